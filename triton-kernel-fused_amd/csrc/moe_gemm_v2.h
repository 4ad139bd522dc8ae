// Grouped GEMM, second generation (16-bit operands): 256x256 output tile per workgroup, four
// waves of 128x128 each (16 MFMA 32x32x16 tiles, 256 accumulator registers per lane), K steps of
// 64 elements double-buffered in 128 KB of LDS.
//
// LDS layout: each operand tile is 256 rows x 128 bytes (one K step), unpadded, with the 16-byte
// chunk index XOR-ed by ((row >> 1) & 7). A row is half of the 64 four-byte banks, so even and
// odd rows use different halves and the XOR spreads 8 rows of each parity over all chunks: the
// MFMA operand reads (16 consecutive rows per 256-byte LDS cycle, one 16-byte chunk each) are
// conflict-free. A wave fills 8 whole rows with one direct-to-LDS load (global_load_lds_dwordx4:
// lane l writes bytes [16l, 16l+16) of a 1 KB block; the lane loads the global chunk that belongs
// in that slot).
//
// K-contiguous operands (activations, weights in the forward) go global->LDS by DMA without
// touching registers. Row-contiguous operands (weights in the dX GEMMs, both wgrad operands) are
// loaded as 8x8 blocks of 16-bit values, transposed in registers and stored; one block per thread
// per K step, with the K chunk running fastest across lanes so each store instruction covers
// whole LDS rows.
#pragma once
#include "moe_common.h"

namespace moe {
namespace v2 {

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

constexpr int NT = 256;
constexpr int TILE = 256;        // rows of each operand tile (P and Q)
constexpr int WT = 128;          // rows of a wave's sub-tile
constexpr int TN = WT / 32;      // MFMA tiles per wave side (4)
constexpr int ROWB = 128;        // bytes per LDS row = one K step (64 16-bit or 128 fp8 values)
constexpr int BK = 64;           // K elements per step for 16-bit operands
template <typename T> constexpr int bk() { return ROWB / (int)sizeof(T); }
constexpr int OPB = TILE * ROWB; // 32 KB per operand per stage
constexpr int STAGEB = 2 * OPB;
constexpr int LDSB = 2 * STAGEB; // 128 KB

__device__ __forceinline__ int swz(int row, int chunk) {
  return row * ROWB + ((chunk ^ ((row >> 1) & 7)) << 4);
}

__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// K-contiguous operand loaded by DMA. Lane l of wave w fills tile row R = w*64 + i*8 + l/8 (i < 8),
// physical chunk l%8, i.e. logical chunk (l%8) ^ ((R >> 1) & 7) = (l%8) ^ ((4*(i&1) + l/16) & 7).
struct DmaKc {
  const char* rowp[8];  // global start of this lane's 8 rows (clamped to a valid row if unused)
  int cbyte[2];         // byte offset of this lane's logical chunk for even / odd i

  __device__ __forceinline__ void init() {
    const int lane = threadIdx.x & 63;
    cbyte[0] = ((lane & 7) ^ (lane >> 4)) << 4;
    cbyte[1] = ((lane & 7) ^ ((4 + (lane >> 4)) & 7)) << 4;
  }
  __device__ __forceinline__ static int row_of(int i) {
    return (int)(threadIdx.x >> 6) * 64 + i * 8 + (int)((threadIdx.x & 63) >> 3);
  }
  template <typename T>
  __device__ __forceinline__ void issue(char* op, int k) {
    char* base = op + (int)(threadIdx.x >> 6) * 64 * ROWB;
    const int kb = k * (int)sizeof(T);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      __builtin_amdgcn_global_load_lds((glb_void*)(rowp[i] + kb + cbyte[i & 1]),
                                       (lds_void*)(base + i * 8 * ROWB), 16, 0, 0);
  }
  __device__ __forceinline__ void prime(int) {}
  __device__ __forceinline__ void commit(char*) const {}
};

// Row-contiguous operand (element (r, k) at src + row(k)*ld + r*2 bytes) through registers.
// Thread t owns the 8x8 block rc = t/8 (rows 8rc..8rc+7), kc = t%8 (K 8kc..8kc+7).
// Loads are unconditional (out-of-range K rows and columns read a clamped, valid address and are
// zeroed at commit), so the 8 loads of a step issue back to back. With GATHER the row index of K
// value k is gather[k]; those indices are fetched one K step ahead of the data that needs them.
template <bool GATHER>
struct RcReg {
  const char* src;      // column r0 of K-row 0
  size_t ld;            // bytes between K rows
  const int32_t* gather;
  int kend;             // K values >= kend are zero
  int rc, kc;
  bool rin;             // this thread's 8 rows are inside the operand
  int nrow[8];          // row indices of the next step to issue (GATHER)
  unsigned valid;       // bit j: K row j of the step in flight is inside [.., kend)
  i32x4 reg[8];

  __device__ __forceinline__ void init(int rvalid) {
    rc = (int)threadIdx.x >> 3;
    kc = (int)threadIdx.x & 7;
    rin = rc * 8 < rvalid;
  }
  __device__ __forceinline__ void fetch_rows(int k0) {
    if constexpr (GATHER) {
#pragma unroll
      for (int j = 0; j < 8; ++j) nrow[j] = gather[min(k0 + kc * 8 + j, kend - 1)];
    }
  }
  // Called once before the first issue(k0).
  __device__ __forceinline__ void prime(int k0) { fetch_rows(k0); }

  template <typename T>
  __device__ __forceinline__ void issue(char*, int k0) {
    const char* base = src + (rin ? rc * 16 : 0);
    unsigned v = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = k0 + kc * 8 + j;
      v |= (rin && k < kend) ? (1u << j) : 0u;
      const int row = GATHER ? nrow[j] : min(k, kend - 1);
      reg[j] = ldg16(base + (size_t)row * ld);
    }
    valid = v;
    fetch_rows(k0 + BK);
  }
  __device__ __forceinline__ void commit(char* op) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (!((valid >> j) & 1u)) reg[j] = zero4();
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      i32x4 t;
      const unsigned sel = (r & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
      for (int w = 0; w < 4; ++w)
        t[w] = (int)__builtin_amdgcn_perm((unsigned)reg[2 * w + 1][r >> 1], (unsigned)reg[2 * w][r >> 1], sel);
      *(i32x4*)(op + swz(rc * 8 + r, kc)) = t;
    }
  }
};

// acc[ti][tj] += P(wave rows) . Q(wave cols) over K in [k0, k1). T is the operand element type;
// a K step is ROWB bytes, i.e. SLABS MFMAs of 2*CPL 16-byte chunks each.
template <typename T, class LP, class LQ>
__device__ __forceinline__ void mainloop(f32x16 (&acc)[TN][TN], LP& lp, LQ& lq, int k0, int k1,
                                         char* smem) {
  constexpr int KS = bk<T>();
  constexpr int CPL = Mfma<T>::CPL;
  constexpr int SLABS = ROWB / (32 * CPL);
  const int nk = (k1 - k0 + KS - 1) / KS;
  if (nk <= 0) return;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int wr = w >> 1, wc = w & 1;
  const int pbase = (wr * WT + (lane & 31)) * ROWB;
  const int qbase = OPB + (wc * WT + (lane & 31)) * ROWB;
  const int half = lane >> 5, sw = (lane >> 1) & 7;  // rows wbase + t*32 + (lane&31)

  lp.prime(k0);
  lq.prime(k0);
  lp.template issue<T>(smem, k0);
  lq.template issue<T>(smem + OPB, k0);
  lp.commit(smem);
  lq.commit(smem + OPB);
  wait_vm();
  __syncthreads();
  for (int it = 0; it < nk; ++it) {
    char* cur = smem + (it & 1) * STAGEB;
    char* nxt = smem + ((it + 1) & 1) * STAGEB;
    const bool more = it + 1 < nk;
    if (more) {
      lp.template issue<T>(nxt, k0 + (it + 1) * KS);
      lq.template issue<T>(nxt + OPB, k0 + (it + 1) * KS);
    }
    // Operand fragments are double-buffered in registers: slab s+1 is read from LDS while the 16
    // MFMAs of slab s execute.
    i32x4 a[2][TN][CPL], b[2][TN][CPL];
    auto load = [&](int f, int s) {
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int cb = (((2 * s + half) * CPL + c) ^ sw) << 4;
#pragma unroll
        for (int t = 0; t < TN; ++t) a[f][t][c] = *(const i32x4*)(cur + pbase + t * 32 * ROWB + cb);
#pragma unroll
        for (int t = 0; t < TN; ++t) b[f][t][c] = *(const i32x4*)(cur + qbase + t * 32 * ROWB + cb);
      }
    };
    load(0, 0);
#pragma unroll
    for (int s = 0; s < SLABS; ++s) {
      const int f = s & 1;
      if (s + 1 < SLABS) load(f ^ 1, s + 1);
      // Keep the prefetch above the MFMAs (the scheduler would otherwise sink each read to its use).
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ti = 0; ti < TN; ++ti)
#pragma unroll
        for (int tj = 0; tj < TN; ++tj) Mfma<T>::stepf(acc[ti][tj], a[f][ti], b[f][tj]);
    }
    if (more) {
      lp.commit(nxt);
      lq.commit(nxt + OPB);
    }
    wait_vm();
    __syncthreads();
  }
}

// Block -> logical tile with XCD grouping: workgroups are dealt to the 8 XCDs round-robin, so
// logical = (b % 8) * (G8 / 8) + b / 8 gives every XCD a contiguous run of logical tiles (shared
// operands stay in that XCD's L2). G8 = gridDim.x, a multiple of 8.
__device__ __forceinline__ int xcd_logical(int b, int g8) { return (b & 7) * (g8 >> 3) + (b >> 3); }

}  // namespace v2
}  // namespace moe
