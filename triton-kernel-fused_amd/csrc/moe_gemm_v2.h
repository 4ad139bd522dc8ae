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

// One direct-to-LDS load: lane l copies 16 bytes from g to LDS byte (l_base + 16 l); l_base is
// wave-uniform. Written as inline asm so that the compiler does not track it: its own tracking
// treats every later LDS read as dependent on every DMA in flight and waits for all of them,
// which would drain the pipeline each step. The K loops order these loads themselves with
// explicit vmcnt waits.
__device__ __forceinline__ void dma16(const void* g, char* l_base) {
  const unsigned m0 = (unsigned)(uintptr_t)(lds_void*)l_base;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(m0)
               : "memory", "m0");
}

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

// ---------------------------------------------------------------------------------------------
// Epilogue staging. The MFMA accumulator gives a lane four consecutive output channels of one
// output row, so storing it directly writes 8 bytes into each of 32 rows per instruction. Instead
// each wave writes its 128x128 block, rounded to T, into its own 32 KB of LDS transposed to
// [q][p] (q = MFMA column = output row, p = MFMA row = output channel; 256 bytes per q row, the
// 16-byte chunk index XOR-ed by (q & 15), so the 8-byte writes of 32 lanes cover all 64 banks
// once), and reads it back as 16-byte chunks with 16 lanes per row: every store instruction then
// writes whole 256-byte row segments.
constexpr int EPI_ROWB = WT * 2;  // bytes per staged row

template <typename T> __device__ __forceinline__ unsigned pack2(float a, float b);
template <> __device__ __forceinline__ unsigned pack2<bf16>(float a, float b) {
  return __builtin_bit_cast(unsigned, bf16x2{(bf16)a, (bf16)b});
}
template <> __device__ __forceinline__ unsigned pack2<f16>(float a, float b) {
  typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 h2;
  return __builtin_bit_cast(unsigned, h2{(f16)a, (f16)b});
}

// Eight 16-bit values of a 16-byte chunk as floats (whole-word conversions only).
template <typename T> __device__ __forceinline__ void unpack8(i32x4 v, float (&f)[8]);
template <> __device__ __forceinline__ void unpack8<bf16>(i32x4 v, float (&f)[8]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const unsigned u = (unsigned)v[w];
    f[2 * w] = __builtin_bit_cast(float, u << 16);
    f[2 * w + 1] = __builtin_bit_cast(float, u & 0xffff0000u);
  }
}
template <> __device__ __forceinline__ void unpack8<f16>(i32x4 v, float (&f)[8]) {
  typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 h2;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const h2 h = __builtin_bit_cast(h2, (unsigned)v[w]);
    f[2 * w] = (float)h[0];
    f[2 * w + 1] = (float)h[1];
  }
}
template <typename T> __device__ __forceinline__ i32x4 pack8(const float (&f)[8]) {
  return i32x4{(int)pack2<T>(f[0], f[1]), (int)pack2<T>(f[2], f[3]), (int)pack2<T>(f[4], f[5]),
               (int)pack2<T>(f[6], f[7])};
}

__device__ __forceinline__ int staged_off(int q, int c) { return q * EPI_ROWB + ((c ^ (q & 15)) << 4); }

// Write this wave's accumulators to its LDS block wl (the mainloop's last barrier has released
// the LDS). Channel p = ti*32 + 8g + 4h + j sits in chunk p/8 = 4ti + g, half h.
template <typename T, int TJ = TN>
__device__ __forceinline__ void stage_acc(const f32x16 (&acc)[TN][TJ], char* wl) {
  const int lane = threadIdx.x & 63, h = lane >> 5;
#pragma unroll
  for (int tj = 0; tj < TJ; ++tj) {
    const int q = tj * 32 + (lane & 31);
#pragma unroll
    for (int ti = 0; ti < TN; ++ti)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        uint2 v = {pack2<T>(acc[ti][tj][4 * g], acc[ti][tj][4 * g + 1]),
                   pack2<T>(acc[ti][tj][4 * g + 2], acc[ti][tj][4 * g + 3])};
        *(uint2*)(wl + staged_off(q, 4 * ti + g) + 8 * h) = v;
      }
  }
}

// The same for 16x16 MFMA tiles (acc[ti][tj]: lane l holds channels ti*16 + 4(l/16) + v, v < 4,
// of output row tj*16 + l%16): chunk 2ti + l/32, half (l/16) & 1. A 32-lane half writes each of
// its 16 rows' chunk once, all 64 banks.
template <typename T, int TI_, int TJ_>
__device__ __forceinline__ void stage_acc(const f32x4 (&acc)[TI_][TJ_], char* wl) {
  const int lane = threadIdx.x & 63, h = (lane >> 4) & 1, g = lane >> 5;
#pragma unroll
  for (int tj = 0; tj < TJ_; ++tj) {
    const int q = tj * 16 + (lane & 15);
#pragma unroll
    for (int ti = 0; ti < TI_; ++ti) {
      uint2 v = {pack2<T>(acc[ti][tj][0], acc[ti][tj][1]), pack2<T>(acc[ti][tj][2], acc[ti][tj][3])};
      *(uint2*)(wl + staged_off(q, 2 * ti + g) + 8 * h) = v;
    }
  }
}

__device__ __forceinline__ i32x4 staged(const char* wl, int q, int c) {
  return *(const i32x4*)(wl + staged_off(q, c));
}

// GEMM outputs are written once and read by a later kernel: stored nontemporal so they do not
// displace operand lines in L2 (measured 1-3% faster on the 256x256 GEMMs).
template <typename P>
__device__ __forceinline__ void st_stream(i32x4 v, P* p) {
  __builtin_nontemporal_store(v, (i32x4*)p);
}

// Plain store of a staged block of WQ rows: out row (row0 + q) gets channels ch0 + 8c .. +7 for
// the rows below row_end and channels below n_ch (a multiple of 8).
template <typename T, int WQ = WT>
__device__ __forceinline__ void store_staged(const char* wl, T* out, long long ld, int row0,
                                             int row_end, int ch0, int n_ch) {
  const int lane = threadIdx.x & 63, c = lane & 15;
  const int ch = ch0 + 8 * c;
#pragma unroll 8
  for (int it = 0; it < WQ / 4; ++it) {
    const int q = it * 4 + (lane >> 4);
    const i32x4 v = staged(wl, q, c);
    if (row0 + q < row_end && ch < n_ch) st_stream(v, out + (size_t)(row0 + q) * ld + ch);
  }
}

}  // namespace v2
}  // namespace moe
