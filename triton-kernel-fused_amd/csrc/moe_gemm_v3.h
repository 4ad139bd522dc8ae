// Grouped GEMM main loop, third generation (16-bit operands): 256x256 output tile per workgroup,
// four waves of 128x128 (16 MFMA 32x32x16 tiles, 256 accumulator registers per lane), K steps of
// 32 elements in a five-deep ring of LDS stages (5 x 32 KB = 160 KB, all of gfx950's LDS).
//
// Every operand reaches LDS by direct-to-LDS DMA (global_load_lds_dwordx4: lane l of a wave
// writes bytes [16l, 16l+16) of a 1 KB block, from any global address it chooses), issued four
// K steps ahead of its use: with one wave per SIMD nothing else hides memory latency, and four
// steps (~4000 cycles of MFMA work) cover an HBM miss under load. The waits are partial
// (s_waitcnt vmcnt(N) retires loads in issue order), so later stages stay in flight.
//
// Two LDS layouts, chosen by how the operand lies in memory:
//  * K-contiguous rows (activations; weights in the forward): [256 rows][64 bytes], the 16-byte
//    chunk index XOR-ed by (row >> 2) & 3. MFMA operands are read with ds_read_b128 (16 rows of
//    one chunk per 256-byte LDS cycle, conflict-free).
//  * Row-contiguous (weights in the dX GEMMs, both weight-gradient operands: element (r, k) at
//    row(k) * ld + r): [32 K rows][256 r x 2 bytes], the 16-byte chunk index XOR-ed by
//    4 * (k & 3). MFMA operands are read with ds_read_b64_tr_b16, which transposes 16-bit
//    elements across each group of 16 lanes: if lane j of the group addresses 4 consecutive
//    elements D[j][0..3], lane i receives D[4q + i/4][i%4] for q = 0..3. Pointing lane 4q + p at
//    X[k + q][r + 4p .. 4p + 3] hands lane i the values X[k .. k+3][r + i], i.e. four consecutive
//    K of one row, which is the MFMA operand layout. A 32-lane half reads 4 K rows x 64 bytes and
//    the XOR puts them on disjoint banks.
// K values at or past the operand's end (ragged weight-gradient K) read a zero block instead.
#pragma once
#include "moe_gemm_v2.h"

namespace moe {
namespace v3 {

using v2::glb_void;
using v2::lds_void;

constexpr int NT = 256;
constexpr int TILE = 256;
constexpr int WT = 128;
constexpr int TN = WT / 32;
constexpr int KS = 32;                 // K elements per stage
constexpr int KC_ROWB = KS * 2;        // 64 bytes per K-contiguous row
constexpr int RC_ROWB = TILE * 2;      // 512 bytes per K row of a row-contiguous tile
constexpr int OPB = TILE * KC_ROWB;    // 16 KB per operand per stage (both layouts)
constexpr int STAGEB = 2 * OPB;
constexpr int NSTAGE = 5;
constexpr int LDSB = NSTAGE * STAGEB;  // 160 KB
constexpr int LOADS = 4;               // DMA instructions per wave per operand per stage
static_assert(OPB == KS * RC_ROWB, "both layouts fill one operand buffer");

// Source of the K values past an operand's end.
__device__ __attribute__((aligned(1024))) const i32x4 g_zero_block[32] = {};

__device__ __forceinline__ int lane_id() { return (int)threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6); }

// Wave-wide load of a 32-bit value at a uniform address through the scalar cache.
typedef const __attribute__((address_space(4))) int32_t cint32;
__device__ __forceinline__ int sload(const int32_t* p) { return *(cint32*)p; }

using v2::dma16;

// ---------------------------------------------------------------------------------------------
// K-contiguous operand. Lane l of wave w fills row w*64 + 16i + l/4 (i < 4), physical chunk l%4,
// i.e. logical chunk (l%4) ^ ((row >> 2) & 3) = (l%4) ^ (l/16).
struct KcDma {
  const char* rowp[LOADS];  // this lane's rows (clamped to a valid row when outside the operand)
  int cb;                   // byte offset of this lane's logical chunk
  int fbase;                // fragment reads: byte offset of row rbase + (l & 31)
  int coff[2];              // fragment reads: chunk offset of slab 0 / 1

  __device__ __forceinline__ static int row_of(int i) {
    return ((int)threadIdx.x >> 6) * 64 + i * 16 + (lane_id() >> 2);
  }
  // rbase: first operand row of this wave's 128-row block.
  __device__ __forceinline__ void init(int rbase) {
    const int l = lane_id(), h = l >> 5, sw = (l >> 2) & 3;
    cb = ((l & 3) ^ (l >> 4)) << 4;
    fbase = (rbase + (l & 31)) * KC_ROWB;
    coff[0] = ((0 + h) ^ sw) << 4;
    coff[1] = ((2 + h) ^ sw) << 4;
  }
  __device__ __forceinline__ void prime(int) {}
  template <int I>
  __device__ __forceinline__ void issue_one(char* op, int k) {
    dma16(rowp[I] + k * 2 + cb, op + wave_id() * (64 * KC_ROWB) + I * 1024);
  }
  __device__ __forceinline__ void issue(char* op, int k) {
    static_for<0, LOADS>([&](auto i) { issue_one<decltype(i)::value>(op, k); });
  }
  // MFMA operand of tile t (rows rbase + 32t + (l & 31)), slab s (K 16s + 8h .. +7).
  template <int S>
  __device__ __forceinline__ i32x4 frag(const char* op, int t) const {
    return *(const i32x4*)(op + fbase + t * 32 * KC_ROWB + coff[S]);
  }
};

// ---------------------------------------------------------------------------------------------
// Row-contiguous operand: element (r, k) at src + row(k) * ld + 2r (src already at column r0),
// row(k) = gather[k] or k. Lane l of wave w fills K row w*8 + 2i + h (h = l/32), physical chunk
// l%32, i.e. logical chunk (l%32) ^ 4*((2i + h) & 3) = columns 8c .. 8c+7.
template <bool GATHER>
struct RcDma {
  const char* src;
  size_t ld;
  const int32_t* gather;
  int kend;           // K values >= kend read zeros
  int cbyte[2];       // column byte offsets for even / odd i (clamped inside the operand)
  int zoff[2];        // zero-block offsets of the same chunks
  int toff[TN];       // fragment reads: byte offset of tile t for slab 0, first half
  int gi[8];          // GATHER: row indices of this wave's 8 K rows of the next stage

  __device__ __forceinline__ void init(int rbase, int rvalid) {
    const int l = lane_id(), h = l >> 5;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int c = (l & 31) ^ (4 * ((2 * par + h) & 3));
      cbyte[par] = min(8 * c, rvalid - 8) * 2;
      zoff[par] = c * 16;
    }
    const int G = (l >> 4) & 1, j = l & 15, q = j >> 2, p = j & 3;
#pragma unroll
    for (int t = 0; t < TN; ++t)
      toff[t] = (8 * h + q) * RC_ROWB + ((rbase >> 3) + ((4 * t + 2 * G + (p >> 1)) ^ (4 * q))) * 16 +
                8 * (p & 1);
  }
  __device__ __forceinline__ void fetch_rows(int k) {
    if constexpr (GATHER) {
      const int kw = k + wave_id() * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) gi[j] = sload(gather + min(kw + j, kend - 1));
    }
  }
  __device__ __forceinline__ void prime(int k) { fetch_rows(k); }
  // Instruction I of a stage; the last one also fetches the next stage's gather indices.
  template <int I>
  __device__ __forceinline__ void issue_one(char* op, int k) {
    const int w = wave_id(), h = lane_id() >> 5;
    const int kk = k + w * 8 + 2 * I;  // K row of lanes 0-31; lanes 32-63 take kk + 1
    int row;
    if constexpr (GATHER) row = h ? gi[2 * I + 1] : gi[2 * I];
    else row = kk + h;
    const char* g = (kk + h < kend) ? src + (size_t)row * ld + cbyte[I & 1]
                                    : (const char*)g_zero_block + zoff[I & 1];
    dma16(g, op + w * (8 * RC_ROWB) + I * 1024);
    if constexpr (I == LOADS - 1) fetch_rows(k + KS);
  }
  __device__ __forceinline__ void issue(char* op, int k) {
    static_for<0, LOADS>([&](auto i) { issue_one<decltype(i)::value>(op, k); });
  }
  template <int S>
  __device__ __forceinline__ i32x4 frag(const char* op, int t) const {
    typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s4;
    typedef __attribute__((address_space(3))) s4 lds_s4;
    const char* p0 = op + toff[t] + S * 16 * RC_ROWB;
    const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)p0);
    const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p0 + 4 * RC_ROWB));
    typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i2;
    const i2 a = __builtin_bit_cast(i2, lo), b = __builtin_bit_cast(i2, hi);
    return i32x4{a[0], a[1], b[0], b[1]};
  }
};

template <int N>
__device__ __forceinline__ void wait_vm_n() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Wait until at most n stages of DMA (2 * LOADS instructions each) are still in flight.
__device__ __forceinline__ void wait_stages(int n) {
  if (n >= 4) wait_vm_n<8 * LOADS>();
  else if (n == 3) wait_vm_n<6 * LOADS>();
  else if (n == 2) wait_vm_n<4 * LOADS>();
  else if (n == 1) wait_vm_n<2 * LOADS>();
  else wait_vm_n<0>();
}
// Block barrier that also orders this wave's LDS reads before the DMA writes issued after it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// acc[ti][tj] += P(wave rows) . Q(wave cols) over K in [k0, k1). Stage j of the K loop lives in
// buffer j % NSTAGE. Per iteration: MFMAs of slab 0, then (stage it+1 landed, block barrier) the
// DMA of stage it+NSTAGE into the buffer just drained and the slab-0 reads of stage it+1, then
// the MFMAs of slab 1, whose operands were read before the barrier.
template <typename T, class LP, class LQ>
__device__ __forceinline__ void mainloop(f32x16 (&acc)[TN][TN], LP& lp, LQ& lq, int k0, int k1,
                                         char* smem) {
  const int nk = (k1 - k0 + KS - 1) / KS;
  if (nk <= 0) return;
  lp.prime(k0);
  lq.prime(k0);
#pragma unroll
  for (int j = 0; j < NSTAGE; ++j)
    if (j < nk) {
      lp.issue(smem + j * STAGEB, k0 + j * KS);
      lq.issue(smem + j * STAGEB + OPB, k0 + j * KS);
    }
  i32x4 a0[TN], b0[TN], a1[TN], b1[TN];
  wait_stages(min(NSTAGE - 1, nk - 1));
  lds_barrier();
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    a0[t] = lp.template frag<0>(smem, t);
    b0[t] = lq.template frag<0>(smem + OPB, t);
  }
  // Each batch of fragment reads is issued after the first MFMA row of the slab that does not need
  // it, so the in-order LDS counter never makes an MFMA wait for reads issued just before it.
  auto mfma_row = [&](int ti, const i32x4 (&a)[TN], const i32x4 (&b)[TN]) {
#pragma unroll
    for (int tj = 0; tj < TN; ++tj) Mfma<T>::step(acc[ti][tj], a[ti], b[tj]);
  };
  int buf = 0;
  for (int it = 0; it < nk; ++it) {
    const char* cur = smem + buf * STAGEB;
    mfma_row(0, a0, b0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      a1[t] = lp.template frag<1>(cur, t);
      b1[t] = lq.template frag<1>(cur + OPB, t);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ti = 1; ti < TN; ++ti) mfma_row(ti, a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    const bool more = it + 1 < nk;
    const int nbuf = buf + 1 == NSTAGE ? 0 : buf + 1;
    if (more) {
      // Stages issued after stage it+1: it+2 .. min(it+NSTAGE-1, nk-1).
      wait_stages(min(NSTAGE - 2, nk - 2 - it));
      lds_barrier();
      if (it + NSTAGE < nk) {
        lp.issue(smem + buf * STAGEB, k0 + (it + NSTAGE) * KS);
        lq.issue(smem + buf * STAGEB + OPB, k0 + (it + NSTAGE) * KS);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    mfma_row(0, a1, b1);
    __builtin_amdgcn_sched_barrier(0);
    if (more) {
      const char* nxt = smem + nbuf * STAGEB;
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        a0[t] = lp.template frag<0>(nxt, t);
        b0[t] = lq.template frag<0>(nxt + OPB, t);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ti = 1; ti < TN; ++ti) mfma_row(ti, a1, b1);
    __builtin_amdgcn_sched_barrier(0);
    buf = nbuf;
  }
  // The epilogue reuses the LDS.
  lds_barrier();
}

}  // namespace v3
}  // namespace moe
