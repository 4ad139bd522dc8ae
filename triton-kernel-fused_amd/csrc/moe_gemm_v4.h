// Grouped GEMM, fourth generation (16-bit operands, both K-contiguous): 256x256 output tile per
// workgroup of EIGHT waves, two per SIMD. Each wave owns a 128 (P) x 64 (Q) sub-tile: 4 x 2 MFMA
// 32x32x16 tiles, 128 accumulators per lane, so two waves fit one SIMD's register file.
//
// Why eight waves: with one wave per SIMD, every LDS-read wait and barrier of that wave idles its
// SIMD's MFMA pipe; with two, the other wave's MFMAs fill the gap. Measured on the config-3 gate/up
// GEMM with the loads switched off, the K loop runs at ~1.6-1.8 PFLOP/s against ~1.3-1.45 for the
// four-wave 128x128-per-wave kernel. LDS read traffic grows 1.5x (6 fragment reads per 8 MFMAs
// instead of 8 per 16), which gfx950's LDS (about 230 bytes per clock per CU for 16-byte reads)
// absorbs.
//
// LDS row layout and K step are those of moe_gemm_v2.h: K steps of 64 16-bit values (one 128-byte
// row per operand row), 16-byte chunk index XOR-ed by ((row >> 1) & 7), held in a ring of five
// 32 KB slots (below). Wave w DMAs rows 32w .. 32w+31 of an operand: four global_load_lds_dwordx4,
// each covering 8 whole 128-byte rows.
#pragma once
#include "moe_gemm_v2.h"

namespace moe {
namespace v4 {

using v2::dma16;
using v2::ROWB;
using v2::swz;

constexpr int NT = 512;
constexpr int NW = NT / 64;
constexpr int TILE = 256;
constexpr int WP = 128;          // P rows (MFMA A side, output channels) per wave
constexpr int WQ = 64;           // Q rows (MFMA B side, tokens) per wave
constexpr int TI = WP / 32;      // 4
constexpr int TJ = WQ / 32;      // 2
constexpr int OPB = TILE * ROWB; // 32 KB: one operand's K step
constexpr int LOADS = TILE / NW / 8;  // DMA instructions per wave per operand per step (4)

__device__ __forceinline__ int lane_id() { return (int)threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6); }
// Wave w: P half wr = w & 1, Q quarter wc = w >> 1.
__device__ __forceinline__ int wave_r() { return wave_id() & 1; }
__device__ __forceinline__ int wave_c() { return wave_id() >> 1; }

// K-contiguous operand. Lane l of wave w fills tile row R = 32w + 8i + l/8 (i < 4), physical
// chunk l%8, i.e. logical chunk (l%8) ^ ((R >> 1) & 7) = (l%8) ^ ((4*(i&1) + l/16) & 7).
struct DmaKc {
  const char* rowp[LOADS];  // this lane's rows (clamped to a valid row when outside the operand)
  int cbyte[2];             // byte offset of this lane's logical chunk for even / odd i

  __device__ __forceinline__ void init() {
    const int l = lane_id();
    cbyte[0] = ((l & 7) ^ (l >> 4)) << 4;
    cbyte[1] = ((l & 7) ^ ((4 + (l >> 4)) & 7)) << 4;
  }
  __device__ __forceinline__ static int row_of(int i) {
    return ((int)threadIdx.x >> 6) * 32 + i * 8 + (lane_id() >> 3);
  }
  template <typename T>
  __device__ __forceinline__ void issue(char* op, int k) {
    char* base = op + wave_id() * 32 * ROWB;
    const int kb = k * (int)sizeof(T);
#pragma unroll
    for (int i = 0; i < LOADS; ++i) dma16(rowp[i] + kb + cbyte[i & 1], base + i * 8 * ROWB);
  }
};

// ---------------------------------------------------------------------------------------------
// Ring pipeline. HIP's __syncthreads() is a workgroup release fence plus s_barrier: the fence
// waits for every outstanding global load of the wave, so a K loop that synchronises with it
// drains its whole load queue once per step, and the queue depth never exceeds one step (about
// 45 GB/s per CU delivered). Here the LDS holds a ring of NSLOT = 5 slots of 32 KB, each one
// operand's K step (256 rows x 128 bytes), filled in the order P0 Q0 P1 Q1 P2 ...; a slot is
// refilled as soon as the step that read it is over, so 1-3 slots (32-96 KB per CU) stay in
// flight across every step boundary. Waits are per wave and partial (s_waitcnt vmcnt(N), loads
// retire in issue order); the block barrier is a bare s_barrier after the wave's own LDS reads
// have returned (s_waitcnt lgkmcnt(0)), which orders (a) every wave's DMA of the slots about to be
// read before any wave reads them and (b) every wave's reads of the slots about to be refilled
// before any wave's DMA into them.
constexpr int NSLOT = 5;
constexpr int SLOTB = OPB;                 // 32 KB
constexpr int RING_LDSB = NSLOT * SLOTB;   // 160 KB

__device__ __forceinline__ void bare_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// Wait until at most n slots (LOADS instructions each) of this wave's DMA are in flight.
__device__ __forceinline__ void wait_slots(int n) {
  if (n >= 3) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * LOADS) : "memory");
  else if (n == 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * LOADS) : "memory");
  else if (n == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LOADS) : "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// K loop over the ring. Step s reads P_s from slot (2s) % NSLOT and Q_s from (2s+1) % NSLOT. The
// synchronisation sits before the last slab of each step: wait for this wave's loads of step s+1,
// barrier, refill the two slots step s has finished reading (with Q_{s+2} and P_{s+3}), read the
// first slab of step s+1, then run the last slab's MFMAs, whose operands were read before the
// barrier and which cover the latency of those reads.
template <typename T>
__device__ __forceinline__ void mainloop_ring(f32x16 (&acc)[TI][TJ], DmaKc& lp, DmaKc& lq, int k0,
                                              int k1, char* smem) {
  constexpr int KS = v2::bk<T>();
  constexpr int CPL = Mfma<T>::CPL;
  constexpr int SLABS = ROWB / (32 * CPL);
  static_assert(SLABS >= 2, "the mid-step barrier needs at least two slabs per step");
  const int nk = (k1 - k0 + KS - 1) / KS;
  if (nk <= 0) return;
  const int lane = lane_id();
  const int pbase = (wave_r() * WP + (lane & 31)) * ROWB;
  const int qbase = (wave_c() * WQ + (lane & 31)) * ROWB;
  const int half = lane >> 5, sw = (lane >> 1) & 7;
  const int nslab = 2 * nk;  // ring loads of the whole loop: P_j is load 2j, Q_j is load 2j+1

  // Prologue: loads 0..NSLOT-1 (P0 Q0 P1 Q1 P2) into slots 0..4.
  int issued = 0;
  for (; issued < NSLOT && issued < nslab; ++issued) {
    char* slot = smem + issued * SLOTB;
    const int k = k0 + (issued >> 1) * KS;
    if (issued & 1) lq.template issue<T>(slot, k);
    else lp.template issue<T>(slot, k);
  }
  wait_slots(issued - 2);
  bare_barrier();

  i32x4 a[2][TI][CPL], b[2][TJ][CPL];
  auto load = [&](int f, const char* ps, const char* qs, int sl) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int cb = (((2 * sl + half) * CPL + c) ^ sw) << 4;
#pragma unroll
      for (int t = 0; t < TI; ++t) a[f][t][c] = *(const i32x4*)(ps + t * 32 * ROWB + cb);
#pragma unroll
      for (int t = 0; t < TJ; ++t) b[f][t][c] = *(const i32x4*)(qs + t * 32 * ROWB + cb);
    }
  };
  int sp = 0, sq = 1;  // slots of P_s, Q_s
  load(0, smem + sp * SLOTB + pbase, smem + sq * SLOTB + qbase, 0);
  for (int s = 0; s < nk; ++s) {
    const char* ps = smem + sp * SLOTB + pbase;
    const char* qs = smem + sq * SLOTB + qbase;
    const int np = sp + 2 >= NSLOT ? sp + 2 - NSLOT : sp + 2;
    const int nq = sq + 2 >= NSLOT ? sq + 2 - NSLOT : sq + 2;
#pragma unroll
    for (int sl = 0; sl < SLABS; ++sl) {
      const int f = sl & 1;
      if (sl + 1 < SLABS) {
        load(f ^ 1, ps, qs, sl + 1);
      } else if (s + 1 < nk) {
        wait_slots(issued - (2 * s + 4));
        bare_barrier();
        // Slot sp (P_s) takes load 2s+5 = Q_{s+2}; slot sq (Q_s) takes load 2s+6 = P_{s+3}.
        if (issued < nslab) {
          lq.template issue<T>(smem + sp * SLOTB, k0 + (s + 2) * KS);
          ++issued;
        }
        if (issued < nslab) {
          lp.template issue<T>(smem + sq * SLOTB, k0 + (s + 3) * KS);
          ++issued;
        }
        load(f ^ 1, smem + np * SLOTB + pbase, smem + nq * SLOTB + qbase, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ti = 0; ti < TI; ++ti)
#pragma unroll
        for (int tj = 0; tj < TJ; ++tj) Mfma<T>::stepf(acc[ti][tj], a[f][ti], b[f][tj]);
      __builtin_amdgcn_sched_barrier(0);
    }
    sp = np;
    sq = nq;
  }
  // The epilogue reuses the LDS: every wave's reads of the last step must be over.
  bare_barrier();
}

// Block -> logical tile with XCD grouping (see v2::xcd_logical).
using v2::xcd_logical;

}  // namespace v4
}  // namespace moe
