// Grouped GEMM, fourth generation (16-bit and fp8 operands): 256x256 output tile per
// workgroup of EIGHT waves, two per SIMD. Each wave owns a 128 (P) x 64 (Q) sub-tile: 8 x 4 MFMA
// 16x16x32 tiles (token GEMMs) or 4 x 2 32x32x16 / 32x32x64-fp8 tiles (weight gradients, fp8),
// 128 accumulators per lane either way, so two waves fit one SIMD's register file.
//
// Why eight waves: with one wave per SIMD, every LDS-read wait and barrier of that wave idles its
// SIMD's MFMA pipe; with two, the other wave's MFMAs fill the gap. Measured on the config-3 gate/up
// GEMM with the loads switched off, the K loop runs at ~1.6-1.8 PFLOP/s against ~1.3-1.45 for the
// four-wave 128x128-per-wave kernel. LDS read traffic per FLOP grows 1.5x (a 128x64 wave block
// instead of 128x128), which gfx950's LDS (about 230 bytes per clock per CU for 16-byte reads)
// absorbs.
//
// LDS row layout and K step are those of moe_gemm_v2.h: K steps of 64 16-bit values (one 128-byte
// row per operand row), 16-byte chunk index XOR-ed by ((row >> 1) & 7), held in a ring of five
// 32 KB slots (below). Wave w DMAs rows 32w .. 32w+31 of an operand: four global_load_lds_dwordx4,
// each covering 8 whole 128-byte rows.
#pragma once
#include "moe_gemm_v3.h"

namespace moe {
namespace v4 {

using v2::dma16;
using v2::ROWB;
using v2::swz;

constexpr int NT = 512;
constexpr int NW = NT / 64;
constexpr int TILE = 256;
constexpr int WP = 128;          // P rows (MFMA A side, output channels) per wave
constexpr int WQ = TILE / (NW / 2);  // Q rows (MFMA B side, tokens) per wave
constexpr int RPW = TILE / NW;   // operand rows (Kc) or K rows x 4 (Rc) each wave loads per slot
constexpr int TI = WP / 32;      // 4   (32x32 MFMA tiles: fp8)
constexpr int TJ = WQ / 32;      // 2
constexpr int TI16 = WP / 16;    // 8   (16x16x32 MFMA tiles: 16-bit operands)
constexpr int TJ16 = WQ / 16;    // 4
constexpr int OPB = TILE * ROWB; // 32 KB: one operand's K step
constexpr int LOADS = TILE / NW / 8;  // DMA instructions per wave per operand per step (4)
// K-split of the last partial wave: only for K of at least SPLIT_MIN_STEPS ring steps (the
// handoff's device-scope acquire invalidates the XCD's L2, which costs short-K GEMMs more than
// the split saves: measured +20% on a 88-step dX GEMM, -2 to -8% at 16-32 steps), at most
// SPLIT_MAX pieces of at least 8 steps.
constexpr int SPLIT_MIN_STEPS = 40;
constexpr int SPLIT_MAX = 4;

__device__ __forceinline__ int lane_id() { return (int)threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6); }
// Wave w: P half wr = w & 1, Q quarter wc = w >> 1.
__device__ __forceinline__ int wave_r() { return wave_id() & 1; }
__device__ __forceinline__ int wave_c() { return wave_id() >> 1; }

// ---------------------------------------------------------------------------------------------
// Operand loaders. Each fills one ring slot (one operand's 64-value K step, 32 KB) with four DMA
// instructions per wave (issue) and reads MFMA operand fragments from a slot (frag): fragment t
// (FR rows of this wave's block), slab sl, chunk c (< CPL). FR = 32 (32x32 MFMAs): lane l holds
// row l%32 and the K chunk l/32 of a 16-value (16-bit) or 64-value (fp8, CPL = 2) slab. FR = 16
// (16x16x32 MFMAs, 16-bit only): lane l holds row l%16 and K chunk l/16 of a 32-value slab.

// K-contiguous operand: [256 rows][128 bytes], chunk index XOR-ed by (row >> 1) & 7. Lane l of
// wave w fills row R = 32w + 8i + l/8 (i < 4), physical chunk l%8, i.e. logical chunk
// (l%8) ^ ((R >> 1) & 7) = (l%8) ^ ((4*(i&1) + l/16) & 7).
template <int FR>
struct KcLoadT {
  const char* rowp[LOADS];  // this lane's rows (clamped to a valid row when outside the operand)
  int cbyte[2];             // byte offset of this lane's logical chunk for even / odd i
  int fbase;                // fragment reads: byte offset of row rbase + l % FR
  int half, sw;             // K chunk of the lane within a slab (l / FR); swizzle of its rows

  // rbase: first operand row of this wave's fragment block.
  __device__ __forceinline__ void init(int rbase) {
    const int l = lane_id();
    cbyte[0] = ((l & 7) ^ (l >> 4)) << 4;
    cbyte[1] = ((l & 7) ^ ((4 + (l >> 4)) & 7)) << 4;
    fbase = (rbase + (l & (FR - 1))) * ROWB;
    half = l / FR;
    sw = (l >> 1) & 7;  // ((row >> 1) & 7) for row = rbase + 16u + l % FR (rbase % 16 == 0)
  }
  __device__ __forceinline__ static int row_of(int i) {
    return ((int)threadIdx.x >> 6) * RPW + i * 8 + (lane_id() >> 3);
  }
  __device__ __forceinline__ void prime(int) {}
  template <typename T>
  __device__ __forceinline__ void issue(char* slot, int k) {
    char* base = slot + wave_id() * RPW * ROWB;
    const int kb = k * (int)sizeof(T);
#pragma unroll
    for (int i = 0; i < LOADS; ++i) dma16(rowp[i] + kb + cbyte[i & 1], base + i * 8 * ROWB);
  }
  // One of the LOADS instructions of issue(), then issue_done() after the last.
  template <typename T, int I>
  __device__ __forceinline__ void issue_i(char* slot, int k) {
    dma16(rowp[I] + k * (int)sizeof(T) + cbyte[I & 1], slot + wave_id() * RPW * ROWB + I * 8 * ROWB);
  }
  __device__ __forceinline__ void issue_done(int) {}
  template <int CPL>
  __device__ __forceinline__ i32x4 frag(const char* slot, int t, int sl, int c) const {
    static_assert(FR == 32 || CPL == 1, "16-row fragments are for 16-bit operands");
    const int cb = ((((64 / FR) * sl + half) * CPL + c) ^ sw) << 4;
    return *(const i32x4*)(slot + fbase + t * FR * ROWB + cb);
  }
};
using KcLoad = KcLoadT<32>;
using KcLoad16 = KcLoadT<16>;

// K-contiguous fp8 operand with one E8M0 scale per (row, K step of 128) for the B side of
// v_mfma_scale_f32_32x32x64_f8f6f4. The scales of K step s sit in byte row s of a table (row
// pitch s_ld) with 256 bytes per token tile (tile index mt at byte 256 mt), two per lane: bytes
// 2j and 2j+1 of a wave's 64 are its rows j and j+32, so one 16-bit load gives lane l the scales
// of its two fragment rows (selected by the MFMA's op_sel, 0 for tj = 0, 1 for tj = 1). The loads
// are inline asm, like the DMAs, so the compiler adds no waits of its own, and the ring's waits
// cover them: steps 0 and 1 go out before the prologue's DMAs; step s+2's right after its Q
// refill in step s's last slab, ahead of the P refill that the next per-step wait leaves in
// flight. Three registers hold the scales of steps s-1 / s / s+1 (x0 / x1 / x2); shift_scale
// moves them down and loads step s+2's into x2. fence_scales (after each wait) re-defines x1 and
// x2 there, so no compiler copy of them can come before it. The prologue must run inside
// mainloop_ring (PRE = false): its loads are then in flight in straight-line code only.
struct KcLoadS : KcLoadT<32> {
  static constexpr bool SCALED = true;
  const char* sp;  // this lane's scale pair in the table's row 0
  long long s_ld;
  unsigned x0 = 0, x1 = 0, x2 = 0;
  __device__ __forceinline__ const char* at(int k) const { return sp + (long long)(k >> 7) * s_ld; }
  // The scales of K steps k0 and k1, loaded ahead of the prologue's DMAs. The loads (and the
  // shift below) write the registers in place through tied asm operands, so the three values keep
  // their registers across the loop and no compiler copy reads a register whose load is still in
  // flight.
  __device__ __forceinline__ void prologue_scales(int k0, int k1) {
    asm volatile("global_load_ushort %0, %2, off\n\tglobal_load_ushort %1, %3, off"
                 : "+v"(x1), "+v"(x2)
                 : "v"(at(k0)), "v"(at(k1))
                 : "memory");
  }
  __device__ __forceinline__ void shift_scale(int k) {
    asm volatile("v_mov_b32 %0, %1\n\tv_mov_b32 %1, %2\n\tglobal_load_ushort %2, %3, off"
                 : "+v"(x0), "+v"(x1), "+v"(x2)
                 : "v"(at(k))
                 : "memory");
  }
  __device__ __forceinline__ void fence_scales() { asm volatile("" : "+v"(x1), "+v"(x2)); }
};
// Loaders with per-step B scales (KcLoadS) declare SCALED = true.
template <class L, class = void>
struct Scaled : std::false_type {};
template <class L>
struct Scaled<L, std::void_t<decltype(L::SCALED)>> : std::bool_constant<L::SCALED> {};
template <class L>
__device__ __forceinline__ void shift_scale_of(L& l, int k) {
  if constexpr (Scaled<L>::value) l.shift_scale(k);
}

// Row-contiguous operand (element (r, k) at src + row(k) * ld + 2r, src at column r0; row(k) =
// gather[k] or k): [64 K rows][256 r x 2 bytes], the 16-byte chunk index XOR-ed by 4 * (k & 3)
// (the XOR applies to the whole chunk index: wave blocks of 64 columns start at odd multiples of 8).
// Fragments are read with ds_read_b64_tr_b16, which transposes 16-bit elements across each group
// of 16 lanes: if lane j of the group addresses 4 consecutive elements D[j][0..3], lane i receives
// D[4q + i/4][i%4] for q = 0..3. Pointing lane 4q + p at X[k + q][r + 4p .. 4p + 3] hands lane i
// the values X[k .. k+3][r + i], i.e. four consecutive K of one row, the MFMA operand layout; a
// 32-lane half reads 4 K rows x 64 bytes and the XOR puts them on disjoint banks. Lane l of wave w
// fills K row 8w + 2i + h (h = l/32), physical chunk l%32, i.e. logical chunk
// (l%32) ^ 4*((2i + h) & 3) = columns 8c .. 8c+7. K values at or past kend read a zero block.
// FR = 32: the two 16-lane groups of a 32-lane half take columns 16G .. 16G+15 of the fragment
// and the halves K rows 8h .. 8h+7 of a 16-row slab; FR = 16: the four 16-lane groups g take the
// fragment's 16 columns and K rows 8g .. 8g+7 of a 32-row slab, and the chunk XOR also takes
// 2 * ((k >> 3) & 3) (= 2g): a 32-lane half (g, g+1) then varies chunk bits 0 (p), 1 (g) and
// 2-3 (q) and covers the 64 banks once.
constexpr int RC_ROWB = TILE * 2;  // 512 bytes per K row
template <bool GATHER, int NFRAG, int FR = 32>
struct RcLoad {
  const char* src;
  size_t ld;
  const int32_t* gather;
  int kend;           // K values >= kend read zeros
  int cbyte[2];       // column byte offsets for even / odd i (clamped inside the operand)
  int zoff[2];        // zero-block offsets of the same chunks
  int toff[NFRAG];    // fragment reads: byte offset of fragment t for slab 0
  int gi[GATHER ? 2 * LOADS : 1];  // GATHER: row indices of this wave's K rows of the next issue

  // rbase: first column (r) of this wave's fragment block; rvalid: columns inside the operand.
  __device__ __forceinline__ void init(int rbase, int rvalid) {
    const int l = lane_id(), h = l >> 5;
    // FR = 16 also XORs 2 * ((k >> 3) & 3) (k >> 3 = w for this wave's K rows 8w .. 8w+7).
    const int wx = FR == 16 ? 2 * (wave_id() & 3) : 0;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int c = (l & 31) ^ (4 * ((2 * par + h) & 3)) ^ wx;
      cbyte[par] = min(8 * c, rvalid - 8) * 2;
      zoff[par] = c * 16;
    }
    const int G = (l >> 4) & 1, j = l & 15, q = j >> 2, p = j & 3;
#pragma unroll
    for (int t = 0; t < NFRAG; ++t) {
      if constexpr (FR == 32)
        toff[t] = (8 * h + q) * RC_ROWB +
                  ((((rbase >> 3) + 4 * t + 2 * G + (p >> 1)) ^ (4 * q)) * 16) + 8 * (p & 1);
      else
        toff[t] = (8 * (l >> 4) + q) * RC_ROWB +
                  ((((rbase >> 3) + 2 * t + (p >> 1)) ^ (4 * q) ^ (2 * (l >> 4))) * 16) + 8 * (p & 1);
    }
  }
  // The column clamp of a new r range (rvalid columns inside the operand); the rest of init()
  // depends only on the lane and rbase.
  __device__ __forceinline__ void set_rvalid(int rvalid) {
    const int l = lane_id(), h = l >> 5;
    const int wx = FR == 16 ? 2 * (wave_id() & 3) : 0;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int c = (l & 31) ^ (4 * ((2 * par + h) & 3)) ^ wx;
      cbyte[par] = min(8 * c, rvalid - 8) * 2;
    }
  }
  __device__ __forceinline__ void fetch_rows(int k) {
    if constexpr (GATHER) {
      const int kw = k + wave_id() * 2 * LOADS;
#pragma unroll
      for (int j = 0; j < 2 * LOADS; ++j) gi[j] = v3::sload(gather + min(kw + j, kend - 1));
    }
  }
  // Called once with the first K of the operand's first issue.
  __device__ __forceinline__ void prime(int k) { fetch_rows(k); }
  template <typename T, int I>
  __device__ __forceinline__ void issue_i(char* slot, int k) {
    const int w = wave_id(), h = lane_id() >> 5;
    const int kk = k + w * 2 * LOADS + 2 * I;  // K row of lanes 0-31; lanes 32-63 take kk + 1
    int row;
    if constexpr (GATHER) row = h ? gi[2 * I + 1] : gi[2 * I];
    else row = kk + h;
    const char* g = (kk + h < kend) ? src + (size_t)row * ld + cbyte[I & 1]
                                    : (const char*)v3::g_zero_block + zoff[I & 1];
    dma16(g, slot + w * (2 * LOADS * RC_ROWB) + I * 1024);
  }
  // After the last issue_i of a slot: the gathered row indices of the next issue.
  __device__ __forceinline__ void issue_done(int k) { fetch_rows(k + 64); }
  template <typename T>
  __device__ __forceinline__ void issue(char* slot, int k) {
    static_for<0, LOADS>([&](auto ic) { issue_i<T, decltype(ic)::value>(slot, k); });
    issue_done(k);
  }
  template <int CPL>
  __device__ __forceinline__ i32x4 frag(const char* slot, int t, int sl, int) const {
    typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s4;
    typedef __attribute__((address_space(3))) s4 lds_s4;
    const char* p0 = slot + toff[t] + sl * (FR == 32 ? 16 : 32) * RC_ROWB;
    const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)p0);
    const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p0 + 4 * RC_ROWB));
    typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i2;
    const i2 x = __builtin_bit_cast(i2, lo), y = __builtin_bit_cast(i2, hi);
    return i32x4{x[0], x[1], y[0], y[1]};
  }
};

// ---------------------------------------------------------------------------------------------
// Ring pipeline. HIP's __syncthreads() is a workgroup release fence plus s_barrier: the fence
// waits for every outstanding global load of the wave, so a K loop that synchronises with it
// drains its whole load queue once per step, and the queue depth never exceeds one step (about
// 45 GB/s per CU delivered). Here the LDS holds a ring of NSLOT = 5 slots of 32 KB, each one
// operand's K step, filled in the order P0 Q0 P1 Q1 P2 ...; a slot is refilled as soon as the step
// that read it is over, so 1-3 slots (32-96 KB per CU) stay in flight across every step boundary.
// Waits are per wave and partial (s_waitcnt vmcnt(N), loads retire in issue order); the block
// barrier is a bare s_barrier after the wave's own LDS reads have returned (s_waitcnt
// lgkmcnt(0)), which orders (a) every wave's DMA of the slots about to be read before any wave
// reads them and (b) every wave's reads of the slots about to be refilled before any wave's DMA
// into them.
constexpr int NSLOT = 5;
constexpr int SLOTB = OPB;                 // 32 KB
constexpr int RING_LDSB = NSLOT * SLOTB;   // 160 KB
static_assert(64 * RC_ROWB == SLOTB, "both layouts fill one slot");

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

// K loop over the ring: acc[ti][tj] += P(wave block) . Q(wave block) over K in [k0, k1). Step s
// reads P_s from slot (2s) % NSLOT and Q_s from (2s+1) % NSLOT. The synchronisation sits at the
// last slab of each step and is the same at every step: wait for this wave's loads of step s+1
// (one slot, P_{s+2}, may stay in flight), barrier, read the first slab of step s+1, then run the
// last slab's MFMAs. The refills of the slots step s has finished go out between MFMAs: Q_{s+2}
// one DMA after every second MFMA of that slab, P_{s+3} one DMA per four MFMAs over the first two
// slabs of step s+1; every other slab interleaves the next slab's fragment reads with its MFMAs. Spreading the
// DMAs and LDS reads over the MFMAs and keeping the loop free of branches measured ~8% faster
// than issuing them in bursts. Refills past the end re-read the last K step into slots nobody
// reads again, and the prologue fills the slots the same way at every K length, so every wait is
// a constant; the loop end waits for all DMAs.
// COMPUTE false (a wave whose token rows are all past the group end): the same loads and
// barriers, no fragment reads and no MFMAs, so the SIMD's other wave has the LDS and the matrix
// pipe to itself.
// Prologue DMAs of the ring over K in [k0, k1): loads [first, first + count) of the sequence
// P0 Q0 P1 Q1 P2, load i into slot (base + i) % NSLOT. A persistent kernel issues the next tile's
// first loads while the current tile's epilogue runs (mainloop_ring with PRE = true then skips
// them).
template <typename T, class LP, class LQ>
__device__ __forceinline__ void ring_prologue(LP& lp, LQ& lq, int k0, int k1, char* smem, int base,
                                              int first, int count) {
  constexpr int KS = v2::bk<T>();
  const int nk = (k1 - k0 + KS - 1) / KS;
  const int klast = k0 + (nk - 1) * KS;
  if (first == 0) {
    lp.prime(k0);
    lq.prime(k0);
    if constexpr (Scaled<LQ>::value) lq.prologue_scales(k0, min(k0 + KS, klast));
  }
  for (int i = first; i < first + count; ++i) {
    const int si = base + i >= NSLOT ? base + i - NSLOT : base + i;
    char* slot = smem + si * SLOTB;
    const int k = min(k0 + (i >> 1) * KS, klast);
    if (i & 1) lq.template issue<T>(slot, k);
    else lp.template issue<T>(slot, k);
  }
}

// PRE: the caller has issued all NSLOT prologue loads with ring_prologue(..., base, ...) (and
// possibly other memory operations after them, which the first wait then also covers).
template <typename T, bool COMPUTE = true, bool PRE = false, typename AccV, int TI_, int TJ_,
          class LP, class LQ>
__device__ __forceinline__ void mainloop_ring(AccV (&acc)[TI_][TJ_], LP& lp, LQ& lq, int k0, int k1,
                                              char* smem, int base = 0) {
  constexpr int KS = v2::bk<T>();
  constexpr int CPL = Mfma<T>::CPL;
  constexpr int FR = sizeof(AccV) == sizeof(f32x4) ? 16 : 32;  // MFMA tile rows
  static_assert(TI_ * FR == WP && TJ_ * FR == WQ, "accumulators cover the wave's block");
  constexpr int SLABS = ROWB / ((FR == 16 ? 64 : 32) * CPL);
  static_assert(SLABS >= 2, "the mid-step barrier needs at least two slabs per step");
  // Fragment schedule: 32x32 16-bit tiles double-buffer both operands' fragments and defer the P
  // refill to the next step (FB == 2); fp8 and 16x16x32 tiles roll the A fragments and
  // double-buffer B (ROLL), every refill in the synchronising slab.
  constexpr bool ROLL = FR == 16 || CPL > 1;
  // Only the ROLL schedule has a non-computing copy; the FB == 2 schedule always reads fragments
  // and issues its MFMAs.
  static_assert(COMPUTE || ROLL, "COMPUTE = false is implemented for the ROLL schedule only");
  constexpr int NM = TI_ * TJ_;  // MFMAs per slab
  const int nk = (k1 - k0 + KS - 1) / KS;
  if (nk <= 0) return;

  // Prologue: loads 0..NSLOT-1 (P0 Q0 P1 Q1 P2) into slots base .. base+4 (mod NSLOT).
  const int klast = k0 + (nk - 1) * KS;
  constexpr int PRO = ROLL ? NSLOT : NSLOT - 1;  // FB == 2: P2 goes out with step 0's slab 0
  static_assert(!PRE || ROLL, "a pre-issued prologue is implemented for the ROLL schedule");
  if constexpr (!PRE) ring_prologue<T>(lp, lq, k0, k1, smem, base, 0, PRO);
  static_assert(!Scaled<LQ>::value || (ROLL && !PRE), "block scales need the ROLL schedule and an in-loop prologue");
  wait_slots(PRO - 2);
  // Pending P refill (slot, K) issued during the next step's first slab.
  int pp_slot = base == 0 ? NSLOT - 1 : base - 1, pp_k = min(k0 + 2 * KS, klast);
  bare_barrier();
  if constexpr (Scaled<LQ>::value) lq.fence_scales();

  constexpr int FB = ROLL ? 1 : 2;
  i32x4 a[FB][TI_][CPL], b[FB][TJ_][CPL];
  auto load = [&](int f, const char* ps, const char* qs, int sl) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
#pragma unroll
      for (int t = 0; t < TI_; ++t) a[f][t][c] = lp.template frag<CPL>(ps, t, sl, c);
#pragma unroll
      for (int t = 0; t < TJ_; ++t) b[f][t][c] = lq.template frag<CPL>(qs, t, sl, c);
    }
  };
  // ROLL: one A buffer, two B buffers.
  i32x4 ra[TI_][CPL], rb[2][TJ_][CPL];
  int sp = base, sq = base + 1 == NSLOT ? 0 : base + 1;  // slots of P_s, Q_s
  if constexpr (FB == 2) load(0, smem + sp * SLOTB, smem + sq * SLOTB, 0);
  if constexpr (ROLL) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
#pragma unroll
      for (int t = 0; t < TI_; ++t) ra[t][c] = lp.template frag<CPL>(smem + sp * SLOTB, t, 0, c);
#pragma unroll
      for (int t = 0; t < TJ_; ++t) rb[0][t][c] = lq.template frag<CPL>(smem + sq * SLOTB, t, 0, c);
    }
    // lgkmcnt(0) (vmcnt and expcnt at their maxima) as a real waitcnt instruction, so the
    // compiler's loop-entry state holds no LDS reads and the in-loop waits stay partial.
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  for (int s = 0; s < nk; ++s) {
    const char* ps = smem + sp * SLOTB;
    const char* qs = smem + sq * SLOTB;
    const int np = sp + 2 >= NSLOT ? sp + 2 - NSLOT : sp + 2;
    const int nq = sq + 2 >= NSLOT ? sq + 2 - NSLOT : sq + 2;
#pragma unroll
    for (int sl = 0; sl < SLABS; ++sl) {
      if constexpr (ROLL) {
        // B fragments double-buffered (the next slab's reads after the slab's first MFMAs), A
        // fragments rolled: each is re-read for the next slab right after its last MFMA of this
        // slab, so every read has the rest of the slab's MFMAs to land, within the register
        // budget of one buffer. The synchronising slab waits, barriers, then reads step s+1's
        // first slab the same way and issues both refills, one DMA per NM / 8 MFMAs.
        const int f = sl & 1;
        const bool sync = sl + 1 == SLABS;
        const char* nps = sync ? smem + np * SLOTB : ps;
        const char* nqs = sync ? smem + nq * SLOTB : qs;
        const int nsl = sync ? 0 : sl + 1;
        int kq = 0, kp = 0;
        char* qslot = smem + sp * SLOTB;
        char* pslot = smem + sq * SLOTB;
        if (sync) {
          wait_slots(1);
          bare_barrier();
          if constexpr (Scaled<LQ>::value) lq.fence_scales();
          kq = min(k0 + (s + 2) * KS, klast);
          kp = min(k0 + (s + 3) * KS, klast);
        }
        constexpr int DI = NM / (2 * LOADS);
        static_assert(DI * 2 * LOADS == NM, "refill DMAs spread evenly over the slab");
        __builtin_amdgcn_sched_barrier(0);
        static_for<0, NM>([&](auto ic) {
          constexpr int I = decltype(ic)::value;
          if constexpr (COMPUTE) {
            if constexpr (Scaled<LQ>::value) {
              // MFMAs after this slab's shift_scale find step s's scales in x0.
              const unsigned sc = (sync && I >= LOADS * DI) ? lq.x0 : lq.x1;
              Mfma<T>::template stepf_sb<I % TJ_>(acc[I / TJ_][I % TJ_], ra[I / TJ_], rb[f][I % TJ_], sc);
            } else {
              Mfma<T>::stepf(acc[I / TJ_][I % TJ_], ra[I / TJ_], rb[f][I % TJ_]);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (COMPUTE && I < TJ_) {
#pragma unroll
            for (int c = 0; c < CPL; ++c) rb[f ^ 1][I][c] = lq.template frag<CPL>(nqs, I, nsl, c);
          }
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (COMPUTE && I % TJ_ == TJ_ - 1) {
#pragma unroll
            for (int c = 0; c < CPL; ++c) ra[I / TJ_][c] = lp.template frag<CPL>(nps, I / TJ_, nsl, c);
          }
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (I % DI == DI - 1) {
            constexpr int d = I / DI;
            if (sync) {
              if constexpr (d < LOADS) lq.template issue_i<T, d>(qslot, kq);
              else lp.template issue_i<T, d - LOADS>(pslot, kp);
              if constexpr (d == LOADS - 1) shift_scale_of(lq, kq);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        });
        if (sync) {
          lq.issue_done(kq);
          lp.issue_done(kp);
        }
      } else {
        const int f = sl & 1;
        if (sl + 1 == SLABS) {
          // Synchronisation step, the same at every step (no branches around the MFMAs): wait for
          // step s+1, barrier, read its first slab, and issue the Q refill one DMA per two MFMAs;
          // the P refill goes out over the next step's first two slabs. Past the last
          // step the refills re-read the last K step into slots that are never read again, and
          // the reads of "step s+1" read stale LDS into unused registers; the loop end drains the
          // DMAs.
          wait_slots(1);
          bare_barrier();
          load(f ^ 1, smem + np * SLOTB, smem + nq * SLOTB, 0);
          const int kq = min(k0 + (s + 2) * KS, klast), kp = min(k0 + (s + 3) * KS, klast);
          char* qslot = smem + sp * SLOTB;
          __builtin_amdgcn_sched_barrier(0);
          static_assert(NM == 2 * LOADS, "one refill DMA per two MFMAs");
          static_for<0, NM>([&](auto ic) {
            constexpr int I = decltype(ic)::value;
            Mfma<T>::step(acc[I / TJ_][I % TJ_], a[f][I / TJ_][0], b[f][I % TJ_][0]);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (I % 2 == 1) lq.template issue_i<T, I / 2>(qslot, kq);
            __builtin_amdgcn_sched_barrier(0);
          });
          lq.issue_done(kq);
          pp_slot = sq;
          pp_k = kp;
        } else {
          // Next slab's fragment reads (and, in slabs 0 and 1, the pending P refill) between the
          // MFMAs.
          static_for<0, NM>([&](auto ic) {
            constexpr int I = decltype(ic)::value;
            if constexpr (I < TI_) a[f ^ 1][I][0] = lp.template frag<CPL>(ps, I, sl + 1, 0);
            else if constexpr (I < TI_ + TJ_) b[f ^ 1][I - TI_][0] = lq.template frag<CPL>(qs, I - TI_, sl + 1, 0);
            __builtin_amdgcn_sched_barrier(0);
            Mfma<T>::step(acc[I / TJ_][I % TJ_], a[f][I / TJ_][0], b[f][I % TJ_][0]);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (I % 4 == 3) {
              if (sl == 0) lp.template issue_i<T, I / 4>(smem + pp_slot * SLOTB, pp_k);
              if (sl == 1) lp.template issue_i<T, 2 + I / 4>(smem + pp_slot * SLOTB, pp_k);
            }
            __builtin_amdgcn_sched_barrier(0);
          });
          if (sl == 1) lp.issue_done(pp_k);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    sp = np;
    sq = nq;
  }
  // The epilogue reuses the LDS: every wave's reads of the last step must be over (and, with the
  // interleaved refills, every DMA into the ring has landed).
  wait_slots(0);
  bare_barrier();
}

// Expert lookup of token tiles from the sorted-row offsets, in scalar registers: a walk over the
// experts that resumes where the previous lookup stopped (a workgroup's token tiles come in
// non-decreasing order when its tile stride is a multiple of the tile group; otherwise the walk
// steps back from where it is). The offsets are read with scalar loads (scalar cache, counted
// apart from the vector memory operations whose waits the ring relies on).
struct Experts {
  const int32_t* off;
  int E;
  int n_mt;     // token tiles in total
  int e, pref;  // walk state: expert e and the index of its first token tile
  __device__ __forceinline__ void init(const int32_t* offsets, int n_experts) {
    off = offsets;
    E = n_experts;
    const int l = lane_id();
    int tot = 0;
    for (int base = 0; base < E; base += 64) {
      const int x = base + l;
      int c = x < E ? (offsets[x + 1] - offsets[x] + TILE - 1) / TILE : 0;
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) c += __shfl_xor(c, d, 64);
      tot += c;
    }
    n_mt = __builtin_amdgcn_readfirstlane(tot);
    e = 0;
    pref = 0;
  }
  // Expert of token tile mt (< n_mt) and its rows [m0, m_end).
  __device__ __forceinline__ void lookup(int mt, int& ex, int& m0, int& m_end) {
    int o0 = v3::sload(off + e), o1 = v3::sload(off + e + 1);
    // With tile groups a workgroup's token tiles can step back by up to a group: walk back
    // from the current expert rather than restarting at expert 0 (O(distance), not O(E)).
    while (mt < pref) {
      --e;
      o1 = o0;
      o0 = v3::sload(off + e);
      pref -= (o1 - o0 + TILE - 1) / TILE;
    }
    while (mt >= pref + (o1 - o0 + TILE - 1) / TILE) {
      pref += (o1 - o0 + TILE - 1) / TILE;
      ++e;
      o0 = o1;
      o1 = v3::sload(off + e + 1);
    }
    ex = e;
    m0 = o0 + (mt - pref) * TILE;
    m_end = o1;
  }
};

// Logical tile -> (token tile mt, weight tile rt) of a token GEMM. Up to 8 weight tiles: row-major
// (rt fastest), so the 32 workgroups an XCD runs at once (32 consecutive logical tiles) cover 4+
// token tiles x every weight tile. More weight tiles: groups of TGM token tiles with the token tile
// fastest inside a group, so those 32 workgroups cover 8 token tiles x 4 weight tiles (12 operand
// blocks for the XCD's L2) instead of 2-3 x 12-16 (15-18 blocks); measured +2% on the fp8 forward
// (12 and 16 weight tiles), -1% when applied to 8 weight tiles.
constexpr int TGM = 8;
__host__ __device__ inline int tile_group(int n_rt) { return n_rt > 8 ? TGM : 1; }
__device__ __forceinline__ void tile_of(int lid, int n_rt, int& mt, int& rt) {
  const int gm = tile_group(n_rt);
  const int per = gm * n_rt;
  const int g = lid / per, w = lid - g * per;
  mt = g * gm + w % gm;
  rt = w / gm;
}
// Block -> (mt, rt) of a token GEMM from the actual token-tile count n_mt (the launch is sized
// for an upper bound, logical_tiles below): workgroup b runs on XCD b % 8, which takes the
// contiguous logical range [x * R, x * R + R) in order, so every XCD gets an equal share of the
// real tiles. (An XCD grouping over the launch size left the upper bound's unused tiles all on
// the last XCD; measured 4-7% slower on the bf16 token GEMMs.) False: nothing to do.
__device__ __forceinline__ bool block_tile(int n_mt, int n_rt, int& mt, int& rt) {
  const int gm = tile_group(n_rt);
  const int n_idx = (n_mt + gm - 1) / gm * gm * n_rt;
  const int x = (int)blockIdx.x & 7, bi = (int)blockIdx.x >> 3;
  const int R = (n_idx + 7) >> 3;
  const int lid = x * R + bi;
  if (bi >= R || lid >= n_idx) return false;
  tile_of(lid, n_rt, mt, rt);
  return mt < n_mt;
}
// Logical tiles to launch for up to max_mt token tiles: whole groups, so every valid (mt, rt)
// has a logical index below the count (and 8 * ceil(count / 8) blocks cover every XCD's range).
inline int64_t logical_tiles(int64_t max_mt, int n_rt) {
  const int gm = tile_group(n_rt);
  return (max_mt + gm - 1) / gm * gm * n_rt;
}

}  // namespace v4
}  // namespace moe
