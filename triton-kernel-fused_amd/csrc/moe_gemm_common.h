// Pieces shared by the grouped GEMM kernels (bf16 / fp16 / fp32 in moe_gemm.hip, fp8 in
// moe_fp8.hip): tile-shape constants, the token-GEMM argument block, the per-workgroup expert tile
// scan, four-element row stores and the fused GLU activations.
#pragma once
#include "moe_common.h"

namespace moe {

constexpr int MAX_GLU_EXPERTS = 1024;
constexpr int BK_BYTES = 128;            // bytes of K per LDS row (first-generation kernels)
constexpr int LDS_ROW = BK_BYTES + 16;   // padded LDS row

// EPI_GLU_BWD_GATED: as EPI_GLU_BWD, with the token operand = grad_out rows (ungated) and the gate
// weight applied in the epilogue, which also writes gate * inter and the gate-gradient partials.
enum EpiMode { EPI_STORE = 0, EPI_GLU_FWD = 1, EPI_GLU_BWD = 2, EPI_GLU_BWD_GATED = 3 };

template <typename T_, int BR_, int BC_, int WR_, int WC_>
struct Cfg {
  typedef T_ T;
  static constexpr int BR = BR_, BC = BC_, WR = WR_, WC = WC_;
  static constexpr int NT = WR * WC * 64;
  static constexpr int VEC = 16 / (int)sizeof(T);
  static constexpr int BK = BK_BYTES / (int)sizeof(T);
  static constexpr int WTR = BR / WR;
  static constexpr int WTC = BC / WC;
  static constexpr int TI = WTR / 32;
  static constexpr int TJ = WTC / 32;
  static constexpr int SLABS = BK_BYTES / 32;
  static constexpr int LDS_P = BR * LDS_ROW;
  static constexpr int LDS_Q = BC * LDS_ROW;
  static constexpr int STAGE = LDS_P + LDS_Q;
  static constexpr int LDS_BYTES = 2 * STAGE;
  static_assert(WTR % 32 == 0 && WTC % 32 == 0, "wave tile must be whole 32x32 MFMA tiles");
};

// ---------------------------------------------------------------------------------------------
// Output helpers: four consecutive elements of one row.
template <typename T> struct Store4;
template <> struct Store4<bf16> {
  __device__ __forceinline__ static void st(bf16* p, float a, float b, float c, float d) {
    bf16x2 lo = {(bf16)a, (bf16)b}, hi = {(bf16)c, (bf16)d};
    uint2 v = {__builtin_bit_cast(unsigned, lo), __builtin_bit_cast(unsigned, hi)};
    *(uint2*)p = v;
  }
  __device__ __forceinline__ static void ld(const bf16* p, float (&v)[4]) {
    uint2 u = *(const uint2*)p;
    bf16x2 lo = __builtin_bit_cast(bf16x2, u.x), hi = __builtin_bit_cast(bf16x2, u.y);
    v[0] = (float)lo[0]; v[1] = (float)lo[1]; v[2] = (float)hi[0]; v[3] = (float)hi[1];
  }
};
template <> struct Store4<f16> {
  __device__ __forceinline__ static void st(f16* p, float a, float b, float c, float d) {
    typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 h4;
    h4 v = {(f16)a, (f16)b, (f16)c, (f16)d};
    *(h4*)p = v;
  }
  __device__ __forceinline__ static void ld(const f16* p, float (&v)[4]) {
    typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 h4;
    h4 u = *(const h4*)p;
    v[0] = (float)u[0]; v[1] = (float)u[1]; v[2] = (float)u[2]; v[3] = (float)u[3];
  }
};
template <> struct Store4<float> {
  __device__ __forceinline__ static void st(float* p, float a, float b, float c, float d) {
    *(f32x4*)p = f32x4{a, b, c, d};
  }
  __device__ __forceinline__ static void ld(const float* p, float (&v)[4]) {
    f32x4 u = *(const f32x4*)p;
    v[0] = u[0]; v[1] = u[1]; v[2] = u[2]; v[3] = u[3];
  }
};

// GLU activation and its derivative for the codes the GEMM epilogues fuse (0 = SiLU, 1 = ReLU^2),
// kernels/sm75/moe.py:176-183 (forward) and :206-225 (backward).
__device__ __forceinline__ float glu_act(int code, float g) {
  if (code == 1) { float r = fmaxf(g, 0.f); return r * r; }
  return silu(g);
}
__device__ __forceinline__ float glu_dact(int code, float g) {
  if (code == 1) return 2.f * fmaxf(g, 0.f);
  const float s = sigmoid(g);
  return s * (1.f + g * (1.f - s));
}
// act(g) and act'(g) together (one sigmoid for SiLU).
__device__ __forceinline__ void glu_act_dact(int code, float g, float& act, float& dact) {
  if (code == 1) {
    const float r = fmaxf(g, 0.f);
    act = r * r;
    dact = 2.f * r;
  } else {
    const float s = sigmoid(g);
    act = g * s;
    dact = s * (1.f + g * (1.f - s));
  }
}

// ---------------------------------------------------------------------------------------------
// Token-grouped GEMM: for each expert e < E_glu and each tile of its sorted rows,
//   acc[r, m] = sum_k P_e[r, k] * Q[qrow(m), k].
struct TokenArgs {
  const void* P;      // expert weights base
  long long p_e;      // elements between experts
  long long p_ld;     // elements between rows (P_KC) or between K rows (P_RC)
  int R;              // P rows per expert (output row dim); EPI_GLU_FWD: 2*I
  int K;
  const void* Q;      // token-side operand rows (K-contiguous)
  long long q_ld;     // elements between rows
  const int32_t* q_gather;  // sorted row -> Q row (sorted_token), or null for identity
  const int32_t* offsets;   // E_glu + 1 sorted-row offsets
  int E_glu;
  int n_rtiles;
  const int32_t* act_codes;
  int I;              // intermediate size (GLU epilogues)
  void* out;          // EPI_STORE: (M, R); EPI_GLU_FWD: gate_up (M, 2I); EPI_GLU_BWD: ggu (M, 2I)
  long long out_ld;
  void* out2;         // EPI_GLU_FWD: inter (M, I); EPI_GLU_BWD: grad_inter (M, I);
                      // EPI_GLU_BWD_GATED: gate * inter (M, I), may be null
  const void* aux;    // EPI_GLU_BWD(_GATED): gate_up (M, 2I)
  // EPI_GLU_BWD_GATED only:
  const void* gate;        // top_k_weights (N*k), indexed by sorted_flat
  const int32_t* sflat;    // sorted row -> flat slot t*k+j
  float* part;             // gate-gradient partials (2 * n_rtiles, M): sum over a wave's 128
                           // channels of (grad_out @ down_proj) * inter
  // K-split of each XCD's last partial wave (v4 kernel, EPI_STORE; null split_ws = off): fp32
  // partial tiles, one per workgroup slot (xcd_cus per XCD), then per-tile arrival counters (zero
  // on entry, left zero).
  float* split_ws;
  int* split_cnt;
  int xcd_cus;
};

// Block-wide exclusive scan of the per-expert tile counts into s_pref[0..E]; returns the total.
template <int NT>
__device__ __forceinline__ void tile_prefix(const int32_t* offsets, int E, int BC, int* s_pref,
                                            int* s_wsum) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int per = (E + NT - 1) / NT;
  const int e0 = tid * per;
  int local = 0;
  for (int j = 0; j < per; ++j) {
    const int e = e0 + j;
    if (e < E) local += (offsets[e + 1] - offsets[e] + BC - 1) / BC;
  }
  int incl = local;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int v = __shfl_up(incl, d, 64);
    if (lane >= d) incl += v;
  }
  if (lane == 63) s_wsum[wid] = incl;
  __syncthreads();
  int run = incl - local;
  for (int w = 0; w < wid; ++w) run += s_wsum[w];
  for (int j = 0; j < per; ++j) {
    const int e = e0 + j;
    if (e < E) {
      s_pref[e] = run;
      run += (offsets[e + 1] - offsets[e] + BC - 1) / BC;
    }
  }
  if (tid == NT - 1) s_pref[E] = run;
  __syncthreads();
}

// Physical weight row of tile row rr for the gate/up forward GEMM: in each wave's WTR rows the
// first half are gate channels and the second half the same up channels.
template <class C>
__device__ __forceinline__ int glu_prow(int rr, int rt, int I, bool& ok) {
  const int wr = rr / C::WTR, w = rr % C::WTR;
  const int ch = rt * (C::BR / 2) + wr * (C::WTR / 2) + (w % (C::WTR / 2));
  ok = ch < I;
  return (w >= C::WTR / 2 ? I : 0) + ch;
}

}  // namespace moe
