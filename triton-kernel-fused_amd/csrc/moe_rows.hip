// Memory-bound row kernels of the MoE pipeline: the gate-weighted combine, its backward, the
// un-permute of the input gradient, and the row-wise PolyGLU activation (BatchedGLU) forward and
// backward for every activation code.
//
// Combine and un-permute are gathers, not scatters: one wave owns one token's 64*V-column chunk
// and sums its k routed rows in slot order in fp32, so results are deterministic and need no
// atomics (the reference scatters with fp32 atomics or index_add_,
// /root/reference/kernels/sm75/moe.py:673-682,593-595).
#include "moe_common.h"

namespace moe {

constexpr int ROW_THREADS = 256;  // 4 waves, one token / routed row per wave

template <typename T> struct Vec8;  // 16 bytes of T as floats
template <> struct Vec8<bf16> {
  static constexpr int N = 8;
  // bf16 -> fp32 is exact: the bf16 bits are the top half of the fp32 bits.
  __device__ __forceinline__ static void ld(const bf16* p, float* v) { cvt(*(const uint4*)p, v); }
  __device__ __forceinline__ static void cvt(const uint4& u, float* v) {
    const unsigned w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static void st(bf16* p, const float* v) {
    unsigned w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bf16x2 t = {(bf16)v[2 * i], (bf16)v[2 * i + 1]};
      w[i] = __builtin_bit_cast(unsigned, t);
    }
    *(uint4*)p = uint4{w[0], w[1], w[2], w[3]};
  }
};
template <> struct Vec8<f16> {
  static constexpr int N = 8;
  typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 h2;
  __device__ __forceinline__ static void ld(const f16* p, float* v) { cvt(*(const uint4*)p, v); }
  __device__ __forceinline__ static void cvt(const uint4& u, float* v) {
    const unsigned w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h2 t = __builtin_bit_cast(h2, w[i]);
      v[2 * i] = (float)t[0]; v[2 * i + 1] = (float)t[1];
    }
  }
  __device__ __forceinline__ static void st(f16* p, const float* v) {
    unsigned w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h2 t = {(f16)v[2 * i], (f16)v[2 * i + 1]};
      w[i] = __builtin_bit_cast(unsigned, t);
    }
    *(uint4*)p = uint4{w[0], w[1], w[2], w[3]};
  }
};
template <> struct Vec8<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void ld(const float* p, float* v) {
    f32x4 u = *(const f32x4*)p;
    v[0] = u[0]; v[1] = u[1]; v[2] = u[2]; v[3] = u[3];
  }
  __device__ __forceinline__ static void cvt(const uint4& u, float* v) {
    v[0] = __uint_as_float(u.x); v[1] = __uint_as_float(u.y);
    v[2] = __uint_as_float(u.z); v[3] = __uint_as_float(u.w);
  }
  __device__ __forceinline__ static void st(float* p, const float* v) {
    *(f32x4*)p = f32x4{v[0], v[1], v[2], v[3]};
  }
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

// Kind of routed slot: 0 = GLU expert row, 1 = Identity (code 3), 2 = Zero (code 4) or invalid.
__device__ __forceinline__ int slot_kind(int64_t e, const int32_t* codes, int E_glu, int E_all,
                                         int pos) {
  if (e < 0 || e >= E_all || pos < 0) return 2;
  if (e < E_glu) return 0;
  const int c = codes[e];
  return c == 3 ? 1 : 2;
}

// Per-token gathers (combine forward, un-permute backward). One wave owns CPW 64*V-column chunks
// of one token; the k routed rows are loaded BATCH at a time, all BATCH x CPW loads in flight
// together (the token's routing reads are wave-uniform), and summed in slot order in fp32:
//   acc = sum_j g_j * row_j,  row_j = rows[f2s[t,j]] for a GLU expert (g_j = gate if GATE_GLU,
//   else 1) or self[t] for an Identity expert (g_j = gate); Zero experts and invalid ids add
//   nothing.
// CPW (column chunks per wave): two put 16 loads in flight behind one round of routing reads
// (measured ~4% faster than one at H = 2048; four is level); one when a row is a single chunk
// (H <= 512 for 16-bit types). BATCH: k rounded up to 2, 4 or 8, so a small top-k does not load
// (and discard) rows for slots that do not exist.
template <typename T, bool GATE_GLU, int BATCH, int CPW>
__device__ __forceinline__ void token_gather(const T* __restrict__ rows, const T* __restrict__ self,
                                             int64_t self_ld, const T* __restrict__ wt,
                                             const int64_t* __restrict__ idx,
                                             const int32_t* __restrict__ codes, int E_glu,
                                             int E_all, const int32_t* __restrict__ f2s,
                                             int64_t N, int k, int H, T* __restrict__ out) {
  constexpr int V = Vec8<T>::N;
  const int nchunk = (H + 64 * V - 1) / (64 * V);
  const int ncw = (nchunk + CPW - 1) / CPW;
  const int64_t wv = (int64_t)blockIdx.x * (ROW_THREADS / 64) + (threadIdx.x >> 6);
  if (wv >= N * ncw) return;
  const int64_t t = wv / ncw;
  const int lane = threadIdx.x & 63;
  int c[CPW];
  bool col_ok[CPW];
  float acc[CPW][V];
#pragma unroll
  for (int u = 0; u < CPW; ++u) {
    c[u] = ((int)(wv % ncw) * CPW + u) * 64 * V + lane * V;
    col_ok[u] = c[u] < H;
#pragma unroll
    for (int i = 0; i < V; ++i) acc[u][i] = 0.f;
  }
  for (int j0 = 0; j0 < k; j0 += BATCH) {
    // Branch-free: every slot's 16 bytes are loaded (a skipped slot reads the token's own row)
    // before any is used, so the BATCH x CPW loads are in flight together.
    const T* src[BATCH];
    float w[BATCH];
    bool used[BATCH];
#pragma unroll
    for (int jj = 0; jj < BATCH; ++jj) {
      const int j = j0 + jj;
      const int64_t f = t * k + (j < k ? j : 0);
      const int pos = f2s[f];
      const int kind = j < k ? slot_kind(idx[f], codes, E_glu, E_all, pos) : 2;
      used[jj] = kind != 2;
      w[jj] = (kind == 0 && !GATE_GLU) ? 1.f : to_f32(wt[f]);
      src[jj] = kind == 0 ? rows + (size_t)pos * H : self + (size_t)t * self_ld;
    }
    i32x4 raw[CPW][BATCH];
#pragma unroll
    for (int u = 0; u < CPW; ++u) {
      const int cc = col_ok[u] ? c[u] : 0;
#pragma unroll
      for (int jj = 0; jj < BATCH; ++jj) raw[u][jj] = *(const i32x4*)(src[jj] + cc);
    }
#pragma unroll
    for (int u = 0; u < CPW; ++u)
#pragma unroll
      for (int jj = 0; jj < BATCH; ++jj) {
        float v[V];
        Vec8<T>::ld((const T*)&raw[u][jj], v);
        // A skipped slot contributes nothing (not even 0 * inf).
#pragma unroll
        for (int i = 0; i < V; ++i) acc[u][i] += used[jj] ? w[jj] * v[i] : 0.f;
      }
  }
#pragma unroll
  for (int u = 0; u < CPW; ++u)
    if (col_ok[u]) Vec8<T>::st(out + (size_t)t * H + c[u], acc[u]);
}

// out[t] = sum_j w[t,j] * row(t,j); GATE_GLU false: GLU rows already carry their gate.
template <typename T, bool GATE_GLU, int BATCH, int CPW>
__global__ void __launch_bounds__(ROW_THREADS)
combine_fwd_kernel(const T* __restrict__ eo, const T* __restrict__ hidden,
                   const T* __restrict__ wt, const int64_t* __restrict__ idx,
                   const int32_t* __restrict__ codes, int E_glu, int E_all,
                   const int32_t* __restrict__ f2s, int64_t N, int k, int H, T* __restrict__ out) {
  token_gather<T, GATE_GLU, BATCH, CPW>(eo, hidden, H, wt, idx, codes, E_glu, E_all, f2s, N, k, H,
                                        out);
}

// Per sorted row r (token t, flat f): grad_eo[r] = go[t]*w; grad_wt[f] = sum_h go[t,h]*row[h].
// Rows past the routed count carry t = f = -1 (dispatch) and are skipped.
template <typename T>
__global__ void __launch_bounds__(ROW_THREADS)
combine_bwd_kernel(const T* __restrict__ go, int64_t go_ld, const T* __restrict__ eo,
                   const T* __restrict__ hidden, const T* __restrict__ wt,
                   const int64_t* __restrict__ idx, const int32_t* __restrict__ codes, int E_glu,
                   int E_all, const int32_t* __restrict__ st, const int32_t* __restrict__ sflat,
                   int64_t M, int H, T* __restrict__ grad_eo, T* __restrict__ grad_wt) {
  constexpr int V = Vec8<T>::N;
  const int64_t r = (int64_t)blockIdx.x * (ROW_THREADS / 64) + (threadIdx.x >> 6);
  if (r >= M) return;
  const int lane = threadIdx.x & 63;
  const int t = st[r];
  const int f = sflat[r];
  if (f < 0 || t < 0) return;  // past the routed count (dropped ids): no slot
  const int kind = slot_kind(idx[f], codes, E_glu, E_all, 0);
  const float w = to_f32(wt[f]);
  float dot = 0.f;
  for (int c = lane * V; c < H; c += 64 * V) {
    float g[V], v[V];
    Vec8<T>::ld(go + (size_t)t * go_ld + c, g);
    if (kind == 0) {
      Vec8<T>::ld(eo + (size_t)r * H + c, v);
      float ge[V];
#pragma unroll
      for (int i = 0; i < V; ++i) ge[i] = g[i] * w;
      Vec8<T>::st(grad_eo + (size_t)r * H + c, ge);
    } else if (kind == 1) {
      Vec8<T>::ld(hidden + (size_t)t * H + c, v);
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) v[i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < V; ++i) dot += g[i] * v[i];
  }
  dot = wave_sum(dot);
  if (lane == 0) grad_wt[f] = from_f32<T>(dot);
}

// Gate gradients from the fused down-dX GEMM: one wave per token; for each routed slot f = t*k+j,
// GLU expert: grad_wt[f] = sum of the n_parts partial dots of its sorted row (fixed order, so the
// result is deterministic); Identity: <grad_out[t], hidden[t]>; Zero or invalid: 0
// (kernels/sm75/moe.py:712-720).
template <typename T, bool LANES>
__global__ void __launch_bounds__(ROW_THREADS)
gate_grad_kernel(const float* __restrict__ part, int n_parts, int64_t n_rows,
                 const T* __restrict__ go, int64_t go_ld, const T* __restrict__ hidden,
                 const int64_t* __restrict__ idx, const int32_t* __restrict__ codes, int E_glu,
                 int E_all, const int32_t* __restrict__ f2s, int64_t N, int k, int H,
                 T* __restrict__ grad_wt) {
  constexpr int V = Vec8<T>::N;
  const int64_t t = (int64_t)blockIdx.x * (ROW_THREADS / 64) + (threadIdx.x >> 6);
  if (t >= N) return;
  const int lane = threadIdx.x & 63;
  if (LANES) {
    // k * n_parts <= 64, n_parts a power of two: lane = j * n_parts + p loads partial p of slot
    // j, all in flight together, and each slot's n_parts lanes sum them (butterfly within the
    // segment, a fixed order). Identity slots are handled by the loop below.
    float v = 0.f;
    int kind = 2;
    const int j = lane / n_parts, p = lane & (n_parts - 1);
    const int64_t f = t * k + (j < k ? j : 0);
    if (j < k) {
      const int pos = f2s[f];
      kind = slot_kind(idx[f], codes, E_glu, E_all, pos);
      if (kind == 0) v = part[(size_t)p * n_rows + pos];
    }
    for (int d = 1; d < n_parts; d <<= 1) v += __shfl_xor(v, d, 64);
    if (j < k && p == 0 && kind != 1) grad_wt[f] = from_f32<T>(v);
  }
  for (int j = 0; j < k; ++j) {
    const int64_t f = t * k + j;
    const int pos = f2s[f];
    const int kind = slot_kind(idx[f], codes, E_glu, E_all, pos);
    if (LANES && kind != 1) continue;
    float v = 0.f;
    if (kind == 0) {
      for (int p = lane; p < n_parts; p += 64) v += part[(size_t)p * n_rows + pos];
    } else if (kind == 1) {
      for (int c = lane * V; c < H; c += 64 * V) {
        float g[V], x[V];
        Vec8<T>::ld(go + (size_t)t * go_ld + c, g);
        Vec8<T>::ld(hidden + (size_t)t * H + c, x);
#pragma unroll
        for (int i = 0; i < V; ++i) v += g[i] * x[i];
      }
    }
    v = wave_sum(v);
    if (lane == 0) grad_wt[f] = from_f32<T>(v);
  }
}

// grad_x[t] = sum_j (GLU: grad_xs[pos]; Identity: w*go[t]; Zero: 0)
template <typename T, int BATCH, int CPW>
__global__ void __launch_bounds__(ROW_THREADS)
unpermute_bwd_kernel(const T* __restrict__ gxs, const T* __restrict__ go, int64_t go_ld,
                     const T* __restrict__ wt, const int64_t* __restrict__ idx,
                     const int32_t* __restrict__ codes, int E_glu, int E_all,
                     const int32_t* __restrict__ f2s, int64_t N, int k, int H,
                     T* __restrict__ gx) {
  // GLU expert rows of grad_xs already carry the gate weight; Identity slots add w * grad_out.
  token_gather<T, false, BATCH, CPW>(gxs, go, go_ld, wt, idx, codes, E_glu, E_all, f2s, N, k, H,
                                     gx);
}

// ---------------------------------------------------------------------------------------------
// Row-wise PolyGLU (kernels/sm75/moe.py:163-232): one workgroup per row, the full intermediate
// row in one pass, so the RMS of codes 2/6/7, the RMS-coupling sum S of their backward and the
// SiTU parameter sums are block reductions in the same kernel.
constexpr float NS_EPS = 1e-6f;
constexpr int GLU_THREADS = 256;

__device__ __forceinline__ float tanh_via_sigmoid(float x) { return 2.f / (1.f + __expf(-2.f * x)) - 1.f; }

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < GLU_THREADS / 64; ++w) s += red[w];
  return s;
}

__device__ __forceinline__ bool is_norm_code(int c) { return c == 2 || c == 6 || c == 7; }

template <typename T>
__global__ void __launch_bounds__(GLU_THREADS)
glu_fwd_kernel(const T* __restrict__ gu, int64_t gu_ld, const int32_t* __restrict__ row_act,
               const float* __restrict__ alpha, const float* __restrict__ gamma, int ap_stride,
               int I, T* __restrict__ out, int64_t out_ld) {
  __shared__ float red[GLU_THREADS / 64];
  const int64_t row = blockIdx.x;
  const T* g = gu + row * gu_ld;
  const T* u = g + I;
  const int code = row_act[row];
  const float aa = alpha ? alpha[row * ap_stride] : 1.f;
  const float gg = gamma ? gamma[row * ap_stride] : 1.f;
  float r = 1.f;
  if (is_norm_code(code)) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < I; i += GLU_THREADS) { float x = to_f32(g[i]); ss += x * x; }
    ss = block_sum(ss, red);
    r = sqrtf(ss / I + NS_EPS);
  }
  for (int i = threadIdx.x; i < I; i += GLU_THREADS) {
    const float gate = to_f32(g[i]);
    const float up = to_f32(u[i]);
    const float gn = is_norm_code(code) ? gate / r : gate;
    const float sig = sigmoid(gn);
    float act;
    if (code == 1 || code == 6) { float rl = fmaxf(gn, 0.f); act = rl * rl; }
    else if (code == 5) act = gg * tanh_via_sigmoid(aa * gate) * sig;
    else if (code == 7) act = tanh_via_sigmoid(gn) * sig;
    else act = gn * sig;  // codes 0, 2
    out[row * out_ld + i] = from_f32<T>(act * up);
  }
}

template <typename T>
__global__ void __launch_bounds__(GLU_THREADS)
glu_bwd_kernel(const T* __restrict__ go_, int64_t go_rs, int64_t go_cs, const T* __restrict__ gu,
               int64_t gu_ld, const int32_t* __restrict__ row_act,
               const float* __restrict__ alpha, const float* __restrict__ gamma, int ap_stride,
               int I, T* __restrict__ ggu, int64_t ggu_ld, float* __restrict__ da,
               float* __restrict__ dg) {
  __shared__ float red[GLU_THREADS / 64];
  const int64_t row = blockIdx.x;
  const T* g = gu + row * gu_ld;
  const T* u = g + I;
  const T* gop = go_ + row * go_rs;
  const int code = row_act[row];
  const bool norm = is_norm_code(code);
  const float aa = alpha ? alpha[row * ap_stride] : 1.f;
  const float gg = gamma ? gamma[row * ap_stride] : 1.f;
  float r = 1.f, S = 0.f;
  if (norm) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < I; i += GLU_THREADS) { float x = to_f32(g[i]); ss += x * x; }
    ss = block_sum(ss, red);
    r = sqrtf(ss / I + NS_EPS);
    float s = 0.f;
    for (int i = threadIdx.x; i < I; i += GLU_THREADS) {
      const float gn = to_f32(g[i]) / r;
      const float sig = sigmoid(gn);
      float df;
      if (code == 6) df = 2.f * fmaxf(gn, 0.f);
      else if (code == 7) { float tg = tanh_via_sigmoid(gn); df = (1.f - tg * tg) * sig + tg * sig * (1.f - sig); }
      else df = sig * (1.f + gn * (1.f - sig));
      s += to_f32(gop[i * go_cs]) * to_f32(u[i]) * df * gn;
    }
    S = block_sum(s, red);
  }
  float sda = 0.f, sdg = 0.f;
  for (int i = threadIdx.x; i < I; i += GLU_THREADS) {
    const float gate = to_f32(g[i]);
    const float up = to_f32(u[i]);
    const float go = to_f32(gop[i * go_cs]);
    const float gn = norm ? gate / r : gate;
    const float sig = sigmoid(gn);
    const float gup = go * up;
    float act, grad_gate;
    if (code == 1) {
      float rl = fmaxf(gn, 0.f); act = rl * rl; grad_gate = gup * 2.f * rl;
    } else if (code == 5) {
      const float t5 = tanh_via_sigmoid(aa * gate);
      act = gg * t5 * sig;
      grad_gate = gup * gg * (aa * (1.f - t5 * t5) * sig + t5 * sig * (1.f - sig));
      sda += gup * gg * gate * (1.f - t5 * t5) * sig;
      sdg += gup * t5 * sig;
    } else if (norm) {
      float df;
      if (code == 6) { float rl = fmaxf(gn, 0.f); act = rl * rl; df = 2.f * rl; }
      else if (code == 7) { float tg = tanh_via_sigmoid(gn); act = tg * sig; df = (1.f - tg * tg) * sig + tg * sig * (1.f - sig); }
      else { act = gn * sig; df = sig * (1.f + gn * (1.f - sig)); }
      grad_gate = (gup * df - (S / I) * gn) / r;
    } else {  // code 0
      act = gn * sig;
      grad_gate = gup * sig * (1.f + gn * (1.f - sig));
    }
    ggu[row * ggu_ld + i] = from_f32<T>(grad_gate);
    ggu[row * ggu_ld + I + i] = from_f32<T>(go * act);
  }
  if (da) {
    sda = block_sum(sda, red);
    sdg = block_sum(sdg, red);
    if (threadIdx.x == 0) {
      da[row] = code == 5 ? sda : 0.f;
      dg[row] = code == 5 ? sdg : 0.f;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Row-wise PolyGLU, vector form: one wave per row and 16-byte loads and stores (V elements per
// lane and chunk), for rows whose element offsets are multiples of V and 16-byte aligned. A lane
// keeps chunks lane, lane + 64, ... (up to NJ of them, NJ * 64 * V >= I) in registers, so the RMS
// pass of codes 2/6/7 and the main pass read each element once, and every reduction is a wave
// reduction (no block barrier; a wave past the last row leaves at once). The per-element math is
// the scalar kernels' above.
constexpr int GLU_VEC_WAVES = 4;

// act(gate) and act'(gn) of the codes (the derivative with respect to the normalised gate gn for
// 2/6/7, to gate otherwise; code 5's pieces are computed by the callers).
__device__ __forceinline__ void glu_row_act_dact(int code, float gn, float sig, float& act,
                                                 float& df) {
  if (code == 1 || code == 6) {
    const float rl = fmaxf(gn, 0.f);
    act = rl * rl;
    df = 2.f * rl;
  } else if (code == 7) {
    const float tg = tanh_via_sigmoid(gn);
    act = tg * sig;
    df = (1.f - tg * tg) * sig + tg * sig * (1.f - sig);
  } else {  // 0, 2 (and any other code, as the scalar kernels)
    act = gn * sig;
    df = sig * (1.f + gn * (1.f - sig));
  }
}

template <typename T, int NJ>
__global__ void __launch_bounds__(64 * GLU_VEC_WAVES)
glu_fwd_vec_kernel(const T* __restrict__ gu, int64_t gu_ld, const int32_t* __restrict__ row_act,
                   const float* __restrict__ alpha, const float* __restrict__ gamma,
                   int ap_stride, int64_t n_rows, int I, T* __restrict__ out, int64_t out_ld) {
  constexpr int V = Vec8<T>::N;
  const int64_t row = (int64_t)blockIdx.x * GLU_VEC_WAVES + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int lane = threadIdx.x & 63;
  const int nch = I / V;
  const T* g = gu + row * gu_ld;
  const T* u = g + I;
  const int code = row_act[row];
  const float aa = alpha ? alpha[row * ap_stride] : 1.f;
  const float gg = gamma ? gamma[row * ap_stride] : 1.f;
  // The row's chunks stay packed in registers (16 bytes each) and are unpacked where used.
  uint4 graw[NJ], uraw[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = lane + 64 * j;
    graw[j] = uraw[j] = uint4{0u, 0u, 0u, 0u};
    if (c < nch) {
      graw[j] = *(const uint4*)(g + c * V);
      uraw[j] = *(const uint4*)(u + c * V);
    }
  }
  float rinv = 1.f;
  if (is_norm_code(code)) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      float gv[V];
      Vec8<T>::cvt(graw[j], gv);
#pragma unroll
      for (int i = 0; i < V; ++i) ss += gv[i] * gv[i];
    }
    ss = wave_sum(ss);
    rinv = 1.f / sqrtf(ss / I + NS_EPS);
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = lane + 64 * j;
    if (c >= nch) continue;
    float o[V], gv[V], uv[V];
    Vec8<T>::cvt(graw[j], gv);
    Vec8<T>::cvt(uraw[j], uv);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float gate = gv[i];
      const float gn = is_norm_code(code) ? gate * rinv : gate;
      const float sig = sigmoid(gn);
      float act, df;
      if (code == 5) act = gg * tanh_via_sigmoid(aa * gate) * sig;
      else glu_row_act_dact(code, gn, sig, act, df);
      o[i] = act * uv[i];
    }
    Vec8<T>::st(out + row * out_ld + c * V, o);
  }
}

template <typename T, int NJ>
__global__ void __launch_bounds__(64 * GLU_VEC_WAVES)
glu_bwd_vec_kernel(const T* __restrict__ go_, int64_t go_rs, const T* __restrict__ gu,
                   int64_t gu_ld, const int32_t* __restrict__ row_act,
                   const float* __restrict__ alpha, const float* __restrict__ gamma,
                   int ap_stride, int64_t n_rows, int I, T* __restrict__ ggu, int64_t ggu_ld,
                   float* __restrict__ da, float* __restrict__ dg) {
  constexpr int V = Vec8<T>::N;
  const int64_t row = (int64_t)blockIdx.x * GLU_VEC_WAVES + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int lane = threadIdx.x & 63;
  const int nch = I / V;
  const T* g = gu + row * gu_ld;
  const T* u = g + I;
  const T* gop = go_ + row * go_rs;
  const int code = row_act[row];
  const bool norm = is_norm_code(code);
  const float aa = alpha ? alpha[row * ap_stride] : 1.f;
  const float gg = gamma ? gamma[row * ap_stride] : 1.f;
  uint4 graw[NJ], uraw[NJ], oraw[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = lane + 64 * j;
    graw[j] = uraw[j] = oraw[j] = uint4{0u, 0u, 0u, 0u};
    if (c < nch) {
      graw[j] = *(const uint4*)(g + c * V);
      uraw[j] = *(const uint4*)(u + c * V);
      oraw[j] = *(const uint4*)(gop + c * V);
    }
  }
  float r = 1.f, rinv = 1.f, S = 0.f;
  if (norm) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      float gv[V];
      Vec8<T>::cvt(graw[j], gv);
#pragma unroll
      for (int i = 0; i < V; ++i) ss += gv[i] * gv[i];
    }
    ss = wave_sum(ss);
    r = sqrtf(ss / I + NS_EPS);
    rinv = 1.f / r;
    float sacc = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      float gv[V], uv[V], ov[V];
      Vec8<T>::cvt(graw[j], gv);
      Vec8<T>::cvt(uraw[j], uv);
      Vec8<T>::cvt(oraw[j], ov);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float gn = gv[i] * rinv;
        float act, df;
        glu_row_act_dact(code, gn, sigmoid(gn), act, df);
        sacc += ov[i] * uv[i] * df * gn;  // zero-filled chunks add nothing
      }
    }
    S = wave_sum(sacc);
  }
  float sda = 0.f, sdg = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = lane + 64 * j;
    if (c >= nch) continue;
    float dgt[V], dup[V], gv[V], uv[V], ov[V];
    Vec8<T>::cvt(graw[j], gv);
    Vec8<T>::cvt(uraw[j], uv);
    Vec8<T>::cvt(oraw[j], ov);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float gate = gv[i];
      const float gn = norm ? gate * rinv : gate;
      const float sig = sigmoid(gn);
      const float gup = ov[i] * uv[i];
      float act, df;
      if (code == 5) {
        const float t5 = tanh_via_sigmoid(aa * gate);
        act = gg * t5 * sig;
        dgt[i] = gup * gg * (aa * (1.f - t5 * t5) * sig + t5 * sig * (1.f - sig));
        sda += gup * gg * gate * (1.f - t5 * t5) * sig;
        sdg += gup * t5 * sig;
      } else {
        glu_row_act_dact(code, gn, sig, act, df);
        dgt[i] = norm ? (gup * df - (S / I) * gn) / r : gup * df;
      }
      dup[i] = ov[i] * act;
    }
    Vec8<T>::st(ggu + row * ggu_ld + c * V, dgt);
    Vec8<T>::st(ggu + row * ggu_ld + I + c * V, dup);
  }
  if (da) {
    sda = wave_sum(sda);
    sdg = wave_sum(sdg);
    if (lane == 0) {
      da[row] = code == 5 ? sda : 0.f;
      dg[row] = code == 5 ? sdg : 0.f;
    }
  }
}

}  // namespace moe

using namespace moe;

static int vec_of(int dtype) { return dtype == MOE_DT_F32 ? 4 : 8; }
static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Launch KERNEL<T_> with T_ bound to the element type of `dtype` (the argument list may use T_).
#define MOE_BY_DTYPE(dtype, KERNEL, GRID, BLOCK, STREAM, ...)      \
  do {                                                             \
    if ((dtype) == MOE_DT_BF16) {                                  \
      typedef bf16 T_;                                             \
      hipLaunchKernelGGL(KERNEL<T_>, GRID, BLOCK, 0, STREAM, __VA_ARGS__); \
    } else if ((dtype) == MOE_DT_F16) {                            \
      typedef f16 T_;                                              \
      hipLaunchKernelGGL(KERNEL<T_>, GRID, BLOCK, 0, STREAM, __VA_ARGS__); \
    } else {                                                       \
      typedef float T_;                                            \
      hipLaunchKernelGGL(KERNEL<T_>, GRID, BLOCK, 0, STREAM, __VA_ARGS__); \
    }                                                              \
  } while (0)
// The same for kernels with a second (integer) template parameter B.
#define MOE_BY_DTYPE_B(dtype, KERNEL, B, GRID, BLOCK, STREAM, ...)      \
  do {                                                             \
    if ((dtype) == MOE_DT_BF16) {                                  \
      typedef bf16 T_;                                             \
      hipLaunchKernelGGL((KERNEL<T_, B>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); \
    } else if ((dtype) == MOE_DT_F16) {                            \
      typedef f16 T_;                                              \
      hipLaunchKernelGGL((KERNEL<T_, B>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); \
    } else {                                                       \
      typedef float T_;                                            \
      hipLaunchKernelGGL((KERNEL<T_, B>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); \
    }                                                              \
  } while (0)

static int check_rows(int dtype, int64_t n, int top_k, int64_t H, int n_experts, int E_glu) {
  if (dtype < 0 || dtype > 2) return MOE_ERR_DTYPE;
  if (n < 0 || top_k <= 0 || H <= 0 || H >= (1 << 30) || n_experts <= 0 || E_glu < 0 ||
      E_glu > n_experts)
    return MOE_ERR_SHAPE;
  if (H % vec_of(dtype)) return MOE_ERR_ALIGN;
  return MOE_OK;
}

static unsigned row_grid(int64_t rows) { return (unsigned)((rows + 3) / 4); }

// Register chunks per lane of the vector GLU kernels (1, 2, 4 ... max_nj: I <= 64 * NJ * v), or 0
// when I is not a multiple of the vector width v or too long (the scalar kernels then run).
static int glu_vec_chunks(int64_t I, int v, int max_nj) {
  if (I % v) return 0;
  const int64_t nch = I / v;
  for (int nj = 1; nj <= max_nj; nj *= 2)
    if (nch <= 64 * nj) return nj;
  return 0;
}

// Per-token gathers (combine, un-permute): CPW column chunks of 64*vec per wave, BATCH routed rows
// loaded together. Each wave keeps its token's row loads in flight together; whole-token waves
// loading one row at a time measured ~20% slower even when the grid alone fills the GPU.
struct GatherCfg {
  int batch, cpw;
  int64_t col_waves;  // waves per token
};
static GatherCfg gather_cfg(int64_t H, int vec, int k) {
  GatherCfg g;
  const int64_t nchunk = (H + 64 * vec - 1) / (64 * vec);
  g.batch = k <= 2 ? 2 : k <= 4 ? 4 : 8;
  g.cpw = nchunk >= 2 ? 2 : 1;
  g.col_waves = (nchunk + g.cpw - 1) / g.cpw;
  return g;
}
// Calls f(integral_constant<BATCH>, integral_constant<CPW>) for the configuration g.
template <class F>
static void with_gather_cfg(const GatherCfg& g, F&& f) {
  using B2 = std::integral_constant<int, 2>;
  using B4 = std::integral_constant<int, 4>;
  using B8 = std::integral_constant<int, 8>;
  using C1 = std::integral_constant<int, 1>;
  using C2 = std::integral_constant<int, 2>;
  if (g.cpw == 1) {
    if (g.batch == 2) f(B2{}, C1{});
    else if (g.batch == 4) f(B4{}, C1{});
    else f(B8{}, C1{});
  } else {
    if (g.batch == 2) f(B2{}, C2{});
    else if (g.batch == 4) f(B4{}, C2{});
    else f(B8{}, C2{});
  }
}
// Calls f(T{}) with T the element type of dtype (bf16, f16 or float).
template <class F>
static void with_dtype(int dtype, F&& f) {
  if (dtype == MOE_DT_BF16) f(bf16{});
  else if (dtype == MOE_DT_F16) f(f16{});
  else f(float{});
}

extern "C" int moe_combine_fwd(int dtype, const void* eo, const void* hidden,
                               const void* top_k_weights, const int64_t* top_k_indices,
                               const int32_t* act_codes, int n_experts, int E_glu,
                               const int32_t* flat_to_sorted, int64_t n_tokens, int top_k,
                               int64_t H, int glu_rows_weighted, void* out, void* stream) {
  int st = check_rows(dtype, n_tokens, top_k, H, n_experts, E_glu);
  if (st) return st;
  if (n_tokens == 0) return MOE_OK;
  if (!hidden || !top_k_weights || !top_k_indices || !act_codes || !flat_to_sorted || !out ||
      (E_glu > 0 && !eo))
    return MOE_ERR_SHAPE;
  if (!al16(hidden) || !al16(out) || (eo && !al16(eo))) return MOE_ERR_ALIGN;
  const GatherCfg gc = gather_cfg(H, vec_of(dtype), top_k);
  if (n_tokens * gc.col_waves >= ((int64_t)1 << 32)) return MOE_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(row_grid(n_tokens * gc.col_waves));
  with_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    with_gather_cfg(gc, [&](auto b, auto c) {
      constexpr int B = decltype(b)::value, C = decltype(c)::value;
      auto kern = glu_rows_weighted ? combine_fwd_kernel<T, false, B, C> : combine_fwd_kernel<T, true, B, C>;
      hipLaunchKernelGGL(kern, grid, dim3(ROW_THREADS), 0, s, (const T*)eo, (const T*)hidden,
                         (const T*)top_k_weights, top_k_indices, act_codes, E_glu, n_experts,
                         flat_to_sorted, n_tokens, top_k, (int)H, (T*)out);
    });
  });
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}

extern "C" int moe_combine_bwd(int dtype, const void* grad_out, int64_t grad_out_ld,
                               const void* eo, const void* hidden, const void* top_k_weights,
                               const int64_t* top_k_indices, const int32_t* act_codes,
                               int n_experts, int E_glu, const int32_t* sorted_token,
                               const int32_t* sorted_flat, int64_t n_rows, int top_k, int64_t H,
                               void* grad_eo_out, void* grad_wt_out, void* stream) {
  int st = check_rows(dtype, n_rows, top_k, H, n_experts, E_glu);
  if (st) return st;
  if (n_rows == 0) return MOE_OK;
  if (!grad_out || !hidden || !top_k_weights || !top_k_indices || !act_codes || !sorted_token ||
      !sorted_flat || !grad_wt_out || (E_glu > 0 && (!eo || !grad_eo_out)))
    return MOE_ERR_SHAPE;
  if (grad_out_ld < H || grad_out_ld % vec_of(dtype)) return MOE_ERR_ALIGN;
  if (!al16(grad_out) || !al16(hidden) || (eo && !al16(eo)) || (grad_eo_out && !al16(grad_eo_out)))
    return MOE_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  MOE_BY_DTYPE(dtype, combine_bwd_kernel, dim3(row_grid(n_rows)), dim3(ROW_THREADS), s,
               (const T_*)grad_out, grad_out_ld, (const T_*)eo, (const T_*)hidden,
               (const T_*)top_k_weights, top_k_indices, act_codes, E_glu, n_experts, sorted_token,
               sorted_flat, n_rows, (int)H, (T_*)grad_eo_out, (T_*)grad_wt_out);
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}

extern "C" int moe_gate_grad(int dtype, const float* wt_partial, int n_parts, int64_t n_rows,
                             const void* grad_out, int64_t grad_out_ld, const void* hidden,
                             const int64_t* top_k_indices, const int32_t* act_codes,
                             int n_experts, int E_glu, const int32_t* flat_to_sorted,
                             int64_t n_tokens, int top_k, int64_t H, void* grad_wt_out,
                             void* stream) {
  int st = check_rows(dtype, n_tokens, top_k, H, n_experts, E_glu);
  if (st) return st;
  if (n_parts < 0 || n_rows < 0) return MOE_ERR_SHAPE;
  if (n_tokens == 0) return MOE_OK;
  if (!grad_out || !hidden || !top_k_indices || !act_codes || !flat_to_sorted || !grad_wt_out ||
      (E_glu > 0 && n_rows > 0 && n_parts > 0 && !wt_partial))
    return MOE_ERR_SHAPE;
  if (grad_out_ld < H || grad_out_ld % vec_of(dtype)) return MOE_ERR_ALIGN;
  if (!al16(grad_out) || !al16(hidden)) return MOE_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const bool lanes = n_parts > 0 && (n_parts & (n_parts - 1)) == 0 && (int64_t)top_k * n_parts <= 64;
  if (lanes)
    MOE_BY_DTYPE_B(dtype, gate_grad_kernel, true, dim3(row_grid(n_tokens)), dim3(ROW_THREADS), s,
                   wt_partial, n_parts, n_rows, (const T_*)grad_out, grad_out_ld, (const T_*)hidden,
                   top_k_indices, act_codes, E_glu, n_experts, flat_to_sorted, n_tokens, top_k,
                   (int)H, (T_*)grad_wt_out);
  else
    MOE_BY_DTYPE_B(dtype, gate_grad_kernel, false, dim3(row_grid(n_tokens)), dim3(ROW_THREADS), s,
                   wt_partial, n_parts, n_rows, (const T_*)grad_out, grad_out_ld, (const T_*)hidden,
                   top_k_indices, act_codes, E_glu, n_experts, flat_to_sorted, n_tokens, top_k,
                   (int)H, (T_*)grad_wt_out);
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}

extern "C" int moe_unpermute_bwd(int dtype, const void* grad_xs, const void* grad_out,
                                 int64_t grad_out_ld, const void* top_k_weights,
                                 const int64_t* top_k_indices, const int32_t* act_codes,
                                 int n_experts, int E_glu, const int32_t* flat_to_sorted,
                                 int64_t n_tokens, int top_k, int64_t H, void* grad_x_out,
                                 void* stream) {
  int st = check_rows(dtype, n_tokens, top_k, H, n_experts, E_glu);
  if (st) return st;
  if (n_tokens == 0) return MOE_OK;
  if (!grad_out || !top_k_weights || !top_k_indices || !act_codes || !flat_to_sorted ||
      !grad_x_out || (E_glu > 0 && !grad_xs))
    return MOE_ERR_SHAPE;
  if (grad_out_ld < H || grad_out_ld % vec_of(dtype)) return MOE_ERR_ALIGN;
  if (!al16(grad_out) || !al16(grad_x_out) || (grad_xs && !al16(grad_xs))) return MOE_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const GatherCfg gc = gather_cfg(H, vec_of(dtype), top_k);
  if (n_tokens * gc.col_waves >= ((int64_t)1 << 32)) return MOE_ERR_SHAPE;
  const dim3 grid(row_grid(n_tokens * gc.col_waves));
  with_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    with_gather_cfg(gc, [&](auto b, auto c) {
      constexpr int B = decltype(b)::value, C = decltype(c)::value;
      hipLaunchKernelGGL((unpermute_bwd_kernel<T, B, C>), grid, dim3(ROW_THREADS), 0, s,
                         (const T*)grad_xs, (const T*)grad_out, grad_out_ld,
                         (const T*)top_k_weights, top_k_indices, act_codes, E_glu, n_experts,
                         flat_to_sorted, n_tokens, top_k, (int)H, (T*)grad_x_out);
    });
  });
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}

extern "C" int moe_glu_fwd(int dtype, const void* gate_up, int64_t gu_ld, const int32_t* row_act,
                           const float* alpha, const float* gamma, int ap_stride, int64_t n_rows,
                           int64_t I, void* out, int64_t out_ld, void* stream) {
  if (dtype < 0 || dtype > 2) return MOE_ERR_DTYPE;
  if (n_rows < 0 || I <= 0 || I >= (1 << 30) || gu_ld < 2 * I || out_ld < I) return MOE_ERR_SHAPE;
  if (n_rows == 0) return MOE_OK;
  if (!gate_up || !row_act || !out || n_rows >= (1ll << 31)) return MOE_ERR_SHAPE;
  if ((alpha == nullptr) != (gamma == nullptr)) return MOE_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const int v = vec_of(dtype);
  const int nj = glu_vec_chunks(I, v, 8);
  if (nj && gu_ld % v == 0 && out_ld % v == 0 && al16(gate_up) && al16(out)) {
    const dim3 grid((unsigned)((n_rows + GLU_VEC_WAVES - 1) / GLU_VEC_WAVES)), block(64 * GLU_VEC_WAVES);
#define MOE_GLU_FWD_VEC(NJ_)                                                                     \
  MOE_BY_DTYPE_B(dtype, glu_fwd_vec_kernel, NJ_, grid, block, s, (const T_*)gate_up, gu_ld,     \
                 row_act, alpha, gamma, ap_stride, n_rows, (int)I, (T_*)out, out_ld)
    if (nj == 1) MOE_GLU_FWD_VEC(1);
    else if (nj == 2) MOE_GLU_FWD_VEC(2);
    else if (nj == 4) MOE_GLU_FWD_VEC(4);
    else MOE_GLU_FWD_VEC(8);
#undef MOE_GLU_FWD_VEC
  } else {
    MOE_BY_DTYPE(dtype, glu_fwd_kernel, dim3((unsigned)n_rows), dim3(GLU_THREADS), s,
                 (const T_*)gate_up, gu_ld, row_act, alpha, gamma, ap_stride, (int)I, (T_*)out,
                 out_ld);
  }
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}

extern "C" int moe_glu_bwd(int dtype, const void* grad_out, int64_t go_row_stride,
                           int64_t go_col_stride, const void* gate_up, int64_t gu_ld,
                           const int32_t* row_act, const float* alpha, const float* gamma,
                           int ap_stride, int64_t n_rows, int64_t I, void* ggu_out,
                           int64_t ggu_ld, float* da_out, float* dg_out, void* stream) {
  if (dtype < 0 || dtype > 2) return MOE_ERR_DTYPE;
  if (n_rows < 0 || I <= 0 || I >= (1 << 30) || gu_ld < 2 * I || ggu_ld < 2 * I) return MOE_ERR_SHAPE;
  if (n_rows == 0) return MOE_OK;
  if (!grad_out || !gate_up || !row_act || !ggu_out || n_rows >= (1ll << 31)) return MOE_ERR_SHAPE;
  if ((alpha == nullptr) != (gamma == nullptr) || (da_out == nullptr) != (dg_out == nullptr))
    return MOE_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const int v = vec_of(dtype);
  // At most 4 chunks per lane: the backward holds three rows' worth (gate, up, grad).
  const int nj = glu_vec_chunks(I, v, 4);
  if (nj && go_col_stride == 1 && go_row_stride % v == 0 && gu_ld % v == 0 && ggu_ld % v == 0 &&
      al16(grad_out) && al16(gate_up) && al16(ggu_out)) {
    const dim3 grid((unsigned)((n_rows + GLU_VEC_WAVES - 1) / GLU_VEC_WAVES)), block(64 * GLU_VEC_WAVES);
#define MOE_GLU_BWD_VEC(NJ_)                                                                     \
  MOE_BY_DTYPE_B(dtype, glu_bwd_vec_kernel, NJ_, grid, block, s, (const T_*)grad_out,           \
                 go_row_stride, (const T_*)gate_up, gu_ld, row_act, alpha, gamma, ap_stride,    \
                 n_rows, (int)I, (T_*)ggu_out, ggu_ld, da_out, dg_out)
    if (nj == 1) MOE_GLU_BWD_VEC(1);
    else if (nj == 2) MOE_GLU_BWD_VEC(2);
    else MOE_GLU_BWD_VEC(4);
#undef MOE_GLU_BWD_VEC
  } else {
    MOE_BY_DTYPE(dtype, glu_bwd_kernel, dim3((unsigned)n_rows), dim3(GLU_THREADS), s,
                 (const T_*)grad_out, go_row_stride, go_col_stride, (const T_*)gate_up, gu_ld,
                 row_act, alpha, gamma, ap_stride, (int)I, (T_*)ggu_out, ggu_ld, da_out, dg_out);
  }
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}

extern "C" const char* moe_version(void) { return "moe_gfx950 0.1.0"; }
