// Router epilogue: the step between the router logits (N, E) and dispatch. Scores (sigmoid or
// softmax over the experts), selection on scores + bias (bias only steers the choice), top-k, the
// unbiased scores gathered at the picks, optional sum-to-1 normalisation, routed scaling, and the
// per-expert pick counts for auxiliary-loss-free load balancing; its backward; and the bias update
// (kernels/sm75/router.py:40-150,152-170,293-301).
//
// One wave owns one token row: lane l holds experts l, l+64, ... (EJ per lane). The top-k is a
// radix select over distinct integer keys (selection value, then the lower expert index first) by
// wave ballots: about 40 ballot rounds per row instead of an O(E) scan per lane, then each pick's
// slot is the count of larger picks. Ties pick the lowest expert index. Counts are summed per
// workgroup in LDS and added to the global counters with one integer atomic per expert, so the
// totals do not depend on the order of the atomics.
#include <algorithm>

#include "moe_common.h"

namespace moe {

constexpr int RT_THREADS = 256;  // 4 waves = 4 token rows per workgroup
constexpr int RT_MAX_E = 1024;
constexpr int RT_MAX_K = 32;
#ifndef RT_FWD_GRID
#define RT_FWD_GRID 2048
#endif
constexpr int RT_MAX_GRID = RT_FWD_GRID;  // forward workgroups (grid-stride over rows beyond)
constexpr int RT_COUNT_GRID = 64;    // count workgroups

__device__ __forceinline__ float sigmoid_acc(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
  return v;
}
__device__ __forceinline__ float wave_add(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

// This lane's logits of one row (invalid experts: -inf).
template <typename T, int EJ>
__device__ __forceinline__ void row_load(const T* row, int E, int lane, float (&x)[EJ]) {
#pragma unroll
  for (int j = 0; j < EJ; ++j) {
    const int e = lane + 64 * j;
    x[j] = e < E ? to_f32(row[e]) : -INFINITY;
  }
}

// Scores of this lane's experts for one row from its logits (invalid experts: score 0).
template <int EJ>
__device__ __forceinline__ void row_scores_of(const float (&x)[EJ], int E, int softmax, int lane,
                                              float (&s)[EJ]) {
  if (softmax) {
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < EJ; ++j) m = fmaxf(m, x[j]);
    m = wave_max(m);
    float z = 0.f;
#pragma unroll
    for (int j = 0; j < EJ; ++j) {
      s[j] = lane + 64 * j < E ? expf(x[j] - m) : 0.f;
      z += s[j];
    }
    z = wave_add(z);
    const float rz = 1.0f / z;
#pragma unroll
    for (int j = 0; j < EJ; ++j) s[j] *= rz;
  } else {
#pragma unroll
    for (int j = 0; j < EJ; ++j) s[j] = lane + 64 * j < E ? sigmoid_acc(x[j]) : 0.f;
  }
}

template <typename T, int EJ>
__global__ void __launch_bounds__(RT_THREADS)
router_fwd_kernel(const T* __restrict__ logits, int64_t ld, int64_t N, int E,
                  const float* __restrict__ bias, int top_k, int softmax, int norm, float scale,
                  int64_t* __restrict__ idx_out, float* __restrict__ w_out) {
  __shared__ unsigned long long s_keys[(RT_THREADS / 64) * RT_MAX_K];
  const int lane = threadIdx.x & 63;
  // Selection keys: the selection value as an order-preserving unsigned integer, then the
  // complemented expert index in the low ib bits, so keys are distinct and a larger key is the
  // better pick (ties in value go to the lower expert index). Invalid experts: key 0.
  const int ib = E > 1 ? 32 - __clz(E - 1) : 0;
  float bv[EJ];
#pragma unroll
  for (int j = 0; j < EJ; ++j) {
    const int e = lane + 64 * j;
    bv[j] = bias && e < E ? bias[e] : 0.f;
  }
  // Grid-stride over rows; the next row's logits are loaded while this row is processed.
  const int64_t step = (int64_t)gridDim.x * (RT_THREADS / 64);
  int64_t n = (int64_t)blockIdx.x * (RT_THREADS / 64) + (threadIdx.x >> 6);
  float xn[EJ];
  if (n < N) row_load<T, EJ>(logits + n * ld, E, lane, xn);
  for (; n < N; n += step) {
    float s[EJ], x[EJ];
#pragma unroll
    for (int j = 0; j < EJ; ++j) x[j] = xn[j];
    if (n + step < N) row_load<T, EJ>(logits + (n + step) * ld, E, lane, xn);
    row_scores_of<EJ>(x, E, softmax, lane, s);
    unsigned long long key[EJ];
#pragma unroll
    for (int j = 0; j < EJ; ++j) {
      const int e = lane + 64 * j;
      const unsigned u = __float_as_uint(s[j] + bv[j]);
      const unsigned k32 = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
      key[j] = e < E ? ((unsigned long long)k32 << ib) | (unsigned long long)(E - 1 - e) : 0ull;
    }
    // Bits above the highest one in which two valid keys differ are common to all of them: the
    // threshold starts with them (two wave reductions on the vector side instead of one scalar
    // round per bit).
    unsigned kmax = 0, kmin = 0xffffffffu;
#pragma unroll
    for (int j = 0; j < EJ; ++j)
      if (lane + 64 * j < E) {
        const unsigned k32 = (unsigned)(key[j] >> ib);
        kmax = max(kmax, k32);
        kmin = min(kmin, k32);
      }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
      kmax = max(kmax, (unsigned)__shfl_xor((int)kmax, d, 64));
      kmin = min(kmin, (unsigned)__shfl_xor((int)kmin, d, 64));
    }
    const int top = kmax == kmin ? -1 : 31 - __clz(kmax ^ kmin);  // highest differing value bit
    // A threshold that exactly top_k keys reach, one bit at a time from there down: keep a bit
    // when at least top_k keys reach the threshold with it set, stop as soon as exactly top_k do
    // (one ballot per bit and expert slot; the threshold is wave-uniform, the counting runs on the
    // scalar unit, which one CU's four SIMDs share, so the fewer rounds the better).
    unsigned long long thr =
        top >= 31 ? 0ull : ((unsigned long long)((kmax >> (top + 1)) << (top + 1)) << ib);
    for (int b = top + ib; b >= 0; --b) {
      const unsigned long long c = thr | (1ull << b);
      int cnt = 0;
#pragma unroll
      for (int j = 0; j < EJ; ++j) cnt += __popcll(__ballot(key[j] >= c));
      if (cnt >= top_k) {
        thr = c;
        if (cnt == top_k) break;  // exactly top_k keys reach thr: the lower bits change nothing
      }
    }
    // The picks are the top_k keys >= thr. They are compacted into this wave's LDS row, and a
    // pick's slot is the number of picked keys larger than its own.
    unsigned long long* sk = s_keys + (threadIdx.x >> 6) * RT_MAX_K;
    bool pick[EJ];
    float tsum = 0.f;
    int base = 0;
#pragma unroll
    for (int j = 0; j < EJ; ++j) {
      pick[j] = key[j] >= thr;
      tsum += pick[j] ? s[j] : 0.f;
      const unsigned long long m = __ballot(pick[j]);
      const int before = __builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
      if (pick[j]) sk[base + before] = key[j];
      base += __popcll(m);
    }
    int rank[EJ];
#pragma unroll
    for (int j = 0; j < EJ; ++j) rank[j] = 0;
    for (int i = 0; i < top_k; ++i) {
      const unsigned long long kp = sk[i];
#pragma unroll
      for (int j = 0; j < EJ; ++j) rank[j] += kp > key[j];
    }
    tsum = wave_add(tsum);
    const float f = norm ? scale / (tsum + 1e-20f) : scale;
#pragma unroll
    for (int j = 0; j < EJ; ++j) {
      if (pick[j]) {
        idx_out[n * top_k + rank[j]] = lane + 64 * j;
        w_out[n * top_k + rank[j]] = s[j] * f;
      }
    }
  }
}

// counts[e] += #{picks == e}: per-workgroup LDS histogram, then one global atomic per expert and
// workgroup (a small grid keeps the atomics on each counter few).
__global__ void __launch_bounds__(RT_THREADS)
router_count_kernel(const int64_t* __restrict__ idx, int64_t n_picks, int E, int32_t* counts) {
  __shared__ int s_cnt[RT_MAX_E];
  for (int e = threadIdx.x; e < E; e += RT_THREADS) s_cnt[e] = 0;
  __syncthreads();
  for (int64_t i = (int64_t)blockIdx.x * RT_THREADS + threadIdx.x; i < n_picks;
       i += (int64_t)gridDim.x * RT_THREADS)
    atomicAdd(&s_cnt[(int)idx[i]], 1);
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += RT_THREADS)
    if (s_cnt[e]) atomicAdd(&counts[e], s_cnt[e]);
}

// grad_logits[n, e] from grad_w (fp32, (N, k)): with picked raw scores w_k and T = sum w_k + 1e-20,
// the scattered score gradient is g_e = sum_{k: idx_k = e} G'_k with G'_k = scale/T (G_k - <G,w>/T)
// (normalised) or scale G_k; sigmoid: grad = g_e s_e (1 - s_e); softmax: s_e (g_e - sum_k G'_k w_k)
// (kernels/sm75/router.py:105-150).
template <typename T, int EJ>
__global__ void __launch_bounds__(RT_THREADS)
router_bwd_kernel(const T* __restrict__ logits, int64_t ld, int64_t N, int E,
                  const int64_t* __restrict__ idx, const float* __restrict__ gw, int top_k,
                  int softmax, int norm, float scale, T* __restrict__ gout, int64_t gout_ld) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * (RT_THREADS / 64) + (threadIdx.x >> 6);
  if (n >= N) return;
  float s[EJ];
  {
    float x[EJ];
    row_load<T, EJ>(logits + n * ld, E, lane, x);
    row_scores_of<EJ>(x, E, softmax, lane, s);
  }
  // Lane k (< top_k) holds slot k: its expert, upstream gradient and raw picked score.
  int ek = -1;
  float gk = 0.f, wk = 0.f;
  if (lane < top_k) {
    ek = (int)idx[n * top_k + lane];
    gk = gw[n * top_k + lane];
  }
  // Raw score of expert ek lives in lane ek % 64, slot ek / 64.
  {
    const int src = ek >= 0 ? (ek & 63) : 0, jj = ek >= 0 ? (ek >> 6) : 0;
    float mine = 0.f;
#pragma unroll
    for (int j = 0; j < EJ; ++j) {
      const float o = __shfl(s[j], src, 64);
      if (j == jj) mine = o;
    }
    wk = ek >= 0 ? mine : 0.f;
  }
  float gp;
  if (norm) {
    const float t = wave_add(wk) + 1e-20f;
    const float dot = wave_add(gk * wk);
    gp = scale / t * (gk - dot / t);
  } else {
    gp = scale * gk;
  }
  if (ek < 0) gp = 0.f;
  const float gs = softmax ? wave_add(gp * wk) : 0.f;
  float g[EJ];
#pragma unroll
  for (int j = 0; j < EJ; ++j) g[j] = 0.f;
  for (int k = 0; k < top_k; ++k) {
    const int e = __shfl(ek, k, 64);
    const float v = __shfl(gp, k, 64);
#pragma unroll
    for (int j = 0; j < EJ; ++j)
      if (lane + 64 * j == e) g[j] += v;
  }
  T* orow = gout + n * gout_ld;
#pragma unroll
  for (int j = 0; j < EJ; ++j) {
    const int e = lane + 64 * j;
    if (e < E) {
      const float r = softmax ? s[j] * (g[j] - gs) : g[j] * s[j] * (1.f - s[j]);
      orow[e] = from_f32<T>(r);
    }
  }
}

// bias[e] += u * sign(mean(counts) - counts[e]) in fp32, one workgroup.
__global__ void __launch_bounds__(1024) router_bias_kernel(float* bias, const int32_t* counts, int E, float u) {
  __shared__ float s_part[16];
  float acc = 0.f;
  for (int e = threadIdx.x; e < E; e += blockDim.x) acc += (float)counts[e];
  acc = wave_add(acc);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = acc;
  __syncthreads();
  float tot = 0.f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) tot += s_part[i];
  const float mean = tot / (float)E;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    const float d = mean - (float)counts[e];
    const float sg = d > 0.f ? 1.f : (d < 0.f ? -1.f : 0.f);
    bias[e] += u * sg;
  }
}

}  // namespace moe

using namespace moe;

static int ej_of(int E) { return E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : 16; }

#define RT_DISPATCH(dtype, EJV, KERNEL, GRID, STREAM, ...)                                   \
  do {                                                                                       \
    auto launch = [&]<typename T_>() {                                                       \
      switch (EJV) {                                                                         \
        case 1: hipLaunchKernelGGL((KERNEL<T_, 1>), GRID, dim3(RT_THREADS), 0, STREAM, __VA_ARGS__); break; \
        case 2: hipLaunchKernelGGL((KERNEL<T_, 2>), GRID, dim3(RT_THREADS), 0, STREAM, __VA_ARGS__); break; \
        case 4: hipLaunchKernelGGL((KERNEL<T_, 4>), GRID, dim3(RT_THREADS), 0, STREAM, __VA_ARGS__); break; \
        case 8: hipLaunchKernelGGL((KERNEL<T_, 8>), GRID, dim3(RT_THREADS), 0, STREAM, __VA_ARGS__); break; \
        default: hipLaunchKernelGGL((KERNEL<T_, 16>), GRID, dim3(RT_THREADS), 0, STREAM, __VA_ARGS__); break; \
      }                                                                                      \
    };                                                                                       \
    if ((dtype) == MOE_DT_BF16) launch.template operator()<bf16>();                          \
    else if ((dtype) == MOE_DT_F16) launch.template operator()<f16>();                       \
    else launch.template operator()<float>();                                                \
  } while (0)

static int check_router(int dtype, int64_t N, int E, int top_k, int64_t ld) {
  if (dtype != MOE_DT_F32 && dtype != MOE_DT_F16 && dtype != MOE_DT_BF16) return MOE_ERR_DTYPE;
  if (N < 0 || N >= ((int64_t)1 << 31) / 4 || E <= 0 || E > RT_MAX_E || top_k <= 0 ||
      top_k > RT_MAX_K || top_k > E || ld < E)
    return MOE_ERR_SHAPE;
  return MOE_OK;
}

extern "C" int moe_router_topk_fwd(int dtype, const void* logits, int64_t ld, int64_t n_tokens,
                                   int n_experts, const float* bias, int top_k, int softmax,
                                   int norm, float scale, int64_t* idx_out, float* w_out,
                                   int32_t* counts, void* stream) {
  int st = check_router(dtype, n_tokens, n_experts, top_k, ld);
  if (st) return st;
  if (n_tokens == 0) return MOE_OK;
  if (!logits || !idx_out || !w_out) return MOE_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const dim3 fgrid((unsigned)std::min<int64_t>((n_tokens + 3) / 4, RT_MAX_GRID));
  RT_DISPATCH(dtype, ej_of(n_experts), router_fwd_kernel, fgrid, s, (const T_*)logits, ld, n_tokens,
              n_experts, bias, top_k, softmax, norm, scale, idx_out, w_out);
  if (counts) {
    const int64_t picks = n_tokens * top_k;
    const unsigned cg = (unsigned)std::min<int64_t>((picks + RT_THREADS - 1) / RT_THREADS, RT_COUNT_GRID);
    hipLaunchKernelGGL(router_count_kernel, dim3(cg), dim3(RT_THREADS), 0, s, idx_out, picks,
                       n_experts, counts);
  }
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}

extern "C" int moe_router_topk_bwd(int dtype, const void* logits, int64_t ld, int64_t n_tokens,
                                   int n_experts, const int64_t* idx, const float* grad_w,
                                   int top_k, int softmax, int norm, float scale,
                                   void* grad_logits_out, int64_t out_ld, void* stream) {
  int st = check_router(dtype, n_tokens, n_experts, top_k, ld);
  if (st) return st;
  if (out_ld < n_experts) return MOE_ERR_SHAPE;
  if (n_tokens == 0) return MOE_OK;
  if (!logits || !idx || !grad_w || !grad_logits_out) return MOE_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)((n_tokens + 3) / 4));
  RT_DISPATCH(dtype, ej_of(n_experts), router_bwd_kernel, grid, s, (const T_*)logits, ld, n_tokens,
              n_experts, idx, grad_w, top_k, softmax, norm, scale, (T_*)grad_logits_out, out_ld);
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}

extern "C" int moe_router_bias_update(float* bias, const int32_t* counts, int n_experts, float u,
                                      void* stream) {
  if (n_experts <= 0) return MOE_ERR_SHAPE;
  if (!(u > 0.f)) return MOE_OK;  // u <= 0 (or NaN): no update, as the reference returns early
  if (!bias || !counts) return MOE_ERR_SHAPE;
  hipLaunchKernelGGL(router_bias_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, bias, counts,
                     n_experts, u);
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}
