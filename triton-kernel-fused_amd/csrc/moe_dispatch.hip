// Token dispatch for the grouped expert GEMMs: per-expert histogram, prefix scan and a stable
// permutation of the N*k routed rows ordered by (expert id, flat index t*k+j).
//
// The reference sorts the flattened expert ids with torch's (unstable) sort and then syncs the
// host with bincount(...).tolist() (/root/reference/kernels/sm75/moe.py:564-572); its grouped
// schedule is a host loop (:535-543). Here everything stays on the device:
//   pass 1 (hist):    each chunk of DISPATCH_CHUNK flat rows counts its experts in LDS;
//   pass 2 (scan):    one workgroup turns the chunk histograms into per-chunk base offsets,
//                     per-expert counts, offsets and token-tile offsets;
//   pass 3 (scatter): each chunk re-reads its rows and ranks them stably. Within a wave the rank
//                     of a row among equal experts comes from a ballot match (one ballot per id
//                     bit) and a popcount; waves of one step are ordered through LDS counters.
// A batch that fits one chunk runs all three passes in one workgroup (dispatch_small_kernel).
#include <mutex>
#include <unordered_map>

#include "moe_common.h"

namespace moe {

constexpr int DISPATCH_THREADS = 256;
constexpr int DISPATCH_CHUNK = 1024;  // flat rows per chunk (4 steps of 256)
constexpr int MAX_EXPERTS = 1024;
constexpr int TILE_ROWS = 128;        // token-tile height of the grouped GEMMs

// Exclusive prefix sums over the block of up to NT * 2 values, two consecutive values per thread
// (v0 at index 2t, v1 at 2t+1): p0/p1 get the sums of everything before them, the return value is
// the total. s_w holds NT / 64 partial sums.
template <int NT>
__device__ __forceinline__ int block_scan2(int v0, int v1, int& p0, int& p1, int* s_w) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int x = v0 + v1;  // inclusive scan of the pair sums over the wave
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) s_w[w] = x;
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) {
    const int s = s_w[i];
    before += i < w ? s : 0;
    total += s;
  }
  p0 = before + x - v0 - v1;
  p1 = p0 + v0;
  return total;
}

__device__ __forceinline__ int load_expert(const int64_t* idx, int64_t f, int E, bool& valid) {
  int64_t v = idx[f];
  valid = (v >= 0) && (v < E);
  return valid ? (int)v : E;
}

// Writes -1 to sorted_token / sorted_flat at the positions of [f0, f0 + n) that lie in
// [routed, M): the tail of the sorted arrays when some ids were dropped (out of range), so a
// kernel walking all M sorted rows finds no stale indices there.
__device__ __forceinline__ void fill_tail(int64_t f0, int n, int nthreads, int routed, int64_t M,
                                          int32_t* sorted_token, int32_t* sorted_flat) {
  for (int i = threadIdx.x; i < n; i += nthreads) {
    const int64_t p = f0 + i;
    if (p >= routed && p < M) {
      sorted_token[p] = -1;
      sorted_flat[p] = -1;
    }
  }
}

__global__ void __launch_bounds__(DISPATCH_THREADS)
dispatch_hist_kernel(const int64_t* __restrict__ idx, int64_t M, int E, int32_t* __restrict__ hist,
                     int32_t* __restrict__ status) {
  __shared__ int cnt[MAX_EXPERTS + 1];
  const int b = blockIdx.x;
  for (int e = threadIdx.x; e <= E; e += DISPATCH_THREADS) cnt[e] = 0;
  __syncthreads();
  const int64_t f0 = (int64_t)b * DISPATCH_CHUNK;
  int bad = 0;
  for (int i = threadIdx.x; i < DISPATCH_CHUNK; i += DISPATCH_THREADS) {
    int64_t f = f0 + i;
    if (f < M) {
      bool valid;
      int e = load_expert(idx, f, E, valid);
      atomicAdd(&cnt[e], 1);
      bad += valid ? 0 : 1;
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += DISPATCH_THREADS) hist[(int64_t)b * E + e] = cnt[e];
  if (bad) atomicAdd(status, bad);
}

// One workgroup. hist (nchunks, E) is rewritten in place into exclusive per-chunk bases. The
// chunks are cut into G groups (thread g*E + e takes expert e of group g) so the group sums load
// in parallel; a scan over the groups in LDS gives each group's base.
__global__ void __launch_bounds__(1024)
dispatch_scan_kernel(int32_t* __restrict__ hist, int nchunks, int E, int32_t* __restrict__ counts,
                     int32_t* __restrict__ offsets, int32_t* __restrict__ tile_offsets,
                     int32_t* __restrict__ expert_order) {
  __shared__ int s_cnt[MAX_EXPERTS];
  __shared__ int s_tiles[MAX_EXPERTS];
  __shared__ int s_part[1024];  // [group][expert] chunk-group sums
  const int G = max(1, min(1024 / E, nchunks));
  const int g = threadIdx.x / E, e = threadIdx.x % E;
  const bool act = g < G;
  const int c_lo = act ? g * nchunks / G : 0, c_hi = act ? (g + 1) * nchunks / G : 0;
  // Eight chunks' counts are loaded before any is used, so the loads overlap.
  int sum = 0;
  for (int c0 = c_lo; c0 < c_hi; c0 += 8) {
    int v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = c0 + j < c_hi ? hist[(int64_t)(c0 + j) * E + e] : 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += v[j];
  }
  if (act) s_part[g * E + e] = sum;
  __syncthreads();
  if (act) {
    int run = 0, total = 0;
    for (int gg = 0; gg < G; ++gg) {
      const int p = s_part[gg * E + e];
      run += gg < g ? p : 0;
      total += p;
    }
    for (int c0 = c_lo; c0 < c_hi; c0 += 8) {
      int v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = c0 + j < c_hi ? hist[(int64_t)(c0 + j) * E + e] : 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (c0 + j < c_hi) hist[(int64_t)(c0 + j) * E + e] = run;
        run += v[j];
      }
    }
    if (g == 0) {
      counts[e] = total;
      s_cnt[e] = total;
      s_tiles[e] = (total + TILE_ROWS - 1) / TILE_ROWS;
    }
  }
  __syncthreads();
  // Experts by descending count (ties by id): rank = experts that sort before this one.
  if (threadIdx.x < E) {
    const int e = threadIdx.x;
    const int c = s_cnt[e];
    int rank = 0;
    for (int j = 0; j < E; ++j) {
      const int cj = s_cnt[j];
      rank += (cj > c) || (cj == c && j < e);
    }
    expert_order[rank] = e;
  }
  // E <= 1024: a serial scan by one thread is a few microseconds at most and keeps this exact.
  if (threadIdx.x == 0) {
    int o = 0, t = 0;
    for (int i = 0; i < E; ++i) {
      offsets[i] = o;
      tile_offsets[i] = t;
      o += s_cnt[i];
      t += s_tiles[i];
    }
    offsets[E] = o;
    tile_offsets[E] = t;
  }
}

__global__ void __launch_bounds__(DISPATCH_THREADS)
dispatch_scatter_kernel(const int64_t* __restrict__ idx, int64_t M, int top_k, int E,
                        const int32_t* __restrict__ chunk_base, const int32_t* __restrict__ offsets,
                        int32_t* __restrict__ sorted_token, int32_t* __restrict__ sorted_flat,
                        int32_t* __restrict__ flat_to_sorted) {
  constexpr int NW = DISPATCH_THREADS / 64;
  __shared__ int run[MAX_EXPERTS + 1];        // rows of each expert already placed by this chunk
  __shared__ int wcnt[NW][MAX_EXPERTS + 1];   // rows of each expert in each wave of this step
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  for (int e = threadIdx.x; e <= E; e += DISPATCH_THREADS) {
    run[e] = (e < E) ? offsets[e] + chunk_base[(int64_t)b * E + e] : 0;
  }
  int nbits = 0;
  while ((1 << nbits) <= E) ++nbits;  // ids 0..E (E = invalid bucket)
  const unsigned long long lt_mask = (1ull << lane) - 1ull;
  const int64_t f0 = (int64_t)b * DISPATCH_CHUNK;
  // Sorted positions past the routed count (one per dropped id) hold -1: this chunk's share of
  // [offsets[E], M) is its own index range, which no valid row's position reaches.
  fill_tail(f0, DISPATCH_CHUNK, DISPATCH_THREADS, offsets[E], M, sorted_token, sorted_flat);
  for (int s = 0; s < DISPATCH_CHUNK; s += DISPATCH_THREADS) {
    for (int i = threadIdx.x; i < NW * (E + 1); i += DISPATCH_THREADS) wcnt[i / (E + 1)][i % (E + 1)] = 0;
    __syncthreads();
    const int64_t f = f0 + s + threadIdx.x;
    const bool live = f < M;
    bool valid = false;
    int e = live ? load_expert(idx, f, E, valid) : E;
    // Lanes holding the same id: intersect the ballots of every id bit.
    unsigned long long match = ballot64(live);
#pragma unroll 1
    for (int bit = 0; bit < nbits; ++bit) {
      const bool on = (e >> bit) & 1;
      const unsigned long long bl = ballot64(live && on);
      match &= on ? bl : ~bl;
    }
    if (!live) match = 0;
    const int rank = __popcll(match & lt_mask);
    if (live && rank == 0) wcnt[w][e] = __popcll(match);
    __syncthreads();
    if (live) {
      if (valid) {
        int pos = run[e] + rank;
        for (int ww = 0; ww < w; ++ww) pos += wcnt[ww][e];
        sorted_token[pos] = (int32_t)(f / top_k);
        sorted_flat[pos] = (int32_t)f;
        flat_to_sorted[f] = pos;
      } else {
        flat_to_sorted[f] = -1;
      }
    }
    __syncthreads();
    for (int ee = threadIdx.x; ee < E; ee += DISPATCH_THREADS) {
      int add = 0;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) add += wcnt[ww][ee];
      run[ee] += add;
    }
    // The next step's clear of wcnt is ordered after these reads by its own barrier below.
    __syncthreads();
  }
}

// All three passes in one workgroup when every row fits one chunk (decode-sized batches), with
// block barriers in place of kernel launches: LDS histogram, the scans of dispatch_scan_kernel,
// and the stable scatter of dispatch_scatter_kernel over steps of SMALL_THREADS rows.
constexpr int SMALL_THREADS = 512;
__global__ void __launch_bounds__(SMALL_THREADS)
dispatch_small_kernel(const int64_t* __restrict__ idx, int64_t M, int top_k, int E,
                      int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                      int32_t* __restrict__ tile_offsets, int32_t* __restrict__ expert_order,
                      int32_t* __restrict__ sorted_token, int32_t* __restrict__ sorted_flat,
                      int32_t* __restrict__ flat_to_sorted, int32_t* __restrict__ status) {
  constexpr int NW = SMALL_THREADS / 64;
  __shared__ int cnt[MAX_EXPERTS + 1];
  __shared__ int run[MAX_EXPERTS + 1];
  __shared__ int wcnt[NW][MAX_EXPERTS + 1];
  __shared__ int s_bad;
  __shared__ int s_scan[NW];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int e = tid; e <= E; e += SMALL_THREADS) cnt[e] = 0;
  if (tid == 0) s_bad = 0;
  __syncthreads();
  // Every row fits one chunk (M <= DISPATCH_CHUNK): each thread loads its PER ids once and keeps
  // them for the scatter below.
  constexpr int PER = DISPATCH_CHUNK / SMALL_THREADS;
  static_assert(PER * SMALL_THREADS == DISPATCH_CHUNK, "whole rows per thread");
  int ev[PER];
  bool vv[PER];
  int bad = 0;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int64_t f = tid + (int64_t)u * SMALL_THREADS;
    vv[u] = false;
    ev[u] = E;
    if (f < M) {
      ev[u] = load_expert(idx, f, E, vv[u]);
      atomicAdd(&cnt[ev[u]], 1);
      bad += vv[u] ? 0 : 1;
    }
  }
  if (bad) atomicAdd(&s_bad, bad);
  __syncthreads();
  {
    // Offsets and tile offsets: block-wide exclusive scans (experts 2*tid and 2*tid + 1).
    static_assert(2 * SMALL_THREADS >= MAX_EXPERTS, "two experts per thread");
    const int e0 = 2 * tid, e1 = 2 * tid + 1;
    const int c0 = e0 < E ? cnt[e0] : 0, c1 = e1 < E ? cnt[e1] : 0;
    int o0, o1, t0, t1;
    const int o_tot = block_scan2<SMALL_THREADS>(c0, c1, o0, o1, s_scan);
    __syncthreads();  // s_scan is reused
    const int t_tot = block_scan2<SMALL_THREADS>((c0 + TILE_ROWS - 1) / TILE_ROWS,
                                                 (c1 + TILE_ROWS - 1) / TILE_ROWS, t0, t1, s_scan);
    if (e0 < E) { offsets[e0] = o0; tile_offsets[e0] = t0; run[e0] = o0; }
    if (e1 < E) { offsets[e1] = o1; tile_offsets[e1] = t1; run[e1] = o1; }
    if (tid == 0) {
      offsets[E] = o_tot;
      tile_offsets[E] = t_tot;
      if (s_bad) atomicAdd(status, s_bad);
    }
    fill_tail(0, DISPATCH_CHUNK, SMALL_THREADS, o_tot, M, sorted_token, sorted_flat);
  }
  // Experts by descending count (ties by id).
  for (int e = tid; e < E; e += SMALL_THREADS) {
    const int c = cnt[e];
    counts[e] = c;
    int rank = 0;
    for (int j = 0; j < E; ++j) {
      const int cj = cnt[j];
      rank += (cj > c) || (cj == c && j < e);
    }
    expert_order[rank] = e;
  }
  int nbits = 0;
  while ((1 << nbits) <= E) ++nbits;  // ids 0..E (E = invalid bucket)
  const unsigned long long lt_mask = (1ull << lane) - 1ull;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int64_t s = (int64_t)u * SMALL_THREADS;
    if (s >= M) break;
    for (int i = tid; i < NW * (E + 1); i += SMALL_THREADS) wcnt[i / (E + 1)][i % (E + 1)] = 0;
    __syncthreads();  // also orders run[] (first step) after thread 0's scan
    const int64_t f = s + tid;
    const bool live = f < M;
    const bool valid = vv[u];
    const int e = ev[u];
    unsigned long long match = ballot64(live);
#pragma unroll 1
    for (int bit = 0; bit < nbits; ++bit) {
      const bool on = (e >> bit) & 1;
      const unsigned long long bl = ballot64(live && on);
      match &= on ? bl : ~bl;
    }
    if (!live) match = 0;
    const int rank = __popcll(match & lt_mask);
    if (live && rank == 0) wcnt[w][e] = __popcll(match);
    __syncthreads();
    if (live) {
      if (valid) {
        int pos = run[e] + rank;
        for (int ww = 0; ww < w; ++ww) pos += wcnt[ww][e];
        sorted_token[pos] = (int32_t)(f / top_k);
        sorted_flat[pos] = (int32_t)f;
        flat_to_sorted[f] = pos;
      } else {
        flat_to_sorted[f] = -1;
      }
    }
    __syncthreads();
    for (int ee = tid; ee < E; ee += SMALL_THREADS) {
      int add = 0;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) add += wcnt[ww][ee];
      run[ee] += add;
    }
    __syncthreads();
  }
}

}  // namespace moe

using namespace moe;

static int64_t n_chunks(int64_t M) { return (M + DISPATCH_CHUNK - 1) / DISPATCH_CHUNK; }

extern "C" int moe_tile_rows(void) { return TILE_ROWS; }

extern "C" size_t moe_get_workspace_size(int64_t n_tokens, int top_k, int n_experts) {
  if (n_tokens < 0 || top_k <= 0 || n_experts <= 0) return 0;
  int64_t M = n_tokens * top_k;
  int64_t nc = n_chunks(M);
  if (nc < 1) nc = 1;
  size_t bytes = (size_t)nc * (size_t)n_experts * sizeof(int32_t);
  return (bytes + 255) & ~(size_t)255;
}

// The three passes on a given histogram buffer (nchunks * E int32, fully written by the
// histogram pass, so it needs no clearing).
static int dispatch_launch(const int64_t* top_k_indices, int64_t M, int top_k, int n_experts,
                           int32_t* counts, int32_t* offsets, int32_t* tile_offsets,
                           int32_t* expert_order, int32_t* sorted_token, int32_t* sorted_flat,
                           int32_t* flat_to_sorted, int32_t* status, int32_t* hist,
                           hipStream_t s) {
  const int nc = (int)n_chunks(M);
  if (nc <= 1) {
    hipLaunchKernelGGL(dispatch_small_kernel, dim3(1), dim3(SMALL_THREADS), 0, s, top_k_indices, M,
                       top_k, n_experts, counts, offsets, tile_offsets, expert_order, sorted_token,
                       sorted_flat, flat_to_sorted, status);
    return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
  }
  hipLaunchKernelGGL(dispatch_hist_kernel, dim3(nc), dim3(DISPATCH_THREADS), 0, s, top_k_indices,
                     M, n_experts, hist, status);
  hipLaunchKernelGGL(dispatch_scan_kernel, dim3(1), dim3(1024), 0, s, hist, nc, n_experts, counts,
                     offsets, tile_offsets, expert_order);
  hipLaunchKernelGGL(dispatch_scatter_kernel, dim3(nc), dim3(DISPATCH_THREADS), 0, s,
                     top_k_indices, M, top_k, n_experts, hist, offsets, sorted_token,
                     sorted_flat, flat_to_sorted);
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}

static int dispatch_check(const int64_t* top_k_indices, int64_t n_tokens, int top_k,
                          int n_experts, const int32_t* counts, const int32_t* offsets,
                          const int32_t* tile_offsets, const int32_t* expert_order,
                          const int32_t* sorted_token, const int32_t* sorted_flat,
                          const int32_t* flat_to_sorted, const int32_t* status) {
  if (n_tokens < 0 || top_k <= 0 || n_experts <= 0 || n_experts > MAX_EXPERTS) return MOE_ERR_SHAPE;
  const int64_t M = n_tokens * top_k;
  if (M >= (int64_t)1 << 31) return MOE_ERR_SHAPE;
  if (!counts || !offsets || !tile_offsets || !expert_order || !status) return MOE_ERR_SHAPE;
  if (M > 0 && (!top_k_indices || !sorted_token || !sorted_flat || !flat_to_sorted))
    return MOE_ERR_SHAPE;
  return MOE_OK;
}

extern "C" int moe_dispatch(const int64_t* top_k_indices, int64_t n_tokens, int top_k,
                            int n_experts, int32_t* counts, int32_t* offsets,
                            int32_t* tile_offsets, int32_t* expert_order, int32_t* sorted_token,
                            int32_t* sorted_flat, int32_t* flat_to_sorted, int32_t* status,
                            void* workspace, size_t workspace_bytes, void* stream) {
  int st = dispatch_check(top_k_indices, n_tokens, top_k, n_experts, counts, offsets, tile_offsets,
                          expert_order, sorted_token, sorted_flat, flat_to_sorted, status);
  if (st) return st;
  if (!workspace || workspace_bytes < moe_get_workspace_size(n_tokens, top_k, n_experts))
    return MOE_ERR_WORKSPACE;
  return dispatch_launch(top_k_indices, n_tokens * top_k, top_k, n_experts, counts, offsets,
                         tile_offsets, expert_order, sorted_token, sorted_flat, flat_to_sorted,
                         status, (int32_t*)workspace, (hipStream_t)stream);
}

// ───────────────────────── allocation-free dispatch ─────────────────────────
// For callers that cannot allocate device memory (code under HIP graph capture, serving loops):
// the histogram lives in a file-scope device array instead of a caller workspace. Each GPU holds
// its own copy for the life of the process; its device address is looked up once per device with
// hipGetSymbolAddress (the array's name is only a host-side stand-in in host code).
constexpr size_t DISPATCH_SCRATCH_BYTES = (size_t)4 << 20;  // 4 MiB: nchunks * E <= 2^20
static __device__ __align__(256) int32_t scratch[DISPATCH_SCRATCH_BYTES / sizeof(int32_t)];

static std::mutex g_scratch_mu;
static std::unordered_map<int, int32_t*> g_scratch_ptr;  // device ordinal -> device address

static int32_t* scratch_for_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  auto it = g_scratch_ptr.find(dev);
  if (it != g_scratch_ptr.end()) return it->second;
  void* ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
  g_scratch_ptr[dev] = (int32_t*)ptr;
  return (int32_t*)ptr;
}

extern "C" int moe_dispatch_noalloc(const int64_t* top_k_indices, int64_t n_tokens, int top_k,
                                    int n_experts, int32_t* counts, int32_t* offsets,
                                    int32_t* tile_offsets, int32_t* expert_order,
                                    int32_t* sorted_token, int32_t* sorted_flat,
                                    int32_t* flat_to_sorted, int32_t* status, void* stream) {
  int st = dispatch_check(top_k_indices, n_tokens, top_k, n_experts, counts, offsets, tile_offsets,
                          expert_order, sorted_token, sorted_flat, flat_to_sorted, status);
  if (st) return st;
  if (moe_get_workspace_size(n_tokens, top_k, n_experts) > DISPATCH_SCRATCH_BYTES)
    return MOE_ERR_WORKSPACE;
  int32_t* hist = scratch_for_current_device();
  if (!hist) return MOE_ERR_LAUNCH;
  return dispatch_launch(top_k_indices, n_tokens * top_k, top_k, n_experts, counts, offsets,
                         tile_offsets, expert_order, sorted_token, sorted_flat, flat_to_sorted,
                         status, hist, (hipStream_t)stream);
}
