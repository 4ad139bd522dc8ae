// Grouped expert GEMMs for gfx950: forward gate/up (+GLU epilogue), forward down, backward dX of
// both projections (+GLU-backward epilogue on the down one) and the ragged weight gradients; the
// C-ABI entry points at the end of the file pick the kernel.
//
// 16-bit operands with K a multiple of 64 run the eight-wave ring kernels of moe_gemm_v4.h
// (token_gemm_v4_kernel, wgrad_v4_kernel below); row-contiguous weights with other K run the
// five-stage kernel of moe_gemm_v3.h. The first-generation kernels described next serve fp32 and
// the remaining 16-bit shapes.
//
// First generation: one MFMA mainloop. The output tile is BR "P rows" x BC "Q columns"; P feeds
// the MFMA A side and is always the operand whose index is contiguous in the output, so each lane
// ends up owning four consecutive output elements (one 8-byte bf16 store). Both operands are
// staged through LDS as [row][128 bytes of K] with a 16-byte pad per row (conflict-free 16-byte
// reads for 16 consecutive rows), double-buffered with one barrier per K step. Operands that are
// K-contiguous in HBM are copied as 16-byte chunks; operands that are row-contiguous (weights
// read transposed, and every wgrad operand) are loaded as VECxVEC blocks and transposed in
// registers before the LDS store, so the MFMA always reads 16 contiguous K bytes per lane.
//
// Token GEMMs walk variable-size expert groups: every workgroup rebuilds the per-expert tile
// prefix from the dispatch offsets in LDS (a block scan), finds its expert by binary search and
// exits if its tile is past the end, so the grid is a host-side upper bound and nothing syncs.
#include "moe_common.h"
#include "moe_gemm_common.h"
#include "moe_gemm_v3.h"
#include "moe_gemm_v4.h"



namespace moe {

// ---------------------------------------------------------------------------------------------
// Loaders. fetch() issues the global loads of one K step into registers, store() writes them to
// one LDS stage. Rows outside the valid range and K beyond the end load zeros.

// K-contiguous rows: chunk c = tid + i*NT covers tile row c/8, 16-byte K chunk c%8.
template <typename T, int ROWS, int NT>
struct KcLoader {
  static constexpr int VEC = 16 / (int)sizeof(T);
  static constexpr int CPR = BK_BYTES / 16;
  static constexpr int CPT = ROWS * CPR / NT;
  static_assert((ROWS * CPR) % NT == 0 && NT % CPR == 0, "chunk split");
  const char* row[CPT];
  i32x4 reg[CPT];
  int kc;
  int K;

  __device__ __forceinline__ static int row_of(int i) {
    return (int)(threadIdx.x / CPR) + i * (NT / CPR);
  }
  __device__ __forceinline__ void fetch(int k0) {
    const int k = k0 + kc * VEC;
    const bool kin = k < K;
#pragma unroll
    for (int i = 0; i < CPT; ++i)
      reg[i] = (row[i] != nullptr && kin) ? ldg16(row[i] + (size_t)k * sizeof(T)) : zero4();
  }
  __device__ __forceinline__ void store(char* lds) const {
#pragma unroll
    for (int i = 0; i < CPT; ++i) *(i32x4*)(lds + row_of(i) * LDS_ROW + kc * 16) = reg[i];
  }
};

// in[j] = VEC values (index r) of K row j  ->  out[r] = the VEC K values of column r.
__device__ __forceinline__ void transpose_unit(const i32x4 (&in)[8], i32x4 (&out)[8]) {
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const unsigned sel = (r & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      out[r][w] = (int)__builtin_amdgcn_perm((unsigned)in[2 * w + 1][r >> 1],
                                             (unsigned)in[2 * w][r >> 1], sel);
  }
}
__device__ __forceinline__ void transpose_unit(const i32x4 (&in)[4], i32x4 (&out)[4]) {
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) out[r][j] = in[j][r];
}

// Row-contiguous operand: element (r, k) at src + row(k)*ld + r with row(k) = gather ? gather[k]
// : k. Unit u = tid + i*NT covers VEC rows r (chunk rc = u % RCH) x VEC K values (kc = u / RCH);
// rc runs fastest so a wave's loads of one K row are contiguous.
template <typename T, int ROWS, int NT>
struct RcLoader {
  static constexpr int VEC = 16 / (int)sizeof(T);
  static constexpr int RCH = ROWS / VEC;
  static constexpr int KCH = BK_BYTES / 16;
  static constexpr int UNITS = RCH * KCH;
  static constexpr int UPT = (UNITS + NT - 1) / NT;
  const char* src;  // column r0 of row 0
  size_t ld;        // bytes between rows
  const int32_t* gather;
  int kend;    // K values >= kend load zeros
  int rvalid;  // tile rows >= rvalid load zeros (a multiple of VEC)
  i32x4 reg[UPT][VEC];

  __device__ __forceinline__ void fetch(int k0) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = (int)threadIdx.x + i * NT;
      if (UNITS % NT == 0 || u < UNITS) {
        const int rc = u % RCH, kc = u / RCH;
        const bool rin = rc * VEC < rvalid;
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          const int k = k0 + kc * VEC + j;
          if (rin && k < kend) {
            const int rowi = gather ? gather[k] : k;
            reg[i][j] = ldg16(src + (size_t)rowi * ld + (size_t)rc * 16);
          } else {
            reg[i][j] = zero4();
          }
        }
      }
    }
  }
  __device__ __forceinline__ void store(char* lds) const {
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = (int)threadIdx.x + i * NT;
      if (UNITS % NT == 0 || u < UNITS) {
        const int rc = u % RCH, kc = u / RCH;
        i32x4 t[VEC];
        transpose_unit(reg[i], t);
#pragma unroll
        for (int r = 0; r < VEC; ++r) *(i32x4*)(lds + (rc * VEC + r) * LDS_ROW + kc * 16) = t[r];
      }
    }
  }
};

// ---------------------------------------------------------------------------------------------
// Mainloop: acc[ti][tj] += P_tile(rows) . Q_tile(cols) over K in [k_begin, k_end).
template <class C, class LP, class LQ>
__device__ __forceinline__ void mainloop(f32x16 (&acc)[C::TI][C::TJ], LP& lp, LQ& lq, int k_begin,
                                         int k_end, char* smem) {
  const int nk = (k_end - k_begin + C::BK - 1) / C::BK;
  if (nk <= 0) return;
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int wr = wid / C::WC, wc = wid % C::WC;
  const int pa_off = (wr * C::WTR + (lane & 31)) * LDS_ROW + (lane >> 5) * 16;
  const int qb_off = C::LDS_P + (wc * C::WTC + (lane & 31)) * LDS_ROW + (lane >> 5) * 16;

  lp.fetch(k_begin);
  lq.fetch(k_begin);
  lp.store(smem);
  lq.store(smem + C::LDS_P);
  __syncthreads();
  for (int it = 0; it < nk; ++it) {
    char* cur = smem + (it & 1) * C::STAGE;
    const bool more = it + 1 < nk;
    if (more) {
      lp.fetch(k_begin + (it + 1) * C::BK);
      lq.fetch(k_begin + (it + 1) * C::BK);
    }
#pragma unroll
    for (int s = 0; s < C::SLABS; ++s) {
      i32x4 a[C::TI], b[C::TJ];
#pragma unroll
      for (int ti = 0; ti < C::TI; ++ti)
        a[ti] = *(const i32x4*)(cur + pa_off + ti * 32 * LDS_ROW + s * 32);
#pragma unroll
      for (int tj = 0; tj < C::TJ; ++tj)
        b[tj] = *(const i32x4*)(cur + qb_off + tj * 32 * LDS_ROW + s * 32);
#pragma unroll
      for (int ti = 0; ti < C::TI; ++ti)
#pragma unroll
        for (int tj = 0; tj < C::TJ; ++tj) Mfma<typename C::T>::step(acc[ti][tj], a[ti], b[tj]);
    }
    if (more) {
      char* nxt = smem + ((it + 1) & 1) * C::STAGE;
      lp.store(nxt);
      lq.store(nxt + C::LDS_P);
    }
    __syncthreads();
  }
}

// Token-GEMM epilogue: acc holds P rows x token columns of tile (rt, sorted rows m0..) of expert e.
template <class C, int EPI>
__device__ __forceinline__ void token_epilogue(f32x16 (&acc)[C::TI][C::TJ], const TokenArgs& a, int e,
                                               int m0, int m_end, int rt) {
  typedef typename C::T T;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const int wr = wid / C::WC, wc = wid % C::WC;
  const int h = lane >> 5;
  // act_codes is NULL when the epilogue only writes raw GEMM results (grad_inter mode).
  const int code = (EPI == EPI_STORE || a.act_codes == nullptr) ? 0 : a.act_codes[e];
  static_for<0, C::TJ>([&](auto tj_c) {
    constexpr int tj = decltype(tj_c)::value;
    const int m = m0 + wc * C::WTC + tj * 32 + (lane & 31);
    if (m >= m_end) return;
    if constexpr (EPI == EPI_STORE) {
      T* o = (T*)a.out + (size_t)m * a.out_ld;
#pragma unroll
      for (int ti = 0; ti < C::TI; ++ti)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int r = rt * C::BR + wr * C::WTR + ti * 32 + 8 * g + 4 * h;
          if (r < a.R)
            Store4<T>::st(o + r, acc[ti][tj][4 * g], acc[ti][tj][4 * g + 1],
                          acc[ti][tj][4 * g + 2], acc[ti][tj][4 * g + 3]);
        }
    } else if constexpr (EPI == EPI_GLU_FWD) {
      T* gu = (T*)a.out + (size_t)m * 2 * a.I;
      T* it = a.out2 ? (T*)a.out2 + (size_t)m * a.I : nullptr;
#pragma unroll
      for (int ti = 0; ti < C::TI / 2; ++ti)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int ch = rt * (C::BR / 2) + wr * (C::WTR / 2) + ti * 32 + 8 * g + 4 * h;
          if (ch >= a.I) continue;
          float gv[4], uv[4], iv[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            gv[j] = round_through<T>(acc[ti][tj][4 * g + j]);
            uv[j] = round_through<T>(acc[ti + C::TI / 2][tj][4 * g + j]);
            iv[j] = glu_act(code, gv[j]) * uv[j];
          }
          Store4<T>::st(gu + ch, gv[0], gv[1], gv[2], gv[3]);
          Store4<T>::st(gu + a.I + ch, uv[0], uv[1], uv[2], uv[3]);
          if (it) Store4<T>::st(it + ch, iv[0], iv[1], iv[2], iv[3]);
        }
    } else {  // EPI_GLU_BWD: acc = grad_inter[m, i]
      const T* gu = (const T*)a.aux + (size_t)m * 2 * a.I;
      T* ggu = a.out ? (T*)a.out + (size_t)m * 2 * a.I : nullptr;
      T* gi = a.out2 ? (T*)a.out2 + (size_t)m * a.I : nullptr;
#pragma unroll
      for (int ti = 0; ti < C::TI; ++ti) {
        // The gate/up values of this lane's 16 channels in tile row ti, loaded together.
        float gv[4][4], uv[4][4];
        const int ib = rt * C::BR + wr * C::WTR + ti * 32 + 4 * h;
        if (ggu) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int i0 = min(ib + 8 * g, a.I - 4);
            Store4<T>::ld(gu + i0, gv[g]);
            Store4<T>::ld(gu + a.I + i0, uv[g]);
          }
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int i0 = ib + 8 * g;
          float go[4], dg[4], du[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            go[j] = round_through<T>(acc[ti][tj][4 * g + j]);
            float act, dact;
            glu_act_dact(code, gv[g][j], act, dact);
            dg[j] = go[j] * uv[g][j] * dact;
            du[j] = go[j] * act;
          }
          if (i0 < a.I) {
            if (gi) Store4<T>::st(gi + i0, go[0], go[1], go[2], go[3]);
            if (ggu) {
              Store4<T>::st(ggu + i0, dg[0], dg[1], dg[2], dg[3]);
              Store4<T>::st(ggu + a.I + i0, du[0], du[1], du[2], du[3]);
            }
          }
        }
      }
    }
  });
}

template <class C, int EPI, bool P_RC>
__global__ void __launch_bounds__(C::NT)
token_gemm_kernel(TokenArgs a) {
  typedef typename C::T T;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  __shared__ int s_pref[MAX_GLU_EXPERTS + 1];
  __shared__ int s_wsum[C::NT / 64];

  tile_prefix<C::NT>(a.offsets, a.E_glu, C::BC, s_pref, s_wsum);
  const int mt = (int)(blockIdx.x / a.n_rtiles);
  const int rt = (int)(blockIdx.x % a.n_rtiles);
  if (mt >= s_pref[a.E_glu]) return;
  int lo = 0, hi = a.E_glu - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_pref[mid] <= mt) lo = mid; else hi = mid - 1;
  }
  const int e = lo;
  const int m0 = a.offsets[e] + (mt - s_pref[e]) * C::BC;
  const int m_end = a.offsets[e + 1];

  const int tid = threadIdx.x;
  const T* Pe = (const T*)a.P + (size_t)e * a.p_e;

  // Q: sorted token rows m0 .. m0+BC (K-contiguous, optionally gathered).
  KcLoader<T, C::BC, C::NT> lq;
  lq.kc = tid % lq.CPR;
  lq.K = a.K;
#pragma unroll
  for (int i = 0; i < lq.CPT; ++i) {
    const int m = m0 + lq.row_of(i);
    if (m < m_end) {
      const int qr = a.q_gather ? a.q_gather[m] : m;
      lq.row[i] = (const char*)((const T*)a.Q + (size_t)qr * a.q_ld);
    } else {
      lq.row[i] = nullptr;
    }
  }

  f32x16 acc[C::TI][C::TJ];
#pragma unroll
  for (int ti = 0; ti < C::TI; ++ti)
#pragma unroll
    for (int tj = 0; tj < C::TJ; ++tj)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[ti][tj][v] = 0.f;

  if constexpr (P_RC) {
    // P[r, k] at Pe + k*p_ld + r (a weight read transposed).
    RcLoader<T, C::BR, C::NT> lp;
    const int r0 = rt * C::BR;
    lp.src = (const char*)(Pe + r0);
    lp.ld = (size_t)a.p_ld * sizeof(T);
    lp.gather = nullptr;
    lp.kend = a.K;
    lp.rvalid = a.R - r0;
    mainloop<C>(acc, lp, lq, 0, a.K, smem);
  } else {
    KcLoader<T, C::BR, C::NT> lp;
    lp.kc = tid % lp.CPR;
    lp.K = a.K;
#pragma unroll
    for (int i = 0; i < lp.CPT; ++i) {
      const int rr = lp.row_of(i);
      int prow;
      bool ok;
      if (EPI == EPI_GLU_FWD) {
        // Interleave gate and up: in each wave's WTR rows the first half are gate channels and
        // the second half the same up channels, so the epilogue pairs them in registers.
        const int wr = rr / C::WTR, w = rr % C::WTR;
        const int ch = rt * (C::BR / 2) + wr * (C::WTR / 2) + (w % (C::WTR / 2));
        ok = ch < a.I;
        prow = (w >= C::WTR / 2 ? a.I : 0) + ch;
      } else {
        prow = rt * C::BR + rr;
        ok = prow < a.R;
      }
      lp.row[i] = ok ? (const char*)(Pe + (size_t)prow * a.p_ld) : nullptr;
    }
    mainloop<C>(acc, lp, lq, 0, a.K, smem);
  }

  token_epilogue<C, EPI>(acc, a, e, m0, m_end, rt);
}

// ---------------------------------------------------------------------------------------------
// Ragged weight gradient: out[e, c, r] = sum_{m in rows(e)} rsrc[rrow(m), r] * csrc[crow(m), c].
struct WgradArgs {
  const void* rsrc; long long r_ld; const int32_t* r_gather;
  const void* csrc; long long c_ld; const int32_t* c_gather;
  int R, C;
  const int32_t* offsets;
  int n_rtiles, n_ctiles;
  void* out;
  // K split (ring kernel only): S pieces per tile (1 = none), workgroups b = piece * Lp + tile
  // index; fp32 partials in split_ws (one 256x256 slot per piece), one arrival counter per tile.
  int S, Lp;
  float* split_ws;
  int* split_cnt;
};

template <class C>
__device__ __forceinline__ void wgrad_epilogue(f32x16 (&acc)[C::TI][C::TJ], const WgradArgs& a, int e,
                                               int r0, int c0) {
  typedef typename C::T T;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wr = wid / C::WC, wc = wid % C::WC;
  const int h = lane >> 5;
  T* outE = (T*)a.out + (size_t)e * a.C * a.R;
#pragma unroll
  for (int tj = 0; tj < C::TJ; ++tj) {
    const int c = c0 + wc * C::WTC + tj * 32 + (lane & 31);
    if (c >= a.C) continue;
    T* o = outE + (size_t)c * a.R;
#pragma unroll
    for (int ti = 0; ti < C::TI; ++ti)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int r = r0 + wr * C::WTR + ti * 32 + 8 * g + 4 * h;
        if (r < a.R)
          Store4<T>::st(o + r, acc[ti][tj][4 * g], acc[ti][tj][4 * g + 1], acc[ti][tj][4 * g + 2],
                        acc[ti][tj][4 * g + 3]);
      }
  }
}

template <class C>
__global__ void __launch_bounds__(C::NT)
wgrad_kernel(WgradArgs a) {
  typedef typename C::T T;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int per_e = a.n_rtiles * a.n_ctiles;
  const int e = (int)(blockIdx.x / per_e);
  const int rem = (int)(blockIdx.x % per_e);
  const int ct = rem / a.n_rtiles, rt = rem % a.n_rtiles;
  const int k0 = a.offsets[e], k1 = a.offsets[e + 1];
  const int r0 = rt * C::BR, c0 = ct * C::BC;

  RcLoader<T, C::BR, C::NT> lp;
  lp.src = (const char*)((const T*)a.rsrc + r0);
  lp.ld = (size_t)a.r_ld * sizeof(T);
  lp.gather = a.r_gather;
  lp.kend = k1;
  lp.rvalid = a.R - r0;
  RcLoader<T, C::BC, C::NT> lq;
  lq.src = (const char*)((const T*)a.csrc + c0);
  lq.ld = (size_t)a.c_ld * sizeof(T);
  lq.gather = a.c_gather;
  lq.kend = k1;
  lq.rvalid = a.C - c0;

  f32x16 acc[C::TI][C::TJ];
#pragma unroll
  for (int ti = 0; ti < C::TI; ++ti)
#pragma unroll
    for (int tj = 0; tj < C::TJ; ++tj)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[ti][tj][v] = 0.f;
  mainloop<C>(acc, lp, lq, k0, k1, smem);

  wgrad_epilogue<C>(acc, a, e, r0, c0);
}

// ---------------------------------------------------------------------------------------------
// Second-generation kernels (16-bit types; 256x256 tiles, DMA-fed LDS; see moe_gemm_v2.h).

template <typename T> using V2Cfg = Cfg<T, v2::TILE, v2::TILE, 2, 2>;

// Token-GEMM epilogue of the 256x256 kernels through LDS (v2::stage_acc): same values as
// token_epilogue, written as whole 16-byte chunks. Wave (wr, wc) owns sorted rows
// m0 + wc*128 + q and, per mode, these channels of its staged block:
//   EPI_STORE   chunk c -> out channel rt*256 + wr*128 + 8c
//   EPI_GLU_FWD chunk c < 8 -> gate channel rt*128 + wr*64 + 8c, chunk c + 8 -> the same up channel
//   EPI_GLU_BWD chunk c -> grad_inter channel rt*256 + wr*128 + 8c
// WQ = token rows per wave; the wave holds channels wr*128..+127
// of the 256-channel tile and token rows wc*WQ..+WQ-1.
// wrow (WQ = 64): the gate of token row row0 + lane when a.gate is set (1 otherwise), fetched by
// the caller before its K loop.
template <typename T, int EPI, int WQ = 32 * v2::TN, class Acc>
__device__ __forceinline__ void token_epilogue_v2(const Acc& acc, const TokenArgs& a, int e, int m0,
                                                  int m_end, int rt, char* smem, int wr, int wc,
                                                  float wrow = 1.f) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  char* wl = smem + w * (WQ * v2::EPI_ROWB);
  const int row0 = m0 + wc * WQ;
  v2::stage_acc<T>(acc, wl);
  __syncthreads();
  if (row0 >= m_end) return;  // this wave's token rows all lie past the group end
  if constexpr (EPI == EPI_STORE) {
    v2::store_staged<T, WQ>(wl, (T*)a.out, a.out_ld, row0, m_end, rt * v2::TILE + wr * v2::WT, a.R);
  } else if constexpr (EPI == EPI_GLU_FWD) {
    const int code = a.act_codes ? a.act_codes[e] : 0;
    const int c = lane & 7;
    const int ch = rt * (v2::TILE / 2) + wr * (v2::WT / 2) + 8 * c;
    T* gu = (T*)a.out;
    T* it = (T*)a.out2;
#pragma unroll 4
    for (int i = 0; i < WQ / 8; ++i) {
      const int q = i * 8 + (lane >> 3);
      const int m = row0 + q;
      const i32x4 gq = v2::staged(wl, q, c), uq = v2::staged(wl, q, c + 8);
      // Weighted intermediate (a.gate set): w * act(g) * u, so the down projection yields w * eo
      // and the combine only sums; w = 1 (exact) otherwise. Shuffled with every lane active.
      const float w = __shfl(wrow, q & 63, 64);
      if (m < m_end && ch < a.I) {
        T* r = gu + (size_t)m * 2 * a.I + ch;
        v2::st_stream(gq, r);
        v2::st_stream(uq, r + a.I);
        if (it) {
          float gv[8], uv[8], iv[8];
          v2::unpack8<T>(gq, gv);
          v2::unpack8<T>(uq, uv);
#pragma unroll
          for (int j = 0; j < 8; ++j) iv[j] = w * (glu_act(code, gv[j]) * uv[j]);
          v2::st_stream(v2::pack8<T>(iv), it + (size_t)m * a.I + ch);
        }
      }
    }
  } else if constexpr (EPI == EPI_GLU_BWD_GATED) {
    // Staged value = grad_out[t] @ down_proj[e] (no gate). With w = gate of the row, inter =
    // act(g) * u recomputed in fp32: grad_inter = w * staged, the GLU backward of grad_inter,
    // gate*inter for the down weight gradient, and the gate gradient's partial dot
    // sum_ch staged * inter (kernels/sm75/moe.py:712-720: <grad_out, eo> = <grad_out @ W_d, inter>).
    const int code = a.act_codes ? a.act_codes[e] : 0;
    const int c = lane & 15;
    const int ch = rt * v2::TILE + wr * v2::WT + 8 * c;
    const int chc = min(ch, a.I - 8);
    const bool cok = ch < a.I;
    static_assert(WQ == 64, "one gate per lane of the wave's token rows");
    const T* gu = (const T*)a.aux;
    T* ggu = (T*)a.out;
    T* iw = (T*)a.out2;
    float* part = a.part + (size_t)(2 * rt + wr) * a.out_ld;  // out_ld = M (partials row length)
    // Rows per batch of gate_up loads: 4 measured ~1% faster than 8 and ~4% faster than all 16 at
    // once (the epilogues of all CUs compete for HBM).
    constexpr int NB = 4;
#pragma unroll 1
    for (int i0 = 0; i0 < WQ / 4; i0 += NB) {
      i32x4 gq[NB], uq[NB];
      float wv[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int m = min(row0 + (i0 + b) * 4 + (lane >> 4), m_end - 1);
        const T* r = gu + (size_t)m * 2 * a.I + chc;
        gq[b] = *(const i32x4*)r;
        uq[b] = *(const i32x4*)(r + a.I);
        wv[b] = __shfl(wrow, (i0 + b) * 4 + (lane >> 4), 64);
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int q = (i0 + b) * 4 + (lane >> 4);
        const int m = row0 + q;
        const i32x4 oq = v2::staged(wl, q, c);
        float go[8], gv[8], uv[8], dg[8], du[8], ia[8];
        v2::unpack8<T>(oq, go);
        v2::unpack8<T>(gq[b], gv);
        v2::unpack8<T>(uq[b], uv);
        float dot = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float act, dact;
          glu_act_dact(code, gv[j], act, dact);
          const float inter = act * uv[j];
          dot += cok ? go[j] * inter : 0.f;
          const float gi = wv[b] * go[j];
          dg[j] = gi * uv[j] * dact;
          du[j] = gi * act;
          ia[j] = wv[b] * inter;
        }
        // The row's 16 lanes (channels 8c .. 8c+7 each) sum their partial dots.
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) dot += __shfl_xor(dot, d, 64);
        if (m < m_end) {
          if (c == 0) part[m] = dot;
          if (cok) {
            if (ggu) {
              T* r = ggu + (size_t)m * 2 * a.I + ch;
              v2::st_stream(v2::pack8<T>(dg), r);
              v2::st_stream(v2::pack8<T>(du), r + a.I);
            }
            if (iw) v2::st_stream(v2::pack8<T>(ia), iw + (size_t)m * a.I + ch);
          }
        }
      }
    }
  } else {  // EPI_GLU_BWD
    const int code = a.act_codes ? a.act_codes[e] : 0;
    const int c = lane & 15;
    const int ch = rt * v2::TILE + wr * v2::WT + 8 * c;
    const int chc = min(ch, a.I - 8);
    const T* gu = (const T*)a.aux;
    T* ggu = (T*)a.out;
    T* gi = (T*)a.out2;
    constexpr int NB = 8;  // rows per batch of loads
#pragma unroll 1
    for (int i0 = 0; i0 < WQ / 4; i0 += NB) {
      i32x4 gq[NB], uq[NB];
      if (ggu) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int m = min(row0 + (i0 + b) * 4 + (lane >> 4), m_end - 1);
          const T* r = gu + (size_t)m * 2 * a.I + chc;
          gq[b] = *(const i32x4*)r;
          uq[b] = *(const i32x4*)(r + a.I);
        }
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int q = (i0 + b) * 4 + (lane >> 4);
        const int m = row0 + q;
        const i32x4 oq = v2::staged(wl, q, c);
        if (m < m_end && ch < a.I) {
          if (gi) v2::st_stream(oq, gi + (size_t)m * a.I + ch);
          if (ggu) {
            float go[8], gv[8], uv[8], dg[8], du[8];
            v2::unpack8<T>(oq, go);
            v2::unpack8<T>(gq[b], gv);
            v2::unpack8<T>(uq[b], uv);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              float act, dact;
              glu_act_dact(code, gv[j], act, dact);
              dg[j] = go[j] * uv[j] * dact;
              du[j] = go[j] * act;
            }
            T* r = ggu + (size_t)m * 2 * a.I + ch;
            v2::st_stream(v2::pack8<T>(dg), r);
            v2::st_stream(v2::pack8<T>(du), r + a.I);
          }
        }
      }
    }
  }
}

// Weight-gradient epilogue of the 256x256 kernel: out[e, c, r], c = MFMA column, r contiguous.
// WQ = output rows c per wave; the wave holds r = wr*128..+127.
template <typename T, int WQ = 32 * v2::TN, class Acc>
__device__ __forceinline__ void wgrad_epilogue_v2(const Acc& acc, const WgradArgs& a, int e, int r0,
                                                  int c0, char* smem, int wr, int wc) {
  const int w = threadIdx.x >> 6;
  char* wl = smem + w * (WQ * v2::EPI_ROWB);
  v2::stage_acc<T>(acc, wl);
  __syncthreads();
  v2::store_staged<T, WQ>(wl, (T*)a.out + (size_t)e * a.C * a.R, a.R, c0 + wc * WQ, a.C,
                          r0 + wr * v2::WT, a.R);
}

// MFMA tile shape of the 16-bit ring kernels: 16x16x32 (8 x 4 tiles of f32x4 per wave) or
// 32x32x16 (4 x 2 tiles of f32x16). Measured on the config-3 GEMMs, the token GEMMs run 3-6%
// faster on 16x16x32 tiles (same LDS and operand traffic, half the accumulator register traffic
// per FLOP), the weight gradients (both operands read transposed) 3-7% slower.
template <class AccV, int TI_, int TJ_, int FR_, class Kc_>
struct V4Shape {
  using Acc = AccV;
  using Kc = Kc_;
  static constexpr int TI = TI_, TJ = TJ_, FR = FR_;
  __device__ __forceinline__ static void zero(Acc (&acc)[TI][TJ]) {
#pragma unroll
    for (int ti = 0; ti < TI; ++ti)
#pragma unroll
      for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
        for (int v = 0; v < (int)(sizeof(Acc) / sizeof(float)); ++v) acc[ti][tj][v] = 0.f;
  }
};
using V4Sh16 = V4Shape<f32x4, v4::TI16, v4::TJ16, 16, v4::KcLoad16>;
using V4Sh32 = V4Shape<f32x16, v4::TI, v4::TJ, 32, v4::KcLoad>;

// K-split handoff between the S pieces of one output tile (slots slot0 .. slot0 + S - 1 of the
// split workspace, one arrival counter). Every piece stores its fp32 partial accumulators with
// device-coherent stores (agent-scope relaxed atomic stores: written through the XCD's L2), waits
// for them and counts itself in with a device-scope atomic; the last to arrive reads every
// piece's partials with device-coherent loads (they miss the XCD's L2), sums them in piece order
// (the same result whichever piece arrives last), clears the counter and returns true. No L2
// write-back or invalidate fence: an agent-scope release / acquire fence writes back or drops the
// whole L2 of the XCD, and with it the operands the XCD's other workgroups are streaming
// (measured: a weight gradient split 2-way ran 2.2x slower with them). Each store and load
// instruction of a wave covers 256 contiguous bytes.
// TWO: the caller always splits in exactly two pieces; the last piece then adds the other's
// partials to its own accumulators (p0 + p1 = p1 + p0 exactly, the same sum in either arrival
// order) instead of re-reading both, which keeps the sum within the register budget.
template <bool TWO = false, class AccV, int TI_, int TJ_>
__device__ __forceinline__ bool split_handoff(AccV (&acc)[TI_][TJ_], float* ws, int* cnt,
                                              int slot0, int piece, int S, char* smem) {
  constexpr int VL = (int)(sizeof(AccV) / sizeof(float));
  constexpr int NV = TI_ * TJ_;
  constexpr int SLOT = NV * VL * v4::NT;
  static_assert(SLOT == 65536, "one 256 KB slot per piece");
  const int tid = (int)threadIdx.x;
  // Within a slot: [wave][element][lane], so consecutive elements of a thread are 256 bytes apart
  // (16 of them reachable from one address register with the instruction's immediate offset).
  const int toff = (tid >> 6) * (NV * VL * 64) + (tid & 63);
  float* mine = ws + (size_t)(slot0 + piece) * SLOT + toff;
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int i = 0; i < VL; ++i)
      __hip_atomic_store(mine + (v * VL + i) * 64, acc[v / TJ_][v % TJ_][i], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  int* s_flag = (int*)smem;  // the ring is drained and idle between the K loop and the epilogue
  if (tid == 0)
    *s_flag = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const bool last = *s_flag == S - 1;
  __syncthreads();  // every wave has read the flag before the epilogue reuses the LDS
  if (!last) return false;
  if constexpr (TWO) {
    const float* src = ws + (size_t)(slot0 + (piece ^ 1)) * SLOT + toff;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
      for (int i = 0; i < VL; ++i)
        acc[v / TJ_][v % TJ_][i] += __hip_atomic_load(src + (v * VL + i) * 64, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
      // Groups of 32 loads: the sums of the group are complete at the empty asm that "modifies"
      // its vectors, so the loads of later groups cannot be hoisted above it and pile up in
      // registers (hoisted all together they spilled).
      if ((v + 1) * VL % 32 == 0 || v + 1 == NV) {
        asm volatile("" : "+v"(acc[v / TJ_][v % TJ_]));
        if (v > 0) asm volatile("" : "+v"(acc[(v - 1) / TJ_][(v - 1) % TJ_]));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
  }
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int i = 0; i < VL; ++i) acc[v / TJ_][v % TJ_][i] = 0.f;
  for (int q = 0; q < S; ++q) {
    const float* src = ws + (size_t)(slot0 + q) * SLOT + toff;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
      for (int i = 0; i < VL; ++i)
        acc[v / TJ_][v % TJ_][i] += __hip_atomic_load(src + (v * VL + i) * 64, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// Phase timestamps for experiments (built only with -DMOE_PHASE_TRACE): per workgroup, the
// 100 MHz wall clock at kernel start, K-loop start, K-loop end and epilogue end.
#ifdef MOE_PHASE_TRACE
__device__ unsigned long long g_phase[16 * 65536 * 4];
#define MOE_PHASE(slot, i)                                                                   \
  do {                                                                                       \
    if (threadIdx.x == 0) g_phase[((size_t)(slot) * 65536 + blockIdx.x) * 4 + (i)] = wall_clock64(); \
  } while (0)
#else
#define MOE_PHASE(slot, i) do {} while (0)
#endif

// Token GEMMs on the eight-wave ring kernel of moe_gemm_v4.h. The token side Q is K-contiguous
// (gathered or sorted rows); the weights P are K-contiguous in the forward and row-contiguous
// (P_RC) in the dX GEMMs.
template <typename T, int EPI, bool P_RC>
__global__ void __launch_bounds__(v4::NT, 1)
token_gemm_v4_kernel(TokenArgs a) {
  using C = V2Cfg<T>;
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  constexpr int PH = EPI * 2 + (P_RC ? 1 : 0);
  MOE_PHASE(PH, 0);
  // The expert tile scan borrows the last ring slot (free until the K loop's prologue).
  int* s_pref = (int*)(smem + (v4::NSLOT - 1) * v4::SLOTB);
  tile_prefix<v4::NT>(a.offsets, a.E_glu, v4::TILE, s_pref, s_pref + MAX_GLU_EXPERTS + 1);
  // Block -> tile as v4::block_tile. With a split workspace (plain-store GEMMs, K of at least
  // SPLIT_MIN_STEPS steps), each XCD's last partial wave -- rem tiles for its xcd_cus slots -- is
  // cut along K into S pieces per tile, all on that XCD.
  const int nk = a.K / 64;
  int mt, rt, piece = 0, S = 1, slot0 = 0;
  {
    const int n_mt = s_pref[a.E_glu];
    const int gm = v4::tile_group(a.n_rtiles);
    const int n_idx = (n_mt + gm - 1) / gm * gm * a.n_rtiles;
    const int x = (int)blockIdx.x & 7, bi = (int)blockIdx.x >> 3;
    const int R = (n_idx + 7) >> 3;
    const int t_lo = x * R, t_cnt = max(0, min(n_idx, t_lo + R) - t_lo);
    const int cus = a.xcd_cus;
    const bool split = EPI == EPI_STORE && a.split_ws && nk >= v4::SPLIT_MIN_STEPS;
    const int full = split ? t_cnt / cus * cus : t_cnt;
    const int rem = t_cnt - full;
    S = rem > 0 ? min(min(cus / rem, nk / 8), v4::SPLIT_MAX) : 1;
    int lid;
    if (bi < full || S <= 1) {
      if (bi >= t_cnt) return;
      lid = t_lo + bi;
      S = 1;
    } else {
      const int j = bi - full;
      if (j >= rem * S) return;
      lid = t_lo + full + j / S;
      piece = j % S;
      slot0 = x * cus + (j / S) * S;
    }
    v4::tile_of(lid, a.n_rtiles, mt, rt);
    if (mt >= n_mt) return;
  }
  const int kb = piece * nk / S * 64, ke = (piece + 1) * nk / S * 64;
  int lo = 0, hi = a.E_glu - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_pref[mid] <= mt) lo = mid; else hi = mid - 1;
  }
  const int e = lo;
  const int m0 = a.offsets[e] + (mt - s_pref[e]) * v4::TILE;
  const int m_end = a.offsets[e + 1];
  const T* Pe = (const T*)a.P + (size_t)e * a.p_e;
  const int wr = v4::wave_r(), wc = v4::wave_c();
  // Waves whose 64 token rows all lie past the group end (tail tiles) skip their MFMAs.
  const bool wave_rows = m0 + wc * v4::WQ < m_end;

  // Gate of this lane's token row (gated backward; weighted forward intermediate), needed only by
  // the epilogue, loaded with the token-row indices below. sflat null: the gates are already in
  // sorted-row order (one load); else indexed through sflat (two dependent loads).
  // The load is unconditional (a readable dummy address without gates) and its value is first
  // touched after the K loop, so nothing waits for it before then.
  constexpr bool WGATE = EPI == EPI_GLU_BWD_GATED || EPI == EPI_GLU_FWD;
  unsigned short wbits = 0;
  if constexpr (WGATE) {
    const int m = min(m0 + wc * v4::WQ + v4::lane_id(), m_end - 1);
    const unsigned short* gp = (const unsigned short*)a.offsets;
    if (a.gate) gp = (const unsigned short*)a.gate + (a.sflat ? a.sflat[m] : m);
    wbits = *gp;
  }
  // Token rows past the group end read row m0 (their results are never stored).
  typename V4Sh16::Kc lq;
  lq.init(wc * v4::WQ);
#pragma unroll
  for (int i = 0; i < v4::LOADS; ++i) {
    int m = m0 + v4::KcLoad::row_of(i);
    if (m >= m_end) m = m0;
    const int qr = a.q_gather ? a.q_gather[m] : m;
    lq.rowp[i] = (const char*)((const T*)a.Q + (size_t)qr * a.q_ld);
  }

  typename V4Sh16::Acc acc[V4Sh16::TI][V4Sh16::TJ];
  V4Sh16::zero(acc);

  if constexpr (P_RC) {
    v4::RcLoad<false, V4Sh16::TI, V4Sh16::FR> lp;
    const int r0 = rt * v4::TILE;
    lp.src = (const char*)(Pe + r0);
    lp.ld = (size_t)a.p_ld * sizeof(T);
    lp.gather = nullptr;
    lp.kend = a.K;
    lp.init(wr * v4::WP, a.R - r0);
    v4::bare_barrier();  // s_pref is read; the LDS now belongs to the K loop (LDS-only)
    MOE_PHASE(PH, 1);
    if (wave_rows) v4::mainloop_ring<T, true>(acc, lp, lq, kb, ke, smem);
    else v4::mainloop_ring<T, false>(acc, lp, lq, kb, ke, smem);
  } else {
    typename V4Sh16::Kc lp;
    lp.init(wr * v4::WP);
#pragma unroll
    for (int i = 0; i < v4::LOADS; ++i) {
      const int rr = v4::KcLoad::row_of(i);
      bool ok;
      int prow;
      if (EPI == EPI_GLU_FWD) {
        prow = glu_prow<C>(rr, rt, a.I, ok);
      } else {
        prow = rt * v4::TILE + rr;
        ok = prow < a.R;
      }
      lp.rowp[i] = (const char*)(Pe + (size_t)(ok ? prow : 0) * a.p_ld);
    }
    v4::bare_barrier();  // s_pref is read; the LDS now belongs to the K loop (LDS-only)
    MOE_PHASE(PH, 1);
    if (wave_rows) v4::mainloop_ring<T, true>(acc, lp, lq, kb, ke, smem);
    else v4::mainloop_ring<T, false>(acc, lp, lq, kb, ke, smem);
  }
  MOE_PHASE(PH, 2);
  if (S > 1) {
    // Split piece: the last piece to arrive sums all pieces' partials and runs the epilogue;
    // nothing waits on another workgroup.
    if (!split_handoff(acc, a.split_ws, a.split_cnt + slot0, slot0, piece, S, smem)) return;
  }
  float wrow = 1.f;
  if constexpr (WGATE) {
    if (a.gate) wrow = to_f32(__builtin_bit_cast(T, wbits));
  }
  token_epilogue_v2<T, EPI, v4::WQ>(acc, a, e, m0, m_end, rt, smem, wr, wc, wrow);
#ifdef MOE_PHASE_TRACE
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
#endif
  MOE_PHASE(PH, 3);
}

// ---------------------------------------------------------------------------------------------
// Persistent token GEMMs (no K split). One workgroup per CU slot of an XCD runs the XCD's logical
// tiles bi, bi + n_wg, bi + 2 n_wg, ... (the same tiles the XCD's CUs ran at once in the
// one-tile-per-workgroup kernel above, so the L2 sharing is unchanged). That kernel spends ~2.5 us
// per tile on set-up (the expert tile scan and its barrier, token-row indices) before the ring's
// first loads; here the next tile's expert comes from a scalar walk over the offsets (no barrier,
// no vector memory access) and only its token-row indices are loaded. The epilogue stages 16
// token rows at a time through ring slot 0 (4 KB per wave); each tile's ring starts at slot 1.
// Measured on config 3: gate/up forward -4.7%, down forward -4.3%, gated down dX -1.4%, gate/up
// dX -1%.
// 0, opaque to the optimiser (kept in an SGPR).
__device__ __forceinline__ int opaque_zero() {
  int z = 0;
  asm volatile("" : "+s"(z));
  return z;
}

namespace v5 {
constexpr int BASE = 1;            // ring slot of each tile's P0
constexpr int STAGE_B = 4096;      // per-wave staging: 16 rows x 256 bytes
static_assert(v4::NW * STAGE_B == v4::SLOTB, "the staging of all waves is ring slot 0");

struct Tile {
  int e, m0, m_end, rt;
};

// Accumulator rows tj*16 .. tj*16+15 of the wave (16x16 MFMA tiles: lane l holds channels
// ti*16 + 4(l/16) + v of row l%16) to the wave's staging block, rounded to T.
template <typename T, int TI_, int TJ_>
__device__ __forceinline__ void stage_rows(const f32x4 (&acc)[TI_][TJ_], int tj, char* wl) {
  const int lane = v4::lane_id(), h = (lane >> 4) & 1, g = lane >> 5;
  const int q = lane & 15;
#pragma unroll
  for (int ti = 0; ti < TI_; ++ti) {
    uint2 v = {v2::pack2<T>(acc[ti][tj][0], acc[ti][tj][1]),
               v2::pack2<T>(acc[ti][tj][2], acc[ti][tj][3])};
    *(uint2*)(wl + v2::staged_off(q, 2 * ti + g) + 8 * h) = v;
  }
}

// Epilogue of one tile: the token_epilogue_v2 operations, 16 rows per pass through the wave's
// staging block.
template <typename T, int EPI, class Acc>
__device__ __forceinline__ void epilogue(const Acc& acc, const TokenArgs& a, const Tile& t,
                                         char* wl, int wr, int wc, float wrow) {
  const int lane = v4::lane_id();
  const int row0 = t.m0 + wc * v4::WQ;
  const bool rows = row0 < t.m_end;  // false: this wave's token rows all lie past the group end
  const int code = (EPI != EPI_STORE && a.act_codes) ? a.act_codes[t.e] : 0;
  static_for<0, V4Sh16::TJ>([&](auto tjc) {
    constexpr int TJ = decltype(tjc)::value;
    const bool live = rows && row0 + TJ * 16 < t.m_end;
    if constexpr (EPI == EPI_STORE) {
      if (!live) return;
      stage_rows<T>(acc, TJ, wl);
      const int c = lane & 15;
      const int ch = t.rt * v4::TILE + wr * v2::WT + 8 * c;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int q = it * 4 + (lane >> 4);
        const int m = row0 + TJ * 16 + q;
        const i32x4 v = v2::staged(wl, q, c);
        if (m < t.m_end && ch < a.R) v2::st_stream(v, (T*)a.out + (size_t)m * a.out_ld + ch);
      }
    } else if constexpr (EPI == EPI_GLU_FWD) {
      if (!live) return;
      stage_rows<T>(acc, TJ, wl);
      const int c = lane & 7;
      const int ch = t.rt * (v2::TILE / 2) + wr * (v2::WT / 2) + 8 * c;
      T* gu = (T*)a.out;
      T* it = (T*)a.out2;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int q = i * 8 + (lane >> 3);
        const int m = row0 + TJ * 16 + q;
        const i32x4 gq = v2::staged(wl, q, c), uq = v2::staged(wl, q, c + 8);
        const float w = __shfl(wrow, TJ * 16 + q, 64);  // every lane active
        if (m < t.m_end && ch < a.I) {
          T* r = gu + (size_t)m * 2 * a.I + ch;
          v2::st_stream(gq, r);
          v2::st_stream(uq, r + a.I);
          if (it) {
            float gv[8], uv[8], iv[8];
            v2::unpack8<T>(gq, gv);
            v2::unpack8<T>(uq, uv);
#pragma unroll
            for (int j = 0; j < 8; ++j) iv[j] = w * (glu_act(code, gv[j]) * uv[j]);
            v2::st_stream(v2::pack8<T>(iv), it + (size_t)m * a.I + ch);
          }
        }
      }
    } else if constexpr (EPI == EPI_GLU_BWD_GATED) {
      if (!live) return;
      stage_rows<T>(acc, TJ, wl);
      const int c = lane & 15;
      const int ch = t.rt * v2::TILE + wr * v2::WT + 8 * c;
      const int chc = min(ch, a.I - 8);
      const bool cok = ch < a.I;
      const T* gu = (const T*)a.aux;
      T* ggu = (T*)a.out;
      T* iw = (T*)a.out2;
      float* part = a.part + (size_t)(2 * t.rt + wr) * a.out_ld;
      i32x4 gq[4], uq[4];
      float wv[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int q = b * 4 + (lane >> 4);
        const int m = min(row0 + TJ * 16 + q, t.m_end - 1);
        const T* r = gu + (size_t)m * 2 * a.I + chc;
        gq[b] = *(const i32x4*)r;
        uq[b] = *(const i32x4*)(r + a.I);
        wv[b] = __shfl(wrow, TJ * 16 + q, 64);
      }
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int q = b * 4 + (lane >> 4);
        const int m = row0 + TJ * 16 + q;
        const i32x4 oq = v2::staged(wl, q, c);
        float go[8], gv[8], uv[8], dg[8], du[8], ia[8];
        v2::unpack8<T>(oq, go);
        v2::unpack8<T>(gq[b], gv);
        v2::unpack8<T>(uq[b], uv);
        float dot = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float act, dact;
          glu_act_dact(code, gv[j], act, dact);
          const float inter = act * uv[j];
          dot += cok ? go[j] * inter : 0.f;
          const float gi = wv[b] * go[j];
          dg[j] = gi * uv[j] * dact;
          du[j] = gi * act;
          ia[j] = wv[b] * inter;
        }
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) dot += __shfl_xor(dot, d, 64);
        if (m < t.m_end) {
          if (c == 0) part[m] = dot;
          if (cok) {
            if (ggu) {
              T* r = ggu + (size_t)m * 2 * a.I + ch;
              v2::st_stream(v2::pack8<T>(dg), r);
              v2::st_stream(v2::pack8<T>(du), r + a.I);
            }
            if (iw) v2::st_stream(v2::pack8<T>(ia), iw + (size_t)m * a.I + ch);
          }
        }
      }
    }
  });
}
}  // namespace v5

template <typename T, int EPI, bool P_RC>
__global__ void __launch_bounds__(v4::NT, 1)
token_gemm_v5_kernel(TokenArgs a) {
  using C = V2Cfg<T>;
  using LQ = typename V4Sh16::Kc;
  using LP = std::conditional_t<P_RC, v4::RcLoad<false, V4Sh16::TI, V4Sh16::FR>, typename V4Sh16::Kc>;
  constexpr bool WGATE = EPI == EPI_GLU_BWD_GATED || EPI == EPI_GLU_FWD;
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  v4::Experts ex;
  ex.init(a.offsets, a.E_glu);
  const int gm = v4::tile_group(a.n_rtiles);
  const int n_idx = (ex.n_mt + gm - 1) / gm * gm * a.n_rtiles;
  const int x = (int)blockIdx.x & 7, bi = (int)blockIdx.x >> 3, nwg = (int)gridDim.x >> 3;
  const int R = (n_idx + 7) >> 3;
  const int t_lo = x * R, t_cnt = max(0, min(n_idx, t_lo + R) - t_lo);
  const int wr = v4::wave_r(), wc = v4::wave_c();

  // First valid logical tile at local index j or later (stride nwg); t_cnt if none.
  auto find = [&](int j, v5::Tile& t) {
    for (; j < t_cnt; j += nwg) {
      int mt, rt;
      v4::tile_of(t_lo + j, a.n_rtiles, mt, rt);
      if (mt < ex.n_mt) {
        ex.lookup(mt, t.e, t.m0, t.m_end);
        t.rt = rt;
        return j;
      }
    }
    return t_cnt;
  };
  // Operand row pointers (and the gate of this lane's token row) of tile t.
  auto setup = [&](const v5::Tile& t, LP& lp, LQ& lq, unsigned short& wbits) {
    const T* Pe = (const T*)a.P + (size_t)t.e * a.p_e;
    if constexpr (WGATE) {
      const int m = min(t.m0 + wc * v4::WQ + v4::lane_id(), t.m_end - 1);
      const unsigned short* gp = (const unsigned short*)a.offsets;
      if (a.gate) gp = (const unsigned short*)a.gate + (a.sflat ? a.sflat[m] : m);
      wbits = *gp;
    }
    // (The loaders' lane constants are set once, before the tile loop: recomputed per tile they
    // were kept twice and spilled.)
#pragma unroll
    for (int i = 0; i < v4::LOADS; ++i) {
      int m = t.m0 + v4::KcLoad::row_of(i);
      if (m >= t.m_end) m = t.m0;
      // The plain-store GEMMs read sorted rows (no gather; checked at launch): no index load,
      // whose wait would also wait for the previous tile's epilogue stores.
      const int qr = (EPI != EPI_STORE && a.q_gather) ? a.q_gather[m] : m;
      lq.rowp[i] = (const char*)((const T*)a.Q + (size_t)qr * a.q_ld);
    }
    if constexpr (P_RC) {
      const int r0 = t.rt * v4::TILE;
      lp.src = (const char*)(Pe + r0);
      lp.set_rvalid(a.R - r0);
    } else {
#pragma unroll
      for (int i = 0; i < v4::LOADS; ++i) {
        const int rr = v4::KcLoad::row_of(i);
        bool ok;
        int prow;
        if (EPI == EPI_GLU_FWD) {
          prow = glu_prow<C>(rr, t.rt, a.I, ok);
        } else {
          prow = t.rt * v4::TILE + rr;
          ok = prow < a.R;
        }
        lp.rowp[i] = (const char*)(Pe + (size_t)(ok ? prow : 0) * a.p_ld);
      }
    }
  };

  v5::Tile cur;
  int j = find(bi, cur);
  if (j >= t_cnt) return;
  LP lp;
  LQ lq;
  lq.init(wc * v4::WQ);
  if constexpr (P_RC) {
    lp.ld = (size_t)a.p_ld * sizeof(T);
    lp.gather = nullptr;
    lp.kend = a.K;
    lp.init(wr * v4::WP, a.R);
  } else {
    lp.init(wr * v4::WP);
  }
  unsigned short wbits = 0;
  setup(cur, lp, lq, wbits);
  v4::ring_prologue<T>(lp, lq, opaque_zero(), a.K, smem, v5::BASE, 0, v4::NSLOT - 1);
  char* wl = smem + (threadIdx.x >> 6) * v5::STAGE_B;  // staging: ring slot 0
#ifdef MOE_PHASE_TRACE
  constexpr int PH = 8 + EPI * 2 + (P_RC ? 1 : 0);
  int n_tile = 0;
#define MOE_PHASE5(i)                                                                         \
  do {                                                                                        \
    if (threadIdx.x == 0 && n_tile < 64)                                                      \
      g_phase[((size_t)PH * 65536 + blockIdx.x * 64 + n_tile) * 4 + (i)] = wall_clock64();     \
  } while (0)
#else
#define MOE_PHASE5(i) do {} while (0)
#endif
  while (true) {
    MOE_PHASE5(0);
    // K starts at 0 for every tile, but as a value the compiler cannot see: otherwise it computes
    // the prologue's row and address terms once, keeps them live across the tile loop and spills
    // them, and each reload's wait then drains the ring loads already in flight.
    const int kz = opaque_zero();
    v4::ring_prologue<T>(lp, lq, kz, a.K, smem, v5::BASE, v4::NSLOT - 1, 1);  // P2 -> slot 0
    typename V4Sh16::Acc acc[V4Sh16::TI][V4Sh16::TJ];
    V4Sh16::zero(acc);
    if (cur.m0 + wc * v4::WQ < cur.m_end)
      v4::mainloop_ring<T, true, true>(acc, lp, lq, kz, a.K, smem, v5::BASE);
    else
      v4::mainloop_ring<T, false, true>(acc, lp, lq, kz, a.K, smem, v5::BASE);
    // The ring is drained and every wave is past its last read: slots 1-4 take the next tile's
    // first loads while this tile's epilogue stages through slot 0.
    MOE_PHASE5(1);
    v5::Tile nxt;
    const int jn = find(j + nwg, nxt);
    float wrow = 1.f;
    if constexpr (WGATE) {
      if (a.gate) wrow = to_f32(__builtin_bit_cast(T, wbits));
    }
#ifdef MOE_PHASE_TRACE
    if (threadIdx.x == 0 && n_tile < 64)  // slot 2: the tile's valid token rows
      g_phase[((size_t)PH * 65536 + blockIdx.x * 64 + n_tile) * 4 + 2] =
          (unsigned long long)min(cur.m_end - cur.m0, v4::TILE);
#endif
    v5::epilogue<T, EPI>(acc, a, cur, wl, wr, wc, wrow);
#ifdef MOE_PHASE_TRACE
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#endif
    MOE_PHASE5(3);
#ifdef MOE_PHASE_TRACE
    ++n_tile;
#endif
    // The next tile's set-up and first ring loads (slots 1-4; nobody reads the ring between K
    // loops), then the barrier that frees the staging slot for P2. Measured on config 3, issuing
    // these loads during the epilogue instead gained nothing on the plain-store and forward
    // epilogues and cost the gated one (its gate_up loads then wait behind them). The set-up runs
    // for the last tile too (on valid, unused values): unconditional, it keeps the register
    // allocation free of spills.
    setup(jn < t_cnt ? nxt : cur, lp, lq, wbits);
    if (jn < t_cnt) v4::ring_prologue<T>(lp, lq, opaque_zero(), a.K, smem, v5::BASE, 0, v4::NSLOT - 1);
    if (jn >= t_cnt) break;
    v4::bare_barrier();  // every wave is done with slot 0 before P2 lands in it
    cur = nxt;
    j = jn;
  }
}

// Weight gradients on the eight-wave ring kernel: out[e, c, r] = sum over expert e's sorted rows m
// of rsrc[rrow(m), r] * csrc[crow(m), c]; both operands row-contiguous (optionally gathered rows).
template <typename T, bool RG, bool CG, bool SPLIT>
__global__ void __launch_bounds__(v4::NT, 1)
wgrad_v4_kernel(WgradArgs a, const int32_t* order, int E_glu, int n_logical, int xr, int xc) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  constexpr int PH = 4 + (RG ? 2 : 0) + (CG ? 1 : 0);
  MOE_PHASE(PH, 0);
  // `order` puts the largest experts first and each expert's tiles are spread over all 8 XCDs
  // (workgroups are dealt to XCDs round-robin, so tile j of an expert runs on XCD j % 8 when the
  // tile count is a multiple of 8). With xr > 0 the r x c tile grid is cut into 8 rectangles of
  // xr x xc tiles and XCD x takes rectangle x, so the tiles sharing one L2 read xr r-slices and
  // xc c-slices; otherwise tiles sharing an XCD share their r-slice (rt fastest).
  // SPLIT: a separate instantiation, so the unsplit kernel's code is the same as without it.
  const int piece = SPLIT ? (int)blockIdx.x / a.Lp : 0;
  const int lid = SPLIT ? (int)blockIdx.x % a.Lp : (int)blockIdx.x;
  if (lid >= n_logical) return;
  const int per_e = a.n_rtiles * a.n_ctiles;
  const int ei = lid / per_e, rem = lid % per_e;
  const int e = order ? order[ei] : ei;
  if (e < 0 || e >= E_glu) return;  // weightless special expert
  int ct, rt;
  if (xr > 0) {
    const int x = rem & 7, i = rem >> 3;              // XCD, index within its rectangle
    const int nrx = a.n_rtiles / xr;                  // rectangles along r
    rt = (x % nrx) * xr + i % xr;
    ct = (x / nrx) * xc + i / xr;
  } else {
    ct = rem / a.n_rtiles;
    rt = rem % a.n_rtiles;
  }
  int k0 = a.offsets[e], k1 = a.offsets[e + 1];
  if constexpr (SPLIT) {
    // Piece `piece` of the expert's rows: whole 64-row K steps, the last piece takes the rest;
    // pieces past the end are empty (they add zero partials).
    const int len = ((k1 - k0 + a.S - 1) / a.S + 63) & ~63;
    const int kb = min(k1, k0 + piece * len);
    k1 = min(k1, kb + len);
    k0 = kb;
  }
  const int r0 = rt * v4::TILE, c0 = ct * v4::TILE;
  const int wr = v4::wave_r(), wc = v4::wave_c();

  // kend = the piece's end: K rows at or past it read zeros (the next piece's rows are not added).
  v4::RcLoad<RG, V4Sh32::TI, V4Sh32::FR> lp;
  lp.src = (const char*)((const T*)a.rsrc + r0);
  lp.ld = (size_t)a.r_ld * sizeof(T);
  lp.gather = a.r_gather;
  lp.kend = k1;
  lp.init(wr * v4::WP, a.R - r0);
  v4::RcLoad<CG, V4Sh32::TJ, V4Sh32::FR> lq;
  lq.src = (const char*)((const T*)a.csrc + c0);
  lq.ld = (size_t)a.c_ld * sizeof(T);
  lq.gather = a.c_gather;
  lq.kend = k1;
  lq.init(wc * v4::WQ, a.C - c0);

  typename V4Sh32::Acc acc[V4Sh32::TI][V4Sh32::TJ];
  V4Sh32::zero(acc);
  MOE_PHASE(PH, 1);
  v4::mainloop_ring<T>(acc, lp, lq, k0, k1, smem);
  MOE_PHASE(PH, 2);
  if constexpr (SPLIT) {
    // Split piece: the last piece of the tile to arrive sums the partials and runs the epilogue.
    // The launch sets a.S = 2 whenever it picks this instantiation (launch_wgrad_v2), which the
    // two-piece handoff relies on.
    const int tile = e * per_e + rem;  // < E_glu * per_e, checked at launch against the slots
    if (!split_handoff<true>(acc, a.split_ws, a.split_cnt + tile, tile * 2, piece, 2, smem)) return;
  }
  wgrad_epilogue_v2<T, v4::WQ>(acc, a, e, r0, c0, smem, wr, wc);
#ifdef MOE_PHASE_TRACE
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#endif
  MOE_PHASE(PH, 3);
}

// dX GEMMs (weights row-contiguous): the five-stage pipeline of moe_gemm_v3.h.
template <typename T, int EPI, bool P_RC>
__global__ void __launch_bounds__(v3::NT, 1)
token_gemm_v3_kernel(TokenArgs a) {
  using C = V2Cfg<T>;
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  // The expert tile scan borrows the last LDS stage (free until the K loop's prologue).
  int* s_pref = (int*)(smem + (v3::NSTAGE - 1) * v3::STAGEB);
  tile_prefix<v3::NT>(a.offsets, a.E_glu, v3::TILE, s_pref, s_pref + MAX_GLU_EXPERTS + 1);
  int mt, rt;
  if (!v4::block_tile(s_pref[a.E_glu], a.n_rtiles, mt, rt)) return;
  int lo = 0, hi = a.E_glu - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_pref[mid] <= mt) lo = mid; else hi = mid - 1;
  }
  const int e = lo;
  const int m0 = a.offsets[e] + (mt - s_pref[e]) * v3::TILE;
  const int m_end = a.offsets[e + 1];
  const T* Pe = (const T*)a.P + (size_t)e * a.p_e;
  const int w = (int)threadIdx.x >> 6, wr = w >> 1, wc = w & 1;

  // Token rows past the group end read row m0 (their results are never stored).
  v3::KcDma lq;
  lq.init(wc * v3::WT);
#pragma unroll
  for (int i = 0; i < v3::LOADS; ++i) {
    int m = m0 + v3::KcDma::row_of(i);
    if (m >= m_end) m = m0;
    const int qr = a.q_gather ? a.q_gather[m] : m;
    lq.rowp[i] = (const char*)((const T*)a.Q + (size_t)qr * a.q_ld);
  }

  f32x16 acc[v3::TN][v3::TN];
#pragma unroll
  for (int ti = 0; ti < v3::TN; ++ti)
#pragma unroll
    for (int tj = 0; tj < v3::TN; ++tj)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[ti][tj][v] = 0.f;
  __syncthreads();  // s_pref is read; the LDS now belongs to the K loop

  if constexpr (P_RC) {
    v3::RcDma<false> lp;
    const int r0 = rt * v3::TILE;
    lp.src = (const char*)(Pe + r0);
    lp.ld = (size_t)a.p_ld * sizeof(T);
    lp.gather = nullptr;
    lp.kend = a.K;
    lp.init(wr * v3::WT, a.R - r0);
    v3::mainloop<T>(acc, lp, lq, 0, a.K, smem);
  } else {
    v3::KcDma lp;
    lp.init(wr * v3::WT);
#pragma unroll
    for (int i = 0; i < v3::LOADS; ++i) {
      const int rr = v3::KcDma::row_of(i);
      bool ok;
      int prow;
      if (EPI == EPI_GLU_FWD) {
        prow = glu_prow<C>(rr, rt, a.I, ok);
      } else {
        prow = rt * v3::TILE + rr;
        ok = prow < a.R;
      }
      lp.rowp[i] = (const char*)(Pe + (size_t)(ok ? prow : 0) * a.p_ld);
    }
    v3::mainloop<T>(acc, lp, lq, 0, a.K, smem);
  }
  token_epilogue_v2<T, EPI>(acc, a, e, m0, m_end, rt, smem, (int)(threadIdx.x >> 7), (int)(threadIdx.x >> 6) & 1);
}

// ---------------------------------------------------------------------------------------------
// Host-side launch helpers.

template <typename T> using TokCfg = Cfg<T, 128, 128, 2, 2>;
template <typename T> using WgCfg = Cfg<T, 128, 128, 2, 2>;

template <class C, int EPI, bool P_RC>
static int launch_token(const TokenArgs& a, int64_t n_rows, hipStream_t s) {
  const int64_t max_mt = (n_rows + C::BC - 1) / C::BC + a.E_glu;
  const int64_t grid = max_mt * a.n_rtiles;
  if (grid <= 0 || n_rows == 0) return MOE_OK;
  if (grid >= (int64_t)1 << 31) return MOE_ERR_SHAPE;
  auto kern = token_gemm_kernel<C, EPI, P_RC>;
  (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS_BYTES);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(C::NT), C::LDS_BYTES, s, a);
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}

template <class C>
static int launch_wgrad(const WgradArgs& a, int E, hipStream_t s) {
  const int64_t grid = (int64_t)E * a.n_rtiles * a.n_ctiles;
  if (grid <= 0) return MOE_OK;
  if (grid >= (int64_t)1 << 31) return MOE_ERR_SHAPE;
  auto kern = wgrad_kernel<C>;
  (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS_BYTES);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(C::NT), C::LDS_BYTES, s, a);
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}


// CUs of the current device (cached per device ordinal; 0 on error).
static int device_cus() {
  static int cache[64];
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64 && cache[dev] > 0) return cache[dev];
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) cache[dev] = n;
  return n;
}

// 256x256 token GEMMs: the persistent ring kernel (any expert count, no K split), else the
// one-tile-per-workgroup ring kernel when K is a multiple of its 64-value step, otherwise (dX
// GEMMs with K a multiple of 32) the four-wave five-stage kernel.
template <typename T, int EPI, bool P_RC>
static int launch_token_v2(TokenArgs a, int64_t n_rows, hipStream_t s) {
  a.n_rtiles = EPI == EPI_GLU_FWD ? (int)((a.I + v2::TILE / 2 - 1) / (v2::TILE / 2))
                                  : (int)((a.R + v2::TILE - 1) / v2::TILE);
  const int64_t max_mt = (n_rows + v2::TILE - 1) / v2::TILE + a.E_glu;
  const int64_t logical = v4::logical_tiles(max_mt, a.n_rtiles);
  if (logical <= 0 || n_rows == 0) return MOE_OK;
#ifndef MOE_NO_PERSISTENT
  const bool split = EPI == EPI_STORE && a.split_ws && a.K / 64 >= v4::SPLIT_MIN_STEPS;
  const int cus = device_cus();
  if constexpr (EPI != EPI_GLU_BWD) {
  if (a.K % 64 == 0 && !split && cus >= 8 && (EPI != EPI_STORE || !a.q_gather)) {
    const int64_t per_xcd = (logical + 7) / 8;
    const int64_t grid = 8 * std::min<int64_t>(cus / 8, per_xcd);
    auto kern = token_gemm_v5_kernel<T, EPI, P_RC>;
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, v4::RING_LDSB);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(v4::NT), v4::RING_LDSB, s, a);
    return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
  }
  }
#endif
  int64_t grid = (logical + 7) / 8 * 8;
  if (a.split_ws && a.K % 64 == 0) grid += 8 * (int64_t)a.xcd_cus;  // the split pieces
  if (grid >= (int64_t)1 << 31) return MOE_ERR_SHAPE;
  if (a.K % 64 == 0) {
    auto kern = token_gemm_v4_kernel<T, EPI, P_RC>;
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, v4::RING_LDSB);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(v4::NT), v4::RING_LDSB, s, a);
  } else {
    if constexpr (P_RC && EPI != EPI_GLU_BWD_GATED) {  // the gated epilogue needs the v4 kernel
      auto kern = token_gemm_v3_kernel<T, EPI, P_RC>;
      (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, v3::LDSB);
      hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(v3::NT), v3::LDSB, s, a);
    } else {
      return MOE_ERR_SHAPE;  // callers route K % 64 != 0 forwards to the first-generation kernel
    }
  }
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}

// n_entries = length of `order` (every expert id, GLU or special) or E_glu without an order.
template <typename T>
static int launch_wgrad_v2(WgradArgs a, const int32_t* order, int n_entries, int E_glu, hipStream_t s) {
  a.n_rtiles = (a.R + v2::TILE - 1) / v2::TILE;
  a.n_ctiles = (a.C + v2::TILE - 1) / v2::TILE;
  const int64_t logical = (int64_t)n_entries * a.n_rtiles * a.n_ctiles;
  if (logical <= 0) return MOE_OK;
  const int64_t grid = (logical + 7) / 8 * 8;
  if (grid >= (int64_t)1 << 31) return MOE_ERR_SHAPE;
  // Per-XCD rectangles (see wgrad_v4_kernel): 8 equal rectangles of xr x xc tiles with the fewest
  // slices per rectangle (xr + xc); 0 = the r-slice mapping (grids that do not split into 8).
  int xr = 0, xc = 0;
  for (int nrx : {1, 2, 4, 8}) {  // rectangles along r; 8 / nrx along c
    const int ncx = 8 / nrx;
    if (a.n_rtiles % nrx == 0 && a.n_ctiles % ncx == 0) {
      const int r = a.n_rtiles / nrx, c = a.n_ctiles / ncx;
      if (xr == 0 || r + c < xr + xc) {
        xr = r;
        xc = c;
      }
    }
  }
  // K split in two when the expert tiles fill at most a quarter of the CUs (few experts and small
  // weights, e.g. E = 9, H = 512, I = 768: 54 down tiles); the partials fit the token GEMMs'
  // split workspace (one 256x256 fp32 slot per CU). Measured on that shape: down 72 -> 53 us
  // with 2 pieces, 72 us with 4; the 108-tile gate/up gradient 92 -> 111 us with 2 pieces (more
  // concurrent row streams than its L2 reuse absorbs), hence the quarter.
  a.S = 1;
  a.Lp = (int)grid;
  const int n_cus = device_cus();
  const int64_t glu_tiles = (int64_t)E_glu * a.n_rtiles * a.n_ctiles;
  if (a.split_ws && n_cus >= 8 && 4 * glu_tiles <= n_cus) a.S = 2;
  const int64_t grid_s = grid * a.S;
  auto pick = [&]<bool SPLIT>() {
    return a.r_gather ? (a.c_gather ? wgrad_v4_kernel<T, true, true, SPLIT> : wgrad_v4_kernel<T, true, false, SPLIT>)
                      : (a.c_gather ? wgrad_v4_kernel<T, false, true, SPLIT> : wgrad_v4_kernel<T, false, false, SPLIT>);
  };
  auto kern = a.S > 1 ? pick.template operator()<true>() : pick.template operator()<false>();
  (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, v4::RING_LDSB);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid_s), dim3(v4::NT), v4::RING_LDSB, s, a, order, E_glu,
                     (int)logical, xr, xc);
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

static int check_common(int dtype, int64_t H, int64_t I, int E_glu, int64_t n_rows) {
  if (dtype != MOE_DT_F32 && dtype != MOE_DT_F16 && dtype != MOE_DT_BF16) return MOE_ERR_DTYPE;
  if (H <= 0 || I <= 0 || E_glu <= 0 || E_glu > MAX_GLU_EXPERTS || n_rows < 0) return MOE_ERR_SHAPE;
  if (H >= (1 << 30) || I >= (1 << 29) || n_rows >= ((int64_t)1 << 31)) return MOE_ERR_SHAPE;
  if (H % 8 != 0 || I % 8 != 0) return MOE_ERR_ALIGN;
  return MOE_OK;
}

}  // namespace moe

using namespace moe;

#define MOE_DISPATCH_DTYPE(dtype, FN)                  \
  switch (dtype) {                                     \
    case MOE_DT_BF16: return FN<bf16>();               \
    case MOE_DT_F16: return FN<f16>();                 \
    case MOE_DT_F32: return FN<float>();               \
    default: return MOE_ERR_DTYPE;                     \
  }

extern "C" int moe_grouped_gateup_swiglu_fwd(int dtype, const void* hidden, int64_t n_tokens,
                                             int64_t H, const void* gate_up_proj, int E_glu,
                                             int64_t I, const int32_t* act_codes,
                                             const int32_t* offsets, const int32_t* tile_offsets,
                                             const int32_t* sorted_token, int64_t n_rows,
                                             void* gate_up_out, void* inter_out,
                                             const void* top_k_weights,
                                             const int32_t* sorted_flat, void* stream) {
  (void)tile_offsets;
  int st = check_common(dtype, H, I, E_glu, n_rows);
  if (st) return st;
  if (n_rows == 0) return MOE_OK;
  if (!hidden || !gate_up_proj || !offsets || !sorted_token || !gate_up_out || !act_codes)
    return MOE_ERR_SHAPE;
  // Gate-weighted intermediate: 16-bit operands, H a multiple of 64 (the ring kernel's epilogue).
  if (top_k_weights && (!inter_out || dtype == MOE_DT_F32 || H % 64 != 0)) return MOE_ERR_SHAPE;
  if (!aligned16(hidden) || !aligned16(gate_up_proj) || !aligned16(gate_up_out) ||
      (inter_out && !aligned16(inter_out)))
    return MOE_ERR_ALIGN;
  (void)n_tokens;
  TokenArgs a = {};
  a.P = gate_up_proj; a.p_e = 2 * I * H; a.p_ld = H; a.R = (int)(2 * I); a.K = (int)H;
  a.Q = hidden; a.q_ld = H; a.q_gather = sorted_token;
  a.offsets = offsets; a.E_glu = E_glu; a.act_codes = act_codes; a.I = (int)I;
  a.out = gate_up_out; a.out_ld = 2 * I; a.out2 = inter_out;
  a.gate = top_k_weights; a.sflat = sorted_flat;
  hipStream_t s = (hipStream_t)stream;
  auto go = [&]<typename T>() {
    if constexpr (sizeof(T) == 2) {
      if (a.K % v2::BK == 0) return launch_token_v2<T, EPI_GLU_FWD, false>(a, n_rows, s);
    }
    using C = TokCfg<T>;
    a.n_rtiles = (int)((I + C::BR / 2 - 1) / (C::BR / 2));
    return launch_token<C, EPI_GLU_FWD, false>(a, n_rows, s);
  };
  switch (dtype) {
    case MOE_DT_BF16: return go.template operator()<bf16>();
    case MOE_DT_F16: return go.template operator()<f16>();
    default: return go.template operator()<float>();
  }
}

// Workgroup slots of the current device (CUs; one 160 KB-LDS workgroup each).

extern "C" size_t moe_token_split_workspace_size(void) {
  const int n = device_cus();
  if (n <= 0) return 0;
  return (size_t)n * 65536 * sizeof(float) + (((size_t)n * sizeof(int) + 255) & ~(size_t)255);
}

// Attach a caller's split workspace (NULL: none). MOE_OK or MOE_ERR_WORKSPACE.
static int attach_split(TokenArgs& a, void* workspace, size_t workspace_bytes) {
  if (!workspace) return MOE_OK;
  const int n = device_cus();
  if (n < 8 || workspace_bytes < moe_token_split_workspace_size() || ((uintptr_t)workspace & 255))
    return MOE_ERR_WORKSPACE;
  a.split_ws = (float*)workspace;
  a.split_cnt = (int*)((char*)workspace + (size_t)n * 65536 * sizeof(float));
  a.xcd_cus = n / 8;
  return MOE_OK;
}

extern "C" int moe_grouped_down_fwd(int dtype, const void* inter, const void* down_proj, int E_glu,
                                    int64_t H, int64_t I, const int32_t* offsets,
                                    const int32_t* tile_offsets, int64_t n_rows, void* eo_out,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  (void)tile_offsets;
  int st = check_common(dtype, H, I, E_glu, n_rows);
  if (st) return st;
  if (n_rows == 0) return MOE_OK;
  if (!inter || !down_proj || !offsets || !eo_out) return MOE_ERR_SHAPE;
  if (!aligned16(inter) || !aligned16(down_proj) || !aligned16(eo_out)) return MOE_ERR_ALIGN;
  TokenArgs a = {};
  a.P = down_proj; a.p_e = H * I; a.p_ld = I; a.R = (int)H; a.K = (int)I;
  a.Q = inter; a.q_ld = I; a.q_gather = nullptr;
  a.offsets = offsets; a.E_glu = E_glu; a.I = (int)I;
  a.out = eo_out; a.out_ld = H;
  if ((st = attach_split(a, workspace, workspace_bytes))) return st;
  hipStream_t s = (hipStream_t)stream;
  auto go = [&]<typename T>() {
    if constexpr (sizeof(T) == 2) {
      if (a.K % v2::BK == 0) return launch_token_v2<T, EPI_STORE, false>(a, n_rows, s);
    }
    using C = TokCfg<T>;
    a.n_rtiles = (int)((H + C::BR - 1) / C::BR);
    return launch_token<C, EPI_STORE, false>(a, n_rows, s);
  };
  switch (dtype) {
    case MOE_DT_BF16: return go.template operator()<bf16>();
    case MOE_DT_F16: return go.template operator()<f16>();
    default: return go.template operator()<float>();
  }
}

extern "C" int moe_grouped_down_dx_swiglu_bwd(int dtype, const void* grad_eo,
                                              const void* down_proj, int E_glu, int64_t H,
                                              int64_t I, const void* gate_up,
                                              const int32_t* act_codes, const int32_t* offsets,
                                              const int32_t* tile_offsets, int64_t n_rows,
                                              void* ggu_out, void* grad_inter_out, void* stream) {
  (void)tile_offsets;
  int st = check_common(dtype, H, I, E_glu, n_rows);
  if (st) return st;
  if (n_rows == 0) return MOE_OK;
  if (!grad_eo || !down_proj || !offsets || (!ggu_out && !grad_inter_out)) return MOE_ERR_SHAPE;
  if (ggu_out && (!gate_up || !act_codes)) return MOE_ERR_SHAPE;
  if (!aligned16(grad_eo) || !aligned16(down_proj) || (ggu_out && !aligned16(ggu_out)) ||
      (gate_up && !aligned16(gate_up)) || (grad_inter_out && !aligned16(grad_inter_out)))
    return MOE_ERR_ALIGN;
  TokenArgs a = {};
  // P[r = i, k = h] = down_proj[e, h, i]: row-contiguous, K rows I elements apart.
  a.P = down_proj; a.p_e = H * I; a.p_ld = I; a.R = (int)I; a.K = (int)H;
  a.Q = grad_eo; a.q_ld = H; a.q_gather = nullptr;
  a.offsets = offsets; a.E_glu = E_glu; a.act_codes = act_codes; a.I = (int)I;
  a.out = ggu_out; a.out2 = grad_inter_out; a.aux = gate_up;
  hipStream_t s = (hipStream_t)stream;
  auto go = [&]<typename T>() {
    if constexpr (sizeof(T) == 2) {
      if (a.K % v3::KS == 0) return launch_token_v2<T, EPI_GLU_BWD, true>(a, n_rows, s);
    }
    using C = TokCfg<T>;
    a.n_rtiles = (int)((I + C::BR - 1) / C::BR);
    return launch_token<C, EPI_GLU_BWD, true>(a, n_rows, s);
  };
  switch (dtype) {
    case MOE_DT_BF16: return go.template operator()<bf16>();
    case MOE_DT_F16: return go.template operator()<f16>();
    default: return go.template operator()<float>();
  }
}

extern "C" int moe_gate_grad_parts(int64_t I) { return (int)(2 * ((I + v4::TILE - 1) / v4::TILE)); }

extern "C" int moe_grouped_down_dx_gated_bwd(int dtype, const void* grad_out, int64_t grad_out_ld,
                                             const void* down_proj, int E_glu, int64_t H,
                                             int64_t I, const void* gate_up,
                                             const int32_t* act_codes, const void* top_k_weights,
                                             const int32_t* offsets, const int32_t* sorted_token,
                                             const int32_t* sorted_flat, int64_t n_rows,
                                             void* ggu_out, void* inter_w_out, float* wt_partial,
                                             void* stream) {
  if (dtype != MOE_DT_BF16 && dtype != MOE_DT_F16) return MOE_ERR_DTYPE;
  int st = check_common(dtype, H, I, E_glu, n_rows);
  if (st) return st;
  if (H % 64 != 0) return MOE_ERR_ALIGN;
  if (n_rows == 0) return MOE_OK;
  if (!grad_out || !down_proj || !gate_up || !act_codes || !top_k_weights || !offsets ||
      !sorted_token || !wt_partial)
    return MOE_ERR_SHAPE;
  if (grad_out_ld < H || grad_out_ld % 8 != 0) return MOE_ERR_ALIGN;
  if (!aligned16(grad_out) || !aligned16(down_proj) || !aligned16(gate_up) ||
      (ggu_out && !aligned16(ggu_out)) || (inter_w_out && !aligned16(inter_w_out)))
    return MOE_ERR_ALIGN;
  TokenArgs a = {};
  // P[r = i, k = h] = down_proj[e, h, i]: row-contiguous; Q = grad_out rows gathered per token.
  a.P = down_proj; a.p_e = H * I; a.p_ld = I; a.R = (int)I; a.K = (int)H;
  a.Q = grad_out; a.q_ld = grad_out_ld; a.q_gather = sorted_token;
  a.offsets = offsets; a.E_glu = E_glu; a.act_codes = act_codes; a.I = (int)I;
  a.out = ggu_out; a.out2 = inter_w_out; a.aux = gate_up;
  a.gate = top_k_weights; a.sflat = sorted_flat; a.part = wt_partial; a.out_ld = n_rows;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == MOE_DT_BF16) return launch_token_v2<bf16, EPI_GLU_BWD_GATED, true>(a, n_rows, s);
  return launch_token_v2<f16, EPI_GLU_BWD_GATED, true>(a, n_rows, s);
}

extern "C" int moe_grouped_gateup_dx(int dtype, const void* ggu, const void* gate_up_proj,
                                     int E_glu, int64_t H, int64_t I, const int32_t* offsets,
                                     const int32_t* tile_offsets, int64_t n_rows,
                                     void* grad_xs_out, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  (void)tile_offsets;
  int st = check_common(dtype, H, I, E_glu, n_rows);
  if (st) return st;
  if (n_rows == 0) return MOE_OK;
  if (!ggu || !gate_up_proj || !offsets || !grad_xs_out) return MOE_ERR_SHAPE;
  if (!aligned16(ggu) || !aligned16(gate_up_proj) || !aligned16(grad_xs_out)) return MOE_ERR_ALIGN;
  TokenArgs a = {};
  // P[r = h, k = n] = gate_up_proj[e, n, h]: row-contiguous, K rows H elements apart.
  a.P = gate_up_proj; a.p_e = 2 * I * H; a.p_ld = H; a.R = (int)H; a.K = (int)(2 * I);
  a.Q = ggu; a.q_ld = 2 * I; a.q_gather = nullptr;
  a.offsets = offsets; a.E_glu = E_glu; a.I = (int)I;
  a.out = grad_xs_out; a.out_ld = H;
  if ((st = attach_split(a, workspace, workspace_bytes))) return st;
  hipStream_t s = (hipStream_t)stream;
  auto go = [&]<typename T>() {
    if constexpr (sizeof(T) == 2) {
      if (a.K % v3::KS == 0) return launch_token_v2<T, EPI_STORE, true>(a, n_rows, s);
    }
    using C = TokCfg<T>;
    a.n_rtiles = (int)((H + C::BR - 1) / C::BR);
    return launch_token<C, EPI_STORE, true>(a, n_rows, s);
  };
  switch (dtype) {
    case MOE_DT_BF16: return go.template operator()<bf16>();
    case MOE_DT_F16: return go.template operator()<f16>();
    default: return go.template operator()<float>();
  }
}

extern "C" int moe_grouped_wgrad(int dtype, const void* rsrc, int64_t r_ld, const int32_t* r_gather,
                                 const void* csrc, int64_t c_ld, const int32_t* c_gather, int64_t R,
                                 int64_t C, const int32_t* offsets, const int32_t* expert_order,
                                 int n_experts, int E_glu, void* out, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  if (dtype != MOE_DT_F32 && dtype != MOE_DT_F16 && dtype != MOE_DT_BF16) return MOE_ERR_DTYPE;
  if (R <= 0 || C <= 0 || E_glu <= 0 || E_glu > MAX_GLU_EXPERTS || R >= (1 << 30) || C >= (1 << 30))
    return MOE_ERR_SHAPE;
  if (expert_order && (n_experts < E_glu || n_experts > MAX_GLU_EXPERTS)) return MOE_ERR_SHAPE;
  if (!rsrc || !csrc || !offsets || !out) return MOE_ERR_SHAPE;
  if (R % 8 != 0 || C % 8 != 0 || r_ld % 8 != 0 || c_ld % 8 != 0) return MOE_ERR_ALIGN;
  if (!aligned16(rsrc) || !aligned16(csrc) || !aligned16(out)) return MOE_ERR_ALIGN;
  WgradArgs a = {};
  a.rsrc = rsrc; a.r_ld = r_ld; a.r_gather = r_gather;
  a.csrc = csrc; a.c_ld = c_ld; a.c_gather = c_gather;
  a.R = (int)R; a.C = (int)C; a.offsets = offsets; a.out = out;
  if (workspace) {
    const int n = device_cus();
    if (n < 8 || workspace_bytes < moe_token_split_workspace_size() || ((uintptr_t)workspace & 255))
      return MOE_ERR_WORKSPACE;
    a.split_ws = (float*)workspace;
    a.split_cnt = (int*)((char*)workspace + (size_t)n * 65536 * sizeof(float));
  }
  hipStream_t s = (hipStream_t)stream;
  auto go = [&]<typename T>() {
    if constexpr (sizeof(T) == 2) {
      return launch_wgrad_v2<T>(a, expert_order, expert_order ? n_experts : E_glu, E_glu, s);
    }
    using Cc = WgCfg<T>;
    a.n_rtiles = (int)((R + Cc::BR - 1) / Cc::BR);
    a.n_ctiles = (int)((C + Cc::BC - 1) / Cc::BC);
    return launch_wgrad<Cc>(a, E_glu, s);
  };
  switch (dtype) {
    case MOE_DT_BF16: return go.template operator()<bf16>();
    case MOE_DT_F16: return go.template operator()<f16>();
    default: return go.template operator()<float>();
  }
}

#ifdef MOE_PHASE_TRACE
extern "C" int moe_phase_read(void* host, size_t bytes) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_phase), bytes, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : 1;
}
extern "C" int moe_phase_reset(void) {
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_phase)) != hipSuccess) return 1;
  return hipMemset(p, 0, sizeof(g_phase)) == hipSuccess ? 0 : 1;
}
#endif
