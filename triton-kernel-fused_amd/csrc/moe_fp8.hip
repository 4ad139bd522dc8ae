// fp8-e4m3 MoE forward (inference): grouped gate/up GEMM with scales + SwiGLU + re-quantisation
// of the intermediate, grouped down GEMM with scales.
//
// Operands are OCP e4m3fn: activations with an fp32 scale per token, weights with an fp32 scale
// per output channel. The GEMMs run the eight-wave 256x256 ring pipeline of moe_gemm_v4.h on
// v_mfma_scale_f32_32x32x64_f8f6f4; the fp32 scales factor out of the K sum and are applied in
// the epilogue: gate_up[m, n] = (sum_k xq[m,k] wq[n,k]) * sx[m] * sw[n].
// The gate/up epilogue quantises the intermediate itself, one power-of-two (E8M0) scale per
// token row and 128-channel block: a block is the tile's channel range, so its absmax is known in
// the epilogue (the two P-half waves exchange theirs through LDS), and a block is one K step of
// the down GEMM, whose MFMAs take the scales through their B-scale operand (v4::KcLoadS):
// eo[m, h] = (sum_k 2^e[m, k/128] iq[m,k] wq[h,k]) * sw[h].
#include "moe_gemm_common.h"
#include "moe_gemm_v4.h"

namespace moe {

struct Fp8Args {
  const fp8e4m3* P;        // weight rows, K contiguous
  long long p_e, p_ld;     // elements between experts / rows
  const float* p_scale;    // per (expert, weight row) fp32 scales
  long long ps_e;          // scales between experts
  int R, K, I;
  const fp8e4m3* Q;        // token-side rows, K contiguous
  long long q_ld;
  const int32_t* q_gather; // sorted row -> Q row, or null
  const float* q_scale;    // GLU: per Q row (indexed like Q rows)
  const uint8_t* q_bscale; // down: E8M0 block scales of the intermediate (KcLoadS table layout)
  long long bs_ld;         // scale table row pitch (bytes)
  const int32_t* offsets;
  int E_glu, n_rtiles;
  bf16* out;               // down: (M, out_ld) bf16
  long long out_ld;
  fp8e4m3* out_q;          // GLU: intermediate (M, I) e4m3
  uint8_t* out_bscale;     // GLU: its E8M0 block scales (written in the KcLoadS table layout)
};

// Persistent: one workgroup per CU slot of an XCD runs the XCD's logical tiles bi, bi + n_wg, ...
// (as the bf16 persistent token GEMMs: a scalar expert walk instead of a per-tile scan, and the
// next tile's ring loads issued as soon as the epilogue has released the LDS).
template <bool GLU>
__global__ void __launch_bounds__(v4::NT, 1)
fp8_gemm_kernel(Fp8Args a) {
  using C = Cfg<fp8e4m3, v4::TILE, v4::TILE, 2, 2>;  // GLU row interleave per 128-row P half
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  v4::Experts ex;
  ex.init(a.offsets, a.E_glu);
  const int gm = v4::tile_group(a.n_rtiles);
  const int n_idx = (ex.n_mt + gm - 1) / gm * gm * a.n_rtiles;
  const int xcd = (int)blockIdx.x & 7, bi = (int)blockIdx.x >> 3, nwg = (int)gridDim.x >> 3;
  const int R8 = (n_idx + 7) >> 3;
  const int t_lo = xcd * R8, t_cnt = max(0, min(n_idx, t_lo + R8) - t_lo);
  const int wr = v4::wave_r(), wc = v4::wave_c();
  struct Tile { int e, m0, m_end, rt, mt; };
  auto find = [&](int j, Tile& t) {
    for (; j < t_cnt; j += nwg) {
      int mt, rt;
      v4::tile_of(t_lo + j, a.n_rtiles, mt, rt);
      if (mt < ex.n_mt) {
        ex.lookup(mt, t.e, t.m0, t.m_end);
        t.rt = rt;
        t.mt = mt;
        return j;
      }
    }
    return t_cnt;
  };
  std::conditional_t<GLU, v4::KcLoad, v4::KcLoadS> lq;
  v4::KcLoad lp;
  auto setup = [&](const Tile& t) {
    const fp8e4m3* Pe = a.P + (size_t)t.e * a.p_e;
    lq.init(wc * v4::WQ);
    if constexpr (!GLU) {
      // The gate/up epilogue writes scale codes only for rows below its group end, so the bytes
      // of a tail tile's rows past m_end are stale; they scale only accumulator rows that the
      // epilogue does not store.
      lq.sp = (const char*)a.q_bscale + (size_t)t.mt * v4::TILE + wc * v4::WQ +
              2 * (v4::lane_id() & 31);
      lq.s_ld = a.bs_ld;
    }
#pragma unroll
    for (int i = 0; i < v4::LOADS; ++i) {
      int m = t.m0 + v4::KcLoad::row_of(i);
      if (m >= t.m_end) m = t.m0;
      const int qr = a.q_gather ? a.q_gather[m] : m;
      lq.rowp[i] = (const char*)(a.Q + (size_t)qr * a.q_ld);
    }
    lp.init(wr * v4::WP);
#pragma unroll
    for (int i = 0; i < v4::LOADS; ++i) {
      const int rr = v4::KcLoad::row_of(i);
      bool ok;
      int prow;
      if (GLU) {
        prow = glu_prow<C>(rr, t.rt, a.I, ok);
      } else {
        prow = t.rt * v4::TILE + rr;
        ok = prow < a.R;
      }
      lp.rowp[i] = (const char*)(Pe + (size_t)(ok ? prow : 0) * a.p_ld);
    }
  };

  Tile cur;
  int jt = find(bi, cur);
  if (jt >= t_cnt) return;
  // The gate/up GEMM issues the next tile's ring loads right after the epilogue; the down GEMM's
  // K loop issues them itself (its block-scale loads must not be in flight across the tile loop).
  constexpr bool PRE = GLU;
  setup(cur);
  if (PRE) v4::ring_prologue<fp8e4m3>(lp, lq, 0, a.K, smem, 0, 0, v4::NSLOT);
  while (true) {
    const int e = cur.e, m0 = cur.m0, m_end = cur.m_end, rt = cur.rt, mt = cur.mt;
    f32x16 acc[v4::TI][v4::TJ];
#pragma unroll
    for (int ti = 0; ti < v4::TI; ++ti)
#pragma unroll
      for (int tj = 0; tj < v4::TJ; ++tj)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[ti][tj][v] = 0.f;
    // Waves whose 64 token rows all lie past the group end (tail tiles) skip their MFMAs.
    if (m0 + wc * v4::WQ < m_end) v4::mainloop_ring<fp8e4m3, true, PRE>(acc, lp, lq, 0, a.K, smem);
    else v4::mainloop_ring<fp8e4m3, false, PRE>(acc, lp, lq, 0, a.K, smem);
    {
    // Epilogue: scales applied in fp32 in registers, then the bf16 results of each wave are staged
    // in its own LDS block (the ring's final barrier has released the LDS) and stored as whole row
    // segments: lane (l & 31) of fragment tj is token row q = 32 tj + (l & 31) and holds four
    // consecutive output channels per 8-channel group g (half h of the lane).
    const int lane = threadIdx.x & 63;
    const int h = lane >> 5;
    const int w = threadIdx.x >> 6;
    const float* ps = a.p_scale + (size_t)e * a.ps_e;
    const int row0 = m0 + wc * v4::WQ;
    if constexpr (GLU) {
      float qsv[v4::TJ];
#pragma unroll
      for (int tj = 0; tj < v4::TJ; ++tj) {
        const int m = row0 + tj * 32 + (lane & 31);
        qsv[tj] = m < m_end ? a.q_scale[a.q_gather ? a.q_gather[m] : m] : 0.f;
      }
      // SiLU(gate) * up in fp32, in place of the gate accumulators: lane (l & 31) of fragment tj
      // is token row q = 32 tj + (l & 31) and holds channels 32 ti + 8 g + 4 h + j of the wave's
      // 64 (h = l / 32, the partner lane l ^ 32 holds the other half).
      float am[v4::TJ] = {0.f, 0.f};
#pragma unroll
      for (int ti = 0; ti < v4::TI / 2; ++ti)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int ch = rt * (v4::TILE / 2) + wr * (v4::WP / 2) + ti * 32 + 8 * g + 4 * h;
          const bool cok = ch < a.I;
          const f32x4 sg = cok ? *(const f32x4*)(ps + ch) : f32x4{0.f, 0.f, 0.f, 0.f};
          const f32x4 su = cok ? *(const f32x4*)(ps + a.I + ch) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int tj = 0; tj < v4::TJ; ++tj)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float gv = acc[ti][tj][4 * g + j] * qsv[tj] * sg[j];
              const float uv = acc[ti + v4::TI / 2][tj][4 * g + j] * qsv[tj] * su[j];
              const float iv = silu(gv) * uv;
              acc[ti][tj][4 * g + j] = iv;
              am[tj] = fmaxf(am[tj], fabsf(iv));
            }
        }
      // Block absmax over the tile's 128 channels of each token row: the partner lane, then the
      // other P-half wave (same token rows) through LDS (above the 32 KB of staging blocks).
      float* xam = (float*)(smem + 32768) + wc * (2 * v4::WQ);
#pragma unroll
      for (int tj = 0; tj < v4::TJ; ++tj) {
        am[tj] = fmaxf(am[tj], __shfl_xor(am[tj], 32, 64));
        if (h == 0) xam[wr * v4::WQ + tj * 32 + lane] = am[tj];
      }
      __syncthreads();
      // E8M0 exponent per token row: the smallest e with 448 * 2^e >= absmax (for absmax =
      // 1.f * 2^E: e = E - 8, plus one when 1.f > 1.75), clamped to [-127, ...]; byte = e + 127.
      unsigned code[v4::TJ];
      float inv[v4::TJ];
#pragma unroll
      for (int tj = 0; tj < v4::TJ; ++tj) {
        const int q = tj * 32 + (lane & 31);
        const float amax = fmaxf(xam[q], xam[v4::WQ + q]);
        const unsigned b = __float_as_uint(amax);
        const int c = (int)(b >> 23) - 8 + ((b & 0x7fffff) > 0x600000u ? 1 : 0);
        code[tj] = (unsigned)max(c, 0);
        inv[tj] = __uint_as_float((254u - code[tj]) << 23);  // 2^-e, exact
      }
      // e4m3 bytes of the wave's 64 rows x 64 channels, staged per wave as [row q][64 bytes]:
      // 16-byte chunk c of row q at c ^ ((q >> 2) & 3).
      char* wl = smem + w * (v4::WQ * 64);
#pragma unroll
      for (int ti = 0; ti < v4::TI / 2; ++ti)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int tj = 0; tj < v4::TJ; ++tj) {
            const f32x16& v = acc[ti][tj];
            int p = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * g] * inv[tj], v[4 * g + 1] * inv[tj], 0,
                                                    false);
            p = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * g + 2] * inv[tj], v[4 * g + 3] * inv[tj], p,
                                                true);
            const int q = tj * 32 + (lane & 31);
            const int chunk = ti * 2 + (g >> 1), pos = 2 * (g & 1) + h;
            *(int*)(wl + q * 64 + ((chunk ^ ((q >> 2) & 3)) << 4) + 4 * pos) = p;
          }
      // Scales: table row rt (the down GEMM's K step), the token tile's 256 bytes, bytes 2j /
      // 2j+1 of the wave's 64 = its rows j / j+32.
      if (wr == 0 && h == 0) {
#pragma unroll
        for (int tj = 0; tj < v4::TJ; ++tj)
          if (row0 + tj * 32 + lane < m_end)
            a.out_bscale[(size_t)rt * a.bs_ld + (size_t)mt * v4::TILE + wc * v4::WQ + 2 * lane + tj] =
                (uint8_t)code[tj];
      }
      __syncthreads();
      const int c = lane & 3;
      const int ch = rt * (v4::TILE / 2) + wr * (v4::WP / 2);
#pragma unroll
      for (int it = 0; it < v4::WQ / 16; ++it) {
        const int q = it * 16 + (lane >> 2);
        const i32x4 v = *(const i32x4*)(wl + q * 64 + (c << 4));
        const int lc = c ^ ((q >> 2) & 3);
        if (row0 + q < m_end && ch < a.I)
          *(i32x4*)(a.out_q + (size_t)(row0 + q) * a.I + ch + 16 * lc) = v;
      }
    } else {
#pragma unroll
      for (int ti = 0; ti < v4::TI; ++ti)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int r = rt * v4::TILE + wr * v4::WP + ti * 32 + 8 * g + 4 * h;
          const f32x4 sr = r < a.R ? *(const f32x4*)(ps + r) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int tj = 0; tj < v4::TJ; ++tj)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[ti][tj][4 * g + j] *= sr[j];
        }
      char* wl = smem + w * (v4::WQ * v2::EPI_ROWB);
      v2::stage_acc<bf16, v4::TJ>(acc, wl);
      __syncthreads();
      v2::store_staged<bf16, v4::WQ>(wl, a.out, a.out_ld, row0, m_end, rt * v4::TILE + wr * v4::WP, a.R);
    }

    }
    Tile nxt;
    const int jn = find(jt + nwg, nxt);
    if (jn >= t_cnt) break;
    setup(nxt);
    v4::bare_barrier();  // every wave is done with its staging block
    if (PRE) v4::ring_prologue<fp8e4m3>(lp, lq, 0, a.K, smem, 0, 0, v4::NSLOT);
    cur = nxt;
    jt = jn;
  }
}

// Per-row absmax fp8 quantisation of a bf16 matrix (one wave per row):
// scale[m] = absmax(row) / 448 (1 for an all-zero row), q[m, :] = e4m3(x / scale).
__global__ void __launch_bounds__(256)
rowquant_fp8_kernel(const bf16* __restrict__ x, int64_t M, int K, fp8e4m3* __restrict__ q,
                    float* __restrict__ scale) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const int lane = threadIdx.x & 63;
  const bf16* xr = x + row * K;
  float amax = 0.f;
  for (int c = lane * 8; c < K; c += 512) {
    const uint4 u = *(const uint4*)(xr + c);
    const unsigned w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      amax = fmaxf(amax, fmaxf(fabsf(__uint_as_float(w[i] << 16)),
                               fabsf(__uint_as_float(w[i] & 0xffff0000u))));
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) amax = fmaxf(amax, __shfl_xor(amax, d, 64));
  const float s = amax > 0.f ? amax / 448.f : 1.f;
  if (lane == 0) scale[row] = s;
  fp8e4m3* qr = q + row * K;
  for (int c = lane * 8; c < K; c += 512) {
    const uint4 u = *(const uint4*)(xr + c);
    const unsigned w[4] = {u.x, u.y, u.z, u.w};
    int packed[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float v0 = __uint_as_float(w[2 * i] << 16) / s;
      const float v1 = __uint_as_float(w[2 * i] & 0xffff0000u) / s;
      const float v2 = __uint_as_float(w[2 * i + 1] << 16) / s;
      const float v3 = __uint_as_float(w[2 * i + 1] & 0xffff0000u) / s;
      int p = __builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
      p = __builtin_amdgcn_cvt_pk_fp8_f32(v2, v3, p, true);
      packed[i] = p;
    }
    *(uint2*)(qr + c) = uint2{(unsigned)packed[0], (unsigned)packed[1]};
  }
}

template <bool GLU>
static int launch_fp8(Fp8Args a, int64_t n_rows, hipStream_t s) {
  a.n_rtiles = GLU ? (a.I + v2::TILE / 2 - 1) / (v2::TILE / 2) : (a.R + v2::TILE - 1) / v2::TILE;
  const int64_t max_mt = (n_rows + v2::TILE - 1) / v2::TILE + a.E_glu;
  const int64_t logical = v4::logical_tiles(max_mt, a.n_rtiles);
  if (logical <= 0) return MOE_OK;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 8)
    return MOE_ERR_LAUNCH;
  const int64_t grid = 8 * std::min<int64_t>(cus / 8, (logical + 7) / 8);
  auto kern = fp8_gemm_kernel<GLU>;
  (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, v4::RING_LDSB);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(v4::NT), v4::RING_LDSB, s, a);
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}

}  // namespace moe

using namespace moe;

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Scale table of the intermediate: one row per K step of the down GEMM (I / 128), 256 bytes per
// possible token tile (the grouped tiling gives at most ceil(n_rows / 256) + E of them).
static int64_t bscale_pitch(int64_t n_rows, int E) {
  return (int64_t)v4::TILE * ((n_rows + v4::TILE - 1) / v4::TILE + E);
}

extern "C" int64_t moe_fp8_inter_bscale_bytes(int64_t I, int64_t n_rows, int E) {
  if (I <= 0 || n_rows < 0 || E <= 0) return 0;
  return (I / 128) * bscale_pitch(n_rows, E);
}

extern "C" int moe_fp8_fwd(const void* x_q, const float* x_scale, int64_t n_tokens, int64_t H,
                           const void* w13_q, const float* w13_scale, const void* w2_q,
                           const float* w2_scale, int E, int64_t I, const int32_t* offsets,
                           const int32_t* sorted_token, int64_t n_rows, void* inter_q,
                           void* inter_bscale, void* eo, void* stream) {
  if (n_tokens < 0 || H <= 0 || I <= 0 || E <= 0 || E > MAX_GLU_EXPERTS || n_rows < 0)
    return MOE_ERR_SHAPE;
  if (H >= (1 << 30) || I >= (1 << 29) || n_rows >= ((int64_t)1 << 31)) return MOE_ERR_SHAPE;
  if (H % 128 != 0 || I % 128 != 0) return MOE_ERR_ALIGN;
  if (n_rows == 0) return MOE_OK;
  if (!x_q || !x_scale || !w13_q || !w13_scale || !w2_q || !w2_scale || !offsets ||
      !sorted_token || !inter_q || !inter_bscale || !eo)
    return MOE_ERR_SHAPE;
  if (!al16(x_q) || !al16(w13_q) || !al16(w2_q) || !al16(w13_scale) || !al16(w2_scale) ||
      !al16(inter_q) || !al16(eo))
    return MOE_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  const int64_t bs_ld = bscale_pitch(n_rows, E);
  Fp8Args g = {};
  g.P = (const fp8e4m3*)w13_q; g.p_e = 2 * I * H; g.p_ld = H;
  g.p_scale = w13_scale; g.ps_e = 2 * I;
  g.R = (int)(2 * I); g.K = (int)H; g.I = (int)I;
  g.Q = (const fp8e4m3*)x_q; g.q_ld = H; g.q_gather = sorted_token; g.q_scale = x_scale;
  g.offsets = offsets; g.E_glu = E;
  g.out_q = (fp8e4m3*)inter_q; g.out_bscale = (uint8_t*)inter_bscale; g.bs_ld = bs_ld;
  int st = launch_fp8<true>(g, n_rows, s);
  if (st) return st;
  Fp8Args d = {};
  d.P = (const fp8e4m3*)w2_q; d.p_e = H * I; d.p_ld = I;
  d.p_scale = w2_scale; d.ps_e = H;
  d.R = (int)H; d.K = (int)I; d.I = (int)I;
  d.Q = (const fp8e4m3*)inter_q; d.q_ld = I; d.q_gather = nullptr;
  d.q_bscale = (const uint8_t*)inter_bscale; d.bs_ld = bs_ld;
  d.offsets = offsets; d.E_glu = E;
  d.out = (bf16*)eo; d.out_ld = H;
  return launch_fp8<false>(d, n_rows, s);
}

extern "C" int moe_rowquant_fp8(const void* x, int64_t n_rows, int64_t K, void* q, float* scale,
                                void* stream) {
  if (n_rows < 0 || K <= 0 || K >= (1 << 30)) return MOE_ERR_SHAPE;
  if (K % 8 != 0) return MOE_ERR_ALIGN;
  if (n_rows == 0) return MOE_OK;
  if (!x || !q || !scale) return MOE_ERR_SHAPE;
  if (!al16(x) || ((uintptr_t)q & 7)) return MOE_ERR_ALIGN;
  hipLaunchKernelGGL(rowquant_fp8_kernel, dim3((unsigned)((n_rows + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, (const bf16*)x, n_rows, (int)K, (fp8e4m3*)q, scale);
  return hipGetLastError() == hipSuccess ? MOE_OK : MOE_ERR_LAUNCH;
}
