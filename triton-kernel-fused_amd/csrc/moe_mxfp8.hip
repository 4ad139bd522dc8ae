// MXFP8-weight MoE forward for decode-sized batches (a few tokens per expert): the weight stream
// is the whole cost, so the kernels are built to read every touched expert's weights once at full
// HBM bandwidth and to do nothing else expensive.
//
// Weights are e4m3 bytes with one E8M0 scale per 32 consecutive K values of a row (OCP MX).
// Activations stay bf16. A workgroup owns one expert and 64 weight rows (gate/up: 32 gate rows and
// the same 32 up rows; down: 64 rows of H); its four waves split K. Each lane streams 64
// contiguous weight bytes of one row per 128-byte K chunk (the two lane halves cover the chunk,
// so every row read is a whole 128-byte line), converts them to bf16 with
// v_cvt_scalef32_pk_bf16_fp8 (the block scale 2^(s-127) applied in the conversion, exact in
// bf16), and feeds v_mfma_f32_32x32x16_bf16 with the expert's tokens as the other operand
// (token rows read from L2: decode batches are small). The four partial accumulators are summed
// through LDS; the gate/up kernel applies SwiGLU and writes the bf16 intermediate, the down
// kernel writes the expert outputs, and the gate-weighted combine (moe_combine_fwd) finishes.
#include "moe_common.h"

namespace moe {

struct MxArgs {
  const uint8_t* W;        // e4m3 weight rows, K bytes contiguous
  long long w_e, w_ld;     // bytes between experts / rows
  const uint8_t* S;        // E8M0 scales, one per 32 K values of a row
  long long s_e, s_ld;
  int R, K, I;             // rows per expert, K, intermediate size (gate/up)
  const bf16* X;           // token-side rows (bf16), K contiguous
  long long x_ld;
  const int32_t* x_gather; // sorted row -> X row (gate/up: sorted_token), null = identity
  const int32_t* offsets;
  int n_rtiles;
  bf16* out;
  long long out_ld;
};

// 2^(s-127) as an fp32 value (s = 0 is 2^-127, a denormal).
__device__ __forceinline__ float e8m0_to_f32(unsigned s) {
  return __uint_as_float(s ? (s << 23) : 0x00400000u);
}

// 8 e4m3 bytes (two dwords) times 2^(s-127) -> eight bf16 as one MFMA operand.
__device__ __forceinline__ i32x4 dequant8(unsigned lo, unsigned hi, float sc) {
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, sc, false);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, sc, true);
  const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, sc, false);
  const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, sc, true);
  return i32x4{__builtin_bit_cast(int, a), __builtin_bit_cast(int, b), __builtin_bit_cast(int, c),
               __builtin_bit_cast(int, d)};
}

// KSPLIT waves share one row tile and split its K range (partials summed through LDS); the
// block's 4/KSPLIT tiles are consecutive row tiles. a.n_rtiles counts row tiles.
// LDS per block: staged token rows (up to MX_XLDS bytes), reused for the K-split partial sums.
constexpr size_t MX_XLDS = 80 * 1024;
static_assert(MX_XLDS >= sizeof(f32x16) * 4 * 2 * 64, "partial sums fit");

template <bool GLU, int KSPLIT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
mx_gemm_kernel(MxArgs a) {
  constexpr int TPB = 4 / KSPLIT;  // row tiles per block
  const int nb = (a.n_rtiles + TPB - 1) / TPB;
  const int e = (int)blockIdx.x / nb;
  const int m_begin = a.offsets[e], m_end = a.offsets[e + 1];
  if (m_begin >= m_end) return;
  extern __shared__ __attribute__((aligned(16))) char xlds[];  // token rows, then partial sums
  f32x16 (*red)[2][64] = (f32x16 (*)[2][64])xlds;

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int w = wv % KSPLIT;                                      // K part of this wave
  const int rt = ((int)blockIdx.x % nb) * TPB + wv / KSPLIT;      // row tile of this wave
  const bool tile_ok = rt < a.n_rtiles;
  const int r = lane & 31, h = lane >> 5;
  int row0, row1;
  bool ok0, ok1;
  if (GLU) {
    const int ch = rt * 32 + r;
    ok0 = ok1 = ch < a.I;
    row0 = ok0 ? ch : 0;
    row1 = ok1 ? a.I + ch : 0;
  } else {
    row0 = rt * 64 + r;
    row1 = rt * 64 + 32 + r;
    ok0 = row0 < a.R;
    ok1 = row1 < a.R;
    row0 = ok0 ? row0 : 0;
    row1 = ok1 ? row1 : 0;
  }
  const uint8_t* w0 = a.W + (size_t)e * a.w_e + (size_t)row0 * a.w_ld;
  const uint8_t* w1 = a.W + (size_t)e * a.w_e + (size_t)row1 * a.w_ld;
  const uint8_t* s0 = a.S + (size_t)e * a.s_e + (size_t)row0 * a.s_ld;
  const uint8_t* s1 = a.S + (size_t)e * a.s_e + (size_t)row1 * a.s_ld;
  const int nc = a.K / 128;
  const int c_begin = w * nc / KSPLIT, c_end = tile_ok ? (w + 1) * nc / KSPLIT : c_begin;

  for (int mb = m_begin; mb < m_end; mb += 32) {
    const int m = mb + r;
    const bool tok = m < m_end;
    // Lanes past the group's last token read the first token's row: they only feed output
    // columns that are never stored, and unconditional loads keep the pipeline's waits partial.
    const int mm = tok ? m : m_begin;
    const int xr = a.x_gather ? a.x_gather[mm] : mm;
    const bf16* xrow = a.X + (size_t)xr * a.x_ld;
    f32x16 acc0, acc1;
#pragma unroll
    for (int v = 0; v < 16; ++v) { acc0[v] = 0.f; acc1[v] = 0.f; }

    // When this block's tokens fit in LDS (a decode batch gives an expert a handful), they are
    // staged once and every wave reads its token fragments from LDS instead of re-reading 8 KB
    // from L2 per 128-byte weight chunk; padding lanes read the last real token's row.
    const int nt = min(32, m_end - mb);
    const bool x_lds = (size_t)nt * a.K * sizeof(bf16) <= MX_XLDS;
    if (x_lds) {
      const int units = a.K / 8;  // 16-byte units per token row
      for (int u = threadIdx.x; u < nt * units; u += blockDim.x) {
        const int tt = u / units, o = u % units;
        const int gm = mb + tt;
        const int gr = a.x_gather ? a.x_gather[gm] : gm;
        *(i32x4*)(xlds + ((size_t)tt * a.K + 8 * o) * sizeof(bf16)) =
            ldg16(a.X + (size_t)gr * a.x_ld + 8 * o);
      }
      __syncthreads();
    }
    const char* xl = xlds + (size_t)min(r, nt - 1) * a.K * sizeof(bf16);

    // Software pipeline over two register buffers (no copies): everything chunk c+1 needs (token
    // fragments, weights, scales) is issued before chunk c computes. Vector loads retire in issue
    // order, so chunk c waits only for loads issued an iteration earlier. The prefetch is
    // unconditional (the last one re-reads a valid chunk) so every path has the same count of
    // loads in flight and the compiler's waits stay partial.
    auto kloop = [&](auto xl_c) {
      constexpr bool XL = decltype(xl_c)::value;
      struct Buf {
        i32x4 x[XL ? 1 : 8];
        uint4 a[4], b[4];
        unsigned short sa, sb;
      };
      Buf p0, p1;
      auto fetch = [&](int c, Buf& f) {
        const int kb = c * 128 + h * 64;
        if constexpr (!XL) {
#pragma unroll
          for (int j = 0; j < 8; ++j) f.x[j] = ldg16(xrow + kb + 8 * j);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f.a[i] = *(const uint4*)(w0 + kb + 16 * i);
          f.b[i] = *(const uint4*)(w1 + kb + 16 * i);
        }
        f.sa = *(const unsigned short*)(s0 + kb / 32);
        f.sb = *(const unsigned short*)(s1 + kb / 32);
        __builtin_amdgcn_sched_barrier(0);  // issue the whole batch before the compute that follows
      };
      auto compute = [&](const Buf& f, int c) {
        i32x4 xv[8];
        if constexpr (XL) {
          const int kb = c * 128 + h * 64;
#pragma unroll
          for (int j = 0; j < 8; ++j) xv[j] = *(const i32x4*)(xl + (kb + 8 * j) * sizeof(bf16));
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) xv[j] = f.x[j];
        }
        const float sa0 = e8m0_to_f32(f.sa & 0xff), sa1 = e8m0_to_f32(f.sa >> 8);
        const float sb0 = e8m0_to_f32(f.sb & 0xff), sb1 = e8m0_to_f32(f.sb >> 8);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint4 ua = f.a[j >> 1], ub = f.b[j >> 1];
          const i32x4 av = (j & 1) ? dequant8(ua.z, ua.w, j < 4 ? sa0 : sa1)
                                   : dequant8(ua.x, ua.y, j < 4 ? sa0 : sa1);
          const i32x4 bv = (j & 1) ? dequant8(ub.z, ub.w, j < 4 ? sb0 : sb1)
                                   : dequant8(ub.x, ub.y, j < 4 ? sb0 : sb1);
          Mfma<bf16>::step(acc0, av, xv[j]);
          Mfma<bf16>::step(acc1, bv, xv[j]);
        }
      };
      const int c_last = c_end - 1;
      if (c_begin <= c_last) {
        fetch(c_begin, p0);
        for (int c = c_begin; c <= c_last; c += 2) {
          fetch(min(c + 1, c_last), p1);
          compute(p0, c);
          if (c + 1 > c_last) break;
          fetch(min(c + 2, c_last), p0);
          compute(p1, c + 1);
        }
      }
    };
    if (x_lds) kloop(std::true_type{});
    else kloop(std::false_type{});
    // The partial-sum exchange below reuses the LDS that held the tokens.
    if (KSPLIT > 1 && x_lds) __syncthreads();

    if (KSPLIT > 1) {
      if (w > 0) {
        red[wv][0][lane] = acc0;
        red[wv][1][lane] = acc1;
      }
      __syncthreads();
      if (w == 0) {
#pragma unroll
        for (int q = 1; q < KSPLIT; ++q) {
          const f32x16 p0 = red[wv + q][0][lane], p1 = red[wv + q][1][lane];
#pragma unroll
          for (int v = 0; v < 16; ++v) { acc0[v] += p0[v]; acc1[v] += p1[v]; }
        }
      }
    }
    if (w == 0 && tok && tile_ok) {
      bf16* o = a.out + (size_t)m * a.out_ld;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int i0 = 8 * g + 4 * h;  // row within the 32-row tile
        if (GLU) {
          if (rt * 32 + i0 < a.I) {
            float iv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) iv[j] = silu(acc0[4 * g + j]) * acc1[4 * g + j];
            const bf16x2 p = {(bf16)iv[0], (bf16)iv[1]}, q = {(bf16)iv[2], (bf16)iv[3]};
            *(uint2*)(o + rt * 32 + i0) =
                uint2{__builtin_bit_cast(unsigned, p), __builtin_bit_cast(unsigned, q)};
          }
        } else {
          if (rt * 64 + i0 < a.R) {
            const bf16x2 p = {(bf16)acc0[4 * g], (bf16)acc0[4 * g + 1]};
            const bf16x2 q = {(bf16)acc0[4 * g + 2], (bf16)acc0[4 * g + 3]};
            *(uint2*)(o + rt * 64 + i0) =
                uint2{__builtin_bit_cast(unsigned, p), __builtin_bit_cast(unsigned, q)};
          }
          if (rt * 64 + 32 + i0 < a.R) {
            const bf16x2 p = {(bf16)acc1[4 * g], (bf16)acc1[4 * g + 1]};
            const bf16x2 q = {(bf16)acc1[4 * g + 2], (bf16)acc1[4 * g + 3]};
            *(uint2*)(o + rt * 64 + 32 + i0) =
                uint2{__builtin_bit_cast(unsigned, p), __builtin_bit_cast(unsigned, q)};
          }
        }
      }
    }
    if (KSPLIT > 1) __syncthreads();
  }
}

}  // namespace moe

using namespace moe;

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// ksplit = waves per row tile (4: each block is one row tile with K split four ways; measured
// within a few percent of 2 and 1 for both kernels at the decode shape).
template <bool GLU>
static bool launch_mx(const MxArgs& a, int E, int ksplit, hipStream_t s) {
  const int tpb = 4 / ksplit;
  const unsigned grid = (unsigned)(E * ((a.n_rtiles + tpb - 1) / tpb));
  auto go = [&](auto kern) {
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)MX_XLDS);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), MX_XLDS, s, a);
  };
  if (ksplit == 1) go(mx_gemm_kernel<GLU, 1>);
  else if (ksplit == 2) go(mx_gemm_kernel<GLU, 2>);
  else go(mx_gemm_kernel<GLU, 4>);
  return hipGetLastError() == hipSuccess;
}

extern "C" int moe_mxfp8_fwd(const void* hidden, int64_t n_tokens, int64_t H, const void* w13_q,
                             const void* w13_scale, const void* w2_q, const void* w2_scale, int E,
                             int64_t I, const int32_t* offsets, const int32_t* sorted_token,
                             int64_t n_rows, void* inter, void* eo, void* stream) {
  if (n_tokens < 0 || H <= 0 || I <= 0 || E <= 0 || n_rows < 0) return MOE_ERR_SHAPE;
  if (H >= (1 << 30) || I >= (1 << 29) || n_rows >= ((int64_t)1 << 31)) return MOE_ERR_SHAPE;
  if (H % 512 != 0 || I % 512 != 0) return MOE_ERR_ALIGN;
  if (n_rows == 0) return MOE_OK;
  if (!hidden || !w13_q || !w13_scale || !w2_q || !w2_scale || !offsets || !sorted_token ||
      !inter || !eo)
    return MOE_ERR_SHAPE;
  if (!al16(hidden) || !al16(w13_q) || !al16(w2_q) || !al16(inter) || !al16(eo) ||
      ((uintptr_t)w13_scale & 1) || ((uintptr_t)w2_scale & 1))
    return MOE_ERR_ALIGN;
  if ((int64_t)E * ((2 * I + 63) / 64) >= ((int64_t)1 << 31)) return MOE_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  MxArgs g = {};
  g.W = (const uint8_t*)w13_q; g.w_e = 2 * I * H; g.w_ld = H;
  g.S = (const uint8_t*)w13_scale; g.s_e = 2 * I * (H / 32); g.s_ld = H / 32;
  g.R = (int)(2 * I); g.K = (int)H; g.I = (int)I;
  g.X = (const bf16*)hidden; g.x_ld = H; g.x_gather = sorted_token;
  g.offsets = offsets; g.n_rtiles = (int)((I + 31) / 32);
  g.out = (bf16*)inter; g.out_ld = I;
  if (!launch_mx<true>(g, E, 4, s)) return MOE_ERR_LAUNCH;
  MxArgs d = {};
  d.W = (const uint8_t*)w2_q; d.w_e = H * I; d.w_ld = I;
  d.S = (const uint8_t*)w2_scale; d.s_e = H * (I / 32); d.s_ld = I / 32;
  d.R = (int)H; d.K = (int)I; d.I = (int)I;
  d.X = (const bf16*)inter; d.x_ld = I; d.x_gather = nullptr;
  d.offsets = offsets; d.n_rtiles = (int)((H + 63) / 64);
  d.out = (bf16*)eo; d.out_ld = H;
  return launch_mx<false>(d, E, 4, s) ? MOE_OK : MOE_ERR_LAUNCH;
}
