// MXFP8-weight MoE forward for decode-sized batches (a few tokens per expert): the weight stream
// is the whole cost, so the kernels are built to read every touched expert's weights once at full
// HBM bandwidth and to do nothing else expensive.
//
// Weights are e4m3 bytes with one E8M0 scale per 32 consecutive K values of a row (OCP MX).
// Activations stay bf16. A workgroup owns one expert and a few row tiles of 64 weight rows
// (gate/up: 32 gate rows and the same 32 up rows; down: 64 rows of H). For the gate/up projection
// (long K) its four waves split K and sum their partial accumulators through LDS; for the down
// projection (short K) each wave runs whole row tiles of its own. Each load instruction reads
// whole 128-byte lines of 8 rows with a nontemporal hint, a lane exchange puts each lane's 32
// bytes of one row in place, and the lane converts them to bf16 with
// v_cvt_scalef32_pk_bf16_fp8 (the block scale 2^(s-127) applied in the conversion, exact in
// bf16), and feeds v_mfma_f32_16x16x32_bf16 with the expert's tokens as the other operand
// (token rows staged in LDS: decode batches are small). The gate/up kernel applies SwiGLU and
// writes the bf16 intermediate, the down kernel writes the expert outputs, and the gate-weighted
// combine (moe_combine_fwd) finishes.
#include "moe_gemm_common.h"

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

// LDS per block (two blocks per CU): the E8M0 scale table of the block's 64 rows, then the
// staged token rows, whose space the K-split partial sums reuse after the K loop.
constexpr int MX_LDS = 80 * 1024;
constexpr int MX_WAVES = 4;       // waves per block; they split K
constexpr int MX_ROWS = 64;       // weight rows per block (4 MFMA tiles of 16)
constexpr int MX_TOK = 16;        // tokens per MFMA tile (v_mfma_f32_16x16x32_bf16 B side)
constexpr int MX_BATCH = 8;       // staging loads in flight per lane

// Scale-table row stride in 4-byte words for nc K chunks split over the waves: one word (four
// E8M0 bytes) per chunk, rounded up to an odd count so the 16 rows of a tile hit distinct banks.
__host__ __device__ inline int mx_scale_words(int nc, bool ks) {
  return (ks ? (nc + MX_WAVES - 1) / MX_WAVES : nc) | 1;
}

// One block per (expert, RT consecutive row tiles of 64 weight rows): gate/up tile = rows
// ch..ch+31 of the gate and the same channels of up (GLU), down tile = 64 rows. The block stages
// the expert's token rows once and runs its row tiles over them. KS (K split, long K): wave w
// streams K chunks [w*nc/4, (w+1)*nc/4) of every tile of the block, one tile after the other, and
// the partial sums meet in LDS. Otherwise (short K) wave w streams the whole K of tiles w, w+4,
// ... on its own and stores them: no exchange and no barrier between tiles.
//
// MFMA layout (16x16x32): lane l holds row l%16 of a 16-row weight tile and token l%16 of the
// token tile; q = l/16 selects K. Within a 128-byte chunk lane q owns the weight bytes
// [32q, 32q+32) (after the load exchange below), consumed as four K steps of 8; the token
// fragments use the same K order. Those 32 bytes are exactly scale block q of the chunk.
//
// LDS: the scale tables ([64 rows][sw words] each; KS: RT x 4 per wave and tile, else RT, one per
// tile), then (KS, RT > 1) the partial-sum exchange, then the staged token rows (KS, RT == 1: the
// exchange reuses the token rows' space).
constexpr int MX_RED_BYTES = MX_WAVES * 4 * 64 * 16;  // [wave][tile][lane] f32x4
__host__ __device__ inline int mx_table_bytes(int nc, int rt, bool ks) {
  return rt * (ks ? MX_WAVES : 1) * MX_ROWS * mx_scale_words(nc, ks) * 4;
}
__host__ __device__ inline int mx_x_offset(int nc, int rt, bool ks) {
  return mx_table_bytes(nc, rt, ks) + (ks && rt > 1 ? MX_RED_BYTES : 0);
}

template <bool GLU, int RT, bool KS>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
mx_gemm_kernel(MxArgs a) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int ng = (a.n_rtiles + RT - 1) / RT;
  const int e = (int)blockIdx.x / ng;
  const int rt0 = ((int)blockIdx.x % ng) * RT;
  const int nrt = min(RT, a.n_rtiles - rt0);
  const int m_begin = a.offsets[e], m_end = a.offsets[e + 1];
  if (m_begin >= m_end) return;

  // The wave index as a scalar, so the K range, the item counters and the weight base below stay
  // in scalar registers.
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rr = lane & 15, q = lane >> 4;
  const int nc = a.K / 128;
  // >= 1 chunk per wave: K % 512 == 0
  const int c0 = KS ? w * nc / MX_WAVES : 0, nch = KS ? (w + 1) * nc / MX_WAVES - c0 : nc;
  auto chunk = [&](int i) { return c0 + i; };  // the wave's i-th K chunk
  // The wave's tiles: tile(j), j < nrt_w.
  const int nrt_w = KS ? nrt : (w < nrt ? (nrt - w + MX_WAVES - 1) / MX_WAVES : 0);
  auto tile = [&](int j) { return rt0 + (KS ? j : w + MX_WAVES * j); };
  const int total = nrt_w * nch;    // (tile, chunk) items of this wave, tile-major
  const int sw = mx_scale_words(nc, KS);
  auto stab_of = [&](int j) {
    return (uint32_t*)lds + (KS ? j * MX_WAVES + w : w + MX_WAVES * j) * MX_ROWS * sw;
  };
  char* xlds = lds + mx_x_offset(nc, RT, KS);
  f32x4* red = (f32x4*)(RT > 1 ? lds + mx_table_bytes(nc, RT, KS) : xlds);
  const int x_bytes = MX_LDS - mx_x_offset(nc, RT, KS);
  // Block barrier without HIP's release fence: weight loads stay in flight across it.
  auto barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

  // Weight row i of tile rt (clamped into the matrix; rows outside it feed unstored outputs).
  auto wrow = [&](int rt, int i) {
    if (GLU) {
      const int ch = min(rt * 32 + 16 * ((i >> 4) & 1) + (i & 15), a.I - 1);
      return ((i >> 4) < 2 ? 0 : a.I) + ch;
    }
    return min(rt * MX_ROWS + i, a.R - 1);
  };
  // Loads: one instruction reads whole 128-byte lines of 8 rows (lane l: row 8*jj + l%8 of a
  // 16-row group, 16-byte piece l/8 of the K chunk), nontemporal (each weight byte is read once);
  // measured ~7.0 TB/s against ~5.6 TB/s for half lines per instruction. The MFMA wants lane l to
  // hold row l%16, so a row_ror:8 DPP exchange between lanes l and l^8 (compute()) turns the two
  // loads of a group into pieces 2q and 2q+1 (K bytes [32q, 32q+32)) of row l%16, q = l/16.
  // A load's address is the expert's weights plus the chunk's byte offset (both wave-uniform)
  // plus the lane's 32-bit row offset within the expert, set once per row tile.
  const int r8 = lane & 7, pc = lane >> 3;
  const uint8_t* wexp = a.W + (size_t)e * a.w_e;
  uint32_t roff[4][2];
  auto set_rows = [&](int j) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        roff[t][jj] = (uint32_t)wrow(tile(j), 16 * t + 8 * jj + r8) * (uint32_t)a.w_ld + 16 * pc;
  };
  set_rows(0);

  // Two register buffers of weight bytes (no copies): item i+1 is in flight while item i
  // computes, and across tile ends the next tile's first chunk is in flight during the partial-sum
  // exchange and the epilogue. Fetches past the last item re-read it (every path has the same
  // loads in flight, so the compiler's waits stay partial).
  struct Buf { i32x4 v[4][2]; };
  Buf p0, p1;
  int fj = 0, fc = 0;  // next item to fetch (tile, chunk index of the wave)
  auto fetch = [&](Buf& f) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        f.v[t][jj] = __builtin_nontemporal_load(
            (const i32x4*)(wexp + (size_t)chunk(fc) * 128 + roff[t][jj]));
    __builtin_amdgcn_sched_barrier(0);
    if (++fc == nch) {
      if (fj + 1 < nrt_w) {
        ++fj;
        fc = 0;
        set_rows(fj);
      } else {
        fc = nch - 1;
      }
    }
  };

  // The first weight chunk goes out before the scale tables and token rows are staged. Staging
  // loads go out in batches of MX_BATCH per lane before any of them is written to LDS, so a
  // block start waits for a few load latencies rather than one per element.
  fetch(p0);
  for (int j = 0; j < nrt_w; ++j) {
    uint32_t* stab = stab_of(j);
    const int n = MX_ROWS * nch;
    for (int u0 = lane; u0 < n; u0 += 64 * MX_BATCH) {
      uint32_t v[MX_BATCH];
#pragma unroll
      for (int b = 0; b < MX_BATCH; ++b) {
        const int u = min(u0 + 64 * b, n - 1);  // past the end: re-read the last word
        const int i = u / nch, c = u % nch;
        v[b] = *(const uint32_t*)(a.S + (size_t)e * a.s_e + (size_t)wrow(tile(j), i) * a.s_ld +
                                  chunk(c) * 4);
      }
#pragma unroll
      for (int b = 0; b < MX_BATCH; ++b) {
        const int u = u0 + 64 * b;
        if (u < n) stab[(u / nch) * sw + u % nch] = v[b];
      }
    }
  }

  for (int mb = m_begin; mb < m_end; mb += MX_TOK) {
    const int nt = min(MX_TOK, m_end - mb);
    const int m = mb + rr;
    if (mb != m_begin) {
      fj = 0;
      fc = 0;
      set_rows(0);
      fetch(p0);
    }
    // Token rows: staged in LDS when they fit (a decode batch gives an expert a handful), else
    // read from L2 per chunk. Lanes past the last token read the last token's row: they only
    // feed output columns that are never stored.
    const bool x_lds = (size_t)nt * a.K * sizeof(bf16) <= (size_t)x_bytes;
    barrier();  // scale tables written; the previous token block is done with the LDS
    if (x_lds) {
      const int units = a.K / 8;  // 16-byte units per token row
      const int n = nt * units;
      for (int u0 = threadIdx.x; u0 < n; u0 += 64 * MX_WAVES * MX_BATCH) {
        i32x4 v[MX_BATCH];
#pragma unroll
        for (int b = 0; b < MX_BATCH; ++b) {
          const int u = min(u0 + 64 * MX_WAVES * b, n - 1);
          const int tt = u / units, o = u % units;
          const int gr = a.x_gather ? a.x_gather[mb + tt] : mb + tt;
          v[b] = ldg16(a.X + (size_t)gr * a.x_ld + 8 * o);
        }
#pragma unroll
        for (int b = 0; b < MX_BATCH; ++b) {
          const int u = u0 + 64 * MX_WAVES * b;
          if (u < n)
            *(i32x4*)(xlds + ((size_t)(u / units) * a.K + 8 * (u % units)) * sizeof(bf16)) = v[b];
        }
      }
      barrier();
    }
    const int mt = mb + min(rr, nt - 1);
    const int xr = a.x_gather ? a.x_gather[mt] : mt;
    const bf16* xrow = a.X + (size_t)xr * a.x_ld;
    const char* xl = xlds + (size_t)min(rr, nt - 1) * a.K * sizeof(bf16);

    auto run = [&](auto xl_c) {
      constexpr bool XL = decltype(xl_c)::value;
      f32x4 acc[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
      int cj = 0, cc = 0;  // item being computed
      auto compute = [&](const Buf& f) {
        i32x4 xv[4];  // token fragments of the four K steps: K [32q + 8ks, 32q + 8ks + 8)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const int k = chunk(cc) * 128 + 32 * q + 8 * ks;
          if constexpr (XL) xv[ks] = *(const i32x4*)(xl + k * sizeof(bf16));
          else xv[ks] = ldg16(xrow + k);
        }
        const uint32_t* stab = stab_of(cj);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          // Lanes with l%16 < 8 keep their first load and take the partner's (l^8) first load as
          // their second piece; lanes with l%16 >= 8 take the partner's second load as their first
          // piece and keep their own second load.
          i32x4 lo, hi;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            lo[d] = __builtin_amdgcn_update_dpp(f.v[t][0][d], f.v[t][1][d], 0x128, 0xf, 0xc, false);
            hi[d] = __builtin_amdgcn_update_dpp(f.v[t][1][d], f.v[t][0][d], 0x128, 0xf, 0x3, false);
          }
          // K bytes [32q, 32q+32) of the chunk are exactly 32-value scale block q.
          const uint32_t sc = stab[(16 * t + rr) * sw + cc];
          const float s0 = e8m0_to_f32((sc >> (8 * q)) & 0xff);
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            const i32x4 u = ks < 2 ? lo : hi;
            const i32x4 av = (ks & 1) ? dequant8((unsigned)u[2], (unsigned)u[3], s0)
                                      : dequant8((unsigned)u[0], (unsigned)u[1], s0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av),
                                                             __builtin_bit_cast(bf16x8, xv[ks]),
                                                             acc[t], 0, 0, 0);
          }
        }
      };
      // After the last chunk of tile cj. KS: partial sums of waves 1-3 meet wave 0's in LDS,
      // wave 0 stores the tile. Otherwise the wave stores its own tile.
      auto finish_tile = [&]() {
        if (KS) {
          if (RT == 1) barrier();  // the exchange reuses the token rows' space
          if (w > 0) {
#pragma unroll
            for (int t = 0; t < 4; ++t) red[(w * 4 + t) * 64 + lane] = acc[t];
          }
          barrier();
        }
        if (!KS || w == 0) {
          if (KS) {
#pragma unroll
            for (int v = 1; v < MX_WAVES; ++v)
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                const f32x4 p = red[(v * 4 + t) * 64 + lane];
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) acc[t][jj] += p[jj];
              }
          }
          const int rt = tile(cj);
          // Lane (token rr, q) holds rows 4q .. 4q+3 of each 16-row tile.
          if (rr < nt) {
            bf16* o = a.out + (size_t)m * a.out_ld;
            if (GLU) {
#pragma unroll
              for (int t = 0; t < 2; ++t) {
                const int ch = rt * 32 + 16 * t + 4 * q;
                if (ch < a.I) {
                  float iv[4];
#pragma unroll
                  for (int jj = 0; jj < 4; ++jj) iv[jj] = silu(acc[t][jj]) * acc[t + 2][jj];
                  Store4<bf16>::st(o + ch, iv[0], iv[1], iv[2], iv[3]);
                }
              }
            } else {
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                const int row = rt * MX_ROWS + 16 * t + 4 * q;
                if (row < a.R) Store4<bf16>::st(o + row, acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
              }
            }
          }
        }
        if (KS && RT > 1) barrier();  // wave 0 has read the exchange before the next tile writes it
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
      };
      auto advance = [&]() {
        if (++cc == nch) {
          finish_tile();
          ++cj;
          cc = 0;
        }
      };
      for (int it = 0; it < total; it += 2) {
        // Every two chunks the wave lets its loads drain (s_waitcnt vmcnt(0)) before it issues
        // the next chunk: measured ~1% faster over the whole weight stream than keeping one
        // chunk in flight throughout.
        __builtin_amdgcn_s_waitcnt(0x0F70);
        fetch(p1);
        compute(p0);
        advance();
        if (it + 1 >= total) break;
        fetch(p0);
        compute(p1);
        advance();
      }
    };
    if (x_lds) run(std::true_type{});
    else run(std::false_type{});
  }
}

}  // namespace moe

using namespace moe;

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Row tiles per block: several when the scale tables of that many tiles, the partial-sum
// exchange and at least 16 KB of token rows fit the block's LDS. The gate/up projection (long K)
// splits K over the waves, two tiles per block (level with one); the down projection (short K,
// K = I) gives each wave a tile of its own, four per block.
#ifndef MX_RT_GLU
#define MX_RT_GLU 2
#endif
#ifndef MX_RT_DOWN
#define MX_RT_DOWN 4
#endif
#ifndef MX_KS_DOWN
#define MX_KS_DOWN false
#endif
#ifndef MX_KS_GLU
#define MX_KS_GLU true
#endif
template <bool GLU>
static bool launch_mx(const MxArgs& a, int E, hipStream_t s) {
  constexpr int MX_RT = GLU ? MX_RT_GLU : MX_RT_DOWN;
  const int nc = a.K / 128;
  auto go = [&](auto kern, int rt) {
    const unsigned grid = (unsigned)(E * ((a.n_rtiles + rt - 1) / rt));
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, MX_LDS);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * MX_WAVES), MX_LDS, s, a);
  };
  constexpr bool KS = GLU ? MX_KS_GLU : MX_KS_DOWN;
  if (MX_RT > 1 && mx_x_offset(nc, MX_RT, KS) + 16384 <= MX_LDS) go(mx_gemm_kernel<GLU, MX_RT, KS>, MX_RT);
  else go(mx_gemm_kernel<GLU, 1, KS>, 1);
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
      ((uintptr_t)w13_scale & 3) || ((uintptr_t)w2_scale & 3))
    return MOE_ERR_ALIGN;
  // The scale tables of a block plus the partial sums (16 KB) must fit the block's LDS.
  if (mx_x_offset((int)(H / 128), 1, MX_KS_GLU) + MX_RED_BYTES > MX_LDS ||
      mx_x_offset((int)(I / 128), 1, MX_KS_DOWN) + MX_RED_BYTES > MX_LDS)
    return MOE_ERR_SHAPE;
  if ((int64_t)E * ((2 * I + 63) / 64) >= ((int64_t)1 << 31)) return MOE_ERR_SHAPE;
  // Row offsets within one expert's weights are 32-bit.
  if (2 * I * H >= ((int64_t)1 << 32)) return MOE_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  MxArgs g = {};
  g.W = (const uint8_t*)w13_q; g.w_e = 2 * I * H; g.w_ld = H;
  g.S = (const uint8_t*)w13_scale; g.s_e = 2 * I * (H / 32); g.s_ld = H / 32;
  g.R = (int)(2 * I); g.K = (int)H; g.I = (int)I;
  g.X = (const bf16*)hidden; g.x_ld = H; g.x_gather = sorted_token;
  g.offsets = offsets; g.n_rtiles = (int)((I + 31) / 32);  // 32 channels: 32 gate + 32 up rows
  g.out = (bf16*)inter; g.out_ld = I;
  if (!launch_mx<true>(g, E, s)) return MOE_ERR_LAUNCH;
  MxArgs d = {};
  d.W = (const uint8_t*)w2_q; d.w_e = H * I; d.w_ld = I;
  d.S = (const uint8_t*)w2_scale; d.s_e = H * (I / 32); d.s_ld = I / 32;
  d.R = (int)H; d.K = (int)I; d.I = (int)I;
  d.X = (const bf16*)inter; d.x_ld = I; d.x_gather = nullptr;
  d.offsets = offsets; d.n_rtiles = (int)((H + MX_ROWS - 1) / MX_ROWS);
  d.out = (bf16*)eo; d.out_ld = H;
  return launch_mx<false>(d, E, s) ? MOE_OK : MOE_ERR_LAUNCH;
}
