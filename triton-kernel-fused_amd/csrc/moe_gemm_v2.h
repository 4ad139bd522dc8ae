// Shared pieces of the 256x256 grouped GEMMs (the ring kernels of moe_gemm_v4.h, the fallback of
// moe_gemm_v3.h): tile constants, the swizzled LDS row layout, the direct-to-LDS load, and the
// epilogue staging through LDS.
//
// LDS layout: each operand tile is 256 rows x 128 bytes (one K step), unpadded, with the 16-byte
// chunk index XOR-ed by ((row >> 1) & 7). A row is half of the 64 four-byte banks, so even and
// odd rows use different halves and the XOR spreads 8 rows of each parity over all chunks: the
// MFMA operand reads (16 consecutive rows per 256-byte LDS cycle, one 16-byte chunk each) are
// conflict-free. A wave fills 8 whole rows with one direct-to-LDS load (global_load_lds_dwordx4:
// lane l writes bytes [16l, 16l+16) of a 1 KB block; the lane loads the global chunk that belongs
// in that slot).
#pragma once
#include "moe_common.h"

namespace moe {
namespace v2 {

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

constexpr int TILE = 256;        // rows of each operand tile (P and Q)
constexpr int WT = 128;          // rows of a wave's sub-tile
constexpr int TN = WT / 32;      // MFMA tiles per wave side (4)
constexpr int ROWB = 128;        // bytes per LDS row = one K step (64 16-bit or 128 fp8 values)
constexpr int BK = 64;           // K elements per step for 16-bit operands
template <typename T> constexpr int bk() { return ROWB / (int)sizeof(T); }
constexpr int OPB = TILE * ROWB; // 32 KB per operand per stage

__device__ __forceinline__ int swz(int row, int chunk) {
  return row * ROWB + ((chunk ^ ((row >> 1) & 7)) << 4);
}

// One direct-to-LDS load: lane l copies 16 bytes from g to LDS byte (l_base + 16 l); l_base is
// wave-uniform. Written as inline asm so that the compiler does not track it: its own tracking
// treats every later LDS read as dependent on every DMA in flight and waits for all of them,
// which would drain the pipeline each step. The K loops order these loads themselves with
// explicit vmcnt waits.
__device__ __forceinline__ void dma16(const void* g, char* l_base) {
  const unsigned m0 = (unsigned)(uintptr_t)(lds_void*)l_base;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(m0)
               : "memory", "m0");
}

// ---------------------------------------------------------------------------------------------
// Epilogue staging. The MFMA accumulator gives a lane four consecutive output channels of one
// output row, so storing it directly writes 8 bytes into each of 32 rows per instruction. Instead
// each wave writes its 128x128 block, rounded to T, into its own 32 KB of LDS transposed to
// [q][p] (q = MFMA column = output row, p = MFMA row = output channel; 256 bytes per q row, the
// 16-byte chunk index XOR-ed by (q & 15), so the 8-byte writes of 32 lanes cover all 64 banks
// once), and reads it back as 16-byte chunks with 16 lanes per row: every store instruction then
// writes whole 256-byte row segments.
constexpr int EPI_ROWB = WT * 2;  // bytes per staged row

template <typename T> __device__ __forceinline__ unsigned pack2(float a, float b);
template <> __device__ __forceinline__ unsigned pack2<bf16>(float a, float b) {
  return __builtin_bit_cast(unsigned, bf16x2{(bf16)a, (bf16)b});
}
template <> __device__ __forceinline__ unsigned pack2<f16>(float a, float b) {
  typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 h2;
  return __builtin_bit_cast(unsigned, h2{(f16)a, (f16)b});
}

// Eight 16-bit values of a 16-byte chunk as floats (whole-word conversions only).
template <typename T> __device__ __forceinline__ void unpack8(i32x4 v, float (&f)[8]);
template <> __device__ __forceinline__ void unpack8<bf16>(i32x4 v, float (&f)[8]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const unsigned u = (unsigned)v[w];
    f[2 * w] = __builtin_bit_cast(float, u << 16);
    f[2 * w + 1] = __builtin_bit_cast(float, u & 0xffff0000u);
  }
}
template <> __device__ __forceinline__ void unpack8<f16>(i32x4 v, float (&f)[8]) {
  typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 h2;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const h2 h = __builtin_bit_cast(h2, (unsigned)v[w]);
    f[2 * w] = (float)h[0];
    f[2 * w + 1] = (float)h[1];
  }
}
template <typename T> __device__ __forceinline__ i32x4 pack8(const float (&f)[8]) {
  return i32x4{(int)pack2<T>(f[0], f[1]), (int)pack2<T>(f[2], f[3]), (int)pack2<T>(f[4], f[5]),
               (int)pack2<T>(f[6], f[7])};
}

__device__ __forceinline__ int staged_off(int q, int c) { return q * EPI_ROWB + ((c ^ (q & 15)) << 4); }

// Write this wave's accumulators to its LDS block wl (the mainloop's last barrier has released
// the LDS). Channel p = ti*32 + 8g + 4h + j sits in chunk p/8 = 4ti + g, half h.
template <typename T, int TJ = TN>
__device__ __forceinline__ void stage_acc(const f32x16 (&acc)[TN][TJ], char* wl) {
  const int lane = threadIdx.x & 63, h = lane >> 5;
#pragma unroll
  for (int tj = 0; tj < TJ; ++tj) {
    const int q = tj * 32 + (lane & 31);
#pragma unroll
    for (int ti = 0; ti < TN; ++ti)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        uint2 v = {pack2<T>(acc[ti][tj][4 * g], acc[ti][tj][4 * g + 1]),
                   pack2<T>(acc[ti][tj][4 * g + 2], acc[ti][tj][4 * g + 3])};
        *(uint2*)(wl + staged_off(q, 4 * ti + g) + 8 * h) = v;
      }
  }
}

// The same for 16x16 MFMA tiles (acc[ti][tj]: lane l holds channels ti*16 + 4(l/16) + v, v < 4,
// of output row tj*16 + l%16): chunk 2ti + l/32, half (l/16) & 1. A 32-lane half writes each of
// its 16 rows' chunk once, all 64 banks.
template <typename T, int TI_, int TJ_>
__device__ __forceinline__ void stage_acc(const f32x4 (&acc)[TI_][TJ_], char* wl) {
  const int lane = threadIdx.x & 63, h = (lane >> 4) & 1, g = lane >> 5;
#pragma unroll
  for (int tj = 0; tj < TJ_; ++tj) {
    const int q = tj * 16 + (lane & 15);
#pragma unroll
    for (int ti = 0; ti < TI_; ++ti) {
      uint2 v = {pack2<T>(acc[ti][tj][0], acc[ti][tj][1]), pack2<T>(acc[ti][tj][2], acc[ti][tj][3])};
      *(uint2*)(wl + staged_off(q, 2 * ti + g) + 8 * h) = v;
    }
  }
}

__device__ __forceinline__ i32x4 staged(const char* wl, int q, int c) {
  return *(const i32x4*)(wl + staged_off(q, c));
}

// GEMM outputs are written once and read by a later kernel: stored nontemporal so they do not
// displace operand lines in L2 (measured 1-3% faster on the 256x256 GEMMs).
template <typename P>
__device__ __forceinline__ void st_stream(i32x4 v, P* p) {
  __builtin_nontemporal_store(v, (i32x4*)p);
}

// Plain store of a staged block of WQ rows: out row (row0 + q) gets channels ch0 + 8c .. +7 for
// the rows below row_end and channels below n_ch (a multiple of 8).
template <typename T, int WQ = WT>
__device__ __forceinline__ void store_staged(const char* wl, T* out, long long ld, int row0,
                                             int row_end, int ch0, int n_ch) {
  const int lane = threadIdx.x & 63, c = lane & 15;
  const int ch = ch0 + 8 * c;
#pragma unroll 8
  for (int it = 0; it < WQ / 4; ++it) {
    const int q = it * 4 + (lane >> 4);
    const i32x4 v = staged(wl, q, c);
    if (row0 + q < row_end && ch < n_ch) st_stream(v, out + (size_t)(row0 + q) * ld + ch);
  }
}

}  // namespace v2
}  // namespace moe
