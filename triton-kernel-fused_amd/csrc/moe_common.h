// Shared device helpers for the gfx950 MoE kernels: element types, 16-byte vector access,
// MFMA wrappers and the dtype / status codes of the C ABI (declared in include/moe_gfx950.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/moe_gfx950.h"

namespace moe {

typedef __bf16 bf16;
typedef _Float16 f16;

typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
typedef __attribute__((__vector_size__(8 * sizeof(int)))) int i32x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(f16 v) { return (float)v; }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) { return (bf16)v; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float v) { return (f16)v; }

// Round a float through T and back (the value a stored-then-reloaded T would have).
template <typename T> __device__ __forceinline__ float round_through(float v) {
  return to_f32(from_f32<T>(v));
}

// fp8 e4m3 (OCP "fn": bias 7, max 448, no infinities) operand tag; one byte per element.
struct fp8e4m3 { unsigned char bits; };

// MFMA traits per operand element type. A lane holds CPL 16-byte chunks of K per MFMA: the two
// lane halves (lanes 0-31 and 32-63) hold consecutive CPL-chunk runs, so one MFMA ("slab") spans
// 32*CPL bytes of K. Only the pairing of A and B elements matters to the sum, so any K order
// shared by both operands is valid. Operand P feeds the MFMA A side (rows of the 32x32 output),
// operand Q the B side (columns).
template <typename T> struct Mfma;

template <> struct Mfma<bf16> {
  static constexpr int VEC = 8;  // elements per 16 bytes
  static constexpr int CPL = 1;
  __device__ __forceinline__ static void step(f32x16& c, i32x4 a, i32x4 b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static void stepf(f32x16& c, const i32x4* a, const i32x4* b) {
    step(c, a[0], b[0]);
  }
  // 16x16x32: lane l holds row (A) / column (B) l%16, K values 8(l/16) .. 8(l/16)+7.
  __device__ __forceinline__ static void step(f32x4& c, i32x4 a, i32x4 b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static void stepf(f32x4& c, const i32x4* a, const i32x4* b) {
    step(c, a[0], b[0]);
  }
};

template <> struct Mfma<f16> {
  static constexpr int VEC = 8;
  static constexpr int CPL = 1;
  __device__ __forceinline__ static void step(f32x16& c, i32x4 a, i32x4 b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                               __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static void stepf(f32x16& c, const i32x4* a, const i32x4* b) {
    step(c, a[0], b[0]);
  }
  __device__ __forceinline__ static void step(f32x4& c, i32x4 a, i32x4 b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                               __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static void stepf(f32x4& c, const i32x4* a, const i32x4* b) {
    step(c, a[0], b[0]);
  }
};

template <> struct Mfma<float> {
  static constexpr int VEC = 4;
  static constexpr int CPL = 1;
  // v_mfma_f32_32x32x2f32 consumes one fp32 per lane and K=2 per instruction (one value per lane
  // half), so a 16-byte chunk (4 consecutive K values per lane) is four instructions.
  __device__ __forceinline__ static void step(f32x16& c, i32x4 a, i32x4 b) {
    // Bit-cast whole vectors: this compiler folds a bit-cast of a single vector element to
    // element 0, so per-element casts (vec[j]) must not be used.
    const f32x4 af = __builtin_bit_cast(f32x4, a), bf = __builtin_bit_cast(f32x4, b);
#pragma unroll
    for (int j = 0; j < 4; ++j) c = __builtin_amdgcn_mfma_f32_32x32x2f32(af[j], bf[j], c, 0, 0, 0);
  }
  __device__ __forceinline__ static void stepf(f32x16& c, const i32x4* a, const i32x4* b) {
    step(c, a[0], b[0]);
  }
};

// fp8 x fp8 on the gfx950 f8f6f4 MFMA (32x32x64, 32 e4m3 bytes per lane). The scaled form with
// both E8M0 scales = 127 (2^0) is the unscaled product; format code 0 = fp8 e4m3 for A and B.
template <> struct Mfma<fp8e4m3> {
  static constexpr int VEC = 16;
  static constexpr int CPL = 2;
  __device__ __forceinline__ static void stepf(f32x16& c, const i32x4* a, const i32x4* b) {
    const i32x8 a8 = __builtin_shufflevector(a[0], a[1], 0, 1, 2, 3, 4, 5, 6, 7);
    const i32x8 b8 = __builtin_shufflevector(b[0], b[1], 0, 1, 2, 3, 4, 5, 6, 7);
    c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, c, 0, 0, 0, 127, 0, 127);
  }
  // The same with a per-lane E8M0 scale for B: byte SEL of sb scales the 32 K values the lane
  // holds (one block of one B column); A unscaled.
  template <int SEL>
  __device__ __forceinline__ static void stepf_sb(f32x16& c, const i32x4* a, const i32x4* b,
                                                  unsigned sb) {
    const i32x8 a8 = __builtin_shufflevector(a[0], a[1], 0, 1, 2, 3, 4, 5, 6, 7);
    const i32x8 b8 = __builtin_shufflevector(b[0], b[1], 0, 1, 2, 3, 4, 5, 6, 7);
    c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, c, 0, 0, 0, 127, SEL, (int)sb);
  }
};

__device__ __forceinline__ i32x4 ldg16(const void* p) { return *(const i32x4*)p; }
__device__ __forceinline__ void stg16(void* p, i32x4 v) { *(i32x4*)p = v; }
__device__ __forceinline__ i32x4 zero4() { return i32x4{0, 0, 0, 0}; }

// sigma(g) = 1 / (1 + e^-g) with the hardware reciprocal (v_rcp_f32, 1 ulp) instead of an IEEE
// division sequence. A large negative finite g gives e^-g = inf, sigma = 0 and silu = -0; g = -inf
// gives silu = -inf * 0 = NaN, the same as with a division.
__device__ __forceinline__ float sigmoid(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}
__device__ __forceinline__ float silu(float g) { return g * sigmoid(g); }

// Compile-time loop: f(std::integral_constant<int, i>) for i in [I, N). Each iteration is its own
// code instance, so arrays indexed by the loop variable stay in registers however large the body.
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// 64-bit wave ballot.
__device__ __forceinline__ unsigned long long ballot64(bool p) { return __ballot(p); }

}  // namespace moe
