// Device-side building blocks shared by the gfx950 paged-attention kernels.
//
// MFMA used throughout: v_mfma_f32_16x16x32_{bf16,f16} (CDNA4). Per lane l of a wave64,
// with j = l / 16 and n = l % 16:
//   A operand (16 x 32): row n,    k = 8j .. 8j+7   (8 packed 16-bit values)
//   B operand (32 x 16): column n, k = 8j .. 8j+7
//   C/D       (16 x 16): column n, rows 4j .. 4j+3  (4 fp32 values)
// The order of the 32 k-slots is free as long as A and B agree; the kernels use that
// freedom to keep every lane's global loads contiguous.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvh {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;

// Storage-type tags. `bits16` is the raw 16-bit encoding.
struct BF16 {
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    // one v_cvt_pk_bf16_f32 (round to nearest even)
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
  }
  static __device__ __forceinline__ float to_f32(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }
  // Two E4M3 values (bytes 0-1 of w, or 2-3 when HI) as a packed bf16 pair, low byte in the
  // low half; every E4M3 value is exact in bf16, so the conversion (scale 1) rounds nothing.
  template <bool HI>
  static __device__ __forceinline__ uint32_t from_fp8x2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, HI));
  }
  // acc + lo + hi of a packed pair (v_dot2_f32_bf16 against {1, 1})
  static __device__ __forceinline__ float dot2_ones(uint32_t x, float acc) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x), __builtin_bit_cast(bf16x2_t, 0x3f803f80u),
                                           acc, false);
  }
};

struct F16 {
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    // one packed conversion (round to nearest even)
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, f16x2_t));
  }
  static __device__ __forceinline__ float to_f32(uint16_t x) {
    return (float)__builtin_bit_cast(_Float16, x);
  }
  // Two E4M3 values as a packed fp16 pair (exact, as for bf16).
  template <bool HI>
  static __device__ __forceinline__ uint32_t from_fp8x2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.f, HI));
  }
  // acc + lo + hi of a packed pair (v_dot2_f32_f16 against {1, 1})
  static __device__ __forceinline__ float dot2_ones(uint32_t x, float acc) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x), __builtin_bit_cast(f16x2_t, 0x3c003c00u), acc, false);
  }
};

// OCP FP8 E4M3 (float8_e4m3fn, bias 7, no infinities, 0x7f / 0xff NaN, largest finite 448):
// the KV-cache storage format of the *_fp8 entry points. A value x is stored as
// e4m3(clamp(x / scale, -448, 448)) with round-to-nearest-even, PyTorch's
// (x.float() / scale).clamp(-448, 448).to(torch.float8_e4m3fn): an IEEE fp32 division, then
// a clamp that lets NaN through, then the conversion.
constexpr float kFp8Max = 448.f;

__device__ __forceinline__ float fp8_prep(float x, float scale) {
  const float y = x / scale;
  return y > kFp8Max ? kFp8Max : (y < -kFp8Max ? -kFp8Max : y);
}

// Four prepared values to four E4M3 bytes (a in byte 0); v_cvt_pk_fp8_f32 rounds to nearest
// even, and the inputs are already within range.
__device__ __forceinline__ uint32_t fp8_pack4(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// Interleave the low (SEL = 0) or high (SEL = 1) 16-bit halves of two dwords:
// result = {half(a), half(b)} with half(a) in the low 16 bits.
template <int SEL>
__device__ __forceinline__ uint32_t pick_halves(uint32_t a, uint32_t b) {
  // v_perm_b32 byte selectors: bytes 0-3 come from the second operand, 4-7 from the first.
  return SEL == 0 ? __builtin_amdgcn_perm(b, a, 0x05040100u) : __builtin_amdgcn_perm(b, a, 0x07060302u);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Cross-lane reductions over the four 16-lane groups (lanes n, n+16, n+32, n+48) with the
// CDNA4 VALU swaps (no LDS round trip). With both operands equal, v_permlane32_swap returns
// {x[l % 32], x[l % 32 + 32]} and v_permlane16_swap returns the even and the odd 16-lane row
// of each 32-lane half, so combining the pair reduces over lanes l ^ 32, then l ^ 16.
__device__ __forceinline__ float max_over_groups(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_over_groups(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Wave-uniform copies: values loaded through pointers the compiler cannot prove read-only
// land in VGPRs; readfirstlane moves them to SGPRs so that control flow on them is scalar.
__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ int64_t uni64(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ int64_t clamp64(int64_t x, int64_t lo, int64_t hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

}  // namespace kvh
