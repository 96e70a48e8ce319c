// Element-type traits for the gfx950 kernels: storage type, accumulation type, and
// the 16-byte MFMA fragment of eight 16-bit values.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace convnd {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Acc {
  using type = float;
};
template <>
struct Acc<double> {
  using type = double;
};

template <typename A, typename T>
__device__ __forceinline__ A widen(T v) {
  return static_cast<A>(v);
}

template <typename T, typename A>
__device__ __forceinline__ T narrow(A v) {
  return static_cast<T>(v);
}

// fp32 operands on the bf16 MFMA: each value v splits into three bf16 parts taken by
// truncation (p0 = v with its low 16 bits cleared, p1 the same of v - p0, p2 of v - p0 - p1;
// every subtraction is exact), so v = p0 + p1 + p2 exactly for fp32 v and every part has
// the sign of v, |p1| < 2^-7 |v|, |p2| < 2^-15 |v|. A product x*w keeps the six part
// products (0,0) (0,1) (1,0) (0,2) (2,0) (1,1) accumulated in fp32 (the dropped ones are
// below 2^-21 |x w| together): the GEMM runs over six copies of the channel (or batch)
// dimension, the data operand contributing parts kSplitData[s] and the other operand parts
// kSplitOther[s].
// Non-finite values and the other operand: a non-finite v gives v in all three parts, and a
// part of a finite nonzero v that would be zero is replaced by p0 * 2^-40 (same sign), so
// every product that meets an infinity carries the sign of x*w and a zero only meets it
// where w or x itself is zero -- as in an fp32 GEMM (inf * 0 = NaN; inf * w = +-inf).
constexpr int kSplitProducts = 6;
__host__ __device__ __forceinline__ int split_data_part(int s) {
  return s == 2 || s == 5 ? 1 : (s == 4 ? 2 : 0);
}
__host__ __device__ __forceinline__ int split_other_part(int s) {
  return s == 1 || s == 5 ? 1 : (s == 3 ? 2 : 0);
}
// Part of image block s of a split-precision copy with part map `map` (kSplitDataMap ... in
// convnd_internal.h).
__host__ __device__ __forceinline__ int split_map_part(unsigned map, int s) {
  return static_cast<int>((map >> (4 * s)) & 15u);
}
__host__ __device__ __forceinline__ unsigned short bf16_part_bits(float v, int part) {
  const unsigned bits = __builtin_bit_cast(unsigned, v);
  const unsigned short b0 = static_cast<unsigned short>(bits >> 16);
  if (part == 0 || (bits & 0x7f800000u) == 0x7f800000u) return b0;  // p0, or inf / NaN
  const float p0 = __builtin_bit_cast(float, bits & 0xffff0000u);
  const float r1 = v - p0;
  const unsigned b1 = __builtin_bit_cast(unsigned, r1) & 0xffff0000u;
  const float r = part == 1 ? r1 : r1 - __builtin_bit_cast(float, b1);
  unsigned out = __builtin_bit_cast(unsigned, r) & 0xffff0000u;
  if ((out & 0x7fffffffu) == 0 && (bits & 0x7fffffffu) != 0)
    out = __builtin_bit_cast(unsigned, p0 * 0x1p-40f) & 0xffff0000u;
  return static_cast<unsigned short>(out >> 16);
}

// 16x16x32 MFMA with fp32 accumulation for the two 16-bit element types.
template <typename T>
struct Mfma16;

template <>
struct Mfma16<__bf16> {
  using frag = bf16x8;
  __device__ __forceinline__ static f32x4 run(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma16<_Float16> {
  using frag = f16x8;
  __device__ __forceinline__ static f32x4 run(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

}  // namespace convnd
