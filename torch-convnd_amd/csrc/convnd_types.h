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

// fp32 operands on the bf16 MFMA: each value v splits into three bf16 parts (each the
// nearest bf16 of what the previous parts leave; every subtraction is exact), so
// v = p0 + p1 + p2 + r with |r| <= 2^-24 |v|. A product x*w keeps the six part products of
// order >= 2^-16 relative -- (0,0) (0,1) (1,0) (0,2) (2,0) (1,1) -- accumulated in fp32:
// the GEMM runs over six copies of the channel (or batch) dimension, the data operand
// contributing parts kSplitData[s] and the other operand parts kSplitOther[s].
constexpr int kSplitProducts = 6;
__device__ __forceinline__ int split_data_part(int s) {
  return s == 2 || s == 5 ? 1 : (s == 4 ? 2 : 0);
}
__device__ __forceinline__ int split_other_part(int s) {
  return s == 1 || s == 5 ? 1 : (s == 3 ? 2 : 0);
}
__device__ __forceinline__ unsigned short bf16_part_bits(float v, int part) {
  const __bf16 h0 = static_cast<__bf16>(v);
  float r = v;
  __bf16 h = h0;
  if (part >= 1) {
    r = v - static_cast<float>(h0);
    h = static_cast<__bf16>(r);
    if (part >= 2) h = static_cast<__bf16>(r - static_cast<float>(h));
  }
  return __builtin_bit_cast(unsigned short, h);
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
