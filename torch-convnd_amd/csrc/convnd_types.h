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
