// Shared device/host helpers for libhmx (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "hmx.h"

namespace hmx {

// ----------------------------------------------------------------------------
// host-side error reporting (thread-local message, status codes from hmx.h)
// ----------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

#define HMX_REQUIRE(cond, code, ...)                 \
  do {                                               \
    if (!(cond)) return ::hmx::set_error(code, __VA_ARGS__); \
  } while (0)

// ----------------------------------------------------------------------------
// element types
// ----------------------------------------------------------------------------
typedef __bf16 bf16;
typedef _Float16 f16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(f16 x) { return (float)x; }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float x) { return (f16)x; }

// Loads N consecutive elements of type T starting at p (N*sizeof(T) must be a
// multiple of 4 and p suitably aligned) and widens them to float.
template <int N, typename T>
__device__ __forceinline__ void load_vec(const T* __restrict__ p, float* out) {
  if constexpr (sizeof(T) == 4) {
    static_assert(N % 4 == 0, "f32 vector loads are float4");
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      float4 t = *reinterpret_cast<const float4*>(p + i);
      out[i] = t.x; out[i + 1] = t.y; out[i + 2] = t.z; out[i + 3] = t.w;
    }
  } else {
    static_assert(N % 4 == 0, "16-bit vector loads are 4 elements (8 bytes)");
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      typedef T T4 __attribute__((ext_vector_type(4)));
      T4 t = *reinterpret_cast<const T4*>(p + i);
      out[i] = to_f32(t[0]); out[i + 1] = to_f32(t[1]);
      out[i + 2] = to_f32(t[2]); out[i + 3] = to_f32(t[3]);
    }
  }
}

// store_vec with non-temporal stores: for streams written once and not re-read
// by the same kernel (a recurrent state's write-back).
template <int N, typename T>
__device__ __forceinline__ void store_vec_nt(T* __restrict__ p, const float* in) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < N; i += 4)
      __builtin_nontemporal_store(f32x4{in[i], in[i + 1], in[i + 2], in[i + 3]},
                                  reinterpret_cast<f32x4*>(p + i));
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      typedef T T4 __attribute__((ext_vector_type(4)));
      T4 t;
      t[0] = from_f32<T>(in[i]); t[1] = from_f32<T>(in[i + 1]);
      t[2] = from_f32<T>(in[i + 2]); t[3] = from_f32<T>(in[i + 3]);
      __builtin_nontemporal_store(t, reinterpret_cast<T4*>(p + i));
    }
  }
}

template <int N, typename T>
__device__ __forceinline__ void store_vec(T* __restrict__ p, const float* in) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < N; i += 4)
      *reinterpret_cast<float4*>(p + i) = make_float4(in[i], in[i + 1], in[i + 2], in[i + 3]);
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      typedef T T4 __attribute__((ext_vector_type(4)));
      T4 t;
      t[0] = from_f32<T>(in[i]); t[1] = from_f32<T>(in[i + 1]);
      t[2] = from_f32<T>(in[i + 2]); t[3] = from_f32<T>(in[i + 3]);
      *reinterpret_cast<T4*>(p + i) = t;
    }
  }
}

// ----------------------------------------------------------------------------
// wave64 helpers
// ----------------------------------------------------------------------------
__device__ __forceinline__ float shfl_xor(float x, int mask) {
  return __shfl_xor(x, mask, 64);
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += shfl_xor(x, m);
  return x;
}

// exp via exp2 with the log2(e) factor folded in (hardware v_exp_f32).
__device__ __forceinline__ float fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// softplus with mamba's threshold (x for x > 20): max(x, 0) + log1p(e^{-|x|}),
// log1p by Goldberg's correction log(w) u / (w - 1), w = 1 + u (exact for u
// below w's rounding), on the hardware exp/log.
__device__ __forceinline__ float softplus20(float x) {
  if (x > 20.f) return x;
  const float u = fast_exp(-fabsf(x));
  const float w = 1.f + u;
  const float l1p = (w == 1.f) ? u : __logf(w) * (u / (w - 1.f));
  return fmaxf(x, 0.f) + l1p;
}

}  // namespace hmx
