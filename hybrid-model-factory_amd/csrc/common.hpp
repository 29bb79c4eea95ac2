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


// ----------------------------------------------------------------------------
// gates from the layer's raw projections (hmx_gate_proj): one definition for the
// standalone gating kernels and the mixer kernels' fused loads, so both paths
// give the same values
// ----------------------------------------------------------------------------
// Element i of a tensor whose dtype is known only at run time.  Two 16-bit loads,
// the element's low and high halves (for a 16-bit type the same half twice), both in
// bounds for every dtype and issued unconditionally: a load inside a branch on the
// dtype would be waited for inside the branch (a full round trip per call), while
// here the wait lands at the value's first use and the loads overlap the caller's.
__device__ __forceinline__ float load_any(const void* p, int64_t i, int dtype) {
  const uint16_t* u = static_cast<const uint16_t*>(p);
  const bool f32 = dtype == HMX_F32;
  const int64_t e = f32 ? 2 * i : i;
  const uint32_t lo = u[e], hi = u[f32 ? e + 1 : e];
  const float vf = __uint_as_float(lo | (hi << 16));
  const float vb = __uint_as_float(lo << 16);
  const float vh = (float)__builtin_bit_cast(f16, (uint16_t)lo);
  return f32 ? vf : dtype == HMX_BF16 ? vb : vh;
}

// x as stored in a tensor of `dtype` and read back
__device__ __forceinline__ float round_to(float x, int dtype) {
  if (dtype == HMX_BF16) return (float)(bf16)x;
  if (dtype == HMX_F16) return (float)(f16)x;
  return x;
}

// log(1 + e^y) = max(y, 0) + log1p(e^{-|y|}), log1p by Goldberg's correction
// log(w) u / (w - 1), w = 1 + u (exact for u below w's rounding), on the hardware
// exp / log: a few fp32 ulps, cheap enough for the mixer kernels' gate loads
__device__ __forceinline__ float softplus_core(float y) {
  const float u = fast_exp(-fabsf(y));
  const float w = 1.f + u;
  const float l1p = (w == 1.f) ? u : __logf(w) * (u / (w - 1.f));
  return fmaxf(y, 0.f) + l1p;
}

// softplus with mamba's threshold (x for x > 20)
__device__ __forceinline__ float softplus20(float x) { return x > 20.f ? x : softplus_core(x); }

// -exp(A_log) * softplus(x), softplus(x) = log(1 + e^{beta x}) / beta, or x past
// the threshold (fused_gdn_gating.py:66-71); eA = exp(A_log)
__device__ __forceinline__ float gate_decay_e(float eA, float x, float sp_beta, float threshold) {
  const float bx = sp_beta * x;
  const float sp = (bx <= threshold) ? softplus_core(bx) / sp_beta : x;
  return -eA * sp;
}
__device__ __forceinline__ float gate_exp(float A_log) { return fast_exp(A_log); }
__device__ __forceinline__ float gate_decay(float A_log, float x, float sp_beta, float threshold) {
  return gate_decay_e(gate_exp(A_log), x, sp_beta, threshold);
}

__device__ __forceinline__ float gate_sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.0f + fast_exp(-x));
}

// the gates as the reference's gate tensors hold them, from the raw projection
// values a, b, alpha_in of one token (eA_h, dtb_h: the head's exp(A_log) and dt_bias)
__device__ __forceinline__ float gp_g_of(const hmx_gate_proj& gp, float a, float eA_h, float dtb_h) {
  return round_to(gate_decay_e(eA_h, a + dtb_h, gp.softplus_beta, gp.softplus_threshold),
                  gp.in_dtype);
}
__device__ __forceinline__ float gp_beta_of(const hmx_gate_proj& gp, float b) {
  const float s = round_to(gate_sigmoid(b), gp.in_dtype);
  return gp.beta_scale == 1.f ? s : round_to(s * gp.beta_scale, gp.in_dtype);
}
__device__ __forceinline__ float gp_alpha_of(const hmx_gate_proj& gp, float ai) {
  if (gp.alpha_zero) return 0.f;
  const float s = round_to(gate_sigmoid(ai), gp.in_dtype);
  return gp.alpha_add == 0.f ? s : round_to(s + gp.alpha_add, gp.in_dtype);
}
// the same, loading token t, head h
__device__ __forceinline__ float gp_g(const hmx_gate_proj& gp, int64_t t, int h) {
  if (!gp.A_log) return 0.f;
  return gp_g_of(gp, load_any(gp.a, t * gp.a_token_stride + h * gp.a_head_stride, gp.in_dtype),
                 gate_exp(load_any(gp.A_log, h, gp.A_log_dtype)),
                 load_any(gp.dt_bias, h, gp.dt_bias_dtype));
}
__device__ __forceinline__ float gp_beta(const hmx_gate_proj& gp, int64_t t, int h) {
  return gp_beta_of(gp, load_any(gp.b, t * gp.b_token_stride + h * gp.b_head_stride, gp.in_dtype));
}
__device__ __forceinline__ float gp_alpha(const hmx_gate_proj& gp, int64_t t, int h) {
  if (gp.alpha_zero) return 0.f;
  return gp_alpha_of(gp, load_any(gp.alpha_in, t * gp.alpha_token_stride + h * gp.alpha_head_stride,
                                  gp.in_dtype));
}

// host-side check of a gate descriptor
int check_gates(const hmx_gate_proj* gp, bool gka, const char* what);

}  // namespace hmx
