// Gated RMSNorm over rows of D elements (the GDN/GKA output norm o_norm(o, z)):
//   norm_before_gate:  out = x / sqrt(mean(x^2) + eps) * w * silu(z)
//   otherwise:         u = x silu(z);  out = u / sqrt(mean(u^2) + eps) * w
// fp32 arithmetic on the upcast inputs, one rounding to the output dtype
// (vLLM RMSNormGated / fla FusedRMSNormGated with group_size None; called at
// vllm-inference/src/primed_vllm/primed_gdn_layer.py:621-626 and
// primed_gka_layer.py:944-949).
//
// Layout: a row is held by D/8 consecutive lanes, 8 elements (one or two
// 16-byte vectors) each; the sum of squares is an xor butterfly over those
// lanes.  HBM-bound: x, z and out move once.
#include "common.hpp"

namespace hmx {
namespace gnorm {

__device__ __forceinline__ float silu(float z) {
  return z * __builtin_amdgcn_rcpf(1.0f + fast_exp(-z));
}

__device__ __forceinline__ float ld_w(const void* w, int i, int dt) {
  if (dt == HMX_F32) return static_cast<const float*>(w)[i];
  if (dt == HMX_BF16) return (float)static_cast<const bf16*>(w)[i];
  return (float)static_cast<const f16*>(w)[i];
}

template <typename T, int LPR>
__global__ __launch_bounds__(256) void rms_norm_gated_kernel(
    const T* __restrict__ x, int64_t xs, const T* __restrict__ z, int64_t zs,
    const void* __restrict__ w, int w_dt, T* __restrict__ out, int64_t os, int64_t rows,
    float eps, int before) {
  constexpr int D = 8 * LPR;
  constexpr int RPB = 256 / LPR;                // rows per workgroup pass
  const int sub = threadIdx.x % LPR, c0 = 8 * sub;
  float wv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) wv[j] = ld_w(w, c0 + j, w_dt);
  for (int64_t r = blockIdx.x * (int64_t)RPB + threadIdx.x / LPR; r < rows;
       r += (int64_t)gridDim.x * RPB) {
    float u[8], g[8];
    load_vec<8>(x + r * xs + c0, u);
    if (z) {
      load_vec<8>(z + r * zs + c0, g);
#pragma unroll
      for (int j = 0; j < 8; ++j) g[j] = silu(g[j]);
      if (!before) {
#pragma unroll
        for (int j = 0; j < 8; ++j) u[j] *= g[j];
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += u[j] * u[j];
#pragma unroll
    for (int m = LPR / 2; m >= 1; m >>= 1) ss += shfl_xor(ss, m);
    const float rstd = __builtin_amdgcn_rsqf(ss * (1.0f / D) + eps);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      u[j] *= rstd * wv[j];
      if (z && before) u[j] *= g[j];
    }
    store_vec<8>(out + r * os + c0, u);
  }
}

template <typename T>
void launch(const void* x, int64_t xs, const void* z, int64_t zs, const void* w, int w_dt,
            void* out, int64_t os, int64_t rows, int D, float eps, int before, hipStream_t s) {
  const int lpr = D / 8, rpb = 256 / lpr;
  const int64_t need = (rows + rpb - 1) / rpb;
  const int grid = (int)(need < 2048 ? need : 2048);
  const T* X = static_cast<const T*>(x);
  const T* Z = static_cast<const T*>(z);
  T* O = static_cast<T*>(out);
  if (lpr == 8)
    hipLaunchKernelGGL((rms_norm_gated_kernel<T, 8>), dim3(grid), dim3(256), 0, s, X, xs, Z, zs, w,
                       w_dt, O, os, rows, eps, before);
  else if (lpr == 16)
    hipLaunchKernelGGL((rms_norm_gated_kernel<T, 16>), dim3(grid), dim3(256), 0, s, X, xs, Z, zs,
                       w, w_dt, O, os, rows, eps, before);
  else
    hipLaunchKernelGGL((rms_norm_gated_kernel<T, 32>), dim3(grid), dim3(256), 0, s, X, xs, Z, zs,
                       w, w_dt, O, os, rows, eps, before);
}

}  // namespace gnorm
}  // namespace hmx

using namespace hmx;

extern "C" int hmx_rms_norm_gated(const void* x, int64_t x_row_stride, const void* z,
                                  int64_t z_row_stride, int32_t dtype, const void* weight,
                                  int32_t weight_dtype, void* out, int64_t out_row_stride,
                                  int64_t rows, int32_t D, float eps, int32_t norm_before_gate,
                                  void* stream) {
  HMX_REQUIRE(D == 64 || D == 128 || D == 256, HMX_EUNSUPPORTED,
              "hmx_rms_norm_gated: row length %d not in {64, 128, 256}", D);
  HMX_REQUIRE(dtype >= 0 && dtype <= 2 && weight_dtype >= 0 && weight_dtype <= 2,
              HMX_EUNSUPPORTED, "hmx_rms_norm_gated: dtype codes %d / %d", dtype, weight_dtype);
  HMX_REQUIRE(rows >= 0, HMX_EINVAL, "hmx_rms_norm_gated: rows %lld", (long long)rows);
  if (rows == 0) return HMX_OK;
  HMX_REQUIRE(x && weight && out, HMX_EINVAL, "hmx_rms_norm_gated: null pointer");
  const int64_t vec = dtype == HMX_F32 ? 4 : 8;   // elements per 16 bytes
  HMX_REQUIRE(x_row_stride % vec == 0 && out_row_stride % vec == 0 &&
                  (!z || z_row_stride % vec == 0),
              HMX_EINVAL, "hmx_rms_norm_gated: row strides must be multiples of 16 bytes");
  const uintptr_t al = (uintptr_t)x | (uintptr_t)out | (uintptr_t)z;
  HMX_REQUIRE(al % 16 == 0, HMX_EINVAL, "hmx_rms_norm_gated: pointers must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == HMX_BF16)
    gnorm::launch<bf16>(x, x_row_stride, z, z_row_stride, weight, weight_dtype, out,
                        out_row_stride, rows, D, eps, norm_before_gate, s);
  else if (dtype == HMX_F16)
    gnorm::launch<f16>(x, x_row_stride, z, z_row_stride, weight, weight_dtype, out,
                       out_row_stride, rows, D, eps, norm_before_gate, s);
  else
    gnorm::launch<float>(x, x_row_stride, z, z_row_stride, weight, weight_dtype, out,
                         out_row_stride, rows, D, eps, norm_before_gate, s);
  return check_launch("hmx_rms_norm_gated");
}
