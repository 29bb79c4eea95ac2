// Mixer gating kernels (elementwise over [num_tokens, num_heads]).
//  GDN: g = -exp(A_log) * softplus(a + dt_bias), beta = sigmoid(b)
//       (vllm-inference/src/primed_vllm/gdn/ops/fused_gdn_gating.py:66-76)
//  GKA: the same g, alpha = sigmoid(alpha_in), optional beta = sigmoid(b)
//       (vllm-inference/src/primed_vllm/primed_gka_layer.py:224-300)
// Inputs may be strided views of a fused projection.  One thread per
// (token, head), grid-stride loop; [num_heads] parameters come from L1.
#include "common.hpp"

namespace hmx {

__device__ __forceinline__ void store_any(void* p, int64_t i, int dtype, float x) {
  if (dtype == HMX_F32) static_cast<float*>(p)[i] = x;
  else if (dtype == HMX_BF16) static_cast<bf16*>(p)[i] = (bf16)x;
  else static_cast<f16*>(p)[i] = (f16)x;
}

__global__ __launch_bounds__(256) void gdn_gating_kernel(
    const void* __restrict__ A_log, int A_dt, const void* __restrict__ a, int64_t as0, int64_t as1,
    const void* __restrict__ b, int64_t bs0, int64_t bs1, int ab_dt,
    const void* __restrict__ dt_bias, int db_dt, void* __restrict__ g, void* __restrict__ beta,
    int out_dt, int64_t total, int H, float sp_beta, float threshold) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / H;
    const int h = (int)(i - t * H);
    const float x = load_any(a, t * as0 + h * as1, ab_dt) + load_any(dt_bias, h, db_dt);
    const float gv = gate_decay(load_any(A_log, h, A_dt), x, sp_beta, threshold);
    const float bv = gate_sigmoid(load_any(b, t * bs0 + h * bs1, ab_dt));
    store_any(g, i, out_dt, gv);
    store_any(beta, i, out_dt, bv);
  }
}

__global__ __launch_bounds__(256) void gka_gating_kernel(
    const void* __restrict__ A_log, int A_dt, const void* __restrict__ a, int64_t as0, int64_t as1,
    const void* __restrict__ ai, int64_t is0, int64_t is1, const void* __restrict__ b, int64_t bs0,
    int64_t bs1, int in_dt, const void* __restrict__ dt_bias, int db_dt, void* __restrict__ g,
    void* __restrict__ alpha, void* __restrict__ beta, int out_dt, int64_t total, int H,
    float sp_beta, float threshold) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / H;
    const int h = (int)(i - t * H);
    const float x = load_any(a, t * as0 + h * as1, in_dt) + load_any(dt_bias, h, db_dt);
    store_any(g, i, out_dt, gate_decay(load_any(A_log, h, A_dt), x, sp_beta, threshold));
    store_any(alpha, i, out_dt, gate_sigmoid(load_any(ai, t * is0 + h * is1, in_dt)));
    if (b) store_any(beta, i, out_dt, gate_sigmoid(load_any(b, t * bs0 + h * bs1, in_dt)));
  }
}

int check_gates(const hmx_gate_proj* gp, bool gka, const char* what) {
  auto dt_ok = [](int d) { return d == HMX_F32 || d == HMX_BF16 || d == HMX_F16; };
  HMX_REQUIRE(gp->a || !gp->A_log, HMX_EINVAL, "%s: gates.A_log needs gates.a", what);
  HMX_REQUIRE(!gp->A_log || (gp->dt_bias && dt_ok(gp->A_log_dtype) && dt_ok(gp->dt_bias_dtype)),
              HMX_EINVAL, "%s: gates.A_log needs gates.dt_bias (dtype codes 0-2)", what);
  HMX_REQUIRE(dt_ok(gp->in_dtype), HMX_EUNSUPPORTED, "%s: gates.in_dtype code %d", what,
              gp->in_dtype);
  HMX_REQUIRE(gp->softplus_beta > 0.f, HMX_EINVAL, "%s: gates.softplus_beta must be > 0", what);
  if (gka) {
    HMX_REQUIRE(gp->alpha_in || gp->alpha_zero, HMX_EINVAL, "%s: gates.alpha_in is NULL", what);
  } else {
    HMX_REQUIRE(gp->A_log && gp->b, HMX_EINVAL, "%s: GDN gates need A_log, a, dt_bias and b",
                what);
  }
  return HMX_OK;
}

}  // namespace hmx

extern "C" int hmx_gka_gating(const void* A_log, int32_t A_log_dtype, const void* a,
                              int64_t a_stride0, int64_t a_stride1, const void* alpha_in,
                              int64_t alpha_in_stride0, int64_t alpha_in_stride1, const void* b,
                              int64_t b_stride0, int64_t b_stride1, int32_t in_dtype,
                              const void* dt_bias, int32_t dt_bias_dtype, void* g, void* alpha,
                              void* beta_out, int32_t out_dtype, int64_t num_tokens,
                              int32_t num_heads, float sp_beta, float threshold, void* stream) {
  HMX_REQUIRE(num_tokens >= 0 && num_heads > 0, HMX_EINVAL, "hmx_gka_gating: bad sizes");
  for (int dt : {A_log_dtype, in_dtype, dt_bias_dtype, out_dtype})
    HMX_REQUIRE(dt == HMX_F32 || dt == HMX_BF16 || dt == HMX_F16, HMX_EUNSUPPORTED,
                "hmx_gka_gating: unsupported dtype code %d", dt);
  HMX_REQUIRE(A_log && a && alpha_in && dt_bias && g && alpha && (!b || beta_out), HMX_EINVAL,
              "hmx_gka_gating: null pointer");
  const int64_t total = num_tokens * num_heads;
  if (total == 0) return HMX_OK;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(hmx::gka_gating_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, A_log, A_log_dtype, a, a_stride0, a_stride1, alpha_in,
                     alpha_in_stride0, alpha_in_stride1, b, b_stride0, b_stride1, in_dtype, dt_bias,
                     dt_bias_dtype, g, alpha, beta_out, out_dtype, total, num_heads, sp_beta,
                     threshold);
  return hmx::check_launch("hmx_gka_gating");
}

extern "C" int hmx_gdn_gating(const void* A_log, int32_t A_log_dtype, const void* a,
                              int64_t a_stride0, int64_t a_stride1, const void* b,
                              int64_t b_stride0, int64_t b_stride1, int32_t ab_dtype,
                              const void* dt_bias, int32_t dt_bias_dtype, void* g, void* beta_out,
                              int32_t out_dtype, int64_t num_tokens, int32_t num_heads,
                              float sp_beta, float threshold, void* stream) {
  HMX_REQUIRE(num_tokens >= 0 && num_heads > 0, HMX_EINVAL,
              "hmx_gdn_gating: bad sizes num_tokens=%lld num_heads=%d", (long long)num_tokens,
              num_heads);
  for (int dt : {A_log_dtype, ab_dtype, dt_bias_dtype, out_dtype})
    HMX_REQUIRE(dt == HMX_F32 || dt == HMX_BF16 || dt == HMX_F16, HMX_EUNSUPPORTED,
                "hmx_gdn_gating: unsupported dtype code %d", dt);
  HMX_REQUIRE(A_log && a && b && dt_bias && g && beta_out, HMX_EINVAL,
              "hmx_gdn_gating: null pointer");
  const int64_t total = num_tokens * num_heads;
  if (total == 0) return HMX_OK;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(hmx::gdn_gating_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, A_log, A_log_dtype, a, a_stride0, a_stride1, b,
                     b_stride0, b_stride1, ab_dtype, dt_bias, dt_bias_dtype, g, beta_out,
                     out_dtype, total, num_heads, sp_beta, threshold);
  return hmx::check_launch("hmx_gdn_gating");
}
