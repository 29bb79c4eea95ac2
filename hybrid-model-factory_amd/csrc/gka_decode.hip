// GKA (Gated KalmaNet) decode step: fused h_kk update, Chebyshev ridge solve,
// alpha blend, h_kv update and readout, in place on slot-indexed state pools.
//
// Per sequence n (first token only) and head h
// (vllm-inference/src/primed_vllm/gka/ops/chebyshev_iteration_gqa.py:79-170):
//   q, k <- q/|q|, k/|k|;  k~ = (beta+1e-6) k;  v~ = (beta+1e-6) v
//   H <- e^{gk} H + k~ k~^T                       (stored)
//   f = |H|_F, lam = r f, tau = 2/(2lam+f), c = (f/(2lam+f)/2)^2
//   x = tau q, x_prev = 0, w = 2; num_iter x { w <- 1/(1-cw);
//       x, x_prev <- w x - tau w (H x + lam x - q) - (w-1) x_prev, x }
//   x <- q + alpha (x - q);  S <- e^{gk} S + k~ v~^T (stored);  o = scale S^T x
//
// Mapping: one 256-thread workgroup per (sequence, head); wave w owns state
// columns [32w, 32w+32) of both H and S, lane l owns 4 columns (l&7) of 16
// consecutive rows (l>>3), all in registers.  Column sums (H x, S^T x) are a
// per-lane partial plus a 3-step xor butterfly; the iterate x is exchanged
// through a double-buffered 128-float LDS vector, one barrier per iteration.
// Roofline: HBM-bound read-modify-write of two fp32 128x128 states (256 KiB
// per (sequence, head)) plus num_iter matvecs of 2*128^2 flops.
#include "common.hpp"

namespace hmx {
namespace gkad {

constexpr int D = 128;

// The decode's gates from the raw projections.
__device__ __forceinline__ void proj_gates(const hmx_gate_proj& gp, int64_t t, int h,
                                           float& alpha, float& egk, float& bscale) {
  alpha = gp_alpha(gp, t, h);
  egk = gp.gk_from_g ? expf(gp_g(gp, t, h)) : 1.0f;
  bscale = gp.b ? gp_beta(gp, t, h) + 1e-6f : 1.0f;
}

struct Params {
  const void* q; const void* k; const void* v;
  int64_t q_ts, k_ts, v_ts;           // token strides (elements); heads are D apart
  const void* alpha; int alpha_dt;
  const void* gk; int gk_dt;          // may be null (no decay)
  const void* beta; int beta_dt;      // may be null
  hmx_gate_proj gp; int fused;        // fused: alpha, gk, beta from the raw projections
  void* o;
  const float* hkk_in; float* hkk_out; int64_t hkk_in_rs, hkk_out_rs;
  const void* hkv_in; void* hkv_out; int64_t hkv_in_rs, hkv_out_rs;
  const int32_t* cu_seqlens;
  const int32_t* idx; int64_t idx_stride;
  int64_t T;
  int H, HKV;
  int num_iter;
  float ridge_ratio, scale;
  // optional gated RMSNorm of the output row (NORM kernels)
  const void* zg; int64_t zg_ts, zg_hs;   // gate rows in q's dtype, or null
  const void* onw; int onw_dt;            // weight [D]
  float on_eps;
};

__device__ __forceinline__ float ld_scalar(const void* p, int64_t i, int dt) {
  if (dt == HMX_F32) return static_cast<const float*>(p)[i];
  if (dt == HMX_BF16) return (float)static_cast<const bf16*>(p)[i];
  return (float)static_cast<const f16*>(p)[i];
}

__device__ __forceinline__ float rowgroup_sum(float x) {
  x += shfl_xor(x, 8);
  x += shfl_xor(x, 16);
  x += shfl_xor(x, 32);
  return x;
}

// NORM: the output row passes through the gated RMSNorm of hmx_rms_norm_gated
// (norm before gate), from o as rounded to q's dtype.
template <typename TQ, typename TKV, bool NORM>
__global__ __launch_bounds__(256) void gka_decode_kernel(Params p) {
  __shared__ float sx[2][D];
  __shared__ float sred[4];
  __shared__ float spart[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 7, r = lane >> 3;
  const int n = blockIdx.x / p.H, h = blockIdx.x - n * p.H;
  const int hk = h / (p.H / p.HKV);
  const int col = wave * 32 + c * 4;   // this lane's 4 columns
  const int row0 = r * 16;             // this lane's 16 rows

  int64_t bos, len;
  if (p.cu_seqlens) {
    bos = p.cu_seqlens[n];
    len = (int64_t)p.cu_seqlens[n + 1] - bos;
  } else {
    bos = (int64_t)n * p.T;
    len = p.T;
  }
  if (len <= 0) return;
  const int64_t slot = p.idx ? (int64_t)p.idx[(int64_t)n * p.idx_stride] : n;
  if (slot < 0) return;

  // ---- h_kk loads (issued first).  h_kv is loaded after the iteration, once
  // h_kk's registers are free: the iteration phase then holds one state, which
  // doubles the workgroups a CU keeps in flight.
  float Hs[16][4];
  {
    const float* hsrc = p.hkk_in + slot * p.hkk_in_rs + (int64_t)h * D * D + row0 * D + col;
#pragma unroll
    for (int i = 0; i < 16; ++i) load_vec<4>(hsrc + i * D, Hs[i]);
  }
  // ---- token inputs
  const TQ* qp = static_cast<const TQ*>(p.q) + bos * p.q_ts + (int64_t)h * D;
  const TQ* kp = static_cast<const TQ*>(p.k) + bos * p.k_ts + (int64_t)hk * D;
  const TQ* vp = static_cast<const TQ*>(p.v) + bos * p.v_ts + (int64_t)hk * D;
  float kr[16], qr[16], kc[4], qc[4], vc[4];
  load_vec<16>(kp + row0, kr);
  load_vec<16>(qp + row0, qr);
  load_vec<4>(kp + col, kc);
  load_vec<4>(qp + col, qc);
  load_vec<4>(vp + col, vc);
  const int64_t si = bos * p.H + h;
  float alpha, egk, bscale;
  if (p.fused) {          // the gates from the layer's raw projections
    proj_gates(p.gp, bos, h, alpha, egk, bscale);
  } else {
    alpha = ld_scalar(p.alpha, si, p.alpha_dt);
    egk = p.gk ? expf(ld_scalar(p.gk, si, p.gk_dt)) : 1.0f;
    bscale = p.beta ? ld_scalar(p.beta, si, p.beta_dt) + 1e-6f : 1.0f;
  }
  // The state updates below spell out their fused multiply-adds: every kernel
  // variant (with or without the output norm, gates loaded or formed) then rounds
  // them identically, whatever the compiler would contract in each.

  float sk = 0.f, sq = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) { sk += kr[i] * kr[i]; sq += qr[i] * qr[i]; }
  sk = rowgroup_sum(sk);
  sq = rowgroup_sum(sq);
  const float ik = bscale / sqrtf(sk), iq = 1.0f / sqrtf(sq);
#pragma unroll
  for (int i = 0; i < 16; ++i) { kr[i] *= ik; qr[i] *= iq; }
#pragma unroll
  for (int j = 0; j < 4; ++j) { kc[j] *= ik; qc[j] *= iq; vc[j] *= bscale; }

  // ---- H <- e^{gk} H + k~ k~^T, stored; |H|_F^2
  float fro2 = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      Hs[i][j] = __builtin_fmaf(kr[i], kc[j], Hs[i][j] * egk);
      fro2 += Hs[i][j] * Hs[i][j];
    }
  {
    float* hdst = p.hkk_out + slot * p.hkk_out_rs + (int64_t)h * D * D + row0 * D + col;
#pragma unroll
    for (int i = 0; i < 16; ++i) store_vec<4>(hdst + i * D, Hs[i]);
  }
  fro2 = wave_sum(fro2);
  if (lane == 0) sred[wave] = fro2;
  if (tid < D) sx[0][tid] = 0.f;
  __syncthreads();
  const float fro = sqrtf(sred[0] + sred[1] + sred[2] + sred[3]);
  const float lam = p.ridge_ratio * fro;
  const float inv_den = 1.0f / (2.0f * lam + fro);
  const float tau = 2.0f * inv_den;
  const float cc = (fro * inv_den * 0.5f) * (fro * inv_den * 0.5f);

  // ---- Chebyshev iteration; lanes keep x, x_prev for their 4 columns
  float xc[4], xp[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) { xc[j] = tau * qc[j]; xp[j] = 0.f; }
  float xr[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) xr[i] = tau * qr[i];
  float w = 2.0f;
  int buf = 0;
  for (int it = 0; it < p.num_iter; ++it) {
    // w <= 2 (c <= 1/4, omega <= 2): the hardware reciprocal (1 ulp) suffices
    w = __builtin_amdgcn_rcpf(1.0f - cc * w);
    float hx[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) hx[j] += xr[i] * Hs[i][j];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float hxj = rowgroup_sum(hx[j]);
      const float grad = tau * w * (hxj + lam * xc[j] - qc[j]) + (w - 1.0f) * xp[j];
      xp[j] = xc[j];
      xc[j] = w * xc[j] - grad;
    }
    buf ^= 1;
    if (r == 0) *reinterpret_cast<float4*>(&sx[buf][col]) = make_float4(xc[0], xc[1], xc[2], xc[3]);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const float4 t = *reinterpret_cast<const float4*>(&sx[buf][row0 + i]);
      xr[i] = t.x; xr[i + 1] = t.y; xr[i + 2] = t.z; xr[i + 3] = t.w;
    }
  }
  // ---- h_kv loads; k and q rows again (L2 hits) instead of keeping them live
  float Ss[16][4];
  {
    const TKV* ssrc = static_cast<const TKV*>(p.hkv_in) + slot * p.hkv_in_rs +
                      (int64_t)h * D * D + row0 * D + col;
#pragma unroll
    for (int i = 0; i < 16; ++i) load_vec<4>(ssrc + i * D, Ss[i]);
  }
  load_vec<16>(kp + row0, kr);
  load_vec<16>(qp + row0, qr);
#pragma unroll
  for (int i = 0; i < 16; ++i) { kr[i] *= ik; qr[i] *= iq; }
  // ---- alpha blend (rows), S update, readout o = scale S^T x
#pragma unroll
  for (int i = 0; i < 16; ++i) xr[i] = (qr[i] + alpha * (xr[i] - qr[i])) * p.scale;
  float ov[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      Ss[i][j] = __builtin_fmaf(kr[i], vc[j], Ss[i][j] * egk);
      ov[j] += Ss[i][j] * xr[i];
    }
  {
    TKV* sdst = static_cast<TKV*>(p.hkv_out) + slot * p.hkv_out_rs + (int64_t)h * D * D +
                row0 * D + col;
#pragma unroll
    for (int i = 0; i < 16; ++i) store_vec<4>(sdst + i * D, Ss[i]);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) ov[j] = rowgroup_sum(ov[j]);
  if constexpr (NORM) {
    float zz[4] = {0.f, 0.f, 0.f, 0.f};
    if (p.zg) load_vec<4>(static_cast<const TQ*>(p.zg) + bos * p.zg_ts + h * p.zg_hs + col, zz);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ov[j] = to_f32(from_f32<TQ>(ov[j]));   // o as the op returns it
      ss += ov[j] * ov[j];
    }
    ss += shfl_xor(ss, 1);
    ss += shfl_xor(ss, 2);
    ss += shfl_xor(ss, 4);
    if (lane == 0) spart[wave] = ss;
    __syncthreads();
    const float rstd = 1.0f / sqrtf((spart[0] + spart[1] + spart[2] + spart[3]) / D + p.on_eps);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ov[j] *= rstd * ld_scalar(p.onw, col + j, p.onw_dt);
      if (p.zg) ov[j] *= zz[j] / (1.0f + expf(-zz[j]));
    }
  }
  if (r == 0) store_vec<4>(static_cast<TQ*>(p.o) + (bos * p.H + h) * D + col, ov);
}

template <typename TQ, typename TKV>
static void launch(const Params& p, int64_t N, hipStream_t s) {
  if (p.onw)
    hipLaunchKernelGGL((gka_decode_kernel<TQ, TKV, true>), dim3((unsigned)(N * p.H)), dim3(256), 0,
                       s, p);
  else
    hipLaunchKernelGGL((gka_decode_kernel<TQ, TKV, false>), dim3((unsigned)(N * p.H)), dim3(256), 0,
                       s, p);
}

template <typename TQ>
static int dispatch_kv(const Params& p, int64_t N, int kv_dt, hipStream_t s) {
  if (kv_dt == HMX_F32)
    launch<TQ, float>(p, N, s);
  else if (kv_dt == HMX_BF16)
    launch<TQ, bf16>(p, N, s);
  else
    return set_error(HMX_EUNSUPPORTED, "hmx_gka_decode_fwd: h_kv dtype %d", kv_dt);
  return HMX_OK;
}

}  // namespace gkad
}  // namespace hmx

extern "C" int hmx_gka_decode_fwd(const void* q, int64_t q_token_stride, const void* k,
                                  int64_t k_token_stride, const void* v, int64_t v_token_stride,
                                  int32_t qkv_dtype,
                                  const void* alpha, int32_t alpha_dtype, const void* gk,
                                  int32_t gk_dtype, const void* beta, int32_t beta_dtype, void* o,
                                  const float* h_kk_in, int64_t h_kk_in_row_stride,
                                  float* h_kk_out, int64_t h_kk_out_row_stride,
                                  const void* h_kv_in, int64_t h_kv_in_row_stride, void* h_kv_out,
                                  int64_t h_kv_out_row_stride, int32_t h_kv_dtype,
                                  const int32_t* cu_seqlens, const int32_t* ssm_state_indices,
                                  int64_t idx_stride, int64_t B, int64_t T, int64_t N, int32_t H,
                                  int32_t HKV, int32_t D, int32_t V, int32_t num_iter,
                                  float ridge_ratio, float scale, const hmx_gated_norm* o_norm,
                                  const hmx_gate_proj* gates, void* stream) {
  using namespace hmx;
  if (gates) {
    const int rc = check_gates(gates, true, "hmx_gka_decode_fwd");
    if (rc != HMX_OK) return rc;
  }
  HMX_REQUIRE(D == gkad::D && V == gkad::D, HMX_EUNSUPPORTED,
              "hmx_gka_decode_fwd: only D == V == 128 is supported (got D=%d V=%d)", D, V);
  HMX_REQUIRE(H > 0 && HKV > 0 && H % HKV == 0, HMX_EINVAL,
              "hmx_gka_decode_fwd: H=%d must be a positive multiple of HKV=%d", H, HKV);
  HMX_REQUIRE(q && k && v && (alpha || gates) && o && h_kk_in && h_kk_out && h_kv_in && h_kv_out, HMX_EINVAL,
              "hmx_gka_decode_fwd: null tensor pointer");
  HMX_REQUIRE(num_iter >= 0, HMX_EINVAL, "hmx_gka_decode_fwd: num_iter=%d", num_iter);
  HMX_REQUIRE(cu_seqlens || N == B, HMX_EINVAL, "hmx_gka_decode_fwd: N != B without cu_seqlens");
  if (N == 0) return HMX_OK;
  gkad::Params p;
  HMX_REQUIRE(q_token_stride % 4 == 0 && k_token_stride % 4 == 0 && v_token_stride % 4 == 0 &&
                  ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) % 16 == 0,
              HMX_EINVAL, "hmx_gka_decode_fwd: q/k/v token strides must be multiples of 4 "
              "elements and the bases 16-byte aligned");
  p.q = q; p.k = k; p.v = v;
  p.q_ts = q_token_stride; p.k_ts = k_token_stride; p.v_ts = v_token_stride;
  p.alpha = alpha; p.alpha_dt = alpha_dtype; p.gk = gk; p.gk_dt = gk_dtype;
  p.beta = beta; p.beta_dt = beta_dtype; p.o = o;
  p.fused = gates != nullptr;
  p.gp = gates ? *gates : hmx_gate_proj{};
  p.hkk_in = h_kk_in; p.hkk_out = h_kk_out; p.hkk_in_rs = h_kk_in_row_stride;
  p.hkk_out_rs = h_kk_out_row_stride;
  p.hkv_in = h_kv_in; p.hkv_out = h_kv_out; p.hkv_in_rs = h_kv_in_row_stride;
  p.hkv_out_rs = h_kv_out_row_stride;
  p.cu_seqlens = cu_seqlens; p.idx = ssm_state_indices; p.idx_stride = idx_stride;
  p.T = T; p.H = H; p.HKV = HKV; p.num_iter = num_iter; p.ridge_ratio = ridge_ratio;
  p.scale = scale;
  p.zg = nullptr; p.zg_ts = p.zg_hs = 0; p.onw = nullptr; p.onw_dt = HMX_F32; p.on_eps = 0.f;
  if (o_norm) {
    HMX_REQUIRE(o_norm->weight && o_norm->weight_dtype >= 0 && o_norm->weight_dtype <= 2,
                HMX_EINVAL, "hmx_gka_decode_fwd: o_norm needs a weight (dtype code 0-2)");
    const int64_t vec = qkv_dtype == HMX_F32 ? 4 : 8;
    HMX_REQUIRE(!o_norm->gate || ((uintptr_t)o_norm->gate % 8 == 0 &&
                                  o_norm->gate_token_stride % vec == 0 &&
                                  o_norm->gate_head_stride % vec == 0),
                HMX_EINVAL, "hmx_gka_decode_fwd: o_norm gate rows must be aligned");
    p.zg = o_norm->gate; p.zg_ts = o_norm->gate_token_stride; p.zg_hs = o_norm->gate_head_stride;
    p.onw = o_norm->weight; p.onw_dt = o_norm->weight_dtype; p.on_eps = o_norm->eps;
  }
  hipStream_t s = (hipStream_t)stream;
  int rc;
  if (qkv_dtype == HMX_BF16) rc = gkad::dispatch_kv<bf16>(p, N, h_kv_dtype, s);
  else if (qkv_dtype == HMX_F16) rc = gkad::dispatch_kv<f16>(p, N, h_kv_dtype, s);
  else if (qkv_dtype == HMX_F32) rc = gkad::dispatch_kv<float>(p, N, h_kv_dtype, s);
  else rc = set_error(HMX_EUNSUPPORTED, "hmx_gka_decode_fwd: qkv dtype %d", qkv_dtype);
  if (rc != HMX_OK) return rc;
  return check_launch("hmx_gka_decode_fwd");
}
