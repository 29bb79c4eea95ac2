// GDN fused recurrent forward (decode / speculative decode), GQA-native, with a
// slot-indexed fp32 (or bf16) state pool updated in place.
//
// Per sequence n, query head h, token t (reference kernel
// vllm-inference/src/primed_vllm/gdn/ops/fused_recurrent_gqa.py:111-144):
//   q,k <- q/sqrt(|q|^2+1e-6), k/sqrt(|k|^2+1e-6);  q <- q*scale
//   S <- exp(g) S;  u <- beta (v - S^T k);  S <- S + k u^T;  o <- S^T q
//
// Layout & mapping.  One workgroup per (sequence, head, 128 state columns) with
// up to 4 waves; wave w owns 32 state columns for all K rows, kept in registers for
// the whole token loop.  Lane l owns 4 consecutive columns (c = l&7) of
// R = K/8 rows r, r+8, ..., r+8(R-1) (r = l>>3).  One load instruction of the
// wave touches 8 consecutive rows x 128 contiguous bytes, so the four waves of a
// workgroup stream the head's K*V*4-byte state in contiguous 8-row blocks.  Column sums over
// k (S^T k, S^T q) are a per-lane partial over R rows plus a 3-step xor
// butterfly over the row-group lane bits — no LDS, no barriers.
//
// Roofline: HBM-bound read-modify-write of the state, 2*K*V*sizeof(state)
// bytes per (sequence, head) per call (q/k/v/o add 6*K*2 bytes).
#include <type_traits>

#include "common.hpp"

namespace hmx {

struct RecurrentParams {
  const void* q; const void* k; const void* v;
  int64_t q_ts, k_ts, v_ts;   // token strides (elements); heads are K (V for v) apart
  const void* g; int g_dt;
  const void* beta; int beta_dt; int beta_headwise;
  hmx_gate_proj gp;          // ProjG kernels: g, beta from the raw projections
  void* o;
  const void* h0; int64_t h0_rs;
  void* ht; int64_t ht_rs;
  const int32_t* cu_seqlens;
  const int32_t* idx; int64_t idx_stride;
  const int32_t* num_accepted;
  int64_t T;
  int H, HKV, V;
  float scale;
  int l2norm, inplace;
  // optional gated RMSNorm of each output row (NORM kernels; V <= 128)
  const void* zg; int64_t zg_ts, zg_hs;   // gate rows in q's dtype, or null
  const void* onw; int onw_dt;            // weight [V]
  float on_eps;
};

__device__ __forceinline__ float load_scalar(const void* p, int64_t i, int dtype) {
  return load_any(p, i, dtype);
}

// Loads of g and beta: a fixed element type (one code path, so the state and
// per-token loads of a thread are all in flight together), DynG (the dtype code
// decides at run time) or ProjG (formed from the layer's raw projections).
struct DynG {};
struct ProjG {};

template <typename TG>
__device__ __forceinline__ float load_gate(const void* p, int64_t i, int dtype) {
  if constexpr (std::is_same_v<TG, DynG>) return load_scalar(p, i, dtype);
  else return (float)static_cast<const TG*>(p)[i];
}

// Sum a value over the 8 row-group lanes (lane bits 3..5) of a wave.
__device__ __forceinline__ float rowgroup_sum(float x) {
  x += shfl_xor(x, 8);
  x += shfl_xor(x, 16);
  x += shfl_xor(x, 32);
  return x;
}

// NORM: each output row (one workgroup holds all V <= 128 columns) passes through
// the gated RMSNorm of hmx_rms_norm_gated (norm before gate) on its way out, from
// o as rounded to q's dtype; the sum of squares crosses the waves through LDS.
template <int K, typename TQ, typename TS, bool NORM, typename TG>
__global__ __launch_bounds__(256) void gdn_recurrent_kernel(RecurrentParams p) {
  constexpr int R = K / 8;  // rows per lane
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 7, r = lane >> 3;
  const int n = blockIdx.x / p.H;
  const int h = blockIdx.x - n * p.H;
  const int hk = h / (p.H / p.HKV);
  const int V = p.V;
  if ((int)(blockIdx.y * 4 + wave) * 32 >= p.V) return;  // tail workgroup of a V not a multiple of 128
  const int col = (blockIdx.y * 4 + wave) * 32 + c * 4;

  int64_t bos, T;
  if (p.cu_seqlens) {
    bos = p.cu_seqlens[n];
    T = (int64_t)p.cu_seqlens[n + 1] - bos;
  } else {
    bos = (int64_t)n * p.T;
    T = p.T;
  }
  if (T <= 0) return;

  // resolve state rows
  int64_t read_row = -1, write_row;
  if (p.h0) {
    if (p.idx) {
      const int64_t cidx = p.num_accepted ? (int64_t)p.num_accepted[n] - 1 : 0;
      read_row = p.idx[(int64_t)n * p.idx_stride + cidx];
      if (read_row < 0) return;
    } else {
      read_row = bos;
    }
  }
  if (p.inplace) {
    write_row = p.idx[(int64_t)n * p.idx_stride];
    if (write_row < 0) return;
  } else {
    write_row = bos;   // fused_recurrent_gqa.py:137-139: row bos of the [B*T] rows
  }

  __shared__ float part[2][4];   // NORM: per-wave sums of squares, by token parity
  float wn[4] = {0.f, 0.f, 0.f, 0.f};
  if (NORM) {
#pragma unroll
    for (int j = 0; j < 4; ++j) wn[j] = load_scalar(p.onw, col + j, p.onw_dt);
  }

  float S[R][4];
  if (read_row >= 0) {
    const TS* src = static_cast<const TS*>(p.h0) + read_row * p.h0_rs + (int64_t)h * K * V +
                    (int64_t)r * V + col;
#pragma unroll
    for (int i = 0; i < R; ++i) load_vec<4>(src + (int64_t)(8 * i) * V, S[i]);
  } else {
#pragma unroll
    for (int i = 0; i < R; ++i) S[i][0] = S[i][1] = S[i][2] = S[i][3] = 0.f;
  }

  for (int64_t t = 0; t < T; ++t) {
    const int64_t tok = bos + t;
    float kr[R], qr[R], vv[4], bb[4];
    {
      const TQ* kp = static_cast<const TQ*>(p.k) + tok * p.k_ts + (int64_t)hk * K + r;
      const TQ* qp = static_cast<const TQ*>(p.q) + tok * p.q_ts + (int64_t)h * K + r;
#pragma unroll
      for (int i = 0; i < R; ++i) {
        kr[i] = to_f32(kp[8 * i]);
        qr[i] = to_f32(qp[8 * i]);
      }
    }
    load_vec<4>(static_cast<const TQ*>(p.v) + tok * p.v_ts + (int64_t)hk * V + col, vv);
    float gt;
    if constexpr (std::is_same_v<TG, ProjG>) {
      gt = gp_g(p.gp, tok, h);
      bb[0] = bb[1] = bb[2] = bb[3] = gp_beta(p.gp, tok, h);
    } else {
    gt = load_gate<TG>(p.g, tok * p.H + h, p.g_dt);
    if (p.beta_headwise) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bb[j] = load_gate<TG>(p.beta, (tok * p.H + h) * V + col + j, p.beta_dt);
    } else {
      const float bs = load_gate<TG>(p.beta, tok * p.H + h, p.beta_dt);
      bb[0] = bb[1] = bb[2] = bb[3] = bs;
    }
    }

    float qs = p.scale;
    if (p.l2norm) {
      float sk = 0.f, sq = 0.f;
#pragma unroll
      for (int i = 0; i < R; ++i) { sk += kr[i] * kr[i]; sq += qr[i] * qr[i]; }
      sk = rowgroup_sum(sk);
      sq = rowgroup_sum(sq);
      const float ik = 1.0f / sqrtf(sk + 1e-6f);
#pragma unroll
      for (int i = 0; i < R; ++i) kr[i] *= ik;
      qs *= 1.0f / sqrtf(sq + 1e-6f);
    }
#pragma unroll
    for (int i = 0; i < R; ++i) qr[i] *= qs;

    const float eg = fast_exp(gt);
    float kv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < R; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        S[i][j] *= eg;
        kv[j] += S[i][j] * kr[i];
      }
    }
    float u[4], ov[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) u[j] = (vv[j] - rowgroup_sum(kv[j])) * bb[j];
#pragma unroll
    for (int i = 0; i < R; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        S[i][j] += kr[i] * u[j];
        ov[j] += S[i][j] * qr[i];
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) ov[j] = rowgroup_sum(ov[j]);
    if constexpr (NORM) {
      float zz[4] = {0.f, 0.f, 0.f, 0.f};
      if (p.zg) load_vec<4>(static_cast<const TQ*>(p.zg) + tok * p.zg_ts + h * p.zg_hs + col, zz);
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ov[j] = to_f32(from_f32<TQ>(ov[j]));   // o as the op returns it
        ss += ov[j] * ov[j];
      }
      ss += shfl_xor(ss, 1);
      ss += shfl_xor(ss, 2);
      ss += shfl_xor(ss, 4);
      if (lane == 0) part[t & 1][wave] = ss;
      __syncthreads();
      float tot = 0.f;
      for (int w = 0; w < (int)(blockDim.x >> 6); ++w) tot += part[t & 1][w];
      const float rstd = 1.0f / sqrtf(tot / V + p.on_eps);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ov[j] *= rstd * wn[j];
        if (p.zg) ov[j] *= zz[j] / (1.0f + expf(-zz[j]));
      }
    }
    if (r == 0) store_vec<4>(static_cast<TQ*>(p.o) + (tok * p.H + h) * V + col, ov);
  }

  TS* dst = static_cast<TS*>(p.ht) + write_row * p.ht_rs + (int64_t)h * K * V +
            (int64_t)r * V + col;
#pragma unroll
  for (int i = 0; i < R; ++i) store_vec_nt<4>(dst + (int64_t)(8 * i) * V, S[i]);
}

template <int K, typename TQ, typename TS, typename TG>
static void launch_g(const RecurrentParams& p, const dim3& grid, const dim3& block, hipStream_t s) {
  if (p.onw)
    hipLaunchKernelGGL((gdn_recurrent_kernel<K, TQ, TS, true, TG>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((gdn_recurrent_kernel<K, TQ, TS, false, TG>), grid, block, 0, s, p);
}

template <int K, typename TQ, typename TS>
static void launch(const RecurrentParams& p, int64_t N, hipStream_t s) {
  // at most 4 waves (128 state columns) per workgroup; wider V spans grid.y
  const int waves = p.V / 32;
  const dim3 grid((unsigned)(N * p.H), (unsigned)((waves + 3) / 4)),
      block(64 * (waves < 4 ? waves : 4));
  // typed g/beta paths for bf16 q/k/v with g and beta both fp32 or both bf16
  if (p.gp.a)
    launch_g<K, TQ, TS, ProjG>(p, grid, block, s);
  else if (std::is_same_v<TQ, bf16> && p.g_dt == p.beta_dt && p.g_dt == HMX_F32)
    launch_g<K, TQ, TS, float>(p, grid, block, s);
  else if (std::is_same_v<TQ, bf16> && p.g_dt == p.beta_dt && p.g_dt == HMX_BF16)
    launch_g<K, TQ, TS, bf16>(p, grid, block, s);
  else
    launch_g<K, TQ, TS, DynG>(p, grid, block, s);
}

template <int K, typename TQ>
static int dispatch_state(const RecurrentParams& p, int64_t N, int state_dt, hipStream_t s) {
  if (state_dt == HMX_F32) launch<K, TQ, float>(p, N, s);
  else if (state_dt == HMX_BF16) launch<K, TQ, bf16>(p, N, s);
  else return set_error(HMX_EUNSUPPORTED, "hmx_gdn_recurrent_fwd: state dtype %d", state_dt);
  return HMX_OK;
}

template <int K>
static int dispatch_qkv(const RecurrentParams& p, int64_t N, int qkv_dt, int state_dt,
                        hipStream_t s) {
  if (qkv_dt == HMX_BF16) return dispatch_state<K, bf16>(p, N, state_dt, s);
  if (qkv_dt == HMX_F16) return dispatch_state<K, f16>(p, N, state_dt, s);
  if (qkv_dt == HMX_F32) return dispatch_state<K, float>(p, N, state_dt, s);
  return set_error(HMX_EUNSUPPORTED, "hmx_gdn_recurrent_fwd: qkv dtype %d", qkv_dt);
}

}  // namespace hmx

extern "C" int hmx_gdn_recurrent_fwd(
    const void* q, int64_t q_token_stride, const void* k, int64_t k_token_stride, const void* v,
    int64_t v_token_stride, int32_t qkv_dtype, const void* g,
    int32_t g_dtype, const void* beta, int32_t beta_dtype, int32_t beta_headwise, void* o,
    const void* h0, int64_t h0_row_stride, void* ht, int64_t ht_row_stride, int32_t state_dtype,
    const int32_t* cu_seqlens, const int32_t* ssm_state_indices, int64_t idx_stride,
    const int32_t* num_accepted_tokens, int64_t B, int64_t T, int64_t N, int32_t H, int32_t HKV,
    int32_t K, int32_t V, float scale, int32_t use_qk_l2norm, int32_t inplace_final_state,
    const hmx_gated_norm* o_norm, const hmx_gate_proj* gates, void* stream) {
  using namespace hmx;
  HMX_REQUIRE(H > 0 && HKV > 0 && H % HKV == 0, HMX_EINVAL,
              "hmx_gdn_recurrent_fwd: H=%d must be a positive multiple of HKV=%d", H, HKV);
  if (gates) {
    const int rc = check_gates(gates, false, "hmx_gdn_recurrent_fwd");
    if (rc != HMX_OK) return rc;
    HMX_REQUIRE(!beta_headwise, HMX_EINVAL,
                "hmx_gdn_recurrent_fwd: gates give one beta per head (beta_headwise = 0)");
  }
  HMX_REQUIRE(K == 64 || K == 128 || K == 256, HMX_EUNSUPPORTED,
              "hmx_gdn_recurrent_fwd: K=%d not in {64,128,256}", K);
  HMX_REQUIRE(V > 0 && V % 32 == 0 && V <= 256, HMX_EUNSUPPORTED,
              "hmx_gdn_recurrent_fwd: V=%d must be a multiple of 32 and <= 256", V);
  HMX_REQUIRE(q && k && v && (gates || (g && beta)) && o && ht, HMX_EINVAL,
              "hmx_gdn_recurrent_fwd: null tensor pointer");
  HMX_REQUIRE(!inplace_final_state || ssm_state_indices, HMX_EINVAL,
              "hmx_gdn_recurrent_fwd: in-place final state needs ssm_state_indices");
  HMX_REQUIRE(!num_accepted_tokens || ssm_state_indices, HMX_EINVAL,
              "hmx_gdn_recurrent_fwd: num_accepted_tokens needs ssm_state_indices");
  HMX_REQUIRE(cu_seqlens || N == B, HMX_EINVAL,
              "hmx_gdn_recurrent_fwd: N=%lld must equal B=%lld without cu_seqlens",
              (long long)N, (long long)B);
  HMX_REQUIRE(gates || (g_dtype >= 0 && g_dtype <= 2 && beta_dtype >= 0 && beta_dtype <= 2),
              HMX_EUNSUPPORTED, "hmx_gdn_recurrent_fwd: g/beta dtype");
  HMX_REQUIRE(q_token_stride % 4 == 0 && k_token_stride % 4 == 0 && v_token_stride % 4 == 0 &&
                  ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) % 16 == 0,
              HMX_EINVAL, "hmx_gdn_recurrent_fwd: q/k/v token strides must be multiples of 4 "
              "elements and the bases 16-byte aligned");
  if (N == 0) return HMX_OK;
  RecurrentParams p;
  p.q = q; p.k = k; p.v = v; p.g = g; p.g_dt = g_dtype;
  p.q_ts = q_token_stride; p.k_ts = k_token_stride; p.v_ts = v_token_stride;
  p.beta = beta; p.beta_dt = beta_dtype; p.beta_headwise = beta_headwise;
  p.gp = gates ? *gates : hmx_gate_proj{};
  p.o = o; p.h0 = h0; p.h0_rs = h0_row_stride; p.ht = ht; p.ht_rs = ht_row_stride;
  p.cu_seqlens = cu_seqlens; p.idx = ssm_state_indices; p.idx_stride = idx_stride;
  p.num_accepted = num_accepted_tokens; p.T = T; p.H = H; p.HKV = HKV; p.V = V;
  p.scale = scale; p.l2norm = use_qk_l2norm; p.inplace = inplace_final_state;
  p.zg = nullptr; p.zg_ts = p.zg_hs = 0; p.onw = nullptr; p.onw_dt = HMX_F32; p.on_eps = 0.f;
  if (o_norm) {
    HMX_REQUIRE(V <= 128, HMX_EUNSUPPORTED,
                "hmx_gdn_recurrent_fwd: the fused output norm needs V <= 128 (got %d)", V);
    HMX_REQUIRE(o_norm->weight && o_norm->weight_dtype >= 0 && o_norm->weight_dtype <= 2,
                HMX_EINVAL, "hmx_gdn_recurrent_fwd: o_norm needs a weight (dtype code 0-2)");
    const int64_t vec = qkv_dtype == HMX_F32 ? 4 : 8;
    HMX_REQUIRE(!o_norm->gate || ((uintptr_t)o_norm->gate % 8 == 0 &&
                                  o_norm->gate_token_stride % vec == 0 &&
                                  o_norm->gate_head_stride % vec == 0),
                HMX_EINVAL, "hmx_gdn_recurrent_fwd: o_norm gate rows must be aligned");
    p.zg = o_norm->gate; p.zg_ts = o_norm->gate_token_stride; p.zg_hs = o_norm->gate_head_stride;
    p.onw = o_norm->weight; p.onw_dt = o_norm->weight_dtype; p.on_eps = o_norm->eps;
  }
  hipStream_t s = (hipStream_t)stream;
  int rc;
  if (K == 64) rc = dispatch_qkv<64>(p, N, qkv_dtype, state_dtype, s);
  else if (K == 128) rc = dispatch_qkv<128>(p, N, qkv_dtype, state_dtype, s);
  else rc = dispatch_qkv<256>(p, N, qkv_dtype, state_dtype, s);
  if (rc != HMX_OK) return rc;
  return check_launch("hmx_gdn_recurrent_fwd");
}
