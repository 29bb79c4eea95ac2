// Mamba2 single-token state update (selective_state_update) for gfx950: an
// in-place read-modify-write of one slot of the SSM state pool per (sequence,
// head), HBM-bound on the state.
//
// Semantics (mamba_ssm / vLLM selective_state_update; reference calls at
// training/.../layers/mamba/mamba2.py:776-800 and
// vllm-inference/src/primed_vllm/primed_mamba2_layer.py:1000-1021):
//   d      = dt[p] + dt_bias[p]; d = softplus_20(d) if dt_softplus
//   S[p,n] = S[p,n] e^{A[p,n] d} + d x[p] B[n]
//   out[p] = sum_n S[p,n] C[n] + D[p] x[p];  out *= z sigmoid(z) if z is given
// The source slot is state_batch_indices[i] (or i); entries equal to
// pad_slot_id are skipped; the result goes to dst_state_batch_indices[i] when
// given, else back to the source slot.
//
// Layout: one 256-thread workgroup per (sequence, head).  Thread t owns the
// 4 consecutive n of columns 4 (t mod N/4) for rows p = t / (N/4) + k (1024/N),
// so every state load and store is a fully coalesced 16-byte (fp32) access.
#include <type_traits>

#include "common.hpp"
#include "mfma.hpp"

namespace hmx {
namespace ssdd {

// Sum over the GN lanes that share a state row (GN = 16: one DPP row; GN = 32:
// two rows combined by row_bcast:15 into the odd rows).  Valid in the row's
// leader lane: lane 16 of each 32 (GN = 32) or lane 0 of each 16.
template <int GN>
__device__ __forceinline__ float row_total(float x) {
  x = row16_sum(x);
  if constexpr (GN == 32)
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x142, 0xA, 0xF, false));
  return x;
}

constexpr int NTHR = 256;

struct Params {
  void* state; int64_t slot_stride;          // [slots][H][P][N], inner contiguous
  const void* x; int x_dt; int64_t x_bs, x_hs, x_ps;
  const void* dt; int dt_dt; int64_t dt_bs, dt_hs, dt_ps;
  const float* A; int64_t a_hs, a_ps, a_ns;  // fp32 [H][P][N] (any strides)
  const void* B; int b_dt; int64_t b_bs, b_gs;
  const void* C; int c_dt; int64_t c_bs, c_gs;
  const float* D; int64_t d_hs, d_ps;        // or null
  const float* dt_bias; int64_t db_hs, db_ps; // or null
  const void* z; int z_dt; int64_t z_bs, z_hs, z_ps;  // or null
  void* out; int out_dt; int64_t o_bs, o_hs, o_ps;
  const int* src_idx; const int* dst_idx; int pad_slot;
  // x has HX heads, B G groups and C GC groups (each divides H): head h reads
  // x head h / (H/HX), B group h / (H/G) and C group h / (H/GC).
  int H, HX, G, GC, softplus;
};

__device__ __forceinline__ float ld_any(const void* p, int64_t i, int dt) {
  if (dt == HMX_F32) return static_cast<const float*>(p)[i];
  if (dt == HMX_BF16) return (float)static_cast<const bf16*>(p)[i];
  return (float)static_cast<const f16*>(p)[i];
}

__device__ __forceinline__ void st_any(void* p, int64_t i, int dt, float v) {
  if (dt == HMX_F32) static_cast<float*>(p)[i] = v;
  else if (dt == HMX_BF16) static_cast<bf16*>(p)[i] = (bf16)v;
  else static_cast<f16*>(p)[i] = (f16)v;
}

// Element loads of the per-token operands: a fixed type (one code path, so every
// load of a thread is in flight at once), or Any (the dtype code decides).
struct Any {};

template <typename T>
__device__ __forceinline__ float ld_t(const void* p, int64_t i, int dt) {
  if constexpr (std::is_same_v<T, Any>) return ld_any(p, i, dt);
  else return (float)static_cast<const T*>(p)[i];
}

template <typename T>
__device__ __forceinline__ void st_t(void* p, int64_t i, int dt, float v) {
  if constexpr (std::is_same_v<T, Any>) st_any(p, i, dt, v);
  else static_cast<T*>(p)[i] = (T)v;
}

template <typename TS>
__device__ __forceinline__ f32x4 ld4(const TS* p) {
  if constexpr (sizeof(TS) == 4) {
    return *reinterpret_cast<const f32x4*>(p);
  } else {
    const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
    return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
  }
}

// The updated state is written once and not read again in this step:
// non-temporal stores keep it from displacing the state still being read.
template <typename TS>
__device__ __forceinline__ void st4(TS* p, const f32x4& v) {
  if constexpr (sizeof(TS) == 4) {
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
  } else {
    *reinterpret_cast<bf16x4*>(p) = bf16x4{(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
  }
}

// TIO: the type of x, B, C, z and out (Any: per-tensor dtype codes); TDT: dt's.
template <typename TS, int P, int N, bool A_TIED, typename TIO, typename TDT>
__global__ __launch_bounds__(NTHR) void ssd_state_update_kernel(Params p) {
  constexpr int GN = N / 4;            // threads per row
  constexpr int RPP = NTHR / GN;       // rows per pass
  constexpr int PASSES = P / RPP;
  const int i = blockIdx.x / p.H, h = blockIdx.x % p.H;
  const int g = h / (p.H / p.G), gc = h / (p.H / p.GC), hx = h / (p.H / p.HX);
  const int src = p.src_idx ? p.src_idx[i] : i;
  if (src == p.pad_slot) return;
  const int dst = p.dst_idx ? p.dst_idx[i] : src;
  const int tid = threadIdx.x, n0 = 4 * (tid % GN), r0 = tid / GN;

  float bv[4], cv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    bv[j] = ld_t<TIO>(p.B, (int64_t)i * p.b_bs + (int64_t)g * p.b_gs + n0 + j, p.b_dt);
    cv[j] = ld_t<TIO>(p.C, (int64_t)i * p.c_bs + (int64_t)gc * p.c_gs + n0 + j, p.c_dt);
  }
  const TS* sin = static_cast<const TS*>(p.state) + (int64_t)src * p.slot_stride + (int64_t)h * P * N;
  TS* sout = static_cast<TS*>(p.state) + (int64_t)dst * p.slot_stride + (int64_t)h * P * N;

  f32x4 st[PASSES];
#pragma unroll
  for (int k = 0; k < PASSES; ++k) st[k] = ld4(sin + (int64_t)(r0 + k * RPP) * N + n0);
  float xs[PASSES], ds[PASSES];
#pragma unroll
  for (int k = 0; k < PASSES; ++k) {
    const int pr = r0 + k * RPP;
    xs[k] = ld_t<TIO>(p.x, (int64_t)i * p.x_bs + (int64_t)hx * p.x_hs + (int64_t)pr * p.x_ps, p.x_dt);
    ds[k] = ld_t<TDT>(p.dt, (int64_t)i * p.dt_bs + (int64_t)h * p.dt_hs + (int64_t)pr * p.dt_ps, p.dt_dt);
  }

#pragma unroll
  for (int k = 0; k < PASSES; ++k) {
    const int pr = r0 + k * RPP;
    const float xv = xs[k];
    float d = ds[k];
    if (p.dt_bias) d += p.dt_bias[(int64_t)h * p.db_hs + (int64_t)pr * p.db_ps];
    if (p.softplus) d = softplus20(d);
    const float dx = d * xv;
    float acc = 0.f;
    if constexpr (A_TIED) {
      const float da = fast_exp(p.A[(int64_t)h * p.a_hs] * d);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        st[k][j] = st[k][j] * da + dx * bv[j];
        acc += st[k][j] * cv[j];
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = p.A[(int64_t)h * p.a_hs + (int64_t)pr * p.a_ps + (int64_t)(n0 + j) * p.a_ns];
        st[k][j] = st[k][j] * fast_exp(a * d) + dx * bv[j];
        acc += st[k][j] * cv[j];
      }
    }
    acc = row_total<GN>(acc);
    if (GN == 32 ? (tid & 31) == 16 : (tid & 15) == 0) {   // the row's leader lane
      float o = acc;
      if (p.D) o += p.D[(int64_t)h * p.d_hs + (int64_t)pr * p.d_ps] * xv;
      if (p.z) {
        const float zz = ld_t<TIO>(p.z, (int64_t)i * p.z_bs + (int64_t)h * p.z_hs + (int64_t)pr * p.z_ps, p.z_dt);
        o *= zz * __builtin_amdgcn_rcpf(1.f + fast_exp(-zz));
      }
      st_t<TIO>(p.out, (int64_t)i * p.o_bs + (int64_t)h * p.o_hs + (int64_t)pr * p.o_ps, p.out_dt, o);
    }
  }
#pragma unroll
  for (int k = 0; k < PASSES; ++k) st4(sout + (int64_t)(r0 + k * RPP) * N + n0, st[k]);
}

template <typename TS, int P, int N, typename TIO, typename TDT>
void launch_t(const Params& p, int batch, bool tied, hipStream_t s) {
  if (tied)
    hipLaunchKernelGGL((ssd_state_update_kernel<TS, P, N, true, TIO, TDT>), dim3(batch * p.H),
                       dim3(NTHR), 0, s, p);
  else
    hipLaunchKernelGGL((ssd_state_update_kernel<TS, P, N, false, TIO, TDT>), dim3(batch * p.H),
                       dim3(NTHR), 0, s, p);
}

// The layers' dtypes get fixed-type kernels: x, B, C, z and out all bf16 (or all
// fp32), dt bf16 or fp32; anything else takes the per-tensor dtype codes.
template <typename TS, int P, int N>
void launch(const Params& p, int batch, bool tied, hipStream_t s) {
  const int io = p.x_dt;
  const bool same = p.b_dt == io && p.c_dt == io && p.out_dt == io && (!p.z || p.z_dt == io);
  if (same && io == HMX_BF16 && p.dt_dt == HMX_BF16) launch_t<TS, P, N, bf16, bf16>(p, batch, tied, s);
  else if (same && io == HMX_BF16 && p.dt_dt == HMX_F32) launch_t<TS, P, N, bf16, float>(p, batch, tied, s);
  else if (same && io == HMX_F32 && p.dt_dt == HMX_F32) launch_t<TS, P, N, float, float>(p, batch, tied, s);
  else launch_t<TS, P, N, Any, Any>(p, batch, tied, s);
}

}  // namespace ssdd
}  // namespace hmx

using namespace hmx;
using namespace hmx::ssdd;

extern "C" int hmx_ssd_state_update(
    void* state, int32_t state_dtype, int64_t slot_stride, const void* x, int32_t x_dtype,
    int64_t x_bs, int64_t x_hs, int64_t x_ps, const void* dt, int32_t dt_dtype, int64_t dt_bs,
    int64_t dt_hs, int64_t dt_ps, const float* A, int64_t a_hs, int64_t a_ps, int64_t a_ns,
    const void* B, int32_t b_dtype, int64_t b_bs, int64_t b_gs, const void* C, int32_t c_dtype,
    int64_t c_bs, int64_t c_gs, const float* D, int64_t d_hs, int64_t d_ps, const float* dt_bias,
    int64_t db_hs, int64_t db_ps, const void* z, int32_t z_dtype, int64_t z_bs, int64_t z_hs,
    int64_t z_ps, void* out, int32_t out_dtype, int64_t o_bs, int64_t o_hs, int64_t o_ps,
    const int32_t* state_batch_indices, const int32_t* dst_state_batch_indices,
    int32_t pad_slot_id, int32_t batch, int32_t H, int32_t HX, int32_t G, int32_t GC, int32_t P,
    int32_t N,
    int32_t dt_softplus, void* stream) {
  HMX_REQUIRE(state_dtype == HMX_F32 || state_dtype == HMX_BF16, HMX_EUNSUPPORTED,
              "hmx_ssd_state_update: state must be float32 or bfloat16 (dtype code %d)", state_dtype);
  HMX_REQUIRE((P == 64 || P == 128) && (N == 64 || N == 128), HMX_EUNSUPPORTED,
              "hmx_ssd_state_update: headdim in {64,128} and d_state in {64,128} (got %d, %d)", P, N);
  HMX_REQUIRE(H > 0 && HX > 0 && G > 0 && GC > 0 && H % HX == 0 && H % G == 0 && H % GC == 0,
              HMX_EINVAL, "hmx_ssd_state_update: H=%d must be a multiple of HX=%d, G=%d and GC=%d",
              H, HX, G, GC);
  HMX_REQUIRE(state && x && dt && A && B && C && out, HMX_EINVAL,
              "hmx_ssd_state_update: null tensor pointer");
  HMX_REQUIRE(slot_stride % 4 == 0, HMX_EINVAL,
              "hmx_ssd_state_update: the state slot stride must be a multiple of 4 elements");
  if (batch == 0) return HMX_OK;
  Params p;
  p.state = state; p.slot_stride = slot_stride;
  p.x = x; p.x_dt = x_dtype; p.x_bs = x_bs; p.x_hs = x_hs; p.x_ps = x_ps;
  p.dt = dt; p.dt_dt = dt_dtype; p.dt_bs = dt_bs; p.dt_hs = dt_hs; p.dt_ps = dt_ps;
  p.A = A; p.a_hs = a_hs; p.a_ps = a_ps; p.a_ns = a_ns;
  p.B = B; p.b_dt = b_dtype; p.b_bs = b_bs; p.b_gs = b_gs;
  p.C = C; p.c_dt = c_dtype; p.c_bs = c_bs; p.c_gs = c_gs;
  p.D = D; p.d_hs = d_hs; p.d_ps = d_ps;
  p.dt_bias = dt_bias; p.db_hs = db_hs; p.db_ps = db_ps;
  p.z = z; p.z_dt = z_dtype; p.z_bs = z_bs; p.z_hs = z_hs; p.z_ps = z_ps;
  p.out = out; p.out_dt = out_dtype; p.o_bs = o_bs; p.o_hs = o_hs; p.o_ps = o_ps;
  p.src_idx = state_batch_indices; p.dst_idx = dst_state_batch_indices; p.pad_slot = pad_slot_id;
  p.H = H; p.HX = HX; p.G = G; p.GC = GC; p.softplus = dt_softplus;
  const bool tied = a_ps == 0 && a_ns == 0;
  hipStream_t s = (hipStream_t)stream;
#define HMX_SSDD(TS)                                          \
  if (P == 64 && N == 128) launch<TS, 64, 128>(p, batch, tied, s);        \
  else if (P == 128 && N == 128) launch<TS, 128, 128>(p, batch, tied, s); \
  else if (P == 64 && N == 64) launch<TS, 64, 64>(p, batch, tied, s);     \
  else launch<TS, 128, 64>(p, batch, tied, s);
  if (state_dtype == HMX_F32) { HMX_SSDD(float) } else { HMX_SSDD(bf16) }
#undef HMX_SSDD
  return check_launch("hmx_ssd_state_update");
}
