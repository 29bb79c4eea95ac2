// Short causal depthwise conv1d (the mixers' input convolution), prefill and
// slot-indexed decode, for gfx950.
//
// Semantics (vLLM causal_conv1d_fn / causal_conv1d_update, un-vendored; called at
// vllm-inference/src/primed_vllm/primed_gdn_layer.py:700-780; torch form
// training/.../qwen3_5_moe_hmf/modeling_qwen3_5_moe_hmf.py:306-321), per channel c
// with width W <= 4:
//   out[t, c] = act(bias[c] + sum_i w[c, i] x[t - (W-1) + i, c])
// positions before a sequence's first token read its conv state (the previous
// inputs; zeros without an initial state), and afterwards the state holds the last
// state_len inputs.  State pool layout [slots, state_len, dim] with channels
// contiguous (primed_utils.py:174-177).
//
// Layout: a thread owns 8 consecutive channels (one 16-byte vector of a bf16 row)
// and walks a tile of tokens with the last W-1 inputs in registers; rows of x are
// read once.  The prefill writes the new states in a second launch, after every
// tile has read the old ones (a sequence's first tile reads its slot while its last
// tile would write it).  HBM-bound: x read once, out written once.
#include "common.hpp"

namespace hmx {
namespace conv {

constexpr int TT = 64;         // tokens per prefill tile
constexpr int NT = 256;        // threads per workgroup (2048 channels)

__device__ __forceinline__ float ld_any(const void* p, int64_t i, int dt) {
  if (dt == HMX_F32) return static_cast<const float*>(p)[i];
  if (dt == HMX_BF16) return (float)static_cast<const bf16*>(p)[i];
  return (float)static_cast<const f16*>(p)[i];
}

struct Params {
  const void* x; int64_t xs;          // [tokens, dim] rows
  void* out; int64_t os;
  const void* w; int w_dt; int W;     // [dim, W]
  const void* bias; int b_dt;         // [dim] or null
  void* st; int64_t st_slot, st_row; int st_len;   // [slots, st_len, dim] or null
  const int32_t* qs; int batch; int64_t total;
  const int32_t* idx;                 // slot per sequence, or null (slot = sequence)
  const uint8_t* has_init;            // per sequence, or null (all true)
  int dim, act, pad;
};

template <typename T>
struct Taps {
  float w[4][8], b[8];
  __device__ __forceinline__ void load(const Params& p, int c0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i][j] = i < p.W ? ld_any(p.w, (int64_t)(c0 + j) * p.W + i, p.w_dt) : 0.f;
      b[j] = p.bias ? ld_any(p.bias, c0 + j, p.b_dt) : 0.f;
    }
  }
  // window[0..2] = inputs at t-3..t-1 (taps shifted so tap W-1 is the current input)
  __device__ __forceinline__ void apply(const float (&win)[3][8], const float (&xt)[8], int W,
                                        int act, float (&y)[8]) const {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float a = b[j];
      // tap i reads t - (W-1) + i: the window row 3 - (W-1) + i for i < W-1, x_t for i = W-1
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const int r = 3 - (W - 1) + i;
        if (i < W - 1) a += w[i][j] * win[r][j];
      }
      a += w[W - 1][j] * xt[j];
      y[j] = act ? a / (1.0f + fast_exp(-a)) : a;
    }
  }
};

// sequence of token t: largest b with qs[b] <= t (non-empty sequences only)
__device__ __forceinline__ int seq_of(const int32_t* qs, int batch, int64_t t) {
  int lo = 0, hi = batch - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (qs[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

template <typename T>
__device__ __forceinline__ bool seq_slot(const Params& p, int b, int64_t& slot, bool& init) {
  slot = p.idx ? p.idx[b] : b;
  const bool ok = slot != p.pad;
  init = ok && p.st && (p.has_init ? p.has_init[b] != 0 : true);   // never read a pad slot
  return ok;
}

// The W-1 inputs before token t of sequence b (starting at token s): from x, or
// from the state rows (init), or zeros.
template <typename T>
__device__ __forceinline__ void load_window(const Params& p, int64_t t, int64_t s, int64_t slot,
                                            bool init, int c0, float (&win)[3][8]) {
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    const int64_t pos = t - 3 + r;   // window row r holds position t - 3 + r
#pragma unroll
    for (int j = 0; j < 8; ++j) win[r][j] = 0.f;
    if (pos >= s) {
      load_vec<8>(static_cast<const T*>(p.x) + pos * p.xs + c0, win[r]);
    } else if (init) {
      const int64_t row = p.st_len + (pos - s);   // state row of position pos (< 0 -> none)
      if (row >= 0)
        load_vec<8>(static_cast<const T*>(p.st) + slot * p.st_slot + row * p.st_row + c0, win[r]);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(NT) void conv_fwd_kernel(Params p) {
  const int c0 = (blockIdx.y * NT + threadIdx.x) * 8;
  if (c0 >= p.dim) return;
  const int64_t t0 = (int64_t)blockIdx.x * TT;
  const int64_t t1 = min(t0 + TT, p.total);
  Taps<T> tp;
  tp.load(p, c0);
  int b = seq_of(p.qs, p.batch, t0);
  int64_t s = p.qs[b], e = p.qs[b + 1];
  int64_t slot;
  bool init;
  bool ok = seq_slot<T>(p, b, slot, init);
  float win[3][8];
  load_window<T>(p, t0, s, slot, init, c0, win);
  for (int64_t t = t0; t < t1; ++t) {
    if (t >= e) {   // next non-empty sequence starts at t
      while (p.qs[b + 1] <= t) ++b;
      s = p.qs[b];
      e = p.qs[b + 1];
      ok = seq_slot<T>(p, b, slot, init);
      load_window<T>(p, t, s, slot, init, c0, win);
    }
    float xt[8], y[8];
    load_vec<8>(static_cast<const T*>(p.x) + t * p.xs + c0, xt);
    tp.apply(win, xt, p.W, p.act, y);
    if (!ok) {
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = 0.f;
    }
    store_vec<8>(static_cast<T*>(p.out) + t * p.os + c0, y);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      win[0][j] = win[1][j];
      win[1][j] = win[2][j];
      win[2][j] = xt[j];
    }
  }
}

// New prefill states: the last st_len inputs of each sequence (older state rows in
// front when it is shorter).  One thread per (sequence, 8 channels); each thread
// reads only its own slot's rows before writing them.
template <typename T>
__global__ __launch_bounds__(NT) void conv_state_kernel(Params p) {
  const int c0 = (blockIdx.y * NT + threadIdx.x) * 8;
  const int b = blockIdx.x;
  if (c0 >= p.dim) return;
  int64_t slot;
  bool init;
  if (!seq_slot<T>(p, b, slot, init)) return;
  const int64_t s = p.qs[b], e = p.qs[b + 1], len = e - s;
  if (len == 0) return;   // an empty sequence keeps its state
  float rows[8][8];       // st_len <= 8
  for (int r = 0; r < p.st_len; ++r) {
    const int64_t pos = e - p.st_len + r;   // sequence position of new state row r
#pragma unroll
    for (int j = 0; j < 8; ++j) rows[r & 7][j] = 0.f;
    if (pos >= s) {
      load_vec<8>(static_cast<const T*>(p.x) + pos * p.xs + c0, rows[r & 7]);
    } else if (init) {
      const int64_t row = p.st_len + (pos - s);
      if (row >= 0)
        load_vec<8>(static_cast<const T*>(p.st) + slot * p.st_slot + row * p.st_row + c0, rows[r & 7]);
    }
  }
  for (int r = 0; r < p.st_len; ++r)
    store_vec<8>(static_cast<T*>(p.st) + slot * p.st_slot + r * p.st_row + c0, rows[r & 7]);
}

// Decode: one token per sequence against its slot; the state shifts by one row.
template <typename T>
__global__ __launch_bounds__(NT) void conv_update_kernel(Params p) {
  const int c0 = (blockIdx.y * NT + threadIdx.x) * 8;
  const int b = blockIdx.x;
  if (c0 >= p.dim) return;
  const int64_t slot = p.idx ? p.idx[b] : b;
  T* orow = static_cast<T*>(p.out) + (int64_t)b * p.os + c0;
  if (slot == p.pad) {   // padded entry: zero output, no state access
    const float zero[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    store_vec<8>(orow, zero);
    return;
  }
  Taps<T> tp;
  tp.load(p, c0);
  T* srow = static_cast<T*>(p.st) + slot * p.st_slot + c0;
  float rows[8][8];   // st_len <= 8
  for (int r = 0; r < p.st_len; ++r) load_vec<8>(srow + r * p.st_row, rows[r & 7]);
  float win[3][8], xt[8], y[8];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    const int sr = p.st_len - 3 + r;   // window row r = state row st_len - 3 + r
#pragma unroll
    for (int j = 0; j < 8; ++j) win[r][j] = sr >= 0 ? rows[sr & 7][j] : 0.f;
  }
  load_vec<8>(static_cast<const T*>(p.x) + (int64_t)b * p.xs + c0, xt);
  tp.apply(win, xt, p.W, p.act, y);
  store_vec<8>(orow, y);
  for (int r = 0; r + 1 < p.st_len; ++r) store_vec<8>(srow + r * p.st_row, rows[(r + 1) & 7]);
  store_vec<8>(srow + (int64_t)(p.st_len - 1) * p.st_row, xt);
}

template <typename T>
void launch_fwd(const Params& p, hipStream_t s) {
  const unsigned cg = (unsigned)((p.dim / 8 + NT - 1) / NT);
  if (p.total > 0)
    hipLaunchKernelGGL(conv_fwd_kernel<T>, dim3((unsigned)((p.total + TT - 1) / TT), cg),
                       dim3(NT), 0, s, p);
  if (p.st && p.batch > 0)
    hipLaunchKernelGGL(conv_state_kernel<T>, dim3((unsigned)p.batch, cg), dim3(NT), 0, s, p);
}

template <typename T>
void launch_update(const Params& p, hipStream_t s) {
  const unsigned cg = (unsigned)((p.dim / 8 + NT - 1) / NT);
  hipLaunchKernelGGL(conv_update_kernel<T>, dim3((unsigned)p.batch, cg), dim3(NT), 0, s, p);
}

int check_common(const char* fn, int32_t dtype, int32_t width, int32_t dim, int32_t state_len,
                 int32_t weight_dtype, const void* bias, int32_t bias_dtype, int64_t xs,
                 int64_t os, int64_t st_row, int64_t st_slot, const void* st) {
  HMX_REQUIRE(dtype >= 0 && dtype <= 2, HMX_EUNSUPPORTED, "%s: dtype code %d", fn, dtype);
  HMX_REQUIRE(width >= 2 && width <= 4, HMX_EUNSUPPORTED, "%s: kernel width %d not in 2..4", fn,
              width);
  HMX_REQUIRE(dim > 0 && dim % 8 == 0, HMX_EUNSUPPORTED, "%s: dim %d must be a multiple of 8", fn,
              dim);
  HMX_REQUIRE(weight_dtype >= 0 && weight_dtype <= 2 && (!bias || (bias_dtype >= 0 && bias_dtype <= 2)),
              HMX_EUNSUPPORTED, "%s: weight/bias dtype", fn);
  const int64_t vec = dtype == HMX_F32 ? 4 : 8;
  HMX_REQUIRE(xs % vec == 0 && os % vec == 0 && (!st || (st_row % vec == 0 && st_slot % vec == 0)),
              HMX_EINVAL, "%s: token / state strides must be multiples of 16 bytes", fn);
  HMX_REQUIRE(!st || (state_len >= width - 1 && state_len <= 8), HMX_EUNSUPPORTED,
              "%s: state_len %d must be in [width-1, 8]", fn, state_len);
  return HMX_OK;
}

}  // namespace conv
}  // namespace hmx

using namespace hmx;
using namespace hmx::conv;

extern "C" int hmx_causal_conv1d_fwd(const void* x, int64_t x_token_stride, void* out,
                                     int64_t out_token_stride, int32_t dtype, const void* weight,
                                     int32_t weight_dtype, int32_t width, const void* bias,
                                     int32_t bias_dtype, void* conv_states,
                                     int64_t state_slot_stride, int64_t state_row_stride,
                                     int32_t state_len, const int32_t* query_start_loc,
                                     int32_t batch, int64_t total_tokens,
                                     const int32_t* cache_indices,
                                     const uint8_t* has_initial_state, int32_t dim,
                                     int32_t activation, int32_t pad_slot_id, void* stream) {
  // total_tokens must equal query_start_loc[batch] (the kernels walk sequences up to it)
  const int rc = check_common("hmx_causal_conv1d_fwd", dtype, width, dim, state_len, weight_dtype,
                              bias, bias_dtype, x_token_stride, out_token_stride, state_row_stride,
                              state_slot_stride, conv_states);
  if (rc != HMX_OK) return rc;
  HMX_REQUIRE(batch >= 0 && total_tokens >= 0, HMX_EINVAL, "hmx_causal_conv1d_fwd: sizes");
  if (batch == 0 || total_tokens == 0) return HMX_OK;
  HMX_REQUIRE(x && out && weight && query_start_loc, HMX_EINVAL,
              "hmx_causal_conv1d_fwd: null pointer");
  Params p{x, x_token_stride, out, out_token_stride, weight, weight_dtype, width, bias,
           bias_dtype, conv_states, state_slot_stride, state_row_stride,
           conv_states ? state_len : width - 1, query_start_loc, batch, total_tokens,
           cache_indices, has_initial_state, dim, activation, pad_slot_id};
  hipStream_t s = (hipStream_t)stream;
  if (dtype == HMX_BF16) launch_fwd<bf16>(p, s);
  else if (dtype == HMX_F16) launch_fwd<f16>(p, s);
  else launch_fwd<float>(p, s);
  return check_launch("hmx_causal_conv1d_fwd");
}

extern "C" int hmx_causal_conv1d_update(const void* x, int64_t x_token_stride, void* out,
                                        int64_t out_token_stride, int32_t dtype, const void* weight,
                                        int32_t weight_dtype, int32_t width, const void* bias,
                                        int32_t bias_dtype, void* conv_state,
                                        int64_t state_slot_stride, int64_t state_row_stride,
                                        int32_t state_len, const int32_t* conv_state_indices,
                                        int32_t batch, int32_t dim, int32_t activation,
                                        int32_t pad_slot_id, void* stream) {
  const int rc = check_common("hmx_causal_conv1d_update", dtype, width, dim, state_len,
                              weight_dtype, bias, bias_dtype, x_token_stride, out_token_stride,
                              state_row_stride, state_slot_stride, conv_state);
  if (rc != HMX_OK) return rc;
  HMX_REQUIRE(batch >= 0, HMX_EINVAL, "hmx_causal_conv1d_update: batch %d", batch);
  if (batch == 0) return HMX_OK;
  HMX_REQUIRE(x && out && weight && conv_state, HMX_EINVAL,
              "hmx_causal_conv1d_update: null pointer");
  Params p{x, x_token_stride, out, out_token_stride, weight, weight_dtype, width, bias,
           bias_dtype, conv_state, state_slot_stride, state_row_stride, state_len, nullptr,
           batch, batch, conv_state_indices, nullptr, dim, activation, pad_slot_id};
  hipStream_t s = (hipStream_t)stream;
  if (dtype == HMX_BF16) launch_update<bf16>(p, s);
  else if (dtype == HMX_F16) launch_update<f16>(p, s);
  else launch_update<float>(p, s);
  return check_launch("hmx_causal_conv1d_update");
}
