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
// read once.  Width and activation are template parameters so every register
// array is indexed at compile time (no scratch).  The prefill writes the new states in a second launch, after every
// tile has read the old ones (a sequence's first tile reads its slot while its last
// tile would write it).  HBM-bound: x read once, out written once.
#include "common.hpp"

namespace hmx {
namespace conv {

constexpr int TT = 64;         // tokens per prefill tile
constexpr int U = 8;           // rows loaded ahead per thread (memory-level parallelism)
constexpr int NT = 256;        // threads per workgroup (2048 channels)

// 8 consecutive channels: one 16-byte load for 16-bit rows, two for fp32
template <typename T>
__device__ __forceinline__ void ld8(const T* __restrict__ p, float (&o)[8]) {
  if constexpr (sizeof(T) == 4) {
    load_vec<8>(p, o);
  } else {
    typedef T T8 __attribute__((ext_vector_type(8)));
    const T8 v = *reinterpret_cast<const T8*>(p);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = to_f32(v[j]);
  }
}

template <typename T>
__device__ __forceinline__ void st8(T* __restrict__ p, const float (&y)[8]) {
  if constexpr (sizeof(T) == 4) {
    store_vec<8>(p, y);
  } else {
    typedef T T8 __attribute__((ext_vector_type(8)));
    T8 v;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = from_f32<T>(y[j]);
    *reinterpret_cast<T8*>(p) = v;
  }
}

struct Params {
  const void* x; int64_t xs;          // [tokens, dim] rows
  void* out; int64_t os;
  const void* w; int w_dt;            // [dim, W]
  const void* bias; int b_dt;         // [dim] or null
  void* st; int64_t st_slot, st_row; int st_len;   // [slots, st_len, dim] or null
  const int32_t* qs; int batch; int64_t total;
  const int32_t* idx;                 // slot per sequence, or null (slot = sequence)
  const uint8_t* has_init;            // per sequence, or null (none: every sequence starts from zeros)
  int dim, pad;
  int64_t tile0;                      // prefill: first token tile of this launch
  const int32_t* nacc;                // speculative update: accepted tokens per sequence
  // slot table rows: idx[b * idx_stride + column], idx_cols columns (1 and 1 for a
  // plain [batch] table).  Prefix caching (vLLM's block arguments) picks columns:
  int64_t idx_stride; int idx_cols;
  const int32_t* blk_in;              // column of the slot read (initial_state_idx), or null: 0
  const int32_t* blk_last;            // column of the slot written last (block_idx_last_scheduled_token)
  const int32_t* blk_first;           // prefill: block_idx_first_scheduled_token
  const int32_t* ncomp;               // prefill: tokens computed before this step
  int blk_size;                       // prefill: block_size_to_align
};

// Taps of 8 channels; the window holds the W-1 inputs before the current one
// (win[0] oldest), so tap i < W-1 reads win[i] and tap W-1 the current input.
template <int W, bool ACT>
struct Taps {
  float w[W][8], b[8];
  // The 8W weights of channels c0..c0+7 are contiguous ([dim, W] rows): vector
  // loads of one dtype branch, all in flight together.
  template <typename WT>
  __device__ __forceinline__ void load_t(const Params& p, int c0) {
    float f[8 * W];
    const WT* wp = static_cast<const WT*>(p.w) + (int64_t)c0 * W;
#pragma unroll
    for (int k = 0; k < W; ++k) {
      float v[8];
      ld8(wp + 8 * k, v);
#pragma unroll
      for (int j = 0; j < 8; ++j) f[8 * k + j] = v[j];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < W; ++i) w[i][j] = f[j * W + i];
  }
  template <typename BT>
  __device__ __forceinline__ void load_b(const Params& p, int c0) {
    ld8(static_cast<const BT*>(p.bias) + c0, b);
  }
  __device__ __forceinline__ void load(const Params& p, int c0) {
    if (p.w_dt == HMX_F32) load_t<float>(p, c0);
    else if (p.w_dt == HMX_BF16) load_t<bf16>(p, c0);
    else load_t<f16>(p, c0);
    if (!p.bias) {
#pragma unroll
      for (int j = 0; j < 8; ++j) b[j] = 0.f;
    } else if (p.b_dt == HMX_F32) load_b<float>(p, c0);
    else if (p.b_dt == HMX_BF16) load_b<bf16>(p, c0);
    else load_b<f16>(p, c0);
  }
  __device__ __forceinline__ void apply(const float (&win)[W - 1][8], const float (&xt)[8],
                                        float (&y)[8]) const {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float a = b[j];
#pragma unroll
      for (int i = 0; i < W - 1; ++i) a += w[i][j] * win[i][j];
      a += w[W - 1][j] * xt[j];
      y[j] = ACT ? a * __builtin_amdgcn_rcpf(1.0f + fast_exp(-a)) : a;
    }
  }
};

template <int W>
__device__ __forceinline__ void shift_in(float (&win)[W - 1][8], const float (&xt)[8]) {
#pragma unroll
  for (int i = 0; i + 1 < W - 1; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) win[i][j] = win[i + 1][j];
#pragma unroll
  for (int j = 0; j < 8; ++j) win[W - 2][j] = xt[j];
}

// Token range [s, e) of sequence b, clamped to [0, total) so that a malformed
// query_start_loc (not checked on the host, which would need a device sync) cannot
// move an access outside x; identity for a well-formed one.
__device__ __forceinline__ void seq_range(const Params& p, int b, int64_t& s, int64_t& e) {
  s = min(max((int64_t)p.qs[b], (int64_t)0), p.total);
  e = min(max((int64_t)p.qs[b + 1], s), p.total);
}

// sequence of token t: largest b with qs[b] <= t (non-empty sequences only)
__device__ __forceinline__ int seq_of(const int32_t* qs, int batch, int64_t t) {
  int lo = 0, hi = batch - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (qs[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Slot of sequence b at table column col[b] (column 0 when col is null), the
// column clamped into the table.
__device__ __forceinline__ int64_t slot_col(const Params& p, int b, const int32_t* col) {
  if (!p.idx) return b;
  const int c = col ? min(max(col[b], 0), p.idx_cols - 1) : 0;
  return p.idx[(int64_t)b * p.idx_stride + c];
}

// The slot sequence b reads its initial state from; false for a padded entry (its
// written slot is pad_slot_id: zero output, no state access).
__device__ __forceinline__ bool seq_slot(const Params& p, int b, int64_t& slot, bool& init) {
  slot = slot_col(p, b, p.blk_in);
  const int64_t wslot = p.blk_last ? slot_col(p, b, p.blk_last) : slot;
  const bool ok = wslot != p.pad;
  // never read a pad slot
  init = ok && slot != p.pad && p.st && p.has_init && p.has_init[b] != 0;
  return ok;
}

// The W-1 inputs before token t of sequence b (starting at token s): from x, or
// from the state rows (init), or zeros.
template <typename T, int W>
__device__ __forceinline__ void load_window(const Params& p, int64_t t, int64_t s, int64_t slot,
                                            bool init, int c0, float (&win)[W - 1][8]) {
#pragma unroll
  for (int r = 0; r < W - 1; ++r) {
    const int64_t pos = t - (W - 1) + r;   // window row r holds position t - (W-1) + r
#pragma unroll
    for (int j = 0; j < 8; ++j) win[r][j] = 0.f;
    if (pos >= s) {
      ld8(static_cast<const T*>(p.x) + pos * p.xs + c0, win[r]);
    } else if (init) {
      const int64_t row = p.st_len + (pos - s);   // state row of position pos (< 0 -> none)
      if (row >= 0) ld8(static_cast<const T*>(p.st) + slot * p.st_slot + row * p.st_row + c0, win[r]);
    }
  }
}

// Prefill: a workgroup owns TT tokens x 2048 channels; each thread walks its 8
// channels through the tile, loading U rows ahead before computing them.  Token
// and sequence indices are uniform across the workgroup, so the sequence-boundary
// branch is scalar.
template <typename T, int W, bool ACT>
__global__ __launch_bounds__(NT) void conv_fwd_kernel(Params p) {
  const int c0 = (blockIdx.x * NT + threadIdx.x) * 8;
  if (c0 >= p.dim) return;
  const int64_t t0 = (p.tile0 + blockIdx.y) * TT;
  const int64_t t1 = min(t0 + TT, p.total);
  Taps<W, ACT> tp;
  tp.load(p, c0);
  // tokens from qs[batch] on belong to no sequence: zero output
  const int64_t tend = min(max((int64_t)p.qs[p.batch], (int64_t)0), p.total);
  int b = 0;
  int64_t s = 0, e = p.total, slot = 0;
  bool init = false, ok = false;
  float win[W - 1][8];
  if (t0 < tend) {
    b = seq_of(p.qs, p.batch, t0);
    seq_range(p, b, s, e);
    ok = seq_slot(p, b, slot, init);
    load_window<T, W>(p, t0, s, slot, init, c0, win);
  } else {
#pragma unroll
    for (int r = 0; r < W - 1; ++r)
#pragma unroll
      for (int j = 0; j < 8; ++j) win[r][j] = 0.f;
  }
  const T* __restrict__ xp = static_cast<const T*>(p.x) + c0;
  T* __restrict__ op = static_cast<T*>(p.out) + c0;
  for (int64_t tb = t0; tb < t1; tb += U) {
    // unconditional loads (rows past the tile end re-read its last row, unused) so
    // all U are in flight before the first is converted
    float xt[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) ld8(xp + min(tb + u, t1 - 1) * p.xs, xt[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = tb + u;
      if (t < t1) {
        if (t >= e) {
          if (t >= tend) {   // past the last sequence
            ok = false;
            e = p.total;
          } else {           // next non-empty sequence starts at t
            while (b + 1 < p.batch && p.qs[b + 1] <= t) ++b;
            seq_range(p, b, s, e);
            ok = seq_slot(p, b, slot, init);
            load_window<T, W>(p, t, s, slot, init, c0, win);
          }
        }
        float y[8];
        tp.apply(win, xt[u], y);
        if (!ok) {
#pragma unroll
          for (int j = 0; j < 8; ++j) y[j] = 0.f;
        }
        st8(op + t * p.os, y);
        shift_in<W>(win, xt[u]);
      }
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
  if (!seq_slot(p, b, slot, init)) return;
  int64_t s, e;
  seq_range(p, b, s, e);
  if (e == s) return;     // an empty sequence keeps its state
  float rows[8][8];       // st_len <= 8
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    if (r < p.st_len) {
      const int64_t pos = e - p.st_len + r;   // sequence position of new state row r
#pragma unroll
      for (int j = 0; j < 8; ++j) rows[r][j] = 0.f;
      if (pos >= s) {
        ld8(static_cast<const T*>(p.x) + pos * p.xs + c0, rows[r]);
      } else if (init) {
        const int64_t row = p.st_len + (pos - s);
        if (row >= 0) ld8(static_cast<const T*>(p.st) + slot * p.st_slot + row * p.st_row + c0, rows[r]);
      }
    }
  }
  T* srow = static_cast<T*>(p.st) + slot * p.st_slot + c0;
#pragma unroll
  for (int r = 0; r < 8; ++r)
    if (r < p.st_len) st8(srow + r * p.st_row, rows[r]);
}

// New prefill states with prefix caching (vLLM's block arguments, as the Mamba2
// layer passes them, vllm-inference/src/primed_vllm/primed_mamba2_layer.py:770-792):
// sequence b's tokens continue ncomp[b] computed ones, and the blocks of
// blk_size tokens from blk_first[b] to blk_last[b] - 1 end inside this step.  Block
// k's slot (table column k) receives the state at its end, the last st_len inputs
// before absolute position (k + 1) * blk_size; column blk_last[b] receives the state
// after the sequence's last token.  Rows before the sequence's first token come
// from the initial state (zeros without one), read into registers before any row is
// written (the read slot may be one of the written ones).  The block range is
// clamped to the table's columns, so the loop is bounded.
template <typename T>
__global__ __launch_bounds__(NT) void conv_state_blocks_kernel(Params p) {
  const int c0 = (blockIdx.y * NT + threadIdx.x) * 8;
  const int b = blockIdx.x;
  if (c0 >= p.dim) return;
  int64_t rslot;
  bool init;
  if (!seq_slot(p, b, rslot, init)) return;
  int64_t s, e;
  seq_range(p, b, s, e);
  if (e == s) return;     // an empty sequence keeps its state
  const int L = p.st_len;
  float old[8][8];        // the initial state's rows, st_len <= 8
#pragma unroll
  for (int r = 0; r < 8; ++r) {
#pragma unroll
    for (int j = 0; j < 8; ++j) old[r][j] = 0.f;
    if (r < L && init)
      ld8(static_cast<const T*>(p.st) + rslot * p.st_slot + (int64_t)r * p.st_row + c0, old[r]);
  }
  const int last = min(max(p.blk_last[b], 0), p.idx_cols - 1);
  const int first = min(max(p.blk_first[b], 0), last);
  const int64_t nc = max(p.ncomp[b], 0);
  for (int k = first; k <= last; ++k) {
    // the state after `end` of the sequence's tokens
    int64_t end = k < last ? (int64_t)(k + 1) * p.blk_size - nc : e - s;
    end = min(max(end, (int64_t)0), e - s);
    const int64_t wslot = p.idx[(int64_t)b * p.idx_stride + k];
    if (wslot == p.pad) continue;
    T* srow = static_cast<T*>(p.st) + wslot * p.st_slot + c0;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      if (r >= L) continue;
      const int64_t pos = end - L + r;    // sequence position of state row r (>= -L)
      float v[8];
      if (pos >= 0) {
        ld8(static_cast<const T*>(p.x) + (s + pos) * p.xs + c0, v);
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q)
          if (q == L + pos)
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = old[q][j];
      }
      st8(srow + (int64_t)r * p.st_row, v);
    }
  }
}

// Decode: one token per sequence against its slot; the state shifts by one row.
// With prefix caching the state is read from table column blk_in[b] and written
// to column blk_last[b] (every read precedes the writes).
template <typename T, int W, bool ACT>
__global__ __launch_bounds__(NT) void conv_update_kernel(Params p) {
  const int c0 = (blockIdx.y * NT + threadIdx.x) * 8;
  const int b = blockIdx.x;
  if (c0 >= p.dim) return;
  const int64_t slot = slot_col(p, b, p.blk_in);
  const int64_t wslot = p.blk_last ? slot_col(p, b, p.blk_last) : slot;
  T* orow = static_cast<T*>(p.out) + (int64_t)b * p.os + c0;
  if (slot == p.pad || wslot == p.pad) {   // padded entry: zero output, no state access
    const float zero[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    st8(orow, zero);
    return;
  }
  const T* sin = static_cast<const T*>(p.st) + slot * p.st_slot + c0;
  T* srow = static_cast<T*>(p.st) + wslot * p.st_slot + c0;
  const int L = p.st_len;
  float xt[8], win[W - 1][8], y[8];
  ld8(static_cast<const T*>(p.x) + (int64_t)b * p.xs + c0, xt);
#pragma unroll
  for (int i = 0; i < W - 1; ++i) ld8(sin + (int64_t)(L - (W - 1) + i) * p.st_row, win[i]);
  float rows[8][8];      // rows 1 .. L-1 of a state longer than the window
  const bool slack = L > W - 1;
  if (slack) {
#pragma unroll
    for (int r = 1; r < 8; ++r)
      if (r < L - (W - 1)) ld8(sin + r * p.st_row, rows[r]);
  }
  Taps<W, ACT> tp;
  tp.load(p, c0);
  tp.apply(win, xt, y);
  st8(orow, y);
  // shift: row r <- row r+1; the window rows are the last W-1 rows
  if (slack) {
#pragma unroll
    for (int r = 0; r + 1 < 8; ++r)
      if (r + 1 < L - (W - 1)) st8(srow + r * p.st_row, rows[r + 1]);
  }
#pragma unroll
  for (int i = 0; i < W - 1; ++i) {
    const int r = L - (W - 1) + i - 1;       // destination of window row i
    if (r >= 0) st8(srow + (int64_t)r * p.st_row, win[i]);
  }
  st8(srow + (int64_t)(L - 1) * p.st_row, xt);
}

// Speculative update (multi-token, vLLM's num_accepted_tokens convention): sequence
// b's tokens [qs[b], qs[b+1]) continue the history whose last W-1 inputs are state
// rows a-1 .. a+W-3, a = num_accepted_tokens[b] (the previous step's accepted
// tokens; the rows after them are its rejected drafts).  Afterwards the state is
// rows a .. a+L-n-1 followed by the n new inputs, so the next step's window again
// starts at its accepted count minus one.  a is clamped to [1, L-W+2] and n to at
// most L-W+2 (the rows the state holds), so every access stays inside the slot; the
// token offsets are clamped to [0, total] (rows of x and out).
template <typename T, int W, bool ACT>
__global__ __launch_bounds__(NT) void conv_spec_update_kernel(Params p) {
  const int c0 = (blockIdx.y * NT + threadIdx.x) * 8;
  const int b = blockIdx.x;
  if (c0 >= p.dim) return;
  const int L = p.st_len;
  const int64_t t0 = min(max((int64_t)p.qs[b], (int64_t)0), p.total);
  const int64_t t1 = min(max((int64_t)p.qs[b + 1], t0), p.total);
  const int n = (int)min(t1 - t0, (int64_t)(L - W + 2));
  const int64_t slot = p.idx ? p.idx[b] : b;
  const float zero[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (slot == p.pad) {   // padded entry: zero outputs, no state access
    for (int t = 0; t < n; ++t) st8(static_cast<T*>(p.out) + (t0 + t) * p.os + c0, zero);
    return;
  }
  const int a = min(max(p.nacc[b], 1), L - W + 2);
  T* srow = static_cast<T*>(p.st) + slot * p.st_slot + c0;
  float rows[8][8];   // the slot's L (<= 8) rows of these channels
#pragma unroll
  for (int r = 0; r < 8; ++r)
    if (r < L) ld8(srow + (int64_t)r * p.st_row, rows[r]);
  Taps<W, ACT> tp;
  tp.load(p, c0);
  float win[W - 1][8];
#pragma unroll
  for (int i = 0; i < W - 1; ++i)
#pragma unroll
    for (int r = 0; r < 8; ++r)
      if (r == a - 1 + i)
#pragma unroll
        for (int j = 0; j < 8; ++j) win[i][j] = rows[r][j];
  float xs[8][8];     // the new inputs, for the state (n <= 8)
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    if (t < n) {
      ld8(static_cast<const T*>(p.x) + (t0 + t) * p.xs + c0, xs[t]);
      float y[8];
      tp.apply(win, xs[t], y);
      st8(static_cast<T*>(p.out) + (t0 + t) * p.os + c0, y);
#pragma unroll
      for (int i = 0; i + 1 < W - 1; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) win[i][j] = win[i + 1][j];
#pragma unroll
      for (int j = 0; j < 8; ++j) win[W - 2][j] = xs[t][j];
    }
  }
  // new state: rows a .. a+L-n-1, then the n inputs
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    if (r >= L) continue;
    float v[8];
    if (r < L - n) {
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (q == a + r)
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = rows[q][j];
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t)
        if (t == r - (L - n))
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = xs[t][j];
    }
    st8(srow + (int64_t)r * p.st_row, v);
  }
}

template <typename T, int W, bool ACT>
void launch_fwd_w(const Params& p, hipStream_t s) {
  const unsigned cg = (unsigned)((p.dim / 8 + NT - 1) / NT);
  // channel groups on x, so the groups of one token tile run together and read
  // whole rows; token tiles on y, in launches of at most 65535 (grid y's limit)
  const int64_t tiles = (p.total + TT - 1) / TT;
  for (int64_t t = 0; t < tiles; t += 65535) {
    Params q = p;
    q.tile0 = t;
    hipLaunchKernelGGL((conv_fwd_kernel<T, W, ACT>), dim3(cg, (unsigned)min(tiles - t, (int64_t)65535)),
                       dim3(NT), 0, s, q);
  }
  if (p.st && p.batch > 0) {
    if (p.blk_first)
      hipLaunchKernelGGL(conv_state_blocks_kernel<T>, dim3((unsigned)p.batch, cg), dim3(NT), 0, s, p);
    else
      hipLaunchKernelGGL(conv_state_kernel<T>, dim3((unsigned)p.batch, cg), dim3(NT), 0, s, p);
  }
}

template <typename T, int W, bool ACT>
void launch_update_w(const Params& p, hipStream_t s) {
  const unsigned cg = (unsigned)((p.dim / 8 + NT - 1) / NT);
  hipLaunchKernelGGL((conv_update_kernel<T, W, ACT>), dim3((unsigned)p.batch, cg), dim3(NT), 0, s,
                     p);
}

template <typename T, int W, bool ACT>
void launch_spec_w(const Params& p, hipStream_t s) {
  const unsigned cg = (unsigned)((p.dim / 8 + NT - 1) / NT);
  hipLaunchKernelGGL((conv_spec_update_kernel<T, W, ACT>), dim3((unsigned)p.batch, cg), dim3(NT), 0,
                     s, p);
}

// KIND 0: prefill, 1: decode update, 2: speculative update
template <typename T, int KIND>
void dispatch(const Params& p, int W, int act, hipStream_t s) {
#define HMX_CONV_CASE(WW, AA)                                            \
  if (W == WW && (act != 0) == AA) {                                      \
    if (KIND == 1) launch_update_w<T, WW, AA>(p, s);                      \
    else if (KIND == 2) launch_spec_w<T, WW, AA>(p, s);                   \
    else launch_fwd_w<T, WW, AA>(p, s);                                   \
    return;                                                               \
  }
  HMX_CONV_CASE(2, false) HMX_CONV_CASE(2, true) HMX_CONV_CASE(3, false)
  HMX_CONV_CASE(3, true) HMX_CONV_CASE(4, false) HMX_CONV_CASE(4, true)
#undef HMX_CONV_CASE
}

int check_common(const char* fn, const void* x, const void* out, const void* weight,
                 int32_t dtype, int32_t width, int32_t dim, int32_t state_len,
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
  const uintptr_t any = (uintptr_t)x | (uintptr_t)out | (uintptr_t)weight | (uintptr_t)bias |
                        (uintptr_t)st;
  HMX_REQUIRE(any % 16 == 0, HMX_EINVAL,
              "%s: x, out, weight, bias and state pointers must be 16-byte aligned", fn);
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
  const int rc = check_common("hmx_causal_conv1d_fwd", x, out, weight, dtype, width, dim,
                              state_len, weight_dtype, bias, bias_dtype, x_token_stride,
                              out_token_stride, state_row_stride, state_slot_stride, conv_states);
  if (rc != HMX_OK) return rc;
  HMX_REQUIRE(batch >= 0 && total_tokens >= 0, HMX_EINVAL, "hmx_causal_conv1d_fwd: sizes");
  if (total_tokens == 0) return HMX_OK;   // batch 0: every token gets output 0
  HMX_REQUIRE(x && out && weight && query_start_loc, HMX_EINVAL,
              "hmx_causal_conv1d_fwd: null pointer");
  Params p{x, x_token_stride, out, out_token_stride, weight, weight_dtype, bias, bias_dtype,
           conv_states, state_slot_stride, state_row_stride,
           conv_states ? state_len : width - 1, query_start_loc, batch, total_tokens,
           cache_indices, has_initial_state, dim, pad_slot_id};
  p.idx_stride = 1;
  p.idx_cols = 1;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == HMX_BF16) dispatch<bf16, 0>(p, width, activation, s);
  else if (dtype == HMX_F16) dispatch<f16, 0>(p, width, activation, s);
  else dispatch<float, 0>(p, width, activation, s);
  return check_launch("hmx_causal_conv1d_fwd");
}

extern "C" int hmx_causal_conv1d_fwd_blocks(
    const void* x, int64_t x_token_stride, void* out, int64_t out_token_stride, int32_t dtype,
    const void* weight, int32_t weight_dtype, int32_t width, const void* bias, int32_t bias_dtype,
    void* conv_states, int64_t state_slot_stride, int64_t state_row_stride, int32_t state_len,
    const int32_t* query_start_loc, int32_t batch, int64_t total_tokens,
    const int32_t* cache_indices, int64_t cache_indices_row_stride, int32_t cache_indices_cols,
    const uint8_t* has_initial_state, const int32_t* initial_state_idx,
    const int32_t* block_idx_first_scheduled_token, const int32_t* block_idx_last_scheduled_token,
    const int32_t* num_computed_tokens, int32_t block_size, int32_t dim, int32_t activation,
    int32_t pad_slot_id, void* stream) {
  const char* fn = "hmx_causal_conv1d_fwd_blocks";
  const int rc = check_common(fn, x, out, weight, dtype, width, dim, state_len, weight_dtype,
                              bias, bias_dtype, x_token_stride, out_token_stride,
                              state_row_stride, state_slot_stride, conv_states);
  if (rc != HMX_OK) return rc;
  HMX_REQUIRE(batch >= 0 && total_tokens >= 0, HMX_EINVAL, "%s: sizes", fn);
  HMX_REQUIRE(block_size > 0 && cache_indices_cols > 0 &&
              cache_indices_row_stride >= cache_indices_cols, HMX_EINVAL,
              "%s: block_size %d, cache_indices [batch, %d] with row stride %lld", fn, block_size,
              cache_indices_cols, (long long)cache_indices_row_stride);
  if (total_tokens == 0) return HMX_OK;
  HMX_REQUIRE(x && out && weight && query_start_loc && conv_states && cache_indices &&
              initial_state_idx && block_idx_first_scheduled_token &&
              block_idx_last_scheduled_token && num_computed_tokens, HMX_EINVAL,
              "%s: null pointer", fn);
  Params p{x, x_token_stride, out, out_token_stride, weight, weight_dtype, bias, bias_dtype,
           conv_states, state_slot_stride, state_row_stride, state_len, query_start_loc, batch,
           total_tokens, cache_indices, has_initial_state, dim, pad_slot_id};
  p.idx_stride = cache_indices_row_stride;
  p.idx_cols = cache_indices_cols;
  p.blk_in = initial_state_idx;
  p.blk_last = block_idx_last_scheduled_token;
  p.blk_first = block_idx_first_scheduled_token;
  p.ncomp = num_computed_tokens;
  p.blk_size = block_size;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == HMX_BF16) dispatch<bf16, 0>(p, width, activation, s);
  else if (dtype == HMX_F16) dispatch<f16, 0>(p, width, activation, s);
  else dispatch<float, 0>(p, width, activation, s);
  return check_launch(fn);
}

extern "C" int hmx_causal_conv1d_update(const void* x, int64_t x_token_stride, void* out,
                                        int64_t out_token_stride, int32_t dtype, const void* weight,
                                        int32_t weight_dtype, int32_t width, const void* bias,
                                        int32_t bias_dtype, void* conv_state,
                                        int64_t state_slot_stride, int64_t state_row_stride,
                                        int32_t state_len, const int32_t* conv_state_indices,
                                        int32_t batch, int32_t dim, int32_t activation,
                                        int32_t pad_slot_id, void* stream) {
  const int rc = check_common("hmx_causal_conv1d_update", x, out, weight, dtype, width, dim,
                              state_len, weight_dtype, bias, bias_dtype, x_token_stride,
                              out_token_stride, state_row_stride, state_slot_stride, conv_state);
  if (rc != HMX_OK) return rc;
  HMX_REQUIRE(batch >= 0, HMX_EINVAL, "hmx_causal_conv1d_update: batch %d", batch);
  if (batch == 0) return HMX_OK;
  HMX_REQUIRE(x && out && weight && conv_state, HMX_EINVAL,
              "hmx_causal_conv1d_update: null pointer");
  Params p{x, x_token_stride, out, out_token_stride, weight, weight_dtype, bias, bias_dtype,
           conv_state, state_slot_stride, state_row_stride, state_len, nullptr, batch, batch,
           conv_state_indices, nullptr, dim, pad_slot_id};
  p.idx_stride = 1;
  p.idx_cols = 1;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == HMX_BF16) dispatch<bf16, 1>(p, width, activation, s);
  else if (dtype == HMX_F16) dispatch<f16, 1>(p, width, activation, s);
  else dispatch<float, 1>(p, width, activation, s);
  return check_launch("hmx_causal_conv1d_update");
}

extern "C" int hmx_causal_conv1d_update_spec(
    const void* x, int64_t x_token_stride, void* out, int64_t out_token_stride, int32_t dtype,
    const void* weight, int32_t weight_dtype, int32_t width, const void* bias, int32_t bias_dtype,
    void* conv_state, int64_t state_slot_stride, int64_t state_row_stride, int32_t state_len,
    const int32_t* conv_state_indices, const int32_t* num_accepted_tokens,
    const int32_t* query_start_loc, int32_t batch, int64_t total_tokens, int32_t dim,
    int32_t activation, int32_t pad_slot_id, void* stream) {
  const int rc = check_common("hmx_causal_conv1d_update_spec", x, out, weight, dtype, width, dim,
                              state_len, weight_dtype, bias, bias_dtype, x_token_stride,
                              out_token_stride, state_row_stride, state_slot_stride, conv_state);
  if (rc != HMX_OK) return rc;
  HMX_REQUIRE(batch >= 0, HMX_EINVAL, "hmx_causal_conv1d_update_spec: batch %d", batch);
  if (batch == 0) return HMX_OK;
  HMX_REQUIRE(x && out && weight && conv_state && num_accepted_tokens && query_start_loc,
              HMX_EINVAL, "hmx_causal_conv1d_update_spec: null pointer");
  Params p{x, x_token_stride, out, out_token_stride, weight, weight_dtype, bias, bias_dtype,
           conv_state, state_slot_stride, state_row_stride, state_len, query_start_loc, batch,
           total_tokens, conv_state_indices, nullptr, dim, pad_slot_id, 0, num_accepted_tokens};
  p.idx_stride = 1;
  p.idx_cols = 1;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == HMX_BF16) dispatch<bf16, 2>(p, width, activation, s);
  else if (dtype == HMX_F16) dispatch<f16, 2>(p, width, activation, s);
  else dispatch<float, 2>(p, width, activation, s);
  return check_launch("hmx_causal_conv1d_update_spec");
}

extern "C" int hmx_causal_conv1d_update_blocks(
    const void* x, int64_t x_token_stride, void* out, int64_t out_token_stride, int32_t dtype,
    const void* weight, int32_t weight_dtype, int32_t width, const void* bias, int32_t bias_dtype,
    void* conv_state, int64_t state_slot_stride, int64_t state_row_stride, int32_t state_len,
    const int32_t* conv_state_indices, int64_t indices_row_stride, int32_t indices_cols,
    const int32_t* initial_state_idx, const int32_t* block_idx_last_scheduled_token,
    int32_t batch, int32_t dim, int32_t activation, int32_t pad_slot_id, void* stream) {
  const char* fn = "hmx_causal_conv1d_update_blocks";
  const int rc = check_common(fn, x, out, weight, dtype, width, dim, state_len, weight_dtype,
                              bias, bias_dtype, x_token_stride, out_token_stride,
                              state_row_stride, state_slot_stride, conv_state);
  if (rc != HMX_OK) return rc;
  HMX_REQUIRE(batch >= 0 && indices_cols > 0 && indices_row_stride >= indices_cols, HMX_EINVAL,
              "%s: batch %d, conv_state_indices [batch, %d] with row stride %lld", fn, batch,
              indices_cols, (long long)indices_row_stride);
  if (batch == 0) return HMX_OK;
  HMX_REQUIRE(x && out && weight && conv_state && conv_state_indices && initial_state_idx &&
              block_idx_last_scheduled_token, HMX_EINVAL, "%s: null pointer", fn);
  Params p{x, x_token_stride, out, out_token_stride, weight, weight_dtype, bias, bias_dtype,
           conv_state, state_slot_stride, state_row_stride, state_len, nullptr, batch, batch,
           conv_state_indices, nullptr, dim, pad_slot_id};
  p.idx_stride = indices_row_stride;
  p.idx_cols = indices_cols;
  p.blk_in = initial_state_idx;
  p.blk_last = block_idx_last_scheduled_token;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == HMX_BF16) dispatch<bf16, 1>(p, width, activation, s);
  else if (dtype == HMX_F16) dispatch<f16, 1>(p, width, activation, s);
  else dispatch<float, 1>(p, width, activation, s);
  return check_launch(fn);
}
