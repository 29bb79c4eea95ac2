// GDN chunked prefill (gated delta rule, WY/UT form), GQA-native, varlen,
// bf16 q/k/v with an fp32 recurrent state, for gfx950.
//
// Semantics: vllm-inference/src/primed_vllm/gdn/ops/chunk_gqa.py:15-83 (the op
// chain l2norm -> chunk cumsum -> KK^T -> (I+A)^-1 -> w,u -> h,v_new -> o), with
// per-chunk maths (C tokens per chunk, G = in-chunk cumsum of g):
//   A_ij = beta_i (k_i.k_j) e^{G_i-G_j} (j<i);  T = (I+A)^-1
//   V_new = T diag(beta) (V - diag(e^G) K S)
//         (= U - W S with U = T diag(beta) V, W = T diag(beta e^G) K)
//   O = scale [e^G (Q S) + tril(Q K^T e^{G_i-G_j}) V_new]
//   S <- e^{G_last} S + K^T (e^{G_last-G} V_new)
// Forming V_new from K S instead of W S needs no W: T is applied to the 32 x 32
// right-hand side in registers, by blockwise substitution over its two 16-row
// blocks (no merged T_10), with beta folded into T's columns (T' = T diag(beta))
// and A = diag(beta) M, M_ij = k_i.k_j e^{G_i-G_j} (j < i):
//   V_new_0 = T'_00 Y_0,  V_new_1 = T'_11 (Y_1 - M_10 V_new_0),  Y = V - e^G K S.
//
// The chunk length is an internal choice (the result is the same recurrence at
// any chunk length, up to fp32 rounding): C = 32 keeps a workgroup's LDS under
// 80 KB so two workgroups share a CU.
//
// Parallel decomposition (segmented chunk scan).  Each sequence's chunks are
// split into segments; one 256-thread workgroup owns one (segment, head) and
// walks its chunks serially with the 128x128 fp32 state held in MFMA
// accumulator registers (wave w owns state columns [32w, 32w+32)).  A segment's
// initial state comes from one of:
//   * the sequence's initial state (first segment);
//   * a warm-up: the chain is re-run from a zero state over the preceding
//     chunks, far enough back that the dropped history is bounded by
//     prod e^{g_t} max(1,|1-beta_t|) < e^{-decay_threshold} (the transition
//     e^{g}(I - beta k k^T) has spectral norm <= e^{g} max(1,|1-beta|) for
//     |k| <= 1, which in-kernel L2 normalisation guarantees) - exact to fp32;
//   * the exact segment scan when that bound is not reached within a few chunks
//     (weak decay): per-segment zero-start end states S0_s and transitions
//     Phi_s (chain started from I with V = 0), then S_{s+1} = Phi_s S_s + S0_s.
//
// Chunk pipeline: two barriers per chunk.  Phase 1 forms the chunk's T blocks
// (waves 0-1) and P (waves 2-3) while every wave computes K S and Q S for its
// state columns, stores the previous chunk's O, and prepares the next chunk
// (prefetched one chunk ahead into registers): its row norms and g cumsum.
// Phase 2 forms V_new, O and the state update, then stages the next chunk into
// the other of two LDS buffers.
//
// Numerics: every MFMA operand is fp16 (one round-to-nearest-even rounding) with
// fp32 accumulation.  k and q enter as k_n = rk k and q_n = scale rq q with the
// in-kernel L2 factors applied in fp32 before the rounding (|k_n|, |q_n| <= 1),
// so no product needs row factors afterwards; the state, T, M_10, P and the
// substitution right-hand sides are rounded from their fp32 accumulators.  fp16
// keeps 11 significant bits where bf16 keeps 8: one rounding per operand gives
// ~5e-4 relative state error, inside the 1e-3 bound, where bf16 needed hi + lo
// pairs (two MFMAs and a split per product).  Without in-kernel normalisation
// |k|, |q| must stay below 65504.  The state, the substitution's right-hand sides
// and V_new are O(|v|) and may pass fp16's range for large v or a large initial
// state: such a walk is detected (the inf reaches its end state, V_new through the
// fp16 copy from which the state update is formed) and walked again with those
// operands scaled per wave by a power of two from a running bound on the state's
// column norms (chunk_walk), which is exact.  The state is kept in fp32 and
// decayed explicitly each chunk.
//
// Roofline: HBM-bound at the algorithmic minimum (q,k,v,o bf16 + g,beta +
// final state); FLOPs 2*T*H*(5*C*d + 3*d^2).
#include <type_traits>

#include "common.hpp"
#include "mfma.hpp"

namespace hmx {
namespace gdnp {

constexpr int C = 32;          // chunk length (tokens)
constexpr int MT = C / 16;     // 16-row tiles per chunk
constexpr int D = 128;         // head dim (K == V == 128)
constexpr int NTHR = 256;      // 4 waves
// [C][128] row stride (k, q, v and O staging): 72 dwords = 8 mod 64 banks, which
// makes the 128-bit row-fragment reads and the transposing reads of natural-order
// rows (ds_read_b64_tr_b16) bank-conflict-free.  k and q are staged in the
// interleaved feature order (icol), so every k / q operand is one 128-bit read.
constexpr int LDQ = D + 16;
// O staging row stride: 68 dwords (4 mod 64 banks).  The O tile is written as
// 8-byte pieces (4 features of one token per lane), conflict-free for the
// 16-lane groups that a 64-bit write serves together (rows 4 banks apart), and
// read back by rows r and r + 16 per half-wave (68 * 16 = 64 mod 128 dwords),
// which a 128-bit read serves together.
constexpr int LDO = D + 8;
constexpr int LDT = C + 8;     // [C][C] row stride (P, T blocks)
static_assert(C == 32, "chunk length: the substitution and the g scan are written for 32");

// MODE_OUT: the output walk.  MODE_PRE: the exact scan's pre-pass walk of a
// segment, from zero with the values (S0) or from I without them (Phi).
enum Mode { MODE_OUT = 0, MODE_PRE = 1 };

// shared-memory layout (bytes): two staging buffers (K, Q as normalised fp16,
// V raw bf16, per-token scalars), the O staging tile, T/M blocks, P
constexpr int SZ_Q = C * LDQ * 2;
constexpr int SZ_SC = 4 * C * 4;                 // per-token scalars (see Stage)
constexpr int SZ_BUF = 3 * SZ_Q + SZ_SC;
constexpr int SZ_P = C * LDT * 2;
constexpr int SZ_O = C * LDO * 2;
constexpr int OFF_O = 2 * SZ_BUF;
constexpr int OFF_T = OFF_O + SZ_O;    // rows 0-15: T'_00 | rows 16-31: -M_10, T'_11 (fp16)
constexpr int OFF_P = OFF_T + SZ_P;    // P (fp16, lower triangle; the upper tile stays 0)
constexpr int OFF_NW = OFF_P + SZ_P;   // fp32 [D] output-norm weight (NORM)
constexpr int OFF_FLAG = OFF_NW + D * 4;   // int [4]: the waves' range flags
constexpr int SMEM = OFF_FLAG + 16;
static_assert(SMEM <= 80 * 1024, "LDS budget: two workgroups per CU");

struct SegInfo {     // one row of the host-built segment table (int32 x 8)
  int n, bos, eos, c_start, c_end, seg_idx, first_seg, nseg;
};

struct Params {
  const bf16* q; const bf16* k; const bf16* v;
  int64_t q_ts, kv_ts;       // token strides (elements; k and v share one); heads are D apart
  const void* g; int g_dt;
  const void* beta; int beta_dt;
  hmx_gate_proj gp; int fused;   // fused: g, beta from the raw projections in gp
  bf16* o;
  // States: slot sidx[n] (or n) of the h0 / ht bases, st_ss elements apart, in
  // st_dt (f32 or bf16); a negative slot or hinit[n] == 0 starts from zero, and a
  // negative slot writes no end state.  With sidx the two may alias (one pool):
  // the end states of split sequences then go through ws_ht (copied after the
  // launch that may still read the pool).
  const void* h0;            // or null (zero start)
  void* ht;                  // or null (no end state)
  int64_t st_ss; int st_dt;
  const int* sidx;           // [N] or null
  const uint8_t* hinit;      // [N] or null
  float* ws_ht;              // [N][H][D][D] or null
  const int* seg;            // [nseg_total][8]
  int* plan;                 // [nseg_total][H]: warm-up start chunk, or -1 (null: 1 seg/seq)
  int* redo;                 // [nseg_total][H]: 1 where the output walk left fp16's range
  float* ws_s0;              // [nseg_total][H][D][D]
  float* ws_phi;
  float* ws_init;
  int nseg_total;
  int H, HKV;
  float scale;
  int l2norm;
  int max_warm;
  float decay_thresh;
  // optional gated RMSNorm of each output row (NORM kernels)
  const bf16* zg; int64_t zg_ts, zg_hs;   // gate rows, or null (plain RMSNorm)
  const void* onw; int onw_dt;            // weight [D]
  float on_eps;
  // training: the fp16 state entering each output chunk, [cu_chunk[n] + c][H][D][D]
  f16* ws_hc = nullptr;
  const int* cu_chunk = nullptr;
};

__device__ __forceinline__ float ld_scalar(const void* p, int64_t i, int dt) {
  if (dt == HMX_F32) return static_cast<const float*>(p)[i];
  if (dt == HMX_BF16) return (float)static_cast<const bf16*>(p)[i];
  return (float)static_cast<const f16*>(p)[i];
}

// The element's bits, zero-extended (no conversion: a conversion right after the
// load would make the wave wait for it, and for every load issued before it).
__device__ __forceinline__ uint32_t ld_bits(const void* p, int64_t i, int dt) {
  if (dt == HMX_F32) return static_cast<const uint32_t*>(p)[i];
  return static_cast<const uint16_t*>(p)[i];
}

__device__ __forceinline__ float bits_f32(uint32_t b, int dt) {
  if (dt == HMX_F32) return __builtin_bit_cast(float, b);
  if (dt == HMX_BF16) return __builtin_bit_cast(float, b << 16);
  return (float)__builtin_bit_cast(f16, (uint16_t)b);
}

__device__ __forceinline__ SegInfo load_seg(const int* seg, int s) {
  const int* r = seg + s * 8;
  return SegInfo{r[0], r[1], r[2], r[3], r[4], r[5], r[6], r[7]};
}

// How a chunk's loaded gate bits become g and beta: as stored (g_dt / beta_dt),
// or, with fused gates, from the raw projection bits (gp.in_dtype) and the head's
// A_log and dt_bias.  Lanes past the sequence end hold NO_TOKEN (zero bits read
// as a gate give g = 0, but a zero projection does not) and give g = beta = 0.
constexpr uint32_t NO_TOKEN = 0xffffffffu;   // no 16-bit load yields it
template <bool FG>
struct GateConv {
  const Params& p;
  float eA_h, dtb_h;   // fused: the head's exp(A_log), dt_bias
  __device__ __forceinline__ float g(uint32_t bits) const {
    if constexpr (FG)
      return bits == NO_TOKEN ? 0.f : gp_g_of(p.gp, bits_f32(bits, p.gp.in_dtype), eA_h, dtb_h);
    else return bits_f32(bits, p.g_dt);
  }
  __device__ __forceinline__ float beta(uint32_t bits) const {
    if constexpr (FG)
      return bits == NO_TOKEN ? 0.f : gp_beta_of(p.gp, bits_f32(bits, p.gp.in_dtype));
    else return bits_f32(bits, p.beta_dt);
  }
};
template <bool FG>
__device__ __forceinline__ GateConv<FG> gate_conv(const Params& p, int h) {
  if constexpr (FG)
    return GateConv<FG>{p, gate_exp(load_any(p.gp.A_log, h, p.gp.A_log_dtype)),
                        load_any(p.gp.dt_bias, h, p.gp.dt_bias_dtype)};
  else return GateConv<FG>{p, 0.f, 0.f};
}
// the token's gate bits as stored, or its raw projection bits (fused)
template <bool FG>
__device__ __forceinline__ void ld_gate_bits(const Params& p, int64_t tok, int h, uint32_t& gb,
                                             uint32_t& bb) {
  if constexpr (FG) {
    gb = ld_bits(p.gp.a, tok * p.gp.a_token_stride + h * p.gp.a_head_stride, p.gp.in_dtype);
    bb = ld_bits(p.gp.b, tok * p.gp.b_token_stride + h * p.gp.b_head_stride, p.gp.in_dtype);
  } else {
    const int64_t gi = tok * p.H + h;
    gb = ld_bits(p.g, gi, p.g_dt);
    bb = ld_bits(p.beta, gi, p.beta_dt);
  }
}

// A sequence/head pair needs the exact segment scan when any of its later
// segments found no warm-up start (plan == -1).  The lanes of a wave read 64
// plan entries at a time (one load latency, not one per segment); the result
// is wave-uniform.
__device__ __forceinline__ bool seq_exact(const int* plan, const SegInfo& si, int H, int h,
                                          int lane) {
  if (!plan) return false;
  const int end = si.first_seg + si.nseg;
  for (int s0 = si.first_seg + 1; s0 < end; s0 += 64) {
    const int s = s0 + lane;
    if (__ballot(s < end && plan[s * H + h] < 0)) return true;
  }
  return false;
}

// The first segment-table row of sequence n (rows are grouped by sequence), or
// -1; 64 rows per load round.
__device__ __forceinline__ int find_seq_row(const int* seg, int nseg_total, int n, int lane) {
  for (int s0 = 0; s0 < nseg_total; s0 += 64) {
    const int s = s0 + lane;
    const unsigned long long m = __ballot(s < nseg_total && seg[s * 8] == n);
    if (m) return s0 + __builtin_ctzll(m);
  }
  return -1;
}

// One chunk's raw inputs for this thread: 2 rows x 8 features of k, v, q and
// (lanes 0-31 of wave 0) one token's g and beta, loaded one chunk ahead; then
// the row factors of those rows and (wave 0) the token's g cumsum, e^G and
// e^{G_last-G}, formed while the current chunk's MFMA work runs (prep_*).
struct RawChunk {
  bf16x8 k[MT], v[MT], q[MT];
  uint32_t gb, bb;              // g, beta as loaded (converted in prep_scan)
  float rk[MT], rq[MT];
  float gs, eg, edl;
};

// A raw buffer resource over rows 0 .. nrows-1 (D bf16 features each, ts elements
// apart) from base: loads past them return zeros without touching memory, which
// pads a chunk's missing rows with no per-row masks.  The base is uniform, so the
// per-chunk addressing is scalar; each lane's offset within a chunk is fixed.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const bf16* base, int nrows,
                                                           int64_t ts) {
  const uint32_t bytes = nrows > 0 ? (uint32_t)(((int64_t)(nrows - 1) * ts + D) * 2) : 0u;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(base), 0, bytes, 0x00020000);
}
__device__ __forceinline__ bf16x8 ld_rows(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Byte offsets of a thread's row pieces within a chunk (row pass*16 + tid/16,
// features 8 (tid % 16) ..), for k / v rows (kv_ts) and q rows (q_ts).
struct RowOffs {
  uint32_t kv[MT], q[MT];
};
__device__ __forceinline__ RowOffs row_offs(const Params& p, int tid) {
  RowOffs o;
#pragma unroll
  for (int pass = 0; pass < MT; ++pass) {
    const int64_t row = pass * 16 + (tid >> 4), f0 = (tid & 15) * 8;
    o.kv[pass] = (uint32_t)((row * p.kv_ts + f0) * 2);
    o.q[pass] = (uint32_t)((row * p.q_ts + f0) * 2);
  }
  return o;
}

template <int MODE, bool FG>
__device__ __forceinline__ void load_raw(RawChunk& r, const Params& p, const RowOffs& ro,
                                         const bf16* qh, const bf16* kh, const bf16* vh,
                                         int tok0, int nval, bool need_q, bool with_v, int tid,
                                         int h) {
  const __amdgpu_buffer_rsrc_t rk = rows_rsrc(kh + (int64_t)tok0 * p.kv_ts, nval, p.kv_ts);
  const __amdgpu_buffer_rsrc_t rv =
      rows_rsrc(vh + (int64_t)tok0 * p.kv_ts, (MODE == MODE_OUT || with_v) ? nval : 0, p.kv_ts);
  const __amdgpu_buffer_rsrc_t rq =
      rows_rsrc(qh + (int64_t)tok0 * p.q_ts, (MODE == MODE_OUT && need_q) ? nval : 0, p.q_ts);
#pragma unroll
  for (int pass = 0; pass < MT; ++pass) {
    r.k[pass] = ld_rows(rk, ro.kv[pass]);
    if (MODE == MODE_OUT || with_v) r.v[pass] = ld_rows(rv, ro.kv[pass]);
    if (MODE == MODE_OUT) r.q[pass] = ld_rows(rq, ro.q[pass]);
  }
  r.gb = r.bb = FG ? NO_TOKEN : 0u;
  if (tid < nval && tid < C) ld_gate_bits<FG>(p, (int64_t)(tok0 + tid), h, r.gb, r.bb);
}

// One staged chunk in LDS.  K and Q hold the rows as the products use them, in
// fp16: k_n = rk k and q_n = scale rq q, with rk, rq the in-kernel L2
// normalisation (1 without it); V holds the raw bf16 rows.
struct Stage {
  f16* K; f16* Q; bf16* V;
  float* G; float* B; float* EG; float* EDL;   // G, beta, e^G, e^{G_last-G}
};

__device__ __forceinline__ Stage stage_at(unsigned char* smem, int bi) {
  unsigned char* b = smem + bi * SZ_BUF;
  Stage s;
  s.K = reinterpret_cast<f16*>(b);
  s.Q = reinterpret_cast<f16*>(b + SZ_Q);
  s.V = reinterpret_cast<bf16*>(b + 2 * SZ_Q);
  s.G = reinterpret_cast<float*>(b + 3 * SZ_Q);
  s.B = s.G + C;
  s.EG = s.B + C;
  s.EDL = s.EG + C;
  return s;
}

// 1 / ||row|| of the row whose 8-feature slices the 16 lanes of a DPP row hold.
__device__ __forceinline__ float row_inv_norm(const bf16x8& raw) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; j += 2)
    ss = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{raw[j], raw[j + 1]}, bf16x2{raw[j], raw[j + 1]},
                                         ss, false);
  return __builtin_amdgcn_rsqf(row16_sum(ss) + 1e-6f);
}

// Row factors of the prefetched rows (1 without in-kernel normalisation).
template <int MODE>
__device__ __forceinline__ void prep_rows(RawChunk& r, bool norm, float scale) {
#pragma unroll
  for (int pass = 0; pass < MT; ++pass) {
    r.rk[pass] = norm ? row_inv_norm(r.k[pass]) : 1.f;
    if (MODE == MODE_OUT) r.rq[pass] = (norm ? row_inv_norm(r.q[pass]) : 1.f) * scale;
  }
}

// In-chunk cumsum of g and the decay factors (wave 0; lanes 0-31 = tokens).
template <bool FG>
__device__ __forceinline__ void prep_scan(RawChunk& r, int lane, const GateConv<FG>& gc) {
  const float gv = scan32(lane < C ? gc.g(r.gb) : 0.f);
  const float glast = __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gv), C - 1));
  r.gs = gv;
  r.eg = fast_exp(gv);
  r.edl = fast_exp(glast - gv);
}

__device__ __forceinline__ f16x8 scale_h8(const bf16x8& x, float s) {
  f16x8 y;
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = (f16)((float)x[j] * s);
  return y;
}

// Write a prefetched, prepared chunk into staging buffer st.
template <int MODE, typename GC>
__device__ __forceinline__ void stage_chunk(const Stage& st, const RawChunk& r, bool with_q,
                                            bool with_v, int tid, int wave, int lane,
                                            const GC& gc) {
#pragma unroll
  for (int pass = 0; pass < MT; ++pass) {
    const int row = pass * 16 + (tid >> 4);
    const int f0 = (tid & 15) * 8;
    store8_i(st.K + row * LDQ, f0, scale_h8(r.k[pass], r.rk[pass]));
    if (MODE == MODE_OUT || with_v)
      *reinterpret_cast<bf16x8*>(st.V + row * LDQ + f0) = r.v[pass];
    if (MODE == MODE_OUT && with_q)
      store8_i(st.Q + row * LDQ, f0, scale_h8(r.q[pass], r.rq[pass]));
  }
  if (wave == 0 && lane < C) {
    st.G[lane] = r.gs;
    st.B[lane] = gc.beta(r.bb);
    st.EG[lane] = r.eg;
    st.EDL[lane] = r.edl;
  }
}

// ((I + A)^-1)^T of a strictly-lower 16x16 block held in C layout (A) together
// with its transpose (At), by the exact identity for nilpotent A (A^16 = 0):
//   ((I + A)^-1)^T = (I + (A^8)^T)(I + (A^4)^T)(I + (A^2)^T)(I - A^T)
// (the factors commute).  Each product X.Y is one 16x16x16 fp16 MFMA on the C
// layout of X^T and of Y, so the chain forms A^2, A^4, A^8 and (A^2)^T, (A^4)^T.
// The result in C layout gives each lane 4 consecutive columns of one row of
// (I + A)^-1.
__device__ __forceinline__ f32x4 inv_unit_lower16_t(const f32x4& A, const f32x4& At, int q4,
                                                    int l16) {
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  const f16x4 a = h4(A), at = h4(At);
  const f16x4 a2 = h4(mfma16h_k16(at, a, z)), a2t = h4(mfma16h_k16(a, at, z));
  const f16x4 a4 = h4(mfma16h_k16(a2t, a2, z)), a4t = h4(mfma16h_k16(a2, a2t, z));
  const f16x4 a8 = h4(mfma16h_k16(a4t, a4, z));
  f32x4 R;
#pragma unroll
  for (int v = 0; v < 4; ++v) R[v] = ((4 * q4 + v == l16) ? 1.f : 0.f) - At[v];
  R = mfma16h_k16(a2, h4(R), R);
  R = mfma16h_k16(a4, h4(R), R);
  return mfma16h_k16(a8, h4(R), R);
}

// 4 consecutive fp16 of one row of a [C][LDT] tile (one 8-byte LDS write)
__device__ __forceinline__ void put_row4(f16* m, int r, int c, const f32x4& x) {
  *reinterpret_cast<f16x4*>(m + r * LDT + c) = h4(x);
}

// A operand (16x16x16) of the 16x16 block at (r0, c0) of an fp16 [C][LDT] matrix
__device__ __forceinline__ f16x4 ld_blk(const f16* m, int r0, int c0, int lane) {
  return *reinterpret_cast<const f16x4*>(m + (r0 + (lane & 15)) * LDT + c0 + 4 * (lane >> 4));
}

// ---------------------------------------------------------------------------
// the chunk-scan workgroup
// ---------------------------------------------------------------------------
// NORM: the output rows pass through the gated RMSNorm of hmx_rms_norm_gated
// (norm before gate) on their way out of sO.
// One workgroup's walk of segment s_id for head h: its output (OUT), or the S0
// (phi false) or Phi (phi true) pre-pass walk of an exact pair's segment (PRE).
template <int MODE, bool NORM, bool FG, bool SAFE>
__device__ __forceinline__ bool chunk_walk(const Params& p, unsigned char* smem, int s_id, int h,
                                           bool phi) {
  bf16* sO = reinterpret_cast<bf16*>(smem + OFF_O);
  f16* sT = reinterpret_cast<f16*>(smem + OFF_T);
  f16* sP = reinterpret_cast<f16*>(smem + OFF_P);

  const int tid = threadIdx.x, lane = tid & 63;
  // the wave index as a scalar: branches on it are uniform (an EXEC-masked region
  // would still run its MFMAs, which ignore EXEC)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, l16 = lane & 15;
  const GateConv<FG> gc = gate_conv<FG>(p, h);
  const SegInfo si = load_seg(p.seg, s_id);
  const int H = p.H;
  const int hk = h / (H / p.HKV);

  // ---- decide the chunk range and the initial state ------------------------
  const bool exact = seq_exact(p.plan, si, H, h, lane);
  const bool with_v = MODE == MODE_OUT || !phi;
  int c_begin = si.c_start;            // first chunk processed
  const int c_out = si.c_start;        // first chunk whose output is written
  int init_kind;                       // 0 zero, 1 h0, 2 ws_init, 3 identity
  if (MODE == MODE_OUT) {
    if (si.seg_idx == 0) {
      init_kind = 1;
    } else if (exact) {
      init_kind = 2;
    } else {
      const int w = p.plan[s_id * H + h];
      c_begin = w;
      init_kind = (w == 0) ? 1 : 0;
    }
  } else {
    if (!exact || si.seg_idx == si.nseg - 1) return true;
    if (phi) {
      if (si.seg_idx == 0) return true;
      init_kind = 3;
    } else {
      init_kind = (si.seg_idx == 0) ? 1 : 0;
    }
  }
  const int64_t slot = p.sidx ? (int64_t)p.sidx[si.n] : si.n;
  if (init_kind == 1 && (!p.h0 || slot < 0 || (p.hinit && !p.hinit[si.n]))) init_kind = 0;

  // ---- state registers: S[rt][ct] is the 16x16 tile (rows 16rt.., cols 32w+16ct..)
  f32x4 S[8][2];
  {
    const float* src = nullptr;
    const bf16* src16 = nullptr;
    if (init_kind == 1) {
      const int64_t off = slot * p.st_ss + (int64_t)h * D * D;
      if (p.st_dt == HMX_BF16) src16 = static_cast<const bf16*>(p.h0) + off;
      else src = static_cast<const float*>(p.h0) + off;
    }
    if (init_kind == 2) src = p.ws_init + ((int64_t)s_id * H + h) * D * D;
    // one uniform branch per source type (a per-element choice costs registers)
    if (src) {
#pragma unroll
      for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            S[rt][ct][v] = src[(16 * rt + 4 * q4 + v) * D + 32 * wave + 16 * ct + l16];
    } else if (src16) {
#pragma unroll
      for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            S[rt][ct][v] = (float)src16[(16 * rt + 4 * q4 + v) * D + 32 * wave + 16 * ct + l16];
    } else {
#pragma unroll
      for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int row = 16 * rt + 4 * q4 + v, col = 32 * wave + 16 * ct + l16;
            S[rt][ct][v] = (init_kind == 3 && row == col) ? 1.f : 0.f;
          }
    }
  }

  // ---- fp16 range.  The plain walk (SAFE false) rounds the state, Y, the
  // substitution's right-hand sides and V_new to fp16 as they are; an entry past
  // fp16's range becomes inf, which reaches the end state (V_new through its fp16
  // copy, from which the state update is formed), so the walk reports it instead of
  // writing the end state and the caller walks again with SAFE true.  The SAFE walk keeps
  // 2^-se S in the registers (se >= 0, per wave) and bnd, a bound on the 2-norm of
  // each of this wave's state columns at true scale.  A column s of the state
  // follows s <- e^g (I - beta k k^T) s + beta k v_j, whose transition has norm
  // <= 1 for |k| <= 1, beta in [0, 2] and g <= 0, so a chunk whose entries of v
  // (this wave's columns) are at most vmax in magnitude keeps
  //   |S|, |Y|, |V_new|, |e^{G_last-G} V_new|, the substitution's right-hand sides
  //     <= 2 (bnd + vmax + 2 C vmax),   bnd <- e^{G_last} bnd + 2 C vmax.
  // Each chunk scales its fp16 operands by 2^-fp16_range_exp of that bound; the
  // scale enters only through multiplications by powers of two, which are exact,
  // so both walks give the same result wherever the plain one stays in range.
  float bnd = 0.f;
  int se = 0;
  if (!SAFE) {
  } else if (init_kind == 1 || init_kind == 2) {
    float ss = 0.f;   // the Frobenius norm of this wave's columns bounds each column's norm
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int v = 0; v < 4; ++v) ss += S[rt][ct][v] * S[rt][ct][v];
    bnd = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(
                                        __builtin_bit_cast(int, sqrtf(wave_sum(ss)))));
    se = fp16_range_exp(2.f * bnd);
    if (se) {
      const float sig = pow2f(-se);
#pragma unroll
      for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v) S[rt][ct][v] *= sig;
    }
  } else {
    bnd = init_kind == 3 ? 1.f : 0.f;
  }

  // P's strictly-upper 16x16 tile is never written by phase 1: zero it once.
  if (MODE == MODE_OUT) {
    for (int i = tid; i < 16 * 16; i += NTHR) sP[(i >> 4) * LDT + 16 + (i & 15)] = (f16)0.f;
  }

  const int64_t o_rs = (int64_t)H * D;
  const bf16* qh = p.q + (int64_t)h * D;
  const bf16* kh = p.k + (int64_t)hk * D;
  const bf16* vh = p.v + (int64_t)hk * D;
  bf16* oh = p.o + (int64_t)h * D;

  // The O tile staged in sO (rows LDO apart) leaves through coalesced 16-byte
  // reads and stores: lane group g of wave w handles, in pass p, row 8p + 2w +
  // (g >> 1) + 16 (g & 1) (rows r and r + 16 share a half-wave), features
  // 8 (lane & 15) .. +7.
  const int og = (tid & 63) >> 4;
  const int o_f = (tid & 15) * 8;
  auto o_row = [&](int pass) { return 8 * pass + 2 * wave + (og >> 1) + 16 * (og & 1); };
  auto store_o = [&](int tok0, int nval) {
#pragma unroll
    for (int pass = 0; pass < MT; ++pass) {
      const int row = o_row(pass);
      if (row < nval)
        *reinterpret_cast<bf16x8*>(oh + (int64_t)(tok0 + row) * o_rs + o_f) =
            *reinterpret_cast<const bf16x8*>(sO + row * LDO + o_f);
    }
  };
  // NORM: the gate slices of this thread's two output rows (loaded a phase ahead),
  // then out = o / sqrt(mean(o^2) + eps) * w * silu(z) over each 128-wide row
  // (16 lanes x 8), o as rounded into sO.
  const float* sNW = reinterpret_cast<const float*>(smem + OFF_NW);
  const bf16* zh = NORM && p.zg ? p.zg + (int64_t)h * p.zg_hs : nullptr;
  auto load_gate = [&](bf16x8* zr, int tok0, int nval) {
#pragma unroll
    for (int pass = 0; pass < MT; ++pass) {
      const int row = o_row(pass);
      zr[pass] = (zh && row < nval)
                     ? *reinterpret_cast<const bf16x8*>(zh + (int64_t)(tok0 + row) * p.zg_ts + o_f)
                     : bf16x8{};
    }
  };
  auto store_o_norm = [&](int tok0, int nval, const bf16x8* zr) {
#pragma unroll
    for (int pass = 0; pass < MT; ++pass) {
      const int row = o_row(pass);
      const bf16x8 ov = *reinterpret_cast<const bf16x8*>(sO + row * LDO + o_f);
      float f[8], ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        f[j] = (float)ov[j];
        ss += f[j] * f[j];
      }
      // the 16 lanes of a row group hold the whole row
      const float rstd = 1.0f / sqrtf(row16_sum(ss) * (1.0f / D) + p.on_eps);
      const f32x4 w0 = *reinterpret_cast<const f32x4*>(sNW + o_f);
      const f32x4 w1 = *reinterpret_cast<const f32x4*>(sNW + o_f + 4);
      const float w[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
      bf16x8 out;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float y = f[j] * rstd * w[j];
        if (zh) {
          const float z = (float)zr[pass][j];
          y *= z * __builtin_amdgcn_rcpf(1.0f + fast_exp(-z));
        }
        out[j] = (bf16)y;
      }
      if (row < nval) *reinterpret_cast<bf16x8*>(oh + (int64_t)(tok0 + row) * o_rs + o_f) = out;
    }
  };
  if (NORM && tid < D) {
    float wv;
    if (p.onw_dt == HMX_F32) wv = static_cast<const float*>(p.onw)[tid];
    else if (p.onw_dt == HMX_BF16) wv = (float)static_cast<const bf16*>(p.onw)[tid];
    else wv = (float)static_cast<const f16*>(p.onw)[tid];
    reinterpret_cast<float*>(smem + OFF_NW)[tid] = wv;
  }

  if (c_begin < si.c_end) {
    const RowOffs ro = row_offs(p, tid);
    RawChunk raw;
    {
      const int t0 = si.bos + c_begin * C;
      load_raw<MODE, FG>(raw, p, ro, qh, kh, vh, t0, min(C, si.eos - t0), c_begin >= c_out,
                         with_v, tid, h);
      prep_rows<MODE>(raw, p.l2norm, p.scale);
      if (wave == 0) prep_scan(raw, lane, gc);
      stage_chunk<MODE>(stage_at(smem, 0), raw, c_begin >= c_out, with_v, tid, wave, lane, gc);
      if (c_begin + 1 < si.c_end) {
        const int t1 = t0 + C;
        load_raw<MODE, FG>(raw, p, ro, qh, kh, vh, t1, min(C, si.eos - t1),
                           c_begin + 1 >= c_out, with_v, tid, h);
      }
    }
    lds_barrier();

    for (int c = c_begin; c < si.c_end; ++c) {
      const int bi = (c - c_begin) & 1;
      const Stage cur = stage_at(smem, bi);
      const int tok0 = si.bos + c * C;
      const bool out_chunk = (MODE == MODE_OUT) && (c >= c_out);
      if (MODE == MODE_OUT && out_chunk && p.ws_hc) {
        // the state entering this chunk, fp16 row-major (the backward's S0; at true
        // scale, so its entries must stay inside fp16's range)
        f16* dst = p.ws_hc + ((int64_t)(p.cu_chunk[si.n] + c) * H + h) * D * D + 32 * wave + l16;
        const float isig = pow2f(se);
#pragma unroll
        for (int rt = 0; rt < 8; ++rt)
#pragma unroll
          for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int v = 0; v < 4; ++v)
              dst[(16 * rt + 4 * q4 + v) * D + 16 * ct] = (f16)(S[rt][ct][v] * isig);
      }

      // ---- phase 1: stage the next chunk (its buffer was last read in the previous
      // chunk's phase 2) and prefetch the one after, so the loads have a whole chunk
      // to arrive; T blocks / P; K S and (Q S)^T; store the previous chunk's O -------
      if (c + 1 < si.c_end) {
        prep_rows<MODE>(raw, p.l2norm, p.scale);
        if (wave == 0) prep_scan(raw, lane, gc);
        stage_chunk<MODE>(stage_at(smem, bi ^ 1), raw, c + 1 >= c_out, with_v, tid, wave, lane,
                          gc);
        if (c + 2 < si.c_end) {
          const int t2 = tok0 + 2 * C;
          load_raw<MODE, FG>(raw, p, ro, qh, kh, vh, t2, min(C, si.eos - t2), c + 2 >= c_out,
                             with_v, tid, h);
        }
      }
      bf16x8 zr[MT];
      if constexpr (NORM) {
        if (MODE == MODE_OUT && c > c_out) load_gate(zr, tok0 - C, C);
      }

      // X[mt][ct] = (K S) tile (tokens 16mt.., state cols 32w+16ct..);
      // QT[ct][mt] = (Q S)^T tile (state cols 32w+16ct.., tokens 16mt..)
      f32x4 X[MT][2], QT[2][MT];
      // VF: this wave's tile of the chunk's V (fp32), read in phase 1 so that the
      // reduction of its magnitude overlaps the MFMAs; vmax bounds its entries
      f32x4 VF[MT][2];
      float vmax = 0.f;
      auto phase1 = [&](auto role_c, auto outq_c) {
        constexpr int R = decltype(role_c)::value;
        constexpr bool OQ = decltype(outq_c)::value;
        // Role work, balanced over the waves (16x16x32-MFMA units in brackets):
        //   wave 0: T'_00 [4 + 8 half]; wave 1: T'_11 [4 + 8 half];
        //   wave 2: -M_10 and P_00 [4 + 4]; wave 3: P_10 and P_11 [4 + 4].
        // Tiles are formed transposed (keys as rows), so each lane holds 4
        // consecutive columns of one row and writes them with one 8-byte store.
        auto gram = [&](const f16* X, int rx, const f16* Y, int ry) {
          // C layout of X[rx..rx+15] . Y[ry..ry+15]^T (128-long rows)
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks)
            acc = mfma16h(frag_i(X, LDQ, rx, 32 * ks, lane), frag_i(Y, LDQ, ry, 32 * ks, lane), acc);
          return acc;
        };
        if constexpr (R < MT) {
          // T'_RR = (I + A_RR)^-1 diag(beta), A = diag(beta) M on the diagonal block
          const int o = 16 * R;
          const f32x4 kk = gram(cur.K, o, cur.K, o);   // symmetric
          const float gc = cur.G[o + l16], bc = cur.B[o + l16];
          f32x4 Ad, At_;
          float br[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int row = 4 * q4 + v;
            br[v] = cur.B[o + row];
            const float d = cur.G[o + row] - gc;
            const float e = kk[v] * fast_exp(row > l16 ? d : -d);
            Ad[v] = row > l16 ? br[v] * e : 0.f;
            At_[v] = l16 > row ? bc * e : 0.f;
          }
          f32x4 Tt = inv_unit_lower16_t(Ad, At_, q4, l16);   // T[l16][4q4+v]
#pragma unroll
          for (int v = 0; v < 4; ++v) Tt[v] *= br[v];
          put_row4(sT, o + l16, o + 4 * q4, Tt);
        } else if constexpr (R == MT) {
          // -M_10: row 16+l16, cols 4q4+v: -(k_i.k_j) e^{G_i-G_j}
          const f32x4 m = gram(cur.K, 0, cur.K, 16);
          const float gi = cur.G[16 + l16];
          f32x4 nm;
#pragma unroll
          for (int v = 0; v < 4; ++v) nm[v] = -m[v] * fast_exp(gi - cur.G[4 * q4 + v]);
          put_row4(sT, 16 + l16, 4 * q4, nm);
          if constexpr (OQ) {
            // P_00: row l16 (query), cols 4q4+v (keys), c <= r
            const f32x4 pt = gram(cur.K, 0, cur.Q, 0);
            const float gr = cur.G[l16];
            f32x4 pv;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int c = 4 * q4 + v;
              pv[v] = c <= l16 ? pt[v] * fast_exp(gr - cur.G[c]) : 0.f;
            }
            put_row4(sP, l16, 4 * q4, pv);
          }
        } else if constexpr (OQ) {
          // P_10 (all c < r) and P_11 (c <= r): row 16+l16
          const float gr = cur.G[16 + l16];
          const f32x4 p0 = gram(cur.K, 0, cur.Q, 16);
          const f32x4 p1 = gram(cur.K, 16, cur.Q, 16);
          f32x4 v0, v1;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int c = 4 * q4 + v;
            v0[v] = p0[v] * fast_exp(gr - cur.G[c]);
            v1[v] = c <= l16 ? p1[v] * fast_exp(gr - cur.G[16 + c]) : 0.f;
          }
          put_row4(sP, 16 + l16, 4 * q4, v0);
          put_row4(sP, 16 + l16, 16 + 4 * q4, v1);
        }
        if constexpr (SAFE) {
          float vm = 0.f;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
              bf16x4 vt = {};
              if (with_v) vt = ld_tr(cur.V, LDQ, 16 * mt + 4 * q4, 32 * wave + 16 * ct, lane);
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                VF[mt][ct][v] = (float)vt[v];
                vm = fmaxf(vm, fabsf(VF[mt][ct][v]));
              }
            }
          vmax = with_v ? wave_max_nonneg(vm) : 0.f;
        }
        // K S and (Q S)^T for this wave's columns; one fp16 copy of the state
        // serves as the B operand of K S and the A operand of (Q S)^T
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) {
            X[mt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
            QT[ct][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          f16x8 Sb[2];
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) Sb[ct] = h8(S[2 * ks][ct], S[2 * ks + 1][ct]);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const f16x8 a = frag_i(cur.K, LDQ, 16 * mt, 32 * ks, lane);
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) X[mt][ct] = mfma16h(a, Sb[ct], X[mt][ct]);
            if constexpr (OQ) {
              const f16x8 bq = frag_i(cur.Q, LDQ, 16 * mt, 32 * ks, lane);
#pragma unroll
              for (int ct = 0; ct < 2; ++ct) QT[ct][mt] = mfma16h(Sb[ct], bq, QT[ct][mt]);
            }
          }
        }
      };
      using I0 = std::integral_constant<int, 0>;
      using I1 = std::integral_constant<int, 1>;
      using I2 = std::integral_constant<int, 2>;
      using I3 = std::integral_constant<int, 3>;
      using BT = std::true_type;
      using BF = std::false_type;
      if (MODE == MODE_OUT && out_chunk) {
        if (wave == 0) phase1(I0{}, BT{});
        else if (wave == 1) phase1(I1{}, BT{});
        else if (wave == 2) phase1(I2{}, BT{});
        else phase1(I3{}, BT{});
      } else {
        if (wave == 0) phase1(I0{}, BF{});
        else if (wave == 1) phase1(I1{}, BF{});
        else if (wave == 2) phase1(I2{}, BF{});
        else phase1(I3{}, BF{});
      }
      if (MODE == MODE_OUT && c > c_out) {
        if constexpr (NORM) store_o_norm(tok0 - C, C, zr);
        else store_o(tok0 - C, C);
      }
      lds_barrier();

      __builtin_amdgcn_s_setprio(1);
      // ---- phase 2: Y = V - e^G K S; V_new by blockwise substitution --------------
      // (SAFE: at operand scale 2^-te, with the registers' S, and so K S and Q S, at
      // 2^-se: Y = 2^-te V - 2^(se-te) e^G K (2^-se S))
      int te = 0;
      float tau = 1.f, rho = 1.f, itau = 1.f;
      if constexpr (SAFE) {
        te = fp16_range_exp(2.f * (bnd + (2 * C + 1) * vmax));
        tau = pow2f(-te);
        rho = pow2f(se - te);
        itau = pow2f(te);
      }
      f32x4 Vn[MT][2];
      {
        f32x4 Y[MT][2];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) {
            if constexpr (SAFE) {
#pragma unroll
              for (int v = 0; v < 4; ++v)
                Y[mt][ct][v] = VF[mt][ct][v] * tau -
                               (cur.EG[16 * mt + 4 * q4 + v] * rho) * X[mt][ct][v];
            } else {
              bf16x4 vt = {};
              if (with_v) vt = ld_tr(cur.V, LDQ, 16 * mt + 4 * q4, 32 * wave + 16 * ct, lane);
#pragma unroll
              for (int v = 0; v < 4; ++v)
                Y[mt][ct][v] = (float)vt[v] - cur.EG[16 * mt + 4 * q4 + v] * X[mt][ct][v];
            }
          }
        const f16x4 t00 = ld_blk(sT, 0, 0, lane);
        const f16x4 nm10 = ld_blk(sT, 16, 0, lane);
        const f16x4 t11 = ld_blk(sT, 16, 16, lane);
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          Vn[0][ct] = mfma16h_k16(t00, h4(Y[0][ct]), z);
          const f32x4 r1 = mfma16h_k16(nm10, h4(Vn[0][ct]), Y[1][ct]);
          Vn[1][ct] = mfma16h_k16(t11, h4(r1), z);
        }
      }

      // V_new's fp16 copy: the B operand of O and, widened again, the state update's
      // right-hand side, so that an entry past fp16's range reaches the state
      f16x8 Va[2];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) Va[ct] = h8(Vn[0][ct], Vn[1][ct]);

      // ---- O^T = e^G (Q S)^T + V_new^T P^T -> sO (4 features of a token per lane) ----
      if (out_chunk) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const f16x8 bp = frag_perm_h(sP, LDT, 16 * mt, 0, lane);
          const float eg = SAFE ? cur.EG[16 * mt + l16] * rho : cur.EG[16 * mt + l16];
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) {
            f32x4 O;
#pragma unroll
            for (int v = 0; v < 4; ++v) O[v] = QT[ct][mt][v] * eg;
            O = mfma16h(Va[ct], bp, O);   // SAFE: 2^-te O
            if constexpr (SAFE) {
#pragma unroll
              for (int v = 0; v < 4; ++v) O[v] *= itau;
            }
            *reinterpret_cast<bf16x4*>(sO + (16 * mt + l16) * LDO + 32 * wave + 16 * ct + 4 * q4) =
                bf16x4{(bf16)O[0], (bf16)O[1], (bf16)O[2], (bf16)O[3]};
          }
        }
      }

      // ---- S <- e^{G_last} S + K_n^T (e^{G_last-G} V_new) (SAFE: leaving the
      // registers at 2^-te) ----------------------------------------------------------
      {
        float egl = cur.EG[C - 1];
        if constexpr (SAFE)
          egl = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, egl)));
        const float egs = SAFE ? egl * rho : egl;
#pragma unroll
        for (int rt = 0; rt < 8; ++rt)
#pragma unroll
          for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int v = 0; v < 4; ++v) S[rt][ct][v] *= egs;
        if constexpr (SAFE) {
          bnd = egl * bnd + (2 * C) * vmax;
          se = te;
        }
        float e0[4], e1[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          e0[v] = cur.EDL[4 * q4 + v];
          e1[v] = cur.EDL[16 + 4 * q4 + v];
        }
        // W = e^{G_last-G} V_new from V_new's fp16 copy (mixed-precision multiplies)
        f16x8 Wb[2];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          f32x4 w0, w1;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            // fma with a zero addend: one v_fma_mix_f32 (widening in the instruction)
            w0[v] = __builtin_fmaf((float)Va[ct][v], e0[v], 0.f);
            w1[v] = __builtin_fmaf((float)Va[ct][4 + v], e1[v], 0.f);
          }
          Wb[ct] = h8(w0, w1);
        }
#pragma unroll
        for (int rt = 0; rt < 8; ++rt) {
          const f16x8 a = frag_t_i(cur.K, LDQ, 0, 16 * rt, lane);
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) S[rt][ct] = mfma16h(a, Wb[ct], S[rt][ct]);
        }
      }
      __builtin_amdgcn_s_setprio(0);

      lds_barrier();
    }
    if (MODE == MODE_OUT && si.c_end > c_out) {
      const int tl = si.bos + (si.c_end - 1) * C;
      if constexpr (NORM) {
        bf16x8 zl[MT];
        load_gate(zl, tl, min(C, si.eos - tl));
        store_o_norm(tl, min(C, si.eos - tl), zl);
      } else {
        store_o(tl, min(C, si.eos - tl));
      }
    }
  }

  // ---- plain walk: did an fp16 operand leave its range?  Any inf there reaches the
  // end state as inf or NaN (the sum below overflows to inf only when entries
  // approach fp32's range, which the SAFE walk then handles as well).
  if constexpr (!SAFE) {
    float acc = 0.f;
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc += S[rt][ct][v];
    int* flag = reinterpret_cast<int*>(smem + OFF_FLAG);
    const bool bad = __ballot(!__builtin_isfinite(acc)) != 0;
    if (lane == 0) flag[wave] = bad;
    lds_barrier();
    const int redo = flag[0] | flag[1] | flag[2] | flag[3];
    if (MODE == MODE_OUT && tid == 0) p.redo[s_id * H + h] = redo;
    if (redo) return false;   // the end state is not written
  }

  // ---- write the end state ---------------------------------------------------
  float* dst = nullptr;
  bf16* dst16 = nullptr;
  if (MODE == MODE_OUT) {
    if (si.seg_idx == si.nseg - 1 && p.ht && slot >= 0) {
      if (p.ws_ht && si.nseg > 1) {
        dst = p.ws_ht + ((int64_t)si.n * H + h) * D * D;
      } else {
        const int64_t off = slot * p.st_ss + (int64_t)h * D * D;
        if (p.st_dt == HMX_BF16) dst16 = static_cast<bf16*>(p.ht) + off;
        else dst = static_cast<float*>(p.ht) + off;
      }
    }
  } else {
    dst = (phi ? p.ws_phi : p.ws_s0) + ((int64_t)s_id * H + h) * D * D;
  }
  if (dst || dst16) {
    const float isig = pow2f(se);   // back to true scale (exact)
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int i = (16 * rt + 4 * q4 + v) * D + 32 * wave + 16 * ct + l16;
          if (dst) dst[i] = S[rt][ct][v] * isig;
          else dst16[i] = (bf16)(S[rt][ct][v] * isig);
        }
  }
  return true;
}

// The output walks (after the exact pairs' segment combine).
// A walk whose fp16 operands left their range writes no end state and sets its
// redo flag; gdn_redo_kernel walks it again with scaled operands.
template <bool NORM, bool FG>
__global__ __launch_bounds__(NTHR, 2) void gdn_chunk_kernel(Params p) {
  __shared__ __align__(16) unsigned char smem[SMEM];
  chunk_walk<MODE_OUT, NORM, FG, false>(p, smem, blockIdx.x, blockIdx.y, false);
}

// The flagged output walks again, with scaled fp16 operands (their outputs and end
// states are written again); the other workgroups return at once.
template <bool NORM, bool FG>
__global__ __launch_bounds__(NTHR, 2) void gdn_redo_kernel(Params p) {
  __shared__ __align__(16) unsigned char smem[SMEM];
  if (!p.redo[blockIdx.x * p.H + blockIdx.y]) return;
  chunk_walk<MODE_OUT, NORM, FG, true>(p, smem, blockIdx.x, blockIdx.y, false);
}

// The exact pairs' pre-pass: blockIdx.z 0 walks S0, 1 walks Phi.  The two are
// independent and share the GPU in one launch; the output walks follow in a
// launch of their own, which the warm-up pairs fill alongside the exact ones.  A
// walk whose fp16 operands left their range is walked again at once with scaled
// operands (its end state feeds the segment combine).
template <bool FG>
__global__ __launch_bounds__(NTHR, 2) void gdn_pre_kernel(Params p) {
  __shared__ __align__(16) unsigned char smem[SMEM];
  if (!chunk_walk<MODE_PRE, false, FG, false>(p, smem, blockIdx.x, blockIdx.y, blockIdx.z == 1))
    chunk_walk<MODE_PRE, false, FG, true>(p, smem, blockIdx.x, blockIdx.y, blockIdx.z == 1);
}

// ---------------------------------------------------------------------------
// plan: warm-up start chunk per (segment, head); exact flag per (sequence, head)
// ---------------------------------------------------------------------------
template <bool FG>
__global__ __launch_bounds__(64) void gdn_plan_kernel(Params p) {
  const int s = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int H = p.H;
  const GateConv<FG> gc = gate_conv<FG>(p, h);
  const SegInfo si = load_seg(p.seg, s);
  int plan = 0;
  if (si.seg_idx > 0) {
    plan = -1;
    if (p.l2norm) {
      // Walk back from the segment start over at most max_warm chunks, summing each
      // chunk's decay bound, until the sum drops below -decay_thresh (start there)
      // or the sequence start is reached (start from h0).  4 chunks per round:
      // lanes 16j..16j+15 load chunk c_hi - 1 - j, 2 tokens each, in one go.
      const int lo = max(0, si.c_start - p.max_warm);
      float acc = 0.f;
      for (int c_hi = si.c_start; c_hi > lo && plan < 0; c_hi -= 4) {
        const int c = c_hi - 1 - (lane >> 4);
        float b = 0.f;
        if (c >= lo) {
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const int t = si.bos + c * C + (lane & 15) * 2 + i;
            if (t < si.eos) {
              uint32_t gbits, bbits;
              ld_gate_bits<FG>(p, t, h, gbits, bbits);
              b += gc.g(gbits) + logf(fmaxf(1.f, fabsf(1.f - gc.beta(bbits))));
            }
          }
        }
        b = row16_sum(b);
        bool done = false;
        for (int j = 0; j < 4 && !done; ++j) {   // uniform: every lane holds every sum
          const int cj = c_hi - 1 - j;
          if (cj < lo) break;
          acc += __shfl(b, 16 * j);
          if (acc < -p.decay_thresh) { plan = cj; done = true; }
          else if (cj == 0) { plan = 0; done = true; }  // sequence start: exact from h0
        }
      }
    }
  }
  if (lane == 0) p.plan[s * H + h] = plan;
}

// ---------------------------------------------------------------------------
// exact segment scan: S_1 = S0_0; S_{s+1} = Phi_s S_s + S0_s, in fp32 MFMAs
// (16x16x4 f32).  One 512-thread workgroup per (sequence, head, 16-column slice
// of the state); wave w forms rows [16w, 16w+16) of the slice, two waves per
// SIMD.  The slice of S_s lives in LDS transposed (column-major, 132-dword
// columns: the 4 K-values a lane feeds are one conflict-free 128-bit read),
// double-buffered so a step needs one barrier.  Phi_s and S0_s do not depend on
// the chain: they are loaded into registers two steps ahead.  The 8 slices of a
// (sequence, head) are blocks b with equal b mod 8, which the dispatcher places
// on one XCD, so each Phi_s is fetched into one L2 once.
// ---------------------------------------------------------------------------
constexpr int CMB_LD = D + 4;
constexpr int CMB_THR = 512;

__global__ __launch_bounds__(CMB_THR) void gdn_seg_combine_kernel(Params p, int N) {
  __shared__ __align__(16) float sST[2][16 * CMB_LD];
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, l16 = lane & 15;
  const int cb = (b >> 3) & 7, nh = (b & 7) + 8 * (b >> 6);
  const int H = p.H;
  if (nh >= N * H) return;
  const int n = nh / H, h = nh % H;
  const int row = find_seq_row(p.seg, p.nseg_total, n, lane);
  if (row < 0) return;
  const SegInfo si = load_seg(p.seg, row);
  const int first = si.first_seg, nseg = si.nseg;
  if (nseg < 2 || !seq_exact(p.plan, si, H, h, lane)) return;
  const int64_t hoff = (int64_t)h * D * D, sstride = (int64_t)H * D * D;
  const int col = cb * 16 + l16, r0 = 16 * wave;
  // Phi_s rows r0 + l16, features 16j + 4q4..+3 (A operands) and S0_s in the
  // accumulator layout (rows r0 + 4q4 + v, column col)
  struct StepIn { f32x4 phi[8], s0; };
  auto load_step = [&](StepIn& in, int s) {
    const float* ph = p.ws_phi + (first + s) * sstride + hoff;
    const float* z = p.ws_s0 + (first + s) * sstride + hoff;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      in.phi[j] = *reinterpret_cast<const f32x4*>(ph + (r0 + l16) * D + 16 * j + 4 * q4);
#pragma unroll
    for (int v = 0; v < 4; ++v) in.s0[v] = z[(r0 + 4 * q4 + v) * D + col];
  };
  auto put = [&](int buf, const f32x4& x) {
    *reinterpret_cast<f32x4*>(&sST[buf][l16 * CMB_LD + r0 + 4 * q4]) = x;
  };
  // S_s (LDS buffer buf, after a barrier) -> its ws_init slice: thread tid writes
  // row tid / 4, columns 4 (tid & 3)..+3 (the stores never read the MFMA
  // accumulators, so the next step need not wait for them)
  auto flush = [&](int buf, int s) {
    float* init = p.ws_init + (first + s) * sstride + hoff;
    const int r = tid >> 2, c0 = (tid & 3) * 4;
    f32x4 x;
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = sST[buf][(c0 + e) * CMB_LD + r];
    *reinterpret_cast<f32x4*>(init + r * D + cb * 16 + c0) = x;
  };
  const int last = nseg - 2;   // the last step forms S_{nseg-1}
  // three input sets in rotation: step s consumes one while the loads of steps
  // s + 1 and s + 2 are in flight (issued at the starts of steps s - 1 and s)
  StepIn b0, b1, b2;
  auto step = [&](StepIn& in, StepIn& ahead, int s) {
    const int cur = (s - 1) & 1;
    load_step(ahead, min(s + 2, last));   // unconditional: the last steps reload their own
    __builtin_amdgcn_sched_barrier(0);
    f32x4 acc[2] = {in.s0, f32x4{0.f, 0.f, 0.f, 0.f}};   // two chains: even / odd j
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const f32x4 bk = *reinterpret_cast<const f32x4*>(&sST[cur][l16 * CMB_LD + 16 * j + 4 * q4]);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[j & 1] = mfma16f(in.phi[j][e], bk[e], acc[j & 1]);
    }
    put(cur ^ 1, acc[0] + acc[1]);
    __syncthreads();
    flush(cur ^ 1, s + 1);
  };
  // S_1 = S0_0
  load_step(b0, 0);
  put(0, b0.s0);
  load_step(b1, min(1, last));
  load_step(b2, min(2, last));
  __syncthreads();
  flush(0, 1);
  // step s reads b[s % 3] and loads step s + 2 into b[(s + 2) % 3], whose step
  // s - 1 is done
  for (int s = 1; s <= last; s += 3) {
    step(b1, b0, s);
    if (s + 1 > last) break;
    step(b2, b1, s + 1);
    if (s + 2 > last) break;
    step(b0, b2, s + 2);
  }
}

// ---------------------------------------------------------------------------
// pooled end states of split sequences: ws_ht -> the pool slot, after every launch
// that may still read the pool.  One workgroup per (sequence, head).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(NTHR) void gdn_state_copy_kernel(Params p) {
  const int n = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int row = find_seq_row(p.seg, p.nseg_total, n, tid & 63);
  const int64_t slot = p.sidx[n];
  if (row < 0 || p.seg[row * 8 + 7] < 2 || slot < 0) return;
  const float* src = p.ws_ht + ((int64_t)n * p.H + h) * D * D;
  const int64_t off = slot * p.st_ss + (int64_t)h * D * D;
  for (int i = tid * 4; i < D * D; i += NTHR * 4) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(src + i);
    if (p.st_dt == HMX_BF16) {
      bf16x4 y{(bf16)x[0], (bf16)x[1], (bf16)x[2], (bf16)x[3]};
      *reinterpret_cast<bf16x4*>(static_cast<bf16*>(p.ht) + off + i) = y;
    } else {
      *reinterpret_cast<f32x4*>(static_cast<float*>(p.ht) + off + i) = x;
    }
  }
}

}  // namespace gdnp
}  // namespace hmx

using namespace hmx;
using namespace hmx::gdnp;

// hmx_gdn_chunk_fwd, and with block_states / cu_blocks the training forward
// (hmx_gdn_train_fwd) that also writes the state entering every chunk
static int chunk_fwd_impl(const void* q, int64_t q_token_stride, const void* k,
                          int64_t k_token_stride, const void* v, int64_t v_token_stride,
                          int32_t qkv_dtype, const void* g, int32_t g_dtype, const void* beta,
                          int32_t beta_dtype, void* o, const void* h0, void* ht,
                          int64_t state_slot_stride, int32_t state_dtype,
                          const int32_t* state_indices, const uint8_t* has_initial_state,
                          const int32_t* seg_table, int32_t nseg_total, int32_t N, int32_t H,
                          int32_t HKV, int32_t K, int32_t V, float scale, int32_t use_qk_l2norm,
                          int32_t max_warm_chunks, float decay_threshold, void* workspace,
                          size_t workspace_bytes, const hmx_gated_norm* o_norm,
                          const hmx_gate_proj* gates, void* stream, f16* block_states,
                          const int32_t* cu_blocks) {
  HMX_REQUIRE(qkv_dtype == HMX_BF16, HMX_EUNSUPPORTED,
              "hmx_gdn_chunk_fwd: q/k/v must be bfloat16 (got dtype code %d)", qkv_dtype);
  HMX_REQUIRE(K == D && V == D, HMX_EUNSUPPORTED,
              "hmx_gdn_chunk_fwd: only K == V == 128 is supported (got K=%d V=%d)", K, V);
  HMX_REQUIRE(H > 0 && HKV > 0 && H % HKV == 0, HMX_EINVAL,
              "hmx_gdn_chunk_fwd: H=%d must be a positive multiple of HKV=%d", H, HKV);
  HMX_REQUIRE(q && k && v && (gates || (g && beta)) && o && seg_table, HMX_EINVAL,
              "hmx_gdn_chunk_fwd: null tensor pointer");
  HMX_REQUIRE(gates || (g_dtype >= 0 && g_dtype <= 2 && beta_dtype >= 0 && beta_dtype <= 2),
              HMX_EUNSUPPORTED, "hmx_gdn_chunk_fwd: g/beta dtype");
  if (gates) {
    const int rc = check_gates(gates, false, "hmx_gdn_chunk_fwd");
    if (rc != HMX_OK) return rc;
  }
  HMX_REQUIRE(q_token_stride % 8 == 0 && k_token_stride % 8 == 0 && v_token_stride % 8 == 0 &&
                  ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)o) % 16 == 0,
              HMX_EINVAL, "hmx_gdn_chunk_fwd: q/k/v/o rows must be 16-byte aligned");
  HMX_REQUIRE(k_token_stride == v_token_stride, HMX_EINVAL,
              "hmx_gdn_chunk_fwd: k and v must share a token stride (%lld vs %lld)",
              (long long)k_token_stride, (long long)v_token_stride);
  // a chunk's rows are addressed by 32-bit byte offsets from its first row
  HMX_REQUIRE(q_token_stride > 0 && k_token_stride > 0 && q_token_stride < (1 << 26) &&
                  k_token_stride < (1 << 26),
              HMX_EINVAL, "hmx_gdn_chunk_fwd: token strides must lie in [1, 2^26) elements");
  HMX_REQUIRE(!(h0 || ht) || ((state_dtype == HMX_F32 || state_dtype == HMX_BF16) &&
                              state_slot_stride % 4 == 0 &&
                              ((uintptr_t)h0 | (uintptr_t)ht) % 16 == 0),
              HMX_EINVAL, "hmx_gdn_chunk_fwd: states must be f32/bf16 with 16-byte aligned "
              "slots (slot stride %lld)", (long long)state_slot_stride);
  if (nseg_total == 0) return HMX_OK;
  const int32_t pooled = state_indices != nullptr;
  const size_t need = hmx_gdn_chunk_workspace_bytes(nseg_total, N, H, pooled);
  HMX_REQUIRE(workspace && workspace_bytes >= need, HMX_EINVAL,
              "hmx_gdn_chunk_fwd: workspace of %zu bytes needed, %zu given", need,
              workspace_bytes);
  Params p;
  p.q = static_cast<const bf16*>(q); p.k = static_cast<const bf16*>(k);
  p.v = static_cast<const bf16*>(v);
  p.q_ts = q_token_stride; p.kv_ts = k_token_stride;
  p.g = g; p.g_dt = g_dtype; p.beta = beta; p.beta_dt = beta_dtype;
  p.fused = gates != nullptr;
  p.gp = gates ? *gates : hmx_gate_proj{};
  p.o = static_cast<bf16*>(o); p.h0 = h0; p.ht = ht;
  p.st_ss = state_slot_stride; p.st_dt = state_dtype;
  p.sidx = state_indices; p.hinit = has_initial_state;
  p.seg = seg_table; p.nseg_total = nseg_total; p.H = H; p.HKV = HKV; p.scale = scale;
  p.l2norm = use_qk_l2norm; p.max_warm = max_warm_chunks; p.decay_thresh = decay_threshold;
  p.zg = nullptr; p.zg_ts = p.zg_hs = 0; p.onw = nullptr; p.onw_dt = HMX_F32; p.on_eps = 0.f;
  p.ws_hc = block_states; p.cu_chunk = cu_blocks;
  if (o_norm) {
    HMX_REQUIRE(o_norm->weight && o_norm->weight_dtype >= 0 && o_norm->weight_dtype <= 2,
                HMX_EINVAL, "hmx_gdn_chunk_fwd: o_norm needs a weight (dtype code 0-2)");
    HMX_REQUIRE(!o_norm->gate || ((uintptr_t)o_norm->gate % 16 == 0 &&
                                  o_norm->gate_token_stride % 8 == 0 &&
                                  o_norm->gate_head_stride % 8 == 0),
                HMX_EINVAL, "hmx_gdn_chunk_fwd: o_norm gate rows must be 16-byte aligned");
    p.zg = static_cast<const bf16*>(o_norm->gate);
    p.zg_ts = o_norm->gate_token_stride; p.zg_hs = o_norm->gate_head_stride;
    p.onw = o_norm->weight; p.onw_dt = o_norm->weight_dtype; p.on_eps = o_norm->eps;
  }
  // workspace carve-up: state buffers first (256-byte aligned), then plan/exact
  const size_t st = (size_t)nseg_total * H * D * D * sizeof(float);
  char* ws = static_cast<char*>(workspace);
  const bool multi = nseg_total > N;
  p.ws_s0 = multi ? reinterpret_cast<float*>(ws) : nullptr;
  p.ws_phi = multi ? reinterpret_cast<float*>(ws + st) : nullptr;
  p.ws_init = multi ? reinterpret_cast<float*>(ws + 2 * st) : nullptr;
  const bool staged = multi && pooled && ht;
  p.ws_ht = staged ? reinterpret_cast<float*>(ws + 3 * st) : nullptr;
  char* tail = ws + (multi ? 3 * st : 0) + (multi && pooled ? (size_t)N * H * D * D * 4 : 0);
  p.plan = reinterpret_cast<int*>(tail);
  p.redo = p.plan + (size_t)nseg_total * H;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(nseg_total, H);
  // multi-segment: plan; the exact pairs' S0 / Phi pre-pass; their segment
  // combine; every output walk.  One segment per sequence: every walk starts
  // from h0.
  if (multi) {
    const dim3 pre(nseg_total, H, 2);
    if (p.fused) {
      hipLaunchKernelGGL(gdn_plan_kernel<true>, grid, dim3(64), 0, s, p);
      hipLaunchKernelGGL(gdn_pre_kernel<true>, pre, dim3(NTHR), 0, s, p);
    } else {
      hipLaunchKernelGGL(gdn_plan_kernel<false>, grid, dim3(64), 0, s, p);
      hipLaunchKernelGGL(gdn_pre_kernel<false>, pre, dim3(NTHR), 0, s, p);
    }
    // blocks b: slice (b / 8) % 8 of pair (b % 8) + 8 (b / 64)
    hipLaunchKernelGGL(gdn_seg_combine_kernel, dim3((N * H + 7) / 8 * 64), dim3(CMB_THR), 0, s,
                       p, N);
  } else {
    p.plan = nullptr;
  }
  // every output walk, then again (scaled) the ones that left fp16's range
  if (o_norm && p.fused) {
    hipLaunchKernelGGL((gdn_chunk_kernel<true, true>), grid, dim3(NTHR), 0, s, p);
    hipLaunchKernelGGL((gdn_redo_kernel<true, true>), grid, dim3(NTHR), 0, s, p);
  } else if (o_norm) {
    hipLaunchKernelGGL((gdn_chunk_kernel<true, false>), grid, dim3(NTHR), 0, s, p);
    hipLaunchKernelGGL((gdn_redo_kernel<true, false>), grid, dim3(NTHR), 0, s, p);
  } else if (p.fused) {
    hipLaunchKernelGGL((gdn_chunk_kernel<false, true>), grid, dim3(NTHR), 0, s, p);
    hipLaunchKernelGGL((gdn_redo_kernel<false, true>), grid, dim3(NTHR), 0, s, p);
  } else {
    hipLaunchKernelGGL((gdn_chunk_kernel<false, false>), grid, dim3(NTHR), 0, s, p);
    hipLaunchKernelGGL((gdn_redo_kernel<false, false>), grid, dim3(NTHR), 0, s, p);
  }
  if (staged) hipLaunchKernelGGL(gdn_state_copy_kernel, dim3(N, H), dim3(NTHR), 0, s, p);
  return check_launch("hmx_gdn_chunk_fwd");
}

extern "C" int hmx_gdn_chunk_fwd(const void* q, int64_t q_token_stride, const void* k,
                                 int64_t k_token_stride, const void* v, int64_t v_token_stride,
                                 int32_t qkv_dtype, const void* g, int32_t g_dtype,
                                 const void* beta, int32_t beta_dtype, void* o, const void* h0,
                                 void* ht, int64_t state_slot_stride, int32_t state_dtype,
                                 const int32_t* state_indices, const uint8_t* has_initial_state,
                                 const int32_t* seg_table, int32_t nseg_total, int32_t N,
                                 int32_t H, int32_t HKV, int32_t K, int32_t V, float scale,
                                 int32_t use_qk_l2norm, int32_t max_warm_chunks,
                                 float decay_threshold, void* workspace, size_t workspace_bytes,
                                 const hmx_gated_norm* o_norm, const hmx_gate_proj* gates,
                                 void* stream) {
  return chunk_fwd_impl(q, q_token_stride, k, k_token_stride, v, v_token_stride, qkv_dtype, g,
                        g_dtype, beta, beta_dtype, o, h0, ht, state_slot_stride, state_dtype,
                        state_indices, has_initial_state, seg_table, nseg_total, N, H, HKV, K, V,
                        scale, use_qk_l2norm, max_warm_chunks, decay_threshold, workspace,
                        workspace_bytes, o_norm, gates, stream, nullptr, nullptr);
}

extern "C" size_t hmx_gdn_chunk_workspace_bytes(int32_t nseg_total, int32_t N, int32_t H,
                                                int32_t pooled) {
  const bool multi = nseg_total > N;
  size_t b = multi ? 3 * (size_t)nseg_total * H * D * D * sizeof(float) : 0;
  if (multi && pooled) b += (size_t)N * H * D * D * sizeof(float);   // staged end states
  b += 2 * (size_t)nseg_total * H * sizeof(int);                    // plan, redo flags
  return b;
}

// ===========================================================================
// Training: the backward of the chunked gated delta rule.
//
// Per 32-token block (the forward's chunk) with S0 the state entering it (written
// by the training forward), gamma the in-block cumsum of g, E = diag(e^gamma),
// F = diag(e^{gamma_L - gamma}), Gm_ij = e^{gamma_i - gamma_j}, unit rows q^, k^
// (in-kernel L2 normalisation) and the forward's
//   Mm = strict_lower(K^K^T . Gm),  T = (I + diag(beta) Mm)^-1,
//   Ut = V - E K^ S0,  W = T diag(beta) Ut,  S_L = e^{gamma_L} S0 + K^T F W,
//   O  = scale (E Q^ S0 + lower(Q^K^T . Gm) W),
// the gradient dS of S_L gives
//   dW = scale lower(Q^K^T . Gm)^T dO + F K^ dS,  Z = T^T dW,  dV = diag(beta) Z,
//   dN = -strict_lower(Z W^T),  Dm = diag(beta) dN . Gm,  Dp = scale lower(dO W^T) . Gm,
//   dQ^ = scale E dO S0^T + Dp K^,
//   dK^ = -E diag(beta) Z S0^T + F W dS^T + Dp^T Q^ + (Dm + Dm^T) K^,
//   dbeta = rowdot(Z, Ut) + rowsum(dN . Mm),
//   dgamma = rowdot(Q^, scale E dO S0^T) + rowdot(K^, -E diag(beta) Z S0^T - F W dS^T)
//            + (rowsum - colsum)(Dp . Q^K^T) + (rowsum - colsum)(Dm . K^K^T),
//   dgamma_L += e^{gamma_L} <dS, S0> + sum_j k^_j . (F W dS^T)_j,
//   dS0 = e^{gamma_L} dS + scale Q^T E dO - K^T E diag(beta) Z,
// then dg = the in-block reverse cumsum of dgamma and the L2 backward
// dq = (dq^ - q^ (q^ . dq^)) / sqrt(|q|^2 + 1e-6) (k likewise).
//
// Three launches: a block-parallel prep (T and scale lower(Q^K^T . Gm), fp16), the
// reverse chain of dS over each sequence's blocks (one workgroup per sequence and
// head, wave w owning value columns 16w.., the fp32 dS in MFMA accumulators; it
// writes each block's dS in fp16), and the block-parallel gradient kernel.  Every
// MFMA operand is fp16 (one rounding) with fp32 accumulation.
// ===========================================================================
namespace hmx {
namespace gdnp {
namespace train {

constexpr int LR = 144;       // fp16 row stride of [rows][128] LDS arrays (72 dwords)
constexpr int LL = 40;        // fp16 row stride of [32][32] LDS arrays
constexpr int LF = 33;        // fp32 row stride of [32][32] LDS arrays
constexpr int BNTHR = 512;    // 8 waves

struct Bwd {
  const bf16* q; const bf16* k; const bf16* v;
  int64_t q_ts, kv_ts;        // token strides (elements); heads are D apart
  const void* g; int g_dt;
  const void* beta; int beta_dt;
  const bf16* dout; int64_t do_ts;
  const float* dht;           // [N][H][D][D] gradient of the final states, or null
  const f16* hc;              // [nblk][H][D][D] state entering each block
  f16* dhc;                   // [nblk][H][D][D] gradient of the state leaving each block
  f16* tm;                    // [nblk][H][C][C] T
  f16* pm;                    // [nblk][H][C][C] scale lower(Q^K^T . Gm)
  const int* ctab;            // [nblk][4]: first token, tokens, sequence, block in sequence
  const int* cu_blk;          // [N+1]
  const int* cseg;            // [nseg][3]: sequence, first block, end block of a chain run
  int nseg;
  int max_warm;               // warm-up blocks a chain run may add past its end
  float decay_thresh;         // ... to bring the dropped history under e^-decay_thresh
  int* cplan;                 // [nseg][H]: where a run's chain starts (its warm-up end), or -1
  // Exact runs, compact over the runs that need them (rows grouped by ascending
  // sequence, each sequence's runs tiling its blocks in order; row s of sequence n):
  float* cR;                  // [nseg-N][H][D][D] at s-n-1, runs after a sequence's first:
                              //   the chain from zero over the run
  float* cPsi;                // [nseg-N][H][D][D] ... and the product of its transposed transitions
  float* cstart;              // [nseg-N][H][D][D] at s-n, runs before a sequence's last:
                              //   the exact dS at the run's end
  bf16* dq; bf16* dk; bf16* dv;   // [tokens][H][D]
  float* dg; float* dbeta;        // [tokens][H]
  float* dh0;                 // [N][H][D][D] or null
  int H, nblk;
  float scale;
  int l2norm;
};

// B (or A^T) operand from a row-major fp16 array M: column c0 + (l & 15), k = rows
// k0 + 8 (l >> 4) .. +7 (natural order; pairs with frag_h)
__device__ __forceinline__ f16x8 frag_col(const f16* b, int ld, int k0, int c0, int lane) {
  const int kq = k0 + 8 * (lane >> 4);
  const f16x4 x = ld_tr_h(b, ld, kq, c0, lane);
  const f16x4 y = ld_tr_h(b, ld, kq + 4, c0, lane);
  return f16x8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
}

// the row of a block that thread tid stages (features 8 (tid & 15) .. +7 of row
// tid >> 4), or zeros past the block's tokens
__device__ __forceinline__ bf16x8 ld_row(const bf16* src, int64_t ts, int tok0, int nval, int tid) {
  const int row = tid >> 4, f0 = (tid & 15) * 8;
  return row < nval ? *reinterpret_cast<const bf16x8*>(src + (int64_t)(tok0 + row) * ts + f0)
                    : bf16x8{};
}
// ... and its store into an fp16 [32][LR] array, times 1 / sqrt(|x|^2 + 1e-6) with l2
// (that factor into rnorm[row] when given)
__device__ __forceinline__ void put_row(f16* dst, const bf16x8& x, bool l2, float* rnorm, int tid) {
  const int row = tid >> 4, f0 = (tid & 15) * 8;
  const float r = l2 ? row_inv_norm(x) : 1.f;
  *reinterpret_cast<f16x8*>(dst + row * LR + f0) = scale_h8(x, r);
  if (rnorm && (tid & 15) == 0) rnorm[row] = r;
}

struct Sc { float* G; float* E; float* F; float* B; };

// wave 0: the block's in-block cumsum of g, e^gamma, e^{gamma_L - gamma} and beta
// into LDS (lanes 0-31; 0 / 0 past the block's tokens)
__device__ __forceinline__ void ld_gates(const Bwd& p, int tok0, int nval, int h, int lane,
                                         float& gv, float& bv) {
  const bool ok = lane < nval;
  const int64_t i = (int64_t)(tok0 + lane) * p.H + h;
  gv = ok ? ld_scalar(p.g, i, p.g_dt) : 0.f;
  bv = ok ? ld_scalar(p.beta, i, p.beta_dt) : 0.f;
}
__device__ __forceinline__ void block_scalars(const Sc& s, float gv, float bv, int lane) {
  const float gam = scan32(gv);
  const float gl = __builtin_bit_cast(float,
                                      __builtin_amdgcn_readlane(__builtin_bit_cast(int, gam), C - 1));
  if (lane < C) {
    s.G[lane] = gam;
    s.E[lane] = fast_exp(gam);
    s.F[lane] = fast_exp(gl - gam);
    s.B[lane] = bv;
  }
}

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xF, 0xF, false));
}
// The sums of x[0..3] over the 16 lanes of a DPP row, by a transposing reduction
// (five DPP additions instead of sixteen): lane l16 receives the sum of x[l16 & 3].
__device__ __forceinline__ float row16_sum4(const f32x4& x, int l16) {
  const bool b = l16 & 1, c = l16 & 2;
  const float y0 = (b ? x[1] : x[0]) + dppf<0xB1>(b ? x[0] : x[1]);   // x[b], lanes l, l ^ 1
  const float y1 = (b ? x[3] : x[2]) + dppf<0xB1>(b ? x[2] : x[3]);   // x[b + 2]
  float z = (c ? y1 : y0) + dppf<0x4E>(c ? y0 : y1);                   // x[l & 3], l ^ 2 too
  z += dppf<0x124>(z);                                                  // row_ror:4
  z += dppf<0x128>(z);                                                  // row_ror:8
  return z;
}

// rows 16 mt + 4 q4 .. +3 of a per-token LDS array (one 16-byte read)
__device__ __forceinline__ f32x4 row4(const float* a, int mt, int q4) {
  return *reinterpret_cast<const f32x4*>(a + 16 * mt + 4 * q4);
}

__device__ __forceinline__ Sc sc_at(unsigned char* base) {
  float* f = reinterpret_cast<float*>(base);
  return Sc{f, f + C, f + 2 * C, f + 3 * C};
}

// ---- prep: T and scale lower(Q^K^T . Gm) of every block ----------------------
constexpr int PR_OFF_K = 0, PR_OFF_Q = C * LR * 2, PR_OFF_N = 2 * C * LR * 2;
constexpr int PR_OFF_T = PR_OFF_N + C * LF * 4, PR_OFF_SC = PR_OFF_T + C * LF * 4;
constexpr int PR_SMEM = PR_OFF_SC + 4 * C * 4;

__global__ __launch_bounds__(BNTHR) void gdn_bwd_prep_kernel(Bwd p) {
  __shared__ __align__(16) unsigned char smem[PR_SMEM];
  f16* sK = reinterpret_cast<f16*>(smem + PR_OFF_K);
  f16* sQ = reinterpret_cast<f16*>(smem + PR_OFF_Q);
  float* sN = reinterpret_cast<float*>(smem + PR_OFF_N);
  float* sT = reinterpret_cast<float*>(smem + PR_OFF_T);
  const Sc sc = sc_at(smem + PR_OFF_SC);
  const int cb = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, l16 = lane & 15;
  const int tok0 = p.ctab[cb * 4], nval = p.ctab[cb * 4 + 1];
  {
    const bf16x8 xk = ld_row(p.k + (int64_t)h * D, p.kv_ts, tok0, nval, tid);
    const bf16x8 xq = ld_row(p.q + (int64_t)h * D, p.q_ts, tok0, nval, tid);
    float gv = 0.f, bv = 0.f;
    if (wave == 0) ld_gates(p, tok0, nval, h, lane, gv, bv);
    put_row(sK, xk, p.l2norm, nullptr, tid);
    put_row(sQ, xq, p.l2norm, nullptr, tid);
    if (wave == 0) block_scalars(sc, gv, bv, lane);
  }
  lds_barrier();
  const int64_t mo = ((int64_t)cb * p.H + h) * C * C;
  {  // waves 0-3: a tile of Q^K^T -> P; waves 4-7: a tile of K^K^T -> N = beta Mm
    const int t = wave & 3, mt = t >> 1, nt = t & 1;
    const f16* A = wave < 4 ? sQ : sK;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      acc = mfma16h(frag_h(A, LR, 16 * mt, 32 * ks, lane), frag_h(sK, LR, 16 * nt, 32 * ks, lane),
                    acc);
    const int j = 16 * nt + l16;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int i = 16 * mt + 4 * q4 + v;
      const float gm = j <= i ? fast_exp(sc.G[i] - sc.G[j]) : 0.f;
      if (wave < 4) p.pm[mo + i * C + j] = (f16)(p.scale * acc[v] * gm);
      else sN[i * LF + j] = j < i ? sc.B[i] * acc[v] * gm : 0.f;
    }
  }
  lds_barrier();
  // T = (I + N)^-1: the diagonal 16x16 blocks by forward substitution (lane l of
  // each half solves for column l of its block) ...
  if (wave == 0 && lane < C) {
    const int o = (lane >> 4) * 16, l = lane & 15;
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float s = (i == l) ? 1.f : 0.f;
#pragma unroll
      for (int j = 0; j < i; ++j) s -= sN[(o + i) * LF + o + j] * t[j];
      t[i] = s;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sT[(o + i) * LF + o + l] = t[i];
  }
  lds_barrier();
  // ... then T_10 = -T_11 (N_10 T_00), the inner product held in T's upper-right block
  if (tid < 256) {
    const int i = tid >> 4, j = tid & 15;
    float y = 0.f;
    for (int k = j; k < 16; ++k) y += sN[(16 + i) * LF + k] * sT[k * LF + j];
    sT[i * LF + 16 + j] = y;
  }
  lds_barrier();
  if (tid < 256) {
    const int i = tid >> 4, j = tid & 15;
    float y = 0.f;
    for (int k = 0; k <= i; ++k) y += sT[(16 + i) * LF + 16 + k] * sT[k * LF + 16 + j];
    sT[(16 + i) * LF + j] = -y;
  }
  lds_barrier();
  for (int e = tid; e < C * C; e += BNTHR) {
    const int i = e >> 5, j = e & 31;
    p.tm[mo + e] = (f16)(j > i ? 0.f : sT[i * LF + j]);
  }
}

// ---- the reverse chain of the state gradient ---------------------------------
constexpr int CH_OFF_K = 0, CH_OFF_Q = C * LR * 2, CH_OFF_DO = 2 * C * LR * 2;
constexpr int CH_OFF_T = 3 * C * LR * 2, CH_OFF_P = CH_OFF_T + C * LL * 2;
constexpr int CH_OFF_SC = CH_OFF_P + C * LL * 2;
constexpr int CH_SMEM = CH_OFF_SC + 4 * C * 4;     // 33 KB: three workgroups per CU

// One block's global inputs for this thread, loaded a block or two ahead of use:
// its row of k, q and dO (features 8 (tid & 15) .. +7 of row tid >> 4), two
// entries of T and P, and (wave 0, lanes 0-31) the token's g and beta.
struct ChainPre {
  bf16x8 k, q, o;
  uint32_t t, pm;
  float g, b;
};

__device__ __forceinline__ void chain_load(const Bwd& p, ChainPre& r, int cb, int tok0, int nval,
                                           int h, int tid, int wave, int lane) {
  const int row = tid >> 4, f0 = (tid & 15) * 8;
  const bool ok = row < nval;
  const int64_t t = tok0 + row;
  r.k = ok ? *reinterpret_cast<const bf16x8*>(p.k + t * p.kv_ts + (int64_t)h * D + f0) : bf16x8{};
  r.q = ok ? *reinterpret_cast<const bf16x8*>(p.q + t * p.q_ts + (int64_t)h * D + f0) : bf16x8{};
  r.o = ok ? *reinterpret_cast<const bf16x8*>(p.dout + t * p.do_ts + (int64_t)h * D + f0) : bf16x8{};
  const int64_t mo = ((int64_t)cb * p.H + h) * C * C + 2 * tid;
  r.t = *reinterpret_cast<const uint32_t*>(p.tm + mo);
  r.pm = *reinterpret_cast<const uint32_t*>(p.pm + mo);
  r.g = r.b = 0.f;
  if (wave == 0 && lane < nval) {
    const int64_t i = (int64_t)(tok0 + lane) * p.H + h;
    r.g = ld_scalar(p.g, i, p.g_dt);
    r.b = ld_scalar(p.beta, i, p.beta_dt);
  }
}

enum ChainMode { CH_WALK = 0, CH_R = 1, CH_PSI = 2 };

// The first chain-run row whose sequence is >= n (rows are grouped by ascending
// sequence): a wave-uniform binary search, log2(nseg) dependent loads.
__device__ __forceinline__ int seq_lower_bound(const Bwd& p, int n) {
  int lo = 0, hi = p.nseg;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (p.cseg[mid * 3] < n) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// The rows of the chain-run table that belong to sequence n: [r0, r1).
__device__ __forceinline__ void seq_runs(const Bwd& p, int n, int lane, int& r0, int& r1) {
  (void)lane;
  r0 = seq_lower_bound(p, n);
  r1 = seq_lower_bound(p, n + 1);
}

// Whether any run of sequence n needs the exact combine for head h (wave-uniform).
__device__ __forceinline__ bool head_exact(const Bwd& p, int n, int h, int lane) {
  int r0, r1;
  seq_runs(p, n, lane, r0, r1);
  for (int s0 = r0; s0 < r1; s0 += 64) {
    const int s = s0 + lane;
    if (__ballot(s < r1 && p.cplan[s * p.H + h] < 0)) return true;
  }
  return false;
}

// ---- plan: where each run's chain starts --------------------------------------
// A run that ends before its sequence does starts from zero at the end of a
// warm-up over the following blocks, long enough that the dropped history, bounded
// by prod_t e^{g_t} max(1, |1 - beta_t|) (the spectral norm of e^g (I - beta k k^T)
// for |k| = 1, which the in-kernel L2 normalisation guarantees), is below
// e^-decay_thresh.  Without that bound within max_warm blocks, or without the
// normalisation, the run is exact (-1): its head then takes the combine.  One wave
// per (run, head) reads 16 blocks' gates at a time: lane l sums tokens 8 (l & 3) ..
// +7 of block l >> 2, then a prefix over the blocks finds the first one that brings
// the bound below the threshold.
__global__ __launch_bounds__(64) void gdn_bwd_plan_kernel(Bwd p) {
  const int sg = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int n = p.cseg[sg * 3], bb = p.cseg[sg * 3 + 2];
  const int first = p.cu_blk[n], last = p.cu_blk[n + 1];
  int w = last;
  if (bb < last) {
    w = -1;
    if (p.l2norm) {
      const int bos = p.ctab[first * 4];
      const int eos = p.ctab[(last - 1) * 4] + p.ctab[(last - 1) * 4 + 1];
      float acc = 0.f;
      const int lim = min(last, bb + p.max_warm);
      for (int base = bb; base < lim; base += 16) {
        const int cb = base + (lane >> 2);
        float x = 0.f;
        if (cb < lim) {
          const int t0 = bos + (cb - first) * C + 8 * (lane & 3), t1 = min(t0 + 8, eos);
          for (int t = t0; t < t1; ++t) {
            const int64_t i = (int64_t)t * p.H + h;
            x += ld_scalar(p.g, i, p.g_dt) +
                 __logf(fmaxf(1.f, fabsf(1.f - ld_scalar(p.beta, i, p.beta_dt))));
          }
        }
        x += __shfl_xor(x, 1, 64);
        x += __shfl_xor(x, 2, 64);          // the block's sum, in its four lanes
        float pre = x;                      // inclusive prefix over the blocks
#pragma unroll
        for (int off = 4; off < 64; off <<= 1) {
          const float y = __shfl_up(pre, off, 64);
          if (lane >= off) pre += y;
        }
        const unsigned long long hit = __ballot(cb < lim && acc + pre < -p.decay_thresh);
        if (hit) {
          w = base + (__builtin_ctzll(hit) >> 2) + 1;
          break;
        }
        acc += __shfl(pre, 63, 64);
      }
    }
  }
  if (lane == 0) p.cplan[sg * p.H + h] = w;
}

// ---- combine: the exact dS at every run end of a head with an exact run ---------
// Backward over the runs of sequence n: X = dht (or 0) at the sequence end; run r
// starts from X, and X <- Psi_r X + R_r is the dS at the end of run r - 1.  X is
// kept in fp32 accumulators (wave w owns columns 16w..); each product splits X into
// fp16 hi + lo and rounds Psi_r (a product of contractions) to fp16 once.
constexpr int CB_SMEM = D * LR * 2;
__global__ __launch_bounds__(BNTHR, 1) void gdn_bwd_combine_kernel(Bwd p) {
  __shared__ __align__(16) unsigned char smem[CB_SMEM];
  f16* sPsi = reinterpret_cast<f16*>(smem);
  const int n = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, l16 = lane & 15, c0 = 16 * wave;
  if (!head_exact(p, n, h, lane)) return;
  int r0, r1;
  seq_runs(p, n, lane, r0, r1);
  const int64_t DD = (int64_t)D * D;
  f32x4 X[8];
  const float* src = p.dht ? p.dht + ((int64_t)n * p.H + h) * DD : nullptr;
#pragma unroll
  for (int rt = 0; rt < 8; ++rt)
#pragma unroll
    for (int v = 0; v < 4; ++v) X[rt][v] = src ? src[(16 * rt + 4 * q4 + v) * D + c0 + l16] : 0.f;
  for (int r = r1 - 1; r >= r0; --r) {
    if (r < r1 - 1) {   // the last run starts from dht itself
      const int64_t os = ((int64_t)(r - n) * p.H + h) * DD;
#pragma unroll
      for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int v = 0; v < 4; ++v) p.cstart[os + (16 * rt + 4 * q4 + v) * D + c0 + l16] = X[rt][v];
    }
    if (r == r0) break;
    const int64_t o = ((int64_t)(r - n - 1) * p.H + h) * DD;
    lds_barrier();   // the previous run's Psi reads are done
    for (int e = tid * 8; e < D * D; e += BNTHR * 8) {   // Psi_r into LDS, fp16, interleaved
      float f[8];
      load_vec<8>(p.cPsi + o + e, f);
      f16x8 y;
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = (f16)f[j];
      store8_i(sPsi + (e >> 7) * LR, e & 127, y);
    }
    lds_barrier();
    f16x8 xh[4], xl[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      f32x4 lo0, lo1;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        lo0[v] = X[2 * m][v] - (float)(f16)X[2 * m][v];
        lo1[v] = X[2 * m + 1][v] - (float)(f16)X[2 * m + 1][v];
      }
      xh[m] = h8(X[2 * m], X[2 * m + 1]);
      xl[m] = h8(lo0, lo1);
    }
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) {
      f32x4 acc;
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[v] = p.cR[o + (16 * rt + 4 * q4 + v) * D + c0 + l16];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const f16x8 a = frag_i(sPsi, LR, 16 * rt, 32 * m, lane);
        acc = mfma16h(a, xh[m], acc);
        acc = mfma16h(a, xl[m], acc);
      }
      X[rt] = acc;
    }
  }
}

__global__ __launch_bounds__(BNTHR, 3) void gdn_bwd_chain_kernel(Bwd p, int mode) {
  __shared__ __align__(16) unsigned char smem[CH_SMEM];
  f16* sK = reinterpret_cast<f16*>(smem + CH_OFF_K);
  f16* sQ = reinterpret_cast<f16*>(smem + CH_OFF_Q);
  f16* sDO = reinterpret_cast<f16*>(smem + CH_OFF_DO);
  f16* sT = reinterpret_cast<f16*>(smem + CH_OFF_T);
  f16* sP = reinterpret_cast<f16*>(smem + CH_OFF_P);
  const Sc sc = sc_at(smem + CH_OFF_SC);
  const int sg = blockIdx.x, h = blockIdx.y;
  if (mode != CH_WALK) mode = blockIdx.z ? CH_PSI : CH_R;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, l16 = lane & 15;
  const int c0 = 16 * wave;                      // this wave's value columns
  const int64_t DD = (int64_t)D * D;
  const int n = p.cseg[sg * 3], ba = p.cseg[sg * 3 + 1], bb = p.cseg[sg * 3 + 2];
  const int first = p.cu_blk[n], last = p.cu_blk[n + 1];   // the sequence's blocks
  // a sequence's blocks are consecutive 32-token runs from its first token
  int bos = 0, eos = 0;
  if (last > first) {
    bos = p.ctab[first * 4];
    eos = p.ctab[(last - 1) * 4] + p.ctab[(last - 1) * 4 + 1];
  }
  auto blk_tok = [&](int cb) { return bos + (cb - first) * C; };
  // Where this run's chain starts and from what (the plan kernel's choice): after a
  // warm-up from zero, or from the sequence end (the last run); for a head with an
  // exact run, every run starts at its own end from the combine's exact dS.
  const bool hexact = head_exact(p, n, h, lane);
  int wend = p.cplan[sg * p.H + h];
  const float* src = nullptr;
  bool ident = false;
  if (mode == CH_WALK) {
    if (hexact) {
      wend = bb;
      if (bb < last) src = p.cstart + ((int64_t)(sg - n) * p.H + h) * DD;
    }
    if (wend == last && p.dht) src = p.dht + ((int64_t)n * p.H + h) * DD;
  } else {           // pre-pass of an exact head's run: R from zero, Psi from I
    if (!hexact || ba == first) return;
    wend = bb;
    ident = mode == CH_PSI;
  }
  // dS[rt]: rows 16 rt + 4 q4 + v, column c0 + l16
  f32x4 dS[8];
#pragma unroll
  for (int rt = 0; rt < 8; ++rt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = 16 * rt + 4 * q4 + v, col = c0 + l16;
      dS[rt][v] = src ? src[row * D + col] : ((ident && row == col) ? 1.f : 0.f);
    }
  const bool with_do = mode != CH_PSI;
  ChainPre pa, pb;                               // blocks cb and cb - 1
  if (wend > ba) chain_load(p, pa, wend - 1, blk_tok(wend - 1), min(C, eos - blk_tok(wend - 1)), h, tid, wave, lane);
  if (wend - 1 > ba) chain_load(p, pb, wend - 2, blk_tok(wend - 2), C, h, tid, wave, lane);
  for (int cb = wend - 1; cb >= ba; --cb) {
    if (mode == CH_WALK && cb < bb) {   // the gradient of the state leaving block cb
      f16* dst = p.dhc + ((int64_t)cb * p.H + h) * DD + c0 + l16;
#pragma unroll
      for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int v = 0; v < 4; ++v) dst[(16 * rt + 4 * q4 + v) * D] = (f16)dS[rt][v];
    }
    lds_barrier();   // the previous block's LDS reads are done
    {  // stage block cb from registers
      const int row = tid >> 4, f0 = (tid & 15) * 8;
      const float rk = p.l2norm ? row_inv_norm(pa.k) : 1.f;
      const float rq = p.l2norm ? row_inv_norm(pa.q) : 1.f;
      store8_i(sK + row * LR, f0, scale_h8(pa.k, rk));   // interleaved feature order
      *reinterpret_cast<f16x8*>(sQ + row * LR + f0) = scale_h8(pa.q, rq);
      *reinterpret_cast<f16x8*>(sDO + row * LR + f0) = scale_h8(pa.o, 1.f);
      const int e = 2 * tid, i = e >> 5, j = e & 31;
      *reinterpret_cast<uint32_t*>(sT + i * LL + j) = pa.t;
      *reinterpret_cast<uint32_t*>(sP + i * LL + j) = pa.pm;
      if (wave == 0) {
        const float gam = scan32(pa.g);
        const float gl = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gam), C - 1));
        if (lane < C) {
          sc.G[lane] = gam;
          sc.E[lane] = fast_exp(gam);
          sc.F[lane] = fast_exp(gl - gam);
          sc.B[lane] = pa.b;
        }
      }
    }
    // the loads two blocks ahead, in flight through this block's products
    pa = pb;
    if (cb - 2 >= ba) chain_load(p, pb, cb - 2, blk_tok(cb - 2), C, h, tid, wave, lane);
    lds_barrier();
    // dW = F K^ dS + P^T dO (tokens x this wave's columns), Z' = -E beta T^T dW
    f32x4 dW[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < 4; ++m)
        acc = mfma16h(frag_i(sK, LR, 16 * mt, 32 * m, lane), h8(dS[2 * m], dS[2 * m + 1]), acc);
#pragma unroll
      for (int v = 0; v < 4; ++v) dW[mt][v] = sc.F[16 * mt + 4 * q4 + v] * acc[v];
    }
    const f16x8 bdo = frag_col(sDO, LR, 0, c0, lane);
    if (with_do) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) dW[mt] = mfma16h(frag_col(sP, LL, 0, 16 * mt, lane), bdo, dW[mt]);
    }
    f32x4 Zp[2];
    {
      const f16x8 bw = h8(dW[0], dW[1]);
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const f32x4 Z = mfma16h(frag_t_perm_h(sT, LL, 0, 16 * mt, lane), bw, z);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int r = 16 * mt + 4 * q4 + v;
          Zp[mt][v] = -sc.E[r] * sc.B[r] * Z[v];
        }
      }
    }
    // dS <- e^{gamma_L} dS + K^T Z' + Q^T (scale E dO)
    f16x8 bqe;
#pragma unroll
    for (int j = 0; j < 8; ++j) bqe[j] = (f16)((float)bdo[j] * p.scale * sc.E[8 * q4 + j]);
    const f16x8 bz = h8(Zp[0], Zp[1]);
    const float eL = sc.E[C - 1];
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) {
#pragma unroll
      for (int v = 0; v < 4; ++v) dS[rt][v] *= eL;
      dS[rt] = mfma16h(frag_t_i(sK, LR, 0, 16 * rt, lane), bz, dS[rt]);
      if (with_do) dS[rt] = mfma16h(frag_col(sQ, LR, 0, 16 * rt, lane), bqe, dS[rt]);
    }
  }
  if (mode != CH_WALK) {   // the run's R or Psi
    float* dst = (mode == CH_R ? p.cR : p.cPsi) + ((int64_t)(sg - n - 1) * p.H + h) * DD + c0 + l16;
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
#pragma unroll
      for (int v = 0; v < 4; ++v) dst[(16 * rt + 4 * q4 + v) * D] = dS[rt][v];
    return;
  }
  if (p.dh0 && ba == first) {
    float* dst = p.dh0 + ((int64_t)n * p.H + h) * DD + c0 + l16;
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
#pragma unroll
      for (int v = 0; v < 4; ++v) dst[(16 * rt + 4 * q4 + v) * D] = dS[rt][v];
  }
}

// ---- the per-block gradients -------------------------------------------------
constexpr int SZR = C * LR * 2, SZS = D * LR * 2, SZL = C * LL * 2;
constexpr int G_OFF_K = 0, G_OFF_Q = SZR, G_OFF_DO = 2 * SZR, G_OFF_X = 3 * SZR;
constexpr int G_OFF_W = 4 * SZR, G_OFF_Z = 5 * SZR;
constexpr int G_OFF_S0 = 6 * SZR, G_OFF_DS = G_OFF_S0 + SZS;
constexpr int G_OFF_T = G_OFF_DS + SZS, G_OFF_PM = G_OFF_T + SZL;
constexpr int G_OFF_DP = G_OFF_PM + SZL, G_OFF_DM = G_OFF_DP + SZL;
constexpr int G_OFF_QK = G_OFF_DM + SZL, G_OFF_KK = G_OFF_QK + C * LF * 4;
constexpr int G_OFF_SC = G_OFF_KK + C * LF * 4;            // G, E, F, B, rq, rk
constexpr int NPG = 16, NPB = 10;
constexpr int G_OFF_PG = G_OFF_SC + 6 * C * 4;             // [16][32] dgamma pieces
constexpr int G_OFF_PB = G_OFF_PG + NPG * C * 4;           // [10][32] dbeta pieces
constexpr int G_OFF_PC = G_OFF_PB + NPB * C * 4;           // [8] sum_j k^_j . (F W dS^T)_j per wave
constexpr int G_OFF_PQ = G_OFF_PC + 8 * C * 4;             // [8][32] q^ . dq^ per wave
constexpr int G_OFF_PK = G_OFF_PQ + 8 * C * 4;             // [8][32] k^ . dk^ per wave
constexpr int G_OFF_PD = G_OFF_PK + 8 * C * 4;             // [8] <dS, S0> per wave
constexpr int G_SMEM = G_OFF_PD + 8 * 4;
static_assert(G_SMEM <= 160 * 1024, "LDS budget");

// One block's global inputs for this thread (loaded while the previous block is
// processed): its rows of k, q, dO, v; 1/4 of S0 and of dS; two entries of T and P;
// (wave 0, lanes 0-31) the token's g and beta.
struct GradPre {
  bf16x8 k, q, o, v;
  f16x8 s0[4], ds[4];
  uint32_t t, pm;
  float g, b;
};

__device__ __forceinline__ void grad_load(const Bwd& p, GradPre& r, int64_t bh, int h, int tok0,
                                          int nval, int tid, int wave, int lane) {
  r.k = ld_row(p.k + (int64_t)h * D, p.kv_ts, tok0, nval, tid);
  r.q = ld_row(p.q + (int64_t)h * D, p.q_ts, tok0, nval, tid);
  r.o = ld_row(p.dout + (int64_t)h * D, p.do_ts, tok0, nval, tid);
  r.v = ld_row(p.v + (int64_t)h * D, p.kv_ts, tok0, nval, tid);
  const int64_t DD = (int64_t)D * D;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int e = (pass * BNTHR + tid) * 8;
    r.s0[pass] = *reinterpret_cast<const f16x8*>(p.hc + bh * DD + e);
    r.ds[pass] = *reinterpret_cast<const f16x8*>(p.dhc + bh * DD + e);
  }
  r.t = *reinterpret_cast<const uint32_t*>(p.tm + bh * C * C + 2 * tid);
  r.pm = *reinterpret_cast<const uint32_t*>(p.pm + bh * C * C + 2 * tid);
  r.g = r.b = 0.f;
  if (wave == 0) ld_gates(p, tok0, nval, h, lane, r.g, r.b);
}

// Persistent: workgroup w takes blocks (block, head) = w, w + gridDim.x, ... and
// loads each one's inputs while it processes the one before.
__global__ __launch_bounds__(BNTHR, 1) void gdn_bwd_grad_kernel(Bwd p) {
  __shared__ __align__(16) unsigned char smem[G_SMEM];
  f16* sK = reinterpret_cast<f16*>(smem + G_OFF_K);
  f16* sQ = reinterpret_cast<f16*>(smem + G_OFF_Q);
  f16* sDO = reinterpret_cast<f16*>(smem + G_OFF_DO);
  f16* sX = reinterpret_cast<f16*>(smem + G_OFF_X);
  f16* sW = reinterpret_cast<f16*>(smem + G_OFF_W);
  f16* sZ = reinterpret_cast<f16*>(smem + G_OFF_Z);
  f16* sS0 = reinterpret_cast<f16*>(smem + G_OFF_S0);
  f16* sDS = reinterpret_cast<f16*>(smem + G_OFF_DS);
  f16* sT = reinterpret_cast<f16*>(smem + G_OFF_T);
  f16* sPm = reinterpret_cast<f16*>(smem + G_OFF_PM);
  f16* sDp = reinterpret_cast<f16*>(smem + G_OFF_DP);
  f16* sDm = reinterpret_cast<f16*>(smem + G_OFF_DM);
  float* sQK = reinterpret_cast<float*>(smem + G_OFF_QK);
  float* sKK = reinterpret_cast<float*>(smem + G_OFF_KK);
  const Sc sc = sc_at(smem + G_OFF_SC);
  float* sRq = sc.B + C;
  float* sRk = sRq + C;
  float* sPG = reinterpret_cast<float*>(smem + G_OFF_PG);
  float* sPB = reinterpret_cast<float*>(smem + G_OFF_PB);
  float* sPC = reinterpret_cast<float*>(smem + G_OFF_PC);
  float* sPQ = reinterpret_cast<float*>(smem + G_OFF_PQ);
  float* sPK = reinterpret_cast<float*>(smem + G_OFF_PK);
  float* sPD = reinterpret_cast<float*>(smem + G_OFF_PD);

  const int H = p.H, total = p.nblk * H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, l16 = lane & 15;
  const int c0 = 16 * wave;      // this wave's value columns (P1-P2) / key features (P3-P5)
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  int it = blockIdx.x;
  if (it >= total) return;
  int cb = it / H, h = it - cb * H;
  int tok0 = p.ctab[cb * 4], nval = p.ctab[cb * 4 + 1];
  GradPre pre;
  grad_load(p, pre, (int64_t)cb * H + h, h, tok0, nval, tid, wave, lane);
  for (;;) {
    const int nxt = it + gridDim.x;
    int ncb = 0, nh = 0, ntok0 = 0, nnval = 0;
    if (nxt < total) {
      ncb = nxt / H;
      nh = nxt - ncb * H;
      ntok0 = p.ctab[ncb * 4];
      nnval = p.ctab[ncb * 4 + 1];
    }
    const int64_t bh = (int64_t)cb * H + h;

    // ---- P0: stage this block from registers; the next block's loads go out -------
    lds_barrier();   // the previous block's LDS reads are done
    {
      put_row(sK, pre.k, p.l2norm, sRk, tid);
      put_row(sQ, pre.q, p.l2norm, sRq, tid);
      put_row(sDO, pre.o, false, nullptr, tid);
      put_row(sX, pre.v, false, nullptr, tid);
      if (wave == 0) block_scalars(sc, pre.g, pre.b, lane);
#pragma unroll
      for (int pass = 0; pass < 4; ++pass) {
        const int e = (pass * BNTHR + tid) * 8, row = e >> 7, col = e & 127;
        *reinterpret_cast<f16x8*>(sS0 + row * LR + col) = pre.s0[pass];
        *reinterpret_cast<f16x8*>(sDS + row * LR + col) = pre.ds[pass];
      }
      const int e2 = 2 * tid, i = e2 >> 5, j = e2 & 31;
      *reinterpret_cast<uint32_t*>(sT + i * LL + j) = pre.t;
      *reinterpret_cast<uint32_t*>(sPm + i * LL + j) = pre.pm;
    }
    if (nxt < total) grad_load(p, pre, (int64_t)ncb * H + nh, nh, ntok0, nnval, tid, wave, lane);
    lds_barrier();

    // ---- P1: K^ S0 and K^ dS (tokens x this wave's value columns), a tile of Q^K^T
    // or K^K^T, this wave's share of <dS, S0>; Ut = V - E K^ S0, beta Ut over V ----
    f32x4 Ut[2], KD[2];
    {
      f32x4 KS[2] = {zero, zero};
      KD[0] = KD[1] = zero;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const f16x8 bs = frag_col(sS0, LR, 32 * ks, c0, lane), bd = frag_col(sDS, LR, 32 * ks, c0, lane);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const f16x8 a = frag_h(sK, LR, 16 * mt, 32 * ks, lane);
          KS[mt] = mfma16h(a, bs, KS[mt]);
          KD[mt] = mfma16h(a, bd, KD[mt]);
        }
      }
      {
        const int t = wave & 3, mt = t >> 1, nt = t & 1;
        const f16* A = wave < 4 ? sQ : sK;
        f32x4 acc = zero;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          acc = mfma16h(frag_h(A, LR, 16 * mt, 32 * ks, lane), frag_h(sK, LR, 16 * nt, 32 * ks, lane), acc);
        float* dst = wave < 4 ? sQK : sKK;
#pragma unroll
        for (int v = 0; v < 4; ++v) dst[(16 * mt + 4 * q4 + v) * LF + 16 * nt + l16] = acc[v];
      }
      {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 16 * wave + 4 * i + q4, col = 8 * l16;
          const f16x8 a = *reinterpret_cast<const f16x8*>(sS0 + row * LR + col);
          const f16x8 b = *reinterpret_cast<const f16x8*>(sDS + row * LR + col);
#pragma unroll
          for (int j = 0; j < 8; ++j) d += (float)a[j] * (float)b[j];
        }
        d = wave_sum(d);
        if (lane == 0) sPD[wave] = d;
      }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const f32x4 e4 = row4(sc.E, mt, q4), b4 = row4(sc.B, mt, q4);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int r = 16 * mt + 4 * q4 + v, idx = r * LR + c0 + l16;
          Ut[mt][v] = (float)sX[idx] - e4[v] * KS[mt][v];
          sX[idx] = (f16)(b4[v] * Ut[mt][v]);
        }
      }
    }
    lds_barrier();

    // ---- P2: W = T (beta Ut); dW = P^T dO + F K^ dS; Z = T^T dW; dv; rowdot(Z, Ut) --
    {
      const f16x8 bx = frag_col(sX, LR, 0, c0, lane), bdo = frag_col(sDO, LR, 0, c0, lane);
      f32x4 W[2], dW[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        W[mt] = mfma16h(frag_h(sT, LL, 16 * mt, 0, lane), bx, zero);
        const f32x4 f4r = row4(sc.F, mt, q4);
#pragma unroll
        for (int v = 0; v < 4; ++v) dW[mt][v] = f4r[v] * KD[mt][v];
        dW[mt] = mfma16h(frag_col(sPm, LL, 0, 16 * mt, lane), bdo, dW[mt]);
      }
      const f16x8 bw = h8(dW[0], dW[1]);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const f32x4 Z = mfma16h(frag_t_perm_h(sT, LL, 0, 16 * mt, lane), bw, zero);
        const f32x4 b4 = row4(sc.B, mt, q4);
        f32x4 zu;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int r = 16 * mt + 4 * q4 + v, idx = r * LR + c0 + l16;
          sW[idx] = (f16)W[mt][v];
          sZ[idx] = (f16)Z[v];
          if (r < nval) p.dv[((int64_t)(tok0 + r) * H + h) * D + c0 + l16] = (bf16)(b4[v] * Z[v]);
          zu[v] = Z[v] * Ut[mt][v];
        }
        const float zs = row16_sum4(zu, l16);
        if (l16 < 4) sPB[wave * C + 16 * mt + 4 * q4 + l16] = zs;
      }
    }
    lds_barrier();

    // ---- P3: dO S0^T, Z S0^T, W dS^T (tokens x this wave's key features); a tile of
    // Z W^T (-> dN, Dm) or dO W^T (-> Dp) with their row and column sums -------------
    f32x4 DQ[2], DK[2];
    f32x4 qh[2], kh[2];      // q^, k^ at this lane's accumulator positions
    {
      float cs = 0.f;
      f32x4 A0[2] = {zero, zero}, A1[2] = {zero, zero}, A2[2] = {zero, zero};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const f16x8 bs = frag_h(sS0, LR, c0, 32 * ks, lane), bd = frag_h(sDS, LR, c0, 32 * ks, lane);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          A0[mt] = mfma16h(frag_h(sDO, LR, 16 * mt, 32 * ks, lane), bs, A0[mt]);
          A1[mt] = mfma16h(frag_h(sZ, LR, 16 * mt, 32 * ks, lane), bs, A1[mt]);
          A2[mt] = mfma16h(frag_h(sW, LR, 16 * mt, 32 * ks, lane), bd, A2[mt]);
        }
      }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const f32x4 e4 = row4(sc.E, mt, q4), b4 = row4(sc.B, mt, q4), f4r = row4(sc.F, mt, q4);
        f32x4 gq;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int r = 16 * mt + 4 * q4 + v, idx = r * LR + c0 + l16;
          const float qt = p.scale * e4[v] * A0[mt][v];
          const float ut = -e4[v] * b4[v] * A1[mt][v];
          const float st = f4r[v] * A2[mt][v];
          qh[mt][v] = (float)sQ[idx];
          kh[mt][v] = (float)sK[idx];
          DQ[mt][v] = qt;
          DK[mt][v] = ut + st;
          gq[v] = qh[mt][v] * qt + kh[mt][v] * (ut - st);
          cs += kh[mt][v] * st;
        }
        const float gs = row16_sum4(gq, l16);
        if (l16 < 4) sPG[(8 + wave) * C + 16 * mt + 4 * q4 + l16] = gs;
      }
      cs = wave_sum(cs);
      if (lane == 0) sPC[wave] = cs;
    }
    {
      const int t = wave & 3, mt = t >> 1, nt = t & 1;
      const f16* A = wave < 4 ? sZ : sDO;
      f32x4 acc = zero;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        acc = mfma16h(frag_h(A, LR, 16 * mt, 32 * ks, lane), frag_h(sW, LR, 16 * nt, 32 * ks, lane), acc);
      const int j = 16 * nt + l16;
      const float gj = sc.G[j];
      const f32x4 gi4 = row4(sc.G, mt, q4), bi4 = row4(sc.B, mt, q4);
      float csum = 0.f;
      f32x4 xs, dbs;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 16 * mt + 4 * q4 + v;
        const float gm = j <= i ? fast_exp(gi4[v] - gj) : 0.f;
        float x;
        if (wave < 4) {   // dN = -strict_lower(Z W^T), Dm = beta dN . Gm
          const float dn = j < i ? -acc[v] : 0.f;
          const float kk = sKK[i * LF + j];
          const float d = bi4[v] * dn * gm;
          sDm[i * LL + j] = (f16)d;
          x = d * kk;
          dbs[v] = dn * kk * gm;
        } else {          // Dp = scale lower(dO W^T) . Gm
          const float d = p.scale * acc[v] * gm;
          sDp[i * LL + j] = (f16)d;
          x = d * sQK[i * LF + j];
          dbs[v] = 0.f;
        }
        xs[v] = x;
        csum += x;
      }
      const int ri = 16 * mt + 4 * q4 + l16;   // the row whose sums this lane holds (l16 < 4)
      if (wave < 4) {
        const float db = row16_sum4(dbs, l16);
        if (l16 < 4) sPB[(8 + nt) * C + ri] = db;
      }
      const float rs = row16_sum4(xs, l16);
      if (l16 < 4) sPG[((wave < 4 ? 0 : 2) + nt) * C + ri] = rs;
      csum += __shfl_xor(csum, 16, 64);
      csum += __shfl_xor(csum, 32, 64);
      if (q4 == 0) sPG[((wave < 4 ? 4 : 6) + mt) * C + j] = -csum;
    }
    lds_barrier();

    // ---- P4: dQ^ += Dp K^; dK^ += Dp^T Q^ + (Dm + Dm^T) K^; the L2 backward's row dots
    {
      const f16x8 bk = frag_col(sK, LR, 0, c0, lane), bq = frag_col(sQ, LR, 0, c0, lane);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        DQ[mt] = mfma16h(frag_h(sDp, LL, 16 * mt, 0, lane), bk, DQ[mt]);
        DK[mt] = mfma16h(frag_col(sDp, LL, 0, 16 * mt, lane), bq, DK[mt]);
        DK[mt] = mfma16h(frag_h(sDm, LL, 16 * mt, 0, lane), bk, DK[mt]);
        DK[mt] = mfma16h(frag_col(sDm, LL, 0, 16 * mt, lane), bk, DK[mt]);
      }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        f32x4 xq, xk;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          xq[v] = qh[mt][v] * DQ[mt][v];
          xk[v] = kh[mt][v] * DK[mt][v];
        }
        const float sq = row16_sum4(xq, l16), sk = row16_sum4(xk, l16);
        if (l16 < 4) {
          sPQ[wave * C + 16 * mt + 4 * q4 + l16] = sq;
          sPK[wave * C + 16 * mt + 4 * q4 + l16] = sk;
        }
      }
    }
    lds_barrier();

    // ---- P5: dq, dk (through the L2 normalisation); dg, dbeta --------------------
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      f32x4 sq = zero, sk = zero;
      if (p.l2norm) {
#pragma unroll
        for (int w = 0; w < 8; ++w) {
          sq += row4(sPQ + w * C, mt, q4);
          sk += row4(sPK + w * C, mt, q4);
        }
      }
      const f32x4 rq4 = row4(sRq, mt, q4), rk4 = row4(sRk, mt, q4);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = 16 * mt + 4 * q4 + v;
        float dq = DQ[mt][v], dk = DK[mt][v];
        if (p.l2norm) {
          dq = rq4[v] * (dq - qh[mt][v] * sq[v]);
          dk = rk4[v] * (dk - kh[mt][v] * sk[v]);
        }
        if (r < nval) {
          const int64_t o = ((int64_t)(tok0 + r) * H + h) * D + c0 + l16;
          p.dq[o] = (bf16)dq;
          p.dk[o] = (bf16)dk;
        }
      }
    }
    if (wave == 0) {
      float dgam = 0.f, db = 0.f, ctot = 0.f, dd = 0.f;
      if (lane < C) {
#pragma unroll
        for (int s = 0; s < NPG; ++s) dgam += sPG[s * C + lane];
#pragma unroll
        for (int s = 0; s < NPB; ++s) db += sPB[s * C + lane];
      }
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        dd += sPD[w];
        ctot += sPC[w];
      }
      if (lane == C - 1) dgam += sc.E[C - 1] * dd + ctot;
      // in-block reverse inclusive cumsum over lanes 0-31
#pragma unroll
      for (int off = 1; off < C; off <<= 1) {
        const float y = __shfl_down(dgam, off, 64);
        if (lane + off < C) dgam += y;
      }
      if (lane < nval) {
        const int64_t o = (int64_t)(tok0 + lane) * H + h;
        p.dg[o] = dgam;
        p.dbeta[o] = db;
      }
    }
    if (nxt >= total) break;
    it = nxt;
    cb = ncb;
    h = nh;
    tok0 = ntok0;
    nval = nnval;
  }
}

}  // namespace train
}  // namespace gdnp
}  // namespace hmx

extern "C" int hmx_gdn_train_fwd(const void* q, int64_t q_token_stride, const void* k,
                                 const void* v, int64_t kv_token_stride, const void* g,
                                 int32_t g_dtype, const void* beta, int32_t beta_dtype, void* o,
                                 const float* h0, float* ht, const int32_t* seg_table,
                                 int32_t nseg_total, int32_t N, int32_t H, float scale,
                                 int32_t use_qk_l2norm, int32_t max_warm_chunks,
                                 float decay_threshold, void* workspace, size_t workspace_bytes,
                                 void* block_states, const int32_t* cu_blocks, void* stream) {
  HMX_REQUIRE(block_states && cu_blocks && (uintptr_t)block_states % 16 == 0, HMX_EINVAL,
              "hmx_gdn_train_fwd: block_states (16-byte aligned) and cu_blocks are required");
  return chunk_fwd_impl(q, q_token_stride, k, kv_token_stride, v, kv_token_stride, HMX_BF16, g,
                        g_dtype, beta, beta_dtype, o, h0, ht, (int64_t)H * D * D, HMX_F32,
                        nullptr, nullptr, seg_table, nseg_total, N, H, H, D, D, scale,
                        use_qk_l2norm, max_warm_chunks, decay_threshold, workspace,
                        workspace_bytes, nullptr, nullptr, stream,
                        static_cast<f16*>(block_states), cu_blocks);
}

extern "C" size_t hmx_gdn_train_bwd_workspace_bytes(int32_t nblock_total,
                                                    int32_t nchain_segments, int32_t N,
                                                    int32_t H) {
  // dS per block (fp16 D x D), T and P per block (fp16 C x C each); per chain run
  // the plan entry; per run beyond a sequence's first, R, Psi and an exact start
  // (fp32 D x D each): nothing for sequences walked as one run
  const size_t extra = nchain_segments > N ? (size_t)(nchain_segments - N) : 0;
  return (size_t)nblock_total * H * ((size_t)D * D + 2 * C * C) * sizeof(f16) +
         (size_t)nchain_segments * H * sizeof(int) +
         extra * H * 3 * (size_t)D * D * sizeof(float) + 256;
}

extern "C" int hmx_gdn_train_bwd(const void* q, int64_t q_token_stride, const void* k,
                                 const void* v, int64_t kv_token_stride, const void* g,
                                 int32_t g_dtype, const void* beta, int32_t beta_dtype,
                                 const void* dout, int64_t dout_token_stride, const float* dht,
                                 const void* block_states, const int32_t* block_table,
                                 const int32_t* cu_blocks, int32_t nblock_total, int32_t N,
                                 const int32_t* chain_segments, int32_t nchain_segments,
                                 int32_t max_warm_blocks, float decay_threshold, int32_t H,
                                 float scale, int32_t use_qk_l2norm, void* dq, void* dk,
                                 void* dv, float* dg, float* dbeta, float* dh0, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  using namespace hmx::gdnp::train;
  HMX_REQUIRE(q && k && v && g && beta && dout && block_states && block_table && cu_blocks &&
                  chain_segments && dq && dk && dv && dg && dbeta,
              HMX_EINVAL, "hmx_gdn_train_bwd: null pointer");
  HMX_REQUIRE(N > 0 && H > 0 && nblock_total >= 0 && nchain_segments >= N && max_warm_blocks >= 0,
              HMX_EINVAL, "hmx_gdn_train_bwd: bad sizes (N=%d H=%d nblock=%d nseg=%d warm=%d)", N,
              H, nblock_total, nchain_segments, max_warm_blocks);
  HMX_REQUIRE(g_dtype >= 0 && g_dtype <= 2 && beta_dtype >= 0 && beta_dtype <= 2,
              HMX_EUNSUPPORTED, "hmx_gdn_train_bwd: g/beta dtype");
  HMX_REQUIRE(q_token_stride % 8 == 0 && kv_token_stride % 8 == 0 && dout_token_stride % 8 == 0 &&
                  ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)dout |
                   (uintptr_t)block_states) % 16 == 0,
              HMX_EINVAL, "hmx_gdn_train_bwd: rows must be 16-byte aligned");
  const size_t need = hmx_gdn_train_bwd_workspace_bytes(nblock_total, nchain_segments, N, H);
  HMX_REQUIRE(workspace && workspace_bytes >= need && (uintptr_t)workspace % 16 == 0, HMX_EINVAL,
              "hmx_gdn_train_bwd: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  Bwd p;
  p.q = static_cast<const bf16*>(q); p.k = static_cast<const bf16*>(k);
  p.v = static_cast<const bf16*>(v);
  p.q_ts = q_token_stride; p.kv_ts = kv_token_stride;
  p.g = g; p.g_dt = g_dtype; p.beta = beta; p.beta_dt = beta_dtype;
  p.dout = static_cast<const bf16*>(dout); p.do_ts = dout_token_stride;
  p.dht = dht;
  p.hc = static_cast<const f16*>(block_states);
  f16* ws = static_cast<f16*>(workspace);
  p.dhc = ws;
  p.tm = ws + (size_t)nblock_total * H * D * D;
  p.pm = p.tm + (size_t)nblock_total * H * C * C;
  {
    const size_t runs_hd = (size_t)(nchain_segments - N) * H * D * D;
    char* tail = reinterpret_cast<char*>(p.pm + (size_t)nblock_total * H * C * C);
    tail += (256 - reinterpret_cast<uintptr_t>(tail) % 256) % 256;
    p.cR = reinterpret_cast<float*>(tail);
    p.cPsi = p.cR + runs_hd;
    p.cstart = p.cPsi + runs_hd;
    p.cplan = reinterpret_cast<int*>(p.cstart + runs_hd);
  }
  p.ctab = block_table; p.cu_blk = cu_blocks;
  p.cseg = chain_segments; p.nseg = nchain_segments;
  p.max_warm = max_warm_blocks; p.decay_thresh = decay_threshold;
  p.dq = static_cast<bf16*>(dq); p.dk = static_cast<bf16*>(dk); p.dv = static_cast<bf16*>(dv);
  p.dg = dg; p.dbeta = dbeta; p.dh0 = dh0;
  p.H = H; p.nblk = nblock_total; p.scale = scale; p.l2norm = use_qk_l2norm;
  hipStream_t s = (hipStream_t)stream;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  const int64_t work = (int64_t)nblock_total * H;
  const int grad_grid = (int)std::min<int64_t>(work, (int64_t)cus);
  if (nblock_total > 0)
    hipLaunchKernelGGL(gdn_bwd_prep_kernel, dim3(nblock_total, H), dim3(BNTHR), 0, s, p);
  // where each chain run starts; for heads with an exact run, every run's R and
  // Psi, then their exact starts; then the chain walk
  hipLaunchKernelGGL(gdn_bwd_plan_kernel, dim3(nchain_segments, H), dim3(64), 0, s, p);
  hipLaunchKernelGGL(gdn_bwd_chain_kernel, dim3(nchain_segments, H, 2), dim3(BNTHR), 0, s, p,
                     (int)CH_R);
  hipLaunchKernelGGL(gdn_bwd_combine_kernel, dim3(N, H), dim3(BNTHR), 0, s, p);
  hipLaunchKernelGGL(gdn_bwd_chain_kernel, dim3(nchain_segments, H), dim3(BNTHR), 0, s, p,
                     (int)CH_WALK);
  if (nblock_total > 0)
    hipLaunchKernelGGL(gdn_bwd_grad_kernel, dim3(grad_grid), dim3(BNTHR), 0, s, p);
  return check_launch("hmx_gdn_train_bwd");
}
