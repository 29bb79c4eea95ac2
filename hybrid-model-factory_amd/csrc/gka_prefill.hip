// GKA (Gated KalmaNet) chunked prefill: per-token Chebyshev ridge solve against
// the running key Gram matrix H (h_kk), alpha blend, and beta^2-weighted gated
// linear attention over the value state S (h_kv); bf16 q/k/v, fp32 states.
//
// Semantics (per token t, head h; reference files under
// vllm-inference/src/primed_vllm/gka/):
//   q, k <- q/|q|, k/|k| (no eps)                          gka_forward.py:114-159
//   k~ = (beta+1e-6) k,  v~ = (beta+1e-6) v
//   H_t = e^{Gk_t} H_c + sum_{j<=t} e^{Gk_t-Gk_j} k~_j k~_j^T  chebyshev_prefill_gqa.py:28-106
//   f_t = |H_t|_F (closed form, :227-235); lam = r f; tau = 2/(2lam+f);
//   c = (f/(2lam+f)/2)^2; x = tau q; num_iter x { w <- 1/(1-cw);
//   x, x_prev <- w x - tau w (H_t x + lam x - q) - (w-1) x_prev, x }  :243-263
//   q <- q + alpha (x - q)                                  gka_forward.py:225
//   o_t = scale [e^{G_t} q^T S_c + sum_{j<=t} e^{G_t-G_j} (q.k~_j) v~_j]   ops/chunk_o_gqa.py:25-114
//   S <- e^{g} S + k~ v~^T,  H <- e^{gk} H + k~ k~^T        chunk_simple_gla_gqa.py:33-101
//
// Decomposition (the reference's split of the state recurrence from the solve,
// chebyshev_prefill_gqa.py:291-314).  The solve and the output of a token need
// only the states at its 64-token block's start; nothing they compute feeds the
// recurrences.  So:
//   * gka_walk_kernel: one workgroup per (segment, head) walks 32-token chunks
//     from a zero state with H and S in MFMA accumulators (wave w owns columns
//     [32w, 32w+32)), writing the zero-start states at every 64-token block start
//     (fp16) and the segment's end states (fp32).
//   * gka_combine_kernel: both recurrences have a scalar decay, so a segment's
//     true start state is the exact combine e^{D_s} X_s + dX_s of the segments
//     before it; it also reads and writes the caller's state pools.
//   * gka_solve_kernel: one workgroup per (64-token block, head), all blocks in
//     parallel: block-start states H_c = dH_b + e^{Gk(seg..b)} H_seg (same for S),
//     |H_t|_F in closed form, the Chebyshev iterations and the GLA output.  Wave w
//     owns the block's tokens [16w, 16w+16) and keeps its iterate transposed
//     (X^T, state dimension as rows) in C-layout registers, which is the B operand
//     layout of the next product: the iterations need no LDS exchange and no
//     barrier.
//
// Numerics.  MFMA operands are fp16 with fp32 accumulation: k~, v~, the block-start
// states (one rounding each).  The solve runs in direction form (x and the
// residual in fp32; only the step d enters the products): d is one fp16 rounding
// against H_c and an fp16 hi + lo pair against the in-block keys, as are the
// masked in-block products d.k~ and the blended query (the iterate is large off
// the key span, and a single rounding of it moves o by ~3e-2).  The walk keeps H
// and S in fp32 accumulators; its update operands are single fp16 roundings.
//
// Roofline: MFMA-bound at num_iter >= 8 (2*num_iter*(C*d^2 + 2*C^2*d) flops per
// block-head for the solver) plus the HBM minimum (q,k,v,o bf16 + gates +
// states) and the block-start states (2 * 32 KiB per 64-token block and head).
#include "common.hpp"
#include "mfma.hpp"

namespace hmx {
namespace gkap {

constexpr int D = 128;
constexpr int CB = 64;          // block: the solve's unit and the state-storage interval
constexpr int CW = 32;          // walk chunk
constexpr int NTHR = 256;       // 4 waves
// fp16 [rows][128] LDS row stride of the walk's tiles: 72 dwords = 8 mod 64 banks,
// so the transposing reads (ds_read_b64_tr_b16: 8 rows of 8 dwords per 32 lanes)
// are bank-conflict-free
constexpr int LDQ = D + 16;
constexpr float EPS = 1e-6f;

// Element (r, c) of a block-start state in its tile-major layout: 16x16 tiles,
// row-major within a tile and in tile order (the walk writes whole tiles; a row
// segment of 8 elements stays contiguous for the solve's 16-byte loads)
__device__ __forceinline__ int blk_index(int r, int c) {
  return ((r >> 4) * (D / 16) + (c >> 4)) * 256 + (r & 15) * 16 + (c & 15);
}

struct SegInfo { int n, bos, eos, c_start, c_end, seg_idx, first_seg, nseg; };

// A state pool: slots of [H, D, D] states, ss elements apart, f32 or bf16; `in`
// and `out` may be the same pool (read at the start, written at the end).
struct Pool {
  const void* in; void* out; int64_t ss; int dt;
};

struct Params {
  const bf16* q; const bf16* k; const bf16* v;
  int64_t q_ts, kv_ts;                    // token strides (elements; k and v share one)
  const void* alpha; int alpha_dt;
  const void* g; int g_dt;
  const void* gk; int gk_dt;              // null: no h_kk decay
  const void* beta; int beta_dt;          // null: no beta
  hmx_gate_proj gp; int fused;            // fused: the gates from the raw projections in gp
  bf16* o;
  // Sequence n's states: slot sidx[n] (or n) of the h_kk / h_kv pools; a negative
  // slot or hinit[n] == 0 starts from zero, and a negative slot writes nothing.
  // Only the combine launch reads and writes the pools.
  Pool hkk, hkv;
  const int* sidx;                        // [N] or null
  const uint8_t* hinit;                   // [N] or null
  const int* seg; int nseg_total; int nblk_total;
  int* segblk;                            // [nseg+1]: first global block of each segment
  f16* ws_hb; f16* ws_sb;                 // [nblk][H][D][D]: zero-start block-start H, S^T
                                          // (tile-major, see blk_index)
  float* ws_boff;                         // [nblk][H][2]: sum gk, sum g, segment start -> block
  float* ws_dh; float* ws_ds;             // [nseg][H][D][D]: zero-start end states H, S^T
  float* ws_dec;                          // [nseg][H][2]: sum gk, sum g over the segment
  f16* ws_h0; f16* ws_s0;                 // [nseg][H][D][D]: segment start states H, S^T
  int H, HKV, num_iter;
  float ridge_ratio, scale;
  int l2norm;                             // 0: q, k are used as given
  // optional gated RMSNorm of each output row (NORM kernels)
  const bf16* zg; int64_t zg_ts, zg_hs;   // gate rows, or null (plain RMSNorm)
  const void* onw; int onw_dt;            // weight [D]
  float on_eps;
  // the training solve (SM_X / SM_DQ / SM_GLA_SAVE solve kernels): |H_t|_F per token
  // [tokens][H] (written by SM_X and SM_GLA_SAVE, read by SM_DQ), the fp32 solution
  // of SM_DQ [tokens][H][D] (added to what it holds when xo32_acc), and the solution
  // x (before the alpha blend) saved by SM_GLA_SAVE [tokens][H][D] bf16
  float* fro; float* xo32; int xo32_acc; bf16* xs;
  const float* rhs32;                     // SM_DQ: an fp32 right-hand side in place of p.q
};

// The fused gates' raw projection values as bits (one load in either dtype
// branch), held in a float register and converted where the gates are formed: a
// conversion at the load would wait there for the rows loaded just before.
__device__ __forceinline__ uint32_t ld_bits(const void* p, int64_t i, int dt) {
  if (dt == HMX_F32) return static_cast<const uint32_t*>(p)[i];
  return static_cast<const uint16_t*>(p)[i];
}
__device__ __forceinline__ float bits_as_f(uint32_t b) { return __builtin_bit_cast(float, b); }
__device__ __forceinline__ float bits_f32(float held, int dt) {
  const uint32_t b = __builtin_bit_cast(uint32_t, held);
  if (dt == HMX_F32) return held;
  if (dt == HMX_BF16) return __builtin_bit_cast(float, b << 16);
  return (float)__builtin_bit_cast(f16, (uint16_t)b);
}
__device__ __forceinline__ float ldsc(const void* p, int64_t i, int dt) {
  if (dt == HMX_F32) return static_cast<const float*>(p)[i];
  if (dt == HMX_BF16) return (float)static_cast<const bf16*>(p)[i];
  return (float)static_cast<const f16*>(p)[i];
}

__device__ __forceinline__ SegInfo load_seg(const int* seg, int s) {
  const int* r = seg + s * 8;
  return SegInfo{r[0], r[1], r[2], r[3], r[4], r[5], r[6], r[7]};
}

// Sum of squares of an 8-feature slice over the 16 lanes of its DPP row.
__device__ __forceinline__ float row_sumsq(const bf16x8& x) {
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) s += (float)x[j] * (float)x[j];
  return row16_sum(s);
}

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ float scan64(float x) {
  const float lo = scan32(x);          // lanes 0-31 and 32-63 scanned separately
  const float carry = __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lo), 31));
  return (threadIdx.x & 63) >= 32 ? lo + carry : lo;
}

// Gate reads: the op's gate tensors, or (fused) the gates formed from the raw
// projections in gp.  Token tok is the op's flattened token index.
__device__ __forceinline__ bool has_beta(const Params& p) {
  return p.fused ? p.gp.b != nullptr : p.beta != nullptr;
}
__device__ __forceinline__ bool has_gk(const Params& p) {
  return p.fused ? p.gp.gk_from_g != 0 : p.gk != nullptr;
}
__device__ __forceinline__ float beta_at(const Params& p, int64_t tok, int h) {
  return p.fused ? gp_beta(p.gp, tok, h) : ldsc(p.beta, tok * p.H + h, p.beta_dt);
}
__device__ __forceinline__ float g_at(const Params& p, int64_t tok, int h) {
  return p.fused ? gp_g(p.gp, tok, h) : ldsc(p.g, tok * p.H + h, p.g_dt);
}
__device__ __forceinline__ float gk_at(const Params& p, int64_t tok, int h) {   // has_gk(p)
  return p.fused ? gp_g(p.gp, tok, h) : ldsc(p.gk, tok * p.H + h, p.gk_dt);
}
__device__ __forceinline__ float alpha_at(const Params& p, int64_t tok, int h) {
  return p.fused ? gp_alpha(p.gp, tok, h) : ldsc(p.alpha, tok * p.H + h, p.alpha_dt);
}

// The k~ scale of a row: (beta+1e-6) / |k| (or without the norm / without beta).
__device__ __forceinline__ float key_scale(const Params& p, float ss, int64_t tok, int h, bool ok) {
  if (!ok) return 0.f;
  const float be = has_beta(p) ? beta_at(p, tok, h) + EPS : 1.f;
  return p.l2norm ? be / sqrtf(ss) : be;
}

__device__ __forceinline__ float beta_eps(const Params& p, int64_t tok, int h, bool ok) {
  if (!ok) return 0.f;
  return has_beta(p) ? beta_at(p, tok, h) + EPS : 1.f;
}

__device__ __forceinline__ f16x8 scale_h8(const bf16x8& x, float s) {
  f16x8 y;
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = (f16)((float)x[j] * s);
  return y;
}

// ===========================================================================
// Pass A: the state walk
// ===========================================================================
namespace walk {
constexpr int SZ_T = CW * LDQ * 2;                 // one fp16 [32][LDQ] tile
constexpr int SZ_BUF = 3 * SZ_T + 2 * CW * 4;      // K~, K~ e^{GkL-Gk}, V~ e^{GL-G}; sum gk, sum g
constexpr int SMEM = 2 * SZ_BUF;
static_assert(SMEM <= 80 * 1024, "LDS budget");

struct Stage {
  f16* K; f16* KD; f16* VD; float* tot;   // tot[0] = chunk sum gk, tot[1] = chunk sum g
};
__device__ __forceinline__ Stage stage_at(unsigned char* smem, int bi) {
  unsigned char* b = smem + bi * SZ_BUF;
  return Stage{reinterpret_cast<f16*>(b), reinterpret_cast<f16*>(b + SZ_T),
               reinterpret_cast<f16*>(b + 2 * SZ_T), reinterpret_cast<float*>(b + 3 * SZ_T)};
}

struct Raw {
  bf16x8 k[2], v[2];
  float b[2];                 // beta of the thread's two rows
  float g, gk;                // gates of token `lane` (lanes 0-31 of every wave)
};

template <bool FG>
__device__ __forceinline__ void load_raw(Raw& r, const Params& p, const bf16* kh, const bf16* vh,
                                         int tok0, int nval, int tid, int h) {
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int row = pass * 16 + (tid >> 4), f0 = (tid & 15) * 8;
    const bool ok = row < nval;
    const int64_t tok = tok0 + row;
    r.k[pass] = ok ? *reinterpret_cast<const bf16x8*>(kh + tok * p.kv_ts + f0) : bf16x8{};
    r.v[pass] = ok ? *reinterpret_cast<const bf16x8*>(vh + tok * p.kv_ts + f0) : bf16x8{};
    // fused: b itself (the gate is formed at staging, so no load is waited for here)
    r.b[pass] = !(ok && has_beta(p)) ? 0.f
                : FG ? bits_as_f(ld_bits(p.gp.b, tok * p.gp.b_token_stride + h * p.gp.b_head_stride,
                                         p.gp.in_dtype))
                          : ldsc(p.beta, tok * p.H + h, p.beta_dt);
  }
  const int lane = tid & 63;
  const bool okg = lane < nval && lane < CW;
  const int64_t tk = tok0 + lane, gi = tk * p.H + h;
  if constexpr (FG) {     // a itself (fused: g and gk are formed at staging)
    r.g = (okg && p.gp.A_log)
              ? bits_as_f(ld_bits(p.gp.a, tk * p.gp.a_token_stride + h * p.gp.a_head_stride,
                                  p.gp.in_dtype))
              : 0.f;
    r.gk = 0.f;
  } else {
    r.g = (okg && p.g) ? ldsc(p.g, gi, p.g_dt) : 0.f;
    r.gk = (okg && p.gk) ? ldsc(p.gk, gi, p.gk_dt) : 0.f;
  }
}

// Stage one chunk: rows as the update uses them (fp16, k~ and v~ with the decay to
// the chunk end folded into the B-operand copies) and the chunk's gate sums.  Every
// wave forms the 32 in-chunk cumsums itself (lanes 0-31) and hands each staging
// lane its row's decay with a lane permute, so no LDS round trip is needed.
template <bool FG>
__device__ __forceinline__ void stage(const Stage& st, const Raw& r, const Params& p, int tid,
                                      int lane, int tok0, int nval, int h, bool track_h) {
  float gt = r.g, gkt = r.gk;
  if constexpr (FG) {     // the gates from the raw a (lanes of valid tokens)
    gt = (lane < nval && p.gp.A_log)
             ? gp_g_of(p.gp, bits_f32(r.g, p.gp.in_dtype), gate_exp(load_any(p.gp.A_log, h, p.gp.A_log_dtype)),
                       load_any(p.gp.dt_bias, h, p.gp.dt_bias_dtype))
             : 0.f;
    gkt = p.gp.gk_from_g ? gt : 0.f;
  }
  const float G = scan32(lane < CW ? gt : 0.f);
  const float Gk = scan32(lane < CW ? gkt : 0.f);
  const float GL = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, G), CW - 1));
  const float GkL = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, Gk), CW - 1));
  const float dl = fast_exp(GL - G), dlk = fast_exp(GkL - Gk);   // per token `lane`
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int row = pass * 16 + (tid >> 4), f0 = (tid & 15) * 8;
    const bool ok = row < nval;
    const float ss = row_sumsq(r.k[pass]);
    const float be = !ok ? 0.f
                     : !has_beta(p) ? 1.f
                     : (FG ? gp_beta_of(p.gp, bits_f32(r.b[pass], p.gp.in_dtype)) : r.b[pass]) + EPS;
    const float sk = !ok ? 0.f : (p.l2norm ? be / sqrtf(ss) : be);
    const float sv = be;
    const float drow = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(row << 2, __builtin_bit_cast(int, dl)));
    const float dkrow = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(row << 2, __builtin_bit_cast(int, dlk)));
    *reinterpret_cast<f16x8*>(st.K + row * LDQ + f0) = scale_h8(r.k[pass], sk);
    if (track_h) *reinterpret_cast<f16x8*>(st.KD + row * LDQ + f0) = scale_h8(r.k[pass], sk * dkrow);
    *reinterpret_cast<f16x8*>(st.VD + row * LDQ + f0) = scale_h8(r.v[pass], sv * drow);
  }
  if (tid == 0) {
    st.tot[0] = GkL;
    st.tot[1] = GL;
  }
}

template <bool TRACK_H, bool FG>
__global__ __launch_bounds__(NTHR, 2) void gka_walk_kernel(Params p) {
  __shared__ __align__(16) unsigned char smem[SMEM];
  const int tid = threadIdx.x, lane = tid & 63;
  // the wave index as a scalar: branches on it are uniform (an EXEC-masked region
  // would still run its MFMAs, which ignore EXEC)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, l16 = lane & 15;
  const int s_id = blockIdx.x, h = blockIdx.y, H = p.H;
  const SegInfo si = load_seg(p.seg, s_id);
  const int hk = h / (H / p.HKV);

  // this segment's first global block: the blocks of the segments before it
  __shared__ int red[NTHR / 64];
  {
    int cnt = 0;
    for (int s = tid; s < s_id; s += NTHR) {
      const int* r = p.seg + s * 8;
      cnt += r[4] - r[3];
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) cnt += __shfl_xor(cnt, m, 64);
    if (lane == 0) red[wave] = cnt;
  }
  __syncthreads();
  const int base = red[0] + red[1] + red[2] + red[3];
  if (h == 0 && tid == 0) {
    p.segblk[s_id] = base;
    if (s_id == p.nseg_total - 1) p.segblk[p.nseg_total] = base + si.c_end - si.c_start;
  }

  const int t_begin = si.bos + si.c_start * CB;
  const int t_end = min(si.eos, si.bos + si.c_end * CB);
  f32x4 Hs[8][2], Ss[8][2];
#pragma unroll
  for (int rt = 0; rt < 8; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      Hs[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
      Ss[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  float acc_gk = 0.f, acc_g = 0.f;        // decay sums from the segment start
  const bf16* kh = p.k + (int64_t)hk * D;
  const bf16* vh = p.v + (int64_t)hk * D;
  const int64_t DD = (int64_t)D * D;

  // the zero-start block-start states of block gb, transposed (H is symmetric) and
  // tile-major: a C-layout tile is 4 consecutive elements of one stored row per
  // lane, and the 64 lanes' 8-byte stores fill one contiguous 512-byte tile
  auto store_block = [&](int gb) {
    f16* hb = p.ws_hb + ((int64_t)gb * H + h) * DD;
    f16* sb = p.ws_sb + ((int64_t)gb * H + h) * DD;
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const int64_t off = blk_index(32 * wave + 16 * ct + l16, 16 * rt + 4 * q4);
        // H is symmetric: only its upper tiles (tile row <= tile column) are kept
        if (TRACK_H && 2 * wave + ct <= rt) *reinterpret_cast<f16x4*>(hb + off) = h4(Hs[rt][ct]);
        *reinterpret_cast<f16x4*>(sb + off) = h4(Ss[rt][ct]);
      }
    if (tid == 0) {
      p.ws_boff[((int64_t)gb * H + h) * 2 + 0] = acc_gk;
      p.ws_boff[((int64_t)gb * H + h) * 2 + 1] = acc_g;
    }
  };

  if (t_begin < t_end) {
    // rows are prefetched two chunks ahead: ra holds chunk t0 + CW, rb chunk t0 + 2 CW
    Raw ra, rb;
    load_raw<FG>(ra, p, kh, vh, t_begin, min(CW, t_end - t_begin), tid, h);
    stage<FG>(stage_at(smem, 0), ra, p, tid, lane, t_begin, min(CW, t_end - t_begin), h, TRACK_H);
    if (t_begin + CW < t_end)
      load_raw<FG>(ra, p, kh, vh, t_begin + CW, min(CW, t_end - t_begin - CW), tid, h);
    if (t_begin + 2 * CW < t_end)
      load_raw<FG>(rb, p, kh, vh, t_begin + 2 * CW, min(CW, t_end - t_begin - 2 * CW), tid, h);
    lds_barrier();
    int bi = 0;
    for (int t0 = t_begin; t0 < t_end; t0 += CW, bi ^= 1) {
      const Stage cur = stage_at(smem, bi);
      // stage the next chunk (its buffer was last read before the previous barrier)
      if (t0 + CW < t_end) {
        const int t1 = t0 + CW;
        stage<FG>(stage_at(smem, bi ^ 1), ra, p, tid, lane, t1, min(CW, t_end - t1), h, TRACK_H);
        ra = rb;
        if (t1 + 2 * CW < t_end)
          load_raw<FG>(rb, p, kh, vh, t1 + 2 * CW, min(CW, t_end - t1 - 2 * CW), tid, h);
      }
      // block start: the zero-start states so far (block 0 of a segment starts at zero)
      if (((t0 - t_begin) % CB) == 0) {
        const int gb = base + (t0 - t_begin) / CB;
        if (t0 > t_begin) store_block(gb);
        else if (tid == 0) {
          p.ws_boff[((int64_t)gb * H + h) * 2 + 0] = 0.f;
          p.ws_boff[((int64_t)gb * H + h) * 2 + 1] = 0.f;
        }
      }
      // S <- e^{GL} S + K~^T (e^{GL-G} V~);  H <- e^{GkL} H + K~^T (e^{GkL-Gk} K~)
      const float egl = fast_exp(cur.tot[1]), egkl = fast_exp(cur.tot[0]);
      acc_g += cur.tot[1];
      acc_gk += cur.tot[0];
#pragma unroll
      for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            Ss[rt][ct][v] *= egl;
            if (TRACK_H) Hs[rt][ct][v] *= egkl;
          }
      f16x8 bs[2], bh[2];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        bs[ct] = frag_t_perm_h(cur.VD, LDQ, 0, 32 * wave + 16 * ct, lane);
        if (TRACK_H) bh[ct] = frag_t_perm_h(cur.KD, LDQ, 0, 32 * wave + 16 * ct, lane);
      }
#pragma unroll
      for (int rt = 0; rt < 8; ++rt) {
        const f16x8 a = frag_t_perm_h(cur.K, LDQ, 0, 16 * rt, lane);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          Ss[rt][ct] = mfma16h(a, bs[ct], Ss[rt][ct]);
          if (TRACK_H) Hs[rt][ct] = mfma16h(a, bh[ct], Hs[rt][ct]);
        }
      }
      lds_barrier();
    }
  }

  // zero-start end states (H as is, S transposed) and the segment's decay sums
  float* hd = p.ws_dh + ((int64_t)s_id * H + h) * DD;
  float* sd = p.ws_ds + ((int64_t)s_id * H + h) * DD;
#pragma unroll
  for (int rt = 0; rt < 8; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int64_t off = (int64_t)(32 * wave + 16 * ct + l16) * D + 16 * rt + 4 * q4;
      if (TRACK_H) *reinterpret_cast<f32x4*>(hd + off) = Hs[rt][ct];
      *reinterpret_cast<f32x4*>(sd + off) = Ss[rt][ct];
    }
  if (tid == 0) {
    p.ws_dec[((int64_t)s_id * H + h) * 2 + 0] = acc_gk;
    p.ws_dec[((int64_t)s_id * H + h) * 2 + 1] = acc_g;
  }
}
}  // namespace walk

// ===========================================================================
// combine: segment start states and the final states (the only pool access)
// ===========================================================================
// One workgroup per (sequence, head, 32x32 tile of the state).  H is kept as is
// and S transposed in the workspace; the pools hold S as [K][V], so the S tile is
// read and written through an LDS transpose.
__global__ __launch_bounds__(256) void gka_combine_kernel(Params p, int track_h) {
  __shared__ float tile[32][33];
  const int nh = blockIdx.x, H = p.H;
  const int n = nh / H, h = nh % H;
  const int tr = blockIdx.y >> 2, tc = blockIdx.y & 3;      // tile row / column (of 4x4)
  const int tid = threadIdx.x;
  int first = -1, nseg = 0;
  for (int s = 0; s < p.nseg_total; ++s) {
    const SegInfo si = load_seg(p.seg, s);
    if (si.n == n) { first = si.first_seg; nseg = si.nseg; break; }
  }
  if (first < 0) return;
  const int64_t slot = p.sidx ? (int64_t)p.sidx[n] : n;
  const bool init = slot >= 0 && (!p.hinit || p.hinit[n]);
  const int64_t DD = (int64_t)D * D;
  const int64_t hoff = (int64_t)h * DD;
  // element (r, c) of this thread's 4 elements: r = 32 tr + (tid >> 3), c = 32 tc + 4 (tid & 7) + j
  const int r = 32 * tr + (tid >> 3), c0 = 32 * tc + 4 * (tid & 7);
  auto pool_f = [&](const Pool& pl, int64_t i) -> float {
    return pl.dt == HMX_BF16 ? (float)static_cast<const bf16*>(pl.in)[i]
                             : static_cast<const float*>(pl.in)[i];
  };
  auto pool_w = [&](const Pool& pl, int64_t i, float x) {
    if (pl.dt == HMX_BF16) static_cast<bf16*>(pl.out)[i] = (bf16)x;
    else static_cast<float*>(pl.out)[i] = x;
  };
  // h_kk: start states in the stored layout [r][c] (symmetric, no transpose)
  if (track_h) {
    float x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      x[j] = (init && p.hkk.in) ? pool_f(p.hkk, slot * p.hkk.ss + hoff + r * D + c0 + j) : 0.f;
    for (int s = 0; s < nseg; ++s) {
      const int64_t b = (int64_t)(first + s) * H + h;
      *reinterpret_cast<f16x4*>(p.ws_h0 + b * DD + r * D + c0) = f16x4{(f16)x[0], (f16)x[1], (f16)x[2], (f16)x[3]};
      const float dk = expf(p.ws_dec[b * 2 + 0]);
      const f32x4 e = *reinterpret_cast<const f32x4*>(p.ws_dh + b * DD + r * D + c0);
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = x[j] * dk + e[j];
    }
    if (slot >= 0 && p.hkk.out) {
#pragma unroll
      for (int j = 0; j < 4; ++j) pool_w(p.hkk, slot * p.hkk.ss + hoff + r * D + c0 + j, x[j]);
    }
  } else if (slot >= 0 && p.hkk.out && p.hinit && !p.hinit[n]) {
    // without the solver h_kk is not tracked: a pooled slot of a sequence without an
    // initial state is cleared, the others keep their value
#pragma unroll
    for (int j = 0; j < 4; ++j) pool_w(p.hkk, slot * p.hkk.ss + hoff + r * D + c0 + j, 0.f);
  }
  // h_kv: the workspace holds S^T; this thread owns S^T rows r (= S columns),
  // S^T columns c0..c0+3.  The pool tile is read / written transposed via LDS.
  {
    float x[4];
    // pool S[c][r] for c in this tile's columns: thread reads S[32 tr' ...] coalesced
    // as (row = 32 tc + (tid >> 3), cols 32 tr + 4 (tid & 7) + j), then transposes
    const int pr = 32 * tc + (tid >> 3), pc0 = 32 * tr + 4 * (tid & 7);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      tile[tid >> 3][4 * (tid & 7) + j] =
          (init && p.hkv.in) ? pool_f(p.hkv, slot * p.hkv.ss + hoff + pr * D + pc0 + j) : 0.f;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = tile[4 * (tid & 7) + j][tid >> 3];
    for (int s = 0; s < nseg; ++s) {
      const int64_t b = (int64_t)(first + s) * H + h;
      *reinterpret_cast<f16x4*>(p.ws_s0 + b * DD + r * D + c0) = f16x4{(f16)x[0], (f16)x[1], (f16)x[2], (f16)x[3]};
      const float dg = expf(p.ws_dec[b * 2 + 1]);
      const f32x4 e = *reinterpret_cast<const f32x4*>(p.ws_ds + b * DD + r * D + c0);
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = x[j] * dg + e[j];
    }
    if (slot >= 0 && p.hkv.out) {
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 4; ++j) tile[4 * (tid & 7) + j][tid >> 3] = x[j];
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 4; ++j)
        pool_w(p.hkv, slot * p.hkv.ss + hoff + pr * D + pc0 + j, tile[tid >> 3][4 * (tid & 7) + j]);
    }
  }
}

// ===========================================================================
// Pass B: the parallel solve and GLA output
// ===========================================================================
namespace solve {
// LDS rows of H_c / S_c, k~ and v~ are 72 dwords apart (8 mod 64 banks): 128-bit
// row-fragment reads (lane pairs q, q+1 of 8 rows share a cycle) and transposed
// ds_read_b64_tr_b16 reads of natural-order rows (8 rows of 8 dwords per 32 lanes)
// are then bank-conflict-free.  H_c, S_c and k~ keep their features in the
// interleaved order (icol), so each of their MFMA operands is one 128-bit read;
// v~ (read transposed only) keeps the natural order.
constexpr int LDP = D + 16;
constexpr int SZ_K = CB * LDP * 2;        // fp16 [64][LDP]
constexpr int SZ_H = D * LDP * 2;         // fp16 [128][LDP]
constexpr int OFF_K = 0;
constexpr int OFF_V = OFF_K + SZ_K;
constexpr int OFF_H = OFF_V + SZ_K;       // H_c, then S_c
constexpr int OFF_SC = OFF_H + SZ_H;
enum { SC_G, SC_GK, SC_AL, SC_D, SC_G2, SC_HN, NSC };
constexpr int OFF_NW = OFF_SC + NSC * CB * 4;
constexpr int SMEM = OFF_NW + D * 4;
static_assert(2 * SMEM <= 160 * 1024, "two workgroups per CU");

// hi/lo fp16 pair of a B operand built from two stacked C-layout tiles:
// hi = fp16 of x rounded toward zero (v_cvt_pkrtz, two per register), lo =
// fp16(x - hi), where x - hi is exact in fp32 and comes from v_fma_mix reading the
// packed hi halves directly.  hi + lo carries x to 2^-21 relative.  `one` is 1.0
// held in a register the compiler cannot see through, so that x*one - hi stays a
// fused multiply-add (which selects v_fma_mix) instead of being folded into a
// subtraction of a separately converted hi.
__device__ __forceinline__ float opaque_one() {
  float one;
  asm volatile("v_mov_b32 %0, 1.0" : "=v"(one));
  return one;
}
__device__ __forceinline__ void h8_hilo(const f32x4& t0, const f32x4& t1, f16x8& hi, f16x8& lo,
                                        float one) {
  typedef f16 f16x2 __attribute__((ext_vector_type(2)));
  const f16x2 h0 = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(t0[0], t0[1]));
  const f16x2 h1 = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(t0[2], t0[3]));
  const f16x2 h2 = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(t1[0], t1[1]));
  const f16x2 h3 = __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(t1[2], t1[3]));
  hi = f16x8{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
  lo = f16x8{(f16)__builtin_fmaf(t0[0], one, -(float)h0[0]), (f16)__builtin_fmaf(t0[1], one, -(float)h0[1]),
             (f16)__builtin_fmaf(t0[2], one, -(float)h1[0]), (f16)__builtin_fmaf(t0[3], one, -(float)h1[1]),
             (f16)__builtin_fmaf(t1[0], one, -(float)h2[0]), (f16)__builtin_fmaf(t1[1], one, -(float)h2[1]),
             (f16)__builtin_fmaf(t1[2], one, -(float)h3[0]), (f16)__builtin_fmaf(t1[3], one, -(float)h3[1])};
}

// A block-start state X = dX_b + e^{off} X_seg (both fp16; dX_b is zero for a
// segment's first block), this thread's 64 elements: row tid/2, half tid&1.
struct StateLd { f16x8 b[8], s[8]; };

// The loads of a block-start state (tile-major; null: zero) and of its segment's
// start state (rows; null: dropped), issued separately so the second can wait for
// the decay that decides whether it is needed.
// SYM (H): only the pieces in upper 16x16 tiles (tile row <= tile column) are
// loaded; state_fill_lower mirrors the rest in LDS.
template <bool SYM>
__device__ __forceinline__ bool piece_kept(int r, int c) {
  return !SYM || (r >> 4) <= (c >> 4);
}
template <bool SYM>
__device__ __forceinline__ void state_issue_b(StateLd& L, const f16* xb, int tid) {
  const int r = tid >> 1, c0 = (tid & 1) * 64;
  const f16* xbr = xb ? xb + blk_index(r, c0) : nullptr;   // 8-element pieces: fixed offsets
#pragma unroll
  for (int j = 0; j < 8; ++j)
    L.b[j] = (xbr && piece_kept<SYM>(r, c0 + 8 * j))
                 ? *reinterpret_cast<const f16x8*>(xbr + (j >> 1) * 256 + (j & 1) * 8)
                 : f16x8{};
}
template <bool SYM>
__device__ __forceinline__ void state_issue_s(StateLd& L, const f16* xs, int tid) {
  const int r = tid >> 1, c0 = (tid & 1) * 64;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    L.s[j] = (xs && piece_kept<SYM>(r, c0 + 8 * j))
                 ? *reinterpret_cast<const f16x8*>(xs + r * D + c0 + 8 * j)
                 : f16x8{};
}
// A segment's start state enters a block's state decayed by e^{off}; below e^-20
// (2e-9 of its norm, under fp32 rounding) it is dropped and not loaded.
constexpr float SEG_STATE_DROP = -20.f;

// Writes the state into LDS as fp16 rows; returns this thread's sum of squares.
// (SYM: of the upper tiles, each off-diagonal tile standing for itself and its
// mirror in the sum of squares.)
template <bool SYM>
__device__ __forceinline__ float state_store(f16* dst, const StateLd& L, float dec, int tid) {
  const int r = tid >> 1, c0 = (tid & 1) * 64;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int c = c0 + 8 * j;
    if (!piece_kept<SYM>(r, c)) continue;
    f16x8 y;
    float sj = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float u = (float)L.b[j][i] + dec * (float)L.s[j][i];
      sj += u * u;
      y[i] = (f16)u;
    }
    ss += (SYM && (r >> 4) != (c >> 4)) ? 2.f * sj : sj;
    store8_i(dst + r * LDP, c, y);
  }
  return ss;
}

// The lower 16x16 tiles of the symmetric H in LDS from their upper mirrors: a
// transposing read of 4 rows x 16 columns of tile (C, R) is 4 consecutive columns
// of one row of tile (R, C) per lane.  Wave w of nw fills lower tiles w, w+nw, ... (28).
__device__ __forceinline__ void state_fill_lower(f16* sH, int wave, int lane, int nw = 4) {
  const int q4 = lane >> 4, l16 = lane & 15;
  for (int k = wave; k < 28; k += nw) {
    int R = 1, m = k;                   // k-th lower tile (R, C), C < R, row-major
    while (m >= R) { m -= R; ++R; }
    const int C = m;
    const f16x4 x = ld_tr_i(sH, LDP, 16 * C + 4 * q4, 16 * R, lane);
    *reinterpret_cast<f16x4*>(sH + (16 * R + l16) * LDP + icol(16 * C + 4 * q4)) = x;
  }
}

// Runs f(WaveIdx<w>{}) for the workgroup's wave w.  Wave w's tokens are
// 16w..16w+15, so its causal key range is tiles 0..w; with w a compile-time
// constant the loops over that range are straight-line code.  Only the
// w-dependent stages go through this (the rest is shared, which keeps the kernel
// within the instruction cache).
template <int N> struct WaveIdx { static constexpr int value = N; };
template <typename F>
__device__ __forceinline__ void with_wave(int wave, F&& f) {
  switch (wave) {
    case 0: f(WaveIdx<0>{}); break;
    case 1: f(WaveIdx<1>{}); break;
    case 2: f(WaveIdx<2>{}); break;
    default: f(WaveIdx<3>{}); break;
  }
}

// What the solve kernel produces: the GLA output (serving prefill), or the solution
// x of the Chebyshev solve itself (training): SM_X writes x (bf16, into p.o) and
// |H_t|_F; SM_DQ solves for the right-hand side in p.q with the |H_t|_F of the
// forward read back (the backward's dq) and writes fp32 (p.xo32); SM_GLA_SAVE is
// the GLA output that also saves x (p.xs) and |H_t|_F for the training backward.
enum SolveMode { SM_GLA = 0, SM_X = 1, SM_DQ = 2, SM_GLA_SAVE = 3 };

template <bool SOLVE, bool NORM, int MODE = SM_GLA>
__global__ __launch_bounds__(NTHR, 2) void gka_solve_kernel(Params p) {
  static_assert(MODE == SM_GLA || (SOLVE && !NORM), "the x outputs need the solver");
  constexpr bool GLA = MODE == SM_GLA || MODE == SM_GLA_SAVE;
  __shared__ __align__(16) unsigned char smem[SMEM];
  f16* sK = reinterpret_cast<f16*>(smem + OFF_K);
  f16* sV = reinterpret_cast<f16*>(smem + OFF_V);
  f16* sH = reinterpret_cast<f16*>(smem + OFF_H);
  float* sc = reinterpret_cast<float*>(smem + OFF_SC);
  auto SC = [&](int slot, int t) -> float& { return sc[slot * CB + t]; };
  const int tid = threadIdx.x, lane = tid & 63;
  // the wave index as a scalar: branches on it are uniform
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const float one = opaque_one();
  const int q4 = lane >> 4, l16 = lane & 15;
  const int gb = blockIdx.x, h = blockIdx.y, H = p.H;
  const int hk = h / (H / p.HKV);
  const int64_t DD = (int64_t)D * D;

  // ---- which segment / block -------------------------------------------------
  int lo = 0, hi = p.nseg_total;        // last s with segblk[s] <= gb
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (p.segblk[mid] <= gb) lo = mid; else hi = mid;
  }
  const int s_id = lo;
  const SegInfo si = load_seg(p.seg, s_id);
  const int lb = gb - p.segblk[s_id];                 // block index within the segment
  const int tok0 = si.bos + (si.c_start + lb) * CB;
  const int nval = min(CB, si.eos - tok0);
  if (nval <= 0) return;

  // block-start decay offsets (segment start -> this block); the state loads go
  // out first so their latency overlaps the staging below
  const int64_t bo = ((int64_t)gb * H + h) * 2;
  const int64_t so = ((int64_t)s_id * H + h) * DD;
  const int64_t bso = ((int64_t)gb * H + h) * DD;
  StateLd hst;
  if constexpr (SOLVE) state_issue_b<true>(hst, lb > 0 ? p.ws_hb + bso : nullptr, tid);
  const float off_gk = p.ws_boff[bo + 0], off_g = p.ws_boff[bo + 1];
  if constexpr (SOLVE)
    state_issue_s<true>(hst, (lb == 0 || off_gk > SEG_STATE_DROP) ? p.ws_h0 + so : nullptr, tid);

  // ---- stage k~, v~ (fp16), gates; q rows into registers --------------------
#pragma unroll
  for (int pass = 0; pass < CB / 16; ++pass) {
    const int row = pass * 16 + (tid >> 4), f0 = (tid & 15) * 8;
    const bool ok = row < nval;
    const int64_t tok = tok0 + row;
    const bf16x8 kr = ok ? *reinterpret_cast<const bf16x8*>(p.k + tok * p.kv_ts + hk * D + f0) : bf16x8{};
    const bf16x8 vr = ok ? *reinterpret_cast<const bf16x8*>(p.v + tok * p.kv_ts + hk * D + f0) : bf16x8{};
    const float sk = key_scale(p, row_sumsq(kr), tok, h, ok);
    store8_i(sK + row * LDP, f0, scale_h8(kr, sk));
    if constexpr (GLA)
      *reinterpret_cast<f16x8*>(sV + row * LDP + f0) = scale_h8(vr, beta_eps(p, tok, h, ok));
  }
  if (wave == 0) {
    const bool ok = lane < nval;
    const int64_t tk = tok0 + lane;
    const float gt = (GLA && ok) ? g_at(p, tk, h) : 0.f;
    const float G = scan64(gt);
    const float Gk = scan64((ok && has_gk(p)) ? (p.fused ? gt : gk_at(p, tk, h)) : 0.f);
    SC(SC_G, lane) = G;
    SC(SC_GK, lane) = Gk;
    SC(SC_AL, lane) = (GLA && ok) ? alpha_at(p, tk, h) : 0.f;
  }
  if (NORM && tid < D) {
    float wv;
    if (p.onw_dt == HMX_F32) wv = static_cast<const float*>(p.onw)[tid];
    else if (p.onw_dt == HMX_BF16) wv = (float)static_cast<const bf16*>(p.onw)[tid];
    else wv = (float)static_cast<const f16*>(p.onw)[tid];
    reinterpret_cast<float*>(smem + OFF_NW)[tid] = wv;
  }
  float* red = sc + SC_HN * CB;           // 4 partial sums
  if constexpr (SOLVE) {
    const float ss = wave_sum(state_store<true>(sH, hst, fast_exp(off_gk), tid));
    if (lane == 0) red[wave] = ss;
  }
  // this lane's token t (16 per wave) and its q^ slice: Q[nt][v] = q^[t][16 nt + 4 q4 + v]
  const int tb = 16 * wave + l16;
  const bool tok_ok = tb < nval;
  f32x4 Q[8];
  const bf16* qr = p.q + (int64_t)(tok0 + tb) * p.q_ts + (int64_t)h * D + 4 * q4;
  float rq;
  {
    float ss = 0.f;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      if (MODE == SM_DQ && p.rhs32) {
        Q[nt] = tok_ok ? *reinterpret_cast<const f32x4*>(p.rhs32 + ((int64_t)(tok0 + tb) * H + h) * D +
                                                         4 * q4 + 16 * nt)
                       : f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
        const bf16x4 x = tok_ok ? *reinterpret_cast<const bf16x4*>(qr + 16 * nt) : bf16x4{};
#pragma unroll
        for (int v = 0; v < 4; ++v) Q[nt][v] = (float)x[v];
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) ss += Q[nt][v] * Q[nt][v];
    }
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    rq = (!tok_ok) ? 0.f : (p.l2norm ? 1.0f / sqrtf(ss) : 1.f);
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) Q[nt][v] *= rq;
  }

  f32x4 X[8];                             // the query fed to the GLA, transposed C layout
  if constexpr (SOLVE) {
    lds_barrier();
    state_fill_lower(sH, wave, lane);
    lds_barrier();
    const float hn = red[0] + red[1] + red[2] + red[3];   // |H_c|^2
    const float GkT = SC(SC_GK, tb);

    // d_j = k~_j^T H_c k~_j for this wave's tokens j = 16 wave + l16
    if constexpr (MODE != SM_DQ) {
      f32x4 Pd[8];
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) Pd[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const f16x8 b = frag_i(sK, LDP, 16 * wave, 32 * ks, lane);
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) Pd[nt] = mfma16h(frag_i(sH, LDP, 16 * nt, 32 * ks, lane), b, Pd[nt]);
      }
      float d = 0.f;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        const f16x4 kk = *reinterpret_cast<const f16x4*>(sK + tb * LDP + icol(16 * nt + 4 * q4));
#pragma unroll
        for (int v = 0; v < 4; ++v) d += Pd[nt][v] * (float)kk[v];
      }
      d += __shfl_xor(d, 16, 64);
      d += __shfl_xor(d, 32, 64);
      if (q4 == 0) SC(SC_D, tb) = d;
    }
    // Gram part of |H_t|^2: g2_t = sum_{i,j<=t} a_ti a_tj (k~_i.k~_j)^2, a_tj = e^{Gk_t-Gk_j},
    // as the row sums of a . (A B) with B = (K K^T)^2 over this wave's key range
    if constexpr (MODE != SM_DQ) with_wave(wave, [&](auto Wc) {
      constexpr int W = decltype(Wc)::value;
      f32x4 U[4];
#pragma unroll
      for (int I = 0; I < 4; ++I) U[I] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        if (J > W) break;
        // a[t = tb][j = 16J + 4q4 + v]
        f16x4 aJ;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int j = 16 * J + 4 * q4 + v;
          aJ[v] = (f16)(j <= tb ? fast_exp(GkT - SC(SC_GK, j)) : 0.f);
        }
#pragma unroll
        for (int I = 0; I < 4; ++I) {
          if (I > W) break;
          f32x4 kk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks)
            kk = mfma16h(frag_i(sK, LDP, 16 * J, 32 * ks, lane), frag_i(sK, LDP, 16 * I, 32 * ks, lane), kk);
          f32x4 sq;
#pragma unroll
          for (int v = 0; v < 4; ++v) sq[v] = kk[v] * kk[v];
          U[I] = mfma16h_k16(aJ, h4(sq), U[I]);
        }
      }
      // U[I][v]: row t = 16 wave + 4 q4 + v, column i = 16 I + l16
      float g2[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        if (I > W) break;
        const int i = 16 * I + l16;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int t = 16 * W + 4 * q4 + v;
          g2[v] += (i <= t) ? U[I][v] * fast_exp(SC(SC_GK, t) - SC(SC_GK, i)) : 0.f;
        }
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float s = row16_sum(g2[v]);
        if (l16 == 0) SC(SC_G2, 16 * W + 4 * q4 + v) = s;
      }
    });
    lds_barrier();
    // f_t, lam, tau, c for this lane's token
    float tau, lam, cc;
    {
      float f;
      if constexpr (MODE == SM_DQ) {
        f = tok_ok ? p.fro[(int64_t)(tok0 + tb) * H + h] : 0.f;
      } else {
        float cross = 0.f;
        for (int j = q4; j <= tb; j += 4) cross += fast_exp(GkT - SC(SC_GK, j)) * SC(SC_D, j);
        cross += __shfl_xor(cross, 16, 64);
        cross += __shfl_xor(cross, 32, 64);
        const float e = fast_exp(GkT);
        f = sqrtf(fmaxf(e * e * hn + 2.f * e * cross + SC(SC_G2, tb), 0.f));
        if ((MODE == SM_X || MODE == SM_GLA_SAVE) && tok_ok && q4 == 0)
          p.fro[(int64_t)(tok0 + tb) * H + h] = f;
      }
      lam = p.ridge_ratio * f;
      const float inv = 1.0f / (2.f * lam + f);
      tau = 2.f * inv;
      const float c = f * inv * 0.5f;
      cc = c * c;
      if (!tok_ok) { tau = 0.f; lam = 0.f; cc = 0.f; }
    }

    // ---- the Chebyshev iterations ------------------------------------------
    // In direction form: with rho_k = q - A x_k (A = H_t + lam I) and d_k = x_{k+1} - x_k,
    //   x_0 = tau q, d_{-1} = tau q, rho_0 = q - A d_{-1};  per step (w as the reference
    //   updates it): d_k = w tau rho_k + (w - 1) d_{k-1}, x_{k+1} = x_k + d_k,
    //   rho_{k+1} = rho_k - A d_k
    // - the reference's x_{k+1} = w x_k - tau w (A x_k - q) - (w-1) x_{k-1} exactly.
    // x and rho stay in fp32; only d enters the products.  d and rho carry no
    // 1/lam growth (x does, off the key span), so the history part e^{Gk_t} H_c d
    // takes d as one fp16 rounding; the in-block part K~^T (M . K~ d), which carries
    // the early tokens, keeps the hi + lo pairs.  (A CPU emulation of both orders of
    // rounding against the fp64 recurrence gives the same output error as hi + lo
    // for every product.)
    {
    f32x4 R[8], Dd[8];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        Dd[nt][v] = tau * Q[nt][v];
        X[nt][v] = Dd[nt][v];
        R[nt][v] = Q[nt][v];
      }
    // minus the in-block decays -m_tj = -e^{Gk_t-Gk_j} (j <= t, else 0) of the four key tiles
    f32x4 mz[4];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      const f32x4 gkj = *reinterpret_cast<const f32x4*>(&SC(SC_GK, 16 * jt + 4 * q4));
#pragma unroll
      for (int v = 0; v < 4; ++v)
        mz[jt][v] = (16 * jt + 4 * q4 + v <= tb) ? -fast_exp(GkT - gkj[v]) : 0.f;
    }
    const float egk = fast_exp(GkT);
    // R <- R - A d: R - lam d - e^{Gk_t} H_c d first, then the in-block part
    // accumulates on top through -Z~ (eight 16-row tiles in two groups of four, four
    // independent accumulation chains)
    auto apply = [&]() {
      f16x8 dh[4], dl[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) h8_hilo(Dd[2 * ks], Dd[2 * ks + 1], dh[ks], dl[ks], one);
      // -Z~^T[j][t] = -m_tj (k~_j . d_t), hi/lo B operands over all four key tiles (the
      // keys past this wave's tokens get m = 0; one uniform instruction stream)
      f16x8 zh[2], zl[2];
      {
        f32x4 Z[4];
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) Z[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          f16x8 a[4];
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) a[jt] = frag_i(sK, LDP, 16 * jt, 32 * ks, lane);
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) Z[jt] = mfma16h(a[jt], dh[ks], Z[jt]);
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) Z[jt] = mfma16h(a[jt], dl[ks], Z[jt]);
        }
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
          for (int v = 0; v < 4; ++v) Z[jt][v] *= mz[jt][v];
#pragma unroll
        for (int jk = 0; jk < 2; ++jk) h8_hilo(Z[2 * jk], Z[2 * jk + 1], zh[jk], zl[jk], one);
      }
#pragma unroll
      for (int g4 = 0; g4 < 8; g4 += 4) {
        f32x4 hx[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) hx[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          f16x8 a[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) a[u] = frag_i(sH, LDP, 16 * (g4 + u), 32 * ks, lane);
#pragma unroll
          for (int u = 0; u < 4; ++u) hx[u] = mfma16h(a[u], dh[ks], hx[u]);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            hx[u][v] = R[g4 + u][v] - lam * Dd[g4 + u][v] - egk * hx[u][v];
#pragma unroll
        for (int jk = 0; jk < 2; ++jk) {
          f16x8 a[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) a[u] = frag_t_i(sK, LDP, 32 * jk, 16 * (g4 + u), lane);
#pragma unroll
          for (int u = 0; u < 4; ++u) hx[u] = mfma16h(a[u], zh[jk], hx[u]);
#pragma unroll
          for (int u = 0; u < 4; ++u) hx[u] = mfma16h(a[u], zl[jk], hx[u]);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) R[g4 + u] = hx[u];
        // bound the scheduler's hoisting of LDS operands to one group of tiles
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    if (p.num_iter > 0) apply();
    // w <= 2 since c <= 1/4, so the hardware reciprocal suffices
    float om = 2.f;
    for (int it = 0; it < p.num_iter; ++it) {
      om = __builtin_amdgcn_rcpf(1.0f - cc * om);
      const float wt = om * tau, wm = om - 1.0f;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          Dd[nt][v] = wt * R[nt][v] + wm * Dd[nt][v];
          X[nt][v] += Dd[nt][v];
        }
      if (it + 1 < p.num_iter) apply();
    }
    }
    if constexpr (MODE != SM_GLA) {
      // the solution of this lane's token: X[nt][v] = x[16 nt + 4 q4 + v]
      if (tok_ok) {
        const int64_t ro = ((int64_t)(tok0 + tb) * H + h) * D + 4 * q4;
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
          if constexpr (MODE == SM_X || MODE == SM_GLA_SAVE) {
            bf16x4 y;
#pragma unroll
            for (int v = 0; v < 4; ++v) y[v] = (bf16)X[nt][v];
            *reinterpret_cast<bf16x4*>((MODE == SM_X ? p.o : p.xs) + ro + 16 * nt) = y;
          } else {
            f32x4 y = X[nt];
            if (p.xo32_acc) {
              const f32x4 o0 = *reinterpret_cast<const f32x4*>(p.xo32 + ro + 16 * nt);
#pragma unroll
              for (int v = 0; v < 4; ++v) y[v] += o0[v];
            }
            *reinterpret_cast<f32x4*>(p.xo32 + ro + 16 * nt) = y;
          }
        }
      }
      if constexpr (!GLA) return;
    }
    // alpha blend (q read again: the iterations keep x, d and rho in registers)
    const float al = SC(SC_AL, tb);
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const bf16x4 xq = tok_ok ? *reinterpret_cast<const bf16x4*>(qr + 16 * nt) : bf16x4{};
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float qv = (float)xq[v] * rq;
        X[nt][v] = qv + al * (X[nt][v] - qv);
      }
    }
    lds_barrier();      // every wave is done with H_c
  } else {
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) X[nt] = Q[nt];
  }

  // ---- GLA output: o^T = scale [e^{G_t} S_c^T x^ + V~^T Z'^T] ---------------
  // The S_c loads go out first; the in-block products (they need only k~) run while
  // they arrive.
  StateLd sst;
  state_issue_b<false>(sst, lb > 0 ? p.ws_sb + bso : nullptr, tid);
  state_issue_s<false>(sst, (lb == 0 || off_g > SEG_STATE_DROP) ? p.ws_s0 + so : nullptr, tid);
  if constexpr (!SOLVE) lds_barrier();     // the staged k~, v~ and gates
  f32x4 O[8];
  {
    f16x8 xh[4], xl[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) h8_hilo(X[2 * ks], X[2 * ks + 1], xh[ks], xl[ks], one);
    const float GT = SC(SC_G, tb), eg = fast_exp(GT);
    // Z'^T[j][t] = e^{G_t-G_j} (k~_j . x^_t), j <= t
    f16x8 zb0, zb1 = {};
    with_wave(wave, [&](auto Wc) {
      constexpr int W = decltype(Wc)::value;
      f32x4 Z[4];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) Z[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        f16x8 a[W + 1];
#pragma unroll
        for (int jt = 0; jt <= W; ++jt) a[jt] = frag_i(sK, LDP, 16 * jt, 32 * ks, lane);
#pragma unroll
        for (int jt = 0; jt <= W; ++jt) Z[jt] = mfma16h(a[jt], xh[ks], Z[jt]);
#pragma unroll
        for (int jt = 0; jt <= W; ++jt) Z[jt] = mfma16h(a[jt], xl[ks], Z[jt]);
      }
#pragma unroll
      for (int jt = 0; jt <= W; ++jt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int j = 16 * jt + 4 * q4 + v;
          Z[jt][v] = (j <= tb) ? Z[jt][v] * fast_exp(GT - SC(SC_G, j)) : 0.f;
        }
      zb0 = h8(Z[0], Z[1]);
      if constexpr (W >= 2) zb1 = h8(Z[2], Z[3]);
    });
    // S_c into LDS (every wave is past its last read of H_c)
    state_store<false>(sH, sst, fast_exp(off_g), tid);
    lds_barrier();
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) O[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        const f16x8 a = frag_i(sH, LDP, 16 * nt, 32 * ks, lane);
        O[nt] = mfma16h(a, xh[ks], O[nt]);
        O[nt] = mfma16h(a, xl[ks], O[nt]);
      }
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) O[nt][v] *= eg;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      O[nt] = mfma16h(frag_t_perm_h(sV, LDP, 0, 16 * nt, lane), zb0, O[nt]);
      if (wave >= 2) O[nt] = mfma16h(frag_t_perm_h(sV, LDP, 32, 16 * nt, lane), zb1, O[nt]);
    }
  }

  // ---- store (NORM: out = o / sqrt(mean(o^2) + eps) * w * silu(z) per token) ---
  if (tok_ok) {
    bf16* orow = p.o + (int64_t)(tok0 + tb) * H * D + (int64_t)h * D + 4 * q4;
    float rstd = 1.f;
    if constexpr (NORM) {
      float ss = 0.f;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float y = (float)(bf16)(O[nt][v] * p.scale);   // o as rounded to bf16
          O[nt][v] = y;
          ss += y * y;
        }
      ss += __shfl_xor(ss, 16, 64);
      ss += __shfl_xor(ss, 32, 64);
      rstd = 1.0f / sqrtf(ss * (1.0f / D) + p.on_eps);
    }
    const bf16* zr = (NORM && p.zg) ? p.zg + (int64_t)(tok0 + tb) * p.zg_ts + (int64_t)h * p.zg_hs + 4 * q4
                                    : nullptr;
    const float* sNW = reinterpret_cast<const float*>(smem + OFF_NW);
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      bf16x4 out;
      if constexpr (NORM) {
        bf16x4 z = {};
        if (zr) z = *reinterpret_cast<const bf16x4*>(zr + 16 * nt);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float y = O[nt][v] * rstd * sNW[16 * nt + 4 * q4 + v];
          if (zr) {
            const float zz = (float)z[v];
            y *= zz * __builtin_amdgcn_rcpf(1.0f + fast_exp(-zz));
          }
          out[v] = (bf16)y;
        }
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) out[v] = (bf16)(O[nt][v] * p.scale);
      }
      *reinterpret_cast<bf16x4*>(orow + 16 * nt) = out;
    }
  }
}

}  // namespace solve

}  // namespace gkap
}  // namespace hmx

using namespace hmx;
using namespace hmx::gkap;

// Workspace carve-up (256-byte aligned pieces), in this order: block states (H, S^T
// fp16), segment states (dH, dS^T, H0, S0^T fp32), block offsets, segment decays,
// the segment -> block prefix.
namespace {
struct WsLayout { size_t hb, sb, dh, ds, h0, s0, boff, dec, segblk, total; };
size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }
WsLayout ws_layout(int32_t nseg, int32_t nblk, int32_t H) {
  WsLayout w;
  const size_t blk_st = (size_t)nblk * H * D * D * sizeof(f16);
  const size_t seg_st = (size_t)nseg * H * D * D * sizeof(float);
  const size_t seg_h = (size_t)nseg * H * D * D * sizeof(f16);
  size_t o = 0;
  w.hb = o; o = al256(o + blk_st);
  w.sb = o; o = al256(o + blk_st);
  w.dh = o; o = al256(o + seg_st);
  w.ds = o; o = al256(o + seg_st);
  w.h0 = o; o = al256(o + seg_h);
  w.s0 = o; o = al256(o + seg_h);
  w.boff = o; o = al256(o + (size_t)nblk * H * 2 * sizeof(float));
  w.dec = o; o = al256(o + (size_t)nseg * H * 2 * sizeof(float));
  w.segblk = o; o = al256(o + (size_t)(nseg + 1) * sizeof(int));
  w.total = o;
  return w;
}
}  // namespace

extern "C" size_t hmx_gka_chunk_workspace_bytes(int32_t nseg_total, int32_t nblock_total,
                                                int32_t N, int32_t H) {
  (void)N;
  return ws_layout(nseg_total, nblock_total, H).total;
}

extern "C" int hmx_gka_chunk_fwd(const void* q, int64_t q_token_stride, const void* k,
                                 int64_t k_token_stride, const void* v, int64_t v_token_stride,
                                 int32_t qkv_dtype, const void* alpha, int32_t alpha_dtype,
                                 const void* g, int32_t g_dtype, const void* gk, int32_t gk_dtype,
                                 const void* beta, int32_t beta_dtype, void* o,
                                 const void* h_kk0, void* h_kk_final, int64_t h_kk_slot_stride,
                                 int32_t h_kk_dtype, const void* h_kv0, void* h_kv_final,
                                 int64_t h_kv_slot_stride, int32_t h_kv_dtype,
                                 const int32_t* state_indices, const uint8_t* has_initial_state,
                                 const int32_t* seg_table, int32_t nseg_total,
                                 int32_t nblock_total, int32_t N, int32_t H, int32_t HKV,
                                 int32_t D_, int32_t V, int32_t num_iter, float ridge_ratio,
                                 float scale, int32_t use_qk_l2norm, void* workspace,
                                 size_t workspace_bytes, const hmx_gated_norm* o_norm,
                                 const hmx_gate_proj* gates, void* stream) {
  HMX_REQUIRE(qkv_dtype == HMX_BF16, HMX_EUNSUPPORTED,
              "hmx_gka_chunk_fwd: q/k/v must be bfloat16 (got dtype code %d)", qkv_dtype);
  if (gates) {
    const int rc = check_gates(gates, true, "hmx_gka_chunk_fwd");
    if (rc != HMX_OK) return rc;
  }
  HMX_REQUIRE(D_ == D && V == D, HMX_EUNSUPPORTED,
              "hmx_gka_chunk_fwd: only D == V == 128 is supported (got D=%d V=%d)", D_, V);
  HMX_REQUIRE(H > 0 && HKV > 0 && H % HKV == 0, HMX_EINVAL, "hmx_gka_chunk_fwd: H/HKV");
  HMX_REQUIRE(q && k && v && (gates || (alpha && g)) && o && seg_table, HMX_EINVAL,
              "hmx_gka_chunk_fwd: null tensor pointer");
  HMX_REQUIRE(num_iter >= 0, HMX_EINVAL, "hmx_gka_chunk_fwd: num_iter=%d", num_iter);
  HMX_REQUIRE(nseg_total >= 0 && nblock_total >= 0, HMX_EINVAL,
              "hmx_gka_chunk_fwd: nseg_total=%d nblock_total=%d", nseg_total, nblock_total);
  HMX_REQUIRE(q_token_stride % 8 == 0 && k_token_stride % 8 == 0 && v_token_stride % 8 == 0 &&
                  ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)o) % 16 == 0,
              HMX_EINVAL, "hmx_gka_chunk_fwd: q/k/v/o rows must be 16-byte aligned");
  HMX_REQUIRE(k_token_stride == v_token_stride, HMX_EINVAL,
              "hmx_gka_chunk_fwd: k and v must share a token stride (%lld vs %lld)",
              (long long)k_token_stride, (long long)v_token_stride);
  HMX_REQUIRE((h_kk_dtype == HMX_F32 || h_kk_dtype == HMX_BF16) &&
                  (h_kv_dtype == HMX_F32 || h_kv_dtype == HMX_BF16),
              HMX_EUNSUPPORTED, "hmx_gka_chunk_fwd: state dtypes must be f32 or bf16");
  if (nseg_total == 0) return HMX_OK;
  const WsLayout wl = ws_layout(nseg_total, nblock_total, H);
  HMX_REQUIRE(workspace && workspace_bytes >= wl.total, HMX_EINVAL,
              "hmx_gka_chunk_fwd: workspace of %zu bytes needed, %zu given", wl.total,
              workspace_bytes);
  Params p;
  p.q = static_cast<const bf16*>(q); p.k = static_cast<const bf16*>(k);
  p.v = static_cast<const bf16*>(v);
  p.alpha = alpha; p.alpha_dt = alpha_dtype; p.g = g; p.g_dt = g_dtype;
  p.gk = gk; p.gk_dt = gk_dtype; p.beta = beta; p.beta_dt = beta_dtype;
  p.fused = gates != nullptr;
  p.gp = gates ? *gates : hmx_gate_proj{};
  p.zg = nullptr; p.zg_ts = p.zg_hs = 0; p.onw = nullptr; p.onw_dt = HMX_F32; p.on_eps = 0.f;
  if (o_norm) {
    HMX_REQUIRE(o_norm->weight && o_norm->weight_dtype >= 0 && o_norm->weight_dtype <= 2,
                HMX_EINVAL, "hmx_gka_chunk_fwd: o_norm needs a weight (dtype code 0-2)");
    HMX_REQUIRE(!o_norm->gate || ((uintptr_t)o_norm->gate % 8 == 0 &&
                                  o_norm->gate_token_stride % 4 == 0 &&
                                  o_norm->gate_head_stride % 4 == 0),
                HMX_EINVAL, "hmx_gka_chunk_fwd: o_norm gate rows must be 8-byte aligned");
    p.zg = static_cast<const bf16*>(o_norm->gate);
    p.zg_ts = o_norm->gate_token_stride; p.zg_hs = o_norm->gate_head_stride;
    p.onw = o_norm->weight; p.onw_dt = o_norm->weight_dtype; p.on_eps = o_norm->eps;
  }
  p.o = static_cast<bf16*>(o);
  p.q_ts = q_token_stride; p.kv_ts = k_token_stride;
  p.hkk = Pool{h_kk0, h_kk_final, h_kk_slot_stride, h_kk_dtype};
  p.hkv = Pool{h_kv0, h_kv_final, h_kv_slot_stride, h_kv_dtype};
  p.sidx = state_indices; p.hinit = has_initial_state;
  p.seg = seg_table; p.nseg_total = nseg_total; p.nblk_total = nblock_total;
  p.H = H; p.HKV = HKV; p.num_iter = num_iter; p.ridge_ratio = ridge_ratio; p.scale = scale;
  p.l2norm = use_qk_l2norm;
  char* ws = static_cast<char*>(workspace);
  p.ws_hb = reinterpret_cast<f16*>(ws + wl.hb);
  p.ws_sb = reinterpret_cast<f16*>(ws + wl.sb);
  p.ws_dh = reinterpret_cast<float*>(ws + wl.dh);
  p.ws_ds = reinterpret_cast<float*>(ws + wl.ds);
  p.ws_h0 = reinterpret_cast<f16*>(ws + wl.h0);
  p.ws_s0 = reinterpret_cast<f16*>(ws + wl.s0);
  p.ws_boff = reinterpret_cast<float*>(ws + wl.boff);
  p.ws_dec = reinterpret_cast<float*>(ws + wl.dec);
  p.segblk = reinterpret_cast<int*>(ws + wl.segblk);
  const bool solve_ = num_iter > 0;
  hipStream_t s = (hipStream_t)stream;
  const dim3 wgrid(nseg_total, H);
  if (solve_ && p.fused) hipLaunchKernelGGL((walk::gka_walk_kernel<true, true>), wgrid, dim3(NTHR), 0, s, p);
  else if (solve_) hipLaunchKernelGGL((walk::gka_walk_kernel<true, false>), wgrid, dim3(NTHR), 0, s, p);
  else if (p.fused) hipLaunchKernelGGL((walk::gka_walk_kernel<false, true>), wgrid, dim3(NTHR), 0, s, p);
  else hipLaunchKernelGGL((walk::gka_walk_kernel<false, false>), wgrid, dim3(NTHR), 0, s, p);
  hipLaunchKernelGGL(gka_combine_kernel, dim3(N * H, 16), dim3(256), 0, s, p, (int)solve_);
  if (nblock_total > 0) {
    const dim3 grid(nblock_total, H);
    if (solve_ && o_norm) hipLaunchKernelGGL((solve::gka_solve_kernel<true, true>), grid, dim3(NTHR), 0, s, p);
    else if (solve_) hipLaunchKernelGGL((solve::gka_solve_kernel<true, false>), grid, dim3(NTHR), 0, s, p);
    else if (o_norm) hipLaunchKernelGGL((solve::gka_solve_kernel<false, true>), grid, dim3(NTHR), 0, s, p);
    else hipLaunchKernelGGL((solve::gka_solve_kernel<false, false>), grid, dim3(NTHR), 0, s, p);
  }
  return check_launch("hmx_gka_chunk_fwd");
}

// ===========================================================================
// The training backward of the Chebyshev solve: dk and dgk
// ===========================================================================
// With x treated as the exact solution, dL/dH_t = G_t = -dq_t x_t^T + a_t H_t, where
// a_t = -r (dq_t . x_t) / |H_t|_F carries the ridge's dependence on |H_t|_F (0
// without bp_lambda).  Per 64-token block c with in-block decays g_t (inclusive
// cumsum of gk from the block start), block total Gam = g at the last token, and
// block-start state h_c (H_t = e^{g_t} h_c + sum_{s<=t} e^{g_t-g_s} k_s k_s^T):
//   E_c = sum_t e^{g_t} (G_t + G_t^T)   (the block's share of dL/dh_c, symmetrised;
//         stored bf16, the reverse scan accumulating in fp32)
//   Dn_c = sum over later blocks, decayed to block c's end: Dn_c = E_{c+1} + e^{Gam_{c+1}} Dn_{c+1}
//   dk_s = -sum_{t>=s} e^{g_t-g_s} [dq_t (x_t.k_s) + x_t (dq_t.k_s)]
//          + 2 beta_s h_c k_s + 2 sum_u W_su (k_u.k_s) k_u + e^{Gam-g_s} Dn k_s
//   with rho_m = sum_{t>=m} a_t e^{2(g_t-g_m)}, beta_s = e^{g_s} rho_s,
//   W_su = e^{(g_m-g_s)+(g_m-g_u)} rho_m (m = max(s,u));
//   dL/dg_t = <G_t, H_t> - sum_{t'>=t} e^{g_t'-g_t} <G_t', k_t k_t^T> - e^{Gam-g_t} k_t^T Dn k_t / 2
//             (+ <Dn, h_{c+1}> / 2 at the block's last token),
//   and dgk is its in-block reverse cumsum (the derivative through the chunk-local
//   cumsum of gk).  These are the terms of chunk_dk_backward_gating.py's two passes
//   and chunk_bwd_dh (chebyshev_iteration.py:646-688), in this kernel's arrangement.
namespace hmx {
namespace gkap {
namespace train {
using solve::LDP;
using solve::SZ_K;
using solve::SZ_H;
using solve::StateLd;

struct Bwd {
  const bf16* x;          // [tokens][H][D] the forward's solution
  const float* dq;        // [tokens][H][D] the backward's solve of dx
  const float* fro;       // [tokens][H]
  bf16* e;                // [nblk][H][D][D] bf16 tile-major: E_c, then Dn_c
  float* gam;             // [nblk][H] block totals of gk
  bf16* dk;               // [tokens][H][D] the gradient of k (+ dk_add when given)
  const float* dk_add;    // null, or [tokens][H][D] fp32 added to dk
  bf16* dq_out;           // [tokens][H][D] the gradient of the right-hand side (+ dq_add)
  const float* dq_add;    // null, or [tokens][H][D] fp32 added to dq_out
  float* dgk;             // [tokens][H]
  int bp_lambda;
};

struct Blk { int s_id, lb, tok0, nval; };
__device__ __forceinline__ Blk block_of(const Params& p, int gb) {
  int lo = 0, hi = p.nseg_total;         // last s with segblk[s] <= gb
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (p.segblk[mid] <= gb) lo = mid; else hi = mid;
  }
  const SegInfo si = load_seg(p.seg, lo);
  const int lb = gb - p.segblk[lo];
  const int tok0 = si.bos + (si.c_start + lb) * CB;
  return Blk{lo, lb, tok0, min(CB, si.eos - tok0)};
}

// h_c of block gb into sH (fp16, interleaved rows, both triangles), as the solve
// forms it; the first 256 threads load, all nw waves mirror
__device__ __forceinline__ void load_hc(const Params& p, f16* sH, const Blk& b, int gb, int h,
                                        int tid, int wave, int lane, int nw = 4) {
  if (tid < NTHR) {
    const int64_t DD = (int64_t)D * D;
    const int64_t so = ((int64_t)b.s_id * p.H + h) * DD;
    const int64_t bso = ((int64_t)gb * p.H + h) * DD;
    StateLd hst;
    solve::state_issue_b<true>(hst, b.lb > 0 ? p.ws_hb + bso : nullptr, tid);
    const float off_gk = p.ws_boff[((int64_t)gb * p.H + h) * 2];
    solve::state_issue_s<true>(hst, (b.lb == 0 || off_gk > solve::SEG_STATE_DROP) ? p.ws_h0 + so : nullptr, tid);
    solve::state_store<true>(sH, hst, fast_exp(off_gk), tid);
  }
  lds_barrier();
  solve::state_fill_lower(sH, wave, lane, nw);
}

// in-block inclusive cumsum of gk for lanes 0-63 (wave 0); 0 past the block's tokens
__device__ __forceinline__ float block_decay(const Params& p, const Blk& b, int h, int lane) {
  const bool ok = lane < b.nval;
  return scan64((ok && p.gk) ? ldsc(p.gk, (int64_t)(b.tok0 + lane) * p.H + h, p.gk_dt) : 0.f);
}

// a_t = -r (dq_t . x_t) / |H_t|_F for token row `row` from the row's staged
// pieces (features 8 l16 .. 8 l16 + 7 in each lane of its 16-lane group)
__device__ __forceinline__ float lambda_weight(const Params& p, const Bwd& w, const Blk& b, int row,
                                               int h, const f32x4& q0, const f32x4& q1,
                                               const bf16x8& xv) {
  float d = 0.f;
#pragma unroll
  for (int v = 0; v < 4; ++v) d += q0[v] * (float)xv[v] + q1[v] * (float)xv[4 + v];
  d = row16_sum(d);
  const float f = (row < b.nval && w.bp_lambda) ? w.fro[(int64_t)(b.tok0 + row) * p.H + h] : 0.f;
  return f > 0.f ? -p.ridge_ratio * d / f : 0.f;
}

// x, dq and the ridge weights grow like 1 / |H_t|_F, which is small at a
// sequence's start: the fp16 operands built from them are scaled by a power of two
// (exact) chosen from their largest magnitude, and the products unscaled in fp32.
// pow2_scale(m): 2^j with m 2^j < 2^8 (1 when m is below that already)
__device__ __forceinline__ float pow2_scale(float m) {
  int e;
  (void)frexpf(m, &e);                   // m < 2^e
  return e > 8 ? ldexpf(1.f, 8 - e) : 1.f;
}
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m, 64));
  return x;
}
__device__ __forceinline__ float absmax8(const bf16x8& x) {
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf((float)x[j]));
  return m;
}
__device__ __forceinline__ float absmax4(const f32x4& x) {
  return fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
}
// The workgroup's maxima of NV per-thread values over NW waves: slot[NV * NW] of
// LDS scratch; includes a barrier.
template <int NV, int NW = 4>
__device__ __forceinline__ void block_max(float (&v)[NV], float* slot, int wave, int lane) {
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    v[i] = wave_max(v[i]);
    if (lane == 0) slot[NW * i + wave] = v[i];
  }
  lds_barrier();
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    float m = slot[NW * i];
#pragma unroll
    for (int j = 1; j < NW; ++j) m = fmaxf(m, slot[NW * i + j]);
    v[i] = m;
  }
}
__device__ __forceinline__ bf16x4 bf4(const f32x4& x) {
  return bf16x4{(bf16)x[0], (bf16)x[1], (bf16)x[2], (bf16)x[3]};
}
__device__ __forceinline__ f32x4 f4(const bf16x4& x) {
  return f32x4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]};
}
__device__ __forceinline__ f16x8 h8_of(const f32x4& a, const f32x4& b, float s) {
  return f16x8{(f16)(s * a[0]), (f16)(s * a[1]), (f16)(s * a[2]), (f16)(s * a[3]),
               (f16)(s * b[0]), (f16)(s * b[1]), (f16)(s * b[2]), (f16)(s * b[3])};
}

constexpr int E_OFF_K = 0, E_OFF_KB = SZ_K, E_OFF_Q = 2 * SZ_K, E_OFF_X = 3 * SZ_K;
constexpr int E_OFF_H = 4 * SZ_K, E_OFF_SC = E_OFF_H + SZ_H;
constexpr int E_SMEM = E_OFF_SC + 3 * CB * 4 + 32 * 4;
constexpr int E_NTHR = 512;             // 8 waves: wave w forms tile row w of E_c
static_assert(E_SMEM <= 160 * 1024, "LDS budget");

// E_c = -(Ql^T X + X^T Ql) + 2 (alpha h_c + K^T diag(beta) K), Ql = e^{g} dq, of block gb
__global__ __launch_bounds__(E_NTHR, 1) void cheb_e_kernel(Params p, Bwd w) {
  __shared__ __align__(16) unsigned char smem[E_SMEM];
  f16* sK = reinterpret_cast<f16*>(smem + E_OFF_K);
  f16* sKb = reinterpret_cast<f16*>(smem + E_OFF_KB);
  f16* sQ = reinterpret_cast<f16*>(smem + E_OFF_Q);
  f16* sX = reinterpret_cast<f16*>(smem + E_OFF_X);
  f16* sH = reinterpret_cast<f16*>(smem + E_OFF_H);
  float* sG = reinterpret_cast<float*>(smem + E_OFF_SC);     // g_t
  float* sA = sG + CB;                                        // a_t
  float* sB = sA + CB;                                        // 2 beta_t, then [CB-1 + 1] unused
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, l16 = lane & 15;
  const int gb = blockIdx.x, h = blockIdx.y, H = p.H;
  const Blk b = block_of(p, gb);
  if (b.nval <= 0) return;
  constexpr int NP = CB * 16 / E_NTHR;     // staging passes of 32 rows

  load_hc(p, sH, b, gb, h, tid, wave, lane, E_NTHR / 64);
  if (wave == 0) {
    const float g = block_decay(p, b, h, lane);
    sG[lane] = g;
    if (lane == b.nval - 1) w.gam[(int64_t)gb * H + h] = g;
  }
  // the rows, and a_t from them
  bf16x8 kr[NP], xr[NP];
  f32x4 q0[NP], q1[NP];
#pragma unroll
  for (int pass = 0; pass < NP; ++pass) {
    const int row = pass * 32 + (tid >> 4), f0 = (tid & 15) * 8;
    const bool ok = row < b.nval;
    const int64_t ro = ((int64_t)(b.tok0 + row) * H + h) * D + f0;
    kr[pass] = ok ? *reinterpret_cast<const bf16x8*>(p.k + (int64_t)(b.tok0 + row) * p.kv_ts + h * D + f0) : bf16x8{};
    xr[pass] = ok ? *reinterpret_cast<const bf16x8*>(w.x + ro) : bf16x8{};
    q0[pass] = ok ? *reinterpret_cast<const f32x4*>(w.dq + ro) : f32x4{0.f, 0.f, 0.f, 0.f};
    q1[pass] = ok ? *reinterpret_cast<const f32x4*>(w.dq + ro + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
    const float a = lambda_weight(p, w, b, row, h, q0[pass], q1[pass], xr[pass]);
    if (l16 == 0) sA[row] = a;
  }
  lds_barrier();
  // rho_t = sum_{t'>=t} a_t' e^{2(g_t'-g_t)} (lane t of wave 0), beta_t = e^{g_t} rho_t
  float alpha = 0.f;
  if (wave == 0) {
    float rho = 0.f;
    const float gt = sG[lane];
    for (int t2 = lane; t2 < b.nval; ++t2) rho += sA[t2] * fast_exp(2.f * (sG[t2] - gt));
    sB[lane] = lane < b.nval ? 2.f * fast_exp(gt) * rho : 0.f;
    alpha = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                          __builtin_bit_cast(int, fast_exp(2.f * gt) * rho), 0));
  }
  __shared__ float s_alpha;
  if (tid == 0) s_alpha = alpha;
  lds_barrier();
  // stage k, 2 beta k, -e^{g} dq, x (fp16, interleaved; the last three scaled)
  float mx[3] = {0.f, 0.f, 0.f};            // max |x|, |e^g dq|, |2 beta k|
#pragma unroll
  for (int pass = 0; pass < NP; ++pass) {
    const int row = pass * 32 + (tid >> 4);
    const float eg = row < b.nval ? -fast_exp(sG[row]) : 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      q0[pass][v] *= eg;
      q1[pass][v] *= eg;
    }
    mx[0] = fmaxf(mx[0], absmax8(xr[pass]));
    mx[1] = fmaxf(mx[1], fmaxf(absmax4(q0[pass]), absmax4(q1[pass])));
    mx[2] = fmaxf(mx[2], fabsf(sB[row]) * absmax8(kr[pass]));
  }
  block_max<3, E_NTHR / 64>(mx, reinterpret_cast<float*>(smem + E_OFF_SC + 3 * CB * 4), wave, lane);
  const float sx = pow2_scale(mx[0]), sq = pow2_scale(mx[1]), sb = pow2_scale(mx[2]);
#pragma unroll
  for (int pass = 0; pass < NP; ++pass) {
    const int row = pass * 32 + (tid >> 4), f0 = (tid & 15) * 8;
    store8_i(sK + row * LDP, f0, scale_h8(kr[pass], 1.f));
    store8_i(sKb + row * LDP, f0, scale_h8(kr[pass], sb * sB[row]));
    store8_i(sX + row * LDP, f0, scale_h8(xr[pass], sx));
    store8_i(sQ + row * LDP, f0, h8_of(q0[pass], q1[pass], sq));
  }
  lds_barrier();
  const float a2 = 2.f * s_alpha;
  const float u12 = 1.f / (sx * sq), u3 = 1.f / sb;
  // wave w: tile row w (state rows 16w..16w+15), all 8 tile columns
  bf16* eo = w.e + ((int64_t)gb * H + h) * D * D;
  {
    const int it = wave;
    f32x4 E[8], E3[8];
#pragma unroll
    for (int jt = 0; jt < 8; ++jt) {
      E[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
      E3[jt] = E[jt];
    }
#pragma unroll
    for (int jk = 0; jk < 2; ++jk) {
      const f16x8 aq = frag_t_i(sQ, LDP, 32 * jk, 16 * it, lane);
      const f16x8 ax = frag_t_i(sX, LDP, 32 * jk, 16 * it, lane);
      const f16x8 ab = frag_t_i(sKb, LDP, 32 * jk, 16 * it, lane);
#pragma unroll
      for (int jt = 0; jt < 8; ++jt) {
        E[jt] = mfma16h(aq, frag_t_i(sX, LDP, 32 * jk, 16 * jt, lane), E[jt]);
        E[jt] = mfma16h(ax, frag_t_i(sQ, LDP, 32 * jk, 16 * jt, lane), E[jt]);
        E3[jt] = mfma16h(ab, frag_t_i(sK, LDP, 32 * jk, 16 * jt, lane), E3[jt]);
      }
    }
    // E[jt][v] = E_c[16 it + 4 q4 + v][16 jt + l16]; E_c is symmetric, so the lane
    // writes it as row 16 jt + l16, columns 16 it + 4 q4 .. +3 of the tile-major store
#pragma unroll
    for (int jt = 0; jt < 8; ++jt) {
      const f16x4 hc = *reinterpret_cast<const f16x4*>(sH + (16 * jt + l16) * LDP + icol(16 * it + 4 * q4));
      f32x4 y;
#pragma unroll
      for (int v = 0; v < 4; ++v) y[v] = u12 * E[jt][v] + u3 * E3[jt][v] + a2 * (float)hc[v];
      *reinterpret_cast<bf16x4*>(eo + blk_index(16 * jt + l16, 16 * it + 4 * q4)) = bf4(y);
    }
  }
}

// Dn_c = sum over the later blocks of the sequence: one workgroup per (sequence,
// head, 1024 elements), the sequence's blocks in reverse.  E_c is replaced by Dn_c.
__global__ __launch_bounds__(256) void cheb_dscan_kernel(Params p, Bwd w) {
  const int nh = blockIdx.x, H = p.H;
  const int n = nh / H, h = nh % H;
  int first = -1, nseg = 0;
  for (int s = 0; s < p.nseg_total; ++s) {
    const SegInfo si = load_seg(p.seg, s);
    if (si.n == n) { first = si.first_seg; nseg = si.nseg; break; }
  }
  if (first < 0) return;
  const int b0 = p.segblk[first], b1 = p.segblk[first + nseg];
  const int64_t DD = (int64_t)D * D;
  const int64_t el = (int64_t)blockIdx.y * 1024 + 4 * threadIdx.x;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int c = b1 - 1; c >= b0; --c) {
    bf16* ec = w.e + ((int64_t)c * H + h) * DD + el;
    const f32x4 e = f4(*reinterpret_cast<const bf16x4*>(ec));
    const float dg = fast_exp(w.gam[(int64_t)c * H + h]);
    *reinterpret_cast<bf16x4*>(ec) = bf4(acc);
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[v] = e[v] + dg * acc[v];
  }
}

constexpr int C_OFF_K = 0, C_OFF_X = SZ_K, C_OFF_Q = 2 * SZ_K, C_OFF_H = 3 * SZ_K;
constexpr int C_OFF_DN = C_OFF_H + SZ_H, C_OFF_SC = C_OFF_DN + SZ_H;
enum { CS_G, CS_A, CS_RHO, CS_DG, CS_COL0, NCS = CS_COL0 + 4 };
// 8 waves: wave w takes the 16 columns s of group w & 3 and the feature half w >> 2
constexpr int C_NTHR = 512;
constexpr int C_OFF_RED = C_OFF_SC + NCS * CB * 4;        // 16 floats of cross-wave sums
constexpr int C_OFF_MS = C_OFF_RED + 16 * 4;              // 24 floats for block_max
constexpr int C_OFF_XCH = C_OFF_MS + 24 * 4;              // [2][64][4] feature-half dot products
constexpr int C_SMEM = C_OFF_XCH + 2 * CB * 4 * 4;
static_assert(C_SMEM <= 160 * 1024, "LDS budget");

// dk and dgk of block gb (see the section comment)
__global__ __launch_bounds__(C_NTHR, 1) void cheb_dk_kernel(Params p, Bwd w) {
  __shared__ __align__(16) unsigned char smem[C_SMEM];
  f16* sK = reinterpret_cast<f16*>(smem + C_OFF_K);
  f16* sX = reinterpret_cast<f16*>(smem + C_OFF_X);
  f16* sQ = reinterpret_cast<f16*>(smem + C_OFF_Q);
  f16* sH = reinterpret_cast<f16*>(smem + C_OFF_H);
  f16* sDn = reinterpret_cast<f16*>(smem + C_OFF_DN);
  float* sc = reinterpret_cast<float*>(smem + C_OFF_SC);
  float* red = reinterpret_cast<float*>(smem + C_OFF_RED);
  float* mslot = reinterpret_cast<float*>(smem + C_OFF_MS);
  float* xch = reinterpret_cast<float*>(smem + C_OFF_XCH);
  auto SC = [&](int slot, int t) -> float& { return sc[slot * CB + t]; };
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cg = wave & 3, fh = wave >> 2;   // column group, feature half (nt 4 fh .. 4 fh + 3)
  const int q4 = lane >> 4, l16 = lane & 15;
  const int gb = blockIdx.x, h = blockIdx.y, H = p.H;
  const Blk b = block_of(p, gb);
  if (b.nval <= 0) return;
  const int64_t DD = (int64_t)D * D;
  constexpr int NP = CB * 16 / C_NTHR;     // staging passes of 32 rows

  load_hc(p, sH, b, gb, h, tid, wave, lane, C_NTHR / 64);
  if (wave == 0) SC(CS_G, lane) = block_decay(p, b, h, lane);
  // the rows (x, dq and Dn scaled into fp16's range) and a_t
  bf16x8 kr[NP], xr[NP];
  f32x4 q0[NP], q1[NP];
  const bf16* dn = w.e + ((int64_t)gb * H + h) * DD;
  const int dr = tid >> 2, dc0 = (tid & 3) * 32;    // this thread's Dn: row dr, columns dc0..+31
  f32x4 u[8];
  float mx[3] = {0.f, 0.f, 0.f};            // max |x|, |dq|, |Dn|
#pragma unroll
  for (int pass = 0; pass < NP; ++pass) {
    const int row = pass * 32 + (tid >> 4), f0 = (tid & 15) * 8;
    const bool ok = row < b.nval;
    const int64_t ro = ((int64_t)(b.tok0 + row) * H + h) * D + f0;
    kr[pass] = ok ? *reinterpret_cast<const bf16x8*>(p.k + (int64_t)(b.tok0 + row) * p.kv_ts + h * D + f0) : bf16x8{};
    xr[pass] = ok ? *reinterpret_cast<const bf16x8*>(w.x + ro) : bf16x8{};
    q0[pass] = ok ? *reinterpret_cast<const f32x4*>(w.dq + ro) : f32x4{0.f, 0.f, 0.f, 0.f};
    q1[pass] = ok ? *reinterpret_cast<const f32x4*>(w.dq + ro + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
    mx[0] = fmaxf(mx[0], absmax8(xr[pass]));
    mx[1] = fmaxf(mx[1], fmaxf(absmax4(q0[pass]), absmax4(q1[pass])));
    const float a = lambda_weight(p, w, b, row, h, q0[pass], q1[pass], xr[pass]);
    if (l16 == 0) SC(CS_A, row) = a;
    if (ok) {                             // the caller's dq: this solve's (+ dq_add), bf16
      f32x4 y0 = q0[pass], y1 = q1[pass];
      if (w.dq_add) {
        const f32x4 o0 = *reinterpret_cast<const f32x4*>(w.dq_add + ro);
        const f32x4 o1 = *reinterpret_cast<const f32x4*>(w.dq_add + ro + 4);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          y0[v] += o0[v];
          y1[v] += o1[v];
        }
      }
      *reinterpret_cast<bf16x8*>(w.dq_out + ro) =
          bf16x8{(bf16)y0[0], (bf16)y0[1], (bf16)y0[2], (bf16)y0[3],
                 (bf16)y1[0], (bf16)y1[1], (bf16)y1[2], (bf16)y1[3]};
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    u[j] = f4(*reinterpret_cast<const bf16x4*>(dn + blk_index(dr, dc0 + 4 * j)));
    mx[2] = fmaxf(mx[2], absmax4(u[j]));
  }
  block_max<3, C_NTHR / 64>(mx, mslot, wave, lane);   // (its barrier also orders h_c's lower tiles)
  const float sx = pow2_scale(mx[0]), sq = pow2_scale(mx[1]), sd = pow2_scale(mx[2]);
#pragma unroll
  for (int pass = 0; pass < NP; ++pass) {
    const int row = pass * 32 + (tid >> 4), f0 = (tid & 15) * 8;
    store8_i(sK + row * LDP, f0, scale_h8(kr[pass], 1.f));
    store8_i(sX + row * LDP, f0, scale_h8(xr[pass], sx));
    store8_i(sQ + row * LDP, f0, h8_of(q0[pass], q1[pass], sq));
  }
  // Dn into LDS and <Dn, h_c> in fp32
  float dnh = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = dc0 + 8 * j;
    const f16x4 h0 = *reinterpret_cast<const f16x4*>(sH + dr * LDP + icol(c));
    const f16x4 h1 = *reinterpret_cast<const f16x4*>(sH + dr * LDP + icol(c + 4));
#pragma unroll
    for (int v = 0; v < 4; ++v) dnh += u[2 * j][v] * (float)h0[v] + u[2 * j + 1][v] * (float)h1[v];
    store8_i(sDn + dr * LDP, c, h8_of(u[2 * j], u[2 * j + 1], sd));
  }
  dnh = wave_sum(dnh);
  // rho_t (lane t of wave 0)
  if (wave == 0) {
    float rho = 0.f;
    const float gt = SC(CS_G, lane);
    for (int t2 = lane; t2 < b.nval; ++t2) rho += SC(CS_A, t2) * fast_exp(2.f * (SC(CS_G, t2) - gt));
    SC(CS_RHO, lane) = rho;
  }
  if (lane == 0) red[wave] = dnh;
  lds_barrier();

  const int s = 16 * cg + l16;              // this lane's key / token column
  const bool s_ok = s < b.nval;
  const float gs = SC(CS_G, s);
  const float Gam = SC(CS_G, b.nval - 1);
  // products with h_c and Dn over this wave's feature half: HK = h_c k_s, HX = h_c x_s,
  // P = Dn k_s (rows f = 16 (4 fh + i) + 4 q4 + v, column s)
  f32x4 HK[4], HX[4], P[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    HK[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    HX[i] = HK[i];
    P[i] = HK[i];
  }
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const f16x8 bk = frag_i(sK, LDP, 16 * cg, 32 * ks, lane);
    const f16x8 bx = frag_i(sX, LDP, 16 * cg, 32 * ks, lane);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int nt = 4 * fh + i;
      const f16x8 ah = frag_i(sH, LDP, 16 * nt, 32 * ks, lane);
      HK[i] = mfma16h(ah, bk, HK[i]);
      HX[i] = mfma16h(ah, bx, HX[i]);
      P[i] = mfma16h(frag_i(sDn, LDP, 16 * nt, 32 * ks, lane), bk, P[i]);
    }
  }
  // in-block products over the 64 tokens t (rows) for this wave's columns s:
  // XK = x_t . k_s, QK = dq_t . k_s, KK = k_t . k_s (both feature halves form them)
  f32x4 XK[4], QK[4], KK[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    XK[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    QK[tt] = XK[tt];
    KK[tt] = XK[tt];
  }
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const f16x8 bk = frag_i(sK, LDP, 16 * cg, 32 * ks, lane);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      XK[tt] = mfma16h(frag_i(sX, LDP, 16 * tt, 32 * ks, lane), bk, XK[tt]);
      QK[tt] = mfma16h(frag_i(sQ, LDP, 16 * tt, 32 * ks, lane), bk, QK[tt]);
      KK[tt] = mfma16h(frag_i(sK, LDP, 16 * tt, 32 * ks, lane), bk, KK[tt]);
    }
  }
  // masks and the scalar sums: m_ts = e^{g_t - g_s} (t >= s); dm = (x_t.k_s)(dq_t.k_s) m_ts
  // (XK carries the scale sx and QK sq: S1 and S2 keep them, dm is unscaled)
  const float rho_s = SC(CS_RHO, s);
  const float uxq = 1.f / (sx * sq);
  float rowdm = 0.f, sw;
  f16x8 s1[2], s2[2], wk[2];
  {
    f32x4 S1[4], S2[4], WK[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const f32x4 gt4 = *reinterpret_cast<const f32x4*>(&SC(CS_G, 16 * tt + 4 * q4));
      const f32x4 rt4 = *reinterpret_cast<const f32x4*>(&SC(CS_RHO, 16 * tt + 4 * q4));
      float col[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int t = 16 * tt + 4 * q4 + v;
        const float m = (t >= s && t < b.nval) ? fast_exp(gt4[v] - gs) : 0.f;
        S1[tt][v] = -XK[tt][v] * m;
        S2[tt][v] = -QK[tt][v] * m;
        const float dm = XK[tt][v] * QK[tt][v] * m * uxq;
        rowdm += dm;
        col[v] = dm;
        // W_st with mm = max(s, t): e^{(g_mm - g_s) + (g_mm - g_t)} rho_mm
        const bool sl = t >= s;
        const float gm = sl ? gt4[v] : gs;
        const float wst = (t < b.nval && s_ok) ? fast_exp((gm - gs) + (gm - gt4[v])) * (sl ? rt4[v] : rho_s) : 0.f;
        WK[tt][v] = 2.f * wst * KK[tt][v];
      }
      // column sums over this wave's s (the 16 lanes of each row group)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float cs = row16_sum(col[v]);
        if (fh == 0 && l16 == 0) SC(CS_COL0 + cg, 16 * tt + 4 * q4 + v) = cs;
      }
    }
    float mw = 0.f;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) mw = fmaxf(mw, absmax4(WK[tt]));
    sw = pow2_scale(wave_max(mw));
#pragma unroll
    for (int jk = 0; jk < 2; ++jk) {
      s1[jk] = h8(S1[2 * jk], S1[2 * jk + 1]);
      s2[jk] = h8(S2[2 * jk], S2[2 * jk + 1]);
      wk[jk] = h8_of(WK[2 * jk], WK[2 * jk + 1], sw);
    }
  }
  rowdm += __shfl_xor(rowdm, 16, 64);
  rowdm += __shfl_xor(rowdm, 32, 64);
  // dk^T accumulators over this wave's feature half: in-block terms, then the lambda terms L
  f32x4 DK[4], L[4];
  const float beta2 = 2.f * fast_exp(gs) * rho_s;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    DK[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    L[i] = DK[i];
  }
#pragma unroll
  for (int jk = 0; jk < 2; ++jk)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int nt = 4 * fh + i;
      DK[i] = mfma16h(frag_t_i(sQ, LDP, 32 * jk, 16 * nt, lane), s1[jk], DK[i]);
      DK[i] = mfma16h(frag_t_i(sX, LDP, 32 * jk, 16 * nt, lane), s2[jk], DK[i]);
      L[i] = mfma16h(frag_t_i(sK, LDP, 32 * jk, 16 * nt, lane), wk[jk], L[i]);
    }
  // unscale: DK (sx sq), L's MFMA part (sw), P (sd), HX (sx)
  const float uw = 1.f / sw, ud = 1.f / sd, ux = 1.f / sx;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      DK[i][v] *= uxq;
      L[i][v] = uw * L[i][v] + beta2 * HK[i][v];
      P[i][v] *= ud;
      HX[i][v] *= ux;
    }
  // per-column dot products with k_s, dq_s (fp32 from memory) over both feature halves
  const float ec = fast_exp(Gam - gs);
  const int64_t ro = ((int64_t)(b.tok0 + s) * H + h) * D + 4 * q4;
  float kl = 0.f, kp = 0.f, qhx = 0.f;
  {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int nt = 4 * fh + i;
      const f16x4 kk = *reinterpret_cast<const f16x4*>(sK + s * LDP + icol(16 * nt + 4 * q4));
      const f32x4 dq = s_ok ? *reinterpret_cast<const f32x4*>(w.dq + ro + 16 * nt) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        kl += (float)kk[v] * L[i][v];
        kp += (float)kk[v] * P[i][v];
        qhx += dq[v] * HX[i][v];
      }
    }
    kl += __shfl_xor(kl, 16, 64);
    kl += __shfl_xor(kl, 32, 64);
    kp += __shfl_xor(kp, 16, 64);
    kp += __shfl_xor(kp, 32, 64);
    qhx += __shfl_xor(qhx, 16, 64);
    qhx += __shfl_xor(qhx, 32, 64);
    if (q4 == 0) {
      float* xo = xch + (fh * CB + s) * 4;
      xo[0] = kl; xo[1] = kp; xo[2] = qhx;
    }
  }
  // store this feature half of dk_s = DK + L + e^{Gam - g_s} P
  if (s_ok) {
    const int64_t dko = ((int64_t)(b.tok0 + s) * H + h) * D + 4 * q4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int nt = 4 * fh + i;
      f32x4 y;
#pragma unroll
      for (int v = 0; v < 4; ++v) y[v] = DK[i][v] + L[i][v] + ec * P[i][v];
      if (w.dk_add) {
        const f32x4 o0 = *reinterpret_cast<const f32x4*>(w.dk_add + dko + 16 * nt);
#pragma unroll
        for (int v = 0; v < 4; ++v) y[v] += o0[v];
      }
      *reinterpret_cast<bf16x4*>(w.dk + dko + 16 * nt) = bf4(y);
    }
  }
  lds_barrier();       // the column sums, the feature halves' dot products, red[0..7]
  // dL/dg_s (waves of the first feature half; the second has the same inputs)
  float dg = 0.f, phi = 0.f;
  if (fh == 0 && s_ok) {
    const float* xo = xch + s * 4;
    const float* xp = xch + (CB + s) * 4;
    kl = xo[0] + xp[0];
    kp = xo[1] + xp[1];
    qhx = xo[2] + xp[2];
    phi = 0.5f * ec * kp;
    const float f = w.fro[(int64_t)(b.tok0 + s) * H + h];
    dg = rowdm - fast_exp(gs) * qhx + SC(CS_A, s) * f * f - 0.5f * kl - phi;
    dg -= SC(CS_COL0 + 0, s) + SC(CS_COL0 + 1, s) + SC(CS_COL0 + 2, s) + SC(CS_COL0 + 3, s);
  }
  // sum of phi over the block (for the last token)
  float ph = phi;
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) ph += __shfl_xor(ph, m, 64);
  float dnh_all = 0.f;
#pragma unroll
  for (int j = 0; j < C_NTHR / 64; ++j) dnh_all += red[j];
  lds_barrier();       // every read of red[0..7]
  if (fh == 0 && lane == 0) red[8 + cg] = ph;
  lds_barrier();
  if (fh == 0 && s_ok && s == b.nval - 1)
    dg += 0.5f * fast_exp(Gam) * dnh_all + red[8] + red[9] + red[10] + red[11];
  // dgk_u = sum_{t >= u} dL/dg_t within the block
  if (fh == 0 && q4 == 0) SC(CS_DG, s) = s_ok ? dg : 0.f;
  lds_barrier();
  if (w.dgk && wave == 0 && lane < b.nval) {
    float acc = 0.f;
    for (int t2 = lane; t2 < b.nval; ++t2) acc += SC(CS_DG, t2);
    w.dgk[(int64_t)(b.tok0 + lane) * H + h] = acc;
  }
}

// ===========================================================================
// The training backward of the GLA readout (chunk_simple_gla's backward)
// ===========================================================================
// o_t = scale (e^{G_t} S_c^T u_t + sum_{s<=t in block} e^{G_t-G_s} (u_t.k_s) v_s), with
// u_t = q_t + alpha_t (x_t - q_t) the blended query, G the in-block cumsum of g and
// S_c the block-start K x V state.  With dSn_c the gradient of S_{c+1} (the later
// blocks' share, the same reverse scan as the solve's):
//   E'_c = scale sum_t e^{G_t} u_t do_t^T,   dSn_c = E'_{c+1} + e^{Gam_{c+1}} dSn_{c+1}
//   du_t = scale (e^{G_t} S_c do_t + sum_{s<=t} e^{G_t-G_s} (do_t.v_s) k_s)
//   dk_s = scale sum_{t>=s} e^{G_t-G_s} (do_t.v_s) u_t + e^{Gam-G_s} dSn v_s
//   dv_s = scale sum_{t>=s} e^{G_t-G_s} (u_t.k_s) do_t + e^{Gam-G_s} dSn^T k_s
//   dL/dG_t = u_t.du_t - k_t.dk_t (+ <dSn, S_{c+1}> at the block's last token)
// and dg is its in-block reverse cumsum; the blend gives dx = alpha du,
// dq = (1 - alpha) du, dalpha = du.(x - q).
struct GlaBwd {
  const bf16* q; const bf16* x; const bf16* v; const bf16* dout;   // [tokens][H][D]
  const void* alpha; int alpha_dt;        // [tokens][H]
  bf16* e; float* gam;                    // as Bwd
  float* dx;                              // [tokens][H][D]: alpha du (the solve's dx)
  // [tokens][H][D]: dq and dk in fp32 when the solve's backward adds to them
  // (dq32, dk32), else in bf16 (dq_bf, dk_bf); dv in bf16
  float* dq32; float* dk32; bf16* dq_bf; bf16* dk_bf; bf16* dv;
  float* dalpha; float* dg;               // [tokens][H]
  float scale;
  int solve;                              // 0: num_iter == 0 (u = q, no x, alpha unused)
};

__device__ __forceinline__ float gla_alpha(const GlaBwd& w, int64_t i) {
  return w.solve ? ldsc(w.alpha, i, w.alpha_dt) : 0.f;
}

// E'_c of block gb (tile-major, row-major K x V) and the block's g total
constexpr int GE_OFF_U = 0, GE_OFF_DO = SZ_K, GE_OFF_SC = 2 * SZ_K;
constexpr int GE_SMEM = GE_OFF_SC + CB * 4 + 16 * 4;
__global__ __launch_bounds__(NTHR, 2) void gla_e_kernel(Params p, GlaBwd w) {
  __shared__ __align__(16) unsigned char smem[GE_SMEM];
  f16* sU = reinterpret_cast<f16*>(smem + GE_OFF_U);
  f16* sDo = reinterpret_cast<f16*>(smem + GE_OFF_DO);
  float* sG = reinterpret_cast<float*>(smem + GE_OFF_SC);
  float* mslot = sG + CB;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, l16 = lane & 15;
  const int gb = blockIdx.x, h = blockIdx.y, H = p.H;
  const Blk b = block_of(p, gb);
  if (b.nval <= 0) return;
  if (wave == 0) {
    const bool ok = lane < b.nval;
    const float G = scan64(ok ? ldsc(p.g, (int64_t)(b.tok0 + lane) * H + h, p.g_dt) : 0.f);
    sG[lane] = G;
    if (lane == b.nval - 1) w.gam[(int64_t)gb * H + h] = G;
  }
  lds_barrier();
  // rows: e^{G_t} scale u_t and do_t (fp32), then scaled into fp16
  f32x4 u0[CB / 16], u1[CB / 16];
  bf16x8 dr[CB / 16];
  float mx[2] = {0.f, 0.f};
#pragma unroll
  for (int pass = 0; pass < CB / 16; ++pass) {
    const int row = pass * 16 + (tid >> 4), f0 = (tid & 15) * 8;
    const bool ok = row < b.nval;
    const int64_t ti = (int64_t)(b.tok0 + row) * H + h, ro = ti * D + f0;
    const bf16x8 qr = ok ? *reinterpret_cast<const bf16x8*>(w.q + ro) : bf16x8{};
    const bf16x8 xr = (ok && w.solve) ? *reinterpret_cast<const bf16x8*>(w.x + ro) : bf16x8{};
    dr[pass] = ok ? *reinterpret_cast<const bf16x8*>(w.dout + ro) : bf16x8{};
    const float al = ok ? gla_alpha(w, ti) : 0.f;
    const float eg = ok ? w.scale * fast_exp(sG[row]) : 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      u0[pass][v] = eg * ((float)qr[v] + al * ((float)xr[v] - (float)qr[v]));
      u1[pass][v] = eg * ((float)qr[4 + v] + al * ((float)xr[4 + v] - (float)qr[4 + v]));
    }
    mx[0] = fmaxf(mx[0], fmaxf(absmax4(u0[pass]), absmax4(u1[pass])));
    mx[1] = fmaxf(mx[1], absmax8(dr[pass]));
  }
  block_max(mx, mslot, wave, lane);
  const float su = pow2_scale(mx[0]), sd = pow2_scale(mx[1]);
#pragma unroll
  for (int pass = 0; pass < CB / 16; ++pass) {
    const int row = pass * 16 + (tid >> 4), f0 = (tid & 15) * 8;
    store8_i(sU + row * LDP, f0, h8_of(u0[pass], u1[pass], su));
    store8_i(sDo + row * LDP, f0, scale_h8(dr[pass], sd));
  }
  lds_barrier();
  const float un = 1.f / (su * sd);
  bf16* eo = w.e + ((int64_t)gb * H + h) * D * D;
  // wave w: E'^T tile rows (V) 2w, 2w+1 by all 8 tile columns (K); the lane's 4
  // values are 4 consecutive V columns of one K row of E'
#pragma unroll
  for (int ir = 0; ir < 2; ++ir) {
    const int jt = 2 * wave + ir;
    f32x4 E[8];
#pragma unroll
    for (int it = 0; it < 8; ++it) E[it] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int jk = 0; jk < 2; ++jk) {
      const f16x8 ad = frag_t_i(sDo, LDP, 32 * jk, 16 * jt, lane);
#pragma unroll
      for (int it = 0; it < 8; ++it) E[it] = mfma16h(ad, frag_t_i(sU, LDP, 32 * jk, 16 * it, lane), E[it]);
    }
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      f32x4 y;
#pragma unroll
      for (int v = 0; v < 4; ++v) y[v] = un * E[it][v];
      *reinterpret_cast<bf16x4*>(eo + blk_index(16 * it + l16, 16 * jt + 4 * q4)) = bf4(y);
    }
  }
}

constexpr int GB_OFF_K = 0, GB_OFF_V = SZ_K, GB_OFF_DO = 2 * SZ_K, GB_OFF_U = 3 * SZ_K;
constexpr int GB_OFF_S = 4 * SZ_K, GB_OFF_DS = GB_OFF_S + SZ_H, GB_OFF_SC = GB_OFF_DS + SZ_H;
enum { GS_G, GS_DG, NGS };
// 8 waves: wave w takes the 16 columns s of group w & 3 and the feature half w >> 2
constexpr int GB_NTHR = 512;
constexpr int GB_OFF_RED = GB_OFF_SC + NGS * CB * 4;       // 16 floats of cross-wave sums
constexpr int GB_OFF_MS = GB_OFF_RED + 16 * 4;             // 24 floats for block_max
constexpr int GB_OFF_XCH = GB_OFF_MS + 24 * 4;             // [2][64][4] feature-half dot products
constexpr int GB_SMEM = GB_OFF_XCH + 2 * CB * 4 * 4;
static_assert(GB_SMEM <= 160 * 1024, "LDS budget");

// du (-> dx, dq, dalpha), dk, dv, dg of block gb (see the section comment)
__global__ __launch_bounds__(GB_NTHR, 1) void gla_bwd_kernel(Params p, GlaBwd w) {
  __shared__ __align__(16) unsigned char smem[GB_SMEM];
  f16* sK = reinterpret_cast<f16*>(smem + GB_OFF_K);
  f16* sV = reinterpret_cast<f16*>(smem + GB_OFF_V);
  f16* sDo = reinterpret_cast<f16*>(smem + GB_OFF_DO);
  f16* sU = reinterpret_cast<f16*>(smem + GB_OFF_U);
  f16* sS = reinterpret_cast<f16*>(smem + GB_OFF_S);      // S_c^T: rows V, columns K
  f16* sDS = reinterpret_cast<f16*>(smem + GB_OFF_DS);    // dSn: rows K, columns V
  float* sc = reinterpret_cast<float*>(smem + GB_OFF_SC);
  float* red = reinterpret_cast<float*>(smem + GB_OFF_RED);
  float* mslot = reinterpret_cast<float*>(smem + GB_OFF_MS);
  float* xch = reinterpret_cast<float*>(smem + GB_OFF_XCH);
  auto SC = [&](int slot, int t) -> float& { return sc[slot * CB + t]; };
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cg = wave & 3, fh = wave >> 2;   // column group, feature half (nt 4 fh .. 4 fh + 3)
  const int q4 = lane >> 4, l16 = lane & 15;
  const int gb = blockIdx.x, h = blockIdx.y, H = p.H;
  const Blk b = block_of(p, gb);
  if (b.nval <= 0) return;
  const int64_t DD = (int64_t)D * D;
  constexpr int NP = CB * 16 / GB_NTHR;    // staging passes of 32 rows

  // S_c (as the solve forms it: zero-start block state + decayed segment start)
  if (tid < NTHR) {
    const int64_t so = ((int64_t)b.s_id * H + h) * DD;
    const int64_t bso = ((int64_t)gb * H + h) * DD;
    StateLd sst;
    solve::state_issue_b<false>(sst, b.lb > 0 ? p.ws_sb + bso : nullptr, tid);
    const float off_g = p.ws_boff[((int64_t)gb * H + h) * 2 + 1];
    solve::state_issue_s<false>(sst, (b.lb == 0 || off_g > solve::SEG_STATE_DROP) ? p.ws_s0 + so : nullptr, tid);
    solve::state_store<false>(sS, sst, fast_exp(off_g), tid);
  }
  if (wave == 0) {
    const bool ok = lane < b.nval;
    SC(GS_G, lane) = scan64(ok ? ldsc(p.g, (int64_t)(b.tok0 + lane) * H + h, p.g_dt) : 0.f);
  }
  lds_barrier();
  // rows k, v (fp16 as given), do and u (scaled); dSn (scaled) and <dSn, S_c>
  bf16x8 kr[NP], vr[NP], dr[NP];
  f32x4 u0[NP], u1[NP];
  const bf16* dn = w.e + ((int64_t)gb * H + h) * DD;
  const int drw = tid >> 2, dc0 = (tid & 3) * 32;    // this thread's dSn: row drw, columns dc0..+31
  f32x4 dsv[8];
  float mx[3] = {0.f, 0.f, 0.f};          // max |do|, |u|, |dSn|
#pragma unroll
  for (int pass = 0; pass < NP; ++pass) {
    const int row = pass * 32 + (tid >> 4), f0 = (tid & 15) * 8;
    const bool ok = row < b.nval;
    const int64_t ti = (int64_t)(b.tok0 + row) * H + h, ro = ti * D + f0;
    kr[pass] = ok ? *reinterpret_cast<const bf16x8*>(p.k + (int64_t)(b.tok0 + row) * p.kv_ts + h * D + f0) : bf16x8{};
    vr[pass] = ok ? *reinterpret_cast<const bf16x8*>(w.v + ro) : bf16x8{};
    dr[pass] = ok ? *reinterpret_cast<const bf16x8*>(w.dout + ro) : bf16x8{};
    const bf16x8 qr = ok ? *reinterpret_cast<const bf16x8*>(w.q + ro) : bf16x8{};
    const bf16x8 xr = (ok && w.solve) ? *reinterpret_cast<const bf16x8*>(w.x + ro) : bf16x8{};
    const float al = ok ? gla_alpha(w, ti) : 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      u0[pass][v] = (float)qr[v] + al * ((float)xr[v] - (float)qr[v]);
      u1[pass][v] = (float)qr[4 + v] + al * ((float)xr[4 + v] - (float)qr[4 + v]);
    }
    mx[0] = fmaxf(mx[0], absmax8(dr[pass]));
    mx[1] = fmaxf(mx[1], fmaxf(absmax4(u0[pass]), absmax4(u1[pass])));
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    dsv[j] = f4(*reinterpret_cast<const bf16x4*>(dn + blk_index(drw, dc0 + 4 * j)));
    mx[2] = fmaxf(mx[2], absmax4(dsv[j]));
  }
  block_max<3, GB_NTHR / 64>(mx, mslot, wave, lane);
  const float sdo = pow2_scale(mx[0]), su = pow2_scale(mx[1]), sds = pow2_scale(mx[2]);
#pragma unroll
  for (int pass = 0; pass < NP; ++pass) {
    const int row = pass * 32 + (tid >> 4), f0 = (tid & 15) * 8;
    store8_i(sK + row * LDP, f0, scale_h8(kr[pass], 1.f));
    store8_i(sV + row * LDP, f0, scale_h8(vr[pass], 1.f));
    store8_i(sDo + row * LDP, f0, scale_h8(dr[pass], sdo));
    store8_i(sU + row * LDP, f0, h8_of(u0[pass], u1[pass], su));
  }
  float dss = 0.f;                        // <dSn, S_c> over this thread's elements
#pragma unroll
  for (int j = 0; j < 8; ++j) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int c = dc0 + 4 * j + v;      // V index; S_c^T[c][drw] in sS
      dss += dsv[j][v] * (float)sS[c * LDP + icol(drw)];
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
    store8_i(sDS + drw * LDP, dc0 + 8 * j, h8_of(dsv[2 * j], dsv[2 * j + 1], sds));
  dss = wave_sum(dss);
  if (lane == 0) red[wave] = dss;
  lds_barrier();

  const int s = 16 * cg + l16;            // this lane's token / key column
  const bool s_ok = s < b.nval;
  const float Gs = SC(GS_G, s), Gam = SC(GS_G, b.nval - 1);
  const float ec = fast_exp(Gam - Gs), egs = fast_exp(Gs);
  const int64_t ti = (int64_t)(b.tok0 + s) * H + h;
  const int64_t ro = ti * D + 4 * q4;     // + 16 nt: features 16 nt + 4 q4 .. +3
  float* xo = xch + (fh * CB + s) * 4;    // this half's dot products of column s

  // ---- du (rows f = K of this half, column t = s) ---------------------------
  {
    f32x4 DQ[4], DI[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      DQ[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      DI[i] = DQ[i];
    }
    // S_c do_t: A = S_c rows (K) over V, read transposed from S_c^T
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const f16x8 bd = frag_i(sDo, LDP, 16 * cg, 32 * ks, lane);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        DQ[i] = mfma16h(frag_t_i(sS, LDP, 32 * ks, 16 * (4 * fh + i), lane), bd, DQ[i]);
    }
    // P[j][t] = e^{G_t-G_j} (do_t.v_j), j <= t: rows j over the block, column t
    f16x8 pb[2];
    {
      f32x4 P[4];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) P[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const f16x8 bd = frag_i(sDo, LDP, 16 * cg, 32 * ks, lane);
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) P[jt] = mfma16h(frag_i(sV, LDP, 16 * jt, 32 * ks, lane), bd, P[jt]);
      }
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const f32x4 gj = *reinterpret_cast<const f32x4*>(&SC(GS_G, 16 * jt + 4 * q4));
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int j = 16 * jt + 4 * q4 + v;
          P[jt][v] = (j <= s && j < b.nval) ? P[jt][v] * fast_exp(Gs - gj[v]) : 0.f;
        }
      }
      pb[0] = h8(P[0], P[1]);
      pb[1] = h8(P[2], P[3]);
    }
#pragma unroll
    for (int jk = 0; jk < 2; ++jk)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        DI[i] = mfma16h(frag_t_i(sK, LDP, 32 * jk, 16 * (4 * fh + i), lane), pb[jk], DI[i]);
    // du = scale (e^{G_t} DQ + DI) / sdo; dx, dq, dalpha and u.du over this half
    const float cu = w.scale / sdo;
    const float al = s_ok ? gla_alpha(w, ti) : 0.f;
    float dal = 0.f, udu = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int nt = 4 * fh + i;
      const bf16x4 qv = s_ok ? *reinterpret_cast<const bf16x4*>(w.q + ro + 16 * nt) : bf16x4{};
      const bf16x4 xv = (s_ok && w.solve) ? *reinterpret_cast<const bf16x4*>(w.x + ro + 16 * nt) : bf16x4{};
      f32x4 du, dqo, dxo;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        du[v] = cu * (egs * DQ[i][v] + DI[i][v]);
        const float qf = (float)qv[v], xf = (float)xv[v];
        dal += du[v] * (xf - qf);
        udu += du[v] * (qf + al * (xf - qf));
        dqo[v] = (1.f - al) * du[v];
        dxo[v] = al * du[v];
      }
      if (s_ok) {
        if (w.dq32) *reinterpret_cast<f32x4*>(w.dq32 + ro + 16 * nt) = dqo;
        else *reinterpret_cast<bf16x4*>(w.dq_bf + ro + 16 * nt) = bf4(dqo);
        if (w.solve) *reinterpret_cast<f32x4*>(w.dx + ro + 16 * nt) = dxo;
      }
    }
    dal += __shfl_xor(dal, 16, 64);
    dal += __shfl_xor(dal, 32, 64);
    udu += __shfl_xor(udu, 16, 64);
    udu += __shfl_xor(udu, 32, 64);
    if (q4 == 0) {
      xo[0] = udu;
      xo[1] = dal;
    }
  }
  // ---- dk (rows f = K of this half, column s) ----------------------------------
  {
    f32x4 DK[4], DX[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      DK[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      DX[i] = DK[i];
    }
    // R[t][s] = e^{G_t-G_s} (do_t.v_s), t >= s
    f16x8 rb[2];
    {
      f32x4 R[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) R[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const f16x8 bv = frag_i(sV, LDP, 16 * cg, 32 * ks, lane);
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) R[tt] = mfma16h(frag_i(sDo, LDP, 16 * tt, 32 * ks, lane), bv, R[tt]);
      }
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const f32x4 gt = *reinterpret_cast<const f32x4*>(&SC(GS_G, 16 * tt + 4 * q4));
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int t = 16 * tt + 4 * q4 + v;
          R[tt][v] = (t >= s && t < b.nval) ? R[tt][v] * fast_exp(gt[v] - Gs) : 0.f;
        }
      }
      rb[0] = h8(R[0], R[1]);
      rb[1] = h8(R[2], R[3]);
    }
#pragma unroll
    for (int jk = 0; jk < 2; ++jk)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        DK[i] = mfma16h(frag_t_i(sU, LDP, 32 * jk, 16 * (4 * fh + i), lane), rb[jk], DK[i]);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const f16x8 bv = frag_i(sV, LDP, 16 * cg, 32 * ks, lane);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        DX[i] = mfma16h(frag_i(sDS, LDP, 16 * (4 * fh + i), 32 * ks, lane), bv, DX[i]);
    }
    const float ci = w.scale / (su * sdo), cx = ec / sds;
    float kdk = 0.f, kdkx = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int nt = 4 * fh + i;
      const f16x4 kk = *reinterpret_cast<const f16x4*>(sK + s * LDP + icol(16 * nt + 4 * q4));
      f32x4 y;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float xpart = cx * DX[i][v];
        y[v] = ci * DK[i][v] + xpart;
        kdk += (float)kk[v] * y[v];
        kdkx += (float)kk[v] * xpart;
      }
      if (s_ok) {
        if (w.dk32) *reinterpret_cast<f32x4*>(w.dk32 + ro + 16 * nt) = y;
        else *reinterpret_cast<bf16x4*>(w.dk_bf + ro + 16 * nt) = bf4(y);
      }
    }
    kdk += __shfl_xor(kdk, 16, 64);
    kdk += __shfl_xor(kdk, 32, 64);
    kdkx += __shfl_xor(kdkx, 16, 64);
    kdkx += __shfl_xor(kdkx, 32, 64);
    if (q4 == 0) {
      xo[2] = kdk;
      xo[3] = kdkx;
    }
  }
  // ---- dv (rows f = V of this half, column s) ----------------------------------
  {
    f32x4 DV[4], DX[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      DV[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      DX[i] = DV[i];
    }
    // U[t][s] = e^{G_t-G_s} (u_t.k_s), t >= s
    f16x8 ub[2];
    {
      f32x4 U[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) U[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const f16x8 bk = frag_i(sK, LDP, 16 * cg, 32 * ks, lane);
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) U[tt] = mfma16h(frag_i(sU, LDP, 16 * tt, 32 * ks, lane), bk, U[tt]);
      }
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const f32x4 gt = *reinterpret_cast<const f32x4*>(&SC(GS_G, 16 * tt + 4 * q4));
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int t = 16 * tt + 4 * q4 + v;
          U[tt][v] = (t >= s && t < b.nval) ? U[tt][v] * fast_exp(gt[v] - Gs) : 0.f;
        }
      }
      ub[0] = h8(U[0], U[1]);
      ub[1] = h8(U[2], U[3]);
    }
#pragma unroll
    for (int jk = 0; jk < 2; ++jk)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        DV[i] = mfma16h(frag_t_i(sDo, LDP, 32 * jk, 16 * (4 * fh + i), lane), ub[jk], DV[i]);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const f16x8 bk = frag_i(sK, LDP, 16 * cg, 32 * ks, lane);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        DX[i] = mfma16h(frag_t_i(sDS, LDP, 32 * ks, 16 * (4 * fh + i), lane), bk, DX[i]);
    }
    const float ci = w.scale / (su * sdo), cx = ec / sds;
    if (s_ok) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4 y;
#pragma unroll
        for (int v = 0; v < 4; ++v) y[v] = ci * DV[i][v] + cx * DX[i][v];
        *reinterpret_cast<bf16x4*>(w.dv + ro + 16 * (4 * fh + i)) = bf4(y);
      }
    }
  }
  lds_barrier();       // both halves' dot products, red[0..7]
  // ---- dg: dL/dG_t, the last token's <dSn, S_{c+1}>, the in-block reverse cumsum
  float dG = 0.f, kx = 0.f;
  if (fh == 0 && s_ok) {
    const float* xa = xch + s * 4;
    const float* xb = xch + (CB + s) * 4;
    dG = (xa[0] + xb[0]) - (xa[2] + xb[2]);
    kx = xa[3] + xb[3];
    if (q4 == 0 && w.solve) w.dalpha[ti] = xa[1] + xb[1];
  }
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) kx += __shfl_xor(kx, m, 64);
  float dss_all = 0.f;
#pragma unroll
  for (int j = 0; j < GB_NTHR / 64; ++j) dss_all += red[j];
  lds_barrier();       // every read of red[0..7]
  if (fh == 0 && lane == 0) red[8 + cg] = kx;
  lds_barrier();
  if (fh == 0 && s_ok && q4 == 0) {
    float d = dG;
    if (s == b.nval - 1) d += fast_exp(Gam) * dss_all + red[8] + red[9] + red[10] + red[11];
    SC(GS_DG, s) = d;
  }
  lds_barrier();
  if (wave == 0 && lane < b.nval) {
    float acc = 0.f;
    for (int t2 = lane; t2 < b.nval; ++t2) acc += SC(GS_DG, t2);
    w.dg[(int64_t)(b.tok0 + lane) * H + h] = acc;
  }
}
}  // namespace train
}  // namespace gkap
}  // namespace hmx

// ---------------------------------------------------------------------------
// The training-side Chebyshev solve (ChebyshevIteration of the training layer):
// k, q [tokens, H, D] bf16 with k at H heads, the h_kk recurrence only (no GLA),
// no initial state.  The forward leaves the walk's block-start states in the
// workspace; the backward's dq solve reads them from there.
// ---------------------------------------------------------------------------
namespace {
int cheb_params(Params& p, const char* fn, const void* k, int64_t k_ts, const void* rhs,
                int64_t rhs_ts, int32_t dtype, const void* gk, int32_t gk_dtype,
                const int32_t* seg_table, int32_t nseg_total, int32_t nblock_total, int32_t N,
                int32_t H, int32_t D_, int32_t num_iter, float ridge_ratio, void* workspace,
                size_t workspace_bytes) {
  HMX_REQUIRE(dtype == HMX_BF16, HMX_EUNSUPPORTED, "%s: k and q must be bfloat16 (dtype code %d)",
              fn, dtype);
  HMX_REQUIRE(D_ == D, HMX_EUNSUPPORTED, "%s: only D == 128 is supported (got %d)", fn, D_);
  HMX_REQUIRE(H > 0 && N >= 0 && num_iter >= 0, HMX_EINVAL, "%s: H=%d N=%d num_iter=%d", fn, H,
              N, num_iter);
  HMX_REQUIRE(k && rhs && seg_table, HMX_EINVAL, "%s: null tensor pointer", fn);
  HMX_REQUIRE(k_ts % 8 == 0 && rhs_ts % 8 == 0 && ((uintptr_t)k | (uintptr_t)rhs) % 16 == 0,
              HMX_EINVAL, "%s: k / q rows must be 16-byte aligned", fn);
  HMX_REQUIRE(!gk || gk_dtype == HMX_F32 || gk_dtype == HMX_BF16 || gk_dtype == HMX_F16,
              HMX_EUNSUPPORTED, "%s: gk dtype code %d", fn, gk_dtype);
  HMX_REQUIRE(nseg_total >= 0 && nblock_total >= 0, HMX_EINVAL, "%s: nseg_total=%d nblock_total=%d",
              fn, nseg_total, nblock_total);
  const WsLayout wl = ws_layout(nseg_total, nblock_total, H);
  HMX_REQUIRE(nseg_total == 0 || (workspace && workspace_bytes >= wl.total), HMX_EINVAL,
              "%s: workspace of %zu bytes needed, %zu given", fn, wl.total, workspace_bytes);
  p = Params{};
  p.k = static_cast<const bf16*>(k); p.v = p.k; p.kv_ts = k_ts;
  p.q = static_cast<const bf16*>(rhs); p.q_ts = rhs_ts;
  p.gk = gk; p.gk_dt = gk_dtype;
  p.fused = 0; p.gp = hmx_gate_proj{};
  p.onw_dt = HMX_F32;
  p.hkk = Pool{nullptr, nullptr, (int64_t)H * D * D, HMX_F32};
  p.hkv = Pool{nullptr, nullptr, (int64_t)H * D * D, HMX_F32};
  p.seg = seg_table; p.nseg_total = nseg_total; p.nblk_total = nblock_total;
  p.H = H; p.HKV = H; p.num_iter = num_iter; p.ridge_ratio = ridge_ratio; p.scale = 1.f;
  p.l2norm = 0;
  char* ws = static_cast<char*>(workspace);
  p.ws_hb = reinterpret_cast<f16*>(ws + wl.hb);
  p.ws_sb = reinterpret_cast<f16*>(ws + wl.sb);
  p.ws_dh = reinterpret_cast<float*>(ws + wl.dh);
  p.ws_ds = reinterpret_cast<float*>(ws + wl.ds);
  p.ws_h0 = reinterpret_cast<f16*>(ws + wl.h0);
  p.ws_s0 = reinterpret_cast<f16*>(ws + wl.s0);
  p.ws_boff = reinterpret_cast<float*>(ws + wl.boff);
  p.ws_dec = reinterpret_cast<float*>(ws + wl.dec);
  p.segblk = reinterpret_cast<int*>(ws + wl.segblk);
  return HMX_OK;
}
}  // namespace

extern "C" int hmx_gka_cheb_fwd(const void* k, int64_t k_token_stride, const void* q,
                                int64_t q_token_stride, int32_t qk_dtype, const void* gk,
                                int32_t gk_dtype, void* x, float* fro, float* h_kk_final,
                                const int32_t* seg_table, int32_t nseg_total,
                                int32_t nblock_total, int32_t N, int32_t H, int32_t D_,
                                int32_t num_iter, float ridge_ratio, void* workspace,
                                size_t workspace_bytes, void* stream) {
  Params p;
  const int rc = cheb_params(p, "hmx_gka_cheb_fwd", k, k_token_stride, q, q_token_stride, qk_dtype,
                             gk, gk_dtype, seg_table, nseg_total, nblock_total, N, H, D_,
                             num_iter, ridge_ratio, workspace, workspace_bytes);
  if (rc != HMX_OK) return rc;
  HMX_REQUIRE(x && fro && ((uintptr_t)x % 16) == 0, HMX_EINVAL,
              "hmx_gka_cheb_fwd: x (16-byte aligned) and fro are required");
  if (nseg_total == 0) return HMX_OK;
  p.o = static_cast<bf16*>(x);
  p.fro = fro;
  p.hkk.out = h_kk_final;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL((walk::gka_walk_kernel<true, false>), dim3(nseg_total, H), dim3(NTHR), 0, s, p);
  hipLaunchKernelGGL(gka_combine_kernel, dim3(N * H, 16), dim3(256), 0, s, p, 1);
  if (nblock_total > 0)
    hipLaunchKernelGGL((solve::gka_solve_kernel<true, false, solve::SM_X>), dim3(nblock_total, H),
                       dim3(NTHR), 0, s, p);
  return check_launch("hmx_gka_cheb_fwd");
}

// backward workspace: E/Dn (bf16), the blocks' gk totals, the solve's dq (fp32)
extern "C" size_t hmx_gka_cheb_bwd_workspace_bytes(int32_t nblock_total, int32_t H,
                                                   int64_t tokens) {
  return al256((size_t)nblock_total * H * D * D * sizeof(bf16)) +
         al256((size_t)nblock_total * H * sizeof(float)) +
         al256((size_t)tokens * H * D * sizeof(float));
}

extern "C" int hmx_gka_cheb_bwd(const void* k, int64_t k_token_stride, const void* x,
                                const void* dx, int64_t dx_token_stride, int32_t dtype,
                                const void* gk, int32_t gk_dtype, const float* fro, void* dq,
                                void* dk, float* dgk, const int32_t* seg_table,
                                int32_t nseg_total, int32_t nblock_total, int32_t N, int32_t H,
                                int32_t D_, int64_t tokens, int32_t num_iter, float ridge_ratio,
                                int32_t bp_lambda, void* fwd_workspace, size_t fwd_workspace_bytes,
                                void* bwd_workspace, size_t bwd_workspace_bytes, void* stream) {
  Params p;
  const int rc = cheb_params(p, "hmx_gka_cheb_bwd", k, k_token_stride, dx, dx_token_stride, dtype,
                             gk, gk_dtype, seg_table, nseg_total, nblock_total, N, H, D_,
                             num_iter, ridge_ratio, fwd_workspace, fwd_workspace_bytes);
  if (rc != HMX_OK) return rc;
  HMX_REQUIRE(x && fro && dq && dk && (!gk || dgk) &&
                  (((uintptr_t)x | (uintptr_t)dq | (uintptr_t)dk) % 16) == 0,
              HMX_EINVAL, "hmx_gka_cheb_bwd: x, fro, dq, dk (16-byte aligned) and dgk (with gk) "
                          "are required");
  const size_t need = hmx_gka_cheb_bwd_workspace_bytes(nblock_total, H, tokens);
  HMX_REQUIRE(tokens >= 0 && (nblock_total == 0 || (bwd_workspace && bwd_workspace_bytes >= need)),
              HMX_EINVAL, "hmx_gka_cheb_bwd: backward workspace of %zu bytes needed, %zu given",
              need, bwd_workspace_bytes);
  if (nseg_total == 0 || nblock_total == 0) return HMX_OK;
  char* bw = static_cast<char*>(bwd_workspace);
  const size_t e_bytes = al256((size_t)nblock_total * H * D * D * sizeof(bf16));
  float* dq32 = reinterpret_cast<float*>(bw + e_bytes + al256((size_t)nblock_total * H * sizeof(float)));
  p.fro = const_cast<float*>(fro);
  p.xo32 = dq32;
  train::Bwd w{};
  w.x = static_cast<const bf16*>(x);
  w.dq = dq32; w.fro = fro;
  w.e = reinterpret_cast<bf16*>(bw);
  w.gam = reinterpret_cast<float*>(bw + e_bytes);
  w.dk = static_cast<bf16*>(dk); w.dq_out = static_cast<bf16*>(dq);
  w.dgk = gk ? dgk : nullptr;
  w.bp_lambda = bp_lambda;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(nblock_total, H);
  hipLaunchKernelGGL((solve::gka_solve_kernel<true, false, solve::SM_DQ>), grid, dim3(NTHR), 0, s, p);
  hipLaunchKernelGGL(train::cheb_e_kernel, grid, dim3(train::E_NTHR), 0, s, p, w);
  hipLaunchKernelGGL(train::cheb_dscan_kernel, dim3(N * H, 16), dim3(256), 0, s, p, w);
  hipLaunchKernelGGL(train::cheb_dk_kernel, grid, dim3(train::C_NTHR), 0, s, p, w);
  return check_launch("hmx_gka_cheb_bwd");
}

// ---------------------------------------------------------------------------
// The training GKA forward with its backward (gka_chebyshev_gla): the solve, the
// alpha blend and the GLA readout; q, k, v [tokens][H][D] bf16 (contiguous, k and
// v at H heads), no initial states, beta already applied by the layer.
// ---------------------------------------------------------------------------
namespace {
int train_params(Params& p, const char* fn, const void* q, const void* k, const void* v,
                 int32_t dtype, const void* alpha, int32_t alpha_dtype, const void* g,
                 int32_t g_dtype, const void* gk, int32_t gk_dtype, const int32_t* seg_table,
                 int32_t nseg_total, int32_t nblock_total, int32_t N, int32_t H, int32_t D_,
                 int32_t num_iter, float ridge_ratio, float scale, void* workspace,
                 size_t workspace_bytes) {
  const int rc = cheb_params(p, fn, k, (int64_t)H * D, q, (int64_t)H * D, dtype, gk, gk_dtype,
                             seg_table, nseg_total, nblock_total, N, H, D_, num_iter,
                             ridge_ratio, workspace, workspace_bytes);
  if (rc != HMX_OK) return rc;
  HMX_REQUIRE(v && g && alpha && ((uintptr_t)v % 16) == 0, HMX_EINVAL,
              "%s: v (16-byte aligned), g and alpha are required", fn);
  HMX_REQUIRE(g_dtype >= 0 && g_dtype <= 2 && (!alpha || (alpha_dtype >= 0 && alpha_dtype <= 2)),
              HMX_EUNSUPPORTED, "%s: gate dtype codes must be 0-2", fn);
  p.v = static_cast<const bf16*>(v);
  p.alpha = alpha; p.alpha_dt = alpha_dtype; p.g = g; p.g_dt = g_dtype;
  p.scale = scale;
  return HMX_OK;
}
}  // namespace

extern "C" int hmx_gka_train_fwd(const void* q, const void* k, const void* v, int32_t dtype,
                                 const void* alpha, int32_t alpha_dtype, const void* g,
                                 int32_t g_dtype, const void* gk, int32_t gk_dtype, void* o,
                                 void* x, float* fro, float* h_kk_final, float* h_kv_final,
                                 const int32_t* seg_table, int32_t nseg_total,
                                 int32_t nblock_total, int32_t N, int32_t H, int32_t D_,
                                 int32_t num_iter, float ridge_ratio, float scale,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  Params p;
  const int rc = train_params(p, "hmx_gka_train_fwd", q, k, v, dtype, alpha, alpha_dtype, g,
                              g_dtype, gk, gk_dtype, seg_table, nseg_total, nblock_total, N, H,
                              D_, num_iter, ridge_ratio, scale, workspace, workspace_bytes);
  if (rc != HMX_OK) return rc;
  HMX_REQUIRE(o && h_kv_final && ((uintptr_t)o % 16) == 0 &&
                  (num_iter == 0 || (x && fro && h_kk_final && ((uintptr_t)x % 16) == 0)),
              HMX_EINVAL, "hmx_gka_train_fwd: o, h_kv_final (and with the solver x, fro, "
                          "h_kk_final) are required, 16-byte aligned");
  if (nseg_total == 0) return HMX_OK;
  p.o = static_cast<bf16*>(o);
  p.xs = static_cast<bf16*>(x);
  p.fro = fro;
  p.hkk.out = num_iter > 0 ? h_kk_final : nullptr;
  p.hkv.out = h_kv_final;
  const bool solve_ = num_iter > 0;
  hipStream_t s = (hipStream_t)stream;
  if (solve_) hipLaunchKernelGGL((walk::gka_walk_kernel<true, false>), dim3(nseg_total, H), dim3(NTHR), 0, s, p);
  else hipLaunchKernelGGL((walk::gka_walk_kernel<false, false>), dim3(nseg_total, H), dim3(NTHR), 0, s, p);
  hipLaunchKernelGGL(gka_combine_kernel, dim3(N * H, 16), dim3(256), 0, s, p, (int)solve_);
  if (nblock_total > 0) {
    if (solve_)
      hipLaunchKernelGGL((solve::gka_solve_kernel<true, false, solve::SM_GLA_SAVE>),
                         dim3(nblock_total, H), dim3(NTHR), 0, s, p);
    else
      hipLaunchKernelGGL((solve::gka_solve_kernel<false, false>), dim3(nblock_total, H),
                         dim3(NTHR), 0, s, p);
  }
  return check_launch("hmx_gka_train_fwd");
}

// backward workspace: the solve's backward workspace (with its dq), then dx, the
// GLA's dq and dk (fp32)
extern "C" size_t hmx_gka_train_bwd_workspace_bytes(int32_t nblock_total, int32_t H,
                                                    int64_t tokens) {
  return hmx_gka_cheb_bwd_workspace_bytes(nblock_total, H, tokens) +
         3 * al256((size_t)tokens * H * D * sizeof(float));
}

extern "C" int hmx_gka_train_bwd(const void* q, const void* k, const void* v, int32_t dtype,
                                 const void* alpha, int32_t alpha_dtype, const void* g,
                                 int32_t g_dtype, const void* gk, int32_t gk_dtype,
                                 const void* x, const float* fro, const void* dout, void* dq,
                                 void* dk, void* dv, float* dalpha, float* dg, float* dgk,
                                 const int32_t* seg_table, int32_t nseg_total,
                                 int32_t nblock_total, int32_t N, int32_t H, int32_t D_,
                                 int64_t tokens, int32_t num_iter, float ridge_ratio, float scale,
                                 int32_t bp_lambda, void* fwd_workspace,
                                 size_t fwd_workspace_bytes, void* bwd_workspace,
                                 size_t bwd_workspace_bytes, void* stream) {
  Params p;
  const int rc = train_params(p, "hmx_gka_train_bwd", q, k, v, dtype, alpha, alpha_dtype, g,
                              g_dtype, gk, gk_dtype, seg_table, nseg_total, nblock_total, N, H,
                              D_, num_iter, ridge_ratio, scale, fwd_workspace,
                              fwd_workspace_bytes);
  if (rc != HMX_OK) return rc;
  const bool solve_ = num_iter > 0;
  HMX_REQUIRE(dout && dq && dk && dv && dg && tokens >= 0 &&
                  (!solve_ || (x && fro && dalpha && (!gk || dgk))) &&
                  (((uintptr_t)dout | (uintptr_t)dq | (uintptr_t)dk | (uintptr_t)dv |
                    (uintptr_t)x) % 16) == 0,
              HMX_EINVAL, "hmx_gka_train_bwd: dout, dq, dk, dv, dg (and with the solver x, fro, "
                          "dalpha, dgk) are required, 16-byte aligned");
  const size_t need = hmx_gka_train_bwd_workspace_bytes(nblock_total, H, tokens);
  HMX_REQUIRE(nblock_total == 0 || (bwd_workspace && bwd_workspace_bytes >= need), HMX_EINVAL,
              "hmx_gka_train_bwd: backward workspace of %zu bytes needed, %zu given", need,
              bwd_workspace_bytes);
  if (nseg_total == 0 || nblock_total == 0) return HMX_OK;
  char* bw = static_cast<char*>(bwd_workspace);
  const size_t e_bytes = al256((size_t)nblock_total * H * D * D * sizeof(bf16));
  const size_t cb_bytes = hmx_gka_cheb_bwd_workspace_bytes(nblock_total, H, tokens);
  const size_t tok_bytes = al256((size_t)tokens * H * D * sizeof(float));
  train::GlaBwd gw{};
  gw.q = static_cast<const bf16*>(q); gw.x = static_cast<const bf16*>(x);
  gw.v = static_cast<const bf16*>(v); gw.dout = static_cast<const bf16*>(dout);
  gw.alpha = alpha; gw.alpha_dt = alpha_dtype;
  gw.e = reinterpret_cast<bf16*>(bw);
  gw.gam = reinterpret_cast<float*>(bw + e_bytes);
  gw.dx = reinterpret_cast<float*>(bw + cb_bytes);
  float* dq_cheb = reinterpret_cast<float*>(bw + e_bytes + al256((size_t)nblock_total * H * sizeof(float)));
  float* dq_gla = reinterpret_cast<float*>(bw + cb_bytes + tok_bytes);
  float* dk_gla = reinterpret_cast<float*>(bw + cb_bytes + 2 * tok_bytes);
  if (solve_) {           // the solve's backward adds its dq and dk, then writes bf16
    gw.dq32 = dq_gla; gw.dk32 = dk_gla;
  } else {
    gw.dq_bf = static_cast<bf16*>(dq); gw.dk_bf = static_cast<bf16*>(dk);
  }
  gw.dv = static_cast<bf16*>(dv); gw.dalpha = dalpha; gw.dg = dg;
  gw.scale = scale; gw.solve = solve_;
  train::Bwd cw{};
  cw.e = gw.e; cw.gam = gw.gam;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(nblock_total, H), sgrid(N * H, 16);
  hipLaunchKernelGGL(train::gla_e_kernel, grid, dim3(NTHR), 0, s, p, gw);
  hipLaunchKernelGGL(train::cheb_dscan_kernel, sgrid, dim3(256), 0, s, p, cw);
  hipLaunchKernelGGL(train::gla_bwd_kernel, grid, dim3(train::GB_NTHR), 0, s, p, gw);
  if (solve_) {
    // the solve's backward on dx = alpha du: its dq is added to dq, its dk to dk
    Params pc = p;
    pc.rhs32 = gw.dx;
    pc.fro = const_cast<float*>(fro);
    pc.xo32 = dq_cheb; pc.xo32_acc = 0;
    cw.x = gw.x; cw.dq = dq_cheb; cw.fro = fro;
    cw.dk = static_cast<bf16*>(dk); cw.dk_add = dk_gla;
    cw.dq_out = static_cast<bf16*>(dq); cw.dq_add = dq_gla;
    cw.dgk = gk ? dgk : nullptr;
    cw.bp_lambda = bp_lambda;
    hipLaunchKernelGGL((solve::gka_solve_kernel<true, false, solve::SM_DQ>), grid, dim3(NTHR), 0, s, pc);
    hipLaunchKernelGGL(train::cheb_e_kernel, grid, dim3(train::E_NTHR), 0, s, pc, cw);
    hipLaunchKernelGGL(train::cheb_dscan_kernel, sgrid, dim3(256), 0, s, pc, cw);
    hipLaunchKernelGGL(train::cheb_dk_kernel, grid, dim3(train::C_NTHR), 0, s, pc, cw);
  }
  return check_launch("hmx_gka_train_bwd");
}
