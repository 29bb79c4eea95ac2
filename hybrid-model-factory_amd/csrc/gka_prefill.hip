// GKA (Gated KalmaNet) chunked prefill: per-token Chebyshev ridge solve against
// the running key Gram matrix H (h_kk), alpha blend, and beta^2-weighted gated
// linear attention over the value state S (h_kv); bf16 q/k/v, fp32 states.
//
// Semantics (per token t, head h; reference files under
// vllm-inference/src/primed_vllm/gka/):
//   q, k <- q/|q|, k/|k| (no eps)                          gka_forward.py:114-159
//   k~ = (beta+1e-6) k
//   H_t = e^{Gk_t} H_c + sum_{j<=t} e^{Gk_t-Gk_j} k~_j k~_j^T  chebyshev_prefill_gqa.py:28-106
//   f_t = |H_t|_F (closed form, :227-235); lam = r f; tau = 2/(2lam+f);
//   c = (f/(2lam+f)/2)^2; x = tau q; num_iter x { w <- 1/(1-cw);
//   x, x_prev <- w x - tau w (H_t x + lam x - q) - (w-1) x_prev, x }  :243-263
//   q <- q + alpha (x - q)                                  gka_forward.py:225
//   o_t = scale [e^{G_t} q^T S_c + sum_{j<=t} e^{G_t-G_j} (q.k_j)(beta_j+1e-6)^2 v_j]
//                                                           ops/chunk_o_gqa.py:25-114
//   S_{c+1} = e^{G_last} S_c + K^T (e^{G_last-G} (beta+1e-6)^2 V)   chunk_simple_gla_gqa.py:33-101
//   H_{c+1} = e^{Gk_last} H_c + K~^T (e^{Gk_last-Gk} K~)
//
// Decomposition.  One 256-thread workgroup per (segment, head) walks 32-token
// chunks with H and S in MFMA accumulator registers (wave w owns columns
// [32w, 32w+32) of both).  Both state recurrences are linear with a scalar
// decay, so a segment's start state is exact from a scalar-decay combine of the
// other segments' zero-start end states (pass LOCAL + combine), no transition
// matrices needed.
//
// Numerics.  Raw k stays exact in bf16; the L2 normalisation and (beta+1e-6)
// become fp32 per-token scales folded into fp32 epilogues or into B operands
// that are then split into bf16 hi + lo.  The Chebyshev iterate and H are used
// as hi/lo pairs in the solver's products; the GLA output uses bf16 operands.
//
// Roofline: MFMA-bound at num_iter >= 8 (2*num_iter*(C*d^2 + 2*C^2*d) flops per
// chunk-head for the solver) plus the HBM minimum (q,k,v,o bf16 + gates +
// states).
#include "common.hpp"
#include "mfma.hpp"

namespace hmx {
namespace gkap {

constexpr int C = 32;           // tokens per chunk
constexpr int MT = C / 16;
constexpr int D = 128;
#ifndef HMX_GKA_WAVES
#define HMX_GKA_WAVES 8
#endif
constexpr int NW = HMX_GKA_WAVES;   // waves per workgroup (one workgroup per CU)
constexpr int NTHR = 64 * NW;
constexpr int CW = D / NW;          // state columns owned by one wave
constexpr int NCT = CW / 16;        // 16-column tiles per wave
constexpr int RPP = NTHR / 16;      // chunk rows staged per pass (16 lanes per row)
constexpr int NPASS = C / RPP;      // staging passes per chunk
static_assert(NW == 4 || NW == 8, "4 or 8 waves");
constexpr int LDQ = D + 8;      // bf16 [C][D] row stride (q, k, v, O)
constexpr int LDX = C + 8;      // bf16 [D][C] row stride (X^T hi/lo, Q^T)
constexpr int LDZ = C + 8;      // bf16 [C][C] row stride (Z, A2)
constexpr int LDK = C + 1;      // fp32 [C][C] (scaled k.k Gram)
constexpr float EPS = 1e-6f;

enum Mode { MODE_OUT = 0, MODE_LOCAL = 1 };

// LDS layout (bytes)
constexpr int SZ_Q = C * LDQ * 2;   // 8704
constexpr int SZ_XT = D * LDX * 2;  // 10240
constexpr int SZ_Z = C * LDZ * 2;   // 2560
constexpr int OFF_Q = 0;
constexpr int OFF_K = OFF_Q + SZ_Q;
constexpr int OFF_V = OFF_K + SZ_Q;
constexpr int OFF_O = OFF_V + SZ_Q;
constexpr int OFF_XH = OFF_O + SZ_Q;
constexpr int OFF_XL = OFF_XH + SZ_XT;
constexpr int OFF_ZH = OFF_XL + SZ_XT;
constexpr int OFF_ZL = OFF_ZH + SZ_Z;
constexpr int OFF_KK = OFF_ZL + SZ_Z;              // fp32 [C][LDK]
constexpr int OFF_S = OFF_KK + C * LDK * 4;         // fp32 per-token scalars
constexpr int NSC = 25;                             // scalar arrays of C floats
constexpr int OFF_NW = OFF_S + NSC * C * 4;        // fp32 [D] output-norm weight (NORM)
constexpr int SMEM = OFF_NW + D * 4;
static_assert(SMEM <= 80 * 1024, "LDS budget");
// per-token scalar array indices
enum { S_G, S_GK, S_EG, S_EGK, S_EDL, S_EDLK, S_BE, S_SK, S_IQ, S_ALPHA, S_KN2, S_QN2,
       S_U0 };                                        // S_U0 .. S_U0 + NW - 1: per-wave u partials
constexpr int S_F0 = S_U0 + NW, S_F1 = S_F0 + 1, S_TAU = S_F1 + 1, S_LAM = S_TAU + 1,
              S_CC = S_LAM + 1;
static_assert(S_CC < NSC, "scalar slots");

struct SegInfo { int n, bos, eos, c_start, c_end, seg_idx, first_seg, nseg; };

// A state pool: slots of [H, D, D] states, ss elements apart, f32 or bf16; `in`
// and `out` may be the same pool (read at the start, written at the end).
struct Pool {
  const void* in; void* out; int64_t ss; int dt;
};

__device__ __forceinline__ float pool_ld(const Pool& pl, int64_t i) {
  return pl.dt == HMX_BF16 ? (float)static_cast<const bf16*>(pl.in)[i]
                           : static_cast<const float*>(pl.in)[i];
}

__device__ __forceinline__ void pool_st(const Pool& pl, int64_t i, float x) {
  if (pl.dt == HMX_BF16) static_cast<bf16*>(pl.out)[i] = (bf16)x;
  else static_cast<float*>(pl.out)[i] = x;
}

struct Params {
  const bf16* q; const bf16* k; const bf16* v;
  int64_t q_ts, kv_ts;                    // token strides (elements; k and v share one)
  const void* alpha; int alpha_dt;
  const void* g; int g_dt;
  const void* gk; int gk_dt;       // null: no h_kk decay
  const void* beta; int beta_dt;   // null: no beta
  bf16* o;
  // Sequence n's states: slot sidx[n] (or n) of the h_kk / h_kv pools; a negative
  // slot or hinit[n] == 0 starts from zero, and a negative slot writes nothing.
  // Only the combine launch and single-segment workgroups read the pools, so the
  // last segment may write its end state straight into the slot.
  Pool hkk, hkv;
  const int* sidx;                        // [N] or null
  const uint8_t* hinit;                   // [N] or null
  const int* seg; int nseg_total;
  float* ws_dh; float* ws_ds;             // [nseg][H][D][D] zero-start segment end states
  float* ws_dec;                          // [nseg][H][2]: sum gk, sum g over the segment
  float* ws_h0; float* ws_s0;             // [nseg][H][D][D] segment start states
  int H, HKV, num_iter;
  float ridge_ratio, scale;
  int l2norm;                             // 0: q, k are used as given
  // optional gated RMSNorm of each output row (NORM kernels)
  const bf16* zg; int64_t zg_ts, zg_hs;   // gate rows, or null (plain RMSNorm)
  const void* onw; int onw_dt;            // weight [D]
  float on_eps;
};

__device__ __forceinline__ float ldsc(const void* p, int64_t i, int dt) {
  if (dt == HMX_F32) return static_cast<const float*>(p)[i];
  if (dt == HMX_BF16) return (float)static_cast<const bf16*>(p)[i];
  return (float)static_cast<const f16*>(p)[i];
}

__device__ __forceinline__ SegInfo load_seg(const int* seg, int s) {
  const int* r = seg + s * 8;
  return SegInfo{r[0], r[1], r[2], r[3], r[4], r[5], r[6], r[7]};
}

// One [D][D] state into accumulator tiles (rows 16rt+4q4+v, columns CW wave +
// 16ct + l16): from fp32 workspace, or from a pool slot (f32 or bf16), or zeros.
// (The pool comes by value: a pointer into the kernel's argument struct would move
// the whole struct to scratch.)
__device__ __forceinline__ void load_state(f32x4 (&X)[8][NCT], const float* ws, bool use_pool,
                                           Pool pl, int64_t slot, int64_t hoff, int wave, int q4,
                                           int l16) {
#define HMX_GKA_STATE_LOOP(EXPR)                                                   \
  _Pragma("unroll") for (int rt = 0; rt < 8; ++rt)                                \
  _Pragma("unroll") for (int ct = 0; ct < NCT; ++ct)                              \
  _Pragma("unroll") for (int v = 0; v < 4; ++v) {                                 \
    const int off = (16 * rt + 4 * q4 + v) * D + CW * wave + 16 * ct + l16;      \
    X[rt][ct][v] = (EXPR);                                                        \
  }
  if (ws) {
    HMX_GKA_STATE_LOOP(ws[off])
  } else if (use_pool && pl.dt == HMX_BF16) {
    const bf16* b = static_cast<const bf16*>(pl.in) + slot * pl.ss + hoff;
    HMX_GKA_STATE_LOOP((float)b[off])
  } else if (use_pool) {
    const float* f = static_cast<const float*>(pl.in) + slot * pl.ss + hoff;
    HMX_GKA_STATE_LOOP(f[off])
  } else {
    HMX_GKA_STATE_LOOP(0.f)
  }
#undef HMX_GKA_STATE_LOOP
}

// One [D][D] state from accumulator tiles into a pool slot (f32 or bf16), or
// zeros into it (clear).
__device__ __forceinline__ void store_state(const f32x4 (&X)[8][NCT], Pool pl, int64_t slot,
                                            int64_t hoff, int wave, int q4, int l16, bool clear) {
#define HMX_GKA_STORE_LOOP(STMT)                                                   \
  _Pragma("unroll") for (int rt = 0; rt < 8; ++rt)                                \
  _Pragma("unroll") for (int ct = 0; ct < NCT; ++ct)                              \
  _Pragma("unroll") for (int v = 0; v < 4; ++v) {                                 \
    const int off = (16 * rt + 4 * q4 + v) * D + CW * wave + 16 * ct + l16;      \
    const float x = clear ? 0.f : X[rt][ct][v];                                   \
    STMT;                                                                         \
  }
  if (pl.dt == HMX_BF16) {
    bf16* b = static_cast<bf16*>(pl.out) + slot * pl.ss + hoff;
    HMX_GKA_STORE_LOOP(b[off] = (bf16)x)
  } else {
    float* f = static_cast<float*>(pl.out) + slot * pl.ss + hoff;
    HMX_GKA_STORE_LOOP(f[off] = x)
  }
#undef HMX_GKA_STORE_LOOP
}

struct Raw {
  bf16x8 k[NPASS], v[NPASS], q[NPASS];
  float g, gk, b, a;
};

template <int MODE>
__device__ __forceinline__ void load_raw(Raw& r, const Params& p, const bf16* qh, const bf16* kh,
                                         const bf16* vh, int tok0, int nval, int tid, int h) {
#pragma unroll
  for (int pass = 0; pass < NPASS; ++pass) {
    const int row = pass * RPP + (tid >> 4), f0 = (tid & 15) * 8;
    const bool ok = row < nval;
    const int64_t tok = tok0 + row;
    r.k[pass] = ok ? *reinterpret_cast<const bf16x8*>(kh + tok * p.kv_ts + f0) : bf16x8{};
    r.v[pass] = ok ? *reinterpret_cast<const bf16x8*>(vh + tok * p.kv_ts + f0) : bf16x8{};
    if (MODE == MODE_OUT)
      r.q[pass] = ok ? *reinterpret_cast<const bf16x8*>(qh + tok * p.q_ts + f0) : bf16x8{};
  }
  if (tid < C) {
    const bool ok = tid < nval;
    const int64_t i = (int64_t)(tok0 + tid) * p.H + h;
    r.g = ok ? ldsc(p.g, i, p.g_dt) : 0.f;
    r.gk = (ok && p.gk) ? ldsc(p.gk, i, p.gk_dt) : 0.f;
    r.b = (ok && p.beta) ? ldsc(p.beta, i, p.beta_dt) : 0.f;
    r.a = (ok && MODE == MODE_OUT) ? ldsc(p.alpha, i, p.alpha_dt) : 0.f;
  }
}

// Sum of squares of a staged 8-feature slice over its 16-lane row.
__device__ __forceinline__ float row_sumsq(const bf16x8& x) {
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) s += (float)x[j] * (float)x[j];
  return row16_sum(s);
}

// Writes a C-layout 16x16 register tile transposed (M^T[col][row]) as bf16 hi/lo,
// 4 consecutive rows per lane -> one 8-byte store each.
__device__ __forceinline__ void put_t_hilo(bf16* th, bf16* tl, int ld, int r0, int c0,
                                           const f32x4& x, int q4, int l16) {
  bf16x4 hi, lo;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    hi[v] = (bf16)x[v];
    lo[v] = (bf16)(x[v] - (float)hi[v]);
  }
  const int a = (c0 + l16) * ld + r0 + 4 * q4;
  *reinterpret_cast<bf16x4*>(th + a) = hi;
  if (tl) *reinterpret_cast<bf16x4*>(tl + a) = lo;
}

// One workgroup per CU: NW / 4 waves per SIMD (the second bound is waves per SIMD).
// NORM: the output rows pass through the gated RMSNorm of hmx_rms_norm_gated (norm
// before gate) on their way out of sO.
template <int MODE, bool NORM = false>
__global__ __launch_bounds__(NTHR, NW / 4) void gka_chunk_kernel(Params p) {
  __shared__ __align__(16) unsigned char smem[SMEM];
  bf16* sQ = reinterpret_cast<bf16*>(smem + OFF_Q);
  bf16* sK = reinterpret_cast<bf16*>(smem + OFF_K);
  bf16* sV = reinterpret_cast<bf16*>(smem + OFF_V);
  bf16* sO = reinterpret_cast<bf16*>(smem + OFF_O);
  bf16* sXh = reinterpret_cast<bf16*>(smem + OFF_XH);
  bf16* sXl = reinterpret_cast<bf16*>(smem + OFF_XL);
  bf16* sZh = reinterpret_cast<bf16*>(smem + OFF_ZH);
  bf16* sZl = reinterpret_cast<bf16*>(smem + OFF_ZL);
  float* sKK = reinterpret_cast<float*>(smem + OFF_KK);
  float* sc = reinterpret_cast<float*>(smem + OFF_S);
  auto SC = [&](int slot, int t) -> float& { return sc[slot * C + t]; };

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q4 = lane >> 4, l16 = lane & 15;
  const int s_id = blockIdx.x, h = blockIdx.y;
  const SegInfo si = load_seg(p.seg, s_id);
  const int H = p.H, hk = h / (H / p.HKV);
  const bool solve = (MODE == MODE_OUT) && p.num_iter > 0;
  const bool track_h = p.num_iter > 0;

  if (MODE == MODE_LOCAL && si.seg_idx == si.nseg - 1) return;
  if (NORM && tid < D) {
    float wv;
    if (p.onw_dt == HMX_F32) wv = static_cast<const float*>(p.onw)[tid];
    else if (p.onw_dt == HMX_BF16) wv = (float)static_cast<const bf16*>(p.onw)[tid];
    else wv = (float)static_cast<const f16*>(p.onw)[tid];
    reinterpret_cast<float*>(smem + OFF_NW)[tid] = wv;   // read after the chunk's barriers
  }

  // ---- initial states ----------------------------------------------------
  // A split sequence's segments (its first included) start from the workspace
  // the combine launch filled; a single-segment sequence reads its pool slot.
  const int64_t slot = p.sidx ? (int64_t)p.sidx[si.n] : si.n;
  const int64_t hoff = (int64_t)h * D * D;
  f32x4 Hs[8][NCT], Ss[8][NCT];
  {
    const float *hsrc = nullptr, *ssrc = nullptr;
    bool pooled = false;
    if (MODE == MODE_OUT) {
      if (si.nseg == 1) {
        pooled = slot >= 0 && (!p.hinit || p.hinit[si.n]);
      } else {
        hsrc = p.ws_h0 + ((int64_t)s_id * H + h) * D * D;
        ssrc = p.ws_s0 + ((int64_t)s_id * H + h) * D * D;
      }
    }
    // h_kk then h_kv, each from one source chosen by a uniform branch (a per-element
    // choice costs registers)
    load_state(Hs, hsrc && track_h ? hsrc : nullptr, pooled && track_h && p.hkk.in, p.hkk, slot,
               hoff, wave, q4, l16);
    load_state(Ss, ssrc, pooled && p.hkv.in, p.hkv, slot, hoff, wave, q4, l16);
  }

  const int64_t o_rs = (int64_t)H * D;
  const bf16* qh = p.q + (int64_t)h * D;
  const bf16* kh = p.k + (int64_t)hk * D;
  const bf16* vh = p.v + (int64_t)hk * D;
  float seg_gk = 0.f, seg_g = 0.f;

  Raw raw;
  if (si.c_start < si.c_end)
    load_raw<MODE>(raw, p, qh, kh, vh, si.bos + si.c_start * C,
                   min(C, si.eos - (si.bos + si.c_start * C)), tid, h);

  for (int c = si.c_start; c < si.c_end; ++c) {
    const int tok0 = si.bos + c * C;
    const int nval = min(C, si.eos - tok0);

    // ---- P0: stage raw rows, row norms, per-token gates ---------------------
#pragma unroll
    for (int pass = 0; pass < NPASS; ++pass) {
      const int row = pass * RPP + (tid >> 4), f0 = (tid & 15) * 8;
      *reinterpret_cast<bf16x8*>(sK + row * LDQ + f0) = raw.k[pass];
      *reinterpret_cast<bf16x8*>(sV + row * LDQ + f0) = raw.v[pass];
      const float kn2 = row_sumsq(raw.k[pass]);
      if ((tid & 15) == 0) SC(S_KN2, row) = kn2;
      if (MODE == MODE_OUT) {
        *reinterpret_cast<bf16x8*>(sQ + row * LDQ + f0) = raw.q[pass];
        const float qn2 = row_sumsq(raw.q[pass]);
        if ((tid & 15) == 0) SC(S_QN2, row) = qn2;
      }
    }
    if (wave == 0) {
      const bool ok = lane < C;
      const float G = scan32(ok ? raw.g : 0.f);
      const float Gk = scan32(ok ? raw.gk : 0.f);
      const float GL = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, G), C - 1));
      const float GkL = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, Gk), C - 1));
      if (ok) {
        SC(S_G, lane) = G;
        SC(S_GK, lane) = Gk;
        SC(S_EG, lane) = fast_exp(G);
        SC(S_EGK, lane) = fast_exp(Gk);
        SC(S_EDL, lane) = fast_exp(GL - G);
        SC(S_EDLK, lane) = fast_exp(GkL - Gk);
        SC(S_BE, lane) = p.beta ? raw.b + EPS : 1.0f;
        SC(S_ALPHA, lane) = raw.a;
      }
      seg_g += GL;
      seg_gk += GkL;
    }
    if (c + 1 < si.c_end) {
      const int t1 = tok0 + C;
      load_raw<MODE>(raw, p, qh, kh, vh, t1, min(C, si.eos - t1), tid, h);
    }
    lds_barrier();
    // per-token scales: s_t = (beta_t+eps)/|k_t| (k~ = s k), iq_t = 1/|q_t|
    // (without in-kernel normalisation: s_t = beta_t+eps or 1, iq_t = 1)
    if (tid < C) {
      const float kn2 = SC(S_KN2, tid);
      SC(S_SK, tid) = tid < nval ? SC(S_BE, tid) * (p.l2norm ? 1.0f / sqrtf(kn2) : 1.f) : 0.f;
      if (MODE == MODE_OUT)
        SC(S_IQ, tid) = tid < nval ? (p.l2norm ? 1.0f / sqrtf(SC(S_QN2, tid)) : 1.f) : 0.f;
    }

    lds_barrier();
    // q^ for this wave's columns (C layout), fp32
    f32x4 qv[MT][NCT];
    if (MODE == MODE_OUT) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int t = 16 * mt + 4 * q4 + v;
            qv[mt][ct][v] = (float)sQ[t * LDQ + CW * wave + 16 * ct + l16] * SC(S_IQ, t);
          }
    }

    // ---- P1: the Chebyshev solve (OUT, num_iter > 0) -------------------------
    f32x4 xq[MT][NCT];  // the query fed to the GLA (solved + alpha-blended, or q^)
    if (MODE == MODE_OUT) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) xq[mt][ct] = qv[mt][ct];
    }
    if (solve) {
      // P1a: u_j = k~_j H_c k~_j^T (per-wave partials), |H_c|^2, scaled Gram k~.k~
      {
        float u[MT][4];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int v = 0; v < 4; ++v) u[mt][v] = 0.f;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          bf16x8 Hh[NCT], Hl[NCT];
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) pack_b_hilo(Hs[2 * ks][ct], Hs[2 * ks + 1][ct], Hh[ct], Hl[ct]);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const bf16x8 a = frag_perm(sK, LDQ, 16 * mt, 32 * ks, lane);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
              f32x4 acc = {0.f, 0.f, 0.f, 0.f};
              acc = mfma16(a, Hh[ct], acc);
              acc = mfma16(a, Hl[ct], acc);
#pragma unroll
              for (int v = 0; v < 4; ++v)
                u[mt][v] += acc[v] *
                            (float)sK[(16 * mt + 4 * q4 + v) * LDQ + CW * wave + 16 * ct + l16];
            }
          }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float s = row16_sum(u[mt][v]);
            if (l16 == 0) SC(S_U0 + wave, 16 * mt + 4 * q4 + v) = s;
          }
        float hn = 0.f;
#pragma unroll
        for (int rt = 0; rt < 8; ++rt)
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
            for (int v = 0; v < 4; ++v) hn += Hs[rt][ct][v] * Hs[rt][ct][v];
        hn = wave_sum(hn);
        if (lane == 0) SC(S_F0, C - 1 - wave) = hn;  // |H_c|^2 partials in the F0 tail
        // Gram tiles (0,0), (1,0), (1,1) on waves 0..2: sKK[t][j] = s_t s_j k_t.k_j
        if (wave < 3) {
          const int a = (wave == 0) ? 0 : 1, b = (wave == 2) ? 1 : 0;
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks)
            acc = mfma16(frag(sK, LDQ, 16 * a, 32 * ks, lane), frag(sK, LDQ, 16 * b, 32 * ks, lane), acc);
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int t = 16 * a + 4 * q4 + v, j = 16 * b + l16;
            sKK[t * LDK + j] = acc[v] * SC(S_SK, t) * SC(S_SK, j);
          }
        }
      }
      lds_barrier();
      // P1b: in-chunk part of |H_t|_F^2 = sum_l M_tl (M . KK^2)_tl, M_tj = e^{Gk_t-Gk_j} (t>=j)
      float hc2 = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) hc2 += SC(S_F0, C - 1 - w);
      lds_barrier();
      if (wave < 3) {
        const int a = (wave == 0) ? 0 : 1, b = (wave == 2) ? 1 : 0;
        f32x4 R = {0.f, 0.f, 0.f, 0.f};
        // R_tl = sum_j M_tj KK_jl^2 over j <= t (KK symmetric; only j >= l contributes via M? no:
        // every j <= t contributes); k in natural order j = 4s + q (two 16-blocks)
        for (int jb = 0; jb <= a; ++jb) {
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int t = 16 * a + l16, j = 16 * jb + 4 * s + q4, l = 16 * b + l16;
            const float m = (t >= j) ? fast_exp(SC(S_GK, t) - SC(S_GK, j)) : 0.f;
            const float kk = (j >= l) ? sKK[j * LDK + l] : sKK[l * LDK + j];
            R = mfma16f(m, kk * kk, R);
          }
        }
        float fp[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int t = 16 * a + 4 * q4 + v, l = 16 * b + l16;
          const float m = (t >= l) ? fast_exp(SC(S_GK, t) - SC(S_GK, l)) : 0.f;
          fp[v] = row16_sum(R[v] * m);
        }
        if (l16 == 0) {
#pragma unroll
          for (int v = 0; v < 4; ++v) SC(b == 0 ? S_F0 : S_F1, 16 * a + 4 * q4 + v) = fp[v];
        }
        if (a == 0 && l16 == 0) {
#pragma unroll
          for (int v = 0; v < 4; ++v) SC(S_F1, 4 * q4 + v) = 0.f;  // tile (0,1) is empty
        }
      }
      lds_barrier();
      // P1c: per-token f, lam, tau, c
      if (tid < C) {
        const int t = tid;
        float cross = 0.f;
        for (int j = 0; j <= t; ++j) {
          float usum = 0.f;
#pragma unroll
          for (int w = 0; w < NW; ++w) usum += SC(S_U0 + w, j);
          const float uj = usum * SC(S_SK, j) * SC(S_SK, j);
          cross += fast_exp(SC(S_GK, t) - SC(S_GK, j)) * uj;
        }
        const float egk = SC(S_EGK, t);
        const float f2 = egk * egk * hc2 + 2.f * egk * cross + SC(S_F0, t) + SC(S_F1, t);
        const float f = sqrtf(f2);
        const float lam = p.ridge_ratio * f;
        const float inv = 1.0f / (2.f * lam + f);
        SC(S_TAU, t) = 2.f * inv;
        SC(S_LAM, t) = lam;
        const float cc = f * inv * 0.5f;
        SC(S_CC, t) = cc * cc;
      }
      lds_barrier();

      // P1d: the iteration.  Each wave owns X[:, 32w..32w+32) in registers.
      float tau[MT][4], lam[MT][4], ccv[MT][4], om[MT][4];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int t = 16 * mt + 4 * q4 + v;
          tau[mt][v] = SC(S_TAU, t);
          lam[mt][v] = SC(S_LAM, t);
          ccv[mt][v] = SC(S_CC, t);
          om[mt][v] = 2.0f;
        }
      f32x4 X[MT][NCT], Xp[MT][NCT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            X[mt][ct][v] = tau[mt][v] * qv[mt][ct][v];
            Xp[mt][ct][v] = 0.f;
          }
        }
      // Z~ weights M_tj s_j^2 (j <= t) of this wave's tile, fixed over the iterations
      f32x4 zw = {0.f, 0.f, 0.f, 0.f};
      if (wave < 3) {
        const int a = (wave == 0) ? 0 : 1, b = (wave == 2) ? 1 : 0;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int t = 16 * a + 4 * q4 + v, j = 16 * b + l16;
          const float sj = SC(S_SK, j);
          zw[v] = (t >= j) ? sj * sj * fast_exp(SC(S_GK, t) - SC(S_GK, j)) : 0.f;
        }
      }
      for (int it = 0; it < p.num_iter; ++it) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct)
            put_t_hilo(sXh, sXl, LDX, 16 * mt, CW * wave + 16 * ct, X[mt][ct], q4, l16);
        lds_barrier();
        // Z~_tj = M_tj s_j^2 (x_t . k_j) for j <= t on waves 0..2
        if (wave < 3) {
          const int a = (wave == 0) ? 0 : 1, b = (wave == 2) ? 1 : 0;
          f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            const bf16x8 bk = frag(sK, LDQ, 16 * b, 32 * ks, lane);
            z = mfma16(frag_t(sXh, LDX, 32 * ks, 16 * a, lane), bk, z);
            z = mfma16(frag_t(sXl, LDX, 32 * ks, 16 * a, lane), bk, z);
          }
          f32x4 zs;
#pragma unroll
          for (int v = 0; v < 4; ++v) zs[v] = z[v] * zw[v];
          // store Z~ row-major (t, j): 2-byte writes
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int t = 16 * a + 4 * q4 + v, j = 16 * b + l16;
            const bf16 hi = (bf16)zs[v];
            sZh[t * LDZ + j] = hi;
            sZl[t * LDZ + j] = (bf16)(zs[v] - (float)hi);
          }
        } else if (wave == 3) {
          // wave 3 zeroes the empty upper tile (0,1)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            sZh[(4 * q4 + v) * LDZ + 16 + l16] = (bf16)0.f;
            sZl[(4 * q4 + v) * LDZ + 16 + l16] = (bf16)0.f;
          }
        }
        // Y = e^{Gk} (X H_c) for this wave's columns (X, H as hi/lo)
        f32x4 Y[MT][NCT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) Y[mt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          bf16x8 Hh[NCT], Hl[NCT];
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) pack_b_hilo(Hs[2 * ks][ct], Hs[2 * ks + 1][ct], Hh[ct], Hl[ct]);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const bf16x8 ah = frag_t_perm(sXh, LDX, 32 * ks, 16 * mt, lane);
            const bf16x8 al = frag_t_perm(sXl, LDX, 32 * ks, 16 * mt, lane);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
              Y[mt][ct] = mfma16(ah, Hh[ct], Y[mt][ct]);
              Y[mt][ct] = mfma16(ah, Hl[ct], Y[mt][ct]);
              Y[mt][ct] = mfma16(al, Hh[ct], Y[mt][ct]);
            }
          }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float e = SC(S_EGK, 16 * mt + 4 * q4 + v);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) Y[mt][ct][v] *= e;
          }
        lds_barrier();
        // Y += Z~ K (Z~ hi/lo, raw K exact)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
          const bf16x8 bk = frag_t(sK, LDQ, 0, CW * wave + 16 * ct, lane);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            Y[mt][ct] = mfma16(frag(sZh, LDZ, 16 * mt, 0, lane), bk, Y[mt][ct]);
            Y[mt][ct] = mfma16(frag(sZl, LDZ, 16 * mt, 0, lane), bk, Y[mt][ct]);
          }
        }
        // Chebyshev update
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            // w <= 2 (c <= 1/4, omega <= 2): the hardware reciprocal (1 ulp) suffices
            const float w = __builtin_amdgcn_rcpf(1.0f - ccv[mt][v] * om[mt][v]);
            om[mt][v] = w;
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
              const float x = X[mt][ct][v];
              const float grad = tau[mt][v] * w * (Y[mt][ct][v] + lam[mt][v] * x - qv[mt][ct][v]) +
                                 (w - 1.0f) * Xp[mt][ct][v];
              Xp[mt][ct][v] = x;
              X[mt][ct][v] = w * x - grad;
            }
          }
      }
      // alpha blend
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float al = SC(S_ALPHA, 16 * mt + 4 * q4 + v);
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct)
            xq[mt][ct][v] = qv[mt][ct][v] + al * (X[mt][ct][v] - qv[mt][ct][v]);
        }
    }

    // ---- P2: GLA output (OUT) ------------------------------------------------
    if (MODE == MODE_OUT) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
          put_t_hilo(sXh, sXl, LDX, 16 * mt, CW * wave + 16 * ct, xq[mt][ct], q4, l16);
      lds_barrier();
      // A2_tj = e^{G_t-G_j} (xq_t . k_j) s_j (beta_j+eps)  (j <= t), waves 0..2
      if (wave < 3) {
        const int a = (wave == 0) ? 0 : 1, b = (wave == 2) ? 1 : 0;
        f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16x8 bk = frag(sK, LDQ, 16 * b, 32 * ks, lane);
          z = mfma16(frag_t(sXh, LDX, 32 * ks, 16 * a, lane), bk, z);
          z = mfma16(frag_t(sXl, LDX, 32 * ks, 16 * a, lane), bk, z);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int t = 16 * a + 4 * q4 + v, j = 16 * b + l16;
          const float w = (t >= j) ? fast_exp(SC(S_G, t) - SC(S_G, j)) * SC(S_SK, j) * SC(S_BE, j) : 0.f;
          sZh[t * LDZ + j] = (bf16)(z[v] * w);
        }
      } else if (wave == 3) {
#pragma unroll
        for (int v = 0; v < 4; ++v) sZh[(4 * q4 + v) * LDZ + 16 + l16] = (bf16)0.f;
      }
      f32x4 O[MT][NCT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) O[mt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        // The solved query is large off the key span, so both operands carry a
        // bf16 remainder: a single bf16 rounding of either costs ~3% of |o|.
        bf16x8 Sh[NCT], Sl[NCT];
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) pack_b_hilo(Ss[2 * ks][ct], Ss[2 * ks + 1][ct], Sh[ct], Sl[ct]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const bf16x8 ah = frag_t_perm(sXh, LDX, 32 * ks, 16 * mt, lane);
          const bf16x8 al = frag_t_perm(sXl, LDX, 32 * ks, 16 * mt, lane);
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) {
            O[mt][ct] = mfma16(ah, Sh[ct], O[mt][ct]);
            O[mt][ct] = mfma16(al, Sh[ct], O[mt][ct]);
            O[mt][ct] = mfma16(ah, Sl[ct], O[mt][ct]);
          }
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float e = SC(S_EG, 16 * mt + 4 * q4 + v);
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) O[mt][ct][v] *= e;
        }
      lds_barrier();
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const bf16x8 bv = frag_t(sV, LDQ, 0, CW * wave + 16 * ct, lane);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) O[mt][ct] = mfma16(frag(sZh, LDZ, 16 * mt, 0, lane), bv, O[mt][ct]);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            sO[(16 * mt + 4 * q4 + v) * LDQ + CW * wave + 16 * ct + l16] = (bf16)(O[mt][ct][v] * p.scale);
    }

    // ---- P3: state updates (hi/lo B operands); the output-norm gate is loaded
    // here, a phase before the O store uses it ---------------------------------
    bf16x8 zr[NPASS];
    if constexpr (NORM) {
#pragma unroll
      for (int pass = 0; pass < NPASS; ++pass) {
        const int row = pass * RPP + (tid >> 4);
        zr[pass] = (p.zg && row < nval)
                       ? *reinterpret_cast<const bf16x8*>(p.zg + (int64_t)(tok0 + row) * p.zg_ts +
                                                          (int64_t)h * p.zg_hs + (tid & 15) * 8)
                       : bf16x8{};
      }
    }
    {
      const float egl = SC(S_EG, C - 1), egkl = SC(S_EGK, C - 1);
#pragma unroll
      for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            Ss[rt][ct][v] *= egl;
            if (track_h) Hs[rt][ct][v] *= egkl;
          }
      float fs[8], fh[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int t = 8 * q4 + j;
        const float s = SC(S_SK, t);
        fs[j] = s * SC(S_BE, t) * SC(S_EDL, t);
        fh[j] = s * s * SC(S_EDLK, t);
      }
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const bf16x8 vr = frag_t(sV, LDQ, 0, CW * wave + 16 * ct, lane);
        const bf16x8 kr = frag_t(sK, LDQ, 0, CW * wave + 16 * ct, lane);
        bf16x8 vh, vl, kh_, kl_;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float x = (float)vr[j] * fs[j];
          vh[j] = (bf16)x;
          vl[j] = (bf16)(x - (float)vh[j]);
          const float y = (float)kr[j] * fh[j];
          kh_[j] = (bf16)y;
          kl_[j] = (bf16)(y - (float)kh_[j]);
        }
#pragma unroll
        for (int rt = 0; rt < 8; ++rt) {
          const bf16x8 a = frag_t(sK, LDQ, 0, 16 * rt, lane);
          Ss[rt][ct] = mfma16(a, vh, Ss[rt][ct]);
          Ss[rt][ct] = mfma16(a, vl, Ss[rt][ct]);
          if (track_h) {
            Hs[rt][ct] = mfma16(a, kh_, Hs[rt][ct]);
            Hs[rt][ct] = mfma16(a, kl_, Hs[rt][ct]);
          }
        }
      }
    }
    lds_barrier();

    // ---- store O (NORM: out = o / sqrt(mean(o^2) + eps) * w * silu(z) per row) -
    if (MODE == MODE_OUT) {
      bf16* oh = p.o + (int64_t)h * D;
#pragma unroll
      for (int pass = 0; pass < NPASS; ++pass) {
        const int row = pass * RPP + (tid >> 4), f0 = (tid & 15) * 8;
        bf16x8 ov = *reinterpret_cast<const bf16x8*>(sO + row * LDQ + f0);
        if constexpr (NORM) {
          const float* sNW = reinterpret_cast<const float*>(smem + OFF_NW);
          float f[8], ss = 0.f;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            f[j] = (float)ov[j];
            ss += f[j] * f[j];
          }
          const float rstd = 1.0f / sqrtf(row16_sum(ss) * (1.0f / D) + p.on_eps);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            float y = f[j] * rstd * sNW[f0 + j];
            if (p.zg) {
              const float z = (float)zr[pass][j];
              y *= z * __builtin_amdgcn_rcpf(1.0f + fast_exp(-z));
            }
            ov[j] = (bf16)y;
          }
        }
        if (row < nval) *reinterpret_cast<bf16x8*>(oh + (int64_t)(tok0 + row) * o_rs + f0) = ov;
      }
    }
  }

  // ---- end states ----------------------------------------------------------
  float *hd = nullptr, *sd = nullptr;
  if (MODE == MODE_OUT) {
    if (si.seg_idx == si.nseg - 1 && slot >= 0) {
      // without the solver (num_iter 0) h_kk is not tracked: a pooled h_kk slot of a
      // sequence without an initial state is cleared, the others keep their value
      if (p.hkk.out && (track_h || (p.hinit && !p.hinit[si.n])))
        store_state(Hs, p.hkk, slot, hoff, wave, q4, l16, !track_h);
      if (p.hkv.out) store_state(Ss, p.hkv, slot, hoff, wave, q4, l16, false);
    }
  } else {
    hd = track_h ? p.ws_dh + ((int64_t)s_id * H + h) * D * D : nullptr;
    sd = p.ws_ds + ((int64_t)s_id * H + h) * D * D;
    if (tid == 0) {
      p.ws_dec[((int64_t)s_id * H + h) * 2 + 0] = seg_gk;
      p.ws_dec[((int64_t)s_id * H + h) * 2 + 1] = seg_g;
    }
  }
#pragma unroll
  for (int rt = 0; rt < 8; ++rt)
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int off = (16 * rt + 4 * q4 + v) * D + CW * wave + 16 * ct + l16;
        if (hd) hd[off] = Hs[rt][ct][v];
        if (sd) sd[off] = Ss[rt][ct][v];
      }
}

// Segment start states: X_0 = initial, X_{s+1} = e^{D_s} X_s + dX_s (elementwise).
__global__ __launch_bounds__(256) void gka_seg_combine_kernel(Params p) {
  const int nh = blockIdx.x, H = p.H;
  const int n = nh / H, h = nh % H;
  int first = -1, nseg = 0;
  for (int s = 0; s < p.nseg_total; ++s) {
    const SegInfo si = load_seg(p.seg, s);
    if (si.n == n) { first = si.first_seg; nseg = si.nseg; break; }
  }
  if (first < 0 || nseg < 2) return;
  const bool track_h = p.num_iter > 0;
  const int64_t slot = p.sidx ? (int64_t)p.sidx[n] : n;
  const bool init = slot >= 0 && (!p.hinit || p.hinit[n]);
  const int64_t hoff = (int64_t)h * D * D;
  for (int e = blockIdx.y * 256 + threadIdx.x; e < D * D; e += gridDim.y * 256) {
    float hx = (track_h && init && p.hkk.in) ? pool_ld(p.hkk, slot * p.hkk.ss + hoff + e) : 0.f;
    float sx = (init && p.hkv.in) ? pool_ld(p.hkv, slot * p.hkv.ss + hoff + e) : 0.f;
    {   // the first segment's start state, so that no OUT workgroup reads the pool
      const int64_t fb = ((int64_t)first * H + h) * D * D + e;
      if (track_h) p.ws_h0[fb] = hx;
      p.ws_s0[fb] = sx;
    }
    for (int s = 0; s < nseg - 1; ++s) {
      const int64_t b = ((int64_t)(first + s) * H + h);
      const float dk = expf(p.ws_dec[b * 2 + 0]), dg = expf(p.ws_dec[b * 2 + 1]);
      if (track_h) hx = hx * dk + p.ws_dh[b * D * D + e];
      sx = sx * dg + p.ws_ds[b * D * D + e];
      const int64_t nb = ((int64_t)(first + s + 1) * H + h) * D * D + e;
      if (track_h) p.ws_h0[nb] = hx;
      p.ws_s0[nb] = sx;
    }
  }
}

}  // namespace gkap
}  // namespace hmx

using namespace hmx;
using namespace hmx::gkap;

extern "C" size_t hmx_gka_chunk_workspace_bytes(int32_t nseg_total, int32_t N, int32_t H) {
  if (nseg_total <= N) return 16;
  const size_t st = (size_t)nseg_total * H * D * D * sizeof(float);
  return 4 * st + (size_t)nseg_total * H * 2 * sizeof(float);
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
                                 int32_t N, int32_t H, int32_t HKV, int32_t D_, int32_t V,
                                 int32_t num_iter, float ridge_ratio, float scale,
                                 int32_t use_qk_l2norm, void* workspace, size_t workspace_bytes,
                                 const hmx_gated_norm* o_norm, void* stream) {
  HMX_REQUIRE(qkv_dtype == HMX_BF16, HMX_EUNSUPPORTED,
              "hmx_gka_chunk_fwd: q/k/v must be bfloat16 (got dtype code %d)", qkv_dtype);
  HMX_REQUIRE(D_ == D && V == D, HMX_EUNSUPPORTED,
              "hmx_gka_chunk_fwd: only D == V == 128 is supported (got D=%d V=%d)", D_, V);
  HMX_REQUIRE(H > 0 && HKV > 0 && H % HKV == 0, HMX_EINVAL, "hmx_gka_chunk_fwd: H/HKV");
  HMX_REQUIRE(q && k && v && alpha && g && o && seg_table, HMX_EINVAL,
              "hmx_gka_chunk_fwd: null tensor pointer");
  HMX_REQUIRE(num_iter >= 0, HMX_EINVAL, "hmx_gka_chunk_fwd: num_iter=%d", num_iter);
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
  const size_t need = hmx_gka_chunk_workspace_bytes(nseg_total, N, H);
  HMX_REQUIRE(workspace && workspace_bytes >= need, HMX_EINVAL,
              "hmx_gka_chunk_fwd: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  Params p;
  p.q = static_cast<const bf16*>(q); p.k = static_cast<const bf16*>(k);
  p.v = static_cast<const bf16*>(v);
  p.alpha = alpha; p.alpha_dt = alpha_dtype; p.g = g; p.g_dt = g_dtype;
  p.gk = gk; p.gk_dt = gk_dtype; p.beta = beta; p.beta_dt = beta_dtype;
  p.zg = nullptr; p.zg_ts = p.zg_hs = 0; p.onw = nullptr; p.onw_dt = HMX_F32; p.on_eps = 0.f;
  if (o_norm) {
    HMX_REQUIRE(o_norm->weight && o_norm->weight_dtype >= 0 && o_norm->weight_dtype <= 2,
                HMX_EINVAL, "hmx_gka_chunk_fwd: o_norm needs a weight (dtype code 0-2)");
    HMX_REQUIRE(!o_norm->gate || ((uintptr_t)o_norm->gate % 16 == 0 &&
                                  o_norm->gate_token_stride % 8 == 0 &&
                                  o_norm->gate_head_stride % 8 == 0),
                HMX_EINVAL, "hmx_gka_chunk_fwd: o_norm gate rows must be 16-byte aligned");
    p.zg = static_cast<const bf16*>(o_norm->gate);
    p.zg_ts = o_norm->gate_token_stride; p.zg_hs = o_norm->gate_head_stride;
    p.onw = o_norm->weight; p.onw_dt = o_norm->weight_dtype; p.on_eps = o_norm->eps;
  }
  p.o = static_cast<bf16*>(o);
  p.q_ts = q_token_stride; p.kv_ts = k_token_stride;
  p.hkk = Pool{h_kk0, h_kk_final, h_kk_slot_stride, h_kk_dtype};
  p.hkv = Pool{h_kv0, h_kv_final, h_kv_slot_stride, h_kv_dtype};
  p.sidx = state_indices; p.hinit = has_initial_state;
  p.seg = seg_table; p.nseg_total = nseg_total;
  p.H = H; p.HKV = HKV; p.num_iter = num_iter; p.ridge_ratio = ridge_ratio; p.scale = scale;
  p.l2norm = use_qk_l2norm;
  const bool multi = nseg_total > N;
  const size_t st = (size_t)nseg_total * H * D * D;
  float* ws = static_cast<float*>(workspace);
  p.ws_dh = multi ? ws : nullptr;
  p.ws_ds = multi ? ws + st : nullptr;
  p.ws_h0 = multi ? ws + 2 * st : nullptr;
  p.ws_s0 = multi ? ws + 3 * st : nullptr;
  p.ws_dec = multi ? ws + 4 * st : nullptr;
  hipStream_t s = (hipStream_t)stream;
  if (multi) {
    hipLaunchKernelGGL(gka_chunk_kernel<MODE_LOCAL>, dim3(nseg_total, H), dim3(NTHR), 0, s, p);
    hipLaunchKernelGGL(gka_seg_combine_kernel, dim3(N * H, 16), dim3(256), 0, s, p);
  }
  if (o_norm)
    hipLaunchKernelGGL((gka_chunk_kernel<MODE_OUT, true>), dim3(nseg_total, H), dim3(NTHR), 0, s, p);
  else
    hipLaunchKernelGGL(gka_chunk_kernel<MODE_OUT>, dim3(nseg_total, H), dim3(NTHR), 0, s, p);
  return check_launch("hmx_gka_chunk_fwd");
}
