// GDN chunked prefill (gated delta rule, WY/UT form), GQA-native, varlen,
// bf16 q/k/v with an fp32 recurrent state, for gfx950.
//
// Semantics: vllm-inference/src/primed_vllm/gdn/ops/chunk_gqa.py:15-83 (the op
// chain l2norm -> chunk cumsum -> KK^T -> (I+A)^-1 -> w,u -> h,v_new -> o), with
// per-chunk maths (C = 64 tokens, G = in-chunk cumsum of g):
//   A_ij = beta_i (k_i.k_j) e^{G_i-G_j} (j<i);  T = (I+A)^-1
//   U = T diag(beta) V;   W = T diag(beta e^G) K
//   V_new = U - W S;      O = scale [e^G (Q S) + tril(Q K^T e^{G_i-G_j}) V_new]
//   S <- e^{G_last} S + K^T (e^{G_last-G} V_new)
//
// Parallel decomposition (segmented chunk scan).  Each sequence's chunks are
// split into segments; one 256-thread workgroup owns one (segment, head) and
// walks its chunks serially with the 128x128 fp32 state held in MFMA
// accumulator registers (wave w owns state columns [32w, 32w+32)).  A segment's
// initial state comes from one of:
//   * the sequence's initial state (first segment);
//   * a warm-up: the chain is re-run from a zero state over the preceding
//     chunks, far enough back that the dropped history is bounded by
//     prod e^{g_t} max(1,|1-beta_t|) < e^{-60} (the transition
//     e^{g}(I - beta k k^T) has spectral norm <= e^{g} max(1,|1-beta|) for
//     |k| <= 1, which in-kernel L2 normalisation guarantees) - exact to fp32;
//   * the exact segment scan when that bound is not reached within a few chunks
//     (weak decay): per-segment zero-start end states S0_s and transitions
//     Phi_s (chain started from I with V = 0), then S_{s+1} = Phi_s S_s + S0_s.
//
// Numerics: MFMA operands are bf16 with fp32 accumulation.  T (with beta and
// beta e^G folded in, so K and V enter exactly) and the decayed V_new of the
// state update are split into bf16 hi + lo pairs, giving ~fp32 accuracy where
// the state is sensitive; W, Q, P and the state as a B operand are bf16.
//
// Roofline: HBM-bound at the algorithmic minimum (q,k,v,o bf16 + g,beta +
// final state); FLOPs 2*T*H*(5*C*d + 3*d^2).
#include "common.hpp"

namespace hmx {
namespace gdnp {

constexpr int C = 64;          // chunk length
constexpr int D = 128;         // head dim (K == V == 128)
constexpr int NTHR = 256;      // 4 waves
constexpr int LDQ = D + 8;     // bf16 [64][128] row stride (q, k, W, O staging)
constexpr int LDT = C + 8;     // bf16 [128][64] row stride (K^T, V^T) and [64][64] (P, T hi/lo)
constexpr int LDA = C + 8;     // fp32 [64][64] row stride (A, T)

enum Mode { MODE_OUT = 0, MODE_S0 = 1, MODE_PHI = 2 };

// shared-memory layout (bytes)
constexpr int SZ_Q = C * LDQ * 2;           // 17408
constexpr int SZ_KT = D * LDT * 2;          // 18432
constexpr int SZ_F32 = C * LDA * 4;         // 18432
constexpr int SZ_P = C * LDT * 2;           // 9216
constexpr int OFF_Q = 0;
constexpr int OFF_K = OFF_Q + SZ_Q;
constexpr int OFF_KT = OFF_K + SZ_Q;
constexpr int OFF_VT = OFF_KT + SZ_KT;      // also the O staging buffer
constexpr int OFF_A = OFF_VT + SZ_KT;       // fp32 A, then bf16 T hi/lo (4 x SZ_P)
constexpr int OFF_T = OFF_A + SZ_F32;       // fp32 T
constexpr int OFF_W = OFF_T + SZ_F32;
constexpr int OFF_P = OFF_W + SZ_Q;
constexpr int OFF_X = OFF_P + SZ_P;         // fp32 scratch 3 x 16 x 16
constexpr int OFF_G = OFF_X + 3 * 256 * 4;  // fp32 G[64], beta[64], eG[64], edl[64]
constexpr int SMEM = OFF_G + 4 * C * 4;
static_assert(4 * SZ_P <= 2 * SZ_F32, "T hi/lo must fit over A and T");
static_assert(SMEM <= 160 * 1024, "LDS budget");

struct SegInfo {     // one row of the host-built segment table (int32 x 8)
  int n, bos, eos, c_start, c_end, seg_idx, first_seg, nseg;
};

struct Params {
  const bf16* q; const bf16* k; const bf16* v;
  const void* g; int g_dt;
  const void* beta; int beta_dt;
  bf16* o;
  const float* h0;           // [N,H,K,V] or null
  float* ht;                 // [N,H,K,V] or null
  const int* seg;            // [nseg_total][8]
  int* plan;                 // [nseg_total][H]: warm-up start chunk, or -1
  int* exact;                // [N][H]
  float* ws_s0;              // [nseg_total][H][D][D]
  float* ws_phi;
  float* ws_init;
  int nseg_total;
  int H, HKV;
  float scale;
  int l2norm;
  int max_warm;
  float decay_thresh;
};

__device__ __forceinline__ float ld_scalar(const void* p, int64_t i, int dt) {
  if (dt == HMX_F32) return static_cast<const float*>(p)[i];
  if (dt == HMX_BF16) return (float)static_cast<const bf16*>(p)[i];
  return (float)static_cast<const f16*>(p)[i];
}

__device__ __forceinline__ SegInfo load_seg(const int* seg, int s) {
  const int* r = seg + s * 8;
  return SegInfo{r[0], r[1], r[2], r[3], r[4], r[5], r[6], r[7]};
}

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// A (or B^T) fragment in natural k order: lane holds row r0+(l&15), k0+8(l>>4)..+7.
__device__ __forceinline__ bf16x8 frag(const bf16* base, int ld, int r0, int k0, int lane) {
  return *reinterpret_cast<const bf16x8*>(base + (r0 + (lane & 15)) * ld + k0 + 8 * (lane >> 4));
}

// A fragment whose k order matches a B operand built from two C-layout tiles:
// lane holds row r0+(l&15), k = k0+4q+{0..3} and k0+16+4q+{0..3}, q = l>>4.
__device__ __forceinline__ bf16x8 frag_perm(const bf16* base, int ld, int r0, int k0, int lane) {
  const bf16* p = base + (r0 + (lane & 15)) * ld + k0 + 4 * (lane >> 4);
  const bf16x4 a = *reinterpret_cast<const bf16x4*>(p);
  const bf16x4 b = *reinterpret_cast<const bf16x4*>(p + 16);
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// B fragment from two vertically stacked C-layout 16x16 tiles (rows 0-15 in t0,
// rows 16-31 in t1); pairs with frag_perm.
__device__ __forceinline__ bf16x8 pack_b(const f32x4& t0, const f32x4& t1) {
  return bf16x8{(bf16)t0[0], (bf16)t0[1], (bf16)t0[2], (bf16)t0[3],
                (bf16)t1[0], (bf16)t1[1], (bf16)t1[2], (bf16)t1[3]};
}

// hi/lo split of the same pair: x ~= hi + lo with both in bf16.
__device__ __forceinline__ void pack_b_hilo(const f32x4& t0, const f32x4& t1, bf16x8& hi,
                                            bf16x8& lo) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16 h0 = (bf16)t0[j], h1 = (bf16)t1[j];
    hi[j] = h0; hi[4 + j] = h1;
    lo[j] = (bf16)(t0[j] - (float)h0);
    lo[4 + j] = (bf16)(t1[j] - (float)h1);
  }
}

// ---------------------------------------------------------------------------
// the chunk-scan workgroup
// ---------------------------------------------------------------------------
template <int MODE>
__global__ __launch_bounds__(NTHR, 1) void gdn_chunk_kernel(Params p) {
  __shared__ __align__(16) unsigned char smem[SMEM];
  bf16* sQ = reinterpret_cast<bf16*>(smem + OFF_Q);
  bf16* sK = reinterpret_cast<bf16*>(smem + OFF_K);
  bf16* sKt = reinterpret_cast<bf16*>(smem + OFF_KT);
  bf16* sVt = reinterpret_cast<bf16*>(smem + OFF_VT);
  bf16* sO = sVt;  // O staging reuses V^T after U is formed
  float* sA = reinterpret_cast<float*>(smem + OFF_A);
  float* sT = reinterpret_cast<float*>(smem + OFF_T);
  bf16* sTkh = reinterpret_cast<bf16*>(smem + OFF_A);
  bf16* sTkl = sTkh + C * LDT;
  bf16* sTvh = sTkl + C * LDT;
  bf16* sTvl = sTvh + C * LDT;
  bf16* sW = reinterpret_cast<bf16*>(smem + OFF_W);
  bf16* sP = reinterpret_cast<bf16*>(smem + OFF_P);
  float* sX = reinterpret_cast<float*>(smem + OFF_X);
  float* sG = reinterpret_cast<float*>(smem + OFF_G);
  float* sB = sG + C;
  float* sEG = sB + C;    // e^{G}
  float* sEDL = sEG + C;  // e^{G_last - G}

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q4 = lane >> 4, l16 = lane & 15;
  const int s_id = blockIdx.x, h = blockIdx.y;
  const SegInfo si = load_seg(p.seg, s_id);
  const int H = p.H;
  const int hk = h / (H / p.HKV);

  // ---- decide the chunk range and the initial state ------------------------
  const bool exact = p.exact && p.exact[si.n * H + h];
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
    if (!exact || si.seg_idx == si.nseg - 1) return;
    if (MODE == MODE_PHI) {
      if (si.seg_idx == 0) return;
      init_kind = 3;
    } else {
      init_kind = (si.seg_idx == 0) ? 1 : 0;
    }
  }
  if (init_kind == 1 && !p.h0) init_kind = 0;

  // ---- state registers: S[rt][ct] is the 16x16 tile (rows 16rt.., cols 32w+16ct..)
  f32x4 S[8][2];
  {
    const float* src = nullptr;
    if (init_kind == 1) src = p.h0 + ((int64_t)si.n * H + h) * D * D;
    if (init_kind == 2) src = p.ws_init + ((int64_t)s_id * H + h) * D * D;
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = 16 * rt + 4 * q4 + v, col = 32 * wave + 16 * ct + l16;
          float x = 0.f;
          if (src) x = src[row * D + col];
          if (init_kind == 3) x = (row == col) ? 1.f : 0.f;
          S[rt][ct][v] = x;
        }
  }

  // P's strictly-upper 16x16 tiles are never written by phase 1: zero them once.
  if (MODE == MODE_OUT) {
    for (int i = tid; i < C * C; i += NTHR) {
      const int r = i / C, c = i % C;
      if ((c >> 4) > (r >> 4)) sP[r * LDT + c] = (bf16)0.f;
    }
  }

  const int64_t q_rs = (int64_t)H * D, kv_rs = (int64_t)p.HKV * D;
  const bf16* qh = p.q + (int64_t)h * D;
  const bf16* kh = p.k + (int64_t)hk * D;
  const bf16* vh = p.v + (int64_t)hk * D;

  for (int c = c_begin; c < si.c_end; ++c) {
    const int tok0 = si.bos + c * C;
    const int nval = min(C, si.eos - tok0);
    const bool out_chunk = (MODE == MODE_OUT) && (c >= c_out);

    // ---- phase 0: load the chunk (L2-normalise q,k rows), g cumsum --------
    {
      // 16 threads per 128-wide row, 16 rows per pass, 4 passes
#pragma unroll
      for (int pass = 0; pass < 4; ++pass) {
        const int row = pass * 16 + (tid >> 4);
        const int f0 = (tid & 15) * 8;
        const bool ok = row < nval;
        const int64_t tok = tok0 + row;
        // k
        bf16x8 kv8 = {};
        if (ok) kv8 = *reinterpret_cast<const bf16x8*>(kh + tok * kv_rs + f0);
        float kf[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) kf[j] = (float)kv8[j];
        if (p.l2norm) {
          float ss = 0.f;
#pragma unroll
          for (int j = 0; j < 8; ++j) ss += kf[j] * kf[j];
          ss += shfl_xor(ss, 1); ss += shfl_xor(ss, 2);
          ss += shfl_xor(ss, 4); ss += shfl_xor(ss, 8);
          const float inv = 1.0f / sqrtf(ss + 1e-6f);
#pragma unroll
          for (int j = 0; j < 8; ++j) kf[j] *= inv;
        }
        bf16x8 kb;
#pragma unroll
        for (int j = 0; j < 8; ++j) kb[j] = (bf16)kf[j];
        *reinterpret_cast<bf16x8*>(sK + row * LDQ + f0) = kb;
#pragma unroll
        for (int j = 0; j < 8; ++j) sKt[(f0 + j) * LDT + row] = kb[j];
        // v (transposed only)
        if (MODE != MODE_PHI) {
          bf16x8 vv8 = {};
          if (ok) vv8 = *reinterpret_cast<const bf16x8*>(vh + tok * kv_rs + f0);
#pragma unroll
          for (int j = 0; j < 8; ++j) sVt[(f0 + j) * LDT + row] = vv8[j];
        }
        // q
        if (out_chunk) {
          bf16x8 qv8 = {};
          if (ok) qv8 = *reinterpret_cast<const bf16x8*>(qh + tok * q_rs + f0);
          float qf[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) qf[j] = (float)qv8[j];
          if (p.l2norm) {
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) ss += qf[j] * qf[j];
            ss += shfl_xor(ss, 1); ss += shfl_xor(ss, 2);
            ss += shfl_xor(ss, 4); ss += shfl_xor(ss, 8);
            const float inv = 1.0f / sqrtf(ss + 1e-6f);
#pragma unroll
            for (int j = 0; j < 8; ++j) qf[j] *= inv;
          }
          bf16x8 qb;
#pragma unroll
          for (int j = 0; j < 8; ++j) qb[j] = (bf16)qf[j];
          *reinterpret_cast<bf16x8*>(sQ + row * LDQ + f0) = qb;
        }
      }
      if (wave == 0) {
        const int t = lane;
        const bool ok = t < nval;
        const int64_t gi = (int64_t)(tok0 + t) * H + h;
        float gv = ok ? ld_scalar(p.g, gi, p.g_dt) : 0.f;
        float bv = ok ? ld_scalar(p.beta, gi, p.beta_dt) : 0.f;
        // inclusive scan over the 64 lanes
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const float y = __shfl_up(gv, off, 64);
          if (lane >= off) gv += y;
        }
        const float glast = __shfl(gv, 63, 64);
        sG[t] = gv;
        sB[t] = bv;
        sEG[t] = fast_exp(gv);
        sEDL[t] = fast_exp(glast - gv);
      }
    }
    __syncthreads();

    // ---- phase 1: A = beta_i (k_i.k_j) e^{G_i-G_j} (j<i), P = q_i.k_j e^{G_i-G_j} (j<=i)
    {
      const int nitems = out_chunk ? 20 : 10;
      for (int it = wave; it < nitems; it += 4) {
        const int pair = out_chunk ? (it >> 1) : it;
        const bool isP = out_chunk && (it & 1);
        int i = 0, j = pair;
        while (j > i) { j -= i + 1; ++i; }  // pair -> (i, j), 0 <= j <= i < 4
        const bf16* Am = isP ? sQ : sK;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          acc = mfma16(frag(Am, LDQ, 16 * i, 32 * ks, lane), frag(sK, LDQ, 16 * j, 32 * ks, lane),
                       acc);
        const int col = 16 * j + l16;
        const float gc = sG[col];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = 16 * i + 4 * q4 + v;
          const float dcy = (row >= col) ? fast_exp(sG[row] - gc) : 0.f;
          if (isP) {
            sP[row * LDT + col] = (bf16)(row >= col ? acc[v] * dcy : 0.f);
          } else {
            sA[row * LDA + col] = row > col ? sB[row] * acc[v] * dcy : 0.f;
          }
        }
      }
    }
    __syncthreads();

    // ---- phase 2: T = (I + A)^-1 in fp32 --------------------------------------
    {
      // 2a: 16x16 diagonal blocks by forward substitution, one wave per block
      {
        const int b = wave, cc = l16;
        float x[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float acc = (r == cc) ? 1.f : 0.f;
#pragma unroll
          for (int m = 0; m < r; ++m) acc -= sA[(16 * b + r) * LDA + 16 * b + m] * x[m];
          x[r] = acc;
        }
        if (lane < 16) {
#pragma unroll
          for (int r = 0; r < 16; ++r) sT[(16 * b + r) * LDA + 16 * b + cc] = x[r];
        }
        // zero the strictly-upper blocks of T in this block row
        for (int e = lane; e < 16 * 64; e += 64) {
          const int r = 16 * b + (e >> 6), col = e & 63;
          if ((col >> 4) > b) sT[r * LDA + col] = 0.f;
        }
      }
      __syncthreads();
      // 2b: off-diagonal blocks by distance d: T_ij = -T_ii sum_{m=j}^{i-1} A_im T_mj
      for (int d = 1; d < 4; ++d) {
        const int nblk = 4 - d;
        for (int e = tid; e < nblk * 256; e += NTHR) {
          const int bj = e >> 8, r = (e >> 4) & 15, cc = e & 15;
          const int bi = bj + d;
          float acc = 0.f;
          for (int m = bj; m < bi; ++m)
#pragma unroll
            for (int kk = 0; kk < 16; ++kk)
              acc += sA[(16 * bi + r) * LDA + 16 * m + kk] * sT[(16 * m + kk) * LDA + 16 * bj + cc];
          sX[e] = acc;
        }
        __syncthreads();
        for (int e = tid; e < nblk * 256; e += NTHR) {
          const int bj = e >> 8, r = (e >> 4) & 15, cc = e & 15;
          const int bi = bj + d;
          float acc = 0.f;
#pragma unroll
          for (int kk = 0; kk < 16; ++kk)
            acc += sT[(16 * bi + r) * LDA + 16 * bi + kk] * sX[(bj << 8) + kk * 16 + cc];
          sT[(16 * bi + r) * LDA + 16 * bj + cc] = -acc;
        }
        __syncthreads();
      }
      // 2c: Tk = T diag(beta e^G), Tv = T diag(beta), split into bf16 hi + lo
      float tk[16], tv[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int idx = tid + e * NTHR, r = idx >> 6, cc = idx & 63;
        const float t = sT[r * LDA + cc];
        tk[e] = t * sB[cc] * sEG[cc];
        tv[e] = t * sB[cc];
      }
      __syncthreads();
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int idx = tid + e * NTHR, r = idx >> 6, cc = idx & 63;
        const bf16 kh_ = (bf16)tk[e];
        sTkh[r * LDT + cc] = kh_;
        sTkl[r * LDT + cc] = (bf16)(tk[e] - (float)kh_);
        if (MODE != MODE_PHI) {
          const bf16 vh_ = (bf16)tv[e];
          sTvh[r * LDT + cc] = vh_;
          sTvl[r * LDT + cc] = (bf16)(tv[e] - (float)vh_);
        }
      }
      __syncthreads();
    }

    // ---- phase 3: W = Tk K (to LDS, negated), U = Tv V (registers) -----------
    f32x4 Vn[4][2];  // U, then V_new: rows 16mt.., cols 32w+16ct..
    {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          const int nt = 2 * wave + ct;
          f32x4 w = {0.f, 0.f, 0.f, 0.f};
          f32x4 u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const bf16x8 bk = frag(sKt, LDT, 16 * nt, 32 * ks, lane);
            w = mfma16(frag(sTkh, LDT, 16 * mt, 32 * ks, lane), bk, w);
            w = mfma16(frag(sTkl, LDT, 16 * mt, 32 * ks, lane), bk, w);
            if (MODE != MODE_PHI) {
              const bf16x8 bv = frag(sVt, LDT, 16 * nt, 32 * ks, lane);
              u = mfma16(frag(sTvh, LDT, 16 * mt, 32 * ks, lane), bv, u);
              u = mfma16(frag(sTvl, LDT, 16 * mt, 32 * ks, lane), bv, u);
            }
          }
#pragma unroll
          for (int v = 0; v < 4; ++v)
            sW[(16 * mt + 4 * q4 + v) * LDQ + 16 * nt + l16] = (bf16)(-w[v]);
          Vn[mt][ct] = u;
        }
    }
    __syncthreads();

    // ---- phase 4: V_new = U - W S (state as bf16 B operand) -------------------
    bf16x8 Sb[4][2];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) Sb[ks][ct] = pack_b(S[2 * ks][ct], S[2 * ks + 1][ct]);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 a = frag_perm(sW, LDQ, 16 * mt, 32 * ks, lane);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) Vn[mt][ct] = mfma16(a, Sb[ks][ct], Vn[mt][ct]);
      }

    // ---- phase 5: O = scale [e^G (Q S) + P V_new] ------------------------------
    if (out_chunk) {
      f32x4 O[4][2];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) O[mt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16x8 a = frag_perm(sQ, LDQ, 16 * mt, 32 * ks, lane);
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) O[mt][ct] = mfma16(a, Sb[ks][ct], O[mt][ct]);
        }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float e = sEG[16 * mt + 4 * q4 + v];
          O[mt][0][v] *= e;
          O[mt][1][v] *= e;
        }
      bf16x8 Vb[2][2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) Vb[ks][ct] = pack_b(Vn[2 * ks][ct], Vn[2 * ks + 1][ct]);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          if (32 * ks > 16 * mt + 15) continue;  // P is lower triangular
          const bf16x8 a = frag_perm(sP, LDT, 16 * mt, 32 * ks, lane);
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) O[mt][ct] = mfma16(a, Vb[ks][ct], O[mt][ct]);
        }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            sO[(16 * mt + 4 * q4 + v) * LDQ + 32 * wave + 16 * ct + l16] =
                (bf16)(O[mt][ct][v] * p.scale);
    }

    // ---- phase 6: S <- e^{G_last} S + K^T (e^{G_last-G} V_new), hi/lo ---------
    {
      const float egl = sEG[C - 1];
#pragma unroll
      for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v) S[rt][ct][v] *= egl;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float e = sEDL[16 * mt + 4 * q4 + v];
          Vn[mt][0][v] *= e;
          Vn[mt][1][v] *= e;
        }
      bf16x8 Vh[2][2], Vl[2][2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
          pack_b_hilo(Vn[2 * ks][ct], Vn[2 * ks + 1][ct], Vh[ks][ct], Vl[ks][ct]);
#pragma unroll
      for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const bf16x8 a = frag_perm(sKt, LDT, 16 * rt, 32 * ks, lane);
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) {
            S[rt][ct] = mfma16(a, Vh[ks][ct], S[rt][ct]);
            S[rt][ct] = mfma16(a, Vl[ks][ct], S[rt][ct]);
          }
        }
    }
    __syncthreads();

    // ---- store O (coalesced 16-byte rows) --------------------------------------
    if (out_chunk) {
      bf16* oh = p.o + (int64_t)h * D;
#pragma unroll
      for (int pass = 0; pass < 4; ++pass) {
        const int row = pass * 16 + (tid >> 4);
        const int f0 = (tid & 15) * 8;
        if (row < nval)
          *reinterpret_cast<bf16x8*>(oh + (int64_t)(tok0 + row) * q_rs + f0) =
              *reinterpret_cast<const bf16x8*>(sO + row * LDQ + f0);
      }
      __syncthreads();
    }
  }

  // ---- write the end state ---------------------------------------------------
  float* dst = nullptr;
  if (MODE == MODE_OUT) {
    if (si.seg_idx == si.nseg - 1 && p.ht) dst = p.ht + ((int64_t)si.n * H + h) * D * D;
  } else if (MODE == MODE_S0) {
    dst = p.ws_s0 + ((int64_t)s_id * H + h) * D * D;
  } else {
    dst = p.ws_phi + ((int64_t)s_id * H + h) * D * D;
  }
  if (dst) {
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          dst[(16 * rt + 4 * q4 + v) * D + 32 * wave + 16 * ct + l16] = S[rt][ct][v];
  }
}

// ---------------------------------------------------------------------------
// plan: warm-up start chunk per (segment, head); exact flag per (sequence, head)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void gdn_plan_kernel(Params p, int N) {
  const int n = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int H = p.H;
  int any_exact = 0;
  // find this sequence's segments: the table is sorted by sequence
  for (int s = 0; s < p.nseg_total; ++s) {
    const SegInfo si = load_seg(p.seg, s);
    if (si.n != n) continue;
    int plan = 0;
    if (si.seg_idx > 0) {
      plan = -1;
      if (p.l2norm) {
        float acc = 0.f;
        const int lo = max(0, si.c_start - p.max_warm);
        for (int c = si.c_start - 1; c >= lo; --c) {
          const int t = si.bos + c * C + lane;
          float b = 0.f;
          if (t < si.eos) {
            const int64_t gi = (int64_t)t * H + h;
            const float gv = ld_scalar(p.g, gi, p.g_dt);
            const float bv = ld_scalar(p.beta, gi, p.beta_dt);
            b = gv + logf(fmaxf(1.f, fabsf(1.f - bv)));
          }
          acc += wave_sum(b);
          if (acc < -p.decay_thresh) { plan = c; break; }
          if (c == 0) { plan = 0; break; }  // reached the sequence start: exact from h0
        }
      }
    }
    if (plan < 0) any_exact = 1;
    if (lane == 0) p.plan[s * H + h] = plan;
  }
  if (lane == 0) p.exact[n * H + h] = any_exact;
}

// ---------------------------------------------------------------------------
// exact segment scan: S_1 = S0_0; S_{s+1} = Phi_s S_s + S0_s  (fp32)
// one workgroup per (sequence, head, 16-column slice)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(NTHR) void gdn_seg_combine_kernel(Params p, int N) {
  __shared__ float sS[D * 16];
  const int nh = blockIdx.x, cb = blockIdx.y, tid = threadIdx.x;
  const int H = p.H, n = nh / H, h = nh % H;
  if (!p.exact[n * H + h]) return;
  int first = -1, nseg = 0;
  for (int s = 0; s < p.nseg_total; ++s) {
    const SegInfo si = load_seg(p.seg, s);
    if (si.n == n) { first = si.first_seg; nseg = si.nseg; break; }
  }
  if (first < 0 || nseg < 2) return;
  const int row = tid >> 1, c0 = (tid & 1) * 8;
  const int64_t hoff = (int64_t)h * D * D;
  // S_1
  {
    const float* s0 = p.ws_s0 + (int64_t)first * H * D * D + hoff;
    float* init = p.ws_init + (int64_t)(first + 1) * H * D * D + hoff;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float x = s0[row * D + cb * 16 + c0 + j];
      sS[row * 16 + c0 + j] = x;
      init[row * D + cb * 16 + c0 + j] = x;
    }
  }
  __syncthreads();
  for (int s = 1; s < nseg - 1; ++s) {
    const float* phi = p.ws_phi + (int64_t)(first + s) * H * D * D + hoff;
    const float* s0 = p.ws_s0 + (int64_t)(first + s) * H * D * D + hoff;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = s0[row * D + cb * 16 + c0 + j];
    for (int kk = 0; kk < D; ++kk) {
      const float a = phi[row * D + kk];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += a * sS[kk * 16 + c0 + j];
    }
    __syncthreads();
    float* init = p.ws_init + (int64_t)(first + s + 1) * H * D * D + hoff;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      sS[row * 16 + c0 + j] = acc[j];
      init[row * D + cb * 16 + c0 + j] = acc[j];
    }
    __syncthreads();
  }
}

}  // namespace gdnp
}  // namespace hmx

using namespace hmx;
using namespace hmx::gdnp;

extern "C" int hmx_gdn_chunk_fwd(const void* q, const void* k, const void* v, int32_t qkv_dtype,
                                 const void* g, int32_t g_dtype, const void* beta,
                                 int32_t beta_dtype, void* o, const float* h0, float* ht,
                                 const int32_t* seg_table, int32_t nseg_total, int32_t N,
                                 int32_t H, int32_t HKV, int32_t K, int32_t V, float scale,
                                 int32_t use_qk_l2norm, int32_t max_warm_chunks,
                                 float decay_threshold, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  HMX_REQUIRE(qkv_dtype == HMX_BF16, HMX_EUNSUPPORTED,
              "hmx_gdn_chunk_fwd: q/k/v must be bfloat16 (got dtype code %d)", qkv_dtype);
  HMX_REQUIRE(K == D && V == D, HMX_EUNSUPPORTED,
              "hmx_gdn_chunk_fwd: only K == V == 128 is supported (got K=%d V=%d)", K, V);
  HMX_REQUIRE(H > 0 && HKV > 0 && H % HKV == 0, HMX_EINVAL,
              "hmx_gdn_chunk_fwd: H=%d must be a positive multiple of HKV=%d", H, HKV);
  HMX_REQUIRE(q && k && v && g && beta && o && seg_table, HMX_EINVAL,
              "hmx_gdn_chunk_fwd: null tensor pointer");
  HMX_REQUIRE(g_dtype >= 0 && g_dtype <= 2 && beta_dtype >= 0 && beta_dtype <= 2,
              HMX_EUNSUPPORTED, "hmx_gdn_chunk_fwd: g/beta dtype");
  if (nseg_total == 0) return HMX_OK;
  const size_t need = hmx_gdn_chunk_workspace_bytes(nseg_total, N, H);
  HMX_REQUIRE(workspace && workspace_bytes >= need, HMX_EINVAL,
              "hmx_gdn_chunk_fwd: workspace of %zu bytes needed, %zu given", need,
              workspace_bytes);
  Params p;
  p.q = static_cast<const bf16*>(q); p.k = static_cast<const bf16*>(k);
  p.v = static_cast<const bf16*>(v);
  p.g = g; p.g_dt = g_dtype; p.beta = beta; p.beta_dt = beta_dtype;
  p.o = static_cast<bf16*>(o); p.h0 = h0; p.ht = ht;
  p.seg = seg_table; p.nseg_total = nseg_total; p.H = H; p.HKV = HKV; p.scale = scale;
  p.l2norm = use_qk_l2norm; p.max_warm = max_warm_chunks; p.decay_thresh = decay_threshold;
  // workspace carve-up: state buffers first (256-byte aligned), then plan/exact
  const size_t st = (size_t)nseg_total * H * D * D * sizeof(float);
  char* ws = static_cast<char*>(workspace);
  const bool multi = nseg_total > N;
  p.ws_s0 = multi ? reinterpret_cast<float*>(ws) : nullptr;
  p.ws_phi = multi ? reinterpret_cast<float*>(ws + st) : nullptr;
  p.ws_init = multi ? reinterpret_cast<float*>(ws + 2 * st) : nullptr;
  char* tail = ws + (multi ? 3 * st : 0);
  p.plan = reinterpret_cast<int*>(tail);
  p.exact = reinterpret_cast<int*>(tail + (size_t)nseg_total * H * sizeof(int));
  hipStream_t s = (hipStream_t)stream;
  if (multi) {
    hipLaunchKernelGGL(gdn_plan_kernel, dim3(N, H), dim3(64), 0, s, p, N);
    hipLaunchKernelGGL(gdn_chunk_kernel<MODE_S0>, dim3(nseg_total, H), dim3(NTHR), 0, s, p);
    hipLaunchKernelGGL(gdn_chunk_kernel<MODE_PHI>, dim3(nseg_total, H), dim3(NTHR), 0, s, p);
    hipLaunchKernelGGL(gdn_seg_combine_kernel, dim3(N * H, D / 16), dim3(NTHR), 0, s, p, N);
  } else {
    p.exact = nullptr;  // one segment per sequence: every segment starts from h0
  }
  hipLaunchKernelGGL(gdn_chunk_kernel<MODE_OUT>, dim3(nseg_total, H), dim3(NTHR), 0, s, p);
  return check_launch("hmx_gdn_chunk_fwd");
}

extern "C" size_t hmx_gdn_chunk_workspace_bytes(int32_t nseg_total, int32_t N, int32_t H) {
  const bool multi = nseg_total > N;
  size_t b = multi ? 3 * (size_t)nseg_total * H * D * D * sizeof(float) : 0;
  b += (size_t)nseg_total * H * sizeof(int) + (size_t)N * H * sizeof(int);
  return b;
}
