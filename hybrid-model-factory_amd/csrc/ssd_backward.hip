// Mamba2 SSD chunk scan backward (the gradients of mamba_chunk_scan_combined) for
// gfx950: bf16 MFMA products with fp32 accumulation, fp32 scalar chains.
//
// The forward (ssd_prefill.hip) per head h, chunk of L = 64 tokens, a_t = dt'_t A_h,
// A_t = sum_{s<=t} a_s from the chunk start (inclusive), chunk start state S0 and
// end state S1 (both P x N):
//   y'_t = sum_{s<=t} (C_t . B_s) e^{A_t - A_s} dt'_s x_s + e^{A_t} S0 C_t + D x_t
//   y_t  = y'_t silu(z_t)                        (y_t = y'_t without z)
//   S1   = e^{A_L} S0 + sum_s e^{A_L - A_s} dt'_s x_s B_s^T
// With g_t = dy_t silu(z_t) (dy_t without z), the gradient dS1 of the chunk's end
// state and, for s <= t,
//   M_ts = (C_t . B_s) e^{A_t - A_s},  Q_ts = g_t . x_s,  W_ts = dt'_s Q_ts e^{A_t - A_s}
// the backward is:
//   dS0   = e^{A_L} dS1 + sum_t e^{A_t} g_t C_t^T           (reverse scan over chunks)
//   dx_s  = sum_t M_ts dt'_s g_t + e^{A_L - A_s} dt'_s dS1 B_s + D g_s
//   dC_t  = sum_s W_ts B_s + e^{A_t} S0^T g_t
//   dB_s  = sum_t W_ts C_t + e^{A_L - A_s} dt'_s dS1^T x_s
//   ddt'_s = sum_t M_ts Q_ts + e^{A_L - A_s} x_s . (dS1 B_s)  +  A_h da_s
//   dA_t  (the cumulated log-decay): sum_s W_ts (C_t.B_s) - sum_u W_ut (C_u.B_t)
//           + g_t . (e^{A_t} S0 C_t) - dt'_t e^{A_L - A_t} x_t . (dS1 B_t)
//           + [t = L-1] <dS1, S1>
//   da_s  = sum_{t>=s} dA_t,   dA_h += sum_s dt'_s da_s
//   dz    = dy y' silu'(z),    dD_p += sum_t g_t[p] x_t[p]
//   d dt  = ddt' * [dt_min <= dt' <= dt_max] * (softplus ? sigmoid(dt + bias) : 1)
// with <dS1, S1> = e^{A_L} <dS1, S0> + sum_s dt'_s e^{A_L - A_s} x_s . (dS1 B_s), so
// S1 is never read.  These are the chain rule through the recurrence of
// oracle/ssd.py; mamba_ssm's backward (un-vendored) computes the same gradients
// with its own kernels (training/.../layers/mamba/mamba2.py:555-580 calls it).
//
// Three launches over 64-token chunks (rows of a segment table, one chunk each):
//   ssd_bwd_local_kernel  (chunk, C group's heads in turn; chunk, head at headdim
//                          128): the chunk's zero-start end state
//                          sum_s e^{A_L - A_s} dt'_s x_s B_s^T, its share
//                          sum_t e^{A_t} g_t C_t^T of dS0, and e^{A_L}
//   ssd_bwd_scan_kernel   (sequence, head, 1024 state elements): the forward chain
//                          S0(c+1) = e^{A_L(c)} S0(c) + local(c) gives every chunk's
//                          start state, the reverse chain dS1 of every chunk and dS0
//                          of the sequence's start
//   ssd_bwd_chunk_kernel  (chunk, C group): everything else, for the group's heads
//                          in turn, the next head's inputs loading into registers
//                          during the current head's products
// dC (and dB when B's groups are C's) sum over the workgroup's heads in registers;
// x shared by several heads (HX < H), or B shared wider than a C group, accumulate
// with fp32 atomics; everything else is stored.

#include <type_traits>

#include "common.hpp"
#include "mfma.hpp"

namespace hmx {
namespace ssdb {

constexpr int L = 64;
constexpr int NTHR = 256;

struct Params {
  const bf16* x; int64_t x_ts, x_hs;         // [T][HX][P]
  const bf16* B; int64_t b_ts, b_gs;         // [T][G][N]
  const bf16* C; int64_t c_ts, c_gs;         // [T][GC][N]
  const void* dt; int dt_dt; int64_t dt_ts, dt_hs;   // raw dt [T][H]
  const float* A;                            // [H]
  const float* D;                            // [H][P] or null
  const float* dt_bias;                      // [H] or null
  const bf16* z; int64_t z_ts, z_hs;         // [T][H][P] or null
  const bf16* dy; int64_t dy_ts, dy_hs;      // [T][H][P]
  const float* h0;                           // [nseq][H][P][N] or null (zero start)
  const float* dT;                           // [nseq][H][P][N] end-state gradients, or null
  const int* seg;                            // [nrows][8] segment rows (one chunk each)
  const int* seqs;                           // [nseq][2]: first row, rows
  int nrows, nseq;
  bf16* loc;                                 // ws [nrows][H][P][N]: dS0 shares
  bf16* sloc;                                // ws [nrows][H][P][N]: zero-start end states
  float* edec;                               // ws [nrows][H]: e^{A_L}
  bf16* S0;                                  // ws [nrows][H][P][N]: chunk start states
  bf16* dS1;                                 // ws [nrows][H][P][N]: end-state gradients
  // outputs (contiguous)
  void* dx;    int x_shared;                 // [T][HX][P]
  void* dB;    int b_shared;                 // [T][G][N]
  void* dC;                                  // [T][GC][N]
  int gbf16;                                 // dx, dB, dC stored in bf16 (else fp32)
  bf16* dz;                                  // [T][H][P] or null
  float* ddt;                                // [T][H]
  float* dA;                                 // [H] (accumulated)
  float* dD;                                 // [H][P] (accumulated) or null
  float* dbias;                              // [H] (accumulated) or null
  float* dh0;                                // [nseq][H][P][N] or null
  int H, HX, G, GC, softplus;
  float dt_min, dt_max;
};

// segment row: sequence, first token, end token, chunk range, index in the
// sequence, first row of the sequence, rows of the sequence
struct Row { int n, bos, eos, c0, c1, idx, first, nseg; };
__device__ __forceinline__ Row load_row(const int* seg, int r) {
  const int* q = seg + r * 8;
  return Row{q[0], q[1], q[2], q[3], q[4], q[5], q[6], q[7]};
}

__device__ __forceinline__ float scan64(float x, int lane) {
  x = scan32(x);
  const float lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 31));
  return lane >= 32 ? x + lo : x;
}

__device__ __forceinline__ float silu(float z) { return z * __builtin_amdgcn_rcpf(1.f + fast_exp(-z)); }

// a stored (not accumulated) gradient element, bf16 or fp32
__device__ __forceinline__ void st_grad(void* base, int64_t i, float v, int bf) {
  if (bf) static_cast<bf16*>(base)[i] = (bf16)v;
  else static_cast<float*>(base)[i] = v;
}

// Per-token scalars of a chunk, lane t of one wave: dt' (0 past the chunk's
// tokens), A_t, and the factor d dt'/d dt (clamp pass times the softplus slope).
struct Tok { float dtv, acs, fac; };
// dt prefetched for the next head: its raw bits (one load in either dtype
// branch), converted where the scalars are formed.  Converting at the load (as
// load_any does) would wait there for every load issued before it, the rest of
// the prefetch included.
__device__ __forceinline__ uint32_t ld_bits(const void* p, int64_t i, int dt) {
  if (dt == HMX_F32) return static_cast<const uint32_t*>(p)[i];
  return static_cast<const uint16_t*>(p)[i];
}
__device__ __forceinline__ float bits_f32(uint32_t b, int dt) {
  if (dt == HMX_F32) return __builtin_bit_cast(float, b);
  if (dt == HMX_BF16) return __builtin_bit_cast(float, b << 16);
  return (float)__builtin_bit_cast(f16, (uint16_t)b);
}
__device__ __forceinline__ Tok token_scalars_raw(const Params& p, int h, float dt_raw, int nval,
                                                 int lane) {
  float d = dt_raw + (p.dt_bias ? p.dt_bias[h] : 0.f);
  float sp = d, slope = 1.f;
  if (p.softplus) {
    sp = softplus20(d);
    slope = d > 20.f ? 1.f : 1.f / (1.f + fast_exp(-d));
  }
  float dtv = fminf(fmaxf(sp, p.dt_min), p.dt_max);
  // torch.clamp's gradient passes on [min, max]
  float fac = (sp >= p.dt_min && sp <= p.dt_max) ? slope : 0.f;
  if (lane >= nval) { dtv = 0.f; fac = 0.f; }
  const float acs = scan64(dtv * p.A[h], lane);
  return Tok{dtv, acs, fac};
}
__device__ __forceinline__ Tok token_scalars(const Params& p, int h, int tok0, int nval, int lane) {
  float d = 0.f;
  if (lane < nval) d = load_any(p.dt, (int64_t)(tok0 + lane) * p.dt_ts + (int64_t)h * p.dt_hs, p.dt_dt);
  return token_scalars_raw(p, h, d, nval, lane);
}

// ---------------------------------------------------------------------------
// local: sloc[r][h] = sum_s dt'_s e^{A_L - A_s} x_s B_s^T, loc[r][h] = sum_t e^{A_t}
// g_t C_t^T (P x N each, stored in bf16: the scans accumulate them in fp32),
// edec[r][h] = e^{A_L}
// ---------------------------------------------------------------------------
template <int P, int N>
constexpr int local_lds_bytes() { return 2 * L * (P + 8) * 2 + 2 * L * (N + 8) * 2 + 2 * L * 4; }

template <int P, int N>
__global__ __launch_bounds__(NTHR) void ssd_bwd_local_kernel(Params p) {
  constexpr int LDX = P + 8, LDB = N + 8;
  constexpr int VX = L * P / 8 / NTHR, VB = L * N / 8 / NTHR;
  extern __shared__ __align__(16) unsigned char lsm[];
  bf16* sG = reinterpret_cast<bf16*>(lsm);                     // e^{A_t} g_t       [L][LDX]
  bf16* sXW = sG + L * LDX;                                    // dt'_s e^{A_L-A_s} x_s
  bf16* sC = sXW + L * LDX;                                    // [L][LDB]
  bf16* sB = sC + L * LDB;
  float* sEA = reinterpret_cast<float*>(sB + L * LDB);
  float* sWT = sEA + L;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, l16 = lane & 15;
  const int H = p.H, GC = p.GC, HC = H / GC, HB = H / p.G, HXS = H / p.HX;
  // headdim 64: one workgroup per (chunk, C group), C staged once (B too when its
  // groups are C's), the group's heads in turn with the next one's rows loading
  // into registers during the current one's products.  Headdim 128: one workgroup
  // per (chunk, head) (the rows of a second head would not fit in registers).
  constexpr bool AHEAD = P == 64;
  const int per_row = AHEAD ? GC : H, nh = AHEAD ? HC : 1;
  const int r = blockIdx.x / per_row;
  const int h_first = AHEAD ? (blockIdx.x % per_row) * HC : blockIdx.x % per_row;
  const int gc = h_first / HC;
  const Row ro = load_row(p.seg, r);
  const int tok0 = ro.bos, nval = ro.eos - ro.bos;
  const bool b_once = AHEAD && p.G == GC;
#pragma unroll
  for (int i = 0; i < VB; ++i) {
    const int e = (i * NTHR + tid) * 8, t = e / N, c = e % N;
    bf16x8 cv = {}, bv = {};
    if (t < nval) {
      cv = *reinterpret_cast<const bf16x8*>(p.C + (int64_t)(tok0 + t) * p.c_ts + (int64_t)gc * p.c_gs + c);
      if (b_once)
        bv = *reinterpret_cast<const bf16x8*>(p.B + (int64_t)(tok0 + t) * p.b_ts +
                                              (int64_t)(h_first / HB) * p.b_gs + c);
    }
    *reinterpret_cast<bf16x8*>(sC + t * LDB + c) = cv;
    if (b_once) *reinterpret_cast<bf16x8*>(sB + t * LDB + c) = bv;
  }
  constexpr int VZ = P == 64 ? VX : 1;
  struct In { bf16x8 x[VX], dy[VX], z[VZ], b[VB]; uint32_t dt; };
  const auto fetch = [&](int h, In& q) {
    const int hx = h / HXS, g = h / HB;
#pragma unroll
    for (int i = 0; i < VX; ++i) {
      const int e = (i * NTHR + tid) * 8, t = e / P, c = e % P;
      q.x[i] = q.dy[i] = bf16x8{};
      if constexpr (P == 64) q.z[i] = bf16x8{};
      if (t < nval) {
        q.dy[i] = *reinterpret_cast<const bf16x8*>(p.dy + (int64_t)(tok0 + t) * p.dy_ts + (int64_t)h * p.dy_hs + c);
        q.x[i] = *reinterpret_cast<const bf16x8*>(p.x + (int64_t)(tok0 + t) * p.x_ts + (int64_t)hx * p.x_hs + c);
        if constexpr (P == 64) {
          if (p.z) q.z[i] = *reinterpret_cast<const bf16x8*>(p.z + (int64_t)(tok0 + t) * p.z_ts + (int64_t)h * p.z_hs + c);
        }
      }
    }
    if (!b_once) {
#pragma unroll
      for (int i = 0; i < VB; ++i) {
        const int e = (i * NTHR + tid) * 8, t = e / N, c = e % N;
        q.b[i] = bf16x8{};
        if (t < nval)
          q.b[i] = *reinterpret_cast<const bf16x8*>(p.B + (int64_t)(tok0 + t) * p.b_ts + (int64_t)g * p.b_gs + c);
      }
    }
    q.dt = (wave == 0 && lane < nval)
               ? ld_bits(p.dt, (int64_t)(tok0 + lane) * p.dt_ts + (int64_t)h * p.dt_hs, p.dt_dt) : 0u;
  };
  In in;
  if constexpr (AHEAD) fetch(h_first, in);
  constexpr int PBW = P / 16 / 4;   // p blocks per wave
  for (int ih = 0; ih < nh; ++ih) {
    const int h = h_first + ih;
    if (wave == 0) {
      const Tok tk = AHEAD ? token_scalars_raw(p, h, bits_f32(in.dt, p.dt_dt), nval, lane)
                           : token_scalars(p, h, tok0, nval, lane);
      const float aend = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, tk.acs), 63));
      sEA[lane] = fast_exp(tk.acs);
      sWT[lane] = tk.dtv * fast_exp(aend - tk.acs);
      if (lane == L - 1) p.edec[(int64_t)r * H + h] = expf(aend);
    }
    __syncthreads();   // the scalars; the previous head's products have read the tiles
    if constexpr (!AHEAD) {   // headdim 128: the rows straight from memory
      const int hx = h / HXS, g = h / HB;
#pragma unroll
      for (int i = 0; i < VX; ++i) {
        const int e = (i * NTHR + tid) * 8, t = e / P, c = e % P;
        in.x[i] = in.dy[i] = bf16x8{};
        if (t < nval) {
          in.dy[i] = *reinterpret_cast<const bf16x8*>(p.dy + (int64_t)(tok0 + t) * p.dy_ts + (int64_t)h * p.dy_hs + c);
          in.x[i] = *reinterpret_cast<const bf16x8*>(p.x + (int64_t)(tok0 + t) * p.x_ts + (int64_t)hx * p.x_hs + c);
        }
      }
#pragma unroll
      for (int i = 0; i < VB; ++i) {
        const int e = (i * NTHR + tid) * 8, t = e / N, c = e % N;
        bf16x8 bv = {};
        if (t < nval)
          bv = *reinterpret_cast<const bf16x8*>(p.B + (int64_t)(tok0 + t) * p.b_ts + (int64_t)g * p.b_gs + c);
        *reinterpret_cast<bf16x8*>(sB + t * LDB + c) = bv;
      }
    }
#pragma unroll
    for (int i = 0; i < VX; ++i) {
      const int e = (i * NTHR + tid) * 8, t = e / P, c = e % P;
      const float ea = sEA[t], wt = sWT[t];
      bf16x8 o, xw;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float v = (float)in.dy[i][j];
        if constexpr (P == 64) {
          if (p.z) v *= silu((float)in.z[i][j]);
        }
        o[j] = (bf16)(v * ea);
        xw[j] = (bf16)((float)in.x[i][j] * wt);
      }
      *reinterpret_cast<bf16x8*>(sG + t * LDX + c) = o;
      *reinterpret_cast<bf16x8*>(sXW + t * LDX + c) = xw;
    }
    if (AHEAD && !b_once) {
#pragma unroll
      for (int i = 0; i < VB; ++i) {
        const int e = (i * NTHR + tid) * 8, t = e / N, c = e % N;
        *reinterpret_cast<bf16x8*>(sB + t * LDB + c) = in.b[i];
      }
    }
    __syncthreads();
    if constexpr (AHEAD) {
      if (ih + 1 < nh) fetch(h + 1, in);
    }
    // wave w: p rows [16 (w PBW + i), ...), all n tiles, for both products (one after
    // the other: their tiles would not fit in registers together at headdim 128)
#pragma unroll 1
    for (int which = 0; which < 2; ++which) {
      const bf16* sa = which ? sXW : sG;
      const bf16* sb = which ? sB : sC;
      f32x4 acc[PBW][N / 16];
#pragma unroll
      for (int i = 0; i < PBW; ++i)
#pragma unroll
        for (int j = 0; j < N / 16; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k0 = 0; k0 < L; k0 += 32) {
        bf16x8 bf[N / 16];
#pragma unroll
        for (int j = 0; j < N / 16; ++j) bf[j] = frag_t(sb, LDB, k0, 16 * j, lane);
#pragma unroll
        for (int i = 0; i < PBW; ++i) {
          const bf16x8 af = frag_t(sa, LDX, k0, 16 * (wave * PBW + i), lane);
#pragma unroll
          for (int j = 0; j < N / 16; ++j) acc[i][j] = mfma16(af, bf[j], acc[i][j]);
        }
      }
      bf16* dst = (which ? p.sloc : p.loc) + ((int64_t)r * H + h) * P * N;
#pragma unroll
      for (int i = 0; i < PBW; ++i)
#pragma unroll
        for (int j = 0; j < N / 16; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            dst[(16 * (wave * PBW + i) + 4 * q4 + v) * N + 16 * j + l16] = (bf16)acc[i][j][v];
    }
  }
}

// ---------------------------------------------------------------------------
// scans over a sequence's chunks, 4 state elements per thread, PF chunks' loads in
// flight ahead of the dependent chain:
//   forward: S0(first) = h0 (or 0), S0(c+1) = e^{A_L(c)} S0(c) + sloc(c)
//   reverse: dS1(last) = dT (or 0), dS1(c-1) = e^{A_L(c)} dS1(c) + loc(c); dh0 =
//            the value before the first chunk
// ---------------------------------------------------------------------------
constexpr int PF = 4;
__device__ __forceinline__ f32x4 ld4(const float* q) { return *reinterpret_cast<const f32x4*>(q); }
__device__ __forceinline__ f32x4 ld4(const bf16* q) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(q);
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
__device__ __forceinline__ void st4b(bf16* q, f32x4 v) {
  *reinterpret_cast<bf16x4*>(q) = bf16x4{(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
}

__global__ __launch_bounds__(256) void ssd_bwd_scan_kernel(Params p, int PN) {
  const int H = p.H;
  const int n = blockIdx.x / H, h = blockIdx.x % H;
  const int first = p.seqs[2 * n], cnt = p.seqs[2 * n + 1];
  const int e = (blockIdx.y * 256 + threadIdx.x) * 4;
  if (e >= PN) return;
  const int64_t sb = ((int64_t)n * H + h) * PN + e;
  auto off = [&](int k) { return ((int64_t)(first + k) * H + h) * PN + e; };
  auto dec = [&](int k) { return p.edec[(int64_t)(first + k) * H + h]; };
  // Chain position m of a direction: chunk k = m (forward) or cnt-1-m (reverse).
  // Full groups of PF run without branches (the prefetch index is clamped in
  // bounds), so each load is waited for only where it is used; the tail is guarded.
  auto chain = [&](bool fwd, f32x4 X, const bf16* src, bf16* dst) -> f32x4 {
    if (cnt == 0) return X;
    auto kk = [&](int m) { return fwd ? m : cnt - 1 - m; };
    f32x4 buf[PF];
#pragma unroll
    for (int j = 0; j < PF; ++j) buf[j] = ld4(src + off(kk(min(j, cnt - 1))));
    int m = 0;
    for (; m + PF <= cnt; m += PF) {
#pragma unroll
      for (int j = 0; j < PF; ++j) {
        const int k = kk(m + j);
        st4b(dst + off(k), X);
        const float d = dec(k);
        const f32x4 l = buf[j];
        buf[j] = ld4(src + off(kk(min(m + j + PF, cnt - 1))));
        X = X * d + l;
      }
    }
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      if (m + j < cnt) {
        const int k = kk(m + j);
        st4b(dst + off(k), X);
        X = X * dec(k) + buf[j];
      }
    }
    return X;
  };
  chain(true, p.h0 ? ld4(p.h0 + sb) : f32x4{0.f, 0.f, 0.f, 0.f}, p.sloc, p.S0);
  {
    const f32x4 G = chain(false, p.dT ? ld4(p.dT + sb) : f32x4{0.f, 0.f, 0.f, 0.f}, p.loc, p.dS1);
    if (p.dh0) *reinterpret_cast<f32x4*>(p.dh0 + sb) = G;
  }
}

// ---------------------------------------------------------------------------
// chunk kernel
// ---------------------------------------------------------------------------
template <int P, int N>
struct Lay {
  static constexpr int LDX = P + 8, LDB = N + 8, LDM = L + 8;
  static constexpr int OFF_X = 0;                          // x        [L][LDX]
  static constexpr int OFF_G = OFF_X + L * LDX * 2;        // g        [L][LDX]
  // dy and z (for dz) fit only at P = 64; headdim 128 takes no z
  static constexpr int ZW = P == 64 ? L * LDX * 2 : 0;
  static constexpr int OFF_DY = OFF_G + L * LDX * 2;       // dy       [L][LDX] (z only)
  static constexpr int OFF_Z = OFF_DY + ZW;                // z        [L][LDX] (z only)
  static constexpr int OFF_B = OFF_Z + ZW;                 // B        [L][LDB]
  static constexpr int OFF_C = OFF_B + L * LDB * 2;        // C        [L][LDB]
  static constexpr int OFF_S = OFF_C + L * LDB * 2;        // S0       [P][LDB]
  static constexpr int OFF_DS = OFF_S + P * LDB * 2;       // dS1      [P][LDB]
  static constexpr int OFF_M = OFF_DS + P * LDB * 2;       // M dt'    [L][LDM]
  static constexpr int OFF_W = OFF_M + L * LDM * 2;        // W        [L][LDM]
  static constexpr int OFF_F = OFF_W + L * LDM * 2;        // fp32 scalars
  static constexpr int FDD = 16, FDV = 16 + P / L;         // dD and D: P floats each
  static constexpr int NF = 16 + 2 * (P / L);              // scalar arrays of L floats
  static constexpr int BYTES = OFF_F + NF * L * 4 + 64;
  static_assert(BYTES <= 160 * 1024, "LDS budget");
};
// scalar arrays
enum { F_DT, F_ACS, F_EA, F_E, F_FAC, F_ROWR, F_DAS, F_DDS,
       F_CMQ0, F_CR0 = F_CMQ0 + 4 };   // F_CR0 + 4 = 16 arrays, then dD and D (Lay)

// One head's inputs for the chunk, loaded into registers while the head before it
// is computed: x, dy, z rows (2 vectors per thread), S0 and dS1 (4 each), B rows
// (4, when B is not staged once per workgroup), the raw dt of token `lane` (wave 0)
// and D of feature `tid` (tid < 64).
template <int P, int N>
struct HeadIn {
  bf16x8 x[L * P / 8 / NTHR], dy[L * P / 8 / NTHR], z[L * P / 8 / NTHR];
  bf16x8 s0[P * N / 8 / NTHR], ds[P * N / 8 / NTHR], b[L * N / 8 / NTHR];
  uint32_t dt;   // as stored (converted where the scalars are formed)
  float d;
};

template <int P, int N>
__global__ __launch_bounds__(NTHR, 1) void ssd_bwd_chunk_kernel(Params p) {
  static_assert((P == 64 || P == 128) && (N == 64 || N == 128), "tile shape");
  // headdim 64 loads the next head's inputs during the current head's products;
  // at 128 they would not fit in registers beside the products' tiles
  constexpr bool AHEAD = P == 64;
  using K = Lay<P, N>;
  constexpr int LDX = K::LDX, LDB = K::LDB, LDM = K::LDM, NT = N / 16;
  extern __shared__ __align__(16) unsigned char smem[];
  bf16* sX = reinterpret_cast<bf16*>(smem + K::OFF_X);
  bf16* sG = reinterpret_cast<bf16*>(smem + K::OFF_G);
  bf16* sDY = reinterpret_cast<bf16*>(smem + K::OFF_DY);
  bf16* sZ = reinterpret_cast<bf16*>(smem + K::OFF_Z);
  bf16* sB = reinterpret_cast<bf16*>(smem + K::OFF_B);
  bf16* sC = reinterpret_cast<bf16*>(smem + K::OFF_C);
  bf16* sS = reinterpret_cast<bf16*>(smem + K::OFF_S);
  bf16* sDS = reinterpret_cast<bf16*>(smem + K::OFF_DS);
  bf16* sM = reinterpret_cast<bf16*>(smem + K::OFF_M);
  bf16* sW = reinterpret_cast<bf16*>(smem + K::OFF_W);
  float* sF = reinterpret_cast<float*>(smem + K::OFF_F);
  auto F = [&](int a, int t) -> float& { return sF[a * L + t]; };
  float* sHD = sF + K::NF * L;   // [0]: <dS1, S0>

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, l16 = lane & 15;
  const int H = p.H, GC = p.GC, HC = H / GC, HB = H / p.G, HXS = H / p.HX;
  // one workgroup per (chunk, C group): the group's HC heads in turn
  const int r = blockIdx.x / GC, gc = blockIdx.x % GC;
  const Row ro = load_row(p.seg, r);
  const int tok0 = ro.bos, nval = ro.eos - ro.bos;
  const int h_first = gc * HC;
  // B staged once when the workgroup's heads are exactly one B group; dB then sums
  // over them in registers.  Otherwise B is per head (stored) or shared wider
  // (atomics).
  const bool b_once = p.G == GC;
  constexpr int VX = L * P / 8 / NTHR, VS = P * N / 8 / NTHR, VB = L * N / 8 / NTHR;

  if (tid == 0) sHD[0] = 0.f;
  if (tid < P) F(K::FDD, tid) = 0.f;
  // C (and B when shared by all the heads) once
#pragma unroll
  for (int i = 0; i < VB; ++i) {
    const int e = (i * NTHR + tid) * 8, t = e / N, c = e % N;
    bf16x8 cv = {}, bv = {};
    if (t < nval) {
      cv = *reinterpret_cast<const bf16x8*>(p.C + (int64_t)(tok0 + t) * p.c_ts + (int64_t)gc * p.c_gs + c);
      if (b_once)
        bv = *reinterpret_cast<const bf16x8*>(p.B + (int64_t)(tok0 + t) * p.b_ts +
                                              (int64_t)(h_first / HB) * p.b_gs + c);
    }
    *reinterpret_cast<bf16x8*>(sC + t * LDB + c) = cv;
    if (b_once) *reinterpret_cast<bf16x8*>(sB + t * LDB + c) = bv;
  }

  const auto fetch = [&](int h, HeadIn<P, N>& q) {
    const int hx = h / HXS, g = h / HB;
#pragma unroll
    for (int i = 0; i < VX; ++i) {
      const int e = (i * NTHR + tid) * 8, t = e / P, c = e % P;
      q.x[i] = q.dy[i] = q.z[i] = bf16x8{};
      if (t < nval) {
        q.x[i] = *reinterpret_cast<const bf16x8*>(p.x + (int64_t)(tok0 + t) * p.x_ts + (int64_t)hx * p.x_hs + c);
        q.dy[i] = *reinterpret_cast<const bf16x8*>(p.dy + (int64_t)(tok0 + t) * p.dy_ts + (int64_t)h * p.dy_hs + c);
        if (p.z) q.z[i] = *reinterpret_cast<const bf16x8*>(p.z + (int64_t)(tok0 + t) * p.z_ts + (int64_t)h * p.z_hs + c);
      }
    }
    const bf16* s0 = p.S0 + ((int64_t)r * H + h) * P * N;
    const bf16* ds = p.dS1 + ((int64_t)r * H + h) * P * N;
#pragma unroll
    for (int i = 0; i < VS; ++i) {
      const int e = (i * NTHR + tid) * 8;
      q.s0[i] = *reinterpret_cast<const bf16x8*>(s0 + e);
      q.ds[i] = *reinterpret_cast<const bf16x8*>(ds + e);
    }
    if (!b_once) {
#pragma unroll
      for (int i = 0; i < VB; ++i) {
        const int e = (i * NTHR + tid) * 8, t = e / N, c = e % N;
        q.b[i] = bf16x8{};
        if (t < nval)
          q.b[i] = *reinterpret_cast<const bf16x8*>(p.B + (int64_t)(tok0 + t) * p.b_ts + (int64_t)g * p.b_gs + c);
      }
    }
    q.dt = (wave == 0 && lane < nval)
               ? ld_bits(p.dt, (int64_t)(tok0 + lane) * p.dt_ts + (int64_t)h * p.dt_hs, p.dt_dt) : 0u;
    q.d = (p.D && tid < P) ? p.D[(int64_t)h * P + tid] : 0.f;
  };

  HeadIn<P, N> in;
  if constexpr (AHEAD) fetch(h_first, in);
  f32x4 dCacc[NT], dBacc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) { dCacc[j] = f32x4{0.f, 0.f, 0.f, 0.f}; dBacc[j] = dCacc[j]; }

  for (int ih = 0; ih < HC; ++ih) {
  const int h = h_first + ih, hx = h / HXS, g = h / HB;
  const float A_h = p.A[h];
  if constexpr (!AHEAD) fetch(h, in);

  // ---- staging from registers: x, g = dy silu(z), dy and z with the dD partials;
  // S0 and dS1 with <dS1, S0>; B when per head; the token scalars and D ----------
  {
    float dd[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < VX; ++i) {
      const int e = (i * NTHR + tid) * 8, t = e / P, c = e % P;
      bf16x8 gv;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float gj = (float)in.dy[i][j];
        if (p.z) gj *= silu((float)in.z[i][j]);
        gv[j] = (bf16)gj;
        dd[j] += gj * (float)in.x[i][j];
      }
      *reinterpret_cast<bf16x8*>(sX + t * LDX + c) = in.x[i];
      *reinterpret_cast<bf16x8*>(sG + t * LDX + c) = gv;
      if constexpr (P == 64) {
        if (p.z) {
          *reinterpret_cast<bf16x8*>(sDY + t * LDX + c) = in.dy[i];
          *reinterpret_cast<bf16x8*>(sZ + t * LDX + c) = in.z[i];
        }
      }
    }
    if (p.dD) {
      const int c = (tid * 8) % P;
#pragma unroll
      for (int j = 0; j < 8; ++j) atomicAdd(&F(K::FDD, c + j), dd[j]);
    }
    float hd = 0.f;
#pragma unroll
    for (int i = 0; i < VS; ++i) {
      const int e = (i * NTHR + tid) * 8, pr = e / N, c = e % N;
      *reinterpret_cast<bf16x8*>(sS + pr * LDB + c) = in.s0[i];
      *reinterpret_cast<bf16x8*>(sDS + pr * LDB + c) = in.ds[i];
#pragma unroll
      for (int j = 0; j < 8; ++j) hd += (float)in.s0[i][j] * (float)in.ds[i][j];
    }
    hd = wave_sum(hd);
    if (lane == 0) atomicAdd(sHD, hd);
    if (!b_once) {
#pragma unroll
      for (int i = 0; i < VB; ++i) {
        const int e = (i * NTHR + tid) * 8, t = e / N, c = e % N;
        *reinterpret_cast<bf16x8*>(sB + t * LDB + c) = in.b[i];
      }
    }
    if (tid < P) F(K::FDV, tid) = in.d;
    if (wave == 0) {
      const Tok tk = token_scalars_raw(p, h, bits_f32(in.dt, p.dt_dt), nval, lane);
      const float aend = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, tk.acs), 63));
      F(F_DT, lane) = tk.dtv;
      F(F_ACS, lane) = tk.acs;
      F(F_EA, lane) = fast_exp(tk.acs);
      F(F_E, lane) = fast_exp(aend - tk.acs);
      F(F_FAC, lane) = tk.fac;
    }
  }
  __syncthreads();
  // the next head's inputs load during this head's products (no other vector load
  // is issued until they are used)
  if constexpr (AHEAD) {
    if (ih + 1 < HC) fetch(h + 1, in);
  }
  if (p.dD && tid < P) {
    unsafeAtomicAdd(p.dD + (int64_t)h * P + tid, F(K::FDD, tid));
    F(K::FDD, tid) = 0.f;   // the next head's staging adds after the closing barrier
  }

  // ---- step A: CB and Q (rows t of wave's block, all s), M dt' and W to LDS ----
  {
    f32x4 cb[4], qq[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) { cb[j] = f32x4{0.f, 0.f, 0.f, 0.f}; qq[j] = cb[j]; }
#pragma unroll
    for (int k0 = 0; k0 < N; k0 += 32) {
      const bf16x8 a = frag(sC, LDB, 16 * wave, k0, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) cb[j] = mfma16(a, frag(sB, LDB, 16 * j, k0, lane), cb[j]);
    }
#pragma unroll
    for (int k0 = 0; k0 < P; k0 += 32) {
      const bf16x8 a = frag(sG, LDX, 16 * wave, k0, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) qq[j] = mfma16(a, frag(sX, LDX, 16 * j, k0, lane), qq[j]);
    }
    float rowr[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int s = 16 * j + l16;
      const float acs_s = F(F_ACS, s), dt_s = F(F_DT, s);
      float cmq = 0.f, cr = 0.f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int t = 16 * wave + 4 * q4 + v;
        const float dec = s <= t ? fast_exp(F(F_ACS, t) - acs_s) : 0.f;
        const float m = cb[j][v] * dec;
        const float w = dt_s * qq[j][v] * dec;
        const float rr = w * cb[j][v];
        cmq += m * qq[j][v];
        cr += rr;
        rowr[v] += rr;
        sM[t * LDM + s] = (bf16)(m * dt_s);
        sW[t * LDM + s] = (bf16)w;
      }
      // column sums over the wave's 16 rows: the four lane groups
      cmq += shfl_xor(cmq, 16);
      cmq += shfl_xor(cmq, 32);
      cr += shfl_xor(cr, 16);
      cr += shfl_xor(cr, 32);
      if (q4 == 0) {
        F(F_CMQ0 + wave, s) = cmq;
        F(F_CR0 + wave, s) = cr;
      }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float rs = row16_sum(rowr[v]);
      if (l16 == 0) F(F_ROWR, 16 * wave + 4 * q4 + v) = rs;
    }
  }
  __syncthreads();

  // ---- step B1: y' = M dt' x + e^{A_t} C S0^T + D x -> dz, and g . (e^A C S0^T) --
  {
    f32x4 yi[P / 16], ys[P / 16];
#pragma unroll
    for (int i = 0; i < P / 16; ++i) { yi[i] = f32x4{0.f, 0.f, 0.f, 0.f}; ys[i] = yi[i]; }
    if (P == 64 && p.z) {   // y' only feeds dz
#pragma unroll
      for (int k0 = 0; k0 < L; k0 += 32) {
        const bf16x8 a = frag(sM, LDM, 16 * wave, k0, lane);
#pragma unroll
        for (int i = 0; i < P / 16; ++i) yi[i] = mfma16(a, frag_t(sX, LDX, k0, 16 * i, lane), yi[i]);
      }
    }
#pragma unroll
    for (int k0 = 0; k0 < N; k0 += 32) {
      const bf16x8 a = frag(sC, LDB, 16 * wave, k0, lane);
#pragma unroll
      for (int i = 0; i < P / 16; ++i) ys[i] = mfma16(a, frag(sS, LDB, 16 * i, k0, lane), ys[i]);
    }
    float das[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int t = 16 * wave + 4 * q4 + v;
      const float ea = F(F_EA, t);
#pragma unroll
      for (int i = 0; i < P / 16; ++i) {
        const int pc = 16 * i + l16;
        const float y_s = ea * ys[i][v];
        das[v] += (float)sG[t * LDX + pc] * y_s;
        if (P == 64 && p.z && t < nval) {
          float yp = yi[i][v] + y_s;
          if (p.D) yp += F(K::FDV, pc) * (float)sX[t * LDX + pc];
          const float zf = (float)sZ[t * LDX + pc];
          const float sg = __builtin_amdgcn_rcpf(1.f + fast_exp(-zf));
          const float dsilu = sg * (1.f + zf * (1.f - sg));
          p.dz[(int64_t)(tok0 + t) * H * P + (int64_t)h * P + pc] =
              (bf16)((float)sDY[t * LDX + pc] * yp * dsilu);
        }
      }
      const float rs = row16_sum(das[v]);
      if (l16 == 0) F(F_DAS, t) = rs;
    }
  }

  // ---- step B2: dx = (M dt')^T g + e dt' (dS1 B)^T + D g, and x . (dS1 B) -------
  {
    f32x4 dxi[P / 16], dhb[P / 16];
#pragma unroll
    for (int i = 0; i < P / 16; ++i) { dxi[i] = f32x4{0.f, 0.f, 0.f, 0.f}; dhb[i] = dxi[i]; }
#pragma unroll
    for (int k0 = 0; k0 < L; k0 += 32) {
      const bf16x8 a = frag_t(sM, LDM, k0, 16 * wave, lane);
#pragma unroll
      for (int i = 0; i < P / 16; ++i) dxi[i] = mfma16(a, frag_t(sG, LDX, k0, 16 * i, lane), dxi[i]);
    }
#pragma unroll
    for (int k0 = 0; k0 < N; k0 += 32) {
      const bf16x8 a = frag(sB, LDB, 16 * wave, k0, lane);
#pragma unroll
      for (int i = 0; i < P / 16; ++i) dhb[i] = mfma16(a, frag(sDS, LDB, 16 * i, k0, lane), dhb[i]);
    }
    float dds[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int s = 16 * wave + 4 * q4 + v;
      const float e = F(F_E, s), dt_s = F(F_DT, s);
#pragma unroll
      for (int i = 0; i < P / 16; ++i) {
        const int pc = 16 * i + l16;
        dds[v] += (float)sX[s * LDX + pc] * dhb[i][v];
        if (s < nval) {
          float d = dxi[i][v] + e * dt_s * dhb[i][v];
          if (p.D) d += F(K::FDV, pc) * (float)sG[s * LDX + pc];
          const int64_t ix = (int64_t)(tok0 + s) * p.HX * P + (int64_t)hx * P + pc;
          if (p.x_shared) unsafeAtomicAdd(static_cast<float*>(p.dx) + ix, d);
          else st_grad(p.dx, ix, d, p.gbf16);
        }
      }
      const float rs = row16_sum(dds[v]);
      if (l16 == 0) F(F_DDS, s) = e * rs;
    }
  }

  // ---- step B3: dC += e^{A_t} g S0 + W B (summed over the workgroup's heads) -------
  {
    f32x4 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k0 = 0; k0 < P; k0 += 32) {
      const bf16x8 a = frag(sG, LDX, 16 * wave, k0, lane);
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[j] = mfma16(a, frag_t(sS, LDB, k0, 16 * j, lane), acc[j]);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float ea = F(F_EA, 16 * wave + 4 * q4 + v);
#pragma unroll
      for (int j = 0; j < NT; ++j) dCacc[j][v] += acc[j][v] * ea;
    }
#pragma unroll
    for (int k0 = 0; k0 < L; k0 += 32) {
      const bf16x8 a = frag(sW, LDM, 16 * wave, k0, lane);
#pragma unroll
      for (int j = 0; j < NT; ++j) dCacc[j] = mfma16(a, frag_t(sB, LDB, k0, 16 * j, lane), dCacc[j]);
    }
  }

  // ---- step B4: dB = e dt' x dS1 + W^T C (summed over the heads when B is staged
  // once; otherwise this head's, stored or added) ------------------------------------
  {
    f32x4 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k0 = 0; k0 < P; k0 += 32) {
      const bf16x8 a = frag(sX, LDX, 16 * wave, k0, lane);
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[j] = mfma16(a, frag_t(sDS, LDB, k0, 16 * j, lane), acc[j]);
    }
    if (!b_once) {
#pragma unroll
      for (int j = 0; j < NT; ++j) dBacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int s_ = 16 * wave + 4 * q4 + v;
      const float f = F(F_E, s_) * F(F_DT, s_);
#pragma unroll
      for (int j = 0; j < NT; ++j) dBacc[j][v] += acc[j][v] * f;
    }
#pragma unroll
    for (int k0 = 0; k0 < L; k0 += 32) {
      const bf16x8 a = frag_t(sW, LDM, k0, 16 * wave, lane);
#pragma unroll
      for (int j = 0; j < NT; ++j) dBacc[j] = mfma16(a, frag_t(sC, LDB, k0, 16 * j, lane), dBacc[j]);
    }
    if (!b_once) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int s_ = 16 * wave + 4 * q4 + v;
        if (s_ >= nval) continue;
        const int64_t row = (int64_t)(tok0 + s_) * p.G * N + (int64_t)g * N;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          if (p.b_shared) unsafeAtomicAdd(static_cast<float*>(p.dB) + row + 16 * j + l16, dBacc[j][v]);
          else st_grad(p.dB, row + 16 * j + l16, dBacc[j][v], p.gbf16);
        }
      }
    }
  }
  __syncthreads();

  // ---- scalar chain: dA_t, da (reverse cumsum), d dt, dA_h, d dt_bias --------------
  if (wave == 0) {
    const int t = lane;
    const float dt_t = F(F_DT, t), dds = F(F_DDS, t);
    float dacs = F(F_ROWR, t) + F(F_DAS, t) - dt_t * dds;
    float cmq = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      dacs -= F(F_CR0 + w, t);
      cmq += F(F_CMQ0 + w, t);
    }
    // <dS1, S1> = e^{A_L} <dS1, S0> + sum_s dt'_s e_s x_s . (dS1 B_s), on the last token
    const float tail = wave_sum(dt_t * dds);
    const float aend = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
        __builtin_bit_cast(int, F(F_ACS, t)), 63));
    if (t == L - 1) dacs += fast_exp(aend) * sHD[0] + tail;
    const float incl = scan64(dacs, lane);
    const float total = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, incl), 63));
    const float da = total - incl + dacs;   // sum_{u >= t} dA_u
    const float ddtv = cmq + dds + A_h * da;
    const float ddt_raw = ddtv * F(F_FAC, t);
    if (t < nval) p.ddt[(int64_t)(tok0 + t) * H + h] = ddt_raw;
    const float sa = wave_sum(dt_t * da);
    const float sb = wave_sum(ddt_raw);
    if (lane == 0) {
      unsafeAtomicAdd(p.dA + h, sa);
      if (p.dbias) unsafeAtomicAdd(p.dbias + h, sb);
      sHD[0] = 0.f;   // lane 63 read it above; the next head adds after the barrier
    }
  }
  __syncthreads();   // LDS free for the next head
  }   // heads

  // dC of the C group (and dB of the B group staged once), summed over the heads
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int t = 16 * wave + 4 * q4 + v;
    if (t >= nval) continue;
    const int64_t rc = (int64_t)(tok0 + t) * GC * N + (int64_t)gc * N;
    const int64_t rb = (int64_t)(tok0 + t) * p.G * N + (int64_t)gc * N;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      st_grad(p.dC, rc + 16 * j + l16, dCacc[j][v], p.gbf16);
      if (b_once) st_grad(p.dB, rb + 16 * j + l16, dBacc[j][v], p.gbf16);
    }
  }
}

template <int P, int N>
void launch(const Params& p, hipStream_t s) {
  constexpr int lsm = local_lds_bytes<P, N>();
  constexpr int smem = Lay<P, N>::BYTES;
  (void)hipFuncSetAttribute((const void*)ssd_bwd_local_kernel<P, N>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, lsm);
  (void)hipFuncSetAttribute((const void*)ssd_bwd_chunk_kernel<P, N>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, smem);
  hipLaunchKernelGGL((ssd_bwd_local_kernel<P, N>), dim3(p.nrows * (P == 64 ? p.GC : p.H)),
                     dim3(NTHR), lsm, s, p);
  hipLaunchKernelGGL(ssd_bwd_scan_kernel, dim3(p.nseq * p.H, (P * N + 1023) / 1024), dim3(256), 0,
                     s, p, P * N);
  hipLaunchKernelGGL((ssd_bwd_chunk_kernel<P, N>), dim3(p.nrows * p.GC), dim3(NTHR), smem, s, p);
}

}  // namespace ssdb
}  // namespace hmx

using namespace hmx;
using namespace hmx::ssdb;

extern "C" size_t hmx_ssd_chunk_bwd_workspace_bytes(int32_t nrows, int32_t H, int32_t P, int32_t N) {
  const size_t st = (size_t)nrows * H * P * N;
  return st * (2 + 2 + 2 + 2) + (size_t)nrows * H * 4 + 256;
}

extern "C" int hmx_ssd_chunk_bwd(
    const void* x, int64_t x_ts, int64_t x_hs, const void* B, int64_t b_ts, int64_t b_gs,
    const void* C, int64_t c_ts, int64_t c_gs, int32_t xbc_dtype, const void* dt, int32_t dt_dtype,
    int64_t dt_ts, int64_t dt_hs, const float* A, const float* D, const float* dt_bias,
    const void* z, int64_t z_ts, int64_t z_hs, const void* dy, int64_t dy_ts, int64_t dy_hs,
    const float* h0, const float* d_final, const int32_t* seg_table,
    int32_t nrows, const int32_t* seq_table, int32_t nseq, int32_t H, int32_t HX, int32_t G,
    int32_t GC, int32_t P, int32_t N, int32_t dt_softplus, float dt_min, float dt_max, void* dx,
    void* dB, void* dC, int32_t grad_dtype, void* dz, float* ddt, float* dA, float* dD, float* ddt_bias,
    float* dh0, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "hmx_ssd_chunk_bwd";
  HMX_REQUIRE(xbc_dtype == HMX_BF16, HMX_EUNSUPPORTED, "%s: x/B/C/z/dy must be bfloat16", fn);
  HMX_REQUIRE((P == 64 || P == 128) && (N == 64 || N == 128), HMX_EUNSUPPORTED,
              "%s: headdim and d_state in {64,128} (got %d, %d)", fn, P, N);
  HMX_REQUIRE(P == 64 || !z, HMX_EUNSUPPORTED, "%s: the z gate needs headdim 64", fn);
  HMX_REQUIRE(grad_dtype == HMX_F32 ||
                  (grad_dtype == HMX_BF16 && HX == H && (G == H || G == GC)),
              HMX_EUNSUPPORTED,
              "%s: dx / dB / dC in bf16 need unshared x and B (HX = H; G = H or G = GC)", fn);
  HMX_REQUIRE(H > 0 && HX > 0 && G > 0 && GC > 0 && H % HX == 0 && H % G == 0 && H % GC == 0,
              HMX_EINVAL, "%s: H=%d must be a multiple of HX=%d, G=%d and GC=%d", fn, H, HX, G, GC);
  HMX_REQUIRE(x && B && C && dt && A && dy && seg_table && seq_table && dx && dB && dC && ddt && dA &&
                  (!z || dz) && nrows >= 0 && nseq >= 0,
              HMX_EINVAL, "%s: null pointer", fn);
  HMX_REQUIRE(dt_dtype == HMX_F32 || dt_dtype == HMX_BF16 || dt_dtype == HMX_F16, HMX_EINVAL,
              "%s: dt dtype code %d", fn, dt_dtype);
  const int64_t strides[] = {x_ts, x_hs, b_ts, b_gs, c_ts, c_gs, dy_ts, dy_hs,
                             z ? z_ts : 8, z ? z_hs : 8};
  for (int64_t st : strides)
    HMX_REQUIRE(st % 8 == 0, HMX_EINVAL, "%s: token/head strides must be multiples of 8", fn);
  HMX_REQUIRE(((uintptr_t)x | (uintptr_t)B | (uintptr_t)C | (uintptr_t)dy | (uintptr_t)z |
               (uintptr_t)h0 | (uintptr_t)d_final | (uintptr_t)dh0) % 16 == 0,
              HMX_EINVAL, "%s: operands must be 16-byte aligned", fn);
  if (nrows == 0 && nseq == 0) return HMX_OK;
  const size_t need = hmx_ssd_chunk_bwd_workspace_bytes(nrows, H, P, N);
  HMX_REQUIRE(workspace && workspace_bytes >= need, HMX_EINVAL,
              "%s: workspace of %zu bytes needed, %zu given", fn, need, workspace_bytes);
  Params p;
  p.x = static_cast<const bf16*>(x); p.x_ts = x_ts; p.x_hs = x_hs;
  p.B = static_cast<const bf16*>(B); p.b_ts = b_ts; p.b_gs = b_gs;
  p.C = static_cast<const bf16*>(C); p.c_ts = c_ts; p.c_gs = c_gs;
  p.dt = dt; p.dt_dt = dt_dtype; p.dt_ts = dt_ts; p.dt_hs = dt_hs;
  p.A = A; p.D = D; p.dt_bias = dt_bias;
  p.z = static_cast<const bf16*>(z); p.z_ts = z_ts; p.z_hs = z_hs;
  p.dy = static_cast<const bf16*>(dy); p.dy_ts = dy_ts; p.dy_hs = dy_hs;
  p.h0 = h0; p.dT = d_final;
  p.seg = seg_table; p.seqs = seq_table; p.nrows = nrows; p.nseq = nseq;
  const size_t st = (size_t)nrows * H * P * N;
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  p.loc = reinterpret_cast<bf16*>(ws);
  p.sloc = reinterpret_cast<bf16*>(ws + st * 2);
  p.S0 = reinterpret_cast<bf16*>(ws + st * 4);
  p.dS1 = reinterpret_cast<bf16*>(ws + st * 6);
  p.edec = reinterpret_cast<float*>(ws + st * 8);
  p.dx = dx; p.x_shared = HX < H;
  p.dB = dB; p.b_shared = G < H;
  p.dC = dC; p.gbf16 = grad_dtype == HMX_BF16;
  p.dz = static_cast<bf16*>(dz); p.ddt = ddt; p.dA = dA; p.dD = dD; p.dbias = ddt_bias;
  p.dh0 = dh0;
  p.H = H; p.HX = HX; p.G = G; p.GC = GC; p.softplus = dt_softplus;
  p.dt_min = dt_min; p.dt_max = dt_max;
  hipStream_t s = (hipStream_t)stream;
  if (nrows == 0) {   // empty sequences only: dh0 = dT
    hipLaunchKernelGGL(ssd_bwd_scan_kernel, dim3(nseq * H, (P * N + 1023) / 1024), dim3(256), 0, s,
                       p, P * N);
    return check_launch(fn);
  }
  if (P == 64 && N == 128) launch<64, 128>(p, s);
  else if (P == 64) launch<64, 64>(p, s);
  else if (N == 128) launch<128, 128>(p, s);
  else launch<128, 64>(p, s);
  return check_launch(fn);
}
