// Mamba2 SSD chunk scan (mamba_chunk_scan_combined / _varlen) for gfx950:
// bf16 x/B/C/z/y, fp32 dt math and fp32 states.
//
// Semantics (per head h, group g = h / (H/G), state S in R^{P x N}; the
// reference calls sit at training/.../layers/mamba/mamba2.py:555-580 and
// vllm-inference/src/primed_vllm/primed_mamba2_layer.py:844-863; the kernels
// there are mamba_ssm 2.3.0 / vLLM 0.15.1, not vendored):
//   dt'_t = clamp(softplus_20(dt_t + dt_bias_h), dt_min, dt_max)
//   S_t   = e^{dt'_t A_h} S_{t-1} + dt'_t x_t B_t^T
//   y_t   = S_t C_t + D_hp x_t ;  y_t *= z_t sigmoid(z_t) if z is given
//
// Chunked form over L = 64 tokens with a_t = dt'_t A_h and A_t = sum_{s<=t} a_s
// (inclusive, from the chunk start):
//   M[t][j] = (C_t . B_j) e^{A_t - A_j} dt'_j        (j <= t)
//   Y       = diag(e^{A}) C S^T + M X  (+ D x, z gate)
//   S^T    <- e^{A_L} S^T + B^T diag(dt' e^{A_L - A}) X
// The state lives transposed (S^T, rows n, columns p) in MFMA accumulator
// registers: wave w owns p-columns [16 PB w, 16 PB (w+1)) for every n, so the
// products with the state never leave the wave.  The output is formed
// transposed too (Y^T = S C^T + X^T M^T, rows p, columns t), and M as M^T = B C^T,
// so every tile leaves the accumulators as 4 consecutive features of one row (one
// 8-byte LDS write).  The state is linear with a scalar decay per chunk, so a
// segment's start state is exact from a scalar-decay combine of the other
// segments' zero-start end states (pass LOCAL + combine, the carry of
// mamba_mixer_cp_utils.py:44-65).
//
// Numerics: every MFMA operand is fp16 with fp32 accumulation.  x, B and C are
// bf16 inputs, which fp16 holds exactly within its range (|v| < 65504; below
// 6.1e-5 it keeps an absolute 6e-8); the fp32 factors S, M and w x are rounded
// to fp16 once each (11 significant bits, against bf16's 8: one bf16 rounding of
// M cost ~6e-3 absolute at |y| ~ 7, fp16's ~8e-4).  B and C are staged in the
// interleaved feature order (icol) so the operands that pair with a state built
// from two C-layout tiles are single 128-bit reads; row strides of 36 or 72
// dwords keep those reads bank-conflict-free.
//
// Workgroup order: the 1-D grid maps block ids so that the heads sharing one
// B/C group and segment have ids equal mod 8, i.e. land on one XCD and share
// its L2 for the B/C chunk reads.
//
// Roofline: HBM-bound at the C4 shape (x, y, B, C, dt and the final state move
// once; the LOCAL pass re-reads x, B and dt of all but the last segment).
#include <type_traits>

#include "common.hpp"
#include "mfma.hpp"

namespace hmx {
namespace ssd {

constexpr int L = 64;          // tokens per chunk
constexpr int NTHR = 256;

enum Mode { MODE_OUT = 0, MODE_LOCAL = 1 };

struct SegInfo { int n, bos, eos, c_start, c_end, seg_idx, first_seg, nseg; };

struct Params {
  const bf16* x; int64_t x_ts, x_hs;
  const bf16* B; int64_t b_ts, b_gs;
  const bf16* C; int64_t c_ts, c_gs;
  const void* dt; int dt_dt; int64_t dt_ts, dt_hs;
  const float* A;          // [H]
  const float* D;          // [H][P] or null
  const float* dt_bias;    // [H] or null
  const bf16* z; int64_t z_ts, z_hs;   // or null
  bf16* y; int64_t y_ts, y_hs;
  // Sequence n's state: slot sidx[n] (or n) of the h0 / hT bases ([H][P][N] slots
  // st_ss elements apart, f32 or bf16; they may be one pool).  A negative slot or
  // hinit[n] == 0 starts from zero; a negative slot writes nothing.  Only the
  // combine launch and single-segment workgroups read h0, so the last segment
  // writes its end state straight into the slot.
  const void* h0;          // or null
  void* hT;                // or null
  int64_t st_ss; int st_dt;
  const int* sidx;         // [nseq] or null
  const uint8_t* hinit;    // [nseq] or null
  const int* seg; int nseg_total;
  float* ws_loc;           // [nseg][H][P][N] zero-start segment end states
  float* ws_s0;            // [nseg][H][P][N] segment start states
  float* ws_dec;           // [nseg][H] segment log-decay sum_t a_t
  int* redo;               // [nseg][H]: 1 where the pass's walk left fp16's range
  // x has HX heads and C has GC groups, B has G groups (each divides H): head h
  // reads x head h / (H/HX), B group h / (H/G) and C group h / (H/GC).
  int H, HX, G, GC, softplus;
  float dt_min, dt_max;
};

// fp16 row strides (elements) for 64- and 128-wide rows: 36 and 72 dwords
constexpr int row_ld(int w) { return w == 64 ? w + 8 : w + 16; }

template <int P, int N>
struct Cfg {
  static constexpr int LDX = row_ld(P);   // fp16 [L][P] x; bf16 [L][P] y / z staging
  static constexpr int LDB = row_ld(N);   // fp16 [L][N] B, C (interleaved features)
  static constexpr int LDM = row_ld(L);   // fp16 [L][L] M (interleaved columns)
  static constexpr int PB = P / 64;       // 16-wide p-blocks per wave
  static constexpr int NB = N / 16;       // 16-row n-blocks of S^T
  static constexpr int VX = L * P / 8 / NTHR;   // 16-byte x vectors per thread
  static constexpr int VB = L * N / 8 / NTHR;   // 16-byte B (or C) vectors per thread
  static constexpr int OFF_X = 0;
  static constexpr int OFF_B = OFF_X + L * LDX * 2;
  static constexpr int OFF_S = OFF_B + L * LDB * 2;
  static constexpr int OFF_C = OFF_S + 2 * 4 * L * 4;   // two buffers of 4 scalar arrays
  static constexpr int OFF_M = OFF_C + L * LDB * 2;
  static constexpr int OFF_Y = OFF_M + L * LDM * 2;
  static constexpr int SMEM_LOCAL = OFF_C;              // x, B, scalars
  static constexpr int SMEM_OUT = OFF_Y + L * LDX * 2;
  static constexpr int OFF_ML = SMEM_OUT;               // bf16 [L][L] M's low parts (SAFE)
  static constexpr int SMEM_OUT_SAFE = OFF_ML + L * LDM * 2;
  // two workgroups per CU, except the OUT pass at P = 128 (one; see the kernel)
  static_assert(SMEM_LOCAL <= 80 * 1024, "LDS budget: two workgroups per CU");
  static_assert(SMEM_OUT <= (P == 128 ? 160 : 80) * 1024, "LDS budget");
  static_assert(SMEM_OUT_SAFE <= (P == 128 ? 160 : 80) * 1024, "LDS budget");
  static_assert(P % 64 == 0 && N % 32 == 0, "tile shape");
};

// per-token scalar arrays (fp32 [L] each)
enum { S_DT, S_ACS, S_W, S_EA };

// The raw bits of element i (one load in either dtype branch, so the wait for it
// can be placed where the value is used, after the loads issued later) and their
// value as a float.
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

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ float scan64(float x, int lane) {
  x = scan32(x);
  const float lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 31));
  return lane >= 32 ? x + lo : x;
}

template <int P, int N>
struct Raw {
  bf16x8 x[Cfg<P, N>::VX], z[Cfg<P, N>::VX], b[Cfg<P, N>::VB], c[Cfg<P, N>::VB];
  uint32_t dt;   // dt of token `lane` (last wave) as stored: converted when used
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// A raw buffer resource over rows 0 .. nrows-1 (w bf16 features each, ts elements
// apart) from base: accesses past them read zeros and write nothing, which masks a
// chunk's missing rows.  The base is uniform, so a chunk's addressing is scalar and
// each lane keeps one fixed byte offset per array (row tid / (w/8), features
// 8 (tid % (w/8)) ..); the i-th vector of a thread adds the uniform i * (rows per
// pass) * ts (the hardware's scalar offset).  The host keeps 64 rows of any stride
// inside 32-bit offsets.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const bf16* base, int nrows,
                                                           int64_t ts, int w) {
  const uint32_t bytes = nrows > 0 ? (uint32_t)(((int64_t)(nrows - 1) * ts + w) * 2) : 0u;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(base), 0, bytes, 0x00020000);
}
__device__ __forceinline__ bf16x8 ld_rows(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, off, soff, 0));
}
__device__ __forceinline__ uint32_t lane_off(int tid, int w, int64_t ts) {
  return (uint32_t)(((int64_t)(tid / (w / 8)) * ts + (tid % (w / 8)) * 8) * 2);
}

template <int P, int N, int MODE>
__device__ __forceinline__ void load_raw(Raw<P, N>& r, const Params& p, int tok0, int nval,
                                         int h, int hx, int g, int gc, int tid) {
  using K = Cfg<P, N>;
  constexpr int RX = NTHR / (P / 8), RB = NTHR / (N / 8);   // rows per pass
  const auto rx = rows_rsrc(p.x + (int64_t)tok0 * p.x_ts + (int64_t)hx * p.x_hs, nval, p.x_ts, P);
  const uint32_t ox = lane_off(tid, P, p.x_ts);
#pragma unroll
  for (int i = 0; i < K::VX; ++i) r.x[i] = ld_rows(rx, ox, (uint32_t)(i * RX * p.x_ts * 2));
  if (MODE == MODE_OUT) {
    if (p.z) {
      const auto rz = rows_rsrc(p.z + (int64_t)tok0 * p.z_ts + (int64_t)h * p.z_hs, nval, p.z_ts, P);
      const uint32_t oz = lane_off(tid, P, p.z_ts);
#pragma unroll
      for (int i = 0; i < K::VX; ++i) r.z[i] = ld_rows(rz, oz, (uint32_t)(i * RX * p.z_ts * 2));
    } else {
#pragma unroll
      for (int i = 0; i < K::VX; ++i) r.z[i] = bf16x8{};
    }
  }
  const auto rb = rows_rsrc(p.B + (int64_t)tok0 * p.b_ts + (int64_t)g * p.b_gs, nval, p.b_ts, N);
  const uint32_t ob = lane_off(tid, N, p.b_ts);
#pragma unroll
  for (int i = 0; i < K::VB; ++i) r.b[i] = ld_rows(rb, ob, (uint32_t)(i * RB * p.b_ts * 2));
  if (MODE == MODE_OUT) {
    const auto rc = rows_rsrc(p.C + (int64_t)tok0 * p.c_ts + (int64_t)gc * p.c_gs, nval, p.c_ts, N);
    const uint32_t oc = lane_off(tid, N, p.c_ts);
#pragma unroll
    for (int i = 0; i < K::VB; ++i) r.c[i] = ld_rows(rc, oc, (uint32_t)(i * RB * p.c_ts * 2));
  }
  const int t = tid - (NTHR - L);   // the last wave loads dt (lane t = token t)
  if (t >= 0)
    r.dt = t < nval ? ld_bits(p.dt, (int64_t)(tok0 + t) * p.dt_ts + h * p.dt_hs, p.dt_dt) : 0u;
}

// bf16 rows staged as they are (the SAFE pass): the 16-bit loads of the fp16 path
// move them unchanged
__device__ __forceinline__ f16x8 bits_h8(const bf16x8& x) { return __builtin_bit_cast(f16x8, x); }
__device__ __forceinline__ bf16x8 bits_b8(const f16x8& x) { return __builtin_bit_cast(bf16x8, x); }

__device__ __forceinline__ f16x8 to_h8(const bf16x8& x) {
  f16x8 y;
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = (f16)(float)x[j];
  return y;
}

// Two workgroups per CU, except the OUT pass at P = 128: its 128x128 state needs
// more than 256 registers, which at two waves per SIMD spill; at one wave per
// SIMD it keeps them in VGPRs + AGPRs.
//
// fp16 range.  The plain pass (SAFE false) rounds x, B, C, the state, M and w x to
// fp16 as they are; an entry past fp16's range becomes inf, which reaches the end
// state (x, B, w x) or y (C, M, the state's copy): the pass sums both and, when
// the sum is not finite, writes no end state and sets the walk's redo flag.  The
// SAFE pass walks the flagged ones again with bf16 operands: x, B and C as they
// are (exact), the state, M and w x as bf16 hi + lo pairs (~16 significant bits,
// two MFMAs per product), so any finite input stays in range.
template <int P, int N, int MODE, bool SAFE>
__global__ __launch_bounds__(NTHR, (P == 128 && MODE == MODE_OUT) ? 1 : 2) void ssd_chunk_kernel(Params p) {
  using K = Cfg<P, N>;
  constexpr int LDX = K::LDX, LDB = K::LDB, LDM = K::LDM, PB = K::PB, NB = K::NB;
  __shared__ __align__(16) unsigned char
      smem[MODE == MODE_OUT ? (SAFE ? K::SMEM_OUT_SAFE : K::SMEM_OUT) : K::SMEM_LOCAL];
  f16* sX = reinterpret_cast<f16*>(smem + K::OFF_X);
  f16* sB = reinterpret_cast<f16*>(smem + K::OFF_B);
  float* sc = reinterpret_cast<float*>(smem + K::OFF_S);
  f16* sC = reinterpret_cast<f16*>(smem + K::OFF_C);     // OUT only
  f16* sM = reinterpret_cast<f16*>(smem + K::OFF_M);     // OUT only
  bf16* sY = reinterpret_cast<bf16*>(smem + K::OFF_Y);   // OUT only
  f16* sML = reinterpret_cast<f16*>(smem + K::OFF_ML);   // OUT, SAFE only
  // per-token scalars, double-buffered by chunk parity: SC(buf, slot, t)
  auto SC = [&](int buf, int slot, int t) -> float& { return sc[(buf * 4 + slot) * L + t]; };
  auto SC4 = [&](int buf, int slot, int t) -> f32x4 {
    return *reinterpret_cast<const f32x4*>(&sc[(buf * 4 + slot) * L + t]);
  };

  const int tid = threadIdx.x, lane = tid & 63;
  // the wave index as a scalar: branches on it are uniform (MFMAs ignore EXEC)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, l16 = lane & 15;
  // XCD-aware block order: ids of the heads of one (segment, group) agree mod 8.
  const int H = p.H, G = p.G, HG = H / G;
  const int id = blockIdx.x, sg = id % (p.nseg_total * G);
  const int s_id = sg / G, g = sg % G, h = g * HG + id / (p.nseg_total * G);
  const int hx = h / (H / p.HX), gc = h / (H / p.GC);
  const SegInfo si = load_seg(p.seg, s_id);
  if (MODE == MODE_LOCAL && si.seg_idx == si.nseg - 1) {
    if (!SAFE && tid == 0) p.redo[s_id * H + h] = 0;   // no LOCAL walk here
    return;
  }
  if (SAFE && !p.redo[s_id * H + h]) return;

  const float A_h = p.A[h];
  const float bias = p.dt_bias ? p.dt_bias[h] : 0.f;

  // ---- initial state S^T: tile (nb, i) holds rows n = 16nb+4q4+v, column
  // p = 16(PB wave + i) + l16 --------------------------------------------------
  const int64_t slot = p.sidx ? (int64_t)p.sidx[si.n] : si.n;
  const int64_t soff = slot * p.st_ss + (int64_t)h * P * N;
  f32x4 ST[NB][PB];
  {
    const float* src = nullptr;
    const bf16* src16 = nullptr;
    if (MODE == MODE_OUT) {
      if (si.nseg == 1) {
        if (p.h0 && slot >= 0 && (!p.hinit || p.hinit[si.n])) {
          if (p.st_dt == HMX_BF16) src16 = static_cast<const bf16*>(p.h0) + soff;
          else src = static_cast<const float*>(p.h0) + soff;
        }
      } else {   // split: every segment's start state comes from the combine launch
        src = p.ws_s0 + ((int64_t)s_id * H + h) * P * N;
      }
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < PB; ++i) {
        const int pc = 16 * (PB * wave + i) + l16;
        const int64_t e = (int64_t)pc * N + 16 * nb + 4 * q4;
        f32x4 x = {0.f, 0.f, 0.f, 0.f};
        if (src) x = *reinterpret_cast<const f32x4*>(src + e);
        if (src16) {
          const bf16x4 b = *reinterpret_cast<const bf16x4*>(src16 + e);
          x = f32x4{(float)b[0], (float)b[1], (float)b[2], (float)b[3]};
        }
        ST[nb][i] = x;
      }
  }
  float dsum = 0.f;   // segment log-decay (LOCAL)

  // Raw chunks in flight: the light LOCAL pass keeps two (the loop is unrolled by
  // two so the register sets alternate statically: chunk c in `cur`, chunk c+1
  // arriving in `nxt`); the OUT pass, whose chunk work covers the load latency,
  // keeps one (cur == nxt, refilled with chunk c+1 after staging).
  constexpr int AHEAD = (MODE == MODE_LOCAL) ? 2 : 1;
  Raw<P, N> ra, rb;
  const auto nval_of = [&](int c) { return min(L, si.eos - (si.bos + c * L)); };
  if (si.c_start < si.c_end)
    load_raw<P, N, MODE>(ra, p, si.bos + si.c_start * L, nval_of(si.c_start), h, hx, g, gc, tid);
  if (AHEAD == 2 && si.c_start + 1 < si.c_end)
    load_raw<P, N, MODE>(rb, p, si.bos + (si.c_start + 1) * L, nval_of(si.c_start + 1), h, hx, g, gc, tid);

  // dt' = clamp(softplus(dt + bias)), A_t = cumsum(dt' A), w_t = dt' e^{A_L - A_t},
  // e^{A_t} of chunk c into scalar buffer `buf` (the last wave; lane = token)
  const auto make_scalars = [&](uint32_t dt_bits, int c, int buf) {
    float d = bits_f32(dt_bits, p.dt_dt) + bias;
    if (p.softplus) d = softplus20(d);
    d = fminf(fmaxf(d, p.dt_min), p.dt_max);
    if (lane >= nval_of(c)) d = 0.f;
    const float acs = scan64(d * A_h, lane);
    const float alast = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acs), 63));
    SC(buf, S_DT, lane) = d;
    SC(buf, S_ACS, lane) = acs;
    SC(buf, S_W, lane) = d * fast_exp(alast - acs);
    SC(buf, S_EA, lane) = fast_exp(acs);
  };
  if (MODE == MODE_LOCAL && si.c_start < si.c_end && wave == NTHR / 64 - 1)
    make_scalars(ra.dt, si.c_start, 0);
  // D of this wave's p-rows, loaded once (a load inside the loop would be waited
  // for with everything issued before it, the next chunk's rows included)
  f32x4 dreg[PB];
#pragma unroll
  for (int i = 0; i < PB; ++i)
    dreg[i] = (MODE == MODE_OUT && p.D)
                  ? *reinterpret_cast<const f32x4*>(p.D + h * P + 16 * (PB * wave + i) + 4 * q4)
                  : f32x4{0.f, 0.f, 0.f, 0.f};

  // coalesced store of the y tile staged in sY (chunk starting at tok0); the plain
  // pass also sums the rows (ysum: inf or NaN there flags the walk)
  float ysum = 0.f;
  const uint32_t oy = lane_off(tid, P, p.y_ts);
  const auto store_y = [&](int tok0, int nval) {
    const auto ry = rows_rsrc(p.y + (int64_t)tok0 * p.y_ts + (int64_t)h * p.y_hs, nval, p.y_ts, P);
#pragma unroll
    for (int i = 0; i < K::VX; ++i) {
      const int e = tid + NTHR * i, row = e / (P / 8), c8 = (e % (P / 8)) * 8;
      const bf16x8 yr = *reinterpret_cast<const bf16x8*>(sY + row * LDX + c8);
      if constexpr (!SAFE) {
#pragma unroll
        for (int j = 0; j < 8; j += 2)
          ysum = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{yr[j], yr[j + 1]},
                                                  bf16x2{(bf16)1.f, (bf16)1.f}, ysum, false);
      }
      // rows from nval on fall outside the resource: not written
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, yr), ry, oy,
                                             (uint32_t)(i * (NTHR / (P / 8)) * p.y_ts * 2), 0);
    }
  };

  // Per chunk (OUT): stage | Y^T = S C^T, M^T, state update | Y^T += X^T M^T +
  // epilogue, with the previous chunk's y stored while this one is staged.
  const auto chunk = [&](Raw<P, N>& cur, Raw<P, N>& nxt, int c) {
    const int tok0 = si.bos + c * L;
    const int cb = (c - si.c_start) & 1;
    // ---- stage chunk c (fp16; B and C interleaved), then refill `cur` ------------
#pragma unroll
    for (int i = 0; i < K::VX; ++i) {
      const int e = tid + NTHR * i, row = e / (P / 8), c8 = (e % (P / 8)) * 8;
      *reinterpret_cast<f16x8*>(sX + row * LDX + c8) = SAFE ? bits_h8(cur.x[i]) : to_h8(cur.x[i]);
    }
#pragma unroll
    for (int i = 0; i < K::VB; ++i) {
      const int e = tid + NTHR * i, row = e / (N / 8), c8 = (e % (N / 8)) * 8;
      store8_i(sB + row * LDB, c8, SAFE ? bits_h8(cur.b[i]) : to_h8(cur.b[i]));
      if (MODE == MODE_OUT)
        store8_i(sC + row * LDB, c8, SAFE ? bits_h8(cur.c[i]) : to_h8(cur.c[i]));
    }
    if (MODE == MODE_OUT && c > si.c_start) store_y(tok0 - L, L);
    bf16x8 zst[K::VX];
    if (MODE == MODE_OUT) {
#pragma unroll
      for (int i = 0; i < K::VX; ++i) zst[i] = cur.z[i];
    }
    // OUT keeps one raw chunk in flight: its scalars come from the chunk's own dt
    // here, before the refill (the staging above has waited for these rows), so the
    // chunk's work never waits for the rows in flight
    if (MODE == MODE_OUT && wave == NTHR / 64 - 1) make_scalars(cur.dt, c, cb);
    if (c + AHEAD < si.c_end)
      load_raw<P, N, MODE>(cur, p, tok0 + AHEAD * L, nval_of(c + AHEAD), h, hx, g, gc, tid);
    lds_barrier();
    const float al = SC(cb, S_ACS, L - 1);

    // X^T operands of this wave's p-columns, t in the paired-tile order
    // (t0 + 4q4 + v, t0 + 16 + 4q4 + v): the B operand of the state update (scaled
    // by w) and the A operand of X^T M^T
    f16x8 xt[PB][2];
#pragma unroll
    for (int i = 0; i < PB; ++i)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        xt[i][ks] = frag_t_perm_h(sX, LDX, 32 * ks, 16 * (PB * wave + i), lane);

    f32x4 YT[PB][4];   // Y^T tile (p rows 16(PB wave + i) + 4q4 + v, t columns 16tb + l16)
    if (MODE == MODE_OUT) {
      // z into the y staging buffer (read back per row by the owner lanes)
      if (p.z) {
#pragma unroll
        for (int i = 0; i < K::VX; ++i) {
          const int e = tid + NTHR * i, row = e / (P / 8), c8 = (e % (P / 8)) * 8;
          *reinterpret_cast<bf16x8*>(sY + row * LDX + c8) = zst[i];
        }
      }
      // ---- Y^T = S C^T diag(e^A): A = S (two C-layout tiles), B = C rows ----------
#pragma unroll
      for (int i = 0; i < PB; ++i)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) YT[i][tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < N / 32; ++ks) {
        if constexpr (SAFE) {
          bf16x8 sh[PB], sl[PB];
#pragma unroll
          for (int i = 0; i < PB; ++i) pack_b_hilo(ST[2 * ks][i], ST[2 * ks + 1][i], sh[i], sl[i]);
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            const bf16x8 bc = bits_b8(frag_i(sC, LDB, 16 * tb, 32 * ks, lane));
#pragma unroll
            for (int i = 0; i < PB; ++i) {
              YT[i][tb] = mfma16(sh[i], bc, YT[i][tb]);
              YT[i][tb] = mfma16(sl[i], bc, YT[i][tb]);
            }
          }
        } else {
          f16x8 sa[PB];
#pragma unroll
          for (int i = 0; i < PB; ++i) sa[i] = h8(ST[2 * ks][i], ST[2 * ks + 1][i]);
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            const f16x8 bc = frag_i(sC, LDB, 16 * tb, 32 * ks, lane);
#pragma unroll
            for (int i = 0; i < PB; ++i) YT[i][tb] = mfma16h(sa[i], bc, YT[i][tb]);
          }
        }
      }
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const float e = SC(cb, S_EA, 16 * tb + l16);
#pragma unroll
        for (int i = 0; i < PB; ++i)
#pragma unroll
          for (int v = 0; v < 4; ++v) YT[i][tb][v] *= e;
      }
      // ---- M^T = B C^T o decay o dt: tile (tb, jb) holds M[t = 16tb + l16][j =
      // 16jb + 4q4 + v], written as 4 consecutive (interleaved) columns of row t.
      // Lower tiles only; (0,1) and (2,3) are zeroed (M X reads them).  Tiles per
      // wave: w0 (0,0)(1,0)(2,0)+zero(0,1); w1 (1,1)(2,1)(3,0)+zero(2,3);
      // w2 (2,2)(3,1); w3 (3,2)(3,3) --------------------------------------------
      constexpr int TT[4][3][2] = {{{0, 0}, {1, 0}, {2, 0}}, {{1, 1}, {2, 1}, {3, 0}},
                                   {{2, 2}, {3, 1}, {-1, -1}}, {{3, 2}, {3, 3}, {-1, -1}}};
      auto m_tile = [&](auto w_c) {
        constexpr int W = decltype(w_c)::value;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          constexpr int tb_[3] = {TT[W][0][0], TT[W][1][0], TT[W][2][0]};
          constexpr int jb_[3] = {TT[W][0][1], TT[W][1][1], TT[W][2][1]};
          const int tb = tb_[k], jb = jb_[k];
          if (tb < 0) continue;
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < N / 32; ++ks) {
            const f16x8 fb = frag_i(sB, LDB, 16 * jb, 32 * ks, lane);
            const f16x8 fc = frag_i(sC, LDB, 16 * tb, 32 * ks, lane);
            acc = SAFE ? mfma16(bits_b8(fb), bits_b8(fc), acc) : mfma16h(fb, fc, acc);
          }
          const int t = 16 * tb + l16, j0 = 16 * jb + 4 * q4;
          const float at = SC(cb, S_ACS, t);
          const f32x4 aj = SC4(cb, S_ACS, j0), dj = SC4(cb, S_DT, j0);
          f32x4 m;
#pragma unroll
          for (int v = 0; v < 4; ++v) m[v] = (t >= j0 + v) ? acc[v] * fast_exp(at - aj[v]) * dj[v] : 0.f;
          if constexpr (SAFE) {
            bf16x2 h01, l01, h23, l23;
            split2(m[0], m[1], h01, l01);
            split2(m[2], m[3], h23, l23);
            *reinterpret_cast<bf16x4*>(sM + t * LDM + icol(j0)) =
                bf16x4{h01[0], h01[1], h23[0], h23[1]};
            *reinterpret_cast<bf16x4*>(sML + t * LDM + icol(j0)) =
                bf16x4{l01[0], l01[1], l23[0], l23[1]};
          } else {
            *reinterpret_cast<f16x4*>(sM + t * LDM + icol(j0)) = h4(m);
          }
        }
        if constexpr (W < 2) {
          constexpr int tb = W == 0 ? 0 : 2;
          const int o = (16 * tb + l16) * LDM + icol(16 * (tb + 1) + 4 * q4);
          *reinterpret_cast<f16x4*>(sM + o) = f16x4{0.f, 0.f, 0.f, 0.f};
          if constexpr (SAFE) *reinterpret_cast<f16x4*>(sML + o) = f16x4{0.f, 0.f, 0.f, 0.f};
        }
      };
      using I0 = std::integral_constant<int, 0>;
      using I1 = std::integral_constant<int, 1>;
      using I2 = std::integral_constant<int, 2>;
      using I3 = std::integral_constant<int, 3>;
      if (wave == 0) m_tile(I0{});
      else if (wave == 1) m_tile(I1{});
      else if (wave == 2) m_tile(I2{});
      else m_tile(I3{});
    } else if (wave == NTHR / 64 - 1 && c + 1 < si.c_end) {
      make_scalars(nxt.dt, c + 1, cb ^ 1);
    }

    // ---- S^T <- e^{A_L} S^T + B^T diag(w) X (after Y^T used the chunk's start
    // state): A = B^T (transposing read), B = w X (one rounding) -----------------
    {
      const float ea = fast_exp(al);
      dsum += al;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < PB; ++i)
#pragma unroll
          for (int v = 0; v < 4; ++v) ST[nb][i][v] *= ea;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const f32x4 w0 = SC4(cb, S_W, 32 * ks + 4 * q4), w1 = SC4(cb, S_W, 32 * ks + 16 + 4 * q4);
        if constexpr (SAFE) {
          bf16x8 bh[PB], bl[PB];
#pragma unroll
          for (int i = 0; i < PB; ++i) {
            const bf16x8 xb = bits_b8(xt[i][ks]);
            f32x4 u0, u1;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              u0[v] = (float)xb[v] * w0[v];
              u1[v] = (float)xb[4 + v] * w1[v];
            }
            pack_b_hilo(u0, u1, bh[i], bl[i]);
          }
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            const bf16x8 a = bits_b8(frag_t_i(sB, LDB, 32 * ks, 16 * nb, lane));
#pragma unroll
            for (int i = 0; i < PB; ++i) {
              ST[nb][i] = mfma16(a, bh[i], ST[nb][i]);
              ST[nb][i] = mfma16(a, bl[i], ST[nb][i]);
            }
          }
        } else {
          f16x8 bw[PB];
#pragma unroll
          for (int i = 0; i < PB; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              bw[i][v] = (f16)((float)xt[i][ks][v] * w0[v]);
              bw[i][4 + v] = (f16)((float)xt[i][ks][4 + v] * w1[v]);
            }
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            const f16x8 a = frag_t_i(sB, LDB, 32 * ks, 16 * nb, lane);
#pragma unroll
            for (int i = 0; i < PB; ++i) ST[nb][i] = mfma16h(a, bw[i], ST[nb][i]);
          }
        }
      }
    }

    if (MODE == MODE_OUT) {
      lds_barrier();   // M complete
      // ---- Y^T += X^T M^T (+ D x, z gate) -> sY ------------------------------------
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int ks = 0; ks <= tb / 2; ++ks) {
          const f16x8 bm = frag_i(sM, LDM, 16 * tb, 32 * ks, lane);
          if constexpr (SAFE) {
            const bf16x8 bl = bits_b8(frag_i(sML, LDM, 16 * tb, 32 * ks, lane));
#pragma unroll
            for (int i = 0; i < PB; ++i) {
              YT[i][tb] = mfma16(bits_b8(xt[i][ks]), bits_b8(bm), YT[i][tb]);
              YT[i][tb] = mfma16(bits_b8(xt[i][ks]), bl, YT[i][tb]);
            }
          } else {
#pragma unroll
            for (int i = 0; i < PB; ++i) YT[i][tb] = mfma16h(xt[i][ks], bm, YT[i][tb]);
          }
        }
#pragma unroll
      for (int i = 0; i < PB; ++i) {
        const int p0 = 16 * (PB * wave + i) + 4 * q4;
        const f32x4 dv = dreg[i];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          const int t = 16 * tb + l16;
          const f16x4 xv = *reinterpret_cast<const f16x4*>(sX + t * LDX + p0);
          const bf16x4 xvb = __builtin_bit_cast(bf16x4, xv);
          bf16x4 zv;
          if (p.z) zv = *reinterpret_cast<const bf16x4*>(sY + t * LDX + p0);
          bf16x4 out;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            float yv = YT[i][tb][v] + dv[v] * (SAFE ? (float)xvb[v] : (float)xv[v]);
            if (p.z) {
              const float zz = (float)zv[v];
              yv *= zz * __builtin_amdgcn_rcpf(1.f + fast_exp(-zz));
            }
            out[v] = (bf16)yv;
          }
          *reinterpret_cast<bf16x4*>(sY + t * LDX + p0) = out;
        }
      }
    }
    lds_barrier();
  };

  if (AHEAD == 2) {
    for (int c = si.c_start; c < si.c_end; c += 2) {
      chunk(ra, rb, c);
      if (c + 1 < si.c_end) chunk(rb, ra, c + 1);
    }
  } else {
    for (int c = si.c_start; c < si.c_end; ++c) chunk(ra, ra, c);
  }
  if (MODE == MODE_OUT && si.c_start < si.c_end) store_y(si.bos + (si.c_end - 1) * L, nval_of(si.c_end - 1));

  // ---- plain pass: did an fp16 operand leave its range? ----------------------------
  if constexpr (!SAFE) {
    float acc = ysum;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < PB; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc += ST[nb][i][v];
    int* flag = reinterpret_cast<int*>(sc);   // the scalar buffers are free after the loop
    if (lane == 0) flag[wave] = __ballot(!__builtin_isfinite(acc)) != 0;
    lds_barrier();
    const int redo = flag[0] | flag[1] | flag[2] | flag[3];
    if (tid == 0) p.redo[s_id * H + h] = redo;
    if (redo) return;   // walked again by the SAFE pass (the end state is not written)
  }

  // ---- segment end state --------------------------------------------------------
  float* dst = nullptr;
  bf16* dst16 = nullptr;
  if (MODE == MODE_LOCAL) {
    dst = p.ws_loc + ((int64_t)s_id * H + h) * P * N;
    if (tid == 0) p.ws_dec[(int64_t)s_id * H + h] = dsum;
  } else if (si.seg_idx == si.nseg - 1 && p.hT && slot >= 0) {
    if (p.st_dt == HMX_BF16) dst16 = static_cast<bf16*>(p.hT) + soff;
    else dst = static_cast<float*>(p.hT) + soff;
  }
  if (dst || dst16) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < PB; ++i) {
        const int pc = 16 * (PB * wave + i) + l16;
        const int64_t e = (int64_t)pc * N + 16 * nb + 4 * q4;
        const f32x4 x = ST[nb][i];
        if (dst) *reinterpret_cast<f32x4*>(dst + e) = x;
        else *reinterpret_cast<bf16x4*>(dst16 + e) = bf16x4{(bf16)x[0], (bf16)x[1], (bf16)x[2],
                                                             (bf16)x[3]};
      }
  }
}

// Segment start states: S0[first] = h0 (or 0); S0[s+1] = e^{dec[s]} S0[s] + loc[s].
// One workgroup row per split (sequence, head); single-segment sequences return.
__global__ __launch_bounds__(256) void ssd_seg_combine_kernel(Params p, int PN) {
  const int nh = blockIdx.x, H = p.H;
  const int n = nh / H, h = nh % H;
  int first = -1, nseg = 0;
  for (int s = 0; s < p.nseg_total; ++s) {
    const SegInfo si = load_seg(p.seg, s);
    if (si.n == n) { first = si.first_seg; nseg = si.nseg; break; }
  }
  if (first < 0 || nseg < 2) return;
  const int64_t slot = p.sidx ? (int64_t)p.sidx[n] : n;
  const bool init = p.h0 && slot >= 0 && (!p.hinit || p.hinit[n]);
  const int64_t soff = slot * p.st_ss + (int64_t)h * PN;
  for (int e = blockIdx.y * 256 + threadIdx.x; e < PN; e += gridDim.y * 256) {
    float sx = 0.f;
    if (init)
      sx = p.st_dt == HMX_BF16 ? (float)static_cast<const bf16*>(p.h0)[soff + e]
                               : static_cast<const float*>(p.h0)[soff + e];
    p.ws_s0[((int64_t)first * H + h) * PN + e] = sx;   // no OUT workgroup reads h0
    for (int s = 0; s < nseg - 1; ++s) {
      const int64_t b = (int64_t)(first + s) * H + h;
      sx = sx * expf(p.ws_dec[b]) + p.ws_loc[b * PN + e];
      p.ws_s0[((int64_t)(first + s + 1) * H + h) * PN + e] = sx;
    }
  }
}

// Each pass, then its flagged walks again with bf16 operands (SAFE).
template <int P, int N>
void launch(const Params& p, int nseq, hipStream_t s) {
  const bool multi = p.nseg_total > nseq;
  const dim3 grid(p.nseg_total * p.H);
  if (multi) {
    hipLaunchKernelGGL((ssd_chunk_kernel<P, N, MODE_LOCAL, false>), grid, dim3(NTHR), 0, s, p);
    hipLaunchKernelGGL((ssd_chunk_kernel<P, N, MODE_LOCAL, true>), grid, dim3(NTHR), 0, s, p);
    hipLaunchKernelGGL(ssd_seg_combine_kernel, dim3(nseq * p.H, (P * N + 1023) / 1024), dim3(256),
                       0, s, p, P * N);
  }
  hipLaunchKernelGGL((ssd_chunk_kernel<P, N, MODE_OUT, false>), grid, dim3(NTHR), 0, s, p);
  hipLaunchKernelGGL((ssd_chunk_kernel<P, N, MODE_OUT, true>), grid, dim3(NTHR), 0, s, p);
}

}  // namespace ssd
}  // namespace hmx

using namespace hmx;
using namespace hmx::ssd;

extern "C" size_t hmx_ssd_chunk_workspace_bytes(int32_t nseg_total, int32_t nseq, int32_t H,
                                                int32_t P, int32_t N) {
  const size_t flags = (size_t)nseg_total * H * sizeof(int);   // redo flags
  if (nseg_total <= nseq) return flags;
  const size_t st = (size_t)nseg_total * H * P * N * sizeof(float);
  return 2 * st + (size_t)nseg_total * H * sizeof(float) + flags;
}

extern "C" int hmx_ssd_chunk_fwd(const void* x, int64_t x_ts, int64_t x_hs, const void* B,
                                 int64_t b_ts, int64_t b_gs, const void* C, int64_t c_ts,
                                 int64_t c_gs, int32_t xbc_dtype, const void* dt, int32_t dt_dtype,
                                 int64_t dt_ts, int64_t dt_hs, const float* A, const float* D,
                                 const float* dt_bias, const void* z, int64_t z_ts, int64_t z_hs,
                                 void* y, int64_t y_ts, int64_t y_hs, const void* h0,
                                 void* h_final, int64_t state_slot_stride, int32_t state_dtype,
                                 const int32_t* state_indices, const uint8_t* has_initial_state,
                                 const int32_t* seg_table, int32_t nseg_total,
                                 int32_t nseq, int32_t H, int32_t HX, int32_t G, int32_t GC,
                                 int32_t P, int32_t N, int32_t dt_softplus, float dt_min, float dt_max, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  HMX_REQUIRE(xbc_dtype == HMX_BF16, HMX_EUNSUPPORTED,
              "hmx_ssd_chunk_fwd: x/B/C/z must be bfloat16 (got dtype code %d)", xbc_dtype);
  HMX_REQUIRE((P == 64 || P == 128) && (N == 64 || N == 128), HMX_EUNSUPPORTED,
              "hmx_ssd_chunk_fwd: headdim in {64,128} and d_state in {64,128} (got %d, %d)", P, N);
  HMX_REQUIRE(H > 0 && HX > 0 && G > 0 && GC > 0 && H % HX == 0 && H % G == 0 && H % GC == 0,
              HMX_EINVAL, "hmx_ssd_chunk_fwd: H=%d must be a multiple of HX=%d, G=%d and GC=%d",
              H, HX, G, GC);
  HMX_REQUIRE(x && B && C && dt && A && y && seg_table, HMX_EINVAL,
              "hmx_ssd_chunk_fwd: null tensor pointer");
  HMX_REQUIRE(dt_dtype == HMX_F32 || dt_dtype == HMX_BF16 || dt_dtype == HMX_F16, HMX_EINVAL,
              "hmx_ssd_chunk_fwd: dt dtype code %d", dt_dtype);
  const int64_t strides[] = {x_ts, x_hs, b_ts, b_gs, c_ts, c_gs, y_ts, y_hs,
                             z ? z_ts : 8, z ? z_hs : 8};
  for (int64_t st : strides)
    HMX_REQUIRE(st % 8 == 0, HMX_EINVAL,
                "hmx_ssd_chunk_fwd: token/head strides must be multiples of 8 elements");
  // a chunk's 64 rows are addressed with 32-bit byte offsets
  for (int64_t ts : {x_ts, b_ts, c_ts, y_ts, z ? z_ts : (int64_t)0})
    HMX_REQUIRE(ts >= 0 && ts < ((int64_t)1 << 24), HMX_EUNSUPPORTED,
                "hmx_ssd_chunk_fwd: token strides must be below 2^24 elements (got %lld)",
                (long long)ts);
  HMX_REQUIRE(!(h0 || h_final) || ((state_dtype == HMX_F32 || state_dtype == HMX_BF16) &&
                                    state_slot_stride % 4 == 0 &&
                                    ((uintptr_t)h0 | (uintptr_t)h_final) % 16 == 0),
              HMX_EINVAL, "hmx_ssd_chunk_fwd: states must be f32/bf16 with 16-byte aligned slots");
  if (nseg_total == 0) return HMX_OK;
  const size_t need = hmx_ssd_chunk_workspace_bytes(nseg_total, nseq, H, P, N);
  HMX_REQUIRE(workspace && workspace_bytes >= need, HMX_EINVAL,
              "hmx_ssd_chunk_fwd: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  Params p;
  p.x = static_cast<const bf16*>(x); p.x_ts = x_ts; p.x_hs = x_hs;
  p.B = static_cast<const bf16*>(B); p.b_ts = b_ts; p.b_gs = b_gs;
  p.C = static_cast<const bf16*>(C); p.c_ts = c_ts; p.c_gs = c_gs;
  p.dt = dt; p.dt_dt = dt_dtype; p.dt_ts = dt_ts; p.dt_hs = dt_hs;
  p.A = A; p.D = D; p.dt_bias = dt_bias;
  p.z = static_cast<const bf16*>(z); p.z_ts = z_ts; p.z_hs = z_hs;
  p.y = static_cast<bf16*>(y); p.y_ts = y_ts; p.y_hs = y_hs;
  p.h0 = h0; p.hT = h_final; p.st_ss = state_slot_stride; p.st_dt = state_dtype;
  p.sidx = state_indices; p.hinit = has_initial_state;
  p.seg = seg_table; p.nseg_total = nseg_total;
  const bool multi = nseg_total > nseq;
  const size_t st = (size_t)nseg_total * H * P * N;
  float* ws = static_cast<float*>(workspace);
  p.ws_loc = multi ? ws : nullptr;
  p.ws_s0 = multi ? ws + st : nullptr;
  p.ws_dec = multi ? ws + 2 * st : nullptr;
  p.redo = reinterpret_cast<int*>(multi ? ws + 2 * st + (size_t)nseg_total * H : ws);
  p.H = H; p.HX = HX; p.G = G; p.GC = GC; p.softplus = dt_softplus; p.dt_min = dt_min; p.dt_max = dt_max;
  hipStream_t s = (hipStream_t)stream;
  if (P == 64 && N == 128) launch<64, 128>(p, nseq, s);
  else if (P == 128 && N == 128) launch<128, 128>(p, nseq, s);
  else if (P == 64 && N == 64) launch<64, 64>(p, nseq, s);
  else launch<128, 64>(p, nseq, s);
  return check_launch("hmx_ssd_chunk_fwd");
}
