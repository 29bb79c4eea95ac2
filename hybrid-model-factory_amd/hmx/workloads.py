"""Seeded synthetic inputs for the benchmark configurations (C0-C4).

Each config draws from ``torch.Generator().manual_seed(20260000 + config_id)`` on
the CPU, in the order the tensors are listed, in fp32 and casts last, so the
CPU checker and the GPU see identical bits.  ``device_gen=True`` draws on the
GPU instead (different bits, same distributions) for large benchmark inputs.

  C0  GDN fwd, B=1 T=2048 H=16 d=128 fp32 (CPU plumbing case)
  C1  GDN chunked prefill, B=1 T=32768 H=32 d=128 bf16 (+ HKV=8, + varlen 8 seqs)
  C2  GDN decode, 256 seqs x 1 token, H=32 d=128, fp32 pool N(0,0.02^2), randperm slots
  C3  GKA prefill, C1 shape
  C4  Mamba2 SSD, B=2 T=16384 H=64 P=64 N=128 G=8 chunk 256
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

SEED_BASE = 20260000


def gen(config_id: int, device: str | torch.device = "cpu") -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(SEED_BASE + config_id)
    return g


def _randn(gen_, shape, device):
    return torch.randn(*shape, generator=gen_, device=device, dtype=torch.float32)


def _l2n(x):
    return x / x.norm(dim=-1, keepdim=True)


def gdn_inputs(T: int, H: int, HKV: int, D: int, dtype=torch.bfloat16, config_id: int = 1,
               B: int = 1, device="cpu", gen_device="cpu"):
    """q,k ~ N(0,1) L2-normalised per head; v ~ N(0,1); beta = sigmoid(N(0,1));
    g = logsigmoid(N(0,1)).  Returns dict of tensors on ``device``."""
    gd = gen(config_id, gen_device)
    q = _l2n(_randn(gd, (B, T, H, D), gen_device))
    k = _l2n(_randn(gd, (B, T, HKV, D), gen_device))
    v = _randn(gd, (B, T, HKV, D), gen_device)
    beta = torch.sigmoid(_randn(gd, (B, T, H), gen_device))
    g = F.logsigmoid(_randn(gd, (B, T, H), gen_device))
    out = dict(q=q.to(dtype), k=k.to(dtype), v=v.to(dtype), g=g, beta=beta)
    return {n: t.to(device) for n, t in out.items()}


def gdn_layer_gates(T: int, H: int, config_id: int = 11, device="cpu", gen_device="cpu"):
    """Gates as a GDN layer forms them (fused_gdn_gating.py:66-76):
    g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b), with A_log = log U(1, 16),
    dt_bias the inverse softplus of dt ~ exp(U(log 1e-3, log 1e-1)) (the Mamba2
    initialisation, training/.../layers/mamba/mamba2.py:194-201) and a, b ~ N(0, 1).
    Many heads then decay by far less than e^-20 over a 512-token window.  Returns
    (g, beta) as fp32 [1, T, H] on ``device``."""
    gd = gen(config_id, gen_device)
    A_log = torch.log(torch.rand(H, generator=gd, device=gen_device) * 15 + 1)
    dt = torch.exp(torch.rand(H, generator=gd, device=gen_device) * (math.log(0.1) - math.log(1e-3))
                   + math.log(1e-3))
    dt_bias = dt + torch.log(-torch.expm1(-dt))
    a = _randn(gd, (T, H), gen_device)
    b = _randn(gd, (T, H), gen_device)
    g = -torch.exp(A_log) * F.softplus(a + dt_bias)
    return g.unsqueeze(0).to(device), torch.sigmoid(b).unsqueeze(0).to(device)


def gdn_exact_pairs(g: torch.Tensor, beta: torch.Tensor, table, max_warm: int = 16,
                    threshold: float = 20.0, chunk: int = 32) -> tuple[int, torch.Tensor]:
    """The prefill plan's use of the exact segment scan, by the kernel's own rule:
    (segment, head) pairs whose preceding max_warm chunks neither decay the dropped
    history below e^-threshold (the decay bound of a token being
    g + log max(1, |1 - beta|)) nor reach the sequence start, and the [H] mask of
    heads with any such segment, which run the scan.  g, beta [1, T, H]; table: the
    plan's [rows, 8] segment table."""
    dec = (g[0].double() + torch.log(torch.clamp((1 - beta[0].double()).abs(), min=1.0))).cpu()
    cs = torch.cat([torch.zeros(1, dec.shape[1], dtype=dec.dtype), dec.cumsum(0)])
    pairs, heads = 0, torch.zeros(dec.shape[1], dtype=torch.bool)
    for r in [list(map(int, x)) for x in table]:
        n, bos, eos, c0 = r[:4]
        if r[5] == 0:
            continue
        lo = max(0, c0 - max_warm)
        if lo == 0:
            continue                       # the warm-up starts at the sequence start
        t0, t1 = bos + lo * chunk, min(eos, bos + c0 * chunk)
        need = (cs[t1] - cs[t0]) > -threshold
        pairs += int(need.sum())
        heads |= need
    return pairs, heads


def varlen_lengths(n_seqs: int = 8, lo: int = 1024, hi: int = 8192, config_id: int = 1):
    """Sequence lengths ~ randint(lo, hi+1) from the config generator (drawn first)."""
    gd = gen(config_id)
    return torch.randint(lo, hi + 1, (n_seqs,), generator=gd)


def cu_from_lengths(lengths: torch.Tensor) -> torch.Tensor:
    return torch.cat([torch.zeros(1, dtype=torch.int64), lengths.cumsum(0)]).to(torch.int32)


def decode_inputs(n_seqs: int = 256, H: int = 32, HKV: int = 32, D: int = 128, steps: int = 1,
                  slots: int | None = None, dtype=torch.bfloat16, config_id: int = 2,
                  device="cpu", gen_device="cpu"):
    """C2: pool fp32 [slots,H,D,D] ~ N(0, 0.02^2); indices = randperm(slots)[:n_seqs];
    per step q,k,v [1,n_seqs,*,D], g, beta [1,n_seqs,H] stacked over ``steps``."""
    slots = slots or n_seqs
    gd = gen(config_id, gen_device)
    pool = _randn(gd, (slots, H, D, D), gen_device) * 0.02
    idx = torch.randperm(slots, generator=gd, device=gen_device)[:n_seqs].to(torch.int32)
    q = _l2n(_randn(gd, (steps, 1, n_seqs, H, D), gen_device)).to(dtype)
    k = _l2n(_randn(gd, (steps, 1, n_seqs, HKV, D), gen_device)).to(dtype)
    v = _randn(gd, (steps, 1, n_seqs, HKV, D), gen_device).to(dtype)
    beta = torch.sigmoid(_randn(gd, (steps, 1, n_seqs, H), gen_device))
    g = F.logsigmoid(_randn(gd, (steps, 1, n_seqs, H), gen_device))
    cu = torch.arange(n_seqs + 1, dtype=torch.int32, device=gen_device)
    out = dict(pool=pool, idx=idx, q=q, k=k, v=v, g=g, beta=beta, cu_seqlens=cu)
    return {n: t.to(device) for n, t in out.items()}


def gka_inputs(T: int, H: int, HKV: int, D: int, dtype=torch.bfloat16, config_id: int = 3,
               B: int = 1, device="cpu", gen_device="cpu"):
    """C3: q,k L2-normalised, v ~ N(0,1); alpha, beta = sigmoid(N(0,1));
    g = gk = logsigmoid(N(0,1)) (one tensor passed as both gates)."""
    gd = gen(config_id, gen_device)
    q = _l2n(_randn(gd, (B, T, H, D), gen_device))
    k = _l2n(_randn(gd, (B, T, HKV, D), gen_device))
    v = _randn(gd, (B, T, HKV, D), gen_device)
    alpha = torch.sigmoid(_randn(gd, (B, T, H), gen_device))
    beta = torch.sigmoid(_randn(gd, (B, T, H), gen_device))
    g = F.logsigmoid(_randn(gd, (B, T, H), gen_device))
    out = dict(q=q.to(dtype), k=k.to(dtype), v=v.to(dtype), alpha=alpha, beta=beta, g=g)
    out = {n: t.to(device) for n, t in out.items()}
    out["gk"] = out["g"]
    return out


def gka_prefill_flops(T: int, H: int, num_iter: int, d: int = 128, C: int = 64) -> float:
    """2*T*H*[(4+n) d^2 + (3+2n) C d + C^2] (h_kk update, exact-fro terms, n solver
    iterations of x.H_c / x.K^T / .K, and the GLA)."""
    n = num_iter
    return 2.0 * T * H * ((4 + n) * d * d + (3 + 2 * n) * C * d + C * C)


def gka_train_flops(T: int, H: int, num_iter: int, d: int = 128, C: int = 64):
    """(forward, backward) FLOPs of the training Chebyshev solve over T tokens x H heads.
    Forward: 2*T*H*[(2+n) d^2 + (1+2n) C d + C^2] (h_kk update, exact-fro terms, n
    iterations).  Backward: 2*T*H*[(n+6) d^2 + (2n+6) C d] (the dq solve's n
    iterations; the block contributions dq^T x, x^T dq, K^T diag K; h_c k, h_c x,
    Dn k; and the in-block x.k, dq.k, k.k products with their three products back)."""
    n = num_iter
    return (2.0 * T * H * ((2 + n) * d * d + (1 + 2 * n) * C * d + C * C),
            2.0 * T * H * ((n + 6) * d * d + (2 * n + 6) * C * d))


def gdn_train_flops(T: int, H: int, d: int = 128, C: int = 32):
    """(forward, backward) FLOPs of the chunked gated delta rule's training op over T
    tokens x H heads, 32-token blocks.  Forward: the prefill's 2*T*H*(3 d^2 + 5 C d).
    Backward: 2*T*H*(11 d^2 + 20 C d) = the forward's recomputation of the block
    states, the prep (Q^K^T, K^K^T: 2 C d), the state-gradient chain (K^ dS, two
    products back into dS: 3 d^2; P^T dO, T^T dW: 2 C d) and the per-block gradients
    (K^ S0, K^ dS, dO S0^T, Z S0^T, W dS^T: 5 d^2; Q^K^T, K^K^T, W, P^T dO, Z, Z W^T,
    dO W^T and four C x C x d products back: 11 C d)."""
    return (2.0 * T * H * (3 * d * d + 5 * C * d), 2.0 * T * H * (11 * d * d + 20 * C * d))


def gka_prefill_bytes(T: int, H: int, HKV: int, d: int = 128, n_seqs: int = 1) -> float:
    """q,o [T,H,d] + k,v [T,HKV,d] bf16 + alpha,beta,g fp32 + two fp32 final states."""
    return T * H * 2 * d * 2 + T * HKV * 2 * d * 2 + 3 * T * H * 4 + 2 * n_seqs * H * d * d * 4


def ssd_inputs(b: int = 2, T: int = 16384, H: int = 64, P: int = 64, N: int = 128, G: int = 8,
               config_id: int = 4, device="cpu", gen_device="cpu"):
    """C4: x [b,T,H,P], B, C [b,T,G,N] bf16 ~ N(0,1); dt_raw [b,T,H] ~ N(-2, 0.5) fp32
    (passed with dt_softplus=True); dt_bias [H] = softplus^-1(exp(U(ln 1e-3, ln 1e-1)));
    A [H] = -exp(U(ln 1, ln 16)); D [H] ~ N(1, 0.1); drawn in that order."""
    gd = gen(config_id, gen_device)
    x = _randn(gd, (b, T, H, P), gen_device)
    Bm = _randn(gd, (b, T, G, N), gen_device)
    Cm = _randn(gd, (b, T, G, N), gen_device)
    dt = _randn(gd, (b, T, H), gen_device) * 0.5 - 2.0
    u = torch.rand(H, generator=gd, device=gen_device)
    dtv = torch.exp(u * (math.log(0.1) - math.log(1e-3)) + math.log(1e-3))
    dt_bias = dtv + torch.log(-torch.expm1(-dtv))
    A = -torch.exp(torch.rand(H, generator=gd, device=gen_device) * math.log(16.0))
    D = _randn(gd, (H,), gen_device) * 0.1 + 1.0
    out = dict(x=x.to(torch.bfloat16), B=Bm.to(torch.bfloat16), C=Cm.to(torch.bfloat16), dt=dt,
               dt_bias=dt_bias, A=A, D=D)
    return {n: t.to(device) for n, t in out.items()}


def ssd_flops(tokens: int, H: int, G: int, P: int = 64, N: int = 128, L: int = 256) -> float:
    """2*tokens*[H(L*P + 2*N*P) + G*L*N]: per chunk-head the intra-chunk (CB^T)X,
    the state-to-output C S^T and the state update X^T B, plus CB^T once per group."""
    return 2.0 * tokens * (H * (L * P + 2 * N * P) + G * L * N)


def ssd_bytes(tokens: int, H: int, G: int, P: int = 64, N: int = 128, n_seqs: int = 2) -> float:
    """x, y bf16 [tokens,H,P] + B, C bf16 [tokens,G,N] + dt fp32 + final fp32 states."""
    return 2 * tokens * H * P * 2 + 2 * tokens * G * N * 2 + tokens * H * 4 + n_seqs * H * P * N * 4


def ssd_decode_bytes(batch: int, H: int, G: int, P: int = 64, N: int = 128,
                     state_bytes: int = 4) -> float:
    """State read + write per (sequence, head), x/out bf16, dt, B, C."""
    return (2 * batch * H * P * N * state_bytes + 2 * batch * H * P * 2 + batch * H * P * 4
            + 2 * batch * G * N * 2)


# ---------------------------------------------------------------------------
# algorithmic work per unit (used for roofline.achieved)
# ---------------------------------------------------------------------------
def gdn_prefill_flops(T: int, H: int, K: int = 128, V: int = 128, C: int = 64) -> float:
    """2*T*H*(5*C*d + 3*d^2) for d = K = V (KK^T, QK^T, T.(bK), T.(bV), P.Vnew: C x C x d;
    W.h, Q.h, K^T.Vnew: C x d x d); the (I+A)^-1 term is excluded."""
    d = K
    return 2.0 * T * H * (5 * C * d + 3 * d * d)


def gdn_prefill_bytes(T: int, H: int, HKV: int, K: int = 128, V: int = 128, n_seqs: int = 1,
                      in_bytes: int = 2) -> float:
    """q,o [T,H,d] + k,v [T,HKV,d] in bf16, g,beta fp32 [T,H], final state fp32."""
    return (T * H * (K + V) * in_bytes + T * HKV * (K + V) * in_bytes + 2 * T * H * 4
            + n_seqs * H * K * V * 4)


def gdn_decode_bytes(n_seqs: int, H: int, HKV: int, K: int = 128, V: int = 128,
                     state_bytes: int = 4, in_bytes: int = 2) -> float:
    """State read + write per (seq, head) plus q,o [n,H,d] and k,v [n,HKV,d] and g,beta."""
    return (2 * n_seqs * H * K * V * state_bytes + n_seqs * H * (K + V) * in_bytes
            + n_seqs * HKV * (K + V) * in_bytes + 2 * n_seqs * H * 4)


def gka_decode_bytes(n_seqs: int, H: int, HKV: int, D: int = 128, in_bytes: int = 2) -> float:
    """h_kk and h_kv (fp32) read + write per (seq, head) plus q,o [n,H,D], k,v
    [n,HKV,D] and alpha, g, beta fp32."""
    return (4 * n_seqs * H * D * D * 4 + 2 * n_seqs * H * D * in_bytes
            + 2 * n_seqs * HKV * D * in_bytes + 3 * n_seqs * H * 4)


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


__all__ = ["gen", "gdn_inputs", "gka_inputs", "gka_prefill_flops", "gka_prefill_bytes",
           "varlen_lengths", "cu_from_lengths", "decode_inputs", "ssd_inputs", "ssd_flops",
           "ssd_bytes", "ssd_decode_bytes", "gdn_prefill_flops", "gdn_prefill_bytes",
           "gdn_decode_bytes", "ceil_div"]
