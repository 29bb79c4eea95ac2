"""The training layer's Chebyshev solve with its backward, over libhmx.

Entry points (reference paths relative to the reference repository root,
training/src/hmf/model/hybrid_zoo/layers/gated_kalmanet/ops/chebyshev/):

- ``ChebyshevIteration`` — chebyshev_iteration.py:560-688, the autograd function
  ``apply(k, q, gk=None, num_iter=30, ridge_ratio=0.02, bp_lambda=True, h0=None,
  chunk_size=64) -> (x, h_kk_final)``: per token x_t solves
  (H_t + r |H_t|_F I) x_t = q_t by the Chebyshev recurrence, H_t = e^{gk_t} H_{t-1}
  + k_t k_t^T from zero.  Its backward returns (dk, dq, dgk) as the reference's
  does: dq by the same recurrence on dx with the forward's |H_t|_F, dk and dgk
  from dL/dH_t = -dq_t x_t^T (- r (dq_t . x_t) H_t / |H_t|_F with bp_lambda); the
  gradient of h_kk_final is not propagated (the reference drops it, :638).
- ``latent_chebyshev`` — gka_chebyshev_solve.py:74-104, the dispatcher over it.
- ``GkaChebyshevGla`` — the whole training forward gka_chebyshev_gla
  (gka_chebyshev_solve.py:107-164: the solve, the alpha blend, fla's
  chunk_simple_gla) as one autograd function; ``hmx.gka_chebyshev_gla`` routes
  through it when a gradient is needed.  Its backward runs the GLA readout's
  backward (dq~, dk, dv, dg, then dx = alpha dq~, dalpha = dq~ . (x - q)) and the
  solve's backward on dx, adding into dq and dk.  Gradients of the final states
  are not propagated.

Kernels (libhmx ``hmx_gka_cheb_fwd`` / ``hmx_gka_cheb_bwd``): the serving prefill's
state walk and combine, and its solve kernel writing x and |H_t|_F instead of the
GLA output; the backward runs the solve on dx reading the saved |H_t|_F and the
forward's block-start states, then three launches for dk and dgk (the blocks'
contributions to the state gradient, its reverse scan over the blocks, and the
per-block dk / dgk).  k, q must be bfloat16 with head dim 128; ``chunk_size``
only tiles the reference's kernels (the blocks here are 64 tokens) and h0 (the
sequence-parallel initial state) is not supported.
"""
from __future__ import annotations

import torch

from .. import _lib
from .gdn import _device_table, _segment_table


def _check(k, q, gk):
    if q.dim() != 4 or k.shape != q.shape:
        raise ValueError(f"k and q must both be [B, T, H, D], got {tuple(k.shape)} and "
                         f"{tuple(q.shape)}")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise NotImplementedError(f"hmx ChebyshevIteration: k and q must be bfloat16, got "
                                  f"{k.dtype} / {q.dtype}")
    if q.shape[-1] != 128:
        raise NotImplementedError(f"hmx ChebyshevIteration: head dim must be 128, got {q.shape[-1]}")
    if gk is not None and tuple(gk.shape) != tuple(q.shape[:3]):
        raise ValueError(f"gk must be [B, T, H] = {tuple(q.shape[:3])}, got {tuple(gk.shape)}")
    _lib.require_gpu(k, q, gk)


def cheb_forward(k, q, gk, num_iter: int, ridge_ratio: float, segment_chunks=None):
    """The forward launches: (x, |H_t|_F [B,T,H] fp32, h_kk_final [B,H,D,D] fp32,
    and what the backward needs of the call: the workspace with the block-start
    states, the segment table and its sizes).  ``segment_chunks`` cuts every
    sequence into segments of at most that many 64-token blocks (tests)."""
    _check(k, q, gk)
    B, T, H, D = q.shape
    dev = q.device
    k2, q2 = k.contiguous(), q.contiguous()
    gk2 = None if gk is None else gk.contiguous()
    rows, nblk = _segment_table(_lib.PLAN_GKA, [(n * T, n * T + T) for n in range(B)],
                                B * T, H, dev, segment_chunks)
    seg = _device_table(rows, dev)
    lib = _lib.load()
    ws = torch.empty(max(int(lib.hmx_gka_chunk_workspace_bytes(len(rows), nblk, B, H)), 16),
                     dtype=torch.uint8, device=dev)
    x = torch.empty_like(q2)
    fro = torch.empty(B, T, H, dtype=torch.float32, device=dev)
    h_final = torch.empty(B, H, D, D, dtype=torch.float32, device=dev)
    _lib.call("hmx_gka_cheb_fwd", _lib.ptr(k2), H * D, _lib.ptr(q2), H * D,
              _lib.dtype_code(q2), _lib.ptr(gk2), 0 if gk2 is None else _lib.dtype_code(gk2),
              _lib.ptr(x), _lib.ptr(fro), _lib.ptr(h_final), _lib.ptr(seg), len(rows), nblk,
              B, H, D, int(num_iter), float(ridge_ratio), _lib.ptr(ws), ws.numel(),
              _lib.stream_of(q2))
    return x, fro, h_final, (k2, gk2, ws, seg, len(rows), nblk)


class ChebyshevIteration(torch.autograd.Function):
    """chebyshev_iteration.py:560-688 (see the module docstring)."""

    @staticmethod
    def forward(ctx, k, q, gk=None, num_iter: int = 30, ridge_ratio: float = 0.02,
                bp_lambda: bool = True, h0=None, chunk_size: int = 64, _segment_chunks=None):
        if h0 is not None:
            raise NotImplementedError("hmx ChebyshevIteration: an initial state h0 (the "
                                      "sequence-parallel path) is not supported")
        x, fro, h_final, (k2, gk2, ws, seg, nrows, nblk) = cheb_forward(
            k, q, gk, num_iter, ridge_ratio, _segment_chunks)
        ctx.save_for_backward(k2, x, fro, gk2, ws, seg)
        ctx.meta = (nrows, nblk, int(num_iter), float(ridge_ratio), bool(bp_lambda),
                    q.dtype, None if gk is None else gk.dtype)
        return x, h_final

    @staticmethod
    def backward(ctx, dx, d_kk_final=None):
        k, x, fro, gk, ws, seg = ctx.saved_tensors
        nrows, nblk, num_iter, ridge, bp_lambda, q_dtype, gk_dtype = ctx.meta
        B, T, H, D = k.shape
        dev = k.device
        if dx is None:
            dx = torch.zeros_like(x)
        # the kernels read dx as bfloat16 rows (x's dtype, which autograd hands back)
        # and write dq, dk in bf16 (k and q's dtype)
        dx2 = dx.to(torch.bfloat16).contiguous()
        dq = torch.empty(B, T, H, D, dtype=torch.bfloat16, device=dev)
        dk = torch.empty_like(dq)
        dgk = None if gk is None else torch.empty(B, T, H, dtype=torch.float32, device=dev)
        lib = _lib.load()
        bws = torch.empty(max(int(lib.hmx_gka_cheb_bwd_workspace_bytes(nblk, H, B * T)), 16),
                          dtype=torch.uint8, device=dev)
        _lib.call("hmx_gka_cheb_bwd", _lib.ptr(k), H * D, _lib.ptr(x), _lib.ptr(dx2), H * D,
                  _lib.dtype_code(k), _lib.ptr(gk), 0 if gk is None else _lib.dtype_code(gk),
                  _lib.ptr(fro), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dgk), _lib.ptr(seg), nrows,
                  nblk, B, H, D, B * T, num_iter, ridge, int(bp_lambda), _lib.ptr(ws),
                  ws.numel(), _lib.ptr(bws), bws.numel(), _lib.stream_of(k))
        return (dk, dq.to(q_dtype), None if dgk is None else dgk.to(gk_dtype),
                None, None, None, None, None, None)


def latent_chebyshev(k, q, ridge_strength, num_iter, solver_type, bp_lambda, gk, chunk_size):
    """gka_chebyshev_solve.py:74-104: (x, kk_final) of the ridge solve."""
    if solver_type != "chebyshev":
        raise ValueError(f"Unknown GKA solver type: {solver_type}")
    return ChebyshevIteration.apply(k, q, gk, num_iter, ridge_strength, bp_lambda, None,
                                    chunk_size)


class GkaChebyshevGla(torch.autograd.Function):
    """gka_chebyshev_solve.py:107-164 with its backward (see the module docstring).
    apply(q, k, v, alpha, g, gk, gla_scale, ridge_strength, num_iter, bp_lambda,
    _segment_chunks) -> (o, kk_final or None, kv_final)."""

    @staticmethod
    def forward(ctx, q, k, v, alpha, g, gk, gla_scale, ridge_strength, num_iter, bp_lambda,
                _segment_chunks=None):
        _check(k, q, gk)
        if v.shape != q.shape or v.dtype != q.dtype:
            raise ValueError(f"v must match q [B, T, H, 128] bf16, got {tuple(v.shape)} {v.dtype}")
        for name, t in (("alpha", alpha), ("g", g)):
            if tuple(t.shape) != tuple(q.shape[:3]):
                raise ValueError(f"{name} must be [B, T, H] = {tuple(q.shape[:3])}, got "
                                 f"{tuple(t.shape)}")
        _lib.require_gpu(v, alpha, g)
        B, T, H, D = q.shape
        dev = q.device
        q2, k2, v2 = q.contiguous(), k.contiguous(), v.contiguous()
        a2, g2 = alpha.contiguous(), g.contiguous()
        gk2 = None if gk is None else gk.contiguous()
        n = int(num_iter)
        rows, nblk = _segment_table(_lib.PLAN_GKA, [(i * T, i * T + T) for i in range(B)],
                                    B * T, H, dev, _segment_chunks)
        seg = _device_table(rows, dev)
        lib = _lib.load()
        ws = torch.empty(max(int(lib.hmx_gka_chunk_workspace_bytes(len(rows), nblk, B, H)), 16),
                         dtype=torch.uint8, device=dev)
        o = torch.empty_like(q2)
        x = torch.empty_like(q2) if n > 0 else None
        fro = torch.empty(B, T, H, dtype=torch.float32, device=dev) if n > 0 else None
        hkk = torch.empty(B, H, D, D, dtype=torch.float32, device=dev) if n > 0 else None
        hkv = torch.empty(B, H, D, D, dtype=torch.float32, device=dev)
        _lib.call("hmx_gka_train_fwd", _lib.ptr(q2), _lib.ptr(k2), _lib.ptr(v2),
                  _lib.dtype_code(q2), _lib.ptr(a2), _lib.dtype_code(a2), _lib.ptr(g2),
                  _lib.dtype_code(g2), _lib.ptr(gk2), 0 if gk2 is None else _lib.dtype_code(gk2),
                  _lib.ptr(o), _lib.ptr(x), _lib.ptr(fro), _lib.ptr(hkk), _lib.ptr(hkv),
                  _lib.ptr(seg), len(rows), nblk, B, H, D, n, float(ridge_strength),
                  float(gla_scale), _lib.ptr(ws), ws.numel(), _lib.stream_of(q2))
        ctx.save_for_backward(q2, k2, v2, a2, g2, gk2, x, fro, ws, seg)
        # unused outputs give None gradients, so a loss that does use a final state is
        # told apart from one that does not (see backward)
        ctx.set_materialize_grads(False)
        ctx.meta = (len(rows), nblk, n, float(ridge_strength), float(gla_scale), bool(bp_lambda),
                    (q.dtype, k.dtype, v.dtype, alpha.dtype, g.dtype,
                     None if gk is None else gk.dtype))
        return o, hkk, hkv

    @staticmethod
    def backward(ctx, do, d_kk=None, d_kv=None):
        # d_kk is dropped, as the reference's ChebyshevIteration.backward drops
        # d_kk_final (chebyshev_iteration.py:606-688).  fla's chunk_simple_gla
        # (gka_chebyshev_solve.py:159) would carry d_kv into the readout's reverse
        # scan; these kernels seed that scan with zero only, so refuse it.
        if d_kv is not None:
            raise NotImplementedError("hmx gka_chebyshev_gla backward: the gradient of the "
                                      "final state kv_final is not supported; use the output o "
                                      "in the loss")
        q, k, v, alpha, g, gk, x, fro, ws, seg = ctx.saved_tensors
        nrows, nblk, n, ridge, scale, bp_lambda, dts = ctx.meta
        B, T, H, D = q.shape
        dev = q.device
        if do is None:
            do = torch.zeros_like(q)
        do2 = do.to(torch.bfloat16).contiguous()
        f32 = dict(dtype=torch.float32, device=dev)
        dq, dk, dv = (torch.empty(B, T, H, D, dtype=torch.bfloat16, device=dev) for _ in range(3))
        dg = torch.empty(B, T, H, **f32)
        dalpha = torch.empty(B, T, H, **f32) if n > 0 else None
        dgk = torch.empty(B, T, H, **f32) if (n > 0 and gk is not None) else None
        lib = _lib.load()
        bws = torch.empty(max(int(lib.hmx_gka_train_bwd_workspace_bytes(nblk, H, B * T)), 16),
                          dtype=torch.uint8, device=dev)
        _lib.call("hmx_gka_train_bwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.dtype_code(q),
                  _lib.ptr(alpha), _lib.dtype_code(alpha), _lib.ptr(g), _lib.dtype_code(g),
                  _lib.ptr(gk), 0 if gk is None else _lib.dtype_code(gk), _lib.ptr(x),
                  _lib.ptr(fro), _lib.ptr(do2), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv),
                  _lib.ptr(dalpha), _lib.ptr(dg), _lib.ptr(dgk), _lib.ptr(seg), nrows, nblk, B,
                  H, D, B * T, n, ridge, scale, int(bp_lambda), _lib.ptr(ws), ws.numel(),
                  _lib.ptr(bws), bws.numel(), _lib.stream_of(q))
        cast = lambda t, dt: None if (t is None or dt is None) else t.to(dt)
        if gk is None or n == 0:
            dgk = None
        return (cast(dq, dts[0]), cast(dk, dts[1]), cast(dv, dts[2]), cast(dalpha, dts[3]),
                cast(dg, dts[4]), cast(dgk, dts[5]), None, None, None, None, None)
