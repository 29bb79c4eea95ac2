"""Mamba2 SSD chunk scan with its backward (hmx.MambaChunkScanCombined).

The training layer calls mamba_ssm's ``mamba_chunk_scan_combined`` under autograd
(training/src/hmf/model/hybrid_zoo/layers/mamba/mamba2.py:555-580).  The forward
here is the HIP scan of ops/ssd.py.  The backward (csrc/ssd_backward.hip) forms
the state at the start of every 64-token chunk again from the inputs (nothing
beyond them is kept between forward and backward): a local pass per chunk, one
scan launch running the forward state chain and the reverse chain of the state
gradients, then the per-chunk gradient kernel.
"""
from __future__ import annotations

import torch

from .. import _lib
from .gdn import _device_table
from .ssd import (SSD_CHUNK, _prep3, _tokens_view, mamba_chunk_scan_combined, seq_layout,
                  start_states)


def _chunk_table(bounds):
    """Segment rows (n, bos, eos, 0, 1, index in the sequence, first row, rows) with
    one row per 64-token chunk of every sequence (a forward over them forms every
    chunk's start state), and the per-sequence (first row, rows) table."""
    rows, seqs = [], []
    for n, (a, e) in enumerate(bounds):
        first, starts = len(rows), list(range(a, e, SSD_CHUNK))
        for k, c in enumerate(starts):
            rows.append((n, c, min(c + SSD_CHUNK, e), 0, 1, k, first, len(starts)))
        seqs.append((first, len(starts)))
    return rows, seqs


def ssd_chunk_scan_bwd(x, dt, A, B, C, D, z, dt_bias, dt_softplus, dt_limit, bounds, h0, dy,
                       d_final=None, want_dh0=False):
    """Gradients of the flattened scan (the _ssd_scan layout: x [T,HX,P], dt [T,H],
    B [T,G,N], C [T,GC,N], z, dy [T,H,P]; h0 fp32 [nseq,H,P,N] or None; d_final fp32
    [nseq,H,P,N] or None).  Returns (dx, ddt, dA [H], dB, dC, dD [H,P] or None,
    ddt_bias [H] or None, dh0 or None, dz or None): dx, dB, dC in bf16 unless x or B
    is shared by several heads (then fp32), dz bf16, the rest fp32."""
    T, HX, P = x.shape
    H = dt.shape[1]
    G, N, GC = B.shape[1], B.shape[2], C.shape[1]
    dev = x.device
    if P not in (64, 128) or N not in (64, 128):
        raise NotImplementedError(f"hmx SSD backward: headdim and d_state in 64/128 "
                                  f"(got {P}, {N})")
    if P == 128 and z is not None:
        raise NotImplementedError("hmx SSD backward: the z gate needs headdim 64 (the training "
                                  "layer with its RMSNorm passes z = None)")
    rows, seqs = _chunk_table(bounds)
    nseq, nrows = len(bounds), len(rows)
    x, B, C = _prep3(x), _prep3(B), _prep3(C)
    z = None if z is None else _prep3(z.to(torch.bfloat16))
    dy = _prep3(dy.to(torch.bfloat16))
    A32 = A.to(torch.float32).contiguous()
    Dm = None
    if D is not None:
        Dm = (D.to(torch.float32)[:, None].expand(H, P) if D.dim() == 1
              else D.to(torch.float32)).contiguous()
    bias = None if dt_bias is None else dt_bias.to(torch.float32).contiguous()
    f32 = dict(dtype=torch.float32, device=dev)
    # shared operands accumulate (fp32); otherwise dx, dB, dC are written in bf16;
    # tokens outside every sequence keep zero gradients
    full = sum(e - a for a, e in bounds) == T
    alloc = lambda shared: torch.empty if (full and not shared) else torch.zeros
    acc_x, acc_b = HX < H, G < H and G != GC
    gdt = torch.float32 if (acc_x or acc_b) else torch.bfloat16
    dx = alloc(acc_x)(T, HX, P, dtype=gdt, device=dev)
    dB = alloc(acc_b)(T, G, N, dtype=gdt, device=dev)
    dC = alloc(False)(T, GC, N, dtype=gdt, device=dev)
    dz = None if z is None else alloc(False)(T, H, P, dtype=torch.bfloat16, device=dev)
    ddt = alloc(False)(T, H, **f32)
    dA = torch.zeros(H, **f32)
    dD = None if D is None else torch.zeros(H, P, **f32)
    dbias = None if dt_bias is None else torch.zeros(H, **f32)
    dh0 = torch.empty(nseq, H, P, N, **f32) if want_dh0 and nseq else None
    if d_final is not None:
        d_final = d_final.to(torch.float32).contiguous()
    seg = _device_table(rows if rows else [(0,) * 8], dev)
    sq = _device_table(seqs if seqs else [(0, 0)], dev)
    lib = _lib.load()
    ws_bytes = int(lib.hmx_ssd_chunk_bwd_workspace_bytes(nrows, H, P, N))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    lo, hi = float(dt_limit[0]), float(dt_limit[1])
    _lib.call("hmx_ssd_chunk_bwd",
              _lib.ptr(x), x.stride(0), x.stride(1), _lib.ptr(B), B.stride(0), B.stride(1),
              _lib.ptr(C), C.stride(0), C.stride(1), _lib.dtype_code(x),
              _lib.ptr(dt), _lib.dtype_code(dt), dt.stride(0), dt.stride(1),
              _lib.ptr(A32), _lib.ptr(Dm), _lib.ptr(bias),
              _lib.ptr(z), 0 if z is None else z.stride(0), 0 if z is None else z.stride(1),
              _lib.ptr(dy), dy.stride(0), dy.stride(1),
              _lib.ptr(h0), _lib.ptr(d_final),
              _lib.ptr(seg), nrows, _lib.ptr(sq), nseq, H, HX, G, GC, P, N,
              int(bool(dt_softplus)), lo, hi,
              _lib.ptr(dx), _lib.ptr(dB), _lib.ptr(dC), _lib.dtype_code(dx), _lib.ptr(dz),
              _lib.ptr(ddt),
              _lib.ptr(dA), _lib.ptr(dD), _lib.ptr(dbias), _lib.ptr(dh0),
              _lib.ptr(ws), ws.numel(), _lib.stream_of(x))
    return dx, ddt, dA, dB, dC, dD, dbias, dh0, dz


class MambaChunkScanCombined(torch.autograd.Function):
    """mamba_chunk_scan_combined with a backward (mamba2.py:555-580 under autograd).

    Same arguments and returns as ops.ssd.mamba_chunk_scan_combined, except
    return_varlen_states (an inference output) which is not differentiable here.
    Gradients flow to x, dt, A, B, C, D, z, dt_bias and initial_states, from y and
    from final_states when returned."""

    @staticmethod
    def forward(ctx, x, dt, A, B, C, chunk_size, D=None, z=None, dt_bias=None,
                initial_states=None, seq_idx=None, cu_seqlens=None, dt_softplus=False,
                dt_limit=(0.0, float("inf")), return_final_states=False):
        out = mamba_chunk_scan_combined(x, dt, A, B, C, chunk_size, D=D, z=z, dt_bias=dt_bias,
                                        initial_states=initial_states, seq_idx=seq_idx,
                                        cu_seqlens=cu_seqlens, dt_softplus=dt_softplus,
                                        dt_limit=dt_limit, return_final_states=return_final_states)
        ctx.save_for_backward(x, dt, A, B, C, D, z, dt_bias, initial_states)
        ctx.seq_idx = None if seq_idx is None else seq_idx.detach().cpu()
        ctx.cu_seqlens = None if cu_seqlens is None else cu_seqlens.detach().cpu()
        ctx.dt_softplus, ctx.dt_limit = dt_softplus, dt_limit
        ctx.return_final_states = return_final_states
        return out

    @staticmethod
    def backward(ctx, dy, d_fin=None):
        x, dt, A, B, C, D, z, dt_bias, initial_states = ctx.saved_tensors
        b, l, H, P = x.shape
        G, N, GC = B.shape[2], B.shape[3], C.shape[2]
        bounds, first_of_row, last_of_row, _ = seq_layout(b, l, ctx.seq_idx, ctx.cu_seqlens)
        h0 = start_states(initial_states, first_of_row, len(bounds), (H, P, N))
        d_final = None
        if ctx.return_final_states and d_fin is not None:
            d_final = torch.zeros(len(bounds), H, P, N, dtype=torch.float32, device=x.device)
            for r, i in enumerate(last_of_row):
                if i >= 0:
                    d_final[i] = d_fin[r].to(torch.float32)
        need_dh0 = initial_states is not None and ctx.needs_input_grad[9]
        dx, ddt, dA, dB, dC, dD, dbias, dh0, dz = ssd_chunk_scan_bwd(
            _tokens_view(x), _tokens_view(dt), A, _tokens_view(B), _tokens_view(C), D,
            None if z is None else _tokens_view(z), dt_bias, ctx.dt_softplus, ctx.dt_limit,
            bounds, h0, dy.reshape(b * l, H, P), d_final, want_dh0=need_dh0)
        g_init = None
        if need_dh0:
            g_init = torch.zeros(b, H, P, N, dtype=torch.float32, device=x.device)
            for r, f in enumerate(first_of_row):
                if f >= 0:
                    g_init[r] = dh0[f]
            if d_fin is not None:   # a row without tokens returns its initial state
                for r, i in enumerate(last_of_row):
                    if i < 0:
                        g_init[r] += d_fin[r].to(torch.float32)
            g_init = g_init.to(initial_states.dtype)
        gD = None
        if dD is not None:
            gD = (dD.sum(-1) if D.dim() == 1 else dD).to(D.dtype)
        return (dx.view(b, l, H, P).to(x.dtype), ddt.view(b, l, H).to(dt.dtype), dA.to(A.dtype),
                dB.view(b, l, G, N).to(B.dtype), dC.view(b, l, GC, N).to(C.dtype), None, gD,
                None if dz is None else dz.view(b, l, H, P).to(z.dtype),
                None if dbias is None else dbias.to(dt_bias.dtype), g_init,
                None, None, None, None, None)
