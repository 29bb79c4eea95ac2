"""Mamba2 SSD ops: chunk scan (mamba_ssm and vLLM-varlen signatures) and the
single-token selective_state_update, on the HIP kernels in libhmx.so.

The reference calls un-vendored kernels (mamba_ssm 2.3.0, vLLM 0.15.1) from
  training/src/hmf/model/hybrid_zoo/layers/mamba/mamba2.py:555-580 (scan),
  :776-800 (decode step), and
  vllm-inference/src/primed_vllm/primed_mamba2_layer.py:844-863 (varlen scan),
  :1000-1021 (decode step).
These wrappers keep those names, argument orders, defaults and return shapes.
"""
from __future__ import annotations

import torch

from .. import _lib
from .gdn import _cu_count, _device_table, _segment_table, seq_bounds

SSD_CHUNK = 64                 # the kernel's internal chunk length (tokens)
PAD_SLOT_ID = -1


def _vec_ok(t: torch.Tensor, dims: tuple[int, ...]) -> bool:
    """Last dim contiguous, the given dims' strides multiples of 8, 16-byte base."""
    return (t.stride(-1) == 1 and all(t.stride(d) % 8 == 0 for d in dims)
            and t.data_ptr() % 16 == 0)


def _tokens_view(t: torch.Tensor) -> torch.Tensor:
    """[b, l, ...] -> [b*l, ...] as a view when the batch dim steps over whole rows."""
    b, l = t.shape[0], t.shape[1]
    if b == 1 or t.stride(0) == l * t.stride(1):
        return t.as_strided((b * l, *t.shape[2:]), (t.stride(1), *t.stride()[2:]),
                            t.storage_offset())
    return t.contiguous().view(b * l, *t.shape[2:])


def _prep3(t: torch.Tensor) -> torch.Tensor:
    """[tokens, heads, dim] with vector-friendly strides (copy only if needed)."""
    return t if _vec_ok(t, (0, 1)) else t.contiguous()


def _ssd_scan(x, dt, A, B, C, D, z, dt_bias, dt_softplus, dt_limit, bounds, h0, y,
              want_final: bool, segment_chunks=None, pooled=None, seg_rows=None):
    """Core launcher over flattened tokens.  z, y [T,H,P]; dt [T,H]; x [T,HX,P],
    B [T,G,N], C [T,GC,N] with HX, G, GC dividing H (head h reads x head
    h // (H // HX), B group h // (H // G), C group h // (H // GC));
    bounds: list of (bos, eos); h0 fp32 [nseq,H,P,N] or None.  Returns the fp32 end
    states [nseq,H,P,N] (or None).  ``pooled`` = (pool, slot indices, has_initial_state
    or None): sequences read and (with want_final) write the pool's slots in place
    instead, and the pool is returned.  ``seg_rows`` (explicit segment rows, see
    _chunk_rows) replaces the planner's table; the call then returns (states,
    segment start states [rows,H,P,N] fp32 or None when no sequence has two)."""
    T, HX, P = x.shape
    H = dt.shape[1]
    G, N, GC = B.shape[1], B.shape[2], C.shape[1]
    if x.dtype != torch.bfloat16 or B.dtype != torch.bfloat16 or C.dtype != torch.bfloat16:
        raise NotImplementedError("hmx SSD scan: x, B and C must be bfloat16 "
                                  f"(got {x.dtype}, {B.dtype}, {C.dtype})")
    if z is not None and z.dtype != torch.bfloat16:
        z = z.to(torch.bfloat16)
    if H % G != 0 or H % GC != 0 or H % HX != 0:
        raise ValueError(f"nheads {H} must be a multiple of ngroups {G} (B), {GC} (C) and of "
                         f"x's heads {HX}")
    if tuple(C.shape) != (T, GC, N) or tuple(y.shape) != (T, H, P):
        raise ValueError(f"C must be [{T}, groups, {N}] and out [{T}, {H}, {P}]")
    if B.shape[0] != T or tuple(dt.shape) != (T, H):
        raise ValueError(f"B must be [{T}, groups, {N}] and dt [{T}, {H}], got "
                         f"{tuple(B.shape)} and {tuple(dt.shape)}")
    if z is not None and tuple(z.shape) != (T, H, P):
        raise ValueError(f"z must be [{T}, {H}, {P}], got {tuple(z.shape)}")
    if any(a < 0 or b < a or b > T for a, b in bounds):
        raise ValueError(f"sequence bounds must lie within the {T} tokens")
    x, B, C, y = _prep3(x), _prep3(B), _prep3(C), y
    z = None if z is None else _prep3(z)
    if not _vec_ok(y, (0, 1)):
        raise ValueError("output tensor must have a contiguous last dim and 8-element strides")
    A32 = A.to(torch.float32).contiguous()
    Dm = None
    if D is not None:
        Dm = (D.to(torch.float32)[:, None].expand(H, P) if D.dim() == 1
              else D.to(torch.float32)).contiguous()
    bias = None if dt_bias is None else dt_bias.to(torch.float32).contiguous()
    nseq = len(bounds)
    idx = hinit = None
    if pooled is not None:
        pool, idx, hinit = pooled
        h0, hT = pool, (pool if want_final else None)
        st_ss, st_dt = pool.stride(0), _lib.dtype_code(pool)
    else:
        hT = (torch.empty(nseq, H, P, N, dtype=torch.float32, device=x.device)
              if want_final else None)
        st_ss, st_dt = H * P * N, _lib.HMX_F32
    if seg_rows is None:
        rows, _ = _segment_table(_lib.PLAN_SSD, bounds, x.shape[0], H, x.device, segment_chunks)
    else:
        rows = seg_rows
    seg = _device_table(rows, x.device)
    lib = _lib.load()
    ws_bytes = int(lib.hmx_ssd_chunk_workspace_bytes(len(rows), nseq, H, P, N))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=x.device)
    lo, hi = float(dt_limit[0]), float(dt_limit[1])
    _lib.call("hmx_ssd_chunk_fwd",
              _lib.ptr(x), x.stride(0), x.stride(1), _lib.ptr(B), B.stride(0), B.stride(1),
              _lib.ptr(C), C.stride(0), C.stride(1), _lib.dtype_code(x),
              _lib.ptr(dt), _lib.dtype_code(dt), dt.stride(0), dt.stride(1),
              _lib.ptr(A32), _lib.ptr(Dm), _lib.ptr(bias),
              _lib.ptr(z), 0 if z is None else z.stride(0), 0 if z is None else z.stride(1),
              _lib.ptr(y), y.stride(0), y.stride(1), _lib.ptr(h0), _lib.ptr(hT), st_ss, st_dt,
              _lib.ptr(idx), _lib.ptr(hinit),
              _lib.ptr(seg), len(rows), nseq, H, HX, G, GC, P, N, int(bool(dt_softplus)), lo, hi,
              _lib.ptr(ws), ws.numel(), _lib.stream_of(x))
    if seg_rows is None:
        return hT
    starts = None
    if len(rows) > nseq:     # the workspace: local end states, then the segment start states
        st = len(rows) * H * P * N
        starts = ws[:2 * st * 4].view(torch.float32)[st:].view(len(rows), H, P, N)
    return hT, starts


def _chunk_rows(cu_chunk, chunk_seq, bounds):
    """Segment rows (n, bos, eos, c_start, c_end, seg_idx, first_seg, nseg) with one
    segment per vLLM chunk [cu_chunk[c], cu_chunk[c+1]) of sequence chunk_seq[c]:
    each segment walks its own 64-token tiles from its first token, and the
    combine chains the segments of a sequence, so the start state of every chunk
    (the end state of the one before) is formed.  Rejects chunks that are empty,
    out of order or do not tile their sequences exactly."""
    nch = len(chunk_seq)
    if len(cu_chunk) != nch + 1:
        raise ValueError(f"cu_chunk_seqlens must hold {nch + 1} offsets, got {len(cu_chunk)}")
    rows, c = [], 0
    for n, (bos, eos) in enumerate(bounds):
        first, pos = c, bos
        while c < nch and chunk_seq[c] == n:
            a, e = cu_chunk[c], cu_chunk[c + 1]
            if a != pos or e <= a or e > eos:
                raise ValueError(f"chunk {c} [{a}, {e}) does not continue sequence {n} "
                                 f"[{bos}, {eos}) at {pos}")
            pos = e
            c += 1
        if pos != eos or (c == first and eos > bos):
            raise ValueError(f"the chunks of sequence {n} do not cover [{bos}, {eos})")
        for j in range(first, c):
            a, e = cu_chunk[j], cu_chunk[j + 1]
            rows.append((n, a, e, 0, (e - a + 63) // 64, j - first, first, c - first))
    if c != nch:
        raise ValueError("seq_idx must list the chunks' sequences in order")
    return rows


def _runs(row: list[int]) -> list[tuple[int, int]]:
    out, a = [], 0
    for i in range(1, len(row) + 1):
        if i == len(row) or row[i] != row[a]:
            out.append((a, i))
            a = i
    return out


def seq_layout(b: int, l: int, seq_idx=None, cu_seqlens=None):
    """The scan's sequences over the flattened [b*l] token axis: (bounds [(bos,
    eos)], first_of_row [sequence starting row r's tokens or -1], last_of_row
    [sequence ending row r or -1], end_at {(row, end): sequence}).  The state
    restarts where seq_idx changes; without it at the cu_seqlens boundaries (b = 1);
    otherwise each row is one sequence."""
    if seq_idx is not None:
        runs_per_row = [_runs(r) for r in seq_idx.to(torch.int64).cpu().tolist()]
    elif cu_seqlens is not None:
        runs_per_row = [[(a, e) for a, e in seq_bounds(cu_seqlens, 1, l) if e > a]]
    else:
        runs_per_row = [[(0, l)] for _ in range(b)]
    bounds, first_of_row, last_of_row, end_at = [], [], [], {}
    for r, runs in enumerate(runs_per_row):
        first_of_row.append(len(bounds) if runs and runs[0][0] == 0 else -1)
        for s0, s1 in runs:
            end_at[(r, s1)] = len(bounds)
            bounds.append((r * l + s0, r * l + s1))
        last_of_row.append(len(bounds) - 1 if runs else -1)
    return bounds, first_of_row, last_of_row, end_at


def start_states(initial_states, first_of_row, nseq: int, shape):
    """fp32 [nseq, *shape] start states with row r's initial state on the sequence
    that starts it (zeros elsewhere), or None without initial states."""
    if initial_states is None:
        return None
    h0 = torch.zeros(nseq, *shape, dtype=torch.float32, device=initial_states.device)
    for r, f in enumerate(first_of_row):
        if f >= 0:
            h0[f] = initial_states[r].to(torch.float32)
    return h0


def mamba_chunk_scan_combined(x, dt, A, B, C, chunk_size, D=None, z=None, dt_bias=None,
                              initial_states=None, seq_idx=None, cu_seqlens=None,
                              dt_softplus=False, dt_limit=(0.0, float("inf")),
                              return_final_states=False, return_varlen_states=False, *,
                              _segment_chunks: int | None = None):
    """mamba_ssm ``mamba_chunk_scan_combined`` (call site mamba2.py:555-580).

    x [b,l,H,P] bf16; dt [b,l,H]; A [H]; B, C [b,l,G,N] bf16; D [H] or [H,P];
    z [b,l,H,P]; dt_bias [H]; initial_states [b,H,P,N] (seeds the first sequence of
    each row); seq_idx [b,l] (the state restarts where it changes; without it,
    cu_seqlens boundaries restart it); cu_seqlens [n+1] with b == 1 selects the
    varlen_states (state after each sequence's last token).  Returns y
    [b,l,H,P] (x.dtype), then final_states [b,H,P,N] fp32 if return_final_states,
    then varlen_states [n,H,P,N] fp32 if return_varlen_states.  chunk_size is
    accepted for signature compatibility: the kernel tiles by 64 tokens and the
    result does not depend on the chunking beyond fp32 rounding.
    """
    ins = (x, dt, A, B, C, D, z, dt_bias, initial_states)
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ins):
        if return_varlen_states:
            raise NotImplementedError("hmx mamba_chunk_scan_combined: return_varlen_states has "
                                      "no backward here")
        from .ssd_train import MambaChunkScanCombined
        return MambaChunkScanCombined.apply(x, dt, A, B, C, chunk_size, D, z, dt_bias,
                                            initial_states, seq_idx, cu_seqlens, dt_softplus,
                                            dt_limit, return_final_states)
    if return_varlen_states and cu_seqlens is None:
        raise ValueError("return_varlen_states requires cu_seqlens")
    if cu_seqlens is not None and x.shape[0] != 1:
        raise ValueError(f"cu_seqlens needs batch size 1, got {x.shape[0]}")
    # seq_idx and cu_seqlens are read on the host only (a CPU tensor costs no copy)
    _lib.require_gpu(x, dt, A, B, C, D, z, dt_bias, initial_states)
    b, l, H, P = x.shape
    G, N = B.shape[2], B.shape[3]
    if initial_states is not None and tuple(initial_states.shape) != (b, H, P, N):
        raise ValueError(f"initial_states must be {(b, H, P, N)}, got {tuple(initial_states.shape)}")
    bounds, first_of_row, last_of_row, end_at = seq_layout(b, l, seq_idx, cu_seqlens)
    h0 = start_states(initial_states, first_of_row, len(bounds), (H, P, N))
    xf, zf = _tokens_view(x), (None if z is None else _tokens_view(z))
    y = torch.empty(b, l, H, P, dtype=x.dtype, device=x.device)
    want = return_final_states or return_varlen_states
    hT = _ssd_scan(xf, _tokens_view(dt), A, _tokens_view(B), _tokens_view(C), D, zf, dt_bias,
                   dt_softplus, dt_limit, bounds, h0, y.view(b * l, H, P), want, _segment_chunks)
    out = [y]
    if return_final_states:
        fin = torch.zeros(b, H, P, N, dtype=torch.float32, device=x.device)
        for r, i in enumerate(last_of_row):
            if i >= 0:
                fin[r] = hT[i]
            elif initial_states is not None:
                fin[r] = initial_states[r].to(torch.float32)
        out.append(fin)
    if return_varlen_states:
        cs = [int(v) for v in cu_seqlens.tolist()]
        idx = []
        for i in range(len(cs) - 1):
            if (0, cs[i + 1]) not in end_at or cs[i + 1] == cs[i]:
                raise ValueError("cu_seqlens boundaries must coincide with the scan's sequences")
            idx.append(end_at[(0, cs[i + 1])])
        out.append(hT.index_select(0, _device_table(idx, x.device)))
    return out[0] if len(out) == 1 else tuple(out)


def mamba_chunk_scan_combined_varlen(x, dt, A, B, C, chunk_size, cu_seqlens, cu_chunk_seqlens=None,
                                     last_chunk_indices=None, seq_idx=None, out=None, D=None,
                                     z=None, dt_bias=None, initial_states=None, dt_softplus=False,
                                     dt_limit=(0.0, float("inf")),
                                     return_intermediate_states=False, state_dtype=None, *,
                                     ssm_state_indices=None, has_initial_state=None,
                                     _segment_chunks: int | None = None):
    """vLLM ``mamba_chunk_scan_combined_varlen`` (call site primed_mamba2_layer.py:844-863).

    x [T,H,P] bf16; dt [T,H]; A [H]; B, C [T,G,N] bf16; cu_seqlens [n+1];
    initial_states [n,H,P,N] or None (each sequence starts from its own state);
    ``out`` [T,H,P] is written in place (allocated when None).  Returns
    varlen_states [n,H,P,N] in state_dtype (fp32 when None).  cu_chunk_seqlens,
    last_chunk_indices and seq_idx are chunking metadata derived from
    cu_seqlens; the kernel uses its own 64-token tiles.  With
    return_intermediate_states (prefix caching, primed_mamba2_layer.py:862-921) the
    return is instead the state after each chunk [nchunks,H,P,N] (state_dtype), the
    chunks given by cu_chunk_seqlens and their sequences by seq_idx (one entry per
    chunk): each chunk becomes one segment of the scan, whose combine forms every
    chunk's start state (the scan's output y is unchanged).

    Keyword-only extension (no reference counterpart): with ``ssm_state_indices``
    [n], ``initial_states`` is the layer's state pool [slots,H,P,N] (fp32 or bf16):
    sequence i starts from slot ``ssm_state_indices[i]`` (zero where
    ``has_initial_state`` [n] is False or the slot is negative) and its end state
    is written back into that slot in place; the pool is returned.  This replaces
    the layer's gather and scatter around the op (primed_mamba2_layer.py:812-824,
    :941).

    Grouped operands (no reference counterpart): the heads H are dt's; x may hold
    HX heads and C its own GC groups (each dividing H), head h reading x head
    h // (H // HX) and C group h // (H // GC), as B's groups already work.  The
    primed layer's repeat_kv'd x and B (primed_mamba2_layer.py:800-835) are read
    in place this way.
    """
    _lib.require_gpu(x, dt, A, B, C, D, z, dt_bias, initial_states, out)   # cu_seqlens: host or device
    T, P = x.shape[0], x.shape[2]
    H = dt.shape[1]
    N = B.shape[-1]
    bounds = seq_bounds(cu_seqlens, 1, T)
    pooled = h0 = None
    if ssm_state_indices is not None:
        _lib.require_gpu(ssm_state_indices, has_initial_state)
        pool = initial_states
        if (pool is None or pool.dim() != 4 or tuple(pool.shape[1:]) != (H, P, N)
                or not pool[0].is_contiguous() or pool.dtype not in (torch.float32, torch.bfloat16)):
            raise ValueError(f"with ssm_state_indices, initial_states must be the state pool "
                             f"[slots,{H},{P},{N}] fp32/bf16 with contiguous slots")
        idx = ssm_state_indices.to(torch.int32).contiguous()
        if idx.shape != (len(bounds),):
            raise ValueError(f"ssm_state_indices must hold {len(bounds)} slots")
        hinit = None
        if has_initial_state is not None:
            if has_initial_state.shape != (len(bounds),):
                raise ValueError(f"has_initial_state must be [{len(bounds)}]")
            hinit = has_initial_state.to(torch.uint8).contiguous()
        pooled = (pool, idx, hinit)
    else:
        if initial_states is not None and tuple(initial_states.shape) != (len(bounds), H, P, N):
            raise ValueError(f"initial_states must be {(len(bounds), H, P, N)}, "
                             f"got {tuple(initial_states.shape)}")
        if has_initial_state is not None:
            raise ValueError("has_initial_state needs ssm_state_indices")
        h0 = None if initial_states is None else initial_states.to(torch.float32).contiguous()
    if out is None:
        out = torch.empty(T, H, P, dtype=x.dtype, device=x.device)
    if out.dtype != x.dtype:
        raise ValueError(f"out dtype {out.dtype} must match x dtype {x.dtype}")
    if return_intermediate_states:
        if cu_chunk_seqlens is None or seq_idx is None:
            raise ValueError("return_intermediate_states needs cu_chunk_seqlens and seq_idx")
        # host metadata (vLLM's CPU copies) is read without a device sync
        cc = [int(v) for v in cu_chunk_seqlens.tolist()]
        cs_seq = [int(v) for v in seq_idx.reshape(-1).tolist()]
        rows = _chunk_rows(cc, cs_seq, bounds)
        nch = len(rows)
        last = [i for i, r in enumerate(rows) if r[5] == r[7] - 1]
        # checked before the scan writes out and the caller's pool
        if last_chunk_indices is not None and [int(v) for v in last_chunk_indices.tolist()] != last:
            raise ValueError("last_chunk_indices must index each sequence's last chunk")
        hT, starts = _ssd_scan(x, dt, A, B, C, D, z, dt_bias, dt_softplus, dt_limit, bounds, h0,
                               out, True, None, pooled, seg_rows=rows)
        # the state after chunk c: the next chunk's start state, or its sequence's end
        # state; one gather over [starts; end states] with a host-built index
        # (advanced indexing: a negative pad slot wraps around instead of faulting;
        # such a sequence has no state in the pool, so its returned rows mean nothing)
        fin = (hT[pooled[1].long()] if pooled is not None else hT).to(torch.float32)
        src = fin if starts is None else torch.cat([starts, fin])
        nst = 0 if starts is None else starts.shape[0]
        gidx = [nst + r[0] if r[5] == r[7] - 1 else i + 1 for i, r in enumerate(rows)]
        states = src.index_select(0, _device_table(gidx, x.device)) if nch else \
            src.new_empty(0, H, P, N)
        return states if state_dtype in (None, torch.float32) else states.to(state_dtype)
    hT = _ssd_scan(x, dt, A, B, C, D, z, dt_bias, dt_softplus, dt_limit, bounds, h0, out, True,
                   _segment_chunks, pooled)
    if pooled is not None:
        return hT
    return hT if state_dtype in (None, torch.float32) else hT.to(state_dtype)


def selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                           dt_softplus=False, state_batch_indices=None,
                           dst_state_batch_indices=None, pad_slot_id=PAD_SLOT_ID, out=None,
                           num_accepted_tokens=None, cu_seqlens=None):
    """mamba_ssm / vLLM ``selective_state_update``: one decode step, in place on
    ``state`` (calls mamba2.py:789-800, primed_mamba2_layer.py:1007-1021).

    state [slots,H,P,N] (or [slots,P,N]); x, dt [b,H,P] (or [b,P]); A [H,P,N];
    B, C [b,G,N] (or [b,N]); D, dt_bias [H,P]; z [b,H,P]; state_batch_indices
    [b] (entries equal to pad_slot_id are skipped); dst_state_batch_indices [b]
    (write target, default the source slot).  ``out`` is written in place
    (allocated like dt when None, in x's dtype) and returned.

    Grouped operands (no reference counterpart): x may hold HX heads and C its
    own GC groups (each dividing H), head h reading x head h // (H // HX) and C
    group h // (H // GC), so the primed layer's repeat_kv'd x and B
    (primed_mamba2_layer.py:972-985) are read in place.
    """
    if num_accepted_tokens is not None or cu_seqlens is not None:
        raise NotImplementedError("multi-token (speculative) selective_state_update is not "
                                  "supported by hmx")
    _lib.require_gpu(state, x, dt, A, B, C, D, z, dt_bias, state_batch_indices,
                     dst_state_batch_indices, out)
    headless = state.dim() == 3
    if headless:   # no head dim
        state, x, dt, A = state.unsqueeze(1), x.unsqueeze(1), dt.unsqueeze(1), A.unsqueeze(0)
        B, C = B.unsqueeze(1), C.unsqueeze(1)
        D = None if D is None else D.unsqueeze(0)
        z = None if z is None else z.unsqueeze(1)
        dt_bias = None if dt_bias is None else dt_bias.unsqueeze(0)
        if out is not None:
            out = out.unsqueeze(1)
    slots, H, P, N = state.shape
    bsz = x.shape[0]
    G, GC, HX = B.shape[1], C.shape[1], x.shape[1]
    if (x.dim() != 3 or x.shape[0] != bsz or x.shape[2] != P or H % HX != 0
            or tuple(dt.shape) != (bsz, H, P)):
        raise ValueError(f"x must be [{bsz}, heads dividing {H}, {P}] and dt {(bsz, H, P)}, got "
                         f"{tuple(x.shape)}, {tuple(dt.shape)}")
    if tuple(A.shape) != (H, P, N):
        raise ValueError(f"A must be {(H, P, N)}, got {tuple(A.shape)}")
    if H % G != 0 or H % GC != 0 or tuple(B.shape) != (bsz, G, N) or tuple(C.shape) != (bsz, GC, N):
        raise ValueError(f"B, C must be [{bsz}, groups, {N}] with groups dividing {H}")
    if state.stride(3) != 1 or state.stride(2) != N or state.stride(1) != P * N:
        raise ValueError("state must be contiguous within a slot ([H,P,N] row-major)")
    if out is None:
        out = torch.empty(bsz, H, P, dtype=x.dtype, device=x.device)
    if tuple(out.shape) != (bsz, H, P):
        raise ValueError(f"out must be {(bsz, H, P)}, got {tuple(out.shape)}")
    A = A if A.dtype == torch.float32 else A.to(torch.float32)
    B = B if B.stride(-1) == 1 else B.contiguous()
    C = C if C.stride(-1) == 1 else C.contiguous()
    D = None if D is None else D.to(torch.float32)
    dt_bias = None if dt_bias is None else dt_bias.to(torch.float32)

    def i32(t):
        return None if t is None else t.to(torch.int32).contiguous()

    src, dst = i32(state_batch_indices), i32(dst_state_batch_indices)
    st = lambda t, i: 0 if t is None else t.stride(i)
    _lib.call("hmx_ssd_state_update",
              _lib.ptr(state), _lib.dtype_code(state), state.stride(0),
              _lib.ptr(x), _lib.dtype_code(x), x.stride(0), x.stride(1), x.stride(2),
              _lib.ptr(dt), _lib.dtype_code(dt), dt.stride(0), dt.stride(1), dt.stride(2),
              _lib.ptr(A), A.stride(0), A.stride(1), A.stride(2),
              _lib.ptr(B), _lib.dtype_code(B), B.stride(0), B.stride(1),
              _lib.ptr(C), _lib.dtype_code(C), C.stride(0), C.stride(1),
              _lib.ptr(D), st(D, 0), st(D, 1), _lib.ptr(dt_bias), st(dt_bias, 0), st(dt_bias, 1),
              _lib.ptr(z), 0 if z is None else _lib.dtype_code(z), st(z, 0), st(z, 1), st(z, 2),
              _lib.ptr(out), _lib.dtype_code(out), out.stride(0), out.stride(1), out.stride(2),
              _lib.ptr(src), _lib.ptr(dst), int(pad_slot_id), bsz, H, HX, G, GC, P, N,
              int(bool(dt_softplus)), _lib.stream_of(x))
    return out.squeeze(1) if headless else out


__all__ = ["mamba_chunk_scan_combined", "mamba_chunk_scan_combined_varlen",
           "selective_state_update"]
