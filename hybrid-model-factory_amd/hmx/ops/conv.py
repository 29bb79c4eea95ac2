"""Short causal depthwise conv1d: the mixers' input convolution.

vLLM's ``causal_conv1d_fn`` (prefill) and ``causal_conv1d_update`` (decode), as the
layers call them (vllm-inference/src/primed_vllm/primed_gdn_layer.py:700-780): x is
the [dim, tokens] transposed view of the [tokens, dim] projection output, the
weight [dim, width], and the conv state pool the [slots, dim, state_len] view
``self_kv_cache[0].transpose(-1, -2)`` (primed_gdn_layer.py:669) of the cache
tensor [slots, state_len, dim] with channels contiguous (primed_utils.py:174-177).
Per channel,

    out[t] = act(bias + sum_i w[i] x[t - (width-1) + i]),  act = silu ("silu"/"swish") or none,

with positions before a sequence's first token taken from its state (zeros
without an initial state); the state then holds the sequence's last state_len
inputs.  Speculative decoding (``num_accepted_tokens`` with ``query_start_loc``) runs
several tokens per sequence against a state with draft slack (see
``causal_conv1d_update``).  Prefix caching (vLLM's block arguments, which the
Mamba2 layer passes with ``mamba_cache_mode == "all"``) reads and writes the
states of a [batch, blocks] slot table by block (see ``causal_conv1d_fn``).
"""
from __future__ import annotations

import torch

from .. import _lib
from .gdn import _device_table

PAD_SLOT_ID = -1


def _act(activation) -> int:
    if activation in (None, False):
        return 0
    if activation is True or activation in ("silu", "swish"):
        return 1
    raise NotImplementedError(f"activation {activation!r} (silu, swish or None)")


def _rows(t: torch.Tensor) -> torch.Tensor:
    """[tokens, dim] rows with channels contiguous and 16-byte aligned rows."""
    if t.stride(-1) != 1 or t.stride(0) % (16 // t.element_size()) or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def _aligned(t):
    """Contiguous with a 16-byte aligned start (the kernels load 16-byte vectors)."""
    if t is None:
        return None
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _pool(st: torch.Tensor, dim: int, dtype, name: str):
    """(state_len, slot stride, row stride) of a [slots, dim, state_len] pool view
    whose channel axis is contiguous."""
    if st.dim() != 3 or st.shape[1] != dim or st.dtype != dtype or st.stride(1) != 1:
        raise ValueError(f"{name} must be the [slots, {dim}, state_len] {dtype} view of a "
                         f"[slots, state_len, {dim}] cache (channels contiguous), got "
                         f"{tuple(st.shape)} strides {st.stride()} {st.dtype}")
    return st.shape[2], st.stride(0), st.stride(2)


def _out_rows(out, rows: int, dim: int, x: torch.Tensor) -> torch.Tensor:
    if out is None:
        return torch.empty(rows, dim, dtype=x.dtype, device=x.device)
    vec = 16 // x.element_size()
    if (tuple(out.shape) != (rows, dim) or out.dtype != x.dtype or out.stride(-1) != 1
            or (rows > 1 and out.stride(0) % vec) or out.data_ptr() % 16):
        raise ValueError(f"out must be [{rows}, {dim}] {x.dtype} with contiguous, 16-byte "
                         f"aligned rows, got {tuple(out.shape)} {out.dtype}")
    return out


def _i32(t):
    return None if t is None else t.to(torch.int32).contiguous()


def causal_conv1d_fn(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
                     conv_states: torch.Tensor | None = None,
                     query_start_loc: torch.Tensor | None = None,
                     cache_indices: torch.Tensor | None = None,
                     has_initial_state: torch.Tensor | None = None,
                     activation: str | None = "silu", pad_slot_id: int = PAD_SLOT_ID,
                     metadata=None, validate_data: bool = False,
                     block_idx_first_scheduled_token: torch.Tensor | None = None,
                     block_idx_last_scheduled_token: torch.Tensor | None = None,
                     initial_state_idx: torch.Tensor | None = None,
                     num_computed_tokens: torch.Tensor | None = None,
                     block_size_to_align: int = 0) -> torch.Tensor:
    """Prefill conv over concatenated sequences.  x [dim, total] (the transposed
    view of [total, dim]); returns the same layout.  ``conv_states`` [slots, dim,
    state_len] (channels contiguous) is updated in place at ``cache_indices``
    (default: sequence b uses slot b).  A sequence starts from its slot's state
    where ``has_initial_state`` [batch] is True, and from zeros elsewhere and when
    it is None (as vLLM's kernel loads initial states only given the flags).

    Prefix caching (the block arguments, primed_mamba2_layer.py:770-793):
    ``cache_indices`` is the [batch, blocks] slot table of block_size_to_align-token
    blocks; sequence b continues num_computed_tokens[b] tokens, reads its initial
    state at column initial_state_idx[b], writes the state at the end of every block
    block_idx_first_scheduled_token[b] .. block_idx_last_scheduled_token[b] - 1 into
    that block's column (the last state_len inputs before the block boundary), and
    the state after its last token into column block_idx_last_scheduled_token[b]."""
    blocks = block_args(initial_state_idx, block_idx_first_scheduled_token,
                        block_idx_last_scheduled_token, num_computed_tokens, block_size_to_align)
    return conv_fwd_rows(x, weight, bias, conv_states, query_start_loc, cache_indices,
                         has_initial_state, activation, pad_slot_id, validate_data,
                         blocks=blocks).t()


def block_args(initial_state_idx, first, last, num_computed_tokens, block_size):
    """The prefix-cache block arguments as ``conv_fwd_rows``'s ``blocks`` tuple, or
    None when none is given; all of them or none."""
    blocks = (initial_state_idx, first, last, num_computed_tokens)
    if all(v is None for v in blocks):
        return None
    if any(v is None for v in blocks) or not block_size or block_size <= 0:
        raise ValueError("prefix caching needs initial_state_idx, block_idx_first_scheduled_token, "
                         "block_idx_last_scheduled_token, num_computed_tokens and "
                         "block_size_to_align > 0 together")
    return blocks + (int(block_size),)


def _table(idx: torch.Tensor, batch: int, name: str):
    """(int32 table, row stride, columns) of a [batch, columns] slot table."""
    t = idx.to(torch.int32)
    if t.dim() != 2 or t.shape[0] < batch or t.shape[1] < 1:
        raise ValueError(f"{name} must be a [batch >= {batch}, blocks] slot table with prefix "
                         f"caching, got {tuple(idx.shape)}")
    if t.stride(1) != 1:
        t = t.contiguous()
    return t, t.stride(0), t.shape[1]


def _per_seq(ts, batch: int, names):
    out = []
    for t, nm in zip(ts, names):
        if t.numel() < batch:
            raise ValueError(f"{nm} needs {batch} entries, got {t.numel()}")
        out.append(_i32(t.reshape(-1)))
    return out


def conv_fwd_rows(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                  conv_states: torch.Tensor | None, query_start_loc: torch.Tensor | None,
                  cache_indices: torch.Tensor | None, has_initial_state: torch.Tensor | None,
                  activation, pad_slot_id: int = PAD_SLOT_ID,
                  validate_data: bool = False, out: torch.Tensor | None = None,
                  blocks=None) -> torch.Tensor:
    """``causal_conv1d_fn`` returning the output as contiguous [total, dim] rows.
    Tokens from ``query_start_loc[-1]`` on belong to no sequence and give 0.  No
    device value is read back unless ``validate_data`` (the kernels clamp sequence
    bounds to the token count, so a malformed ``query_start_loc`` cannot move an
    access outside x).  ``out`` [total, dim] (x's dtype, channels contiguous) receives
    the rows when given.  ``blocks`` = (initial_state_idx, block_idx_first_scheduled_token,
    block_idx_last_scheduled_token, num_computed_tokens, block_size) selects prefix
    caching over the [batch, blocks] table ``cache_indices`` (``causal_conv1d_fn``)."""
    _lib.require_gpu(x, weight, bias, conv_states, query_start_loc, cache_indices,
                     has_initial_state, *(blocks[:4] if blocks else ()))
    dim, total = x.shape
    W = weight.shape[-1]
    if weight.shape != (dim, W):
        raise ValueError(f"weight must be [{dim}, width], got {tuple(weight.shape)}")
    xr = _rows(x.t())
    if query_start_loc is None:
        query_start_loc = _device_table([[0, total]], x.device)[0]
    qs = _i32(query_start_loc)
    batch = qs.shape[0] - 1
    if validate_data:
        bounds = [int(v) for v in qs.tolist()]
        if bounds[0] != 0 or any(b < a for a, b in zip(bounds, bounds[1:])) or \
                bounds[-1] > total:
            raise ValueError(f"query_start_loc must be non-decreasing from 0 to <= {total}: "
                             f"{bounds}")
    out = _out_rows(out, total, dim, x)
    st_len, sst, srs = 0, 0, 0
    if conv_states is not None:
        st_len, sst, srs = _pool(conv_states, dim, x.dtype, "conv_states")
    hinit = None if has_initial_state is None else has_initial_state.to(torch.uint8).contiguous()
    w, b = _aligned(weight), _aligned(bias)
    if blocks is not None:
        if conv_states is None or cache_indices is None:
            raise ValueError("prefix caching needs conv_states and the cache_indices table")
        tab, rs, cols = _table(cache_indices, batch, "cache_indices")
        ini, first, last, ncomp = _per_seq(blocks[:4], batch, (
            "initial_state_idx", "block_idx_first_scheduled_token",
            "block_idx_last_scheduled_token", "num_computed_tokens"))
        _lib.call("hmx_causal_conv1d_fwd_blocks", _lib.ptr(xr), xr.stride(0), _lib.ptr(out),
                  out.stride(0), _lib.dtype_code(x), _lib.ptr(w), _lib.dtype_code(w), W,
                  _lib.ptr(b), 0 if b is None else _lib.dtype_code(b), _lib.ptr(conv_states),
                  sst, srs, st_len, _lib.ptr(qs), batch, total, _lib.ptr(tab), rs, cols,
                  _lib.ptr(hinit), _lib.ptr(ini), _lib.ptr(first), _lib.ptr(last),
                  _lib.ptr(ncomp), blocks[4], dim, _act(activation), int(pad_slot_id),
                  _lib.stream_of(x))
        return out
    _lib.call("hmx_causal_conv1d_fwd", _lib.ptr(xr), xr.stride(0), _lib.ptr(out), out.stride(0),
              _lib.dtype_code(x), _lib.ptr(w), _lib.dtype_code(w), W, _lib.ptr(b),
              0 if b is None else _lib.dtype_code(b), _lib.ptr(conv_states), sst, srs, st_len,
              _lib.ptr(qs), batch, total, _lib.ptr(_i32(cache_indices)), _lib.ptr(hinit),
              dim, _act(activation), int(pad_slot_id), _lib.stream_of(x))
    return out


def causal_conv1d_update(x: torch.Tensor, conv_state: torch.Tensor, weight: torch.Tensor,
                         bias: torch.Tensor | None = None, activation=None,
                         conv_state_indices: torch.Tensor | None = None,
                         num_accepted_tokens: torch.Tensor | None = None,
                         query_start_loc: torch.Tensor | None = None, max_query_len: int = -1,
                         pad_slot_id: int = PAD_SLOT_ID, validate_data: bool = False,
                         block_idx_last_scheduled_token: torch.Tensor | None = None,
                         initial_state_idx: torch.Tensor | None = None, *,
                         out: torch.Tensor | None = None) -> torch.Tensor:
    """Decode conv: x [batch, dim], one token per sequence, against the slot pool
    ``conv_state`` [slots, dim, state_len] (channels contiguous; updated in place:
    the state shifts by one position).  Returns [batch, dim]; padded entries (slot ==
    pad_slot_id) give 0.  ``out`` [batch, dim] (keyword-only, no reference
    counterpart) receives the rows when given.

    Speculative form (``num_accepted_tokens`` and ``query_start_loc`` given, as
    primed_gdn_layer.py:700-712 calls it): x is [tokens, dim], sequence b owning
    rows query_start_loc[b] .. query_start_loc[b+1]-1 (at most state_len - width + 2
    of them).  With a = num_accepted_tokens[b] (the previous step's accepted tokens)
    the window before its first token is state positions a-1 .. a+width-3; the slot
    then holds positions a .. a+state_len-n-1 followed by the n new inputs, so the
    next step's window ends at its last accepted input.  vLLM's kernel is not
    vendored: this position arithmetic is pinned by the invariant that a speculative
    step followed by a step accepting a tokens computes the plain causal convolution
    over the accepted inputs (tests/test_conv_gpu.py).

    Prefix caching (``block_idx_last_scheduled_token`` and ``initial_state_idx``, as
    primed_mamba2_layer.py:964-973 passes them): ``conv_state_indices`` is the
    [batch, blocks] slot table; the window is read from the slot at column
    initial_state_idx[b] and the shifted state written to the slot at column
    block_idx_last_scheduled_token[b]."""
    if block_idx_last_scheduled_token is not None or initial_state_idx is not None:
        if num_accepted_tokens is not None or query_start_loc is not None:
            raise NotImplementedError("speculative decoding with prefix-cache block arguments")
        return _update_blocks(x, conv_state, weight, bias, activation, conv_state_indices,
                              initial_state_idx, block_idx_last_scheduled_token, pad_slot_id,
                              out)
    if num_accepted_tokens is not None or query_start_loc is not None:
        return _update_spec(x, conv_state, weight, bias, activation, conv_state_indices,
                            num_accepted_tokens, query_start_loc, pad_slot_id, out)
    _lib.require_gpu(x, conv_state, weight, bias, conv_state_indices)
    if x.dim() != 2:
        raise NotImplementedError(f"x must be [batch, dim], got {tuple(x.shape)}")
    batch, dim = x.shape
    W = weight.shape[-1]
    if weight.shape != (dim, W):
        raise ValueError(f"weight must be [{dim}, width], got {tuple(weight.shape)}")
    st_len, sst, srs = _pool(conv_state, dim, x.dtype, "conv_state")
    xr = _rows(x)
    out = _out_rows(out, batch, dim, x)
    w, b = _aligned(weight), _aligned(bias)
    _lib.call("hmx_causal_conv1d_update", _lib.ptr(xr), xr.stride(0), _lib.ptr(out), out.stride(0),
              _lib.dtype_code(x), _lib.ptr(w), _lib.dtype_code(w), W, _lib.ptr(b),
              0 if b is None else _lib.dtype_code(b), _lib.ptr(conv_state), sst, srs, st_len,
              _lib.ptr(_i32(conv_state_indices)),
              batch, dim, _act(activation), int(pad_slot_id), _lib.stream_of(x))
    return out


def _update_blocks(x, conv_state, weight, bias, activation, conv_state_indices,
                   initial_state_idx, last_idx, pad_slot_id, out):
    if initial_state_idx is None or last_idx is None or conv_state_indices is None:
        raise ValueError("prefix caching needs conv_state_indices, initial_state_idx and "
                         "block_idx_last_scheduled_token together")
    _lib.require_gpu(x, conv_state, weight, bias, conv_state_indices, initial_state_idx,
                     last_idx)
    if x.dim() != 2:
        raise NotImplementedError(f"x must be [batch, dim], got {tuple(x.shape)}")
    batch, dim = x.shape
    W = weight.shape[-1]
    if weight.shape != (dim, W):
        raise ValueError(f"weight must be [{dim}, width], got {tuple(weight.shape)}")
    st_len, sst, srs = _pool(conv_state, dim, x.dtype, "conv_state")
    tab, rs, cols = _table(conv_state_indices, batch, "conv_state_indices")
    ini, last = _per_seq((initial_state_idx, last_idx), batch,
                         ("initial_state_idx", "block_idx_last_scheduled_token"))
    xr = _rows(x)
    out = _out_rows(out, batch, dim, x)
    w, b = _aligned(weight), _aligned(bias)
    _lib.call("hmx_causal_conv1d_update_blocks", _lib.ptr(xr), xr.stride(0), _lib.ptr(out),
              out.stride(0), _lib.dtype_code(x), _lib.ptr(w), _lib.dtype_code(w), W, _lib.ptr(b),
              0 if b is None else _lib.dtype_code(b), _lib.ptr(conv_state), sst, srs, st_len,
              _lib.ptr(tab), rs, cols, _lib.ptr(ini), _lib.ptr(last), batch, dim,
              _act(activation), int(pad_slot_id), _lib.stream_of(x))
    return out


def _update_spec(x, conv_state, weight, bias, activation, conv_state_indices,
                 num_accepted_tokens, query_start_loc, pad_slot_id, out):
    if num_accepted_tokens is None or query_start_loc is None:
        raise ValueError("the speculative causal_conv1d_update needs both num_accepted_tokens "
                         "and query_start_loc")
    _lib.require_gpu(x, conv_state, weight, bias, conv_state_indices, num_accepted_tokens,
                     query_start_loc)
    if x.dim() != 2:
        raise NotImplementedError(f"x must be [tokens, dim], got {tuple(x.shape)}")
    tokens, dim = x.shape
    batch = query_start_loc.numel() - 1
    if num_accepted_tokens.numel() < batch or (conv_state_indices is not None and
                                               conv_state_indices.numel() < batch):
        raise ValueError(f"num_accepted_tokens / conv_state_indices need {batch} entries")
    W = weight.shape[-1]
    if weight.shape != (dim, W):
        raise ValueError(f"weight must be [{dim}, width], got {tuple(weight.shape)}")
    st_len, sst, srs = _pool(conv_state, dim, x.dtype, "conv_state")
    xr = _rows(x)
    out = _out_rows(out, tokens, dim, x)
    w, b = _aligned(weight), _aligned(bias)
    _lib.call("hmx_causal_conv1d_update_spec", _lib.ptr(xr), xr.stride(0), _lib.ptr(out),
              out.stride(0), _lib.dtype_code(x), _lib.ptr(w), _lib.dtype_code(w), W, _lib.ptr(b),
              0 if b is None else _lib.dtype_code(b), _lib.ptr(conv_state), sst, srs, st_len,
              _lib.ptr(_i32(conv_state_indices)), _lib.ptr(_i32(num_accepted_tokens)),
              _lib.ptr(_i32(query_start_loc)), batch, tokens, dim, _act(activation),
              int(pad_slot_id),
              _lib.stream_of(x))
    return out
