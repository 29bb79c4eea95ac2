"""Short causal depthwise conv1d CPU oracle — test infrastructure only (see package doc).

The input-side convolution of the GDN / GKA / Mamba2 layers (vLLM's
``causal_conv1d_fn`` for prefill and ``causal_conv1d_update`` for decode, called at
vllm-inference/src/primed_vllm/primed_gdn_layer.py:700-780; both un-vendored).
Semantics, per channel c with kernel width W and weight w[c, 0..W-1]:

    out[t, c] = act(bias[c] + sum_i w[c, i] x[t - (W-1) + i, c]),  act = silu or none

where x at positions before a sequence's first token comes from its conv state
(the previous W-1 inputs; zeros without an initial state).  After the call the
state holds the last state_len inputs of the sequence (older state rows shifted
in front when the sequence is shorter).  This is the reference's torch form
``torch_causal_conv1d_update`` (training/src/hmf/model/hybrid_zoo/models/
qwen3_5_moe_hmf/modeling_qwen3_5_moe_hmf.py:306-321: concatenate state and
inputs, depthwise conv1d, keep the last seq_len outputs, silu, state <- last
state_len inputs) applied per sequence.  The vLLM state layout is
[slots, state_len, dim] (primed_utils.py:174-177, "V1 format: swapped
dimensions"), state_len = W - 1 (+ speculative tokens).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

DEFAULT = torch.float64


def conv_sequence(x: torch.Tensor, state: torch.Tensor | None, weight: torch.Tensor,
                  bias: torch.Tensor | None, activation: str | None, dtype=DEFAULT):
    """One sequence: x [T, dim], state [state_len, dim] or None (zeros, state_len =
    W - 1).  Returns (out [T, dim], new_state [state_len, dim]) in ``dtype``."""
    W = weight.shape[-1]
    xs = x.to(dtype)
    st = (torch.zeros(W - 1, x.shape[-1], dtype=dtype) if state is None else state.to(dtype))
    full = torch.cat([st, xs], dim=0)                     # [state_len + T, dim]
    T = xs.shape[0]
    w = weight.to(dtype)
    out = torch.zeros(T, x.shape[-1], dtype=dtype)
    for i in range(W):
        # tap i reads position t - (W-1) + i, i.e. row (state_len - (W-1) + t + i) of full
        off = st.shape[0] - (W - 1) + i
        out += w[:, i] * full[off:off + T]
    if bias is not None:
        out += bias.to(dtype)
    if activation in ("silu", "swish"):
        out = F.silu(out)
    return out, full[-st.shape[0]:].clone()


def causal_conv1d_varlen(x, weight, bias, conv_states, query_start_loc, cache_indices,
                         has_initial_state, activation="silu", pad_slot_id=-1, dtype=DEFAULT):
    """Prefill over concatenated sequences.  x [total, dim]; conv_states [slots,
    state_len, dim] (updated copy returned); returns (out [total, dim], states)."""
    qs = [int(v) for v in query_start_loc.tolist()]
    states = conv_states.to(dtype).clone()
    out = torch.zeros(x.shape, dtype=dtype)
    for b in range(len(qs) - 1):
        slot = int(cache_indices[b]) if cache_indices is not None else b
        if slot == pad_slot_id:
            continue
        # no flags: no initial states (vLLM's causal_conv1d_fn loads the cached state
        # only where a has_initial_state tensor says so)
        init = bool(has_initial_state[b]) if has_initial_state is not None else False
        st = states[slot] if init else torch.zeros_like(states[slot])
        o, ns = conv_sequence(x[qs[b]:qs[b + 1]], st, weight, bias, activation, dtype)
        out[qs[b]:qs[b + 1]] = o
        states[slot] = ns
    return out, states


def causal_conv1d_update(x, conv_state, weight, bias, activation, conv_state_indices,
                         pad_slot_id=-1, dtype=DEFAULT):
    """Decode: x [batch, dim] (one token per sequence) against the slot pool
    [slots, state_len, dim].  Returns (out [batch, dim], updated pool copy)."""
    states = conv_state.to(dtype).clone()
    out = torch.zeros(x.shape, dtype=dtype)
    for b in range(x.shape[0]):
        slot = int(conv_state_indices[b]) if conv_state_indices is not None else b
        if slot == pad_slot_id:
            continue
        o, ns = conv_sequence(x[b:b + 1], states[slot], weight, bias, activation, dtype)
        out[b] = o[0]
        states[slot] = ns
    return out, states


def causal_conv1d_varlen_blocks(x, weight, bias, conv_states, query_start_loc, cache_indices,
                                has_initial_state, initial_state_idx, first_block, last_block,
                                num_computed_tokens, block_size, activation="silu",
                                pad_slot_id=-1, dtype=DEFAULT):
    """Prefill with prefix caching (vLLM's block arguments, as the Mamba2 layer passes
    them, vllm-inference/src/primed_vllm/primed_mamba2_layer.py:770-793).
    cache_indices [batch, blocks] holds one slot per block of block_size tokens.
    Sequence b continues num_computed_tokens[b] tokens: it reads its initial state
    from column initial_state_idx[b] (where has_initial_state[b]); block k in
    first_block[b] .. last_block[b] - 1 ends inside this step and column k receives
    the state at its end, the last state_len inputs before absolute position
    (k + 1) * block_size (the position the layer's SSD states use for the same
    blocks, :864-933); column last_block[b] receives the state after the last
    token.  A sequence whose last column's slot is pad_slot_id is skipped (output
    0); reads see the pool as it was before the call.  Returns (out, states)."""
    qs = [int(v) for v in query_start_loc.tolist()]
    before = conv_states.to(dtype)
    states = before.clone()
    L = before.shape[1]
    out = torch.zeros(x.shape, dtype=dtype)
    for b in range(len(qs) - 1):
        row = [int(v) for v in cache_indices[b].tolist()]
        last, first = int(last_block[b]), int(first_block[b])
        if row[last] == pad_slot_id:
            continue
        rslot = row[int(initial_state_idx[b])]
        init = has_initial_state is not None and bool(has_initial_state[b]) and \
            rslot != pad_slot_id
        st = before[rslot] if init else torch.zeros(L, x.shape[-1], dtype=dtype)
        xb = x[qs[b]:qs[b + 1]].to(dtype)
        o, _ = conv_sequence(xb, st, weight, bias, activation, dtype)
        out[qs[b]:qs[b + 1]] = o
        hist = torch.cat([st, xb])                 # position p of the sequence is row L + p
        nc, T = int(num_computed_tokens[b]), xb.shape[0]
        for k in range(first, last + 1):
            end = (k + 1) * block_size - nc if k < last else T
            if row[k] != pad_slot_id:
                states[row[k]] = hist[end:end + L]
    return out, states


def causal_conv1d_update_blocks(x, conv_state, weight, bias, activation, cache_indices,
                                initial_state_idx, last_block, pad_slot_id=-1, dtype=DEFAULT):
    """Decode with prefix caching (primed_mamba2_layer.py:964-973): the window comes
    from the slot at column initial_state_idx[b] of the [batch, blocks] table and
    the shifted state goes to the slot at column last_block[b]; entries with a pad
    slot are skipped.  Reads see the pool as it was before the call."""
    before = conv_state.to(dtype)
    states = before.clone()
    out = torch.zeros(x.shape, dtype=dtype)
    for b in range(x.shape[0]):
        rs = int(cache_indices[b, int(initial_state_idx[b])])
        ws = int(cache_indices[b, int(last_block[b])])
        if rs == pad_slot_id or ws == pad_slot_id:
            continue
        o, ns = conv_sequence(x[b:b + 1], before[rs], weight, bias, activation, dtype)
        out[b] = o[0]
        states[ws] = ns
    return out, states
