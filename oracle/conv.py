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
