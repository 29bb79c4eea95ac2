"""The vLLM layers' mixer cores over hmx ops: ``gdn_forward_core``,
``gka_forward_core`` and ``mamba2_conv_ssm_forward``.

These restate ``PrimedGatedDeltaNetAttention._forward_core``
(vllm-inference/src/primed_vllm/primed_gdn_layer.py:635-936) and
``PrimedGKAAttention._forward_core`` (primed_gka_layer.py:962-1338) for the
non-speculative batches (pure decode, pure prefill, and mixed batches with the
decodes first) and the speculative ones (``spec_sequence_masks``), with the same
inputs and the same effect: ``core_attn_out`` rows written, the conv and recurrent
state pools updated in place.  Compared with the
reference sequence of calls they drop every copy around the ops:

- the decode and prefill convs write one buffer (no ``torch.cat``);
- q, k and v are column views of that buffer (the reference's
  ``rearrange_mixed_qkv`` makes them contiguous, :485-560);
- the prefill reads and writes the state pool by slot with ``has_initial_state``
  (no gather, zeroing and scatter, :868-879 / primed_gka_layer.py:1245-1266);
- the ops write into ``core_attn_out`` directly (no ``torch.cat`` and no final
  copy, :925-936);
- optionally (``o_norm=(weight, z, eps)``) the layer's output norm runs in the
  ops' epilogue, so ``forward`` skips ``self.o_norm`` (:621-626).

``layer`` is the vLLM layer object (or anything with the attributes the
reference reads: conv1d.weight, activation, A, dt_bias, key_dim, kv_k_dim,
kv_v_dim, num_heads, num_kv_heads, head_k_dim, head_v_dim, tp_size, proj_k / proj_v
(None without the low-rank projection), k_rep / v_rep, and allow_neg_eigval for
GDN / the gka_config attributes for GKA);
``attn_metadata`` is the layer's GDNAttentionMetadata (the fields the reference
reads, with the primed builder's ``non_spec_query_start_loc_d/_p`` in mixed
batches, primed_gdn_attn.py:40-113); ``conv_state`` is
``self_kv_cache[0].transpose(-1, -2)`` and the recurrent pools the other cache
entries, as the reference takes them from the forward context (:667-670).

One deliberate difference: in mixed batches the reference hands the prefill conv
the whole batch's ``has_initial_state`` (primed_gdn_layer.py:753,
primed_gka_layer.py:1083) while its recurrent prefill uses the prefill slice
(primed_gdn_layer.py:870, primed_gka_layer.py:1247); here both use the prefill
slice.

With the low-rank k/v projection (``proj_k``, ``proj_v`` and the optional
learnable residual mixes ``k_rep`` / ``v_rep``), k and v are upsampled to the
query heads before the ops, as the layers' rearrange step does (a library GEMM
through the layer's own modules plus the residual); it needs ``tp_size == 1``.

Speculative batches follow primed_gdn_layer.py:686-712 / :819-836 and
primed_gka_layer.py:1017-1040 / :1185-1205: the spec tokens' conv is the
speculative ``causal_conv1d_update`` (slot ``spec_state_indices_tensor[:, 0]``,
``num_accepted_tokens``), then GDN's recurrent decode reads slot
``spec_state_indices_tensor[n, num_accepted_tokens[n] - 1]`` and leaves the state
after the sequence's last token in slot ``[n, 0]`` (fused_recurrent_gqa.py:95-105,
:135-144); GKA's decode, as the reference's, advances each spec sequence by its
first token only (slot ``[n, 0]``); the rows of its other draft tokens are left
undefined, as the reference's ``new_empty`` output leaves them
(chebyshev_iteration_gqa.py:211).  With non-spec
tokens in the batch too, each part runs on its index-selected rows and the outputs
return by index (the reference's ``index_copy_``, :923-934); the host offsets
(``query_start_loc_cpu``) then describe the whole batch, not the non-spec prefill,
and are not used.

``mamba2_conv_ssm_forward`` restates ``PrimedMamba2Layer.conv_ssm_forward``
(primed_mamba2_layer.py:615-1021) the same way: the decode and prefill convs write
one buffer, the repeat_kv'd x and B and the per-head C are read in place from it
by the SSD ops' grouped operands (no rearrange / repeat_kv / permute copies,
:800-835, :972-985), the prefill scan reads and writes the state pool by slot (no
gather and scatter, :812-824, :941), and both scans write ``output`` directly.
The B/C RMSNorms and the rotary position embedding of B and C
(``use_pos_embed``) run through the layer's own modules, where and as the
reference calls them (:663-671).  With prefix caching (``mamba_cache_mode ==
"all"``, :728-792, :864-933, :943-1021) the state tables are [requests, blocks]:
the conv reads and writes its states by block through the conv ops' block
arguments; the prefill scan starts from the slot of the last computed token's
block, returns the state after every chunk, and the states at the blocks' ends
and after each sequence's last token are copied into the blocks' slots with the
layer's chunk arithmetic (the block and chunk metadata are read on the host, as
the layer's loop does); the decode reads the last computed token's block and
writes the scheduled token's.  In the profile run (``attn_metadata`` None,
:676-697) nothing is written and the x columns repeated over the heads are
returned, as the layer returns them.
"""
from __future__ import annotations

import torch

from . import ops


def _check(layer, md):
    if getattr(layer, "proj_k", None) is not None and layer.tp_size != 1:
        raise NotImplementedError("the low-rank k/v projection needs the k/v all-gather of "
                                  "tensor parallelism, which the hmx mixer cores do not run; "
                                  "tp_size must be 1")


def _conv(layer, md, mixed_qkv, cs):
    """(conv output [n, conv_dim], decode / prefill split) of the non-spec tokens,
    decodes first, in one buffer; updates the conv state pool in place."""
    w = layer.conv1d.weight
    w = w.view(w.size(0), w.size(2))
    x = torch.empty_like(mixed_qkv)
    nd, ndt, npf = md.num_decodes, md.num_decode_tokens, md.num_prefills
    idx, has = md.non_spec_state_indices_tensor, md.has_initial_state
    act = layer.activation
    if nd > 0 and npf > 0:
        ops.causal_conv1d_update(mixed_qkv[:ndt], cs, w, None, act,
                                 conv_state_indices=idx[:nd], out=x[:ndt])
        ops.conv.conv_fwd_rows(mixed_qkv[ndt:].t(), w, None, cs, md.non_spec_query_start_loc_p,
                               idx[nd:], None if has is None else has[nd:], act, out=x[ndt:])
    elif npf > 0:
        ops.conv.conv_fwd_rows(mixed_qkv.t(), w, None, cs, md.non_spec_query_start_loc, idx, has,
                               act, out=x)
    elif nd > 0:
        ops.causal_conv1d_update(mixed_qkv, cs, w, None, act,
                                 conv_state_indices=idx[:mixed_qkv.shape[0]], out=x)
    return x


def _qkv(layer, x):
    """q [1,n,H,Dk], k [1,n,HKV,Dk], v [1,n,HKV,Dv] as column views of x."""
    tp = layer.tp_size
    kd, kk = layer.key_dim // tp, layer.kv_k_dim // tp
    H, HKV = layer.num_heads // tp, layer.num_kv_heads // tp
    n = x.shape[0]
    q = x[:, :kd].view(1, n, H, layer.head_k_dim)
    k = x[:, kd:kd + kk].view(1, n, HKV, layer.head_k_dim)
    v = x[:, kd + kk:].view(1, n, HKV, layer.head_v_dim)
    if getattr(layer, "proj_k", None) is None:
        return q, k, v
    return (q, _low_rank(layer.proj_k, getattr(layer, "k_rep", None), k[0], H),
            _low_rank(layer.proj_v, getattr(layer, "v_rep", None), v[0], H))


def _low_rank(proj, rep, kv, H):
    """k (or v) upsampled from HKV to H heads at tp_size 1, as the layers'
    rearrange step forms it (primed_gdn_layer.py:511-545, primed_gka_layer.py:794-829):
    proj(kv) plus kv repeated over each head group, or plus rep @ kv per token when
    the residual is learnable (rep [H, HKV]).  kv [n, HKV, d] -> [1, n, H, d]."""
    n, HKV, d = kv.shape
    y = proj(kv.reshape(n, HKV * d))
    if isinstance(y, tuple):                 # vLLM linear layers return (out, bias)
        y = y[0]
    y = y.view(n, H, d)
    if rep is None:                          # repeat_interleave residual, added in place
        y.view(n, HKV, H // HKV, d).add_(kv.unsqueeze(2))
    else:
        y = y + torch.matmul(rep, kv.contiguous())
    return y.unsqueeze(0)


def _host_prefill_offsets(num_decodes: int, query_start_loc_cpu):
    """The prefill sequences' offsets from the host copy of the batch's
    query_start_loc (decodes come first in the batch), so that the prefill plans
    its segments without reading a device tensor back."""
    if query_start_loc_cpu is None:
        return None
    q = query_start_loc_cpu[num_decodes:]
    return q - q[0]


def _split(md, query_start_loc_cpu=None):
    nd, ndt, npf = md.num_decodes, md.num_decode_tokens, md.num_prefills
    idx, has = md.non_spec_state_indices_tensor, md.has_initial_state
    mixed = nd > 0 and npf > 0
    dec = None
    if nd > 0:
        cu_d = md.non_spec_query_start_loc_d if mixed else md.non_spec_query_start_loc[:nd + 1]
        dec = (cu_d, idx[:nd] if mixed else idx)
    pre = None
    if npf > 0:
        cu_p = _host_prefill_offsets(nd, query_start_loc_cpu)
        if cu_p is None:
            cu_p = md.non_spec_query_start_loc_p if mixed else md.non_spec_query_start_loc
        pre = (cu_p, idx[nd:] if mixed else idx,
               None if has is None else (has[nd:] if mixed else has))
    return ndt, dec, pre


def _spec_conv(layer, md, mixed_qkv, cs):
    """The speculative tokens' conv (primed_gdn_layer.py:700-712): one call over
    every spec sequence's draft tokens against slot spec_state_indices_tensor[n, 0]."""
    w = layer.conv1d.weight
    w = w.view(w.size(0), w.size(2))
    nsd, sidx = md.num_spec_decodes, md.spec_state_indices_tensor
    return ops.causal_conv1d_update(mixed_qkv, cs, w, None, layer.activation,
                                    conv_state_indices=sidx[:nsd, 0],
                                    num_accepted_tokens=md.num_accepted_tokens,
                                    query_start_loc=md.spec_query_start_loc[:nsd + 1],
                                    max_query_len=sidx.size(-1))


def _by_spec(md, n, rows, core_attn_out, o_norm, run_spec, run_rest):
    """A speculative batch: every token speculative -> run_spec(rows, out, o_norm) in
    place; otherwise each part on its index-selected rows (spec_token_indx,
    non_spec_token_indx) into a scratch output that is copied back by index."""
    if md.num_prefills == 0 and md.num_decodes == 0:
        run_spec(rows, core_attn_out[:n], o_norm)
        return
    z = None if o_norm is None or o_norm[1] is None else o_norm[1][:n]
    for idx, run in ((md.spec_token_indx, run_spec), (md.non_spec_token_indx, run_rest)):
        sub = [None if t is None else t.index_select(0, idx) for t in rows]
        out = core_attn_out.new_empty((idx.numel(),) + tuple(core_attn_out.shape[1:]))
        on = None if o_norm is None else (o_norm[0], None if z is None else z.index_select(0, idx),
                                          o_norm[2])
        run(sub, out, on)
        core_attn_out.index_copy_(0, idx, out)


def _norm_args(o_norm, lo, hi):
    if o_norm is None:
        return {}
    w, z, eps = o_norm
    return dict(o_norm_weight=w, o_norm_gate=None if z is None else z[lo:hi].unsqueeze(0),
                o_norm_eps=eps)


def gdn_forward_core(layer, mixed_qkv: torch.Tensor, b: torch.Tensor, a: torch.Tensor,
                     core_attn_out: torch.Tensor, attn_metadata, conv_state: torch.Tensor,
                     ssm_state: torch.Tensor, *, o_norm=None, query_start_loc_cpu=None) -> None:
    """primed_gdn_layer.py:635-936 over hmx ops (see the module docstring).
    ``o_norm=(weight, z [tokens, H, V], eps)`` fuses the layer's output norm;
    ``query_start_loc_cpu`` (vLLM's host copy of the batch's query_start_loc) lets
    the prefill plan without a device-to-host copy."""
    md = attn_metadata
    if md is None:
        return
    _check(layer, md)
    n = md.num_actual_tokens
    mixed_qkv, b, a = mixed_qkv[:n], b[:n], a[:n]
    beta_scale = 2.0 if getattr(layer, "allow_neg_eigval", False) else 1.0

    def rest(rows, out, on, qsl_cpu=None):
        mq, aa, bb = rows
        x = _conv(layer, md, mq, conv_state)
        q, k, v = _qkv(layer, x)
        # g and beta as fused_gdn_gating and the layer form them (:798-802), computed
        # in the mixer kernels' loads instead of a separate launch
        gates = ops.ProjGates(layer.A, layer.dt_bias, aa, bb, beta_scale=beta_scale)
        o = out.unsqueeze(0)
        m = mq.shape[0]
        ndt, dec, pre = _split(md, qsl_cpu)
        if dec is not None:
            cu_d, idx_d = dec
            ops.fused_recurrent_gated_delta_rule_gqa(
                q[:, :ndt], k[:, :ndt], v[:, :ndt], None, None,
                initial_state=ssm_state, inplace_final_state=True, cu_seqlens=cu_d,
                ssm_state_indices=idx_d, use_qk_l2norm_in_kernel=True, out=o[:, :ndt],
                gates=gates.tokens(0, ndt), **_norm_args(on, 0, ndt))
        if pre is not None:
            cu_p, idx_p, has_p = pre
            ops.chunk_gated_delta_rule_gqa(
                q[:, ndt:], k[:, ndt:], v[:, ndt:], None, None,
                initial_state=ssm_state, output_final_state=True, cu_seqlens=cu_p,
                use_qk_l2norm_in_kernel=True, ssm_state_indices=idx_p, has_initial_state=has_p,
                out=o[:, ndt:], gates=gates.tokens(ndt, m), **_norm_args(on, ndt, m))

    def spec(rows, out, on):
        mq, aa, bb = rows
        q, k, v = _qkv(layer, _spec_conv(layer, md, mq, conv_state))
        gates = ops.ProjGates(layer.A, layer.dt_bias, aa, bb, beta_scale=beta_scale)
        nsd = md.num_spec_decodes
        ops.fused_recurrent_gated_delta_rule_gqa(
            q, k, v, None, None, initial_state=ssm_state, inplace_final_state=True,
            cu_seqlens=md.spec_query_start_loc[:nsd + 1],
            ssm_state_indices=md.spec_state_indices_tensor,
            num_accepted_tokens=md.num_accepted_tokens, use_qk_l2norm_in_kernel=True,
            out=out.unsqueeze(0), gates=gates, **_norm_args(on, 0, mq.shape[0]))

    if md.spec_sequence_masks is None:
        rest((mixed_qkv, a, b), core_attn_out[:n], o_norm, query_start_loc_cpu)
    else:
        _by_spec(md, n, (mixed_qkv, a, b), core_attn_out, o_norm, spec, rest)


def gka_forward_core(layer, mixed_qkv: torch.Tensor, a: torch.Tensor, alpha_in: torch.Tensor,
                     b: torch.Tensor | None, core_attn_out: torch.Tensor, attn_metadata,
                     conv_state: torch.Tensor, h_kk_state: torch.Tensor,
                     h_kv_state: torch.Tensor, *, o_norm=None, query_start_loc_cpu=None) -> None:
    """primed_gka_layer.py:962-1338 over hmx ops (see the module docstring).
    ``o_norm=(weight, z [tokens, H, V], eps)`` fuses the layer's output norm;
    ``query_start_loc_cpu`` as for gdn_forward_core."""
    md = attn_metadata
    if md is None:
        return
    _check(layer, md)
    n = md.num_actual_tokens
    mixed_qkv, a, alpha_in = mixed_qkv[:n], a[:n], alpha_in[:n]
    use_beta = layer.use_beta_gate
    if use_beta:
        b = b[:n]
    fg = layer.use_forgetting_gate
    common = dict(gla_scale=layer.gla_scale, ridge_ratio=layer.ridge_strength,
                  num_iter=layer.num_iter)

    def gates_of(aa, ai, bb):
        # gates as primed_gka_layer.py:1138-1153 form them (fused_gka_gating, or the
        # sigmoids without a forgetting gate; alpha zeroed for num_iter 0 or + 0.5),
        # computed in the mixer kernels' loads instead of separate launches
        return ops.ProjGates(
            layer.A if fg else None, layer.dt_bias, aa, bb if use_beta else None, ai,
            alpha_add=0.5 if (layer.num_iter != 0 and layer._alpha_idx is None) else 0.0,
            alpha_zero=layer.num_iter == 0, gk_from_g=fg and layer.use_forgetting_gate_kk)

    def rest(rows, out, on, qsl_cpu=None):
        mq, aa, ai, bb = rows
        x = _conv(layer, md, mq, conv_state)
        q, k, v = _qkv(layer, x)
        gates = gates_of(aa, ai, bb)
        o = out.unsqueeze(0)
        m = mq.shape[0]
        ndt, dec, pre = _split(md, qsl_cpu)
        if dec is not None:
            cu_d, idx_d = dec
            ops.gka_chebyshev_gla_decode(
                q[:, :ndt], k[:, :ndt], v[:, :ndt], None, None, None, None,
                h_kk=h_kk_state, h_kv=h_kv_state, cu_seqlens=cu_d, ssm_state_indices=idx_d,
                out=o[:, :ndt], gates=gates.tokens(0, ndt), **common,
                **_norm_args(on, 0, ndt))
        if pre is not None:
            cu_p, idx_p, has_p = pre
            ops.gka_chebyshev_gla_prefill(
                q[:, ndt:], k[:, ndt:], v[:, ndt:], None, None, None, None,
                h_kk_initial=h_kk_state, h_kv_initial=h_kv_state, output_final_state=True,
                cu_seqlens=cu_p, ssm_state_indices=idx_p, has_initial_state=has_p,
                out=o[:, ndt:], gates=gates.tokens(ndt, m), **common, **_norm_args(on, ndt, m))

    def spec(rows, out, on):
        mq, aa, ai, bb = rows
        q, k, v = _qkv(layer, _spec_conv(layer, md, mq, conv_state))
        nsd = md.num_spec_decodes
        ops.gka_chebyshev_gla_decode(
            q, k, v, None, None, None, None, h_kk=h_kk_state, h_kv=h_kv_state,
            cu_seqlens=md.spec_query_start_loc[:nsd + 1],
            ssm_state_indices=md.spec_state_indices_tensor, out=out.unsqueeze(0),
            gates=gates_of(aa, ai, bb), **common, **_norm_args(on, 0, mq.shape[0]))

    rows = (mixed_qkv, a, alpha_in, b if use_beta else None)
    if md.spec_sequence_masks is None:
        rest(rows, core_attn_out[:n], o_norm, query_start_loc_cpu)
    else:
        _by_spec(md, n, rows, core_attn_out, o_norm, spec, rest)


def mamba2_conv_ssm_forward(layer, projected_states: torch.Tensor, output: torch.Tensor,
                            attn_metadata, conv_state: torch.Tensor,
                            ssm_state: torch.Tensor, *, query_start_loc_cpu=None,
                            positions: torch.Tensor | None = None) -> torch.Tensor | None:
    """primed_mamba2_layer.py:615-1021 over hmx ops (see the module docstring).

    ``layer`` carries the reference's attributes (tped_intermediate_size,
    tped_conv_size, dt_pad, num_heads, tp_size, xb_size, ssm_state_size, head_dim,
    n_groups, conv_weights [conv_dim, W], conv1d.bias, activation, A, D, dt_bias,
    B_norm / C_norm (or None), use_pos_embed with rotary_emb, cache_config);
    ``positions`` are the tokens' positions the layer's forward receives (needed
    with use_pos_embed); ``attn_metadata`` is
    the layer's Mamba2AttentionMetadata (num_prefills, num_decode_tokens,
    num_prefill_tokens, state_indices_tensor, has_initial_states_p,
    prep_initial_states, query_start_loc_p); ``conv_state`` is
    ``kv_cache[0].transpose(-1, -2)`` and ``ssm_state`` ``kv_cache[1]``
    (:650-653).  Writes ``output[:num_actual_tokens]`` ([tokens, intermediate],
    decodes first) and updates both pools in place.  ``query_start_loc_cpu``
    (vLLM's host copy of the batch's query_start_loc) lets the prefill scan plan
    without a device-to-host copy.

    With ``cache_config.mamba_cache_mode == "all"`` the metadata also carries
    block_idx_last_computed_token, block_idx_last_scheduled_token,
    block_idx_first_scheduled_token_p, num_computed_tokens_p, chunk_size,
    cu_chunk_seqlen_p, seq_idx_p and last_chunk_indices_p (:728-754, :844-863), the
    state table is [requests, blocks] and ``cache_config.mamba_block_size`` is the
    block size.  With ``attn_metadata`` None (the profile run) nothing is written and
    the x columns repeated over the heads [tokens, H * head_dim] are returned."""
    md = attn_metadata
    cc = getattr(layer, "cache_config", None)
    apc = cc is not None and getattr(cc, "mamba_cache_mode", None) == "all"
    rope = getattr(layer, "use_pos_embed", False)
    if rope and positions is None:
        raise ValueError("use_pos_embed needs the tokens' positions")
    tp = layer.tp_size
    I, CD = layer.tped_intermediate_size, layer.tped_conv_size
    H = layer.num_heads // tp
    P, N = layer.head_dim, layer.ssm_state_size
    xb = layer.xb_size // tp
    HX = xb // N                                         # x and B heads before repeat_kv
    if HX * N != xb or P != N or H % HX != 0:
        raise NotImplementedError(f"hmx Mamba2 core needs head_dim == d_state and xb_size a "
                                  f"multiple of d_state dividing the heads (P={P}, N={N}, "
                                  f"xb={xb}, H={H})")
    hbc = projected_states[:, I:I + CD]                  # :622-631
    dt = projected_states[:, I + CD:I + CD + H]          # dt_pad columns dropped (:633-634)
    if layer.B_norm is not None or rope:                 # :663-671
        hs, B, C = torch.split(hbc, [xb, xb, CD - 2 * xb], dim=-1)
        if layer.B_norm is not None:
            B = layer.B_norm(B.reshape(-1, layer.head_dim)).view(B.shape)
            C = layer.C_norm(C.reshape(-1, layer.head_dim)).view(C.shape)
        if rope:
            C, B = layer.rotary_emb(positions, C, B)
        hbc = torch.cat([hs, B, C], dim=-1)
    if md is None:                                       # profile run (:676-697)
        return hbc[:, :xb].reshape(-1, HX, P).repeat_interleave(H // HX, dim=1).reshape(-1, H * P)
    nd, npf = md.num_decode_tokens, md.num_prefills
    n = nd + md.num_prefill_tokens
    idx = md.state_indices_tensor
    w = layer.conv_weights
    bias = getattr(layer.conv1d, "bias", None)
    act = layer.activation
    x = torch.empty(n, CD, dtype=hbc.dtype, device=hbc.device)
    out = output[:n].view(n, H, P)
    if apc:                                              # (:728-754)
        lc, ls = md.block_idx_last_computed_token, md.block_idx_last_scheduled_token
    if npf > 0 and apc:
        _mamba2_prefill_blocks(layer, md, hbc[nd:n], dt[nd:n], x[nd:], out[nd:], idx[nd:nd + npf],
                               lc[nd:nd + npf], ls[nd:nd + npf], conv_state, ssm_state, cc,
                               (H, HX, P, N, xb))
    elif npf > 0:
        idx_p = idx[nd:nd + npf]
        has_c = md.has_initial_states_p                  # the conv takes the flags as given (:788)
        has = has_c
        if has is None or not md.prep_initial_states:    # the scan starts from zeros (:811-824)
            has = torch.zeros(npf, dtype=torch.bool, device=hbc.device)
        qsl = md.query_start_loc_p
        ops.conv.conv_fwd_rows(hbc[nd:n].t(), w, bias, conv_state, qsl, idx_p, has_c, act,
                               out=x[nd:])
        xp = x[nd:]
        qsl_h = _host_prefill_offsets(nd, query_start_loc_cpu)
        ops.mamba_chunk_scan_combined_varlen(
            xp[:, :xb].view(-1, HX, P), dt[nd:n], layer.A, xp[:, xb:2 * xb].view(-1, HX, N),
            xp[:, 2 * xb:].view(-1, H, N), layer.chunk_size,
            cu_seqlens=qsl if qsl_h is None else qsl_h, out=out[nd:],
            D=layer.D, dt_bias=layer.dt_bias, initial_states=ssm_state, dt_softplus=True,
            dt_limit=(0.0, float("inf")), ssm_state_indices=idx_p, has_initial_state=has)
    if nd > 0:
        idx_d = idx[:nd]
        src = dst = idx_d
        if apc:                                          # (:943-973)
            src = idx_d.gather(1, lc[:nd, None].long()).squeeze(1)
            dst = idx_d.gather(1, ls[:nd, None].long()).squeeze(1)
            ops.causal_conv1d_update(hbc[:nd], conv_state, w, bias, act, conv_state_indices=idx_d,
                                     block_idx_last_scheduled_token=ls[:nd],
                                     initial_state_idx=lc[:nd], out=x[:nd])
        else:
            ops.causal_conv1d_update(hbc[:nd], conv_state, w, bias, act, conv_state_indices=idx_d,
                                     out=x[:nd])
        xd = x[:nd]
        ops.selective_state_update(
            ssm_state, xd[:, :xb].view(nd, HX, P), dt[:nd, :, None].expand(nd, H, P),
            layer.A[:, None, None].expand(H, P, N), xd[:, xb:2 * xb].view(nd, HX, N),
            xd[:, 2 * xb:].view(nd, H, N), layer.D[:, None].expand(H, P), z=None,
            dt_bias=layer.dt_bias[:, None].expand(H, P), dt_softplus=True,
            state_batch_indices=src, dst_state_batch_indices=dst, out=out[:nd])


def _mamba2_prefill_blocks(layer, md, hbc, dt, x, out, idx_p, lc_p, ls_p, conv_state, ssm_state,
                           cc, dims):
    """The prefill of primed_mamba2_layer.py:768-933 with prefix caching: the conv
    with its block arguments (:782-793); the scan from the slot of each sequence's
    last computed block (:811-824), returning the state after every chunk
    (:844-863); the states at the ends of the blocks that end in this step and after
    each sequence's last token copied into the blocks' slots (:864-933)."""
    H, HX, P, N, xb = dims
    npf = idx_p.shape[0]
    bs = int(cc.mamba_block_size)
    chunk = int(getattr(md, "chunk_size", layer.chunk_size))
    fs_p, ncomp = md.block_idx_first_scheduled_token_p, md.num_computed_tokens_p
    ops.conv.conv_fwd_rows(hbc.t(), layer.conv_weights, getattr(layer.conv1d, "bias", None),
                           conv_state, md.query_start_loc_p, idx_p, md.has_initial_states_p,
                           layer.activation, out=x, blocks=(lc_p, fs_p, ls_p, ncomp, bs))
    h0 = None
    has = md.has_initial_states_p
    if has is not None and md.prep_initial_states:
        src = idx_p.gather(1, lc_p[:, None].long()).squeeze(1)
        h0 = torch.where(has[:, None, None, None], ssm_state[src.long()].float(), 0.0)
    states = ops.mamba_chunk_scan_combined_varlen(
        x[:, :xb].view(-1, HX, P), dt, layer.A, x[:, xb:2 * xb].view(-1, HX, N),
        x[:, 2 * xb:].view(-1, H, N), chunk, cu_seqlens=md.query_start_loc_p,
        cu_chunk_seqlens=md.cu_chunk_seqlen_p, last_chunk_indices=md.last_chunk_indices_p,
        seq_idx=md.seq_idx_p, out=out, D=layer.D, dt_bias=layer.dt_bias, initial_states=h0,
        dt_softplus=True, dt_limit=(0.0, float("inf")), return_intermediate_states=True,
        state_dtype=ssm_state.dtype)
    # which chunk's state goes to which slot: the layer's loop (:864-933) on host values
    stride = bs // chunk
    tab = idx_p.tolist()
    fs, ls = [int(v) for v in fs_p.tolist()], [int(v) for v in ls_p.tolist()]
    nc = [int(v) for v in ncomp.tolist()]
    last_chunk = [int(v) for v in md.last_chunk_indices_p.tolist()]
    blk_dst, blk_src, fin_dst, fin_src = [], [], [], []
    for s in range(npf):
        first_chunk = 0 if s == 0 else 1 + last_chunk[s - 1]
        aligned = first_chunk + stride - 1 - (nc[s] % bs) // chunk
        for k in range(ls[s] - fs[s]):
            blk_dst.append(tab[s][fs[s] + k])
            blk_src.append(aligned + k * stride)
        fin_dst.append(tab[s][ls[s]])
        fin_src.append(last_chunk[s])
    for dst, src in ((blk_dst, blk_src), (fin_dst, fin_src)):   # block states, then final ones
        keep = [i for i, d in enumerate(dst) if d >= 0]
        if keep:
            dev = ssm_state.device
            ssm_state.index_copy_(0, torch.tensor([dst[i] for i in keep], device=dev),
                                  states.index_select(0, torch.tensor([src[i] for i in keep],
                                                                      device=dev)))
