"""Gated delta rule (GDN) CPU oracle — test infrastructure only (see package doc).

Reference files (paths relative to the reference repository root):
  M  = training/src/hmf/model/hybrid_zoo/models/qwen3_5_moe_hmf/modeling_qwen3_5_moe_hmf.py
  FR = vllm-inference/src/primed_vllm/gdn/ops/fused_recurrent_gqa.py
  CG = vllm-inference/src/primed_vllm/gdn/ops/chunk_gqa.py
  GT = vllm-inference/src/primed_vllm/gdn/ops/fused_gdn_gating.py

Layouts follow the reference ops: tokens-major ``[B, T, H, D]`` tensors, GQA
key/value heads ``HKV`` with query head ``h`` reading kv head ``h // (H/HKV)``
(FR:54), states ``[H, K, V]`` (k-major, v contiguous).

All arithmetic runs in ``dtype`` (float64 by default) on upcast copies of the
inputs, so bf16 inputs are used at their exact values.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

DEFAULT = torch.float64


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x / sqrt(sum(x^2) + eps) over the last dim (M:324-327, FR:116-118)."""
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)


def gdn_gating(A_log, a, b, dt_bias, softplus_beta: float = 1.0,
               threshold: float = 20.0, dtype=DEFAULT):
    """g = -exp(A_log) * softplus(a + dt_bias); beta = sigmoid(b) (GT:66-76).

    softplus(x) = log(1 + exp(beta*x)) / beta when beta*x <= threshold, else x.
    Returns (g, beta) shaped [1, T, H] in ``dtype``.
    """
    x = a.to(dtype) + dt_bias.to(dtype)
    bx = softplus_beta * x
    sp = torch.where(bx <= threshold, torch.log1p(torch.exp(bx)) / softplus_beta, x)
    g = -torch.exp(A_log.to(dtype)) * sp
    beta = torch.sigmoid(b.to(dtype))
    return g.unsqueeze(0), beta.unsqueeze(0)


def _expand_kv(x: torch.Tensor, H: int) -> torch.Tensor:
    """[T, HKV, D] -> [T, H, D] with query head h reading kv head h // (H/HKV)."""
    HKV = x.shape[1]
    return x.repeat_interleave(H // HKV, dim=1)


def recurrent_seq(q, k, v, g, beta, scale, S0=None, use_qk_l2norm=True,
                  dtype=DEFAULT, return_states=False):
    """Per-token gated delta rule over ONE sequence (M:410-449, FR:111-154).

    q [T,H,K]; k [T,HKV,K]; v [T,HKV,V]; g [T,H]; beta [T,H] or [T,H,V];
    S0 [H,K,V] or None.  Per token t and head h (FR:116-133):
        q,k <- l2norm(q), l2norm(k);  q <- q*scale;  S <- exp(g_t) S
        u <- beta_t (v_t - S^T k_t);  S <- S + k_t u^T;  o_t <- S^T q_t
    Returns o [T,H,V] and S_T [H,K,V] (and all S_t if ``return_states``).
    """
    T, H, K = q.shape
    V = v.shape[-1]
    q = q.to(dtype)
    k = _expand_kv(k.to(dtype), H)
    v = _expand_kv(v.to(dtype), H)
    g = g.to(dtype)
    beta = beta.to(dtype)
    if use_qk_l2norm:
        q, k = l2norm(q), l2norm(k)
    q = q * scale
    S = torch.zeros(H, K, V, dtype=dtype) if S0 is None else S0.to(dtype).clone()
    o = torch.zeros(T, H, V, dtype=dtype)
    states = []
    for t in range(T):
        S = S * torch.exp(g[t])[:, None, None]
        kv = torch.einsum("hkv,hk->hv", S, k[t])
        bt = beta[t] if beta.dim() == 3 else beta[t][:, None]
        u = (v[t] - kv) * bt
        S = S + k[t][:, :, None] * u[:, None, :]
        o[t] = torch.einsum("hkv,hk->hv", S, q[t])
        if return_states:
            states.append(S.clone())
    if return_states:
        return o, S, torch.stack(states) if states else torch.zeros(0, H, K, V, dtype=dtype)
    return o, S


def wy_inverse_row_recursion(A: torch.Tensor) -> torch.Tensor:
    """(I + A)^-1 for strictly-lower A by the reference's row recursion (M:373-378).

    The reference builds attn = -A (masked), then for i = 1..C-1:
    attn[i,:i] += sum_j attn[i,j] * attn[j,:i], and finally adds I.
    """
    C = A.shape[-1]
    attn = -A.clone()
    for i in range(1, C):
        row = attn[..., i, :i].clone()
        sub = attn[..., :i, :i].clone()
        attn[..., i, :i] = row + (row.unsqueeze(-1) * sub).sum(-2)
    return attn + torch.eye(C, dtype=A.dtype)


def chunked_seq(q, k, v, g, beta, scale, S0=None, use_qk_l2norm=True,
                chunk: int = 64, dtype=DEFAULT, return_chunk_states=False):
    """Chunked (WY / UT-transform) gated delta rule over ONE sequence.

    Follows M:330-407 and the op chain of CG:58-81.  Per chunk of C tokens with
    G = in-chunk cumsum of g (the padded tail chunk uses g=beta=k=v=0):
        A_ij = beta_i (k_i . k_j) exp(G_i - G_j)  (j < i);   T = (I + A)^-1
        U = T (beta * V);  W = T (beta exp(G) * K)
        V_new = U - W S_c
        O = scale * [exp(G) * (Q S_c) + tril(Q K^T * exp(G_i - G_j)) V_new]
        S_{c+1} = exp(G_last) S_c + (K * exp(G_last - G))^T V_new
    Same I/O as ``recurrent_seq``; beta must be [T,H].
    """
    T, H, K = q.shape
    V = v.shape[-1]
    q = q.to(dtype)
    k = _expand_kv(k.to(dtype), H)
    v = _expand_kv(v.to(dtype), H)
    g = g.to(dtype)
    beta = beta.to(dtype)
    if use_qk_l2norm:
        q, k = l2norm(q), l2norm(k)
    q = q * scale
    pad = (-T) % chunk
    if pad:
        q = F.pad(q, (0, 0, 0, 0, 0, pad))
        k = F.pad(k, (0, 0, 0, 0, 0, pad))
        v = F.pad(v, (0, 0, 0, 0, 0, pad))
        g = F.pad(g, (0, 0, 0, pad))
        beta = F.pad(beta, (0, 0, 0, pad))
    NT = (T + pad) // chunk
    # [NT, H, C, D]
    qc = q.view(NT, chunk, H, K).transpose(1, 2)
    kc = k.view(NT, chunk, H, K).transpose(1, 2)
    vc = v.view(NT, chunk, H, V).transpose(1, 2)
    gc = g.view(NT, chunk, H).transpose(1, 2)
    bc = beta.view(NT, chunk, H).transpose(1, 2)
    G = gc.cumsum(-1)
    lower = torch.tril(torch.ones(chunk, chunk, dtype=torch.bool), -1)
    lower_eq = torch.tril(torch.ones(chunk, chunk, dtype=torch.bool), 0)
    decay = torch.exp((G[..., :, None] - G[..., None, :]).masked_fill(~lower_eq, 0.0))
    A = (bc[..., :, None] * (kc @ kc.transpose(-1, -2)) * decay).masked_fill(~lower, 0.0)
    eye = torch.eye(chunk, dtype=dtype)
    Tinv = torch.linalg.solve_triangular(eye + A, eye.expand_as(A), upper=False,
                                         unitriangular=True)
    U = Tinv @ (bc[..., None] * vc)
    W = Tinv @ ((bc * torch.exp(G))[..., None] * kc)
    P = ((qc @ kc.transpose(-1, -2)) * decay).masked_fill(~lower_eq, 0.0)
    S = torch.zeros(H, K, V, dtype=dtype) if S0 is None else S0.to(dtype).clone()
    o = torch.empty(NT, H, chunk, V, dtype=dtype)
    chunk_states = []
    for c in range(NT):
        if return_chunk_states:
            chunk_states.append(S.clone())
        v_new = U[c] - W[c] @ S
        o[c] = torch.exp(G[c])[..., None] * (qc[c] @ S) + P[c] @ v_new
        g_last = G[c][:, -1]
        kd = kc[c] * torch.exp(g_last[:, None] - G[c])[..., None]
        S = torch.exp(g_last)[:, None, None] * S + kd.transpose(-1, -2) @ v_new
    o = o.transpose(1, 2).reshape(NT * chunk, H, V)[:T]
    if return_chunk_states:
        return o, S, torch.stack(chunk_states)
    return o, S


def _seq_bounds(B, T, cu_seqlens):
    if cu_seqlens is None:
        return [(n, n * T, n * T + T) for n in range(B)]
    cs = [int(x) for x in cu_seqlens.tolist()]
    return [(n, cs[n], cs[n + 1]) for n in range(len(cs) - 1)]


def chunk_gated_delta_rule_gqa(q, k, v, g, beta, scale=None, initial_state=None,
                               output_final_state=False, cu_seqlens=None,
                               use_qk_l2norm_in_kernel=False, chunk=64,
                               dtype=DEFAULT, form="chunked"):
    """The prefill op's semantics (CG:15-83) over B sequences or cu_seqlens.

    q [B,T,H,K]; k,v [B,T,HKV,*]; g, beta [B,T,H]; initial_state [N,H,K,V].
    Returns (o [B,T,H,V] in ``dtype``, final [N,H,K,V] or None).
    ``form`` picks the chunked WY restatement or the per-token recurrence.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    if scale is None:
        scale = K ** -0.5
    o = torch.zeros(B, T, H, V, dtype=dtype)
    seqs = _seq_bounds(B, T, cu_seqlens)
    finals = torch.zeros(len(seqs), H, K, V, dtype=dtype)
    qf, kf, vf = q.reshape(B * T, H, K), k.reshape(B * T, -1, K), v.reshape(B * T, -1, V)
    gf, bf = g.reshape(B * T, H), beta.reshape(B * T, H)
    of = o.view(B * T, H, V)
    for n, bos, eos in seqs:
        S0 = None if initial_state is None else initial_state[n]
        if eos == bos:
            finals[n] = 0 if S0 is None else S0.to(dtype)
            continue
        fn = chunked_seq if form == "chunked" else recurrent_seq
        kw = dict(chunk=chunk) if form == "chunked" else {}
        on, Sn = fn(qf[bos:eos], kf[bos:eos], vf[bos:eos], gf[bos:eos], bf[bos:eos],
                    scale, S0, use_qk_l2norm_in_kernel, dtype=dtype, **kw)
        of[bos:eos] = on
        finals[n] = Sn
    return o, (finals if output_final_state else None)


def fused_recurrent_gated_delta_rule_gqa(q, k, v, g, beta=None, scale=None,
                                         initial_state=None, inplace_final_state=True,
                                         cu_seqlens=None, ssm_state_indices=None,
                                         num_accepted_tokens=None,
                                         use_qk_l2norm_in_kernel=False, dtype=DEFAULT):
    """The decode op's semantics (FR:227-277, kernel FR:25-154), out of place.

    Returns (o [B,T,H,V] in ``dtype``, final) where ``final`` is an updated
    COPY of the state pool when ``inplace_final_state`` (slot
    ``ssm_state_indices[n, 0]`` receives sequence n's last state, FR:135-144), else
    a new [B,T,H,K,V] tensor whose flat row ``bos`` (over B*T; the sequence's first
    token) holds sequence n's final state (FR:137-139: the store pointer is not
    advanced without ``inplace_final_state``).  The initial state of sequence n is pool row
    ``ssm_state_indices[n, num_accepted_tokens[n]-1]`` (column 0 without
    ``num_accepted_tokens``, FR:95-105), or row ``bos`` of ``initial_state``
    without indices (FR:107).  Zero-length sequences are skipped (FR:67-68).
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    if scale is None:
        scale = K ** -0.5
    if beta is None:
        beta = torch.ones_like(g)
    o = torch.zeros(B, T, H, V, dtype=dtype)
    if inplace_final_state:
        final = initial_state.to(dtype).clone()
    else:
        final = torch.zeros(B, T, H, K, V, dtype=dtype)
    idx = None
    if ssm_state_indices is not None:
        idx = ssm_state_indices if ssm_state_indices.dim() == 2 else ssm_state_indices[:, None]
    qf, kf, vf = q.reshape(B * T, H, K), k.reshape(B * T, -1, K), v.reshape(B * T, -1, V)
    gf = g.reshape(B * T, H)
    bf = beta.reshape(B * T, H, -1) if beta.dim() == 4 else beta.reshape(B * T, H)
    of = o.view(B * T, H, V)
    ff = final.view(-1, H, K, V)
    for n, bos, eos in _seq_bounds(B, T, cu_seqlens):
        if eos == bos:
            continue
        S0 = None
        if initial_state is not None:
            if idx is not None:
                col = 0 if num_accepted_tokens is None else int(num_accepted_tokens[n]) - 1
                S0 = initial_state[int(idx[n, col])]
            else:
                S0 = initial_state.reshape(-1, H, K, V)[bos]
        on, Sn = recurrent_seq(qf[bos:eos], kf[bos:eos], vf[bos:eos], gf[bos:eos],
                               bf[bos:eos], scale, S0, use_qk_l2norm_in_kernel, dtype=dtype)
        of[bos:eos] = on
        if inplace_final_state:
            ff[int(idx[n, 0])] = Sn
        else:
            ff[bos] = Sn
    return o, final
