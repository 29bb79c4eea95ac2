"""Pins the GDN oracle (oracle/gdn.py) without trusting its own formulas.

The reference ships no golden vectors for these ops, so each oracle function
is checked against an independent formulation or a closed form chosen so a
plausible mistake (dropped decay, wrong sign, transposed state, wrong GQA
mapping, off-by-one chunk boundary) fails:
  - recurrence vs the transition-matrix form S_t = e^g (I - b k k^T) S + b k v^T
  - beta=0 pure decay, exact memorisation with orthonormal keys, overwrite
  - chunked WY form == recurrence (chunk 16/32/64, ragged tails, h0 != 0)
  - (I+A)^-1: solve_triangular == the reference's row recursion == linalg.inv
  - varlen == per-sequence; GQA == expanded heads; gating == F.softplus/sigmoid
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn as ref

D64 = torch.float64


def _rand(T, H, HKV, K, V, seed, S0=True):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(T, H, K, generator=g, dtype=D64)
    k = torch.randn(T, HKV, K, generator=g, dtype=D64)
    v = torch.randn(T, HKV, V, generator=g, dtype=D64)
    gg = F.logsigmoid(torch.randn(T, H, generator=g, dtype=D64))
    beta = torch.sigmoid(torch.randn(T, H, generator=g, dtype=D64))
    s0 = torch.randn(H, K, V, generator=g, dtype=D64) * 0.1 if S0 else None
    return q, k, v, gg, beta, s0


def test_recurrent_matches_transition_matrix_form():
    T, H, K, V = 9, 3, 5, 4
    q, k, v, g, beta, S0 = _rand(T, H, H, K, V, 0)
    o, S = ref.recurrent_seq(q, k, v, g, beta, 0.7, S0, use_qk_l2norm=True)
    qn = q / torch.sqrt((q * q).sum(-1, keepdim=True) + 1e-6)
    kn = k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    for h in range(H):
        Sh = S0[h].clone()
        for t in range(T):
            kk = kn[t, h][:, None]
            A = torch.exp(g[t, h]) * (torch.eye(K, dtype=D64) - beta[t, h] * kk @ kk.T)
            Sh = A @ Sh + beta[t, h] * kk @ v[t, h][None, :]
            assert torch.allclose(o[t, h], Sh.T @ (0.7 * qn[t, h]), atol=1e-12)
        assert torch.allclose(S[h], Sh, atol=1e-12)


def test_beta_zero_is_pure_decay():
    T, H, K, V = 6, 2, 4, 3
    q, k, v, g, beta, S0 = _rand(T, H, H, K, V, 1)
    o, S = ref.recurrent_seq(q, k, v, g, torch.zeros_like(beta), 1.0, S0, use_qk_l2norm=False)
    G = g.cumsum(0)
    assert torch.allclose(S, torch.exp(G[-1])[:, None, None] * S0, atol=1e-12)
    want = torch.einsum("th,hkv,thk->thv", torch.exp(G), S0, q)
    assert torch.allclose(o, want, atol=1e-12)


def test_orthonormal_keys_memorise_and_overwrite():
    K = V = 8
    T = 5
    Qm, _ = torch.linalg.qr(torch.randn(K, K, generator=torch.Generator().manual_seed(2), dtype=D64))
    keys = Qm[:T]                                      # orthonormal rows
    vals = torch.randn(T, V, generator=torch.Generator().manual_seed(3), dtype=D64)
    k = keys[:, None, :]
    v = vals[:, None, :]
    g = torch.zeros(T, 1, dtype=D64)
    beta = torch.ones(T, 1, dtype=D64)
    q = keys[[0, 0, 1, 3, 2]][:, None, :]              # read back earlier keys
    o, S = ref.recurrent_seq(q, k, v, g, beta, 1.0, None, use_qk_l2norm=False)
    assert torch.allclose(S[0], keys.T @ vals, atol=1e-12)
    for t, j in enumerate([0, 0, 1, 3, 2]):
        if j <= t:
            assert torch.allclose(o[t, 0], vals[j], atol=1e-12)
    # writing the same key again replaces its value (delta rule, beta = 1)
    k2 = torch.cat([k, keys[1][None, None, :]])
    v2 = torch.cat([v, torch.full((1, 1, V), 5.0, dtype=D64)])
    o2, S2 = ref.recurrent_seq(torch.cat([q, keys[1][None, None, :]]), k2, v2,
                               torch.zeros(T + 1, 1, dtype=D64), torch.ones(T + 1, 1, dtype=D64),
                               1.0, None, use_qk_l2norm=False)
    assert torch.allclose(o2[-1, 0], torch.full((V,), 5.0, dtype=D64), atol=1e-12)


@pytest.mark.parametrize("T,chunk", [(64, 64), (100, 64), (37, 16), (96, 32), (1, 64), (130, 64)])
def test_chunked_equals_recurrent(T, chunk):
    H, HKV, K, V = 4, 2, 16, 12
    q, k, v, g, beta, S0 = _rand(T, H, HKV, K, V, T + chunk)
    o1, S1 = ref.recurrent_seq(q, k, v, g, beta, K ** -0.5, S0)
    o2, S2 = ref.chunked_seq(q, k, v, g, beta, K ** -0.5, S0, chunk=chunk)
    assert torch.allclose(o1, o2, atol=1e-10, rtol=1e-9)
    assert torch.allclose(S1, S2, atol=1e-10, rtol=1e-9)


def test_chunk_states_are_recurrent_states_at_boundaries():
    T, H, K, V, C = 96, 2, 8, 8, 32
    q, k, v, g, beta, S0 = _rand(T, H, H, K, V, 4)
    _, _, states = ref.recurrent_seq(q, k, v, g, beta, 1.0, S0, return_states=True)
    _, _, cstates = ref.chunked_seq(q, k, v, g, beta, 1.0, S0, chunk=C, return_chunk_states=True)
    assert torch.allclose(cstates[0], S0)
    for c in range(1, T // C):
        assert torch.allclose(cstates[c], states[c * C - 1], atol=1e-10)


def test_wy_inverse_three_ways():
    C = 24
    g = torch.Generator().manual_seed(5)
    A = torch.tril(torch.randn(2, C, C, generator=g, dtype=D64) * 0.2, -1)
    eye = torch.eye(C, dtype=D64)
    t_rec = ref.wy_inverse_row_recursion(A)
    t_inv = torch.linalg.inv(eye + A)
    t_tri = torch.linalg.solve_triangular(eye + A, eye.expand_as(A), upper=False, unitriangular=True)
    assert torch.allclose(t_rec, t_inv, atol=1e-10)
    assert torch.allclose(t_tri, t_inv, atol=1e-10)


def test_gqa_equals_expanded_heads():
    T, H, HKV, K, V = 20, 6, 2, 8, 8
    q, k, v, g, beta, S0 = _rand(T, H, HKV, K, V, 6)
    o1, S1 = ref.recurrent_seq(q, k, v, g, beta, 0.5, S0)
    ke, ve = k.repeat_interleave(3, 1), v.repeat_interleave(3, 1)
    o2, S2 = ref.recurrent_seq(q, ke, ve, g, beta, 0.5, S0)
    assert torch.equal(o1, o2) and torch.equal(S1, S2)
    # head h of q reads kv head h // 3: permuting kv heads must change the result
    o3, _ = ref.recurrent_seq(q, k.flip(1), v.flip(1), g, beta, 0.5, S0)
    assert not torch.allclose(o1, o3)


def test_varlen_equals_per_sequence_and_forms_agree():
    H, K, V = 2, 8, 8
    lens = [5, 0, 70, 33]
    T = sum(lens)
    q, k, v, g, beta, _ = _rand(T, H, H, K, V, 7, S0=False)
    h0 = torch.randn(len(lens), H, K, V, generator=torch.Generator().manual_seed(8), dtype=D64)
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)))
    args = (q[None], k[None], v[None], g[None], beta[None])
    o_c, f_c = ref.chunk_gated_delta_rule_gqa(*args, initial_state=h0, output_final_state=True,
                                              cu_seqlens=cu, use_qk_l2norm_in_kernel=True,
                                              chunk=16)
    o_r, f_r = ref.chunk_gated_delta_rule_gqa(*args, initial_state=h0, output_final_state=True,
                                              cu_seqlens=cu, use_qk_l2norm_in_kernel=True,
                                              form="recurrent")
    assert torch.allclose(o_c, o_r, atol=1e-10) and torch.allclose(f_c, f_r, atol=1e-10)
    assert torch.equal(f_r[1], h0[1])  # zero-length sequence keeps its state
    for n, (a, b) in enumerate(zip(cu[:-1].tolist(), cu[1:].tolist())):
        if b > a:
            o_n, s_n = ref.recurrent_seq(q[a:b], k[a:b], v[a:b], g[a:b], beta[a:b], K ** -0.5, h0[n])
            assert torch.allclose(o_r[0, a:b], o_n) and torch.allclose(f_r[n], s_n)


def test_decode_pool_routing():
    """Slot routing of the decode op: read column nacc-1, write column 0, skip empty."""
    H, K, V = 1, 4, 4
    lens = [2, 0, 1]
    cu = torch.tensor([0, 2, 2, 3])
    q, k, v, g, beta, _ = _rand(3, H, H, K, V, 9, S0=False)
    pool = torch.randn(8, H, K, V, generator=torch.Generator().manual_seed(10), dtype=D64)
    idx = torch.tensor([[5, 1], [6, 7], [2, 3]])
    nacc = torch.tensor([2, 1, 1])
    o, new = ref.fused_recurrent_gated_delta_rule_gqa(
        q[None], k[None], v[None], g[None], beta[None], initial_state=pool, cu_seqlens=cu,
        ssm_state_indices=idx, num_accepted_tokens=nacc, use_qk_l2norm_in_kernel=True)
    _, s0 = ref.recurrent_seq(q[0:2], k[0:2], v[0:2], g[0:2], beta[0:2], K ** -0.5, pool[1])
    _, s2 = ref.recurrent_seq(q[2:3], k[2:3], v[2:3], g[2:3], beta[2:3], K ** -0.5, pool[2])
    assert torch.allclose(new[5], s0) and torch.allclose(new[2], s2)
    for untouched in (0, 1, 3, 4, 6, 7):
        assert torch.equal(new[untouched], pool[untouched])


def test_gating_matches_library_softplus():
    g0 = torch.Generator().manual_seed(11)
    a = torch.randn(50, 4, generator=g0, dtype=D64) * 15
    b = torch.randn(50, 4, generator=g0, dtype=D64)
    A_log = torch.randn(4, generator=g0, dtype=D64)
    dt_bias = torch.randn(4, generator=g0, dtype=D64)
    for sp_beta, thr in ((1.0, 20.0), (2.0, 10.0)):
        g, be = ref.gdn_gating(A_log, a, b, dt_bias, sp_beta, thr)
        want = -A_log.exp() * F.softplus(a + dt_bias, beta=sp_beta, threshold=thr)
        assert torch.allclose(g[0], want, rtol=1e-12, atol=1e-12)
        assert torch.allclose(be[0], torch.sigmoid(b))


def test_l2norm_norm_invariant():
    x = torch.randn(7, 3, 16, generator=torch.Generator().manual_seed(12), dtype=D64)
    n = ref.l2norm(x).norm(dim=-1)
    xn = x.norm(dim=-1)
    assert torch.allclose(n, xn / torch.sqrt(xn ** 2 + 1e-6))
    assert torch.allclose(ref.l2norm(x, eps=0.0), F.normalize(x, dim=-1))
