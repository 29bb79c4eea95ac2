"""GPU: hmx.serving's GDN and GKA mixer cores on speculative batches
(``spec_sequence_masks``; primed_gdn_layer.py:686-712, :819-836, :923-934 and
primed_gka_layer.py:1017-1040, :1185-1205), all-spec and mixed with non-spec
decodes and a prefill, against a per-sequence composition of the oracles.

A spec sequence carries 1 + SPEC_S tokens against a conv state with SPEC_S rows
of slack.  Its conv reads the window at state rows a-1 .. a+W-3 of slot
spec_state_indices[n, 0] (a = num_accepted_tokens[n]) and leaves the kept rows
followed by its inputs; GDN's recurrence starts from slot [n, a-1] and leaves the
state after its last token in slot [n, 0] (fused_recurrent_gqa.py:95-105,
:135-144); GKA's decode, as the reference's
(chebyshev_iteration_gqa.py: one token per sequence), advances each spec sequence
by its first token only, from and to slot [n, 0] (its other rows are not
written).  The non-spec part is the composition of test_serving_gpu.py.  With the
output norm fused (o_norm), each part takes its rows of the gate.
"""
from types import SimpleNamespace

import pytest
import torch

import hmx
import hmx.serving as srv
from oracle import conv as cref
from oracle import gdn as gref
from oracle import gka as kref
from util import assert_out_close, assert_state_close, half_ulp

import test_serving_gpu as base

pytestmark = pytest.mark.gpu

D, H, HKV, CONV_DIM = base.D, base.H, base.HKV, base.CONV_DIM
SPEC_S = 2                   # draft tokens per spec sequence
T1 = SPEC_S + 1
W = 4
SLOTS = 12


def _meta(mixed, dev):
    """Token order: spec0, dec0, spec1, dec1, prefill(40) (mixed) or three spec
    sequences.  Spec and non-spec sequences use disjoint slots."""
    if mixed:
        layout, nsd, nd, plens = ["s", "d", "s", "d", "p"], 2, 2, [40]
    else:
        layout, nsd, nd, plens = ["s", "s", "s"], 3, 0, []
    spec_tok, non_tok, t, pi = [], [], 0, 0
    for kind in layout:
        L = T1 if kind == "s" else 1 if kind == "d" else plens[pi]
        pi += kind == "p"
        (spec_tok if kind == "s" else non_tok).extend(range(t, t + L))
        t += L
    sidx = torch.tensor([[8, 9, 10], [3, 11, 1], [5, 6, 7]][:nsd], dtype=torch.int32)
    nacc = torch.tensor([1, 3, 2][:nsd], dtype=torch.int32)
    non_lens = [1] * nd + plens
    qsl = torch.tensor([0] + list(torch.tensor(non_lens, dtype=torch.int64).cumsum(0)),
                       dtype=torch.int32) if non_lens else torch.zeros(1, dtype=torch.int32)
    idx = torch.tensor([4, 0, 2][:len(non_lens)], dtype=torch.int32)
    has = torch.ones(len(non_lens), dtype=torch.bool)
    md = SimpleNamespace(
        spec_sequence_masks=torch.ones(nsd, dtype=torch.bool, device=dev), num_spec_decodes=nsd,
        spec_query_start_loc=torch.arange(0, nsd * T1 + 1, T1, dtype=torch.int32, device=dev),
        spec_state_indices_tensor=sidx.to(dev), num_accepted_tokens=nacc.to(dev),
        spec_token_indx=torch.tensor(spec_tok, device=dev),
        non_spec_token_indx=torch.tensor(non_tok, dtype=torch.int64, device=dev),
        num_actual_tokens=t, num_decodes=nd, num_decode_tokens=nd, num_prefills=len(plens),
        non_spec_query_start_loc=qsl.to(dev), non_spec_state_indices_tensor=idx.to(dev),
        has_initial_state=has.to(dev), non_spec_query_start_loc_d=None,
        non_spec_query_start_loc_p=None)
    if nd and plens:
        md.non_spec_query_start_loc_d = qsl[:nd + 1].to(dev)
        md.non_spec_query_start_loc_p = (qsl[nd:] - qsl[nd]).to(dev)
    return md, dict(spec_tok=spec_tok, non_tok=non_tok, sidx=sidx, nacc=nacc, nsd=nsd, nd=nd,
                    non_lens=non_lens, idx=idx, has=has)


def _qkv(xb):
    L = xb.shape[0]
    return (xb[:, :H * D].view(L, H, D), xb[:, H * D:(H + HKV) * D].view(L, HKV, D),
            xb[:, (H + HKV) * D:].view(L, HKV, D))


def _spec_run(kind, mixed, dev, o_norm):
    """One core call on the spec batch; returns (core [n + pad, H, D], states, z, wn)."""
    lay = base._layer(kind, 31)
    md, m = _meta(mixed, dev)
    n = md.num_actual_tokens
    g0 = torch.Generator().manual_seed(77)
    conv_cache = torch.randn(SLOTS, W - 1 + SPEC_S, CONV_DIM, generator=g0).bfloat16()
    s1 = torch.randn(SLOTS, H, D, D, generator=g0) * 0.05
    xk = torch.randn(SLOTS, H, D, 16, generator=g0) * 0.05
    hkk = xk @ xk.transpose(-1, -2)
    mixed_qkv = torch.randn(n + 5, CONV_DIM, generator=g0).bfloat16()
    a, b, alpha_in = (torch.randn(n + 5, H, generator=g0).bfloat16() for _ in range(3))
    z = torch.randn(n + 5, H, D, generator=g0).bfloat16()
    wn = (torch.rand(D, generator=g0) + 0.5).bfloat16()
    on = (wn.to(dev), z.to(dev), 1e-6) if o_norm else None
    lay_d = base._to(lay, dev)
    core = torch.zeros(n + 5, H, D, dtype=torch.bfloat16, device=dev)
    if kind == "gdn":
        ssm = s1.to(dev)
        srv.gdn_forward_core(lay_d, mixed_qkv.to(dev), b.to(dev), a.to(dev), core, md,
                             conv_cache.to(dev).transpose(1, 2), ssm, o_norm=on)
        states = [ssm]
    else:
        hkv_d, hkk_d = s1.to(dev), hkk.to(dev)
        srv.gka_forward_core(lay_d, mixed_qkv.to(dev), a.to(dev), alpha_in.to(dev), b.to(dev),
                             core, md, conv_cache.to(dev).transpose(1, 2), hkk_d, hkv_d,
                             o_norm=on)
        states = [hkv_d, hkk_d]
    torch.cuda.synchronize()
    return core, [t.cpu() for t in states], z, wn, n


@pytest.mark.parametrize("kind", ["gdn", "gka"])
@pytest.mark.parametrize("mixed", [False, True])
def test_forward_core_spec_fused_o_norm(dev, kind, mixed):
    """o_norm on a speculative batch: the spec and non-spec parts each take their
    rows of the gate z; the result equals the layer's norm of the plain core's
    output (within the rounding of o before the norm), and the states are the same."""
    plain, st_p, z, wn, n = _spec_run(kind, mixed, dev, False)
    fused, st_f, _, _, _ = _spec_run(kind, mixed, dev, True)
    rows = list(range(n))
    if kind == "gka":   # only a spec sequence's first token has an output (as the reference's)
        _, m = _meta(mixed, dev)
        drafts = {t for j in range(m["nsd"]) for t in m["spec_tok"][j * T1 + 1:(j + 1) * T1]}
        rows = [t for t in rows if t not in drafts]
    sel = torch.tensor(rows, device=dev)
    expect = hmx.rms_norm_gated(plain[sel], z.to(dev)[sel], wn.to(dev), 1e-6).cpu()
    got = fused[sel].cpu()
    assert ((got.double() - expect.double()).abs()
            <= 2 * half_ulp(expect.double(), torch.bfloat16) + 1e-30).all()
    assert (got == expect).double().mean().item() >= 0.98
    assert torch.equal(fused[n:].cpu(), torch.zeros_like(fused[n:].cpu()))
    for x, y in zip(st_p, st_f):
        assert torch.equal(x, y)


@pytest.mark.parametrize("kind", ["gdn", "gka"])
@pytest.mark.parametrize("mixed", [False, True])
def test_forward_core_spec_batch(dev, kind, mixed):
    lay = base._layer(kind, 31)
    md, m = _meta(mixed, dev)
    n = md.num_actual_tokens
    g0 = torch.Generator().manual_seed(77)
    conv_cache = torch.randn(SLOTS, W - 1 + SPEC_S, CONV_DIM, generator=g0).bfloat16()
    s1 = torch.randn(SLOTS, H, D, D, generator=g0) * 0.05
    xk = torch.randn(SLOTS, H, D, 16, generator=g0) * 0.05
    hkk = xk @ xk.transpose(-1, -2)
    pad = 5
    mixed_qkv = torch.randn(n + pad, CONV_DIM, generator=g0).bfloat16()
    a = torch.randn(n + pad, H, generator=g0).bfloat16()
    b = torch.randn(n + pad, H, generator=g0).bfloat16()
    alpha_in = torch.randn(n + pad, H, generator=g0).bfloat16()
    lay_d = base._to(lay, dev)
    cc_d = conv_cache.to(dev)
    core = torch.zeros(n + pad, H, D, dtype=torch.bfloat16, device=dev)
    if kind == "gdn":
        ssm = s1.to(dev)
        srv.gdn_forward_core(lay_d, mixed_qkv.to(dev), b.to(dev), a.to(dev), core, md,
                             cc_d.transpose(1, 2), ssm)
        got_states, states = [ssm.cpu()], [s1]
    else:
        hkv_d, hkk_d = s1.to(dev), hkk.to(dev)
        srv.gka_forward_core(lay_d, mixed_qkv.to(dev), a.to(dev), alpha_in.to(dev), b.to(dev),
                             core, md, cc_d.transpose(1, 2), hkk_d, hkv_d)
        got_states, states = [hkv_d.cpu(), hkk_d.cpu()], [s1, hkk]
    torch.cuda.synchronize()
    core = core.cpu()
    assert torch.equal(core[n:], torch.zeros_like(core[n:]))

    # ---- spec sequences --------------------------------------------------------
    w = lay.conv1d.weight.cpu().view(CONV_DIM, W)
    conv_exp = conv_cache.clone()
    st_exp = [s.clone().double() for s in states]
    touched = set()
    checked_rows = []
    for j in range(m["nsd"]):
        rows = m["spec_tok"][j * T1:(j + 1) * T1]
        sl = torch.tensor(rows)
        slot0, acc = int(m["sidx"][j, 0]), int(m["nacc"][j])
        win = conv_cache[slot0, acc - 1:acc + W - 2]
        o_c, _ = cref.conv_sequence(mixed_qkv[sl], win, w, None, "silu")
        conv_exp[slot0] = torch.cat([conv_cache[slot0, acc:acc + SPEC_S + W - 1 - T1],
                                     mixed_qkv[sl]])
        q, k, v = _qkv(o_c.bfloat16())
        if kind == "gdn":
            g, beta = gref.gdn_gating(lay.A.cpu(), a[sl], b[sl], lay.dt_bias.cpu())
            g, beta = g.to(a.dtype), beta.to(a.dtype)
            S0 = states[0][int(m["sidx"][j, acc - 1])]
            o, S = gref.recurrent_seq(q, k, v, g[0], beta[0], D ** -0.5, S0, use_qk_l2norm=True)
            assert_out_close(core[sl], o, what=f"spec {j}")
            st_exp[0][slot0] = S
            touched.add(slot0)
            checked_rows += rows
        else:
            g, alpha, beta = kref.gka_gating(lay.A.cpu(), a[sl], alpha_in[sl], b[sl],
                                             lay.dt_bias.cpu())
            g, alpha, beta = g.to(a.dtype), alpha.to(a.dtype), beta.to(a.dtype)
            alpha = alpha + 0.5
            o, hk, hv = kref.gka_seq(q[:1], k[:1], v[:1], alpha[0, :1], g[0, :1], g[0, :1],
                                     beta[0, :1], lay.gla_scale, lay.ridge_strength,
                                     lay.num_iter, states[1][slot0], states[0][slot0])
            assert_out_close(core[rows[0]:rows[0] + 1], o, what=f"spec {j} first token")
            st_exp[0][slot0], st_exp[1][slot0] = hv, hk
            touched.add(slot0)
            checked_rows.append(rows[0])

    # ---- the non-spec part: base composition over its rows ---------------------
    if m["non_tok"]:
        nt = torch.tensor(m["non_tok"])
        gates = (a[nt], b[nt]) if kind == "gdn" else (a[nt], alpha_in[nt], b[nt])
        o_r, conv_r, st_r = base._expected(kind, lay, m["non_lens"], m["idx"], m["has"], m["nd"],
                                           mixed_qkv[nt], gates, conv_cache, states)
        assert_out_close(core[nt], o_r, what="non-spec rows")
        for s in m["idx"].tolist():
            conv_exp[s] = conv_r[s]
            for e, r in zip(st_exp, st_r):
                e[s] = r[s]
            touched.add(s)

    assert torch.equal(cc_d.cpu(), conv_exp)
    for got, exp, orig in zip(got_states, st_exp, states):
        for s in range(SLOTS):
            if s in touched:
                assert_state_close(got[s], exp[s], what=f"slot {s}")
            else:
                assert torch.equal(got[s], orig[s]), f"slot {s} changed"
