"""GPU: hmx.serving's GDN and GKA mixer cores (the vLLM layers' ``_forward_core``,
primed_gdn_layer.py:635-936, primed_gka_layer.py:962-1338) on mixed, prefill-only
and decode-only batches, against a per-sequence composition of the oracles:
the conv oracle (state from the conv cache slot, or zeros for a prefill without
an initial state), the gating oracle rounded to the gate input dtype (the
reference gatings return a.dtype, fused_gdn_gating.py:112-113,
primed_gka_layer.py:332-338), then the recurrence oracle from the recurrent pool
slot.  The layer and its attention metadata are stand-ins with
the reference's attribute names (vLLM is not installed here).

Checks: core_attn_out rows within the output tolerance (rows past
num_actual_tokens untouched), recurrent pool slots within the state tolerance
(other slots untouched), conv cache bit for bit (it holds raw inputs), and the
fused output norm within 2 half-ulps of the unfused core followed by
hmx.rms_norm_gated.
"""
import copy
from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F

import hmx
import hmx.serving as srv
from oracle import conv as cref
from oracle import gdn as gref
from oracle import gka as kref
from util import assert_out_close, assert_state_close, half_ulp

pytestmark = pytest.mark.gpu

D = 128
H, HKV = 4, 2
CONV_DIM = (H + 2 * HKV) * D
SLOTS = 8


class _LowRank(torch.nn.Module):
    """LinearLowRank's forward without activation (primed_gka_layer.py:59-106):
    x -> linearA (rank) -> linearB, both bias-free, in the weights' dtype."""

    def __init__(self, fin, fout, rank, g0):
        super().__init__()
        self.wa = torch.nn.Parameter((torch.randn(rank, fin, generator=g0) * fin ** -0.5)
                                     .bfloat16(), requires_grad=False)
        self.wb = torch.nn.Parameter((torch.randn(fout, rank, generator=g0) * rank ** -0.5 * 0.3)
                                     .bfloat16(), requires_grad=False)

    def forward(self, x):
        return F.linear(F.linear(x, self.wa), self.wb)


def _layer(kind, seed, low_rank=None, **extra):
    g0 = torch.Generator().manual_seed(seed)
    w = (torch.randn(CONV_DIM, 1, 4, generator=g0) * 0.4).bfloat16()
    lay = SimpleNamespace(
        conv1d=SimpleNamespace(weight=w), activation="silu",
        A=torch.log(torch.rand(H, generator=g0) * 4 + 1), dt_bias=torch.randn(H, generator=g0),
        key_dim=H * D, kv_k_dim=HKV * D, kv_v_dim=HKV * D, num_heads=H, num_kv_heads=HKV,
        head_k_dim=D, head_v_dim=D, tp_size=1, proj_k=None)
    if kind == "gdn":
        lay.allow_neg_eigval = False
    else:
        lay.use_forgetting_gate, lay.use_forgetting_gate_kk, lay.use_beta_gate = True, True, True
        lay.num_iter, lay.ridge_strength, lay.gla_scale, lay._alpha_idx = 8, 0.02, D ** -0.5, None
    if low_rank is not None:     # kv_proj_rank 32; "learnable": kv_learnable_residual
        lay.proj_k = _LowRank(HKV * D, H * D, 32, g0)
        lay.proj_v = _LowRank(HKV * D, H * D, 32, g0)
        lay.k_rep = lay.v_rep = None
        if low_rank == "learnable":
            rep = torch.arange(H)[:, None] // (H // HKV) == torch.arange(HKV)[None]
            lay.k_rep = (rep + 0.3 * torch.randn(H, HKV, generator=g0)).bfloat16()
            lay.v_rep = (rep + 0.3 * torch.randn(H, HKV, generator=g0)).bfloat16()
    lay.__dict__.update(extra)
    return lay


def _to(lay, dev):
    lay.conv1d.weight = lay.conv1d.weight.to(dev)
    lay.A, lay.dt_bias = lay.A.to(dev), lay.dt_bias.to(dev)
    if lay.proj_k is not None:
        lay.proj_k, lay.proj_v = lay.proj_k.to(dev), lay.proj_v.to(dev)
        if lay.k_rep is not None:
            lay.k_rep, lay.v_rep = lay.k_rep.to(dev), lay.v_rep.to(dev)
    return lay


def _low_rank_ref(proj, rep, kv):
    """The layers' k / v upsampling at tp 1 (primed_gdn_layer.py:511-545), on the
    CPU in bf16: proj(kv) + kv repeat_interleaved over the head groups, or + the
    learnable mix einsum("kh,lhd->lkd", rep, kv)."""
    L = kv.shape[0]
    y = copy.deepcopy(proj).cpu()(kv.reshape(L, HKV * D)).view(L, H, D)
    if rep is None:
        res = kv.repeat_interleave(H // HKV, dim=1)
    else:
        res = torch.einsum("kh,lhd->lkd", rep.cpu(), kv)
    return y + res


BATCHES = {   # decode sequences (1 token each) first, then prefill lengths
    "mixed": (3, [100, 37]),
    "prefill": (0, [70, 1, 150]),
    "decode": (5, []),
}


def _meta(kind, dev):
    nd, plens = BATCHES[kind]
    lens = [1] * nd + plens
    qsl = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    idx = torch.tensor([4, 0, 6, 2, 5, 1, 7][:len(lens)], dtype=torch.int32)
    has = torch.tensor([True, True, True, False, True, True, False][:len(lens)])
    if kind == "prefill":
        has = torch.tensor([False, True, True])
    md = SimpleNamespace(
        spec_sequence_masks=None, num_actual_tokens=int(qsl[-1]), num_decodes=nd,
        num_decode_tokens=nd, num_prefills=len(plens), non_spec_query_start_loc=qsl.to(dev),
        non_spec_state_indices_tensor=idx.to(dev), has_initial_state=has.to(dev),
        non_spec_query_start_loc_d=None, non_spec_query_start_loc_p=None,
        query_start_loc_cpu=qsl)
    if nd and plens:
        md.non_spec_query_start_loc_d = qsl[:nd + 1].to(dev)
        md.non_spec_query_start_loc_p = (qsl[nd:] - qsl[nd]).to(dev)
    return md, lens, idx, has


def _pools(seed):
    g0 = torch.Generator().manual_seed(seed)
    conv_cache = torch.randn(SLOTS, 3, CONV_DIM, generator=g0).bfloat16()
    s1 = torch.randn(SLOTS, H, D, D, generator=g0) * 0.05
    x = torch.randn(SLOTS, H, D, 16, generator=g0) * 0.05
    return conv_cache, s1, x @ x.transpose(-1, -2), g0


def _expected(kind, lay, md_lens, idx, has, nd, mixed_qkv, gates, conv_cache, states):
    """Per-sequence oracle composition; returns (o [n,H,D], new conv cache, states)."""
    w = lay.conv1d.weight.cpu().view(CONV_DIM, 4)
    conv_new = conv_cache.clone()
    st_new = [s.clone().double() for s in states]
    outs, t0 = [], 0
    for i, L in enumerate(md_lens):
        slot, sl = int(idx[i]), slice(t0, t0 + L)
        t0 += L
        init = i < nd or bool(has[i])
        o_c, cs = cref.conv_sequence(mixed_qkv[sl], conv_cache[slot] if init else None, w, None,
                                     "silu")
        conv_new[slot] = cs.to(conv_cache.dtype)
        xb = o_c.bfloat16()
        q = xb[:, :H * D].view(L, H, D)
        k = xb[:, H * D:(H + HKV) * D].view(L, HKV, D)
        v = xb[:, (H + HKV) * D:].view(L, HKV, D)
        if lay.proj_k is not None:
            k, v = _low_rank_ref(lay.proj_k, lay.k_rep, k), _low_rank_ref(lay.proj_v, lay.v_rep, v)
        if kind == "gdn":
            a, b = gates
            g, beta = gref.gdn_gating(lay.A.cpu(), a[sl], b[sl], lay.dt_bias.cpu())
            g, beta = g.to(a.dtype), beta.to(a.dtype)   # the gating returns a.dtype
            s0 = states[0][slot] if init else None
            o, S = gref.recurrent_seq(q, k, v, g[0], beta[0], D ** -0.5, s0, use_qk_l2norm=True)
            st_new[0][slot] = S
        else:
            a, alpha_in, b = gates
            if lay.use_forgetting_gate:
                g, alpha, beta = kref.gka_gating(lay.A.cpu(), a[sl], alpha_in[sl], b[sl],
                                                 lay.dt_bias.cpu())
                g, alpha, beta = g.to(a.dtype), alpha.to(a.dtype), beta.to(a.dtype)
            else:    # no forgetting gate: no decay, sigmoid gates in a.dtype (:1144-1148)
                g = torch.zeros(1, L, H, dtype=a.dtype)
                alpha = torch.sigmoid(alpha_in[sl].float()).to(a.dtype)[None]
                beta = torch.sigmoid(b[sl].float()).to(a.dtype)[None]
            alpha = alpha + 0.5                         # in a.dtype, as the layer adds it
            hkv0 = states[0][slot] if init else None
            hkk0 = states[1][slot] if init else None
            o, hkk, hkv = kref.gka_seq(q, k, v, alpha[0], g[0], g[0], beta[0], lay.gla_scale,
                                       lay.ridge_strength, lay.num_iter, hkk0, hkv0)
            st_new[0][slot], st_new[1][slot] = hkv, hkk
        outs.append(o)
    return torch.cat(outs), conv_new, st_new


def _run(kind, batch, dev, o_norm=False, seed=1, host_offsets=False, low_rank=None, **extra):
    lay = _layer(kind, seed, low_rank, **extra)
    md, lens, idx, has = _meta(batch, dev)
    nd = BATCHES[batch][0]
    n = md.num_actual_tokens
    conv_cache, s1, hkk, g0 = _pools(seed + 10)
    pad = 7                                        # rows past num_actual_tokens
    mixed_qkv = torch.randn(n + pad, CONV_DIM, generator=g0).bfloat16()
    a = torch.randn(n + pad, H, generator=g0).bfloat16()
    b = torch.randn(n + pad, H, generator=g0).bfloat16()
    alpha_in = torch.randn(n + pad, H, generator=g0).bfloat16()
    z = torch.randn(n + pad, H, D, generator=g0).bfloat16()
    wn = torch.rand(D, generator=g0) + 0.5
    lay_d = _to(lay, dev)
    cc_d = conv_cache.to(dev)
    core = torch.zeros(n + pad, H, D, dtype=torch.bfloat16, device=dev)
    onorm = (wn.to(dev), z.to(dev), 1e-6) if o_norm else None
    if kind == "gdn":
        ssm = s1.to(dev)
        srv.gdn_forward_core(lay_d, mixed_qkv.to(dev), b.to(dev), a.to(dev), core, md,
                             cc_d.transpose(1, 2), ssm, o_norm=onorm,
                             query_start_loc_cpu=md.query_start_loc_cpu if host_offsets else None)
        states_d, states, gates = [ssm], [s1], (a, b)
    else:
        hkv_d, hkk_d = s1.to(dev), hkk.to(dev)
        srv.gka_forward_core(lay_d, mixed_qkv.to(dev), a.to(dev), alpha_in.to(dev), b.to(dev),
                             core, md, cc_d.transpose(1, 2), hkk_d, hkv_d, o_norm=onorm,
                             query_start_loc_cpu=md.query_start_loc_cpu if host_offsets else None)
        states_d, states, gates = [hkv_d, hkk_d], [s1, hkk], (a, alpha_in, b)
    torch.cuda.synchronize()
    return dict(lay=lay, md=md, lens=lens, idx=idx, has=has, nd=nd, n=n, pad=pad,
                mixed_qkv=mixed_qkv, gates=gates, conv_cache=conv_cache, states=states,
                core=core.cpu(), cc=cc_d.cpu(), states_d=[s.cpu() for s in states_d], z=z, wn=wn)


def _check_against_oracle(kind, r):
    o_r, conv_r, st_r = _expected(kind, r["lay"], r["lens"], r["idx"], r["has"], r["nd"],
                                  r["mixed_qkv"], r["gates"], r["conv_cache"], r["states"])
    n = r["n"]
    assert_out_close(r["core"][:n], o_r)
    assert torch.equal(r["core"][n:], torch.zeros_like(r["core"][n:]))
    assert torch.equal(r["cc"], conv_r)
    used = set(int(i) for i in r["idx"])
    for got, exp, orig in zip(r["states_d"], st_r, r["states"]):
        for s in range(SLOTS):
            if s in used:
                assert_state_close(got[s], exp[s], what=f"slot {s}")
            else:
                assert torch.equal(got[s], orig[s])


@pytest.mark.parametrize("kind", ["gdn", "gka"])
@pytest.mark.parametrize("batch", ["mixed", "prefill", "decode"])
def test_forward_core_matches_oracle(dev, kind, batch):
    _check_against_oracle(kind, _run(kind, batch, dev))


@pytest.mark.parametrize("kind", ["gdn", "gka"])
@pytest.mark.parametrize("low_rank", ["repeat", "learnable"])
def test_forward_core_low_rank_kv(dev, kind, low_rank):
    """kv_proj_rank: k and v upsampled from HKV to H heads by the layer's low-rank
    projection plus the repeat or learnable residual before the ops."""
    _check_against_oracle(kind, _run(kind, "mixed", dev, low_rank=low_rank))


def test_forward_core_low_rank_needs_tp1(dev):
    lay = _layer("gdn", 3, low_rank="repeat")
    lay.tp_size = 2
    md, *_ = _meta("decode", dev)
    with pytest.raises(NotImplementedError):
        srv.gdn_forward_core(lay, None, None, None, None, md, None, None)


@pytest.mark.parametrize("kind", ["gdn", "gka"])
@pytest.mark.parametrize("batch", ["mixed", "prefill"])
def test_forward_core_host_offsets_equal_device(dev, kind, batch):
    """The prefill planned from the host copy of query_start_loc gives the same
    outputs and states as from the device offsets."""
    a, b = _run(kind, batch, dev), _run(kind, batch, dev, host_offsets=True)
    assert torch.equal(a["core"], b["core"]) and torch.equal(a["cc"], b["cc"])
    for x, y in zip(a["states_d"], b["states_d"]):
        assert torch.equal(x, y)


@pytest.mark.parametrize("kind", ["gdn", "gka"])
def test_forward_core_fused_o_norm(dev, kind):
    plain = _run(kind, "mixed", dev)
    fused = _run(kind, "mixed", dev, o_norm=True)
    n = plain["n"]
    o = plain["core"][:n].to(dev)
    expect = hmx.rms_norm_gated(o, plain["z"][:n].to(dev), plain["wn"].to(dev), 1e-6).cpu()
    got = fused["core"][:n]
    assert ((got.double() - expect.double()).abs()
            <= 2 * half_ulp(expect.double(), torch.bfloat16) + 1e-30).all()
    assert (got == expect).double().mean().item() >= 0.98
    for a, b in zip(plain["states_d"], fused["states_d"]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("batch", ["mixed", "decode"])
def test_gka_core_without_forgetting_gate(dev, batch):
    """use_forgetting_gate = False: g = None (no decay) and sigmoid alpha / beta in
    the gate dtype (primed_gka_layer.py:1144-1148)."""
    r = _run("gka", batch, dev, use_forgetting_gate=False, use_forgetting_gate_kk=False)
    o_r, conv_r, st_r = _expected("gka", r["lay"], r["lens"], r["idx"], r["has"], r["nd"],
                                  r["mixed_qkv"], r["gates"], r["conv_cache"], r["states"])
    n = r["n"]
    assert_out_close(r["core"][:n], o_r)
    assert torch.equal(r["cc"], conv_r)
    for got, exp in zip(r["states_d"], st_r):
        for s in set(int(i) for i in r["idx"]):
            assert_state_close(got[s], exp[s], what=f"slot {s}")

