"""GPU: the Mamba2 serving core (hmx.serving.mamba2_conv_ssm_forward, the vLLM
layer's ``conv_ssm_forward``, primed_mamba2_layer.py:615-1021) and the SSD ops'
grouped operands it relies on.

- Grouped operands: the varlen scan and selective_state_update with x and B at
  HX heads (the layer's pre-repeat_kv width, :800-835, :972-985) and C at H
  groups give bit-identical results to the same calls on explicitly repeated,
  contiguous copies (the reference's layout).
- The core on mixed, prefill-only and decode-only batches against a
  per-sequence composition of the oracles: the layer's B/C RMSNorm (a stand-in
  module), the conv oracle with bias (state from the conv cache slot, or zeros
  for a prefill without an initial state), the conv output rounded to bf16 as
  the op stores it, then the SSD recurrence oracle from the state pool slot.
  Checks: output rows within the output tolerance (rows past num_actual_tokens
  untouched), pool slots within the state tolerance (others untouched), conv
  cache bit for bit.  The layer and metadata are stand-ins with the reference's
  attribute names (vLLM is not installed here).
- Prefix caching (mamba_cache_mode "all"): the same composition run piecewise
  between the blocks' ends, every block slot checked.
- The profile run (attn_metadata None) writes nothing.
"""
from types import SimpleNamespace

import pytest
import torch

import hmx
import hmx.serving as srv
from oracle import conv as cref
from oracle import ssd as sref
from util import assert_out_close, assert_state_close

pytestmark = pytest.mark.gpu

H, P, HX = 8, 64, 2
N = P
I, XB = H * P, HX * N
CD = I + 2 * XB
SLOTS = 8
W = 4


def _cu(lens, dev):
    return torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32, device=dev)


def test_varlen_grouped_operands_equal_repeated(dev):
    g0 = torch.Generator().manual_seed(5)
    lens = [130, 1, 300, 64]
    T = sum(lens)
    rep = H // HX
    xg = torch.randn(T, HX, P, generator=g0).bfloat16().to(dev)
    Bg = torch.randn(T, HX, N, generator=g0).bfloat16().to(dev)
    C = torch.randn(T, H, N, generator=g0).bfloat16().to(dev)
    dt = (torch.randn(T, H, generator=g0) * 0.5 - 2).bfloat16().to(dev)
    A = -torch.exp(torch.rand(H, generator=g0) * 2).to(dev)
    D = torch.randn(H, generator=g0).to(dev)
    bias = torch.randn(H, generator=g0).to(dev) * 0.5
    pool = (torch.randn(SLOTS, H, P, N, generator=g0) * 0.1).to(dev)
    idx = torch.tensor([6, 1, 3, 0], dtype=torch.int32, device=dev)
    has = torch.tensor([True, False, True, True], device=dev)
    cu = _cu(lens, dev)
    outs, pools = [], []
    for x, B in ((xg, Bg), (xg.repeat_interleave(rep, 1).contiguous(),
                            Bg.repeat_interleave(rep, 1).contiguous())):
        p2 = pool.clone()
        y = torch.empty(T, H, P, dtype=torch.bfloat16, device=dev)
        hmx.mamba_chunk_scan_combined_varlen(x, dt, A, B, C, 256, cu_seqlens=cu, out=y, D=D,
                                             dt_bias=bias, initial_states=p2, dt_softplus=True,
                                             ssm_state_indices=idx, has_initial_state=has)
        outs.append(y)
        pools.append(p2)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(pools[0], pools[1])


def test_state_update_grouped_operands_equal_repeated(dev):
    g0 = torch.Generator().manual_seed(6)
    b = 6
    rep = H // HX
    xg = torch.randn(b, HX, P, generator=g0).bfloat16().to(dev)
    Bg = torch.randn(b, HX, N, generator=g0).bfloat16().to(dev)
    C = torch.randn(b, H, N, generator=g0).bfloat16().to(dev)
    dt = (torch.randn(b, H, generator=g0) - 1).bfloat16().to(dev)[:, :, None].expand(b, H, P)
    A = (-torch.rand(H, generator=g0) * 3).to(dev)[:, None, None].expand(H, P, N)
    D = torch.randn(H, generator=g0).to(dev)[:, None].expand(H, P)
    pool = (torch.randn(SLOTS, H, P, N, generator=g0) * 0.1).to(dev)
    idx = torch.tensor([4, 0, -1, 7, 2, 5], dtype=torch.int32, device=dev)
    res = []
    for x, B in ((xg, Bg), (xg.repeat_interleave(rep, 1).contiguous(),
                            Bg.repeat_interleave(rep, 1).contiguous())):
        p2 = pool.clone()
        o = hmx.selective_state_update(p2, x, dt, A, B, C, D, dt_softplus=True,
                                       state_batch_indices=idx)
        res.append((o, p2))
    torch.cuda.synchronize()
    live = [0, 1, 3, 4, 5]
    assert torch.equal(res[0][0][live], res[1][0][live]) and torch.equal(res[0][1], res[1][1])


class _RMSNorm:
    """Stand-in for the layer's vLLM RMSNorm modules (B_norm / C_norm, :66-67):
    x * rsqrt(mean(x^2) + eps) in fp32, back to x's dtype, times the weight."""

    def __init__(self, weight, eps=1e-6):
        self.weight, self.eps = weight, eps

    def __call__(self, x):
        xf = x.float()
        y = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)).to(x.dtype)
        return y * self.weight


class _Rope:
    """Stand-in for the layer's vLLM rotary embedding (get_rope, primed_mamba2_layer.py
    :555-566), called as rotary_emb(positions, C, B) -> (C, B): neox-style rotation of
    every head_dim row, its halves (a, b) -> (a cos - b sin, b cos + a sin) at angle
    position * 10000^(-2i/d), in fp32 and back to the input dtype."""

    def __init__(self, d):
        self.d = d

    def _rot(self, positions, x):
        d, half = self.d, self.d // 2
        inv = 10000.0 ** (-torch.arange(half, device=x.device, dtype=torch.float32) * 2 / d)
        ang = positions.float()[:, None] * inv[None]
        cos, sin = ang.cos()[:, None], ang.sin()[:, None]
        xr = x.float().view(x.shape[0], -1, d)
        a, b = xr[..., :half], xr[..., half:]
        y = torch.cat([a * cos - b * sin, b * cos + a * sin], dim=-1)
        return y.to(x.dtype).view(x.shape)

    def __call__(self, positions, q, k):
        return self._rot(positions, q), self._rot(positions, k)


def _layer(seed, dev):
    g0 = torch.Generator().manual_seed(seed)
    pad = (8 - (2 * I + 2 * XB + H) % 8) % 8
    lay = SimpleNamespace(
        tp_size=1, tped_intermediate_size=I, tped_conv_size=CD, dt_pad=pad, num_heads=H,
        xb_size=XB, ssm_state_size=N, head_dim=P, n_groups=H, chunk_size=256,
        conv_weights=(torch.randn(CD, W, generator=g0) * 0.4).bfloat16().to(dev),
        conv1d=SimpleNamespace(bias=(torch.randn(CD, generator=g0) * 0.1).bfloat16().to(dev)),
        activation="silu", A=(-torch.exp(torch.rand(H, generator=g0) * 2)).to(dev),
        D=torch.randn(H, generator=g0).to(dev), dt_bias=(torch.randn(H, generator=g0) * 0.5).to(dev),
        B_norm=_RMSNorm((torch.rand(P, generator=g0) + 0.5).bfloat16().to(dev)),
        C_norm=_RMSNorm((torch.rand(P, generator=g0) + 0.5).bfloat16().to(dev)),
        use_pos_embed=False, cache_config=SimpleNamespace(mamba_cache_mode="none"))
    return lay, 2 * I + 2 * XB + H + pad


BATCHES = {   # decode sequences (1 token each) first, then prefill lengths
    "mixed": (3, [100, 37]),
    "prefill": (0, [70, 1, 300]),
    "decode": (5, []),
}


def _meta(kind, dev):
    nd, plens = BATCHES[kind]
    idx = torch.tensor([4, 0, 6, 2, 5, 1, 7][:nd + len(plens)], dtype=torch.int32)
    has_p = torch.tensor([True, False, True][:len(plens)])
    qsl_p = torch.tensor([0] + list(torch.tensor(plens, dtype=torch.int64).cumsum(0)),
                         dtype=torch.int32)
    md = SimpleNamespace(
        num_prefills=len(plens), num_decode_tokens=nd, num_prefill_tokens=sum(plens),
        state_indices_tensor=idx.to(dev), has_initial_states_p=has_p.to(dev) if plens else None,
        prep_initial_states=bool(plens), query_start_loc_p=qsl_p.to(dev) if plens else None)
    return md, nd, plens, idx, has_p


def _normed(lay, proj, positions=None):
    """The layer's own B/C RMSNorm and rotary steps (:663-671), on proj's device: the
    modules are the layer's, so the expected path applies them where the core does
    (a reduction in another order could round differently)."""
    hs, B, C = torch.split(proj[:, I:I + CD], [XB, XB, CD - 2 * XB], dim=-1)
    B = lay.B_norm(B.reshape(-1, P)).view(B.shape)
    C = lay.C_norm(C.reshape(-1, P)).view(C.shape)
    if lay.use_pos_embed:
        C, B = lay.rotary_emb(positions, C, B)
    return torch.cat([hs, B, C], dim=-1)


def _expected(lay, nd, plens, idx, has_p, hbc, dt, conv_cache, pool):
    """Per-sequence oracle composition over the normed conv input hbc [n, CD] and
    dt [n, H]: (out [n, H, P], conv cache, pool)."""
    w, bias = lay.conv_weights.cpu(), lay.conv1d.bias.cpu()
    conv_new, pool_new = conv_cache.clone(), pool.clone().double()
    lens = [1] * nd + plens
    outs, t0 = [], 0
    for i, L in enumerate(lens):
        slot, sl = int(idx[i]), slice(t0, t0 + L)
        t0 += L
        init = i < nd or bool(has_p[i - nd])
        o_c, cs = cref.conv_sequence(hbc[sl], conv_cache[slot] if init else None, w, bias, "silu")
        conv_new[slot] = cs.to(conv_cache.dtype)
        xc = o_c.bfloat16()
        x = xc[:, :XB].reshape(L, HX, P).repeat_interleave(H // HX, 1)
        Bh = xc[:, XB:2 * XB].reshape(L, HX, N).repeat_interleave(H // HX, 1)
        Ch = xc[:, 2 * XB:].reshape(L, H, N)
        dtp = sref.dt_transform(dt[sl], lay.dt_bias.cpu(), True)
        y, S = sref.ssd_seq(x, dtp, lay.A.cpu(), Bh, Ch, lay.D.cpu(), None,
                            pool[slot] if init else None)
        pool_new[slot] = S
        outs.append(y)
    return torch.cat(outs), conv_new, pool_new


@pytest.mark.parametrize("batch,rope", [("mixed", False), ("prefill", False), ("decode", False),
                                        ("mixed", True)])
def test_conv_ssm_forward_matches_oracle(dev, batch, rope):
    """rope: use_pos_embed with the layer's rotary embedding of B and C before the
    conv (primed_mamba2_layer.py:664-671)."""
    lay, dproj = _layer(1, dev)
    lay.use_pos_embed = rope
    lay.rotary_emb = _Rope(P)
    md, nd, plens, idx, has_p = _meta(batch, dev)
    n = nd + sum(plens)
    g0 = torch.Generator().manual_seed(20)
    extra = 5                                         # rows past num_actual_tokens
    proj = torch.randn(n + extra, dproj, generator=g0).bfloat16()
    proj[:, I + CD:I + CD + H] = proj[:, I + CD:I + CD + H] * 0.5 - 1.5   # dt
    conv_cache = torch.randn(SLOTS, W - 1, CD, generator=g0).bfloat16()
    pool = torch.randn(SLOTS, H, P, N, generator=g0) * 0.1
    cc_d, pool_d = conv_cache.to(dev), pool.to(dev)
    output = torch.zeros(n + extra, I, dtype=torch.bfloat16, device=dev)
    positions = torch.randint(0, 4000, (n + extra,), generator=g0).to(dev)
    srv.mamba2_conv_ssm_forward(lay, proj.to(dev), output, md, cc_d.transpose(1, 2), pool_d,
                                positions=positions)
    torch.cuda.synchronize()
    o_r, conv_r, pool_r = _expected(lay, nd, plens, idx, has_p,
                                    _normed(lay, proj.to(dev), positions).cpu(),
                                    proj[:, I + CD:I + CD + H], conv_cache, pool)
    got = output.cpu()
    assert_out_close(got[:n].view(n, H, P), o_r)
    assert torch.equal(got[n:], torch.zeros_like(got[n:]))
    assert torch.equal(cc_d.cpu(), conv_r)
    used = set(int(i) for i in idx)
    pool_g = pool_d.cpu()
    for s in range(SLOTS):
        if s in used:
            assert_state_close(pool_g[s], pool_r[s], what=f"slot {s}")
        else:
            assert torch.equal(pool_g[s], pool[s])


def test_conv_ssm_forward_needs_positions_for_rope(dev):
    lay, _ = _layer(2, dev)
    md, *_ = _meta("decode", dev)
    lay.use_pos_embed = True
    with pytest.raises(ValueError):                 # the rotary embedding needs positions
        srv.mamba2_conv_ssm_forward(lay, None, None, md, None, None)


def test_conv_ssm_forward_profile_run(dev):
    """attn_metadata None (vLLM's profile run, :676-697): nothing is written, and the
    x columns repeated over the heads are returned, as the layer returns them."""
    lay, dproj = _layer(4, dev)
    g0 = torch.Generator().manual_seed(41)
    proj = torch.randn(9, dproj, generator=g0).bfloat16().to(dev)
    output = torch.zeros(9, I, dtype=torch.bfloat16, device=dev)
    got = srv.mamba2_conv_ssm_forward(lay, proj, output, None, None, None)
    torch.cuda.synchronize()
    hs = proj[:, I:I + XB].reshape(9, HX, P)
    assert torch.equal(got, hs.repeat_interleave(H // HX, 1).reshape(9, H * P))
    assert torch.equal(output, torch.zeros_like(output))


APC_BS, APC_CHUNK, APC_SLOTS = 128, 64, 24


def _prefix_chunks(lens, computed, chunk):
    """vLLM's prefix-cache chunking: a chunk ends where the absolute position
    (num_computed_tokens plus the offset) is a multiple of chunk."""
    cu, seq, last, pos = [0], [], [], 0
    for n, (L, nc) in enumerate(zip(lens, computed)):
        off = 0
        while off < L:
            off += min(chunk - (nc + off) % chunk, L - off)
            cu.append(pos + off)
            seq.append(n)
        pos += L
        last.append(len(seq) - 1)
    return cu, seq, last


def _meta_apc(dev, dec_nc, pre):
    """Prefix-caching metadata (the fields primed_mamba2_layer.py:728-754, :844-863
    read) for decodes continuing dec_nc tokens and prefills (num_computed, length),
    with vLLM's block indices: the blocks of the last computed token, the first and
    the last scheduled token (block 0 before any token)."""
    reqs = [(nc, 1) for nc in dec_nc] + list(pre)
    nblk = max((nc + L - 1) // APC_BS + 1 for nc, L in reqs)
    g = torch.Generator().manual_seed(3)
    table = torch.randperm(APC_SLOTS, generator=g)[:len(reqs) * nblk].view(len(reqs), nblk)
    table = table.to(torch.int32)
    lc = torch.tensor([max(nc - 1, 0) // APC_BS for nc, _ in reqs], dtype=torch.int32)
    ls = torch.tensor([(nc + L - 1) // APC_BS for nc, L in reqs], dtype=torch.int32)
    nd = len(dec_nc)
    plens, pnc = [L for _, L in pre], [nc for nc, _ in pre]
    cu_c, seq, last = _prefix_chunks(plens, pnc, APC_CHUNK)
    t = lambda v: torch.tensor(v, dtype=torch.int32, device=dev)
    md = SimpleNamespace(
        num_prefills=len(pre), num_decode_tokens=nd, num_prefill_tokens=sum(plens),
        state_indices_tensor=table.to(dev), has_initial_states_p=torch.tensor(
            [nc > 0 for nc in pnc], device=dev), prep_initial_states=True,
        query_start_loc_p=t([0] + list(torch.tensor(plens).cumsum(0).tolist())),
        chunk_size=APC_CHUNK, cu_chunk_seqlen_p=t(cu_c), seq_idx_p=t(seq),
        last_chunk_indices_p=t(last), block_idx_last_computed_token=lc.to(dev),
        block_idx_last_scheduled_token=ls.to(dev),
        block_idx_first_scheduled_token_p=t([nc // APC_BS for nc in pnc]),
        num_computed_tokens_p=t(pnc))
    return md, reqs, table


def _expected_apc(lay, reqs, table, hbc, dt, conv_cache, pool):
    """Per request: the conv and the SSD recurrence from the slot of its last
    computed block (zeros for a request with no computed token), run piecewise
    between the block ends of this step; each block's slot gets the conv and SSD
    states at its end, the last scheduled block's slot those after the last token."""
    w, bias = lay.conv_weights.cpu(), lay.conv1d.bias.cpu()
    conv_new, pool_new = conv_cache.clone(), pool.clone().double()
    outs, t0 = [], 0
    for r, (nc, L) in enumerate(reqs):
        lc, fs, ls = max(nc - 1, 0) // APC_BS, nc // APC_BS, (nc + L - 1) // APC_BS
        rs, sl = int(table[r, lc]), slice(t0, t0 + L)
        t0 += L
        cst = conv_cache[rs] if nc > 0 else torch.zeros(W - 1, CD, dtype=conv_cache.dtype)
        o_c, _ = cref.conv_sequence(hbc[sl], cst, w, bias, "silu")
        hist = torch.cat([cst, hbc[sl]])
        xc = o_c.bfloat16()
        x = xc[:, :XB].reshape(L, HX, P).repeat_interleave(H // HX, 1)
        Bh = xc[:, XB:2 * XB].reshape(L, HX, N).repeat_interleave(H // HX, 1)
        Ch = xc[:, 2 * XB:].reshape(L, H, N)
        dtp = sref.dt_transform(dt[sl], lay.dt_bias.cpu(), True)
        S = pool[rs] if nc > 0 else None
        ends = [(k + 1) * APC_BS - nc for k in range(fs, ls)] + [L]
        a, ys = 0, []
        for j, e in enumerate(ends):
            y, S = sref.ssd_seq(x[a:e], dtp[a:e], lay.A.cpu(), Bh[a:e], Ch[a:e], lay.D.cpu(),
                                None, S)
            ys.append(y)
            slot = int(table[r, fs + j])
            pool_new[slot] = S
            conv_new[slot] = hist[e:e + W - 1]
            a = e
        outs.append(torch.cat(ys))
    return torch.cat(outs), conv_new, pool_new


@pytest.mark.parametrize("batch", ["mixed", "prefill", "decode"])
def test_conv_ssm_forward_prefix_caching(dev, batch):
    """mamba_cache_mode "all" (primed_mamba2_layer.py:728-1021): requests continuing
    0, unaligned, block-aligned and chunk-unaligned computed tokens, prefills
    crossing several blocks and one ending on a block boundary; decodes in the
    middle of a block and at a block boundary (reading block 0, writing block 1).
    Outputs, every block slot's conv (bit for bit) and SSD state, untouched slots
    unchanged."""
    lay, dproj = _layer(5, dev)
    lay.cache_config = SimpleNamespace(mamba_cache_mode="all", mamba_block_size=APC_BS)
    dec = {"mixed": [127, 128], "prefill": [], "decode": [5, 128, 300]}[batch]
    pre = {"mixed": [(100, 200), (0, 300), (256, 64)], "prefill": [(130, 3), (0, 256), (70, 90)],
           "decode": []}[batch]
    md, reqs, table = _meta_apc(dev, dec, pre)
    n = sum(L for _, L in reqs)
    g0 = torch.Generator().manual_seed(50)
    proj = torch.randn(n + 3, dproj, generator=g0).bfloat16()
    proj[:, I + CD:I + CD + H] = proj[:, I + CD:I + CD + H] * 0.5 - 1.5
    conv_cache = torch.randn(APC_SLOTS, W - 1, CD, generator=g0).bfloat16()
    pool = torch.randn(APC_SLOTS, H, P, N, generator=g0) * 0.1
    cc_d, pool_d = conv_cache.to(dev), pool.to(dev)
    output = torch.zeros(n + 3, I, dtype=torch.bfloat16, device=dev)
    srv.mamba2_conv_ssm_forward(lay, proj.to(dev), output, md, cc_d.transpose(1, 2), pool_d)
    torch.cuda.synchronize()
    o_r, conv_r, pool_r = _expected_apc(lay, reqs, table, _normed(lay, proj.to(dev)).cpu(),
                                        proj[:, I + CD:I + CD + H], conv_cache, pool)
    got = output.cpu()
    assert_out_close(got[:n].view(n, H, P), o_r)
    assert torch.equal(got[n:], torch.zeros_like(got[n:]))
    assert torch.equal(cc_d.cpu(), conv_r)
    pool_g = pool_d.cpu()
    for s in range(APC_SLOTS):
        if not torch.equal(conv_r[s], conv_cache[s]) or not torch.equal(pool_r[s].float(), pool[s]):
            assert_state_close(pool_g[s], pool_r[s], what=f"slot {s}")
        else:
            assert torch.equal(pool_g[s], pool[s]), f"slot {s} changed"


def test_conv_ssm_forward_decode_graph_replays_match_eager(dev):
    """The decode-only core captured in a HIP graph (vLLM captures decode batches)
    and replayed with eager work between replays: every replay equals an eager run
    of the same step from the same pools, bit for bit."""
    lay, dproj = _layer(3, dev)
    md, nd, _, idx, _ = _meta("decode", dev)
    g0 = torch.Generator().manual_seed(30)
    conv = torch.randn(SLOTS, W - 1, CD, generator=g0).bfloat16().to(dev)
    pool = (torch.randn(SLOTS, H, P, N, generator=g0) * 0.1).to(dev)
    proj = torch.randn(nd, dproj, generator=g0).bfloat16().to(dev)
    output = torch.zeros(nd, I, dtype=torch.bfloat16, device=dev)
    step = lambda pr, o, c, s: srv.mamba2_conv_ssm_forward(lay, pr, o, md, c.transpose(1, 2), s)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(proj.clone(), output.clone(), conv.clone(), pool.clone())
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    snap = (conv.clone(), pool.clone())
    with torch.cuda.graph(graph):
        step(proj, output, conv, pool)
    conv.copy_(snap[0])
    pool.copy_(snap[1])
    for r in range(4):
        proj.copy_(torch.randn(nd, dproj, generator=g0).bfloat16().to(dev))
        ref_c, ref_s, ref_o = conv.clone(), pool.clone(), torch.zeros_like(output)
        step(proj.clone(), ref_o, ref_c, ref_s)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(output, ref_o), f"replay {r}: output"
        assert torch.equal(conv, ref_c) and torch.equal(pool, ref_s), f"replay {r}: pools"
        _ = torch.randn(1000, device=dev).sum().item()
