"""GPU: the decode step captured in a HIP graph, as vLLM captures the mixers'
decode batches (primed_gdn_layer.py:85-90 registers the core as a custom op for
exactly that).  hmx.serving's GDN and GKA cores on a decode-only batch, and the
Mamba2 selective_state_update, are captured once and replayed several times
with eager work and synchronisations between the replays; every replay must
equal an eager run of the same step from the same pools, bit for bit.  The
decode paths read nothing back to the host and allocate only through torch's
caching allocator (captured as graph-owned memory), and record no memset.
"""
from types import SimpleNamespace

import pytest
import torch

import hmx
import hmx.serving as srv

pytestmark = pytest.mark.gpu

D, H, HKV, SLOTS, NSEQ = 128, 4, 2, 8, 5
CONV_DIM = (H + 2 * HKV) * D


def _layer(kind, dev):
    g0 = torch.Generator().manual_seed(7)
    lay = SimpleNamespace(
        conv1d=SimpleNamespace(weight=(torch.randn(CONV_DIM, 1, 4, generator=g0) * 0.4)
                               .bfloat16().to(dev)),
        activation="silu", A=torch.rand(H, generator=g0).to(dev),
        dt_bias=torch.randn(H, generator=g0).to(dev), key_dim=H * D, kv_k_dim=HKV * D,
        kv_v_dim=HKV * D, num_heads=H, num_kv_heads=HKV, head_k_dim=D, head_v_dim=D, tp_size=1,
        proj_k=None, allow_neg_eigval=False)
    if kind == "gka":
        lay.use_forgetting_gate = lay.use_forgetting_gate_kk = lay.use_beta_gate = True
        lay.num_iter, lay.ridge_strength, lay.gla_scale, lay._alpha_idx = 8, 0.02, D ** -0.5, None
    return lay


def _meta(dev):
    idx = torch.tensor([3, 7, -1, 0, 5], dtype=torch.int32, device=dev)   # one padded entry
    return SimpleNamespace(
        spec_sequence_masks=None, num_actual_tokens=NSEQ, num_decodes=NSEQ,
        num_decode_tokens=NSEQ, num_prefills=0,
        non_spec_query_start_loc=torch.arange(NSEQ + 1, dtype=torch.int32, device=dev),
        non_spec_state_indices_tensor=idx, has_initial_state=None,
        non_spec_query_start_loc_d=None, non_spec_query_start_loc_p=None)


def _state(dev, kind):
    g0 = torch.Generator().manual_seed(11)
    conv = torch.randn(SLOTS, 3, CONV_DIM, generator=g0).bfloat16().to(dev)
    s1 = (torch.randn(SLOTS, H, D, D, generator=g0) * 0.05).to(dev)
    x = torch.randn(SLOTS, H, D, 16, generator=g0) * 0.05
    s2 = (x @ x.transpose(-1, -2)).to(dev)
    return [conv, s1, s2] if kind == "gka" else [conv, s1]


def _inputs(dev, step):
    g0 = torch.Generator().manual_seed(100 + step)
    return (torch.randn(NSEQ, CONV_DIM, generator=g0).bfloat16().to(dev),
            torch.randn(NSEQ, H, generator=g0).bfloat16().to(dev),
            torch.randn(NSEQ, H, generator=g0).bfloat16().to(dev),
            torch.randn(NSEQ, H, generator=g0).bfloat16().to(dev))


def _step(kind, lay, md, st, xin, core):
    mixed, a, b, alpha_in = xin
    cs = st[0].transpose(1, 2)
    if kind == "gdn":
        srv.gdn_forward_core(lay, mixed, b, a, core, md, cs, st[1])
    else:
        srv.gka_forward_core(lay, mixed, a, alpha_in, b, core, md, cs, st[2], st[1])


@pytest.mark.parametrize("kind", ["gdn", "gka"])
def test_decode_core_graph_replays_match_eager(dev, kind):
    lay, md = _layer(kind, dev), _meta(dev)
    live = [0, 1, 3, 4]                                   # entry 2 is padded
    # static buffers the graph reads / writes
    st = _state(dev, kind)
    xin = [t.clone() for t in _inputs(dev, 0)]
    core = torch.zeros(NSEQ, H, D, dtype=torch.bfloat16, device=dev)
    # warm up on a side stream, then capture one step
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _step(kind, lay, md, [s.clone() for s in st], xin, core.clone())
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    snap = [s.clone() for s in st]
    with torch.cuda.graph(graph):
        _step(kind, lay, md, st, xin, core)
    for s, v in zip(st, snap):   # capture did not run the step: restore regardless
        s.copy_(v)
    for step in range(1, 5):
        new = _inputs(dev, step)
        for t, v in zip(xin, new):
            t.copy_(v)
        ref_st = [s.clone() for s in st]
        ref_core = torch.zeros_like(core)
        _step(kind, lay, md, ref_st, [t.clone() for t in new], ref_core)   # eager
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(core[live], ref_core[live]), f"replay {step}: outputs"
        for s, r in zip(st, ref_st):
            assert torch.equal(s, r), f"replay {step}: pools"
        _ = torch.randn(1000, device=dev).sum().item()     # eager work between replays


def test_selective_state_update_graph_replays_match_eager(dev):
    g0 = torch.Generator().manual_seed(3)
    Hs, P, N, B = 8, 64, 128, 6
    state = (torch.randn(10, Hs, P, N, generator=g0) * 0.1).to(dev)
    x = torch.randn(B, Hs, P, generator=g0).bfloat16().to(dev)
    dt = (torch.randn(B, Hs, generator=g0) - 2).to(dev)[:, :, None].expand(B, Hs, P)
    A = (-torch.rand(Hs, generator=g0) * 4).to(dev)[:, None, None].expand(Hs, P, N)
    Bm = torch.randn(B, 2, N, generator=g0).bfloat16().to(dev)
    idx = torch.tensor([9, 0, 4, -1, 2, 7], dtype=torch.int32, device=dev)
    out = torch.empty_like(x)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        hmx.selective_state_update(state.clone(), x, dt, A, Bm, Bm, dt_softplus=True,
                                   state_batch_indices=idx, out=out.clone())
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    snap = state.clone()
    with torch.cuda.graph(graph):
        hmx.selective_state_update(state, x, dt, A, Bm, Bm, dt_softplus=True,
                                   state_batch_indices=idx, out=out)
    state.copy_(snap)
    live = [0, 1, 2, 4, 5]
    for step in range(4):
        x.copy_(torch.randn(B, Hs, P, device=dev).bfloat16())
        ref_state = state.clone()
        ref_out = hmx.selective_state_update(ref_state, x.clone(), dt, A, Bm, Bm,
                                             dt_softplus=True, state_batch_indices=idx)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[live], ref_out[live]) and torch.equal(state, ref_state)
