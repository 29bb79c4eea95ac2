"""Prefills planned from host sequence offsets: the same results as from device
offsets, with no device-to-host copy (torch's sync debug mode turns any
synchronising copy into an error; the device-offset call is the control that
must trip it)."""
import pytest
import torch

import hmx

pytestmark = pytest.mark.gpu

LENS = [300, 0, 1, 2000, 77]


def _offsets():
    cs = [0]
    for n in LENS:
        cs.append(cs[-1] + n)
    return torch.tensor(cs, dtype=torch.int64)


def _gdn(dev, cs):
    g0 = torch.Generator(device="cpu").manual_seed(5)
    T, H, D = int(cs[-1]), 8, 128
    q, k, v = (torch.randn(1, T, H, D, generator=g0).bfloat16().to(dev) for _ in range(3))
    g = torch.nn.functional.logsigmoid(torch.randn(1, T, H, generator=g0)).to(dev)
    beta = torch.rand(1, T, H, generator=g0).to(dev)
    return lambda c: hmx.chunk_gated_delta_rule_gqa(q, k, v, g, beta, output_final_state=True,
                                                    cu_seqlens=c, use_qk_l2norm_in_kernel=True)


def _gka(dev, cs):
    g0 = torch.Generator(device="cpu").manual_seed(6)
    T, H, D = int(cs[-1]), 4, 128
    q, k, v = (torch.randn(1, T, H, D, generator=g0).bfloat16().to(dev) for _ in range(3))
    alpha = torch.sigmoid(torch.randn(1, T, H, generator=g0)).to(dev)
    g = torch.nn.functional.logsigmoid(torch.randn(1, T, H, generator=g0)).to(dev)
    beta = torch.sigmoid(torch.randn(1, T, H, generator=g0)).to(dev)
    return lambda c: hmx.gka_chebyshev_gla_prefill(q, k, v, alpha, g, g, beta, D ** -0.5,
                                                   ridge_ratio=0.01, num_iter=4, cu_seqlens=c)


def _ssd(dev, cs):
    g0 = torch.Generator(device="cpu").manual_seed(7)
    T, H, P, G, N = int(cs[-1]), 8, 64, 2, 128
    x = torch.randn(T, H, P, generator=g0).bfloat16().to(dev)
    dt = (torch.rand(T, H, generator=g0) * 0.1).to(dev)
    A = (-torch.rand(H, generator=g0)).to(dev)
    B = torch.randn(T, G, N, generator=g0).bfloat16().to(dev)
    C = torch.randn(T, G, N, generator=g0).bfloat16().to(dev)
    return lambda c: hmx.mamba_chunk_scan_combined_varlen(x, dt, A, B, C, 256, c)


def _flat(r):
    return [t for t in (r if isinstance(r, (tuple, list)) else (r,)) if t is not None]


@pytest.mark.parametrize("make", [_gdn, _gka, _ssd], ids=["gdn", "gka", "ssd"])
def test_prefill_host_offsets_sync_free_and_equal(dev, make):
    cs = _offsets()
    run = make(dev, cs)
    ref = _flat(run(cs.to(dev)))
    torch.cuda.synchronize()
    run(cs)                                  # plan once (the segment table upload is cached)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        got = _flat(run(cs))
        with pytest.raises(RuntimeError):    # the control: device offsets are read back
            run(cs.to(dev))
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    assert len(got) == len(ref)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
