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


def _ssd_prefix(dev, pooled):
    """The Mamba2 prefix-caching scan (return_intermediate_states) with vLLM's chunk
    metadata: cu_seqlens, cu_chunk_seqlens, seq_idx, last_chunk_indices."""
    g0 = torch.Generator(device="cpu").manual_seed(8)
    lens, computed = [300, 1, 640, 77], [100, 0, 256, 500]
    cs, cu_c, seq, last = [0], [0], [], []
    for n, (L, nc) in enumerate(zip(lens, computed)):
        off = 0
        while off < L:
            off += min(256 - (nc + off) % 256, L - off)
            cu_c.append(cs[-1] + off)
            seq.append(n)
        cs.append(cs[-1] + L)
        last.append(len(seq) - 1)
    T, H, P, G, N = cs[-1], 4, 64, 2, 128
    x = torch.randn(T, H, P, generator=g0).bfloat16().to(dev)
    dt = (torch.rand(T, H, generator=g0) * 0.1).to(dev)
    A = (-torch.rand(H, generator=g0)).to(dev)
    B = torch.randn(T, G, N, generator=g0).bfloat16().to(dev)
    C = torch.randn(T, G, N, generator=g0).bfloat16().to(dev)
    h0 = (torch.randn(len(lens), H, P, N, generator=g0) * 0.1).to(dev)
    meta = [torch.tensor(v, dtype=torch.int32) for v in (cs, cu_c, seq, last)]
    slots = torch.tensor([3, 0, 5, 1], dtype=torch.int32, device=dev)

    def run(on_dev):
        m = [t.to(dev) if on_dev else t for t in meta]
        out = torch.empty(T, H, P, dtype=torch.bfloat16, device=dev)
        kw = dict(cu_seqlens=m[0], cu_chunk_seqlens=m[1], seq_idx=m[2], last_chunk_indices=m[3],
                  out=out, return_intermediate_states=True)
        if pooled:
            pool = torch.zeros(6, H, P, N, device=dev)
            pool[slots.long()] = h0
            st = hmx.mamba_chunk_scan_combined_varlen(x, dt, A, B, C, 256, initial_states=pool,
                                                      ssm_state_indices=slots, **kw)
            return st, out, pool
        st = hmx.mamba_chunk_scan_combined_varlen(x, dt, A, B, C, 256, initial_states=h0, **kw)
        return st, out
    return run, meta, (x, dt, A, B, C, h0)


@pytest.mark.parametrize("pooled", [False, True], ids=["states", "pool"])
def test_ssd_prefix_cache_host_metadata_sync_free(dev, pooled):
    """The prefix-cache scan reads host chunk metadata with no device-to-host copy
    and returns what device metadata gives."""
    run, _, _ = _ssd_prefix(dev, pooled)
    want = run(True)
    torch.cuda.synchronize()
    run(False)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        got = run(False)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    for a, b in zip(got, want):
        assert torch.equal(a, b)


def test_ssd_prefix_cache_bad_last_chunk_indices_leaves_buffers(dev):
    """A wrong last_chunk_indices raises before the scan writes out or the pool."""
    run, meta, (x, dt, A, B, C, h0) = _ssd_prefix(dev, True)
    T, H, P = x.shape
    pool = torch.randn(6, H, P, 128, device=dev)
    out = torch.full((T, H, P), 7.0, dtype=torch.bfloat16, device=dev)
    pool0, out0 = pool.clone(), out.clone()
    bad = meta[3].clone()
    bad[0] += 1
    with pytest.raises(ValueError):
        hmx.mamba_chunk_scan_combined_varlen(
            x, dt, A, B, C, 256, cu_seqlens=meta[0], cu_chunk_seqlens=meta[1], seq_idx=meta[2],
            last_chunk_indices=bad, out=out, initial_states=pool,
            ssm_state_indices=torch.tensor([3, 0, 5, 1], dtype=torch.int32, device=dev),
            return_intermediate_states=True)
    torch.cuda.synchronize()
    assert torch.equal(pool, pool0) and torch.equal(out, out0)


def test_ssd_seq_idx_host_sync_free(dev):
    """mamba_chunk_scan_combined with a host seq_idx (sequence resets inside a row)
    and final states: no device-to-host copy, the same result as a device seq_idx."""
    g0 = torch.Generator(device="cpu").manual_seed(9)
    b, l, H, P, G, N = 2, 700, 4, 64, 2, 128
    x = torch.randn(b, l, H, P, generator=g0).bfloat16().to(dev)
    dt = (torch.rand(b, l, H, generator=g0) * 0.1).to(dev)
    A = (-torch.rand(H, generator=g0)).to(dev)
    B = torch.randn(b, l, G, N, generator=g0).bfloat16().to(dev)
    C = torch.randn(b, l, G, N, generator=g0).bfloat16().to(dev)
    si = torch.zeros(b, l, dtype=torch.int32)
    si[0, 250:] = 1
    si[1, 600:] = 1
    h0 = (torch.randn(b, H, P, N, generator=g0) * 0.1).to(dev)

    def run(s):
        return hmx.mamba_chunk_scan_combined(x, dt, A, B, C, 256, initial_states=h0, seq_idx=s,
                                             return_final_states=True)
    want = run(si.to(dev))
    torch.cuda.synchronize()
    run(si)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        got = run(si)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    for a, c in zip(got, want):
        assert torch.equal(a, c)
