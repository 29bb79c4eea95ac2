"""GPU check of hmx_gdn_chunk_fwd_noalloc, the GDN prefill entry point whose
workspace is a static device array: called through the C ABI, its outputs and end
states equal hmx_gdn_chunk_fwd's (same kernels, same segment table, caller
workspace) bit for bit, on two calls in a row, the second with a smaller input
(the rejection of oversized tables is a CPU test in test_abi.py), and that the
array is placed in device memory only when the entry point is first called."""
import pytest
import torch
import torch.nn.functional as F

from hmx import _lib
from hmx.ops import gdn as gops

pytestmark = pytest.mark.gpu


def _inputs(T, H, HKV, lens, seed, dev):
    g0 = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(1, T, H, 128, generator=g0), dim=-1).bfloat16().to(dev)
    k = F.normalize(torch.randn(1, T, HKV, 128, generator=g0), dim=-1).bfloat16().to(dev)
    v = torch.randn(1, T, HKV, 128, generator=g0).bfloat16().to(dev)
    g = F.logsigmoid(torch.randn(1, T, H, generator=g0)).to(dev)
    beta = torch.sigmoid(torch.randn(1, T, H, generator=g0)).to(dev)
    h0 = (torch.randn(len(lens), H, 128, 128, generator=g0) * 0.05).to(dev)
    cs = [0]
    for n in lens:
        cs.append(cs[-1] + n)
    bounds = [(cs[i], cs[i + 1]) for i in range(len(lens))]
    return q, k, v, g, beta, h0, bounds


def _call(name, q, k, v, g, beta, h0, bounds, seg_chunks, workspace):
    dev = q.device
    H, HKV = q.shape[2], k.shape[2]
    N = len(bounds)
    rows, _ = _lib.plan_segments(_lib.PLAN_GDN, bounds, q.shape[0] * q.shape[1], H, 256, seg_chunks)
    seg = torch.from_numpy(rows).to(dev)
    o = torch.zeros_like(q)
    ht = torch.zeros(N, H, 128, 128, device=dev)
    args = [_lib.ptr(q), H * 128, _lib.ptr(k), HKV * 128, _lib.ptr(v), HKV * 128, _lib.HMX_BF16,
            _lib.ptr(g), _lib.HMX_F32, _lib.ptr(beta), _lib.HMX_F32, _lib.ptr(o), _lib.ptr(h0),
            _lib.ptr(ht), H * 128 * 128, _lib.HMX_F32, None, None, _lib.ptr(seg), len(rows), N, H,
            HKV, 128, 128, 128 ** -0.5, 1, gops.MAX_WARM_CHUNKS, gops.DECAY_THRESHOLD]
    if workspace:
        lib = _lib.load()
        nb = int(lib.hmx_gdn_chunk_workspace_bytes(len(rows), N, H, 0))
        ws = torch.empty(nb, dtype=torch.uint8, device=dev)
        args += [_lib.ptr(ws), nb]
    _lib.call(name, *args, None, None, _lib.stream_of(q))
    torch.cuda.synchronize()
    return o, ht, len(rows)


def test_noalloc_scratch_reserved_at_first_call(dev):
    """The scratch array sits in a code object of its own (no kernels), which the
    runtime loads at the entry point's first call on a device: after the library's
    other kernels have run (the workspace entry here), device memory still drops
    by the array's size at that first call, and by nothing at the next.  Runs
    first in this file, before any other call of the entry point in the process."""
    inp = _inputs(1000, 4, 4, [300, 0, 700], 71, dev)
    _call("hmx_gdn_chunk_fwd", *inp, 4, True)       # loads the prefill's code object
    _call("hmx_gdn_chunk_fwd", *inp, 4, True)       # and fills torch's cache for o / ht
    free0 = torch.cuda.mem_get_info()[0]
    _call("hmx_gdn_chunk_fwd_noalloc", *inp, 4, False)
    free1 = torch.cuda.mem_get_info()[0]
    _call("hmx_gdn_chunk_fwd_noalloc", *inp, 4, False)
    free2 = torch.cuda.mem_get_info()[0]
    mib = 1 << 20
    print(f"[no_alloc] free before / after the first call / after the second: "
          f"{free0 // mib} / {free1 // mib} / {free2 // mib} MiB", flush=True)
    assert free0 - free1 >= 64 * mib - 2 * mib
    assert abs(free1 - free2) <= 2 * mib


def test_noalloc_equals_workspace_entry(dev):
    cases = [  # (T, H, HKV, lengths, segment chunks): the second call is smaller
        (4096, 8, 4, [4096], 16),
        (1000, 4, 4, [300, 0, 700], 4),
    ]
    for i, (T, H, HKV, lens, sc) in enumerate(cases):
        inp = _inputs(T, H, HKV, lens, 70 + i, dev)
        print(f"[no_alloc] case {i}: T={T} H={H} HKV={HKV} lens={lens}", flush=True)
        o_ws, s_ws, nseg = _call("hmx_gdn_chunk_fwd", *inp, sc, True)
        o_na, s_na, _ = _call("hmx_gdn_chunk_fwd_noalloc", *inp, sc, False)
        assert nseg > len(lens), "the case must run several segments (workspace in use)"
        assert torch.equal(o_na, o_ws), f"case {i}: o differs"
        assert torch.equal(s_na, s_ws), f"case {i}: end states differ"
        # a weak-decay head takes the exact segment scan, which uses most of the workspace
        q, k, v, g, beta, h0, bounds = inp
        gw = F.logsigmoid(torch.randn(g.shape, device=dev) * 0.1 + 7.0)
        o_ws, s_ws, _ = _call("hmx_gdn_chunk_fwd", q, k, v, gw, beta, h0, bounds, sc, True)
        o_na, s_na, _ = _call("hmx_gdn_chunk_fwd_noalloc", q, k, v, gw, beta, h0, bounds, sc, False)
        assert torch.equal(o_na, o_ws) and torch.equal(s_na, s_ws), f"case {i}: exact scan differs"
