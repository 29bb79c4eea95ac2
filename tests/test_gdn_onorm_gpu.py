"""GPU parity: the GDN prefill with its output gated RMSNorm fused into the kernel
epilogue (o_norm_weight / o_norm_gate) against
  - the unfused pair: the same op, then hmx.rms_norm_gated on its bf16 output
    (both norm the same rounded o in fp32, so they agree to one unit in the last
    place), and
  - the fp64 oracles: oracle.gdn then oracle.norm.
Covers a single segment with ragged tails, multi-segment warm-up starts, varlen
with empty and 1-token sequences, no gate (plain RMSNorm), a strided gate (a view
of a fused projection) and a bf16 weight.
"""
import pytest
import torch
import torch.nn.functional as F

import hmx
from oracle import gdn as ref
from oracle import norm as nref
from util import half_ulp

pytestmark = pytest.mark.gpu


def _mk(T, H, HKV, seed, cu=None):
    g0 = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(1, T, H, 128, generator=g0), dim=-1).bfloat16()
    k = F.normalize(torch.randn(1, T, HKV, 128, generator=g0), dim=-1).bfloat16()
    v = torch.randn(1, T, HKV, 128, generator=g0).bfloat16()
    g = F.logsigmoid(torch.randn(1, T, H, generator=g0))
    beta = torch.sigmoid(torch.randn(1, T, H, generator=g0))
    z = (torch.randn(1, T, H, 128, generator=g0) * 1.5).bfloat16()
    w = torch.rand(128, generator=g0) + 0.5
    return q, k, v, g, beta, z, w


def _close_ulp(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    assert ((a - b).abs() <= 2 * half_ulp(b, torch.bfloat16) + 1e-30).all()
    assert (a == b).double().mean().item() >= 0.98


def _check_oracle(on, o_ref, z, w, eps):
    """The op's own bars, in pre-norm units: the norm multiplies element (t, h, j) by
    f = w_j silu(z_j) / rms(o_ref[t, h]) (~20 here), so (on - ref) / f is compared
    with the prefill tolerance (2e-2 beyond bf16 rounding of the normed value,
    1e-2 norm-wise relative)."""
    expect = nref.rms_norm_gated(o_ref, z, w, eps=eps)
    zz = z.double()
    f = (w.double() * zz * torch.sigmoid(zz)
         * torch.rsqrt((o_ref * o_ref).mean(-1, keepdim=True) + eps)).abs()
    err = ((on.double().cpu() - expect).abs() - half_ulp(expect, torch.bfloat16)).clamp(min=0)
    assert (err / f.clamp(min=1e-12)).max().item() <= 2e-2
    assert ((on.double().cpu() - expect).norm() / expect.norm()).item() <= 1e-2


def _run(dev, q, k, v, g, beta, z, w, cu=None, seg=None, eps=1e-5):
    d = [x.to(dev) for x in (q, k, v, g, beta)]
    kw = dict(output_final_state=True, use_qk_l2norm_in_kernel=True, _segment_chunks=seg,
              cu_seqlens=None if cu is None else cu.to(dev))
    o, s = hmx.chunk_gated_delta_rule_gqa(*d, **kw)
    on, s2 = hmx.chunk_gated_delta_rule_gqa(*d, **kw, o_norm_weight=w.to(dev),
                                            o_norm_gate=None if z is None else z.to(dev),
                                            o_norm_eps=eps)
    unf = hmx.rms_norm_gated(o, None if z is None else z.to(dev), w.to(dev), eps=eps)
    torch.cuda.synchronize()
    assert torch.equal(s, s2)        # the epilogue leaves the state alone
    return o, on, unf


@pytest.mark.parametrize("T,seg", [(200, None), (64 * 20 + 17, 3)])
def test_fused_norm_matches_unfused_and_oracle(dev, T, seg):
    q, k, v, g, beta, z, w = _mk(T, 4, 2, T)
    o, on, unf = _run(dev, q, k, v, g, beta, z, w, seg=seg)
    _close_ulp(on, unf)
    o_ref, _ = ref.chunk_gated_delta_rule_gqa(q, k, v, g, beta, use_qk_l2norm_in_kernel=True)
    _check_oracle(on, o_ref, z, w, 1e-5)


def test_fused_norm_varlen_and_plain(dev):
    lens = [130, 0, 64, 33, 1, 77]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    q, k, v, g, beta, z, w = _mk(int(cu[-1]), 4, 1, 21)
    for zz in (z, None):
        o, on, unf = _run(dev, q, k, v, g, beta, zz, w, cu=cu, eps=1e-6)
        _close_ulp(on, unf)


def test_fused_norm_strided_gate_bf16_weight(dev):
    T, H = 150, 2
    q, k, v, g, beta, _, w = _mk(T, H, 2, 22)
    proj = torch.randn(1, T, 3 * H * 128, generator=torch.Generator().manual_seed(5)).bfloat16()
    proj = proj.to(dev)
    z = proj[..., H * 128:2 * H * 128].view(1, T, H, 128)
    wb = w.bfloat16()
    d = [x.to(dev) for x in (q, k, v, g, beta)]
    o, _ = hmx.chunk_gated_delta_rule_gqa(*d, use_qk_l2norm_in_kernel=True)
    on, _ = hmx.chunk_gated_delta_rule_gqa(*d, use_qk_l2norm_in_kernel=True,
                                           o_norm_weight=wb.to(dev), o_norm_gate=z)
    unf = hmx.rms_norm_gated(o, z, wb.to(dev))
    torch.cuda.synchronize()
    _close_ulp(on, unf)


@pytest.mark.parametrize("K,V,lens", [(128, 128, [1] * 9), (128, 128, [3, 0, 5, 1, 4]),
                                      (64, 64, [2, 1, 3]), (128, 256, [1, 2])])
def test_decode_fused_norm(dev, K, V, lens):
    """The decode op with o_norm: fused in the kernel for V <= 128 (per-token
    cross-wave sums, multi-token sequences), a separate norm call for V = 256; both
    against decode-then-norm, with the pool updated identically."""
    H, HKV, slots = 4, 2, 16
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    n_tok, N = int(cu[-1]), len(lens)
    g0 = torch.Generator().manual_seed(K + V + n_tok)
    q = F.normalize(torch.randn(1, n_tok, H, K, generator=g0), dim=-1).bfloat16()
    k = F.normalize(torch.randn(1, n_tok, HKV, K, generator=g0), dim=-1).bfloat16()
    v = torch.randn(1, n_tok, HKV, V, generator=g0).bfloat16()
    g = F.logsigmoid(torch.randn(1, n_tok, H, generator=g0))
    beta = torch.sigmoid(torch.randn(1, n_tok, H, generator=g0))
    z = (torch.randn(1, n_tok, H, V, generator=g0) * 1.5).bfloat16()
    w = torch.rand(V, generator=g0) + 0.5
    pool = torch.randn(slots, H, K, V, generator=g0) * 0.02
    idx = torch.randperm(slots, generator=g0)[:N].to(torch.int32)
    d = [x.to(dev) for x in (q, k, v, g, beta)]
    kw = dict(inplace_final_state=True, cu_seqlens=cu.to(dev), ssm_state_indices=idx.to(dev),
              use_qk_l2norm_in_kernel=True)
    p1, p2 = pool.to(dev), pool.to(dev)
    o, _ = hmx.fused_recurrent_gated_delta_rule_gqa(*d, initial_state=p1, **kw)
    on, _ = hmx.fused_recurrent_gated_delta_rule_gqa(*d, initial_state=p2, **kw,
                                                     o_norm_weight=w.to(dev), o_norm_gate=z.to(dev))
    unf = hmx.rms_norm_gated(o, z.to(dev), w.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(p1, p2)
    _close_ulp(on, unf)
