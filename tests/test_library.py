"""torch.library registrations: schemas, fake (meta) shapes, declared mutations and
the forward-only autograd rule.  Runs on the CPU with meta tensors (no kernels run)."""
import pytest
import torch

import hmx.library  # noqa: F401  (registers torch.ops.hmx.*)

M = torch.device("meta")


def test_ops_registered_with_mutations():
    for name in ("fused_gdn_gating", "chunk_gated_delta_rule_gqa",
                 "fused_recurrent_gated_delta_rule_gqa", "gka_chebyshev_gla_prefill",
                 "gka_chebyshev_gla_decode", "mamba_chunk_scan_combined",
                 "mamba_chunk_scan_combined_varlen", "selective_state_update",
                 "causal_conv1d_fn", "causal_conv1d_update", "rms_norm_gated"):
        assert hasattr(torch.ops.hmx, name), name
    def mutated(op):
        return {a.name for a in op.default._schema.arguments
                if a.alias_info is not None and a.alias_info.is_write}
    assert mutated(torch.ops.hmx.selective_state_update) == {"state", "out"}
    assert mutated(torch.ops.hmx.fused_recurrent_gated_delta_rule_gqa) == {"initial_state"}
    assert mutated(torch.ops.hmx.gka_chebyshev_gla_decode) == {"h_kk", "h_kv"}
    assert mutated(torch.ops.hmx.mamba_chunk_scan_combined_varlen) == {"out"}
    assert mutated(torch.ops.hmx.chunk_gated_delta_rule_gqa) == set()
    assert mutated(torch.ops.hmx.causal_conv1d_fn) == {"conv_states"}
    assert mutated(torch.ops.hmx.causal_conv1d_update) == {"conv_state"}
    assert mutated(torch.ops.hmx.rms_norm_gated) == set()


def test_fake_shapes_gdn_gka():
    B, T, H, HKV, D = 1, 70, 4, 2, 128
    q = torch.empty(B, T, H, D, device=M, dtype=torch.bfloat16)
    k = torch.empty(B, T, HKV, D, device=M, dtype=torch.bfloat16)
    g = torch.empty(B, T, H, device=M)
    cu = torch.empty(4, device=M, dtype=torch.int32)
    o, s = torch.ops.hmx.chunk_gated_delta_rule_gqa(q, k, k, g, g, 0.1, None, True, cu, True)
    assert o.shape == (B, T, H, D) and s.shape == (3, H, D, D) and s.dtype == torch.float32
    o, s = torch.ops.hmx.chunk_gated_delta_rule_gqa(q, k, k, g, g, 0.1, None, False, None, True)
    assert s.numel() == 0
    o, hkk, hkv = torch.ops.hmx.gka_chebyshev_gla_prefill(q, k, k, g, g, g, g, 0.1, 0.02, 0,
                                                          None, None, True, None)
    assert o.shape == (B, T, H, D) and hkk.numel() == 0 and hkv.shape == (1, H, D, D)


def test_fake_shapes_ssd():
    x = torch.empty(2, 50, 8, 64, device=M, dtype=torch.bfloat16)
    dt = torch.empty(2, 50, 8, device=M)
    Bm = torch.empty(2, 50, 2, 128, device=M, dtype=torch.bfloat16)
    A = torch.empty(8, device=M)
    y, fin = torch.ops.hmx.mamba_chunk_scan_combined(x, dt, A, Bm, Bm, 256, None, None, None, None,
                                                     None, True, 0.0, float("inf"))
    assert y.shape == x.shape and fin.shape == (2, 8, 64, 128)
    cu = torch.empty(6, device=M, dtype=torch.int32)
    st = torch.ops.hmx.mamba_chunk_scan_combined_varlen(
        x[0], dt[0], A, Bm[0], Bm[0], 256, cu, torch.empty_like(x[0]), None, None, None, None, True,
        0.0, float("inf"))
    assert st.shape == (5, 8, 64, 128)
    cc = torch.empty(9, device=M, dtype=torch.int32)
    st = torch.ops.hmx.mamba_chunk_scan_combined_varlen_chunks(
        x[0], dt[0], A, Bm[0], Bm[0], 256, cu, cc, cc[:8], torch.empty_like(x[0]), None, None,
        None, None, True, 0.0, float("inf"))
    assert st.shape == (8, 8, 64, 128)


def test_backward_is_refused():
    B, T, H, D = 1, 8, 2, 128
    q = torch.empty(B, T, H, D, device=M, dtype=torch.bfloat16, requires_grad=True)
    g = torch.empty(B, T, H, device=M)
    o, _ = torch.ops.hmx.chunk_gated_delta_rule_gqa(q, q, q, g, g, 0.1, None, False, None, True)
    with pytest.raises(NotImplementedError, match="forward-only"):
        o.sum().backward()


def test_fake_shapes_conv_norm():
    x = torch.empty(300, 96, device=M, dtype=torch.bfloat16)
    w = torch.empty(96, 4, device=M)
    pool = torch.empty(3, 3, 96, device=M, dtype=torch.bfloat16).transpose(1, 2)
    out = torch.ops.hmx.causal_conv1d_fn(x.t(), w, None, pool, None, None, None, "silu", -1)
    assert out.shape == (300, 96)                  # [total, dim] rows; the wrapper transposes
    o = torch.ops.hmx.causal_conv1d_update(x[:5], pool, w, None, "silu", None, -1)
    assert o.shape == (5, 96)
    z = torch.empty(2, 7, 4, 128, device=M, dtype=torch.bfloat16)
    assert torch.ops.hmx.rms_norm_gated(z, z, torch.empty(128, device=M), 1e-6, True).shape == \
        z.shape
