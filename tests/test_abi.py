"""CPU checks of the C ABI boundary: the library loads, exports every entry
point include/*.h declares, and the host wrappers raise the reference's
exception types before any launch (no GPU needed)."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

import hmx
from hmx import _lib

REPO = Path(__file__).resolve().parent.parent


def _declared_symbols():
    names = set()
    for h in (REPO / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(hmx_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    declared = _declared_symbols()
    assert declared, "no declarations found"
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    # and the Python binding knows every declared symbol's signature
    assert set(declared) <= set(_lib.SIGNATURES), set(declared) - set(_lib.SIGNATURES)


def test_abi_version_and_error_string():
    lib = _lib.load()
    assert lib.hmx_abi_version() == 13
    assert isinstance(lib.hmx_last_error(), bytes)


def test_invalid_args_map_to_status_codes():
    """A bad shape is rejected by the C side before any launch (no GPU touched)."""
    lib = _lib.load()
    rc = lib.hmx_gdn_recurrent_fwd(None, 0, None, 0, None, 0, 1, None, 0, None, 0, 0, None, None,
                                   0, None, 0, 0, None, None, 0, None, 1, 1, 1, 4, 4, 96, 128, 1.0,
                                   1, 0, None, None, None)
    assert rc == _lib.HMX_EUNSUPPORTED
    assert b"K=96" in lib.hmx_last_error()
    with pytest.raises(NotImplementedError):
        _lib.call("hmx_gdn_recurrent_fwd", None, 0, None, 0, None, 0, 1, None, 0, None, 0, 0, None,
                  None, 0, None, 0, 0, None, None, 0, None, 1, 1, 1, 4, 4, 96, 128, 1.0, 1, 0, None,
                  None, None)
    with pytest.raises(ValueError):
        _lib.call("hmx_gdn_gating", None, 0, None, 0, 0, None, 0, 0, 1, None, 0, None, None, 1,
                  -1, 4, 1.0, 20.0, None)


def test_wrappers_raise_reference_errors_on_cpu():
    q = torch.zeros(2, 3, 4, 128, dtype=torch.bfloat16)
    g = torch.zeros(2, 3, 4)
    cu = torch.tensor([0, 3, 6])
    with pytest.raises(ValueError, match="Batch size expected to be 1"):
        hmx.fused_recurrent_gated_delta_rule_gqa(q, q, q, g, g, cu_seqlens=cu)
    with pytest.raises(RuntimeError, match="GPU"):
        hmx.fused_recurrent_gated_delta_rule_gqa(q, q, q, g, g, initial_state=None,
                                                 inplace_final_state=False)


@pytest.mark.parametrize("cs", [[1, 4], [0, 5, 3], [0, 4, 9], []])
def test_bad_cu_seqlens_rejected(cs):
    """Sequence bounds are checked on the host before any kernel reads them:
    cu_seqlens must start at 0, not decrease and end within the tokens."""
    from hmx.ops.gdn import seq_bounds
    with pytest.raises(ValueError, match="cu_seqlens"):
        seq_bounds(torch.tensor(cs, dtype=torch.int32), 1, 8)


def test_good_cu_seqlens_bounds():
    from hmx.ops.gdn import seq_bounds
    assert seq_bounds(torch.tensor([0, 0, 3, 8]), 1, 8) == [(0, 0), (0, 3), (3, 8)]
    assert seq_bounds(None, 2, 5) == [(0, 5), (5, 10)]


def test_ssd_scan_rejects_mismatched_operands():
    """The SSD launcher checks every operand's token count (and z's shape) against
    x before launching."""
    from hmx.ops.ssd import _ssd_scan
    T, H, P, G, N = 16, 4, 64, 2, 128
    x = torch.zeros(T, H, P, dtype=torch.bfloat16)
    Bm = torch.zeros(T, G, N, dtype=torch.bfloat16)
    dt = torch.zeros(T, H)
    y = torch.zeros(T, H, P, dtype=torch.bfloat16)
    A = torch.zeros(H)
    bad = [dict(B=Bm[:8]), dict(dt=dt[:8]), dict(z=torch.zeros(T, H, 32, dtype=torch.bfloat16)),
           dict(bounds=[(0, T + 1)])]
    for kw in bad:
        args = dict(x=x, dt=dt, A=A, B=Bm, C=Bm, D=None, z=None, dt_bias=None, dt_softplus=False,
                    dt_limit=(0.0, float("inf")), bounds=[(0, T)], h0=None, y=y, want_final=False)
        args.update(kw)
        with pytest.raises(ValueError):
            _ssd_scan(**args)


def test_noalloc_entry_rejects_oversized_table():
    """hmx_gdn_chunk_fwd_noalloc refuses a segment table whose workspace exceeds its
    static array, before touching the GPU."""
    lib = _lib.load()
    H, N, nseg = 64, 1, 64          # 3 * 64 * 64 * 64 KiB = 768 MiB of workspace
    assert lib.hmx_gdn_chunk_workspace_bytes(nseg, N, H, 0) > (64 << 20)
    with pytest.raises(ValueError, match="static scratch"):
        _lib.call("hmx_gdn_chunk_fwd_noalloc", None, H * 128, None, H * 128, None, H * 128,
                  _lib.HMX_BF16, None, _lib.HMX_F32, None, _lib.HMX_F32, None, None, None, 0,
                  _lib.HMX_F32, None, None, None, nseg, N, H, H, 128, 128, 1.0, 1, 16, 60.0,
                  None, None, None)
