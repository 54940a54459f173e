"""The C-ABI library builds, loads without a GPU, and exports exactly what include/boa_hip.h declares."""
import ctypes
import os
import re
import subprocess

from conftest import REPO


def _declared():
    src = open(os.path.join(REPO, "include", "boa_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b((?:boa|rc|rcb)_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declaration():
    from boa_amd import _native

    lib = _native.load_cdll()  # binding every signature also resolves every symbol
    declared = _declared()
    assert len(declared) >= 25
    bound = {name for name, _, _ in _native.SIGNATURES}
    assert set(declared) == bound, (set(declared) ^ bound)
    for name in declared:
        assert hasattr(lib, name)
    out = subprocess.run(["nm", "-D", "--defined-only", _native.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T ((?:boa|rc|rcb)_[a-z0-9_]+)$", out, flags=re.M))
    assert set(declared) <= exported


def test_no_gpu_calls_fail_cleanly():
    import torch

    from boa_amd import _native

    if torch.cuda.is_available():
        return
    try:
        _native.lib()
    except RuntimeError as e:
        assert "GPU" in str(e)
    else:
        raise AssertionError("lib() must refuse to run without a GPU")


def test_weights_nbytes_matches_layout():
    from boa_amd import _native, weights

    lib = _native.load_cdll()
    for d, L in ((256, 8), (512, 16), (256, 1)):
        c = _native.ModelCfg(d, L, 256, 16, 4, 2, 0)
        assert lib.boa_weights_nbytes(ctypes.byref(c)) == 4 * weights.nfloats(weights.Cfg(d_model=d, n_layers=L))
    assert 4 * weights.nfloats(weights.Cfg()) == 31_688_704


def test_ctx_plan_bytes_host_only():
    """The context memory plan is host arithmetic: callable without a GPU, linear in lanes, exact for the
    per-lane state (checked against the state sizes written out here)."""
    from boa_amd import _native

    lib = _native.load_cdll()
    c = _native.ModelCfg(256, 8, 256, 16, 4, 2, 0)
    out = ctypes.c_int64(0)
    vals = []
    for lanes in (1, 2, 3):
        assert lib.boa_ctx_plan_bytes(ctypes.byref(c), _native.BOA_PREC_BF16X3, lanes, 64, ctypes.byref(out)) == 0
        vals.append(out.value)
    assert vals[2] - vals[1] == vals[1] - vals[0] > 0
    # per lane: state (8 layers x (3 x 512 conv history + 512 x 16 SSM) fp32) + 64 rows of workspace
    # (x, xz, xs, dbc, mm, logits fp32 + LN stats + split activations) + token, encoder and decoder state
    per_row = 4 * (256 + 1024 + 512 + 48 + 256 + 256) + 8 + 2 * 2 * 512
    per_lane = 8 * 4 * (3 * 512 + 512 * 16) + 64 * per_row + 4 + 32 + 32
    assert vals[1] - vals[0] == per_lane
    assert lib.boa_ctx_plan_bytes(ctypes.byref(c), 1, 0, 64, ctypes.byref(out)) == _native.BOA_ERR_ARG
