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
