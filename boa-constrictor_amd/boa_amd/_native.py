"""ctypes binding of libboa_hip.so (C ABI declared in include/boa_hip.h).

torch is imported before the library is loaded, on purpose: torch ships its own HIP runtime
(``libamdhip64.so``, soname ``libamdhip64.so.7``); loading it first lets the dynamic linker resolve this
library's dependency on ``libamdhip64.so.7`` to the same runtime, so device pointers from torch tensors are
valid here.  ``load()`` verifies that with ``boa_is_device_pointer`` on a torch allocation.

There is no fallback: if the library is missing or no GPU is present, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libboa_hip.so")

BOA_OK = 0
BOA_ERR_ARG = 1
BOA_ERR_HIP = 2
BOA_ERR_OVERFLOW = 3
BOA_ERR_STATE = 4

BOA_PREC_F32 = 0      # fp32 MFMA
BOA_PREC_BF16X3 = 1   # split bf16 x3 products (fp32 weights)
BOA_PREC_BF16W = 2    # bf16 weights, split activations


class BoaError(RuntimeError):
    """Raised when a libboa_hip entry point returns a non-zero status."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class ModelCfg(ctypes.Structure):
    _fields_ = [
        ("d_model", ctypes.c_int32),
        ("n_layers", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("d_state", ctypes.c_int32),
        ("d_conv", ctypes.c_int32),
        ("expand", ctypes.c_int32),
        ("dt_rank", ctypes.c_int32),
    ]


class ProfEntry(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 32),
        ("launches", ctypes.c_int64),
        ("sampled", ctypes.c_int64),
        ("ms", ctypes.c_double),
        ("flops", ctypes.c_double),
        ("bytes", ctypes.c_double),
    ]


# (name, restype, argtypes); every declaration of include/boa_hip.h appears here
_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_U64 = ctypes.c_uint64
_F32 = ctypes.c_float
SIGNATURES = [
    ("boa_last_error", ctypes.c_char_p, []),
    ("boa_abi_version", ctypes.c_int, []),
    ("boa_is_device_pointer", ctypes.c_int, [_P]),
    ("boa_weights_nbytes", _I64, [ctypes.POINTER(ModelCfg)]),
    ("boa_ctx_create", ctypes.c_int, [ctypes.POINTER(ModelCfg), _P, _I64, ctypes.c_int, _I32, _I32, _P, ctypes.POINTER(_P)]),
    ("boa_ctx_destroy", ctypes.c_int, [_P]),
    ("boa_ctx_device_bytes", _I64, [_P]),
    ("boa_ctx_plan_bytes", ctypes.c_int, [ctypes.POINTER(ModelCfg), ctypes.c_int, _I32, _I32, ctypes.POINTER(_I64)]),
    ("boa_state_reset", ctypes.c_int, [_P, _I32]),
    ("boa_model_step", ctypes.c_int, [_P, _P, _I32, _P]),
    ("boa_model_forward", ctypes.c_int, [_P, _P, _I64, _I32, _I32, _P]),
    ("boa_profile", ctypes.c_int, [_P, ctypes.c_int]),
    ("boa_profile_read", ctypes.c_int, [_P, _P, _I32, ctypes.POINTER(_I32)]),
    ("boa_compress", ctypes.c_int, [_P, _P, _I64, _P, _I32, _I32, _P, _I64, _P]),
    ("boa_decompress", ctypes.c_int, [_P, _P, _I64, _P, _P, _P, _P, _I32, _I32, _P, _I64]),
    ("boa_xq_cdf", ctypes.c_int, [_P, _I64, _I32, _I32, _P, _P]),
    ("boa_compact", ctypes.c_int, [_P, _I64, _P, _I32, _P, _P, _I64, ctypes.POINTER(_I64), _P]),
    ("boa_compact_noalloc", ctypes.c_int, [_P, _I64, _P, _I32, _P, _P, _I64, ctypes.POINTER(_I64), _P]),
    ("rc_encode_tables", ctypes.c_int, [_I32, _I32, _P, _I32, _P, _I32, _I32, _P, _I64, _P, _P]),
    ("rc_decode_tables", ctypes.c_int, [_I32, _I32, _P, _I32, _P, _I64, _P, _I32, _I32, _P, _P]),
    ("rc_synth_tables", ctypes.c_int, [_U64, _F32, _I32, _I32, _I32, _I32, _I32, _P, _P, _P]),
    ("rcb_create", ctypes.c_int, [_I32, _I32, _I64, _P, ctypes.POINTER(_P)]),
    ("rcb_destroy", ctypes.c_int, [_P]),
    ("rcb_encode_step", ctypes.c_int, [_P, _P, _P, _P]),
    ("rcb_finalize", ctypes.c_int, [_P]),
    ("rcb_get_sizes", ctypes.c_int, [_P, _P]),
    ("rcb_get_words", ctypes.c_int, [_P, _P, _I64, ctypes.POINTER(_I64)]),
    ("rcb_load", ctypes.c_int, [_P, _P, _P]),
    ("rcb_init_decoder", ctypes.c_int, [_P]),
    ("rcb_decode_step", ctypes.c_int, [_P, _P, _P, _P]),
]

_lib = None
_lock = threading.Lock()


def _bind(lib):
    for name, res, args in SIGNATURES:
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


# The C ABI these signatures describe (boa_abi_version); 2: boa_decompress takes the payload's length.
ABI_VERSION = 2


def load_cdll():
    """Loads the shared library, checks its ABI version and binds every signature (no GPU needed)."""
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"libboa_hip.so not built ({LIB_PATH}); run __graft_entry__.build()")
    L = _bind(ctypes.CDLL(LIB_PATH))
    if L.boa_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libboa_hip.so has ABI {L.boa_abi_version()}, this package needs {ABI_VERSION}: "
                           "rebuild it (__graft_entry__.build())")
    return L


def lib():
    """The bound library, checked to share torch's HIP runtime.  Raises if no GPU is available."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not torch.cuda.is_available():
            raise RuntimeError("libboa_hip requires a ROCm GPU (torch.cuda.is_available() is False)")
        L = load_cdll()
        probe = torch.empty(16, dtype=torch.uint8, device="cuda")
        if L.boa_is_device_pointer(ctypes.c_void_p(probe.data_ptr())) != 1:
            raise RuntimeError("libboa_hip.so is bound to a different HIP runtime than torch "
                               "(load order: import torch before loading the library)")
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != BOA_OK:
        msg = _lib.boa_last_error().decode(errors="replace") if _lib is not None else "libboa_hip error"
        if rc == BOA_ERR_ARG:
            raise ValueError(msg)
        raise BoaError(rc, msg)


def ptr(t) -> ctypes.c_void_p:
    """Device (or host) address of a tensor / numpy array, or NULL for None."""
    if t is None:
        return ctypes.c_void_p(0)
    if isinstance(t, torch.Tensor):
        return ctypes.c_void_p(t.data_ptr())
    return ctypes.c_void_p(t.ctypes.data)


def stream_ptr(stream=None) -> ctypes.c_void_p:
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(int(s.cuda_stream))
