"""Drop-in for the reference's ``model`` module: ``BoaConstrictor(d_model, num_layers, vocab_size, device)``.

Reference: model.py:5-134.  The module tree and parameter names are the reference's (``embedding``,
``blocks[i].{ln1, mamba.{in_proj, conv1d, x_proj, dt_proj, A_log, D, out_proj}, ln2, ff}``, ``head``), so
its checkpoints load with ``load_state_dict`` (main.py:262-280) and the weight converter's blob layout
applies.  Compute is not PyTorch: ``forward``, ``init_stream`` and ``step`` run the gfx950 kernels of
libboa_hip.so through its C ABI.  PyTorch holds the parameters and the I/O tensors only.

There is no CPU compute path.  The reference builds a mambapy model when no GPU is present
(model.py:14-15); here step/forward raise on CPU instead of silently falling back.
"""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np
import torch
import torch.nn as nn

from boa_amd import _native as _nat
from boa_amd import weights as _W

__all__ = ["BoaConstrictor", "BoaBytePredictor", "MambaBlock", "Mixer"]

DEFAULT_TILE_LEN = int(os.environ.get("BOA_TILE_LEN", "64"))

# GEMM arithmetic (include/boa_hip.h BOA_PREC_*): "f32" fp32 MFMA (default: the reference's fp32 arithmetic),
# "bf16x3" split-bfloat16 products (fp32 operands as bf16 hi + lo, three products: ~16 significant bits per
# operand, about twice as fast), "bf16w" bfloat16 weight matrices.  Compressor and decompressor must use the
# same mode.
PRECISIONS = {"f32": _nat.BOA_PREC_F32, "bf16x3": _nat.BOA_PREC_BF16X3, "bf16w": _nat.BOA_PREC_BF16W}
DEFAULT_PRECISION = os.environ.get("BOA_PRECISION", "f32")


class Mixer(nn.Module):
    """Parameters of one Mamba mixer, named as mamba_ssm.Mamba / mambapy.MambaBlock name them.

    Shapes (d = d_model, di = 2d, r = ceil(d/16), N = 16): in_proj [2di, d] (no bias), conv1d depthwise
    [di, 1, 4] + bias, x_proj [r + 2N, di] (no bias), dt_proj [di, r] + bias, A_log [di, N], D [di],
    out_proj [d, di] (no bias).  Initialisation follows the public Mamba defaults (dt_proj.weight
    U(+-r^-0.5), dt_proj.bias = softplus^-1(dt) with dt log-uniform in [1e-3, 0.1], A_log = log(1..N), D = 1).
    """

    def __init__(self, d_model: int, d_state: int = 16, d_conv: int = 4, expand: int = 2):
        super().__init__()
        di = expand * d_model
        r = math.ceil(d_model / 16)
        self.d_model, self.d_inner, self.d_state, self.d_conv, self.dt_rank = d_model, di, d_state, d_conv, r
        self.in_proj = nn.Linear(d_model, 2 * di, bias=False)
        self.conv1d = nn.Conv1d(di, di, kernel_size=d_conv, groups=di, padding=d_conv - 1, bias=True)
        self.x_proj = nn.Linear(di, r + 2 * d_state, bias=False)
        self.dt_proj = nn.Linear(r, di, bias=True)
        with torch.no_grad():
            nn.init.uniform_(self.dt_proj.weight, -r ** -0.5, r ** -0.5)
            dt = torch.exp(torch.rand(di) * (math.log(0.1) - math.log(1e-3)) + math.log(1e-3)).clamp(min=1e-4)
            self.dt_proj.bias.copy_(dt + torch.log(-torch.expm1(-dt)))
        self.A_log = nn.Parameter(torch.log(torch.arange(1, d_state + 1, dtype=torch.float32).repeat(di, 1)))
        self.D = nn.Parameter(torch.ones(di))
        self.out_proj = nn.Linear(di, d_model, bias=False)


class MambaBlock(nn.Module):
    """model.py:42-56: x + FF(LN2(Mamba(LN1(x)))), FF = Linear(d, 4d) -> GELU -> Linear(4d, d)."""

    def __init__(self, d_model: int):
        super().__init__()
        self.ln1 = nn.LayerNorm(d_model)
        self.mamba = Mixer(d_model)
        self.ln2 = nn.LayerNorm(d_model)
        self.ff = nn.Sequential(nn.Linear(d_model, 4 * d_model), nn.GELU(), nn.Linear(4 * d_model, d_model))


class _Engine:
    """One libboa_hip model context: device copy of the weights + recurrent state + workspace."""

    def __init__(self, blob: np.ndarray, cfg: _W.Cfg, max_lanes: int, tile_len: int,
                 precision: str = DEFAULT_PRECISION):
        self._lib = _nat.lib()
        self.cfg = cfg
        self.max_lanes = int(max_lanes)
        self.tile_len = int(tile_len)
        if precision not in PRECISIONS:
            raise ValueError(f"precision must be one of {sorted(PRECISIONS)}")
        self.precision = precision
        c = _nat.ModelCfg(cfg.d_model, cfg.n_layers, cfg.vocab, cfg.d_state, cfg.d_conv, cfg.expand, 0)
        h = ctypes.c_void_p()
        blob = np.ascontiguousarray(blob, dtype=np.float32)
        _nat.check(self._lib.boa_ctx_create(ctypes.byref(c), _nat.ptr(blob), blob.nbytes, PRECISIONS[precision],
                                            self.max_lanes, self.tile_len, _nat.stream_ptr(), ctypes.byref(h)))
        self.h = h

    def __del__(self):
        h = getattr(self, "h", None)
        if h is not None and h.value:
            self._lib.boa_ctx_destroy(h)
            self.h = None

    @property
    def device_bytes(self) -> int:
        return int(self._lib.boa_ctx_device_bytes(self.h))

    def reset(self, lanes: int):
        _nat.check(self._lib.boa_state_reset(self.h, int(lanes)))

    def step(self, tokens_i32: torch.Tensor, logits: torch.Tensor):
        _nat.check(self._lib.boa_model_step(self.h, _nat.ptr(tokens_i32), tokens_i32.numel(), _nat.ptr(logits)))

    def forward(self, tokens_i32: torch.Tensor, logits: torch.Tensor):
        B, L = tokens_i32.shape
        _nat.check(self._lib.boa_model_forward(self.h, _nat.ptr(tokens_i32), tokens_i32.stride(0), B, L,
                                               _nat.ptr(logits)))


class _Stream:
    """Streaming state returned by ``init_stream``: its own context, so several streams can coexist."""

    def __init__(self, engine: _Engine, batch_size: int, max_len: int):
        self.engine = engine
        self.batch_size = batch_size
        self.max_len = max_len
        self.seqlen_offset = 0


class BoaBytePredictor(nn.Module):
    """model.py:83-131: embedding -> blocks -> head (Linear-ReLU-Linear) predicting the next byte."""

    def __init__(self, d_model=256, num_layers=4, vocab_size=256):
        super().__init__()
        self.embedding = nn.Embedding(vocab_size, d_model)
        self.blocks = nn.ModuleList([MambaBlock(d_model) for _ in range(num_layers)])
        self.head = nn.Sequential(nn.Linear(d_model, d_model), nn.ReLU(), nn.Linear(d_model, vocab_size))
        self._engines = {}
        self.precision = DEFAULT_PRECISION

    # ---- weights ---------------------------------------------------------------------------------
    @property
    def cfg(self) -> _W.Cfg:
        return _W.Cfg(d_model=self.embedding.embedding_dim, n_layers=len(self.blocks),
                      vocab=self.embedding.num_embeddings)

    def weight_blob(self) -> np.ndarray:
        """Flat float32 blob in convert_boa_weights.py order (see boa_amd.weights)."""
        return _W.pack(self.state_dict(), self.cfg)

    def load_blob(self, blob: np.ndarray) -> "BoaBytePredictor":
        sd = {k: torch.from_numpy(np.array(v)) for k, v in _W.unpack(blob, self.cfg).items()}
        missing = [k for k in self.state_dict() if k not in sd]
        if missing:
            raise KeyError(f"blob lacks {missing}")
        self.load_state_dict({k: sd[k] for k in self.state_dict()}, strict=True)
        return self

    def _weights_key(self):
        return tuple((p.data_ptr(), p._version) for p in self.parameters())

    def _require_gpu(self):
        if not torch.cuda.is_available():
            raise RuntimeError("BoaConstrictor compute runs on the ROCm GPU only (no GPU visible)")

    def engine(self, max_lanes: int, tile_len: int = DEFAULT_TILE_LEN) -> _Engine:
        """Cached context with capacity for max_lanes x tile_len rows (rebuilt when weights change)."""
        self._require_gpu()
        # the context runs on the stream that is current when it is created; a caller on another stream gets
        # its own context, so its input copies and the kernels stay ordered on one stream
        key = (self._weights_key(), self.precision, int(torch.cuda.current_stream().cuda_stream))
        e = self._engines.get("codec")
        if e is not None and e[0] == key and e[1].max_lanes >= max_lanes and e[1].tile_len >= tile_len:
            return e[1]
        self._engines.pop("codec", None)
        eng = _Engine(self.weight_blob(), self.cfg, max_lanes, tile_len, self.precision)
        self._engines["codec"] = (key, eng)
        return eng

    def release_engines(self):
        self._engines.clear()

    def plan_wave_lanes(self, n_chunks: int, chunk_len: int, cap: int = 65536) -> int:
        """Chunks per wave sized from free device memory, as auto_size_params does (boa.cpp:103-150): the
        most lanes (at most n_chunks and cap) whose context (boa_ctx_plan_bytes, exact) plus the wave's own
        buffers (input bytes, pitched words, payload, output bytes: 9 B per position and lane) fit in 90% of
        the memory that is free, counting this model's cached context and torch's cached blocks as free."""
        self._require_gpu()
        lib = _nat.lib()
        cfg = self.cfg
        c = _nat.ModelCfg(cfg.d_model, cfg.n_layers, cfg.vocab, cfg.d_state, cfg.d_conv, cfg.expand, 0)
        prec = PRECISIONS[self.precision]
        tile = int(min(DEFAULT_TILE_LEN, max(chunk_len - 1, 1)))
        free, _total = torch.cuda.mem_get_info()
        e = self._engines.get("codec")
        free += (e[1].device_bytes if e is not None else 0)
        free += torch.cuda.memory_reserved() - torch.cuda.memory_allocated()
        budget = 0.9 * free

        def need(lanes: int) -> float:
            b = ctypes.c_int64(0)
            _nat.check(lib.boa_ctx_plan_bytes(ctypes.byref(c), prec, lanes, tile, ctypes.byref(b)))
            return float(b.value) + lanes * (9.0 * chunk_len + 80.0)

        lo, hi = 1, max(1, min(int(n_chunks), int(cap)))
        if need(hi) <= budget:
            return hi
        while lo < hi:  # largest lanes with need(lanes) <= budget (at least 1)
            mid = (lo + hi + 1) // 2
            if need(mid) <= budget:
                lo = mid
            else:
                hi = mid - 1
        return lo

    # ---- reference API ----------------------------------------------------------------------------
    @torch.inference_mode()
    def forward(self, x, inference_params=None):
        """Teacher-forced logits [B, L, V] for byte tensor x [B, L] (model.py:97-101).

        With ``inference_params`` from ``init_stream`` the positions continue that stream's state and
        advance it; otherwise the state starts from zero."""
        self._require_gpu()
        if x.ndim == 1:
            x = x.unsqueeze(0)
        B, L = x.shape
        tok = x.to("cuda", dtype=torch.int32).contiguous()
        out = torch.empty((B, L, self.embedding.num_embeddings), dtype=torch.float32, device="cuda")
        if isinstance(inference_params, _Stream):
            if B != inference_params.batch_size:
                raise ValueError("batch size differs from the stream's")
            inference_params.engine.forward(tok, out)
            inference_params.seqlen_offset += L
            return out
        eng = self.engine(B, min(DEFAULT_TILE_LEN, max(L, 1)))
        eng.reset(B)
        if L:
            eng.forward(tok, out)
        return out

    @torch.inference_mode()
    def init_stream(self, max_len: int, batch_size: int = 1, device=None, dtype=None):
        """model.py:103-106 / 120-123: fresh (zero) recurrent state for batch_size lanes."""
        self._require_gpu()
        eng = _Engine(self.weight_blob(), self.cfg, batch_size, 1, self.precision)
        eng.reset(batch_size)
        return _Stream(eng, batch_size, max_len)

    @torch.inference_mode()
    def step(self, byte_t, inf) -> torch.Tensor:
        """model.py:108-117 / 125-131: one byte per lane in, next-byte logits [B, V] out; advances state."""
        if not isinstance(inf, _Stream):
            raise TypeError("step() needs the state returned by init_stream()")
        tok = byte_t.reshape(-1).to("cuda", dtype=torch.int32).contiguous()
        if tok.numel() != inf.batch_size:
            raise ValueError(f"expected {inf.batch_size} tokens, got {tok.numel()}")
        out = torch.empty((inf.batch_size, self.embedding.num_embeddings), dtype=torch.float32, device="cuda")
        inf.engine.step(tok, out)
        inf.seqlen_offset += 1
        return out


def BoaConstrictor(d_model=256, num_layers=4, vocab_size=256, device="cuda"):
    """model.py:5-134.  ``device`` is accepted for signature compatibility; parameters are created on the
    CPU (as the reference's modules are) and moved by ``.to(device)``; compute always runs on the GPU."""
    return BoaBytePredictor(d_model=d_model, num_layers=num_layers, vocab_size=vocab_size)
