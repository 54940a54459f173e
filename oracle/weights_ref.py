"""Weight-blob layout restated from the reference converter (TEST INFRASTRUCTURE ONLY).

portability_solved_cpp/convert_boa_weights.py:22-133 writes, as float32, in this order: embedding; per
block ln1.{w,b}, in_proj.{w,b(zeros if absent)}, conv1d.{w,b}, x_proj.w, dt_proj.{w,b}, A_log, D,
out_proj.{w,b(zeros if absent)}, ln2.{w,b}, ff.0.{w,b}, ff.2.{w,b}; then head.0.{w,b}, head.2.{w,b}.
boa_gpu.hpp:173-186,422-437,526-555 reads the same order.  Kept separate from the product's
boa_amd/weights.py so that a layout mistake there fails the tests.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Cfg:
    d_model: int = 256
    n_layers: int = 8
    vocab: int = 256
    d_state: int = 16
    d_conv: int = 4
    expand: int = 2

    @property
    def d_inner(self):
        return self.expand * self.d_model

    @property
    def dt_rank(self):
        return math.ceil(self.d_model / 16)


def entries(cfg: Cfg):
    d, di, N, r, V, K = cfg.d_model, cfg.d_inner, cfg.d_state, cfg.dt_rank, cfg.vocab, cfg.d_conv
    yield "embedding.weight", (V, d)
    for i in range(cfg.n_layers):
        b, m = f"blocks.{i}.", f"blocks.{i}.mamba."
        yield b + "ln1.weight", (d,)
        yield b + "ln1.bias", (d,)
        yield m + "in_proj.weight", (2 * di, d)
        yield m + "in_proj.bias", (2 * di,)
        yield m + "conv1d.weight", (di, 1, K)
        yield m + "conv1d.bias", (di,)
        yield m + "x_proj.weight", (r + 2 * N, di)
        yield m + "dt_proj.weight", (di, r)
        yield m + "dt_proj.bias", (di,)
        yield m + "A_log", (di, N)
        yield m + "D", (di,)
        yield m + "out_proj.weight", (d, di)
        yield m + "out_proj.bias", (d,)
        yield b + "ln2.weight", (d,)
        yield b + "ln2.bias", (d,)
        yield b + "ff.0.weight", (4 * d, d)
        yield b + "ff.0.bias", (4 * d,)
        yield b + "ff.2.weight", (d, 4 * d)
        yield b + "ff.2.bias", (d,)
    yield "head.0.weight", (d, d)
    yield "head.0.bias", (d,)
    yield "head.2.weight", (V, d)
    yield "head.2.bias", (V,)


def unpack(blob, cfg: Cfg):
    blob = np.asarray(blob, dtype=np.float32).reshape(-1)
    out, o = {}, 0
    for name, shape in entries(cfg):
        n = int(np.prod(shape))
        out[name] = blob[o:o + n].reshape(shape)
        o += n
    if o != blob.size:
        raise ValueError(f"blob has {blob.size} floats, layout consumes {o}")
    return out
