"""Flat weight blob of BoaBytePredictor: layout, packing from a state_dict, and the seeded generator.

Blob = little-endian float32 values, no header, tensors in PyTorch ``[out, in]`` order, in exactly the order
the reference converter writes them (portability_solved_cpp/convert_boa_weights.py:22-133, read back by
boa_gpu.hpp:173-186,422-437,526-555):

    embedding.weight [V, d]
    per block i:  ln1.{weight,bias} [d]; mamba.in_proj.{weight [2di, d], bias [2di] (zeros if absent)};
                  mamba.conv1d.{weight [di, 1, 4], bias [di]}; mamba.x_proj.weight [r + 2N, di];
                  mamba.dt_proj.{weight [di, r], bias [di]}; mamba.A_log [di, N]; mamba.D [di];
                  mamba.out_proj.{weight [d, di], bias [d] (zeros if absent)}; ln2.{weight,bias};
                  ff.0.{weight [4d, d], bias}; ff.2.{weight [d, 4d], bias}
    head.0.{weight [d, d], bias}; head.2.{weight [V, d], bias [V]}

The layout has to be the reference's so that its converted ``.bin`` files load unchanged.

``seeded_blob`` is this build's deterministic random initialisation (numpy ``default_rng(seed)``), standing
in for ``torch.manual_seed(seed); BoaConstrictor(...)`` whose RNG consumption inside mamba_ssm / mambapy
cannot be reproduced without those packages.  Distributions follow the public defaults: nn.Linear /
nn.Conv1d weight and bias U(+-1/sqrt(fan_in)), nn.Embedding N(0, 1), LayerNorm (1, 0), and Mamba's
dt_proj.weight U(+-r^-0.5), dt_proj.bias = softplus^-1(dt) with dt log-uniform in [1e-3, 0.1] floored at
1e-4, A_log = log(1..N) per channel, D = 1.
"""
from __future__ import annotations

import argparse
import math
from dataclasses import dataclass
from typing import Dict, List, Tuple

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
    def d_inner(self) -> int:
        return self.expand * self.d_model

    @property
    def dt_rank(self) -> int:
        return math.ceil(self.d_model / 16)


def layout(cfg: Cfg) -> List[Tuple[str, Tuple[int, ...]]]:
    d, di, N, r, V, K = cfg.d_model, cfg.d_inner, cfg.d_state, cfg.dt_rank, cfg.vocab, cfg.d_conv
    out: List[Tuple[str, Tuple[int, ...]]] = [("embedding.weight", (V, d))]
    for i in range(cfg.n_layers):
        p = f"blocks.{i}."
        m = p + "mamba."
        out += [
            (p + "ln1.weight", (d,)), (p + "ln1.bias", (d,)),
            (m + "in_proj.weight", (2 * di, d)), (m + "in_proj.bias", (2 * di,)),
            (m + "conv1d.weight", (di, 1, K)), (m + "conv1d.bias", (di,)),
            (m + "x_proj.weight", (r + 2 * N, di)),
            (m + "dt_proj.weight", (di, r)), (m + "dt_proj.bias", (di,)),
            (m + "A_log", (di, N)), (m + "D", (di,)),
            (m + "out_proj.weight", (d, di)), (m + "out_proj.bias", (d,)),
            (p + "ln2.weight", (d,)), (p + "ln2.bias", (d,)),
            (p + "ff.0.weight", (4 * d, d)), (p + "ff.0.bias", (4 * d,)),
            (p + "ff.2.weight", (d, 4 * d)), (p + "ff.2.bias", (d,)),
        ]
    out += [("head.0.weight", (d, d)), ("head.0.bias", (d,)), ("head.2.weight", (V, d)), ("head.2.bias", (V,))]
    return out


# biases the reference converter writes as zeros when the state_dict lacks them
# (convert_boa_weights.py:55-67, 95-104)
OPTIONAL_ZERO = ("mamba.in_proj.bias", "mamba.out_proj.bias")


def nfloats(cfg: Cfg) -> int:
    return sum(int(np.prod(s)) for _, s in layout(cfg))


def pack(state: Dict[str, object], cfg: Cfg) -> np.ndarray:
    """state_dict (torch tensors or arrays) -> flat float32 blob."""
    parts = []
    for name, shape in layout(cfg):
        if name in state:
            v = state[name]
            if hasattr(v, "detach"):
                v = v.detach().to("cpu").float().numpy()
            a = np.asarray(v, dtype=np.float32)
        elif name.endswith(OPTIONAL_ZERO):
            a = np.zeros(shape, dtype=np.float32)
        else:
            raise KeyError(f"state_dict lacks {name}")
        if a.size != int(np.prod(shape)):
            raise ValueError(f"{name}: expected shape {shape}, got {a.shape}")
        parts.append(a.reshape(-1))
    return np.ascontiguousarray(np.concatenate(parts), dtype=np.float32)


def unpack(blob: np.ndarray, cfg: Cfg) -> Dict[str, np.ndarray]:
    blob = np.asarray(blob, dtype=np.float32).reshape(-1)
    if blob.size != nfloats(cfg):
        raise ValueError(f"blob has {blob.size} floats, layout needs {nfloats(cfg)}")
    out, o = {}, 0
    for name, shape in layout(cfg):
        n = int(np.prod(shape))
        out[name] = blob[o:o + n].reshape(shape)
        o += n
    return out


def seeded_blob(cfg: Cfg, seed: int = 0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    d, di, N, r = cfg.d_model, cfg.d_inner, cfg.d_state, cfg.dt_rank

    def U(bound, shape):
        return rng.uniform(-bound, bound, size=shape).astype(np.float32)

    state: Dict[str, np.ndarray] = {}
    for name, shape in layout(cfg):
        key = name.split(".", 2)[-1] if name.startswith("blocks.") else name
        if name == "embedding.weight":
            v = rng.standard_normal(shape).astype(np.float32)
        elif key.endswith(("ln1.weight", "ln2.weight")):
            v = np.ones(shape, np.float32)
        elif key.endswith(("ln1.bias", "ln2.bias")) or key.endswith(OPTIONAL_ZERO):
            v = np.zeros(shape, np.float32)
        elif key.endswith("conv1d.weight") or key.endswith("conv1d.bias"):
            v = U(1.0 / math.sqrt(cfg.d_conv), shape)  # fan_in = (di / groups) * kernel = 4
        elif key.endswith("dt_proj.weight"):
            v = U(r ** -0.5, shape)
        elif key.endswith("dt_proj.bias"):
            dt = np.exp(rng.uniform(size=shape) * (math.log(0.1) - math.log(1e-3)) + math.log(1e-3))
            dt = np.maximum(dt, 1e-4)
            v = (dt + np.log(-np.expm1(-dt))).astype(np.float32)
        elif key.endswith("A_log"):
            v = np.log(np.tile(np.arange(1, N + 1, dtype=np.float32), (di, 1))).astype(np.float32)
        elif key == "mamba.D" or key.endswith(".D"):
            v = np.ones(shape, np.float32)
        else:  # Linear weights [out, in] and biases: U(+-1/sqrt(fan_in))
            fan_in = shape[1] if len(shape) == 2 else _bias_fan_in(name, cfg)
            v = U(1.0 / math.sqrt(fan_in), shape)
        state[name] = v
    return pack(state, cfg)


def _bias_fan_in(name: str, cfg: Cfg) -> int:
    d = cfg.d_model
    if name.endswith("ff.0.bias"):
        return d
    if name.endswith("ff.2.bias"):
        return 4 * d
    if name.endswith(("head.0.bias", "head.2.bias")):
        return d
    raise KeyError(name)


def write_bin(path: str, blob: np.ndarray) -> None:
    np.asarray(blob, dtype="<f4").tofile(path)


def read_bin(path: str, cfg: Cfg) -> np.ndarray:
    blob = np.fromfile(path, dtype="<f4")
    if blob.size != nfloats(cfg):
        raise ValueError(f"{path}: {blob.size} floats, expected {nfloats(cfg)} for {cfg}")
    return blob.astype(np.float32)


def infer_cfg(state: Dict[str, object]) -> Cfg:
    """Model shape from a state_dict (as main.py loads checkpoints into BoaConstrictor)."""
    V, d = tuple(state["embedding.weight"].shape)
    n = 0
    while f"blocks.{n}.ln1.weight" in state:
        n += 1
    N = int(state["blocks.0.mamba.A_log"].shape[1])
    K = int(state["blocks.0.mamba.conv1d.weight"].shape[-1])
    di = int(state["blocks.0.mamba.D"].shape[0])
    return Cfg(d_model=int(d), n_layers=n, vocab=int(V), d_state=N, d_conv=K, expand=di // int(d))


def convert(model_path: str, output_path: str) -> Cfg:
    """portability_solved_cpp/convert_boa_weights.py:16-135: .pt state_dict -> flat float32 .bin."""
    import torch

    sd = torch.load(model_path, map_location="cpu", weights_only=True)
    if isinstance(sd, dict) and "model_state_dict" in sd:
        sd = sd["model_state_dict"]
    cfg = infer_cfg(sd)
    write_bin(output_path, pack(sd, cfg))
    return cfg


def main(argv=None):
    ap = argparse.ArgumentParser(description="Convert a BoaConstrictor .pt state_dict to the flat .bin blob")
    ap.add_argument("--model", required=True)
    ap.add_argument("--output", required=True)
    a = ap.parse_args(argv)
    cfg = convert(a.model, a.output)
    print(f"wrote {a.output} ({cfg})")


if __name__ == "__main__":
    main()
