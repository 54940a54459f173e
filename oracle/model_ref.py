"""torch-CPU float32 restatement of BoaBytePredictor (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Follows the reference:
  - block:      model.py:57-65 / 75-81     y = LN1(x); y = mixer(y); y = LN2(y); y = FF(y); x + y
  - predictor:  model.py:109-117 / 124-131 embedding -> blocks -> head (Linear, ReLU, Linear)
  - mixer step: the mambapy MambaBlock.step the CPU path calls (model.py:49-50,78); its arithmetic:
        xz = in_proj(u); x, z = chunk(xz)
        x = conv1d(cat([inputs, x]))[..., d_conv-1]      (depthwise, taps oldest-first, + bias)
        x = silu(x); dr, B, C = split(x_proj(x)); dt = softplus(dt_proj(dr))
        h = exp(dt * A) * h + (dt * B) * x ;  y = h @ C + D * x ;  y * silu(z) ;  out_proj
    with A = -exp(A_log) and zero initial cache (model.py:68-73).  mambapy 1.2.0 itself is not installed,
    so this is a restatement of its published algorithm, not an import: parity with it is unpinned.
  - teacher-forced forward (model.py:97-101): ``forward`` runs the same blocks over all positions with a
    full-sequence causal conv and an explicit sequential scan -- a second formulation that must agree with
    running ``step`` position by position.

``numpy_step_f64`` is a float64 numpy brute force of the same step, written with explicit loops, used on
small inputs to pin this module.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, List

import numpy as np
import torch
import torch.nn.functional as F

from . import weights_ref


@dataclass
class Layer:
    ln1_w: torch.Tensor
    ln1_b: torch.Tensor
    in_w: torch.Tensor
    in_b: torch.Tensor
    conv_w: torch.Tensor  # [di, 1, K]
    conv_b: torch.Tensor
    x_w: torch.Tensor
    dt_w: torch.Tensor
    dt_b: torch.Tensor
    A: torch.Tensor       # -exp(A_log) [di, N]
    D: torch.Tensor
    out_w: torch.Tensor
    out_b: torch.Tensor
    ln2_w: torch.Tensor
    ln2_b: torch.Tensor
    ff1_w: torch.Tensor
    ff1_b: torch.Tensor
    ff2_w: torch.Tensor
    ff2_b: torch.Tensor


class RefModel:
    def __init__(self, blob: np.ndarray, cfg: "weights_ref.Cfg"):
        self.cfg = cfg
        sd = {k: torch.from_numpy(np.array(v, dtype=np.float32)) for k, v in weights_ref.unpack(blob, cfg).items()}
        self.emb = sd["embedding.weight"]
        self.layers: List[Layer] = []
        for i in range(cfg.n_layers):
            p, m = f"blocks.{i}.", f"blocks.{i}.mamba."
            self.layers.append(Layer(
                sd[p + "ln1.weight"], sd[p + "ln1.bias"], sd[m + "in_proj.weight"], sd[m + "in_proj.bias"],
                sd[m + "conv1d.weight"], sd[m + "conv1d.bias"], sd[m + "x_proj.weight"],
                sd[m + "dt_proj.weight"], sd[m + "dt_proj.bias"], -torch.exp(sd[m + "A_log"]), sd[m + "D"],
                sd[m + "out_proj.weight"], sd[m + "out_proj.bias"], sd[p + "ln2.weight"], sd[p + "ln2.bias"],
                sd[p + "ff.0.weight"], sd[p + "ff.0.bias"], sd[p + "ff.2.weight"], sd[p + "ff.2.bias"]))
        self.h1_w, self.h1_b = sd["head.0.weight"], sd["head.0.bias"]
        self.h2_w, self.h2_b = sd["head.2.weight"], sd["head.2.bias"]
        self.d, self.di, self.N, self.r = cfg.d_model, cfg.d_inner, cfg.d_state, cfg.dt_rank

    # ---- streaming --------------------------------------------------------------------------------
    def init_state(self, B: int):
        K = self.cfg.d_conv
        return [(torch.zeros(B, self.di, self.N), torch.zeros(B, self.di, K - 1)) for _ in self.layers]

    @torch.no_grad()
    def step(self, tok: torch.Tensor, state) -> torch.Tensor:
        x = F.embedding(tok.long(), self.emb)
        for i, w in enumerate(self.layers):
            h, inputs = state[i]
            u = F.layer_norm(x, (self.d,), w.ln1_w, w.ln1_b, 1e-5)
            xz = F.linear(u, w.in_w, w.in_b)
            xm, z = xz.chunk(2, dim=-1)
            window = torch.cat([inputs, xm.unsqueeze(2)], dim=2)                # [B, di, K]
            xc = F.conv1d(window, w.conv_w, w.conv_b, groups=self.di, padding=self.cfg.d_conv - 1)
            xc = xc[:, :, self.cfg.d_conv - 1]
            inputs = torch.cat([inputs[:, :, 1:], xm.unsqueeze(2)], dim=2)
            xs = F.silu(xc)
            dbc = F.linear(xs, w.x_w)
            dr, Bv, Cv = torch.split(dbc, [self.r, self.N, self.N], dim=-1)
            dt = F.softplus(F.linear(dr, w.dt_w, w.dt_b))
            dA = torch.exp(dt.unsqueeze(-1) * w.A)
            dB = dt.unsqueeze(-1) * Bv.unsqueeze(1)
            h = dA * h + dB * xs.unsqueeze(-1)
            y = (h @ Cv.unsqueeze(-1)).squeeze(2) + w.D * xs
            y = y * F.silu(z)
            m = F.linear(y, w.out_w, w.out_b)
            v = F.layer_norm(m, (self.d,), w.ln2_w, w.ln2_b, 1e-5)
            x = x + F.linear(F.gelu(F.linear(v, w.ff1_w, w.ff1_b)), w.ff2_w, w.ff2_b)
            state[i] = (h, inputs)
        return F.linear(F.relu(F.linear(x, self.h1_w, self.h1_b)), self.h2_w, self.h2_b)

    # ---- teacher forced ---------------------------------------------------------------------------
    @torch.no_grad()
    def forward(self, tokens: torch.Tensor) -> torch.Tensor:
        """tokens [B, T] -> logits [B, T, V], zero initial state."""
        B, T = tokens.shape
        K = self.cfg.d_conv
        x = F.embedding(tokens.long(), self.emb)                                # [B, T, d]
        for w in self.layers:
            u = F.layer_norm(x, (self.d,), w.ln1_w, w.ln1_b, 1e-5)
            xz = F.linear(u, w.in_w, w.in_b)
            xm, z = xz.chunk(2, dim=-1)
            xc = F.conv1d(xm.transpose(1, 2), w.conv_w, w.conv_b, groups=self.di, padding=K - 1)[:, :, :T]
            xs = F.silu(xc.transpose(1, 2))                                    # [B, T, di]
            dbc = F.linear(xs, w.x_w)
            dr, Bv, Cv = torch.split(dbc, [self.r, self.N, self.N], dim=-1)
            dt = F.softplus(F.linear(dr, w.dt_w, w.dt_b))                       # [B, T, di]
            h = torch.zeros(B, self.di, self.N)
            ys = []
            for t in range(T):                                                  # naive sequential scan
                dA = torch.exp(dt[:, t].unsqueeze(-1) * w.A)
                h = dA * h + (dt[:, t].unsqueeze(-1) * Bv[:, t].unsqueeze(1)) * xs[:, t].unsqueeze(-1)
                ys.append((h @ Cv[:, t].unsqueeze(-1)).squeeze(2) + w.D * xs[:, t])
            y = torch.stack(ys, dim=1) * F.silu(z)
            m = F.linear(y, w.out_w, w.out_b)
            v = F.layer_norm(m, (self.d,), w.ln2_w, w.ln2_b, 1e-5)
            x = x + F.linear(F.gelu(F.linear(v, w.ff1_w, w.ff1_b)), w.ff2_w, w.ff2_b)
        return F.linear(F.relu(F.linear(x, self.h1_w, self.h1_b)), self.h2_w, self.h2_b)


def numpy_step_f64(sd: Dict[str, np.ndarray], cfg, tok: np.ndarray, state=None):
    """float64 brute force of one step for all lanes, explicit loops (small inputs only).

    state: list per layer of (h [B, di, N], hist [B, di, K-1]); returns (logits [B, V], state)."""
    d, di, N, r, K = cfg.d_model, cfg.d_inner, cfg.d_state, cfg.dt_rank, cfg.d_conv
    B = tok.shape[0]
    g = {k: np.asarray(v, dtype=np.float64) for k, v in sd.items()}
    if state is None:
        state = [(np.zeros((B, di, N)), np.zeros((B, di, K - 1))) for _ in range(cfg.n_layers)]

    def ln(v, wt, bs):
        mu = v.mean()
        var = ((v - mu) ** 2).mean()
        return (v - mu) / math.sqrt(var + 1e-5) * wt + bs

    def softplus(v):
        return v if v > 20.0 else math.log1p(math.exp(v))

    def silu(v):
        return v / (1.0 + math.exp(-v))

    logits = np.zeros((B, cfg.vocab))
    new_state = [(s[0].copy(), s[1].copy()) for s in state]
    for b in range(B):
        x = g["embedding.weight"][int(tok[b])].copy()
        for i in range(cfg.n_layers):
            p, m = f"blocks.{i}.", f"blocks.{i}.mamba."
            h, hist = new_state[i]
            u = ln(x, g[p + "ln1.weight"], g[p + "ln1.bias"])
            xz = g[m + "in_proj.weight"] @ u + g[m + "in_proj.bias"]
            xm, z = xz[:di], xz[di:]
            xs = np.zeros(di)
            for c in range(di):
                taps = list(hist[b, c]) + [xm[c]]
                acc = g[m + "conv1d.bias"][c]
                for k in range(K):
                    acc += g[m + "conv1d.weight"][c, 0, k] * taps[k]
                xs[c] = silu(acc)
                hist[b, c] = taps[1:]
            dbc = g[m + "x_proj.weight"] @ xs
            dr, Bv, Cv = dbc[:r], dbc[r:r + N], dbc[r + N:]
            y = np.zeros(di)
            for c in range(di):
                dt = softplus(float(g[m + "dt_proj.weight"][c] @ dr) + g[m + "dt_proj.bias"][c])
                acc = 0.0
                for n in range(N):
                    A = -math.exp(g[m + "A_log"][c, n])
                    h[b, c, n] = math.exp(dt * A) * h[b, c, n] + dt * Bv[n] * xs[c]
                    acc += h[b, c, n] * Cv[n]
                y[c] = (acc + g[m + "D"][c] * xs[c]) * silu(z[c])
            mo = g[m + "out_proj.weight"] @ y + g[m + "out_proj.bias"]
            v = ln(mo, g[p + "ln2.weight"], g[p + "ln2.bias"])
            a1 = g[p + "ff.0.weight"] @ v + g[p + "ff.0.bias"]
            gl = np.array([0.5 * t * (1.0 + math.erf(t / math.sqrt(2.0))) for t in a1])
            x = x + g[p + "ff.2.weight"] @ gl + g[p + "ff.2.bias"]
        hh = np.maximum(g["head.0.weight"] @ x + g["head.0.bias"], 0.0)
        logits[b] = g["head.2.weight"] @ hh + g["head.2.bias"]
    return logits, new_state
