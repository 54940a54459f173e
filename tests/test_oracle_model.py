"""Pins the torch-CPU model restatement: a second formulation (teacher-forced with a naive sequential
scan), a float64 loop brute force, and closed forms."""
import numpy as np
import torch

from oracle import model_ref, weights_ref


def _blob(n_layers, seed=0):
    from boa_amd import weights as W

    return W.seeded_blob(W.Cfg(n_layers=n_layers), seed)


def test_step_equals_teacher_forced_forward():
    cfg = weights_ref.Cfg(n_layers=2)
    m = model_ref.RefModel(_blob(2), cfg)
    tok = torch.from_numpy(np.random.default_rng(0).integers(0, 256, (3, 20)))
    lf = m.forward(tok)
    st = m.init_state(3)
    ls = torch.stack([m.step(tok[:, t], st) for t in range(20)], 1)
    assert float((lf - ls).abs().max() / lf.abs().max()) < 2e-6


def test_float64_brute_force():
    cfg = weights_ref.Cfg(n_layers=1)
    blob = _blob(1, 2)
    m = model_ref.RefModel(blob, cfg)
    sd = weights_ref.unpack(blob, cfg)
    tok = np.random.default_rng(1).integers(0, 256, (2, 3))
    st, st64 = m.init_state(2), None
    for t in range(3):
        l32 = m.step(torch.from_numpy(tok[:, t]), st).numpy()
        l64, st64 = model_ref.numpy_step_f64(sd, cfg, tok[:, t], st64)
        assert np.abs(l32 - l64).max() / np.abs(l64).max() < 2e-6


def test_closed_forms():
    from boa_amd import weights as W

    cfg = W.Cfg(n_layers=2)
    sd = W.unpack(W.seeded_blob(cfg, 4).copy(), cfg)
    # all matrices zero -> logits are exactly head.2.bias
    for k, v in sd.items():
        if v.ndim >= 2:
            v[...] = 0.0
    m = model_ref.RefModel(W.pack(sd, cfg), weights_ref.Cfg(n_layers=2))
    out = m.forward(torch.randint(0, 256, (2, 5)))
    assert torch.equal(out, torch.from_numpy(sd["head.2.bias"]).expand_as(out))
    # LayerNorm of a constant row is its bias
    x = torch.full((1, 256), 3.5)
    b = torch.linspace(-1, 1, 256)
    assert torch.equal(torch.nn.functional.layer_norm(x, (256,), torch.ones(256), b, 1e-5), b.unsqueeze(0))


def test_large_A_gives_closed_form_state():
    """A_log = 30: exp(dt*A) underflows to 0, so after each step h = (dt*B)*x exactly (no memory).  dt, B and
    x are recomputed here from the weights by hand, which also pins the conv tap order (the oldest history
    value meets w[..., 0], the current input w[..., 3])."""
    import torch.nn.functional as F

    from boa_amd import weights as W

    cfg = W.Cfg(n_layers=1)
    sd = W.unpack(W.seeded_blob(cfg, 5).copy(), cfg)
    sd["blocks.0.mamba.A_log"][...] = 30.0
    m = model_ref.RefModel(W.pack(sd, cfg), weights_ref.Cfg(n_layers=1))
    g = {k: torch.from_numpy(np.array(v)) for k, v in sd.items()}
    tok = torch.tensor([3, 200])
    tok2 = torch.tensor([17, 5])
    st = m.init_state(2)
    m.step(tok, st)
    m.step(tok2, st)

    def xm_of(t):
        u = F.layer_norm(g["embedding.weight"][t], (256,), g["blocks.0.ln1.weight"], g["blocks.0.ln1.bias"], 1e-5)
        xz = u @ g["blocks.0.mamba.in_proj.weight"].T + g["blocks.0.mamba.in_proj.bias"]
        return xz[:, :512]

    w = g["blocks.0.mamba.conv1d.weight"][:, 0, :]
    x_prev, x_cur = xm_of(tok), xm_of(tok2)
    xc = g["blocks.0.mamba.conv1d.bias"] + w[:, 2] * x_prev + w[:, 3] * x_cur
    xs = xc * torch.sigmoid(xc)
    dbc = xs @ g["blocks.0.mamba.x_proj.weight"].T
    dr, B = dbc[:, :16], dbc[:, 16:32]
    dt = F.softplus(dr @ g["blocks.0.mamba.dt_proj.weight"].T + g["blocks.0.mamba.dt_proj.bias"])
    h_expected = (dt.unsqueeze(-1) * B.unsqueeze(1)) * xs.unsqueeze(-1)
    h = st[0][0]
    assert float((h - h_expected).abs().max() / h_expected.abs().max()) < 1e-5
