"""GPU model vs the torch-CPU fp32 oracle, and encoder/decoder logit identity on the GPU.

Tolerance (floating point): max |logits_gpu - logits_ref| <= 1e-4 * max |logits_ref| (
"logits match the reference's fp32 Mamba step within 1e-4 relative").
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import model_ref, weights_ref

pytestmark = pytest.mark.gpu

REL_TOL = 1e-4


GEMM_MATRICES = ("in_proj.weight", "x_proj.weight", "out_proj.weight", "ff.0.weight", "ff.2.weight",
                 "head.0.weight", "head.2.weight")


def bf16_round(a):
    """Round float32 values to bfloat16 (nearest even), returned as float32."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def _model(n_layers=2, seed=0, d=256, precision="bf16x3"):
    from boa_amd import weights as W

    import model as M

    cfg = W.Cfg(d_model=d, n_layers=n_layers)
    blob = W.seeded_blob(cfg, seed)
    m = M.BoaConstrictor(d_model=d, num_layers=n_layers, vocab_size=256).load_blob(blob)
    m.precision = precision
    ref_blob = blob
    if precision == "bf16w":  # the model's GEMM matrices are bfloat16: the oracle runs with the same values
        sd = W.unpack(blob.copy(), cfg)
        for k in sd:
            if k.endswith(GEMM_MATRICES):
                sd[k][...] = bf16_round(sd[k])
        ref_blob = W.pack(sd, cfg)
    ref = model_ref.RefModel(ref_blob, weights_ref.Cfg(d_model=d, n_layers=n_layers))
    return m, ref


def _rel(a, b):
    return float((a - b).abs().max() / b.abs().max())


@pytest.mark.parametrize("precision", ["f32", "bf16x3", "bf16w"])
@pytest.mark.parametrize("n_layers", [1, 8])
def test_step_logits_vs_oracle(gpu, n_layers, precision):
    m, ref = _model(n_layers, precision=precision)
    rng = np.random.default_rng(n_layers)
    B, T = 24, 12
    tok = torch.from_numpy(rng.integers(0, 256, (B, T)))
    inf = m.init_stream(max_len=T, batch_size=B)
    st = ref.init_state(B)
    for t in range(T):
        g = m.step(tok[:, t].cuda(), inf).cpu()
        r = ref.step(tok[:, t], st)
        err = _rel(g, r)
        print(f"t={t} rel_err={err:.3e}", flush=True)
        assert err <= REL_TOL, (t, err)


@pytest.mark.parametrize("precision", ["f32", "bf16x3", "bf16w"])
def test_forward_vs_oracle_and_step_identity(gpu, precision):
    m, ref = _model(2, precision=precision)
    rng = np.random.default_rng(5)
    B, T = 16, 150  # > tile length: several tiles, state carried between them
    tok = torch.from_numpy(rng.integers(0, 256, (B, T)))
    lf = m(tok.cuda())
    lr = ref.forward(tok)
    assert _rel(lf.cpu(), lr) <= REL_TOL
    # decoder path (one position per launch) must reproduce the encoder path's logits bit for bit
    inf = m.init_stream(max_len=T, batch_size=B)
    ls = torch.stack([m.step(tok[:, t].cuda(), inf) for t in range(T)], dim=1)
    assert torch.equal(ls, lf), float((ls - lf).abs().max())


@pytest.mark.parametrize("precision", ["f32", "bf16x3"])
def test_tile_length_independence(gpu, precision):
    import model as M

    m, _ = _model(2, precision=precision)
    rng = np.random.default_rng(6)
    tok = torch.from_numpy(rng.integers(0, 256, (8, 100))).cuda()
    outs = []
    for tl in (1, 7, 64):
        m.release_engines()
        eng = m.engine(8, tl)
        eng.reset(8)
        out = torch.empty((8, 100, 256), dtype=torch.float32, device="cuda")
        eng.forward(tok.to(torch.int32).contiguous(), out)
        outs.append(out)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    m.release_engines()
    assert M.DEFAULT_TILE_LEN >= 1


def test_quantiser_tables_bit_exact(gpu, ora):
    from boa_amd import _native as N

    m, _ = _model(1)
    rng = np.random.default_rng(8)
    tok = torch.from_numpy(rng.integers(0, 256, (32, 40))).cuda()
    logits = m(tok).reshape(-1, 256).contiguous()
    extra = torch.from_numpy(rng.normal(0, 30, (64, 256)).astype(np.float32)).cuda()
    logits = torch.cat([logits, extra, torch.zeros(1, 256, device="cuda")]).contiguous()
    for P in (16, 24):
        d_cdf = torch.empty((logits.shape[0], 257), dtype=torch.int32, device="cuda")
        N.check(gpu.boa_xq_cdf(N.ptr(logits), logits.shape[0], 256, P, N.ptr(d_cdf), N.stream_ptr()))
        got = d_cdf.cpu().numpy().view(np.uint32)
        ref = ora.xq_cdf(logits.cpu().numpy(), P)
        assert (got == ref).all()


def _dev_f32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def test_quantiser_tables_adversarial_rows(gpu, ora):
    """The XQ quantiser on rows no model emits: infinities, NaN (some or all entries), values whose differences
    overflow to -inf, all entries equal, one peak with every other entry far below it, differences at the
    smallest normal scale, and subnormal logits.  Every GPU table equals the oracle's and is a valid table."""
    from boa_amd import _native as N

    K = 256
    rng = np.random.default_rng(9)
    base = rng.normal(0, 3, K).astype(np.float32)
    rows = []
    for v in (np.inf, -np.inf, np.nan):
        r = base.copy(); r[17] = v; rows.append(r)
    r = base.copy(); r[::3] = np.nan; rows.append(r)
    rows.append(np.full(K, -np.inf, np.float32))
    rows.append(np.full(K, np.inf, np.float32))
    r = np.full(K, -3e38, np.float32); r[200] = 3e38; rows.append(r)
    r = np.where(rng.random(K) < 0.5, 3e38, -3e38).astype(np.float32); rows.append(r)
    rows.append(np.full(K, 7.25, np.float32))
    r = np.full(K, -87.5, np.float32); r[0] = 0.0; rows.append(r)
    r = np.full(K, -86.9, np.float32); r[255] = 0.0; rows.append(r)
    rows.append((rng.integers(-4, 5, K) * np.float32(1.2e-38)).astype(np.float32))
    rows.append((rng.integers(0, 1000, K) * np.float32(1e-45)).astype(np.float32))
    x = np.stack(rows).astype(np.float32)
    d_x = _dev_f32(x)
    for P in (16, 24):
        d_cdf = torch.empty((x.shape[0], K + 1), dtype=torch.int32, device="cuda")
        N.check(gpu.boa_xq_cdf(N.ptr(d_x), x.shape[0], K, P, N.ptr(d_cdf), N.stream_ptr()))
        got = d_cdf.cpu().numpy().view(np.uint32)
        ref = ora.xq_cdf(x, P)
        for i in range(x.shape[0]):
            assert (got[i] == ref[i]).all(), i
        c = got.astype(np.int64)
        assert (c[:, 0] == 0).all() and (c[:, -1] == 1 << P).all() and (np.diff(c, axis=1) >= 1).all()


def test_zero_weights_give_bias_only_logits(gpu):
    """Closed form: with every matrix zero, logits = head.2.bias whatever the input."""
    from boa_amd import weights as W

    import model as M

    cfg = W.Cfg(n_layers=2)
    blob = W.seeded_blob(cfg, 3)
    sd = W.unpack(blob.copy(), cfg)
    for k, v in sd.items():
        if v.ndim >= 2:
            v[...] = 0.0
    blob0 = W.pack(sd, cfg)
    m = M.BoaConstrictor(256, 2, 256).load_blob(blob0)
    out = m(torch.randint(0, 256, (4, 9)).cuda()).cpu()
    hb = torch.from_numpy(sd["head.2.bias"])
    assert torch.equal(out, hb.expand_as(out))


@pytest.mark.parametrize("precision", ["f32", "bf16x3"])
def test_gemm_tiling_independence_at_scale(gpu, precision):
    """4096 lanes: the step path runs the 128x128/BK64 and 64x64/BK128 GEMM configurations, the 8-position
    tile path the 128x128/BK32 one; logits must agree bit for bit (the decoder depends on it)."""
    m, _ = _model(1, precision=precision)
    B, T = 4096, 8
    tok = torch.randint(0, 256, (B, T), generator=torch.Generator().manual_seed(3)).cuda()
    m.release_engines()
    eng = m.engine(B, T)
    eng.reset(B)
    tiled = torch.empty((B, T, 256), dtype=torch.float32, device="cuda")
    eng.forward(tok.to(torch.int32).contiguous(), tiled)
    inf = m.init_stream(max_len=T, batch_size=B)
    for t in range(T):
        st = m.step(tok[:, t], inf)
        assert torch.equal(st, tiled[:, t]), (t, float((st - tiled[:, t]).abs().max()))
    m.release_engines()


def _stream_logits(m, tok, fused):
    """Step logits [B, T, V] from a fresh stream; fused=False builds the context with BOA_FUSED_STEP=0."""
    import os

    old = os.environ.get("BOA_FUSED_STEP")
    os.environ["BOA_FUSED_STEP"] = "1" if fused else "0"
    try:
        inf = m.init_stream(max_len=tok.shape[1], batch_size=tok.shape[0])
    finally:
        if old is None:
            del os.environ["BOA_FUSED_STEP"]
        else:
            os.environ["BOA_FUSED_STEP"] = old
    return torch.stack([m.step(tok[:, t], inf) for t in range(tok.shape[1])], dim=1)


@pytest.mark.parametrize("d,precision", [(256, "bf16x3"), (256, "bf16w"), (256, "f32"), (512, "bf16w"),
                                         (512, "bf16x3")])
def test_fused_step_matches_layer_kernels(gpu, d, precision):
    """The one-launch decompress step (d_model 256: 16 lanes per workgroup, activations in LDS, in each precision
    mode including fp32 MFMA; d_model 512: 32 lanes per workgroup, chunked, with per-lane scratch) against the
    per-layer step kernels: identical bits, including a partial last workgroup (37 lanes) and > 3 positions
    (the conv history ring wraps)."""
    m, ref = _model(8 if d == 256 else 2, seed=0 if d == 256 else 1, d=d, precision=precision)
    tok = torch.from_numpy(np.random.default_rng(11).integers(0, 256, (37, 9))).cuda()
    a = _stream_logits(m, tok, fused=True)
    b = _stream_logits(m, tok, fused=False)
    assert torch.equal(a, b), float((a - b).abs().max())
    lr = ref.forward(tok.cpu())
    assert _rel(a.cpu(), lr) <= REL_TOL


@pytest.mark.parametrize("precision", ["bf16w", "bf16x3"])
def test_d512_config4_shape_vs_oracle_and_identity(gpu, precision):
    """configs[4] shape (d_model 512, d_inner 1024, dt_rank 32), bf16 weights: logits vs the oracle with the
    same bf16-rounded weights, and the decode path (the fused d_model 512 step kernel) equal to the
    teacher-forced tile path bit for bit."""
    m, ref = _model(2, seed=1, d=512, precision=precision)
    rng = np.random.default_rng(21)
    B, T = 20, 70  # > one 64-position tile
    tok = torch.from_numpy(rng.integers(0, 256, (B, T)))
    lf = m(tok.cuda())
    lr = ref.forward(tok)
    err = _rel(lf.cpu(), lr)
    print(f"d512 {precision} rel_err={err:.3e}", flush=True)
    assert err <= REL_TOL
    inf = m.init_stream(max_len=T, batch_size=B)
    ls = torch.stack([m.step(tok[:, t].cuda(), inf) for t in range(T)], dim=1)
    assert torch.equal(ls, lf), float((ls - lf).abs().max())


def test_config4_model_16_layers_vs_oracle(gpu):
    """configs[4]'s model itself: d_model 512 x 16 layers, seed 1, bf16 weights.  Teacher-forced logits
    (compress path, > one 64-position tile) against the oracle with the same bf16-rounded weights, within
    the 1e-4 bar, and the decode path (step by step) bit-identical to them."""
    m, ref = _model(16, seed=1, d=512, precision="bf16w")
    rng = np.random.default_rng(41)
    B, T = 6, 70
    tok = torch.from_numpy(rng.integers(0, 256, (B, T)))
    lf = m(tok.cuda())
    lr = ref.forward(tok)
    err = _rel(lf.cpu(), lr)
    print(f"d512x16L bf16w rel_err={err:.3e}", flush=True)
    assert err <= REL_TOL
    inf = m.init_stream(max_len=T, batch_size=B)
    ls = torch.stack([m.step(tok[:, t].cuda(), inf) for t in range(T)], dim=1)
    assert torch.equal(ls, lf), float((ls - lf).abs().max())
