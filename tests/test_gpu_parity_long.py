"""Parity over long horizons and at configs[0]'s full size.

- configs[0] through the HIP path at its full size: 1 MiB of the order-1 Markov source, 64 chunks of 16384 B,
  d256 x 8 layers seed 0; byte-exact round trip (every chunk decodes 16383 dependent steps,
  codec.py:125-143, boa.cpp:562-569), and the compressed size within 0.5% of the reference protocol run on
  the CPU oracle (fp32 model -> torch.softmax -> Q2 at P = 24 -> coder) on a sample of 8 chunks x 2048 B.
- Teacher-forced logits of configs[2]'s model and records (d256 x 8 layers, seed 0) over 2048 positions, and
  of configs[4]'s model (d512 x 16 layers, bf16 weights, seed 1) over 512 positions, against the oracle at
  every position: the recurrent state's error must not grow past the bar deep into a chunk.
- configs[4]'s compressed size within 0.5% of the oracle pipeline's on 8 chunks x 1024 B (same bf16 weights).

Tolerance (floating point), per position t: max |logits_gpu[:, t] - logits_ref[:, t]| <= 1e-4 *
max |logits_ref[:, t]| (the north-star bar "logits match the reference's fp32 Mamba step within 1e-4
relative", applied position by position instead of over the whole tensor).
"""
import numpy as np
import pytest
import torch

from oracle import model_ref, weights_ref

pytestmark = pytest.mark.gpu

REL_TOL = 1e-4
GEMM_MATRICES = ("in_proj.weight", "x_proj.weight", "out_proj.weight", "ff.0.weight", "ff.2.weight",
                 "head.0.weight", "head.2.weight")


def _bf16_round(a):
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def _models(d, n_layers, seed, precision):
    from boa_amd import weights as W

    import model as M

    cfg = W.Cfg(d_model=d, n_layers=n_layers)
    blob = W.seeded_blob(cfg, seed)
    m = M.BoaConstrictor(d_model=d, num_layers=n_layers, vocab_size=256).load_blob(blob)
    m.precision = precision
    ref_blob = blob
    if precision == "bf16w":  # the GEMM matrices are bfloat16 on the GPU: the oracle gets the same values
        sd = W.unpack(blob.copy(), cfg)
        for k in sd:
            if k.endswith(GEMM_MATRICES):
                sd[k][...] = _bf16_round(sd[k])
        ref_blob = W.pack(sd, cfg)
    return m, model_ref.RefModel(ref_blob, weights_ref.Cfg(d_model=d, n_layers=n_layers))


def _per_position_error(g, r):
    """g, r: [B, T, V] -> per-position relative error [T] (max over lanes and symbols)."""
    num = (g - r).abs().amax(dim=(0, 2))
    den = r.abs().amax(dim=(0, 2))
    return (num / den).numpy()


def _check_horizon(name, g, r):
    err = _per_position_error(g, r)
    worst = int(err.argmax())
    q = [int(len(err) * f) - 1 for f in (0.25, 0.5, 0.75, 1.0)]
    print(f"{name}: worst position {worst} rel_err {err[worst]:.3e}; at positions {q}: "
          + " ".join(f"{err[i]:.2e}" for i in q), flush=True)
    assert err[worst] <= REL_TOL, (name, worst, float(err[worst]))


@pytest.mark.parametrize("precision", ["f32", "bf16x3"])
def test_config2_logits_over_2048_positions(gpu, precision):
    """configs[2]'s model (d256 x 8 layers, seed 0) on 8 of its chunks' first 2049 bytes (float32 records,
    seed 0): logits at positions 0..2047 against the oracle, position by position."""
    from bench import synth_records

    m, ref = _models(256, 8, 0, precision)
    lanes, T = 8, 2048
    data = synth_records(lanes * 16384, 0).reshape(lanes, 16384)[:, :T]
    tok = torch.from_numpy(data.astype(np.int64))
    g = m(tok.cuda()).cpu()
    r = ref.forward(tok)
    _check_horizon(f"configs[2] d256x8L {precision} T={T}", g, r)
    m.release_engines()


def test_config4_logits_over_512_positions(gpu):
    """configs[4]'s model (d512 x 16 layers, bf16 weights, seed 1) on 3 chunks of its int16 / float32
    records: logits at positions 0..511 against the oracle with the same bf16-rounded weights."""
    from bench import config4_data

    m, ref = _models(512, 16, 1, "bf16w")
    T = 512
    data = config4_data(3, 16384, T)
    tok = torch.from_numpy(np.ascontiguousarray(data).astype(np.int64))
    g = m(tok.cuda()).cpu()
    r = ref.forward(tok)
    _check_horizon(f"configs[4] d512x16L bf16w T={T}", g, r)
    m.release_engines()


@pytest.mark.parametrize("precision", ["bf16x3", "f32"])
def test_config0_full_size_round_trip_and_size(gpu, ora, precision):
    """configs[0] on the GPU: the whole 1 MiB Markov input as 64 chunks of 16384 B through boa_compress /
    boa_compact / boa_decompress (codec.compress_payload / decompress_payload), byte-exact; and on 8 chunks x
    their first 2048 B the GPU's compressed size within 0.5% of the oracle pipeline's."""
    import codec
    from bench import markov_bytes
    from oracle import ora as O

    m, ref = _models(256, 8, 0, precision)
    data = markov_bytes(1 << 20, seed=0)
    chunks = [data[i * 16384:(i + 1) * 16384] for i in range(64)]
    payload, nw, fb, Ls = codec.compress_payload(m, chunks)
    assert Ls == [16384] * 64 and fb == [int(c[0]) for c in chunks]
    out = codec.decompress_payload(m, payload, nw, Ls, fb)
    assert np.array_equal(out.reshape(-1), data)
    print(f"configs[0] {precision}: {len(data)} B -> {4 * int(nw.sum())} B of payload", flush=True)
    # compressed size against the reference protocol on a sample
    lanes, L = 8, 2048
    sample = [c[:L] for c in chunks[:lanes]]
    _, snw, _, _ = codec.compress_payload(m, sample)
    X = torch.from_numpy(np.stack(sample).astype(np.int64))
    probs = torch.softmax(ref.forward(X[:, :-1]), dim=-1).to(torch.float32).numpy()
    ref_words = sum(len(O.encode_probs_q2(24, probs[b], X[b, 1:].numpy().astype(np.int32))) for b in range(lanes))
    gpu_words = int(snw.sum())
    print(f"configs[0] sample {lanes}x{L}: gpu words {gpu_words}  oracle words {ref_words}", flush=True)
    assert abs(gpu_words - ref_words) <= 0.005 * ref_words
    m.release_engines()


def test_config4_compressed_size_vs_oracle(gpu, ora):
    """configs[4]'s model (d512 x 16 layers, bf16 weights, seed 1) on 8 chunks of its int16 / float32 records x
    their first 1024 B: byte-exact round trip, and the GPU's compressed size within 0.5% of the reference
    protocol run on the CPU oracle with the same bf16-rounded weights (fp32 model -> torch.softmax -> Q2 at
    P = 24 -> coder)."""
    import codec
    from bench import config4_data
    from oracle import ora as O

    m, ref = _models(512, 16, 1, "bf16w")
    lanes, L = 8, 1024
    data = np.ascontiguousarray(config4_data(lanes, 16384, L))
    chunks = [data[i] for i in range(lanes)]
    payload, nw, fb, Ls = codec.compress_payload(m, chunks)
    out = codec.decompress_payload(m, payload, nw, Ls, fb)
    assert np.array_equal(out, data)
    X = torch.from_numpy(data.astype(np.int64))
    probs = torch.softmax(ref.forward(X[:, :-1]), dim=-1).to(torch.float32).numpy()
    ref_words = sum(len(O.encode_probs_q2(24, probs[b], X[b, 1:].numpy().astype(np.int32))) for b in range(lanes))
    gpu_words = int(nw.sum())
    print(f"configs[4] sample {lanes}x{L}: gpu words {gpu_words}  oracle words {ref_words}", flush=True)
    assert abs(gpu_words - ref_words) <= 0.005 * ref_words
    m.release_engines()
