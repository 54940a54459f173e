"""Pins the CPU baseline restatement (oracle/codec_ref.py) against the reference protocol of
codec.compress_CPU / decompress_CPU (codec.py:153-323): first byte stored raw, one coded symbol per later
position, finished lanes coding nothing more, the lane pool split not changing any word, and the round trip.

Each lane's words are compared with the whole-stream Q2 encoder of rc_oracle.c (``ora.encode_probs_q2``,
one call over the lane's own probability rows) rather than with the per-symbol coder calls codec_ref makes,
so a mistake in the step protocol (a coded first byte, a symbol coded past a lane's end, a skipped step, a
wrong row) changes the words.
"""
import numpy as np
import torch

from oracle import codec_ref, model_ref, ora, weights_ref


def _model(n_layers=2, seed=3):
    from boa_amd import weights as W

    return model_ref.RefModel(W.seeded_blob(W.Cfg(n_layers=n_layers), seed), weights_ref.Cfg(n_layers=n_layers))


def _step_probs(m, X, lens):
    """probs[b, t-1] = softmax(step logits) that code X[b, t], the lanes stepped together with their true
    previous byte (rows past a lane's end are unused)."""
    B, T = X.shape
    st = m.init_state(B)
    rows = []
    for t in range(1, T):
        logits = m.step(torch.from_numpy(X[:, t - 1].copy()), st)
        rows.append(torch.softmax(logits, dim=-1).to(torch.float32).numpy())
    return np.stack(rows, axis=1) if rows else np.zeros((B, 0, 256), np.float32)


def test_codec_ref_protocol_and_words():
    rng = np.random.default_rng(11)
    lens = [1, 37, 90, 64]                                   # ragged, with a lane that codes nothing
    chunks = [rng.integers(0, 256, L).astype(np.uint8) for L in lens]
    m = _model()
    words, fb, Ls, steps = codec_ref.compress_cpu(m, chunks, num_workers=1)
    assert Ls == lens and steps == max(lens) - 1
    assert fb == [int(c[0]) for c in chunks]                 # the first byte is stored raw, never coded
    assert len(words[0]) == 0                                # a one-byte lane codes no symbol at all
    X = np.zeros((len(lens), max(lens)), np.int64)
    for i, c in enumerate(chunks):
        X[i, :lens[i]] = c
    probs = _step_probs(_model(), X, lens)
    for i, L in enumerate(lens):
        exp = ora.encode_probs_q2(codec_ref.P, probs[i, :L - 1], X[i, 1:L].astype(np.int32))
        assert np.array_equal(words[i], exp), (i, len(words[i]), len(exp))
    # a different pool split codes every lane the same
    w3, _, _, _ = codec_ref.compress_cpu(_model(), chunks, num_workers=3)
    assert all(np.array_equal(a, b) for a, b in zip(words, w3))
    out, dsteps = codec_ref.decompress_cpu(_model(), words, lens, fb, num_workers=2)
    assert dsteps == max(lens) - 1
    for i, c in enumerate(chunks):
        assert out[i].dtype == np.uint8 and np.array_equal(out[i], c), i


def test_codec_ref_finished_lanes_are_masked():
    """A short lane's words do not depend on how long the other lanes are, and decoding a lane needs only
    its own words: lengths 5 and 60 coded together give the 5-byte lane the same words as coding it beside
    a 6-byte lane."""
    rng = np.random.default_rng(12)
    a = rng.integers(0, 256, 5).astype(np.uint8)
    b = rng.integers(0, 256, 60).astype(np.uint8)
    w_long, _, _, _ = codec_ref.compress_cpu(_model(), [a, b], num_workers=1)
    w_short, _, _, _ = codec_ref.compress_cpu(_model(), [a, b[:6]], num_workers=1)
    assert np.array_equal(w_long[0], w_short[0])
    out, _ = codec_ref.decompress_cpu(_model(), w_long, [5, 60], [int(a[0]), int(b[0])], num_workers=1)
    assert np.array_equal(out[0], a) and np.array_equal(out[1], b)


def test_codec_ref_step_cap():
    """max_steps bounds the timed sample (bench.py's cpu_baseline): the words are those of the capped
    prefix, and decoding the same prefix returns it."""
    rng = np.random.default_rng(13)
    chunks = [rng.integers(0, 256, 40).astype(np.uint8) for _ in range(3)]
    w, fb, Ls, steps = codec_ref.compress_cpu(_model(), chunks, num_workers=1, max_steps=9)
    assert steps == 9
    pre, _, _, _ = codec_ref.compress_cpu(_model(), [c[:10] for c in chunks], num_workers=1)
    assert all(np.array_equal(x, y) for x, y in zip(w, pre))
    out, _ = codec_ref.decompress_cpu(_model(), w, [10] * 3, fb, num_workers=1)
    assert all(np.array_equal(o, c[:10]) for o, c in zip(out, chunks))
