"""Pins the oracle's range coder and quantisers (CPU only).

Checks that do not restate the oracle's own code: hand-derived known answers, the independent big-integer
interval check, closed-form tables, code-length bounds and round trips.
"""
import json
import math
import os

import numpy as np
import pytest

from oracle import bigint_check

HERE = os.path.dirname(os.path.abspath(__file__))


def _uniform256():
    return np.array([[65536 * i for i in range(257)]], dtype=np.uint32)


def test_known_answers(ora):
    spec = json.load(open(os.path.join(HERE, "golden", "rc_known_answers.json")))
    for case in spec["cases"]:
        P = case["P"]
        syms = np.array(case["syms"], dtype=np.int32)
        if case["cdf"] == "uniform256":
            cdf = np.repeat(_uniform256(), len(syms), axis=0)
        elif len(case["cdf"]) == 0:
            cdf = np.zeros((0, 3), dtype=np.uint32)
        else:
            cdf = np.array(case["cdf"], dtype=np.uint32)
        words = ora.encode_tables(P, cdf, syms)
        assert [int(w) for w in words] == case["words"], case["name"]
        if len(syms):
            assert (ora.decode_tables(P, cdf, words) == syms).all(), case["name"]


def test_bigint_detects_mistakes():
    # the checker must reject a dropped word and flipped bits (a trailing extra word can still decode
    # correctly, so it is not a violation)
    steps = [(0, 32768), (32768, 32768)] * 100
    from oracle import ora

    cdf = np.array([[0, 32768, 65536]] * 200, dtype=np.uint32)
    syms = np.array([0, 1] * 100, dtype=np.int32)
    w = ora.encode_tables(16, cdf, syms)
    bigint_check.check(w, steps, 16)
    assert len(w) >= 3
    flip0 = w.copy(); flip0[0] ^= np.uint32(1 << 31)
    flip1 = w.copy(); flip1[1] ^= np.uint32(1 << 31)
    for bad in (w[:-1], flip0, flip1):
        with pytest.raises(AssertionError):
            bigint_check.check(bad, steps, 16)


@pytest.mark.parametrize("P", [16, 24])
def test_random_streams_bigint(ora, P):
    rng = np.random.default_rng(P)
    for trial in range(40):
        T = int(rng.integers(0, 400))
        K = int(rng.integers(2, 257))
        logits = rng.normal(0, 3 if trial % 2 else 12, (T, K)).astype(np.float32)
        cdf = ora.xq_cdf(logits, P)
        syms = rng.integers(0, K, T).astype(np.int32)
        words = ora.encode_tables(P, cdf, syms)
        steps = [(int(cdf[t, s]), int(cdf[t, s + 1] - cdf[t, s])) for t, s in enumerate(syms)]
        bigint_check.check(words, steps, P)
        assert (ora.decode_tables(P, cdf, words) == syms).all()
        # code length between the information content and it plus 64 bits and the per-step truncation loss
        bits = -sum(math.log2(f / (1 << P)) for _, f in steps)
        assert math.ceil(bits - 1e-9) <= 32 * len(words) < bits + 64 - T * math.log2(1 - 2.0 ** (P - 32)) + 1e-9


def test_carry_heavy_streams(ora):
    # tables concentrated near the top of the range force long runs of inverted (carry-pending) words
    P = 16
    rng = np.random.default_rng(5)
    for trial in range(30):
        T = 300
        cdf = np.zeros((T, 3), dtype=np.uint32)
        cdf[:, 1] = rng.integers(65000, 65535, T)
        cdf[:, 2] = 65536
        syms = (rng.random(T) < 0.97).astype(np.int32) ^ 1
        syms = np.where(rng.random(T) < 0.5, 0, 1).astype(np.int32) if trial % 3 == 0 else syms
        words = ora.encode_tables(P, cdf, syms)
        steps = [(int(cdf[t, s]), int(cdf[t, s + 1] - cdf[t, s])) for t, s in enumerate(syms)]
        bigint_check.check(words, steps, P)
        assert (ora.decode_tables(P, cdf, words) == syms).all()


def test_q2_closed_forms(ora):
    P = 24
    u = np.full((1, 256), 1 / 256, dtype=np.float32)
    assert (ora.q2_cdf(u, P) == _uniform256()).all()          # norm = 1 exactly: cdf[i] = i*(2^24-256)/256 + i
    z = np.zeros((1, 256), dtype=np.float32)                  # degenerate norm: uniform fallback
    assert (ora.q2_cdf(z, P) == _uniform256()).all()
    n = np.full((1, 256), np.nan, dtype=np.float32)
    assert (ora.q2_cdf(n, P) == _uniform256()).all()
    one = np.zeros((1, 4), dtype=np.float32)
    one[0, 2] = 1.0                                           # K=4: free = 2^24-4, point mass on symbol 2
    c = ora.q2_cdf(one, P)[0]
    assert list(c) == [0, 1, 2, (1 << 24) - 1, 1 << 24]


def test_xq_closed_forms(ora):
    P = 24
    flat = np.zeros((1, 256), dtype=np.float32)
    assert (ora.xq_cdf(flat, P) == _uniform256()).all()       # equal logits: f_i = 2^23 for all i
    peak = np.full((1, 256), -200.0, dtype=np.float32)
    peak[0, 0] = 0.0                                          # one symbol: f_0 = 2^23, others 0
    c = ora.xq_cdf(peak, P)[0].astype(np.int64)
    assert c[0] == 0 and all(c[i] == (1 << 24) - 256 + i for i in range(1, 257))
    nan = np.full((1, 256), np.nan, dtype=np.float32)
    assert (ora.xq_cdf(nan, P) == _uniform256()).all()


@pytest.mark.parametrize("P", [16, 24])
def test_table_invariants(ora, P):
    rng = np.random.default_rng(7)
    logits = rng.normal(0, 5, (500, 256)).astype(np.float32)
    for cdf in (ora.xq_cdf(logits, P),
                ora.q2_cdf(np.exp(logits - logits.max(1, keepdims=True)).astype(np.float32), P)):
        c = cdf.astype(np.int64)
        assert (c[:, 0] == 0).all() and (c[:, -1] == 1 << P).all()
        assert (np.diff(c, axis=1) >= 1).all()


def test_expf_accuracy(ora):
    x = np.concatenate([np.linspace(-87, 0, 200001), np.linspace(0, 88, 1001)]).astype(np.float32)
    y = ora.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert (np.abs(y - ref) <= 3 * ulp).all()
    assert ora.expf(np.array([0.0], np.float32))[0] == 1.0
    assert ora.expf(np.array([np.nan, -90.0], np.float32)).tolist() == [0.0, 0.0]


def test_q2_and_xq_round_trip_from_model_outputs(ora):
    rng = np.random.default_rng(11)
    T, K = 300, 256
    logits = rng.normal(0, 3, (T, K)).astype(np.float32)
    probs = np.exp(logits - logits.max(1, keepdims=True))
    probs = (probs / probs.sum(1, keepdims=True)).astype(np.float32)
    syms = np.array([rng.choice(K, p=p / p.sum()) for p in probs.astype(np.float64)], dtype=np.int32)
    w2 = ora.encode_probs_q2(24, probs, syms)
    assert (ora.decode_probs_q2(24, probs, w2) == syms).all()
    wx = ora.encode_logits_xq(24, logits, syms)
    assert (ora.decode_logits_xq(24, logits, wx) == syms).all()
    # both quantisers code within 0.5% of each other on the same distributions
    assert abs(len(w2) - len(wx)) <= max(2, 0.005 * len(w2))


def _tiny_tables(rng, K, T, P, kind):
    """Per-step tables [T, K+1] for the brute-force cases.  "mixed": random frequencies with one symbol at
    frequency 1 on odd steps (paths through it renormalise); "top": most of the mass on the last symbol, which
    pushes the interval's low end up against the carry boundary."""
    one = 1 << P
    cdf = np.zeros((T, K + 1), dtype=np.int64)
    for t in range(T):
        if kind == "mixed":
            f = rng.integers(1, 1 << 12, K).astype(np.float64)
            f = np.maximum(1, np.floor(f / f.sum() * (one - K))).astype(np.int64)
            if t % 2:
                f[t % K] = 1
        else:
            f = np.ones(K, dtype=np.int64)
            f[:-1] = rng.integers(1, 4, K - 1)
        f[-1] += one - f.sum()
        cdf[t, 1:] = np.cumsum(f)
    assert (cdf[:, -1] == one).all() and (np.diff(cdf, axis=1) >= 1).all()
    return cdf.astype(np.uint32)


def _all_sequences(K, T):
    """Every symbol sequence of length T over K symbols, in lexicographic order, [K^T, T]."""
    idx = np.arange(K ** T)
    return np.stack([(idx // K ** (T - 1 - t)) % K for t in range(T)], 1).astype(np.int32)


@pytest.mark.parametrize("K,T", [(2, 8), (3, 6), (4, 5), (2, 1), (4, 1)])
@pytest.mark.parametrize("P", [16, 24])
@pytest.mark.parametrize("kind", ["mixed", "top"])
def test_brute_force_tiny_alphabets(ora, K, T, P, kind):
    """All K^T sequences through one table set.  Each code lies in its final interval (big-integer check) and
    decodes; the codes, read as base-2^32 fractions, increase strictly in the sequences' lexicographic order
    (the sub-intervals are nested and ordered by the cdf); and the length obeys the closed-form bounds
    ceil(I) <= 32 n < I + 64 + T * -log2(1 - 2^(P-32)), with I = sum -log2(f/2^P) the information content and
    the last term the per-step truncation loss of scale = range >> P while range >= 2^32."""
    rng = np.random.default_rng(K * 100 + T * 10 + P + (kind == "top"))
    cdf = _tiny_tables(rng, K, T, P, kind)
    seqs = _all_sequences(K, T)
    loss = -math.log2(1 - 2.0 ** (P - 32))
    codes = []
    for syms in seqs:
        words = ora.encode_tables(P, cdf, syms)
        steps = [(int(cdf[t, s]), int(cdf[t, s + 1] - cdf[t, s])) for t, s in enumerate(syms)]
        bigint_check.check(words, steps, P)
        assert (ora.decode_tables(P, cdf, words) == syms).all()
        info = -sum(math.log2(f / (1 << P)) for _, f in steps)
        assert math.ceil(info - 1e-9) <= 32 * len(words) < info + 64 + T * loss + 1e-9, (syms, len(words))
        codes.append([int(w) for w in words])
    width = max(len(c) for c in codes)
    padded = [tuple(c + [0] * (width - len(c))) for c in codes]
    assert all(a < b for a, b in zip(padded, padded[1:]))


try:
    from hypothesis import HealthCheck, given, settings, strategies as st
except ImportError:  # pragma: no cover
    given = None


@pytest.mark.skipif(given is None, reason="needs hypothesis")
def test_hypothesis_round_trip(ora):
    """Generated tables and symbols (frequencies down to 1, cut points at the ends of [1, 2^P - 1], empty and
    one-symbol streams, one table per step): the words lie in the final interval (big-integer check), decode
    to the symbols, and obey the two-sided length bound."""

    @st.composite
    def case(draw):
        P = draw(st.sampled_from([16, 24]))
        K = draw(st.integers(2, 24))
        T = draw(st.integers(0, 24))
        cuts = st.sets(st.integers(1, (1 << P) - 1), min_size=K - 1, max_size=K - 1)
        shared = draw(st.booleans())
        rows = [sorted(draw(cuts))] * T if shared and T else [sorted(draw(cuts)) for _ in range(T)]
        syms = draw(st.lists(st.integers(0, K - 1), min_size=T, max_size=T))
        return P, K, rows, syms

    @settings(max_examples=400, deadline=None, database=None, suppress_health_check=[HealthCheck.too_slow])
    @given(case())
    def run(c):
        P, K, rows, syms = c
        T = len(syms)
        cdf = np.array([[0] + r + [1 << P] for r in rows], dtype=np.uint32).reshape(T, K + 1)
        s = np.array(syms, dtype=np.int32)
        words = ora.encode_tables(P, cdf, s)
        steps = [(int(cdf[t, v]), int(cdf[t, v + 1] - cdf[t, v])) for t, v in enumerate(syms)]
        bigint_check.check(words, steps, P)
        if T:
            assert (ora.decode_tables(P, cdf, words) == s).all()
            info = -sum(math.log2(f / (1 << P)) for _, f in steps)
            assert math.ceil(info - 1e-9) <= 32 * len(words) < info + 64 - T * math.log2(1 - 2.0 ** (P - 32)) + 1e-9
        else:
            assert len(words) == 0

    run()
