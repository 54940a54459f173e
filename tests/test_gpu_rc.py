"""GPU range coder vs the oracle: bit-exact words on identical CDF tables, drop-in RangeCoderBatch parity."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import bigint_check

pytestmark = pytest.mark.gpu


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _sample(cdf, rng, P):
    # symbol with cdf[s] <= u < cdf[s+1] for a uniform u in [0, 2^P)
    u = rng.integers(0, 1 << P, cdf.shape[:-1])
    return (np.sum(cdf[..., 1:] <= u[..., None], axis=-1)).astype(np.int64)


def _encode_gpu(lib, P, cb, tables, syms, pitch):
    from boa_amd import _native as N

    S, T, K = tables.shape
    d_cdf = _dev(tables)
    d_syms = _dev(syms.astype(np.uint8))
    d_words = torch.zeros((S, pitch), dtype=torch.int32, device="cuda")
    d_n = torch.zeros(S, dtype=torch.int32, device="cuda")
    N.check(lib.rc_encode_tables(P, cb, N.ptr(d_cdf), K, N.ptr(d_syms), S, T, N.ptr(d_words), pitch, N.ptr(d_n),
                                 N.stream_ptr()))
    torch.cuda.synchronize()
    return d_cdf, d_words, d_n


# T = 256 with K = 256 takes the throughput kernels (the block-pipelined encoder; the decoder with eight streams
# per wave for 2-byte tables at P = 16 and T divisible by 8, four streams per wave otherwise, as T = 260);
# T = 257 and K < 256 the one-stream-per-wave ones.  S = 45 leaves part of the last wave without a stream.
@pytest.mark.parametrize("P,cb,K,T", [(16, 2, 256, 257), (16, 4, 256, 257), (24, 4, 256, 257), (16, 2, 100, 257),
                                      (24, 4, 7, 257), (16, 2, 256, 256), (16, 4, 256, 256), (24, 4, 256, 256),
                                      (16, 2, 256, 260)])
def test_tables_bit_exact(gpu, ora, P, cb, K, T):
    from boa_amd import _native as N

    rng = np.random.default_rng(P * 1000 + cb * 100 + K + T)
    S = 45
    logits = rng.normal(0, 3, (S, T, K)).astype(np.float32)
    cdf = ora.xq_cdf(logits, P)
    syms = _sample(cdf, rng, P)
    tables = cdf[..., :K].astype(np.uint16 if cb == 2 else np.uint32)
    pitch = T + 8
    d_cdf, d_words, d_n = _encode_gpu(gpu, P, cb, tables, syms, pitch)
    words = d_words.cpu().numpy().view(np.uint32)
    nw = d_n.cpu().numpy()
    for s in range(S):
        ref = ora.encode_tables(P, cdf[s], syms[s])
        assert nw[s] == len(ref), s
        assert (words[s, :nw[s]] == ref).all(), s
    d_out = torch.zeros((S, T), dtype=torch.uint8, device="cuda")
    N.check(gpu.rc_decode_tables(P, cb, N.ptr(d_cdf), K, N.ptr(d_words), pitch, N.ptr(d_n), S, T, N.ptr(d_out),
                                 N.stream_ptr()))
    assert (d_out.cpu().numpy() == syms).all()


def _zero_runs(cdf, rng, P):
    """The same tables with about a third of the symbols (never the last) at frequency 0, their mass moved to
    the last symbol: runs of equal cdf entries, still below 2^P."""
    freq = np.diff(cdf.astype(np.int64), axis=-1)
    drop = rng.random(freq.shape) < 0.35
    drop[..., -1] = False
    freq[..., -1] += np.where(drop, freq, 0).sum(-1)
    freq[drop] = 0
    out = np.zeros_like(cdf, dtype=np.int64)
    out[..., 1:] = np.cumsum(freq, axis=-1)
    assert (out[..., -1] == 1 << P).all()
    return out.astype(np.uint32)


@pytest.mark.parametrize("P,cb,T,zero", [(16, 2, 256, False), (24, 4, 256, False), (16, 2, 255, False),
                                         (16, 2, 256, True), (16, 2, 260, True)])
def test_decode_tables_arbitrary_words(gpu, ora, P, cb, T, zero):
    """Decoding words that no encoder wrote (random values, random stream lengths 0 .. 2 T, including 0, 1 and
    2 words) on valid tables: every symbol equals the oracle decoder's, which exercises the target division, the
    symbol search at arbitrary targets and the reading of words past the end of a stream (zeros).  With zero,
    the tables hold runs of zero-frequency symbols (equal entries) that the search must step over."""
    from boa_amd import _native as N

    rng = np.random.default_rng(P + T + zero)
    S, K = 45, 256
    cdf = ora.xq_cdf(rng.normal(0, 3, (S, T, K)).astype(np.float32), P)
    if zero:
        cdf = _zero_runs(cdf, rng, P)
    pitch = 2 * T + 8
    words = rng.integers(0, 1 << 32, (S, pitch), dtype=np.uint64).astype(np.uint32)
    nw = rng.integers(0, 2 * T, S).astype(np.int32)
    nw[:4] = [0, 1, 2, 3]
    d_cdf = _dev(cdf[..., :K].astype(np.uint16 if cb == 2 else np.uint32))
    d_words = _dev(words.view(np.int32))
    d_n = _dev(nw)
    d_out = torch.zeros((S, T), dtype=torch.uint8, device="cuda")
    N.check(gpu.rc_decode_tables(P, cb, N.ptr(d_cdf), K, N.ptr(d_words), pitch, N.ptr(d_n), S, T, N.ptr(d_out),
                                 N.stream_ptr()))
    out = d_out.cpu().numpy()
    for s in range(S):
        ref = ora.decode_tables(P, cdf[s], words[s, :nw[s]])
        assert (out[s] == ref).all(), s


@pytest.mark.parametrize("S,T", [(1, 8), (7, 16), (33, 8), (1, 4), (9, 12), (65, 4)])
def test_decode_tables_short_streams(gpu, ora, S, T):
    """The throughput decoders at their smallest shapes: one stream, fewer streams than a wavefront holds, and the
    shortest lengths each takes (8 and 16 steps for eight streams per wave; 4 and 12 for four), on encoder
    words and on arbitrary words (stream lengths 0 .. 2 T + 2), against the oracle decoder."""
    from boa_amd import _native as N

    rng = np.random.default_rng(S * 100 + T)
    K, P = 256, 16
    cdf = ora.xq_cdf(rng.normal(0, 3, (S, T, K)).astype(np.float32), P)
    syms = _sample(cdf, rng, P)
    tables = cdf[..., :K].astype(np.uint16)
    pitch = 2 * T + 8
    d_cdf, d_words, d_n = _encode_gpu(gpu, P, 2, tables, syms, pitch)
    d_out = torch.zeros((S, T), dtype=torch.uint8, device="cuda")
    N.check(gpu.rc_decode_tables(P, 2, N.ptr(d_cdf), K, N.ptr(d_words), pitch, N.ptr(d_n), S, T, N.ptr(d_out),
                                 N.stream_ptr()))
    assert (d_out.cpu().numpy() == syms).all()
    words = rng.integers(0, 1 << 32, (S, pitch), dtype=np.uint64).astype(np.uint32)
    nw = rng.integers(0, 2 * T + 3, S).astype(np.int32)
    d_w, d_nw = _dev(words.view(np.int32)), _dev(nw)  # held: a freed temporary's memory is reused at once
    N.check(gpu.rc_decode_tables(P, 2, N.ptr(d_cdf), K, N.ptr(d_w), pitch, N.ptr(d_nw), S, T, N.ptr(d_out),
                                 N.stream_ptr()))
    out = d_out.cpu().numpy()
    for s in range(S):
        assert (out[s] == ora.decode_tables(P, cdf[s], words[s, :nw[s]])).all(), s


@pytest.mark.parametrize("K,T", [(2, 8), (3, 6), (4, 5)])
@pytest.mark.parametrize("P,cb", [(16, 2), (16, 4), (24, 4)])
@pytest.mark.parametrize("kind", ["mixed", "top"])
def test_tables_brute_force_tiny_alphabets(gpu, ora, K, T, P, cb, kind):
    """Every sequence of length T over K symbols, one stream each, through the same per-step tables (the tables
    the CPU brute-force test pins against the big-integer check and the codes' lexicographic order): the GPU
    words equal the oracle's for every stream, and the GPU decoder returns every sequence."""
    from boa_amd import _native as N
    from test_oracle_rc import _all_sequences, _tiny_tables

    rng = np.random.default_rng(K * 100 + T * 10 + P + (kind == "top"))
    cdf = _tiny_tables(rng, K, T, P, kind)
    seqs = _all_sequences(K, T)
    S = len(seqs)
    tables = np.ascontiguousarray(np.broadcast_to(cdf[:, :K], (S, T, K))).astype(np.uint16 if cb == 2 else np.uint32)
    pitch = T + 8
    d_cdf, d_words, d_n = _encode_gpu(gpu, P, cb, tables, seqs, pitch)
    words = d_words.cpu().numpy().view(np.uint32)
    nw = d_n.cpu().numpy()
    for s in range(S):
        ref = ora.encode_tables(P, cdf, seqs[s])
        assert nw[s] == len(ref) and (words[s, :nw[s]] == ref).all(), seqs[s]
    d_out = torch.zeros((S, T), dtype=torch.uint8, device="cuda")
    N.check(gpu.rc_decode_tables(P, cb, N.ptr(d_cdf), K, N.ptr(d_words), pitch, N.ptr(d_n), S, T, N.ptr(d_out),
                                 N.stream_ptr()))
    assert (d_out.cpu().numpy() == seqs).all()


def test_tables_empty_and_skipped_symbols(gpu, ora):
    P, K, S, T = 16, 16, 8, 40
    rng = np.random.default_rng(3)
    cdf = ora.xq_cdf(rng.normal(0, 2, (S, T, K)).astype(np.float32), P)
    syms = _sample(cdf, rng, P)
    syms[0, :] = 255          # every symbol outside [0, K): skipped -> empty stream
    syms[1, ::3] = 200        # some skipped (gpu_range_coder.py:97)
    _, d_words, d_n = _encode_gpu(gpu, P, 4, cdf[..., :K].astype(np.uint32), syms, T + 8)
    nw = d_n.cpu().numpy()
    words = d_words.cpu().numpy().view(np.uint32)
    assert nw[0] == 0
    for s in range(S):
        keep = syms[s] < K
        ref = ora.encode_tables(P, cdf[s][keep], syms[s][keep])
        assert (words[s, :nw[s]] == ref).all()


def test_synth_tables_round_trip(gpu, ora):
    from boa_amd import _native as N

    P, cb, K, S, T = 16, 2, 256, 256, 512
    d_cdf = torch.empty((S, T, K), dtype=torch.int16, device="cuda")
    d_syms = torch.empty((S, T), dtype=torch.uint8, device="cuda")
    N.check(gpu.rc_synth_tables(12345, 3.0, P, cb, K, S, T, N.ptr(d_cdf), N.ptr(d_syms), N.stream_ptr()))
    pitch = T + 8
    d_words = torch.zeros((S, pitch), dtype=torch.int32, device="cuda")
    d_n = torch.zeros(S, dtype=torch.int32, device="cuda")
    N.check(gpu.rc_encode_tables(P, cb, N.ptr(d_cdf), K, N.ptr(d_syms), S, T, N.ptr(d_words), pitch, N.ptr(d_n),
                                 N.stream_ptr()))
    d_out = torch.zeros((S, T), dtype=torch.uint8, device="cuda")
    N.check(gpu.rc_decode_tables(P, cb, N.ptr(d_cdf), K, N.ptr(d_words), pitch, N.ptr(d_n), S, T, N.ptr(d_out),
                                 N.stream_ptr()))
    torch.cuda.synchronize()
    syms = d_syms.cpu().numpy()
    assert (d_out.cpu().numpy() == syms).all()
    tables = d_cdf.cpu().numpy().view(np.uint16).astype(np.uint32)
    full = np.concatenate([tables, np.full((S, T, 1), 1 << P, np.uint32)], axis=-1)
    assert (full[..., 0] == 0).all() and (np.diff(full.astype(np.int64), axis=-1) >= 1).all()
    words = d_words.cpu().numpy().view(np.uint32)
    nw = d_n.cpu().numpy()
    for s in range(0, S, 37):
        ref = ora.encode_tables(P, full[s], syms[s].astype(np.int32))
        assert (words[s, :nw[s]] == ref).all()
        steps = [(int(full[s, t, v]), int(full[s, t, v + 1]) - int(full[s, t, v])) for t, v in enumerate(syms[s].astype(np.int64))]
        bigint_check.check(ref, steps, P)


def _softmax(x):
    e = np.exp(x - x.max(-1, keepdims=True))
    return (e / e.sum(-1, keepdims=True)).astype(np.float32)


@pytest.mark.parametrize("K", [256, 1000, 3])
def test_range_coder_batch_matches_q2_oracle(gpu, ora, K):
    import gpu_range_coder as gr

    rng = np.random.default_rng(K)
    N, T = 40, 150
    probs = _softmax(rng.normal(0, 3, (T, N, K)))
    p64 = probs.astype(np.float64)
    p64 /= p64.sum(-1, keepdims=True)
    syms = np.array([[rng.choice(K, p=p64[t, i]) for i in range(N)] for t in range(T)], dtype=np.int32)
    lens = rng.integers(0, T + 1, N)
    lens[0], lens[1] = 0, T
    b = gr.gpu.queue.RangeCoderBatch(N, K, T)
    for t in range(T):
        b.encode_step(_dev(syms[t]), _dev(probs[t]), mask=_dev(lens > t))
    b.finalize()
    comp = b.get_compressed_list()
    assert b.get_sizes_list() == [len(c) for c in comp]
    for i in range(N):
        ref = ora.encode_probs_q2(24, probs[:lens[i], i], syms[:lens[i], i])
        assert comp[i].dtype == np.uint32 and (comp[i] == ref).all(), i
    d = gr.gpu.queue.RangeCoderBatch(N, K, T)
    d.load_compressed_list(comp)
    d.init_decoder()
    out = torch.full((N,), -1, dtype=torch.int32, device="cuda")
    got = np.zeros((T, N), dtype=np.int32)
    for t in range(T):
        d.decode_step(_dev(probs[t]), out, mask=_dev(lens > t))
        got[t] = out.cpu().numpy()
    for i in range(N):
        assert (got[:lens[i], i] == syms[:lens[i], i]).all(), i


def test_range_coder_batch_adversarial_probs(gpu, ora):
    """RangeCoderBatch's Q2 on probability rows no softmax emits: all zero, NaN or +inf entries (the uniform
    fallback), entries whose float sum overflows but whose double sum does not, subnormal entries only, one
    nonzero entry, and zeros mixed with ordinary values.  Words equal the oracle's for every lane and decode
    back to the symbols."""
    import gpu_range_coder as gr

    K, T = 256, 40
    rng = np.random.default_rng(21)
    base = _softmax(rng.normal(0, 3, K))
    rows = [np.zeros(K, np.float32)]
    r = base.copy(); r[5] = np.nan; rows.append(r)
    r = base.copy(); r[9] = np.inf; rows.append(r)
    rows.append(np.full(K, 3e38, np.float32))
    r = np.zeros(K, np.float32); r[::7] = 3.3e38; rows.append(r)
    rows.append((rng.integers(1, 100, K) * np.float32(1e-45)).astype(np.float32))
    r = np.zeros(K, np.float32); r[255] = 1.0; rows.append(r)
    r = np.zeros(K, np.float32); r[0] = 1e-45; rows.append(r)
    r = base.copy(); r[rng.random(K) < 0.6] = 0.0; rows.append(r)
    probs = np.stack(rows).astype(np.float32)                  # [N, K], the same rows at every step
    N = probs.shape[0]
    tables = np.stack([ora.q2_cdf(probs[i:i + 1], 24)[0] for i in range(N)]).astype(np.int64)
    assert (np.diff(tables, axis=1) >= 1).all()
    syms = rng.integers(0, K, (T, N)).astype(np.int32)
    d_probs = _dev(probs)
    b = gr.gpu.queue.RangeCoderBatch(N, K, T)
    for t in range(T):
        b.encode_step(_dev(syms[t]), d_probs)
    b.finalize()
    comp = b.get_compressed_list()
    for i in range(N):
        ref = ora.encode_probs_q2(24, np.repeat(probs[i:i + 1], T, 0), syms[:, i])
        assert (comp[i] == ref).all(), i
    d = gr.gpu.queue.RangeCoderBatch(N, K, T)
    d.load_compressed_list(comp)
    d.init_decoder()
    out = torch.full((N,), -1, dtype=torch.int32, device="cuda")
    for t in range(T):
        d.decode_step(d_probs, out)
        assert (out.cpu().numpy() == syms[t]).all(), t


def test_range_coder_batch_errors(gpu):
    import gpu_range_coder as gr

    N, K = 4, 256
    b = gr.gpu.queue.RangeCoderBatch(N, K, 4, pitch_bytes=8)  # 2 words per stream
    rng = np.random.default_rng(0)
    probs = _softmax(rng.normal(0, 0.1, (N, K)))
    for _ in range(8):  # ~8 bits per symbol: overflows 2 words
        b.encode_step(_dev(rng.integers(0, K, N).astype(np.int32)), _dev(probs))
    with pytest.raises(RuntimeError, match="pitch"):
        b.finalize()
    with pytest.raises(RuntimeError, match="length must equal N"):
        b.load_compressed_list([np.zeros(1, np.uint32)])
    with pytest.raises(RuntimeError, match="uint32"):
        b.load_compressed_list([np.zeros(1, np.int64)] * N)
    with pytest.raises(RuntimeError, match="exceeds pitch"):
        b.load_compressed_list([np.zeros(5, np.uint32)] * N)


@pytest.mark.parametrize("bad_lane,bad_count", [(1500, 17), (7, -3), (2999, 17)])
def test_compaction_rejects_counts_outside_pitch(gpu, bad_lane, bad_count):
    """A lane's word count outside [0, pitch] is reported as an argument error and nothing is gathered (the check
    runs in the device scan, in whichever scan workgroup holds the lane).  The words buffer has a spare row and the
    capacity covers the stated counts, so nothing would be touched out of bounds even without the check."""
    from boa_amd import _native as N

    lanes, pitch = 3000, 16
    rng = np.random.default_rng(12)
    nw = rng.integers(0, pitch + 1, lanes).astype(np.int32)
    nw[bad_lane] = bad_count
    words = rng.integers(0, 1 << 31, (lanes + 1, pitch)).astype(np.int32)
    d_words, d_nw = _dev(words), _dev(nw)
    d_off = torch.empty(lanes, dtype=torch.int64, device="cuda")
    cap = int(np.clip(nw, 0, None).astype(np.int64).sum())
    d_pl = torch.full((cap,), 7, dtype=torch.int32, device="cuda")
    got = ctypes.c_int64(-1)
    rc = gpu.boa_compact(N.ptr(d_words), pitch, N.ptr(d_nw), lanes, N.ptr(d_off), N.ptr(d_pl), cap,
                         ctypes.byref(got), N.stream_ptr())
    assert rc == N.BOA_ERR_ARG and b"pitch_words = 16" in gpu.boa_last_error()
    assert got.value == 0 and bool((d_pl == 7).all())
    # the same buffers with the count made valid compact normally (the scratch carries nothing over)
    nw[bad_lane] = pitch
    d_nw = _dev(nw)
    total = int(nw.sum())
    d_pl = torch.zeros(total, dtype=torch.int32, device="cuda")
    N.check(gpu.boa_compact(N.ptr(d_words), pitch, N.ptr(d_nw), lanes, N.ptr(d_off), N.ptr(d_pl), total,
                            ctypes.byref(got), N.stream_ptr()))
    assert got.value == total
    ref = np.concatenate([words[i, :nw[i]] for i in range(lanes)])
    assert (d_pl.cpu().numpy() == ref).all()
    assert (d_off.cpu().numpy() == np.concatenate([[0], np.cumsum(nw)[:-1]])).all()


@pytest.mark.parametrize("lanes,pitch", [(1, 8), (1024, 16), (1025, 16), (3000, 64), (70000, 4)])
def test_compaction(gpu, lanes, pitch):
    """Multi-workgroup scan (1024 lanes per workgroup) + gather vs numpy, at one and several workgroups."""
    from boa_amd import _native as N

    rng = np.random.default_rng(9)
    nw = rng.integers(0, pitch + 1, lanes).astype(np.int32)
    words = rng.integers(0, 1 << 31, (lanes, pitch)).astype(np.int32)
    d_words, d_nw = _dev(words), _dev(nw)
    d_off = torch.empty(lanes, dtype=torch.int64, device="cuda")
    total = int(nw.sum())
    d_pl = torch.empty(total, dtype=torch.int32, device="cuda")
    got = ctypes.c_int64(0)
    N.check(gpu.boa_compact(N.ptr(d_words), pitch, N.ptr(d_nw), lanes, N.ptr(d_off), N.ptr(d_pl), total,
                            ctypes.byref(got), N.stream_ptr()))
    assert got.value == total
    ref = np.concatenate([words[i, :nw[i]] for i in range(lanes)])
    assert (d_pl.cpu().numpy() == ref).all()
    assert (d_off.cpu().numpy() == np.concatenate([[0], np.cumsum(nw)[:-1]])).all()
    small = torch.empty(max(total - 1, 1), dtype=torch.int32, device="cuda")
    with pytest.raises(N.BoaError):
        N.check(gpu.boa_compact(N.ptr(d_words), pitch, N.ptr(d_nw), lanes, N.ptr(d_off), N.ptr(small), total - 1,
                                ctypes.byref(got), N.stream_ptr()))
