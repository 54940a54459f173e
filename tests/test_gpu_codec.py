"""Fused compress/decompress on the GPU: byte-exact round trips, ragged and edge-case chunks, BOA2 files,
and compressed size within 0.5% of the oracle pipeline (CPU fp32 model -> softmax -> Q2 -> coder)."""
import os

import numpy as np
import pytest
import torch

from oracle import model_ref, weights_ref

pytestmark = pytest.mark.gpu


def _model(n_layers=2, seed=0):
    from boa_amd import weights as W

    import model as M

    blob = W.seeded_blob(W.Cfg(n_layers=n_layers), seed)
    return M.BoaConstrictor(256, n_layers, 256).load_blob(blob), blob


def _markov(n, seed=0, alpha=0.1):
    rng = np.random.default_rng(seed)
    P = rng.dirichlet([alpha] * 256, size=256)
    C = np.cumsum(P, axis=1)
    out = np.empty(n, dtype=np.uint8)
    x = 0
    u = rng.random(n)
    for i in range(n):
        out[i] = x
        x = min(int(np.searchsorted(C[x], u[i], side="right")), 255)
    return out


@pytest.mark.parametrize("precision", ["f32", "bf16x3", "bf16w"])
def test_round_trip_ragged(gpu, precision):
    import codec

    m, _ = _model(2)
    m.precision = precision
    rng = np.random.default_rng(1)
    lens = [1, 2, 3, 64, 65, 129, 200, 1, 77]
    chunks = [rng.integers(0, 256, L).astype(np.uint8) for L in lens]
    payload, nw, fb, Ls = codec.compress_payload(m, chunks)
    assert Ls == lens and fb == [int(c[0]) for c in chunks]
    assert nw[0] == 0 and nw[7] == 0  # length-1 chunks code nothing
    out = codec.decompress_payload(m, payload, nw, lens, fb)
    for i, c in enumerate(chunks):
        assert (out[i, :lens[i]] == c).all(), i


def test_round_trip_api_8_layers(gpu):
    import codec

    m, _ = _model(8)
    data = _markov(40 * 300, seed=2)
    x_list = [torch.from_numpy(data[i * 300:(i + 1) * 300]).unsqueeze(0) for i in range(40)]
    comp, fb, Ls = codec.compress_GPU(m, x_list)
    assert all(c.dtype == np.uint32 for c in comp)
    dec = codec.decompress_GPU(m, comp, Ls, fb)
    assert all(d.shape == (1, L) for d, L in zip(dec, Ls))
    assert np.array_equal(np.concatenate([d.reshape(-1) for d in dec]), data)


def test_compressed_size_vs_oracle_pipeline(gpu, ora):
    """Sizes within 0.5% of the reference protocol run on the CPU oracle (Q2 on torch softmax probs)."""
    import codec

    n_layers, B, L = 2, 32, 1500
    m, blob = _model(n_layers, seed=4)
    data = _markov(B * L, seed=3)
    chunks = [data[i * L:(i + 1) * L] for i in range(B)]
    payload, nw, fb, Ls = codec.compress_payload(m, chunks)
    ref = model_ref.RefModel(blob, weights_ref.Cfg(n_layers=n_layers))
    X = torch.from_numpy(np.stack(chunks).astype(np.int64))
    logits = ref.forward(X[:, :-1])                       # [B, L-1, V]
    probs = torch.softmax(logits, dim=-1).to(torch.float32).numpy()
    ref_words = sum(len(ora.encode_probs_q2(24, probs[b], X[b, 1:].numpy().astype(np.int32))) for b in range(B))
    gpu_words = int(nw.sum())
    print(f"gpu words {gpu_words}  oracle words {ref_words}", flush=True)
    assert abs(gpu_words - ref_words) <= 0.005 * ref_words
    out = codec.decompress_payload(m, payload, nw, Ls, fb)
    assert np.array_equal(out.reshape(-1), data)


def test_boa_file_round_trip(gpu, tmp_path):
    import boa

    m, _ = _model(2)
    data = _markov(5000, seed=5).tobytes()
    src = tmp_path / "in.bin"
    src.write_bytes(data)
    f = boa.BOA("cuda", str(tmp_path / "x.boa"), m)
    f.compress(str(src), chunks_count=7, progress=False)
    meta = f.get_metadata()
    assert meta == {"chunk_len": 715, "n_chunks": 7, "uncompressed_len": 5000, "last_chunk_len": 710}
    g = boa.BOA("cuda", str(tmp_path / "x.boa"), m)
    assert g.decompress(progress=False) == data
    # seq_size chunking, and a wave size smaller than the chunk count
    os.environ["BOA_GPU_STREAMS"] = "3"
    try:
        f.compress(str(src), seq_size=1024, progress=False)
        assert boa.BOA("cuda", str(tmp_path / "x.boa"), m).decompress(progress=False) == data
    finally:
        del os.environ["BOA_GPU_STREAMS"]


@pytest.mark.parametrize("data,kw,meta", [
    (b"\x7f", {"chunks_count": 1}, (1, 1, 1)),               # one byte: the first byte only, no coded symbols
    (b"\x00\xff", {"seq_size": 1}, (1, 2, 1)),             # two one-byte chunks: two empty streams
    (bytes(range(5)), {"chunks_count": 7}, (1, 5, 1)),     # more chunks asked for than bytes: 5 chunks
    (bytes(range(9)), {"chunks_count": 4}, (3, 3, 3)),     # ceil(9/4) = 3 leaves an empty 4th chunk: dropped
    (bytes(70), {"seq_size": 65}, (65, 2, 5)),             # a tile boundary inside the first chunk
], ids=["1B", "2x1B", "5B-7chunks", "9B-4chunks", "70B-seq65"])
def test_boa_file_tiny_inputs(gpu, tmp_path, data, kw, meta):
    """BoaFile at its smallest inputs: the header's (chunk_len, n_chunks, last_chunk_len), a byte-exact
    round trip, and the empty file refused with the reference's message (boa.py:162-164)."""
    import boa

    m, _ = _model(2)
    src = tmp_path / "in.bin"
    src.write_bytes(data)
    f = boa.BOA("cuda", str(tmp_path / "x.boa"), m)
    f.compress(str(src), progress=False, **kw)
    got = f.get_metadata()
    assert (got["chunk_len"], got["n_chunks"], got["last_chunk_len"]) == meta
    assert got["uncompressed_len"] == len(data)
    assert boa.BOA("cuda", str(tmp_path / "x.boa"), m).decompress(progress=False) == data
    src.write_bytes(b"")
    with pytest.raises(ValueError, match="Input file is empty"):
        f.compress(str(src), chunks_count=1, progress=False)


@pytest.mark.parametrize("d_model,precision,steps", [(256, "bf16x3", None), (256, "f32", None),
                                                     (512, "bf16w", None), (512, "bf16x3", None),
                                                     (256, "bf16x3", "5"), (512, "bf16w", "5")])
def test_decompress_fused_and_layer_kernels_agree(gpu, d_model, precision, steps):
    """Decompression through the fused step kernel and through the per-layer kernels gives the same bytes
    (both must reproduce the compressor's logits bit for bit to decode at all).  At d_model 512 the 70 ragged
    lanes span three 32-lane workgroups, the last one partly filled, and lanes end at different positions.
    steps: decode steps per fused launch (BOA_FUSED_STEPS_PER_LAUNCH; default 128), so that the conv history
    ring position and the fed-back bytes carry across many launch boundaries."""
    import codec
    from boa_amd import weights as W

    import model as M

    if d_model == 256:
        m, _ = _model(2)
        lens = [300, 17, 1, 256, 45]
    else:
        m = M.BoaConstrictor(512, 2, 256).load_blob(W.seeded_blob(W.Cfg(d_model=512, n_layers=2), 3))
        lens = [int(v) for v in np.random.default_rng(5).integers(1, 90, 70)]
        lens[0], lens[33] = 1, 150
    m.precision = precision
    chunks = [_markov(L, seed=20 + i) for i, L in enumerate(lens)]
    payload, nw, fb, Ls = codec.compress_payload(m, chunks)
    outs = []
    for flag in ("1", "0"):
        os.environ["BOA_FUSED_STEP"] = flag
        if steps:
            os.environ["BOA_FUSED_STEPS_PER_LAUNCH"] = steps
        try:
            m.release_engines()
            outs.append(codec.decompress_payload(m, payload, nw, Ls, fb))
        finally:
            del os.environ["BOA_FUSED_STEP"]
            os.environ.pop("BOA_FUSED_STEPS_PER_LAUNCH", None)
    m.release_engines()
    for out in outs:
        for i, c in enumerate(chunks):
            assert (out[i, :lens[i]] == c).all(), i


@pytest.mark.parametrize("d_model,precision", [(256, "bf16x3"), (256, "f32"), (512, "bf16w")])
def test_decompress_arbitrary_payload(gpu, d_model, precision):
    """Decoding words that no encoder wrote (a random payload, random word counts including 0, chunks of 1 to
    200 bytes): it completes, returns every chunk's first byte as given, decodes the same bytes on a second
    run, and the fused step kernel and the per-layer kernels decode the same bytes (their logits are bit
    identical, so they take the same path through any words)."""
    import codec
    from boa_amd import weights as W

    import model as M

    if d_model == 256:
        m, _ = _model(2)
    else:
        m = M.BoaConstrictor(512, 2, 256).load_blob(W.seeded_blob(W.Cfg(d_model=512, n_layers=2), 3))
    m.precision = precision
    rng = np.random.default_rng(17 + d_model)
    lens = [1, 2, 50, 130, 65, 7, 200, 33]
    nw = rng.integers(0, 60, len(lens)).astype(np.int64)
    nw[1] = 0
    payload = rng.integers(0, 1 << 32, int(nw.sum()), dtype=np.uint64).astype(np.uint32)
    fb = [int(v) for v in rng.integers(0, 256, len(lens))]
    outs = []
    for flag in ("1", "1", "0"):
        os.environ["BOA_FUSED_STEP"] = flag
        try:
            m.release_engines()
            outs.append(codec.decompress_payload(m, payload, nw, lens, fb))
        finally:
            del os.environ["BOA_FUSED_STEP"]
    m.release_engines()
    for i, L in enumerate(lens):
        assert int(outs[0][i, 0]) == fb[i]
        for out in outs[1:]:
            assert (out[i, :L] == outs[0][i, :L]).all(), i


def _decode_raw(m, buf, total, offs, nws, fb, lens):
    """boa_decompress through the C ABI over a device buffer `buf` of which the first `total` words are the
    payload."""
    from boa_amd import _native as nat

    N = len(lens)
    d_buf = torch.from_numpy(np.ascontiguousarray(buf, dtype=np.uint32).view(np.int32)).cuda()
    d_off = torch.tensor(offs, dtype=torch.int64).cuda()
    d_nw = torch.tensor(nws, dtype=torch.int32).cuda()
    d_first = torch.tensor(fb, dtype=torch.uint8).cuda()
    d_lens = torch.tensor(lens, dtype=torch.int32).cuda()
    out = torch.zeros((N, max(lens)), dtype=torch.uint8, device="cuda")
    eng = m.engine(N, 1)
    nat.check(nat.lib().boa_decompress(eng.h, nat.ptr(d_buf), int(total), nat.ptr(d_off), nat.ptr(d_nw),
                                       nat.ptr(d_first), nat.ptr(d_lens), N, max(lens), nat.ptr(out), out.stride(0)))
    return out.cpu().numpy()


@pytest.mark.parametrize("d_model,fused", [(256, "1"), (256, "0"), (512, "1")])
def test_decompress_payload_bound(gpu, d_model, fused):
    """boa_decompress clamps every stream to the payload_words it is given (the bound decompress_v2 checks,
    boa.cpp:240).  The payload sits in a larger buffer whose words past the payload are random: a stream whose
    offset lies past the payload decodes as an empty stream, one that runs past the end as its clamped
    prefix, a negative offset as offset 0 and a negative count as 0 -- each equal to decoding the clamped
    arguments, so no word past the payload was read -- and every consistent lane still round-trips."""
    import codec
    from boa_amd import weights as W

    import model as M

    if d_model == 256:
        m, _ = _model(2)
        m.precision = "bf16x3"
    else:
        m = M.BoaConstrictor(512, 2, 256).load_blob(W.seeded_blob(W.Cfg(d_model=512, n_layers=2), 3))
        m.precision = "bf16w"
    lens = [90, 60, 75, 80, 50, 70, 64]
    chunks = [_markov(L, seed=40 + i) for i, L in enumerate(lens)]
    payload, nw, fb, Ls = codec.compress_payload(m, chunks)
    total = int(nw.sum())
    offs = np.concatenate([[0], np.cumsum(nw)[:-1]]).astype(np.int64)
    rng = np.random.default_rng(9)
    buf = np.concatenate([payload, rng.integers(1, 1 << 32, 4096, dtype=np.uint64).astype(np.uint32)])
    bad_off, bad_nw = offs.copy(), nw.astype(np.int64).copy()
    clamp_off, clamp_nw = offs.copy(), nw.astype(np.int64).copy()
    bad_off[1], bad_nw[1] = total + 100, 50          # past the end: empty
    clamp_off[1], clamp_nw[1] = 0, 0
    bad_off[3], bad_nw[3] = total - 3, 40            # runs past the end: the last 3 words
    clamp_off[3], clamp_nw[3] = total - 3, 3
    bad_off[4], bad_nw[4] = -5, 10                   # negative offset: from word 0
    clamp_off[4], clamp_nw[4] = 0, 10
    bad_nw[5] = -7                                   # negative count: empty
    clamp_nw[5] = 0
    os.environ["BOA_FUSED_STEP"] = fused
    try:
        m.release_engines()
        good = _decode_raw(m, buf, total, offs, nw, fb, lens)
        bad = _decode_raw(m, buf, total, bad_off, bad_nw, fb, lens)
        exp = _decode_raw(m, np.concatenate([payload, np.zeros(4096, np.uint32)]), total, clamp_off, clamp_nw, fb,
                          lens)
    finally:
        del os.environ["BOA_FUSED_STEP"]
        m.release_engines()
    for i, c in enumerate(chunks):
        assert (good[i, :lens[i]] == c).all(), i
        assert (bad[i, :lens[i]] == exp[i, :lens[i]]).all(), i
        if i not in (1, 3, 4, 5):
            assert (bad[i, :lens[i]] == c).all(), i
    assert not (bad[3, :lens[3]] == chunks[3]).all()   # the clamped stream is not the whole stream


def test_boa_decompress_rejects_negative_payload_words(gpu):
    from boa_amd import _native as nat

    m, _ = _model(1)
    eng = m.engine(1, 1)
    z = torch.zeros(16, dtype=torch.int64, device="cuda")
    rc = nat.lib().boa_decompress(eng.h, nat.ptr(z), -1, nat.ptr(z), nat.ptr(z), nat.ptr(z), nat.ptr(z), 1, 4,
                                  nat.ptr(z), 4)
    assert rc != 0 and b"bad arguments" in nat.lib().boa_last_error()
    m.release_engines()


def test_round_trip_d512_bf16w(gpu):
    """configs[4] model shape (d_model 512, bf16 weights), 16 layers, mixed int16 / float32 records."""
    import codec
    from boa_amd import weights as W

    import model as M

    cfg = W.Cfg(d_model=512, n_layers=16)
    m = M.BoaConstrictor(512, 16, 256).load_blob(W.seeded_blob(cfg, 1))
    m.precision = "bf16w"
    rng = np.random.default_rng(1)
    n = 3000
    ints = np.clip(rng.normal(0, 300, n), -32767, 32767).astype(np.int16)
    flts = rng.lognormal(1.0, 1.5, n).astype(np.float32)
    rec = np.empty(n, dtype=[("i", "<i2"), ("f", "<f4")])
    rec["i"], rec["f"] = ints, flts
    data = rec.tobytes()
    data = np.frombuffer(data, dtype=np.uint8)
    L = len(data) // 12
    chunks = [data[i * L:(i + 1) * L] for i in range(12)]
    payload, nw, fb, Ls = codec.compress_payload(m, chunks)
    out = codec.decompress_payload(m, payload, nw, Ls, fb)
    for i, c in enumerate(chunks):
        assert (out[i, :L] == c).all(), i


def test_wave_lanes_from_device_memory(gpu):
    """Without BOA_GPU_STREAMS the wave holds every chunk that fits in free device memory (288 GB: all of
    configs[4]'s 16384 chunks), never more than asked, and the context it implies is exactly what
    boa_ctx_create allocates."""
    import boa

    m, _ = _model(2)
    os.environ.pop("BOA_GPU_STREAMS", None)
    assert boa._wave_lanes(m, 7, 100) == 7
    big = boa._wave_lanes(m, 16384, 16384)
    assert big == 16384
    eng = m.engine(64, 64)
    import ctypes

    from boa_amd import _native as N

    c = N.ModelCfg(256, 2, 256, 16, 4, 2, 0)
    b = ctypes.c_int64(0)
    import model as M

    N.check(gpu.boa_ctx_plan_bytes(ctypes.byref(c), M.PRECISIONS[m.precision], 64, 64, ctypes.byref(b)))
    assert b.value == eng.device_bytes
    os.environ["BOA_GPU_STREAMS"] = "5"
    try:
        assert boa._wave_lanes(m, 7, 100) == 5
    finally:
        del os.environ["BOA_GPU_STREAMS"]


@pytest.mark.parametrize("precision", ["f32", "bf16x3"])
def test_compressed_size_vs_oracle_config2(gpu, ora, precision):
    """configs[2]'s own model (d256 x 8 layers, seed 0) and data (float32 records: in the default f32 mode the
    first 256 of its 4096 chunks, first 2048 B of each, 1/128 of the payload; in bf16x3 the first 32 chunks x
    1024 B): compressed size within 0.5% of the reference protocol run on the CPU oracle (fp32 model ->
    torch.softmax -> Q2 at P = 24 -> coder), and the round trip byte-exact."""
    import codec
    from bench import synth_records
    import model as M

    lanes, L = (256, 2048) if precision == "f32" else (32, 1024)
    m, blob = _model(8, seed=0)
    assert M.DEFAULT_PRECISION == "f32" or "BOA_PRECISION" in os.environ
    m.precision = precision
    data = np.ascontiguousarray(synth_records(lanes * 16384, 0).reshape(lanes, 16384)[:, :L])
    chunks = [data[i] for i in range(lanes)]
    payload, nw, fb, Ls = codec.compress_payload(m, chunks)
    ref = model_ref.RefModel(blob, weights_ref.Cfg(n_layers=8))
    X = torch.from_numpy(data.astype(np.int64))
    probs = torch.softmax(ref.forward(X[:, :-1]), dim=-1).to(torch.float32).numpy()
    ref_words = sum(len(ora.encode_probs_q2(24, probs[b], X[b, 1:].numpy().astype(np.int32))) for b in range(lanes))
    gpu_words = int(nw.sum())
    print(f"gpu words {gpu_words}  oracle words {ref_words}", flush=True)
    assert abs(gpu_words - ref_words) <= 0.005 * ref_words
    out = codec.decompress_payload(m, payload, nw, Ls, fb)
    assert np.array_equal(out, data)


def test_layer_decode_in_two_halves(gpu):
    """Per-layer decode of a wave large enough (>= 512 lanes) to run as two halves of the lanes on two streams,
    their state groups alternating: the same bytes as one stream and as the fused decode kernel."""
    import codec

    m, _ = _model(2)
    rng = np.random.default_rng(7)
    lens = [int(v) for v in rng.integers(1, 40, 600)]
    chunks = [_markov(L, seed=100 + i) for i, L in enumerate(lens)]
    payload, nw, fb, Ls = codec.compress_payload(m, chunks)
    for fused, halves in (("0", "2"), ("0", "1"), ("1", "2")):
        os.environ["BOA_FUSED_STEP"] = fused
        os.environ["BOA_DECODE_HALVES"] = halves
        try:
            m.release_engines()
            out = codec.decompress_payload(m, payload, nw, Ls, fb)
        finally:
            del os.environ["BOA_FUSED_STEP"]
            del os.environ["BOA_DECODE_HALVES"]
        for i, c in enumerate(chunks):
            assert (out[i, :lens[i]] == c).all(), (fused, halves, i)
    m.release_engines()


@pytest.mark.parametrize("flag", ["BOA_HEAD_XQ", "BOA_FFN_OUTP"])
@pytest.mark.parametrize("d_model,precision", [(256, "bf16x3"), (256, "bf16w"), (512, "bf16w")])
def test_fused_compress_kernels_match_separate_kernels(gpu, d_model, precision, flag):
    """Compress tiles with and without one kernel fusion -- BOA_HEAD_XQ: the head + quantiser kernel (logits on
    chip, (lo, width) pairs, sequential coder) against the head GEMMs + per-lane encode kernel; BOA_FFN_OUTP:
    out_proj inside the feed-forward kernel against the separate out_proj GEMM: identical words for every chunk,
    including chunks that end inside a tile, length-1 chunks and the partial last tile; and the stream decodes."""
    _compress_with_and_without(d_model, precision, flag)


@pytest.mark.parametrize("groups", ["1", "2"])
@pytest.mark.parametrize("d_model,precision", [(256, "f32"), (256, "bf16x3"), (256, "bf16w"), (512, "bf16w"),
                                               (512, "bf16x3")])
def test_embedding_gathered_in_ln1_matches_embedding_pass(gpu, d_model, precision, groups):
    """BOA_EMBED_LN1: layer 0 of a full compress tile gathers its embedding rows in the mixer-input kernel's LN1
    prologue (and writes them to x for the residual) instead of reading the rows an embedding pass wrote: identical
    words with and without, on one stream and (groups "2": 512 lanes) on two lane groups, whose byte and length
    pointers start at the second group's first lane; partial tiles keep the embedding pass in both runs."""
    _compress_with_and_without(d_model, precision, "BOA_EMBED_LN1", wide=groups == "2")


def _compress_with_and_without(d_model, precision, flag, wide=False):
    import codec
    from boa_amd import weights as W

    import model as M

    m = M.BoaConstrictor(d_model, 2, 256).load_blob(W.seeded_blob(W.Cfg(d_model=d_model, n_layers=2), 5))
    m.precision = precision
    lens = [1, 2, 63, 64, 65, 66, 129, 200, 191, 130]
    if wide:  # enough lanes for the compress groups (two streams from 512 lanes), ragged in both groups
        lens = (lens * 52)[:512]
    chunks = [_markov(L, seed=40 + i) for i, L in enumerate(lens)]
    res = []
    for val in ("1", "0"):
        os.environ[flag] = val
        try:
            m.release_engines()
            res.append(codec.compress_payload(m, chunks))
        finally:
            del os.environ[flag]
    m.release_engines()
    (p1, n1, f1, L1), (p0, n0, f0, L0) = res
    assert np.array_equal(n1, n0) and f1 == f0 and L1 == L0
    assert np.array_equal(np.asarray(p1), np.asarray(p0))
    out = codec.decompress_payload(m, p1, n1, L1, f1)
    for i, c in enumerate(chunks):
        assert (out[i, :lens[i]] == c).all(), i


@pytest.mark.parametrize("precision", ["bf16x3", "bf16w", "f32"])
def test_compress_in_two_halves(gpu, precision):
    """A wave large enough (>= 512 lanes; 768 for three groups) to compress as groups of the lanes on their own
    streams (two, the default, and three): the same words as one stream, for full and partial tiles, and the
    stream decodes."""
    import codec

    m, _ = _model(2)
    m.precision = precision
    rng = np.random.default_rng(8)
    lens = [int(v) for v in rng.integers(1, 200, 801)]
    chunks = [_markov(L, seed=300 + i) for i, L in enumerate(lens)]
    res = []
    for halves, groups in (("1", "2"), ("1", "3"), ("0", "2")):
        os.environ["BOA_COMPRESS_HALVES"] = halves
        os.environ["BOA_COMPRESS_GROUPS"] = groups
        try:
            m.release_engines()
            res.append(codec.compress_payload(m, chunks))
        finally:
            del os.environ["BOA_COMPRESS_HALVES"]
            del os.environ["BOA_COMPRESS_GROUPS"]
    m.release_engines()
    (p0, n0, f0, L0) = res[-1]
    for p1, n1, f1, L1 in res[:-1]:
        assert np.array_equal(n1, n0)
        assert np.array_equal(np.asarray(p1), np.asarray(p0))
    out = codec.decompress_payload(m, p0, n0, L0, f0)
    for i, c in enumerate(chunks):
        assert (out[i, :lens[i]] == c).all(), i
