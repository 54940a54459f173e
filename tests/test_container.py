"""BOA2 container (boa.py:89-157) on the CPU: closed forms and every host-forceable error path."""
import hashlib
import struct
import zlib

import numpy as np
import pytest


def test_uvarint_known_answers():
    import boa

    cases = {0: b"\x00", 1: b"\x01", 127: b"\x7f", 128: b"\x80\x01", 300: b"\xac\x02", 2**32: b"\x80\x80\x80\x80\x10"}
    for v, enc in cases.items():
        assert boa.uvarint_encode(v) == enc
        assert boa.uvarint_decode(enc, 0) == (v, len(enc))


def test_fingerprint_closed_form():
    import boa

    class BoaBytePredictor:
        pass

    f = boa.BoaFile("/dev/null", BoaBytePredictor())
    assert f._model_fingerprint().hex() == "c257ec9cf5938905c67212f4001ac357"
    assert f._model_fingerprint() == hashlib.blake2s(b"BoaBytePredictor", digest_size=16).digest()


def _write_boa2(path, streams, first, chunk_len, last_len, ulen, fp=b"\x11" * 16, version=1):
    with open(path, "wb") as f:
        f.write(b"BOA2" + struct.pack("<IIQIII", version, 0, ulen, chunk_len, len(streams), last_len))
        f.write(struct.pack("<B", len(fp)) + fp)
        offs, off = [], 0
        for s in streams:
            f.write(s)
            offs.append(off)
            off += len(s)
        import boa

        idx = bytearray(b"IDX1") + bytes(first)
        prev = 0
        for o in offs:
            idx += boa.uvarint_encode(o - prev)
            prev = o
        for s in streams:
            idx += boa.uvarint_encode(len(s))
        f.write(idx + struct.pack("<I", zlib.crc32(idx) & 0xFFFFFFFF))


def test_reader_parses_handmade_file(tmp_path):
    import boa

    streams = [np.arange(3, dtype="<u4").tobytes(), b"", np.arange(5, dtype="<u4").tobytes()]
    p = tmp_path / "a.boa"
    _write_boa2(p, streams, [7, 8, 9], 100, 42, 242)
    f = boa.BoaFile(str(p), object())
    f._read_file()
    assert f.compressed_data == streams
    assert f.first_bytes == [7, 8, 9]
    assert f.lengths == [100, 100, 42]
    assert f.get_metadata() == {"chunk_len": 100, "n_chunks": 3, "last_chunk_len": 42, "uncompressed_len": 242}


@pytest.mark.parametrize("mutate,msg", [
    (lambda b: b"XOA2" + b[4:], "Bad file magic"),
    (lambda b: b[:4] + struct.pack("<I", 2) + b[8:], "Unsupported version"),
    (lambda b: b[:-1] + bytes([b[-1] ^ 1]), "Bad index CRC"),
    (lambda b: b.replace(b"IDX1", b"IDX2"), "Index not found"),
])
def test_reader_errors(tmp_path, mutate, msg):
    import boa

    p = tmp_path / "a.boa"
    _write_boa2(p, [b"\x01\x00\x00\x00"], [0], 10, 10, 10)
    p.write_bytes(mutate(p.read_bytes()))
    with pytest.raises(ValueError, match=msg):
        boa.BoaFile(str(p), object())._read_file()


def test_reader_rejects_out_of_range_payload(tmp_path):
    import boa

    p = tmp_path / "a.boa"
    _write_boa2(p, [b"\x01\x00\x00\x00"], [0], 10, 10, 10)
    raw = bytearray(p.read_bytes())
    i = raw.rfind(b"IDX1")
    # lengths uvarint is the byte after first_bytes (1) and offsets (1): set it to 200
    raw[i + 4 + 1 + 1] = 100
    idx = bytes(raw[i:-4])
    raw[-4:] = struct.pack("<I", zlib.crc32(idx) & 0xFFFFFFFF)
    p.write_bytes(bytes(raw))
    with pytest.raises(ValueError, match="out of range"):
        boa.BoaFile(str(p), object())._read_file()


def _write_boa2_index(path, payload, first, deltas, sizes):
    """A BOA2 file whose index holds the given offset deltas and stream sizes as they are (any values)."""
    import boa

    with open(path, "wb") as f:
        f.write(b"BOA2" + struct.pack("<IIQIII", 1, 0, 100, 50, len(first), 50) + struct.pack("<B", 0))
        f.write(payload)
        idx = bytearray(b"IDX1") + bytes(first)
        for v in list(deltas) + list(sizes):
            idx += boa.uvarint_encode(v)
        f.write(idx + struct.pack("<I", zlib.crc32(idx) & 0xFFFFFFFF))


def test_reader_rejects_wrapping_offsets(tmp_path):
    """Offset deltas whose running sum wraps 2^64 (stream 0 at 2^64 - 4, stream 1 back at 0) are rejected, as are
    a running offset past the payload and a single delta past it; a well-formed index of the same payload reads."""
    import boa

    payload = np.arange(3, dtype="<u4").tobytes()  # 12 bytes
    p = tmp_path / "w.boa"
    bad = [([(1 << 64) - 4, 4], [8, 4]),   # starts [2^64 - 4, 0]: each start + size wraps below 12
           ([4, 12], [4, 0]),              # starts [4, 16]: stream 1 starts past the payload
           ([13, 0], [0, 0])]              # one delta past the payload
    for deltas, sizes in bad:
        _write_boa2_index(p, payload, [1, 2], deltas, sizes)
        with pytest.raises(ValueError, match="out of range"):
            boa.BoaFile(str(p), object())._read_file()
    _write_boa2_index(p, payload, [1, 2], [0, 4], [4, 8])
    f = boa.BoaFile(str(p), object())
    f._read_file()
    assert f.compressed_data == [payload[:4], payload[4:]]


def test_chunking_formula():
    import boa

    ch = boa.BoaFile._chunking
    assert ch(5000, 0, 7) == (715, 7, 710)        # boa.py:171-172: ceil(n / count)
    assert ch(5000, 1024, 0) == (1024, 5, 904)
    assert ch(16, 0, 4) == (4, 4, 4)
    assert ch(9, 0, 4) == (3, 3, 3)               # would leave an empty 4th chunk: dropped
    with pytest.raises(ValueError):
        ch(10, 0, 0)


def test_cpu_device_refused():
    import torch

    import boa

    if torch.cuda.is_available():
        return
    with pytest.raises(RuntimeError):
        boa.BOA("cpu", "/tmp/x.boa", object())


def test_vectorised_uvarints_match_scalar_decoder():
    import boa

    rng = np.random.default_rng(5)
    vals = [0, 1, 127, 128, 16383, 16384, 2**32 - 1, 2**32, 2**56 + 3] + [
        int(v) for v in rng.integers(0, 2**40, 500)]
    buf = b"junk" + b"".join(boa.uvarint_encode(v) for v in vals) + b"tail"
    got = boa._uvarints(buf, 4, len(buf) - 4, len(vals))
    assert [int(v) for v in got] == vals
    pos, ref = 4, []
    for _ in vals:
        v, pos = boa.uvarint_decode(buf, pos)
        ref.append(v)
    assert ref == vals
    with pytest.raises(ValueError, match="out of range"):
        boa._uvarints(buf, 4, 8, len(vals))  # index truncated


def test_vectorised_uvarint_writer_and_index():
    """The writer's vectorised encoder against the scalar LEB128 encoder (closed forms above), including the
    edges of every group count and 2^64 - 1; and the index it builds, byte for byte, against the index of a
    handmade file (offset deltas written from running offsets), which the reader parses back."""
    import boa

    rng = np.random.default_rng(6)
    vals = [0, 1, 127, 128, 16383, 16384, 2**32 - 1, 2**32, 2**56 + 3, 2**63, 2**64 - 1]
    vals += [(1 << (7 * k)) - 1 for k in range(1, 10)] + [1 << (7 * k) for k in range(1, 10)]
    vals += [int(v) for v in rng.integers(0, 2**62, 300)]
    assert boa._uvarints_bytes(vals) == b"".join(boa.uvarint_encode(v) for v in vals)
    assert boa._uvarints_bytes([]) == b""
    lengths = [12, 0, 20, 4, 100000]
    first = [3, 4, 5, 6, 7]
    offs = np.concatenate([[0], np.cumsum(lengths)[:-1]]).tolist()
    ref = bytearray(b"IDX1") + bytes(first)
    prev = 0
    for o in offs:
        ref += boa.uvarint_encode(o - prev)
        prev = o
    for L in lengths:
        ref += boa.uvarint_encode(L)
    assert boa.BoaFile._index(first, lengths) == bytes(ref)
    assert boa.BoaFile._index([], []) == b"IDX1"


def test_reader_many_streams_property(tmp_path):
    import boa

    rng = np.random.default_rng(9)
    streams = [rng.integers(0, 2**32, int(k), dtype=np.uint64).astype("<u4").tobytes()
               for k in rng.integers(0, 300, 257)]
    first = [int(v) for v in rng.integers(0, 256, len(streams))]
    p = tmp_path / "m.boa"
    _write_boa2(p, streams, first, 5000, 17, 5000 * 256 + 17)
    f = boa.BoaFile(str(p), object())
    f._read_file()
    assert f.compressed_data == streams
    assert f.first_bytes == first
    assert f.lengths == [5000] * 256 + [17]


try:
    from hypothesis import given, settings, strategies as st
except ImportError:  # pragma: no cover
    given = None


@pytest.mark.skipif(given is None, reason="needs hypothesis")
def test_hypothesis_uvarints_and_index():
    """Generated values over the whole u64 range: the writer's vectorised encoder equals the scalar LEB128
    encoder, the reader's vectorised decoder returns the values from any offset, and an index built from
    generated lengths parses back to the running offsets."""
    import boa

    @settings(max_examples=300, deadline=None, database=None)
    @given(st.lists(st.integers(0, 2**64 - 1), max_size=40), st.binary(max_size=5))
    def run(vals, junk):
        enc = boa._uvarints_bytes(vals)
        assert enc == b"".join(boa.uvarint_encode(v) for v in vals)
        buf = junk + enc + b"\x00"
        if vals:
            assert [int(v) for v in boa._uvarints(buf, len(junk), len(buf), len(vals))] == vals

    @settings(max_examples=200, deadline=None, database=None)
    @given(st.lists(st.integers(0, 2**40), min_size=1, max_size=30))
    def run_index(lengths):
        first = [(7 * i) & 0xFF for i in range(len(lengths))]
        idx = boa.BoaFile._index(first, lengths)
        n = len(lengths)
        assert idx[:4] == b"IDX1" and list(idx[4:4 + n]) == first
        vals = [int(v) for v in boa._uvarints(idx, 4 + n, len(idx), 2 * n)]
        offs = np.cumsum(vals[:n]).tolist()
        assert offs == np.concatenate([[0], np.cumsum(lengths)[:-1]]).tolist() and vals[n:] == lengths

    run()
    run_index()


def test_wave_lanes_env_override(monkeypatch):
    """BOA_GPU_STREAMS fixes the lanes per wave as in the reference (boa.py:207-210): an unparsable value
    means 5000, and the result is clamped to [1, n_chunks]; the model is not consulted."""
    import boa

    class NoModel:
        def plan_wave_lanes(self, *a):
            raise AssertionError("model consulted despite BOA_GPU_STREAMS")

    for env, n, want in [("3", 10, 3), ("abc", 9000, 5000), ("abc", 40, 40), ("0", 10, 1), ("-5", 10, 1),
                         ("100000", 16384, 16384), (" 7 ", 10, 7)]:
        monkeypatch.setenv("BOA_GPU_STREAMS", env)
        assert boa._wave_lanes(NoModel(), n, 1024) == want, env
