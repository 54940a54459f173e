"""Drop-in for the reference's ``boa`` module: ``BOA(device, filepath, model) -> BoaFile``.

Reference: boa.py:7-311.  Same BOA2 container, byte for byte:

    b"BOA2" | u32 version=1 | u32 flags=0 | u64 uncompressed_len | u32 chunk_len | u32 n_chunks |
    u32 last_chunk_len | u8 fp_len | fingerprint (blake2s-128 of the model class name) |
    payload (every chunk's u32 little-endian words, back to back) |
    b"IDX1" | first_bytes[n] | n x uvarint(offset delta) | n x uvarint(stream bytes) | u32 CRC32(IDX1..)

Chunking: chunk_len = ceil(n / chunks_count), or seq_size.  Chunks are processed in waves of
BOA_GPU_STREAMS lanes if that is set (as in the reference), otherwise of as many lanes as free device
memory holds.  The payload of a wave comes back from the GPU already compacted (one device-to-host copy),
and is written in one piece.  As in the reference, the reader finds the index with rfind(b"IDX1")
(boa.py:130).

Only ``device="cuda"`` (the ROCm GPU under torch-ROCm) is supported; the reference's CPU branch
(mambapy + constriction) is not part of this build and raises.
"""
from __future__ import annotations

import hashlib
import os
import struct
import zlib
from pathlib import Path

import numpy as np
import torch

__all__ = ["BOA", "BoaFile", "uvarint_encode", "uvarint_decode"]


def uvarint_encode(x: int) -> bytes:
    """LEB128 (boa.py:17-23)."""
    out = bytearray()
    while True:
        b = x & 0x7F
        x >>= 7
        out.append(b | (0x80 if x else 0))
        if not x:
            break
    return bytes(out)


def uvarint_decode(buf, pos: int):
    """boa.py:25-31."""
    x = 0
    s = 0
    while True:
        b = buf[pos]
        pos += 1
        x |= (b & 0x7F) << s
        if not (b & 0x80):
            return x, pos
        s += 7


def _wave_lanes(model, n_chunks: int, chunk_len: int) -> int:
    """Chunks per GPU wave.  BOA_GPU_STREAMS, when set, fixes it as in the reference (boa.py:207-210; an
    unparsable value means 5000); otherwise it is sized from free device memory (the model's
    plan_wave_lanes, after boa.cpp:103-150).  Always within [1, n_chunks]."""
    env = os.getenv("BOA_GPU_STREAMS")
    if env is not None:
        try:
            lanes = int(env)
        except ValueError:
            lanes = 5000
    else:
        lanes = model.plan_wave_lanes(n_chunks, chunk_len)
    return max(1, min(int(lanes), int(n_chunks)))


# BOA2 fixed header: magic, version, flags, uncompressed length, chunk length, chunk count, last chunk
# length, fingerprint length (the fingerprint bytes follow).
_HEADER = struct.Struct("<4sIIQIIIB")
_CRC = struct.Struct("<I")


def _uvarints(buf: bytes, lo: int, hi: int, count: int) -> np.ndarray:
    """The first `count` LEB128 values of buf[lo:hi] as uint64, decoded without a per-value loop: a value ends
    at each byte below 0x80; each byte contributes its low 7 bits shifted by 7 x (its index in the value)."""
    if count == 0:
        return np.zeros(0, dtype=np.uint64)
    raw = np.frombuffer(buf, dtype=np.uint8, count=hi - lo, offset=lo)
    ends = np.flatnonzero(raw < 0x80)
    if ends.size < count:
        raise ValueError("BOA2 payload out of range")
    ends = ends[:count]
    heads = np.empty(count, dtype=np.int64)
    heads[0] = 0
    heads[1:] = ends[:-1] + 1
    used = raw[:ends[-1] + 1].astype(np.uint64)
    rank = np.arange(used.size, dtype=np.int64) - np.repeat(heads, ends - heads + 1)
    if int(rank.max()) > 9:
        raise ValueError("BOA2 payload out of range")
    parts = (used & np.uint64(0x7F)) << (np.uint64(7) * rank.astype(np.uint64))
    return np.add.reduceat(parts, heads)


def _uvarints_bytes(values) -> bytes:
    """LEB128 of every value, concatenated (the inverse of _uvarints), built without a per-value loop: row i
    of a [n, 10] table holds value i's 7-bit groups, each flagged 0x80 when a nonzero group follows, and the
    first max(1, significant groups) bytes of each row are kept."""
    v = np.asarray(values, dtype=np.uint64).reshape(-1)
    if v.size == 0:
        return b""
    shifts = np.arange(10, dtype=np.uint64) * np.uint64(7)  # 10 groups cover 64 bits
    groups = (v[:, None] >> shifts[None, :]) & np.uint64(0x7F)
    more = np.zeros(groups.shape, dtype=bool)
    more[:, :9] = (v[:, None] >> (shifts[None, :9] + np.uint64(7))) != 0
    keep = np.arange(10)[None, :] < 1 + more.sum(axis=1)[:, None]
    return (groups | np.where(more, np.uint64(0x80), np.uint64(0))).astype(np.uint8)[keep].tobytes()


class BoaFile:
    MAGIC = b"BOA2"
    IDX = b"IDX1"
    VERSION = 1

    def __init__(self, filepath: str, model, device: str = "cuda"):
        self.filepath = Path(filepath)
        self.model = model
        self.device = device
        self.compressed_data = []
        self.first_bytes = []
        self.lengths = []
        self.metadata = {}

    # boa.py:85-87
    def _model_fingerprint(self) -> bytes:
        name = getattr(self.model, "__class__", type(self.model)).__name__
        return hashlib.blake2s(name.encode(), digest_size=16).digest()

    @staticmethod
    def _chunking(total_size: int, seq_size: int, chunks_count: int):
        """(chunk_len, n_chunks, last_chunk_len) for a file of total_size bytes (boa.py:169-178 semantics).

        seq_size, when given, is the chunk length (it wins over chunks_count); otherwise the file is cut into
        chunks_count pieces of ceil(total / chunks_count) bytes.  A count so large that the tail would hold
        empty chunks yields fewer chunks: the reference's compress would pass empty chunks on to
        compress_GPU's length assertion (boa.py:224-233, codec.py:25), its _split_to_chunks drops them
        (boa.py:73-77), and so does this."""
        if seq_size:
            step = int(seq_size)
        elif chunks_count:
            step = -(-int(total_size) // max(int(chunks_count), 1))
        else:
            raise ValueError("Provide either 'seq_size' or 'chunks_count'.")
        count = max(-(-int(total_size) // step), 1)
        return step, count, int(total_size) - (count - 1) * step

    @classmethod
    def _index(cls, first_bytes, lengths) -> bytes:
        """The BOA2 index (without its CRC): b"IDX1", the first byte of every chunk, then the streams' offsets
        in the payload as deltas from the previous offset (the first is 0, each next one the previous stream's
        length), then the streams' lengths in bytes, all as uvarints."""
        lengths = np.asarray(lengths, dtype=np.uint64)
        deltas = np.concatenate([np.zeros(min(1, lengths.size), dtype=np.uint64), lengths[:-1]])
        return cls.IDX + bytes(first_bytes) + _uvarints_bytes(deltas) + _uvarints_bytes(lengths)

    def _read_file(self):
        """Parses a BOA2 file into compressed_data / first_bytes / lengths / metadata (boa.py:114-157).

        Layout: a fixed header `_HEADER` followed by fp_len fingerprint bytes, the payload, then the index
        b"IDX1" | first_bytes[n] | n uvarint offset deltas | n uvarint stream lengths | u32 CRC32 of the
        index.  The index is located with rfind(b"IDX1"), as the reference reader does (boa.py:130); the
        uvarints are decoded in one vectorised pass; every stream must lie inside the payload and hold
        whole u32 words."""
        blob = Path(self.filepath).read_bytes()
        if len(blob) < _HEADER.size or blob[:4] != self.MAGIC:
            raise ValueError("Bad file magic")
        _magic, version, _flags, ulen, chunk_len, n, last_chunk_len, fp_len = _HEADER.unpack_from(blob, 0)
        if version != self.VERSION:
            raise ValueError(f"Unsupported version {version}")
        body = _HEADER.size + fp_len
        at = blob.rfind(self.IDX)
        if at < 0:
            raise ValueError("Index not found")
        (crc,) = _CRC.unpack_from(blob, len(blob) - _CRC.size)
        if zlib.crc32(blob[at:len(blob) - _CRC.size]) & 0xFFFFFFFF != crc:
            raise ValueError("Bad index CRC")
        fb_at = at + len(self.IDX)
        first = list(blob[fb_at:fb_at + n])
        fields = _uvarints(blob, fb_at + n, len(blob) - _CRC.size, 2 * n)
        deltas, sizes = fields[:n], fields[n:]
        starts = np.cumsum(deltas)
        room = at - body
        # boa.cpp:240's check (the Python reader has none): every stream inside the payload, in whole words.  With
        # each delta at most the payload's size, a running offset that wraps 2^64 shows as a decrease; with the
        # last (largest) offset inside the payload, start + size cannot wrap either.
        if n and (int(deltas.max()) > room or bool((starts[1:] < starts[:-1]).any()) or int(starts[-1]) > room
                  or int(sizes.max()) > room or int((starts + sizes).max()) > room or bool((sizes & 3).any())):
            raise ValueError("BOA2 payload out of range")
        view = memoryview(blob)[body:at]
        self.compressed_data = [bytes(view[s:s + z]) for s, z in zip(starts.tolist(), sizes.tolist())]
        self.first_bytes = first
        self.lengths = [int(chunk_len)] * (n - 1) + [int(last_chunk_len)] if n else []
        self.metadata = {
            "chunk_len": int(chunk_len),
            "n_chunks": int(n),
            "last_chunk_len": int(last_chunk_len),
            "uncompressed_len": int(ulen),
        }

    def compress(self, data_path: str, seq_size: int = 0, chunks_count: int = 0, progress: bool = True):
        # boa.py:159-268
        from codec import compress_payload

        p = Path(data_path)
        total_size = p.stat().st_size
        if total_size <= 0:
            raise ValueError("Input file is empty")
        chunk_len, n_chunks, last_chunk_len = self._chunking(total_size, seq_size, chunks_count)
        self.metadata = {
            "chunk_len": int(chunk_len),
            "n_chunks": int(n_chunks),
            "uncompressed_len": int(total_size),
            "last_chunk_len": int(last_chunk_len if last_chunk_len else chunk_len),
        }
        fp = self._model_fingerprint()
        mm = np.memmap(p, dtype=np.uint8, mode="r")
        streams = _wave_lanes(self.model, n_chunks, chunk_len)
        if progress:
            print(f"[compress] gpu_streams={streams} (chunk_len={chunk_len})")
        lengths, first_bytes = [], []
        with torch.inference_mode(), open(self.filepath, "wb") as f_out:
            f_out.write(_HEADER.pack(self.MAGIC, self.VERSION, 0, total_size, chunk_len, n_chunks, last_chunk_len,
                                     len(fp)) + fp)
            for b0 in range(0, n_chunks, streams):
                b1 = min(b0 + streams, n_chunks)
                chunks = [mm[i * chunk_len:min((i + 1) * chunk_len, total_size)] for i in range(b0, b1)]
                payload, nw, fb, _Ls = compress_payload(self.model, chunks)
                f_out.write(payload.astype("<u4", copy=False).tobytes())
                lengths.extend(int(w) * 4 for w in nw)
                first_bytes.extend(int(b) & 0xFF for b in fb)
            idx = self._index(first_bytes, lengths)
            f_out.write(idx + _CRC.pack(zlib.crc32(idx) & 0xFFFFFFFF))
        self.compressed_data = []
        self.first_bytes = first_bytes
        self.lengths = [chunk_len] * (n_chunks - 1) + [last_chunk_len]
        if progress:
            print(f"Compression complete: {n_chunks} chunks, chunk_len={chunk_len}, last={last_chunk_len}")

    def read_from_disk(self):
        self._read_file()
        print("File loaded successfully")

    def decompress(self, progress: bool = True) -> bytes:
        # boa.py:274-308
        from codec import decompress_payload

        self._read_file()
        if progress:
            print(f"Total compressed size from disk: {sum(len(c) for c in self.compressed_data)} bytes")
        n = len(self.compressed_data)
        streams = _wave_lanes(self.model, max(n, 1), max(self.lengths, default=1))
        parts = []
        with torch.inference_mode():
            for b0 in range(0, n, streams):
                b1 = min(b0 + streams, n)
                comp = self.compressed_data[b0:b1]
                nw = [len(c) // 4 for c in comp]
                payload = np.frombuffer(b"".join(comp), dtype="<u4").astype(np.uint32)
                lens = self.lengths[b0:b1]
                out = decompress_payload(self.model, payload, nw, lens, self.first_bytes[b0:b1])
                for i, L in enumerate(lens):
                    parts.append(out[i, :L].tobytes())
        return b"".join(parts)

    def get_metadata(self):
        return dict(self.metadata)


def BOA(device, filepath: str, model):
    """boa.py:7-15: returns a BoaFile bound to filepath and model.  device must be "cuda"."""
    if not (device == "cuda" and torch.cuda.is_available()):
        raise RuntimeError("BOA: only device='cuda' (the ROCm GPU) is supported by this build")
    return BoaFile(filepath, model, device="cuda")
