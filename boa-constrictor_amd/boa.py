"""Drop-in for the reference's ``boa`` module: ``BOA(device, filepath, model) -> BoaFile``.

Reference: boa.py:7-311.  Same BOA2 container, byte for byte:

    b"BOA2" | u32 version=1 | u32 flags=0 | u64 uncompressed_len | u32 chunk_len | u32 n_chunks |
    u32 last_chunk_len | u8 fp_len | fingerprint (blake2s-128 of the model class name) |
    payload (every chunk's u32 little-endian words, back to back) |
    b"IDX1" | first_bytes[n] | n x uvarint(offset delta) | n x uvarint(stream bytes) | u32 CRC32(IDX1..)

Chunking: chunk_len = ceil(n / chunks_count), or seq_size; chunks are processed in waves of
BOA_GPU_STREAMS (default 5000) lanes.  The payload of a wave comes back from the GPU already compacted
(one device-to-host copy), and is written in one piece.  As in the reference, the reader finds the index
with rfind(b"IDX1") (boa.py:130).

Only ``device="cuda"`` (the ROCm GPU under torch-ROCm) is supported; the reference's CPU branch
(mambapy + constriction) is not part of this build and raises.
"""
from __future__ import annotations

import hashlib
import math
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


def _streams_env() -> int:
    try:
        return int(os.getenv("BOA_GPU_STREAMS", "5000"))
    except Exception:
        return 5000


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
        # boa.py:169-178
        if seq_size and chunks_count:
            chunk_len = int(seq_size); n_chunks = math.ceil(total_size / chunk_len)
        elif seq_size:
            chunk_len = int(seq_size); n_chunks = math.ceil(total_size / chunk_len)
        elif chunks_count:
            n_chunks = max(int(chunks_count), 1); chunk_len = math.ceil(total_size / n_chunks)
        else:
            raise ValueError("Provide either 'seq_size' or 'chunks_count'.")
        # chunks_count larger than ceil(n / chunk_len) would leave empty trailing chunks, which the reference's
        # compress passes on to compress_GPU's length assertion (boa.py:224-233, codec.py:25); they are dropped
        # here instead, as _split_to_chunks does (boa.py:73-77)
        n_chunks = min(n_chunks, math.ceil(total_size / chunk_len))
        last = int(total_size - (n_chunks - 1) * chunk_len) if n_chunks > 1 else int(total_size)
        return int(chunk_len), int(n_chunks), int(last)

    def _read_file(self):
        # boa.py:114-157
        data = Path(self.filepath).read_bytes()
        mm = memoryview(data)
        p = 0
        if bytes(mm[p:p + 4]) != self.MAGIC:
            raise ValueError("Bad file magic")
        p += 4
        version, = struct.unpack_from("<I", mm, p); p += 4
        if version != self.VERSION:
            raise ValueError(f"Unsupported version {version}")
        _flags, = struct.unpack_from("<I", mm, p); p += 4
        ulen, = struct.unpack_from("<Q", mm, p); p += 8
        chunk_len, = struct.unpack_from("<I", mm, p); p += 4
        n, = struct.unpack_from("<I", mm, p); p += 4
        last_chunk_len, = struct.unpack_from("<I", mm, p); p += 4
        hlen = mm[p]; p += 1
        _fp = bytes(mm[p:p + hlen]); p += hlen

        crc = struct.unpack_from("<I", mm, len(mm) - 4)[0]
        idx_pos = data.rfind(self.IDX)
        if idx_pos < 0:
            raise ValueError("Index not found")
        if (zlib.crc32(data[idx_pos:len(data) - 4]) & 0xFFFFFFFF) != crc:
            raise ValueError("Bad index CRC")
        q = idx_pos + len(self.IDX)
        first_bytes = list(mm[q:q + n]); q += n
        offsets = [0] * n; pos = q; prev = 0
        for i in range(n):
            d, pos = uvarint_decode(mm, pos); prev += d; offsets[i] = prev
        comp_lens = [0] * n
        for i in range(n):
            L, pos = uvarint_decode(mm, pos); comp_lens[i] = L
        payload = mm[p:idx_pos]
        for i in range(n):  # boa.cpp:240 bounds check (the Python reader slices silently)
            if offsets[i] + comp_lens[i] > len(payload) or comp_lens[i] % 4:
                raise ValueError("BOA2 payload out of range")
        self.compressed_data = [bytes(payload[offsets[i]:offsets[i] + comp_lens[i]]) for i in range(n)]
        self.first_bytes = first_bytes
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
        streams = max(1, min(_streams_env(), n_chunks))
        if progress:
            print(f"[compress] gpu_streams={streams} (chunk_len={chunk_len})")
        lengths, first_bytes = [], []
        with torch.inference_mode(), open(self.filepath, "wb") as f_out:
            f_out.write(self.MAGIC)
            f_out.write(struct.pack("<I", self.VERSION))
            f_out.write(struct.pack("<I", 0))
            f_out.write(struct.pack("<Q", total_size))
            f_out.write(struct.pack("<I", chunk_len))
            f_out.write(struct.pack("<I", n_chunks))
            f_out.write(struct.pack("<I", last_chunk_len))
            f_out.write(struct.pack("<B", len(fp)))
            f_out.write(fp)
            for b0 in range(0, n_chunks, streams):
                b1 = min(b0 + streams, n_chunks)
                chunks = [mm[i * chunk_len:min((i + 1) * chunk_len, total_size)] for i in range(b0, b1)]
                payload, nw, fb, _Ls = compress_payload(self.model, chunks)
                f_out.write(payload.astype("<u4", copy=False).tobytes())
                lengths.extend(int(w) * 4 for w in nw)
                first_bytes.extend(int(b) & 0xFF for b in fb)
            idx = bytearray(self.IDX)
            idx += bytes(first_bytes)
            prev, off = 0, 0
            for L in lengths:
                idx += uvarint_encode(off - prev)
                prev = off
                off += L
            for L in lengths:
                idx += uvarint_encode(L)
            f_out.write(idx)
            f_out.write(struct.pack("<I", zlib.crc32(idx) & 0xFFFFFFFF))
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
        streams = max(1, min(_streams_env(), max(n, 1)))
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
