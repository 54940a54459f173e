"""Drop-in for the reference's ``codec`` module: ``compress_GPU`` / ``decompress_GPU``.

Reference: codec.py:11-151.  Protocol kept: chunk i's byte 0 is returned raw in ``first_bytes``; bytes
1..L_i-1 are range coded (u32 words, u64 state, PRECISION 24) under next-byte probabilities from the model
run over bytes 0..L_i-2; lanes shorter than the longest chunk stop early; state starts at zero per call.

What runs: one fused C-ABI call each way (libboa_hip.so ``boa_compress`` / ``boa_decompress``) instead
of a Python loop over time steps with host syncs.  Compress runs the model parallel in time (tiles of
positions) and codes each tile; decompress runs one recurrent step per byte on the device, feeding decoded
bytes back without host round trips.  Both use the same kernels and the same deterministic quantiser, so the
decoder sees bit-identical probabilities.  The quantiser is this build's (exact integer cumulative), not
torch.softmax + build_cdf_fast; streams are therefore this build's, not byte-compatible with the
reference's (which are not reproducible across GPUs either, since they depend on float GEMM order).

``compress_CPU`` / ``decompress_CPU`` (codec.py:153-323, the mambapy + constriction path) are not part of
this build; they raise.  The oracle package restates them for the CPU baseline.
"""
from __future__ import annotations

import ctypes
from typing import List, Sequence, Tuple

import numpy as np
import torch

from boa_amd import _native as _nat

__all__ = ["compress_GPU", "decompress_GPU", "compress_payload", "decompress_payload", "compress_CPU",
           "decompress_CPU"]

IS_CUDA = torch.cuda.is_available()


def _pinned(shape, dtype):
    return torch.empty(shape, dtype=dtype, pin_memory=True)


def compress_payload(model, chunks: Sequence[np.ndarray], tile_len: int | None = None):
    """Compresses chunks (1-D uint8 arrays, len >= 1) in one batch.

    Returns (payload uint32 [total], nwords int64 [N], first_bytes list[int], lens list[int]): the lanes'
    streams back to back, which is exactly the BOA2 payload."""
    N = len(chunks)
    Ls = [int(c.shape[-1]) for c in chunks]
    maxL = max(Ls)
    host = _pinned((N, maxL), torch.uint8)
    hv = host.numpy()
    hv[:] = 0
    for i, c in enumerate(chunks):
        hv[i, :Ls[i]] = np.asarray(c, dtype=np.uint8).reshape(-1)
    first_bytes = [int(v) for v in hv[:, 0]]
    dev = torch.device("cuda")
    X = host.to(dev, non_blocking=True)
    lens = torch.tensor(Ls, dtype=torch.int32).to(dev, non_blocking=True)
    eng = model.engine(N, tile_len or min(int(model_tile_len()), max(maxL - 1, 1)))
    pitch = maxL + 8  # at most one word per coded byte plus the finalize words
    words = torch.empty((N, pitch), dtype=torch.int32, device=dev)
    nwords = torch.empty(N, dtype=torch.int32, device=dev)
    L = _nat.lib()
    _nat.check(L.boa_compress(eng.h, _nat.ptr(X), X.stride(0), _nat.ptr(lens), N, maxL, _nat.ptr(words), pitch,
                              _nat.ptr(nwords)))
    nw_host = nwords.cpu().numpy().astype(np.int64)
    total = int(nw_host.sum())
    offs = torch.empty(N, dtype=torch.int64, device=dev)
    payload = torch.empty(max(total, 1), dtype=torch.int32, device=dev)
    got = ctypes.c_int64(0)
    _nat.check(L.boa_compact(_nat.ptr(words), pitch, _nat.ptr(nwords), N, _nat.ptr(offs), _nat.ptr(payload),
                             payload.numel(), ctypes.byref(got), _nat.stream_ptr()))
    out = payload[:total].cpu().numpy().view(np.uint32)
    return out, nw_host, first_bytes, Ls


def decompress_payload(model, payload: np.ndarray, nwords: Sequence[int], full_lens: Sequence[int],
                       first_bytes: Sequence[int]) -> np.ndarray:
    """Inverse of compress_payload.  Returns uint8 [N, max(full_lens)] (row i valid up to full_lens[i])."""
    N = len(full_lens)
    maxL = max(int(v) for v in full_lens)
    nw = np.asarray(nwords, dtype=np.int64)
    offs = np.concatenate([[0], np.cumsum(nw)[:-1]]).astype(np.int64)
    dev = torch.device("cuda")
    pl = np.ascontiguousarray(payload, dtype=np.uint32)
    total = int(pl.size)
    if pl.size == 0:
        pl = np.zeros(1, dtype=np.uint32)
    d_payload = torch.from_numpy(pl.view(np.int32)).to(dev)
    d_off = torch.from_numpy(offs).to(dev)
    d_nw = torch.from_numpy(nw.astype(np.int32)).to(dev)
    d_first = torch.tensor([int(b) & 0xFF for b in first_bytes], dtype=torch.uint8).to(dev)
    d_lens = torch.tensor([int(v) for v in full_lens], dtype=torch.int32).to(dev)
    out = torch.empty((N, maxL), dtype=torch.uint8, device=dev)
    eng = model.engine(N, 1)
    _nat.check(_nat.lib().boa_decompress(eng.h, _nat.ptr(d_payload), total, _nat.ptr(d_off), _nat.ptr(d_nw),
                                         _nat.ptr(d_first), _nat.ptr(d_lens), N, maxL, _nat.ptr(out), out.stride(0)))
    return out.cpu().numpy()


def model_tile_len() -> int:
    from model import DEFAULT_TILE_LEN

    return DEFAULT_TILE_LEN


@torch.inference_mode()
def compress_GPU(model, x_list: List[torch.Tensor], device="cuda", progress=True, num_workers: int = 8):
    """codec.py:11-86.  x_list: N tensors [1, L_i] of bytes.  Returns (list[np.uint32], first_bytes, Ls)."""
    model.eval().to(device)
    N = len(x_list)
    assert N >= 1, "Need at least one chunk."
    chunks = []
    for i, x in enumerate(x_list):
        assert x.ndim == 2 and x.shape[0] == 1, f"Chunk {i} must be [1, L_i]"
        assert x.shape[1] >= 1, f"Chunk {i} must have length >= 1"
        chunks.append(x.detach().to("cpu", dtype=torch.uint8).numpy().reshape(-1))
    payload, nw, first_bytes, Ls = compress_payload(model, chunks)
    offs = np.concatenate([[0], np.cumsum(nw)])
    compressed_list = [payload[offs[i]:offs[i + 1]] for i in range(N)]
    return compressed_list, first_bytes, Ls


def _as_u32(comp) -> np.ndarray:
    # codec.py:257-263
    if isinstance(comp, np.ndarray) and comp.dtype == np.uint32:
        return comp
    if isinstance(comp, np.ndarray) and comp.dtype == np.uint8:
        return comp.view(np.uint32)
    return np.frombuffer(np.asarray(comp).tobytes(), dtype=np.uint32)


def decompress_GPU(model, compressed_list, full_lens: List[int], first_bytes: List[int], device="cuda",
                   progress=True, num_workers: int = 8):
    """codec.py:89-151.  Returns list of np.uint8 arrays shaped (1, L_i)."""
    with torch.inference_mode():
        model.eval().to(device)
        N = len(compressed_list)
        assert N >= 1 and len(full_lens) == N and len(first_bytes) == N
        assert all(L >= 1 for L in full_lens)
        arrs = [_as_u32(c) for c in compressed_list]
        nw = [a.size for a in arrs]
        payload = np.concatenate(arrs) if sum(nw) else np.zeros(0, dtype=np.uint32)
        out = decompress_payload(model, payload, nw, full_lens, first_bytes)
        return [out[i, :int(full_lens[i])].reshape(1, -1) for i in range(N)]


def compress_CPU(*args, **kwargs):
    raise NotImplementedError("the CPU codec (mambapy + constriction, codec.py:153-240) is not part of this build")


def decompress_CPU(*args, **kwargs):
    raise NotImplementedError("the CPU codec (mambapy + constriction, codec.py:242-323) is not part of this build")
