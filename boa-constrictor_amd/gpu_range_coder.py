"""Drop-in for the reference's ``gpu_range_coder`` module: ``gpu.queue.RangeCoderBatch``.

Reference: gpu_range_coder.py:488-550 (Python wrapper) over the pybind holder compiled with nvcc at import
time (gpu_range_coder.py:14-375).  Here the holder is libboa_hip.so's ``rcb_*`` C ABI (include/boa_hip.h),
built ahead of time; nothing is compiled at import.

Semantics kept: one range-coder lane per stream, u64 state / u32 words, PRECISION 24, the reference's Q2
quantiser (build_cdf_fast: sequential double accumulation) applied to the given probabilities, masked
lanes and out-of-range symbols skipped, pitch = max(256, maxL * 8) bytes by default, and the same
exceptions (AssertionError for bad tensors, RuntimeError for list/pitch errors).  Difference: calls are
asynchronous on the current torch stream instead of ending in cudaDeviceSynchronize; methods that return
host data synchronize.

The reference module's constriction look-alike ``stream`` namespace (gpu_range_coder.py:384-485) is not
provided: it depends on extension symbols the reference never builds and cannot run there either.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from boa_amd import _native as _nat

__all__ = ["gpu"]


class _RangeCoderBatch:
    def __init__(self, N: int, K: int, maxL: int, pitch_bytes: int | None = None):
        if pitch_bytes is None:
            pitch_bytes = max(256, maxL * 8)
        self.N, self.K, self.maxL = int(N), int(K), int(maxL)
        self.pitch_words = (int(pitch_bytes) + 3) // 4
        self._lib = _nat.lib()
        h = ctypes.c_void_p()
        _nat.check(self._lib.rcb_create(self.N, self.K, self.pitch_words, _nat.stream_ptr(), ctypes.byref(h)))
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.rcb_destroy(h)
            self._h = None

    # gpu_range_coder.py:505-507 -> :237-253
    def load_compressed_list(self, compressed_list):
        if len(compressed_list) != self.N:
            raise RuntimeError("compressed_list length must equal N")
        arrs, sizes = [], np.zeros(self.N, dtype=np.int32)
        for i, c in enumerate(compressed_list):
            a = np.asarray(c)
            if a.ndim != 1 or a.itemsize != 4 or a.dtype.kind != "u":
                raise RuntimeError("Each compressed item must be uint32[?]")
            if a.shape[0] > self.pitch_words:
                raise RuntimeError("Compressed stream exceeds pitch; increase pitch")
            arrs.append(np.ascontiguousarray(a, dtype=np.uint32))
            sizes[i] = a.shape[0]
        words = np.concatenate(arrs) if sizes.sum() else np.zeros(1, dtype=np.uint32)
        _nat.check(self._lib.rcb_load(self._h, _nat.ptr(words), _nat.ptr(sizes)))

    # gpu_range_coder.py:509-527
    def encode_step(self, symbols_gpu, probs_gpu, mask=None):
        assert symbols_gpu.is_cuda and probs_gpu.is_cuda
        assert symbols_gpu.numel() == self.N and tuple(probs_gpu.shape) == (self.N, self.K)
        if symbols_gpu.dtype != torch.int32:
            symbols_gpu = symbols_gpu.to(torch.int32)
        if probs_gpu.dtype != torch.float32:
            probs_gpu = probs_gpu.to(torch.float32)
        symbols_gpu = symbols_gpu.contiguous()
        probs_gpu = probs_gpu.contiguous()
        if mask is not None:
            assert mask.is_cuda and tuple(mask.shape) == (self.N,)
            if mask.dtype != torch.uint8:
                mask = mask.to(torch.uint8)
            mask = mask.contiguous()
        _nat.check(self._lib.rcb_encode_step(self._h, _nat.ptr(symbols_gpu), _nat.ptr(probs_gpu), _nat.ptr(mask)))

    def finalize(self):
        _nat.check(self._lib.rcb_finalize(self._h))

    def get_sizes_list(self):
        sizes = np.zeros(self.N, dtype=np.int32)
        _nat.check(self._lib.rcb_get_sizes(self._h, _nat.ptr(sizes)))
        return [int(s) for s in sizes]

    def get_compressed_list(self):
        sizes = np.asarray(self.get_sizes_list(), dtype=np.int64)
        total = int(sizes.sum())
        words = np.zeros(max(total, 1), dtype=np.uint32)
        got = ctypes.c_int64(0)
        _nat.check(self._lib.rcb_get_words(self._h, _nat.ptr(words), words.size, ctypes.byref(got)))
        offs = np.concatenate([[0], np.cumsum(sizes)])
        return [words[offs[i]:offs[i + 1]].copy() for i in range(self.N)]

    def init_decoder(self):
        _nat.check(self._lib.rcb_init_decoder(self._h))

    # gpu_range_coder.py:535-550
    def decode_step(self, probs_gpu, out_symbols_gpu, mask=None):
        assert probs_gpu.is_cuda and out_symbols_gpu.is_cuda
        assert tuple(probs_gpu.shape) == (self.N, self.K) and out_symbols_gpu.numel() == self.N
        assert out_symbols_gpu.dtype == torch.int32 and out_symbols_gpu.is_contiguous()
        if probs_gpu.dtype != torch.float32:
            probs_gpu = probs_gpu.to(torch.float32)
        probs_gpu = probs_gpu.contiguous()
        if mask is not None:
            assert mask.is_cuda and tuple(mask.shape) == (self.N,)
            if mask.dtype != torch.uint8:
                mask = mask.to(torch.uint8)
            mask = mask.contiguous()
        _nat.check(self._lib.rcb_decode_step(self._h, _nat.ptr(probs_gpu), _nat.ptr(out_symbols_gpu), _nat.ptr(mask)))


class gpu:  # noqa: N801  (name kept from the reference: gr.gpu.queue.RangeCoderBatch)
    class queue:  # noqa: N801
        RangeCoderBatch = _RangeCoderBatch
