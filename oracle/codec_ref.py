"""CPU restatement of codec.compress_CPU / decompress_CPU (TEST INFRASTRUCTURE ONLY: the reported CPU
baseline of bench.py and a checker in tests).

Follows codec.py:153-323 step for step: first byte raw; for t = 1..maxL-1 one batched model step over all
lanes (torch CPU, float32), softmax, then lane-wise coding in a ThreadPoolExecutor(num_workers) created
anew each step, lanes split into num_workers contiguous ranges; finished lanes are skipped and keep their
previous byte.  The model step is oracle.model_ref (mambapy's MambaBlock.step arithmetic); the per-lane
coder is the C restatement in rc_oracle.c with the Q2 quantiser at PRECISION 24 standing in for
constriction's Categorical(perfect=False) + RangeEncoder (constriction 0.4.1 is not installed; parity with
it is unpinned).  ctypes releases the GIL during each coder call, so the pool runs lanes in parallel as
constriction's Rust calls do.
"""
from __future__ import annotations

import ctypes
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from . import ora


def _bind():
    L = ora.lib()
    if not hasattr(L, "_codec_bound"):
        vp = ctypes.c_void_p
        L.ora_enc_sizeof.restype = ctypes.c_size_t
        L.ora_dec_sizeof.restype = ctypes.c_size_t
        L.ora_enc_init.argtypes = [vp]
        L.ora_enc_finish.argtypes = [vp, vp, ctypes.c_int64]
        L.ora_enc_finish.restype = ctypes.c_int64
        L.ora_dec_init.argtypes = [vp, vp, ctypes.c_int64]
        L.ora_q2_encode_one.argtypes = [vp, ctypes.c_int, vp, ctypes.c_int, ctypes.c_int, vp, ctypes.c_int64]
        L.ora_q2_decode_one.argtypes = [vp, ctypes.c_int, vp, ctypes.c_int, vp, ctypes.c_int64]
        L.ora_q2_decode_one.restype = ctypes.c_int
        L._codec_bound = True
    return L


P = 24


@torch.inference_mode()
def compress_cpu(model, chunks, num_workers: int = 8, max_steps: int | None = None):
    """model: oracle.model_ref.RefModel; chunks: list of 1-D uint8 arrays.  Returns
    (list of uint32 word arrays, first_bytes, lens, steps_run)."""
    L = _bind()
    N = len(chunks)
    Ls = [int(len(c)) for c in chunks]
    maxL = max(Ls)
    X = np.zeros((N, maxL), dtype=np.int64)
    for i, c in enumerate(chunks):
        X[i, :Ls[i]] = c
    first_bytes = X[:, 0].tolist()
    esz = L.ora_enc_sizeof()
    states = ctypes.create_string_buffer(esz * N)
    for i in range(N):
        L.ora_enc_init(ctypes.addressof(states) + i * esz)
    caps = [L_ + 8 for L_ in Ls]
    outs = [np.zeros(c, dtype=np.uint32) for c in caps]
    caches = model.init_state(N)
    prev = torch.from_numpy(X[:, 0].copy())
    Xt = torch.from_numpy(X)
    K = model.cfg.vocab
    last = maxL if max_steps is None else min(maxL, 1 + max_steps)

    def encode_range(r0, r1, t, probs_np):
        base = probs_np.ctypes.data
        for i in range(r0, r1):
            if t < Ls[i]:
                L.ora_q2_encode_one(ctypes.addressof(states) + i * esz, P, base + 4 * K * i, K, int(X[i, t]),
                                    outs[i].ctypes.data, caps[i])

    steps = 0
    for t in range(1, last):
        active = np.asarray(Ls) > t
        if not active.any():
            break
        logits = model.step(prev, caches)
        probs_np = np.ascontiguousarray(torch.softmax(logits, dim=-1).to(torch.float32).numpy())
        if num_workers and num_workers > 1:
            chunk = (N + num_workers - 1) // num_workers
            with ThreadPoolExecutor(max_workers=num_workers) as pool:
                futs = [pool.submit(encode_range, s, min(s + chunk, N), t, probs_np) for s in range(0, N, chunk)]
                for f in futs:
                    f.result()
        else:
            encode_range(0, N, t, probs_np)
        prev = torch.where(torch.from_numpy(active), Xt[:, t], prev)
        steps += 1
    words = []
    for i in range(N):
        n = L.ora_enc_finish(ctypes.addressof(states) + i * esz, outs[i].ctypes.data, caps[i])
        words.append(outs[i][:n].copy())
    return words, first_bytes, Ls, steps


@torch.inference_mode()
def decompress_cpu(model, words, lens, first_bytes, num_workers: int = 8, max_steps: int | None = None):
    """Inverse of compress_cpu (codec.py:242-323).  Returns (list of uint8 arrays, steps_run)."""
    L = _bind()
    N = len(words)
    maxL = max(lens)
    dsz = L.ora_dec_sizeof()
    states = ctypes.create_string_buffer(dsz * N)
    ws = [np.ascontiguousarray(w, dtype=np.uint32) if len(w) else np.zeros(1, np.uint32) for w in words]
    for i in range(N):
        L.ora_dec_init(ctypes.addressof(states) + i * dsz, ws[i].ctypes.data, len(words[i]))
    outs = [np.zeros(n, dtype=np.uint8) for n in lens]
    for i in range(N):
        outs[i][0] = int(first_bytes[i])
    caches = model.init_state(N)
    prev_np = np.array(first_bytes, dtype=np.int64)
    prev = torch.from_numpy(prev_np.copy())
    K = model.cfg.vocab
    last = maxL if max_steps is None else min(maxL, 1 + max_steps)

    def decode_range(r0, r1, t, probs_np):
        base = probs_np.ctypes.data
        for i in range(r0, r1):
            if t < lens[i]:
                s = L.ora_q2_decode_one(ctypes.addressof(states) + i * dsz, P, base + 4 * K * i, K,
                                        ws[i].ctypes.data, len(words[i]))
                outs[i][t] = s
                prev_np[i] = s

    steps = 0
    for t in range(1, last):
        if not (np.asarray(lens) > t).any():
            break
        logits = model.step(prev, caches)
        probs_np = np.ascontiguousarray(torch.softmax(logits, dim=-1).to(torch.float32).numpy())
        if num_workers and num_workers > 1:
            chunk = (N + num_workers - 1) // num_workers
            with ThreadPoolExecutor(max_workers=num_workers) as pool:
                futs = [pool.submit(decode_range, s, min(s + chunk, N), t, probs_np) for s in range(0, N, chunk)]
                for f in futs:
                    f.result()
        else:
            decode_range(0, N, t, probs_np)
        prev = torch.from_numpy(prev_np.copy())
        steps += 1
    return outs, steps
