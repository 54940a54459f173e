"""boa_compact_noalloc (compaction with the scan scratch in a fixed device array, no allocation) gives the
same offsets, payload and total as boa_compact, on two calls in a row, the second with fewer lanes; rejects a
wave beyond its static maximum before touching the GPU; and reports a payload capacity below the total or a word
count beyond the pitch without writing anything."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(rng, lanes, pitch):
    nw = rng.integers(0, pitch + 1, lanes).astype(np.int32)
    words = rng.integers(0, 1 << 31, (lanes, pitch)).astype(np.int32)
    return nw, words


def _run(gpu, fn, nw, words, pitch):
    from boa_amd import _native as N

    lanes = nw.size
    d_words = torch.from_numpy(words).cuda()
    d_nw = torch.from_numpy(nw).cuda()
    d_off = torch.full((lanes,), -1, dtype=torch.int64, device="cuda")
    cap = int(nw.sum())
    d_pl = torch.zeros(max(cap, 1), dtype=torch.int32, device="cuda")
    got = ctypes.c_int64(-1)
    N.check(getattr(gpu, fn)(N.ptr(d_words), pitch, N.ptr(d_nw), lanes, N.ptr(d_off), N.ptr(d_pl), cap,
                             ctypes.byref(got), N.stream_ptr()))
    return got.value, d_off.cpu().numpy(), d_pl.cpu().numpy()[:cap]


def test_noalloc_matches_compact_twice(gpu):
    rng = np.random.default_rng(21)
    for lanes, pitch in ((5000, 40), (1500, 24)):  # the second call is smaller: stale partials must not leak
        nw, words = _case(rng, lanes, pitch)
        t_ref, off_ref, pl_ref = _run(gpu, "boa_compact", nw, words, pitch)
        t_new, off_new, pl_new = _run(gpu, "boa_compact_noalloc", nw, words, pitch)
        assert t_new == t_ref == int(nw.sum())
        assert np.array_equal(off_new, off_ref)
        assert np.array_equal(pl_new, pl_ref)
        assert np.array_equal(off_ref, np.concatenate([[0], np.cumsum(nw)[:-1]]))


def test_noalloc_limits(gpu):
    from boa_amd import _native as N

    got = ctypes.c_int64(0)
    one = torch.zeros(1, dtype=torch.int32, device="cuda")
    off = torch.zeros(1, dtype=torch.int64, device="cuda")
    rc = gpu.boa_compact_noalloc(N.ptr(one), 1, N.ptr(one), 262145, N.ptr(off), N.ptr(one), 1, ctypes.byref(got),
                                 N.stream_ptr())
    assert rc == N.BOA_ERR_ARG and b"262144" in gpu.boa_last_error()
    # a payload capacity below the total is reported, not written past
    rng = np.random.default_rng(3)
    nw, words = _case(rng, 300, 8)
    d_words, d_nw = torch.from_numpy(words).cuda(), torch.from_numpy(nw).cuda()
    d_off = torch.empty(300, dtype=torch.int64, device="cuda")
    small = torch.zeros(4, dtype=torch.int32, device="cuda")
    rc = gpu.boa_compact_noalloc(N.ptr(d_words), 8, N.ptr(d_nw), 300, N.ptr(d_off), N.ptr(small), 4,
                                 ctypes.byref(got), N.stream_ptr())
    assert rc == N.BOA_ERR_OVERFLOW and got.value == int(nw.sum())
    # a word count beyond the pitch is an argument error, nothing gathered; the next valid call is unaffected
    bad = nw.copy()
    bad[150] = 9
    d_bad = torch.from_numpy(bad).cuda()
    cap = int(bad.sum())
    d_pl = torch.full((cap,), 7, dtype=torch.int32, device="cuda")
    rc = gpu.boa_compact_noalloc(N.ptr(d_words), 8, N.ptr(d_bad), 300, N.ptr(d_off), N.ptr(d_pl), cap,
                                 ctypes.byref(got), N.stream_ptr())
    assert rc == N.BOA_ERR_ARG and got.value == 0 and bool((d_pl == 7).all())
    t_ref, off_ref, pl_ref = _run(gpu, "boa_compact", nw, words, 8)
    t_new, off_new, pl_new = _run(gpu, "boa_compact_noalloc", nw, words, 8)
    assert t_new == t_ref and np.array_equal(off_new, off_ref) and np.array_equal(pl_new, pl_ref)
