"""Independent big-integer check of a range coder's output words (TEST INFRASTRUCTURE ONLY).

This does not restate the u64/u32 word-level encoder (carry tracking through "inverted" words, finalize).
It tracks the coder's interval with unbounded Python integers instead:

    interval = [L, L + R) in units of 2^-(64 + shift)

starting from L = 0, R = 2^64 - 1.  Per symbol with quantised sub-interval [left, left + prob) out of 2^P
(the same truncating arithmetic the reference coder defines: scale = R >> P, gpu_range_coder.py:100-105):

    L += (R >> P) * left ;  R = (R >> P) * prob ;  while R < 2^32: L <<= 32; R <<= 32; shift += 32

A correct encoder's words w_0 .. w_{n-1}, read as the base-2^32 fraction x = sum w_i 2^(-32(i+1)) and
padded with zero words as the reference decoder pads (gpu_range_coder.py:177,207), must satisfy

    L / 2^(64+shift)  <=  x  <  (L + R) / 2^(64+shift)

which is what the decoder needs to recover every symbol.  Carry mistakes, dropped or duplicated words and a
wrong point word all violate it.  An empty symbol sequence must give zero words.
"""
from __future__ import annotations

from typing import Iterable, Sequence, Tuple


def interval(steps: Iterable[Tuple[int, int]], P: int):
    L, R, shift = 0, (1 << 64) - 1, 0
    n = 0
    for left, prob in steps:
        scale = R >> P
        L += scale * int(left)
        R = scale * int(prob)
        while R < (1 << 32):
            L <<= 32
            R <<= 32
            shift += 32
        n += 1
    return L, R, shift, n


def check(words: Sequence[int], steps: Sequence[Tuple[int, int]], P: int) -> None:
    """Raise AssertionError unless ``words`` encode ``steps`` (a list of (left, prob)) at precision P."""
    L, R, shift, n = interval(steps, P)
    words = [int(w) & 0xFFFFFFFF for w in words]
    if n == 0:
        assert len(words) == 0, f"empty stream must produce no words, got {len(words)}"
        return
    committed = shift // 32
    assert len(words) in (committed + 1, committed + 2), (
        f"word count {len(words)} not in {{{committed + 1}, {committed + 2}}}")
    W = 0
    for w in words:
        W = (W << 32) | w
    nbits = 32 * len(words)
    # compare x = W / 2^nbits with [L, L+R) / 2^(64+shift) by cross-multiplying
    lhs = W << (64 + shift)
    assert (L << nbits) <= lhs, "code value below the final interval"
    assert lhs < ((L + R) << nbits), "code value above the final interval"
