"""(CPU) The cross-workgroup combine of row pieces, ``tg_mp_commit``, as a
model run under every interleaving of its atomic operations (two pieces) or
under many random ones (three to five pieces).

Each piece is a process whose steps are the atomics one wave performs on the
scratch slots, in program order: for two pieces, one swap into the first
piece's slot (and, for the piece that finds its partner's partial there, a
swap that empties it); for more, a swap into its own slot, then one read per
slot of the row (each its own atomic, in any order against other pieces'
atomics), then, if every read found a partial, one emptying swap per slot.
Whatever the order:

* at least one piece combines, and every combiner gets the sum of the pieces
  in window order, bit for bit (two pieces: mine + other in window order;
  more: a fixed tree over the lane-ordered partials, as the wave's reduction);
* every slot is empty when all pieces are done, so the next launch starts clean.
"""

from __future__ import annotations

import itertools
import random
import struct

import numpy as np

KEY = 0x7FF4A5A5A5A5A5A5


def bits(v: float) -> int:
    return struct.unpack("<Q", struct.pack("<d", v))[0]


def val(b: int) -> float:
    return struct.unpack("<d", struct.pack("<Q", b))[0]


def segsum64(vals):
    """The wave's butterfly sum over 64 lanes (lanes past the row add 0.0), as
    tg_segsum<64>: pairwise exchanges at distances 1, 2, 4, 8, 16, 32."""
    v = list(vals) + [0.0] * (64 - len(vals))
    for m in (1, 2, 4, 8, 16, 32):
        v = [v[i] + v[i ^ m] for i in range(64)]
    return v[0]


def piece(slots, n, w, t, out):
    """Window w's piece (of windows 0..n-1) as a sequence of atomic steps; each
    ``yield`` hands the turn back to the scheduler."""
    if n == 2:
        yield
        other, slots[1] = slots[1], bits(t) ^ KEY      # swap into the first piece's slot
        if other == 0:
            return
        o = val(other ^ KEY)
        out.append(t + o if w == 0 else o + t)
        yield
        slots[1] = 0                                   # empty it
        return
    yield
    slots[2 * w + (1 if w == 0 else 0)] = bits(t) ^ KEY  # the swap (its old value is unused)
    seen = {}
    for j in random.sample(range(n), n):               # the lanes' reads, in any order
        yield
        seen[j] = slots[2 * j + (1 if j == 0 else 0)]
    if any(seen[j] == 0 for j in range(n)):
        return
    out.append(segsum64([val(seen[j] ^ KEY) for j in range(n)]))
    for j in random.sample(range(n), n):
        yield
        slots[2 * j + (1 if j == 0 else 0)] = 0


def run(order_pick, n, parts):
    slots = [0] * (2 * n + 2)
    out = []
    procs = [piece(slots, n, w, parts[w], out) for w in range(n)]
    live = list(range(n))
    while live:
        k = order_pick(live)
        try:
            next(procs[k])
        except StopIteration:
            live.remove(k)
    return slots, out


def _expected(parts):
    if len(parts) == 2:
        return parts[0] + parts[1]
    return segsum64(parts)


def test_two_pieces_every_interleaving():
    rng = np.random.default_rng(0)
    for _ in range(50):
        parts = [float(v) for v in rng.uniform(-1e3, 1e3, 2)]
        want = _expected(parts)
        # every sequence of scheduler choices over the two processes' 2-3 steps
        for seq in itertools.product([0, 1], repeat=8):
            it = iter(seq)

            def pick(live):
                c = next(it, 0)
                return live[c % len(live)]
            slots, out = run(pick, 2, parts)
            assert out and all(bits(o) == bits(want) for o in out), (parts, seq, out)
            assert not any(slots), (parts, seq, slots)


def test_more_pieces_random_interleavings():
    random.seed(1)
    rng = np.random.default_rng(1)
    for n in (3, 4, 5):
        for _ in range(400):
            parts = [float(v) for v in rng.uniform(-1e3, 1e3, n)]
            want = _expected(parts)
            slots, out = run(lambda live: random.choice(live), n, parts)
            assert out and all(bits(o) == bits(want) for o in out), (n, parts, out)
            assert not any(slots), (n, slots)


def test_two_piece_sum_is_in_window_order():
    """The combiner adds in window order whichever piece arrives last, so the
    bits do not depend on arrival (a + b and b + a round alike, and the model
    checks the exact expression the kernel writes)."""
    for first in (0, 1):
        slots, out = run(lambda live: live[0] if first in live and len(live) == 2 and
                         live[0] == first else live[-1], 2, [0.1, 0.2])
        assert out and bits(out[0]) == bits(0.1 + 0.2)
