"""The stream-K partition of the decoding-step projections (csrc/linear.hip), replayed on the CPU:
workgroup w streams units [w U / G, (w + 1) U / G); a piece that ends a tile or a range is stored
whole, or as the workgroup's slot-0 (first) or slot-1 (last) partial; the fixup sums, for each tile
a range boundary falls inside, the pieces of the tile's owners w0..w1. Checked: every unit lands in
exactly one stored tile or one summed piece set, the owners from the exact double quotient equal
the integer ones, and the 32-bit start formula equals floor(w U / G)."""

import random

import pytest


def _start(U, G):
    q, r = U // G, U % G
    return lambda w: w * q + (w * r) // G  # the kernel's 32-bit form


def _owner(U, G):
    return lambda u: int(((u + 1) * G - 1.0) / float(U))  # the kernel's double quotient


def _replay(units, ns, G):
    G = min(G, units)
    start, owner = _start(units, G), _owner(units, G)
    part, whole = {}, {}
    for w in range(G):
        u0, n = start(w), start(w + 1) - start(w)
        assert n >= 1
        tile, step = divmod(u0, ns)
        pstep0, slot, acc = step, 0, set()
        for j in range(n):
            acc.add(tile * ns + step)
            if step == ns - 1 or j == n - 1:  # the piece ends
                if pstep0 == 0 and step == ns - 1:
                    assert tile not in whole
                    whole[tile] = acc
                else:
                    assert (w, slot) not in part
                    part[(w, slot)] = acc
                acc, slot, pstep0 = set(), 1, 0
            step += 1
            if step == ns:
                step, tile = 0, tile + 1
    # the host's list: tiles a boundary falls inside, consecutive duplicates dropped
    listed = []
    for b in range(1, G):
        ub = start(b)
        if ub % ns and (not listed or listed[-1] != ub // ns):
            listed.append(ub // ns)
    assert len(set(listed)) == len(listed)
    for t in range(units // ns):
        t0, full = t * ns, set(range(t * ns, t * ns + ns))
        w0, w1 = owner(t0), owner(t0 + ns - 1)
        if w0 == w1:
            assert whole[t] == full and t not in listed
            continue
        assert t in listed and t not in whole
        got = set()
        for w in range(w0, w1 + 1):
            slot = (0 if start(w) >= t0 else 1) if w == w0 else 0
            piece = part[(w, slot)]
            assert all(u // ns == t for u in piece) and not (got & piece)
            got |= piece
        assert got == full


@pytest.mark.parametrize("ns", [1, 2, 5, 80, 96])
@pytest.mark.parametrize("tiles", [1, 3, 40, 130, 1187])
@pytest.mark.parametrize("G", [1, 2, 7, 256, 1199, 10 ** 6])
def test_every_unit_is_summed_once(ns, tiles, G):
    _replay(tiles * ns, ns, G)


def test_partition_arithmetic_at_the_limits():
    random.seed(0)
    for U, G in [(2 ** 31 - 1, 32768), (2 ** 31 - 7, 256), (94960, 1187), (3840, 256), (10 ** 9 + 7, 32767)]:
        start, owner = _start(U, G), _owner(U, G)
        for w in list(range(0, G + 1, max(1, G // 500))) + [G]:
            assert start(w) == w * U // G
        for u in random.sample(range(U), 3000) + [0, U - 1]:
            assert owner(u) == ((u + 1) * G - 1) // U
