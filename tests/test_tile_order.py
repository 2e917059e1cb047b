"""CPU model of the MFMA core's workgroup -> tile mapping (`xcd_remap` in
pytorch-opt_amd/csrc/gemm_nt.h).

Workgroups go to the 8 XCDs round-robin by linear id (XCD = w % 8). With C
compute units and one tile per CU in flight, workgroups k·C .. k·C + C - 1
run together; the mapping gives them logical tiles k·C .. k·C + C - 1, XCD x
a contiguous block of C/8 of them, and a last partial round (or a launch of
fewer than C tiles) one contiguous range per XCD. Checked here:

* the mapping is a bijection onto 0 .. total - 1 for every total and CU count;
* in every full round the tiles form one contiguous range of C and each XCD's
  share is contiguous (C/8 consecutive tiles);
* in the tail each XCD's share is one contiguous range.

Planted mistakes (the XCD and slot roles swapped, a wrong slot modulus, the
tail without its offset) fail one of these.

The blocked order of upper (symmetric-product) tiles used for bf16 (blocks
of 4 tile rows x 8 tile columns) must enumerate exactly the tiles i <= j.
"""

import pytest

XCDS = 8


def _range(w, total):
    q, r = divmod(total, XCDS)
    xcd, slot = w % XCDS, w // XCDS
    return (xcd * (q + 1) if xcd < r else r * (q + 1) + (xcd - r) * q) + slot


def _remap(w, total, cus, plant=None):
    if cus <= 0 or cus % XCDS:
        return _range(w, total)
    full, per = total // cus * cus, cus // XCDS
    if w < full:
        if plant == "swap":
            return w // cus * cus + (w // XCDS) % per * XCDS + w % XCDS
        if plant == "modulus":
            return w // cus * cus + (w % XCDS) * per + (w // XCDS) % XCDS
        return w // cus * cus + (w % XCDS) * per + (w // XCDS) % per
    if plant == "tail":
        return _range(w - full, total - full)
    return full + _range(w - full, total - full)


def _check(total, cus, plant=None):
    logical = [_remap(w, total, cus, plant) for w in range(total)]
    assert sorted(logical) == list(range(total)), "not a bijection"
    full = total // cus * cus if cus % XCDS == 0 else 0
    per = cus // XCDS
    for k in range(full // cus):
        got = logical[k * cus:(k + 1) * cus]
        assert sorted(got) == list(range(k * cus, (k + 1) * cus)), "round not one contiguous range"
        for x in range(XCDS):
            share = sorted(got[x::XCDS])
            assert share == list(range(share[0], share[0] + per)), "XCD share not contiguous"
    tail = logical[full:]
    for x in range(XCDS):
        share = sorted(tail[x::XCDS])
        if share:
            assert share == list(range(share[0], share[0] + len(share))), "tail share not contiguous"


@pytest.mark.parametrize("cus", [256, 64, 8, 12])
@pytest.mark.parametrize("total", [1, 7, 8, 136, 253, 256, 257, 4352, 8192, 8704, 22016, 30000])
def test_tile_order(total, cus):
    _check(total, cus)


@pytest.mark.parametrize("plant", ["swap", "modulus", "tail"])
def test_tile_order_planted_mistakes_are_caught(plant):
    with pytest.raises(AssertionError):
        for total in (256, 8704, 22016 + 37):
            _check(total, 256, plant)


def _decode_blocked(t, n, br=4, bc=8):
    """decode_tile<UPPER, BLOCKED> of the kernel."""
    rem = t
    for r0 in range(0, n, br):
        r1 = min(r0 + br, n)
        for c0 in range((r0 // bc) * bc, n, bc):
            c1 = min(c0 + bc, n)
            cnt = sum(max(0, c1 - max(c0, i)) for i in range(r0, r1))
            if rem < cnt:
                for i in range(r0, r1):
                    k = max(0, c1 - max(c0, i))
                    if rem < k:
                        return i, max(c0, i) + rem
                    rem -= k
            rem -= cnt
    return None


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 8, 9, 16, 17, 22, 33, 43])
def test_blocked_upper_order_enumerates_upper_tiles(n):
    got = [_decode_blocked(t, n) for t in range(n * (n + 1) // 2)]
    assert None not in got and len(set(got)) == len(got)
    assert all(0 <= i <= j < n for i, j in got)


def test_blocked_upper_order_reads_fewer_panels():
    # a 22 x 22 grid (4096 / 192, the K-FAC Gram): runs of 32 consecutive tiles
    # (what one XCD runs at once) touch 14-18 distinct operand panels against
    # 16-22 for whole upper-triangle rows
    n = 22

    def panels(seq):
        return [len({i for i, _ in seq[s:s + 32]} | {j for _, j in seq[s:s + 32]}) for s in range(0, len(seq), 32)]

    blocked = panels([_decode_blocked(t, n) for t in range(n * (n + 1) // 2)])
    plain = panels([(i, j) for i in range(n) for j in range(i, n)])
    assert max(blocked) < max(plain) and sum(blocked) < sum(plain)


def _upper_order_table():
    """kUpperOrderOff / kUpperOrder of pytorch-opt_amd/csrc/upper_order.h."""
    import os
    import re

    path = os.path.join(os.path.dirname(__file__), "..", "pytorch-opt_amd", "csrc", "upper_order.h")
    text = open(path).read()
    tmax = int(re.search(r"kUpperOrderMaxT = (\d+);", text).group(1))
    off = [int(v) for v in re.search(r"kUpperOrderOff\[\d+\] = \{([^}]*)\}", text).group(1).split(",")]
    flat = [int(v) for v in re.search(r"kUpperOrder\[\d+\] = \{([^}]*)\}", text).group(1).split(",")]
    return tmax, off, flat


def _xcd_chunks(seq):
    """The logical ids XCD x runs in a launch of len(seq) < C tiles: one
    contiguous range per XCD, of the sizes _range gives."""
    by_xcd = {}
    for w in range(len(seq)):
        by_xcd.setdefault(w % XCDS, []).append(seq[_range(w, len(seq))])
    return list(by_xcd.values())


def _chunk_panels(chunks):
    return [len({i for i, _ in c} | {j for _, j in c}) for c in chunks]


def test_one_round_upper_order_table():
    """For every tile-grid side T the table lists each upper tile (i <= j < T)
    once, in T(T+1)/2 entries, at the offset the kernel reads; every XCD's
    share of a one-round launch reads no more operand panels than under the
    blocked order, and at T = 22 (the 4096² products on 192² tiles) at most
    11 against the blocked order's 18."""
    tmax, off, flat = _upper_order_table()
    assert tmax == 22 and len(off) == tmax
    for T in range(1, tmax + 1):
        n = T * (T + 1) // 2
        assert off[T - 1] == sum(t * (t + 1) // 2 for t in range(1, T))
        seq = [(e >> 5, e & 31) for e in flat[off[T - 1]:off[T - 1] + n]]
        assert sorted(seq) == [(i, j) for i in range(T) for j in range(i, T)], T
        table = _chunk_panels(_xcd_chunks(seq))
        blocked = _chunk_panels(_xcd_chunks([_decode_blocked(t, T) for t in range(n)]))
        assert max(table) <= max(blocked), (T, table, blocked)
        if T == 22:
            assert max(table) <= 11 and max(blocked) == 18
    assert len(flat) == off[-1] + tmax * (tmax + 1) // 2
