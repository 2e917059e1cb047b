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
