"""CPU models of the MFMA core's two-group main loops: the ping-pong schedule
(the 256² bf16 tiles) and the K-group schedule (the 192² bf16 tile).

The kernel splits its eight waves into two groups of four (one wave of each
per SIMD). Each wave runs the same phases over K tiles t = 0, 1, ...:

  R(t): LDS reads of tile t (stage t % 4) into its one register set, and the
        global->LDS DMA of tile min(t + 3, KT - 1) into stage (t + 3) % 4;
  M(t): the MFMAs of tile t;

with lgkmcnt(0) + vmcnt(2·IPW) + s_barrier after every phase, the DMA of
tiles 0-2 plus vmcnt(2·IPW) + s_barrier before the loop, group 1 starting
one phase late (an extra barrier before its loop) and group 0 ending with
one (after its loop). This model replays that sequence for both groups and
checks what the kernel relies on:

* both groups execute the same number of barriers (a mismatch would hang);
* every LDS read of tile t sees both groups' DMA parts of tile t issued and
  waited for (landed) before a barrier that precedes the read;
* no DMA refills a stage while a read of the tile it still holds is pending
  (in the same or a later phase).

A planted mistake (group 1 without its extra barrier, a ring of 3 stages,
leaving 3 tiles' loads in flight at each wait) fails one of them.
"""

import pytest


def _phases(group, KT, stages=4, wait_keep=2, g1_extra=True):
    """The ops of one wave of `group` as a list of phases (one per barrier)."""
    prologue = [("dma", t, t % stages) for t in range(min(stages - 1, 3))] + [("wait", wait_keep)]
    ph = [prologue]
    if group == 1 and g1_extra:
        ph.append([])
    for t in range(KT):
        ph.append([("read", t, t % stages), ("dma", min(t + stages - 1, KT - 1), (t + stages - 1) % stages),
                   ("wait", wait_keep)])
        ph.append([("mma", t), ("wait", wait_keep)])
    if group == 0:
        ph.append([])
    ph.append([("wait", 0)])
    return ph


def _check(KT, **kw):
    return _check_seqs({g: _phases(g, KT, **kw) for g in (0, 1)}, KT)


def _check_seqs(seqs, KT):
    if len(seqs[0]) != len(seqs[1]):
        raise AssertionError(f"barrier counts differ: {len(seqs[0])} vs {len(seqs[1])}")
    issued = {0: [], 1: []}   # per group: [tile, stage, phase, landed-by-phase or None]
    reads = []
    for i in range(len(seqs[0])):
        for g in (0, 1):
            for op in seqs[g][i]:
                if op[0] == "dma":
                    issued[g].append([op[1], op[2], i, None])
                elif op[0] == "wait":
                    done = issued[g][:max(len(issued[g]) - op[1], 0)]
                    for rec in done:
                        if rec[3] is None:
                            rec[3] = i
                elif op[0] == "read":
                    reads.append((g, op[1], op[2], i))
    for g, t, s, i in reads:
        for h in (0, 1):
            before = [rec for rec in issued[h] if rec[1] == s and rec[2] < i]
            if not before or before[-1][0] != t:
                raise AssertionError(f"group {g} reads tile {t} from stage {s} in phase {i}, which holds "
                                     f"{before[-1][0] if before else None} of group {h}")
            if before[-1][3] is None or before[-1][3] >= i:
                raise AssertionError(f"group {h}'s part of tile {t} not landed before phase {i}")
    for h in (0, 1):
        for tile, s, i, _ in issued[h]:
            for g, t, rs, ri in reads:
                if rs == s and t < tile and ri >= i:
                    raise AssertionError(f"DMA of tile {tile} into stage {s} in phase {i} while tile {t} "
                                         f"is read in phase {ri}")
    return len(seqs[0])


@pytest.mark.parametrize("KT", [4, 8, 12, 64, 128, 344, 512])
def test_pingpong_schedule_is_hazard_free(KT):
    # the kernel requires K to be a multiple of four tiles; every phase ends
    # in one barrier (the prologue's included)
    assert _check(KT) == 2 * KT + 3


@pytest.mark.parametrize("planted", [dict(g1_extra=False), dict(stages=3), dict(wait_keep=3)])
def test_pingpong_planted_mistakes_are_caught(planted):
    with pytest.raises(AssertionError):
        _check(16, **planted)


def _kgroup_phases(group, KT, stages=4, wait_keep=2, late_start=True):
    """K groups: group g reads and multiplies the K tiles t with t % 2 == g;
    interval j: the reader of tile j reads it, the other group multiplies
    tile j - 1, every wave issues its DMA share of tile j + 3 into stage
    (j + 3) % 4; group 1 starts with an interval of DMA only, group 0 ends
    with one."""
    ph = [[("dma", t, t % stages) for t in range(min(stages - 1, 3))] + [("wait", wait_keep)]]
    j = 0
    if group == 1 and late_start:
        ph.append([("dma", min(3, KT - 1), 3 % stages), ("wait", wait_keep)])
        j = 1
    for t in range(group, KT, 2):  # (without the late start, group 1 runs one interval early)
        ph.append([("read", t, t % stages), ("dma", min(j + 3, KT - 1), (j + 3) % stages), ("wait", wait_keep)])
        j += 1
        ph.append([("mma", t), ("dma", min(j + 3, KT - 1), (j + 3) % stages), ("wait", wait_keep)])
        j += 1
    if group == 0:
        ph.append([("dma", min(j + 3, KT - 1), (j + 3) % stages), ("wait", wait_keep)])
    ph.append([("wait", 0)])
    return ph


def _check_kgroup(KT, **kw):
    seqs = {g: _kgroup_phases(g, KT, **kw) for g in (0, 1)}
    return _check_seqs(seqs, KT)


@pytest.mark.parametrize("KT", [4, 8, 12, 64, 512])
def test_kgroup_schedule_is_hazard_free(KT):
    assert _check_kgroup(KT) == KT + 3


@pytest.mark.parametrize("planted", [dict(late_start=False), dict(stages=3), dict(wait_keep=3)])
def test_kgroup_planted_mistakes_are_caught(planted):
    with pytest.raises(AssertionError):
        _check_kgroup(16, **planted)
