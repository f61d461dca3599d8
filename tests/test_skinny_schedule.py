"""CPU model of the skinny entry's loader-split schedule (SkinnyTile::run_deep in
csrc/gemm_skinny.h): loader and computing wavefronts must pass the same barriers, a ring slot may
be refilled only once every fragment read from it has been consumed, a read may only touch a
stage that a barrier has published after the loads landed, and the loaders' vmcnt waits must
imply that the stage a barrier publishes has landed.  A broken rule hangs a GPU (unequal
barriers) or corrupts results silently, so it is checked here for every stage count up to 64.
The constants restate the kernel's: 8 K steps per stage (4 pairs), a ring of 4 slots,
fragments read 3 pairs ahead, 3 stages issued before barrier 0, barrier t >= 1 (reached at
pair 1 of stage t - 1) issuing stage t + 2 into the slot of stage t - 2."""

import pytest

PPS = 4        # K-step pairs per stage (UD = 8)
DSTAGES = 4    # ring slots
DA = 3         # read-ahead in pairs


def loader_events(ns, refill=DSTAGES - 2, tail_wait=DSTAGES - 3):
    """One loader wavefront: ('issue', stage), ('wait', stages left in flight), ('barrier', t)."""
    ev = []
    for s in range(DSTAGES - 1):
        if s < ns:
            ev.append(("issue", s))
    ev.append(("wait", min(DSTAGES - 2, ns - 1)))
    ev.append(("barrier", 0))
    for t in range(1, ns):
        ev.append(("wait", tail_wait if t + DSTAGES - 3 < ns else 0))
        ev.append(("barrier", t))
        if t + refill < ns:
            ev.append(("issue", t + refill))
    return ev


def compute_events(ns, barrier_pair=PPS - DA):
    """One computing wavefront: ('barrier', t), ('read', pair), ('use', pair)."""
    ev = [("barrier", 0)]
    for i in range(DA):
        ev.append(("read", i))
    t = 1
    for s in range(ns):
        for d in range(PPS):
            if d == barrier_pair and s + 1 < ns:
                ev.append(("barrier", t))
                t += 1
            p = s * PPS + d
            ev.append(("use", p))
            ev.append(("read", p + DA))
    return ev


def check_schedule(ns, lev, cev):
    lb = [e[1] for e in lev if e[0] == "barrier"]
    cb = [e[1] for e in cev if e[0] == "barrier"]
    assert lb == cb == list(range(ns)), "both sides pass barriers 0 .. NS-1 once, in order"

    # Loads land in issue order (vmcnt): after a wait leaving x in flight, all but the last x
    # issued have landed; the barrier that follows must publish a landed stage.
    issued, landed, slot_of_issue = [], set(), {}
    for kind, x in lev:
        if kind == "issue":
            assert x not in slot_of_issue, f"stage {x} loaded twice"
            slot_of_issue[x] = x % DSTAGES
            issued.append(x)
        elif kind == "wait":
            landed = set(issued[:len(issued) - x])
        elif kind == "barrier":
            assert x in landed, f"barrier {x} publishes a stage still in flight"
    assert sorted(issued) == list(range(ns)), "every stage loaded exactly once"

    # The computing side: pairs used before each barrier, reads issued after it.
    used, used_before, reads_after, current = set(), {}, {t: [] for t in range(ns)}, None
    seen_reads = set()
    for kind, x in cev:
        if kind == "barrier":
            current = x
            used_before[x] = set(used)
        elif kind == "use":
            assert x in seen_reads, f"pair {x} used before it was read"
            used.add(x)
        else:
            seen_reads.add(x)
            reads_after[current].append(x)
    assert sorted(used) == list(range(ns * PPS))

    # Reads between barrier t and t + 1 touch published stages only (pairs past the last stage
    # read ring bytes that are never used).
    for t, reads in reads_after.items():
        for p in reads:
            if p < ns * PPS:
                assert p // PPS <= t, f"pair {p} read before stage {p // PPS} was published"

    # A stage issued at barrier t overwrites the slot of the stage DSTAGES before it: all of that
    # stage's pairs must be used by then, and no read after barrier t may target it.
    issue_barrier, last_barrier = {}, None
    for kind, x in lev:
        if kind == "barrier":
            last_barrier = x
        elif kind == "issue" and last_barrier is not None:
            issue_barrier[x] = last_barrier
    for stage, t in issue_barrier.items():
        victim = stage - DSTAGES
        if victim < 0:
            continue
        assert set(range(victim * PPS, victim * PPS + PPS)) <= used_before[t], (
            f"barrier {t} refills the slot of stage {victim} before its pairs were used")
        for t2 in range(t, ns):
            for p in reads_after[t2]:
                assert p // PPS != victim, f"pair {p} read from the refilled slot of stage {victim}"


@pytest.mark.parametrize("ns", range(1, 65))
def test_loader_split_schedule_is_safe(ns):
    check_schedule(ns, loader_events(ns), compute_events(ns))


@pytest.mark.parametrize(("ns", "variant"), (
    (8, "refill one stage early"),      # the slot of a stage still being read
    (8, "barrier one pair late"),       # a read of a stage not yet published
    (8, "wait for one stage too few"),  # a barrier publishing a stage still in flight
))
def test_schedule_checker_rejects_broken_variants(ns, variant):
    """The checker fails each variant that breaks one rule of the kernel's schedule."""
    lev, cev = loader_events(ns), compute_events(ns)
    if variant == "refill one stage early":
        lev = loader_events(ns, refill=DSTAGES - 1)
    elif variant == "barrier one pair late":
        cev = compute_events(ns, barrier_pair=PPS - DA + 1)
    else:
        lev = loader_events(ns, tail_wait=DSTAGES - 2)
    with pytest.raises(AssertionError):
        check_schedule(ns, lev, cev)
