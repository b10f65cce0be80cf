"""The reverse scan's hand-off to a bwd_dkw running beside it (csrc/gdn_bwd.hip: bwd_scan_kernel's
loader 1, bwd_dkw_kernel's wait), checked on a model of loader 1's vector-memory queue on the CPU.

Loader 1 of each value-slice workgroup stores every step's dS / dVn (six stores, the copy-out of
step tau-1 at iteration tau) and refills its stage part (18 copies, the part of step tau+3).  A
wave's loads and stores retire in issue order, and it can only wait until at most N of its
operations are in flight, so N must count exactly the operations it issued after the part it waits
for.  Beside a bwd_dkw, loader 1 also announces step tau-3's chunk right after its wait at
iteration tau (one atomic add, in flight with the rest): that wait covers the copy-out of step
tau-3, and the atomic is itself one more operation the next wait must count.  After the loop it
stores the last step, waits for everything and announces the steps the loop did not.

The model replays the kernel's loop and its wait counts against a queue in which exactly the last N
operations are still in flight, and asserts: every wait covers the part it waits for; every
announcement comes after all six stores of its step have retired; every step is announced exactly
once, in the order the scan finishes them (so bwd_dkw, which waits for the count of its chunk to
reach 8, one per value slice, reads a chunk only after every slice's stores of it are visible).  A
count that assumes an announcement that was not issued, or forgets the copy-out, must fail.
"""

import pytest

PART = 18  # BWD_PART_COPIES[1]
STORES = 6  # BWD_OUT_STORES
DEPTH = 3  # BS_DEPTH


class ProtocolError(AssertionError):
    pass


def kernel_wait_count(tau, n, announce):
    """The kernel's vmcnt for loader 1 at iteration tau (bwd_scan_kernel, j == 1)."""
    xn = tau + 1
    later = xn + 1 < n
    stored = tau >= 2
    announced = announce and tau >= 4
    if later and announced:
        return PART + STORES + 1
    if later and stored:
        return PART + STORES
    if later:
        return PART
    if announced:
        return STORES + 1
    if stored:
        return STORES
    return 0


def replay(n, announce=True, wait_count=kernel_wait_count):
    """Loader 1's operations for a document of n chunks; returns the steps announced, in order."""
    ops = []  # issue order: (kind, step)
    announced = []

    def retired_upto(inflight):
        return len(ops) - min(inflight, len(ops))

    def check_retired(kind, step, upto, what):
        idx = [i for i, op in enumerate(ops) if op == (kind, step)]
        if not idx or max(idx) >= upto:
            raise ProtocolError(f"{what}: {kind} of step {step} may still be in flight")

    for tau in range(-DEPTH, n):
        xn, xo, xi = tau + 1, tau - 1, tau + DEPTH
        if 0 <= xn < n:
            upto = retired_upto(wait_count(tau, n, announce))
            check_retired("part", xn, upto, f"iteration {tau}")
            if announce and tau >= 3:
                check_retired("store", tau - 3, upto, f"announcing step {tau - 3}")
                ops.append(("announce", tau - 3))
                announced.append(tau - 3)
        if xo >= 0:
            ops.extend([("store", xo)] * STORES)
        if xi < n:
            ops.extend([("part", xi)] * PART)
    if n > 0:
        ops.extend([("store", n - 1)] * STORES)
        if announce:
            upto = retired_upto(0)  # wait_vmem_all
            for s in range(max(n - 4, 0), n):
                check_retired("store", s, upto, f"announcing step {s} after the loop")
                ops.append(("announce", s))
                announced.append(s)
    return announced


@pytest.mark.parametrize("n", [0, 1, 2, 3, 4, 5, 6, 7, 8, 13, 144])
@pytest.mark.parametrize("announce", [False, True])
def test_reverse_scan_announcements_follow_their_stores(n, announce):
    got = replay(n, announce)
    if announce:
        assert sorted(got) == list(range(n)) and len(set(got)) == n
        # steps are announced in the order they finish: bwd_dkw takes chunks last to first
        assert got == sorted(got)
    else:
        assert got == []


def test_counting_an_announcement_not_yet_issued_is_caught():
    def loose(tau, n, announce):
        xn = tau + 1
        later, stored = xn + 1 < n, tau >= 2
        announced = announce and tau >= 3  # one iteration early: that atomic was never issued
        return (PART if later else 0) + (STORES if stored else 0) + (1 if announced else 0)

    with pytest.raises(ProtocolError, match="may still be in flight"):
        replay(9, True, loose)


def test_forgetting_the_announcement_is_safe_but_forgetting_the_copy_out_is_caught():
    def strict(tau, n, announce):  # one operation fewer in flight than issued: waits longer, still correct
        return max(kernel_wait_count(tau, n, announce) - (1 if announce and tau >= 4 else 0), 0)

    assert replay(9, True, strict) == list(range(9))

    def loose(tau, n, announce):
        return kernel_wait_count(tau, n, announce) + (STORES if tau < 2 else 0)

    with pytest.raises(ProtocolError, match="may still be in flight"):
        replay(9, True, loose)


def test_chunk_counts_reach_eight_only_after_every_slice():
    """Eight value slices announce their steps; a chunk's count (chunk = c_end - 1 - step) reaches 8,
    bwd_dkw's condition, only once every slice has announced that step, each after its own stores."""
    n = 11
    counts = [0] * n
    per_slice = [replay(n) for _ in range(8)]
    for s in range(8):
        for step in per_slice[s]:
            counts[n - 1 - step] += 1
    assert counts == [8] * n

