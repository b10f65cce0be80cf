"""The forward scan's wave hand-off protocol (csrc/gdn_fwd.hip, fwd_scan_kernel), checked on an
event model of the workgroup on the CPU.

The kernel replaces a per-step s_barrier with counts in LDS: each of two loader waves copies
its part of chunk x into stage x % 4 once the consumer wave has finished chunk x - 4 (loader 1
first stores that chunk's outputs from the stage), and publishes chunk x - 2 once its copies
have landed.  A loader cannot wait for one copy: loads and stores retire in issue order and it
can only wait until at most N of its operations are in flight, so N must count exactly the
operations it issued after chunk x - 2 (its part of chunk x - 1 and, for loader 1, the
copy-out before it).  The consumer waits for both loaders' counts and publishes the chunks it
has finished.

The model runs these rules with random retirement delays and random stalls of each wave, and
asserts what the kernel relies on: the consumer reads only landed, not-yet-overwritten stages,
every copy-out reads the outputs of the chunk it stores, and nothing deadlocks.  The same rules
with a looser wait count, or without the wait for the consumer, must fail.
"""

import random

import pytest

STAGES = 4
PART_COPIES = (17, 18)  # FWD_PART_COPIES: loader 0 (-W rows + G_last), loader 1 (KgT + U^T)
OUT_STORES = 6  # FWD_OUT_STORES: stores of one copy-out


class ProtocolError(AssertionError):
    pass


def _check(cond, msg):
    if not cond:
        raise ProtocolError(msg)


def simulate(n, seed, wait_count=None, wait_for_consumer=True):
    """Run the hand-off for a document of n chunks; raise ProtocolError on a violation."""
    rnd = random.Random(seed)
    slots = [{"part": [None, None], "scratch": None} for _ in range(STAGES)]
    flags = [0, 0, 0]  # loader 0, loader 1, consumer
    inflight = [[], []]  # per loader: [finish time, on_retire] in issue order
    now = [0.0]

    def issue(j, on_retire=None):
        last = inflight[j][-1][0] if inflight[j] else now[0]
        inflight[j].append([max(last, now[0]) + rnd.uniform(1, 40), on_retire])

    def retire():
        for q in inflight:
            while q and q[0][0] <= now[0]:
                _, fn = q.pop(0)
                if fn:
                    fn()

    def count(j, x):  # the kernel's wait count for chunk x - 2 at iteration x
        parts = int(x - 1 < n)
        stores = int(0 <= x - 5 < n) if j == 1 else 0
        return (wait_count or (lambda j, p, s: p * PART_COPIES[j] + s * OUT_STORES))(j, parts, stores)

    def loader(j):
        for x in range(n + STAGES):
            y = x - 2
            if 0 <= y < n:
                limit = count(j, x)
                yield lambda: len(inflight[j]) <= limit
                _check(slots[y % STAGES]["part"][j] == y, f"loader {j} published chunk {y} before it landed")
                flags[j] = y + 1
            if x >= STAGES:
                if wait_for_consumer:
                    yield lambda: flags[2] >= x - STAGES + 1
                if j == 1 and x - STAGES < n:
                    got = slots[x % STAGES]["scratch"]
                    _check(got == x - STAGES, f"copy-out of chunk {x - STAGES} read outputs of {got}")
                    for _ in range(OUT_STORES):
                        issue(j)
            if x < n:
                slot = slots[x % STAGES]
                slot["part"][j] = ("pending", x)
                for i in range(PART_COPIES[j]):
                    done = (lambda slot=slot, x=x: slot["part"].__setitem__(j, x)) if i == PART_COPIES[j] - 1 else None
                    issue(j, done)

    def consumer():
        for tau in range(n):
            yield lambda: min(flags[0], flags[1]) >= tau + 1
            slot = slots[tau % STAGES]
            _check(slot["part"] == [tau, tau], f"consumer read chunk {tau} before it landed: {slot['part']}")
            yield None  # computing
            _check(slot["part"] == [tau, tau], f"chunk {tau} overwritten while the consumer read it")
            slot["scratch"] = tau
            flags[2] = tau + 1

    waves = [consumer(), loader(0), loader(1)]
    stall = [rnd.choice([0.0, 0.5, 0.9]) for _ in waves]
    blocked = [None] * 3
    alive = [True] * 3
    for _ in range(2_000_000):
        if not any(alive):
            break
        moved = False
        for i in rnd.sample(range(3), 3):
            if not alive[i] or rnd.random() < stall[i]:
                continue
            if blocked[i] is not None and not blocked[i]():
                continue
            try:
                blocked[i] = next(waves[i])
                moved = True
            except StopIteration:
                alive[i], blocked[i], moved = False, None, True
        now[0] += rnd.uniform(0.5, 25)
        retire()
        idle = not moved and not any(inflight) and all(
            not alive[i] or (blocked[i] is not None and not blocked[i]()) for i in range(3))
        _check(not (idle and any(alive) and max(stall) == 0), f"deadlock at counts {flags}")
    else:
        raise ProtocolError("no progress")
    now[0] = float("inf")
    retire()
    _check(flags == [n, n, n], f"final counts {flags}")


@pytest.mark.parametrize("n", [0, 1, 2, 3, 4, 5, 6, 9, 17])
def test_handoff_protocol_holds(n):
    for seed in range(40):
        simulate(n, seed)


def test_looser_wait_count_is_caught():
    with pytest.raises(ProtocolError, match="before it landed"):
        for seed in range(40):
            simulate(9, seed, wait_count=lambda j, p, s: (p + 1) * PART_COPIES[j] + s * OUT_STORES)


def test_count_with_a_store_group_too_many_is_caught():
    with pytest.raises(ProtocolError, match="before it landed"):
        for seed in range(200):
            simulate(9, seed, wait_count=lambda j, p, s: p * PART_COPIES[j] + (s + 1) * OUT_STORES)


def test_refill_without_waiting_for_the_consumer_is_caught():
    with pytest.raises(ProtocolError):
        for seed in range(40):
            simulate(9, seed, wait_for_consumer=False)
