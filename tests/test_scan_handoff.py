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


def simulate(n, seed, wait_count=None, wait_for_consumer=True, spin_limit=None, hold=None, poison_copy_out=True):
    """Run the hand-off for a document of n chunks; raise ProtocolError on a violation.

    ``spin_limit``: a loader's wait for the consumer gives up after that many polls (the kernel's
    bounded wait); it then publishes the poison flag before refilling.  ``hold = (step, time)``
    stalls the consumer at that step, so that waits do give up.  With a give-up the model checks
    that nothing is silently wrong: a consumer step that read an overwritten stage is followed by
    NaN states, and a copy-out of anything but its own chunk's outputs stores NaN
    (``poison_copy_out=False`` drops the latter, which must be caught)."""
    rnd = random.Random(seed)
    slots = [{"part": [None, None], "scratch": None} for _ in range(STAGES)]
    flags = [0, 0, 0]  # loader 0, loader 1, consumer
    poison = [False]  # flags[3]
    gave_up = [False]
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
                if wait_for_consumer and not (spin_limit and poison[0] and gave_up[0]):
                    polls = [0]

                    def ready(target=x - STAGES + 1, polls=polls):
                        polls[0] += 1
                        return flags[2] >= target or (spin_limit is not None and polls[0] > spin_limit)

                    yield ready
                    if flags[2] < x - STAGES + 1:  # gave up: poison first, then refill without waiting
                        poison[0] = gave_up[0] = True
                if j == 1 and x - STAGES < n:
                    got = slots[x % STAGES]["scratch"]
                    nan = poison_copy_out and poison[0]
                    if got != x - STAGES and not nan:
                        if spin_limit is None:
                            _check(False, f"copy-out of chunk {x - STAGES} read outputs of {got}")
                        _check(False, f"silently wrong copy-out of chunk {x - STAGES} ({got})")
                    for _ in range(OUT_STORES):
                        issue(j)
            if x < n:
                slot = slots[x % STAGES]
                slot["part"][j] = ("pending", x)
                for i in range(PART_COPIES[j]):
                    done = (lambda slot=slot, x=x: slot["part"].__setitem__(j, x)) if i == PART_COPIES[j] - 1 else None
                    issue(j, done)

    def consumer():
        ok, bad_state, seen_poison = True, False, False
        for tau in range(n):
            yield lambda: min(flags[0], flags[1]) >= tau + 1
            if seen_poison:
                ok = False  # the state turns to NaN
            _check(ok or spin_limit is not None, "a wait gave up without a spin limit")
            _check(not (bad_state and ok), f"state silently wrong at chunk {tau}")
            slot = slots[tau % STAGES]
            intact = slot["part"] == [tau, tau]  # the operand reads, issued at the step's start
            if spin_limit is None:
                _check(intact, f"consumer read chunk {tau} before it landed: {slot['part']}")
            seen_poison = poison[0]  # read after the operands, applied at the next step
            if hold is not None and tau == hold[0]:
                until = now[0] + hold[1]
                yield lambda: now[0] >= until
            yield None  # computing
            if spin_limit is None:
                _check(slot["part"] == [tau, tau], f"chunk {tau} overwritten while the consumer read it")
            bad_state = bad_state or not intact
            slot["scratch"] = tau if (ok and intact) else ("nan" if not ok else ("bad", tau))
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
    return gave_up[0]


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


def test_loader_timeout_poisons_instead_of_corrupting():
    """A loader whose wait for the consumer gives up publishes the poison flag before it refills a
    stage: the consumer's later states and every later copy-out are NaN, never silently wrong."""
    gave_up = 0
    for seed in range(60):
        gave_up += simulate(12, seed, spin_limit=3, hold=(2, 3000.0))
    assert gave_up > 0  # the hold made waits give up


def test_copy_out_without_poison_check_is_caught():
    with pytest.raises(ProtocolError, match="silently wrong"):
        for seed in range(60):
            simulate(12, seed, spin_limit=3, hold=(2, 3000.0), poison_copy_out=False)
