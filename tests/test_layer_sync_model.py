"""Host model of the single-launch layer's in-launch wait (layer1.hip): why it cannot deadlock,
and what its bound does when the premise fails.

The model: a grid of workgroups, workgroup b dealt to XCD b mod 8; each XCD dispatches its
share in index order into a limited number of slots; a producer (gate/up workgroup) runs for a
while and then publishes; a consumer (down workgroup) holds its slot from dispatch until every
producer has published (it then finishes) or until its wait bound passes (it gives up). The
layer's grid puts every producer before every consumer. The model shows, over many random
grids, slot counts and run times:
  - producers first: every workgroup finishes and no consumer gives up;
  - consumers first (the order the kernel does not use) with few slots: consumers hold every
    slot while producers wait for one -- only the bound ends it (so the ordering carries the
    argument, and the bound turns a violation into an error, not a hang);
  - producers that never publish (the host-forced give-up test): every consumer gives up after
    the bound and every workgroup still finishes.
It also checks the per-call value the flags are compared with: unique and increasing per
process, so flags left by earlier calls never match a later call's value.
"""
import heapq
import random

XCDS = 8


def simulate(P, C, slots, dur_p, dur_c, bound, producers_first=True, publish=True):
    """Returns (finished workgroups, consumers that gave up, end time)."""
    n = P + C
    is_prod = [(b < P) if producers_first else (b >= C) for b in range(n)]
    queues = [[b for b in range(n) if b % XCDS == x] for x in range(XCDS)]
    heads = [0] * XCDS
    free = [slots] * XCDS
    events = []  # (time, seq, kind, b)
    seq = 0
    published = 0
    waiting = {}  # consumer -> time its wait ends at the latest
    finished = gave_up = 0
    end = 0.0

    def dispatch(t):
        nonlocal seq
        for x in range(XCDS):
            while free[x] > 0 and heads[x] < len(queues[x]):
                b = queues[x][heads[x]]
                heads[x] += 1
                free[x] -= 1
                if is_prod[b]:
                    heapq.heappush(events, (t + dur_p(b), seq, "p_done", b))
                elif published == P:
                    heapq.heappush(events, (t + dur_c(b), seq, "c_done", b))
                else:
                    waiting[b] = t + dur_c(b) + bound
                    heapq.heappush(events, (waiting[b], seq, "c_timeout", b))
                seq += 1

    dispatch(0.0)
    while events:
        now, _, kind, b = heapq.heappop(events)
        if kind == "c_timeout" and b not in waiting:
            continue  # finished before its bound
        end = now
        free[b % XCDS] += 1
        finished += 1
        if kind == "p_done" and publish:
            published += 1
            if published == P:  # every waiting consumer proceeds now
                for c in list(waiting):
                    del waiting[c]
                    heapq.heappush(events, (now, seq, "c_done", c))  # holds its slot until then
                    seq += 1
        elif kind == "c_timeout":
            del waiting[b]
            gave_up += 1
        dispatch(now)
    return finished, gave_up, end


def _random_grid(rng):
    P = rng.randint(1, 200)
    C = rng.randint(1, 600)
    slots = rng.randint(1, 96)
    dp = {b: rng.uniform(5.0, 20.0) for b in range(P + C)}
    dc = {b: rng.uniform(0.5, 3.0) for b in range(P + C)}
    return P, C, slots, dp.__getitem__, dc.__getitem__


def test_producers_first_never_waits_out():
    rng = random.Random(0)
    for _ in range(400):
        P, C, slots, dp, dc = _random_grid(rng)
        fin, gave_up, end = simulate(P, C, slots, dp, dc, bound=1e9)
        assert fin == P + C and gave_up == 0, (P, C, slots)
        assert end < 1e8


def test_consumers_first_needs_the_bound():
    rng = random.Random(1)
    blocked = 0
    for _ in range(200):
        P, C, slots, dp, dc = _random_grid(rng)
        fin, gave_up, end = simulate(P, C, slots, dp, dc, bound=1000.0, producers_first=False)
        assert fin == P + C  # the bound ends every wait
        blocked += gave_up > 0
    assert blocked > 0  # some grids would never finish without it


def test_unpublished_producers_every_consumer_gives_up():
    rng = random.Random(2)
    for _ in range(100):
        P, C, slots, dp, dc = _random_grid(rng)
        fin, gave_up, end = simulate(P, C, slots, dp, dc, bound=50.0, publish=False)
        assert fin == P + C and gave_up == C


def test_call_values_never_repeat():
    """The host's per-call value (capi.hip next_epoch): random high 32 bits per process, a call
    counter below. Flags left by any earlier call, zero-filled or 0xFF-filled workspaces never
    equal a later call's value."""
    rng = random.Random(3)
    high = (rng.getrandbits(32) | 1) << 32
    values = [high + i + 1 for i in range(10000)]
    assert len(set(values)) == len(values) and all(v != 0 for v in values)
    leftovers = {0, (1 << 64) - 1} | set(values[:5000])
    assert not any(v in leftovers for v in values[5000:])
