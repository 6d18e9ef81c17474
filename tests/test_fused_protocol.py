"""CPU model of the one-launch fused decode layer's cross-workgroup protocol (csrc/exl3_moe_fused.h): workgroup g runs
gate|up job g (item g / GU) and then, on the workgroups of item i + 1, the down jobs of item i, which wait for every
gate|up job of item i. The kernel's progress argument is that workgroups are dispatched in id order within each XCD
(ids round-robin over the XCDs) and that a workgroup finishes its own gate|up job before it can wait, so the lowest
waiting workgroup always has its inputs coming, whatever the number of resident slots. The model dispatches the
kernel's job layout onto XCDs with few slots and random job lengths and checks that every launch drains; dispatching
the same layout in reverse id order deadlocks, so the order is what the argument rests on."""
import random

XCDS = 8


def layout(nitems, GU, DN, max_items=None):
    """Per workgroup: (gate|up job's item or -1, item whose down jobs it runs or -1), exactly as the kernel derives them
    from blockIdx.x: grid = J_gu + GU with J_gu = max_items * GU; gi = g // GU; gate|up when g < J_gu and gi < nitems;
    down jobs of item gi - 1 when that item exists and g % GU < DN."""
    max_items = max_items or nitems
    J_gu = max_items * GU
    out = []
    for g in range(J_gu + GU):
        gi, gr0 = divmod(g, GU)
        gu_item = gi if g < J_gu and gi < nitems else -1
        di = gi - 1
        dn_item = di if 0 <= di < nitems and gr0 < DN else -1
        out.append((gu_item, dn_item))
    return out


def simulate(jobs, GU, slots, order, rng, max_steps=200000):
    """Discrete-time run: each XCD holds `slots` workgroups and dispatches its queue (ids on that XCD, in `order`)
    as slots free. A workgroup's gate|up phase lasts a random number of ticks and never waits; its down phase starts
    once every gate|up job of its item has finished, then lasts a random number of ticks. Returns True when every
    workgroup has exited, False on a deadlock (no workgroup can move)."""
    n = len(jobs)
    queues = {x: [g for g in order if g % XCDS == x] for x in range(XCDS)}
    gu_done = [jobs[g][0] < 0 for g in range(n)]
    remaining = {}
    phase = {}
    resident = {x: set() for x in range(XCDS)}
    exited = 0
    item_jobs = {}
    for g, (gi, _) in enumerate(jobs):
        if gi >= 0:
            item_jobs.setdefault(gi, []).append(g)

    def start(g):
        phase[g] = "gu" if jobs[g][0] >= 0 else "wait"
        remaining[g] = rng.randint(1, 20)

    for _ in range(max_steps):
        for x in range(XCDS):
            while len(resident[x]) < slots and queues[x]:
                g = queues[x].pop(0)
                resident[x].add(g)
                start(g)
        moved = False
        for x in range(XCDS):
            for g in list(resident[x]):
                if phase[g] == "gu":
                    remaining[g] -= 1
                    moved = True
                    if remaining[g] == 0:
                        gu_done[g] = True
                        phase[g] = "wait"
                        remaining[g] = rng.randint(1, 20)
                elif phase[g] == "wait":
                    di = jobs[g][1]
                    if di < 0:
                        phase[g] = "exit"
                    elif all(gu_done[d] for d in item_jobs.get(di, [])):
                        phase[g] = "down"
                    moved = moved or phase[g] != "wait"
                elif phase[g] == "down":
                    remaining[g] -= 1
                    moved = True
                    if remaining[g] == 0:
                        phase[g] = "exit"
                if phase[g] == "exit":
                    resident[x].discard(g)
                    exited += 1
                    moved = True
        if exited == n:
            return True
        if not moved:
            return False
    raise AssertionError("simulation did not settle")


def test_in_order_dispatch_always_drains():
    rng = random.Random(7)
    for trial in range(300):
        nitems = rng.randint(1, 12)
        GU = rng.randint(1, 24)
        DN = rng.randint(1, 3 * GU)
        max_items = nitems + rng.randint(0, 3)                 # the grid is sized for up to max_items items
        slots = rng.randint(1, 3)                              # far fewer slots than workgroups
        jobs = layout(nitems, GU, DN, max_items)
        assert simulate(jobs, GU, slots, list(range(len(jobs))), rng), (trial, nitems, GU, DN, slots)


def test_reverse_order_dispatch_can_deadlock():
    """Without in-order dispatch the waits can hold every slot: a deadlock shows up within a few layouts."""
    rng = random.Random(11)
    deadlocks = 0
    for trial in range(100):
        nitems = rng.randint(2, 12)
        GU = rng.randint(1, 24)
        jobs = layout(nitems, GU, rng.randint(1, 3 * GU))
        if not simulate(jobs, GU, 1, list(reversed(range(len(jobs)))), rng):
            deadlocks += 1
    assert deadlocks > 0


def test_layout_matches_the_kernel_indexing():
    """Every gate|up job of every item runs exactly once, every item's down jobs 0 .. DN - 1 run on its successor's
    workgroups (job r on workgroup r % GU of that item), and each down workgroup has a higher id than every gate|up
    job it waits for."""
    for nitems, GU, DN in ((5, 6, 16), (1, 1, 1), (10, 24, 16), (3, 4, 9)):
        jobs = layout(nitems, GU, DN, nitems + 2)
        gu = [g for g, (gi, _) in enumerate(jobs) if gi >= 0]
        assert len(gu) == nitems * GU and len(set(jobs[g][0] for g in gu)) == nitems
        for item in range(nitems):
            runners = [g for g, (_, di) in enumerate(jobs) if di == item]
            covered = sorted(r for g in runners for r in range(g % GU, DN, GU))
            assert covered == list(range(DN))
            deps = [g for g, (gi, _) in enumerate(jobs) if gi == item]
            assert min(runners) > max(deps)
