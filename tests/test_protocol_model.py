"""A CPU model of the expert kernels' task-claim and dependency-wait protocol,
explored exhaustively on small instances under every interleaving of the
blocks and with only some blocks resident (another kernel holding CUs).

What is modelled (final_amd/csrc/moe_kernels.hip):

* Tasks are numbered in the order the queue counter hands them out.  A task
  may wait only for tasks of smaller number: gate/up tiles for the dispatch
  tasks, down tiles / down row tasks for their unit's or expert's gate/up
  tasks, the ring kernel's combine tasks for their token's down tasks.
* expert_mfma_kernel: a block claims its first task as it starts, then per
  task waits for the task's inputs, computes, claims its next task after the
  MFMAs and finishes the epilogue (which never waits).  Dispatch tasks never
  wait (also when, routing from score bounds, they run the gate chains and
  the exact routing); down tiles wait for every dispatch task.  A down tile above
  128 tokens waits slab by slab for the gate/up tile behind each slab
  (SlabReady) rather than for all of its unit's at once; the model keeps the
  all-at-once wait, which holds the block at least as long on the same set
  of gate/up tasks, so every state the slab waits reach is covered.
* expert_ring_kernel: a block claims its first task as it starts; streaming
  wave 0 claims the next one at an early step of the current task, which may
  come before or after the current task's wait for its inputs (the model
  allows both orders); after the row tasks a block runs the combine tasks
  dealt to it round-robin (block b: tokens b, b+G, ...).
* Residency: of G blocks only R run at once; block b starts when a running
  block exits, in index order.

The model explores every interleaving (memoised depth-first search) and
reports a reachable state in which tasks remain and no block can move.  Both
kernels' protocols are shown free of such states; two variants are shown to
reach one, which is what proves the model can see a deadlock: a first task
given statically by block index (the ring kernel before its first claim came
from the queue: a non-resident block then owns a gate/up task that running
down tasks wait for), and a block that waits for its next task's inputs
before finishing its current one (the shape of a removed ring-kernel variant
that parked down tasks until their expert's values had landed and ended in a
device-side wait timeout: its block could hold the gate/up task that its own
next down task needed).

The ring kernel's routing of a decode batch from score bounds (Ctrl::deferred
2) adds the gate-logit chain jobs and their waits, modelled by
explore_chain:

* J jobs on a counter of their own (chain_head).  As it starts, each of the
  first C blocks claims one (none in lazy mode) and runs it in block form,
  and claims its first row task only after it; every other block claims its
  first row task at once.  A job never waits; it counts itself in
  chain_done when it is stored.
* Prologue (every block plans from the bounds): when a token has more
  possible experts than the plan holds (the fallback), the block claims and
  runs in block form every job still unclaimed, then waits until all J are
  done, holding the row task it may have claimed; otherwise it goes on at
  once.
* After its row tasks, a block's combine of a token (planned path) first
  needs the exact routing: all J jobs done, and while any job is
  unclaimed the waiting wave claims and runs it (wave form,
  ring_route_exact); then the token's expert outputs (its down tasks).  The
  fallback's combine routes from the logits it already has.

Both modes, lazy or not, are shown free of stuck states under partial
residency; the model reaches one when the waits do not run unclaimed jobs
(lazy mode: no block ever would), and when a job waits for another (the
block that holds job 0 waits for job 1, which only a block that is not
resident could claim).

When the MFMA kernel routes from score bounds, its blocks claim their first
tasks from K group counters instead of the queue head (explore_groups):
group g's k-th claim is task k * K + g, for the first F tasks (dispatch and
gate/up tasks, which never wait); a block claims from the head (tasks F, F
+ 1, ...) only after it has found every first-round task claimed, claiming
any left itself; a dispatch task it claims so after a tile it runs last,
and then it ends.  The protocol is shown free of stuck states, with every
task done, under partial residency; without the check before the first
claim from the head the model reaches a stuck state (a down tile waiting
for a gate/up tile whose group's blocks have not started).
"""
from __future__ import annotations

import sys
from dataclasses import dataclass

import pytest

sys.setrecursionlimit(100000)


@dataclass(frozen=True)
class Plan:
    deps: tuple            # deps[t]: frozenset of tasks t waits for (all < t)
    n_row: int             # tasks handed out by the queue
    combine_deps: tuple    # ring kernel: per token, the tasks its combine waits for


def mfma_plan(n_dispatch=2, units=2, p1=2, p2=2, router_slots=False):
    """router_slots: the router assigned the slots (batches of up to 1024
    tokens; with routing from score bounds the dispatch tasks compute the
    logits and exact routing instead), so gate/up tiles do not wait for the
    dispatch tasks, and down tiles wait for all of them (their combine
    counters, and the routing their combines read) and their unit's gate/up
    tiles."""
    deps = [frozenset()] * n_dispatch
    g0 = n_dispatch
    disp = frozenset(range(n_dispatch))
    for u in range(units):
        deps += [frozenset() if router_slots else disp] * p1
    for u in range(units):
        deps += [disp | frozenset(range(g0 + u * p1, g0 + (u + 1) * p1))] * p2
    return Plan(tuple(deps), len(deps), ())


def ring_plan(experts=2, p1=2, p2=2, tokens=((0, 1), (1,))):
    deps = []
    for e in range(experts):
        deps += [frozenset()] * p1
    d0 = experts * p1
    for e in range(experts):
        deps += [frozenset(range(e * p1, (e + 1) * p1))] * p2
    comb = tuple(frozenset(t for e in tok for t in range(d0 + e * p2, d0 + (e + 1) * p2))
                 for tok in tokens)
    return Plan(tuple(deps), len(deps), comb)


# block state: (status, cur, nxt, flags, comb_i)
#   status 0 waiting to start, 1 running, 2 exited
#   flags: bit 0 = current task's inputs awaited, bit 1 = next task claimed
PENDING, RUNNING, EXITED = 0, 1, 2


def explore(plan: Plan, kind: str, G: int, R: int, first="queue", park=False):
    """Returns None if every interleaving finishes, else a description of a
    reachable stuck state."""
    n = plan.n_row
    ncomb = len(plan.combine_deps)
    seen = set()

    def done_set(done_mask, t):
        return (done_mask >> t) & 1

    def deps_done(done_mask, deps):
        return all(done_set(done_mask, d) for d in deps)

    def moves(state):
        head, done, blocks = state
        running = sum(1 for b in blocks if b[0] == RUNNING)
        out = []
        for i, (st, cur, nxt, fl, ci) in enumerate(blocks):
            if st == PENDING:
                # start in index order when a slot is free
                if running < R and all(b[0] != PENDING for b in blocks[:i]):
                    if first == "static":
                        t = i if i < n else n
                        h = head
                    else:
                        t, h = (head, head + 1) if head < n else (n, head)
                    nb = list(blocks)
                    nb[i] = (RUNNING, t, -1, 0, 0)
                    out.append((h, done, tuple(nb)))
                continue
            if st != RUNNING:
                continue
            if cur < n:
                awaited, claimed = fl & 1, fl & 2
                # wait for the current task's inputs
                if not awaited and deps_done(done, plan.deps[cur]):
                    nb = list(blocks)
                    nb[i] = (st, cur, nxt, fl | 1, ci)
                    out.append((head, done, tuple(nb)))
                # claim the next task: the ring kernel at an early step (before
                # or after the wait), the MFMA kernel after the MFMAs
                if not claimed and (kind == "ring" or awaited):
                    if first == "static" and head < G:
                        h = max(head, G)  # static first tasks 0..G-1; the queue starts at G
                    else:
                        h = head
                    t, h = (h, h + 1) if h < n else (n, h)
                    nb = list(blocks)
                    nb[i] = (st, cur, t, fl | 2, ci)
                    out.append((h, done, tuple(nb)))
                # finish the current task (park: only once the next task's
                # inputs are there too)
                if awaited and claimed and (not park or nxt >= n or deps_done(done, plan.deps[nxt])):
                    nb = list(blocks)
                    nb[i] = (st, nxt, -1, 0, ci)
                    out.append((head, done | (1 << cur), tuple(nb)))
                continue
            # row tasks exhausted: the ring kernel's combine tasks for this block
            tok = i + ci * G
            if kind == "ring" and tok < ncomb:
                if deps_done(done, plan.combine_deps[tok]):
                    nb = list(blocks)
                    nb[i] = (st, cur, nxt, fl, ci + 1)
                    out.append((head, done, tuple(nb)))
                continue
            nb = list(blocks)
            nb[i] = (EXITED, cur, nxt, fl, ci)
            out.append((head, done, tuple(nb)))
        return out

    start = (0, 0, tuple((PENDING, -1, -1, 0, 0) for _ in range(G)))
    if first == "static":
        start = (0, 0, start[2])
    stack = [start]
    while stack:
        s = stack.pop()
        if s in seen:
            continue
        seen.add(s)
        nxt_states = moves(s)
        if not nxt_states:
            head, done, blocks = s
            if not all(b[0] == EXITED for b in blocks):
                return f"stuck: done={bin(done)} blocks={blocks}"
        stack.extend(nxt_states)
    return None


CASES = [(G, R) for G in (1, 2, 3) for R in range(1, G + 1)]


@pytest.mark.parametrize("G,R", CASES)
def test_mfma_kernel_protocol_never_sticks(G, R):
    assert explore(mfma_plan(), "mfma", G, R) is None
    assert explore(mfma_plan(n_dispatch=1, units=3, p1=1, p2=2), "mfma", G, R) is None
    assert explore(mfma_plan(router_slots=True), "mfma", G, R) is None
    assert explore(mfma_plan(n_dispatch=2, units=2, p1=1, p2=2, router_slots=True), "mfma",
                   G, R) is None


@pytest.mark.parametrize("G,R", CASES)
def test_ring_kernel_protocol_never_sticks(G, R):
    assert explore(ring_plan(), "ring", G, R) is None
    assert explore(ring_plan(experts=3, p1=1, p2=1, tokens=((0, 2), (1,), (2, 1))), "ring",
                   G, R) is None


def test_static_first_task_sticks_with_partial_residency():
    # with every block resident it finishes ...
    assert explore(ring_plan(experts=1, p1=2, p2=1, tokens=()), "ring", 2, 2, first="static") is None
    # ... but a non-resident block 1 owns gate/up task 1, which the running
    # block's down task waits for
    r = explore(ring_plan(experts=1, p1=2, p2=1, tokens=()), "ring", 2, 1, first="static")
    assert r is not None and "stuck" in r


def test_parking_on_the_next_task_sticks():
    # one block, one expert: it holds gate/up task 0 while its next task, the
    # expert's down task, needs task 0 finished
    r = explore(ring_plan(experts=1, p1=1, p2=1, tokens=()), "ring", 1, 1, park=True)
    assert r is not None and "stuck" in r
    assert explore(ring_plan(experts=1, p1=1, p2=1, tokens=()), "ring", 1, 1) is None


# Chain-job protocol of the deferred decode routing (explore_chain).
# block: (status, phase, cur, nxt, flags, comb_i, job)
#   phase 1 block-form job at start (first row task claimed after it), 2
#   prologue, 6 block-form job in the fallback's prologue, 3 row tasks, 4
#   combines, 5 wave-form job in a combine's routing wait
def explore_chain(plan: Plan, G: int, R: int, J: int, claim_blocks: int, lazy=False,
                  fallback=False, waits_run_jobs=True, job_waits_next=False):
    n = plan.n_row
    ncomb = len(plan.combine_deps)
    all_jobs = (1 << J) - 1
    seen = set()

    def deps_done(done, deps):
        return all((done >> d) & 1 for d in deps)

    def job_can_finish(jdone, j):
        return not job_waits_next or j + 1 >= J or (jdone >> (j + 1)) & 1

    def repl(blocks, i, b):
        nb = list(blocks)
        nb[i] = b
        return tuple(nb)

    def moves(state):
        head, done, chead, jdone, blocks = state
        running = sum(1 for b in blocks if b[0] == RUNNING)
        out = []
        for i, (st, ph, cur, nxt, fl, ci, job) in enumerate(blocks):
            if st == PENDING:
                if running < R and all(b[0] != PENDING for b in blocks[:i]):
                    if not lazy and i < claim_blocks and chead < J:
                        out.append((head, done, chead + 1, jdone,
                                    repl(blocks, i, (RUNNING, 1, -1, -1, 0, 0, chead))))
                    else:
                        t, h = (head, head + 1) if head < n else (n, head)
                        out.append((h, done, chead, jdone,
                                    repl(blocks, i, (RUNNING, 2, t, -1, 0, 0, -1))))
                continue
            if st != RUNNING:
                continue
            if ph in (1, 6, 5):  # a job in progress: it never waits (unless the variant)
                if job_can_finish(jdone, job):
                    nph = 2 if ph in (1, 6) else 4
                    out.append((head, done, chead, jdone | (1 << job),
                                repl(blocks, i, (st, nph, cur, nxt, fl, ci, -1))))
                continue
            if ph == 2:  # prologue
                if fallback and chead < J:
                    out.append((head, done, chead + 1, jdone,
                                repl(blocks, i, (st, 6, cur, nxt, fl, ci, chead))))
                elif not fallback or jdone == all_jobs:
                    t, h = cur, head
                    if t < 0:  # claimed late, after a job
                        t, h = (head, head + 1) if head < n else (n, head)
                    out.append((h, done, chead, jdone, repl(blocks, i, (st, 3, t, -1, 0, ci, -1))))
                continue
            if ph == 3:  # row tasks (ring kernel: the next claim before or after the wait)
                if cur < n:
                    awaited, claimed = fl & 1, fl & 2
                    if not awaited and deps_done(done, plan.deps[cur]):
                        out.append((head, done, chead, jdone,
                                    repl(blocks, i, (st, ph, cur, nxt, fl | 1, ci, job))))
                    if not claimed:
                        t, h = (head, head + 1) if head < n else (n, head)
                        out.append((h, done, chead, jdone,
                                    repl(blocks, i, (st, ph, cur, t, fl | 2, ci, job))))
                    if awaited and claimed:
                        out.append((head, done | (1 << cur), chead, jdone,
                                    repl(blocks, i, (st, ph, nxt, -1, 0, ci, job))))
                else:
                    out.append((head, done, chead, jdone, repl(blocks, i, (st, 4, cur, nxt, 0, ci, job))))
                continue
            if ph == 4:  # combines: routing first (planned path), then the outputs
                tok = i + ci * G
                if tok >= ncomb:
                    out.append((head, done, chead, jdone, repl(blocks, i, (EXITED, ph, cur, nxt, fl, ci, job))))
                    continue
                routed = fallback or jdone == all_jobs
                if not routed:
                    if waits_run_jobs and chead < J:
                        out.append((head, done, chead + 1, jdone,
                                    repl(blocks, i, (st, 5, cur, nxt, fl, ci, chead))))
                    continue
                if deps_done(done, plan.combine_deps[tok]):
                    out.append((head, done, chead, jdone, repl(blocks, i, (st, ph, cur, nxt, fl, ci + 1, job))))
        return out

    stack = [(0, 0, 0, 0, tuple((PENDING, 0, -1, -1, 0, 0, -1) for _ in range(G)))]
    while stack:
        s = stack.pop()
        if s in seen:
            continue
        seen.add(s)
        nxt_states = moves(s)
        if not nxt_states:
            if not all(b[0] == EXITED for b in s[4]):
                return f"stuck: jobs done={bin(s[3])} tasks done={bin(s[1])} blocks={s[4]}"
        stack.extend(nxt_states)
    return None


CHAIN_PLANS = [ring_plan(), ring_plan(experts=1, p1=2, p2=1, tokens=((0,),)),
               ring_plan(experts=3, p1=1, p2=1, tokens=((0, 2), (1,), (2, 1)))]


@pytest.mark.parametrize("G,R", CASES)
@pytest.mark.parametrize("fallback", [False, True])
def test_chain_job_protocol_never_sticks(G, R, fallback):
    for plan in CHAIN_PLANS:
        for J in (1, 2, 3):
            for claim_blocks in range(0, G + 1):
                assert explore_chain(plan, G, R, J, claim_blocks, fallback=fallback) is None
            assert explore_chain(plan, G, R, J, G, lazy=True, fallback=fallback) is None


def test_chain_waits_that_do_not_run_jobs_stick():
    plan = ring_plan(experts=1, p1=1, p2=1, tokens=((0,),))
    # with jobs claimed at the start the waits never need to run one ...
    assert explore_chain(plan, 2, 2, 2, 2, waits_run_jobs=False) is None
    # ... but when no block claims them (lazy mode, or blocks 0..C-1 not yet
    # resident when the combines wait) someone must
    r = explore_chain(plan, 2, 2, 2, 2, lazy=True, waits_run_jobs=False)
    assert r is not None and "stuck" in r
    r = explore_chain(plan, 2, 1, 2, 1, waits_run_jobs=False)
    assert r is not None and "stuck" in r


def test_a_job_that_waits_for_another_sticks():
    plan = ring_plan(experts=1, p1=1, p2=1, tokens=((0,),))
    # block 0 claims job 0, which waits for job 1; with one block resident
    # nobody else can claim it
    r = explore_chain(plan, 2, 1, 2, 2, job_waits_next=True)
    assert r is not None and "stuck" in r
    assert explore_chain(plan, 2, 1, 2, 2) is None


# First round of claims of the MFMA kernel's routing from score bounds
# (explore_groups).  Group g of K counters (blocks b with b % K == g) hands
# out tasks g, g + K, ... below F = min(G, dispatch + gate/up tasks), none of
# which waits; later tasks come from the queue head, F + 0, 1, ...
# block: (status, cur, nxt, flags, first_left, tiles, last)
#   cur -2: first claim (its group's counter) not yet made, -1: a claim past
#   the first round, next_task to be made; flags as in explore; tiles: the
#   block has run a tile (task >= dispatch tasks); last: a dispatch task
#   claimed after a tile, which the block runs and then ends.
def explore_groups(plan: Plan, G: int, R: int, K: int, n_dispatch: int, n_first: int,
                   check=True):
    n = plan.n_row
    F = min(G, n_first)
    seen = set()

    def quota(g):
        return (F - 1 - g) // K + 1 if F > g else 0

    def deps_done(done, deps):
        return all((done >> d) & 1 for d in deps)

    def next_task(head, gc, first_left):
        """expert_mfma_kernel's next_task (first_round_left, then the head),
        as one step: counters only grow, so the loads it makes first can
        only show more tasks left than there are."""
        gc = list(gc)
        if check and first_left:
            for g in range(K):
                if gc[g] < quota(g):
                    t = gc[g] * K + g
                    gc[g] += 1
                    if t < F:
                        return t, head, tuple(gc), True
            first_left = False
        t, h = (F + head, head + 1) if F + head < n else (n, head)
        return t, h, tuple(gc), first_left

    def repl(blocks, i, b):
        nb = list(blocks)
        nb[i] = b
        return tuple(nb)

    def moves(state):
        head, gc, done, blocks = state
        running = sum(1 for b in blocks if b[0] == RUNNING)
        out = []
        for i, (st, cur, nxt, fl, fleft, tiles, last) in enumerate(blocks):
            if st == PENDING:
                if running < R and all(b[0] != PENDING for b in blocks[:i]):
                    out.append((head, gc, done, repl(blocks, i, (RUNNING, -2, -1, 0, True, False, False))))
                continue
            if st != RUNNING:
                continue
            if cur == -2:  # the group claim
                g = i % K
                t = gc[g] * K + g
                ngc = list(gc)
                ngc[g] += 1
                out.append((head, tuple(ngc), done,
                            repl(blocks, i, (st, t if t < F else -1, -1, 0, fleft, tiles, last))))
                continue
            if cur == -1:  # past the first round: claim on
                t, h, ngc, nfl = next_task(head, gc, fleft)
                out.append((h, ngc, done, repl(blocks, i, (st, t, -1, 0, nfl, tiles, last))))
                continue
            if cur >= n:
                out.append((head, gc, done, repl(blocks, i, (EXITED, cur, nxt, fl, fleft, tiles, last))))
                continue
            awaited, claimed = fl & 1, fl & 2
            if not awaited and deps_done(done, plan.deps[cur]):
                out.append((head, gc, done, repl(blocks, i, (st, cur, nxt, fl | 1, fleft, tiles, last))))
            if awaited and not claimed and not last:
                t, h, ngc, nfl = next_task(head, gc, fleft)
                out.append((h, ngc, done, repl(blocks, i, (st, cur, t, fl | 2, nfl, tiles, last))))
            if awaited and (claimed or last):
                ndone = done | (1 << cur)
                if last:
                    out.append((head, gc, ndone, repl(blocks, i, (EXITED, n, -1, 0, fleft, tiles, last))))
                else:
                    nt = tiles or cur >= n_dispatch
                    out.append((head, gc, ndone, repl(blocks, i, (st, nxt, -1, 0, fleft, nt,
                                                                  nt and nxt < n_dispatch))))
        return out

    start = (0, tuple([0] * K), 0, tuple((PENDING, -1, -1, 0, True, False, False) for _ in range(G)))
    stack = [start]
    while stack:
        s = stack.pop()
        if s in seen:
            continue
        seen.add(s)
        nxt_states = moves(s)
        if not nxt_states:
            if not all(b[0] == EXITED for b in s[3]):
                return f"stuck: done={bin(s[2])} blocks={s[3]}"
            if s[2] != (1 << n) - 1:
                return f"unfinished: done={bin(s[2])}"
        stack.extend(nxt_states)
    return None


GROUP_PLANS = [(dict(n_dispatch=1, units=2, p1=1, p2=1), 1, 2),
               (dict(n_dispatch=2, units=1, p1=2, p2=1), 2, 2),
               (dict(n_dispatch=1, units=1, p1=3, p2=1), 1, 1)]


@pytest.mark.parametrize("G,R", [(G, R) for G in (2, 3, 4) for R in range(1, G + 1)])
@pytest.mark.parametrize("K", [1, 2, 3])
def test_first_round_group_claims_never_stick(G, R, K):
    for kw, nd, units in GROUP_PLANS:
        if G <= nd:  # the kernel uses the groups only in grids of more blocks than dispatch tasks
            continue
        plan = mfma_plan(router_slots=True, **kw)
        n_first = nd + units * kw["p1"]
        assert explore_groups(plan, G, R, K, nd, n_first) is None


def test_first_round_without_the_check_sticks():
    # one dispatch task, two gate/up tiles, a down tile: block 0 (group 0)
    # runs task 0; claiming straight from the head it gets the down tile,
    # which waits for gate/up tile 1 of group 1, whose blocks have not started
    kw = dict(n_dispatch=1, units=1, p1=2, p2=1)
    plan = mfma_plan(router_slots=True, **kw)
    assert explore_groups(plan, 3, 1, 2, 1, 3) is None
    r = explore_groups(plan, 3, 1, 2, 1, 3, check=False)
    assert r is not None and "stuck" in r
    assert explore_groups(plan, 3, 3, 2, 1, 3, check=False) is None
