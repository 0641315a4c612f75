"""Operation scripts for the expert slot cache (src/lib/tlm_store.h:49-62),
one runner for every implementation - the oracle's restatement, the
reference's own tlm_store.c, the HIP store - so that their observations can
be compared step by step.

A script is a list of tuples:
  ("acq", layer, ids)      acquire; opens group g = number of acquires so far
  ("wait", g) / ("ready", g) / ("rel", g)   on every entry of group g
  ("pf", layer, ids)       prefetch hints
  ("tick", n)              n decay-clock ticks
  ("settle",)              wait until no load is in flight
  ("warm",)                pin the hottest experts
  ("stats",)               counters
  ("fail", layer, id, on)  while on, loads of that expert fail

Timing: the reference completes reads on I/O threads and the HIP store on the
GPU, so decisions that depend on a load still being in flight differ in time.
The generators below settle before every such decision; within one acquire or
prefetch call the in-flight counts cannot change and need no settle.
"""
import numpy as np


def run(store, script):
    groups, obs = [], []
    for op in script:
        kind = op[0]
        if kind == "acq":
            rc, g = store.acquire(op[1], list(op[2]))
            groups.append((g, len(op[2])))
            obs.append(("acq", rc, store.slots_of(g, len(op[2]))))
        elif kind in ("wait", "ready"):
            g, n = groups[op[1]]
            fn = store.wait if kind == "wait" else store.is_ready
            obs.append((kind, [fn(g, j) for j in range(n)]))
        elif kind == "rel":
            g, n = groups[op[1]]
            for j in range(n):
                store.release(g, j)
        elif kind == "pf":
            store.prefetch(op[1], list(op[2]))
        elif kind == "tick":
            for _ in range(op[1]):
                store.tick()
        elif kind == "settle":
            store.settle()
        elif kind == "warm":
            obs.append(("warm", store.warm()))
        elif kind == "stats":
            obs.append(("stats", store.stats()))
        elif kind == "fail":
            store.set_fail(op[1], op[2], op[3])
        else:
            raise ValueError(op)
    return obs


def first_difference(a, b):
    for i, (x, y) in enumerate(zip(a, b)):
        if x != y:
            return i, x, y
    if len(a) != len(b):
        return min(len(a), len(b)), None, None
    return None


def experts_grid(nl, ne, pruned=(), cpin=(), heat=None):
    """Every (layer, id) of an nl x ne grid; pruned ones are left out (they are
    written as pruned packets by the reference fixture)."""
    out = []
    for l in range(nl):
        for e in range(ne):
            if (l, e) in pruned:
                continue
            x = {"layer": l, "id": e}
            if (l, e) in cpin:
                x["flags"] = 1
            if heat and (l, e) in heat:
                x["heat"] = float(np.float32(heat[(l, e)]))
            out.append(x)
    return out


def model_script(nl, ne, top_k, steps, seed, hints=0, hold_every=0, fail=(), pruned=(), unknown_every=0):
    """A decode-like workload: per step, one layer's top-k (skewed: 70 % of
    picks from experts 0..2), optional router-lookahead hints for the next
    step (one right, one sometimes right, the rest guesses), waits, releases
    and a tick.  hold_every > 0 keeps every such step's references over the
    next step (so acquires meet referenced slots and can fail with EBUSY);
    fail lists (step, layer, id) at which loads of an expert start failing
    (and stop again 5 steps later); unknown_every asks for an absent id."""
    rng = np.random.default_rng(seed)
    seq = []
    for i in range(steps):
        layer = i % nl
        ids = []
        while len(ids) < top_k:
            r = rng.random()
            e = int(rng.integers(0, 3)) if r < 0.7 else int(rng.integers(0, ne))
            if (layer, e) in pruned or e in ids:
                continue
            ids.append(e)
        seq.append((layer, ids))
    script, g, held = [], 0, None
    fails = {s: (l, e) for s, l, e in fail}
    for i, (layer, ids) in enumerate(seq):
        if i in fails:
            script.append(("fail", *fails[i], 1))
        if i - 5 in fails:
            script.append(("fail", *fails[i - 5], 0))
        if unknown_every and i % unknown_every == unknown_every - 1:
            ids = ids + [ne + 3]
        script.append(("acq", layer, ids))
        cur = g
        g += 1
        if hints and i + 1 < len(seq):
            if top_k > 4:   # more than 4 demand reads may still be in flight: settle first
                script.append(("settle",))
            nl_, nxt = seq[i + 1]
            guess = [nxt[0], nxt[1 % len(nxt)] if i % 2 else int(rng.integers(0, ne))]
            guess += [int(rng.integers(0, ne)) for _ in range(hints - 2)]
            script.append(("pf", nl_, guess[:hints]))
        script.append(("settle",))
        script.append(("wait", cur))
        script.append(("ready", cur))
        if held is not None:
            script.append(("rel", held))
            held = None
        if hold_every and i % hold_every == 0:
            held = cur
        else:
            script.append(("rel", cur))
        script.append(("tick", 1))
        if i % 7 == 6:
            script.append(("stats",))
    if held is not None:
        script.append(("rel", held))
    script.append(("settle",))
    script.append(("stats",))
    return script
