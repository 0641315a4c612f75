"""The oracle's slot cache policy (oracle/tlm_oracle_store.c) against the
reference's own tlm_store.c (compiled from its sources into oracle/_ref, over
a packet-store fixture written by the reference's writer), step for step on
the same operation scripts, plus the known answers of the reference's own
store tests (tests/test_store.c:356-560 there).  CPU only."""
import pytest

import oracle
from oracle.store import OracleStore, RefStore
from tests.store_script import experts_grid, first_difference, model_script, run

NL, NE, TOPK = 4, 8, 2
PRUNED = {(2, 7)}
CPIN = {(3, 5)}
HEAT = {(0, 3): 0.9, (1, 6): 0.8, (2, 1): 0.7, (3, 0): 0.6, (3, 5): 0.05}

needs_ref = pytest.mark.skipif(oracle.ref is None, reason="oracle/_ref (the reference's build) not present")


def experts():
    return experts_grid(NL, NE, pruned=PRUNED, cpin=CPIN, heat=HEAT)


def both(script, n_slots, pin_frac=0.0, prefetch=1, top_k=TOPK, ex=None, nl=NL, ne=NE):
    ex = experts() if ex is None else ex
    o = OracleStore(ex, top_k, n_slots, pin_frac, prefetch)
    r = RefStore(ex, top_k, n_slots, pin_frac, prefetch, n_layers=nl, n_experts=ne)
    try:
        assert o.n_slots() == r.n_slots()
        a, b = run(o, script), run(r, script)
    finally:
        o.close()
        r.close()
    return a, b


def assert_same(a, b, script):
    d = first_difference(a, b)
    assert d is None, f"observation {d[0]}: oracle {d[1]} vs reference {d[2]}"


@needs_ref
@pytest.mark.parametrize("n_slots", [2, 3, 5, 64])
@pytest.mark.parametrize("hints", [0, 3])
def test_model_sequences(n_slots, hints):
    script = model_script(NL, NE, TOPK, 160, seed=n_slots * 10 + hints, hints=hints, pruned=PRUNED)
    a, b = both(script, n_slots, prefetch=int(hints > 0))
    assert_same(a, b, script)
    last = a[-1][1]
    assert last["hits"] + last["misses"] == 160 * TOPK and last["in_use"] == 0
    if n_slots <= 3:
        assert last["evictions"] > 0
    if hints and n_slots > TOPK:
        assert last["prefetch_issued"] > 0 and last["prefetch_used"] > 0


@needs_ref
@pytest.mark.parametrize("n_slots,pin_frac", [(5, 0.2), (6, 0.5), (2, 0.9), (8, 0.45)])
def test_pins_then_churn(n_slots, pin_frac):
    script = [("warm",), ("stats",), ("warm",), ("stats",)]
    script += model_script(NL, NE, TOPK, 120, seed=n_slots, hints=3, pruned=PRUNED)
    a, b = both(script, n_slots, pin_frac=pin_frac)
    assert_same(a, b, script)


@needs_ref
@pytest.mark.parametrize("hold_every", [1, 2])
def test_held_references_and_ebusy(hold_every):
    script = model_script(NL, NE, TOPK, 90, seed=7 + hold_every, hints=3, hold_every=hold_every,
                          pruned=PRUNED, unknown_every=9)
    a, b = both(script, 3)
    assert_same(a, b, script)
    rcs = {o[1] for o in a if o[0] == "acq"}
    assert -6 in rcs                      # TLM_ENOTFOUND for the absent id
    if hold_every == 1:
        assert -8 in rcs                  # TLM_EBUSY: every slot referenced


@needs_ref
def test_failed_loads():
    script = model_script(NL, NE, TOPK, 80, seed=3, hints=3, fail=[(4, 0, 1), (20, 1, 0), (33, 2, 2)],
                          pruned=PRUNED)
    a, b = both(script, 4)
    assert_same(a, b, script)
    assert any(o[0] == "wait" and -4 in o[1] for o in a)   # TLM_EFORMAT reaches the holders


@needs_ref
@pytest.mark.parametrize("top_k,ne", [(4, 16), (8, 32)])
def test_wider_top_k(top_k, ne):
    ex = experts_grid(3, ne)
    script = model_script(3, ne, top_k, 90, seed=top_k, hints=6)
    for n_slots in (top_k, top_k + 3, 3 * top_k):
        a, b = both(script, n_slots, top_k=top_k, ex=ex, nl=3, ne=ne)
        assert_same(a, b, script)


# ---- known answers of the reference's store tests, on both implementations --

def kat_stores(n_slots, prefetch=1, pin_frac=0.0):
    out = [OracleStore(experts(), TOPK, n_slots, pin_frac, prefetch)]
    if oracle.ref is not None:
        out.append(RefStore(experts(), TOPK, n_slots, pin_frac, prefetch, n_layers=NL, n_experts=NE))
    return out


def touch(s, layer, e):
    """acquire one expert, wait, release: 1 = hit, 0 = miss (tests/test_store.c:214-236)"""
    before = s.stats()
    rc, g = s.acquire(layer, [e])
    s.settle()
    ok = rc == 0 and s.wait(g, 0) == 0
    s.release(g, 0)
    after = s.stats()
    if not ok:
        return -1
    return 1 if after["hits"] == before["hits"] + 1 else 0


@pytest.mark.parametrize("which", [0, 1])
def test_kat_lfu_decay_and_hints(which):
    """tests/test_store.c:356-414: eviction by lowest (decayed frequency, last
    use); a hint may only take a frequency-0 slot; three halvings clear it."""
    stores = kat_stores(3)
    if which >= len(stores):
        pytest.skip("oracle/_ref not built")
    s = stores[which]
    steps = [(0, 0), (0, 1), (0, 1), (0, 1), (1, 0), (2, 0), (4, 0), (0, 1), (2, 1), (1, 0), (4, 0), (0, 1),
             (1, 1), (2, 0)]
    assert [touch(s, 0, e) for e, _ in steps] == [h for _, h in steps]
    assert s.stats()["evictions"] == 4
    s.prefetch(0, [5])
    s.prefetch(0, [1])
    st = s.stats()
    assert (st["prefetch_issued"], st["prefetch_dropped"]) == (0, 1)
    for _ in range(48):
        s.tick()
    s.prefetch(0, [5])
    s.settle()
    st = s.stats()
    assert (st["prefetch_issued"], st["evictions"]) == (1, 5)
    assert touch(s, 0, 5) == 1 and s.stats()["prefetch_used"] == 1
    assert [touch(s, 0, 0), touch(s, 0, 2), touch(s, 0, 1)] == [0, 1, 0]
    for x in stores:
        x.close()


@pytest.mark.parametrize("which", [0, 1])
def test_kat_prefetch_reserve(which):
    """tests/test_store.c:420-470: hints in flight leave top_k slots for demand."""
    cases = [(3, 0.0, 1, 3), (2, 0.0, 0, 4), (5, 0.2, 2, 2)]
    for n_slots, pin_frac, issued, dropped in cases:
        stores = kat_stores(n_slots, pin_frac=pin_frac)
        if which >= len(stores):
            pytest.skip("oracle/_ref not built")
        s = stores[which]
        if pin_frac:
            assert s.warm() == 0 and s.stats()["pinned"] == 1
        s.prefetch(1, [0, 1, 2, 3])
        st = s.stats()
        assert (st["prefetch_issued"], st["prefetch_dropped"]) == (issued, dropped)
        rc, g = s.acquire(1, [4, 5])
        assert rc == 0 and all(x >= 0 for x in s.slots_of(g, 2))
        s.settle()
        assert [s.wait(g, j) for j in range(2)] == [0, 0]
        s.release(g, 0)
        s.release(g, 1)
        if n_slots == 3:
            assert touch(s, 1, 0) == 1 and s.stats()["prefetch_used"] == 1
        for x in stores:
            x.close()


@pytest.mark.parametrize("which", [0, 1])
def test_kat_pins(which):
    """tests/test_store.c:473-527: the compiler pin first, then manifest heat;
    pin_frac is capped so one streaming slot survives."""
    stores = kat_stores(6, pin_frac=0.5)
    if which >= len(stores):
        pytest.skip("oracle/_ref not built")
    s = stores[which]
    assert s.warm() == 0
    st = s.stats()
    assert (st["pinned"], st["in_use"], st["misses"], st["loads"]) == (3, 0, 0, 3)
    assert s.warm() == 0 and s.stats()["pinned"] == 3
    for l, e in [(3, 5), (0, 3), (1, 6)]:
        assert touch(s, l, e) == 1
    for x in stores:
        x.close()
    stores = kat_stores(2, prefetch=0, pin_frac=0.9)
    s = stores[which]
    assert s.warm() == 0 and s.stats()["pinned"] == 1
    assert [touch(s, 0, 0), touch(s, 0, 1), touch(s, 3, 5)] == [0, 0, 1]
    for x in stores:
        x.close()


@pytest.mark.parametrize("which", [0, 1])
def test_kat_ebusy_and_notfound(which):
    """tests/test_store.c:529-590."""
    stores = kat_stores(2)
    if which >= len(stores):
        pytest.skip("oracle/_ref not built")
    s = stores[which]
    rc, g01 = s.acquire(0, [0, 1])
    s.settle()
    assert rc == 0 and [s.wait(g01, j) for j in range(2)] == [0, 0]
    rc, gx = s.acquire(1, [0])
    assert rc == -8 and s.slots_of(gx, 1) == [-1]
    assert s.wait(gx, 0) == -3 and not s.is_ready(gx, 0)
    assert s.stats()["in_use"] == 2
    rc, gy = s.acquire(0, [0])
    assert rc == 0 and s.slots_of(gy, 1) == s.slots_of(g01, 1)
    s.release(gy, 0)
    s.release(g01, 0)
    rc, gz = s.acquire(1, [0])
    s.settle()
    assert rc == 0 and s.wait(gz, 0) == 0 and s.slots_of(gz, 1)[0] != s.slots_of(g01, 2)[1]
    s.release(gz, 0)
    s.release(g01, 1)
    rc, gp = s.acquire(2, [7])
    assert rc == -6 and s.slots_of(gp, 1) == [-1]
    rc, gm = s.acquire(3, [2, 99])
    s.settle()
    assert rc == -6 and s.slots_of(gm, 2)[0] >= 0 and s.slots_of(gm, 2)[1] == -1
    s.release(gm, 0)
    assert s.acquire(NL, [0])[0] == -6 and s.acquire(-1, [0])[0] == -6
    s.prefetch(2, [7])
    assert s.stats()["in_use"] == 0 and s.stats()["prefetch_issued"] == 0
    for x in stores:
        x.close()


def hint_victim_script():
    """An unused hint publishes with last use 0 (tlm_store.c:185-187), so among
    frequency-0 slots it is the first victim, before older demand loads."""
    return [("acq", 0, [0]), ("settle",), ("wait", 0), ("rel", 0),
            ("acq", 0, [1]), ("settle",), ("wait", 1), ("rel", 1),
            ("tick", 64), ("pf", 0, [4]), ("settle",), ("stats",),
            ("acq", 0, [5]), ("settle",), ("wait", 2), ("rel", 2), ("stats",),
            ("acq", 0, [4]), ("settle",), ("wait", 3), ("rel", 3), ("stats",)]


@pytest.mark.parametrize("which", [0, 1])
def test_kat_unused_hint_is_first_victim(which):
    stores = kat_stores(3)
    if which >= len(stores):
        pytest.skip("oracle/_ref not built")
    obs = run(stores[which], hint_victim_script())
    for x in stores:
        x.close()
    acqs = [o for o in obs if o[0] == "acq"]
    assert acqs[2][2] == [2]                      # expert 5 takes the hint's slot
    assert obs[-1][1]["misses"] == 4 and obs[-1][1]["prefetch_used"] == 0
