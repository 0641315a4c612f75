"""The HBM expert slot cache (tlm_hip_store_*) against the oracle's
restatement of the reference's policy (oracle/tlm_oracle_store.c, itself
checked step for step against the reference's tlm_store.c in
test_store_policy.py), and the bytes it puts in HBM against tlm_hip_pack of
the same payload.

Observations are compared after every settle point (see tests/store_script.py):
slots per acquire, return codes, wait / ready results, every counter."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle
from oracle.store import OracleStore
from tests.store_script import experts_grid, first_difference, model_script, run
from tests.synth import random_code_rows
from tierlm_amd._lib import lib

pytestmark = pytest.mark.gpu

NL, NE, TOPK = 4, 8, 2
PRUNED = {(2, 7)}
CPIN = {(3, 5)}
HEAT = {(0, 3): 0.9, (1, 6): 0.8, (2, 1): 0.7, (3, 0): 0.6, (3, 5): 0.05}
D, DE = 256, 256


def a64(x):
    return (x + 63) // 64 * 64


def make_payload(rng, dt, D=D, de=DE):
    """gate | up | down in the reference's row layout, items 64-byte aligned."""
    g, u, d = (random_code_rows(rng, dt, de, D), random_code_rows(rng, dt, de, D), random_code_rows(rng, dt, D, de))
    off = [0, a64(g.nbytes), a64(g.nbytes) + a64(u.nbytes)]
    buf = np.zeros(off[2] + d.nbytes, np.uint8)
    for o, m in zip(off, (g, u, d)):
        buf[o:o + m.nbytes] = m.reshape(-1)
    return buf, off, (g, u, d)


class HipView:
    """HipStore behind the script interface: loads = bytes_read / payload
    length (every payload has the same length), failures through fetch."""

    def __init__(self, experts, payloads, n_slots, pin_frac=0.0, prefetch=1, top_k=TOPK, use_fetch=False,
                 pinned=False, dt=oracle.Q8_0):
        from tierlm_amd.store import HipStore
        self.failing = set()
        self.payloads = payloads
        self.plen = next(iter(payloads.values()))[0].nbytes
        xs = []
        for x in experts:
            buf, off, _ = payloads[(x["layer"], x["id"])]
            if pinned:
                buf = torch.from_numpy(buf).pin_memory()
            xs.append(dict(x, dtype=dt, item_off=off, payload=None if use_fetch else buf, payload_len=self.plen))
            if pinned:
                self.payloads[(x["layer"], x["id"])] = (buf.numpy(), off, payloads[(x["layer"], x["id"])][2])

        def fetch(user, layer, eid, dst, n):
            if (layer, eid) in self.failing:
                return -4
            src = self.payloads[(layer, eid)][0]
            C.memmove(dst, src.ctypes.data, n)
            return 0

        self.s = HipStore(xs, d_model=D, d_expert=DE, top_k=top_k, pin_frac=pin_frac, prefetch=prefetch,
                          budget_bytes=0, fetch=fetch if use_fetch else None)
        sb = self.s.slot_bytes()
        self.s.close()
        self.s = HipStore(xs, d_model=D, d_expert=DE, top_k=top_k, pin_frac=pin_frac, prefetch=prefetch,
                          budget_bytes=n_slots * sb + sb // 2, fetch=fetch if use_fetch else None)

    def __getattr__(self, name):
        return getattr(self.s, name)

    def set_fail(self, layer, eid, on):
        (self.failing.add if on else self.failing.discard)((layer, eid))

    def stats(self):
        st = self.s.stats()
        st["loads"] = st["bytes_read"] // self.plen
        return {k: st[k] for k in ("hits", "misses", "prefetch_issued", "prefetch_used", "prefetch_dropped",
                                   "evictions", "loads", "slots", "pinned", "in_use")}


def grid_payloads(seed, dt=oracle.Q8_0, nl=NL, ne=NE):
    rng = np.random.default_rng(seed)
    return {(l, e): make_payload(rng, dt) for l in range(nl) for e in range(ne)}


def compare(script, n_slots, pin_frac=0.0, prefetch=1, use_fetch=False, pinned=False, top_k=TOPK, ex=None,
            payloads=None):
    ex = experts_grid(NL, NE, pruned=PRUNED, cpin=CPIN, heat=HEAT) if ex is None else ex
    payloads = grid_payloads(1) if payloads is None else payloads
    o = OracleStore(ex, top_k, n_slots, pin_frac, prefetch)
    h = HipView(ex, payloads, n_slots, pin_frac, prefetch, top_k=top_k, use_fetch=use_fetch, pinned=pinned)
    try:
        assert h.n_slots() == o.n_slots()
        a, b = run(o, script), run(h, script)
    finally:
        o.close()
        h.close()
    d = first_difference(a, b)
    assert d is None, f"observation {d[0]}: oracle {d[1]} vs hip {d[2]}"
    return a


@pytest.mark.parametrize("n_slots,hints", [(2, 0), (3, 3), (5, 3), (64, 0)])
def test_policy_matches_oracle(hip, n_slots, hints):
    script = model_script(NL, NE, TOPK, 120, seed=n_slots * 10 + hints, hints=hints, pruned=PRUNED)
    compare(script, n_slots, prefetch=int(hints > 0))


@pytest.mark.parametrize("n_slots,pin_frac", [(5, 0.2), (6, 0.5), (2, 0.9)])
def test_pins_match_oracle(hip, n_slots, pin_frac):
    script = [("warm",), ("stats",), ("warm",), ("stats",)]
    script += model_script(NL, NE, TOPK, 80, seed=n_slots, hints=3, pruned=PRUNED)
    compare(script, n_slots, pin_frac=pin_frac, pinned=True)


def test_held_references_ebusy_and_unknown_ids(hip):
    script = model_script(NL, NE, TOPK, 60, seed=8, hints=3, hold_every=1, pruned=PRUNED, unknown_every=9)
    obs = compare(script, 3)
    rcs = {o[1] for o in obs if o[0] == "acq"}
    assert {-6, -8} <= rcs


def test_failed_loads_match_oracle(hip):
    """A fetch error is the HIP store's failed read: never READY, every holder
    gets the error, the slot is FREE again (src/lib/tlm_store.c:139-158)."""
    script = model_script(NL, NE, TOPK, 60, seed=3, hints=3, fail=[(4, 0, 1), (20, 1, 0), (33, 2, 2)],
                          pruned=PRUNED)
    obs = compare(script, 4, use_fetch=True)
    assert any(o[0] == "wait" and -4 in o[1] for o in obs)


def test_wider_top_k_matches_oracle(hip):
    ex = experts_grid(3, 16)
    pl = {(l, e): make_payload(np.random.default_rng(l * 16 + e), oracle.Q8_0) for l in range(3) for e in range(16)}
    script = model_script(3, 16, 4, 60, seed=4, hints=6)
    for n_slots in (4, 7, 12):
        compare(script, n_slots, top_k=4, ex=ex, payloads=pl)


def device_bytes(ptr, n):
    out = np.empty(n, np.uint8)
    assert lib.tlm_hip_memcpy_d2h(out.ctypes.data, ptr, n, None) == 0
    assert lib.tlm_hip_sync(None) == 0
    return out


def packed(hip, dt, m, rows, n):
    Wd = torch.from_numpy(np.ascontiguousarray(m).reshape(-1)).cuda()
    return hip.pack(dt, Wd, m.shape[1], rows, n).cpu().numpy()[:hip.packed_bytes(dt, rows, n)]


@pytest.mark.parametrize("dt", [oracle.Q8_0, oracle.Q4_K, oracle.Q5_K, oracle.Q6_K])
@pytest.mark.parametrize("pinned", [False, True])
def test_slot_bytes_are_the_packed_payload(hip, dt, pinned):
    """Through a 3-slot store (so most loads evict): after each wait the slot
    holds the expert's gate / up / down exactly as tlm_hip_pack packs them."""
    from tierlm_amd.store import HipStore
    rng = np.random.default_rng(dt + 10 * pinned)
    ex = [{"layer": 0, "id": e} for e in range(6)]
    pl = {(0, e): make_payload(rng, dt) for e in range(6)}
    view = HipView(ex, pl, 3, pinned=pinned, dt=dt)
    shapes = [(DE, D), (DE, D), (D, DE)]
    want = {e: [packed(hip, dt, m, r, n) for m, (r, n) in zip(pl[(0, e)][2], shapes)] for e in range(6)}
    try:
        for e in [0, 1, 2, 3, 0, 4, 5, 1, 2, 2, 5, 3]:
            rc, g = view.acquire(0, [e])
            assert rc == 0 and view.wait(g, 0) == 0
            for m in range(3):
                got = device_bytes(g[0].mats[m], want[e][m].nbytes)
                assert np.array_equal(got, want[e][m]), (e, m)
            view.release(g, 0)
        st = view.s.stats()
        assert st["evictions"] > 0 and st["bytes_read"] == st["misses"] * view.plen
    finally:
        view.close()
    assert isinstance(view.s, HipStore)


def test_stream_wait_and_release_order(hip, dev):
    """Device-side ordering: a matvec enqueued after stream_wait reads the
    loaded expert, and a slot released while that matvec is queued is not
    overwritten under it by the next load (2 slots, every acquire evicts)."""
    dt = oracle.Q6_K
    rng = np.random.default_rng(5)
    ex = [{"layer": 0, "id": e} for e in range(5)]
    pl = {(0, e): make_payload(rng, dt) for e in range(5)}
    view = HipView(ex, pl, 2, prefetch=0, pinned=True, dt=dt)
    x = torch.randn(D, device=dev)
    act = hip.quantize_act(hip.Q8_K, x)
    want = {}
    for e in range(5):
        Wp = torch.from_numpy(packed(hip, dt, pl[(0, e)][2][0], DE, D)).cuda()
        want[e] = hip.matvec_packed(dt, Wp, DE, D, act).cpu().numpy()
    order = [0, 1, 2, 3, 4, 0, 2, 4, 1, 3] * 3
    outs = [torch.empty(DE, device=dev) for _ in order]
    try:
        for i, e in enumerate(order):
            rc, g = view.acquire(0, [e])
            assert rc == 0 and view.stream_wait(g, 0) == 0
            assert lib.tlm_hip_matvec_packed(dt, g[0].mats[0], DE, D, C.c_void_p(act.data_ptr()),
                                             C.c_void_p(outs[i].data_ptr()),
                                             C.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
            view.release(g, 0)
        torch.cuda.synchronize()
        for i, e in enumerate(order):
            got = outs[i].cpu().numpy()
            assert np.array_equal(got.view(np.uint32), want[e].view(np.uint32)), (i, e)
        st = view.s.stats()
        assert st["hits"] + st["misses"] == len(order) and st["evictions"] == st["misses"] - 2 > 10
    finally:
        view.close()


def test_open_rejects_bad_sources(hip):
    from tierlm_amd._lib import HipError
    from tierlm_amd.store import HipStore
    rng = np.random.default_rng(0)
    buf, off, _ = make_payload(rng, oracle.Q8_0)
    good = {"layer": 0, "id": 0, "dtype": oracle.Q8_0, "item_off": off, "payload": buf}
    kw = dict(d_model=D, d_expert=DE, top_k=2, budget_bytes=1 << 24)
    for bad in ({"dtype": oracle.F32}, {"payload_len": buf.nbytes - 1}, {"payload": None}):
        with pytest.raises(HipError):
            HipStore([dict(good, **bad)], **kw)
    with pytest.raises(HipError):
        HipStore([good, dict(good)], **kw)           # duplicate (layer, id)
    s = HipStore([good, dict(good, id=1, flags=2)], **kw)   # the pruned one is left out
    assert s.n_slots() == 1
    rc, g = s.acquire(0, [1])
    assert rc == -6 and s.slots_of(g, 1) == [-1]
    s.close()
