"""One routed MoE block with its experts in the HBM slot cache
(tlm_hip_moe_layer_store) against the same block with every expert resident
(tlm_hip_moe_layer, itself checked against the oracle in test_hip_moe.py).

The reference's cache changes speed, never results (src/lib/tlm_store.h:10-11):
whatever the budget, pins and lookahead hints, every token must carry the
resident block's bits and routing.  Two layers share one cache, as the
reference's single global cache does (tlm_store.c:15)."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle
from tests.synth import build_moe_case

pytestmark = pytest.mark.gpu


def payload(g, u, dn):
    """gate | up | down, 64-byte aligned items (the EXPERT packet payload)."""
    off, at = [], 0
    for m in (g, u, dn):
        off.append(at)
        at = (at + m.nbytes + 63) // 64 * 64
    buf = np.zeros(at, np.uint8)
    for o, m in zip(off, (g, u, dn)):
        buf[o:o + m.nbytes] = m.reshape(-1)
    return buf, off


def store_block(case, dev):
    """A MoeBlock like case.block whose expert table starts out pointing at a
    zeroed dummy expert (valid memory, wrong bytes): only the cache's writes
    make its results right."""
    from tierlm_amd import MoeBlock
    from tierlm_amd import quant as hq
    b = case.block
    dummy = torch.zeros(hq.packed_bytes(case.expert_dt, max(case.D, case.de), max(case.D, case.de)) + 256,
                        dtype=torch.uint8, device=dev)
    blk = MoeBlock(D=case.D, de=case.de, E=case.E, k=case.k, expert_dt=case.expert_dt, ffn_norm=b.keep[0],
                   router_w=b.keep[1], expert_ptrs=[dummy.data_ptr()] * (3 * case.E), router_bias=b.keep[2],
                   mask=b.keep[3], ds=case.ds, shared_dt=case.shared_dt, shared=b.keep[4],
                   shared_gate_inp=b.keep[5], router=b.desc.router, routed_scale=b.desc.routed_scale,
                   eps=b.desc.eps, device=dev)
    blk.keep.append(dummy)
    return blk


def open_store(cases, slots, hints, pin_frac=0.0, pinned=True):
    from tierlm_amd.store import HipStore
    c0 = cases[0]
    xs = []
    for layer, case in enumerate(cases):
        for e, (g, u, dn) in enumerate(case.experts):
            buf, off = payload(g, u, dn)
            if pinned:
                buf = torch.from_numpy(buf).pin_memory()
            xs.append({"layer": layer, "id": e, "dtype": case.expert_dt, "item_off": off, "payload": buf,
                       "heat": 0.5 if e % 7 == 0 else 0.0})
    probe = HipStore(xs, d_model=c0.D, d_expert=c0.de, top_k=c0.k, budget_bytes=0)
    sb = probe.slot_bytes()
    probe.close()
    return HipStore(xs, d_model=c0.D, d_expert=c0.de, top_k=c0.k, budget_bytes=slots * sb, pin_frac=pin_frac,
                    prefetch=int(hints > 0))


def run_tokens(cases, dev, slots, hints, tokens=12, pin_frac=0.0, pinned=True, seed=0):
    blocks = [store_block(c, dev) for c in cases]
    store = open_store(cases, slots, hints, pin_frac, pinned)
    if pin_frac:
        assert store.warm() == 0
    rng = np.random.default_rng(seed)
    D = cases[0].D
    try:
        for t in range(tokens):
            h0 = (rng.standard_normal(D) * (1 + t % 3)).astype(np.float32)
            h_res = torch.from_numpy(h0.copy()).to(dev)
            h_st = torch.from_numpy(h0.copy()).to(dev)
            for layer, (case, blk) in enumerate(zip(cases, blocks)):
                case.block(h_res)
                want_ids = case.block.ids.cpu().numpy()[:case.k].tolist()
                nxt = (layer + 1) % len(cases)
                hint = [(blocks[nxt], nxt, hints)] if hints else []
                ids, _ = blk.step_store(store, layer, h_st, hints=hint)
                assert ids == want_ids, (t, layer)
            store.tick()
            torch.cuda.synchronize()
            assert np.array_equal(h_st.cpu().numpy().view(np.uint32), h_res.cpu().numpy().view(np.uint32)), t
        store.settle()
        return store.stats()
    finally:
        store.close()


def two_layers(dev, D=512, de=256, E=32, k=4, ds=0, dt=oracle.Q6_K):
    return [build_moe_case(D=D, de=de, E=E, k=k, ds=ds, expert_dt=dt, seed=100 + s, device=dev,
                           weights="random_codes") for s in range(2)]


@pytest.mark.parametrize("slots,hints", [(4, 0), (10, 0), (10, 4), (24, 6), (64, 4)])
def test_store_block_equals_resident(hip, dev, slots, hints):
    st = run_tokens(two_layers(dev), dev, slots, hints)
    assert st["misses"] > 0 and st["in_use"] == 0
    if slots < 64:
        assert st["evictions"] > 0
    if hints and slots > 4:
        assert st["prefetch_issued"] > 0


def test_store_block_pins_pageable_and_shared_expert(hip, dev):
    """Pinned hot experts, pageable payloads (loader-thread copies) and a
    resident shared expert beside the cached routed ones."""
    cases = two_layers(dev, ds=256)
    st = run_tokens(cases, dev, 12, 4, pin_frac=0.25, pinned=False, seed=3)
    assert st["pinned"] == 3 and st["misses"] > 0


@pytest.mark.parametrize("dt", [oracle.Q8_0, oracle.Q4_K, oracle.Q5_K])
def test_store_block_other_dtypes(hip, dev, dt):
    run_tokens(two_layers(dev, dt=dt), dev, 9, 4, tokens=6, seed=int(dt))


def test_budget_below_top_k_is_ebusy_and_leaves_h(hip, dev):
    """Fewer unpinned slots than top_k: the acquire fails (TLM_EBUSY), h is
    unchanged and no reference is left behind (tlm_model.c:983-986)."""
    from tierlm_amd._lib import HipError
    cases = two_layers(dev)
    blk = store_block(cases[0], dev)
    store = open_store(cases, 3, 0)
    try:
        h = torch.randn(cases[0].D, device=dev)
        h0 = h.clone()
        with pytest.raises(HipError) as ei:
            blk.step_store(store, 0, h)
        assert ei.value.code == -8
        torch.cuda.synchronize()
        assert torch.equal(h, h0)
        assert store.stats()["in_use"] == 0
    finally:
        store.close()


def test_two_hints_prefetch_their_own_routes(hip, dev):
    """Two lookahead hints in one call (tlm_model.c:988-991): each prefetches
    the experts its own router picks on the block's input residual, so after
    the loader drains both layers' routes are all hits."""
    cases = [build_moe_case(D=512, de=256, E=32, k=4, ds=0, expert_dt=oracle.Q6_K, seed=120 + s, device=dev,
                            weights="random_codes") for s in range(3)]
    blocks = [store_block(c, dev) for c in cases]
    store = open_store(cases, 40, 4)
    try:
        rng = np.random.default_rng(9)
        h0 = rng.standard_normal(cases[0].D).astype(np.float32)
        want = [c.host.run(h0, trace=True)[1].tolist() for c in cases]
        assert want[1] != want[2]
        h = torch.from_numpy(h0.copy()).to(dev)
        ids, _ = blocks[0].step_store(store, 0, h, hints=[(blocks[1], 1, 4), (blocks[2], 2, 4)])
        assert ids == want[0]
        torch.cuda.synchronize()
        store.settle()
        before = store.stats()
        assert before["prefetch_issued"] == 8
        for layer in (1, 2):
            rc, refs = store.acquire(layer, want[layer])
            assert rc == 0
            for j in range(4):
                assert store.wait(refs, j) == 0
                store.release(refs, j)
        after = store.stats()
        assert after["hits"] - before["hits"] == 8 and after["misses"] == before["misses"]
    finally:
        store.close()


def test_hints_sharing_a_workspace_are_rejected(hip, dev):
    """Routes are read back after all of them ran: a workspace shared by two
    hints (or by a hint and the block) would hand both the last route."""
    import ctypes as C
    from tierlm_amd._lib import MoeDesc, MoeHint, lib
    cases = two_layers(dev)
    blocks = [store_block(c, dev) for c in cases]
    store = open_store(cases, 16, 4)
    try:
        h = torch.randn(cases[0].D, device=dev)
        dsc = MoeDesc.from_buffer_copy(blocks[1].desc)
        ws = torch.empty(int(lib.tlm_hip_moe_workspace_bytes(C.byref(dsc))) + 4096, dtype=torch.uint8, device=dev)
        ids, w = (C.c_int32 * 4)(), (C.c_float * 4)()
        for off_a, off_b in ((0, 0), (0, 256)):
            arr = (MoeHint * 2)(MoeHint(C.pointer(dsc), 1, C.c_void_p(ws.data_ptr() + off_a)),
                                MoeHint(C.pointer(dsc), 0, C.c_void_p(ws.data_ptr() + off_b)))
            rc = lib.tlm_hip_moe_layer_store(C.byref(blocks[0].desc), store.h, 0, C.c_void_p(h.data_ptr()), ids, w,
                                             arr, 2, C.c_void_p(blocks[0].workspace.data_ptr()), None)
            assert rc == -3
        arr = (MoeHint * 1)(MoeHint(C.pointer(dsc), 1, C.c_void_p(blocks[0].workspace.data_ptr())))
        rc = lib.tlm_hip_moe_layer_store(C.byref(blocks[0].desc), store.h, 0, C.c_void_p(h.data_ptr()), ids, w,
                                         arr, 1, C.c_void_p(blocks[0].workspace.data_ptr()), None)
        assert rc == -3
        assert store.stats()["in_use"] == 0
    finally:
        store.close()


@pytest.mark.parametrize("dt,router", [(oracle.Q4_K, 2), (oracle.Q5_K, 0)])
def test_store_block_c5_shape(hip, dev, dt, router):
    """The 94-layer D 4096 model's block: 128 experts top-8 of width 1536,
    Q4_K or Q5_K (10.6 / 13.0 MB per expert), sigmoid + bias selection with a
    routed scale or softmax + renormalise, through a 24-slot cache (fewer
    slots than experts, so tokens evict each other's experts) with a
    lookahead hint - every token's ids, weights and residual bits equal the
    oracle's block."""
    bias = np.linspace(-0.05, 0.05, 128).astype(np.float32) if router == 2 else None
    case = build_moe_case(D=4096, de=1536, E=128, k=8, ds=0, expert_dt=dt, seed=500 + router, device=dev,
                          weights="random_codes", router=router, routed_scale=2.5 if router else 1.0,
                          router_bias=bias)
    blk = store_block(case, dev)
    store = open_store([case], 24, 8)
    rng = np.random.default_rng(router)
    try:
        for t in range(6):
            h0 = (rng.standard_normal(case.D) * (1 + t % 3)).astype(np.float32)
            want_h, want_ids, want_w, _ = case.host.run(h0, trace=True)
            h = torch.from_numpy(h0.copy()).to(dev)
            ids, w = blk.step_store(store, 0, h, hints=[(blk, 0, 8)])
            store.tick()
            assert ids == want_ids.tolist(), t
            assert np.array_equal(np.asarray(w, np.float32).view(np.uint32),
                                  np.asarray(want_w, np.float32).view(np.uint32)), t
            got = h.cpu().numpy()
            nd = int((got.view(np.uint32) != want_h.view(np.uint32)).sum())
            assert nd == 0, f"token {t}: {nd} of {case.D} residual elements differ from the oracle"
        store.settle()
        st = store.stats()
        assert st["misses"] > 0 and st["evictions"] > 0 and st["in_use"] == 0
    finally:
        store.close()


def breadth(hw, hk, top, interest, instinct, seen, heat):
    """The prefetch breadth of a hint, tlm_model.c:863-874 restated: W =
    interest (1 - I) (1 - H) clamped to [0, 1], I the layer's instinct averaged
    with the current top-1 share (the share alone before the layer was seen),
    H its heat; top_k + round(W x (lookahead_k - top_k))."""
    if not (interest > 0.0 and hk > top):
        return hk
    s = float(np.sum(np.asarray(hw[:hk], np.float64)))
    now = float(hw[0]) / s if s > 0.0 else 0.0
    i = 0.5 * (now + instinct) if seen else now
    w = min(1.0, max(0.0, interest * (1.0 - i) * (1.0 - heat)))
    return top + int(w * (hk - top) + 0.5)


def three_layers(dev):
    return [build_moe_case(D=512, de=256, E=32, k=4, ds=0, expert_dt=oracle.Q6_K, seed=300 + s, device=dev,
                           weights="random_codes") for s in range(3)]


def hint_weights(blk, hk, h, dev):
    """The lookahead's routing of block blk with hk experts from residual h
    (tlm_hip_moe_route on a copy of its descriptor), host weights."""
    from tierlm_amd._lib import MoeDesc, check, lib
    from tierlm_amd.quant import stream
    hid = torch.zeros(32, dtype=torch.int32, device=dev)
    hw = torch.zeros(32, dtype=torch.float32, device=dev)
    hd = MoeDesc.from_buffer_copy(blk.desc)
    hd.k = hk
    ws = torch.empty(int(lib.tlm_hip_moe_workspace_bytes(C.byref(hd))), dtype=torch.uint8, device=dev)
    check(lib.tlm_hip_moe_route(C.byref(hd), C.c_void_p(h.data_ptr()), C.c_void_p(hid.data_ptr()),
                                C.c_void_p(hw.data_ptr()), C.c_void_p(ws.data_ptr()), stream()))
    torch.cuda.synchronize()
    return hw.cpu().numpy()


@pytest.mark.parametrize("interest,lk,slots,host_routes", [(0.0, 0, 40, False), (0.0, 8, 40, False),
                                                         (0.8, 10, 36, False), (0.8, 10, 96, False),
                                                         (0.0, 0, 40, True), (0.8, 10, 36, True)])
def test_stack_equals_resident(hip, dev, interest, lk, slots, host_routes):
    """tlm_hip_moe_stack_store over three layers for eight tokens, the slots
    resolved on the device or by the host: every token's h and routing bit
    for bit the resident blocks', the instinct state updated from each
    block's routing as the reference updates it, and one acquire of top_k per
    layer per token in the cache's counters."""
    from tierlm_amd import MoeStack
    cases = three_layers(dev)
    L, k = len(cases), cases[0].k
    store = open_store(cases, slots, 1)
    blocks = [store_block(c, dev) for c in cases]
    stack = MoeStack(blocks, lookahead=1, lookahead_k=lk, interest=interest, heat=[0.1, 0.4, 0.0],
                     host_routes=host_routes)
    instinct, seen = np.zeros(L), np.zeros(L, np.int64)
    rng = np.random.default_rng(5)
    try:
        for t in range(8):
            h0 = (rng.standard_normal(512) * (1 + t % 3)).astype(np.float32)
            h_res = torch.from_numpy(h0.copy()).to(dev)
            h_st = torch.from_numpy(h0.copy()).to(dev)
            stack(store, h_st)
            for layer, case in enumerate(cases):
                case.block(h_res)
                assert stack.ids[layer].tolist() == case.block.ids.cpu().numpy()[:k].tolist(), (t, layer)
                w = case.block.w.cpu().numpy()[:k].astype(np.float64)   # tlm_model.c:974-980
                instinct[layer] += (w[0] / w.sum() - instinct[layer]) * 0.05
                seen[layer] += 1
            torch.cuda.synchronize()
            assert np.array_equal(h_st.cpu().numpy().view(np.uint32), h_res.cpu().numpy().view(np.uint32)), t
            assert np.allclose(stack.instinct, instinct, rtol=0, atol=1e-12) and (stack.seen == seen).all()
        store.settle()
        st = store.stats()
        assert st["hits"] + st["misses"] == 8 * L * k
        if lk or interest:
            assert st["prefetch_issued"] > 0
    finally:
        store.close()


@pytest.mark.parametrize("interest,heat", [(0.8, [0.0, 0.3, 0.6]), (0.35, [0.2, 0.0, 0.1]), (0.0, [0.0] * 3)])
def test_stack_lookahead_breadth(hip, dev, interest, heat):
    """The interest-weighted lookahead breadth: each token through a fresh
    cache with a slot for every expert, so no hinted expert of the next layer
    is there yet; the hints considered - issued, or dropped because too many
    earlier hints are still loading (the admission rule of tlm_store.c:
    694-718, which depends on how far the loads have got) - must be the sum
    over layers of the breadth restated here (tlm_model.c:863-874) from the
    hint's routing, with the instinct state carried from token to token."""
    from tierlm_amd import MoeStack
    cases = three_layers(dev)
    L, k, hk = len(cases), cases[0].k, 10
    blocks = [store_block(c, dev) for c in cases]
    stack = MoeStack(blocks, lookahead=1, lookahead_k=hk, interest=interest, heat=heat)
    instinct, seen = np.zeros(L), np.zeros(L, np.int64)
    rng = np.random.default_rng(9)
    for t in range(3):
        store = open_store(cases, L * cases[0].E, 1)
        try:
            h0 = rng.standard_normal(512).astype(np.float32)
            h_res = torch.from_numpy(h0.copy()).to(dev)
            want = 0
            for layer, case in enumerate(cases):
                if layer + 1 < L:   # the hint reads the residual before this layer's update
                    hw = hint_weights(blocks[layer + 1], hk, h_res, dev)
                    want += breadth(hw, hk, k, interest, instinct[layer + 1], seen[layer + 1], heat[layer + 1])
                case.block(h_res)
                w = case.block.w.cpu().numpy()[:k].astype(np.float64)
                instinct[layer] += (w[0] / w.sum() - instinct[layer]) * 0.05
                seen[layer] += 1
            h_st = torch.from_numpy(h0.copy()).to(dev)
            stack(store, h_st)
            store.settle()
            st = store.stats()
            got = st["prefetch_issued"] + st["prefetch_dropped"]
            assert got == want and st["prefetch_issued"] > 0, (t, got, want)
            if interest == 0.0:
                assert want == (L - 1) * hk
        finally:
            store.close()
