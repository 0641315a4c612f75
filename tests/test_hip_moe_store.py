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
                   shared_gate_inp=b.keep[5], device=dev)
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
