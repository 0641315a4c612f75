"""The whole decode step with the experts in the HBM slot cache
(tlm_hip_model_opts.expert_cache_bytes): the payloads stay in page-locked host
memory, each layer routes on the device, the host acquires the experts (and
hints the next layer's) and the block reads the slots - tierlm's runtime with
its store (src/bin/tierlm.c:286-309, src/lib/tlm_model.c:960-1055).  A block
that reads slots carries the resident block's bits, so:

* on the reference's compiled stores (C1, C2S, C3S) the step must give the
  reference's outputs exactly as the resident step does - teacher-forced
  top-10 logits bit for bit, free-running greedy tokens - with a cache of
  only top_k slots (every token evicts) and with one that holds every expert;
* a synthetic model built with its experts in host memory (one payload per
  expert) gives the resident synthetic model's logits and routing bit for bit,
  for each expert dtype, with and without a shared expert;
* the counters move as a cache's should (evictions on a cache of top_k
  slots, hits and misses, lookahead hints issued and used), and a routing
  heat plus the interest-weighted lookahead run;
* a prompt runs batched through the cache (each chunk's experts acquired in
  passes of the unpinned slots) with the resident batched prefill's and the
  cached step-by-step prefill's bits, and the C3S / C5S references' logits."""
import numpy as np
import pytest

from tests.test_hip_model import C1, C2S, C3S, C5S, greedy_tokens, needs_c1, needs_c2s, needs_c3s, needs_c5s, \
    prompt_tokens, teacher_forced

pytestmark = pytest.mark.gpu

TINY = 1          # raised to top_k slots by the model (src/bin/tierlm.c:273-285)
ALL = 1 << 34     # every expert in a slot


@needs_c1
@pytest.mark.parametrize("budget", [TINY, ALL])
def test_c1_cached_reference_bits(hip, budget):
    from tierlm_amd.model import Model
    m = Model(C1, max_ctx=256, expert_cache=budget)
    try:
        st = m.store_stats()
        assert st is not None
        assert st["slots"] == (m.geom.top_k if budget == TINY else m.geom.n_layers * m.geom.n_experts)
        teacher_forced(m, "c1_oracle.jsonl", prompt_tokens() + greedy_tokens()[:63])
        m.reset()
        assert m.generate(prompt_tokens(), 64) == greedy_tokens()
        st = m.store_stats()
        assert st["misses"] > 0
        if budget == TINY:   # 4 slots for 4 layers' top-4: every layer evicts the previous one's
            assert st["evictions"] > 0
        else:                # every expert stays once loaded
            assert st["hits"] > 0 and st["evictions"] == 0
    finally:
        m.close()


@needs_c2s
def test_c2s_cached_reference_bits(hip):
    """Sigmoid routing with selection bias and routed scale, Q4_K experts."""
    from tierlm_amd.model import Model
    m = Model(C2S, max_ctx=256, expert_cache=TINY)
    try:
        gen = greedy_tokens("c2s_greedy.txt")
        teacher_forced(m, "c2s_oracle.jsonl", prompt_tokens(2048) + gen[:63])
        m.reset()
        assert m.generate(prompt_tokens(2048), 64) == gen
    finally:
        m.close()


@needs_c3s
def test_c3s_cached_reference_bits(hip):
    """Qwen3-30B-A3B attention geometry, 16 experts top-8 through 8 slots,
    over the fixture's 2047 positions."""
    from tierlm_amd.model import Model
    m = Model(C3S, max_ctx=2048, expert_cache=TINY, lookahead_k=12, interest=0.5)
    try:
        assert m.store_stats()["slots"] == 8
        gen = greedy_tokens("c3s_greedy.txt")
        prompt = prompt_tokens(2048, 1920)
        teacher_forced(m, "c3s_oracle.jsonl", prompt + gen[:127])
        m.reset()
        assert m.generate(prompt, 128) == gen
    finally:
        m.close()


@needs_c5s
def test_c5s_cached_reference_bits(hip):
    """16 query heads per key head, 16 Q4_K experts top-8 through 8 slots,
    over the fixture's 1163 positions."""
    from tierlm_amd.model import Model
    m = Model(C5S, max_ctx=1200, expert_cache=TINY)
    try:
        assert m.store_stats()["slots"] == 8
        gen = greedy_tokens("c5s_greedy.txt")
        prompt = prompt_tokens(2048, 1100)
        teacher_forced(m, "c5s_oracle.jsonl", prompt + gen[:63])
        m.reset()
        assert m.generate(prompt, 64) == gen
        assert m.store_stats()["evictions"] > 0
    finally:
        m.close()


def test_synth_qwen3_235b_a22b_cached_equals_resident(hip):
    """Two layers of the full Qwen3-235B-A22B geometry (hidden 4096, 64 / 4
    heads x 128, 128 Q4_K experts top-8 of 1536, vocabulary 151936), the
    experts resident and behind a cache of top_k slots of 10.6 MB: every
    step's logits and routing bit for bit."""
    from tierlm_amd.model import QWEN3_235B_A22B, Model, bench_prompt
    g = dict(QWEN3_235B_A22B, n_layers=2)
    a = Model.synth(g, expert_dt=12, seed=5, max_ctx=48)
    b = Model.synth(g, expert_dt=12, seed=5, max_ctx=48, expert_cache=TINY)
    try:
        assert b.store_stats()["slots"] == 8
        for pos, t in enumerate(bench_prompt(16, g["vocab"], seed=9)):
            la, na = a.step(t)
            lb, nb = b.step(t)
            assert na == nb and np.array_equal(la.view(np.uint32), lb.view(np.uint32)), pos
            ia, wa = a.routes()
            ib, wb = b.routes()
            assert np.array_equal(ia, ib) and np.array_equal(wa.view(np.uint32), wb.view(np.uint32)), pos
        assert b.store_stats()["evictions"] > 0
    finally:
        a.close()
        b.close()


SMALL = dict(n_layers=3, d_model=512, n_heads=8, n_kv_heads=2, head_dim=64, vocab=4096, n_experts=32, top_k=4,
             d_expert=256, n_shared=0, d_shared=0, max_ctx=4096, router=0, rope_theta=1e6, norm_eps=1e-6,
             routed_scale=1.0)


@pytest.mark.parametrize("edt,shared,router", [(14, 0, 0), (12, 1, 0), (13, 0, 2), (8, 1, 2)])
def test_synth_cached_equals_resident(hip, edt, shared, router):
    """The same seed with the experts resident and in host memory behind a
    cache of top_k slots: every step's logits and routing bit for bit."""
    from tierlm_amd.model import Model, bench_prompt
    g = dict(SMALL, n_shared=shared, d_shared=256 * shared, router=router)
    a = Model.synth(g, expert_dt=edt, seed=5, max_ctx=64)
    b = Model.synth(g, expert_dt=edt, seed=5, max_ctx=64, expert_cache=TINY)
    try:
        for pos, t in enumerate(bench_prompt(20, g["vocab"])):
            la, na = a.step(t)
            lb, nb = b.step(t)
            assert na == nb and np.array_equal(la.view(np.uint32), lb.view(np.uint32)), pos
            ia, wa = a.routes()
            ib, wb = b.routes()
            assert np.array_equal(ia, ib) and np.array_equal(wa.view(np.uint32), wb.view(np.uint32)), pos
        a.reset()
        b.reset()
        p = bench_prompt(8, g["vocab"])
        assert a.generate(p, 12) == b.generate(p, 12)
        assert b.store_stats()["evictions"] > 0
    finally:
        a.close()
        b.close()


STORE_COUNTERS = ("hits", "misses", "prefetch_issued", "prefetch_used", "prefetch_dropped", "evictions", "slots",
                  "pinned")


@pytest.mark.parametrize("slots,gamma,prefetch", [(4, 0.0, True), (12, 0.8, True), (40, 0.8, True), (12, 0.0, False)])
def test_device_resolved_slots_equal_host_resolved(hip, slots, gamma, prefetch):
    """The slots resolved on the device (the host replaying acquire, hints
    and release behind it) and resolved by the host between each layer's
    routing and its block: the same logits and routing at every step, over
    caches of top_k slots (every step evicts), twelve and forty slots, with
    and without the lookahead.  Without it every load a step starts has
    landed before the next layer acquires (its block waited for it), so the
    store's decisions, and its counters, are the same step by step; with it
    a victim choice may see a lookahead load still in flight (such a slot is
    not a victim) on either path, so only the acquisitions are compared."""
    from tierlm_amd.model import Model, bench_prompt
    g = dict(SMALL, router=2 if gamma else 0, n_layers=4)
    slot = 3 * 256 * 512 // 256 * 210
    kw = dict(expert_dt=14, seed=9, max_ctx=96, expert_pool=6 if gamma else 0, heat_gamma=gamma,
              expert_cache=slot * slots, prefetch=prefetch, lookahead_k=8 if prefetch else 0,
              interest=0.7 if prefetch else 0.0, prefill_chunk=-1)
    a = Model.synth(g, host_routes=True, **kw)
    b = Model.synth(g, **kw)
    try:
        for pos, t in enumerate(bench_prompt(40, g["vocab"], seed=11)):
            la, na = a.step(t)
            lb, nb = b.step(t)
            assert na == nb and np.array_equal(la.view(np.uint32), lb.view(np.uint32)), pos
            ia, wa = a.routes()
            ib, wb = b.routes()
            assert np.array_equal(ia, ib) and np.array_equal(wa.view(np.uint32), wb.view(np.uint32)), pos
            sa, sb = a.store_stats(), b.store_stats()
            if prefetch:
                assert sa["hits"] + sa["misses"] == sb["hits"] + sb["misses"] == (pos + 1) * 4 * 4, pos
            else:
                assert {c: sa[c] for c in STORE_COUNTERS} == {c: sb[c] for c in STORE_COUNTERS}, pos
        st = b.store_stats()
        assert st["misses"] > 0 and st["in_use"] == 0
        if slots == 4:
            assert st["evictions"] > 0
        a.reset()
        b.reset()
        p = bench_prompt(8, g["vocab"])
        assert a.generate(p, 16) == b.generate(p, 16)
    finally:
        a.close()
        b.close()


def test_synth_cached_heat_lookahead(hip):
    """Sigmoid routing with a Zipf-like selection bias, a pool of 6 distinct
    payloads, the lookahead with interest-weighted breadth: a cache of half
    the experts serves most selections; hints are issued and used.  The
    prompt runs token by token (as the reference's runtime feeds it), so
    every position acquires top_k experts per layer and hints the next."""
    from tierlm_amd.model import Model, bench_prompt
    g = dict(SMALL, router=2, n_layers=4)
    slot = 3 * 256 * 512 // 256 * 210   # three Q6_K matrices of 256 x 512 (no padding at 256-byte alignment)
    m = Model.synth(g, expert_dt=14, seed=9, max_ctx=96, expert_pool=6, heat_gamma=0.8,
                    expert_cache=slot * 64, lookahead_k=8, interest=0.7, prefill_chunk=-1)
    try:
        assert m.store_stats()["slots"] == 64 and not m.prefill_batched()
        p = bench_prompt(16, g["vocab"])
        out = m.generate(p, 48)
        assert len(out) == 48
        lg, _ = m.step(out[-1])
        assert np.isfinite(lg).all()
        st = m.store_stats()
        total = st["hits"] + st["misses"]
        assert total == (16 + 48) * 4 * 4
        assert st["hits"] > st["misses"]
        assert st["prefetch_issued"] > 0 and st["prefetch_used"] > 0
    finally:
        m.close()


@pytest.mark.parametrize("edt,shared,budget,chunk", [(13, 0, TINY, 0), (14, 1, TINY, 24), (12, 0, ALL, 0),
                                                     (14, 0, 12 * 3 * 256 * 512 // 256 * 210, 32)])
def test_cached_prompt_batched_matches_resident(hip, edt, shared, budget, chunk):
    """The prompt of a model with its experts behind the slot cache runs
    batched (the chunk's experts acquired in passes of the unpinned slots:
    top_k slots, twelve, or every expert): the last position's logits and
    routing, and the following steps, are the resident batched model's and
    the cached model's own step-by-step prefill's, bit for bit."""
    from tierlm_amd.model import Model, bench_prompt
    g = dict(SMALL, n_shared=shared, d_shared=256 * shared)
    a = Model.synth(g, expert_dt=edt, seed=4, max_ctx=128)
    b = Model.synth(g, expert_dt=edt, seed=4, max_ctx=128, expert_cache=budget, prefill_chunk=chunk)
    c = Model.synth(g, expert_dt=edt, seed=4, max_ctx=128, expert_cache=budget, prefill_chunk=-1)
    try:
        assert a.prefill_batched() and b.prefill_batched() and not c.prefill_batched()
        p = bench_prompt(70, g["vocab"], seed=3)
        la, lb, lc = a.prefill(p), b.prefill(p), c.prefill(p)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
        assert np.array_equal(lc.view(np.uint32), lb.view(np.uint32))
        ia, wa = a.routes()
        ib, wb = b.routes()
        assert np.array_equal(ia, ib) and np.array_equal(wa.view(np.uint32), wb.view(np.uint32))
        assert a.kv_len() == b.kv_len() == 70
        tok = int(np.argmax(la))
        for s in range(4):
            la, na = a.step(tok)
            lb, nb = b.step(tok)
            assert na == nb and np.array_equal(la.view(np.uint32), lb.view(np.uint32)), s
            tok = na
        st = b.store_stats()
        assert st["misses"] > 0
        if budget == TINY:
            assert st["evictions"] > 0
    finally:
        a.close()
        b.close()
        c.close()


@needs_c3s
def test_c3s_cached_batched_prefill_reference_bits(hip):
    """Qwen3-30B-A3B attention geometry, 16 experts top-8 through 8 slots,
    the 1920-token prompt batched (two passes of 8 experts per layer and
    chunk): the last position's top-10 logits are the reference's bit for
    bit, then its 128 greedy tokens."""
    from tests.test_hip_model_prefill import assert_topk, oracle_row
    from tierlm_amd.model import Model
    m = Model(C3S, max_ctx=2048, expert_cache=TINY)
    try:
        assert m.prefill_batched() and m.store_stats()["slots"] == 8
        prompt = prompt_tokens(2048, 1920)
        lg = m.prefill(prompt)
        assert_topk(lg, oracle_row("c3s_oracle.jsonl", len(prompt) - 1))
        m.reset()
        assert m.generate(prompt, 128) == greedy_tokens("c3s_greedy.txt")
    finally:
        m.close()


@needs_c5s
def test_c5s_cached_batched_prefill_reference_bits(hip):
    """16 query heads per key head, Q4_K experts through 8 slots, the
    1100-token prompt batched: the reference's top-10 logits at its last
    position and its greedy tokens."""
    from tests.test_hip_model_prefill import assert_topk, oracle_row
    from tierlm_amd.model import Model
    m = Model(C5S, max_ctx=1200, expert_cache=TINY)
    try:
        assert m.prefill_batched()
        prompt = prompt_tokens(2048, 1100)
        lg = m.prefill(prompt)
        assert_topk(lg, oracle_row("c5s_oracle.jsonl", len(prompt) - 1))
        m.reset()
        assert m.generate(prompt, 64) == greedy_tokens("c5s_greedy.txt")
    finally:
        m.close()
