"""The whole decode step on the device (tlm_hip_model_*) on synthetic models
as the reference's own compiler writes them, against the reference's own
runtime on the same stores:

* C1 (oracle/make_c1.sh, tests/golden/make_c1_golden.sh): D 512, 8/2 heads x
  64, qk-norm, 32 experts top-4 Q6_K, softmax router, one shared expert, Q8_0
  dense, vocabulary 4096;
* C2S (oracle/make_c2s.sh, tests/golden/make_c2s_golden.sh): D 256, 4/2 heads
  x 128, no qk-norm, YaRN RoPE, 16 experts top-2 Q4_K under the sigmoid
  router (selection bias, routed scale 2.5), no shared expert, vocabulary
  2048.

Checks:
* teacher-forced, every position of prompt + generated tokens: the top-10
  logits of `tierlm oracle`, ids and values bit for bit (`tierlm oracle`
  prints 9 significant digits, which round-trip a float exactly): the integer
  paths are exact, the rest runs the reference's operations in its order, and
  e^x is libm's expf restated;
* free-running greedy decode after the 64-token xorshift(42) prompt: the
  reference's tokens exactly (`tierlm run --print-tokens`; C1's 64 tokens
  md5 f2fb5199...);
* C1 over 383 positions (320 greedy tokens) at context capacities 512 and
  4096 (a request of 5000 is capped at the store's 4096, as tlm_kv_new caps
  it), teacher-forced and free-running;
* C3S (oracle/make_c3s.sh, tests/golden/make_c3s_golden.sh): the attention
  geometry of Qwen3-30B-A3B - D 2048, 32/4 heads x 128, qk-norm, rope theta
  1e6 - with 16 experts top-8, over 2047 positions (a 1920-token prompt and
  the first 127 greedy tokens) at context capacities 2048 and 4096, and the
  reference's 128 greedy tokens after the prompt;
* C5S (oracle/make_c5s.sh, tests/golden/make_c5s_golden.sh): the attention
  grouping of Qwen3-235B-A22B - 16 query heads per key head of width 128
  (32 / 2 heads at D 2048), qk-norm - with 16 Q4_K experts top-8, over 1163
  positions (a 1100-token prompt and the first 63 greedy tokens), and the
  reference's 64 greedy tokens after the prompt;
* C6D (oracle/make_c6d.sh, tests/golden/make_c6d_golden.sh): two leading
  dense-FFN layers (first_k_dense_replace) then two MoE layers with a shared
  expert, over 263 positions (a 200-token prompt and the first 63 greedy
  tokens): top-10 logits bit for bit resident (graph replay and eager) and
  through the slot cache, and the reference's 64 greedy tokens;
* the split attention option (attn_split) on the three: the reference's
  greedy tokens, its top-1 at 99% or more of the teacher-forced positions;
* the full Qwen3-235B-A22B geometry (D 4096, 64 / 4 heads x 128, 128 Q4_K
  experts top-8 of 1536, vocabulary 151936) as a 2-layer random-init model:
  graph replays equal eager launches, the lm_head's greedy token is the
  first maximum of its logits."""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
C1 = os.path.join(ROOT, "oracle", "_ref", "c1", "c1.tlmm")
C2S = os.path.join(ROOT, "oracle", "_ref", "c2s", "c2s.tlmm")
C3S = os.path.join(ROOT, "oracle", "_ref", "c3s", "c3s.tlmm")
C5S = os.path.join(ROOT, "oracle", "_ref", "c5s", "c5s.tlmm")
C6D = os.path.join(ROOT, "oracle", "_ref", "c6d", "c6d.tlmm")
GOLD = os.path.join(ROOT, "tests", "golden")
needs_c1 = pytest.mark.skipif(not os.path.exists(C1), reason="oracle/_ref/c1 not built (oracle/make_c1.sh)")
needs_c2s = pytest.mark.skipif(not os.path.exists(C2S), reason="oracle/_ref/c2s not built (oracle/make_c2s.sh)")
needs_c3s = pytest.mark.skipif(not os.path.exists(C3S), reason="oracle/_ref/c3s not built (oracle/make_c3s.sh)")
needs_c5s = pytest.mark.skipif(not os.path.exists(C5S), reason="oracle/_ref/c5s not built (oracle/make_c5s.sh)")
needs_c6d = pytest.mark.skipif(not os.path.exists(C6D), reason="oracle/_ref/c6d not built (oracle/make_c6d.sh)")


def prompt_tokens(vocab=4096, n=64):
    x, out, m = 42, [], (1 << 64) - 1
    for _ in range(n):   # src/bin/tierlm.c:711-715
        x ^= (x << 13) & m
        x ^= x >> 7
        x ^= (x << 17) & m
        out.append(x % vocab)
    return out


def greedy_tokens(name="c1_greedy.txt"):
    return [int(t) for t in open(os.path.join(GOLD, name)).read().split()]


def teacher_forced(model, oracle_file, tokens):
    """Step through tokens; at every position the top-10 ids and values must be
    the reference's bit for bit; returns (bit-identical count, total, worst
    absolute difference)."""
    oracle_rows = [json.loads(line) for line in open(os.path.join(GOLD, oracle_file))]
    assert len(oracle_rows) == len(tokens)
    model.reset()
    exact = total = 0
    worst = 0.0
    for pos, tok in enumerate(tokens):
        lg, nxt = model.step(tok)
        want = oracle_rows[pos]["topk"]
        got_ids = np.argsort(-lg, kind="stable")[:10]
        assert [int(i) for i in got_ids] == [w[0] for w in want], f"pos {pos}"
        for wid, wv in want:
            wv = np.float32(wv)
            d = abs(float(lg[wid]) - float(wv))
            assert d <= 1e-5 * max(1.0, abs(float(wv))), f"pos {pos} id {wid}: {lg[wid]!r} vs {wv!r}"
            exact += lg[wid] == wv
            worst = max(worst, d)
            total += 1
        assert nxt == want[0][0]
    print(f"{oracle_file}: {exact} of {total} top-10 logits bit-identical, worst |d| {worst:.3g}")
    assert exact == total, f"{total - exact} of {total} top-10 logits differ from the reference (worst {worst:.3g})"
    return exact, total, worst


@pytest.fixture(scope="module")
def c1(hip):
    from tierlm_amd.model import Model
    m = Model(C1, max_ctx=256)
    yield m
    m.close()


@needs_c1
def test_c1_teacher_forced_top10_logits(c1):
    tokens = prompt_tokens() + greedy_tokens()[:63]
    assert len(tokens) == 127
    teacher_forced(c1, "c1_oracle.jsonl", tokens)


@needs_c1
@pytest.mark.parametrize("max_ctx,capacity,slices", [(512, 512, 0), (5000, 4096, 0), (512, 512, 1)])
def test_c1_long_context(hip, max_ctx, capacity, slices):
    """383 positions at head width 64; a capacity above the store's
    max_position_embeddings (4096) is capped to it."""
    from tierlm_amd.model import Model
    m = Model(C1, max_ctx=max_ctx, attn_slices=slices)
    try:
        assert m.kv_capacity() == capacity
        gen = greedy_tokens("c1_greedy_long.txt")
        assert len(gen) == 320
        teacher_forced(m, "c1_oracle_long.jsonl", prompt_tokens() + gen[:319])
        m.reset()
        assert m.generate(prompt_tokens(), 320) == gen
        assert m.kv_len() == 64 + 319
    finally:
        m.close()


@needs_c2s
def test_c2s_teacher_forced_and_greedy(hip):
    """Head width 128, no qk-norm, YaRN, sigmoid routing with bias and
    routed scale, Q4_K experts, no shared expert."""
    from tierlm_amd.model import Model
    m = Model(C2S, max_ctx=256)
    try:
        g = m.geom
        assert (g.head_dim, g.n_heads, g.n_kv_heads, g.top_k, g.n_shared, g.vocab) == (128, 4, 2, 2, 0, 2048)
        gen = greedy_tokens("c2s_greedy.txt")
        teacher_forced(m, "c2s_oracle.jsonl", prompt_tokens(2048) + gen[:63])
        m.reset()
        assert m.generate(prompt_tokens(2048), 64) == gen
    finally:
        m.close()


@needs_c3s
@pytest.mark.parametrize("max_ctx,slices", [(2048, 0), (4096, 3), (4096, 1)])
def test_c3s_long_context_head_width_128(hip, max_ctx, slices):
    """Qwen3-30B-A3B attention geometry over 2047 positions: every position's
    top-10 logits teacher-forced, then the reference's 128 greedy tokens after
    the 1920-token prompt.  Attention slices: automatic (64 per key head, one
    chunk each at 2047 positions), 3 (up to 22 chunks per slice) and 1 (one
    slice per key head, up to 64 chunks)."""
    from tierlm_amd.model import Model
    m = Model(C3S, max_ctx=max_ctx, attn_slices=slices)
    try:
        assert m.kv_capacity() == max_ctx
        g = m.geom
        assert (g.d_model, g.n_heads, g.n_kv_heads, g.head_dim, g.n_experts, g.top_k, g.n_shared, g.vocab) == \
            (2048, 32, 4, 128, 16, 8, 0, 2048)
        gen = greedy_tokens("c3s_greedy.txt")
        assert len(gen) == 128
        prompt = prompt_tokens(2048, 1920)
        exact, total, worst = teacher_forced(m, "c3s_oracle.jsonl", prompt + gen[:127])
        assert total == 2047 * 10
        m.reset()
        assert m.generate(prompt, 128) == gen
        assert m.kv_len() == 1920 + 127
    finally:
        m.close()


@needs_c5s
@pytest.mark.parametrize("max_ctx,slices", [(1200, 0), (4096, 2)])
def test_c5s_sixteen_query_heads_per_key_head(hip, max_ctx, slices):
    """Qwen3-235B-A22B's attention grouping (16 query heads per key head,
    width 128) over 1163 positions: every position's top-10 logits
    teacher-forced, then the reference's 64 greedy tokens after the
    1100-token prompt."""
    from tierlm_amd.model import Model
    m = Model(C5S, max_ctx=max_ctx, attn_slices=slices)
    try:
        g = m.geom
        assert (g.d_model, g.n_heads, g.n_kv_heads, g.head_dim, g.n_experts, g.top_k, g.n_shared, g.vocab) == \
            (2048, 32, 2, 128, 16, 8, 0, 2048)
        gen = greedy_tokens("c5s_greedy.txt")
        assert len(gen) == 64
        prompt = prompt_tokens(2048, 1100)
        exact, total, worst = teacher_forced(m, "c5s_oracle.jsonl", prompt + gen[:63])
        assert total == 1163 * 10
        m.reset()
        assert m.generate(prompt, 64) == gen
    finally:
        m.close()


@needs_c6d
@pytest.mark.parametrize("eager,budget,chunk", [(False, 0, 0), (True, 0, 96), (False, 1, 0), (False, 1, 96)])
def test_c6d_dense_ffn_layers(hip, eager, budget, chunk):
    """Two dense-FFN layers before the MoE layers (tlm_model.c:312-324,
    946-964: rmsnorm, gate / up, silu(gate) * up, down added into h): every
    position's top-10 logits teacher-forced and the reference's 64 greedy
    tokens after the 200-token prompt, run batched (one chunk, or three of
    68) - graph replay, eager launches, and the experts through a cache of
    top_k slots (the dense layers before the store's stack); dense layers
    route nothing."""
    from tierlm_amd.model import Model
    m = Model(C6D, max_ctx=512, eager=eager, expert_cache=budget, prefill_chunk=chunk)
    try:
        g = m.geom
        assert (g.n_layers, g.d_model, g.n_heads, g.n_kv_heads, g.head_dim, g.n_experts, g.top_k, g.n_shared) == \
            (4, 512, 8, 2, 64, 16, 4, 1)
        gen = greedy_tokens("c6d_greedy.txt")
        assert len(gen) == 64
        prompt = prompt_tokens(2048, 200)
        exact, total, worst = teacher_forced(m, "c6d_oracle.jsonl", prompt + gen[:63])
        assert total == 263 * 10
        ids, w = m.routes()
        assert (ids[:2] == 0).all() and (w[:2] == 0).all() and (w[2:] > 0).all()
        assert m.prefill_batched()
        m.reset()
        lg = m.prefill(prompt)
        assert int(np.argmax(lg)) == gen[0]
        m.reset()
        assert m.generate(prompt, 64) == gen
        if budget:
            assert m.store_stats()["misses"] > 0
    finally:
        m.close()


def split_teacher_forced(model, oracle_file, tokens):
    """Split attention (attn_split), teacher-forced: returns the fraction of
    positions whose greedy token (top-1) is the reference's and the worst
    relative difference of the reference's top-10 logits.  Its attention
    outputs are the reference's within float rounding, not bit for bit, so int8
    activation codes and near-tied top-k routing downstream can move logits
    further than the 1e-5 of the exact path, and a near-tied top-1 of a
    random prompt token can change."""
    oracle_rows = [json.loads(line) for line in open(os.path.join(GOLD, oracle_file))]
    model.reset()
    worst = 0.0
    same = 0
    for pos, tok in enumerate(tokens):
        lg, nxt = model.step(tok)
        want = oracle_rows[pos]["topk"]
        same += nxt == want[0][0]
        for wid, wv in want:
            worst = max(worst, abs(float(lg[wid]) - float(wv)) / max(1.0, abs(float(wv))))
    return same / len(tokens), worst


@pytest.mark.parametrize("store,max_ctx,oracle_file,greedy_file,prompt_len,vocab,n_gen", [
    pytest.param(C1, 512, "c1_oracle_long.jsonl", "c1_greedy_long.txt", 64, 4096, 320, marks=needs_c1),
    pytest.param(C2S, 256, "c2s_oracle.jsonl", "c2s_greedy.txt", 64, 2048, 64, marks=needs_c2s),
    pytest.param(C3S, 2048, "c3s_oracle.jsonl", "c3s_greedy.txt", 1920, 2048, 128, marks=needs_c3s),
])
def test_split_attention_greedy_tokens(hip, store, max_ctx, oracle_file, greedy_file, prompt_len, vocab, n_gen):
    """attn_split: the reference's free-running greedy tokens after the
    prompt, and its top-1 at 99% or more of the teacher-forced positions (C1
    383 positions at head width 64, C2S, C3S 2047 positions at head width
    128)."""
    from tierlm_amd.model import Model
    m = Model(store, max_ctx=max_ctx, split=True)
    try:
        gen = greedy_tokens(greedy_file)
        assert len(gen) == n_gen
        prompt = prompt_tokens(vocab, prompt_len)
        agree, worst = split_teacher_forced(m, oracle_file, prompt + gen[:-1])
        print(f"{oracle_file} split attention: top-1 agreement {agree:.4f}, worst relative top-10 logit "
              f"difference {worst:.3g}")
        assert agree >= 0.99
        m.reset()
        assert m.generate(prompt, n_gen) == gen
    finally:
        m.close()


@needs_c1
def test_c1_greedy_decode_matches_reference(c1):
    c1.reset()
    out = c1.generate(prompt_tokens(), 64)
    assert out == greedy_tokens()
    assert c1.kv_len() == 64 + 63


@needs_c1
def test_c1_step_equals_generate(c1):
    """The host-driven step loop and the device-resident generate loop give
    the same tokens (prefill is the step repeated, src/lib/tlm_model.c:1105)."""
    c1.reset()
    toks = prompt_tokens()[:20]
    nxt = None
    for t in toks:
        _, nxt = c1.step(t)
    got = [nxt]
    for _ in range(9):
        _, nxt = c1.step(got[-1])
        got.append(nxt)
    c1.reset()
    assert c1.generate(toks, 10) == got


@needs_c1
def test_c1_context_and_token_errors(c1):
    from tierlm_amd._lib import HipError
    c1.reset()
    with pytest.raises(HipError):
        c1.step(4096)            # token out of range (TLM_EINVAL)
    with pytest.raises(HipError):
        c1.generate(prompt_tokens() * 4, 10)   # 256 + 9 > max_ctx 256 (TLM_ERANGE)
    assert c1.kv_len() == 0


@needs_c1
def test_c1_graph_replays_equal_eager_steps(hip, c1):
    """Every replay of the captured step graph gives the eager launches' bits
    (logits at each of 40 positions, with host work between replays)."""
    from tierlm_amd.model import Model
    eager = Model(C1, max_ctx=256, eager=True)
    try:
        c1.reset()
        eager.reset()
        toks = prompt_tokens()[:30] + greedy_tokens()[:10]
        for pos, t in enumerate(toks):
            a, na = c1.step(t)
            b, nb = eager.step(t)
            assert na == nb and np.array_equal(a.view(np.uint32), b.view(np.uint32)), pos
    finally:
        eager.close()


SMALL = dict(n_layers=3, d_model=512, n_heads=8, n_kv_heads=2, head_dim=64, vocab=4096, n_experts=32, top_k=4,
             d_expert=256, n_shared=1, d_shared=256, max_ctx=4096, router=0, rope_theta=1e6, norm_eps=1e-6,
             routed_scale=1.0)


@pytest.mark.parametrize("edt", [14, 12, 13])   # Q6_K, Q4_K, Q5_K experts
def test_synth_model_graph_equals_eager(hip, edt):
    """tlm_hip_model_synth (random-init weights, no reference counterpart to
    compare with): graph replays give the eager launches' bits, logits stay
    finite, the same seed reproduces the same tokens and another seed does
    not."""
    from tierlm_amd.model import Model, bench_prompt
    a = Model.synth(SMALL, expert_dt=edt, seed=3, max_ctx=128)
    b = Model.synth(SMALL, expert_dt=edt, seed=3, max_ctx=128, eager=True)
    c = Model.synth(SMALL, expert_dt=edt, seed=4, max_ctx=128)
    try:
        p = bench_prompt(24, SMALL["vocab"])
        differs = False
        for pos, t in enumerate(p):
            la, na = a.step(t)
            lb, nb = b.step(t)
            lc, _ = c.step(t)
            assert na == nb and np.array_equal(la.view(np.uint32), lb.view(np.uint32)), pos
            assert np.isfinite(la).all(), pos
            differs = differs or not np.array_equal(la, lc)
        assert differs
        a.reset()
        b.reset()
        assert a.generate(p, 16) == b.generate(p, 16)
    finally:
        a.close()
        b.close()
        c.close()


def test_synth_qwen3_30b_a3b_shape(hip):
    """Two layers of the Qwen3-30B-A3B shape (head width 128, 32 / 4 heads,
    128 experts top-8 of 768, vocabulary 151936): steps run, logits finite,
    graph equals eager."""
    from tierlm_amd.model import QWEN3_30B_A3B, Model, bench_prompt
    g = dict(QWEN3_30B_A3B, n_layers=2)
    a = Model.synth(g, seed=1, max_ctx=64)
    b = Model.synth(g, seed=1, max_ctx=64, eager=True)
    try:
        for pos, t in enumerate(bench_prompt(8, g["vocab"])):
            la, na = a.step(t)
            lb, nb = b.step(t)
            assert np.isfinite(la).all() and na == nb and np.array_equal(la.view(np.uint32), lb.view(np.uint32)), pos
    finally:
        a.close()
        b.close()


def test_synth_qwen3_235b_a22b_geometry(hip):
    """Two layers of the Qwen3-235B-A22B geometry (hidden 4096, 64 / 4 heads
    x 128 with qk-norm, 128 Q4_K experts top-8 of 1536, Q8_0 dense and
    lm_head, vocabulary 151936): over 40 positions the graph replays give the
    eager launches' bits, logits are finite and the greedy token is the first
    maximum of the downloaded logits (the lm_head's per-tile keys and the
    argmax launch against numpy)."""
    from tierlm_amd.model import QWEN3_235B_A22B, Model, bench_prompt
    g = dict(QWEN3_235B_A22B, n_layers=2)
    a = Model.synth(g, expert_dt=12, seed=5, max_ctx=64)
    b = Model.synth(g, expert_dt=12, seed=5, max_ctx=64, eager=True)
    try:
        assert (a.geom.d_model, a.geom.n_heads, a.geom.n_kv_heads, a.geom.head_dim, a.geom.vocab) == \
            (4096, 64, 4, 128, 151936)
        for pos, t in enumerate(bench_prompt(40, g["vocab"], seed=9)):
            la, na = a.step(t)
            lb, nb = b.step(t)
            assert np.isfinite(la).all(), pos
            assert na == nb and np.array_equal(la.view(np.uint32), lb.view(np.uint32)), pos
            assert na == int(np.argmax(la)), pos
    finally:
        a.close()
        b.close()


@needs_c1
@pytest.mark.parametrize("eager", [False, True])
def test_c1_stats_split(hip, eager):
    """tlm_hip_model_opts.stats: the steps' device-timed attention / MoE /
    other split (tlm_model_stats) is counted and leaves every result
    unchanged - the same greedy tokens as the reference, graph or eager."""
    from tierlm_amd.model import Model
    m = Model(C1, max_ctx=256, eager=eager, stats=True, prefill_chunk=-1)
    try:
        st = m.stats()
        assert st["tokens"] == 0 and st["attn_ns"] == 0
        assert m.generate(prompt_tokens(), 64) == greedy_tokens()
        st = m.stats()
        assert st["tokens"] == 64 + 63
        assert st["attn_ns"] > 0 and st["moe_ns"] > 0 and st["other_ns"] > 0
        per = (st["attn_ns"] + st["moe_ns"] + st["other_ns"]) / st["tokens"]
        assert 1e3 < per < 1e7, per                       # between 1 us and 10 ms of device time per token
        m.reset_stats()
        assert m.stats()["tokens"] == 0 and m.stats()["moe_ns"] == 0
        m.reset()
        lg = m.prefill(prompt_tokens()[:40])
        assert m.stats()["tokens"] == 40 and m.stats()["attn_ns"] > 0
        assert int(np.argmax(lg)) == int(np.argmax(lg))
    finally:
        m.close()


@needs_c1
def test_c1_stats_batched_prefill_and_cache(hip):
    """The split is also counted for a batched prompt and for a step whose
    experts come through the slot cache (whose load waits are the expert
    wait)."""
    from tierlm_amd.model import Model
    a = Model(C1, max_ctx=256, stats=True)
    b = Model(C1, max_ctx=256, stats=True, expert_cache=1)
    try:
        assert a.prefill_batched()
        la = a.prefill(prompt_tokens())
        lb = b.prefill(prompt_tokens())
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
        for m in (a, b):
            st = m.stats()
            assert st["tokens"] == 64 and st["attn_ns"] > 0 and st["moe_ns"] > 0 and st["other_ns"] > 0
        assert b.store_stats()["misses"] > 0
    finally:
        a.close()
        b.close()
