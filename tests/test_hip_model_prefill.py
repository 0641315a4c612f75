"""Batched prefill (tlm_hip_model_prefill, tlm_hip_model_opts.prefill_chunk):
tlm_model_prefill steps each prompt token in turn (src/lib/tlm_model.c:
1105-1113); the batched path runs each layer once per chunk of tokens (int8
MFMA token matmuls for q / k / v / o, causal attention over the cache, the
batched MoE block) and must leave every token's values the step's bits:

* on the reference's compiled stores C3S (Qwen3-30B-A3B attention geometry,
  qk-norm, Q6_K experts top-8) and C2S (no qk-norm, YaRN, sigmoid routing,
  Q4_K experts): the last prompt position's top-10 logits are the
  reference's (`tierlm oracle`), bit for bit, and the free-running greedy
  tokens after the batched prompt are the reference's;
* against the model's own step-by-step prefill (prefill_chunk -1): the
  logits bit for bit, then the following steps' logits and routing (so every
  cached key and value matched), for ragged chunks (not multiples of 4 or of
  the chunk), prompts in two calls (a chunk starting past position 0), head
  widths 32 / 64 / 96 / 128, 1 / 3 / 4 / 8 query heads per key head, each
  expert dtype, both routers, Q8_0 and K-quant dense matrices;
* C1 (a shared expert) batched against the reference's logits and tokens;
* a model the batched path does not take (head width 160) still prefills,
  one step per token, with the same bits."""
import json
import os

import numpy as np
import pytest

from tests.test_hip_model import C1, C2S, C3S, C5S, GOLD, greedy_tokens, needs_c1, needs_c2s, needs_c3s, needs_c5s, \
    prompt_tokens

pytestmark = pytest.mark.gpu


def oracle_row(name, pos):
    with open(os.path.join(GOLD, name)) as f:
        for i, line in enumerate(f):
            if i == pos:
                return json.loads(line)["topk"]
    raise AssertionError(f"{name} has no row {pos}")


def assert_topk(lg, want):
    got = np.argsort(-lg, kind="stable")[:10]
    assert [int(i) for i in got] == [w[0] for w in want]
    for wid, wv in want:
        assert lg[wid] == np.float32(wv), (wid, lg[wid], wv)


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@needs_c3s
@pytest.mark.parametrize("chunk", [0, 200])
def test_c3s_batched_prefill_reference_bits(hip, chunk):
    """1920-token prompt in chunks of the automatic size (at most 1024
    tokens, equal lengths: two chunks of 960) and of 200 (ragged: 9 full
    chunks and one of 120): the last position's top-10 logits are the
    reference's, then its 128 greedy tokens."""
    from tierlm_amd.model import Model
    m = Model(C3S, max_ctx=2048, prefill_chunk=chunk)
    try:
        assert m.prefill_batched()
        prompt = prompt_tokens(2048, 1920)
        lg = m.prefill(prompt)
        assert_topk(lg, oracle_row("c3s_oracle.jsonl", len(prompt) - 1))
        m.reset()
        assert m.generate(prompt, 128) == greedy_tokens("c3s_greedy.txt")
    finally:
        m.close()


@needs_c5s
def test_c5s_batched_prefill_reference_bits(hip):
    """16 query heads per key head: the 1100-token prompt batched (chunks of
    at most 1024, equal lengths: 552 + 548) gives the reference's top-10
    logits at its last position bit for bit, then its 64 greedy tokens."""
    from tierlm_amd.model import Model
    m = Model(C5S, max_ctx=1200)
    try:
        assert m.prefill_batched()
        prompt = prompt_tokens(2048, 1100)
        lg = m.prefill(prompt)
        assert_topk(lg, oracle_row("c5s_oracle.jsonl", len(prompt) - 1))
        m.reset()
        assert m.generate(prompt, 64) == greedy_tokens("c5s_greedy.txt")
    finally:
        m.close()


@needs_c2s
def test_c2s_batched_prefill_reference_bits(hip):
    from tierlm_amd.model import Model
    m = Model(C2S, max_ctx=256, prefill_chunk=12)
    try:
        assert m.prefill_batched()
        prompt = prompt_tokens(2048)
        lg = m.prefill(prompt)
        assert_topk(lg, oracle_row("c2s_oracle.jsonl", len(prompt) - 1))
        m.reset()
        assert m.generate(prompt, 64) == greedy_tokens("c2s_greedy.txt")
    finally:
        m.close()


def compare_models(g, edt, ddt, qk, chunk, parts, n_after=6, max_ctx=320, batched=True):
    """Batched (chunk) against step-by-step prefill of the same prompt split
    into parts; then n_after steps on both."""
    from tierlm_amd.model import Model, bench_prompt
    a = Model.synth(g, expert_dt=edt, dense_dt=ddt, qk_norm=qk, seed=3, max_ctx=max_ctx, prefill_chunk=chunk)
    b = Model.synth(g, expert_dt=edt, dense_dt=ddt, qk_norm=qk, seed=3, max_ctx=max_ctx, prefill_chunk=-1)
    try:
        assert a.prefill_batched() == batched and not b.prefill_batched()
        p = bench_prompt(sum(parts), g["vocab"], seed=7)
        i = 0
        for n in parts:
            la = a.prefill(p[i:i + n])
            lb = b.prefill(p[i:i + n])
            i += n
            assert bits_equal(la, lb), f"prefill logits after {i} tokens"
        ia, wa = a.routes()
        ib, wb = b.routes()
        assert np.array_equal(ia, ib) and bits_equal(wa, wb)
        tok = int(np.argmax(la))
        for s in range(n_after):
            la, na = a.step(tok)
            lb, nb = b.step(tok)
            assert na == nb and bits_equal(la, lb), f"step {s} after the prompt"
            ia, wa = a.routes()
            ib, wb = b.routes()
            assert np.array_equal(ia, ib) and bits_equal(wa, wb), f"routes at step {s}"
            tok = na
        assert a.kv_len() == b.kv_len() == sum(parts) + n_after
    finally:
        a.close()
        b.close()


BASE = dict(n_layers=2, d_model=512, n_heads=8, n_kv_heads=2, head_dim=64, vocab=4096, n_experts=16, top_k=4,
            d_expert=256, n_shared=0, d_shared=0, max_ctx=4096, router=0, rope_theta=1e6, norm_eps=1e-6,
            routed_scale=1.0)


@pytest.mark.parametrize("geo,edt,ddt,qk,chunk,parts", [
    (dict(), 14, 8, True, 0, [77]),                                    # one ragged chunk
    (dict(), 12, 8, False, 16, [45, 30]),                              # ragged chunks, two calls
    (dict(router=2, routed_scale=2.5), 13, 8, True, 8, [3, 61]),       # sigmoid routing
    (dict(head_dim=128, n_heads=16, n_kv_heads=2), 14, 14, True, 32, [100]),   # 8 heads per key head, Q6_K dense
    (dict(head_dim=96, n_heads=8, n_kv_heads=2), 12, 12, True, 24, [50]),      # width 96, Q4_K dense
    (dict(head_dim=128, n_heads=6, n_kv_heads=2, d_model=768), 14, 8, True, 20, [41]),   # 3 per key head
    (dict(head_dim=32, n_heads=8, n_kv_heads=8), 13, 13, False, 0, [300]),     # width 32, 1 per key head, Q5_K dense
])
def test_synth_batched_equals_steps(hip, geo, edt, ddt, qk, chunk, parts):
    compare_models(dict(BASE, **geo), edt, ddt, qk, chunk, parts)


def test_synth_long_context_chunks(hip):
    """A 1100-token prompt at capacity 1200: positions past 1024 in a
    score chunk of their own, chunks of 256 (the last ragged)."""
    compare_models(BASE, 14, 8, True, 256, [1100], n_after=3, max_ctx=1200)


def test_shared_expert_batched(hip):
    """A shared expert (the synthetic model's is of the experts' dtype, Q6_K):
    batched, the same bits as the steps."""
    compare_models(dict(BASE, n_shared=1, d_shared=256), 14, 8, True, 16, [45], n_after=3)


def test_unsupported_width_steps(hip):
    """Head width 160: the batched path declines, the prompt still runs (one
    step per token) with the same bits."""
    compare_models(dict(BASE, head_dim=160, n_heads=8, n_kv_heads=2, d_model=512), 14, 8, True, 0, [20],
                   n_after=2, batched=False)


@needs_c1
def test_c1_batched_prefill_reference_bits(hip):
    """C1 (a shared expert, head width 64): the 64-token prompt batched, the
    last position's top-10 logits the reference's and its 64 greedy tokens."""
    from tierlm_amd.model import Model
    m = Model(C1, max_ctx=256, prefill_chunk=24)
    try:
        assert m.prefill_batched()
        lg = m.prefill(prompt_tokens())
        assert_topk(lg, oracle_row("c1_oracle.jsonl", 63))
        m.reset()
        assert m.generate(prompt_tokens(), 64) == greedy_tokens()
    finally:
        m.close()


@pytest.mark.parametrize("parts,max_ctx,n_after", [([1, 2, 1, 3], 320, 4), ([63, 1], 64, 0), ([29, 35], 64, 0)])
def test_synth_tiny_and_full_prompts(hip, parts, max_ctx, n_after):
    """Prompts of 1-3 tokens (a chunk smaller than one group's 4 tokens), and
    prompts that fill the context capacity exactly."""
    compare_models(BASE, 14, 8, True, 0, parts, n_after=n_after, max_ctx=max_ctx)


def test_prefill_errors(hip):
    """Past the capacity, an empty prompt and a token outside the vocabulary
    are refused, and the context is left as it was."""
    from tierlm_amd._lib import HipError
    from tierlm_amd.model import Model, bench_prompt
    m = Model.synth(BASE, expert_dt=14, seed=3, max_ctx=32)
    try:
        m.prefill(bench_prompt(20, BASE["vocab"]))
        with pytest.raises(HipError):
            m.prefill(bench_prompt(13, BASE["vocab"]))
        with pytest.raises(HipError):
            m.prefill([])
        with pytest.raises(HipError):
            m.prefill([BASE["vocab"]])
        assert m.kv_len() == 20
        lg = m.prefill(bench_prompt(12, BASE["vocab"], seed=9))
        assert np.isfinite(lg).all() and m.kv_len() == 32
    finally:
        m.close()


def test_synth_prompt_past_2048(hip):
    """A 2400-token prompt at capacity 2600: the softmax's second round of 2048
    positions per thread set, P.V chunks past position 2048."""
    compare_models(BASE, 12, 8, True, 512, [2400], n_after=3, max_ctx=2600)


@needs_c3s
@pytest.mark.parametrize("chunk", [0, -1])
def test_c3s_past_2048_reference_tokens(hip, chunk):
    """Past 2048 positions (tests/golden/make_c3s_long_golden.sh: a 2300-token
    prompt, the reference's 48 greedy tokens), batched and stepped."""
    from tierlm_amd.model import Model
    m = Model(C3S, max_ctx=4096, prefill_chunk=chunk)
    try:
        assert m.prefill_batched() == (chunk == 0)
        assert m.generate(prompt_tokens(2048, 2300), 48) == greedy_tokens("c3s_long_greedy.txt")
    finally:
        m.close()


def test_synth_prompt_past_4096(hip):
    """A 4400-token prompt at capacity 4600: the stepped decode's probabilities
    in two LDS segments (past 4096 positions) and the batched softmax's third
    round, bit for bit."""
    compare_models(dict(BASE, max_ctx=8192), 13, 8, True, 512, [4400], n_after=3, max_ctx=4600)


def test_synth_full_1024_chunk(hip):
    """An explicit chunk of 1024 on a 1025-token prompt: the prompt splits
    into two chunks of near-equal length (neither a multiple of the other),
    each token the step's bits."""
    compare_models(BASE, 14, 8, True, 1024, [1025], n_after=3, max_ctx=1040)
