"""The whole decode step on the device (tlm_hip_model_*) on the 4-layer
synthetic model as the reference's own compiler writes it (oracle/make_c1.sh:
D 512, 8/2 heads x 64, 32 experts top-4 Q6_K, Q8_0 dense, f32 router, one
shared expert, vocabulary 4096), against the reference's own runtime on the
same store (tests/golden/make_c1_golden.sh):

* teacher-forced, every position of prompt + generated tokens: the top-10
  logits of `tierlm oracle` (ids identical, values within 1e-5 relative; most
  are bit-identical - the integer paths are exact and the rest runs in the
  reference's order);
* free-running greedy decode of 64 tokens after the 64-token xorshift(42)
  prompt: the reference's tokens exactly (`tierlm run --print-tokens`,
  md5 f2fb5199...)."""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
C1 = os.path.join(ROOT, "oracle", "_ref", "c1", "c1.tlmm")
GOLD = os.path.join(ROOT, "tests", "golden")
needs_c1 = pytest.mark.skipif(not os.path.exists(C1), reason="oracle/_ref/c1 not built (oracle/make_c1.sh)")


def prompt_tokens():
    x, out, m = 42, [], (1 << 64) - 1
    for _ in range(64):   # src/bin/tierlm.c:711-715
        x ^= (x << 13) & m
        x ^= x >> 7
        x ^= (x << 17) & m
        out.append(x % 4096)
    return out


def greedy_tokens():
    return [int(t) for t in open(os.path.join(GOLD, "c1_greedy.txt")).read().split()]


@pytest.fixture(scope="module")
def c1(hip):
    from tierlm_amd.model import Model
    m = Model(C1, max_ctx=256)
    yield m
    m.close()


@needs_c1
def test_c1_teacher_forced_top10_logits(c1):
    oracle_rows = [json.loads(line) for line in open(os.path.join(GOLD, "c1_oracle.jsonl"))]
    tokens = prompt_tokens() + greedy_tokens()[:63]
    assert len(oracle_rows) == len(tokens) == 127
    c1.reset()
    exact = worst = 0
    total = 0
    for pos, tok in enumerate(tokens):
        lg, nxt = c1.step(tok)
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
    assert exact >= total // 2, f"only {exact} of {total} top-10 logits bit-identical (worst {worst:.3g})"


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
