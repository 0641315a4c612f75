"""Device activation quantisers vs the oracle, byte for byte
(the reference's rule: src/lib/tlm_quant.c:458-506; KATs tests/test_quant.c:434-536 there)."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _dev_act(hq, kind, x, dev):
    xt = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dev)
    out = hq.quantize_act(kind, xt)
    torch.cuda.synchronize()
    return out.cpu().numpy()[:oracle.qact_bytes(kind, x.size)]


def _cases(rng):
    yield "bell", rng.standard_normal(2048).astype(np.float32)
    yield "zeros", np.zeros(512, np.float32)
    yield "pm1", np.where(rng.integers(0, 2, 1024) > 0, 1.0, -1.0).astype(np.float32)
    spike = (0.001 * rng.standard_normal(768)).astype(np.float32)
    spike[::77] = 1000.0
    yield "spike", spike
    nan = rng.standard_normal(512).astype(np.float32)
    nan[10] = np.nan
    nan[300] = np.inf
    yield "nan_inf", nan
    ninf = rng.standard_normal(256).astype(np.float32)
    ninf[3] = -np.inf
    yield "neg_inf", ninf
    sub = (np.arange(512, dtype=np.float32) - 256) * np.float32(2.0 ** -140)
    yield "subnormal", sub
    tiny = (rng.standard_normal(256) * 2.0 ** -110).astype(np.float32)
    yield "tiny", tiny
    for n in (1, 7, 31, 33, 100, 255, 257, 1003):
        yield f"partial{n}", rng.standard_normal(n).astype(np.float32) * 3
    ties = (np.arange(-300, 300, dtype=np.float32) * 0.5)   # exact .5 ties after scaling
    yield "ties", ties
    big = (rng.standard_normal(4096) * 3e38).astype(np.float32)
    yield "huge", np.clip(big, -3.3e38, 3.3e38)


@pytest.mark.parametrize("kind", [oracle.Q8_K, oracle.Q8_0])
def test_quantize_act_bytes(hip, dev, kind):
    rng = np.random.default_rng(1234)
    for name, x in _cases(rng):
        want = oracle.quantize_act(kind, x)[:oracle.qact_bytes(kind, x.size)]
        got = _dev_act(hip, kind, x, dev)
        if not np.array_equal(got, want):
            bad = np.nonzero(got != want)[0]
            pytest.fail(f"kind {kind} case {name}: {bad.size} bytes differ, first at {bad[:8]}")


def test_quantize_act_random_sweep(hip, dev):
    rng = np.random.default_rng(99)
    for rep in range(40):
        n = int(rng.integers(1, 6000))
        x = (rng.standard_normal(n) * 10.0 ** rng.uniform(-6, 6)).astype(np.float32)
        for kind in (oracle.Q8_K, oracle.Q8_0):
            want = oracle.quantize_act(kind, x)[:oracle.qact_bytes(kind, n)]
            assert np.array_equal(_dev_act(hip, kind, x, dev), want), (rep, n, kind)


def test_quantize_act_f32_copy(hip, dev):
    x = np.random.default_rng(3).standard_normal(77).astype(np.float32)
    got = _dev_act(hip, oracle.F32, x, dev)
    assert np.array_equal(got.view(np.float32), x)


def test_quantize_act_rejects_unknown_kind(hip, dev):
    from tierlm_amd import HipError
    x = torch.zeros(64, device=dev)
    with pytest.raises(HipError):
        hip.quantize_act(oracle.Q6_K, x)
