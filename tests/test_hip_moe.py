"""The device MoE block (tlm_hip_moe_layer) vs the oracle's MoE block
(src/lib/tlm_model.c:940-1055).

Tolerance (from the build's numerics contract): routing ids identical,
weights within an ulp; the updated residual within 1e-5 relative per element,
relative to |ref| + 1e-3 * max|ref|, plus what an ulp of routing weight
contributes through the combine (tests.synth.residual_tolerance).  Integer
block sums, fma chains, quantisation and the combine order are the
reference's, so most elements are bit-identical; the device e^x (silu,
softmax) and the tree-ordered double sum of rmsnorm can move a value by about
an ulp."""
import numpy as np
import pytest
import torch

import oracle
from tests.synth import build_moe_case, residual_tolerance

pytestmark = pytest.mark.gpu

RTOL = 1e-5


def rel_err(got, want):
    return np.abs(got - want) / (np.abs(want) + 1e-3 * np.abs(want).max())


def run_dev(case, h0, dev):
    h = torch.from_numpy(h0.copy()).to(dev)
    case.block(h)
    torch.cuda.synchronize()
    return h.cpu().numpy(), case.block.ids.cpu().numpy()[:case.k], case.block.w.cpu().numpy()[:case.k]


def check_case(case, dev, tokens=3, seed=0):
    rng = np.random.default_rng(seed)
    worst, exact = 0.0, []
    for t in range(tokens):
        h0 = case.h0 if t == 0 else (rng.standard_normal(case.D) * (1 + t)).astype(np.float32)
        want_h, want_ids, want_w, tr = case.host.run(h0, trace=True)
        got_h, got_ids, got_w = run_dev(case, h0, dev)
        assert np.array_equal(got_ids, want_ids), (t, got_ids, want_ids)
        e = rel_err(got_h, want_h)
        worst = max(worst, float(e.max()))
        exact.append(np.mean(got_h.view(np.uint32) == want_h.view(np.uint32)))
        tol = residual_tolerance(want_h, want_w, got_w, tr["eo"], RTOL)
        assert np.all(np.abs(got_h - want_h) <= tol), f"token {t}: max rel err {e.max():.3g}"
    return worst, float(np.mean(exact))


def test_moe_small_config_shape(hip, dev):
    """The synthetic 4-layer config's block: D 512, 32 experts top-4, de 256,
    Q6_K experts, Q8_0 shared expert of width 256, softmax + renormalise."""
    case = build_moe_case(D=512, de=256, E=32, k=4, ds=256, expert_dt=oracle.Q6_K, shared_dt=oracle.Q8_0,
                          seed=21, device=dev)
    worst, exact = check_case(case, dev, tokens=5)
    assert exact > 0.5, f"only {exact:.2%} of outputs bit-identical"


def test_moe_qwen3_30b_shape(hip, dev):
    """D 2048, 128 experts top-8, de 768, Q6_K experts, no shared expert."""
    case = build_moe_case(D=2048, de=768, E=128, k=8, ds=0, expert_dt=oracle.Q6_K, seed=5, device=dev,
                          weights="random_codes")
    check_case(case, dev, tokens=3)


def test_moe_wide_model_dim(hip, dev):
    """D 4864 = 9 full 512-value router chunks + a 256-value tail: the router's
    rolling prefetch past the first 2048 values and its tail chunk."""
    case = build_moe_case(D=4864, de=256, E=16, k=2, ds=0, expert_dt=oracle.Q6_K, seed=44, device=dev,
                          weights="random_codes")
    check_case(case, dev, tokens=2)


def test_moe_many_down_blocks(hip, dev):
    """k * de = 4 x 2304: 36 activation blocks of h per down group, more than
    its first two quantisation passes cover, with a Q6_K shared expert."""
    case = build_moe_case(D=512, de=2304, E=16, k=4, ds=256, expert_dt=oracle.Q6_K, shared_dt=oracle.Q6_K,
                          seed=45, device=dev, weights="random_codes")
    check_case(case, dev, tokens=2)


@pytest.mark.parametrize("router", [0, 1, 2])
def test_moe_routers(hip, dev, router):
    bias = np.linspace(-0.05, 0.05, 16).astype(np.float32) if router == 2 else None
    case = build_moe_case(D=256, de=256, E=16, k=2, ds=0, expert_dt=oracle.Q6_K, seed=30 + router,
                          device=dev, router=router, routed_scale=2.5 if router else 1.0, router_bias=bias)
    check_case(case, dev, tokens=3, seed=router)


@pytest.mark.parametrize("edt,sdt", [(oracle.Q8_0, oracle.Q8_0), (oracle.Q4_K, oracle.Q8_0),
                                     (oracle.Q5_K, oracle.Q6_K), (oracle.Q6_K, oracle.Q6_K)])
def test_moe_dtypes_and_shared(hip, dev, edt, sdt):
    case = build_moe_case(D=512, de=256, E=8, k=3, ds=512, expert_dt=edt, shared_dt=sdt, seed=edt * 7 + sdt,
                          device=dev, shared_gate=True)
    check_case(case, dev, tokens=2)


def test_moe_mask_and_repeat(hip, dev):
    """Pruned experts never route; a second identical call reproduces the bits."""
    mask = np.zeros(32, np.uint8)
    mask[[1, 5, 9, 13, 17, 21, 25, 29]] = 1
    case = build_moe_case(D=512, de=256, E=32, k=4, ds=0, expert_dt=oracle.Q6_K, seed=77, device=dev, mask=mask)
    check_case(case, dev, tokens=2)
    a = run_dev(case, case.h0, dev)
    b = run_dev(case, case.h0, dev)
    assert not np.any(mask[a[1]])
    assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32))


def test_moe_phases_equal_layer(hip, dev):
    case = build_moe_case(D=512, de=256, E=32, k=4, ds=256, expert_dt=oracle.Q6_K, shared_dt=oracle.Q8_0,
                          seed=3, device=dev)
    full = run_dev(case, case.h0, dev)[0]
    h = torch.from_numpy(case.h0.copy()).to(dev)
    case.block.phase(1, h)
    case.block.phase(2, h)
    case.block.phase(1, h)      # re-running phases 1-2 reproduces the same bits
    case.block.phase(2, h)
    case.block.phase(3, h)
    torch.cuda.synchronize()
    assert np.array_equal(h.cpu().numpy().view(np.uint32), full.view(np.uint32))
