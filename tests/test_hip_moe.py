"""The device MoE block (tlm_hip_moe_layer) vs the oracle's MoE block
(src/lib/tlm_model.c:940-1055).

Bar: bit for bit - routing ids, routing weights and every element of the
updated residual.  Integer block sums, fma chains, quantisation, the combine
order and e^x (libm's expf, restated) are the reference's; the one remaining
difference in order, rmsnorm's double sum of squares as a tree, changes the
float result only when that sum lies within a few double ulps of a float
rounding boundary (never met in these cases)."""
import numpy as np
import pytest
import torch

import oracle
from tests.synth import build_moe_case

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def run_dev(case, h0, dev):
    h = torch.from_numpy(h0.copy()).to(dev)
    case.block(h)
    torch.cuda.synchronize()
    return h.cpu().numpy(), case.block.ids.cpu().numpy()[:case.k], case.block.w.cpu().numpy()[:case.k]


def check_case(case, dev, tokens=3, seed=0):
    rng = np.random.default_rng(seed)
    for t in range(tokens):
        h0 = case.h0 if t == 0 else (rng.standard_normal(case.D) * (1 + t)).astype(np.float32)
        want_h, want_ids, want_w, _ = case.host.run(h0, trace=True)
        got_h, got_ids, got_w = run_dev(case, h0, dev)
        assert np.array_equal(got_ids, want_ids), (t, got_ids, want_ids)
        assert np.array_equal(bits(got_w), bits(want_w)), (t, got_w, want_w)
        nd = int((bits(got_h) != bits(want_h)).sum())
        assert nd == 0, f"token {t}: {nd} of {case.D} residual elements differ from the oracle"


def test_moe_small_config_shape(hip, dev):
    """The synthetic 4-layer config's block: D 512, 32 experts top-4, de 256,
    Q6_K experts, Q8_0 shared expert of width 256, softmax + renormalise."""
    case = build_moe_case(D=512, de=256, E=32, k=4, ds=256, expert_dt=oracle.Q6_K, shared_dt=oracle.Q8_0,
                          seed=21, device=dev)
    check_case(case, dev, tokens=5)


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
