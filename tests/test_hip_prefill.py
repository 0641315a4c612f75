"""Prefill through the routed MoE block (tlm_hip_moe_prefill) vs the decode
block run token by token and vs the oracle.

The reference's prefill is the decode step repeated per token
(src/lib/tlm_model.c:1105-1113) and the MoE block has no cross-token terms,
so every token of a prefill must carry exactly the bits the decode block
gives it (routing ids, weights and the updated residual), whatever the mix of
tokens per expert: the expert buckets here range from empty to more than one
32-token tile.  Against the oracle the bar is the decode tests' one: bit for
bit."""
import numpy as np
import pytest
import torch

import oracle
from tests.synth import build_moe_case

pytestmark = pytest.mark.gpu


def prefill_vs_decode(case, dev, T, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    H = (rng.standard_normal((T, case.D)) * scale).astype(np.float32)
    h = torch.from_numpy(H.copy()).to(dev)
    ids = torch.empty((T, case.k), dtype=torch.int32, device=dev)
    w = torch.empty((T, case.k), dtype=torch.float32, device=dev)
    case.block.prefill(h, ids, w)
    torch.cuda.synchronize()
    got, got_ids, got_w = h.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy()
    prefill_vs_decode.last = (got, got_ids, got_w)
    for t in range(T):
        ht = torch.from_numpy(H[t].copy()).to(dev)
        case.block(ht)
        torch.cuda.synchronize()
        assert np.array_equal(got_ids[t], case.block.ids.cpu().numpy()[:case.k]), t
        assert np.array_equal(got_w[t].view(np.uint32), case.block.w.cpu().numpy()[:case.k].view(np.uint32)), t
        assert np.array_equal(got[t].view(np.uint32), ht.cpu().numpy().view(np.uint32)), f"token {t}"
    return H, got, got_ids


@pytest.mark.parametrize("dt", [oracle.Q4_K, oracle.Q5_K, oracle.Q6_K])
@pytest.mark.parametrize("T", [1, 7, 40, 129])
def test_prefill_equals_decode_per_token(hip, dev, dt, T):
    """D 512, 16 experts top-4, de 256: at T = 129 some experts hold more than
    32 tokens (two tiles), at T = 1 most hold none."""
    case = build_moe_case(D=512, de=256, E=16, k=4, ds=0, expert_dt=dt, seed=60 + T, device=dev,
                          weights="random_codes")
    prefill_vs_decode(case, dev, T, seed=T)


@pytest.mark.parametrize("dt", [oracle.Q5_K, oracle.Q6_K])
def test_prefill_qwen3_shape_vs_oracle(hip, dev, dt):
    """D 2048, 128 experts top-8, de 768 at 24 tokens: decode bits per token, and
    the oracle's block's bits (routing ids and weights, residual)."""
    case = build_moe_case(D=2048, de=768, E=128, k=8, ds=0, expert_dt=dt, seed=9, device=dev,
                          weights="random_codes")
    H, got, got_ids = prefill_vs_decode(case, dev, 24, seed=5)
    _, _, got_w = prefill_vs_decode.last
    for t in range(0, 24, 3):
        want_h, want_ids, want_w, _ = case.host.run(H[t], trace=True)
        assert np.array_equal(got_ids[t], want_ids)
        assert np.array_equal(got_w[t].view(np.uint32), np.asarray(want_w, np.float32).view(np.uint32)), t
        assert np.array_equal(got[t].view(np.uint32), np.asarray(want_h, np.float32).view(np.uint32)), t


@pytest.mark.parametrize("dt", [oracle.Q5_K, oracle.Q6_K])
def test_prefill_qwen3_shape_512_tokens(hip, dev, dt):
    """The benchmarked chunk: 512 tokens through D 2048, 128 experts top-8,
    de 768 (every expert holds tokens, many hold two 32-slot tiles); routing
    of every token and the residual of every 8th token carry the decode
    block's bits."""
    case = build_moe_case(D=2048, de=768, E=128, k=8, ds=0, expert_dt=dt, seed=13, device=dev,
                          weights="random_codes")
    T = 512
    rng = np.random.default_rng(21)
    H = rng.standard_normal((T, case.D)).astype(np.float32)
    h = torch.from_numpy(H.copy()).to(dev)
    ids = torch.empty((T, case.k), dtype=torch.int32, device=dev)
    w = torch.empty((T, case.k), dtype=torch.float32, device=dev)
    case.block.prefill(h, ids, w)
    torch.cuda.synchronize()
    got, got_ids, got_w = h.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy()
    counts = np.bincount(got_ids.ravel(), minlength=case.E)
    assert counts.min() > 0 and (counts > 32).any()          # every expert used, some past one tile
    for t in range(T):
        case.block.route(torch.from_numpy(H[t].copy()).to(dev))
        torch.cuda.synchronize()
        assert np.array_equal(got_ids[t], case.block.ids.cpu().numpy()[:case.k]), t
        assert np.array_equal(got_w[t].view(np.uint32), case.block.w.cpu().numpy()[:case.k].view(np.uint32)), t
    for t in range(0, T, 8):
        ht = torch.from_numpy(H[t].copy()).to(dev)
        case.block(ht)
        torch.cuda.synchronize()
        assert np.array_equal(got[t].view(np.uint32), ht.cpu().numpy().view(np.uint32)), f"token {t}"


def test_prefill_many_tokens(hip, dev):
    """20000 tokens x top-4 = 80000 (token, rank) slots, more than a grid's y
    dimension holds: the launches that cover slots put them on x."""
    case = build_moe_case(D=256, de=256, E=16, k=4, ds=0, expert_dt=oracle.Q6_K, seed=17, device=dev,
                          weights="random_codes")
    T = 20000
    rng = np.random.default_rng(22)
    H = rng.standard_normal((T, case.D)).astype(np.float32)
    h = torch.from_numpy(H.copy()).to(dev)
    ids = torch.empty((T, case.k), dtype=torch.int32, device=dev)
    case.block.prefill(h, ids)
    torch.cuda.synchronize()
    got, got_ids = h.cpu().numpy(), ids.cpu().numpy()
    for t in list(range(0, T, 997)) + [T - 1]:
        ht = torch.from_numpy(H[t].copy()).to(dev)
        case.block(ht)
        torch.cuda.synchronize()
        assert np.array_equal(got_ids[t], case.block.ids.cpu().numpy()[:case.k]), t
        assert np.array_equal(got[t].view(np.uint32), ht.cpu().numpy().view(np.uint32)), f"token {t}"


@pytest.mark.parametrize("router", [1, 2])
def test_prefill_routers_and_mask(hip, dev, router):
    mask = np.zeros(16, np.uint8)
    mask[[3, 7, 11]] = 1
    bias = np.linspace(-0.05, 0.05, 16).astype(np.float32) if router == 2 else None
    case = build_moe_case(D=256, de=256, E=16, k=3, ds=0, expert_dt=oracle.Q6_K, seed=70 + router, device=dev,
                          router=router, routed_scale=2.0, router_bias=bias, mask=mask)
    _, _, ids = prefill_vs_decode(case, dev, 50, seed=router, scale=2.0)
    assert not np.any(mask[ids])


@pytest.mark.parametrize("sdt,gate", [(oracle.Q8_0, False), (oracle.Q6_K, True)])
@pytest.mark.parametrize("T", [5, 70])
def test_prefill_shared_expert(hip, dev, sdt, gate, T):
    """A shared expert (C1's kind: Q8_0, or Q6_K with a sigmoid gate input)
    beside the routed ones: its gate / up / down as token matmuls, added
    after the routed sum in the decode block's order - every token's bits."""
    case = build_moe_case(D=512, de=256, E=16, k=4, ds=256, expert_dt=oracle.Q6_K, shared_dt=sdt, seed=80 + T,
                          device=dev, weights="random_codes", shared_gate=gate)
    prefill_vs_decode(case, dev, T, seed=T)


def test_prefill_rejects_unsupported(hip, dev):
    from tierlm_amd._lib import HipError
    case = build_moe_case(D=256, de=256, E=8, k=2, ds=128, expert_dt=oracle.Q6_K, shared_dt=oracle.Q8_0, seed=1,
                          device=dev, weights="random_codes")
    with pytest.raises(HipError):   # a shared width that is not a multiple of 256
        case.block.prefill(torch.zeros((4, 256), device=dev))
    case = build_moe_case(D=256, de=256, E=8, k=2, ds=0, expert_dt=oracle.Q8_0, seed=1, device=dev,
                          weights="random_codes")
    with pytest.raises(HipError):
        case.block.prefill(torch.zeros((4, 256), device=dev))
