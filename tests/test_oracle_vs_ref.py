"""The oracle against the reference itself, compiled from its sources into
oracle/_ref (skipped when that library is not built): weight quantisers and
activation quantiser byte for byte, dot / matvec bit for bit on the scalar and
SIMD tiers over the reference's edge-case generators, and one MoE block
through the reference's kernels."""
import numpy as np
import pytest

import oracle
from oracle import Q4_K, Q5_K, Q6_K, Q8_0, Q8_K
from tests.synth import build_moe_case
from tests.test_hip_gemv import make_act, make_wrow

pytestmark = pytest.mark.skipif(oracle.ref is None, reason="oracle/_ref not built (reference sources absent)")

INT = [Q8_0, Q4_K, Q5_K, Q6_K, Q8_K]


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))


def test_f16_conversions_match_reference():
    codes = np.arange(0, 65536, 7, dtype=np.uint16)
    for c in codes:
        assert same(oracle.orc.orc_f16_to_f32(int(c)), oracle.ref.tlm_f16_to_f32(int(c)))
    rng = np.random.default_rng(0)
    for x in (rng.standard_normal(5000) * 10.0 ** rng.integers(-9, 6, 5000)).astype(np.float32):
        assert oracle.orc.orc_f32_to_f16(float(x)) == oracle.ref.tlm_f32_to_f16(float(x))


@pytest.mark.parametrize("dt", INT)
def test_weight_quantisers_bytes(dt):
    rng = np.random.default_rng(dt)
    for n in (256, 512, 2048):
        for scale in (0.02, 1.0, 300.0):
            x = (rng.standard_normal((6, n)) * scale).astype(np.float32)
            x[1, :40] = 0.0
            x[2, :] = np.abs(x[2, :])
            x[3, ::7] = 0.0
            x[4, :] = 0.0
            x[5, 100] = scale * 50
            assert np.array_equal(oracle.quantize_row(dt, x), oracle.quantize_row(dt, x, use_ref=True)), (n, scale)


def test_activation_quantiser_bytes():
    rng = np.random.default_rng(3)
    cases = [rng.standard_normal(n).astype(np.float32) * s for n, s in
             [(2048, 1.0), (100, 3.0), (1003, 1e-30), (513, 1e30), (37, 1.0)]]
    v = rng.standard_normal(512).astype(np.float32)
    v[10], v[300] = np.nan, np.inf
    cases.append(v)
    cases.append((np.arange(64, dtype=np.float32) - 32) * np.float32(2.0 ** -140))
    for x in cases:
        for kind in (Q8_K, Q8_0):
            assert np.array_equal(oracle.quantize_act(kind, x), oracle.quantize_act(kind, x, use_ref=True))


@pytest.mark.parametrize("tier", ["scalar", "avx2", "avx512"])
@pytest.mark.parametrize("dt", INT)
def test_dots_bit_exact_per_tier(dt, tier):
    oracle.ref.tlm_cpu_force(tier.encode())
    oracle.ref.tlm_quant_init()
    try:
        got_tier = oracle.ref.tlm_quant_tier().decode()
        if got_tier != tier:
            pytest.skip(f"tier {tier} not available on this CPU")
        rng = np.random.default_rng(dt * 17)
        bv = oracle.BLOCK[dt][0]
        for nblk in (1, 2, 3, 8, 9, 17, 33):
            n = nblk * bv
            for rep in range(24):
                w = make_wrow(rng, dt, n, rep % 5)
                a = make_act(rng, dt, n, rep % 5)
                assert same(oracle.vec_dot(dt, w, a, n), oracle.vec_dot(dt, w, a, n, use_ref=True)), (n, rep)
        # matvec with padded stride and unaligned base, absolute row indexing
        n = 3 * bv
        tight = oracle.row_bytes(dt, n)
        rb = tight + 6
        mem = np.full(rb * 24 + 3 + 64, 0xA5, np.uint8)
        for r in range(24):
            mem[3 + rb * r:3 + rb * r + tight] = make_wrow(rng, dt, n, r % 5)
        a = make_act(rng, dt, n, 0)
        want = oracle.matvec_rows(dt, mem, rb, a, n, 5, 21, nrows=24, offset=3)
        got = oracle.matvec_rows(dt, mem, rb, a, n, 5, 21, nrows=24, offset=3, use_ref=True)
        assert np.all(same(got, want))
    finally:
        oracle.ref.tlm_cpu_force(b"auto")
        oracle.ref.tlm_quant_init()
    assert oracle.ref.tlm_quant_selftest_failures() == 0


def test_f32_dot_lane_order():
    rng = np.random.default_rng(2)
    for n in list(range(1, 80)) + [1003, 4099]:
        w = rng.standard_normal(n).astype(np.float32)
        x = rng.standard_normal(n).astype(np.float32)
        assert same(oracle.vec_dot(oracle.F32, w.view(np.uint8), x, n),
                    oracle.vec_dot(oracle.F32, w.view(np.uint8), x, n, use_ref=True))


@pytest.mark.parametrize("threads", [1, 4])
def test_moe_block_matches_reference_kernels(threads):
    case = build_moe_case(D=512, de=256, E=32, k=4, ds=256, expert_dt=Q6_K, shared_dt=Q8_0, seed=44)
    handle = oracle.ref.refmoe_new(threads)
    try:
        for t in range(3):
            h0 = np.random.default_rng(t).standard_normal(512).astype(np.float32) * (t + 1)
            a = case.host.run(h0)
            b = case.host.run_ref(handle, h0)
            assert np.array_equal(a[1], b[1]) and np.array_equal(a[2], b[2])
            assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32))
    finally:
        oracle.ref.refmoe_free(handle)
