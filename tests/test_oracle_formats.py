"""Pins the oracle with facts that do not come from its own code: exhaustive
f16 conversion against numpy's IEEE binary16, the reference's known-answer
tests (tests/test_quant.c:59-119, 396-425, 434-536 there), layouts rebuilt
from the format documentation (src/lib/tlm_quant.h:8-19 there), the
double-precision dot bound (tests/test_quant.c:540-583 there) and float64
restatements of the decoder glue."""
import numpy as np
import pytest

import oracle
from oracle import Q4_K, Q5_K, Q6_K, Q8_0, Q8_K

INT = [Q8_0, Q4_K, Q5_K, Q6_K, Q8_K]


def f32b(x):
    return np.float32(x).view(np.uint32)


# ---------------------------------------------------------------- f16
def test_f16_to_f32_exhaustive():
    codes = np.arange(65536, dtype=np.uint16)
    want = codes.view(np.float16).astype(np.float32)
    got = np.array([oracle.orc.orc_f16_to_f32(int(c)) for c in codes], np.float32)
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    # NaN: quiet bit set, payload kept in the top mantissa bits, sign kept
    for c in codes[~fin]:
        g = int(np.float32(got[c]).view(np.uint32))
        assert (g & 0x7FC00000) == 0x7FC00000
        assert ((g >> 13) & 0x3FF) == (int(c) & 0x3FF) | 0x200
        assert (g >> 31) == (int(c) >> 15)


def test_f32_to_f16_rne():
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
                         np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25,
                                   2.0 ** -25 * 1.0000001, 2.0 ** -26, 6.1e-5, np.inf, -np.inf], np.float32)])
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    got = np.array([oracle.orc.orc_f32_to_f16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, want)
    nan = oracle.orc.orc_f32_to_f16(float("nan"))
    assert (nan & 0x7E00) == 0x7E00


# ---------------------------------------------------------------- layouts
def test_layout_kats():
    rb = oracle.row_bytes
    assert rb(Q6_K, 4096) == 16 * 210 and rb(Q4_K, 4096) == 16 * 144 and rb(Q5_K, 512) == 2 * 176
    assert rb(Q8_0, 64) == 68 and rb(oracle.F32, 7) == 28
    assert rb(Q4_K, 100) == 0 and rb(Q8_0, -32) == 0
    qa = oracle.qact_bytes
    assert qa(Q8_K, 256) == 292 and qa(Q8_K, 257) == 584 and qa(Q8_0, 64) == 72 and qa(Q8_0, 33) == 72
    assert qa(oracle.F32, 10) == 40 and qa(Q6_K, 256) == 0
    for dt in (Q4_K, Q5_K, Q6_K, Q8_K):
        assert oracle.act_kind_for(dt) == Q8_K
    assert oracle.act_kind_for(Q8_0) == Q8_0 and oracle.act_kind_for(oracle.F32) == oracle.F32


def put16(b, off, v):
    b[off:off + 2] = np.frombuffer(np.float16(v).tobytes(), np.uint8)


def test_element_order_kats():
    """tests/test_quant.c:396-425 there."""
    blk = np.zeros(210, np.uint8)
    put16(blk, 0, 1.0)
    put16(blk, 2, 0.0)
    blk[4 + 1] = 2
    blk[4 + 8 + 2] = 3
    blk[16 + 32 * 0 + 5] = 0x70
    blk[16 + 32 * 3 + 9] = 0x04
    y = oracle.dequantize_row(Q4_K, blk[:144], 256)
    assert np.count_nonzero(y) == 2 and y[37] == 14.0 and y[201] == 12.0
    blk = np.zeros(210, np.uint8)
    put16(blk, 208, 1.0)
    blk[192:208] = 1
    blk[128:192] = 0xAA
    blk[64 + 32 + 7] = 0x50
    y = oracle.dequantize_row(Q6_K, blk, 256)
    assert np.count_nonzero(y) == 1 and y[231] == 5.0


# layout packers written from the format documentation, independent of the oracle
def pack_q6k(u, sc, d):
    """u: 256 codes 0..63; element 128h + 32q + l -> ql nibble / qh bit pair."""
    blk = np.zeros(210, np.uint8)
    for e in range(256):
        h, q, l = e // 128, (e % 128) // 32, e % 32
        at = 64 * h + 32 * (q % 2) + l
        blk[at] |= (u[e] & 15) << (4 if q >= 2 else 0)
        blk[128 + 32 * h + l] |= (u[e] >> 4) << (2 * q)
    blk[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    put16(blk, 208, d)
    return blk


def pack_kq(codes, sc, mn, d, dmin, q5):
    """codes 0..15 / 0..31; sub-block s = element // 32; chunk c = e // 64."""
    bb = 176 if q5 else 144
    blk = np.zeros(bb, np.uint8)
    put16(blk, 0, d)
    put16(blk, 2, dmin)
    for j in range(4):
        blk[4 + j] = (sc[j] & 63) | ((sc[4 + j] >> 4) << 6)
        blk[8 + j] = (mn[j] & 63) | ((mn[4 + j] >> 4) << 6)
        blk[12 + j] = (sc[4 + j] & 15) | ((mn[4 + j] & 15) << 4)
    qs = 48 if q5 else 16
    for e in range(256):
        c, hi, l = e // 64, (e // 32) % 2, e % 32
        blk[qs + 32 * c + l] |= (codes[e] & 15) << (4 * hi)
        if q5:
            blk[16 + l] |= ((codes[e] >> 4) & 1) << (2 * c + hi)
    return blk


def act_from_codes(q, d):
    a = np.zeros(292, np.uint8)
    a[0:4] = np.frombuffer(np.float32(d).tobytes(), np.uint8)
    a[4:260] = np.asarray(q, np.int8).view(np.uint8)
    bs = np.asarray(q, np.int64).reshape(16, 16).sum(1).astype(np.int16)
    a[260:292] = bs.view(np.uint8)
    return a


def test_block_isums_from_documented_layout():
    """Integer block sums and dequantisation against codes placed by an
    independent packer: a transposed index or a dropped term fails."""
    rng = np.random.default_rng(1)
    for rep in range(50):
        x = rng.integers(-127, 128, 256)
        a = act_from_codes(x, 0.01)
        u = rng.integers(0, 64, 256)
        sc = rng.integers(-128, 128, 16)
        blk = pack_q6k(u, sc, 0.5)
        want = int(sum(sc[g] * np.dot(u[16 * g:16 * g + 16] - 32, x[16 * g:16 * g + 16]) for g in range(16)))
        assert oracle.block_isum(Q6_K, blk, a)[0] == want
        y = oracle.dequantize_row(Q6_K, blk, 256)
        assert np.array_equal(y, (np.float32(0.5) * np.repeat(sc, 16).astype(np.float32)) * (u - 32).astype(np.float32))
        for q5 in (False, True):
            codes = rng.integers(0, 32 if q5 else 16, 256)
            scs, mns = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
            blk = pack_kq(codes, scs, mns, 0.25, 0.125, q5)
            isum = int(sum(scs[s] * np.dot(codes[32 * s:32 * s + 32], x[32 * s:32 * s + 32]) for s in range(8)))
            msum = int(sum(mns[s] * x[32 * s:32 * s + 32].sum() for s in range(8)))
            assert oracle.block_isum(Q5_K if q5 else Q4_K, blk, a) == (isum, msum)
        w = np.zeros(34, np.uint8)
        qw = rng.integers(-128, 128, 32)
        w[2:] = qw.astype(np.int8).view(np.uint8)
        a8 = np.zeros(36, np.uint8)
        a8[4:] = x[:32].astype(np.int8).view(np.uint8)
        assert oracle.block_isum(Q8_0, w, a8)[0] == int(np.dot(qw, x[:32]))


# ---------------------------------------------------------------- activation quantiser KATs
def fill_row(n, seed):
    return np.random.default_rng(seed).standard_normal(n).astype(np.float32) * 3


def test_act_quant_kats():
    """tests/test_quant.c:434-536 there."""
    x = fill_row(512, 2)
    x[3] = -100.0
    buf = oracle.quantize_act(Q8_K, x)
    for b in range(2):
        blk = buf[292 * b:292 * (b + 1)]
        d = blk[0:4].view(np.float32)[0]
        q = blk[4:260].view(np.int8).astype(int)
        amax = np.abs(x[256 * b:256 * (b + 1)]).max()
        assert d == np.float32(amax) / np.float32(127.0) and d > 0
        assert q.min() >= -127 and (np.abs(q) == 127).any()
        assert np.array_equal(blk[260:292].view(np.int16), q.reshape(16, 16).sum(1))
    assert buf[4 + 3].view(np.int8) == -127
    assert np.array_equal(buf, oracle.quantize_row(Q8_K, x))       # activation layout == Q8_K weight layout
    ab = oracle.quantize_act(Q8_0, x)
    assert ab[36:40].view(np.float32)[0] == np.float32(np.abs(x[32:64]).max()) / np.float32(127.0)
    z = np.zeros(34, np.float32)
    z[33] = 1.0
    zb = oracle.quantize_act(Q8_0, z)
    assert zb[0:4].view(np.float32)[0] == 0.0 and zb[4 + 5] == 0
    assert zb[36:40].view(np.float32)[0] == np.float32(1.0) / np.float32(127.0)
    assert zb[36 + 4 + 1].view(np.int8) == 127 and zb[36 + 4 + 2] == 0 and zb[36 + 4 + 31] == 0
    kb = oracle.quantize_act(Q8_K, x[:100])
    assert np.count_nonzero(kb[4 + 100:260]) == 0 and kb[260 + 30:292].view(np.int16)[0] == 0
    v = fill_row(512, 4)
    v[10] = np.nan
    v[300] = np.inf
    kb = oracle.quantize_act(Q8_K, v)
    assert np.isnan(kb[0:4].view(np.float32)[0]) and kb[292:296].view(np.float32)[0] == np.inf
    assert np.count_nonzero(kb[4:260]) == 0
    ab = oracle.quantize_act(Q8_0, v)
    assert np.isnan(ab[0:4].view(np.float32)[0]) and ab[9 * 36:9 * 36 + 4].view(np.float32)[0] == np.inf
    assert np.isfinite(ab[36:40].view(np.float32)[0])
    tiny = (np.arange(32, dtype=np.float32) - 16) * np.float32(2.0 ** -140)
    tb = oracle.quantize_act(Q8_0, tiny)
    assert tb[4].view(np.int8) == -127 and tb[4 + 16] == 0 and tb[4 + 24] == 64
    c = oracle.quantize_act(oracle.F32, x[:7])
    assert np.array_equal(c[:28].view(np.float32), x[:7])


def test_act_quant_codes_closed_form():
    """codes = round-half-even(x * (127/amax)) in float32, clamped."""
    rng = np.random.default_rng(9)
    for rep in range(30):
        x = (rng.standard_normal(256) * 10.0 ** rng.uniform(-3, 3)).astype(np.float32)
        blk = oracle.quantize_act(Q8_K, x)
        amax = np.abs(x).max()
        idv = np.float32(127.0) / np.float32(amax)
        want = np.clip(np.rint(x * idv), -127, 127).astype(np.int8)
        assert np.array_equal(blk[4:260].view(np.int8), want)


# ---------------------------------------------------------------- dots vs double
def test_dot_vs_double_reference():
    """|dot - sum deq(w)*deq(x)| < 2e-6 * sum|w*x| (tests/test_quant.c:540-583 there)."""
    n = 2048
    for dt in INT + [oracle.F32]:
        for rep in range(12):
            rng = np.random.default_rng(rep * 31 + dt)
            wf = rng.standard_normal(n).astype(np.float32) * [0.02, 1.0, 5.0][rep % 3]
            x = rng.standard_normal(n).astype(np.float32) * [1.0, 0.01, 30.0][rep % 3]
            w = oracle.quantize_row(dt, wf)
            kind = oracle.act_kind_for(dt)
            act = oracle.quantize_act(kind, x)
            wd = oracle.dequantize_row(dt, w, n).astype(np.float64)
            if kind == Q8_K:
                xd = oracle.dequantize_row(Q8_K, act, n).astype(np.float64)
            elif kind == Q8_0:
                blk = act.reshape(-1, 36)
                xd = (blk[:, 0:4].copy().view(np.float32).astype(np.float64) *
                      blk[:, 4:].view(np.int8).astype(np.float64)).reshape(-1)
            else:
                xd = x.astype(np.float64)
            ref = float(np.dot(wd, xd))
            sa = float(np.abs(wd * xd).sum())
            got = float(oracle.vec_dot(dt, w, act, n))
            assert abs(got - ref) <= 2e-6 * sa + 1e-30, (dt, rep, got, ref)


def test_quantiser_roundtrip_error():
    """Quantise -> dequantise error stays within each format's step."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal(4096).astype(np.float32)
    for dt, tol in [(Q8_0, 0.01), (Q6_K, 0.04), (Q5_K, 0.08), (Q4_K, 0.16), (Q8_K, 0.01)]:
        y = oracle.dequantize_row(dt, oracle.quantize_row(dt, x), 4096)
        rel = np.sqrt(np.mean((y - x) ** 2)) / np.sqrt(np.mean(x ** 2))
        assert rel < tol, (dt, rel)


# ---------------------------------------------------------------- decoder glue
def test_rmsnorm_vs_float64():
    rng = np.random.default_rng(3)
    for n in (64, 512, 2048):
        x = rng.standard_normal(n).astype(np.float32) * 5
        w = rng.standard_normal(n).astype(np.float32)
        got = oracle.rmsnorm(x, w, 1e-6)
        r = 1.0 / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6)
        want = x.astype(np.float64) * r * w
        assert np.all(np.abs(got - want) <= 1e-6 * np.abs(want) + 1e-30)


def softmax_topk64(logits, k, mask=None):
    l64 = logits.astype(np.float64)
    ok = ~np.isnan(l64) if mask is None else (~np.isnan(l64) & (mask == 0))
    mx = l64[ok].max()
    p = np.where(ok, np.exp(np.where(ok, l64 - mx, 0.0)), 0.0)
    p /= p.sum()
    order = sorted([e for e in range(len(p)) if ok[e]], key=lambda e: (-p[e], e))
    # once the finite entries run out: lowest unmasked unused ids (NaN ones), weight 0
    order += [e for e in range(len(p)) if not ok[e] and (mask is None or mask[e] == 0)]
    return np.array(order[:k]), p


def test_route_softmax_closed_form():
    rng = np.random.default_rng(4)
    for rep in range(40):
        E, k = int(rng.choice([8, 32, 128])), int(rng.choice([1, 2, 4, 8]))
        logits = (rng.standard_normal(E) * 2).astype(np.float32)
        mask = None
        if rep % 4 == 1:
            mask = (rng.random(E) < 0.3).astype(np.uint8)
            mask[:k] = 0
        if rep % 5 == 2:
            logits[rng.integers(E)] = np.nan
        ids64, p64 = softmax_topk64(logits, k, mask)
        for router in (0, 1):
            ids, w = oracle.route(router, logits, k, mask=mask)
            assert np.array_equal(ids, ids64), (rep, ids, ids64)
            want = p64[ids64] / (p64[ids64].sum() if router == 0 else 1.0)
            assert np.all(np.abs(w - want) <= 2e-6 * want), (rep, router)
            if router == 0:
                assert abs(float(w.astype(np.float64).sum()) - 1.0) < 1e-6


def test_route_ties_nan_and_scale():
    logits = np.array([1.0, 3.0, 3.0, np.nan, 3.0, 0.5], np.float32)
    ids, w = oracle.route(1, logits, 4)
    assert list(ids) == [1, 2, 4, 0]                  # ties -> lowest id, NaN skipped
    allnan = np.full(4, np.nan, np.float32)
    ids, w = oracle.route(0, allnan, 2)
    assert list(ids) == [0, 1] and np.all(w == 0)     # deterministic fallback
    ids2, w2 = oracle.route(0, np.array([2.0, 1.0, 0.0], np.float32), 2, routed_scale=2.5)
    ids1, w1 = oracle.route(0, np.array([2.0, 1.0, 0.0], np.float32), 2)
    assert np.array_equal(ids1, ids2) and np.array_equal(w2, w1 * np.float32(2.5))


def test_route_sigmoid_bias():
    rng = np.random.default_rng(8)
    E, k = 16, 4
    logits = rng.standard_normal(E).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.5).astype(np.float32)
    ids, w = oracle.route(2, logits, k, routed_scale=1.5, bias=bias)
    s = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    sel = sorted(range(E), key=lambda e: (-(np.float32(s[e]) + bias[e]), e))[:k]
    assert list(ids) == sel
    want = s[sel] / s[sel].sum() * 1.5
    assert np.all(np.abs(w - want) <= 3e-6 * want)


def test_moe_layer_stages_vs_float64():
    """Each stage of the oracle's MoE block against float64 math on the
    dequantised operands it consumed (stage inputs from the trace)."""
    from tests.synth import build_moe_case
    case = build_moe_case(D=512, de=256, E=16, k=4, ds=256, expert_dt=Q6_K, shared_dt=Q8_0, seed=12)
    h, ids, w, tr = case.host.run(case.h0, trace=True)
    D, de = 512, 256
    xb64 = case.h0.astype(np.float64) / np.sqrt(np.mean(case.h0.astype(np.float64) ** 2) + 1e-6) * case.ffn_norm
    assert np.all(np.abs(tr["xb"] - xb64) <= 1e-6 * np.abs(xb64) + 1e-12)
    logit64 = case.router_w.astype(np.float64) @ tr["xb"].astype(np.float64)
    scale = np.abs(case.router_w.astype(np.float64)) @ np.abs(tr["xb"].astype(np.float64))
    assert np.all(np.abs(tr["logits"] - logit64) <= 1e-6 * scale)
    ids64, p64 = softmax_topk64(tr["logits"], 4)
    assert np.array_equal(ids, ids64)
    xq = oracle.dequantize_row(Q8_K, oracle.quantize_act(Q8_K, tr["xb"]), D).astype(np.float64)
    for r in range(4):
        g, u, dn = case.experts[ids[r]]
        G = np.stack([oracle.dequantize_row(Q6_K, row, D) for row in g]).astype(np.float64)
        U = np.stack([oracle.dequantize_row(Q6_K, row, D) for row in u]).astype(np.float64)
        tol = 2e-6 * (np.abs(G) @ np.abs(xq)) + 1e-30
        assert np.all(np.abs(tr["gu"][r, :de] - G @ xq) <= tol)
        tol = 2e-6 * (np.abs(U) @ np.abs(xq)) + 1e-30
        assert np.all(np.abs(tr["gu"][r, de:] - U @ xq) <= tol)
        g32, u32 = tr["gu"][r, :de].astype(np.float64), tr["gu"][r, de:].astype(np.float64)
        hh64 = g32 / (1.0 + np.exp(-g32)) * u32
        assert np.all(np.abs(tr["hh"][r] - hh64) <= 1e-6 * np.abs(hh64) + 1e-30)
        hq = oracle.dequantize_row(Q8_K, tr["hq"][r], de).astype(np.float64)
        Dn = np.stack([oracle.dequantize_row(Q6_K, row, de) for row in dn]).astype(np.float64)
        assert np.all(np.abs(tr["eo"][r] - Dn @ hq) <= 2e-6 * (np.abs(Dn) @ np.abs(hq)) + 1e-30)
    ffn64 = sum(np.float64(w[r]) * tr["eo"][r].astype(np.float64) for r in range(4)) + tr["s_out"]
    assert np.all(np.abs(tr["ffn"] - ffn64) <= 1e-6 * (sum(np.abs(w[r] * tr["eo"][r]) for r in range(4))
                                                      + np.abs(tr["s_out"])) + 1e-30)
    assert np.array_equal(h, case.h0 + tr["ffn"])
