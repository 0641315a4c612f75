"""HIP matvec (plain reference layout and packed tile layout) vs the oracle,
bit for bit - the reference's tier bit-exactness matrix with HIP as a fourth
tier (tests/test_quant.c:629-864 there): every integer format, block counts
1..64, the edge weight / activation modes, padded strides, unaligned bases and
row sub-ranges."""
import numpy as np
import pytest
import torch

import oracle
from tests.synth import random_code_rows

pytestmark = pytest.mark.gpu

INT = [oracle.Q8_0, oracle.Q4_K, oracle.Q5_K, oracle.Q6_K, oracle.Q8_K]


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    both_nan = np.isnan(a) & np.isnan(b)
    return (bits(a) == bits(b)) | both_nan


def put_f16(buf, off, v):
    buf[off:off + 2] = np.frombuffer(np.float16(v).tobytes(), np.uint8)


def make_wrow(rng, dt, n, mode):
    """Edge patterns of the reference's make_wrow: 0 random, 1 zero,
    2 max magnitude, 3 quantised from floats, 4 extreme scales."""
    bv, bb = oracle.BLOCK[dt]
    nb = n // bv
    if mode == 3:
        return oracle.quantize_row(dt, (rng.standard_normal(n) * rng.choice([0.02, 1.0, 50.0])).astype(np.float32))
    w = np.zeros(nb * bb, np.uint8) if mode == 1 else rng.integers(0, 256, nb * bb, dtype=np.uint8)
    for b in range(nb):
        o = b * bb
        dv = (65504.0 if rng.integers(2) else 2.0 ** -24) * (-1 if rng.integers(2) else 1) if mode == 4 \
            else rng.uniform(-0.05, 0.05)
        if mode == 1:
            dv = 0.0
        if dt == oracle.Q8_0:
            put_f16(w, o, 0.01 if mode == 2 else dv)
            if mode == 2:
                w[o + 2:o + 34] = np.where(rng.integers(0, 2, 32) > 0, 0x80, 0x7F)
        elif dt in (oracle.Q4_K, oracle.Q5_K):
            put_f16(w, o, 0.01 if mode == 2 else dv)
            put_f16(w, o + 2, 0.01 if mode == 2 else (dv if mode == 4 else rng.uniform(0, 0.05)))
            if mode == 2:
                w[o + 4:o + bb] = 0xFF
        elif dt == oracle.Q6_K:
            put_f16(w, o + 208, 0.01 if mode == 2 else dv)
            if mode == 2:
                w[o:o + 192] = 0xFF if rng.integers(2) else 0x00
                w[o + 192:o + 208] = [0x80 if g & 1 else 0x7F for g in range(16)]
        elif dt == oracle.Q8_K:
            d = np.float32(1e30 if mode == 2 else (dv * 1e3 if mode == 4 else dv))
            w[o:o + 4] = np.frombuffer(d.tobytes(), np.uint8)
            if mode == 2:
                w[o + 4:o + 260] = np.where(rng.integers(0, 2, 256) > 0, 0x80, 0x7F)
    return w


def make_act(rng, dt, n, mode):
    """0 bell, 1 zeros, 2 +-1, 3 spikes, 4 one NaN."""
    if mode == 1:
        x = np.zeros(n, np.float32)
    elif mode == 2:
        x = np.where(rng.integers(0, 2, n) > 0, 1.0, -1.0).astype(np.float32)
    elif mode == 3:
        x = (0.001 * rng.standard_normal(n)).astype(np.float32)
        x[::77] = 1000.0
    else:
        x = rng.standard_normal(n).astype(np.float32)
    if mode == 4:
        x[rng.integers(n)] = np.nan
    return oracle.quantize_act(oracle.act_kind_for(dt), x)


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).reshape(-1).view(np.uint8)).to(dev)


@pytest.mark.parametrize("dt", INT)
def test_matvec_bitexact_matrix(hip, dev, dt):
    """Single rows over block counts 1..64 and edge modes (60 reps each), plain layout."""
    rng = np.random.default_rng(100 + dt)
    bv = oracle.BLOCK[dt][0]
    compared = mismatch = nans = 0
    for nblk in (1, 2, 3, 7, 8, 9, 16, 17, 33, 64):
        n = nblk * bv
        rows, acts, wants = [], [], []
        for rep in range(60):
            wmode = rep if rep < 5 else (2 if rep % 7 == 0 else 4 if rep % 11 == 0 else 3 if rep % 5 == 0 else 0)
            amode = 1 if rep % 13 == 1 else 2 if rep % 13 == 2 else 3 if rep % 13 == 3 else 4 if rep % 29 == 4 else 0
            if rep < 5:
                amode = 2 if rep % 3 == 0 else 0
            w = make_wrow(rng, dt, n, wmode)
            if wmode == 0 and rep & 1:
                bb = oracle.BLOCK[dt][1]
                z = int(rng.integers(nblk))
                w[z * bb:(z + 1) * bb] = 0
            a = make_act(rng, dt, n, amode)
            rows.append(w)
            acts.append(a)
            wants.append(oracle.vec_dot(dt, w, a, n))
        for w, a, want in zip(rows, acts, wants):
            y = hip.matvec_rows(dt, to_dev(w, dev), w.size, to_dev(a, dev), n, 0, 1)
            torch.cuda.synchronize()
            got = y.cpu().numpy()[0]
            compared += 1
            nans += bool(np.isnan(want))
            mismatch += not same(got, want)
    assert mismatch == 0, f"{mismatch}/{compared} mismatches"
    assert nans > 0, "the NaN edge cases were not exercised"


@pytest.mark.parametrize("dt", INT)
def test_matvec_tiles_ranges(hip, dev, dt):
    """48 rows, padded stride, unaligned base, sub-ranges; untouched rows stay."""
    rng = np.random.default_rng(7 + dt)
    ranges = [(0, 1), (0, 7), (0, 8), (3, 11), (3, 30), (0, 40), (5, 45), (13, 13)]
    for shape in range(3):
        n = (1 if shape == 0 else 3 if shape == 1 else 16) * oracle.BLOCK[dt][0]
        tight = oracle.row_bytes(dt, n)
        rb = tight + (6 if shape == 1 else 0)
        off = 3 if shape == 2 else 0
        mem = np.full(rb * 48 + off + 64, 0xA5, np.uint8)
        for r in range(48):
            mem[off + rb * r: off + rb * r + tight] = make_wrow(rng, dt, n, r % 5)
        act = make_act(rng, dt, n, 2 if shape == 2 else 0)
        want = oracle.matvec_rows(dt, mem, rb, act, n, 0, 48, offset=off)
        memd, actd = to_dev(mem, dev), to_dev(act, dev)
        for r0, r1 in ranges:
            y = torch.full((48,), -12345.0, device=dev)
            hip.matvec_rows(dt, memd, rb, actd, n, r0, r1, y=y, offset=off)
            torch.cuda.synchronize()
            got = y.cpu().numpy()
            inside = np.zeros(48, bool)
            inside[r0:r1] = True
            assert np.all(got[~inside] == -12345.0), (shape, r0, r1)
            assert np.all(same(got[inside], want[inside])), (shape, r0, r1)


@pytest.mark.parametrize("dt", INT)
@pytest.mark.parametrize("rows,n", [(16, 256), (48, 512), (37, 768), (768, 2048), (2048, 768), (100, 4096),
                                    (64, 8192), (4096, 8192), (4100, 2048), (16400, 512), (16400, 2048),
                                    (16384, 4096)])
def test_matvec_packed(hip, dev, dt, rows, n):
    """Packed tile layout == oracle, including a partial last tile and rows
    longer than one chunk of blocks (Q8_0: 128 blocks, others 64), through the
    model's launch: quarter tiles per group for few tiles, half tiles from 256
    tiles on (4100 x 2048; 4096 x 8192, the Qwen3-235B-A22B o projection's
    shape, two chunks of blocks per row for Q8_0), whole tiles from 1024
    tiles on (16400 x 512; for Q8_0 at 2048 columns two tiles per group, the
    last group with one, and the activation loaded ahead of the weights; at
    4096 columns two 64-block chunks per tile)."""
    rng = np.random.default_rng(rows * 31 + n + dt)
    W = random_code_rows(rng, dt, rows, n)
    if rows <= 64:
        W[::3] = np.stack([make_wrow(rng, dt, n, m % 5) for m in range(0, rows, 3)])
    x = rng.standard_normal(n).astype(np.float32)
    act = oracle.quantize_act(oracle.act_kind_for(dt), x)
    want = oracle.matvec_rows(dt, W, W.shape[1], act, n, 0, rows)
    Wd = to_dev(W, dev)
    P = hip.pack(dt, Wd, W.shape[1], rows, n)
    y = hip.matvec_packed(dt, P, rows, n, to_dev(act, dev))
    torch.cuda.synchronize()
    got = y.cpu().numpy()[:rows]
    bad = np.nonzero(~same(got, want))[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}: {got[bad[:3]]} vs {want[bad[:3]]}"


def test_matvec_f32_lane_order(hip, dev):
    """f32 rows: lane i mod 32 + the fixed reduce32 tree, odd lengths, unaligned."""
    rng = np.random.default_rng(5)
    for n in list(range(1, 70)) + [1003, 2048, 4099]:
        W = rng.standard_normal((3, n)).astype(np.float32)
        x = rng.standard_normal(n).astype(np.float32)
        want = oracle.matvec_rows(oracle.F32, W.view(np.uint8), 4 * n, x, n, 0, 3)
        y = hip.matvec_rows(oracle.F32, to_dev(W, dev), 4 * n, torch.from_numpy(x).to(dev), n, 0, 3)
        torch.cuda.synchronize()
        assert np.all(same(y.cpu().numpy(), want)), n
    # unaligned base
    n = 515
    W = rng.standard_normal((4, n)).astype(np.float32)
    mem = np.zeros(W.nbytes + 8, np.uint8)
    mem[1:1 + W.nbytes] = W.view(np.uint8).reshape(-1)
    x = rng.standard_normal(n).astype(np.float32)
    want = oracle.matvec_rows(oracle.F32, mem, 4 * n, x, n, 0, 4, offset=1)
    y = hip.matvec_rows(oracle.F32, to_dev(mem, dev), 4 * n, torch.from_numpy(x).to(dev), n, 0, 4, offset=1)
    torch.cuda.synchronize()
    assert np.all(same(y.cpu().numpy(), want))


def test_matvec_errors(hip, dev):
    """Bad dtype / length NaN-fills [r0, r1) and reports TLM_EINVAL (src/lib/tlm_quant.c:1119-1127)."""
    from tierlm_amd import HipError
    buf = torch.zeros(1024, dtype=torch.uint8, device=dev)
    act = torch.zeros(1024, dtype=torch.uint8, device=dev)
    y = torch.ones(4, device=dev)
    with pytest.raises(HipError) as e:
        hip.matvec_rows(oracle.Q4_K, buf, 144, act, 100, 1, 3, y=y)
    assert e.value.code == -3
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.isnan(got[1]) and np.isnan(got[2]) and got[0] == 1 and got[3] == 1
    with pytest.raises(HipError):
        hip.matvec_rows(99, buf, 34, act, 32, 0, 1, y=y)


def test_tier_table_and_selftest(hip):
    assert hip.tier() == "hip"
    assert hip.selftest_failures() == 0
    k, got = hip.kernel_table()
    assert got == 6


def test_tier_table_host_entries(hip):
    """The reference tier ABI entries (host pointers) return the oracle's bits."""
    import ctypes as C
    k, _ = hip.kernel_table()
    rng = np.random.default_rng(42)
    for dt, qk in [(oracle.Q6_K, 6), (oracle.Q8_0, 3), (oracle.Q4_K, 4), (oracle.Q5_K, 5), (oracle.Q8_K, 9)]:
        n = 1024
        W = np.stack([make_wrow(rng, dt, n, m % 5) for m in range(9)])
        act = make_act(rng, dt, n, 0)
        want = oracle.matvec_rows(dt, W, W.shape[1], act, n, 0, 9)
        y = np.zeros(9, np.float32)
        k.mv[qk](W.ctypes.data, W.shape[1], act.ctypes.data, y.ctypes.data, n, 9)
        assert np.all(same(y, want)), dt
        d0 = k.dot[qk](W[4].ctypes.data, act.ctypes.data, n, None)
        assert same(d0, want[4])
    n = 1003
    W = rng.standard_normal((9, n)).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    want = oracle.matvec_rows(oracle.F32, W.view(np.uint8), 4 * n, x, n, 0, 9)
    y = np.zeros(9, np.float32)
    k.mv[0](W.ctypes.data, 4 * n, x.ctypes.data, y.ctypes.data, n, 9)
    assert np.all(same(y, want))
    _ = C


def test_mv_job_segments(hip, dev):
    """Several matrices in one job == separate matvecs (each row by one group)."""
    rng = np.random.default_rng(11)
    segs, wants, keep = [], [], []
    for dt, rows, n, packed in [(oracle.Q6_K, 64, 512, 1), (oracle.Q8_0, 48, 512, 1), (oracle.Q4_K, 32, 256, 0),
                                (oracle.Q6_K, 20, 768, 0), (oracle.F32, 8, 512, 0)]:
        if dt == oracle.F32:
            W = rng.standard_normal((rows, n)).astype(np.float32).view(np.uint8)
            act = rng.standard_normal(n).astype(np.float32)
            want = oracle.matvec_rows(dt, W, 4 * n, act, n, 0, rows)
        else:
            W = random_code_rows(rng, dt, rows, n)
            act = oracle.quantize_act(oracle.act_kind_for(dt), rng.standard_normal(n).astype(np.float32))
            want = oracle.matvec_rows(dt, W, W.shape[1], act, n, 0, rows)
        Wd = to_dev(W, dev)
        if packed:
            Wd = hip.pack(dt, Wd, W.shape[1], rows, n)
        y = torch.zeros(rows, device=dev)
        ad = to_dev(act, dev)
        keep += [Wd, ad, y]
        segs.append(dict(dt=dt, packed=packed, W=Wd, row_bytes=W.shape[1] if W.ndim == 2 else 4 * n, act=ad, y=y,
                         n=n, rows=rows))
        wants.append(want)
    hip.mv_job(segs)
    torch.cuda.synchronize()
    for s, want in zip(segs, wants):
        assert np.all(same(s["y"].cpu().numpy(), want))


def test_mv_job_one_launch_any_mix(hip, dev):
    """30 segments (more than one launch's 24): every format packed and plain,
    the mid Q8_0 tile (2048 columns), f32 rows at an unaligned offset, a
    segment of zero rows; each equals its separate matvec bit for bit.  A
    segment with a bad dtype is NaN-filled and reported while the others run
    (tlm_matvec_rows' rule, src/lib/tlm_quant.c:1119-1127)."""
    from tierlm_amd._lib import HipError
    rng = np.random.default_rng(12)
    specs = [(oracle.Q6_K, 40, 512, 1), (oracle.Q8_0, 33, 2048, 1), (oracle.Q5_K, 17, 768, 1),
             (oracle.Q4_K, 50, 256, 1), (oracle.Q8_K, 9, 512, 1), (oracle.Q8_0, 21, 256, 0),
             (oracle.Q5_K, 6, 512, 0), (oracle.Q8_K, 5, 256, 0), (oracle.F32, 11, 96, 0), (oracle.F32, 7, 64, 2)]
    specs = (specs * 3)[:30]
    segs, wants, keep = [], [], []
    for k, (dt, rows, n, packed) in enumerate(specs):
        if dt == oracle.F32:
            off = 1 if packed == 2 else 0          # packed == 2 here: f32 rows one byte off alignment
            W = rng.standard_normal((rows, n)).astype(np.float32).view(np.uint8)
            act = rng.standard_normal(n).astype(np.float32)
            want = oracle.matvec_rows(dt, W, 4 * n, act, n, 0, rows)
            raw = torch.from_numpy(np.concatenate([np.zeros(off, np.uint8), W.reshape(-1)])).to(dev)
            Wd, rb, pk = raw[off:], 4 * n, 0
        else:
            W = random_code_rows(rng, dt, rows, n)
            act = oracle.quantize_act(oracle.act_kind_for(dt), rng.standard_normal(n).astype(np.float32))
            want = oracle.matvec_rows(dt, W, W.shape[1], act, n, 0, rows)
            Wd, rb, pk = to_dev(W, dev), W.shape[1], packed
            if packed:
                Wd = hip.pack(dt, Wd, W.shape[1], rows, n)
        r = 0 if k == 3 else rows                  # one segment with no rows
        y = torch.zeros(rows, device=dev)
        ad = to_dev(act, dev)
        keep += [Wd, ad, y]
        segs.append(dict(dt=dt, packed=pk, W=Wd, row_bytes=rb, act=ad, y=y, n=n, rows=r))
        wants.append(want if r else np.zeros(rows, np.float32))
    hip.mv_job(segs)
    torch.cuda.synchronize()
    for k, (sg, want) in enumerate(zip(segs, wants)):
        assert np.all(same(sg["y"].cpu().numpy(), want)), k
    bad = dict(segs[0], dt=7, y=torch.zeros(40, device=dev))     # 7: not a dtype of the path
    good = dict(segs[1], y=torch.zeros(33, device=dev))
    with pytest.raises(HipError):
        hip.mv_job([bad, good])
    torch.cuda.synchronize()
    assert np.isnan(bad["y"].cpu().numpy()).all()
    assert np.all(same(good["y"].cpu().numpy(), wants[1]))


def pack_layout_host(dt, W, rows, n):
    """The packed tile layout written out in numpy: unit u = (t*nb + b)*16 + i
    holds row t*16 + i, block b (Q6_K bytes 0..207, Q8_0 codes, other formats
    the whole block), rows past the matrix as zeros; Q6_K / Q8_0 then carry an
    f16 d plane of 2 bytes per unit."""
    bv, bb = oracle.BLOCK[dt]
    nb = n // bv
    T = (rows + 15) // 16
    blocks = np.zeros((T * 16, nb, bb), np.uint8)
    blocks[:rows] = W.reshape(rows, nb, bb)
    units = blocks.reshape(T, 16, nb, bb).transpose(0, 2, 1, 3).reshape(-1, bb)
    if dt == oracle.Q6_K:
        return np.concatenate([units[:, :208].reshape(-1), units[:, 208:210].reshape(-1)])
    if dt == oracle.Q8_0:
        return np.concatenate([units[:, 2:34].reshape(-1), units[:, 0:2].reshape(-1)])
    return units.reshape(-1)


@pytest.mark.parametrize("dt", [oracle.Q8_0, oracle.Q4_K, oracle.Q5_K, oracle.Q6_K, oracle.Q8_K])
@pytest.mark.parametrize("rows,n,offset", [(16, 256, 0), (37, 512, 1), (130, 768, 6), (1, 256, 3)])
def test_pack_layout(hip, dev, dt, rows, n, offset):
    rng = np.random.default_rng(rows * 7 + dt)
    W = rng.integers(0, 256, size=(rows, oracle.row_bytes(dt, n)), dtype=np.uint8)
    raw = np.concatenate([np.full(offset, 0xEE, np.uint8), W.reshape(-1)])
    Wd = torch.from_numpy(raw).to(dev)
    out = hip.pack(dt, Wd[offset:], W.shape[1], rows, n).cpu().numpy()
    want = pack_layout_host(dt, W, rows, n)
    assert np.array_equal(out[:want.size], want)
