"""e^x as the reference evaluates it: libm's expf (silu / sigmoidf_,
src/lib/tlm_model.c:171-172; the routing softmax :823; the attention softmax
:705).  glibc's expf is not correctly rounded (about 8 results in 10^5 differ
from exp in double rounded to float), so the device restates its published
algorithm (N = 32 table of 2^(i/N), cubic, the shift step fused as the x86-64
FMA build fuses it) and is held to libm bit for bit.

CPU: the table against 2^(i/32) from exact arithmetic; the oracle's
restatement against libm over a strided sweep of every float bit pattern plus
the overflow / underflow edges, and the unfused variant shown to differ (two
inputs in 2^32, both kept here).  GPU: tlm_hip_expf against libm over a
strided sweep and the same edges."""
import decimal
import struct

import numpy as np
import pytest

import oracle

H = float.fromhex
HARD = np.array([H("0x1.04845ep+5"), H("-0x1.f8cbb2p+5")], np.float32)   # differ unless the shift is fused
EDGES = np.array([H("0x1.62e42ep6"), H("0x1.62e430p6"), H("-0x1.9fe368p6"), H("-0x1.9fe366p6"), 0.0, -0.0,
                  np.inf, -np.inf, 1e-45, -1e-45, 88.0, -87.0, -103.0], np.float32)


def sweep(stride, start=0):
    u = np.arange(start, 1 << 32, stride, dtype=np.uint64).astype(np.uint32)
    return u.view(np.float32)


def same(a, b):
    return (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))


def test_exp2_table_from_exact_arithmetic():
    decimal.getcontext().prec = 60
    for i in range(32):
        v = float(decimal.Decimal(2) ** (decimal.Decimal(i) / 32))
        bits = struct.unpack("<Q", struct.pack("<d", v))[0]
        assert oracle.orc.orc_exp2_tab(i) == (bits - ((i << 52) // 32)) & ((1 << 64) - 1), i


def test_published_expf_equals_libm():
    for x in (sweep(97), sweep(89, 13), HARD, EDGES):
        assert same(oracle.expf_published(x), oracle.expf(x)).all()
    # the unfused shift is the planted mistake: it misses exactly these two
    assert not same(oracle.expf_published(HARD, fused=False), oracle.expf(HARD)).any()


@pytest.mark.gpu
def test_device_expf_equals_libm(hip, dev):
    import ctypes as C

    import torch

    from tierlm_amd._lib import check, lib
    xs = np.concatenate([sweep(61), sweep(4099, 7), HARD, EDGES])
    chunk = 1 << 24
    bad = 0
    for c0 in range(0, xs.size, chunk):
        x = xs[c0:c0 + chunk]
        xd = torch.from_numpy(x).to(dev)
        yd = torch.empty_like(xd)
        check(lib.tlm_hip_expf(C.c_void_p(xd.data_ptr()), C.c_void_p(yd.data_ptr()), x.size, None))
        torch.cuda.synchronize()
        bad += int((~same(yd.cpu().numpy(), oracle.expf(x))).sum())
    assert bad == 0, f"{bad} of {xs.size} device results differ from libm expf"
