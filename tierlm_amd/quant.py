"""The HIP tier of tlm_quant (src/lib/tlm_quant.h) on device tensors.

Names, argument meaning and error behaviour follow the reference's public
calls: ``quantize_act`` (tlm_quantize_act), ``matvec_rows`` (tlm_matvec_rows,
absolute row indexing into ``y``, NaN-filled rows plus an error on a bad
dtype or length), ``tier`` (tlm_quant_tier), ``init`` (tlm_quant_init) and
``selftest_failures`` (tlm_quant_selftest_failures).  Device memory is torch
tensors on the current HIP device; work goes on torch's current stream.
"""
import ctypes as C

import torch

from ._lib import QuantKernels, Seg, check, lib

F32, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K = 0, 8, 12, 13, 14, 15
# values per block, bytes per block (src/lib/tlm_quant.c:52-63)
BLOCK = {F32: (1, 4), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210),
         Q8_K: (256, 292)}
NAMES = {F32: "f32", Q8_0: "q8_0", Q4_K: "q4_k", Q5_K: "q5_k", Q6_K: "q6_k", Q8_K: "q8_k"}


def act_kind_for(dt):
    """src/lib/tlm_quant.c:709-715"""
    if dt in (Q4_K, Q5_K, Q6_K, Q8_K):
        return Q8_K
    if dt == Q8_0:
        return Q8_0
    return F32


def row_bytes(dt, n):
    """src/lib/tlm_quant.c:106-110 (0 for a bad dtype or length)."""
    if dt not in BLOCK or n < 0 or n % BLOCK[dt][0]:
        return 0
    return n // BLOCK[dt][0] * BLOCK[dt][1]


def qact_bytes(kind, n):
    return int(lib.tlm_hip_qact_bytes(kind, n))


def stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def init(device=0):
    check(lib.tlm_hip_init(device))


def tier():
    return lib.tlm_hip_tier().decode()


def selftest_failures():
    return int(lib.tlm_hip_selftest_failures())


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def quantize_act(kind, x, out=None):
    """f32 device vector -> activation blocks (uint8 device tensor)."""
    assert x.is_cuda and x.dtype == torch.float32 and x.is_contiguous()
    n = x.numel()
    nbytes = qact_bytes(kind, n)
    if out is None:
        out = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=x.device)
    check(lib.tlm_hip_quantize_act(kind, _ptr(x), n, _ptr(out), stream()))
    return out


def matvec_rows(dt, W, rbytes, act, n, r0, r1, y=None, offset=0):
    """y[r] = dot(W row r, act) for r in [r0, r1); W is a uint8 device tensor
    holding rows of ``rbytes`` bytes starting ``offset`` bytes in."""
    if y is None:
        y = torch.zeros(max(r1, 1), dtype=torch.float32, device=W.device)
    check(lib.tlm_hip_matvec_rows(dt, C.c_void_p(W.data_ptr() + offset), rbytes, _ptr(act), _ptr(y),
                                  n, r0, r1, stream()))
    return y


def packed_bytes(dt, rows, n):
    return int(lib.tlm_hip_packed_bytes(dt, rows, n))


def pack(dt, W, rbytes, rows, n, out=None):
    """Plain rows (device) -> packed tile layout (device)."""
    pb = packed_bytes(dt, rows, n)
    if out is None:
        out = torch.empty(max(pb, 16), dtype=torch.uint8, device=W.device)
    check(lib.tlm_hip_pack(dt, _ptr(W), rbytes, rows, n, _ptr(out), stream()))
    return out


def matvec_packed(dt, Wp, rows, n, act, y=None):
    if y is None:
        y = torch.empty(max(rows, 1), dtype=torch.float32, device=Wp.device)
    check(lib.tlm_hip_matvec_packed(dt, _ptr(Wp), rows, n, _ptr(act), _ptr(y), stream()))
    return y


def matmul_tokens(dt, Wp, rows, n, act, ntok, Y=None):
    """Y[t, r] = packed row r . token t's activation (act: ntok consecutive
    activation vectors); the decode result for every token."""
    if Y is None:
        Y = torch.empty((ntok, rows), dtype=torch.float32, device=Wp.device)
    check(lib.tlm_hip_matmul_tokens(dt, _ptr(Wp), rows, n, _ptr(act), ntok, _ptr(Y), stream()))
    return Y


def mv_job(segs):
    """segs: list of dicts with dt, packed, W, row_bytes, act, y, n, rows (tensors)."""
    arr = (Seg * max(len(segs), 1))()
    for i, s in enumerate(segs):
        arr[i] = Seg(s["dt"], int(s.get("packed", 0)), s["W"].data_ptr(), s.get("row_bytes", 0),
                     s["act"].data_ptr(), s["y"].data_ptr(), s["n"], s["rows"])
    check(lib.tlm_hip_mv_job(arr, len(segs), stream()))


def kernel_table():
    """The reference tier table filled with the hip entries (tlm_kern_hip_fill)."""
    k = QuantKernels()
    k.name = b"hip"
    got = lib.tlm_kern_hip_fill(C.byref(k))
    return k, got
