"""Python binding of the oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only to check or time against the HIP path.

  orc  - liboracle.so, this repository's C restatement (tlm_oracle.c)
  ref  - _ref/libtlmref.so, the reference's own tlm_quant / kernel tiers /
         pool compiled from its sources (None when not built), plus ref_moe.c
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORC_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libtlmref.so")

F32, F16, BF16, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K = 0, 1, 2, 8, 12, 13, 14, 15
BLOCK = {F32: (1, 4), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210),
         Q8_K: (256, 292)}
INT_TYPES = (Q8_0, Q4_K, Q5_K, Q6_K, Q8_K)

vp, i32, i64, sz, f32 = C.c_void_p, C.c_int, C.c_int64, C.c_size_t, C.c_float


class OrcMoeDesc(C.Structure):
    """orc_moe_desc (tlm_oracle.h)"""
    _fields_ = [("D", C.c_int64), ("de", C.c_int64), ("ds", C.c_int64),
                ("E", C.c_int), ("k", C.c_int), ("router", C.c_int),
                ("routed_scale", C.c_float), ("eps", C.c_float),
                ("ffn_norm", vp), ("router_dt", C.c_int), ("router_w", vp), ("router_bias", vp),
                ("mask", vp), ("expert_dt", C.c_int), ("gate", vp), ("up", vp), ("down", vp),
                ("shared_dt", C.c_int), ("sg", vp), ("su", vp), ("sd", vp), ("shared_gate_inp", vp)]


class OrcMoeTrace(C.Structure):
    _fields_ = [("xb", vp), ("logits", vp), ("gu", vp), ("hh", vp), ("hq", vp), ("eo", vp),
                ("s_out", vp), ("ffn", vp)]


def _load(path, required):
    if not os.path.exists(path):
        if required:
            raise ImportError(f"oracle: {path} not built; run `make -C oracle` (or __graft_entry__.build())")
        return None
    return C.CDLL(path)


orc = _load(ORC_PATH, True)
ref = _load(REF_PATH, False)

for _n, _r, _a in [
    ("orc_row_bytes", sz, [i32, i64]), ("orc_qact_bytes", sz, [i32, i64]),
    ("orc_act_kind_for", i32, [i32]), ("orc_f16_to_f32", f32, [C.c_uint16]),
    ("orc_f32_to_f16", C.c_uint16, [f32]), ("orc_quantize_row", i32, [i32, vp, vp, i64]),
    ("orc_dequantize_row", i32, [i32, vp, vp, i64]), ("orc_quantize_act", None, [i32, vp, i64, vp]),
    ("orc_vec_dot", f32, [i32, vp, vp, i64]),
    ("orc_matvec_rows", None, [i32, vp, sz, vp, vp, i64, i64, i64]),
    ("orc_block_isum", None, [i32, vp, vp, C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    ("orc_rmsnorm", None, [vp, vp, vp, i64, f32]), ("orc_silu", f32, [f32]), ("orc_sigmoid", f32, [f32]),
    ("orc_expf_many", None, [vp, vp, i64]), ("orc_exp2_tab", C.c_uint64, [i32]),
    ("orc_expf_published_many", None, [vp, vp, i64, i32]),
    ("orc_topk", None, [vp, vp, i32, i32, vp]),
    ("orc_route", None, [i32, vp, vp, vp, i32, i32, f32, vp, vp]),
    ("orc_moe_layer", i32, [C.POINTER(OrcMoeDesc), vp, vp, vp, C.POINTER(OrcMoeTrace)]),
]:
    _f = getattr(orc, _n)
    _f.restype, _f.argtypes = _r, _a

if ref is not None:
    for _n, _r, _a in [
        ("tlm_row_bytes", sz, [i32, i64]), ("tlm_qact_bytes", sz, [i32, i64]),
        ("tlm_f16_to_f32", f32, [C.c_uint16]), ("tlm_f32_to_f16", C.c_uint16, [f32]),
        ("tlm_quantize_row", i32, [i32, vp, vp, i64]), ("tlm_dequantize_row", i32, [i32, vp, vp, i64]),
        ("tlm_quantize_act", None, [i32, vp, i64, vp]), ("tlm_vec_dot", f32, [i32, vp, vp, i64]),
        ("tlm_matvec_rows", None, [i32, vp, sz, vp, vp, i64, i64, i64, vp]),
        ("tlm_quant_tier", C.c_char_p, []), ("tlm_quant_init", None, []),
        ("tlm_cpu_force", None, [C.c_char_p]), ("tlm_quant_selftest_failures", i32, []),
        ("refmoe_new", vp, [i32]), ("refmoe_free", None, [vp]), ("refmoe_tier", C.c_char_p, []),
        ("refmoe_force_tier", None, [C.c_char_p]),
        ("refmoe_layer", i32, [vp, C.POINTER(OrcMoeDesc), vp, vp, vp]),
        ("refmoe_matvecs", None, [vp, i32, vp, vp, i64, vp, vp, i32]),
    ]:
        _f = getattr(ref, _n)
        _f.restype, _f.argtypes = _r, _a


def _p(a):
    return C.c_void_p(a.ctypes.data) if a is not None else None


def row_bytes(dt, n):
    return int(orc.orc_row_bytes(dt, n))


def qact_bytes(kind, n):
    return int(orc.orc_qact_bytes(kind, n))


def act_kind_for(dt):
    return int(orc.orc_act_kind_for(dt))


def f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def quantize_row(dt, x, use_ref=False):
    """float32 [rows, n] or [n] -> uint8 packed rows (reference byte layout)."""
    x = f32(x)
    shp = x.shape
    n = shp[-1]
    rows = int(np.prod(shp[:-1])) if len(shp) > 1 else 1
    rb = row_bytes(dt, n)
    out = np.zeros((rows, rb), np.uint8)
    xr = x.reshape(rows, n)
    q = ref.tlm_quantize_row if use_ref else orc.orc_quantize_row
    for r in range(rows):
        rc = q(dt, xr[r].ctypes.data, out[r].ctypes.data, n)
        if rc != 0:
            raise ValueError(f"quantize_row({dt}, n={n}) -> {rc}")
    return out.reshape(shp[:-1] + (rb,)) if len(shp) > 1 else out[0]


def dequantize_row(dt, w, n, use_ref=False):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    y = np.zeros(n, np.float32)
    fn = ref.tlm_dequantize_row if use_ref else orc.orc_dequantize_row
    fn(dt, w.ctypes.data, y.ctypes.data, n)
    return y


def quantize_act(kind, x, use_ref=False):
    x = f32(x)
    n = x.size
    out = np.zeros(max(qact_bytes(kind, n), 4), np.uint8)
    fn = ref.tlm_quantize_act if use_ref else orc.orc_quantize_act
    fn(kind, x.ctypes.data, n, out.ctypes.data)
    return out


def vec_dot(dt, w, act, n, use_ref=False):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    act = np.ascontiguousarray(act)
    fn = ref.tlm_vec_dot if use_ref else orc.orc_vec_dot
    return np.float32(fn(dt, w.ctypes.data, act.ctypes.data, n))


def matvec_rows(dt, W, rb, act, n, r0, r1, nrows=None, use_ref=False, offset=0):
    """W: uint8 buffer; rows start `offset` bytes in, stride rb.  Returns y
    (length nrows or r1) with untouched rows left at -12345."""
    W = np.ascontiguousarray(W, dtype=np.uint8)
    act = np.ascontiguousarray(act)
    y = np.full(nrows if nrows is not None else max(r1, 1), -12345.0, np.float32)
    base = W.ctypes.data + offset
    if use_ref:
        ref.tlm_matvec_rows(dt, base, rb, act.ctypes.data, y.ctypes.data, n, r0, r1, None)
    else:
        orc.orc_matvec_rows(dt, base, rb, act.ctypes.data, y.ctypes.data, n, r0, r1)
    return y


def block_isum(dt, wblock, ablock):
    wblock = np.ascontiguousarray(wblock, dtype=np.uint8)
    ablock = np.ascontiguousarray(ablock, dtype=np.uint8)
    a, b = C.c_int32(), C.c_int32()
    orc.orc_block_isum(dt, wblock.ctypes.data, ablock.ctypes.data, C.byref(a), C.byref(b))
    return a.value, b.value


def expf(x):
    """libm's expf over a float32 array (the reference's e^x)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    orc.orc_expf_many(_p(x), _p(y), x.size)
    return y


def expf_published(x, fused=True):
    """The published expf algorithm restated (orc_expf_published)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    orc.orc_expf_published_many(_p(x), _p(y), x.size, int(fused))
    return y


def rmsnorm(x, w, eps):
    x, w = f32(x), f32(w)
    out = np.zeros_like(x)
    orc.orc_rmsnorm(out.ctypes.data, x.ctypes.data, w.ctypes.data, x.size, eps)
    return out


def topk(v, k, mask=None):
    v = f32(v)
    ids = np.zeros(k, np.int32)
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
    orc.orc_topk(v.ctypes.data, _p(m), v.size, k, ids.ctypes.data)
    return ids


def route(router, logits, k, routed_scale=1.0, mask=None, bias=None):
    logits = f32(logits)
    ids = np.zeros(k, np.int32)
    w = np.zeros(k, np.float32)
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
    b = None if bias is None else f32(bias)
    orc.orc_route(router, logits.ctypes.data, _p(m), _p(b), logits.size, k, routed_scale,
                  ids.ctypes.data, w.ctypes.data)
    return ids, w


class MoeHost:
    """Host-side MoE block description for orc_moe_layer / refmoe_layer.

    experts: list of (gate, up, down) uint8 arrays in the reference layout."""

    def __init__(self, *, D, de, E, k, expert_dt, ffn_norm, router_w, experts, router=0,
                 routed_scale=1.0, eps=1e-6, router_bias=None, mask=None, ds=0, shared_dt=0,
                 shared=None, shared_gate_inp=None):
        self.keep = []

        def keep(a):
            if a is None:
                return None
            self.keep.append(a)
            return a.ctypes.data

        ptrs = [np.ascontiguousarray(m, dtype=np.uint8) for trip in experts for m in trip]
        self.keep.extend(ptrs)
        g = (C.c_void_p * E)(*[ptrs[3 * e].ctypes.data for e in range(E)])
        u = (C.c_void_p * E)(*[ptrs[3 * e + 1].ctypes.data for e in range(E)])
        dn = (C.c_void_p * E)(*[ptrs[3 * e + 2].ctypes.data for e in range(E)])
        self.keep.extend([g, u, dn])
        sg = su = sd = None
        if shared is not None:
            sg, su, sd = [np.ascontiguousarray(m, dtype=np.uint8) for m in shared]
        self.desc = OrcMoeDesc(D, de, ds, E, k, router, routed_scale, eps, keep(f32(ffn_norm)), F32,
                               keep(f32(router_w)), keep(None if router_bias is None else f32(router_bias)),
                               keep(None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)),
                               expert_dt, C.cast(g, C.c_void_p), C.cast(u, C.c_void_p), C.cast(dn, C.c_void_p),
                               shared_dt, keep(sg), keep(su), keep(sd),
                               keep(None if shared_gate_inp is None else f32(shared_gate_inp)))
        self.D, self.de, self.ds, self.E, self.k = D, de, ds, E, k
        self.expert_dt, self.shared_dt = expert_dt, shared_dt

    def run(self, h, trace=False):
        """Returns (h_out, ids, w, trace dict or None)."""
        h = f32(h).copy()
        ids = np.zeros(self.k, np.int32)
        w = np.zeros(self.k, np.float32)
        tr = None
        trs = None
        if trace:
            ek = act_kind_for(self.expert_dt)
            hqb = qact_bytes(ek, self.de)
            tr = dict(xb=np.zeros(self.D, np.float32), logits=np.zeros(self.E, np.float32),
                      gu=np.zeros((self.k, 2 * self.de), np.float32), hh=np.zeros((self.k, self.de), np.float32),
                      hq=np.zeros((self.k, max(hqb, 4)), np.uint8), eo=np.zeros((self.k, self.D), np.float32),
                      s_out=np.zeros(self.D, np.float32), ffn=np.zeros(self.D, np.float32))
            trs = OrcMoeTrace(*[tr[f].ctypes.data for f in ("xb", "logits", "gu", "hh", "hq", "eo", "s_out", "ffn")])
        orc.orc_moe_layer(C.byref(self.desc), h.ctypes.data, ids.ctypes.data, w.ctypes.data,
                          C.byref(trs) if trs is not None else None)
        return h, ids, w, tr

    def run_ref(self, handle, h):
        """The same block through the compiled reference's kernels (ref_moe.c)."""
        h = f32(h).copy()
        ids = np.zeros(self.k, np.int32)
        w = np.zeros(self.k, np.float32)
        ref.refmoe_layer(handle, C.byref(self.desc), h.ctypes.data, ids.ctypes.data, w.ctypes.data)
        return h, ids, w
