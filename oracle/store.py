"""Expert slot cache policy, two CPU implementations behind one interface
(TEST INFRASTRUCTURE ONLY):

  OracleStore - this repository's restatement (tlm_oracle_store.c)
  RefStore    - the reference's own tlm_store.c over a packet-store fixture
                (ref_store.c), when oracle/_ref is built

Both take the same experts: ``experts`` is a list of dicts with layer, id and
optional flags (bit0 compiler pin, bit1 pruned), heat and seed.  Acquires
return a group: the slots of the call's ids (-1 = not acquired), kept for
wait / is_ready / release by index.
"""
import ctypes as C
import os
import tempfile

from . import orc, ref

vp, i32 = C.c_void_p, C.c_int
I32P = C.POINTER(C.c_int32)

STATS = ("hits", "misses", "prefetch_issued", "prefetch_used", "prefetch_dropped", "evictions", "loads",
         "slots", "pinned", "in_use")


class OStoreSrc(C.Structure):
    _fields_ = [("layer", C.c_uint16), ("id", C.c_uint32), ("flags", C.c_uint16), ("heat", C.c_float),
                ("seed", C.c_uint32)]


class OStoreStats(C.Structure):
    _fields_ = [("hits", C.c_uint64), ("misses", C.c_uint64), ("prefetch_issued", C.c_uint64),
                ("prefetch_used", C.c_uint64), ("prefetch_dropped", C.c_uint64), ("loads", C.c_uint64),
                ("evictions", C.c_uint64), ("slots", C.c_int32), ("pinned", C.c_int32), ("in_use", C.c_int32)]


for _n, _r, _a in [
    ("ostore_open", vp, [C.POINTER(OStoreSrc), i32, i32, i32, C.c_double, i32]),
    ("ostore_close", None, [vp]), ("ostore_n_slots", i32, [vp]), ("ostore_warm", i32, [vp]),
    ("ostore_acquire", i32, [vp, i32, I32P, i32, I32P]), ("ostore_wait", i32, [vp, i32]),
    ("ostore_is_ready", i32, [vp, i32]), ("ostore_release", None, [vp, i32]),
    ("ostore_prefetch", None, [vp, i32, I32P, i32]), ("ostore_tick", None, [vp]), ("ostore_settle", None, [vp]),
    ("ostore_get_stats", None, [vp, C.POINTER(OStoreStats)]), ("ostore_set_fail", None, [vp, i32, i32, i32]),
    ("ostore_slot_expert", C.c_int64, [vp, i32]),
]:
    _f = getattr(orc, _n)
    _f.restype, _f.argtypes = _r, _a


def _ids(ids):
    return (C.c_int32 * max(len(ids), 1))(*ids)


class OracleStore:
    def __init__(self, experts, top_k, n_slots, pin_frac=0.0, prefetch=1):
        src = (OStoreSrc * max(len(experts), 1))()
        for i, x in enumerate(experts):
            src[i] = OStoreSrc(x["layer"], x["id"], x.get("flags", 0), x.get("heat", 0.0), x.get("seed", 0))
        self.h = orc.ostore_open(src, len(experts), top_k, n_slots, pin_frac, prefetch)

    def close(self):
        if self.h:
            orc.ostore_close(self.h)
            self.h = None

    def n_slots(self):
        return orc.ostore_n_slots(self.h)

    def warm(self):
        return orc.ostore_warm(self.h)

    def acquire(self, layer, ids):
        out = (C.c_int32 * max(len(ids), 1))()
        rc = orc.ostore_acquire(self.h, layer, _ids(ids), len(ids), out)
        return rc, list(out[:len(ids)])

    def wait(self, group, j):
        return orc.ostore_wait(self.h, group[j])

    def is_ready(self, group, j):
        return bool(orc.ostore_is_ready(self.h, group[j]))

    def release(self, group, j):
        orc.ostore_release(self.h, group[j])

    def prefetch(self, layer, ids):
        orc.ostore_prefetch(self.h, layer, _ids(ids), len(ids))

    def tick(self):
        orc.ostore_tick(self.h)

    def settle(self):
        orc.ostore_settle(self.h)

    def set_fail(self, layer, eid, on):
        orc.ostore_set_fail(self.h, layer, eid, int(on))

    @staticmethod
    def slots_of(group, n):
        return list(group[:n])

    def stats(self):
        st = OStoreStats()
        orc.ostore_get_stats(self.h, C.byref(st))
        return {k: int(getattr(st, k)) for k in STATS}


class TlmExpertRef(C.Structure):
    """tlm_expert_ref (src/lib/tlm_store.h:34-38)"""
    _fields_ = [("slot", C.c_int), ("payload", vp), ("payload_len", C.c_uint64)]


class TlmStoreStats(C.Structure):
    """tlm_store_stats (src/lib/tlm_store.h:66-70)"""
    _fields_ = [("hits", C.c_uint64), ("misses", C.c_uint64), ("prefetch_issued", C.c_uint64),
                ("prefetch_used", C.c_uint64), ("prefetch_dropped", C.c_uint64), ("bytes_read", C.c_uint64),
                ("evictions", C.c_uint64), ("wait_ns", C.c_uint64), ("slots", C.c_int), ("pinned", C.c_int),
                ("in_use", C.c_int)]


if ref is not None:
    RP = C.POINTER(TlmExpertRef)
    for _n, _r, _a in [
        ("ref_store_fixture", vp, [C.c_char_p, i32, i32, i32, vp, vp, C.c_uint64, i32, C.c_double, i32]),
        ("ref_store_handle", vp, [vp]), ("ref_store_settle", None, [vp]), ("ref_store_corrupt", i32, [vp, i32, i32]),
        ("ref_store_fixture_close", None, [vp]),
        ("tlm_store_warm", i32, [vp]), ("tlm_store_acquire", i32, [vp, i32, I32P, i32, RP]),
        ("tlm_store_wait", i32, [vp, RP]), ("tlm_store_is_ready", i32, [vp, RP]),
        ("tlm_store_release", None, [vp, RP]), ("tlm_store_prefetch", None, [vp, i32, I32P, i32]),
        ("tlm_store_tick", None, [vp]), ("tlm_store_get_stats", None, [vp, C.POINTER(TlmStoreStats)]),
        ("tlm_store_n_slots", i32, [vp]), ("tlm_store_slot_bytes", C.c_uint64, [vp]),
        ("tlm_log_level", None, [i32]),
    ]:
        _f = getattr(ref, _n)
        _f.restype, _f.argtypes = _r, _a


class RefStore:
    """The reference's store over a one-drive fixture of n_layers x n_experts
    packets of payload_len bytes; experts absent from ``experts`` are written
    as pruned packets (flags bit1)."""

    def __init__(self, experts, top_k, n_slots, pin_frac=0.0, prefetch=1, n_layers=None, n_experts=None,
                 payload_len=3000):
        assert ref is not None, "oracle/_ref not built"
        nl = n_layers or (max(x["layer"] for x in experts) + 1)
        ne = n_experts or (max(x["id"] for x in experts) + 1)
        flags = (C.c_uint16 * (nl * ne))(*([2] * (nl * ne)))
        heat = (C.c_float * (nl * ne))()
        for x in experts:
            assert not x.get("seed"), "the fixture carries no warm sidecar"
            flags[x["layer"] * ne + x["id"]] = x.get("flags", 0)
            heat[x["layer"] * ne + x["id"]] = x.get("heat", 0.0)
        self.tmp = tempfile.TemporaryDirectory(prefix="tlmref-store-")
        ref.tlm_log_level(0)   # errors only: failed loads log by design
        self.fx = ref.ref_store_fixture(self.tmp.name.encode(), nl, ne, top_k, C.cast(flags, vp), C.cast(heat, vp),
                                        payload_len, n_slots, pin_frac, prefetch)
        assert self.fx, "reference fixture failed"
        self.s = ref.ref_store_handle(self.fx)
        self.slot_bytes = ref.tlm_store_slot_bytes(self.s)
        self.failing = set()

    def close(self):
        if self.fx:
            for le in list(self.failing):
                self.set_fail(*le, False)
            ref.ref_store_fixture_close(self.fx)
            self.fx = None
            self.tmp.cleanup()

    def n_slots(self):
        return ref.tlm_store_n_slots(self.s)

    def warm(self):
        return ref.tlm_store_warm(self.s)

    def acquire(self, layer, ids):
        refs = (TlmExpertRef * max(len(ids), 1))()
        rc = ref.tlm_store_acquire(self.s, layer, _ids(ids), len(ids), refs)
        return rc, refs

    def wait(self, group, j):
        return ref.tlm_store_wait(self.s, C.byref(group[j]))

    def is_ready(self, group, j):
        return bool(ref.tlm_store_is_ready(self.s, C.byref(group[j])))

    def release(self, group, j):
        ref.tlm_store_release(self.s, C.byref(group[j]))

    def prefetch(self, layer, ids):
        ref.tlm_store_prefetch(self.s, layer, _ids(ids), len(ids))

    def tick(self):
        ref.tlm_store_tick(self.s)

    def settle(self):
        ref.ref_store_settle(self.fx)

    def set_fail(self, layer, eid, on):
        if bool(on) != ((layer, eid) in self.failing):
            assert ref.ref_store_corrupt(self.fx, layer, eid) == 0
            (self.failing.add if on else self.failing.discard)((layer, eid))

    def stats(self):
        st = TlmStoreStats()
        ref.tlm_store_get_stats(self.s, C.byref(st))
        d = {k: int(getattr(st, k)) for k in STATS if k != "loads"}
        d["loads"] = int(st.bytes_read) // int(self.slot_bytes)
        return d

    @staticmethod
    def slots_of(group, n):
        return [group[j].slot for j in range(n)]
