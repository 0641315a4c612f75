"""The HBM expert slot cache (tlm_hip_store_*; the reference's RAM cache is
src/lib/tlm_store.c) through ctypes.

``HipStore`` keeps the source table, the host payloads it points at and the
fetch callback alive for the store's lifetime; it computes nothing itself.
Experts are dicts: layer, id, dtype, payload (a host buffer: numpy array or
CPU tensor, pinned or not) or None to use ``fetch``, item_off (gate, up,
down inside the payload), and optional flags / heat / seed.
"""
import ctypes as C

from ._lib import FETCH, ExpertRef, ExpertSrc, StoreOpts, StoreStats, check, lib
from .quant import stream


def _addr(buf):
    if buf is None:
        return None, 0
    if hasattr(buf, "data_ptr"):
        return buf.data_ptr(), buf.numel() * buf.element_size()
    return buf.ctypes.data, buf.nbytes


class HipStore:
    def __init__(self, experts, *, d_model, d_expert, top_k, budget_bytes, pin_frac=0.0, prefetch=1, fetch=None):
        n = len(experts)
        self.src = (ExpertSrc * max(n, 1))()
        self.keep = []
        for i, x in enumerate(experts):
            ptr, nbytes = _addr(x.get("payload"))
            self.keep.append(x.get("payload"))
            self.src[i] = ExpertSrc(x["layer"], x.get("flags", 0), x["id"], x["dtype"], x.get("heat", 0.0),
                                    x.get("seed", 0), (C.c_uint32 * 3)(*x["item_off"]),
                                    x.get("payload_len", nbytes), ptr)
        # the callback object must outlive the store: it is called from the loader thread
        self._fetch = FETCH(fetch) if fetch is not None else FETCH()
        self.opts = StoreOpts(d_model, d_expert, top_k, prefetch, pin_frac, budget_bytes, self._fetch, None)
        h = C.c_void_p()
        check(lib.tlm_hip_store_open(self.src, n, C.byref(self.opts), C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib.tlm_hip_store_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def n_slots(self):
        return lib.tlm_hip_store_n_slots(self.h)

    def slot_bytes(self):
        return int(lib.tlm_hip_store_slot_bytes(self.h))

    def warm(self):
        return lib.tlm_hip_store_warm(self.h)

    def acquire(self, layer, ids):
        refs = (ExpertRef * max(len(ids), 1))()
        arr = (C.c_int * max(len(ids), 1))(*ids)
        rc = lib.tlm_hip_store_acquire(self.h, layer, arr, len(ids), refs)
        return rc, refs

    @staticmethod
    def slots_of(group, n):
        return [group[j].slot for j in range(n)]

    def wait(self, group, j):
        return lib.tlm_hip_store_wait(self.h, C.byref(group[j]))

    def stream_wait(self, group, j, s=None):
        return lib.tlm_hip_store_stream_wait(self.h, C.byref(group[j]), stream() if s is None else s)

    def is_ready(self, group, j):
        return bool(lib.tlm_hip_store_is_ready(self.h, C.byref(group[j])))

    def release(self, group, j, s=None):
        lib.tlm_hip_store_release(self.h, C.byref(group[j]), stream() if s is None else s)

    def prefetch(self, layer, ids):
        arr = (C.c_int * max(len(ids), 1))(*ids)
        lib.tlm_hip_store_prefetch(self.h, layer, arr, len(ids))

    def tick(self):
        lib.tlm_hip_store_tick(self.h)

    def settle(self):
        check(lib.tlm_hip_store_drain(self.h))

    def stats(self):
        st = StoreStats()
        lib.tlm_hip_store_get_stats(self.h, C.byref(st))
        return {f: int(getattr(st, f)) for f, _ in StoreStats._fields_}
