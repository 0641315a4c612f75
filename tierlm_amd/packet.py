"""Compiled model stores (the reference's .tlmm manifest + .tlmp packet files)
through the library's reader (tlm_hip_manifest_*, tlm_hip_packet_read,
tlm_hip_dir_find).  ``Manifest`` computes nothing; it hands out packet
records, verified payload bytes and tensor-directory entries."""
import ctypes as C

import numpy as np

from ._lib import PacketLoc, TensorRef, check, lib

PK_DENSE, PK_EXPERT, PK_EMBED, PK_META = 1, 2, 5, 7
LAYER_NONE = 0xFFFF


class Manifest:
    def __init__(self, path):
        h = C.c_void_p()
        check(lib.tlm_hip_manifest_load(str(path).encode(), C.byref(h)))
        self.h = h
        self.geom = lib.tlm_hip_manifest_geom(h).contents
        self.name = lib.tlm_hip_manifest_name(h).decode()

    def close(self):
        if self.h:
            lib.tlm_hip_manifest_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def packets(self):
        return [lib.tlm_hip_manifest_packet(self.h, i).contents for i in range(lib.tlm_hip_manifest_n_packets(self.h))]

    def find(self, type_, layer, id_=0):
        p = lib.tlm_hip_manifest_find(self.h, type_, layer, id_)
        return p.contents if p else None

    def read(self, loc):
        """(whole packet bytes, payload view) after the header, length and CRC checks."""
        buf = np.empty(loc.total_len, np.uint8)
        off, plen = C.c_uint64(), C.c_uint64()
        check(lib.tlm_hip_packet_read(self.h, C.byref(loc), buf.ctypes.data, C.byref(off), C.byref(plen)))
        return buf, buf[off.value:off.value + plen.value]

    @staticmethod
    def header(buf):
        dt, off = C.c_uint32(), (C.c_uint32 * 3)()
        check(lib.tlm_hip_packet_header(buf.ctypes.data, C.byref(dt), off))
        return dt.value, list(off)

    @staticmethod
    def tensor(payload, name):
        """(TensorRef, bytes) of a tensor-directory entry, or None if absent."""
        t = TensorRef()
        rc = lib.tlm_hip_dir_find(payload.ctypes.data, payload.nbytes, name.encode(), C.byref(t))
        if rc == -6:
            return None
        check(rc)
        return t, payload[t.offset:t.offset + t.nbytes]
