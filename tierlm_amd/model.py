"""The whole decode step on the device (tlm_hip_model_*; the reference's
tlm_model_step / tlm_model_prefill, src/lib/tlm_model.c:1058-1113) for a
compiled store, through ctypes.  Computes nothing itself."""
import ctypes as C

import numpy as np

from ._lib import check, lib


class ModelOpts(C.Structure):
    """tlm_hip_model_opts"""
    _fields_ = [("max_ctx", C.c_int32), ("eager", C.c_int32)]


class Model:
    def __init__(self, manifest_path, max_ctx=0, eager=False):
        self.opts = ModelOpts(max_ctx, int(eager))
        h = C.c_void_p()
        check(lib.tlm_hip_model_open(str(manifest_path).encode(), C.byref(self.opts), C.byref(h)))
        self.h = h
        self.geom = lib.tlm_hip_model_geom_of(h).contents

    def close(self):
        if self.h:
            lib.tlm_hip_model_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        lib.tlm_hip_model_reset(self.h)

    def kv_len(self):
        return lib.tlm_hip_model_kv_len(self.h)

    def step(self, token, logits=True):
        """One token; returns (logits as float32 [vocab] or None, greedy next token)."""
        lg = np.empty(self.geom.vocab, np.float32) if logits else None
        nxt = C.c_int32()
        check(lib.tlm_hip_model_step(self.h, int(token), lg.ctypes.data if logits else None, C.byref(nxt)))
        return lg, nxt.value

    def generate(self, prompt, n):
        p = (C.c_int32 * len(prompt))(*prompt)
        out = (C.c_int32 * max(n, 1))()
        check(lib.tlm_hip_model_generate(self.h, p, len(prompt), n, out))
        return list(out[:n])
