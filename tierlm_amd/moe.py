"""One routed MoE block on device (src/lib/tlm_model.c:940-1055) through
tlm_hip_moe_layer.

``MoeBlock`` owns nothing but the small device tables the C call needs (the
packed-expert pointer table and the workspace); weights are device tensors
the caller keeps alive.  Expert e's packed gate / up / down pointers sit at
table entries 3e, 3e+1, 3e+2.
"""
import ctypes as C

import torch

import numpy as np

from ._lib import MoeDesc, MoeHint, StackOpts, check, lib
from .quant import stream


class MoeBlock:
    def __init__(self, *, D, de, E, k, expert_dt, ffn_norm, router_w, expert_ptrs,
                 router=0, routed_scale=1.0, eps=1e-6, router_bias=None, mask=None,
                 ds=0, shared_dt=0, shared=None, shared_gate_inp=None, device="cuda"):
        self.keep = [ffn_norm, router_w, router_bias, mask, shared, shared_gate_inp]
        assert len(expert_ptrs) == 3 * E
        self.table = torch.tensor(list(expert_ptrs), dtype=torch.int64, device=device)
        sg, su, sd = shared if shared is not None else (None, None, None)

        def p(t):
            return t.data_ptr() if t is not None else None

        self.desc = MoeDesc(D, de, ds, E, k, router, routed_scale, eps, expert_dt, shared_dt,
                            p(ffn_norm), p(router_w), p(router_bias), p(mask), self.table.data_ptr(),
                            p(sg), p(su), p(sd), p(shared_gate_inp))
        nbytes = int(lib.tlm_hip_moe_workspace_bytes(C.byref(self.desc)))
        self.workspace = torch.empty(nbytes, dtype=torch.uint8, device=device)
        self.ids = torch.zeros(max(k, 1), dtype=torch.int32, device=device)
        self.w = torch.zeros(max(k, 1), dtype=torch.float32, device=device)

    def __call__(self, h):
        """h (f32 device [D]) += MoE(h); routing lands in self.ids / self.w."""
        check(lib.tlm_hip_moe_layer(C.byref(self.desc), C.c_void_p(h.data_ptr()),
                                    C.c_void_p(self.ids.data_ptr()), C.c_void_p(self.w.data_ptr()),
                                    C.c_void_p(self.workspace.data_ptr()), stream()))
        return h

    def phase(self, ph, h):
        check(lib.tlm_hip_moe_layer_phase(C.byref(self.desc), ph, C.c_void_p(h.data_ptr()),
                                          C.c_void_p(self.ids.data_ptr()), C.c_void_p(self.w.data_ptr()),
                                          C.c_void_p(self.workspace.data_ptr()), stream()))

    def prefill(self, h, ids=None, w=None):
        """h (f32 device [T, D]): every token's residual += MoE(token), as
        __call__ would give it one token at a time; routing in ids / w [T, k]
        when given.  The prefill workspace is kept per token count."""
        T = h.shape[0]
        ws = self._pf_ws.get(T) if hasattr(self, "_pf_ws") else None
        if ws is None:
            nbytes = int(lib.tlm_hip_moe_prefill_workspace_bytes(C.byref(self.desc), T))
            ws = torch.empty(nbytes, dtype=torch.uint8, device=h.device)
            self._pf_ws = getattr(self, "_pf_ws", {})
            self._pf_ws[T] = ws

        def p(t):
            return C.c_void_p(t.data_ptr()) if t is not None else None
        check(lib.tlm_hip_moe_prefill(C.byref(self.desc), C.c_void_p(h.data_ptr()), T, p(ids), p(w),
                                      C.c_void_p(ws.data_ptr()), stream()))
        return h

    def route(self, h, ids=None, w=None):
        """Routing alone (device ids / w of k entries), as __call__ routes h."""
        ids = self.ids if ids is None else ids
        w = self.w if w is None else w
        check(lib.tlm_hip_moe_route(C.byref(self.desc), C.c_void_p(h.data_ptr()), C.c_void_p(ids.data_ptr()),
                                    C.c_void_p(w.data_ptr()), C.c_void_p(self.workspace.data_ptr()), stream()))
        return ids, w

    def step_store(self, store, layer, h, hints=()):
        """h += MoE(h) with the experts taken from ``store`` (a HipStore over
        this block's geometry): the block's expert table is rewritten for the
        routed experts.  hints: (block, layer, k) lookahead tuples - the
        block's router predicts k experts of that layer.  Returns the routing
        (ids, w) as host lists."""
        n = len(hints)
        # the hint table is built once per (blocks, layers, k) and kept with
        # the descriptors and workspaces it points at
        key = tuple((id(blk), hl, hk) for blk, hl, hk in hints)
        cache = self.__dict__.setdefault("_hint_cache", {})
        if key not in cache:
            arr = (MoeHint * max(n, 1))()
            keep = []
            for i, (blk, hl, hk) in enumerate(hints):
                dsc = MoeDesc.from_buffer_copy(blk.desc)
                dsc.k = hk
                # one workspace per hint: each route is read back after all of them ran
                ws = torch.empty(int(lib.tlm_hip_moe_workspace_bytes(C.byref(dsc))), dtype=torch.uint8,
                                 device=self.workspace.device)
                keep.append((blk, dsc, ws))
                arr[i] = MoeHint(C.pointer(dsc), hl, C.c_void_p(ws.data_ptr()))
            cache[key] = (arr, keep)
        arr = cache[key][0]
        if getattr(self, "_route_out", None) is None:
            self._route_out = ((C.c_int32 * self.desc.k)(), (C.c_float * self.desc.k)())
        ids, w = self._route_out
        check(lib.tlm_hip_moe_layer_store(C.byref(self.desc), store.h, layer, C.c_void_p(h.data_ptr()), ids, w, arr,
                                          n, C.c_void_p(self.workspace.data_ptr()), stream()))
        return list(ids), list(w)

    def set_expert_ptrs(self, expert_ptrs):
        """Point the block at another set of packed experts (same geometry)."""
        self.table.copy_(torch.tensor(list(expert_ptrs), dtype=torch.int64))


class MoeStack:
    """The routed MoE blocks of a stack of layers run for a token through the
    slot cache in one call (tlm_hip_moe_stack_store): blocks[l] is layer l,
    `lookahead` layers ahead are hinted with lookahead_k experts each, the
    breadth interest-weighted when interest > 0 (heat: per-layer floats or
    None).  The instinct state per layer lives here, as the reference keeps it
    in its model."""

    def __init__(self, blocks, *, lookahead=1, lookahead_k=0, interest=0.0, heat=None, host_routes=False):
        n = len(blocks)
        self.blocks = blocks
        self.descs = (MoeDesc * n)(*[MoeDesc.from_buffer_copy(b.desc) for b in blocks])
        self.instinct = np.zeros(n, np.float64)
        self.seen = np.zeros(n, np.uint32)
        self.heat = None if heat is None else np.ascontiguousarray(heat, np.float32)
        self.opts = StackOpts(lookahead, lookahead_k, interest,
                              None if self.heat is None else self.heat.ctypes.data,
                              self.instinct.ctypes.data, self.seen.ctypes.data, int(host_routes))
        nbytes = int(lib.tlm_hip_moe_stack_workspace_bytes(self.descs, n, C.byref(self.opts)))
        self.workspace = torch.empty(nbytes + 256, dtype=torch.uint8, device=blocks[0].workspace.device)
        self._ws = (self.workspace.data_ptr() + 255) & ~255
        k = blocks[0].desc.k
        self.ids = np.zeros((n, k), np.int32)
        self.w = np.zeros((n, k), np.float32)

    def __call__(self, store, h):
        """h += the stack's MoE blocks for one token; the routing lands in
        self.ids / self.w [n_layers, top_k]."""
        check(lib.tlm_hip_moe_stack_store(self.descs, len(self.blocks), store.h, C.c_void_p(h.data_ptr()),
                                          C.byref(self.opts), self.ids.ctypes.data, self.w.ctypes.data,
                                          C.c_void_p(self._ws), stream()))
        return h
