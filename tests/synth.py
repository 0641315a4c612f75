"""Seeded synthetic MoE blocks for the parity tests and smoke().

Weights follow the shapes of the reference's synthetic model generator
(tlmc synth, src/bin/tlmc.c:340-388 there): router N(0, 1/sqrt(D)) kept f32,
expert gate/up N(0, 1/sqrt(D)), down N(0, 0.5/sqrt(de)), then quantised with
the oracle's restatement of the reference quantisers ("quantized"), or - for
shapes too large to quantise on the CPU inside a test - random code bytes with
finite scale fields ("random_codes", the reference's own matvec bench rows,
tests/test_quant.c:633-690 there).  Both layouts are the reference's bytes.
"""
import types

import numpy as np

import oracle

F16_SCALE_FIELDS = {oracle.Q6_K: (208,), oracle.Q8_0: (0,), oracle.Q4_K: (0, 2), oracle.Q5_K: (0, 2)}


def random_code_rows(rng, dt, rows, n):
    """Random block bytes with finite, modest f16 scale fields (value-independent speed)."""
    bv, bb = oracle.BLOCK[dt]
    nb = n // bv
    w = rng.integers(0, 256, size=(rows, nb, bb), dtype=np.uint8)
    if dt == oracle.Q8_K:
        d = (rng.standard_normal((rows, nb)) * 1e-3).astype(np.float32)
        w[:, :, 0:4] = d.view(np.uint8).reshape(rows, nb, 4)
    else:
        for k, off in enumerate(F16_SCALE_FIELDS[dt]):
            if dt in (oracle.Q4_K, oracle.Q5_K) and k == 1:
                v = np.abs(rng.standard_normal((rows, nb))) * 2e-3
            else:
                v = rng.standard_normal((rows, nb)) * (1e-3 if dt == oracle.Q8_0 else 2e-3)
            w[:, :, off:off + 2] = v.astype(np.float16).view(np.uint8).reshape(rows, nb, 2)
    return w.reshape(rows, nb * bb)


def make_matrix(rng, dt, rows, n, std, weights):
    if weights == "quantized":
        return oracle.quantize_row(dt, (rng.standard_normal((rows, n)) * std).astype(np.float32))
    return random_code_rows(rng, dt, rows, n)


def build_moe_case(*, D, de, E, k, ds=0, expert_dt=oracle.Q6_K, shared_dt=oracle.Q8_0, seed=1,
                   device=None, router=0, routed_scale=1.0, eps=1e-6, weights="quantized",
                   mask=None, router_bias=None, shared_gate=False, h_scale=1.0):
    """Returns a namespace with .host (oracle.MoeHost), .h0 and, when a device
    is given, .block (tierlm_amd.MoeBlock) over the same bytes."""
    rng = np.random.default_rng(seed)
    ffn_norm = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    router_w = (rng.standard_normal((E, D)) / np.sqrt(D)).astype(np.float32)
    experts = []
    for _ in range(E):
        g = make_matrix(rng, expert_dt, de, D, 1.0 / np.sqrt(D), weights)
        u = make_matrix(rng, expert_dt, de, D, 1.0 / np.sqrt(D), weights)
        dn = make_matrix(rng, expert_dt, D, de, 0.5 / np.sqrt(de), weights)
        experts.append((g, u, dn))
    shared = None
    sgi = None
    if ds > 0:
        shared = (make_matrix(rng, shared_dt, ds, D, 1.0 / np.sqrt(D), weights),
                  make_matrix(rng, shared_dt, ds, D, 1.0 / np.sqrt(D), weights),
                  make_matrix(rng, shared_dt, D, ds, 0.5 / np.sqrt(ds), weights))
        if shared_gate:
            sgi = (rng.standard_normal(D) / np.sqrt(D)).astype(np.float32)
    h0 = (rng.standard_normal(D) * h_scale).astype(np.float32)
    host = oracle.MoeHost(D=D, de=de, E=E, k=k, expert_dt=expert_dt, ffn_norm=ffn_norm, router_w=router_w,
                          experts=experts, router=router, routed_scale=routed_scale, eps=eps,
                          router_bias=router_bias, mask=mask, ds=ds, shared_dt=shared_dt, shared=shared,
                          shared_gate_inp=sgi)
    case = types.SimpleNamespace(host=host, h0=h0, experts=experts, shared=shared, ffn_norm=ffn_norm,
                                 router_w=router_w, D=D, de=de, E=E, k=k, ds=ds, expert_dt=expert_dt,
                                 shared_dt=shared_dt, block=None)
    if device is not None:
        case.block, case.dev_keep = device_block(case, device, router=router, routed_scale=routed_scale, eps=eps,
                                                 mask=mask, router_bias=router_bias, shared_gate_inp=sgi)
    return case


def device_block(case, device, *, router=0, routed_scale=1.0, eps=1e-6, mask=None, router_bias=None,
                 shared_gate_inp=None):
    """Upload the case's bytes, pack every matrix on device, build a MoeBlock."""
    import torch

    from tierlm_amd import MoeBlock
    from tierlm_amd import quant as hq

    keep = []

    def packed(W, dt, rows, n):
        Wd = torch.from_numpy(np.ascontiguousarray(W).reshape(-1)).to(device)
        P = hq.pack(dt, Wd, W.shape[1], rows, n)
        keep.append(P)
        return P

    D, de, ds = case.D, case.de, case.ds
    ptrs = []
    for g, u, dn in case.experts:
        ptrs += [packed(g, case.expert_dt, de, D).data_ptr(), packed(u, case.expert_dt, de, D).data_ptr(),
                 packed(dn, case.expert_dt, D, de).data_ptr()]
    shared = None
    if ds > 0:
        sg, su, sd = case.shared
        shared = (packed(sg, case.shared_dt, ds, D), packed(su, case.shared_dt, ds, D),
                  packed(sd, case.shared_dt, D, ds))

    def t(a, dtype=torch.float32):
        return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=dtype)

    block = MoeBlock(D=D, de=de, E=case.E, k=case.k, expert_dt=case.expert_dt, ffn_norm=t(case.ffn_norm),
                     router_w=t(case.router_w), expert_ptrs=ptrs, router=router, routed_scale=routed_scale, eps=eps,
                     router_bias=t(router_bias), mask=t(mask, torch.uint8), ds=ds, shared_dt=case.shared_dt,
                     shared=shared, shared_gate_inp=t(shared_gate_inp), device=device)
    torch.cuda.synchronize()
    return block, keep
