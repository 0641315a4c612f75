"""Writes the golden fixtures of tests/golden/ from the reference compiled out
of its own sources (oracle/_ref/libtlmref.so, built by oracle/Makefile from
/root/reference/src/lib).  Run in the build container:

    make -C oracle && python tests/golden/gen_golden.py

The fixtures are data only (inputs and the reference's outputs):
  quant_rows.npz  float rows -> the reference quantisers' bytes (Q8_0, Q4_K,
                  Q5_K, Q6_K, Q8_K): no closed form pins these searches.
  act.npz         activation vectors (edge cases) -> Q8_K / Q8_0 bytes.
  dots.npz        weight rows x activations -> the reference's scalar-tier
                  float bits (tlm_vec_dot), random-byte and quantised rows.
  moe.npz         one small routed MoE block (D 256, 4 experts top-2,
                  width 256, Q6_K experts, Q8_0 shared expert) through the
                  reference's quantisers and kernels -> updated residual bits.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from oracle import Q4_K, Q5_K, Q6_K, Q8_0, Q8_K  # noqa: E402

INT = [Q8_0, Q4_K, Q5_K, Q6_K, Q8_K]


def main():
    assert oracle.ref is not None, "oracle/_ref/libtlmref.so is not built"
    oracle.ref.tlm_cpu_force(b"scalar")
    oracle.ref.tlm_quant_init()
    assert oracle.ref.tlm_quant_tier() == b"scalar"
    rng = np.random.default_rng(20261201)

    out = {}
    for dt in INT:
        for n, scale in [(256, 0.02), (512, 1.0), (2048, 0.02), (768, 7.0)]:
            x = (rng.standard_normal((3, n)) * scale).astype(np.float32)
            x[1, :32] = 0.0
            out[f"x_{dt}_{n}"] = x
            out[f"q_{dt}_{n}"] = oracle.quantize_row(dt, x, use_ref=True)
    np.savez_compressed(os.path.join(HERE, "quant_rows.npz"), **out)

    out = {}
    vecs = [rng.standard_normal(2048).astype(np.float32), np.zeros(300, np.float32),
            (rng.standard_normal(777) * 1e-3).astype(np.float32),
            (np.arange(64, dtype=np.float32) - 32) * np.float32(2.0 ** -140)]
    v = rng.standard_normal(512).astype(np.float32)
    v[10], v[300] = np.nan, -np.inf
    vecs.append(v)
    sp = (0.001 * rng.standard_normal(1024)).astype(np.float32)
    sp[::77] = 1000.0
    vecs.append(sp)
    for i, x in enumerate(vecs):
        out[f"x{i}"] = x
        out[f"k{i}"] = oracle.quantize_act(Q8_K, x, use_ref=True)
        out[f"a{i}"] = oracle.quantize_act(Q8_0, x, use_ref=True)
    np.savez_compressed(os.path.join(HERE, "act.npz"), **out)

    from tests.synth import random_code_rows
    out = {}
    for dt in INT:
        for n in (256, 768, 2048):
            W = np.concatenate([random_code_rows(rng, dt, 6, n),
                                oracle.quantize_row(dt, (rng.standard_normal((2, n)) * 0.05).astype(np.float32),
                                                    use_ref=True)])
            act = oracle.quantize_act(oracle.act_kind_for(dt), rng.standard_normal(n).astype(np.float32),
                                      use_ref=True)
            y = np.array([oracle.vec_dot(dt, W[r], act, n, use_ref=True) for r in range(W.shape[0])], np.float32)
            out[f"w_{dt}_{n}"], out[f"act_{dt}_{n}"], out[f"y_{dt}_{n}"] = W, act, y
    np.savez_compressed(os.path.join(HERE, "dots.npz"), **out)

    # MoE block: float weights quantised by the reference, run by its kernels
    D, de, E, k, ds = 256, 256, 4, 2, 256
    ffn_norm = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    router_w = (rng.standard_normal((E, D)) / np.sqrt(D)).astype(np.float32)
    experts = []
    for _ in range(E):
        g = oracle.quantize_row(Q6_K, (rng.standard_normal((de, D)) / np.sqrt(D)).astype(np.float32), use_ref=True)
        u = oracle.quantize_row(Q6_K, (rng.standard_normal((de, D)) / np.sqrt(D)).astype(np.float32), use_ref=True)
        dn = oracle.quantize_row(Q6_K, (rng.standard_normal((D, de)) * 0.5 / np.sqrt(de)).astype(np.float32),
                                 use_ref=True)
        experts.append((g, u, dn))
    shared = tuple(oracle.quantize_row(Q8_0, (rng.standard_normal(shp) * s).astype(np.float32), use_ref=True)
                   for shp, s in [((ds, D), 1 / np.sqrt(D)), ((ds, D), 1 / np.sqrt(D)), ((D, ds), 0.5 / np.sqrt(ds))])
    host = oracle.MoeHost(D=D, de=de, E=E, k=k, expert_dt=Q6_K, ffn_norm=ffn_norm, router_w=router_w,
                          experts=experts, ds=ds, shared_dt=Q8_0, shared=shared)
    handle = oracle.ref.refmoe_new(1)
    hs = (rng.standard_normal((4, D)) * 2).astype(np.float32)
    res = [host.run_ref(handle, h) for h in hs]
    oracle.ref.refmoe_free(handle)
    out = dict(ffn_norm=ffn_norm, router_w=router_w, h_in=hs,
               gate=np.stack([e[0] for e in experts]), up=np.stack([e[1] for e in experts]),
               down=np.stack([e[2] for e in experts]), sg=shared[0], su=shared[1], sd=shared[2],
               h_out=np.stack([r[0] for r in res]), ids=np.stack([r[1] for r in res]),
               w=np.stack([r[2] for r in res]))
    np.savez_compressed(os.path.join(HERE, "moe.npz"), **out)
    oracle.ref.tlm_cpu_force(b"auto")
    oracle.ref.tlm_quant_init()
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
