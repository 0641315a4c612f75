"""Decode benchmark of the quantised-MoE hot path on one MI355X.

Workload (one decode step = one token through one routed MoE block at
Qwen3-30B-A3B shape): D 2048, 128 experts, top-8 softmax routing with
renormalisation, expert width 768, Q6_K experts, f32 router, batch 1.  Each
token has its own seeded N(0,1) residual.  To keep "HBM GB/s" honest the
tokens cycle through --layers distinct copies of the layer's 128 experts
(48 copies = the 23.8 GB of Q6_K experts a 48-layer model keeps resident), so
consecutive tokens never re-read an expert from the 256 MB last-level cache.

Timed region: K tokens launched back to back on one stream (HIP graphs of up
to --graph tokens, replayed), bracketed by synchronisation.  value = tokens/s.

roofline: the dominant kernel is the gate/up launch (phase 2).  Its average
duration is measured with HIP events around a graph of --roofline-tokens
back-to-back phase-2 launches (cycling the layer copies), divided by the
count; algorithmic bytes per launch = top-8 x (gate + up) packed Q6_K bytes =
8 x 2 x 1,290,240 = 20,643,840 B.

cpu_baseline: the reference's own kernels (oracle/_ref, AVX-512 tier when the
host has it) running the same block through ref_moe.c on the host cores, on a
bounded sample of tokens over 128 distinct random-code experts.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

D, E, K, DE = 2048, 128, 8, 768
Q6_K = 14
MAT_BYTES = DE * D // 256 * 210          # one packed Q6_K matrix: 1,290,240 B
EXPERT_BYTES = 3 * MAT_BYTES             # 3,870,720 B
TOKEN_BYTES = K * EXPERT_BYTES           # 30,965,760 B per token-layer
GATEUP_BYTES = K * 2 * MAT_BYTES         # 20,643,840 B per gate/up launch
DOWN_BYTES = K * MAT_BYTES               # 10,321,920 B per down launch
HBM_PEAK_GBS = 8000.0
# HBM bytes per gate/up launch from rocprofv3 FETCH_SIZE + WRITE_SIZE (KiB per dispatch), each
# scaled by its reading for a 256 MiB device copy (factors 1.99976 and 1.0); the run and its
# figures: profiles/moe_block_qwen3_30b_hbm_traffic.md
GATEUP_TRAFFIC_BYTES = 20918804


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def make_weights(torch, dev, layers, seed):
    """Random-code Q6_K experts already in the packed tile layout: random code
    bytes, modest f16 block scales in each matrix's scale plane."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    n_mats = layers * E * 3
    W = torch.empty((n_mats, MAT_BYTES), dtype=torch.uint8, device=dev)
    units = MAT_BYTES - (MAT_BYTES // 210) * 2          # 208-byte units, then the f16 scale plane
    chunk = 256
    for m0 in range(0, n_mats, chunk):
        m1 = min(n_mats, m0 + chunk)
        W[m0:m1].random_(0, 256, generator=g)
        d = (torch.randn((m1 - m0, (MAT_BYTES - units) // 2), generator=g, device=dev) * 2e-3).to(torch.float16)
        W[m0:m1, units:] = d.view(torch.uint8)
    return W


PREFILL_T = 512
INT8_PEAK_TOPS = 5000.0                  # MI355X dense int8 MFMA


Q5_K = 13
MAT_BYTES_Q5K = DE * D // 256 * 176      # one packed Q5_K matrix: 1,081,344 B


def make_weights_q5k(torch, dev, seed):
    """128 random-code Q5_K experts in the packed layout (whole 176-byte
    blocks in tile order): random code / scale bytes, modest f16 d and
    non-negative f16 dmin in each block's first four bytes."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    n_mats = E * 3
    W = torch.empty((n_mats, MAT_BYTES_Q5K), dtype=torch.uint8, device=dev)
    W.random_(0, 256, generator=g)
    units = W.view(n_mats, -1, 176)
    d = (torch.randn(units.shape[:2], generator=g, device=dev) * 2e-3).to(torch.float16)
    dm = (torch.randn(units.shape[:2], generator=g, device=dev).abs() * 2e-3).to(torch.float16)
    units[:, :, 0:2] = d.view(torch.uint8).view(n_mats, -1, 2)
    units[:, :, 2:4] = dm.view(torch.uint8).view(n_mats, -1, 2)
    return W


def prefill_bench(torch, dev, W, mat_bytes, dt, router_w, ffn_norm, gen):
    """One 512-token chunk through the block (128 experts of dtype dt, matrix
    stride mat_bytes in W): per-token norm + quantisation, batched router
    logits, routing, tokens bucketed per expert, grouped gate/up + SwiGLU and
    down on int8 MFMA, combine.  Algorithmic bytes = all 128 experts once
    (every expert gets tokens at this size); int8 ops = 2 x tokens x top-8 x
    3 x 768 x 2048."""
    from tierlm_amd import MoeBlock
    ptrs = [W.data_ptr() + (e * 3 + j) * mat_bytes for e in range(E) for j in range(3)]
    blk = MoeBlock(D=D, de=DE, E=E, k=K, expert_dt=dt, ffn_norm=ffn_norm, router_w=router_w, expert_ptrs=ptrs,
                   router=0, eps=1e-6, device=dev)
    H0 = torch.randn((PREFILL_T, D), generator=gen, device=dev)
    h = H0.clone()
    blk.prefill(h)
    torch.cuda.synchronize()
    best = None
    for _ in range(5):
        h.copy_(H0)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        blk.prefill(h)
        ev1.record()
        ev1.synchronize()
        us = ev0.elapsed_time(ev1) * 1e3
        best = us if best is None else min(best, us)
    nbytes = E * 3 * mat_bytes
    ops = 2.0 * PREFILL_T * K * 3 * DE * D
    name = {Q6_K: "Q6_K", Q5_K: "Q5_K"}[dt]
    log(f"bench: prefill {PREFILL_T} tokens ({name}): {best:.1f} us ({PREFILL_T / best * 1e6:.0f} tok/s), "
        f"experts {nbytes / best / 1e3:.0f} GB/s, int8 {ops / best / 1e6:.1f} TOP/s")
    return {"tokens": PREFILL_T, "us": round(best, 1), "tok_s": round(PREFILL_T / best * 1e6, 1),
            "expert_bytes": nbytes, "expert_GBps": round(nbytes / best / 1e3, 1),
            "hbm_frac": round(nbytes / best / 1e3 / HBM_PEAK_GBS, 4), "int8_ops": ops,
            "int8_TOPs": round(ops / best / 1e6, 2), "mfma_util": round(ops / best / 1e6 / INT8_PEAK_TOPS, 4),
            "timing": "HIP events around one tlm_hip_moe_prefill call (best of 5)",
            "workload": f"512-token chunk, Qwen3-30B-A3B-shape block, 128 random-code {name} experts, "
                        "tokens routed by the seeded f32 router and bucketed per expert"}


def host_payloads(torch, n_experts, seed):
    """n_experts Q6_K expert payloads in the reference's packet layout (gate |
    up | down rows of 1680 / 1680 / 630 bytes, random codes, finite f16 block
    scales) in one page-locked host buffer; returns (buffer, payload bytes)."""
    import numpy as np
    rng = np.random.default_rng(seed)
    plen = EXPERT_BYTES
    buf = torch.empty(n_experts * plen, dtype=torch.uint8, pin_memory=True)
    nbl = plen // 210
    for e in range(n_experts):
        blocks = rng.integers(0, 256, size=(nbl, 210), dtype=np.uint8)
        blocks[:, 208:210] = (rng.standard_normal((nbl, 1)) * 2e-3).astype(np.float16).view(np.uint8)
        buf[e * plen:(e + 1) * plen].copy_(torch.from_numpy(blocks.reshape(-1)))
    return buf, plen


def slot_cache_bench(torch, dev, router_w, ffn_norm, gen, tokens):
    """The expert slot cache in HBM (tlm_hip_store_*): (1) fill rate - all 128
    experts of the block loaded into empty slots (pinned host payloads ->
    DMA -> pack), against one plain pinned host-to-device copy of the same
    bytes; (2) decode through the cache (tlm_hip_moe_layer_store) with every
    expert resident, and with half of them (64 slots: misses stream over
    PCIe)."""
    from tierlm_amd import MoeBlock
    from tierlm_amd.store import HipStore
    buf, plen = host_payloads(torch, E, seed=7)
    off = [0, MAT_BYTES, 2 * MAT_BYTES]
    srcs = [{"layer": 0, "id": e, "dtype": Q6_K, "item_off": off, "payload": buf[e * plen:(e + 1) * plen]}
            for e in range(E)]
    out = {"payload_bytes": plen, "experts": E}

    dst = torch.empty(E * plen, dtype=torch.uint8, device=dev)
    best = None
    for _ in range(3):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dst.copy_(buf, non_blocking=True)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        best = dt if best is None else min(best, dt)
    out["h2d_copy_GBps"] = round(E * plen / best / 1e9, 2)
    del dst

    def make_store(slots):
        return HipStore(srcs, d_model=D, d_expert=DE, top_k=K, budget_bytes=slots * (EXPERT_BYTES + 768),
                        prefetch=0)

    best = None
    for _ in range(3):
        st = make_store(E)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for b in range(E // K):
            rc, g = st.acquire(0, list(range(b * K, (b + 1) * K)))
            assert rc == 0
            for j in range(K):
                st.release(g, j)
        st.settle()
        dt = time.perf_counter() - t0
        best = dt if best is None else min(best, dt)
        assert st.stats()["misses"] == E
        st.close()
    out["fill_GBps"] = round(E * plen / best / 1e9, 2)
    out["fill_us_per_expert"] = round(best / E * 1e6, 1)

    dummy = torch.zeros(EXPERT_BYTES, dtype=torch.uint8, device=dev)
    blk = MoeBlock(D=D, de=DE, E=E, k=K, expert_dt=Q6_K, ffn_norm=ffn_norm, router_w=router_w,
                   expert_ptrs=[dummy.data_ptr()] * (3 * E), router=0, eps=1e-6, device=dev)
    for slots, name in ((E, "resident"), (E // 2, "half")):
        st = make_store(slots)
        H = torch.randn((tokens + 20, D), generator=gen, device=dev)
        for t in range(20):                      # warm: fill what fits
            blk.step_store(st, 0, H[t].clone())
            st.tick()
        s0 = st.stats()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for t in range(20, 20 + tokens):
            blk.step_store(st, 0, H[t])
            st.tick()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        s1 = st.stats()
        miss = (s1["misses"] - s0["misses"]) / tokens
        out[name] = {"slots": st.n_slots(), "tok_s": round(tokens / dt, 1), "us_per_token": round(dt / tokens * 1e6, 1),
                     "misses_per_token": round(miss, 2),
                     "miss_GBps": round(miss * plen * tokens / dt / 1e9, 2)}
        st.close()
        log(f"bench: slot cache {name} ({out[name]['slots']} slots): {out[name]['tok_s']:.0f} tok/s, "
            f"{miss:.2f} misses/token")
    log(f"bench: slot fill {out['fill_GBps']} GB/s ({out['fill_us_per_expert']} us/expert), "
        f"plain pinned H2D copy {out['h2d_copy_GBps']} GB/s")
    out["timing"] = "host wall clock around the calls, synchronised (the cache path reads routing back per token)"
    return out


def c5_bench(torch, dev, tokens, cache_gb, pool=64, gamma=0.14, seed=11):
    """The HBM slot cache at the Qwen3-235B-A22B shape: 94 layers x 128
    experts (D 4096, expert width 1536, top-8) of Q4_K, 10.6 MB each (127.7 GB
    in all), served from pinned host memory through tlm_hip_moe_layer_store
    with the cache capped at cache_gb, the next layer's router predicting its
    experts (lookahead hints), one router per layer.  Routing heat: sigmoid
    routing (kind 2) whose selection bias is -gamma * ln(rank + 1) per expert,
    which puts about Zipf(1.1)'s share of the selections on the hottest
    experts (the measured share is reported).  Every (layer, expert) has its
    own slot and is loaded over PCIe on a miss; their payload bytes come from
    a pool of `pool` distinct random-code payloads (the bytes do not change
    the traffic), so host memory stays under 1 GB.  A second, short run caps
    the cache at 8 GB, where most selections miss and stream over PCIe."""
    import numpy as np
    from tierlm_amd import MoeBlock
    from tierlm_amd.store import HipStore
    L5, D5, DE5, Q4_K = 94, 4096, 1536, 12
    rg, rd = D5 // 256 * 144, DE5 // 256 * 144          # gate/up and down row bytes
    off = [0, DE5 * rg, 2 * DE5 * rg]
    plen = 2 * DE5 * rg + D5 * rd                        # 10,616,832 B
    rng = np.random.default_rng(seed)
    buf = torch.empty(pool * plen, dtype=torch.uint8, pin_memory=True)
    nbl = plen // 144
    for i in range(pool):
        blocks = rng.integers(0, 256, size=(nbl, 144), dtype=np.uint8)
        blocks[:, 0:2] = (rng.standard_normal((nbl, 1)) * 2e-3).astype(np.float16).view(np.uint8)
        blocks[:, 2:4] = (np.abs(rng.standard_normal((nbl, 1))) * 2e-3).astype(np.float16).view(np.uint8)
        buf[i * plen:(i + 1) * plen].copy_(torch.from_numpy(blocks.reshape(-1)))
    srcs = [{"layer": l, "id": e, "dtype": Q4_K, "item_off": off,
             "payload": buf[((l * E + e) % pool) * plen:((l * E + e) % pool + 1) * plen]}
            for l in range(L5) for e in range(E)]
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    ffn_norm = torch.ones(D5, device=dev)
    bias = torch.tensor(-gamma * np.log(np.arange(E) + 1.0), dtype=torch.float32, device=dev)
    dummy = torch.zeros(16, dtype=torch.uint8, device=dev)
    blocks = []
    for l in range(L5):
        # each layer's hot experts are a different permutation of the ids
        perm = torch.randperm(E, generator=g, device=dev)
        blocks.append(MoeBlock(D=D5, de=DE5, E=E, k=K, expert_dt=Q4_K, ffn_norm=ffn_norm,
                               router_w=torch.randn((E, D5), generator=g, device=dev) / float(np.sqrt(D5)),
                               expert_ptrs=[dummy.data_ptr()] * (3 * E), router=2, router_bias=bias[perm].contiguous(),
                               eps=1e-6, device=dev))
    H = torch.randn((tokens + 40, D5), generator=g, device=dev)

    def run(cap_gb, ntok, warm):
        st = HipStore(srcs, d_model=D5, d_expert=DE5, top_k=K, budget_bytes=int(cap_gb * (1 << 30)), prefetch=1)
        sel = np.zeros((L5, E), np.int64)

        def token(t, count):
            for l in range(L5):
                hints = [(blocks[l + 1], l + 1, K)] if l + 1 < L5 else []
                ids, _ = blocks[l].step_store(st, l, H[t].clone(), hints)
                if count:
                    sel[l, ids] += 1
                st.tick()

        for t in range(warm):                            # fill the cache and reach the heat's steady state
            token(t, False)
        s0 = st.stats()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for t in range(warm, warm + ntok):
            token(t, True)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        s1 = st.stats()
        miss = (s1["misses"] - s0["misses"]) / ntok
        fs = np.sort(sel, axis=1)[:, ::-1].sum(axis=0)
        r = {"cache_GB": cap_gb, "slots": st.n_slots(), "tokens": ntok, "warmup_tokens": warm,
             "tok_s": round(ntok / dt, 2), "ms_per_token": round(dt / ntok * 1e3, 2),
             "misses_per_token": round(miss, 1), "hit_rate": round(1.0 - miss / (L5 * K), 4),
             "miss_GBps": round(miss * plen * ntok / dt / 1e9, 2),
             # lookahead loads are not misses: they land before the layer asks, but cross PCIe too
             "prefetch_issued_per_token": round((s1["prefetch_issued"] - s0["prefetch_issued"]) / ntok, 1),
             "prefetch_used_per_token": round((s1["prefetch_used"] - s0["prefetch_used"]) / ntok, 1),
             "load_GBps_with_prefetch": round((miss + (s1["prefetch_issued"] - s0["prefetch_issued"]) / ntok)
                                              * plen * ntok / dt / 1e9, 2),
             "heat_top10pct_share": round(float(fs[:13].sum() / fs.sum()), 3)}
        st.close()
        log(f"bench: C5 slot cache ({r['slots']} slots, {cap_gb:.0f} GB): {r['tok_s']:.2f} tok/s, "
            f"{r['misses_per_token']:.1f} misses/token (hit rate {r['hit_rate']:.3f}), {r['miss_GBps']:.1f} GB/s "
            f"of misses; lookahead {r['prefetch_issued_per_token']:.1f} loads/token "
            f"({r['prefetch_used_per_token']:.1f} used); all loads {r['load_GBps_with_prefetch']:.1f} GB/s over PCIe, "
            f"heat top-13 share {r['heat_top10pct_share']}")
        return r

    out = {"model": "Qwen3-235B-A22B shape MoE stack: 94 layers, D 4096, 128 experts top-8 of width 1536, Q4_K, "
                    "random codes (127.7 GB of experts)",
           "expert_bytes": plen, **run(cache_gb, tokens, 40),
           "heat": f"sigmoid routing, selection bias -{gamma} ln(rank + 1) (a Zipf(1.1)-like heat; Zipf(1.1) puts 0.61 "
                   "of top-8 selections on the 13 hottest experts)",
           "timing": "host wall clock around 94 tlm_hip_moe_layer_store calls per token (ctypes, routing read back "
                     "per layer), after the warm-up tokens"}
    out["small_cache"] = run(8.0, max(2, tokens // 4), 4)   # misses stream over PCIe
    del blocks, buf
    return out


C1_STORE = os.path.join(ROOT, "oracle", "_ref", "c1", "c1.tlmm")
C1_TIERLM = os.path.join(ROOT, "oracle", "_ref", "bin", "tierlm")


def c1_bench(reps):
    """The whole decode step on the 4-layer synthetic model (the reference's
    compiled store, oracle/make_c1.sh): 64-token prompt, 64 greedy tokens, as
    `tierlm bench --prompt-len 64 -n 64`; decode tok/s = 63 / decode time.
    Beside it the reference's own runtime on the host cores, same store."""
    import subprocess
    from tierlm_amd.model import bench as model_bench
    r = model_bench(C1_STORE, 64, 64, reps, max_ctx=256)
    out = {"prefill_tok_s": r["prefill_tok_s"], "decode_tok_s": r["decode_tok_s"],
           "decode_us_per_token": r["decode_us_per_token"], "tokens_head": r["tokens"][:4],
           "timing": "host wall clock around tlm_hip_model_generate (prefill 64, then 63 decode steps), best of "
                     f"{reps}; each step one replay of a captured HIP graph"}
    if os.path.exists(C1_TIERLM):
        r = subprocess.run([C1_TIERLM, "bench", C1_STORE, "--prompt-len", "64", "-n", "64", "--cache", "1G"],
                           capture_output=True, text=True, timeout=120)
        line = r.stdout.splitlines()[0] if r.stdout else ""
        try:
            ref_dec = float(line.split("decode 64 tokens in")[1].split("(")[1].split(" tok/s")[0])
            ref_pre = float(line.split("prompt 64 tokens in")[1].split("(")[1].split(" tok/s")[0])
            out["reference_cpu"] = {"prefill_tok_s": ref_pre, "decode_tok_s": ref_dec, "threads": os.cpu_count(),
                                    "kind": "reference", "command": "tierlm bench --prompt-len 64 -n 64 --cache 1G"}
        except (IndexError, ValueError):
            out["reference_cpu"] = None
    log(f"bench: C1 whole step: prefill {out['prefill_tok_s']:.0f} tok/s, decode {out['decode_tok_s']:.0f} tok/s "
        f"({out['decode_us_per_token']:.1f} us/token); reference CPU {out.get('reference_cpu')}")
    return out


def c3_bench(reps, ctx):
    """The whole decode step on a random-init model of the full Qwen3-30B-A3B
    shape (48 layers, hidden 2048, 32 q / 4 kv heads x 128, 128 experts top-8
    of width 768, vocabulary 151936; Q6_K experts, Q8_0 dense; every expert
    resident, 23.8 GB), built in HBM by tlm_hip_model_synth: a 64-token
    prompt, then greedy tokens up to ctx positions.  The reference has no
    store of this size here, so no CPU figure sits beside it."""
    from tierlm_amd.model import QWEN3_30B_A3B, Model, time_model
    t0 = time.perf_counter()
    m = Model.synth(QWEN3_30B_A3B, expert_dt=Q6_K, dense_dt=8, seed=1, max_ctx=ctx)
    built = time.perf_counter() - t0
    try:
        r = time_model(m, 64, ctx - 64, reps, warm_n=8)
        short = time_model(m, 64, 64, reps)
    finally:
        m.close()
    out = {"model": "Qwen3-30B-A3B shape, random init (48 layers, 128 experts top-8, Q6_K experts, Q8_0 dense)",
           "context": ctx, "prefill_tok_s": r["prefill_tok_s"], "decode_tok_s": r["decode_tok_s"],
           "decode_ms_per_token": round(r["decode_us_per_token"] / 1e3, 3),
           "decode_tok_s_first_64": short["decode_tok_s"], "build_s": round(built, 2),
           "timing": f"host wall clock around tlm_hip_model_generate: prefill 64, then {ctx - 64 - 1} decode steps "
                     f"to {ctx} positions, best of {reps}; each step one replay of a captured HIP graph",
           "reference_cpu": None}
    log(f"bench: Qwen3-30B-A3B-shape model: decode {out['decode_tok_s']:.1f} tok/s to {ctx} positions "
        f"({out['decode_ms_per_token']:.3f} ms/token; {out['decode_tok_s_first_64']:.1f} tok/s over the first 64), "
        f"prefill {out['prefill_tok_s']:.1f} tok/s")
    return out


def cpu_baseline(args, threads):
    """Reference kernels on the host (oracle/_ref), bounded sample."""
    import numpy as np

    import oracle
    from tests.synth import random_code_rows
    if oracle.ref is None:
        return None
    rng = np.random.default_rng(3)
    experts = []
    for _ in range(E):
        experts.append((random_code_rows(rng, Q6_K, DE, D), random_code_rows(rng, Q6_K, DE, D),
                        random_code_rows(rng, Q6_K, D, DE)))
    host = oracle.MoeHost(D=D, de=DE, E=E, k=K, expert_dt=Q6_K, ffn_norm=np.ones(D, np.float32),
                          router_w=(rng.standard_normal((E, D)) / np.sqrt(D)).astype(np.float32), experts=experts)
    hs = rng.standard_normal((64, D)).astype(np.float32)
    out = {}
    for nthr in sorted({1, threads}):
        handle = oracle.ref.refmoe_new(nthr)
        host.run_ref(handle, hs[0])            # warm
        t0, n = time.perf_counter(), 0
        while time.perf_counter() - t0 < args.cpu_seconds / 2 or n < 8:
            host.run_ref(handle, hs[n % 64])
            n += 1
        dt = time.perf_counter() - t0
        oracle.ref.refmoe_free(handle)
        out[nthr] = (n / dt, n)
    tier = oracle.ref.refmoe_tier().decode()
    best = out[threads]
    return {"value": round(best[0], 2), "unit": "tok/s", "cores": threads, "kind": "reference",
            "sample": f"{best[1]} tokens of the same block (128 distinct random-code Q6_K experts, 495 MB) "
                      f"through the reference's {tier} tier + pool on {threads} threads",
            "single_thread_tok_s": round(out[1][0], 2), "gpu_over_cpu": None}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10000, help="timed tokens")
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--layers", type=int, default=48, help="distinct layer copies cycled by the tokens")
    ap.add_argument("--graph", type=int, default=100, help="tokens per captured HIP graph (0 = eager launches)")
    ap.add_argument("--roofline-tokens", type=int, default=960, help="launches per phase in the roofline graphs")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the 512-token prefill measurement")
    ap.add_argument("--no-store", action="store_true", help="skip the expert slot cache measurement")
    ap.add_argument("--no-c1", action="store_true", help="skip the whole-step synthetic model measurement")
    ap.add_argument("--no-c3", action="store_true", help="skip the full Qwen3-30B-A3B-shape model measurement")
    ap.add_argument("--c3-context", type=int, default=2048, help="positions the full-model decode runs to")
    ap.add_argument("--store-tokens", type=int, default=400, help="tokens per slot-cache decode measurement")
    ap.add_argument("--no-c5", action="store_true", help="skip the Qwen3-235B-shape slot-cache measurement")
    ap.add_argument("--c5-tokens", type=int, default=20, help="timed tokens of the Qwen3-235B-shape slot-cache run")
    ap.add_argument("--c5-cache-gb", type=float, default=64.0, help="slot cache cap of that run (GB)")
    ap.add_argument("--copy-check-mib", type=int, default=0,
                    help="after the timed work, one device-to-device copy of this many MiB: a plain copy kernel "
                         "of known size, the scale for HBM byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); "
              "multi-GPU runs are not part of it", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import tierlm_amd
    from tierlm_amd import MoeBlock
    from tierlm_amd import quant as hq

    dev = torch.device("cuda", 0)
    hq.init(0)
    assert hq.selftest_failures() == 0, "HIP self-test failures"
    L = args.layers
    log(f"bench: allocating {L} x {E} Q6_K experts ({L * E * EXPERT_BYTES / 1e9:.1f} GB)")
    W = make_weights(torch, dev, L, seed=1)
    gen = torch.Generator(device=dev)
    gen.manual_seed(2)
    router_w = torch.randn((E, D), generator=gen, device=dev) / float(np.sqrt(D))
    ffn_norm = torch.ones(D, device=dev)
    blocks = []
    base = W.data_ptr()
    for layer in range(L):
        ptrs = [base + ((layer * E + e) * 3 + j) * MAT_BYTES for e in range(E) for j in range(3)]
        blocks.append(MoeBlock(D=D, de=DE, E=E, k=K, expert_dt=Q6_K, ffn_norm=ffn_norm, router_w=router_w,
                               expert_ptrs=ptrs, router=0, eps=1e-6, device=dev))
    total = args.warmup + args.steps
    H = torch.randn((max(total, args.roofline_tokens), D), generator=gen, device=dev)
    torch.cuda.synchronize()

    def run_tokens(t0, t1):
        for t in range(t0, t1):
            blocks[t % L](H[t])

    graphs = []
    if args.graph > 0:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            run_tokens(0, min(args.graph, total))          # warm the launch path before capture
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()

        def capture(t0, t1):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                run_tokens(t0, t1)
            return g
        G = args.graph
        warm_chunks = [(t, min(t + G, args.warmup)) for t in range(0, args.warmup, G)]
        timed_chunks = [(t, min(t + G, total)) for t in range(args.warmup, total, G)]
        log(f"bench: capturing {len(warm_chunks) + len(timed_chunks)} graphs of <= {G} tokens")
        warm_graphs = [capture(*c) for c in warm_chunks]
        graphs = [capture(*c) for c in timed_chunks]
        torch.cuda.synchronize()
        for g in warm_graphs:
            g.replay()
    else:
        run_tokens(0, args.warmup)
    torch.cuda.synchronize()

    t0 = time.perf_counter()
    if graphs:
        for g in graphs:
            g.replay()
    else:
        run_tokens(args.warmup, total)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    tok_s = args.steps / elapsed
    ms_per_step = elapsed * 1e3 / args.steps

    # roofline pass: per phase, one HIP graph of R launches of that phase
    # alone, each on the next layer copy (so weights stream from HBM), replayed
    # between two events on the stream it runs on; average launch = elapsed / R
    # (kernel time plus the graph's dispatch gap between dependent launches)
    R = args.roofline_tokens
    hr = torch.randn(D, generator=gen, device=dev)
    for b in blocks:                       # every workspace holds a routed token
        b(hr.clone())
    torch.cuda.synchronize()
    ph = []
    for p in range(1, 4):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            blocks[0].phase(p, hr)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for t in range(R):
                blocks[t % L].phase(p, hr)
        g.replay()
        torch.cuda.synchronize()
        best = None
        for _ in range(3):
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record()
            g.replay()
            ev1.record()
            ev1.synchronize()
            us = ev0.elapsed_time(ev1) * 1e3 / R
            best = us if best is None else min(best, us)
        ph.append(best)
        del g
    p1, p2, p3 = ph
    gu_gbs = GATEUP_BYTES / (p2 * 1e-6) / 1e9
    dn_gbs = DOWN_BYTES / (p3 * 1e-6) / 1e9
    expert_gbs = TOKEN_BYTES / ((p2 + p3) * 1e-6) / 1e9
    log(f"bench: {tok_s:.0f} tok/s ({ms_per_step * 1e3:.2f} us/token); per launch: router {p1:.2f} us, "
        f"gate/up {p2:.2f} us ({gu_gbs:.0f} GB/s), down+combine {p3:.2f} us ({dn_gbs:.0f} GB/s)")
    # on-box streaming-read reference: this library's packed Q6_K GEMV over a span of up to
    # 2 GiB of the resident expert bytes read as one 2048-wide matrix (values irrelevant); the
    # span never exceeds the buffer it reads
    srows = min(2 << 30, W.numel()) // 1680 // 16 * 16
    sbytes = hq.packed_bytes(Q6_K, srows, D)
    assert 0 < sbytes <= W.numel(), (sbytes, W.numel())
    xs = hq.quantize_act(hq.Q8_K, torch.randn(D, generator=gen, device=dev))
    ys = torch.empty(srows, dtype=torch.float32, device=dev)
    hq.matvec_packed(Q6_K, W, srows, D, xs, ys)
    torch.cuda.synchronize()
    stream_us = None
    for _ in range(5):
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        hq.matvec_packed(Q6_K, W, srows, D, xs, ys)
        ev1.record()
        ev1.synchronize()
        us = ev0.elapsed_time(ev1) * 1e3
        stream_us = us if stream_us is None else min(stream_us, us)
    stream_gbs = sbytes / (stream_us * 1e-6) / 1e9
    log(f"bench: streaming GEMV over {sbytes / 1e9:.2f} GB: {stream_gbs:.0f} GB/s")

    if args.copy_check_mib > 0:
        nbytes = args.copy_check_mib << 20
        src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"bench: copy check {args.copy_check_mib} MiB done")
        del src, dst

    prefill = prefill_q5k = None
    if not args.no_prefill:
        prefill = prefill_bench(torch, dev, W, MAT_BYTES, Q6_K, router_w, ffn_norm, gen)
        W5 = make_weights_q5k(torch, dev, seed=5)
        prefill_q5k = prefill_bench(torch, dev, W5, MAT_BYTES_Q5K, Q5_K, router_w, ffn_norm, gen)
        del W5
    slot_cache = None if args.no_store else slot_cache_bench(torch, dev, router_w, ffn_norm, gen, args.store_tokens)
    c1 = None if args.no_c1 or not os.path.exists(C1_STORE) else c1_bench(3)
    if not args.no_c3:
        del W                                  # the block's 23.8 GB of experts; the model builds its own
        torch.cuda.empty_cache()
    c3 = None if args.no_c3 else c3_bench(1, args.c3_context)
    c5 = None
    if not args.no_c5:
        torch.cuda.empty_cache()
        try:
            c5 = c5_bench(torch, dev, args.c5_tokens, args.c5_cache_gb)
        except Exception as e:                 # recorded, so the rest of the line still prints
            c5 = {"error": repr(e)}
            log(f"bench: C5 slot cache failed: {e!r}")
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        log(f"bench: cpu baseline ({threads} threads, ~{args.cpu_seconds:.0f} s)")
        cpu = cpu_baseline(args, threads)
        if cpu:
            cpu["gpu_over_cpu"] = round(tok_s / cpu["value"], 1)

    line = {
        "metric": "decode tok/s batch-1, Qwen3-30B-A3B shape; expert GEMV HBM GB/s vs peak",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8xu6->int32 (Q6_K x Q8_K), f32 chain", "data": "synthetic",
        "config": {"workload": "single routed MoE block at Qwen3-30B-A3B shape (D 2048, 128 experts top-8 softmax+renorm, "
                               "expert width 768, Q6_K random-code experts, f32 router), batch-1 decode, "
                               f"one token per step, {L} resident layer copies cycled",
                   "tokens_timed": args.steps, "graph_tokens": args.graph, "layers_resident": L,
                   "expert_bytes_per_token": TOKEN_BYTES},
        "roofline": {"bound": "hbm", "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": GATEUP_TRAFFIC_BYTES,
                     "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per dispatch, scaled by a 256 MiB copy",
                     "kernel": "k_moe_gateup (routing + gate/up of the top-8 experts + SwiGLU)",
                     "bytes_per_launch": GATEUP_BYTES, "avg_launch_us": round(p2, 3),
                     "down_combine_GBps": round(dn_gbs, 1), "down_combine_avg_launch_us": round(p3, 3),
                     "router_avg_launch_us": round(p1, 3),
                     "timing": "HIP events around a graph of R back-to-back launches of the phase (R = roofline_launches), / R",
                     "roofline_launches": R,
                     "expert_gemv_GBps": round(expert_gbs, 1), "expert_gemv_frac": round(expert_gbs / HBM_PEAK_GBS, 4),
                     "stream_read_peak_GBps": round(stream_gbs, 1),
                     "stream_read_kernel": "k_mv_packed<Q6_K> over ~2 GB of resident expert bytes, one launch (best of 5)"},
        "cpu_baseline": cpu,
        "prefill": prefill,
        "prefill_q5k": prefill_q5k,
        "slot_cache": slot_cache,
        "c1_whole_step": c1,
        "qwen3_30b_a3b_whole_model": c3,
        "qwen3_235b_a22b_slot_cache": c5,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
