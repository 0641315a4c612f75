"""Decode benchmark of the quantised-MoE hot path on one MI355X.

Headline (value): batch-1 greedy decode of the whole Qwen3-30B-A3B-shaped
model to 2048 positions: 48 layers, hidden 2048, 32 q / 4 kv heads x 128
(qk-norm, rope theta 1e6), 128 experts top-8 of width 768 (Q6_K, all 23.8 GB
resident), Q8_0 dense, f32 router, vocabulary 151936; random init built in
HBM (tlm_hip_model_synth).  A 64-token prompt and one greedy pass fill the
context to 2047 positions; a "step" is then one decode token (the captured
step graph: embedding, 48 x (q|k|v, attention scores, softmax + P.V, o,
router, routed gate/up + SwiGLU, down + combine), lm_head + argmax) at a
context position taken evenly from 64..2047 (descending; the context is
rewound to that position first, so the step reads exactly that many cached
positions).  --steps 1984 is the whole sweep.  Timed with HIP events on the
model's stream (and the host clock) around exactly K steps.

roofline (the decode step): algorithmic bytes per token = packed weight
bytes read (48 x (q, k, v, o + router + 8 routed experts) + lm_head =
2,829,893,632 B) + the f32 KV rows read (K and V, 48 layers x 4 kv heads x T x
128 x 4 B each, averaged over the timed positions), over the step time,
against 8 TB/s.  expert_gemv: the routed block alone (one MoE layer per
token, 48 resident layer copies cycled), per-phase launch times from graphs
of back-to-back launches (HIP events), as before.

cpu_baseline: the reference's own kernels (oracle/_ref: AVX-512 tier, its
pool) on the host cores for a bounded sample of the same per-token work -
one layer's q|k|v and o projections (Q8_0) and routed MoE block at this
shape, and the lm_head - scaled to tokens/s as 1 / (48 x layer + lm_head)
(attention's score / softmax / P.V arithmetic and the norms are left out of
the CPU figure).
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
# HBM bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE (KiB per dispatch) of the MoE-block
# and dense-GEMV legs, each scaled by its reading for a 256 MiB device copy (factors 1.99982 and
# 1.0); the runs and their figures: profiles/moe_block_qwen3_30b_hbm_traffic.md
GATEUP_TRAFFIC_BYTES = 20868827
ROUTER_TRAFFIC_BYTES = 1383201
DOWN_TRAFFIC_BYTES = 10892562
DENSE_TRAFFIC_BYTES = {"qkv": 11274251, "o": 9071845, "lm_head": 331571529}
# the decode step's kernels at the Qwen3-30B-A3B shape: per layer q|k|v + o + router + gate/up +
# down, then lm_head once (the attention launches' K / V reads are added at their algorithmic bytes:
# they run only inside the model, which is not profiled under counters)
STEP_LAYER_TRAFFIC_BYTES = (DENSE_TRAFFIC_BYTES["qkv"] + DENSE_TRAFFIC_BYTES["o"] + ROUTER_TRAFFIC_BYTES
                            + GATEUP_TRAFFIC_BYTES + DOWN_TRAFFIC_BYTES)


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
Q4_K = 12
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
    from tierlm_amd import MoeBlock, MoeStack
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

    stack = MoeStack(blocks, lookahead=1, lookahead_k=K)

    def run(cap_gb, ntok, warm):
        st = HipStore(srcs, d_model=D5, d_expert=DE5, top_k=K, budget_bytes=int(cap_gb * (1 << 30)), prefetch=1)
        sel = np.zeros((L5, E), np.int64)

        def token(t, count):
            stack(st, H[t].clone())                      # 94 layers, one tick
            if count:
                for l in range(L5):
                    sel[l, stack.ids[l]] += 1

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
        log(f"bench: Qwen3-235B-A22B-shape MoE stack through the slot cache ({r['slots']} slots, {cap_gb:.0f} GB): {r['tok_s']:.2f} tok/s, "
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
           "timing": "host wall clock around one tlm_hip_moe_stack_store call per token (94 layers, the residual "
                     "carried from layer to layer, each layer's routing read through mapped memory without a stream "
                     "synchronisation, the next layer's routing queued behind each block, lookahead depth 1 of top_k "
                     "experts, one tick per token), after the warm-up tokens"}
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
    log(f"bench: 4-layer synthetic store (D 512, 32 experts top-4), whole step: prefill {out['prefill_tok_s']:.0f} tok/s, decode {out['decode_tok_s']:.0f} tok/s "
        f"({out['decode_us_per_token']:.1f} us/token); reference CPU {out.get('reference_cpu')}")
    return out


def c3_geometry_bytes(g):
    """Packed weight bytes one decode token reads at geometry g (dict), and
    the KV bytes per cached position."""
    q80 = lambda rows, n: rows * (n // 32) * 34            # noqa: E731
    q6k = lambda rows, n: rows * (n // 256) * 210          # noqa: E731
    D, hd, H, KV, E, k, de = (g[x] for x in ("d_model", "head_dim", "n_heads", "n_kv_heads", "n_experts", "top_k",
                                             "d_expert"))
    attn = q80(H * hd, D) + 2 * q80(KV * hd, D) + q80(D, H * hd)
    router = E * D * 4
    experts = k * (2 * q6k(de, D) + q6k(D, de))
    layer = attn + router + experts
    weights = g["n_layers"] * layer + q80(g["vocab"], D)
    kv_per_pos = g["n_layers"] * KV * hd * 4 * 2
    return {"weights_per_token": weights, "attention_per_layer": attn, "router_per_layer": router,
            "experts_per_layer": experts, "lm_head": q80(g["vocab"], D), "kv_per_position": kv_per_pos}


def c3_bench(torch, steps, warmup, ctx, split=False):
    """The headline: whole-model decode at Qwen3-30B-A3B shape, K steps at
    positions spread evenly over 64..ctx-1 (see the module docstring).
    split: the split attention option instead of the reference's order."""
    from tierlm_amd.model import QWEN3_30B_A3B, Model, bench_prompt
    t0 = time.perf_counter()
    m = Model.synth(QWEN3_30B_A3B, expert_dt=Q6_K, dense_dt=8, seed=1, max_ctx=ctx, split=split)
    built = time.perf_counter() - t0
    try:
        prompt = bench_prompt(64, QWEN3_30B_A3B["vocab"])
        m.reset()
        t0 = time.perf_counter()
        toks = m.generate(prompt, ctx - 64)          # fills the context to ctx - 1 positions (graph captured)
        fill_s = time.perf_counter() - t0
        top = ctx - 1
        assert m.kv_len() == top
        # descending, evenly over 64..top, both ends included
        positions = [top - (i * (top - 64)) // (steps - 1) for i in range(steps)] if steps > 1 else [top]
        w = max(1, warmup)
        m.rewind(top - w)
        m.decode(w)                                  # warm-up steps (untimed), back at top positions
        m.sync()
        st = torch.cuda.ExternalStream(m.stream())
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        h0 = time.perf_counter()
        ev0.record(st)
        for p in positions:
            m.rewind(p)
            m.decode(1)
        ev1.record(st)
        m.sync()
        wall = time.perf_counter() - h0
        ev1.synchronize()
        ev_s = ev0.elapsed_time(ev1) * 1e-3
        # batched prefill of a (ctx - 1)-token prompt (tlm_model_prefill's
        # result, 1024-token chunks): first run allocates, best of the next two
        pf_prompt = bench_prompt(ctx - 1, QWEN3_30B_A3B["vocab"], seed=7)
        pf = []
        for _ in range(3):
            m.reset()
            t0 = time.perf_counter()
            m.prefill(pf_prompt)
            pf.append(time.perf_counter() - t0)
        prefill_s = min(pf[1:])
        batched = m.prefill_batched()
    finally:
        m.close()
    gb = c3_geometry_bytes(QWEN3_30B_A3B)
    kv_mean = sum((p + 1) * gb["kv_per_position"] for p in positions) / len(positions)
    per_tok = gb["weights_per_token"] + kv_mean
    sec = ev_s / steps
    achieved = per_tok / sec / 1e9
    log(f"bench: Qwen3-30B-A3B-shape decode{' (split attention)' if split else ''}: {steps / ev_s:.1f} tok/s over "
        f"{steps} steps at positions "
        f"{positions[-1]}..{positions[0]} ({sec * 1e3:.3f} ms/token events, {wall / steps * 1e3:.3f} ms/token host); "
        f"{per_tok / 1e9:.3f} GB/token = {achieved:.0f} GB/s; context fill {ctx - 64} tokens in {fill_s:.1f} s "
        f"({(ctx - 64) / fill_s:.1f} tok/s); prefill {ctx - 1} tokens in {prefill_s * 1e3:.1f} ms "
        f"({(ctx - 1) / prefill_s:.0f} tok/s{'' if batched else ', one step per token'})")
    return {"prefill_tok_s": (ctx - 1) / prefill_s, "prefill_ms": prefill_s * 1e3, "prefill_batched": batched,
            "tok_s": steps / ev_s, "ms_per_step": sec * 1e3, "wall_ms_per_step": wall / steps * 1e3,
            "positions": [positions[-1], positions[0]], "bytes_per_token": per_tok, "weights_per_token":
            gb["weights_per_token"], "kv_bytes_per_token_mean": kv_mean, "achieved_GBps": achieved,
            "build_s": built, "fill_tok_s": (ctx - 64) / fill_s, "tokens_head": toks[:4], "geometry_bytes": gb}


# the Qwen3-235B-A22B geometry with sigmoid routing, whose selection bias
# gives the experts a Zipf-like heat (the slot-cache legs)
QWEN3_235B_A22B = dict(n_layers=94, d_model=4096, n_heads=64, n_kv_heads=4, head_dim=128, vocab=151936,
                      n_experts=128, top_k=8, d_expert=1536, n_shared=0, d_shared=0, max_ctx=40960, router=2,
                      rope_theta=1e6, norm_eps=1e-6, routed_scale=1.0)


def c5_model_bench(torch, tokens, cache_gb, prompt_len=32, warm=40, pool=64, gamma=0.14, pf_len=512, expert_dt=12):
    """The whole Qwen3-235B-A22B-shaped model (94 layers, hidden 4096, 64 q / 4
    kv heads x 128 with qk-norm, 128 experts top-8 of width 1536 in Q4_K
    (expert_dt 12) or Q5_K (13), Q8_0 dense and lm_head, vocabulary 151936,
    random init) decoding with its experts behind the HBM slot cache capped at
    cache_gb: the payloads (Q4_K: 127.7 GB as the cache sees them, 12,032
    experts of 10.6 MB; Q5_K: 156.1 GB, 13.0 MB each; drawn from a pool of
    `pool` distinct payloads in page-locked host memory so the host holds a
    few GB at most) load over PCIe on a miss; sigmoid routing with the
    Zipf-like selection bias -gamma ln(rank + 1) on a per-layer order of the
    experts; the reference runtime's store defaults (pin share 0.30, router
    lookahead one layer ahead, top_k hints).  A prompt, `warm` greedy tokens
    to fill the cache, then `tokens` timed greedy tokens (host clock around
    the steps).  Then, with pf_len > 0, from an empty context and the cache as
    decoding left it, a `pf_len`-token prompt prefilled batched through the
    cache (each layer's union of the prompt's experts acquired once), host
    clock around tlm_hip_model_prefill."""
    from tierlm_amd.model import Model, bench_prompt
    t0 = time.perf_counter()
    m = Model.synth(QWEN3_235B_A22B, expert_dt=expert_dt, dense_dt=8, seed=11,
                    max_ctx=max(prompt_len + warm + tokens, pf_len) + 8,
                    expert_pool=pool, heat_gamma=gamma, expert_cache=int(cache_gb * (1 << 30)))
    built = time.perf_counter() - t0
    try:
        p = bench_prompt(prompt_len, QWEN3_235B_A22B["vocab"])
        m.reset()
        m.generate(p, warm)
        m.sync()
        s0 = m.store_stats()
        h0 = time.perf_counter()
        m.decode(tokens)
        m.sync()
        dt = time.perf_counter() - h0
        s1 = m.store_stats()
        if pf_len > 0:
            assert m.prefill_batched()
            m.reset()
            pp = bench_prompt(pf_len, QWEN3_235B_A22B["vocab"], seed=7)
            m.sync()
            h1 = time.perf_counter()
            m.prefill(pp, logits=False)
            m.sync()
            pf_dt = time.perf_counter() - h1
            s2 = m.store_stats()
    finally:
        m.close()
    L, K = QWEN3_235B_A22B["n_layers"], QWEN3_235B_A22B["top_k"]
    miss = (s1["misses"] - s0["misses"]) / tokens
    pre = (s1["prefetch_issued"] - s0["prefetch_issued"]) / tokens
    bb = 144 if expert_dt == Q4_K else 176
    plen = 2 * 1536 * (4096 // 256 * bb) + 4096 * (1536 // 256 * bb)
    name = "Q4_K" if expert_dt == Q4_K else "Q5_K"
    r = {"model": f"Qwen3-235B-A22B shape, whole model: 94 layers, hidden 4096, 64 q / 4 kv heads x 128, qk-norm, "
                  f"128 experts top-8 of width 1536 ({name}, {plen / 1e6:.1f} MB each, {plen * 12032 / 1e9:.1f} GB) "
                  f"behind the HBM slot cache, Q8_0 dense and lm_head, vocabulary 151936, random init",
         "expert_dtype": name,
         "cache_GB": cache_gb, "slots": s1["slots"], "pinned": s1["pinned"], "tokens": tokens,
         "warmup_tokens": warm, "prompt": prompt_len, "tok_s": round(tokens / dt, 2),
         "ms_per_token": round(dt / tokens * 1e3, 2), "misses_per_token": round(miss, 2),
         "hit_rate": round(1.0 - miss / (L * K), 4), "prefetch_issued_per_token": round(pre, 2),
         "load_GBps": round((miss + pre) * plen * tokens / dt / 1e9, 2), "build_s": round(built, 1),
         "prefill": None if pf_len <= 0 else {"prompt": pf_len, "ms": round(pf_dt * 1e3, 1), "tok_s": round(pf_len / pf_dt, 1),
                     "acquires": s2["hits"] + s2["misses"] - s1["hits"] - s1["misses"],
                     "misses": s2["misses"] - s1["misses"],
                     "load_GBps": round((s2["misses"] - s1["misses"]) * plen / pf_dt / 1e9, 2),
                     "timing": "host wall clock around tlm_hip_model_prefill of the prompt (batched, 1024-token "
                               "chunks, each layer's union of the chunk's experts through the cache) and a sync"},
         "timing": "host wall clock around tlm_hip_model_decode of the timed tokens and a sync, after the prompt and "
                   "the warm-up tokens"}
    log(f"bench: Qwen3-235B-A22B-shape whole model, {name} experts, through the slot cache ({r['slots']} slots, {cache_gb:.0f} GB): {r['tok_s']:.2f} tok/s "
        f"({r['ms_per_token']:.2f} ms/token), {r['misses_per_token']:.2f} misses/token (hit rate {r['hit_rate']:.4f}), "
        f"{r['prefetch_issued_per_token']:.1f} lookahead loads/token, {r['load_GBps']:.2f} GB/s over PCIe")
    q = r["prefill"]
    if q:
        log(f"bench: Qwen3-235B-A22B-shape {pf_len}-token prompt batched through the slot cache: {q['ms']:.1f} ms = "
            f"{q['tok_s']:.1f} tok/s, {q['acquires']} acquires, {q['misses']} misses ({q['load_GBps']:.2f} GB/s over PCIe)")
    return r


def host_cores():
    """Physical cores of the host and of this process's CPU set (distinct
    (package, core) pairs), and the thread count the CPU baseline uses: every
    physical core of the CPU set, at most 16 (the CPU share a one-GPU job
    has on the GPU hosts)."""
    def core_of(c):
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            with open(base + "physical_package_id") as f:
                pkg = f.read().strip()
            with open(base + "core_id") as f:
                core = f.read().strip()
            return (pkg, core)
        except OSError:
            return ("?", str(c))
    online = [int(d[3:]) for d in os.listdir("/sys/devices/system/cpu") if d[3:].isdigit()]
    mine = sorted(os.sched_getaffinity(0))
    phys_host = len({core_of(c) for c in online}) or (os.cpu_count() or 1)
    phys_mine = len({core_of(c) for c in mine}) or len(mine)
    threads = max(1, min(16, phys_mine))
    return {"host_physical_cores": phys_host, "host_logical_cpus": len(online), "process_cpus": len(mine),
            "process_physical_cores": phys_mine, "threads": threads,
            "note": (f"{phys_mine} physical cores in this process's CPU set of {len(mine)} CPUs "
                     f"(host: {phys_host} physical cores, {len(online)} logical CPUs)"
                     + ("; capped at the 16-CPU share of a one-GPU job" if phys_mine > 16 else ""))}


def q6k_kernel_gbps(seconds=0.5):
    """The reference's own single-thread kernel figure (tests/test_quant.c:
    897-938): tlm_matvec_rows of a 4096 x 4096 Q6_K matrix against a Q8_K
    activation, weight bytes / best time (a 13.8 MB matrix may sit in a large
    last-level cache: a kernel, not a memory, figure)."""
    import ctypes as C

    import numpy as np

    import oracle
    from tests.synth import random_code_rows
    rng = np.random.default_rng(5)
    W = random_code_rows(rng, Q6_K, 4096, 4096)
    x = rng.standard_normal(4096).astype(np.float32)
    y = np.empty(4096, np.float32)
    handle = oracle.ref.refmoe_new(1)
    try:
        Wp = (C.c_void_p * 1)(W.ctypes.data)
        R = (C.c_int64 * 1)(4096)
        Y = (C.c_void_p * 1)(y.ctypes.data)
        oracle.ref.refmoe_matvecs(handle, Q6_K, Wp, R, 4096, x.ctypes.data, Y, 1)   # warm
        best, spent, it = 1e30, 0.0, 0
        while (spent < seconds and it < 400) or it < 2:
            t0 = time.perf_counter()
            oracle.ref.refmoe_matvecs(handle, Q6_K, Wp, R, 4096, x.ctypes.data, Y, 1)
            dt = time.perf_counter() - t0
            best = min(best, dt)
            spent += dt
            it += 1
    finally:
        oracle.ref.refmoe_free(handle)
    return {"GBps": round(W.nbytes / best / 1e9, 2), "tier": oracle.ref.refmoe_tier().decode(), "runs": it,
            "note": "tlm_matvec_rows, one thread, best of the runs; the activation quantised inside each run"}


def cpu_baseline(args, threads):
    """The reference's kernels on the host cores for a bounded sample of the
    per-token work at Qwen3-30B-A3B shape (oracle/_ref): one layer's q|k|v
    and o projections and routed MoE block, repeated, and the lm_head; tok/s
    = 1 / (48 x layer + lm_head)."""
    import ctypes as C

    import numpy as np

    import oracle
    from tests.synth import random_code_rows
    if oracle.ref is None:
        return None
    rng = np.random.default_rng(3)
    Q8_0 = 8
    H, KVH, HD, V = 32, 4, 128, 151936
    experts = [(random_code_rows(rng, Q6_K, DE, D), random_code_rows(rng, Q6_K, DE, D),
                random_code_rows(rng, Q6_K, D, DE)) for _ in range(E)]
    host = oracle.MoeHost(D=D, de=DE, E=E, k=K, expert_dt=Q6_K, ffn_norm=np.ones(D, np.float32),
                          router_w=(rng.standard_normal((E, D)) / np.sqrt(D)).astype(np.float32), experts=experts)
    # 8 distinct layers of dense weights (160 MB) beside the 495 MB of experts and the 330 MB
    # lm_head, so the sample streams from memory rather than the host's last-level cache
    NL = 8
    dense = [[random_code_rows(rng, Q8_0, r, D) for r in (H * HD, KVH * HD, KVH * HD)] +
             [random_code_rows(rng, Q8_0, D, H * HD)] for _ in range(NL)]
    wl = random_code_rows(rng, Q8_0, V, D)
    ys = [np.empty(r, np.float32) for r in (H * HD, KVH * HD, KVH * HD, D, V)]
    xs = rng.standard_normal((64, H * HD)).astype(np.float32)

    def mvs(handle, mats, n, x, outs):
        W = (C.c_void_p * len(mats))(*[mm.ctypes.data for mm in mats])
        R = (C.c_int64 * len(mats))(*[mm.shape[0] for mm in mats])
        Y = (C.c_void_p * len(mats))(*[o.ctypes.data for o in outs])
        oracle.ref.refmoe_matvecs(handle, Q8_0, W, R, n, x.ctypes.data, Y, len(mats))

    handle = oracle.ref.refmoe_new(threads)
    try:
        def layer(i):
            x = xs[i % 64]
            wq, wk, wv, wo = dense[i % NL]
            mvs(handle, [wq, wk, wv], D, np.ascontiguousarray(x[:D]), ys[:3])
            mvs(handle, [wo], H * HD, x, [ys[3]])
            host.run_ref(handle, np.ascontiguousarray(x[:D]))

        layer(0)
        t0, n = time.perf_counter(), 0
        while time.perf_counter() - t0 < args.cpu_seconds * 0.8 or n < 4:
            layer(n)
            n += 1
        t_layer = (time.perf_counter() - t0) / n
        mvs(handle, [wl], D, np.ascontiguousarray(xs[0][:D]), [ys[4]])
        t0, nl = time.perf_counter(), 0
        while time.perf_counter() - t0 < args.cpu_seconds * 0.2 or nl < 2:
            mvs(handle, [wl], D, np.ascontiguousarray(xs[nl % 64][:D]), [ys[4]])
            nl += 1
        t_lm = (time.perf_counter() - t0) / nl
    finally:
        oracle.ref.refmoe_free(handle)
    tier = oracle.ref.refmoe_tier().decode()
    per_tok = 48 * t_layer + t_lm
    return {"value": round(1.0 / per_tok, 3), "unit": "tok/s", "cores": threads, "kind": "reference",
            "sample": f"{n} layers (q|k|v + o Q8_0 projections cycling 8 distinct layers, and the routed top-8 Q6_K "
                      f"MoE block over 128 random-code experts, at Qwen3-30B-A3B shape; about 1 GB of weights in "
                      f"all) and {nl} lm_head passes (151936 x 2048 Q8_0) "
                      f"through the reference's {tier} tier + pool on {threads} threads; tok/s = 1 / (48 x "
                      f"{t_layer * 1e3:.2f} ms + {t_lm * 1e3:.2f} ms); attention arithmetic and norms not included",
            "layer_ms": round(t_layer * 1e3, 3), "lm_head_ms": round(t_lm * 1e3, 3)}


def expert_gemv_bench(torch, dev, args, gen):
    """The routed MoE block alone at Qwen3-30B-A3B shape (one layer per token,
    --layers resident copies of the 128 experts cycled, HIP graphs of --graph
    tokens), and per phase the average launch time from a graph of
    back-to-back launches of that phase (HIP events).  Returns the block's
    figures and the weights/tensors the prefill and cache legs reuse."""
    import numpy as np
    from tierlm_amd import MoeBlock
    L = args.layers
    log(f"bench: allocating {L} x {E} Q6_K experts ({L * E * EXPERT_BYTES / 1e9:.1f} GB)")
    W = make_weights(torch, dev, L, seed=1)
    router_w = torch.randn((E, D), generator=gen, device=dev) / float(np.sqrt(D))
    ffn_norm = torch.ones(D, device=dev)
    blocks = []
    base = W.data_ptr()
    for layer in range(L):
        ptrs = [base + ((layer * E + e) * 3 + j) * MAT_BYTES for e in range(E) for j in range(3)]
        blocks.append(MoeBlock(D=D, de=DE, E=E, k=K, expert_dt=Q6_K, ffn_norm=ffn_norm, router_w=router_w,
                               expert_ptrs=ptrs, router=0, eps=1e-6, device=dev))
    ntok, warm = args.c2_tokens, 200
    total = warm + ntok
    H = torch.randn((max(total, args.roofline_tokens), D), generator=gen, device=dev)
    torch.cuda.synchronize()

    def run_tokens(t0, t1):
        for t in range(t0, t1):
            blocks[t % L](H[t])

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run_tokens(0, min(args.graph, total))
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    def capture(t0, t1):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            run_tokens(t0, t1)
        return g
    G = args.graph
    warm_graphs = [capture(t, min(t + G, warm)) for t in range(0, warm, G)]
    graphs = [capture(t, min(t + G, total)) for t in range(warm, total, G)]
    for g in warm_graphs:
        g.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for g in graphs:
        g.replay()
    ev1.record()
    ev1.synchronize()
    block_us = ev0.elapsed_time(ev1) * 1e3 / ntok
    del graphs, warm_graphs

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
    log(f"bench: MoE block {1e6 / block_us:.0f} tok/s ({block_us:.2f} us/token); per launch: router {p1:.2f} us, "
        f"gate/up {p2:.2f} us ({gu_gbs:.0f} GB/s), down+combine {p3:.2f} us ({dn_gbs:.0f} GB/s)")
    block_gbs = TOKEN_BYTES / (block_us * 1e-6) / 1e9
    out = {"workload": "one routed MoE block per token at Qwen3-30B-A3B shape (D 2048, 128 experts top-8 "
                       "softmax+renorm, expert width 768, Q6_K experts, f32 router), "
                       f"{L} resident layer copies cycled; {ntok} timed tokens of N(0,1) residuals (seeded); "
                       "the experts are random 6-bit codes with scales of N(0,0.02)-quantised magnitude, not "
                       "quantised N(0,0.02) draws (the kernels' speed does not depend on the values)",
           "block_tok_s": round(1e6 / block_us, 1),
           "block_us_per_token": round(block_us, 3), "tokens": ntok,
           "expert_bytes_per_token": TOKEN_BYTES, "expert_gemv_GBps": round(expert_gbs, 1),
           "expert_gemv_frac": round(expert_gbs / HBM_PEAK_GBS, 4),
           "block_GBps": round(block_gbs, 1), "block_frac": round(block_gbs / HBM_PEAK_GBS, 4),
           "frac_note": "expert_gemv_frac: expert bytes / (gate/up + down launch times); block_frac: expert bytes "
                        "/ the whole block's time per token (router, routing and launch gaps included)",
           "gateup": {"kernel": "k_moe_gateup (routing + gate/up of the top-8 experts + SwiGLU)",
                      "bytes_per_launch": GATEUP_BYTES, "avg_launch_us": round(p2, 3),
                      "achieved_GBps": round(gu_gbs, 1), "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                      "traffic": GATEUP_TRAFFIC_BYTES,
                      "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per dispatch, scaled by a 256 MiB copy"},
           "down_combine": {"bytes_per_launch": DOWN_BYTES, "avg_launch_us": round(p3, 3),
                            "achieved_GBps": round(dn_gbs, 1)},
           "router_avg_launch_us": round(p1, 3),
           "timing": "HIP events: the block over graphs of --graph tokens; per phase a graph of "
                     f"{R} back-to-back launches of that phase, / {R} (best of 3)"}
    return out, W, router_w, ffn_norm


Q8_0 = 8
# the decode step's dense Q8_0 matrices at the Qwen3-30B-A3B shape: q|k|v (32 + 4 + 4 heads x 128
# rows of 2048), o (2048 rows of 4096), lm_head (151936 rows of 2048)
DENSE_SHAPES = [("qkv", 5120, 2048), ("o", 2048, 4096), ("lm_head", 151936, 2048)]


def dense_gemv_bench(torch, dev, layers, reps, gen):
    """The decode step's dense Q8_0 GEMVs through tlm_hip_matvec_packed (the
    step's segmented launch with one segment, activation given quantised):
    per shape, random code bytes in the packed layout (`layers` copies of
    q|k|v and o and two of lm_head cycled, so that no launch finds its matrix
    in the 256 MB last-level cache), a graph of `reps` back-to-back launches,
    HIP events, best of 3."""
    from tierlm_amd import quant as hq
    out = {}
    for name, rows, n in DENSE_SHAPES:
        copies = 2 if name == "lm_head" else layers
        pb = hq.packed_bytes(Q8_0, rows, n)
        W = torch.empty((copies, pb), dtype=torch.uint8, device=dev).random_(0, 256, generator=gen)
        act = hq.quantize_act(Q8_0, torch.randn(n, generator=gen, device=dev))
        y = torch.empty(rows, dtype=torch.float32, device=dev)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            hq.matvec_packed(Q8_0, W[0], rows, n, act, y)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for t in range(reps):
                hq.matvec_packed(Q8_0, W[t % copies], rows, n, act, y)
        g.replay()
        torch.cuda.synchronize()
        best = None
        for _ in range(3):
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record()
            g.replay()
            ev1.record()
            ev1.synchronize()
            us = ev0.elapsed_time(ev1) * 1e3 / reps
            best = us if best is None else min(best, us)
        del g, W
        gbs = pb / (best * 1e-6) / 1e9
        out[name] = {"rows": rows, "n": n, "bytes_per_launch": pb, "avg_launch_us": round(best, 3),
                     "achieved_GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": DENSE_TRAFFIC_BYTES.get(name)}
    log("bench: dense GEMVs per launch: " + ", ".join(
        f"{k} {v['avg_launch_us']:.2f} us ({v['achieved_GBps']:.0f} GB/s)" for k, v in out.items()))
    out["timing"] = (f"HIP events around a graph of {reps} back-to-back launches per shape, / {reps} (best of 3); "
                     f"random code bytes, activation quantised once; {layers} copies of q|k|v and o, 2 of lm_head, "
                     "cycled")
    out["traffic_source"] = ("rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per dispatch of this leg, each scaled by its "
                             "reading for a 256 MiB device copy")
    return out


def stream_read_peak(torch, dev, nbytes):
    """A plain streaming read (tlm_hip_stream_read) over nbytes of device
    memory, best of 5, HIP events."""
    import ctypes as C

    from tierlm_amd._lib import check, lib
    from tierlm_amd.quant import stream
    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(7)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    check(lib.tlm_hip_stream_read(C.c_void_p(buf.data_ptr()), nbytes, C.c_void_p(sink.data_ptr()), stream()))
    torch.cuda.synchronize()
    best = None
    for _ in range(5):
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        check(lib.tlm_hip_stream_read(C.c_void_p(buf.data_ptr()), nbytes, C.c_void_p(sink.data_ptr()), stream()))
        ev1.record()
        ev1.synchronize()
        us = ev0.elapsed_time(ev1) * 1e3
        best = us if best is None else min(best, us)
    del buf
    gbs = nbytes / (best * 1e-6) / 1e9
    log(f"bench: plain streaming read of {nbytes / 1e9:.2f} GB: {gbs:.0f} GB/s")
    return {"GBps": round(gbs, 1), "bytes": nbytes, "us": round(best, 1),
            "kernel": "k_stream_read: 16-byte loads, eight in flight per lane, 2048 groups of 256, grid-stride"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1984, help="timed decode steps (positions spread over 64..2047)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--c3-context", type=int, default=2048, help="context the decode positions span")
    ap.add_argument("--split-steps", type=int, default=248,
                    help="steps of the same sweep with the split attention option (0: skip)")
    ap.add_argument("--layers", type=int, default=48, help="MoE block: distinct layer copies cycled by the tokens")
    ap.add_argument("--c2-tokens", type=int, default=10000, help="MoE block: timed tokens")
    ap.add_argument("--graph", type=int, default=100, help="MoE block: tokens per captured HIP graph")
    ap.add_argument("--roofline-tokens", type=int, default=960, help="MoE block: launches per phase graph")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-c2", action="store_true", help="skip the MoE-block measurement (and prefill / cache)")
    ap.add_argument("--no-prefill", action="store_true", help="skip the 512-token prefill measurement")
    ap.add_argument("--no-store", action="store_true", help="skip the expert slot cache measurement")
    ap.add_argument("--no-c1", action="store_true", help="skip the whole-step synthetic model measurement")
    ap.add_argument("--no-c3", action="store_true",
                    help="skip the whole-model decode legs (graph replays): for profiler runs, which trace the "
                         "other legs only; the line then carries no value")
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
    if args.steps < 1:
        ap.error("--steps must be at least 1")

    import torch

    from tierlm_amd import quant as hq

    dev = torch.device("cuda", 0)
    hq.init(0)
    assert hq.selftest_failures() == 0, "HIP self-test failures"

    c3 = c3s = None
    if not args.no_c3:
        c3 = c3_bench(torch, args.steps, args.warmup, args.c3_context)
        torch.cuda.empty_cache()
    if args.split_steps > 0 and not args.no_c3:
        c3s = c3_bench(torch, args.split_steps, args.warmup, args.c3_context, split=True)
        torch.cuda.empty_cache()
    peak = stream_read_peak(torch, dev, 2 << 30)

    gen = torch.Generator(device=dev)
    gen.manual_seed(2)
    c2 = prefill = prefill_q5k = slot_cache = None
    dense = None
    if not args.no_c2:
        c2, W, router_w, ffn_norm = expert_gemv_bench(torch, dev, args, gen)
        dense = dense_gemv_bench(torch, dev, args.layers, args.roofline_tokens, gen)
        if args.copy_check_mib > 0:
            nbytes = args.copy_check_mib << 20
            src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
            dst = torch.empty_like(src)
            torch.cuda.synchronize()
            dst.copy_(src)
            torch.cuda.synchronize()
            log(f"bench: copy check {args.copy_check_mib} MiB done")
            del src, dst
        if not args.no_prefill:
            prefill = prefill_bench(torch, dev, W, MAT_BYTES, Q6_K, router_w, ffn_norm, gen)
            W5 = make_weights_q5k(torch, dev, seed=5)
            prefill_q5k = prefill_bench(torch, dev, W5, MAT_BYTES_Q5K, Q5_K, router_w, ffn_norm, gen)
            del W5
        if not args.no_store:
            slot_cache = slot_cache_bench(torch, dev, router_w, ffn_norm, gen, args.store_tokens)
        del W
        torch.cuda.empty_cache()
    c1 = None if args.no_c1 or not os.path.exists(C1_STORE) else c1_bench(3)
    c5 = c5m = c5q5 = None
    if not args.no_c5:
        try:
            c5 = c5_bench(torch, dev, args.c5_tokens, args.c5_cache_gb)
        except Exception as e:                 # recorded, so the rest of the line still prints
            c5 = {"error": repr(e)}
            log(f"bench: Qwen3-235B-A22B-shape slot-cache stack failed: {e!r}")
        torch.cuda.empty_cache()
        try:
            c5m = c5_model_bench(torch, args.c5_tokens, args.c5_cache_gb)
        except Exception as e:
            c5m = {"error": repr(e)}
            log(f"bench: Qwen3-235B-A22B-shape whole model failed: {e!r}")
        torch.cuda.empty_cache()
        try:
            c5q5 = c5_model_bench(torch, args.c5_tokens, args.c5_cache_gb, pf_len=0, expert_dt=13)
        except Exception as e:
            c5q5 = {"error": repr(e)}
            log(f"bench: Qwen3-235B-A22B-shape whole model (Q5_K) failed: {e!r}")
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        cores = host_cores()
        threads = cores["threads"]
        log(f"bench: cpu baseline ({threads} threads: {cores['note']}; ~{args.cpu_seconds:.0f} s), then 1 thread")
        cpu = cpu_baseline(args, threads)
        if cpu:
            cpu["host_cores"] = cores
            one = cpu_baseline(args, 1)
            cpu["one_thread"] = {k: one[k] for k in ("value", "unit", "cores", "layer_ms", "lm_head_ms")}
            cpu["q6_k_4096x4096_1thread"] = q6k_kernel_gbps()
            if c3:
                cpu["gpu_over_cpu"] = round(c3["tok_s"] / cpu["value"], 1)
                cpu["gpu_over_cpu_1thread"] = round(c3["tok_s"] / one["value"], 1)
    if c3 is None:   # --no-c3: the other legs only
        print(json.dumps({"metric": "decode tok/s batch-1, Qwen3-30B-A3B shape; expert GEMV HBM GB/s vs peak",
                          "value": None, "unit": "tok/s", "n_gpus": 1, "note": "--no-c3: whole-model legs skipped",
                          "expert_gemv": c2, "dense_gemv": dense, "cpu_baseline": cpu, "prefill": prefill,
                          "prefill_q5k": prefill_q5k,
                          "slot_cache": slot_cache, "c1_whole_step": c1, "stream_read": peak,
                          "qwen3_235b_a22b_slot_cache": c5, "qwen3_235b_a22b_model": c5m,
                          "qwen3_235b_a22b_model_q5k": c5q5}), flush=True)
        return

    line = {
        "metric": "decode tok/s batch-1, Qwen3-30B-A3B shape; expert GEMV HBM GB/s vs peak",
        "value": round(c3["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(c3["ms_per_step"], 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8xu6/int8->int32 (Q6_K/Q8_0 x Q8_K/a8), f32 chains", "data": "synthetic",
        "config": {"workload": "whole-model batch-1 greedy decode to 2048 positions, Qwen3-30B-A3B shape: 48 layers, "
                               "hidden 2048, 32 q / 4 kv heads x 128, 128 experts top-8 of width 768 (Q6_K, all "
                               "resident), Q8_0 dense, f32 router, vocabulary 151936, random init in HBM; one step = "
                               "one token at a context position spread evenly over 64..2047",
                   "positions": c3["positions"], "context": args.c3_context,
                   "wall_ms_per_step": round(c3["wall_ms_per_step"], 4),
                   "timing": "HIP events on the model's stream around exactly K steps (each a context rewind + "
                             "one replay of the captured step graph)"},
        "roofline": {"bound": "hbm", "achieved": round(c3["achieved_GBps"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(c3["achieved_GBps"] / HBM_PEAK_GBS, 4),
                     "traffic": int(48 * STEP_LAYER_TRAFFIC_BYTES + DENSE_TRAFFIC_BYTES["lm_head"]
                                    + c3["kv_bytes_per_token_mean"]),
                     "traffic_source": "the step's launches summed: per layer the q|k|v, o, router, gate/up and down "
                                       "kernels' HBM bytes per dispatch (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of "
                                       "the same kernels at the same shapes in the MoE-block and dense-GEMV legs, "
                                       "scaled by a 256 MiB copy), 48 layers, plus lm_head's, plus the mean K / V "
                                       "read at its algorithmic bytes",
                     "kernel": "the decode step (its kernels' algorithmic bytes / the step time)",
                     "bytes_per_step": int(c3["bytes_per_token"]),
                     "weights_per_step": c3["weights_per_token"],
                     "kv_bytes_per_step_mean": int(c3["kv_bytes_per_token_mean"]),
                     "avg_step_us": round(c3["ms_per_step"] * 1e3, 2),
                     "stream_read_peak_GBps": peak["GBps"], "stream_read_frac": round(
                         c3["achieved_GBps"] / peak["GBps"], 4),
                     "stream_read_kernel": peak["kernel"]},
        "expert_gemv": c2,
        "dense_gemv": dense,
        "cpu_baseline": cpu,
        "prefill": prefill,
        "prefill_q5k": prefill_q5k,
        "slot_cache": slot_cache,
        "c1_whole_step": c1,
        "qwen3_30b_a3b_context_fill_tok_s": round(c3["fill_tok_s"], 1),
        "qwen3_30b_a3b_prefill": {
            "tokens": args.c3_context - 1, "ms": round(c3["prefill_ms"], 2), "tok_s": round(c3["prefill_tok_s"], 1),
            "batched": c3["prefill_batched"],
            "timing": "host wall clock around tlm_hip_model_prefill (prompt upload, the batched chunks, the last "
                      "token's lm_head and logits download), best of 2 after one run that allocates",
            "note": "each token's cache entries, logits and greedy token are the step-by-step prefill's bits"},
        "qwen3_30b_a3b_split_attention": None if c3s is None else {
            "tok_s": round(c3s["tok_s"], 2), "ms_per_step": round(c3s["ms_per_step"], 4), "steps": args.split_steps,
            "positions": c3s["positions"],
            "note": "the same decode with the attn_split option (per-slice partial softmax and P.V, merged per head): "
                    "attention outputs within float rounding of the reference's, logits not bit-identical (int8 "
                    "activation codes and near-tied top-k routing amplify the differences); greedy tokens equal on "
                    "the reference fixtures"},
        "qwen3_235b_a22b_slot_cache": c5,
        "qwen3_235b_a22b_model": c5m,
        "qwen3_235b_a22b_model_q5k": c5q5,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
