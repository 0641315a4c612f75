"""The whole decode step on the device (tlm_hip_model_*; the reference's
tlm_model_step / tlm_model_prefill, src/lib/tlm_model.c:1058-1113) for a
compiled store, through ctypes.  Computes nothing itself.

    python -m tierlm_amd.model STORE.tlmm [--prompt-len 64] [-n 64] [--eager]
    python -m tierlm_amd.model --synth qwen3-30b-a3b [--layers 48] ...

times the device the way `tierlm bench` times the host runtime
(src/bin/tierlm.c:702-735): a pseudo-random prompt, prefill, then greedy
tokens; decode tok/s = (n - 1) / decode time.  --synth times a random-init
model of that shape built in HBM (tlm_hip_model_synth) instead of a store."""
import ctypes as C
import time

import numpy as np

from ._lib import check, lib


class ModelOpts(C.Structure):
    """tlm_hip_model_opts"""
    _fields_ = [("max_ctx", C.c_int32), ("eager", C.c_int32), ("attn_slices", C.c_int32), ("attn_split", C.c_int32),
                ("expert_cache_bytes", C.c_uint64), ("pin_frac", C.c_double), ("prefetch_off", C.c_int32),
                ("lookahead_k", C.c_int32), ("interest", C.c_double), ("prefill_chunk", C.c_int32),
                ("stats", C.c_int32), ("host_routes", C.c_int32)]


class ModelStats(C.Structure):
    """tlm_hip_model_stats (tlm_model_stats)"""
    _fields_ = [("tokens", C.c_uint64), ("attn_ns", C.c_uint64), ("moe_ns", C.c_uint64),
                ("expert_wait_ns", C.c_uint64), ("other_ns", C.c_uint64)]


def model_opts(max_ctx=0, eager=False, attn_slices=0, split=False, expert_cache=0, pin_frac=0.0, prefetch=True,
               lookahead_k=0, interest=0.0, prefill_chunk=0, stats=False, host_routes=False):
    """tlm_hip_model_opts; expert_cache > 0 (bytes) serves the experts through
    an HBM slot cache of that size from page-locked host memory, as tierlm's
    runtime serves them from its store (pin_frac 0 = its default 0.30,
    prefetch = its router lookahead, lookahead_k / interest its io and nav
    options); prefill_chunk: 0 batched prompts where the model allows them,
    n > 0 at most n tokens per batch, < 0 one step per token; stats: the
    device-timed attention / MoE / other split of tlm_model_stats;
    host_routes: the host resolves each layer's slots instead of the device."""
    return ModelOpts(max_ctx, int(eager), attn_slices, int(split), int(expert_cache), float(pin_frac),
                     0 if prefetch else 1, int(lookahead_k), float(interest), int(prefill_chunk), int(stats),
                     int(host_routes))


# Qwen3-30B-A3B: 48 layers, hidden 2048, 32 q / 4 kv heads x 128, 128
# experts top-8 of width 768, vocabulary 151936, qk-norm, rope theta 1e6
QWEN3_30B_A3B = dict(n_layers=48, d_model=2048, n_heads=32, n_kv_heads=4, head_dim=128, vocab=151936,
                     n_experts=128, top_k=8, d_expert=768, n_shared=0, d_shared=0, max_ctx=40960, router=0,
                     rope_theta=1e6, norm_eps=1e-6, routed_scale=1.0)

# Qwen3-235B-A22B: 94 layers, hidden 4096, 64 q / 4 kv heads x 128 (16 query
# heads per key head), 128 experts top-8 of width 1536, vocabulary 151936,
# qk-norm, rope theta 1e6, softmax routing
QWEN3_235B_A22B = dict(n_layers=94, d_model=4096, n_heads=64, n_kv_heads=4, head_dim=128, vocab=151936,
                       n_experts=128, top_k=8, d_expert=1536, n_shared=0, d_shared=0, max_ctx=40960, router=0,
                       rope_theta=1e6, norm_eps=1e-6, routed_scale=1.0)


class Model:
    def __init__(self, manifest_path, max_ctx=0, eager=False, attn_slices=0, split=False, **cache):
        """cache: expert_cache, pin_frac, prefetch, lookahead_k, interest, prefill_chunk, stats,
        host_routes (model_opts)"""
        self.opts = model_opts(max_ctx, eager, attn_slices, split, **cache)
        h = C.c_void_p()
        check(lib.tlm_hip_model_open(str(manifest_path).encode(), C.byref(self.opts), C.byref(h)))
        self._bind(h)

    @classmethod
    def synth(cls, geom, expert_dt=14, dense_dt=8, qk_norm=True, seed=1, max_ctx=0, eager=False, attn_slices=0,
              split=False, expert_pool=0, heat_gamma=0.0, **cache):
        """tlm_hip_model_synth: a random-init model of geometry geom (a dict of
        tlm_hip_model_geom fields) built in HBM; with cache (model_opts'
        expert_cache ...) its experts stay in page-locked host memory (a pool
        of expert_pool distinct payloads, 0 = one each) behind the slot cache;
        heat_gamma > 0 with sigmoid routing biases selection towards a
        per-layer order of the experts (-heat_gamma ln(rank + 1))."""
        from ._lib import ModelGeom, ModelSynthOpts
        g = ModelGeom()
        g.arch = b"synthetic"
        for k, v in geom.items():
            setattr(g, k, v)
        so = ModelSynthOpts(expert_dt, dense_dt, int(qk_norm), int(expert_pool), seed, float(heat_gamma))
        self = cls.__new__(cls)
        self.opts = model_opts(max_ctx, eager, attn_slices, split, **cache)
        h = C.c_void_p()
        check(lib.tlm_hip_model_synth(C.byref(g), C.byref(so), C.byref(self.opts), C.byref(h)))
        self._bind(h)
        return self

    def _bind(self, h):
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

    def kv_capacity(self):
        """The context capacity in effect: the request, capped at the store's
        max_position_embeddings as tlm_kv_new caps it (src/lib/tlm_model.c:646-650)."""
        return lib.tlm_hip_model_kv_capacity(self.h)

    def rewind(self, n):
        """Keep the first n positions of the context (enqueued)."""
        check(lib.tlm_hip_model_rewind(self.h, int(n)))

    def decode(self, n):
        """n greedy steps from the current position, enqueued (sync() waits)."""
        check(lib.tlm_hip_model_decode(self.h, int(n)))

    def sync(self):
        check(lib.tlm_hip_model_sync(self.h))

    def stream(self):
        """the model's HIP stream handle (an int)"""
        return lib.tlm_hip_model_stream(self.h)

    def store_stats(self):
        """The expert slot cache's counters (tlm_hip_store_get_stats), or None
        when every expert is resident."""
        from ._lib import StoreStats
        st = lib.tlm_hip_model_expert_store(self.h)
        if not st:
            return None
        out = StoreStats()
        lib.tlm_hip_store_get_stats(st, C.byref(out))
        return {f: int(getattr(out, f)) for f, _ in StoreStats._fields_}

    def stats(self):
        """tlm_model_stats of the device steps (tlm_hip_model_get_stats)."""
        out = ModelStats()
        check(lib.tlm_hip_model_get_stats(self.h, C.byref(out)))
        return {f: int(getattr(out, f)) for f, _ in ModelStats._fields_}

    def reset_stats(self):
        lib.tlm_hip_model_reset_stats(self.h)

    def routes(self):
        """The last step's routing: (ids, weights), each [n_layers, top_k] in
        rank order (what the reference's routing hook receives)."""
        L, k = self.geom.n_layers, self.geom.top_k
        ids = np.empty((L, k), np.int32)
        w = np.empty((L, k), np.float32)
        check(lib.tlm_hip_model_routes(self.h, ids.ctypes.data, w.ctypes.data))
        return ids, w

    def step(self, token, logits=True):
        """One token; returns (logits as float32 [vocab] or None, greedy next token)."""
        lg = np.empty(self.geom.vocab, np.float32) if logits else None
        nxt = C.c_int32()
        check(lib.tlm_hip_model_step(self.h, int(token), lg.ctypes.data if logits else None, C.byref(nxt)))
        return lg, nxt.value

    def prefill(self, tokens, logits=True):
        """tlm_model_prefill: the tokens from the current position; the last
        one's logits (float32 [vocab]) or None."""
        p = (C.c_int32 * len(tokens))(*tokens)
        lg = np.empty(self.geom.vocab, np.float32) if logits else None
        check(lib.tlm_hip_model_prefill(self.h, p, len(tokens), lg.ctypes.data if logits else None))
        return lg

    def prefill_batched(self):
        """Whether prompts run batched on this model."""
        return bool(lib.tlm_hip_model_prefill_batched(self.h))

    def generate(self, prompt, n):
        p = (C.c_int32 * len(prompt))(*prompt)
        out = (C.c_int32 * max(n, 1))()
        check(lib.tlm_hip_model_generate(self.h, p, len(prompt), n, out))
        return list(out[:n])


def bench_prompt(n, vocab, seed=42):
    """tierlm bench's prompt: xorshift64 from the seed, each token mod vocab
    (src/bin/tierlm.c:711-715)."""
    x, out, m = seed, [], (1 << 64) - 1
    for _ in range(n):
        x ^= (x << 13) & m
        x ^= x >> 7
        x ^= (x << 17) & m
        out.append(x % vocab)
    return out


def time_model(m, prompt_len=64, n=64, reps=3, warm_n=None):
    """Best of reps: prefill time (generate(prompt, 1)) and decode time (the
    n - 1 further steps of generate(prompt, n)), host wall clock around the
    calls; tokens stay on the device between steps."""
    prompt = bench_prompt(prompt_len, m.geom.vocab)
    m.reset()
    toks = m.generate(prompt, n if warm_n is None else warm_n)   # warm (and graph capture)
    pre = dec = None
    for _ in range(reps):
        m.reset()
        t0 = time.perf_counter()
        m.generate(prompt, 1)
        t1 = time.perf_counter()
        m.reset()
        t2 = time.perf_counter()
        toks = m.generate(prompt, n)
        t3 = time.perf_counter()
        p, d = t1 - t0, (t3 - t2) - (t1 - t0)
        pre = p if pre is None else min(pre, p)
        dec = d if dec is None else min(dec, d)
    return {"prefill_tok_s": round(prompt_len / pre, 1), "decode_tok_s": round((n - 1) / dec, 1),
            "decode_us_per_token": round(dec / (n - 1) * 1e6, 1), "tokens": toks}


def _roctx():
    """roctxProfilerPause / Resume (rocprofv3 --selected-regions traces only
    what runs between a resume and the next pause), or None without the
    library."""
    try:
        lib_ = C.CDLL("librocprofiler-sdk-roctx.so.1")
    except OSError:
        return None
    lib_.roctxProfilerPause.argtypes = lib_.roctxProfilerResume.argtypes = [C.c_uint64]
    return lib_


def time_at_context(m, context, n, rx=None):
    """n decode steps ending at position context - 1: the context is filled to
    context - n positions first (a pseudo-random prompt, greedy from there),
    then the n steps are timed (host clock around the enqueued steps and a
    sync).  With rx (_roctx()), only the timed steps run between
    roctxProfilerResume and roctxProfilerPause."""
    if not 1 <= n < context <= m.kv_capacity():
        raise ValueError(f"context {context}, {n} steps, capacity {m.kv_capacity()}")
    if rx:
        rx.roctxProfilerPause(0)
    m.reset()
    m.generate(bench_prompt(context - n, m.geom.vocab), 1)   # positions 0 .. context - n - 1
    m.sync()
    if rx:
        rx.roctxProfilerResume(0)
    t0 = time.perf_counter()
    m.decode(n)
    m.sync()
    dt = time.perf_counter() - t0
    if rx:
        rx.roctxProfilerPause(0)
    return {"positions": [context - n, context - 1], "decode_tok_s": round(n / dt, 1),
            "decode_us_per_token": round(dt / n * 1e6, 1)}


def bench(path, prompt_len=64, n=64, reps=3, eager=False, max_ctx=0):
    """time_model on a compiled store."""
    m = Model(path, max_ctx=max_ctx or prompt_len + n + 1, eager=eager)
    try:
        return time_model(m, prompt_len, n, reps)
    finally:
        m.close()


if __name__ == "__main__":
    import argparse

    from .quant import init
    ap = argparse.ArgumentParser(prog="python -m tierlm_amd.model")
    ap.add_argument("store", nargs="?")
    ap.add_argument("--synth", choices=["qwen3-30b-a3b"], help="a random-init model of this shape instead of a store")
    ap.add_argument("--layers", type=int, default=0, help="with --synth: layers (default: the model's)")
    ap.add_argument("--prompt-len", type=int, default=64)
    ap.add_argument("-n", type=int, default=64)
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--eager", action="store_true", help="launch kernels directly instead of replaying a graph")
    ap.add_argument("--split", action="store_true", help="split attention (attn_split) instead of the reference's order")
    ap.add_argument("--context", type=int, default=0,
                    help="time only the n decode steps ending at position CONTEXT - 1 (the context filled first)")
    ap.add_argument("--roctx", action="store_true",
                    help="with --context: pause the profiler outside the timed steps (rocprofv3 --selected-regions)")
    a = ap.parse_args()
    if (a.store is None) == (a.synth is None):
        ap.error("give a store or --synth")
    if a.roctx and not a.context:
        ap.error("--roctx needs --context")
    rx = None
    if a.roctx:   # loaded before the runtime starts, so the profiler sees its calls
        rx = _roctx()
        if rx is None:
            raise SystemExit("librocprofiler-sdk-roctx.so.1 not found")
        rx.roctxProfilerPause(0)
    init(0)
    ctx = a.context or a.prompt_len + a.n + 1
    if a.synth:
        geom = dict(QWEN3_30B_A3B, **({"n_layers": a.layers} if a.layers else {}))
        m = Model.synth(geom, seed=1, max_ctx=ctx, eager=a.eager, split=a.split)
        name = f"{a.synth} ({geom['n_layers']} layers, random init)"
    else:
        m = Model(a.store, max_ctx=ctx, eager=a.eager, split=a.split)
        name = a.store
    try:
        if a.context:
            r = time_at_context(m, a.context, a.n, rx)
        else:
            r = time_model(m, a.prompt_len, a.n, a.reps)
    finally:
        m.close()
    if a.context:
        print(f"bench {name}: decode {a.n} tokens at positions {r['positions'][0]}..{r['positions'][1]} "
              f"({r['decode_tok_s']:.1f} tok/s, {r['decode_us_per_token']:.1f} us/token)"
              f"{' eager' if a.eager else ''}", flush=True)
        raise SystemExit(0)
    print(f"bench {name}: prompt {a.prompt_len} tokens ({r['prefill_tok_s']:.1f} tok/s), decode {a.n} tokens "
          f"({r['decode_tok_s']:.1f} tok/s, {r['decode_us_per_token']:.1f} us/token){' eager' if a.eager else ''}",
          flush=True)
