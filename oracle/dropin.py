"""dropin.py - TEST INFRASTRUCTURE ONLY: the reference's own `tierlm` with
libtlm_hip.so dropped in, built from a build-directory copy of the
reference's sources under oracle/_ref/dropin (nothing is written under the
reference, nothing from it is committed here).

    python3 oracle/dropin.py          # -> oracle/_ref/dropin/bin/tierlm

The copy gets the few additions a maintainer would make to take the HIP
library (each one anchored on a line of the reference and asserted to apply):

* src/lib/tlm_platform.c, tlm_cpu_force (:352-358): a request for the tier
  "hip" (--kernel hip, or TIERLM_KERNEL=hip through tlm_cpu) is remembered;
* src/lib/tlm_quant.c, tlm_quant_init (:1069-1088): when it is, a fourth
  tier is built from the best CPU tier, tlm_kern_hip_fill overwrites its
  entries and the reference's own bit-exact self-test (selftest_tier,
  :1015-1056) runs over them against the scalar kernels before the table is
  published - tlm_quant_tier() then reports "hip";
* src/lib/tlm_model.c: a KV cache opened while a device manifest is set
  (tlm_kv_new, :646-664) also opens the store on the device
  (tlm_hip_model_open, with the same capacity); tlm_model_step (:1058-1103)
  then runs the whole step there (tlm_hip_model_step: logits back to the
  host only when asked for), tlm_model_prefill (:1105-1113) hands the whole
  prompt over (tlm_hip_model_prefill: batched where the model allows it, the
  same bits), tlm_kv_reset / tlm_kv_free reset and close it;
* src/bin/tierlm.c, rt_open (:196-202): --kernel hip sets the device manifest
  to the store being opened (TIERLM_HIP_TIER_ONLY=1 keeps the reference's CPU
  step with only the kernel table on the device), and the stats line names
  the self-test failures beside the tier;
* rt_open (:273-310): the expert budget the runtime settles on (--cache /
  memory.expert_cache, raised to top_k slots), its capped pin share, its
  router lookahead, io.lookahead_k and nav.interest_aggressiveness go to the
  device model: when the budget cannot hold every expert, the experts stay
  in page-locked host memory behind an HBM slot cache of that budget
  (tlm_hip_model_opts.expert_cache_bytes), else they are all resident;
* print_stats / print_stats_json (:419-470, :473-480): the store counters
  are the device cache's when the step runs there (the reference's RAM store
  then serves no expert);
* tlm_model_get_stats / tlm_model_reset_stats (tlm_model.c:642-643): with
  --stats / --stats-json the device step's attention / MoE split is timed
  on the device (tlm_hip_model_opts.stats; tlm_hip_model_get_stats), the
  expert wait is its slot cache's, and other is the rest of the host's step
  time.

Every library file is then compiled as oracle/Makefile compiles the reference
(same flags), against include/tlm_hip.h, and linked with
tierlm_amd/libtlm_hip.so (rpath to it).
"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
REF = os.environ.get("REF", "/root/reference")
OUT = os.path.join(HERE, "_ref", "dropin")
CFLAGS = ["-std=c11", "-O2", "-g", "-fPIC", "-pthread", "-fno-math-errno", "-ffp-contract=off", "-D_GNU_SOURCE",
          "-w"]
AVX2 = ["-mavx2", "-mfma", "-mf16c"]
AVX512 = ["-mavx512f", "-mavx512bw", "-mavx512vl", "-mavx512vnni", "-mavx512dq", "-mfma", "-mf16c"]

DROPIN_CACHE = """static uint64_t g_dropin_cache;       /* the device slot budget; 0 = every expert resident */
static double g_dropin_pin, g_dropin_interest;
static int g_dropin_prefetch_off, g_dropin_lookahead_k, g_dropin_stats;
static tlm_hip_model *g_dropin_model;    /* the device model of the open KV cache */
void tlm_model_dropin_cache(uint64_t budget, uint64_t expert_total, double pin_frac, int prefetch,
                            int lookahead_k, double interest, int stats) {
    g_dropin_cache = budget < expert_total ? budget : 0;
    g_dropin_pin = pin_frac > 0 ? pin_frac : -1.0;
    g_dropin_prefetch_off = !prefetch;
    g_dropin_lookahead_k = lookahead_k;
    g_dropin_interest = interest;
    g_dropin_stats = stats;
}
void tlm_model_dropin_store_stats(tlm_store_stats *ss) {
    tlm_hip_store *st = g_dropin_model ? tlm_hip_model_expert_store(g_dropin_model) : NULL;
    if (st) tlm_hip_store_get_stats(st, (tlm_hip_store_stats *)ss);
}
/* the device step's split: attention and MoE timed on the device, the
 * expert wait of its slot cache, the rest of the host's step time as other */
static void dropin_split(tlm_model_stats *out) {
    tlm_hip_model_stats d;
    if (!g_dropin_model || tlm_hip_model_get_stats(g_dropin_model, &d)) return;
    out->attn_ns = d.attn_ns;
    out->moe_ns = d.moe_ns;
    out->expert_wait_ns = d.expert_wait_ns;
    const uint64_t dev = d.attn_ns + d.moe_ns;
    out->other_ns = out->other_ns > dev ? out->other_ns - dev : 0;
}
"""

# (file, anchor, text inserted after the anchor) - or ("replace", old, new)
PATCHES = [
    ("lib/tlm_platform.c", "void tlm_cpu_force(const char *tier) {\n",
     "    tlm_dropin_hip = tier && strcmp(tier, \"hip\") == 0;\n"),
    ("lib/tlm_platform.c", "#include \"tlm_platform.h\"\n",
     "int tlm_dropin_hip;   /* the HIP tier was asked for */\n"),
    ("lib/tlm_quant.c", "#include \"tlm_platform.h\"\n",
     "#include \"tlm_hip.h\"\n"),
    ("lib/tlm_quant.c", "static pthread_mutex_t g_init_mu = PTHREAD_MUTEX_INITIALIZER;\n",
     "extern int tlm_dropin_hip;\n"
     "static tlm_quant_kernels g_tab_hip;\n"
     "static int g_hip_state;   /* 0 not built, 1 ok, -1 unavailable */\n"),
    ("lib/tlm_quant.c", "void tlm_quant_init(void) {\n",
     None),   # the HIP tier builder goes before tlm_quant_init (below)
    ("lib/tlm_quant.c", "    atomic_store_explicit(&g_kern, &g_tab[sel], memory_order_release);\n",
     None),
    ("lib/tlm_model.c", "    int    max_ctx, len;\n",
     "    void  *hip;                  /* the device model when the step runs there */\n"),
    ("lib/tlm_model.c", "#include \"tlm_quant.h\"\n",
     "#include \"tlm_hip.h\"\n"
     "static const char *g_dropin_manifest;   /* the store to open on the device, or NULL */\n"
     "void tlm_model_dropin_manifest(const char *path) { g_dropin_manifest = path; }\n" + DROPIN_CACHE),
    ("lib/tlm_model.c", "void tlm_kv_free(tlm_kv *kv) {\n    if (!kv) return;\n",
     "    if (kv->hip && g_dropin_model == (tlm_hip_model *)kv->hip) g_dropin_model = NULL;\n"
     "    if (kv->hip) tlm_hip_model_close((tlm_hip_model *)kv->hip);\n"),
    ("lib/tlm_model.c", "int tlm_model_step(tlm_model *M, tlm_kv *kv, int token, float *logits) {\n",
     None),
    ("lib/tlm_model.c", "    if (n <= 0) return tlm_seterr(TLM_EINVAL, \"prefill: no tokens\");\n",
     "    if (kv->hip) return dropin_prefill(M, kv, tokens, n, logits);\n"),
    ("lib/tlm_model.c",
     "    if (kv->len >= kv->max_ctx) return tlm_seterr(TLM_ERANGE, \"context full (%d tokens)\", kv->max_ctx);\n",
     "    if (kv->hip) return dropin_step(M, kv, token, logits);\n"),
    ("bin/tierlm.c", "#include \"tlm_store.h\"\n",
     "void tlm_model_dropin_manifest(const char *path);\n"
     "void tlm_model_dropin_cache(uint64_t budget, uint64_t expert_total, double pin_frac, int prefetch,\n"
     "                            int lookahead_k, double interest, int stats);\n"
     "void tlm_model_dropin_store_stats(tlm_store_stats *ss);\n"),
    ("bin/tierlm.c", "    r->mdl = tlm_model_open(&r->m, r->io, r->st, r->pool, &mo);\n",
     "    tlm_model_dropin_cache(r->budget, r->expert_total, r->pin_frac, r->lookahead, r->lookahead_k, mo.interest,\n"
     "                           o->stats || o->stats_json);\n"),
    ("bin/tierlm.c", "        tlm_cpu_force(o->kernel);\n        tlm_quant_init();\n",
     "        if (!strcmp(o->kernel, \"hip\") && !getenv(\"TIERLM_HIP_TIER_ONLY\"))\n"
     "            tlm_model_dropin_manifest(o->manifest);\n"),
]


HIP_TIER = """static void build_hip_tier(int base) {
    if (g_hip_state) return;
    g_hip_state = -1;
    g_tab_hip = g_tab[base];
    if (tlm_hip_init(0) != 0) {
        tlm_log(TLM_LOG_WARN, "tlm_quant: hip tier unavailable: %s", tlm_hip_errmsg());
        return;
    }
    if (tlm_kern_hip_fill((tlm_hip_quant_kernels *)&g_tab_hip) <= 0) return;
    g_tab_hip.name = "hip";
    selftest_tier(&g_tab_hip, &g_tab[base]);
    g_hip_state = 1;
}

"""

HIP_SELECT = """    if (tlm_dropin_hip) {
        build_hip_tier(sel);
        if (g_hip_state > 0) {
            atomic_store_explicit(&g_kern, &g_tab_hip, memory_order_release);
            pthread_mutex_unlock(&g_init_mu);
            return;
        }
    }
"""

DROPIN_STEP = """static int dropin_step(tlm_model *M, tlm_kv *kv, int token, float *logits) {
    uint64_t t0 = tlm_now_ns();
    int rc = tlm_hip_model_step((tlm_hip_model *)kv->hip, token, logits, NULL);
    if (rc) return tlm_seterr(rc, "hip step: %s", tlm_hip_errmsg());
    kv->len++;
    M->st.tokens++;
    M->st.other_ns += tlm_now_ns() - t0;
    return TLM_OK;
}

static int dropin_prefill(tlm_model *M, tlm_kv *kv, const int *tokens, int n, float *logits) {
    uint64_t t0 = tlm_now_ns();
    int rc = tlm_hip_model_prefill((tlm_hip_model *)kv->hip, (const int32_t *)tokens, n, logits);
    if (rc) return tlm_seterr(rc, "hip prefill: %s", tlm_hip_errmsg());
    kv->len += n;
    M->st.tokens += n;
    M->st.other_ns += tlm_now_ns() - t0;
    return TLM_OK;
}

"""

KV_OPEN = """    if (g_dropin_manifest) {
        tlm_hip_model_opts ho;
        memset(&ho, 0, sizeof ho);
        ho.max_ctx = max_ctx;
        ho.expert_cache_bytes = g_dropin_cache;
        ho.pin_frac = g_dropin_pin;
        ho.prefetch_off = g_dropin_prefetch_off;
        ho.lookahead_k = g_dropin_lookahead_k;
        ho.interest = g_dropin_interest;
        ho.stats = g_dropin_stats;
        tlm_hip_model *hm = NULL;
        if (tlm_hip_model_open(g_dropin_manifest, &ho, &hm) != 0) {
            tlm_seterr(TLM_EUNSUP, "hip model: %s", tlm_hip_errmsg());
            tlm_kv_free(kv);
            return NULL;
        }
        kv->hip = hm;
        g_dropin_model = hm;
    }
"""

REPLACES = [
    ("lib/tlm_model.c", "void tlm_model_get_stats(const tlm_model *M, tlm_model_stats *out) { *out = M->st; }\n",
     "void tlm_model_get_stats(const tlm_model *M, tlm_model_stats *out) {\n    *out = M->st;\n"
     "    dropin_split(out);\n}\n"),
    ("lib/tlm_model.c", "void tlm_model_reset_stats(tlm_model *M) { memset(&M->st, 0, sizeof M->st); }\n",
     "void tlm_model_reset_stats(tlm_model *M) {\n    memset(&M->st, 0, sizeof M->st);\n"
     "    if (g_dropin_model) tlm_hip_model_reset_stats(g_dropin_model);\n}\n"),
    ("bin/tierlm.c", "    tlm_store_stats ss;\n    tlm_store_get_stats(r->st, &ss);\n    char b1[32], b2[32], b3[32];\n",
     "    tlm_store_stats ss;\n    tlm_store_get_stats(r->st, &ss);\n    tlm_model_dropin_store_stats(&ss);\n"
     "    char b1[32], b2[32], b3[32];\n"),
    ("bin/tierlm.c", "    tlm_store_stats ss;\n    tlm_store_get_stats(r->st, &ss);\n    uint64_t acc = ss.hits + ss.misses;\n",
     "    tlm_store_stats ss;\n    tlm_store_get_stats(r->st, &ss);\n    tlm_model_dropin_store_stats(&ss);\n"
     "    uint64_t acc = ss.hits + ss.misses;\n"),
    ("lib/tlm_model.c", "void tlm_kv_reset(tlm_kv *kv) { kv->len = 0; }\n",
     "void tlm_kv_reset(tlm_kv *kv) {\n    kv->len = 0;\n"
     "    if (kv->hip) tlm_hip_model_reset((tlm_hip_model *)kv->hip);\n}\n"),
    ("lib/tlm_model.c", "    return kv;\n}\nvoid tlm_kv_free(tlm_kv *kv) {\n",
     KV_OPEN + "    return kv;\n}\nvoid tlm_kv_free(tlm_kv *kv) {\n"),
    ("bin/tierlm.c", "    fprintf(f, \"load        %.3f s (manifest, resident packets, pins); kernel %s, %d thread%s\\n\", r->load_s,\n"
                     "            tlm_quant_tier(), r->threads, r->threads == 1 ? \"\" : \"s\");\n",
     "    fprintf(f, \"load        %.3f s (manifest, resident packets, pins); kernel %s (self-test failures %d), \"\n"
     "               \"%d thread%s\\n\", r->load_s, tlm_quant_tier(), tlm_quant_selftest_failures(), r->threads,\n"
     "            r->threads == 1 ? \"\" : \"s\");\n"),
]


def patch(src):
    def edit(rel, fn):
        p = os.path.join(src, rel)
        s = open(p).read()
        s2 = fn(s)
        open(p, "w").write(s2)

    for rel, anchor, text in PATCHES:
        def ins(s, anchor=anchor, text=text, rel=rel):
            if s.count(anchor) != 1:
                raise SystemExit(f"dropin: anchor not found once in {rel}: {anchor!r}")
            if text is None:
                if anchor.startswith("void tlm_quant_init"):
                    return s.replace(anchor, HIP_TIER + anchor)
                if anchor.startswith("    atomic_store_explicit"):
                    return s.replace(anchor, HIP_SELECT + anchor)
                if anchor.startswith("int tlm_model_step"):
                    return s.replace(anchor, DROPIN_STEP + anchor)
                raise SystemExit(f"dropin: no text for {anchor!r}")
            return s.replace(anchor, anchor + text)
        edit(rel, ins)
    for rel, old, new in REPLACES:
        def rep(s, old=old, new=new, rel=rel):
            if s.count(old) != 1:
                raise SystemExit(f"dropin: text not found once in {rel}: {old[:60]!r}")
            return s.replace(old, new)
        edit(rel, rep)


def build(src):
    obj = os.path.join(OUT, "obj")
    bind = os.path.join(OUT, "bin")
    os.makedirs(obj, exist_ok=True)
    os.makedirs(bind, exist_ok=True)
    inc = ["-I" + os.path.join(src, "lib"), "-I" + os.path.join(ROOT, "include")]
    objs = []
    for f in sorted(os.listdir(os.path.join(src, "lib"))):
        if not f.endswith(".c"):
            continue
        extra = AVX2 if f == "tlm_kern_avx2.c" else AVX512 if f == "tlm_kern_avx512.c" else []
        o = os.path.join(obj, f[:-2] + ".o")
        subprocess.run(["gcc"] + CFLAGS + extra + inc + ["-c", os.path.join(src, "lib", f), "-o", o], check=True)
        objs.append(o)
    libdir = os.path.join(ROOT, "tierlm_amd")
    rpath = "$ORIGIN/" + os.path.relpath(libdir, bind)
    subprocess.run(["gcc"] + CFLAGS + inc + [os.path.join(src, "bin", "tierlm.c"), "-o", os.path.join(bind, "tierlm")]
                   + objs + ["-L" + libdir, "-ltlm_hip", "-Wl,-rpath," + rpath, "-lm", "-pthread"], check=True)


def main():
    if not os.path.isdir(os.path.join(REF, "src", "lib")):
        print(f"dropin: reference sources not found at {REF}; not built")
        return 0
    if not os.path.exists(os.path.join(ROOT, "tierlm_amd", "libtlm_hip.so")):
        raise SystemExit("dropin: build tierlm_amd/libtlm_hip.so first")
    src = os.path.join(OUT, "src")
    shutil.rmtree(OUT, ignore_errors=True)
    os.makedirs(os.path.join(src, "bin"))
    shutil.copytree(os.path.join(REF, "src", "lib"), os.path.join(src, "lib"))
    shutil.copy(os.path.join(REF, "src", "bin", "tierlm.c"), os.path.join(src, "bin", "tierlm.c"))
    patch(src)
    build(src)
    shutil.rmtree(src)   # only the built tool stays; the copied sources do not travel
    shutil.rmtree(os.path.join(OUT, "obj"))
    print("dropin: built", os.path.join(OUT, "bin", "tierlm"))
    return 0


if __name__ == "__main__":
    sys.exit(main())
