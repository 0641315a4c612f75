/* ref_moe.c - CPU-baseline driver over the reference's own kernels.
 *
 * TEST INFRASTRUCTURE ONLY (linked into oracle/_ref/libtlmref.so together with
 * the reference's tlm_quant.c, tlm_pool.c and kernel tiers).
 *
 * Runs one routed MoE block the way src/lib/tlm_model.c:940-1055 does: the
 * reference's tlm_quantize_act for every activation, the reference's
 * tlm_matvec_rows for every matrix (whichever tier tlm_quant_init picked),
 * and the reference's tlm_pool_for to split rows across threads with the same
 * grain and serial cut-off as its mv_exec (src/lib/tlm_model.c:42-44, 205-222).
 * The small glue (rmsnorm, routing, silu, combine) comes from the oracle.
 */
#include "tlm_oracle.h"
#include "tlm_pool.h"
#include "tlm_quant.h"
#include "tlm_platform.h"

#include <stdlib.h>
#include <string.h>

#define SEG_MAX 160
#define GRAIN 16
#define SERIAL_MACS 32768

typedef struct {
    tlm_dtype   dt;
    const void *W;
    size_t      row_bytes;
    const void *act;
    float      *y;
    int64_t     n;
} seg;

typedef struct {
    seg     s[SEG_MAX];
    int64_t first[SEG_MAX + 1];
    int     count;
    int64_t macs;
} job;

typedef struct refmoe {
    tlm_pool *pool;
} refmoe;

static void job_push(job *j, tlm_dtype dt, const void *W, int64_t rows, int64_t n, const void *act, float *y) {
    if (j->count == 0) j->first[0] = 0;
    seg *g = &j->s[j->count];
    g->dt = dt;
    g->W = W;
    g->row_bytes = tlm_row_bytes(dt, n);
    g->act = act;
    g->y = y;
    g->n = n;
    j->first[j->count + 1] = j->first[j->count] + rows;
    j->macs += rows * n;
    j->count++;
}

static void job_rows(void *ctx, int64_t b, int64_t e, int worker) {
    (void)worker;
    const job *j = (const job *)ctx;
    for (int i = 0; i < j->count; i++) {
        int64_t s0 = j->first[i], s1 = j->first[i + 1];
        if (e <= s0) break;
        if (b >= s1) continue;
        int64_t lo = (b > s0 ? b : s0) - s0, hi = (e < s1 ? e : s1) - s0;
        const seg *g = &j->s[i];
        tlm_matvec_rows(g->dt, g->W, g->row_bytes, g->act, g->y, g->n, lo, hi, NULL);
    }
}

static void job_run(refmoe *m, job *j) {
    if (j->count == 0) return;
    tlm_pool_for(j->macs < SERIAL_MACS ? NULL : m->pool, j->first[j->count], GRAIN, job_rows, j);
    j->count = 0;
    j->macs = 0;
}

refmoe *refmoe_new(int nthreads) {
    refmoe *m = (refmoe *)calloc(1, sizeof *m);
    if (!m) return NULL;
    tlm_quant_init();
    if (nthreads > 1) m->pool = tlm_pool_new(nthreads, 0);
    return m;
}

void refmoe_free(refmoe *m) {
    if (!m) return;
    if (m->pool) tlm_pool_free(m->pool);
    free(m);
}

const char *refmoe_tier(void) { return tlm_quant_tier(); }

/* Force a CPU tier ("scalar", "avx2", "avx512", "auto") and re-dispatch. */
void refmoe_force_tier(const char *tier) {
    tlm_cpu_force(tier);
    tlm_quant_init();
}

/* nseg matvecs of one dtype and width n on one activation (quantised here
 * with the reference's quantiser) through the pool as one job, the way mv_exec
 * runs the dense projections of attention() and the lm_head
 * (src/lib/tlm_model.c:175-222, 734-739, 1087-1095). */
void refmoe_matvecs(refmoe *m, int dt, const void *const *W, const int64_t *rows, int64_t n, const float *x,
                    float *const *y, int nseg) {
    tlm_dtype t = (tlm_dtype)dt, ak = tlm_act_kind_for(t);
    uint8_t *act = malloc(tlm_qact_bytes(ak, n) + 64);
    const void *a = x;
    if (ak != TLM_DT_F32) { tlm_quantize_act(ak, x, n, act); a = act; }
    job *j = calloc(1, sizeof *j);
    for (int i = 0; i < nseg && i < SEG_MAX; i++) job_push(j, t, W[i], rows[i], n, a, y[i]);
    job_run(m, j);
    free(j);
    free(act);
}

int refmoe_layer(refmoe *m, const orc_moe_desc *d, float *h, int *ids, float *w) {
    int64_t D = d->D, de = d->de, ds = d->ds;
    int k = d->k;
    if (k > 64 || D <= 0) return -1;
    size_t fsz = sizeof(float);
    float *xb = malloc(fsz * (size_t)D), *logits = malloc(fsz * (size_t)d->E);
    float *eg = malloc(fsz * (size_t)(2 * de * k)), *eh = malloc(fsz * (size_t)(de * k));
    float *eo = malloc(fsz * (size_t)(D * k)), *ffn = malloc(fsz * (size_t)D);
    float *sg = malloc(fsz * (size_t)(2 * (ds > 0 ? ds : 1))), *sh = malloc(fsz * (size_t)(ds > 0 ? ds : 1));
    float *so = malloc(fsz * (size_t)D);
    tlm_dtype et = (tlm_dtype)d->expert_dt, st = (tlm_dtype)d->shared_dt;
    tlm_dtype ek = tlm_act_kind_for(et), sk = tlm_act_kind_for(st);
    size_t hb = tlm_qact_bytes(ek, de);
    uint8_t *xe = malloc(tlm_qact_bytes(TLM_DT_Q8_K, D) + tlm_qact_bytes(TLM_DT_Q8_0, D) + 64);
    uint8_t *xs = malloc(tlm_qact_bytes(TLM_DT_Q8_K, D) + tlm_qact_bytes(TLM_DT_Q8_0, D) + 64);
    uint8_t *he = malloc(hb * (size_t)k + 64);
    uint8_t *hs = malloc(tlm_qact_bytes(TLM_DT_Q8_K, ds) + tlm_qact_bytes(TLM_DT_Q8_0, ds) + 64);
    job *j = calloc(1, sizeof *j);

    orc_rmsnorm(xb, h, d->ffn_norm, D, d->eps);
    tlm_dtype rk = tlm_act_kind_for((tlm_dtype)d->router_dt);
    const void *ract = xb;
    if (rk != TLM_DT_F32) { tlm_quantize_act(rk, xb, D, xs); ract = xs; }
    tlm_matvec_rows((tlm_dtype)d->router_dt, d->router_w, tlm_row_bytes((tlm_dtype)d->router_dt, D), ract,
                    logits, D, 0, d->E, NULL);
    orc_route(d->router, logits, d->mask, d->router_bias, d->E, k, d->routed_scale, ids, w);

    const void *xa = xb;
    if (ek != TLM_DT_F32) { tlm_quantize_act(ek, xb, D, xe); xa = xe; }
    const void *sa = xb;
    if (ds > 0 && sk != TLM_DT_F32) { tlm_quantize_act(sk, xb, D, xs); sa = xs; }
    for (int r = 0; r < k; r++) {
        job_push(j, et, d->gate[ids[r]], de, D, xa, eg + 2 * de * r);
        job_push(j, et, d->up[ids[r]], de, D, xa, eg + 2 * de * r + de);
    }
    if (ds > 0) {
        job_push(j, st, d->sg, ds, D, sa, sg);
        job_push(j, st, d->su, ds, D, sa, sg + ds);
    }
    job_run(m, j);
    for (int r = 0; r < k; r++) {
        const float *g = eg + 2 * de * r, *u = g + de;
        float *hh = eh + de * r;
        for (int64_t i = 0; i < de; i++) hh[i] = orc_silu(g[i]) * u[i];
        const void *ha = hh;
        if (ek != TLM_DT_F32) { tlm_quantize_act(ek, hh, de, he + hb * r); ha = he + hb * r; }
        job_push(j, et, d->down[ids[r]], D, de, ha, eo + D * r);
    }
    if (ds > 0) {
        for (int64_t i = 0; i < ds; i++) sh[i] = orc_silu(sg[i]) * sg[ds + i];
        const void *ha = sh;
        if (sk != TLM_DT_F32) { tlm_quantize_act(sk, sh, ds, hs); ha = hs; }
        job_push(j, st, d->sd, D, ds, ha, so);
    }
    job_run(m, j);

    for (int64_t i = 0; i < D; i++) ffn[i] = 0.0f;
    for (int r = 0; r < k; r++)
        for (int64_t i = 0; i < D; i++) {
            float c = w[r] * eo[D * r + i];
            ffn[i] += c;
        }
    if (ds > 0) {
        float gate = 1.0f;
        if (d->shared_gate_inp) {
            float s = 0.0f;
            for (int64_t i = 0; i < D; i++) s += d->shared_gate_inp[i] * xb[i];
            gate = orc_sigmoid(s);
        }
        for (int64_t i = 0; i < D; i++) ffn[i] += gate * so[i];
    }
    for (int64_t i = 0; i < D; i++) h[i] += ffn[i];

    free(xb); free(logits); free(eg); free(eh); free(eo); free(ffn); free(sg); free(sh); free(so);
    free(xe); free(xs); free(he); free(hs); free(j);
    return 0;
}
