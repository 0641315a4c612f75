/* ref_routes.c - TEST INFRASTRUCTURE ONLY: the reference runtime's routing
 * decisions, position by position, for a fixed token sequence.
 *
 *   ref_routes STORE.tlmm id,id,... > routes.txt
 *
 * Opens a compiled store with the reference's own library (built from its
 * sources by `make -C oracle tools`): tlm_manifest_load, tlm_io_open,
 * tlm_store_open with every expert's slot, tlm_model_open without lookahead,
 * and registers the routing hook the reference calls once per MoE layer per
 * token (tlm_model_set_route_hook, src/lib/tlm_model.h:63-70,
 * src/lib/tlm_model.c:1053).  Then it steps through the tokens
 * (tlm_model_step, teacher-forced) and prints one line per (position, layer):
 *
 *   pos layer id:weight id:weight ...     (rank order, weights as %a)
 *
 * Nothing here is copied from the reference; it sequences its public calls. */
#include "tlm_io.h"
#include "tlm_model.h"
#include "tlm_packet.h"
#include "tlm_platform.h"
#include "tlm_pool.h"
#include "tlm_store.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static void on_route(void *ctx, int layer, int pos, int token, const int *ids, const float *w,
                     const float *out_norm, int k) {
    (void)ctx;
    (void)token;
    (void)out_norm;
    printf("%d %d", pos, layer);
    for (int r = 0; r < k; r++) printf(" %d:%a", ids[r], (double)w[r]);
    printf("\n");
}

static void die(const char *what) {
    fprintf(stderr, "ref_routes: %s: %s\n", what, tlm_errmsg());
    exit(1);
}

int main(int argc, char **argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: ref_routes STORE.tlmm id,id,...\n");
        return 2;
    }
    tlm_manifest m;
    if (tlm_manifest_load(&m, argv[1])) die("manifest");
    char paths[TLM_MAX_DRIVES][1024];
    const char *pp[TLM_MAX_DRIVES];
    for (uint32_t d = 0; d < m.n_drives; d++) {
        tlm_manifest_drive_path(&m, (int)d, paths[d], sizeof paths[d]);
        pp[d] = paths[d];
    }
    tlm_io_opts io;
    memset(&io, 0, sizeof io);
    io.threads_per_drive = 4;
    tlm_io *fio = tlm_io_open(pp, (int)m.n_drives, &io);
    if (!fio) die("io");
    uint64_t slot = 0, total = 0;
    for (uint32_t i = 0; i < m.n_packets; i++)
        if (m.packets[i].type == TLM_PK_EXPERT && !(m.packets[i].flags & 2u)) {
            total += m.packets[i].total_len;
            if (m.packets[i].total_len > slot) slot = m.packets[i].total_len;
        }
    tlm_store_opts so;
    memset(&so, 0, sizeof so);
    so.budget_bytes = total + slot;
    tlm_store *st = tlm_store_open(&m, fio, &so);
    if (!st) die("store");
    tlm_pool *pool = tlm_pool_new(0, 0);
    if (!pool) die("pool");
    tlm_model_opts mo = {0, 0, 0.0};
    tlm_model *mdl = tlm_model_open(&m, fio, st, pool, &mo);
    if (!mdl) die("model");
    tlm_model_set_route_hook(mdl, on_route, NULL);
    int n = 1;
    for (const char *c = argv[2]; *c; c++) n += *c == ',';
    tlm_kv *kv = tlm_kv_new(mdl, n + 1);
    if (!kv) die("kv");
    const char *c = argv[2];
    for (int i = 0; i < n; i++) {
        int tok = (int)strtol(c, (char **)&c, 10);
        if (*c == ',') c++;
        if (tlm_model_step(mdl, kv, tok, NULL)) die("step");
    }
    tlm_kv_free(kv);
    tlm_model_close(mdl);
    tlm_store_close(st);
    tlm_io_close(fio);
    tlm_pool_free(pool);
    tlm_manifest_free(&m);
    return 0;
}
