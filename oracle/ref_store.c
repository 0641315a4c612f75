/* ref_store.c - TEST INFRASTRUCTURE ONLY: puts the reference's own expert
 * slot cache (src/lib/tlm_store.c) over a small packet store written with the
 * reference's writer (src/lib/tlm_packet.c) on one drive directory, so tests
 * can drive tlm_store_* through ctypes and compare it with the oracle's
 * restatement (tlm_oracle_store.c).  Linked only into oracle/_ref/libtlmref.so.
 *
 * Every expert payload has the same length, so every packet has the same
 * total_len and the store's slot size is that length; payload bytes are a
 * function of (layer, id).  No replicas: a corrupted packet fails its load. */
#include "tlm_io.h"
#include "tlm_packet.h"
#include "tlm_platform.h"
#include "tlm_store.h"

#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

typedef struct {
    tlm_manifest m;
    tlm_io *io;
    tlm_store *s;
    char path[512];
} ref_fx;

static void fx_bytes(uint8_t *p, uint64_t n, uint64_t seed) {
    uint64_t x = seed * 0x9E3779B97F4A7C15ull + 1;
    for (uint64_t i = 0; i < n; i++) {
        x ^= x << 13;
        x ^= x >> 7;
        x ^= x << 17;
        p[i] = (uint8_t)(x >> 56);
    }
}

/* flags / heat / seed are per (layer * ne + id); n_slots whole slots. */
ref_fx *ref_store_fixture(const char *dir, int nl, int ne, int top_k, const uint16_t *flags, const float *heat,
                          uint64_t payload_len, int n_slots, double pin_frac, int prefetch) {
    ref_fx *f = (ref_fx *)calloc(1, sizeof *f);
    if (!f) return NULL;
    const char *dirs[1] = {dir};
    tlm_store_writer *w = tlm_writer_open("fx", dirs, 1);
    if (!w) goto fail;
    tlm_packet_loc *locs = (tlm_packet_loc *)calloc((size_t)(nl * ne), sizeof *locs);
    uint8_t *buf = (uint8_t *)malloc(payload_len);
    for (int l = 0; l < nl; l++)
        for (int e = 0; e < ne; e++) {
            fx_bytes(buf, payload_len, (uint64_t)(l * 1000 + e));
            uint32_t item[3] = {0, (uint32_t)(payload_len / 3), (uint32_t)(2 * payload_len / 3)};
            tlm_packet_loc *lc = &locs[l * ne + e];
            if (tlm_writer_add(w, TLM_PK_EXPERT, (uint16_t)l, (uint32_t)e, TLM_DT_Q8_0, buf, payload_len, item, 0, -1,
                               lc) != 0) {
                free(buf);
                free(locs);
                tlm_writer_free(w);
                goto fail;
            }
            lc->heat = heat ? heat[l * ne + e] : 0.0f;
            lc->flags = flags ? flags[l * ne + e] : 0;
        }
    free(buf);
    if (tlm_writer_finish(w, 1) != 0) {
        free(locs);
        tlm_writer_free(w);
        goto fail;
    }
    tlm_writer_free(w);
    tlm_manifest m;
    memset(&m, 0, sizeof m);
    snprintf(m.geom.arch, sizeof m.geom.arch, "tlm-moe");
    m.geom.n_layers = (uint32_t)nl;
    m.geom.n_experts = (uint32_t)ne;
    m.geom.top_k = (uint32_t)top_k;
    m.geom.d_model = 64;
    snprintf(m.name, sizeof m.name, "fx");
    snprintf(m.profile, sizeof m.profile, "exact");
    m.n_drives = 1;
    snprintf(m.drives[0], sizeof m.drives[0], "%.255s", dir);
    m.n_packets = (uint32_t)(nl * ne);
    m.packets = locs;
    char mpath[600];
    snprintf(mpath, sizeof mpath, "%s/fx.tlmm", dir);
    int rc = tlm_manifest_save(&m, mpath);
    free(locs);
    if (rc != 0 || tlm_manifest_load(&f->m, mpath) != 0) goto fail;
    tlm_manifest_drive_path(&f->m, 0, f->path, sizeof f->path);
    const char *pp[1] = {f->path};
    tlm_io_opts io = {TLM_IO_PREAD, 0, 2, 16};
    f->io = tlm_io_open(pp, 1, &io);
    if (!f->io) goto fail;
    uint64_t slot = f->m.n_packets ? f->m.packets[0].total_len : 0;
    tlm_store_opts o;
    memset(&o, 0, sizeof o);
    o.budget_bytes = (uint64_t)n_slots * slot + slot / 2;
    o.pin_frac = pin_frac;
    o.prefetch = prefetch;
    f->s = tlm_store_open(&f->m, f->io, &o);
    if (!f->s) goto fail;
    return f;
fail:
    if (f->io) tlm_io_close(f->io);
    free(f);
    return NULL;
}

tlm_store *ref_store_handle(ref_fx *f) { return f ? f->s : NULL; }

/* Wait until no slot is LOADING: tlm_store_wait on each slot index returns
 * once that slot has left LOADING (it takes and drops no reference). */
void ref_store_settle(ref_fx *f) {
    int n = tlm_store_n_slots(f->s);
    for (int v = 0; v < n; v++) {
        tlm_expert_ref r = {v, NULL, 0};
        (void)tlm_store_wait(f->s, &r);
    }
}

/* Flip one payload byte of packet (layer, id) on disk; a second call repairs it. */
int ref_store_corrupt(ref_fx *f, int layer, int id) {
    const tlm_packet_loc *l = tlm_manifest_find(&f->m, TLM_PK_EXPERT, (uint16_t)layer, (uint32_t)id);
    if (!l) return -1;
    int fd = open(f->path, O_RDWR);
    if (fd < 0) return -1;
    uint8_t b = 0;
    off_t at = (off_t)(l->offset + 64 + 7);
    int ok = pread(fd, &b, 1, at) == 1;
    b ^= 0x5A;
    ok = ok && pwrite(fd, &b, 1, at) == 1;
    close(fd);
    return ok ? 0 : -1;
}

void ref_store_fixture_close(ref_fx *f) {
    if (!f) return;
    tlm_store_close(f->s);
    tlm_io_close(f->io);
    tlm_manifest_free(&f->m);
    free(f);
}
