/* tlm_oracle_store.h - TEST INFRASTRUCTURE ONLY (never linked into the
 * product): a CPU restatement of the reference's routed-expert slot cache
 * policy, src/lib/tlm_store.c:139-740, with loads modelled as explicit events.
 *
 * Slot decisions (which slot a miss or hint takes, which expert is evicted,
 * what is dropped, every counter) follow the reference exactly; the only
 * modelling choice is time: a load started by acquire / prefetch / warm stays
 * LOADING until ostore_settle() or ostore_wait() completes it.  At points
 * where the reference has no read in flight, the two agree state for state. */
#ifndef TLM_ORACLE_STORE_H
#define TLM_ORACLE_STORE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    uint16_t layer;
    uint32_t id;
    uint16_t flags;   /* bit0 compiler pin, bit1 pruned (tlm_store.c:43-44) */
    float    heat;    /* manifest selection frequency */
    uint32_t seed;    /* warm-sidecar count */
} ostore_src;

typedef struct {
    uint64_t hits, misses, prefetch_issued, prefetch_used, prefetch_dropped;
    uint64_t loads, evictions;   /* loads: completed (READY) loads */
    int32_t  slots, pinned, in_use;
} ostore_stats;

typedef struct ostore ostore;

/* n_slots: whole slots the budget holds (clamped to [1, live experts] as
 * tlm_store.c:449-452 does; 0 when no live expert). */
ostore *ostore_open(const ostore_src *src, int n, int top_k, int n_slots, double pin_frac, int prefetch);
void    ostore_close(ostore *o);
int     ostore_n_slots(const ostore *o);
int     ostore_warm(ostore *o);
int     ostore_acquire(ostore *o, int layer, const int32_t *ids, int k, int32_t *slots);
int     ostore_wait(ostore *o, int slot);
int     ostore_is_ready(const ostore *o, int slot);
void    ostore_release(ostore *o, int slot);
void    ostore_prefetch(ostore *o, int layer, const int32_t *ids, int k);
void    ostore_tick(ostore *o);
/* complete every in-flight load */
void    ostore_settle(ostore *o);
void    ostore_get_stats(const ostore *o, ostore_stats *st);
/* while set, loads of (layer, id) complete as failures (TLM_EFORMAT) */
void    ostore_set_fail(ostore *o, int layer, int id, int on);
/* expert held by `slot` as layer << 32 | id, or -1 */
int64_t ostore_slot_expert(const ostore *o, int slot);

#ifdef __cplusplus
}
#endif
#endif
