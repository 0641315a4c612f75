/* tlm_oracle_store.c - TEST INFRASTRUCTURE ONLY: the reference's expert slot
 * cache policy restated on the CPU (declarations and the time model in
 * tlm_oracle_store.h).  Each function cites the reference lines it follows.
 *
 * Pinning: tests/test_store_policy.py runs the same operation scripts through
 * this restatement and through the reference's own tlm_store.c (compiled from
 * its sources into oracle/_ref with a packet-store fixture) and requires
 * identical slots, return codes and counters at every step, plus the
 * reference's known-answer scenarios (tests/test_store.c:356-470 there). */
#include "tlm_oracle_store.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

enum { E_OK = 0, E_IO = -1, E_NOMEM = -2, E_INVAL = -3, E_FORMAT = -4, E_NOTFOUND = -6, E_BUSY = -8 };
enum { S_FREE = 0, S_LOADING = 1, S_READY = 2 };
enum { K_DEMAND = 0, K_HINT = 1, K_PIN = 2 };

#define DECAY_TICKS 16   /* tlm_store.c:41 */
#define HINT_BACKLOG 4   /* tlm_store.c:42 */
#define HINT_INFLIGHT 16 /* tlm_store.c:43 */

typedef struct {
    ostore_src src;
    uint32_t freq;
    int slot;
    int fail;
} o_ex;

typedef struct {
    int state, ex, refs, pinned, hinted, demand, err;
    uint64_t last;
} o_slot;

struct ostore {
    int n_ex, n_slots, reserve, prefetch;
    double pin_frac;
    o_ex *ex;
    o_slot *sl;
    uint64_t clock, ticks;
    int loading, demand_loading, hint_loading, n_pinned;
    ostore_stats st;
};

static int find(const ostore *o, int layer, int id) {
    if (layer < 0 || id < 0) return -1;
    for (int i = 0; i < o->n_ex; i++)
        if (o->ex[i].src.layer == layer && o->ex[i].src.id == (uint32_t)id) return i;
    return -1;
}

ostore *ostore_open(const ostore_src *src, int n, int top_k, int n_slots, double pin_frac, int prefetch) {
    ostore *o = (ostore *)calloc(1, sizeof *o);
    if (!o) return NULL;
    o->ex = (o_ex *)calloc(n > 0 ? (size_t)n : 1, sizeof *o->ex);
    for (int i = 0; i < n; i++) {
        if (src[i].flags & 2u) continue;   /* pruned: not in the store (tlm_store.c:429) */
        o->ex[o->n_ex].src = src[i];
        o->ex[o->n_ex].slot = -1;
        o->n_ex++;
    }
    /* tlm_store.c:406: reserve = top_k clamped to [1, 1024] */
    o->reserve = top_k > 0 ? (top_k > 1024 ? 1024 : top_k) : 1;
    o->prefetch = prefetch;
    o->pin_frac = pin_frac;
    if (o->n_ex) {   /* tlm_store.c:449-452 */
        int ns = n_slots < 1 ? 1 : n_slots;
        o->n_slots = ns > o->n_ex ? o->n_ex : ns;
    }
    o->sl = (o_slot *)calloc(o->n_slots ? (size_t)o->n_slots : 1, sizeof *o->sl);
    for (int i = 0; i < o->n_slots; i++) o->sl[i].ex = -1;
    return o;
}

void ostore_close(ostore *o) {
    if (!o) return;
    free(o->sl);
    free(o->ex);
    free(o);
}

int ostore_n_slots(const ostore *o) { return o ? o->n_slots : 0; }

/* fail_slot, tlm_store.c:139-158 */
static void fail_slot(ostore *o, int v, int err) {
    o_slot *s = &o->sl[v];
    if (s->ex >= 0 && o->ex[s->ex].slot == v) o->ex[s->ex].slot = -1;
    if (s->state == S_LOADING) {
        o->loading--;
        if (s->demand) o->demand_loading--;
        else o->hint_loading--;
    }
    s->state = S_FREE;
    if (s->pinned) o->n_pinned--;
    s->pinned = s->hinted = s->demand = 0;
    s->last = 0;
    if (s->refs > 0) {
        s->err = err;
    } else {
        s->err = 0;
        s->ex = -1;
    }
}

/* start_load, tlm_store.c:162-189 (the submit itself cannot fail here) */
static void start_load(ostore *o, int v, int e, int kind) {
    o_slot *s = &o->sl[v];
    if (s->state == S_READY && s->ex >= 0) {
        o->ex[s->ex].slot = -1;
        o->st.evictions++;
    }
    o->loading++;
    s->state = S_LOADING;
    s->ex = e;
    o->ex[e].slot = v;
    s->refs = kind == K_HINT ? 0 : 1;
    s->pinned = kind == K_PIN;
    if (s->pinned) o->n_pinned++;
    s->hinted = kind == K_HINT;
    s->demand = kind != K_HINT;
    if (s->demand) o->demand_loading++;
    else o->hint_loading++;
    s->err = 0;
    s->last = kind == K_HINT ? 0 : o->clock;
}

/* the publish step of on_read_done, tlm_store.c:249-295 */
static void complete(ostore *o, int v) {
    o_slot *s = &o->sl[v];
    if (s->state != S_LOADING) return;
    if (o->ex[s->ex].fail) {
        fail_slot(o, v, E_FORMAT);
        return;
    }
    s->state = S_READY;
    o->loading--;
    if (s->demand) o->demand_loading--;
    else o->hint_loading--;
    o->st.loads++;
}

/* pick_victim, tlm_store.c:196-214: first FREE slot; else the READY slot of
 * lowest (freq, last use), lowest index on a tie; hints only take freq 0 */
static int pick_victim(const ostore *o, int kind) {
    int best = -1;
    uint32_t bf = 0;
    uint64_t bl = 0;
    for (int i = 0; i < o->n_slots; i++) {
        const o_slot *s = &o->sl[i];
        if (s->refs > 0 || s->pinned) continue;
        if (s->state == S_FREE) return i;
        if (s->state != S_READY) continue;
        uint32_t f = o->ex[s->ex].freq;
        if (kind == K_HINT && f > 0) continue;
        if (best < 0 || f < bf || (f == bf && s->last < bl)) {
            best = i;
            bf = f;
            bl = s->last;
        }
    }
    return best;
}

/* take_ref, tlm_store.c:216-234 */
static void take_ref(ostore *o, int v, uint64_t stamp) {
    o_slot *s = &o->sl[v];
    s->refs++;
    s->last = stamp;
    if (s->hinted) {
        s->hinted = 0;
        o->st.prefetch_used++;
    }
    if (s->state == S_LOADING && !s->demand) {
        s->demand = 1;
        o->hint_loading--;
        o->demand_loading++;
    }
}

/* drop_ref_locked, tlm_store.c:236-246 */
static void drop_ref(ostore *o, int v) {
    o_slot *s = &o->sl[v];
    if (s->refs <= 0) return;
    if (--s->refs == 0 && s->state == S_FREE) {
        s->err = 0;
        s->ex = -1;
    }
}

typedef struct {
    int e, cp;
    float heat;
    uint32_t seed;
    uint16_t layer;
    uint32_t id;
} pin_cand;

/* pin order, tlm_store.c:516-523: compiler pins, heat, sidecar count, then
 * (layer, id) ascending */
static int pin_order(const void *a, const void *b) {
    const pin_cand *x = (const pin_cand *)a, *y = (const pin_cand *)b;
    if (x->cp != y->cp) return x->cp ? -1 : 1;
    if (x->heat != y->heat) return x->heat > y->heat ? -1 : 1;
    if (x->seed != y->seed) return x->seed > y->seed ? -1 : 1;
    if (x->layer != y->layer) return x->layer < y->layer ? -1 : 1;
    return x->id < y->id ? -1 : x->id > y->id;
}

/* tlm_store_warm, tlm_store.c:525-583 */
int ostore_warm(ostore *o) {
    if (!o) return E_INVAL;
    if (o->n_slots == 0) return E_OK;
    double frac = o->pin_frac;
    if (!(frac > 0.0)) return E_OK;
    if (frac > 0.9) frac = 0.9;
    int target = (int)floor(frac * o->n_slots);
    if (target > o->n_slots - 1) target = o->n_slots - 1;
    if (target <= 0) return E_OK;
    pin_cand *c = (pin_cand *)malloc(sizeof *c * (size_t)(o->n_ex ? o->n_ex : 1));
    int *mine = (int *)malloc(sizeof *mine * (size_t)target);
    int nc = 0;
    for (int i = 0; i < o->n_ex; i++) {
        const ostore_src *x = &o->ex[i].src;
        int cp = (x->flags & 1u) != 0;
        if (!cp && !(x->heat > 0.0f) && x->seed == 0) continue;
        c[nc].e = i;
        c[nc].cp = cp;
        c[nc].heat = x->heat;
        c[nc].seed = x->seed;
        c[nc].layer = x->layer;
        c[nc].id = x->id;
        nc++;
    }
    qsort(c, (size_t)nc, sizeof *c, pin_order);
    int pinned = o->n_pinned, n_mine = 0, rc = E_OK;
    for (int i = 0; i < nc && pinned < target; i++) {
        int e = c[i].e, v = o->ex[e].slot;
        if (v >= 0) {
            if (!o->sl[v].pinned) {
                o->sl[v].pinned = 1;
                o->n_pinned++;
                pinned++;
            }
            continue;
        }
        v = pick_victim(o, K_PIN);
        if (v < 0) break;
        start_load(o, v, e, K_PIN);
        mine[n_mine++] = v;
        pinned++;
    }
    for (int i = 0; i < n_mine; i++) {
        complete(o, mine[i]);
        o_slot *s = &o->sl[mine[i]];
        if (s->state != S_READY && rc == E_OK) rc = s->err ? s->err : E_IO;
        drop_ref(o, mine[i]);
    }
    free(c);
    free(mine);
    return rc;
}

/* tlm_store_acquire, tlm_store.c:586-640 */
int ostore_acquire(ostore *o, int layer, const int32_t *ids, int k, int32_t *slots) {
    if (!o || k < 0 || (k > 0 && (!ids || !slots))) return E_INVAL;
    int rc = E_OK;
    uint64_t stamp = ++o->clock;
    for (int i = 0; i < k; i++) {
        slots[i] = -1;
        int e = find(o, layer, ids[i]);
        if (e < 0) {
            if (rc == E_OK) rc = E_NOTFOUND;
            continue;
        }
        if (o->ex[e].freq < UINT32_MAX) o->ex[e].freq++;
    }
    for (int i = 0; i < k; i++) {   /* hits first: a miss never evicts this step's hit */
        int e = find(o, layer, ids[i]);
        if (e < 0 || o->ex[e].slot < 0) continue;
        take_ref(o, o->ex[e].slot, stamp);
        slots[i] = o->ex[e].slot;
        o->st.hits++;
    }
    for (int i = 0; i < k; i++) {
        if (slots[i] >= 0) continue;
        int e = find(o, layer, ids[i]);
        if (e < 0) continue;
        if (o->ex[e].slot >= 0) {   /* repeated id, placed earlier in this pass */
            take_ref(o, o->ex[e].slot, stamp);
            slots[i] = o->ex[e].slot;
            o->st.hits++;
            continue;
        }
        int v = pick_victim(o, K_DEMAND);
        if (v < 0) {
            if (rc == E_OK) rc = E_BUSY;
            continue;
        }
        o->st.misses++;
        start_load(o, v, e, K_DEMAND);
        slots[i] = v;
    }
    return rc;
}

/* tlm_store_wait, tlm_store.c:642-671 (the load completes now) */
int ostore_wait(ostore *o, int slot) {
    if (!o || slot < 0 || slot >= o->n_slots) return E_INVAL;
    complete(o, slot);
    const o_slot *s = &o->sl[slot];
    if (s->state == S_READY) return E_OK;
    return s->err ? s->err : E_IO;
}

int ostore_is_ready(const ostore *o, int slot) {
    return o && slot >= 0 && slot < o->n_slots && o->sl[slot].state == S_READY;
}

/* tlm_store_release, tlm_store.c:681-692 */
void ostore_release(ostore *o, int slot) {
    if (o && slot >= 0 && slot < o->n_slots) drop_ref(o, slot);
}

/* tlm_store_prefetch, tlm_store.c:694-718 */
void ostore_prefetch(ostore *o, int layer, const int32_t *ids, int k) {
    if (!o || !o->prefetch || !ids || k <= 0) return;
    int cap = o->n_slots - o->n_pinned - o->reserve;
    if (cap > HINT_INFLIGHT) cap = HINT_INFLIGHT;
    for (int i = 0; i < k; i++) {
        int e = find(o, layer, ids[i]);
        if (e < 0 || o->ex[e].slot >= 0) continue;
        if (o->demand_loading > HINT_BACKLOG || o->hint_loading >= cap) {
            o->st.prefetch_dropped++;
            continue;
        }
        int v = pick_victim(o, K_HINT);
        if (v < 0) {
            o->st.prefetch_dropped++;
            continue;
        }
        start_load(o, v, e, K_HINT);
        o->st.prefetch_issued++;
    }
}

/* tlm_store_tick, tlm_store.c:720-726 */
void ostore_tick(ostore *o) {
    if (!o) return;
    if (++o->ticks % DECAY_TICKS == 0)
        for (int i = 0; i < o->n_ex; i++) o->ex[i].freq >>= 1;
}

void ostore_settle(ostore *o) {
    if (!o) return;
    for (int v = 0; v < o->n_slots; v++) complete(o, v);
}

/* tlm_store_get_stats, tlm_store.c:728-740 */
void ostore_get_stats(const ostore *o, ostore_stats *st) {
    memset(st, 0, sizeof *st);
    if (!o) return;
    *st = o->st;
    st->slots = o->n_slots;
    st->pinned = o->n_pinned;
    for (int i = 0; i < o->n_slots; i++) st->in_use += o->sl[i].refs > 0;
}

void ostore_set_fail(ostore *o, int layer, int id, int on) {
    int e = o ? find(o, layer, id) : -1;
    if (e >= 0) o->ex[e].fail = on;
}

int64_t ostore_slot_expert(const ostore *o, int slot) {
    if (!o || slot < 0 || slot >= o->n_slots || o->sl[slot].ex < 0) return -1;
    const ostore_src *s = &o->ex[o->sl[slot].ex].src;
    return ((int64_t)s->layer << 32) | s->id;
}
