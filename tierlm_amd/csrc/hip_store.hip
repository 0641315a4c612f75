/* hip_store.hip - the routed-expert slot cache moved into HBM
 * (tlm_hip_store_*; the reference's RAM cache is src/lib/tlm_store.c).
 *
 * Policy - slot lifecycle FREE -> LOADING -> READY, hits referenced before
 * misses choose victims, victims by lowest (decayed selection count, last
 * use), halving every 16 ticks, pins, and the hint rules - is the reference's
 * (src/lib/tlm_store.c:139-740); the same operation scripts give the same
 * slots and counters (tests/test_hip_store.py).  What changes is where the
 * bytes live and how they get there:
 *
 *   - one hipMalloc arena of equal slots; a slot holds an expert's gate, up
 *     and down in the packed tile layout the MoE kernels read;
 *   - a load is three pack kernels on the store's own stream that read the
 *     payload over PCIe straight from page-locked host memory - where it
 *     lies, or a staging buffer the loader thread first copies a pageable
 *     payload into (or the fetch callback fills) - and write the slot; then
 *     an event per slot.  The caller's stream never blocks on a load;
 *   - READY is published when the host sees the slot's event complete;
 *     tlm_hip_store_stream_wait lets a stream wait for a LOADING slot on the
 *     device instead;
 *   - release only notes the caller's stream; the first load that evicts a
 *     released slot records one event on that stream (shared by every such
 *     load until the next release) and the slot's packs wait for it, so a
 *     slot is never overwritten while kernels enqueued before its release
 *     still read it, and all-hit steps make no runtime calls for it.
 *
 * Threading: one mutex guards the policy state; the loader thread takes it
 * only to pick up jobs and to publish a submitted load. */
#include "tlm_hip_internal.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <mutex>
#include <thread>
#include <unordered_map>
#include <vector>

int tlmh_current_device(void);

namespace {

enum { S_FREE = 0, S_LOADING = 1, S_READY = 2 };
enum { K_DEMAND = 0, K_HINT = 1, K_PIN = 2 };
constexpr int DECAY_TICKS = 16;      /* tlm_store.c:41 */
constexpr int HINT_BACKLOG = 4;      /* tlm_store.c:42 */
constexpr int HINT_INFLIGHT = 16;    /* tlm_store.c:43 */
constexpr int NSTAGE = 3;            /* staging buffers for pageable payloads */
constexpr int NLOAD = 2;             /* load streams: consecutive loads overlap */
constexpr size_t MAT_ALIGN = 256;
constexpr int MAX_HINTS = 7;         /* lookahead layers per tlm_hip_moe_layer_store call */
constexpr int ROUTE_BYTES = 256;     /* ids int32[32] at +0, w f32[32] at +128 (moe_route_offset) */
/* a route area: the block's and its hints' routes, then the sequence word the
 * export stores last; NAREA areas, so the host reads one layer's routes while
 * later layers' exports land in the others */
constexpr int ROUTE_AREA = ROUTE_BYTES * (1 + MAX_HINTS) + 64;
constexpr int ROUTE_SEQ = ROUTE_BYTES * (1 + MAX_HINTS);   /* byte offset of the sequence word */
constexpr int NAREA = 4;
constexpr int MOE_MAXK = 32;

struct Expert {
    tlm_hip_expert_src src;
    size_t off[3];          /* packed gate / up / down inside a slot */
    int64_t rows[3], n[3];
    const void *dev_src;    /* the payload's device-visible address when it lies in page-locked
                               host memory, else NULL (copied through staging) */
    uint32_t freq = 0;
    int slot = -1;
};

struct Slot {
    int state = S_FREE, ex = -1, refs = 0, pinned = 0, hinted = 0, demand = 0, err = 0;
    uint64_t last = 0;
    uint64_t gen = 0;           /* bumped by every start_load */
    bool submitted = false;     /* `loaded` recorded for generation gen */
    bool reads_pending = false; /* released since the last load took it: kernels may still read it */
    hipStream_t rel_stream = nullptr;
    hipEvent_t loaded = nullptr;
};

struct Job {
    int v, e;
    uint64_t gen;
    int rel;                    /* release point the packs wait for, or -1 */
};

uint64_t key_of(int layer, int id) { return ((uint64_t)(uint32_t)layer << 32) | (uint32_t)id; }

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

int64_t now_ns() {
    return std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

}  // namespace

struct tlm_hip_store {
    std::mutex mu;
    std::condition_variable cv;
    int device = -1;
    hipStream_t lstream[NLOAD] = {};     /* load streams, used in turn */
    int lnext = 0;                       /* loader thread only */
    tlm_hip_store_opts o{};
    std::vector<Expert> ex;
    std::unordered_map<uint64_t, int> index;
    int n_slots = 0, reserve = 1;
    size_t slot_bytes = 0, stage_bytes = 0;
    uint8_t *arena = nullptr;
    std::vector<Slot> sl;
    uint8_t *stage_host[NSTAGE] = {};   /* page-locked staging for pageable payloads */
    const uint8_t *stage_dev[NSTAGE] = {};  /* their device-visible addresses */
    hipEvent_t stage_packed[NSTAGE] = {};
    int stage_next = 0;                 /* loader thread only */
    std::deque<Job> jobs;
    int unsubmitted = 0;                /* LOADING slots whose job has not been submitted */
    std::thread loader;
    bool stop = false;
    uint64_t clock = 0, ticks = 0;
    int loading = 0, demand_loading = 0, hint_loading = 0, n_pinned = 0;
    tlm_hip_store_stats st{};
    uint8_t *route_host = nullptr;      /* pinned: NAREA route areas (ROUTE_AREA bytes each) */
    uint32_t *route_dev = nullptr;      /* route_host as the device addresses it (mapped, coherent) */
    uint32_t route_seq = 0;             /* the last export's sequence number */
    int route_n[NAREA] = {};            /* routes in each area */
    /* The expert -> slot table the device-resolved blocks read (mapped,
     * coherent host memory; row `layer` of tab_E entries): a slot's index is
     * stored by the load stream right after its packs (so an entry is never
     * ahead of the bytes), and set back to -1 by the host when the slot is
     * chosen as a victim, before its new load is queued. */
    int32_t *tab_host = nullptr, *tab_dev = nullptr;
    int tab_L = 0, tab_E = 0;
    bool uniform = false;               /* every expert's matrices at the same offsets in a slot */
    size_t uoff[3] = {0, 0, 0};
    /* per route area, whether the export resolved every routed slot (1) or
     * handed the layer back (0); mapped, coherent */
    uint32_t *rep_host = nullptr, *rep_dev = nullptr;
    int32_t *res_dev = nullptr;         /* device: the resolved slots, NAREA x 32 */

    size_t tab_index(int e) const { return (size_t)ex[e].src.layer * tab_E + ex[e].src.id; }
    void tab_set(int e, int32_t v) {
        if (tab_host && e >= 0) __atomic_store_n(tab_host + tab_index(e), v, __ATOMIC_RELEASE);
    }
    /* release points: an event recorded on a release stream when a load first
     * needs one, shared by every load that needs a point on that stream
     * before the next release; reused once no queued load waits for it */
    std::vector<hipEvent_t> rel_ev;
    std::vector<int> rel_users;
    int rel_cur = -1;
    hipStream_t rel_cur_stream = nullptr;
    uint64_t release_seq = 0, rel_cur_seq = 0;

    int find(int layer, int id) const {
        if (layer < 0 || id < 0) return -1;
        auto it = index.find(key_of(layer, id));
        return it == index.end() ? -1 : it->second;
    }

    /* ---- policy (all with mu held) ------------------------------------ */
    void fail_slot(int v, int err) {            /* tlm_store.c:139-158 */
        Slot &s = sl[v];
        if (s.ex >= 0) tab_set(s.ex, -1);
        if (s.ex >= 0 && ex[s.ex].slot == v) ex[s.ex].slot = -1;
        if (s.state == S_LOADING) {
            loading--;
            if (s.demand) demand_loading--;
            else hint_loading--;
            if (!s.submitted) unsubmitted--;
        }
        s.state = S_FREE;
        if (s.pinned) n_pinned--;
        s.pinned = s.hinted = s.demand = 0;
        s.last = 0;
        s.submitted = false;
        if (s.refs > 0) {
            s.err = err;
        } else {
            s.err = 0;
            s.ex = -1;
        }
        cv.notify_all();
    }

    void start_load(int v, int e, int kind) {   /* tlm_store.c:162-189 */
        Slot &s = sl[v];
        if (s.state == S_READY && s.ex >= 0) {
            ex[s.ex].slot = -1;
            tab_set(s.ex, -1);
            st.evictions++;
        }
        loading++;
        s.state = S_LOADING;
        s.ex = e;
        ex[e].slot = v;
        s.refs = kind == K_HINT ? 0 : 1;
        s.pinned = kind == K_PIN;
        if (s.pinned) n_pinned++;
        s.hinted = kind == K_HINT;
        s.demand = kind != K_HINT;
        if (s.demand) demand_loading++;
        else hint_loading++;
        s.err = 0;
        s.last = kind == K_HINT ? 0 : clock;
        s.gen++;
        s.submitted = false;
        unsubmitted++;
        int rel = -1;
        if (s.reads_pending) {
            rel = release_point(s.rel_stream);
            s.reads_pending = false;
        }
        jobs.push_back(Job{v, e, s.gen, rel});
        cv.notify_all();
    }

    /* An event on `stream` after every release so far (the slot's readers
     * were all enqueued before it).  Recording it here, at the first load
     * that needs it, rather than at each release keeps all-hit steps free of
     * runtime calls.  -1 if no event could be recorded: then the stream is
     * drained on the host instead. */
    int release_point(hipStream_t stream) {
        if (rel_cur >= 0 && rel_cur_stream == stream && rel_cur_seq == release_seq) {
            rel_users[rel_cur]++;
            return rel_cur;
        }
        int idx = -1;
        for (int i = 0; i < (int)rel_ev.size() && idx < 0; i++)
            if (rel_users[i] == 0) idx = i;
        if (idx < 0) {
            hipEvent_t ev;
            if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
                (void)hipStreamSynchronize(stream);
                return -1;
            }
            rel_ev.push_back(ev);
            rel_users.push_back(0);
            idx = (int)rel_ev.size() - 1;
        }
        if (hipEventRecord(rel_ev[idx], stream) != hipSuccess) {
            (void)hipStreamSynchronize(stream);
            return -1;
        }
        rel_cur = idx;
        rel_cur_stream = stream;
        rel_cur_seq = release_seq;
        rel_users[idx] = 1;
        return idx;
    }

    void complete(int v) {                      /* the publish step, tlm_store.c:273-282 */
        Slot &s = sl[v];
        s.state = S_READY;
        loading--;
        if (s.demand) demand_loading--;
        else hint_loading--;
        st.bytes_read += ex[s.ex].src.payload_len;
        cv.notify_all();
    }

    /* LOADING -> READY once the slot's event has completed on the device */
    void refresh(int v) {
        Slot &s = sl[v];
        if (s.state != S_LOADING || !s.submitted) return;
        hipError_t q = hipEventQuery(s.loaded);
        if (q == hipSuccess) complete(v);
        else if (q != hipErrorNotReady) fail_slot(v, tlmh_check(q, "store: load"));
    }
    void refresh_all() {
        for (int v = 0; v < n_slots; v++) refresh(v);
    }

    /* Victim choice (the rule of tlm_store.c:196-214): among slots that are
     * neither referenced nor pinned, the smallest eviction key - a FREE slot
     * before any READY one, then the lower decayed selection count, then the
     * older last use, then the lower slot index; a LOADING slot never
     * qualifies, and a hint takes only FREE slots or READY slots whose count
     * has decayed to 0.  -1 if nothing qualifies. */
    struct EvictKey {
        int busy;           /* 0 FREE, 1 READY */
        uint32_t freq;
        uint64_t last;
        int slot;
        bool operator<(const EvictKey &o) const {
            if (busy != o.busy) return busy < o.busy;
            if (freq != o.freq) return freq < o.freq;
            if (last != o.last) return last < o.last;
            return slot < o.slot;
        }
    };
    bool evictable(int v, int kind, EvictKey *key) const {
        const Slot &s = sl[v];
        if (s.refs > 0 || s.pinned || s.state == S_LOADING) return false;
        const bool free_slot = s.state == S_FREE;
        const uint32_t f = free_slot ? 0u : ex[s.ex].freq;
        if (!free_slot && kind == K_HINT && f > 0) return false;
        *key = EvictKey{free_slot ? 0 : 1, free_slot ? 0u : f, free_slot ? 0ull : s.last, v};
        return true;
    }
    int pick_victim(int kind) const {
        bool any = false;
        EvictKey best{};
        for (int v = 0; v < n_slots; v++) {
            EvictKey k;
            if (evictable(v, kind, &k) && (!any || k < best)) {
                best = k;
                any = true;
                if (k.busy == 0) break;   /* nothing beats the first FREE slot */
            }
        }
        return any ? best.slot : -1;
    }

    /* where slot v's expert matrices sit */
    void describe(int v, tlm_hip_expert_ref *r) const {
        r->slot = v;
        const Expert &x = ex[sl[v].ex];
        for (int m = 0; m < 3; m++) r->mats[m] = arena + (size_t)v * slot_bytes + x.off[m];
    }
    /* A step takes slot v (its expert is resident or on its way): one more
     * reference, last use now; a hinted expert counts as a used prefetch
     * once, and a hint still loading becomes demand traffic (the rules of
     * tlm_store.c:216-234). */
    void attach(int v, uint64_t stamp, tlm_hip_expert_ref *r) {
        Slot &s = sl[v];
        s.refs += 1;
        s.last = stamp;
        st.prefetch_used += s.hinted ? 1 : 0;
        s.hinted = 0;
        if (s.state == S_LOADING && s.demand == 0) {
            s.demand = 1;
            hint_loading -= 1;
            demand_loading += 1;
        }
        describe(v, r);
    }

    void drop_ref(int v) {                      /* tlm_store.c:236-246 */
        Slot &s = sl[v];
        if (s.refs <= 0) return;
        if (--s.refs == 0 && s.state == S_FREE) {
            s.err = 0;
            s.ex = -1;
        }
    }

    /* ---- the loader thread ------------------------------------------------ */
    /* The pack kernels read the payload straight from page-locked host
     * memory over PCIe (the caller's, or the staging buffer a pageable
     * payload is first copied into) and write the slot: one pass, no DMA
     * engine, no cross-stream dependency. */
    int run_job(const Job &j) {
        const Expert &x = ex[j.e];
        int rc = TLM_HIP_OK;
        hipStream_t packs = lstream[lnext];
        lnext = (lnext + 1) % NLOAD;
        {
            std::lock_guard<std::mutex> lk(mu);
            if (j.rel >= 0) {   /* kernels enqueued before the slot's release may still read it */
                rc = tlmh_check(hipStreamWaitEvent(packs, rel_ev[j.rel], 0), "store: wait for release");
                rel_users[j.rel]--;
                if (rc) return rc;
            }
            const Slot &s = sl[j.v];
            if (s.gen != j.gen || s.state != S_LOADING) return TLM_HIP_OK;   /* superseded */
        }
        const uint8_t *src = (const uint8_t *)x.dev_src;
        int i = -1;
        if (!src) {
            i = stage_next;
            stage_next = (stage_next + 1) % NSTAGE;
            /* the staging buffer is free once the packs that read it have run */
            if ((rc = tlmh_check(hipEventSynchronize(stage_packed[i]), "store: staging buffer"))) return rc;
            if (x.src.payload) {
                memcpy(stage_host[i], x.src.payload, x.src.payload_len);
            } else {
                rc = o.fetch(o.fetch_user, x.src.layer, (int)x.src.id, stage_host[i], x.src.payload_len);
                if (rc) return rc < 0 ? rc : TLM_HIP_EIO;
            }
            src = stage_dev[i];
        }
        uint8_t *base = arena + (size_t)j.v * slot_bytes;
        const int dt = x.src.dtype;
        for (int m = 0; m < 3 && !rc; m++)
            rc = launch_pack(dt, src + x.src.item_off[m], (size_t)(x.n[m] / dt_block_values(dt)) *
                             (size_t)dt_block_bytes(dt), x.rows[m], x.n[m], base + x.off[m], packs);
        if (!rc && tab_dev) rc = launch_publish_slot(tab_dev + tab_index(j.e), j.v, packs);
        if (!rc) rc = tlmh_check(hipEventRecord(sl[j.v].loaded, packs), "store: record load");
        if (rc) (void)hipStreamSynchronize(packs);   /* no half-done load may race a later one into the slot */
        if (i >= 0) {
            const int rc2 = tlmh_check(hipEventRecord(stage_packed[i], packs), "store: record staging");
            if (!rc) rc = rc2;
        }
        return rc;
    }

    void loader_main() {
        (void)hipSetDevice(device);
        for (;;) {
            Job j;
            {
                std::unique_lock<std::mutex> lk(mu);
                cv.wait(lk, [&] { return stop || !jobs.empty(); });
                if (jobs.empty()) return;
                j = jobs.front();
                jobs.pop_front();
            }
            int rc = run_job(j);
            std::lock_guard<std::mutex> lk(mu);
            Slot &s = sl[j.v];
            if (s.gen != j.gen || s.state != S_LOADING) continue;
            if (rc) {
                fail_slot(j.v, rc);
            } else {
                s.submitted = true;
                unsubmitted--;
                cv.notify_all();
            }
        }
    }

    /* A demand miss found no victim while some unreferenced, unpinned slot is
     * still LOADING (a caller that waits on the device runs ahead of the
     * loads): block until one such load has finished, as the reference's
     * read would have by then.  false when there is none (then: EBUSY). */
    bool wait_unreferenced_load(std::unique_lock<std::mutex> &lk) {
        int v = -1;
        for (int i = 0; i < n_slots && v < 0; i++)
            if (sl[i].state == S_LOADING && sl[i].refs == 0 && !sl[i].pinned) v = i;
        if (v < 0) return false;
        const int64_t t0 = now_ns();
        const uint64_t gen = sl[v].gen;
        cv.wait(lk, [&] { return sl[v].gen != gen || sl[v].state != S_LOADING || sl[v].submitted; });
        if (sl[v].gen == gen && sl[v].state == S_LOADING) {
            hipEvent_t ev = sl[v].loaded;
            lk.unlock();
            (void)hipEventSynchronize(ev);
            lk.lock();
            refresh(v);
        }
        st.wait_ns += (uint64_t)(now_ns() - t0);
        return true;
    }

    /* wait (mu held through lk) until no job is queued or unsubmitted */
    void drain_jobs(std::unique_lock<std::mutex> &lk) {
        cv.wait(lk, [&] { return unsubmitted == 0 && jobs.empty(); });
    }

    void destroy() {
        if (loader.joinable()) {
            {
                std::unique_lock<std::mutex> lk(mu);
                drain_jobs(lk);
                stop = true;
                cv.notify_all();
            }
            loader.join();
        }
        for (hipStream_t q : lstream)
            if (q) (void)hipStreamSynchronize(q);
        for (Slot &s : sl)
            if (s.loaded) (void)hipEventDestroy(s.loaded);
        for (hipEvent_t ev : rel_ev) (void)hipEventDestroy(ev);
        for (int i = 0; i < NSTAGE; i++) {
            if (stage_packed[i]) (void)hipEventDestroy(stage_packed[i]);
            if (stage_host[i]) (void)hipHostFree(stage_host[i]);
        }
        if (arena) (void)hipFree(arena);
        if (route_host) (void)hipHostFree(route_host);
        if (tab_host) (void)hipHostFree(tab_host);
        if (rep_host) (void)hipHostFree(rep_host);
        if (res_dev) (void)hipFree(res_dev);
        for (hipStream_t q : lstream)
            if (q) (void)hipStreamDestroy(q);
    }
};

namespace {

struct PinCand {
    int e, cp;
    float heat;
    uint32_t seed;
    uint16_t layer;
    uint32_t id;
};

/* tlm_store.c:516-523: compiler pins, heat, sidecar count, (layer, id) */
bool pin_before(const PinCand &x, const PinCand &y) {
    if (x.cp != y.cp) return x.cp > y.cp;
    if (x.heat != y.heat) return x.heat > y.heat;
    if (x.seed != y.seed) return x.seed > y.seed;
    if (x.layer != y.layer) return x.layer < y.layer;
    return x.id < y.id;
}

/* The device-visible address of a host pointer into page-locked memory that
 * is mapped for the device, else NULL (pageable memory: copied through
 * staging). */
const void *device_view(const void *p) {
    hipPointerAttribute_t a;
    hipError_t e = hipPointerGetAttributes(&a, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();   /* an unknown (pageable) pointer is not an error here */
        return nullptr;
    }
    return a.type == hipMemoryTypeHost ? a.devicePointer : nullptr;
}

}  // namespace

extern "C" {

int tlm_hip_store_open(const tlm_hip_expert_src *src, int n, const tlm_hip_store_opts *o, tlm_hip_store **out) {
    if (!out) return tlmh_seterr(TLM_HIP_EINVAL, "store open: NULL out");
    *out = nullptr;
    if (!o || n < 0 || (n > 0 && !src)) return tlmh_seterr(TLM_HIP_EINVAL, "store open: bad arguments");
    const int dev = tlmh_current_device();
    if (dev < 0) return tlmh_seterr(TLM_HIP_EUNSUP, "store open: tlm_hip_init has not run");
    const int64_t D = o->d_model, de = o->d_expert;
    if (D <= 0 || de <= 0) return tlmh_seterr(TLM_HIP_EINVAL, "store open: d_model %lld, d_expert %lld",
                                              (long long)D, (long long)de);
    tlm_hip_store *s = new (std::nothrow) tlm_hip_store;
    if (!s) return tlmh_seterr(TLM_HIP_ENOMEM, "store open: out of memory");
    s->device = dev;
    s->o = *o;
    s->reserve = o->top_k > 0 ? std::min(o->top_k, 1024) : 1;   /* tlm_store.c:406 */
    for (int i = 0; i < n; i++) {
        const tlm_hip_expert_src &x = src[i];
        if (x.flags & 2u) continue;   /* pruned (tlm_store.c:429) */
        const int dt = x.dtype;
        if (dt != DT_Q8_0 && dt != DT_Q4_K && dt != DT_Q5_K && dt != DT_Q6_K) {
            delete s;
            return tlmh_seterr(TLM_HIP_EUNSUP, "store open: expert %u:%u dtype %d", x.layer, x.id, dt);
        }
        const int bv = dt_block_values(dt);
        if (D % bv || de % bv) {
            delete s;
            return tlmh_seterr(TLM_HIP_EINVAL, "store open: d_model / d_expert not multiples of %d", bv);
        }
        Expert e;
        e.src = x;
        e.rows[0] = e.rows[1] = de;
        e.n[0] = e.n[1] = D;
        e.rows[2] = D;
        e.n[2] = de;
        size_t at = 0;
        for (int m = 0; m < 3; m++) {
            const uint64_t raw = (uint64_t)(e.n[m] / bv) * dt_block_bytes(dt) * (uint64_t)e.rows[m];
            if ((uint64_t)x.item_off[m] + raw > x.payload_len) {
                delete s;
                return tlmh_seterr(TLM_HIP_EFORMAT, "store open: expert %u:%u item %d overruns its payload",
                                   x.layer, x.id, m);
            }
            e.off[m] = at;
            at += align_up(packed_bytes(dt, e.rows[m], e.n[m]), MAT_ALIGN);
        }
        if (!x.payload && !o->fetch) {
            delete s;
            return tlmh_seterr(TLM_HIP_EINVAL, "store open: expert %u:%u has no payload and no fetch", x.layer, x.id);
        }
        e.dev_src = x.payload ? device_view(x.payload) : nullptr;
        s->slot_bytes = std::max(s->slot_bytes, at);
        s->stage_bytes = std::max(s->stage_bytes, (size_t)x.payload_len);
        const uint64_t k = key_of(x.layer, (int)x.id);
        if (s->index.count(k)) {
            delete s;
            return tlmh_seterr(TLM_HIP_EFORMAT, "store open: duplicate expert %u:%u", x.layer, x.id);
        }
        s->index[k] = (int)s->ex.size();
        s->ex.push_back(e);
    }
    int rc = TLM_HIP_OK;
    if (!s->ex.empty()) {   /* tlm_store.c:449-457: whole slots, at least one, at most one per expert */
        uint64_t ns = o->budget_bytes / s->slot_bytes;
        ns = std::max<uint64_t>(ns, 1);
        ns = std::min<uint64_t>(ns, s->ex.size());
        s->n_slots = (int)ns;
        s->sl.resize(ns);
        rc = tlmh_check(hipMalloc((void **)&s->arena, ns * s->slot_bytes), "store: slot arena");
        for (size_t v = 0; v < ns && !rc; v++) {
            rc = tlmh_check(hipEventCreateWithFlags(&s->sl[v].loaded, hipEventDisableTiming), "store: event");
        }
        for (int q = 0; q < NLOAD && !rc; q++)
            rc = tlmh_check(hipStreamCreateWithFlags(&s->lstream[q], hipStreamNonBlocking), "store: load stream");
        for (int i = 0; i < NSTAGE && !rc; i++) {
            rc = tlmh_check(hipHostMalloc((void **)&s->stage_host[i], s->stage_bytes, hipHostMallocMapped),
                            "store: pinned staging");
            void *dp = nullptr;
            if (!rc) rc = tlmh_check(hipHostGetDevicePointer(&dp, s->stage_host[i], 0), "store: staging address");
            s->stage_dev[i] = (const uint8_t *)dp;
            if (!rc) rc = tlmh_check(hipEventCreateWithFlags(&s->stage_packed[i], hipEventDisableTiming), "store: event");
        }
        /* mapped and coherent: k_moe_route_host stores the routing straight into it, its sequence
         * word last; the host waits for that word instead of synchronising the stream */
        if (!rc) rc = tlmh_check(hipHostMalloc((void **)&s->route_host, NAREA * ROUTE_AREA,
                                               hipHostMallocMapped | hipHostMallocCoherent), "store: routing scratch");
        if (!rc) memset(s->route_host, 0, NAREA * ROUTE_AREA);
        if (!rc) rc = tlmh_check(hipHostGetDevicePointer((void **)&s->route_dev, s->route_host, 0),
                                 "store: routing scratch address");
        /* the device-resolved blocks' table and control words */
        int maxl = 0, maxe = 0;
        s->uniform = true;
        for (const Expert &x : s->ex) {
            maxl = std::max(maxl, (int)x.src.layer);
            maxe = std::max(maxe, (int)x.src.id);
            for (int m = 0; m < 3; m++) s->uniform = s->uniform && x.off[m] == s->ex[0].off[m];
        }
        for (int m = 0; m < 3; m++) s->uoff[m] = s->ex[0].off[m];
        s->tab_L = maxl + 1;
        s->tab_E = maxe + 1;
        const size_t tn = (size_t)s->tab_L * s->tab_E;
        if (!rc) rc = tlmh_check(hipHostMalloc((void **)&s->tab_host, tn * 4, hipHostMallocMapped | hipHostMallocCoherent),
                                 "store: slot table");
        if (!rc) {
            for (size_t i = 0; i < tn; i++) s->tab_host[i] = -1;
            rc = tlmh_check(hipHostGetDevicePointer((void **)&s->tab_dev, s->tab_host, 0), "store: slot table address");
        }
        if (!rc) rc = tlmh_check(hipHostMalloc((void **)&s->rep_host, NAREA * 4, hipHostMallocMapped | hipHostMallocCoherent),
                                 "store: export reports");
        if (!rc) {
            memset(s->rep_host, 0, NAREA * 4);
            rc = tlmh_check(hipHostGetDevicePointer((void **)&s->rep_dev, s->rep_host, 0), "store: export reports address");
        }
        if (!rc) rc = tlmh_check(hipMalloc((void **)&s->res_dev, NAREA * 32 * 4), "store: resolved slots");
        if (!rc) rc = tlmh_check(hipMemset(s->res_dev, 0, NAREA * 32 * 4), "store: resolved slots");
        if (!rc) s->loader = std::thread([s] { s->loader_main(); });
    }
    if (rc) {
        s->destroy();
        delete s;
        return rc;
    }
    *out = s;
    return TLM_HIP_OK;
}

void tlm_hip_store_close(tlm_hip_store *s) {
    if (!s) return;
    s->destroy();
    delete s;
}

int tlm_hip_store_n_slots(const tlm_hip_store *s) { return s ? s->n_slots : 0; }
uint64_t tlm_hip_store_slot_bytes(const tlm_hip_store *s) { return s ? s->slot_bytes : 0; }

/* Pinning at start (the rules of tlm_store.c:525-583): a pin budget of
 * floor(min(pin_frac, 0.9) x slots), never all of them; candidates are the
 * experts the compiler flagged, or with heat or a sidecar count, in
 * pin_before order; a resident candidate is pinned where it is, any other is
 * loaded into a victim slot as a pin; the call returns once its own loads
 * have finished. */
static int pin_budget(const tlm_hip_store *s) {
    const double frac = s->o.pin_frac > 0.9 ? 0.9 : s->o.pin_frac;
    if (!(frac > 0.0)) return 0;
    const int want = (int)floor(frac * s->n_slots);
    return std::max(0, std::min(want, s->n_slots - 1));
}

static std::vector<PinCand> pin_candidates(const tlm_hip_store *s) {
    std::vector<PinCand> c;
    for (int i = 0; i < (int)s->ex.size(); i++) {
        const tlm_hip_expert_src &x = s->ex[i].src;
        const PinCand pc{i, (x.flags & 1u) ? 1 : 0, x.heat, x.seed, x.layer, x.id};
        if (pc.cp || pc.heat > 0.0f || pc.seed != 0) c.push_back(pc);
    }
    std::stable_sort(c.begin(), c.end(), pin_before);
    return c;
}

/* block until a slot this call started loading has left LOADING */
static void settle_slot(tlm_hip_store *s, std::unique_lock<std::mutex> &lk, int v) {
    Slot &sl = s->sl[v];
    while (sl.state == S_LOADING) {
        if (!sl.submitted) {
            s->cv.wait(lk);
            continue;
        }
        hipEvent_t ev = sl.loaded;
        lk.unlock();
        (void)hipEventSynchronize(ev);
        lk.lock();
        s->refresh(v);
    }
}

int tlm_hip_store_warm(tlm_hip_store *s) {
    if (!s) return tlmh_seterr(TLM_HIP_EINVAL, "store warm: no store given");
    const int budget = s->n_slots ? pin_budget(s) : 0;
    if (budget <= 0) return TLM_HIP_OK;
    std::unique_lock<std::mutex> lk(s->mu);
    const std::vector<PinCand> cand = pin_candidates(s);
    std::vector<int> started;
    /* start_load counts a pin load in n_pinned at once, as pinning in place does */
    for (size_t i = 0; i < cand.size() && s->n_pinned < budget; i++) {
        const int e = cand[i].e, resident = s->ex[e].slot;
        if (resident >= 0) {
            if (!s->sl[resident].pinned) {
                s->sl[resident].pinned = 1;
                s->n_pinned++;
            }
            continue;
        }
        const int v = s->pick_victim(K_PIN);
        if (v < 0) break;
        s->start_load(v, e, K_PIN);
        started.push_back(v);
    }
    int rc = TLM_HIP_OK;
    for (int v : started) {
        settle_slot(s, lk, v);
        if (s->sl[v].state != S_READY && rc == TLM_HIP_OK) {
            const int err = s->sl[v].err ? s->sl[v].err : TLM_HIP_EIO;
            rc = tlmh_seterr(err, "store warm: a slot chosen for pinning ended without its expert");
        }
        s->drop_ref(v);
    }
    return rc;
}

/* One step's experts of a layer (the rules of tlm_store.c:586-640): every
 * known id is counted as selected; then a pass over the resident experts
 * references them, so that no miss of this step can evict them; then the
 * misses in rank order take victims and start loading (an id repeated in the
 * step finds the slot its first occurrence took). */
int tlm_hip_store_acquire(tlm_hip_store *s, int layer, const int *ids, int k, tlm_hip_expert_ref *out) {
    if (!s || k < 0 || (k > 0 && (!ids || !out)))
        return tlmh_seterr(TLM_HIP_EINVAL, "store acquire: no store, or a negative count, or no ids / output");
    std::unique_lock<std::mutex> lk(s->mu);
    s->refresh_all();
    const uint64_t stamp = ++s->clock;
    int rc = TLM_HIP_OK;
    std::vector<int> exp_of(k);
    for (int i = 0; i < k; i++) {
        out[i] = tlm_hip_expert_ref{};
        out[i].slot = -1;
        exp_of[i] = s->find(layer, ids[i]);
        if (exp_of[i] < 0) {
            if (rc == TLM_HIP_OK)
                rc = tlmh_seterr(TLM_HIP_ENOTFOUND, "store acquire: no routable expert %d in layer %d", ids[i], layer);
        } else if (s->ex[exp_of[i]].freq != UINT32_MAX) {
            s->ex[exp_of[i]].freq += 1;
        }
    }
    for (int pass = 0; pass < 2; pass++) {   /* 0: resident experts, 1: everything still missing */
        for (int i = 0; i < k; i++) {
            const int e = exp_of[i];
            if (e < 0 || out[i].slot >= 0) continue;
            if (s->ex[e].slot >= 0) {
                s->attach(s->ex[e].slot, stamp, &out[i]);
                s->st.hits++;
                continue;
            }
            if (pass == 0) continue;
            int v = s->pick_victim(K_DEMAND);
            while (v < 0 && s->wait_unreferenced_load(lk)) v = s->pick_victim(K_DEMAND);
            if (v < 0) {
                if (rc == TLM_HIP_OK)
                    rc = tlmh_seterr(TLM_HIP_EBUSY, "store acquire: none of the %d slots is free to evict (each is "
                                     "referenced or pinned); keep top_k slots unpinned", s->n_slots);
                continue;
            }
            s->st.misses++;
            s->start_load(v, e, K_DEMAND);
            s->describe(v, &out[i]);
        }
    }
    return rc;
}

static int wait_status(tlm_hip_store *s, int v) {
    const Slot &sl = s->sl[v];
    if (sl.state == S_READY) return TLM_HIP_OK;
    const int rc = sl.err ? sl.err : TLM_HIP_EIO;
    if (sl.ex >= 0)
        return tlmh_seterr(rc, "store: layer %u expert %u could not be loaded", s->ex[sl.ex].src.layer,
                           s->ex[sl.ex].src.id);
    return tlmh_seterr(rc, "store: expert could not be loaded");
}

/* tlm_store.c:642-671: blocks the host until the slot is READY */
int tlm_hip_store_wait(tlm_hip_store *s, tlm_hip_expert_ref *ref) {
    if (!s || !ref) return tlmh_seterr(TLM_HIP_EINVAL, "store wait: no store or slot given");
    if (ref->slot < 0 || ref->slot >= s->n_slots) return tlmh_seterr(TLM_HIP_EINVAL, "store wait: the slot holds no acquired expert");
    const int v = ref->slot;
    std::unique_lock<std::mutex> lk(s->mu);
    int64_t t0 = 0;
    Slot &sl = s->sl[v];
    s->refresh(v);
    while (sl.state == S_LOADING) {
        if (!t0) t0 = now_ns();
        if (!sl.submitted) {
            s->cv.wait(lk);
            continue;
        }
        hipEvent_t ev = sl.loaded;
        lk.unlock();
        (void)hipEventSynchronize(ev);
        lk.lock();
        s->refresh(v);
    }
    if (t0) s->st.wait_ns += (uint64_t)(now_ns() - t0);
    return wait_status(s, v);
}

/* The device-side wait: work enqueued on `stream` after this call runs after
 * the slot's load.  The host blocks only until the load has been submitted. */
int tlm_hip_store_stream_wait(tlm_hip_store *s, const tlm_hip_expert_ref *ref, void *stream) {
    if (!s || !ref) return tlmh_seterr(TLM_HIP_EINVAL, "store stream wait: no store or slot given");
    if (ref->slot < 0 || ref->slot >= s->n_slots)
        return tlmh_seterr(TLM_HIP_EINVAL, "store stream wait: the slot holds no acquired expert");
    const int v = ref->slot;
    std::unique_lock<std::mutex> lk(s->mu);
    Slot &sl = s->sl[v];
    s->refresh(v);
    s->cv.wait(lk, [&] { return sl.state != S_LOADING || sl.submitted; });
    if (sl.state == S_LOADING)
        return tlmh_check(hipStreamWaitEvent((hipStream_t)stream, sl.loaded, 0), "store: stream wait");
    return wait_status(s, v);
}

int tlm_hip_store_is_ready(tlm_hip_store *s, const tlm_hip_expert_ref *ref) {
    if (!s || !ref || ref->slot < 0 || ref->slot >= s->n_slots) return 0;
    std::lock_guard<std::mutex> lk(s->mu);
    s->refresh(ref->slot);
    return s->sl[ref->slot].state == S_READY;
}

/* tlm_store.c:681-692, plus the device-side ordering: the slot is not
 * overwritten before the work enqueued on `stream` up to now has finished */
void tlm_hip_store_release(tlm_hip_store *s, tlm_hip_expert_ref *ref, void *stream) {
    if (!s || !ref) return;
    if (ref->slot >= 0 && ref->slot < s->n_slots) {
        std::lock_guard<std::mutex> lk(s->mu);
        Slot &sl = s->sl[ref->slot];
        if (sl.refs > 0) {
            sl.reads_pending = true;
            sl.rel_stream = (hipStream_t)stream;
            s->release_seq++;
        }
        s->drop_ref(ref->slot);
    }
    ref->slot = -1;
    ref->mats[0] = ref->mats[1] = ref->mats[2] = nullptr;
}

/* A release whose readers have all finished by the time any later load can
 * start (the device-resolved stack's layers before its last): no release
 * point is kept for the slot. */
static void release_retired(tlm_hip_store *s, tlm_hip_expert_ref *ref) {
    if (ref->slot >= 0 && ref->slot < s->n_slots) {
        std::lock_guard<std::mutex> lk(s->mu);
        s->drop_ref(ref->slot);
    }
    ref->slot = -1;
    ref->mats[0] = ref->mats[1] = ref->mats[2] = nullptr;
}

/* Lookahead hints (the rules of tlm_store.c:694-718): an expert not yet
 * resident is loaded ahead only while at most HINT_BACKLOG demand loads are
 * in flight and fewer hints than the hint budget (slots minus pins minus the
 * top_k reserve, at most HINT_INFLIGHT) are, and only into a slot a hint may
 * take (pick_victim); otherwise the hint is dropped and counted. */
static bool hint_admitted(const tlm_hip_store *s) {
    const int budget = std::min(HINT_INFLIGHT, s->n_slots - s->n_pinned - s->reserve);
    return s->demand_loading <= HINT_BACKLOG && s->hint_loading < budget;
}

void tlm_hip_store_prefetch(tlm_hip_store *s, int layer, const int *ids, int k) {
    if (!s || !s->o.prefetch || !ids || k <= 0) return;
    std::lock_guard<std::mutex> lk(s->mu);
    s->refresh_all();
    for (int i = 0; i < k; i++) {
        const int e = s->find(layer, ids[i]);
        if (e < 0 || s->ex[e].slot >= 0) continue;   /* unknown, or resident / already loading */
        const int v = hint_admitted(s) ? s->pick_victim(K_HINT) : -1;
        if (v < 0) {
            s->st.prefetch_dropped++;
            continue;
        }
        s->start_load(v, e, K_HINT);
        s->st.prefetch_issued++;
    }
}

/* One step of time (tlm_store.c:720-726): every DECAY_TICKS ticks the
 * selection counts halve, so old popularity fades. */
void tlm_hip_store_tick(tlm_hip_store *s) {
    if (!s) return;
    std::lock_guard<std::mutex> lk(s->mu);
    s->ticks += 1;
    if (s->ticks % DECAY_TICKS != 0) return;
    for (Expert &x : s->ex) x.freq /= 2;
}

/* Every queued load submitted and finished (READY or failed). */
int tlm_hip_store_drain(tlm_hip_store *s) {
    if (!s) return tlmh_seterr(TLM_HIP_EINVAL, "store drain: NULL");
    std::unique_lock<std::mutex> lk(s->mu);
    s->drain_jobs(lk);
    lk.unlock();
    int rc = TLM_HIP_OK;
    for (hipStream_t q : s->lstream)
        if (q && !rc) rc = tlmh_check(hipStreamSynchronize(q), "store drain");
    lk.lock();
    s->refresh_all();
    return rc;
}

/* tlm_store.c:728-740 */
void tlm_hip_store_get_stats(tlm_hip_store *s, tlm_hip_store_stats *out) {
    if (!out) return;
    memset(out, 0, sizeof *out);
    if (!s) return;
    std::lock_guard<std::mutex> lk(s->mu);
    *out = s->st;
    out->slots = s->n_slots;
    out->pinned = s->n_pinned;
    for (const Slot &sl : s->sl) out->in_use += sl.refs > 0;
}


}  // extern "C"

/* ---- one MoE block through the cache -------------------------------------- */
namespace {


/* the block's route and its hints' routes from h (the residual before the
 * block's update): their routers in one launch, then their routing into route
 * area `area` of the host under a new sequence number (returned in *seq) */
int enqueue_routes(tlm_hip_store *s, const tlm_hip_moe_desc *d, float *h, void *ws, const tlm_hip_moe_desc *hd,
                   void *const *hws, int n_hints, int area, uint32_t *seq, hipStream_t st) {
    const tlm_hip_moe_desc *ds[1 + MAX_HINTS];
    void *wss[1 + MAX_HINTS];
    ds[0] = d;
    wss[0] = ws;
    for (int i = 0; i < n_hints; i++) {
        ds[1 + i] = &hd[i];
        wss[1 + i] = hws[i];
    }
    *seq = ++s->route_seq;
    s->route_n[area] = 1 + n_hints;
    return launch_moe_routes_host(ds, wss, 1 + n_hints, h, s->route_dev + area * (ROUTE_AREA / 4), ROUTE_SEQ, *seq,
                                  st);
}

/* wait (spinning, no stream synchronisation) until every route of area
 * `area` carries sequence number seq; a stream error or a minute without
 * them is an error */
int wait_routes(tlm_hip_store *s, int area, uint32_t seq, hipStream_t st) {
    const uint32_t *w = (const uint32_t *)(s->route_host + (size_t)area * ROUTE_AREA + ROUTE_SEQ);
    const int n = s->route_n[area];
    auto arrived = [&] {
        for (int i = 0; i < n; i++)
            if (__atomic_load_n(w + i, __ATOMIC_ACQUIRE) != seq) return false;
        return true;
    };
    const int64_t t0 = now_ns();
    for (uint64_t i = 0;; i++) {
        if (arrived()) return TLM_HIP_OK;
        if ((i & 4095) == 4095) {
            const hipError_t e = hipStreamQuery(st);
            if (e != hipSuccess && e != hipErrorNotReady) return tlmh_check(e, "moe_layer_store: stream");
            if (e == hipSuccess && !arrived())
                return tlmh_seterr(TLM_HIP_EIO, "moe_layer_store: the routing export did not arrive");
            if (now_ns() - t0 > 60ll * 1000000000ll)
                return tlmh_seterr(TLM_HIP_EIO, "moe_layer_store: no routing export after 60 s");
        }
        __builtin_ia32_pause();
    }
}

/* acquire the routed experts (ids[0..k), weights w), make the stream wait
 * for loads in flight and enqueue phases 2 and 3 on the slots' matrices;
 * refs hold the references (released by the caller, also on an error) */
int run_block(tlm_hip_store *s, const tlm_hip_moe_desc *d, int layer, const int *ids, const float *w, float *h,
              void *ws, tlm_hip_expert_ref *refs, hipStream_t st) {
    const int k = d->k;
    for (int r = 0; r < k; r++) {
        refs[r] = tlm_hip_expert_ref{};
        refs[r].slot = -1;
    }
    for (int r = 0; r < k; r++)   /* the table write below indexes 3 * id + m */
        if (ids[r] < 0 || ids[r] >= d->E)
            return tlmh_seterr(TLM_HIP_EIO, "moe_layer_store: routing produced expert %d of %d", ids[r], d->E);
    int rc = tlm_hip_store_acquire(s, layer, ids, k, refs);
    if (rc) return rc;
    /* the routing and the slots' matrices go to the block as launch
     * arguments: its weight loads start at once, no table is written */
    MoeGiven gv{};
    gv.on = 1;
    for (int r = 0; r < k; r++) {
        gv.ids[r] = ids[r];
        gv.w[r] = w[r];
        for (int m = 0; m < 3; m++) gv.p[3 * r + m] = (const uint8_t *)refs[r].mats[m];
    }
    for (int r = 0; r < k && !rc; r++) rc = tlm_hip_store_stream_wait(s, &refs[r], st);
    if (!rc) rc = launch_moe_phase_given(d, 2, h, ws, &gv, st);
    if (!rc) rc = launch_moe_phase_given(d, 3, h, ws, &gv, st);
    return rc;
}

}  // namespace

extern "C" {

/* moe() with the store, src/lib/tlm_model.c:960-1055: route, acquire the
 * routed experts, issue the lookahead hints (:988-991, lookahead() :844-877),
 * run the block once every expert's load has landed, release. */
int tlm_hip_moe_layer_store(const tlm_hip_moe_desc *d, tlm_hip_store *s, int layer, float *h, int32_t *ids_host,
                            float *w_host, const tlm_hip_moe_hint *hints, int n_hints, void *workspace,
                            void *stream) {
    if (!d || !s || !h || !workspace || n_hints < 0 || n_hints > MAX_HINTS || (n_hints > 0 && !hints))
        return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer_store: bad arguments");
    if (d->k <= 0 || d->k > MOE_MAXK) return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer_store: k=%d", d->k);
    /* each route lands in its own workspace until one export reads them all:
     * no two of them (the block's, the hints') may share a byte */
    const uint8_t *lo[1 + MAX_HINTS];
    size_t len[1 + MAX_HINTS];
    lo[0] = (const uint8_t *)workspace;
    len[0] = moe_workspace_bytes(d);
    for (int i = 0; i < n_hints; i++) {
        if (!hints[i].desc || !hints[i].workspace)
            return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer_store: hint %d has no descriptor or workspace", i);
        lo[1 + i] = (const uint8_t *)hints[i].workspace;
        len[1 + i] = moe_workspace_bytes(hints[i].desc);
    }
    for (int a = 0; a <= n_hints; a++)
        for (int b = a + 1; b <= n_hints; b++)
            if (lo[a] < lo[b] + len[b] && lo[b] < lo[a] + len[a])
                return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer_store: %s%d and hint %d share workspace bytes",
                                   a ? "hint " : "the block's workspace ", a ? a - 1 : 0, b - 1);
    hipStream_t st = (hipStream_t)stream;
    /* every route first (the hints read the same residual, before this
     * block's update), then one round trip for all of them */
    tlm_hip_moe_desc hd[MAX_HINTS];
    void *hws[MAX_HINTS];
    for (int i = 0; i < n_hints; i++) {
        hd[i] = *hints[i].desc;
        hws[i] = hints[i].workspace;
    }
    uint32_t seq = 0;
    int rc = enqueue_routes(s, d, h, workspace, hd, hws, n_hints, 0, &seq, st);
    if (!rc) rc = wait_routes(s, 0, seq, st);
    if (rc) return rc;
    const int k = d->k;
    int ids[MOE_MAXK];
    memcpy(ids, s->route_host, sizeof(int) * k);
    if (ids_host) memcpy(ids_host, ids, sizeof(int) * k);
    if (w_host) memcpy(w_host, s->route_host + 128, sizeof(float) * k);
    tlm_hip_expert_ref refs[MOE_MAXK];
    float w[MOE_MAXK];
    memcpy(w, s->route_host + 128, sizeof(float) * k);
    rc = run_block(s, d, layer, ids, w, h, workspace, refs, st);
    /* hints while this block's experts still hold references (:988-990), issued after the block's
     * launches so that the loader's bookkeeping is off the path to them */
    for (int i = 0; i < n_hints && !rc; i++)
        tlm_hip_store_prefetch(s, hints[i].layer, (const int *)(s->route_host + ROUTE_BYTES * (1 + i)),
                               hints[i].desc->k);
    for (int r = 0; r < k; r++) tlm_hip_store_release(s, &refs[r], stream);
    return rc;
}

/* the lookahead's workspaces after the two block workspaces, each 256-byte
 * aligned: block[2], then hint[2][depth] */
static void stack_layout(const tlm_hip_moe_desc *descs, int n, int depth, int lk, size_t *blk, size_t *hint) {
    size_t b = 0, hb = 0;
    for (int l = 0; l < n; l++) {
        b = std::max(b, moe_workspace_bytes(&descs[l]));
        if (depth > 0) {
            tlm_hip_moe_desc d = descs[l];
            d.k = lk > 0 ? std::min(lk, d.E) : d.k;
            hb = std::max(hb, moe_workspace_bytes(&d));
        }
    }
    *blk = align_up(b, 256);
    *hint = align_up(hb, 256);
}

static int stack_depth(const tlm_hip_stack_opts *o) {
    const int d = o ? o->lookahead : 0;
    return d < 0 ? 0 : d > MAX_HINTS ? MAX_HINTS : d;
}

size_t tlm_hip_moe_stack_workspace_bytes(const tlm_hip_moe_desc *descs, int n_layers, const tlm_hip_stack_opts *o) {
    if (!descs || n_layers <= 0) return 0;
    size_t b, hb;
    const int depth = stack_depth(o);
    stack_layout(descs, n_layers, depth, o ? o->lookahead_k : 0, &b, &hb);
    return 2 * b + 2 * (size_t)depth * hb;
}

}  // extern "C"

/* the instinct update of tlm_model.c:974-980 from a layer's routing */
static void update_instinct(const tlm_hip_stack_opts *o, int l, const float *w, int k) {
    if (!o || !o->instinct || !o->instinct_seen) return;
    double sw = 0.0;
    for (int r = 0; r < k; r++) sw += (double)w[r];
    const double share = sw > 0.0 ? (double)w[0] / sw : 0.0;
    o->instinct[l] += (share - o->instinct[l]) * 0.05;
    o->instinct_seen[l]++;
}

/* lookahead() for layers l+1 .. l+n (tlm_model.c:844-877) from the hint routes
 * of route area `area` (hints routed hd[i].k wide), the breadth
 * interest-weighted (:863-874) */
static void issue_hints(tlm_hip_store *s, const tlm_hip_stack_opts *o, const tlm_hip_moe_desc *descs, int l,
                        const tlm_hip_moe_desc *hd, int n, const uint8_t *area, int layer0) {
    for (int i = 0; i < n; i++) {
        const int tl = l + 1 + i, hk = hd[i].k, top = descs[tl].k;
        const int32_t *hid = (const int32_t *)(area + ROUTE_BYTES * (1 + i));
        const float *hw = (const float *)(area + ROUTE_BYTES * (1 + i) + 128);
        int kk = hk;
        if (o && o->interest > 0.0 && hk > top) {
            double sw = 0.0;
            for (int r = 0; r < hk; r++) sw += (double)hw[r];
            const double now = sw > 0.0 ? (double)hw[0] / sw : 0.0;
            const bool seen = o->instinct_seen && o->instinct && o->instinct_seen[tl];
            const double I = seen ? 0.5 * (now + o->instinct[tl]) : now;
            const double Hh = o->layer_heat ? (double)o->layer_heat[tl] : 0.0;
            double W = o->interest * (1.0 - I) * (1.0 - Hh);
            W = W < 0.0 ? 0.0 : W > 1.0 ? 1.0 : W;
            kk = top + (int)(W * (double)(hk - top) + 0.5);
            kk = std::min(kk, hd[i].E);
        }
        tlm_hip_store_prefetch(s, layer0 + tl, (const int *)hid, kk);
    }
}

/* layer l's hint descriptors: the next n layers' blocks, routed lk wide */
static int hint_descs(const tlm_hip_moe_desc *descs, int n_layers, int l, int depth, int lk, tlm_hip_moe_desc *hd) {
    const int nh = std::min(depth, n_layers - 1 - l);
    for (int i = 0; i < nh; i++) {
        hd[i] = descs[l + 1 + i];
        hd[i].k = lk > 0 ? std::min(lk, hd[i].E) : hd[i].k;
    }
    return nh;
}

/* Whether the blocks can resolve their slots on the device: the slots share
 * one layout, and every layer's experts index the store's table. */
static bool dev_resolvable(const tlm_hip_store *s, const tlm_hip_moe_desc *descs, int n_layers, int layer0) {
    if (!s->uniform || !s->tab_host || !s->rep_host || !s->res_dev || layer0 + n_layers > s->tab_L) return false;
    for (int l = 0; l < n_layers; l++)
        if (descs[l].E > s->tab_E || descs[l].k > MOE_MAXK) return false;
    return true;
}

/* The stack with the slots resolved on the device where they can be (the
 * default).  Per layer the host enqueues what precedes the router (before),
 * the routers, the export - which also reads the routed experts' slots from
 * the store's expert -> slot table - and the two block launches that read
 * those slots; then it replays the layer's store operations from the export
 * in the reference's order (acquire, hints, release; one tick at the end).
 * When every routed expert's load had landed, the block is already running
 * on the slots the export found; otherwise the export handed the layer back
 * (its block launches do nothing) and the host runs it as the host-resolved
 * path does, behind them: the stream waits for the loads, then the block
 * with the slots' matrices as arguments.  Nothing on the device waits for
 * the host or for a load, so no queue the loads share can stall behind it.
 *
 * Why no slot is overwritten while a block reads it: a victim is chosen only
 * while the host replays some layer m - after layer m's export, which runs
 * after every block before layer m (and any block the host ran for one of
 * them) has finished - and never among layer m's routed experts, acquired
 * before any miss chooses a victim and held through the hints; and layer
 * m + 1's export, which reads the table, is enqueued only after that replay
 * has cleared every victim's entry.  The last layer's slots keep a release
 * point on the stream, for whatever the caller enqueues next. */
static int moe_stack_run_dev(const tlm_hip_moe_desc *descs, int n_layers, tlm_hip_store *s, float *h,
                             const tlm_hip_stack_opts *o, int32_t *ids_out, float *w_out, void *workspace,
                             hipStream_t st, const std::function<int(int)> &before, int layer0) {
    const int depth = stack_depth(o), lk = o ? o->lookahead_k : 0;
    size_t bsz, hsz;
    stack_layout(descs, n_layers, depth, lk, &bsz, &hsz);
    uint8_t *base = (uint8_t *)workspace;
    void *blk[2] = {base, base + bsz};
    void *hws[2][MAX_HINTS];
    for (int p = 0; p < 2; p++)
        for (int i = 0; i < depth; i++) hws[p][i] = base + 2 * bsz + ((size_t)p * depth + i) * hsz;
    {
        /* releases on this stream from before: their readers finish before
         * this call's first export, and so before any load it starts */
        std::lock_guard<std::mutex> held(s->mu);
        for (Slot &sl : s->sl)
            if (sl.reads_pending && sl.rel_stream == st) sl.reads_pending = false;
    }
    int rc = TLM_HIP_OK;
    for (int l = 0; l < n_layers && !rc; l++) {
        if (before && (rc = before(l))) break;
        tlm_hip_moe_desc hd[MAX_HINTS];
        const int nh = hint_descs(descs, n_layers, l, depth, lk, hd);
        const tlm_hip_moe_desc *ds[1 + MAX_HINTS];
        void *wss[1 + MAX_HINTS];
        ds[0] = &descs[l];
        wss[0] = blk[l & 1];
        for (int i = 0; i < nh; i++) {
            ds[1 + i] = &hd[i];
            wss[1 + i] = hws[l & 1][i];
        }
        const int area = l % NAREA;
        const uint32_t seq = ++s->route_seq;
        s->route_n[area] = 1 + nh;
        RouteDev rd{};
        rd.tab = s->tab_dev + (size_t)(layer0 + l) * s->tab_E;
        rd.slot_out = s->res_dev + area * 32;
        rd.report = s->rep_dev + area;
        rd.n_slots = s->n_slots;
        rc = launch_moe_routes_host(ds, wss, 1 + nh, h, s->route_dev + area * (ROUTE_AREA / 4), ROUTE_SEQ, seq, st,
                                    &rd);
        const MoeSlots ms{s->res_dev + area * 32, s->arena, s->slot_bytes, {s->uoff[0], s->uoff[1], s->uoff[2]}};
        if (!rc) rc = launch_moe_phase_slots(&descs[l], 2, h, blk[l & 1], &ms, st);
        if (!rc) rc = launch_moe_phase_slots(&descs[l], 3, h, blk[l & 1], &ms, st);
        if (!rc) rc = wait_routes(s, area, seq, st);
        if (rc) break;
        /* the export's routing and whether it kept the layer */
        const uint8_t *ar = s->route_host + (size_t)area * ROUTE_AREA;
        const bool kept = __atomic_load_n(s->rep_host + area, __ATOMIC_ACQUIRE) != 0;
        const int k = descs[l].k;
        int ids[MOE_MAXK];
        float w[MOE_MAXK];
        memcpy(ids, ar, sizeof(int) * k);
        memcpy(w, ar + 128, sizeof(float) * k);
        if (ids_out) memcpy(ids_out + (size_t)l * k, ids, sizeof(int) * k);
        if (w_out) memcpy(w_out + (size_t)l * k, w, sizeof(float) * k);
        update_instinct(o, l, w, k);
        tlm_hip_expert_ref refs[MOE_MAXK];
        if (kept) {
            rc = tlm_hip_store_acquire(s, layer0 + l, ids, k, refs);
        } else {
            rc = run_block(s, &descs[l], layer0 + l, ids, w, h, blk[l & 1], refs, st);
        }
        /* hints while this block's experts hold their references (:988-990) */
        if (!rc) issue_hints(s, o, descs, l, hd, nh, ar, layer0);
        for (int r = 0; r < k; r++) {
            if (l == n_layers - 1 || rc) tlm_hip_store_release(s, &refs[r], st);
            else release_retired(s, &refs[r]);
        }
    }
    if (!rc) tlm_hip_store_tick(s);
    return rc;
}

/* tlm_model_step's loop over moe() with the store (src/lib/tlm_model.c:
 * 1075-1083, 960-1055), lookahead() (:844-877) and the instinct update
 * (:974-980), then tlm_store_tick (:1097); pipelined as described in
 * tlm_hip.h.  before(l), when given, enqueues what precedes layer l's router
 * on the stream (a model's attention); it runs right before that router's
 * launch.  With o->host_routes, or when the slots cannot be resolved on the
 * device, the host resolves each layer's slots: it waits for the layer's
 * routing, acquires, and launches the block with the slots' matrices as
 * arguments, and layer l + 1's attention is queued behind layer l's block. */
int moe_stack_run(const tlm_hip_moe_desc *descs, int n_layers, tlm_hip_store *s, float *h,
                  const tlm_hip_stack_opts *o, int32_t *ids_out, float *w_out, void *workspace, void *stream,
                  const std::function<int(int)> &before, int layer0) {
    if (!descs || n_layers <= 0 || !s || !h || !workspace)
        return tlmh_seterr(TLM_HIP_EINVAL, "moe_stack_store: bad arguments");
    if ((uintptr_t)workspace & 255u)
        return tlmh_seterr(TLM_HIP_EINVAL, "moe_stack_store: workspace must be 256-byte aligned");
    for (int l = 0; l < n_layers; l++)
        if (descs[l].k <= 0 || descs[l].k > MOE_MAXK)
            return tlmh_seterr(TLM_HIP_EINVAL, "moe_stack_store: layer %d (k=%d)", l, descs[l].k);
    if (o && o->lookahead > 0 && o->lookahead_k > MOE_MAXK)
        return tlmh_seterr(TLM_HIP_EINVAL, "moe_stack_store: lookahead_k %d above %d", o->lookahead_k, MOE_MAXK);
    hipStream_t st = (hipStream_t)stream;
    if (!(o && o->host_routes) && dev_resolvable(s, descs, n_layers, layer0))
        return moe_stack_run_dev(descs, n_layers, s, h, o, ids_out, w_out, workspace, st, before, layer0);
    const int depth = stack_depth(o), lk = o ? o->lookahead_k : 0;
    size_t bsz, hsz;
    stack_layout(descs, n_layers, depth, lk, &bsz, &hsz);
    uint8_t *base = (uint8_t *)workspace;
    void *blk[2] = {base, base + bsz};
    void *hws[2][MAX_HINTS];
    for (int p = 0; p < 2; p++)
        for (int i = 0; i < depth; i++) hws[p][i] = base + 2 * bsz + ((size_t)p * depth + i) * hsz;
    tlm_hip_moe_desc hd[MAX_HINTS];
    int nh = 0;
    /* layer l's routes (block + hints for l+1 .. l+depth) into area l mod 2 */
    auto enqueue = [&](int l, uint32_t *seq) {
        if (before) {
            const int rc = before(l);
            if (rc) return rc;
        }
        nh = hint_descs(descs, n_layers, l, depth, lk, hd);
        return enqueue_routes(s, &descs[l], h, blk[l & 1], hd, hws[l & 1], nh, l & 1, seq, st);
    };
    uint32_t seq = 0;
    int rc = enqueue(0, &seq);
    for (int l = 0; l < n_layers && !rc; l++) {
        const int hints_here = nh;   /* the hints routed with this layer */
        tlm_hip_moe_desc hdl[MAX_HINTS];
        for (int i = 0; i < hints_here; i++) hdl[i] = hd[i];
        if ((rc = wait_routes(s, l & 1, seq, st))) break;
        const uint8_t *area = s->route_host + (size_t)(l & 1) * ROUTE_AREA;
        const int k = descs[l].k;
        int ids[MOE_MAXK];
        float w[MOE_MAXK];
        memcpy(ids, area, sizeof(int) * k);
        memcpy(w, area + 128, sizeof(float) * k);
        if (ids_out) memcpy(ids_out + (size_t)l * k, ids, sizeof(int) * k);
        if (w_out) memcpy(w_out + (size_t)l * k, w, sizeof(float) * k);
        update_instinct(o, l, w, k);
        tlm_hip_expert_ref refs[MOE_MAXK];
        rc = run_block(s, &descs[l], layer0 + l, ids, w, h, blk[l & 1], refs, st);
        /* the next layer's routing queued behind this block, before the host's bookkeeping */
        if (!rc && l + 1 < n_layers) rc = enqueue(l + 1, &seq);
        /* hints while this block's experts hold their references (:988-990) */
        if (!rc) issue_hints(s, o, descs, l, hdl, hints_here, area, layer0);
        for (int r = 0; r < k; r++) tlm_hip_store_release(s, &refs[r], stream);
    }
    if (!rc) tlm_hip_store_tick(s);
    return rc;
}

extern "C" {

int tlm_hip_moe_stack_store(const tlm_hip_moe_desc *descs, int n_layers, tlm_hip_store *s, float *h,
                            const tlm_hip_stack_opts *o, int32_t *ids_out, float *w_out, void *workspace,
                            void *stream) {
    if (descs)
        for (int l = 0; l < n_layers; l++)
            if (!descs[l].experts) return tlmh_seterr(TLM_HIP_EINVAL, "moe_stack_store: layer %d has no expert table", l);
    return moe_stack_run(descs, n_layers, s, h, o, ids_out, w_out, workspace, stream, {}, 0);
}

}  // extern "C"
