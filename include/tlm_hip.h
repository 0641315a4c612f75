/* tlm_hip.h - HIP (gfx950 / MI355X) kernel tier for tierlm's quantised-MoE
 * decode path, behind a plain C ABI.
 *
 * Conventions shared with the reference library:
 *   - dtype codes are tlm_dtype values (src/lib/tlm_quant.h:31-42):
 *     F32 0, Q8_0 8, Q4_K 12, Q5_K 13, Q6_K 14, Q8_K 15;
 *   - fallible calls return 0 or a negative TLM_E* code
 *     (src/lib/tlm_platform.h:24-35) and leave a message for
 *     tlm_hip_errmsg(), thread-local like tlm_errmsg();
 *   - numerics follow src/lib/tlm_quant.h:113-128: exact int32 block sums and
 *     one fmaf per block (two for Q4_K/Q5_K) in ascending block order from +0,
 *     so every integer-format result has the bits of the reference's scalar
 *     kernel.
 *
 * Pointers named *_dev, W, act, y, x, h, ids, w, workspace are device
 * pointers (hipMalloc'd or from any allocator of the same device); `stream`
 * is a hipStream_t passed as void* (NULL = the null stream).  Calls enqueue
 * work and return; results are ready after tlm_hip_sync(stream).  No entry
 * point allocates device memory except tlm_hip_malloc, tlm_hip_init (which
 * sizes the staging area behind tlm_kern_hip_fill's host-pointer entries) and
 * tlm_hip_store_open (the slot arena and its staging buffers).
 *
 * Threading: one caller thread per stream.  The host-pointer entries of
 * tlm_kern_hip_fill are serialised internally, so pool workers may call them
 * concurrently.
 */
#ifndef TLM_HIP_H
#define TLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    TLM_HIP_OK = 0, TLM_HIP_EIO = -1, TLM_HIP_ENOMEM = -2, TLM_HIP_EINVAL = -3,
    TLM_HIP_EFORMAT = -4, TLM_HIP_ERANGE = -5, TLM_HIP_ENOTFOUND = -6,
    TLM_HIP_EUNSUP = -7, TLM_HIP_EBUSY = -8
};

/* ---- lifetime / tier ----------------------------------------------------
 * tlm_hip_init replaces tlm_quant_init (src/lib/tlm_quant.c:1069-1088) for the
 * hip tier: it selects `device`, allocates the staging area, and runs the
 * start-up self-test of every HIP kernel against the library's built-in
 * scalar rule on fixed data (src/lib/tlm_quant.c:950-1056).  A kernel that
 * fails is counted and its dtype is refused by the host-pointer tier entries.
 * Idempotent for the same device.  TLM_HIP_EUNSUP when no GPU is present. */
int         tlm_hip_init(int device);
void        tlm_hip_shutdown(void);
/* "hip" after a successful init, else "none" (src/lib/tlm_quant.h:87-88). */
const char *tlm_hip_tier(void);
/* src/lib/tlm_quant.h:131-134 */
int         tlm_hip_selftest_failures(void);
/* src/lib/tlm_platform.h:36 (thread-local message of the last failure) */
const char *tlm_hip_errmsg(void);

/* ---- device memory (the reference's tlm_alloc_aligned,
 *      src/lib/tlm_platform.h:55-56, for device buffers) ------------------ */
int tlm_hip_malloc(void **dptr, size_t bytes);
int tlm_hip_free(void *dptr);
int tlm_hip_memcpy_h2d(void *dst_dev, const void *src_host, size_t bytes, void *stream);
int tlm_hip_memcpy_d2h(void *dst_host, const void *src_dev, size_t bytes, void *stream);
int tlm_hip_sync(void *stream);

/* ---- activations --------------------------------------------------------
 * src/lib/tlm_quant.h:71-74 / src/lib/tlm_quant.c:689-707, on device memory:
 * kind TLM Q8_K (292-byte blocks), Q8_0 (36-byte a8 blocks) or F32 (copy).
 * dst must be 4-byte aligned and tlm_hip_qact_bytes(kind, n) long. */
size_t tlm_hip_qact_bytes(int kind, int64_t n);
int    tlm_hip_quantize_act(int kind, const float *x, int64_t n, void *dst, void *stream);

/* No counterpart in the reference: a plain streaming read of bytes (16-byte
 * aligned) from device memory - the read rate of this device that the GEMVs'
 * HBM figures are set beside.  sink: one device word, written only in the
 * (practically never) event that the folded data equals a fixed constant. */
int    tlm_hip_stream_read(const void *p, size_t bytes, uint32_t *sink, void *stream);

/* ---- the exponential ----------------------------------------------------
 * y[i] = e^(x[i]) on device memory, bit for bit libm's expf as the reference
 * calls it (silu / sigmoidf_, src/lib/tlm_model.c:171-172; the routing softmax
 * :823; the attention softmax :705): the function every softmax, sigmoid and
 * SiLU of this library evaluates, exposed so a caller can check it against
 * its own libm. */
int    tlm_hip_expf(const float *x, float *y, int64_t n, void *stream);

/* ---- matvec on the reference byte layout --------------------------------
 * src/lib/tlm_quant.h:76-85: y[r] = dot(W row r, act) for r in [r0, r1),
 * W row-major with stride row_bytes, any base byte offset.  A bad dtype or n
 * NaN-fills y[r0..r1) on device and returns TLM_HIP_EINVAL. */
int tlm_hip_matvec_rows(int dt, const void *W, size_t row_bytes, const void *act, float *y,
                        int64_t n, int64_t r0, int64_t r1, void *stream);

/* ---- packed (tile) layout for device-resident weights -------------------
 * The packet payload stays in the reference's byte layout on disk and in host
 * RAM (src/lib/tlm_store.h:10-11); after it reaches HBM it is packed once into
 * a tile layout whose every load is a 16-byte aligned vector load.  Packing
 * keeps every byte (no padding beyond the last 16-row tile) and is
 * bit-preserving, so the packed GEMV returns the reference's bits.
 * Q4_K and Q5_K blocks are already 16-byte aligned: their packed layout is the
 * plain layout with tightly packed rows. */
size_t tlm_hip_packed_bytes(int dt, int64_t rows, int64_t n);
int    tlm_hip_pack(int dt, const void *src, size_t row_bytes, int64_t rows, int64_t n,
                    void *dst, void *stream);
/* y[0..rows) for a packed matrix (one launch). */
int    tlm_hip_matvec_packed(int dt, const void *Wp, int64_t rows, int64_t n, const void *act,
                             float *y, void *stream);

/* ---- segment job: several matvecs in one launch --------------------------
 * Mirrors mv_job / mv_exec (src/lib/tlm_model.c:175-222): up to 24 segments of
 * any dtype, width, layout and activation run in one launch (a longer job in
 * one launch per 24); every output row is computed by exactly one work-group,
 * so batching never changes a bit.  An invalid segment (dtype, width,
 * pointers, alignment) has its rows NaN-filled and makes the call return
 * TLM_HIP_EINVAL; the others still run. */
typedef struct {
    int32_t     dt;        /* weight dtype */
    int32_t     packed;    /* 1 = tlm_hip_pack layout, 0 = plain rows (row_bytes) */
    const void *W;
    uint64_t    row_bytes; /* plain layout only */
    const void *act;       /* tlm_hip_quantize_act output of the dtype's kind */
    float      *y;
    int64_t     n, rows;
} tlm_hip_seg;
#define TLM_HIP_MAX_SEGS 136   /* MAX_SEGS, src/lib/tlm_model.c:41-42 */
int tlm_hip_mv_job(const tlm_hip_seg *segs, int nseg, void *stream);

/* ---- many tokens through one packed matrix (prefill) ------------------------
 * The reference's prefill runs the decode step once per token
 * (src/lib/tlm_model.c:1105-1113), i.e. tlm_matvec_rows per token.  This
 * streams a packed matrix once for all ntok tokens (int8 MFMA) and returns,
 * for every token t and row r, exactly the decode result:
 *   Y[t * rows + r] == tlm_hip_matvec_packed(dt, Wp, rows, n, act_t, .)[r]
 * act: ntok activation vectors in the reference layout, consecutive, 4-byte
 * aligned: for Q4_K / Q5_K / Q6_K, Q8_K blocks (n/256 * 292 bytes each;
 * well-formed, i.e. each bsum the sum of its 16 codes, as the quantiser writes
 * them); for Q8_0, a8 blocks (n/32 * 36 bytes each).  n: a multiple of 256. */
int tlm_hip_matmul_tokens(int dt, const void *Wp, int64_t rows, int64_t n, const void *act, int64_t ntok,
                          float *Y, void *stream);

/* ---- one routed MoE block ------------------------------------------------
 * src/lib/tlm_model.c:940-1055 (with run_batch :900-938, route :798-839):
 *   xb = rmsnorm(h, ffn_norm); logits = router xb; (ids, w) = route(logits);
 *   for each rank r: h_r = silu(gate_r xb) * (up_r xb); eo_r = down_r h_r;
 *   ffn = sum_r w_r * eo_r in ascending rank order (+ shared expert);
 *   h += ffn.
 * Every expert is resident (packed) in HBM: experts[3*e + {0,1,2}] point to
 * expert e's packed gate [de x D], up [de x D] and down [D x de].
 * Numerics: router logits, integer block sums, gate/up/down rows, the
 * activation quantisation and the combine order are the reference's; silu /
 * softmax use the device expf and rmsnorm sums squares in double in a tree,
 * so those stages agree with the reference to ~1 ulp. */
typedef struct {
    int64_t D, de, ds;         /* d_model, expert width, shared width (0 = none) */
    int32_t E, k, router;      /* experts, top-k (<= 32), router kind 0/1/2 */
    float   routed_scale, eps;
    int32_t expert_dt, shared_dt;
    const float   *ffn_norm;         /* [D] */
    const float   *router_w;         /* [E x D] f32 rows */
    const float   *router_bias;      /* [E] or NULL */
    const uint8_t *mask;             /* [E] 1 = pruned, or NULL */
    const void *const *experts;      /* device array of 3*E packed matrix pointers */
    const void *sg, *su, *sd;        /* packed shared gate/up [ds x D], down [D x ds] */
    const float   *shared_gate_inp;  /* [D] or NULL */
} tlm_hip_moe_desc;

/* Bytes of caller-owned device workspace one layer call needs. */
size_t tlm_hip_moe_workspace_bytes(const tlm_hip_moe_desc *d);
/* h[D] += MoE(h).  ids[k] / w[k] (device, may be NULL) receive the routing.
 * workspace: tlm_hip_moe_workspace_bytes(d) bytes, 256-byte aligned; calls
 * on different streams need different workspaces. */
int tlm_hip_moe_layer(const tlm_hip_moe_desc *d, float *h, int32_t *ids, float *w,
                      void *workspace, void *stream);
/* No counterpart in the reference: tlm_hip_moe_layer for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The workspace is a static device array of
 * TLM_HIP_MOE_NOALLOC_MAX_BYTES per GPU (the library's, held until the process
 * ends; its address is taken at tlm_hip_init, which must have run on the
 * current device).  Calls no allocator.  Blocks whose
 * tlm_hip_moe_workspace_bytes exceeds the limit get TLM_HIP_ERANGE and no
 * launch.  Every call on one GPU uses that GPU's one array: calls that overlap
 * on one GPU (other streams, other threads) race, so serialise them.  No part
 * of the array needs to start at zero (each call writes what it reads). */
#define TLM_HIP_MOE_NOALLOC_MAX_BYTES (1u << 20)
int tlm_hip_moe_layer_noalloc(const tlm_hip_moe_desc *d, float *h, int32_t *ids, float *w, void *stream);

/* The same block as its launches, one per call, for callers that interleave
 * other work or time each launch (the reference's moe() is likewise route,
 * then the gate/up job, then the down job + combine, src/lib/tlm_model.c:972,
 * 921, 937-1050):
 *   phase 1: rmsnorm + router logits + activation quantisation
 *   phase 2: routing + gate/up + SwiGLU
 *   phase 3: h quantisation + down + rank-order combine + residual update.
 * Phases must run in order on one stream.  Re-running phases 1-2 reproduces
 * the same bits; re-running phase 3 adds the FFN output to h once more. */
int tlm_hip_moe_layer_phase(const tlm_hip_moe_desc *d, int phase, float *h, int32_t *ids, float *w,
                            void *workspace, void *stream);

/* Routing alone: route() of src/lib/tlm_model.c:798-839 after rmsnorm and
 * the router, ids[k] / w[k] (device) exactly as tlm_hip_moe_layer routes the
 * same h.  The expert matrices are not read. */
int tlm_hip_moe_route(const tlm_hip_moe_desc *d, const float *h, int32_t *ids, float *w, void *workspace,
                      void *stream);

/* ---- prefill: T tokens through the routed MoE block ---------------------------
 * src/lib/tlm_model.c:1105-1113 runs the decode step once per token; the MoE
 * block has no cross-token terms, so this gives every token exactly the
 * result of tlm_hip_moe_layer on it: h[t*D .. t*D+D) += MoE(h_t), routing in
 * ids / w [T*k] (either may be NULL).  Tokens are bucketed by expert and each
 * expert's rows stream once per 32 of its tokens (int8 MFMA); a shared expert
 * runs as token matmuls and is added after the routed sum, as the decode
 * block adds it.  Routed Q4_K, Q5_K or Q6_K experts; a shared expert of Q4_K,
 * Q5_K, Q6_K or Q8_0 with D and ds multiples of 256 (others:
 * TLM_HIP_EUNSUP).
 * workspace: tlm_hip_moe_prefill_workspace_bytes bytes, 256-byte aligned. */
size_t tlm_hip_moe_prefill_workspace_bytes(const tlm_hip_moe_desc *d, int64_t T);
int tlm_hip_moe_prefill(const tlm_hip_moe_desc *d, float *h, int64_t T, int32_t *ids, float *w,
                        void *workspace, void *stream);

/* ---- expert slot cache in HBM -------------------------------------------------
 * The reference's routed-expert cache (src/lib/tlm_store.h:24-97; policy
 * src/lib/tlm_store.c:139-740) with its slots in HBM: equal slots allocated
 * once, FREE -> LOADING -> READY, every selection counted, counts halved
 * every 16 ticks, victims by lowest (count, last use) among unreferenced,
 * unpinned READY slots (a FREE slot first), pins by compiler flag / heat /
 * warm count up to pin_frac of the slots, and hints that only take FREE or
 * count-0 slots, bounded in flight so top_k slots stay free for demand.
 * The same calls give the same slots, return codes and counters as the
 * reference.
 *
 * A slot holds one expert's gate, up and down in the tlm_hip_pack layout
 * (the moe block's expert table points into slots); bytes_read counts
 * payload bytes copied into HBM.  Loads run on the store's own stream:
 * payload -> pinned staging (or straight from the payload when it already
 * lies in page-locked memory) -> DMA -> pack.  Each expert's payload is the
 * reference's EXPERT packet payload (gate | up | down at item_off,
 * src/lib/tlm_packet.h:39-54, rows of tlm_row_bytes), read from `payload`
 * (host memory the caller keeps alive until close) or, when NULL, written by
 * the `fetch` callback into staging on the store's loader thread. */
typedef struct tlm_hip_store tlm_hip_store;

typedef struct {
    uint16_t    layer;
    uint16_t    flags;        /* bit0 compiler pin, bit1 pruned (src/lib/tlm_store.c:43-44) */
    uint32_t    id;
    int32_t     dtype;        /* Q8_0, Q4_K, Q5_K or Q6_K */
    float       heat;         /* manifest heat (src/lib/tlm_packet.h:80) */
    uint32_t    seed;         /* warm-sidecar count (src/lib/tlm_store.c:306-340) */
    uint32_t    item_off[3];  /* gate, up, down inside the payload */
    uint64_t    payload_len;
    const void *payload;      /* host bytes, or NULL: use fetch */
} tlm_hip_expert_src;

/* Write expert (layer, id)'s payload_len payload bytes to dst; 0 or TLM_E*.
 * Runs on the store's loader thread. */
typedef int (*tlm_hip_fetch_fn)(void *user, int layer, int id, void *dst, uint64_t len);

typedef struct {
    int64_t          d_model, d_expert;  /* gate / up [d_expert x d_model], down [d_model x d_expert] */
    int32_t          top_k;              /* demand reserve for hints (src/lib/tlm_store.c:406) */
    int32_t          prefetch;           /* accept hints (tlm_store_opts.prefetch) */
    double           pin_frac;           /* tlm_store_opts.pin_frac */
    uint64_t         budget_bytes;       /* HBM for slots, rounded down to whole slots (>= 1) */
    tlm_hip_fetch_fn fetch;
    void            *fetch_user;
} tlm_hip_store_opts;

typedef struct {
    int32_t     slot;      /* >= 0: acquired (release it); -1: not acquired */
    const void *mats[3];   /* device: packed gate, up, down inside the slot */
} tlm_hip_expert_ref;

typedef struct {           /* tlm_store_stats, src/lib/tlm_store.h:66-70 */
    uint64_t hits, misses, prefetch_issued, prefetch_used, prefetch_dropped;
    uint64_t bytes_read, evictions, wait_ns;
    int32_t  slots, pinned, in_use;
} tlm_hip_store_stats;

/* tlm_store_open (src/lib/tlm_store.h:42-46) over n expert sources; pruned
 * sources are left out.  Needs tlm_hip_init. */
int      tlm_hip_store_open(const tlm_hip_expert_src *src, int n, const tlm_hip_store_opts *o,
                            tlm_hip_store **out);
/* Waits for loads in flight; then frees the slots. */
void     tlm_hip_store_close(tlm_hip_store *s);
int      tlm_hip_store_n_slots(const tlm_hip_store *s);
uint64_t tlm_hip_store_slot_bytes(const tlm_hip_store *s);
/* src/lib/tlm_store.h:48-50: pin the hottest experts; loads them synchronously. */
int      tlm_hip_store_warm(tlm_hip_store *s);
/* src/lib/tlm_store.h:52-54, 78-83: every out[i] with slot >= 0 holds a
 * reference (release it whatever the return code); mats are valid device
 * addresses at once, their contents after a wait.  Does not block, except
 * when a miss finds no victim while an unreferenced load is still in flight
 * (a caller that waits on the device runs ahead of its loads): it then waits
 * for that load rather than fail with TLM_HIP_EBUSY. */
int      tlm_hip_store_acquire(tlm_hip_store *s, int layer, const int *ids, int k, tlm_hip_expert_ref *out);
/* src/lib/tlm_store.h:55-56: block the host until READY; 0, or the load's
 * error (TLM_E*, e.g. the fetch callback's). */
int      tlm_hip_store_wait(tlm_hip_store *s, tlm_hip_expert_ref *ref);
/* Device-side wait: work enqueued on `stream` after this call runs after the
 * expert's load; the host blocks only until the load has been queued. */
int      tlm_hip_store_stream_wait(tlm_hip_store *s, const tlm_hip_expert_ref *ref, void *stream);
int      tlm_hip_store_is_ready(tlm_hip_store *s, const tlm_hip_expert_ref *ref);
/* src/lib/tlm_store.h:58-59.  `stream`: where the work reading the slot was
 * enqueued; the slot is not overwritten before that work has finished. */
void     tlm_hip_store_release(tlm_hip_store *s, tlm_hip_expert_ref *ref, void *stream);
/* src/lib/tlm_store.h:60-62, 71-77: advisory hints. */
void     tlm_hip_store_prefetch(tlm_hip_store *s, int layer, const int *ids, int k);
/* src/lib/tlm_store.h:63-64: once per generated token. */
void     tlm_hip_store_tick(tlm_hip_store *s);
/* Block until no load is queued or in flight. */
int      tlm_hip_store_drain(tlm_hip_store *s);
void     tlm_hip_store_get_stats(tlm_hip_store *s, tlm_hip_store_stats *out);

/* One routed MoE block with its experts in the cache: moe() of
 * src/lib/tlm_model.c:960-1055 with tlm_store_acquire, the router lookahead
 * (:844-877, issued at :988-991) and the releases.  Routes on device, reads
 * the routing back (one round trip, shared with the hints, through mapped
 * memory without a stream synchronisation), acquires the k experts, makes
 * `stream` wait for loads still in flight, runs the block (h += MoE(h), as
 * tlm_hip_moe_layer) with the routing and the slots' matrices handed to it
 * at launch (d->experts is not read or written), issues each hint's ids as
 * prefetch hints and releases.  ids_host / w_host (may
 * be NULL) receive the routing.  On an error h is unchanged and every
 * reference is released.  A hint: layer `layer`'s block descriptor with
 * k = the number of experts to hint (lookahead_k, <= 32), and a workspace of
 * its own; at most 7 hints. */
typedef struct {
    const tlm_hip_moe_desc *desc;
    int32_t                 layer;
    void                   *workspace;
} tlm_hip_moe_hint;
int tlm_hip_moe_layer_store(const tlm_hip_moe_desc *d, tlm_hip_store *s, int layer, float *h,
                            int32_t *ids_host, float *w_host, const tlm_hip_moe_hint *hints, int n_hints,
                            void *workspace, void *stream);

/* The routed MoE blocks of a stack of layers for one token through the cache:
 * tlm_model_step's loop over moe() (src/lib/tlm_model.c:1075-1083) with the
 * store (:960-1055), lookahead() for `lookahead` layers ahead with
 * lookahead_k experts routed for each and, when interest > 0, the prefetch
 * breadth weighted as :863-874 (W = interest (1 - I) (1 - H), I the layer's
 * instinct averaged with the current top-1 share, H its heat), the instinct
 * update of :974-980, and one tlm_hip_store_tick at the end (:1097).
 * Pipelined: by default each layer's block is enqueued with its routing and
 * reads the slots its routing export found in the store's expert -> slot
 * table (mapped host memory; an entry is published by its load once the
 * bytes have landed and cleared when its slot is chosen as a victim), while
 * the host replays the layer's acquire, hints and release from the export in
 * the reference's order; a layer whose routed experts have not all landed is
 * handed back by the export and run by the host behind it, as below.
 * Nothing on the device waits on the host.  With host_routes = 1 (or a store
 * whose experts differ in layout) the host waits for each layer's routing
 * through a sequence word the export stores last, acquires and launches the
 * block with the slots' matrices, layer l + 1's routing queued right behind
 * layer l's block.  The store operations and results are the same either
 * way.  descs[l]:
 * layer l's block (its expert table is not used); ids / w (n_layers x top_k,
 * host, may be NULL) receive the routing; workspace: 256-byte aligned,
 * tlm_hip_moe_stack_workspace_bytes bytes.  On an error at layer l the
 * layers before it have updated h and every reference is released. */
typedef struct {
    int32_t      lookahead;      /* layers ahead (0..7), tlm_model_opts.lookahead */
    int32_t      lookahead_k;    /* experts routed for each hint (<= 32; 0 = the layer's top_k) */
    double       interest;       /* tlm_model_opts.interest; 0 = every hint lookahead_k wide */
    const float *layer_heat;     /* per layer, or NULL (0) */
    double      *instinct;       /* per layer, the caller's state (tlm_model's instinct), or NULL */
    uint32_t    *instinct_seen;  /* per layer, or NULL */
    int32_t      host_routes;    /* 1: the host resolves each layer's slots (see above); 0: the device */
} tlm_hip_stack_opts;
size_t tlm_hip_moe_stack_workspace_bytes(const tlm_hip_moe_desc *descs, int n_layers, const tlm_hip_stack_opts *o);
int    tlm_hip_moe_stack_store(const tlm_hip_moe_desc *descs, int n_layers, tlm_hip_store *s, float *h,
                               const tlm_hip_stack_opts *o, int32_t *ids, float *w, void *workspace, void *stream);

/* ---- compiled model stores: manifest + packet files -----------------------
 * Reader of the reference's store format (src/lib/tlm_packet.h:8-151,
 * src/lib/tlm_packet.c:8-34): tlm_manifest_load's checks (one valid layout,
 * header CRC32C, packet-table SHA-256, record ranges, order, no overlapping
 * extents), tlm_packet_read's header / length / CRC checks with the replica
 * fallback, and tensor-directory lookup. */
enum { TLM_HIP_PK_DENSE = 1, TLM_HIP_PK_EXPERT = 2, TLM_HIP_PK_BUNDLE = 3, TLM_HIP_PK_MTP = 4,
       TLM_HIP_PK_EMBED = 5, TLM_HIP_PK_TABLE = 6, TLM_HIP_PK_META = 7, TLM_HIP_PK_TOKEN = 8 };
#define TLM_HIP_LAYER_NONE 0xFFFFu

typedef struct {            /* tlm_packet_loc, src/lib/tlm_packet.h:70-81 */
    uint16_t type, layer;
    uint32_t id;
    uint8_t  drive, replica_drive;   /* 0xFF = no replica */
    uint16_t flags;                  /* bit0 pinned at load, bit1 pruned */
    uint64_t offset, replica_offset, total_len;
    uint32_t crc32c;
    float    heat;
} tlm_hip_packet_loc;

typedef struct {            /* tlm_model_geom, src/lib/tlm_packet.h:84-95 */
    char     arch[32];
    uint32_t n_layers, d_model, n_heads, n_kv_heads, head_dim;
    uint32_t vocab, n_experts, top_k, d_expert, n_shared, d_shared;
    uint32_t max_ctx, router;
    float    rope_theta, norm_eps, routed_scale;
    uint32_t mtp_layers, rope_scale;
    float    rope_factor, rope_beta_fast, rope_beta_slow;
    uint32_t rope_orig_len;
} tlm_hip_model_geom;

typedef struct {            /* tlm_tensor_ref, src/lib/tlm_packet.h:59-66 */
    char     name[48];
    uint32_t dtype, ndim;
    uint64_t shape[2], offset, nbytes;
} tlm_hip_tensor_ref;

typedef struct tlm_hip_manifest tlm_hip_manifest;
/* src/lib/tlm_packet.h:127 (tlm_manifest_load) */
int  tlm_hip_manifest_load(const char *path, tlm_hip_manifest **out);
void tlm_hip_manifest_free(tlm_hip_manifest *m);
const tlm_hip_model_geom *tlm_hip_manifest_geom(const tlm_hip_manifest *m);
const char *tlm_hip_manifest_name(const tlm_hip_manifest *m);
int  tlm_hip_manifest_n_packets(const tlm_hip_manifest *m);
const tlm_hip_packet_loc *tlm_hip_manifest_packet(const tlm_hip_manifest *m, int i);
/* src/lib/tlm_packet.h:129-130 (tlm_manifest_find): binary search */
const tlm_hip_packet_loc *tlm_hip_manifest_find(const tlm_hip_manifest *m, int type, int layer, uint32_t id);
/* src/lib/tlm_packet.h:132: <drive dir>/<name>.tlmp */
const char *tlm_hip_manifest_drive_path(const tlm_hip_manifest *m, int i);
/* src/lib/tlm_packet.h:164-165 (tlm_packet_read): buf holds loc->total_len
 * bytes; the payload is at buf + *payload_off, *payload_len bytes. */
int  tlm_hip_packet_read(tlm_hip_manifest *m, const tlm_hip_packet_loc *loc, void *buf, uint64_t *payload_off,
                         uint64_t *payload_len);
/* dtype and gate / up / down item offsets of a packet header (tlm_packet_hdr) */
int  tlm_hip_packet_header(const void *buf, uint32_t *dtype, uint32_t item_off[3]);
/* src/lib/tlm_packet.h:141 (tlm_dir_find): TLM_HIP_ENOTFOUND if absent */
int  tlm_hip_dir_find(const void *payload, uint64_t len, const char *name, tlm_hip_tensor_ref *out);
/* the format's checksums: CRC32C (src/lib/tlm_platform.h crc32c), SHA-256 */
uint32_t tlm_hip_crc32c(uint32_t crc, const void *p, size_t n);
void     tlm_hip_sha256(const void *p, size_t n, uint8_t out[32]);

/* ---- the whole decode step on the device -----------------------------------
 * tlm_model_open / tlm_model_step / tlm_model_prefill and tierlm bench's
 * greedy loop (src/lib/tlm_model.h:60-125, src/lib/tlm_model.c:486-600,
 * 1058-1113, src/bin/tierlm.c:702-729) for a compiled store: the model is
 * loaded into HBM (every weight packed, every expert resident, an f32 KV cache
 * of max_ctx positions) and each step runs embedding, attention (rmsnorm,
 * q/k/v, qk-norm, RoPE / YaRN, KV append, softmax attention, o, residual),
 * the MoE block, the final norm, lm_head and the greedy argmax on one stream.
 * Dense-FFN layers, MTP heads and head_dim above 256 are not supported
 * (TLM_HIP_EUNSUP).  Needs tlm_hip_init. */
typedef struct tlm_hip_model tlm_hip_model;
typedef struct {
    int32_t max_ctx;     /* KV positions; 0 = the store's max_ctx, else 4096 (tlm_kv_new) */
    int32_t eager;       /* 1: launch each step's kernels directly; 0: replay the step as a HIP graph
                            captured at first use (the position and tokens live in device memory) */
    int32_t attn_slices; /* attention slices per key head; 0 = automatic (enough groups to cover the
                            chip at long contexts) */
    int32_t attn_split;  /* 0: attn_heads' order of operations (src/lib/tlm_model.c:683-719), the
                            reference's bits: one serial P.V chain per output element;
                            1: split attention - softmax and P.V partials per slice of positions,
                            merged per query head: each attention output within float rounding of
                            the reference's, but not its bits, and the int8 activation codes and
                            top-k routing downstream turn such differences into larger ones */
    /* The experts through the HBM slot cache (tlm_hip_store) instead of all
     * resident, as tierlm's runtime opens its store (src/bin/tierlm.c:
     * 286-309: tlm_store_open, tlm_store_warm, tlm_model_open with the
     * lookahead): each expert's packet payload stays in page-locked host
     * memory, the step routes each layer on the device, the host acquires the
     * experts (and hints the next layers') while the device runs on, and the
     * block reads the slots (tlm_model.c:960-1055 through
     * tlm_hip_moe_stack_store's loop with the attention queued before each
     * router).  Such a step is not captured as a graph. */
    uint64_t expert_cache_bytes; /* 0: every expert resident; else the slot budget (at least top_k slots) */
    double   pin_frac;           /* memory.pin_frac: 0 = the reference's default 0.30, < 0 = none; capped so
                                    pins leave top_k slots (src/bin/tierlm.c:288-294) */
    int32_t  prefetch_off;       /* io.prefetch off: no hints, no lookahead (default: lookahead 1) */
    int32_t  lookahead_k;        /* io.lookahead_k: experts hinted per lookahead layer (0 = top_k) */
    double   interest;           /* nav.interest_aggressiveness (0 = fixed breadth) */
    /* Prompts (tlm_hip_model_prefill / _generate): 0 = batched where the
     * model allows it - every resident layer's q/k/v/o Q4_K / Q5_K / Q6_K /
     * Q8_0 with widths multiples of 256, routed Q4_K / Q5_K / Q6_K experts
     * (a shared expert of those dtypes or Q8_0, width a multiple of 256), head
     * width 32 / 64 / 96 / 128, the reference's
     * attention order (attn_split 0) - in chunks sized to the context
     * capacity (at most 1024 tokens); n > 0: chunks of at most n tokens (also
     * bounded by 256 MB of score rows at the context capacity); < 0:
     * one step per token.  A batched chunk runs each layer once for all of
     * its tokens (int8 MFMA token matmuls, the batched MoE block, causal
     * attention over the cache) with each token's result bit for bit the
     * step's. */
    int32_t  prefill_chunk;
    /* 1: every step and prefill chunk stamps the device clock where a layer's
     * attention and its MoE block begin and where the step begins and ends (a
     * one-thread launch each, about 1.5 us, so 2 n_layers + 3 more launches per
     * step), and accumulates the attention / MoE / other split that
     * tlm_model_get_stats reports (src/lib/tlm_model.h:86-90, filled at
     * src/lib/tlm_model.c:1099-1101); 0: no stamps */
    int32_t  stats;
    /* With expert_cache_bytes: 1 = the host resolves each layer's slots
     * between its routing and its block (tlm_hip_stack_opts.host_routes);
     * 0 = the routing export resolves them from the store's table and the
     * block is already queued, the host replaying the store operations
     * behind it (a layer with an expert not yet landed runs as with 1) */
    int32_t  host_routes;
} tlm_hip_model_opts;
int  tlm_hip_model_open(const char *manifest_path, const tlm_hip_model_opts *o, tlm_hip_model **out);
void tlm_hip_model_close(tlm_hip_model *M);
const tlm_hip_model_geom *tlm_hip_model_geom_of(const tlm_hip_model *M);
int  tlm_hip_model_kv_len(const tlm_hip_model *M);
int  tlm_hip_model_kv_capacity(const tlm_hip_model *M);
/* The routing of the last step: per MoE layer, the top_k expert ids and
 * weights in rank order (ids and w each n_layers x top_k, host memory) - what
 * the reference's routing hook receives once per layer per token
 * (tlm_model_set_route_hook, src/lib/tlm_model.h:63-70, called at
 * src/lib/tlm_model.c:1053).  Waits for the step. */
int  tlm_hip_model_routes(tlm_hip_model *M, int32_t *ids, float *w);
void tlm_hip_model_reset(tlm_hip_model *M);   /* tlm_kv_reset */
/* A random-init model of geometry g built directly in HBM, for measuring the
 * decode step at shapes whose compiled stores are too large to write or ship
 * (the role `tlmc synth` + `tlmc compile` play for the reference,
 * src/bin/tlmc.c:270-330): block bytes from a counter-based hash of seed with
 * finite scale fields, weights of about the spread of N(0, 0.02); norms 1;
 * router f32 of variance 1/d_model; embedding and lm_head as dense_dt / Q8_0.
 * Its outputs are not the reference synthesiser's: parity is established on
 * compiled stores (tlm_hip_model_open).  Needs tlm_hip_init. */
typedef struct {
    int32_t  expert_dt, dense_dt;   /* Q4_K, Q5_K, Q6_K or Q8_0 (dtype codes above) */
    int32_t  qk_norm;               /* 1: q_norm / k_norm present */
    int32_t  expert_pool;           /* with expert_cache_bytes: distinct expert payloads kept in host memory,
                                       expert (l, e) using payload (l E + e) mod pool (0 = one each) */
    uint64_t seed;
    double   heat_gamma;            /* > 0 with sigmoid routing: router bias -heat_gamma ln(r + 1) for the
                                       expert of rank r in a seeded per-layer permutation (a Zipf-like heat) */
} tlm_hip_model_synth_opts;
int  tlm_hip_model_synth(const tlm_hip_model_geom *g, const tlm_hip_model_synth_opts *so,
                         const tlm_hip_model_opts *o, tlm_hip_model **out);
/* tlm_model_step: logits (host, vocab floats) and next (the greedy token)
 * may each be NULL. */
int  tlm_hip_model_step(tlm_hip_model *M, int token, float *logits, int32_t *next);
/* tlm_model_prefill (src/lib/tlm_model.c:1105-1113): the n tokens from the
 * current position, logits (host, vocab floats, may be NULL) of the last;
 * the same bits as n steps (batched as tlm_hip_model_opts.prefill_chunk
 * says).  Waits for the work. */
int  tlm_hip_model_prefill(tlm_hip_model *M, const int32_t *tokens, int n, float *logits);
/* 1 when prompts run batched on this model (prefill_chunk and the model's
 * dtypes and geometry allow it), 0 when they run one step per token */
int  tlm_hip_model_prefill_batched(const tlm_hip_model *M);
/* prefill the prompt (as tlm_hip_model_prefill), then n_gen greedy tokens
 * into out; between steps the token stays on the device. */
int  tlm_hip_model_generate(tlm_hip_model *M, const int32_t *prompt, int n_prompt, int n_gen, int32_t *out);
/* No counterpart in the reference (whose KV cache only resets): keep the
 * first len positions of the context (0 <= len <= kv_len) and drop the rest,
 * as after rejected speculative tokens; the next step decodes position len
 * with the token a previous step stored there.  Enqueued on the model's
 * stream, no wait. */
int  tlm_hip_model_rewind(tlm_hip_model *M, int len);
/* n greedy steps from the current position, each on the token the previous
 * step chose (the loop of tierlm bench / generate after its prefill, src/bin/
 * tierlm.c:720-729), enqueued without waiting; tlm_hip_model_sync waits.  The
 * context must hold at least one position. */
int  tlm_hip_model_decode(tlm_hip_model *M, int n);
int  tlm_hip_model_sync(tlm_hip_model *M);
/* the model's stream (hipStream_t), for callers that time or order work
 * against its steps */
void *tlm_hip_model_stream(const tlm_hip_model *M);
/* tlm_model_stats (src/lib/tlm_model.h:86-90) of the device steps since the
 * model opened or the last reset: tokens = positions run; attn_ns / moe_ns =
 * device time from the start of each layer's attention (its q|k|v launch) to
 * the start of its MoE block (the router), and from there to the next layer's
 * attention or the step's tail; other_ns = the embedding and the tail (final
 * norm, lm_head, argmax); expert_wait_ns = host time blocked on expert loads
 * in the slot cache (tlm_hip_store_stats.wait_ns).  The split needs
 * tlm_hip_model_opts.stats; without it tokens and expert_wait_ns alone are
 * counted.  Waits for the model's work. */
typedef struct {
    uint64_t tokens, attn_ns, moe_ns, expert_wait_ns, other_ns;
} tlm_hip_model_stats;
int  tlm_hip_model_get_stats(tlm_hip_model *M, tlm_hip_model_stats *out);
void tlm_hip_model_reset_stats(tlm_hip_model *M);   /* tlm_model_reset_stats (src/lib/tlm_model.c:643) */
/* the model's expert slot cache (expert_cache_bytes > 0), for its counters
 * (tlm_hip_store_get_stats) as tierlm's stats print them (src/bin/tierlm.c:
 * 441-460); NULL when every expert is resident */
tlm_hip_store *tlm_hip_model_expert_store(const tlm_hip_model *M);

/* ---- reference tier ABI --------------------------------------------------
 * Layout-compatible with tlm_quant_kernels (src/lib/tlm_quant.h:152-166, a
 * name and two tables of TLM_QK_COUNT = 10 function pointers indexed F32,
 * F16, BF16, Q8_0, Q4_K, Q5_K, Q6_K, MXFP4, FP8, Q8_K).  tlm_kern_hip_fill
 * overwrites the F32, Q8_0, Q4_K, Q5_K, Q6_K and Q8_K entries with
 * host-pointer kernels that stage through device memory and returns how many
 * entries it filled; 0 when tlm_hip_init has not succeeded.  This is the
 * correctness / self-test path; the device-resident calls above are the fast
 * path. */
typedef float (*tlm_hip_qdot_fn)(const void *wrow, const void *act, int64_t n, const float *aux);
typedef void  (*tlm_hip_qmv_fn)(const void *W, size_t row_bytes, const void *act, float *y,
                                int64_t n, int64_t nrows);
typedef struct {
    const char     *name;
    tlm_hip_qdot_fn dot[10];
    tlm_hip_qmv_fn  mv[10];
} tlm_hip_quant_kernels;
int tlm_kern_hip_fill(tlm_hip_quant_kernels *k);

#ifdef __cplusplus
}
#endif
#endif
