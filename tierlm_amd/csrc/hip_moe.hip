/* hip_moe.hip - one routed MoE block on device in three launches
 * (src/lib/tlm_model.c:940-1055, run_batch :900-938, route :798-839).
 *
 *   K1 moe_router   one wave per work-group, two router rows each.  Every
 *                   group recomputes xb = rmsnorm(h) (same tree, same bits),
 *                   then its rows in the reference's f32 lane order; group b
 *                   also quantises activation block b of xb for the experts
 *                   (and the shared expert) and group 0 publishes xb and the
 *                   shared sigmoid gate.
 *   K2 moe_gateup   one group per (rank, 16-row tile) of gate and up, then the
 *                   shared expert's tiles.  Every group routes (softmax, top-k
 *                   by rank counting, renormalise) from the logits itself -
 *                   the same bits in every group - so no group waits on
 *                   another; each wave then puts all its weight loads in
 *                   flight, copies the activation into its own LDS while they
 *                   land, computes, and the group writes h = silu(g) * u for
 *                   its 16 rows.
 *   K3 moe_down     one group per 8 rows of D: quantises every rank's h (the
 *                   reference's activation rule) into LDS while its down-row
 *                   loads are in flight, computes, and adds
 *                   sum_r w_r * out_r (+ gate * shared) to h in rank order.
 * No launch hands data between its own work-groups, so no cross-XCD cache
 * maintenance is needed inside a kernel.  The kernels are instantiated per
 * (expert dtype, shared dtype) so each holds one or two item paths only.
 * Integer sums, per-row fma chains, activation quantisation and the combine
 * order are the reference's; e^x (double exp rounded to float) and rmsnorm's
 * double sum of squares (a tree) are the device's. */
#include "tlm_hip_internal.h"
#include <type_traits>
#include "tlm_hip_act.h"
#include "tlm_hip_items.h"
#include "tlm_hip_mfma.h"

#include <math.h>

namespace {

constexpr int MAXK = 32;          /* top-k bound of this implementation */
constexpr int MAXE = 256;         /* expert-count bound (4 per lane of one wave) */
constexpr int NWAVE = 4;          /* waves per group in K2 */
constexpr int PARK_MAX = 512;     /* parked items per matrix chunk in K2 */
constexpr int NONE = -1;          /* "no shared expert" instantiation */

__host__ __device__ constexpr int bvals(int kind) { return kind == DT_Q8_K ? 256 : 32; }

/* ---- workspace layout (256-byte aligned regions), computed on the host and
 * passed to every kernel --------------------------------------------------- */
struct WsLayout {
    size_t xb, xe, xs, logits, route, hh, total;
};

__host__ __device__ inline size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

inline WsLayout ws_layout(const tlm_hip_moe_desc &d) {
    WsLayout L;
    const int ek = dt_act_kind(d.expert_dt), sk = d.ds > 0 ? dt_act_kind(d.shared_dt) : DT_Q8_K;
    size_t o = 0;
    L.xb = o;     o += al256((size_t)d.D * 4);
    /* activations of xb in the split (LDS) layout, whole blocks */
    L.xe = o;     o += al256(stage_bytes(ek, (int)((d.D + bvals(ek) - 1) / bvals(ek))));
    L.xs = o;     o += al256(stage_bytes(sk, (int)((d.D + bvals(sk) - 1) / bvals(sk))));
    L.logits = o; o += al256((size_t)d.E * 4);
    L.route = o;  o += 512;                        /* ids int32[32] at +0, w f32[32] at +128, sgate at +256 */
    L.hh = o;     o += al256((size_t)(d.k * d.de + d.ds) * 4);
    L.total = o;
    return L;
}

__device__ __forceinline__ int32_t *ws_ids(uint8_t *ws, const WsLayout &L) { return (int32_t *)(ws + L.route); }
__device__ __forceinline__ float *ws_w(uint8_t *ws, const WsLayout &L) { return (float *)(ws + L.route + 128); }
__device__ __forceinline__ float *ws_sgate(uint8_t *ws, const WsLayout &L) { return (float *)(ws + L.route + 256); }

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* Kernel arguments are read through the scalar cache, and the compiler
 * fetches each field where it is first used: every such batch is a full
 * round trip before the next dependent load can go out.  Naming the fields a
 * kernel needs at its entry makes it fetch them all at once, with one wait. */
template <class T> __device__ __forceinline__ void arg_now(T v) { asm volatile("" ::"s"(v)); }
template <class... T> __device__ __forceinline__ void args_now(T... v) { (arg_now(v), ...); }

/* ---- activation rule (src/lib/tlm_quant.c:458-478) for this lane's 4 values
 * of a block spread over WIDTH lanes: d, and the 4 codes packed in a dword --- */
template <int WIDTH>
__device__ __forceinline__ float act_rule4(f32x4 v, bool ok, uint32_t &codes) {
    /* |v| as bits: for non-negative floats the unsigned order is the float
     * order; above 0x7F800000 is NaN, equal is infinity */
    uint32_t am = 0, fl = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t b = ok ? (__float_as_uint(v[j]) & 0x7FFFFFFFu) : 0u;
        fl |= (b > 0x7F800000u ? 1u : 0u) | (b == 0x7F800000u ? 2u : 0u);
        const uint32_t f = b < 0x7F800000u ? b : 0u;
        am = f > am ? f : am;
    }
    am = group_max_u32<WIDTH>(am);
    fl = group_or_u32<WIDTH>(fl);
    const float amax = __uint_as_float(am);
    codes = 0;
    if (fl) return (fl & 1u) ? __uint_as_float(0x7FC00000u) : INFINITY;
    if (!(amax > 0.0f) || !ok) return amax > 0.0f ? amax / 127.0f : 0.0f;
    const float d = amax / 127.0f;
    if (amax >= 0x1p-100f) {
        const float id = 127.0f / amax;
#pragma unroll
        for (int j = 0; j < 4; j++) codes |= (uint32_t)(uint8_t)(int8_t)rne_clamp(v[j] * id, -127, 127) << (8 * j);
    } else {
        const double id = 127.0 / (double)amax;
#pragma unroll
        for (int j = 0; j < 4; j++)
            codes |= (uint32_t)(uint8_t)(int8_t)rne_clamp((float)((double)v[j] * id), -127, 127) << (8 * j);
    }
    return d;
}

/* Quantise one block (values v of this lane, `ok` = lane inside the block)
 * into the split layout at (q, bs, d) of block index b: Q8_K uses all 64
 * lanes, a8 the 8 lanes of a group. */
template <class QP, class BP, class DP>
__device__ __forceinline__ void quant_block_to(int kind, f32x4 v, bool ok, int sub, QP q, BP bs, DP dd, int b) {
    uint32_t codes;
    if (kind == DT_Q8_K) {
        const float d = act_rule4<64>(v, ok, codes);
        q[b * 64 + sub] = codes;
        int s = byte_sum(codes);
        s += (int)dpp_u32<DPP_XOR1>((uint32_t)s);
        s += (int)dpp_u32<DPP_XOR2>((uint32_t)s);
        if ((sub & 3) == 0) bs[b * 16 + (sub >> 2)] = (int16_t)s;
        if (sub == 0) dd[b] = d;
    } else {
        const float d = act_rule4<8>(v, ok, codes);
        if (ok) {
            q[b * 8 + sub] = codes;
            if (sub == 0) dd[b] = d;
        }
    }
}

/* ---- routing by the group (src/lib/tlm_model.c:776-839) --------------------
 * 256 threads; thread t owns expert t.  Every valid entry (unmasked, selection
 * value not NaN) gets a 64-bit key: the order-preserving bits of its value,
 * then ~index.  Keys are distinct and "larger key" is exactly the reference's
 * "larger value, ties to the lower index", so an entry's rank (the number of
 * larger keys) is its position in the reference's top-k; ranks 0..k-1 are
 * written directly.  With fewer than k valid entries the reference's fallback
 * (lowest unmasked unused index, else 0) fills the remaining ranks. */
struct __align__(16) RouteLds {
    unsigned long long key[MAXE];   /* entries t >= E hold 0 (never larger) */
    float p[MAXE];
    int cnt[MAXE];
    double red[NWAVE];
    float redf[NWAVE];
    int redi[NWAVE];
    int ids[MAXK];
    float w[MAXK];
};

__device__ __forceinline__ uint32_t ord_bits(float f) {
    const uint32_t b = __float_as_uint(f + 0.0f);   /* -0 -> +0: equal values, equal keys */
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

/* ids land in R->ids[0..k) and, with weights, the renormalised weights in
 * R->w[0..k), readable by every thread (without weights R->w holds the
 * unnormalised probabilities).  stash() runs in every thread before a group
 * barrier, once the softmax is done: a place for LDS writes of values loaded
 * at kernel entry. */
struct NoHook {
    __device__ void operator()() const {}
};
template <class Stash, class Issued = NoHook>
__device__ void route_group(const tlm_hip_moe_desc &d, const GAS float *logits, LAS RouteLds *R, Stash stash,
                            const ExpTabLanes &tab, bool weights = true, Issued issued = NoHook{}) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, E = d.E, k = d.k;
    const bool sig = d.router == 2;
    const bool in = t < E;
    const bool unmasked = in && !(d.mask && ((const GAS uint8_t *)d.mask)[t]);
    const float l = in ? logits[t] : 0.0f;
    const float bias = (sig && in && d.router_bias) ? ((const GAS float *)d.router_bias)[t] : 0.0f;
    issued();   /* loads the caller issues here queue behind the routing's own */
    float p;
    if (sig) {   /* sigmoid score = weight; bias for selection only */
        p = 1.0f / (1.0f + expf_ref_with(-l, tab));
    } else {     /* softmax over the routable experts */
        float m = wave_max_f32((unmasked && l > -INFINITY) ? l : -INFINITY);
        if (lane == 0) R->redf[wave] = m;
        __syncthreads();
        float mx = R->redf[0];
#pragma unroll
        for (int q = 1; q < NWAVE; q++) mx = R->redf[q] > mx ? R->redf[q] : mx;
        const bool off = !unmasked || l != l || mx == -INFINITY;
        const float ex = expf_ref_with(l - mx, tab);   /* every lane: the table lives in the lanes */
        const float x = off ? 0.0f : ex;
        const double s = wave_sum_f64((double)x);
        if (lane == 0) R->red[wave] = s;
        __syncthreads();
        const double st = (R->red[0] + R->red[1]) + (R->red[2] + R->red[3]);
        const float inv = st > 0.0 ? (float)(1.0 / st) : 0.0f;
        p = x * inv;
    }
    const float sel = sig ? p + bias : p;
    const bool valid = unmasked && sel == sel;
    const unsigned long long key =
        valid ? ((unsigned long long)ord_bits(sel) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)t) : 0ull;
    R->key[t] = key;
    R->p[t] = p;
    stash();
    const int nv_wave = __builtin_popcountll(__ballot(valid));   /* whole wave active here */
    if (lane == 0) R->redi[wave] = nv_wave;
    __syncthreads();
    const int nvalid = (R->redi[0] + R->redi[1]) + (R->redi[2] + R->redi[3]);
    /* rank = #larger keys; with E <= 128 two threads split the scan of one
     * entry, each over a fixed 64 entries (two keys per 16-byte read; the
     * zero keys past E never count) */
    const bool split = E <= 128;
    const int e = split ? (t & 127) : t;
    const unsigned long long ke = e < E ? R->key[e] : 0ull;
    int c = 0;
    if (ke != 0ull) {
        if (split) {
            const LAS u32x4 *kp = (const LAS u32x4 *)(R->key + (t >= 128 ? 64 : 0));
            int cc[4] = {0, 0, 0, 0};   /* independent counts: no chain through one register */
#pragma unroll
            for (int j = 0; j < 32; j++) {
                const u32x4 w = kp[j];
                const unsigned long long a = ((unsigned long long)w.y << 32) | w.x;
                const unsigned long long b = ((unsigned long long)w.w << 32) | w.z;
                cc[(2 * j) & 3] += a > ke ? 1 : 0;
                cc[(2 * j + 1) & 3] += b > ke ? 1 : 0;
            }
            c = (cc[0] + cc[1]) + (cc[2] + cc[3]);
        } else {
#pragma unroll 16
            for (int f = 0; f < E; f++) c += R->key[f] > ke ? 1 : 0;
        }
    }
    R->cnt[t] = c;
    __syncthreads();
    if (in && key != 0ull) {
        const int rank = split ? R->cnt[t] + R->cnt[t + 128] : c;
        if (rank < k) { R->ids[rank] = t; R->w[rank] = p; }
    }
    __syncthreads();
    if (nvalid < k || weights) {   /* uniform over the group */
      if (wave == 0) {
        if (nvalid < k) {
            if (lane == 0)
                for (int r = nvalid; r < k; r++) {
                    int pick = -1;
                    for (int f = 0; f < E && pick < 0; f++) {
                        if (d.mask && d.mask[f]) continue;
                        bool used = false;
                        for (int q = 0; q < r; q++) used = used || R->ids[q] == f;
                        if (!used) pick = f;
                    }
                    pick = pick < 0 ? 0 : pick;
                    R->ids[r] = pick;
                    R->w[r] = R->p[pick];
                }
            wave_sync();
        }
        if (weights) {   /* renormalise in rank order (double sum), then scale */
            float wr = lane < k ? R->w[lane] : 0.0f;
            if (d.router != 1) {
                double s = 0.0;
                for (int r = 0; r < k; r++) s += (double)rdlane_f32(wr, r);
                if (sig || s > 0.0) wr *= (float)(1.0 / (sig ? s + 1e-20 : s));
            }
            if (sig || d.routed_scale != 1.0f) wr *= d.routed_scale;
            if (lane < k) R->w[lane] = wr;
        }
      }
      __syncthreads();
    }
}

/* ======================================================================
 * K1: rmsnorm + router + activation quantisation (one wave per group)
 * ==================================================================== */
constexpr int RCH = 16;            /* router values per lane per pipelined chunk */
constexpr int RCHV = 32 * RCH;     /* values of one row per chunk */

/* Chunk at c0 of a router row: lane hl takes elements c0 + hl + 32j.  D is a
 * multiple of 32, so a chunk is either full or, as the row's last, holds
 * whole 32-value groups; TAIL loads clamp into the row and fma_chunk skips
 * the groups past D. */
template <bool TAIL>
__device__ __forceinline__ void load_chunk(float (&v)[RCH], const GAS float *wr, int64_t c0, int hl, int64_t D) {
    const GAS float *p = wr + c0 + hl;
#pragma unroll
    for (int j = 0; j < RCH; j++) v[j] = (!TAIL || c0 + 32 * j < D) ? p[32 * j] : 0.0f;
}

template <bool TAIL>
__device__ __forceinline__ float fma_chunk(const float (&v)[RCH], const LAS float *xb, int64_t c0, int hl,
                                           int64_t D, float r) {
    const LAS float *x = xb + c0 + hl;
#pragma unroll
    for (int j = 0; j < RCH; j++)
        if (!TAIL || c0 + 32 * j < D) r = fmaf(v[j], x[32 * j], r);
    return r;
}

/* The 32 lane partials of a router dot (lanes 0-31 and 32-63 separately):
 * lane 0 of each half ends with ((r0 + r16) + (r8 + r24)) + ...: the
 * reference's pairing (i, i+16), (i, i+8), (i, i+4), (i, i+2), (i, i+1)
 * (src/lib/tlm_quant.c:724-738); row_shl:n hands lane i the value of lane i+n */
__device__ __forceinline__ float reduce32(float r) {
    float s = r + __shfl_xor(r, 16, 64);
    s = s + dpp_f32<0x108>(s);
    s = s + dpp_f32<0x104>(s);
    s = s + dpp_f32<DPP_XOR2>(s);
    return s + dpp_f32<DPP_XOR1>(s);
}

/* blockIdx.y = token: its residual at hptr + y * D, its workspace at
 * ws + y * tstride (the decode launches have one token). */
/* NPRE chunks of each router row in flight from the start (4 for rows of up
 * to 2048 values, 8 for wider ones, so a 4096-wide row needs no second round
 * trip for its weights) */
template <int NPRE>
__device__ __forceinline__ void router_body(const tlm_hip_moe_desc &d, const WsLayout &L, const float *__restrict__ hptr,
                                            uint8_t *ws, const int blk) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x, hl = lane & 31;
    const int64_t D = d.D;
    const int64_t row = (int64_t)blk * 2 + (lane >> 5);
    const bool live = row < d.E;
    const GAS float *wr = (const GAS float *)d.router_w + (live ? row : 0) * D;
    const GAS f32x4 *h4 = (const GAS f32x4 *)hptr, *n4 = (const GAS f32x4 *)d.ffn_norm;
    const int64_t nfull = D / RCHV, ctail = nfull * RCHV;

    /* rmsnorm (src/lib/tlm_model.c:164-169): sum of squares in double, lane
     * then wave tree; x and the norm weights parked in LDS (16-byte copies) */
    LAS f32x4 *xb4 = (LAS f32x4 *)lds;
    LAS f32x4 *xw4 = xb4 + D / 4;
    constexpr int NV = 8;   /* 16-byte loads of h and of the weights per lane per batch */
    const int D4 = (int)(D / 4);
    const bool one = D4 <= 64 * NV;   /* D <= 2048: h and the norm weights in one batch */
    /* one batch: h and the norm weights go out first (loads retire in issue
     * order, so the norm then waits for them alone), branch-free (lanes past
     * the row read its last vector), then the router rows */
    f32x4 hv[NV], nv[NV];
    if (one) {
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const int cc = min(lane + 64 * j, D4 - 1);
            hv[j] = h4[cc];
            nv[j] = n4[cc];
        }
    }
    /* the first NPRE full chunks and the partial last chunk in flight
     * during the norm */
    float v[NPRE][RCH], vt[RCH];
#pragma unroll
    for (int c = 0; c < NPRE; c++)
        if (nfull > c) load_chunk<false>(v[c], wr, c * RCHV, hl, D);
    if (ctail < D) load_chunk<true>(vt, wr, ctail, hl, D);

    if (one) {
        /* normalise in registers, write x once */
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < NV; j++)
            if (lane + 64 * j < D4) {
#pragma unroll
                for (int t = 0; t < 4; t++) ss += (double)hv[j][t] * (double)hv[j][t];
            }
        ss = wave_sum_f64(ss);
        const float rn = 1.0f / sqrtf((float)(ss / (double)D) + d.eps);
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const int cc = lane + 64 * j;
            if (cc < D4) {
                f32x4 o;
#pragma unroll
                for (int t = 0; t < 4; t++) o[t] = hv[j][t] * rn * nv[j][t];
                xb4[cc] = o;
            }
        }
    } else {
        /* wider: h and the weights parked in LDS, normalised in batches */
        double ss = 0.0;
        for (int c = lane; c < D4; c += 64 * NV) {
            f32x4 hv[NV], nv[NV];
#pragma unroll
            for (int j = 0; j < NV; j++) {
                const int cc = c + 64 * j;
                if (cc < D4) { hv[j] = h4[cc]; nv[j] = n4[cc]; }
            }
#pragma unroll
            for (int j = 0; j < NV; j++) {
                const int cc = c + 64 * j;
                if (cc < D4) {
#pragma unroll
                    for (int t = 0; t < 4; t++) ss += (double)hv[j][t] * (double)hv[j][t];
                    xb4[cc] = hv[j];
                    xw4[cc] = nv[j];
                }
            }
        }
        ss = wave_sum_f64(ss);
        const float rn = 1.0f / sqrtf((float)(ss / (double)D) + d.eps);
        wave_sync();
        for (int c = lane; c < D4; c += 64 * NV) {
            f32x4 x[NV], w[NV];
#pragma unroll
            for (int j = 0; j < NV; j++)
                if (c + 64 * j < D4) { x[j] = xb4[c + 64 * j]; w[j] = xw4[c + 64 * j]; }
#pragma unroll
            for (int j = 0; j < NV; j++)
                if (c + 64 * j < D4) {
                    f32x4 o;
#pragma unroll
                    for (int t = 0; t < 4; t++) o[t] = x[j][t] * rn * w[j][t];
                    xb4[c + 64 * j] = o;
                }
        }
    }
    wave_sync();
    const LAS float *xb = (const LAS float *)lds;

    /* router row: element i -> lane i mod 32, fmaf in element order, then the
     * reduce32 tree (src/lib/tlm_quant.c:724-738); each buffer is refilled
     * NPRE chunks ahead as soon as it is consumed */
    float r = 0.0f;
    for (int64_t c = 0; c < nfull; c += NPRE) {
#pragma unroll
        for (int i = 0; i < NPRE; i++) {
            if (c + i < nfull) {
                r = fma_chunk<false>(v[i], xb, (c + i) * RCHV, hl, D, r);
                if (c + i + NPRE < nfull) load_chunk<false>(v[i], wr, (c + i + NPRE) * RCHV, hl, D);
            }
        }
    }
    if (ctail < D) r = fma_chunk<true>(vt, xb, ctail, hl, D, r);
    const float res = reduce32(r);
    if (live && hl == 0) ((GAS float *)(ws + L.logits))[row] = res;

    /* group b quantises activation block b for the experts / shared expert
     * into the split layout the gate/up launch copies straight into LDS */
    const int b = blk;
#pragma unroll 1
    for (int which = 0; which < (d.ds > 0 ? 2 : 1); which++) {
        const int kind = dt_act_kind(which ? d.shared_dt : d.expert_dt), bv = bvals(kind);
        const int nb = (int)(D >> (kind == DT_Q8_K ? 8 : 5));   /* D is a multiple of the block */
        if (b >= nb) continue;
        GAS uint8_t *base = (GAS uint8_t *)(ws + (which ? L.xs : L.xe));
        const int sub = kind == DT_Q8_K ? lane : (lane & 7);   /* 4 values per lane */
        const bool ok = kind == DT_Q8_K || lane < 8;
        f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
        if (ok) v = *(const LAS f32x4 *)(xb + (int64_t)b * bv + 4 * sub);
        quant_block_to(kind, v, ok, sub, (GAS uint32_t *)base, (GAS int16_t *)(base + nb * 256),
                       (GAS float *)(base + nb * bv + (kind == DT_Q8_K ? nb * 32 : 0)), b);
    }
    if (b == 0) {
        GAS f32x4 *gxb = (GAS f32x4 *)(ws + L.xb);
        for (int64_t c = lane; c < D / 4; c += 64) gxb[c] = xb4[c];
        if (d.ds > 0) {
            float g = 1.0f;
            if (d.shared_gate_inp) {   /* sequential float dot (src/lib/tlm_model.c:1043-1046) */
                LAS float *gi = (LAS float *)xw4;   /* the norm weights are no longer needed */
                for (int64_t i = lane; i < D; i += 64) gi[i] = ((const GAS float *)d.shared_gate_inp)[i];
                wave_sync();
                float acc = 0.0f;
                if (lane == 0)
                    for (int64_t i = 0; i < D; i++) acc += gi[i] * xb[i];
                g = 1.0f / (1.0f + expf_ref(-acc));
            }
            if (lane == 0) *(GAS float *)ws_sgate(ws, L) = g;
        }
    }
}

template <int NPRE>
__global__ __launch_bounds__(64) void k_moe_router(tlm_hip_moe_desc d, WsLayout L, const float *__restrict__ hptr,
                                                   uint8_t *ws, size_t tstride) {
    args_now(d.D, d.E, d.eps, d.router_w, d.ffn_norm, d.ds, d.expert_dt, d.shared_dt, d.shared_gate_inp, L.logits,
             L.xb, L.xe, L.xs, L.route, hptr, ws, tstride, gridDim.x);
    router_body<NPRE>(d, L, hptr + (size_t)blockIdx.y * d.D, ws + (size_t)blockIdx.y * tstride, blockIdx.x);
}
/* chunks in flight from the start for rows of D values */
inline int router_npre(int64_t D) { return D > 4 * RCHV ? 8 : 4; }

/* Several routers over the same residual in one launch (a block's and its
 * lookahead hints'): blockIdx.y picks the router, each with its own
 * descriptor, workspace and group count. */
constexpr int MULTI_ROUTES = 8;
struct RouterSet {
    tlm_hip_moe_desc d[MULTI_ROUTES];
    WsLayout L[MULTI_ROUTES];
    uint8_t *ws[MULTI_ROUTES];
    int groups[MULTI_ROUTES];
};
template <int NPRE>
__global__ __launch_bounds__(64) void k_moe_router_multi(const RouterSet S, const float *__restrict__ h) {
    const int i = blockIdx.y;
    if ((int)blockIdx.x >= S.groups[i]) return;
    router_body<NPRE>(S.d[i], S.L[i], h, S.ws[i], blockIdx.x);
}

inline int router_groups(const tlm_hip_moe_desc &d) {
    int64_t g = (d.E + 1) / 2;
    const int ek = dt_act_kind(d.expert_dt);
    const int64_t ge = (d.D + bvals(ek) - 1) / bvals(ek);
    if (ge > g) g = ge;
    if (d.ds > 0) {
        const int sk = dt_act_kind(d.shared_dt);
        const int64_t gs = (d.D + bvals(sk) - 1) / bvals(sk);
        if (gs > g) g = gs;
    }
    return (int)g;
}

/* Wave-private copy of a split-layout activation into LDS (16-byte loads,
 * all of a pass in flight first). */
__device__ XLds wave_stage(int kind, const uint8_t *__restrict__ act, int nb, uint8_t *area_g) {
    constexpr int SC = 4;
    const int lane = threadIdx.x & 63;
    const GAS u32x4 *a = (const GAS u32x4 *)act;
    LAS u32x4 *area = (LAS u32x4 *)area_g;
    const int n16 = (int)((stage_bytes(kind, nb) + 15) / 16);
    for (int c0 = 0; c0 < n16; c0 += 64 * SC) {
        u32x4 v[SC];
#pragma unroll
        for (int j = 0; j < SC; j++) {
            const int c = c0 + lane + 64 * j;
            if (c < n16) v[j] = a[c];
        }
#pragma unroll
        for (int j = 0; j < SC; j++) {
            const int c = c0 + lane + 64 * j;
            if (c < n16) area[c] = v[j];
        }
    }
    wave_sync();
    return xlds_at(kind, nb, area_g);
}

/* The wave-private activation copy of wave_stage, issued as direct-to-LDS
 * loads (no registers held): a group can put it in flight before anything
 * else and find it landed when its weights arrive.  Returns false (nothing
 * issued) for an activation of more than 5 16-byte pieces per lane. */
__device__ __forceinline__ bool wave_stage_issue(int kind, const uint8_t *__restrict__ act, int nb, uint8_t *area_g) {
    const int lane = threadIdx.x & 63;
    const int n16 = (int)((stage_bytes(kind, nb) + 15) / 16);
    if (n16 > 64 * 5) return false;
#pragma unroll
    for (int j = 0; j < 5; j++) {
        const int c = lane + 64 * j;
        if (c < n16)
            __builtin_amdgcn_global_load_lds((const void *)(act + (size_t)c * 16),
                                             (LAS void *)(area_g + 64 * 16 * j), 16, 0, 0);
    }
    return true;
}

/* ======================================================================
 * K2: route + gate/up + SwiGLU
 * grid: k * de/16 expert tiles (rank-major), then ds/16 shared tiles
 * LDS: NWAVE wave-private activation copies, then the park of the chunk.
 * ==================================================================== */
template <int DT, int GR>
__device__ void gateup_tile(const tlm_hip_moe_desc &d, const uint8_t *gW, const uint8_t *uW, const uint8_t *act,
                            int64_t F, int64_t t, int i0, float *hh, uint8_t *lds, const ExpTabLanes &tab,
                            bool issued = false) {
    using Fm = Packed<DT>;
    constexpr bool AFF = DT == DT_Q4_K || DT == DT_Q5_K;
    constexpr int IPL = (DT == DT_Q8_0 ? 8 : 4) * GR / TILE_ROWS;
    constexpr int kind = DT == DT_Q8_0 ? DT_Q8_0 : DT_Q8_K;
    const int nb = (int)(d.D / Fm::BV);
    const int wave = threadIdx.x >> 6;
    const size_t xstride = (stage_bytes(kind, nb) + 15) & ~(size_t)15;
    uint8_t *xarea = lds + xstride * wave;
    const int cb = nb < PARK_MAX / TILE_ROWS / 2 ? nb : PARK_MAX / TILE_ROWS / 2;   /* blocks per chunk */
    const Park park = park_at(lds + xstride * NWAVE, 2 * cb * GR);
    const int64_t T = F / TILE_ROWS, units = T * nb * TILE_ROWS;
    const int slots = GROUP_THREADS / Fm::LPI;
    bool staged = false;
    XLds X = xlds_at(kind, nb, xarea);
    float acc = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += cb) {
        const int nbc = nb - b0 < cb ? nb - b0 : cb;
        const int per = nbc * GR, nitems = 2 * per;
        for (int base = 0; base < nitems; base += slots * IPL) {
            auto map = [&](int it, const uint8_t *&W, int64_t &un, int64_t &u, int &b, int &pk) {
                const int g = base + it, m = g >= per, rem = g - m * per;
                W = m ? uW : gW;
                un = units;
                b = b0 + rem / GR;
                u = (t * nb + b) * TILE_ROWS + i0 + rem % GR;
                pk = g;
            };
            auto stage = [&]() {
                if (!staged) {
                    if (issued) {   /* landed by direct-to-LDS loads issued at the group's start */
                        __builtin_amdgcn_s_waitcnt(0);
                        wave_sync();
                    } else {
                        X = wave_stage(kind, act, nb, xarea);
                    }
                    staged = true;
                }
                return X;
            };
            run_items<DT, IPL>(nitems - base, map, stage, park);
        }
        __syncthreads();
        /* threads 0..GR-1: the gate rows' chains, GR..2GR-1: the up rows' */
        if (threadIdx.x < 2 * GR) {
            const int i = threadIdx.x & (GR - 1);
            acc = chain_park<AFF>(park, nbc, threadIdx.x < GR ? 0 : per, GR, i, acc);
        }
        __syncthreads();
    }
    if (threadIdx.x < 64) {   /* wave 0: up value from lane i + GR; e^x in every lane */
        const float up = __shfl_down(acc, GR, 64);
        const float hv = acc / (1.0f + expf_ref_with(-acc, tab)) * up;   /* silu(g) * u (tlm_model.c:171, 927) */
        if (threadIdx.x < GR) hh[t * TILE_ROWS + i0 + threadIdx.x] = hv;
    }
}

/* Where a block's routing and routed matrices come from (MODE): the block
 * routes itself and reads the expert table (ROUTE, no argument); both come as
 * a launch argument (GIVEN, the slot cache's host-resolved blocks); the
 * routing is in the workspace and the slots in device memory (SLOTS, the
 * slot cache's device-resolved blocks) */
constexpr int ROUTE = 0, GIVEN = 1, SLOTS = 2;
struct NoGiven {};
/* a class-template mapping, so that kernel names mangle the same in the host
 * and device passes (an expression over an unnamed enum in a parameter type
 * does not: the two passes number unnamed types differently) */
template <int MODE> struct GivenArgT { using type = NoGiven; };
template <> struct GivenArgT<GIVEN> { using type = MoeGiven; };
template <> struct GivenArgT<SLOTS> { using type = MoeSlots; };
template <int MODE> using GivenArg = typename GivenArgT<MODE>::type;

/* rows of a 16-row tile per routed gate/up group: quarter tiles, 1536
 * groups at the Qwen3-30B-A3B shape (3072 at Qwen3-235B-A22B's), so that
 * while some groups of a compute unit route, others stream their weights (a
 * compute unit's load queue, not HBM, paces each group's weight issue) */
constexpr int GUR = 4;
template <int EDT, int SDT, int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void k_moe_gateup(tlm_hip_moe_desc d, WsLayout L, int32_t *ids_out, float *w_out,
                                                    uint8_t *ws, const GivenArg<MODE> gv) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ RouteLds s_route;
    args_now(d.D, d.de, d.ds, d.E, d.k, d.router, d.routed_scale, d.mask, d.router_bias, d.experts, L.logits, L.route,
             L.hh, L.xe, ids_out, w_out, ws, gridDim.x);
    if constexpr (SDT != NONE) args_now(d.sg, d.su, L.xs);
    ExpTabLanes tab;   /* e^x's table in the lanes (routing, SwiGLU): no global read on the way */
    tab.load();
    constexpr int SPT = TILE_ROWS / GUR;
    const int te = (int)(d.de / TILE_ROWS) * SPT, nexp = d.k * te;
    const bool shared = SDT != NONE && (int)blockIdx.x >= nexp;
    if constexpr (SDT != NONE) {
        if (shared) {
            if constexpr (MODE == SLOTS) {   /* the layer went back to the caller */
                if (((const GAS int32_t *)gv.slot)[0] < 0) return;
            }
            const int t = (int)blockIdx.x - nexp;
            float *hh = (float *)(ws + L.hh) + (size_t)d.k * d.de;
            gateup_tile<SDT, TILE_ROWS>(d, (const uint8_t *)d.sg, (const uint8_t *)d.su, ws + L.xs, d.ds, t, 0, hh,
                                        lds, tab);
            return;
        }
    }
    /* group -> (rank, tile, part): work-groups go to the 8 XCDs round-robin
     * by id, so in each run of 8 SPT ids the parts of 8 (rank, tile) pairs go
     * to one XCD each (ids g, g + 8, ... share the XCD and its L2, whose lines
     * hold neighbouring rows of a tile and its scale plane); ids of a last
     * incomplete run map straight */
    /* the activation (the router's quantised xb) into each wave's copy
     * before the slot, routing or tables are read */
    constexpr int ekind = EDT == DT_Q8_0 ? DT_Q8_0 : DT_Q8_K;
    const int enb = (int)(d.D / Packed<EDT>::BV);
    const bool issued = wave_stage_issue(
        ekind, ws + L.xe, enb, lds + ((stage_bytes(ekind, enb) + 15) & ~(size_t)15) * (threadIdx.x >> 6));
    const int g = (int)blockIdx.x, run = g / (8 * SPT), tpe = te / SPT;
    const bool whole = (run + 1) * 8 * SPT <= nexp;
    const int tau = whole ? run * 8 + g % 8 : g / SPT, part = whole ? (g / 8) % SPT : g % SPT;
    const int r = tau / tpe, t = tau - r * tpe, i0 = part * GUR;
    if constexpr (MODE == SLOTS) {   /* one load for the slot, then the weight loads */
        const int v = ((const GAS int32_t *)gv.slot)[r];
        if (v < 0) {   /* the layer went back to the caller; the LDS loads land first */
            __builtin_amdgcn_s_waitcnt(0);
            return;
        }
        const uint8_t *base = gv.arena + (size_t)v * gv.slot_bytes;
        gateup_tile<EDT, GUR>(d, base + gv.off[0], base + gv.off[1], ws + L.xe, d.de, t, i0,
                              (float *)(ws + L.hh) + (size_t)r * d.de, lds, tab, issued);
        return;
    }
    if constexpr (MODE == GIVEN) {   /* routing and matrices given: the weight loads go out at once */
        if (blockIdx.x == 0 && (int)threadIdx.x < d.k) {
            const int q = threadIdx.x;
            ws_ids(ws, L)[q] = gv.ids[q];
            ws_w(ws, L)[q] = gv.w[q];
            if (ids_out) ids_out[q] = gv.ids[q];
            if (w_out) w_out[q] = gv.w[q];
        }
        gateup_tile<EDT, GUR>(d, gv.p[3 * r], gv.p[3 * r + 1], ws + L.xe, d.de, t, i0,
                              (float *)(ws + L.hh) + (size_t)r * d.de, lds, tab, issued);
        return;
    }
    LAS RouteLds *R = (LAS RouteLds *)&s_route;
    /* every expert's gate / up matrix, loaded with the logits and parked in
     * LDS during routing, so the chosen one costs no extra round trip */
    __shared__ const uint8_t *s_gate[MAXE], *s_up[MAXE];
    const int tid = threadIdx.x;
    const GAS uint64_t *xt = (const GAS uint64_t *)d.experts;
    const uint8_t *tg = tid < d.E ? (const uint8_t *)xt[3 * tid + 0] : nullptr;
    const uint8_t *tu = tid < d.E ? (const uint8_t *)xt[3 * tid + 1] : nullptr;
    /* only group 0 publishes the weights (for the down launch); the others
     * need their expert's id alone */
    route_group(
        d, (const GAS float *)(ws + L.logits), R,
        [&]() {
            s_gate[tid] = tg;
            s_up[tid] = tu;
        },
        tab, blockIdx.x == 0);
    if (blockIdx.x == 0 && (int)threadIdx.x < d.k) {
        const int q = threadIdx.x;
        ws_ids(ws, L)[q] = R->ids[q];
        ws_w(ws, L)[q] = R->w[q];
        if (ids_out) ids_out[q] = R->ids[q];
        if (w_out) w_out[q] = R->w[q];
    }
    const int e = R->ids[r];
    float *hh = (float *)(ws + L.hh) + (size_t)r * d.de;
    gateup_tile<EDT, GUR>(d, s_gate[e], s_up[e], ws + L.xe, d.de, t, i0, hh, lds, tab, issued);
}

/* ======================================================================
 * K3: down + rank-order combine + residual (src/lib/tlm_model.c:921-937,
 * 1029-1050).  Group = 8 rows of D for every rank (and the shared expert):
 * it quantises all ranks' h itself (the reference's activation rule, one
 * block per wave or 8 blocks per wave for Q8_0), streams the ranks' down rows
 * for its 8 rows, and finishes h[row] += sum_r w_r * out_r (+ gate * shared)
 * in rank order, so no launch or group waits for another's rows.
 * ==================================================================== */
constexpr int DROWS = 8;   /* rows of D per K3 group: half a packed tile */

/* Rows row0..row0+7 of nmat matrices F wide (matrix r = wptr(r), activation
 * r = hsrc + r*F); parks (matrix, block, row) results at
 * ((r * nb + b) << 3) + i.  xarea: the activations of all matrices in the split
 * layout; pre() runs once the activation loads are out (all threads call it);
 * the group synchronises before the first compute. */
template <int DT, class WPtr, class Pre>
__device__ void down_rows(int nmat, WPtr wptr, Pre pre, const float *hsrc, int64_t F, int64_t D, int64_t row0,
                          uint8_t *xarea, Park park) {
    using Fm = Packed<DT>;
    constexpr int kind = DT == DT_Q8_0 ? DT_Q8_0 : DT_Q8_K;
    constexpr int BV = Fm::BV, IPL = DT == DT_Q8_0 ? 8 : 4;
    constexpr int LPB = kind == DT_Q8_K ? 16 : 2;  /* lanes per activation block, 16 values each */
    constexpr int BPW = 64 / LPB;                   /* activation blocks per wave per pass */
    constexpr int QB = 2;                           /* passes whose loads go out first */
    const int nb = (int)(F / BV), nq = nmat * nb, nitems = nq * DROWS;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = GROUP_THREADS >> 6;
    const int slots = GROUP_THREADS / Fm::LPI;
    const int64_t units = (D / TILE_ROWS) * nb * TILE_ROWS;
    const int64_t t = row0 / TILE_ROWS, i0 = row0 % TILE_ROWS;
    const XLds X = xlds_at(kind, nq, xarea);
    LAS uint8_t *qx = (LAS uint8_t *)xarea;
    LAS int16_t *bsx = (LAS int16_t *)(xarea + nq * 256);
    LAS float *dx = (LAS float *)(xarea + nq * BV + (kind == DT_Q8_K ? nq * 32 : 0));
    const GAS float *hg = (const GAS float *)hsrc;
    /* activation block of pass m for this lane (blocks of all matrices are
     * contiguous in h: block j starts at value j * BV); the lane takes values
     * 16*sub..16*sub+15 of it */
    const int sub = lane % LPB;
    auto qblock = [&](int m) { return (wave + nw * m) * BPW + lane / LPB; };
    auto qload = [&](int m, f32x4 (&v)[4]) {
        const int j = qblock(m);
        if (j < nq) {
            const GAS f32x4 *src = (const GAS f32x4 *)(hg + (int64_t)j * BV + 16 * sub);
#pragma unroll
            for (int u = 0; u < 4; u++) v[u] = src[u];
        }
    };
    f32x4 hv[QB][4];
#pragma unroll
    for (int m = 0; m < QB; m++) qload(m, hv[m]);
    pre();   /* with the activation loads in flight */
    auto quant = [&](int m, const f32x4 (&v)[4]) { quant16_to(kind, v, qblock(m) < nq, sub, qx, bsx, dx, qblock(m)); };
    for (int base = 0; base < nitems; base += slots * IPL) {
        auto map = [&](int it, const uint8_t *&W, int64_t &un, int64_t &u, int &b, int &pk) {
            const int g = base + it, i = g & (DROWS - 1), j = g >> 3;
            const int r = j / nb, blk = j - r * nb;
            W = wptr(r);
            un = units;
            u = (t * nb + blk) * TILE_ROWS + i0 + i;
            b = j;
            pk = g;
        };
        auto stage = [&]() {
            if (base == 0) {
#pragma unroll
                for (int m = 0; m < QB; m++) quant(m, hv[m]);
                for (int m = QB; (wave + nw * m) * BPW < nq; m++) {   /* wider than QB passes */
                    f32x4 v[4];
                    qload(m, v);
                    quant16_to_ool(kind, v[0], v[1], v[2], v[3], qblock(m) < nq, sub, qx, bsx, dx, qblock(m));
                }
                __syncthreads();
            }
            return X;
        };
        run_items<DT, IPL>(nitems - base, map, stage, park);
    }
}

/* Row i's result for matrix r: the block chain in ascending order. */
template <int DT>
__device__ __forceinline__ float down_chain(const Park &k, int r, int nb, int i) {
    constexpr bool AFF = DT == DT_Q4_K || DT == DT_Q5_K;
    return chain_park<AFF>(k, nb, (r * nb) << 3, DROWS, i, 0.0f);
}

__host__ __device__ inline size_t down_lds_part(int kind, int nq) {
    return ((stage_bytes(kind, nq) + 15) & ~(size_t)15) + park_bytes(nq * DROWS);
}

template <int EDT, int SDT, int MODE>
__global__ __launch_bounds__(256) void k_moe_down(tlm_hip_moe_desc d, WsLayout L, float *__restrict__ h,
                                                  uint8_t *ws, const GivenArg<MODE> gv) {
    extern __shared__ __align__(16) uint8_t lds[];
    args_now(d.D, d.de, d.ds, d.E, d.k, d.experts, L.route, L.hh, h, ws, gridDim.x);
    if constexpr (SDT != NONE) args_now(d.sd);
    constexpr int ek = EDT == DT_Q8_0 ? DT_Q8_0 : DT_Q8_K;
    const int k = d.k;
    /* Work-groups go to the 8 XCDs round-robin by id, so groups g and g + 8
     * share an XCD (and its L2): they take the two halves of one packed tile,
     * whose rows meet inside shared cache lines.  Ids of a last incomplete
     * run of 16 map straight. */
    const int g = blockIdx.x, ng = (int)gridDim.x;
    const int g16 = g & ~15;
    const int64_t row0 = g16 + 16 <= ng ? ((int64_t)(g16 >> 1) + (g & 7)) * TILE_ROWS + ((g >> 3) & 1) * DROWS
                                        : (int64_t)g * DROWS;
    const int nbe = (int)(d.de / Packed<EDT>::BV);
    /* rank t's expert id (thread t < k), clamped so that a stray call before
     * any routing still reads valid memory, and expert t's down matrix (t < E):
     * both reach LDS once the activation loads are in flight */
    __shared__ const uint8_t *s_tab[MAXE];
    __shared__ int s_eid[MAXK];
    __shared__ float s_w[MAXK];
    __shared__ float s_out[(MAXK + 1) * DROWS];
    const int tid = threadIdx.x;
    int eid = 0;
    const uint8_t *tab = nullptr;
    float wl = 0.0f;   /* the combine's inputs, loaded before anything waits; w reaches LDS only
                        * after the rows are done, so no wave stalls on it early */
    if constexpr (MODE == GIVEN) {
        if (tid < k) wl = gv.w[tid];
    } else if constexpr (MODE == SLOTS) {   /* rank t's down matrix from its slot */
        if (((const GAS int32_t *)gv.slot)[0] < 0) return;   /* the layer went back to the caller */
        if (tid < k) {
            const int v = ((const GAS int32_t *)gv.slot)[tid];
            tab = gv.arena + (size_t)v * gv.slot_bytes + gv.off[2];
            wl = ((const GAS float *)ws_w(ws, L))[tid];
        }
    } else {
        eid = tid < k ? ((const GAS int32_t *)ws_ids(ws, L))[tid] : 0;
        tab = tid < d.E ? (const uint8_t *)((const GAS uint64_t *)d.experts)[3 * tid + 2] : nullptr;
        wl = tid < k ? ((const GAS float *)ws_w(ws, L))[tid] : 0.0f;
    }
    float hv = 0.0f, sg = 0.0f;
    if (tid < DROWS) {
        hv = h[row0 + tid];
        if (SDT != NONE) sg = *(const GAS float *)ws_sgate(ws, L);
    }
    auto table = [&]() {
        if (tid < d.E) s_tab[tid] = tab;
        if (tid < k) s_eid[tid] = (eid < 0 || eid >= d.E) ? 0 : eid;
        __syncthreads();
    };
    const Park pe = park_at(lds + ((stage_bytes(ek, k * nbe) + 15) & ~(size_t)15), k * nbe * DROWS);
    if constexpr (MODE == GIVEN)
        down_rows<EDT>(k, [&](int r) { return gv.p[3 * r + 2]; }, []() {}, (const float *)(ws + L.hh), d.de, d.D,
                       row0, lds, pe);
    else if constexpr (MODE == SLOTS)
        down_rows<EDT>(k, [&](int r) { return s_tab[r]; },
                       [&]() {
                           if (tid < k) s_tab[tid] = tab;
                           __syncthreads();
                       },
                       (const float *)(ws + L.hh), d.de, d.D, row0, lds, pe);
    else
        down_rows<EDT>(k, [&](int r) { return s_tab[s_eid[r]]; }, table, (const float *)(ws + L.hh), d.de, d.D, row0,
                       lds, pe);
    Park ps = pe;
    int nbs = 0;
    if constexpr (SDT != NONE) {
        constexpr int sk = SDT == DT_Q8_0 ? DT_Q8_0 : DT_Q8_K;
        nbs = (int)(d.ds / Packed<SDT>::BV);
        uint8_t *xs = lds + down_lds_part(ek, k * nbe);
        ps = park_at(xs + ((stage_bytes(sk, nbs) + 15) & ~(size_t)15), nbs * DROWS);
        down_rows<SDT>(1, [&](int) { return (const uint8_t *)d.sd; }, []() {},
                       (const float *)(ws + L.hh) + (size_t)k * d.de, d.ds, d.D, row0, xs, ps);
    }
    __syncthreads();
    /* row chains, one thread per (matrix, row); then the rank-order sum */
    const int nm = k + (SDT != NONE ? 1 : 0);
    for (int t = tid; t < nm * DROWS; t += GROUP_THREADS) {
        const int r = t >> 3, i = t & (DROWS - 1);
        if constexpr (SDT != NONE) s_out[t] = r < k ? down_chain<EDT>(pe, r, nbe, i) : down_chain<SDT>(ps, 0, nbs, i);
        else s_out[t] = down_chain<EDT>(pe, r, nbe, i);
    }
    if (tid < k) s_w[tid] = wl;
    __syncthreads();
    if (tid < DROWS) {
        float ffn = 0.0f;
        for (int r = 0; r < k; r++) {
            const float c = s_w[r] * s_out[r * DROWS + tid];
            ffn += c;
        }
        if constexpr (SDT != NONE) ffn += sg * s_out[k * DROWS + tid];
        h[row0 + tid] = hv + ffn;
    }
}

/* ======================================================================
 * Prefill: T tokens through the block at once (src/lib/tlm_model.c:1105-1113
 * runs the decode step per token; the MoE block has no cross-token terms, so
 * batching keeps every token's bits).  Each token is normalised and quantised
 * by one wave as K1 does it; router logits come 8 tokens x 8 rows per group
 * in K1's dot order; each token routes as in K2; (token, rank) pairs are
 * bucketed by expert into
 * slots; each expert's gate / up / down rows stream once per 32 of its slots
 * through the int8 MFMA tile; the combine runs per token in rank order.
 * ==================================================================== */
struct PfLayout {
    size_t tok;        /* T per-token decode workspaces (stride tstride) */
    size_t pair_e;     /* int32 [T*k]: expert of (token, rank) */
    size_t pair_w;     /* f32 [T*k]: its routing weight */
    size_t pair_pos;   /* int32 [T*k]: position in its expert's slot run */
    size_t slot_of;    /* int32 [T*k]: slot of (token, rank) */
    size_t slot_tok;   /* int32 [T*k]: token of slot */
    size_t tiles;      /* int32 [MT][3]: expert (-1 unused), first slot, slots */
    size_t hbuf;       /* f32 [T*k][de]: silu(g) * u per slot */
    size_t hq;         /* [T*k] split-layout Q8_K of hbuf rows, stride hq_stride */
    size_t out;        /* f32 [T*k][D]: down output per slot */
    /* the shared expert (ds > 0): its activation per token (reference layout,
     * xb's then h's), gate and up [T][ds], h [T][ds], down output [T][D], gate */
    size_t sact, sg, su, sh, sout, sgate, sact_stride;   /* sact_stride: the larger token row */
    size_t tstride, hq_stride, total;
    int64_t T;
    int MT;
};

inline PfLayout pf_layout(const tlm_hip_moe_desc &d, int64_t T) {
    PfLayout P;
    const WsLayout L = ws_layout(d);
    const size_t pairs = (size_t)T * d.k;
    size_t o = 0;
    P.T = T;
    P.MT = (int)(pairs / tokmm::TM_TOK + d.E);
    P.tstride = L.total;
    P.hq_stride = al256(stage_bytes(DT_Q8_K, (int)(d.de / 256)));
    P.tok = o;      o += P.tstride * T;
    P.pair_e = o;   o += al256(pairs * 4);
    P.pair_w = o;   o += al256(pairs * 4);
    P.pair_pos = o; o += al256(pairs * 4);
    P.slot_of = o;  o += al256(pairs * 4);
    P.slot_tok = o; o += al256(pairs * 4);
    P.tiles = o;    o += al256((size_t)P.MT * 12);
    P.hbuf = o;     o += al256(pairs * d.de * 4);
    P.hq = o;       o += P.hq_stride * pairs;
    P.out = o;      o += al256(pairs * d.D * 4);
    const size_t ds = d.ds > 0 ? (size_t)d.ds : 0, Ts = ds ? (size_t)T : 0;
    const int sk = ds ? dt_act_kind(d.shared_dt) : DT_Q8_K;
    P.sact_stride = ds ? act_bytes(sk, d.D > d.ds ? d.D : d.ds) : 0;
    P.sact = o;     o += al256(Ts * P.sact_stride);
    P.sg = o;       o += al256(Ts * ds * 4);
    P.su = o;       o += al256(Ts * ds * 4);
    P.sh = o;       o += al256(Ts * ds * 4);
    P.sout = o;     o += al256(Ts * d.D * 4);
    P.sgate = o;    o += al256(Ts * 4);
    P.total = o;
    return P;
}

/* Per (block b, token) one wave: xb = rmsnorm(h) with the router launch's
 * lane order and tree (same bits; every wave of a token sums the same
 * squares), block b of xb published to the token's workspace and quantised
 * to Q8_K in the split layout.  D is a multiple of 256, so lane l's f32x4
 * l + 64 b is lane l's part of block b. */
__global__ __launch_bounds__(64) void k_pf_norm(tlm_hip_moe_desc d, WsLayout L, PfLayout P, const float *__restrict__ h,
                                                uint8_t *ws) {
    args_now(d.D, d.eps, d.ffn_norm, L.xb, L.xe, P.tok, P.tstride, h, ws);
    const int lane = threadIdx.x, b = blockIdx.x;
    const int64_t D = d.D;
    const int nb = (int)(D / 256);
    const GAS f32x4 *h4 = (const GAS f32x4 *)(h + (size_t)blockIdx.y * D);
    GAS uint8_t *wst = (GAS uint8_t *)(ws + P.tok + (size_t)blockIdx.y * P.tstride);
    const f32x4 nv = ((const GAS f32x4 *)d.ffn_norm)[lane + 64 * b];
    constexpr int NV = 8;                  /* 16-byte loads per lane per batch, all in flight at once */
    double ss = 0.0;
    f32x4 mine = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j0 = 0; j0 < nb; j0 += NV) {
        f32x4 hv[NV];
#pragma unroll
        for (int j = 0; j < NV; j++)
            if (j0 + j < nb) hv[j] = h4[lane + 64 * (j0 + j)];
#pragma unroll
        for (int j = 0; j < NV; j++)
            if (j0 + j < nb) {
#pragma unroll
                for (int t = 0; t < 4; t++) ss += (double)hv[j][t] * (double)hv[j][t];
                if (j0 + j == b) mine = hv[j];
            }
    }
    ss = wave_sum_f64(ss);
    const float rn = 1.0f / sqrtf((float)(ss / (double)D) + d.eps);
    f32x4 o;
#pragma unroll
    for (int t = 0; t < 4; t++) o[t] = mine[t] * rn * nv[t];
    ((GAS f32x4 *)(wst + L.xb))[lane + 64 * b] = o;
    GAS uint8_t *xe = wst + L.xe;
    quant_block_to(DT_Q8_K, o, true, lane, (GAS uint32_t *)xe, (GAS int16_t *)(xe + nb * 256),
                   (GAS float *)(xe + nb * 288), b);
}

/* Router logits of 8 tokens x 8 router rows per group: the tokens' xb in
 * LDS a 512-value chunk at a time, each thread one row's lane (i mod 32) for
 * all 8 tokens, fmaf in element order, then reduce32 - every (token, row)
 * dot has the decode launch's order and bits.  The chunk is stored
 * transposed, [token][lane][m] for element c0 + lane + 32 m (lane rows 80
 * bytes apart: 16-byte reads of 8 lanes fall on distinct banks), so a lane
 * reads four of its values at once; the next chunk's values and router
 * weights are in flight in registers while a chunk computes. */
constexpr int PFL_ROWS = 8, PFL_TOK = 8, PFL_CH = 512, PFL_M = PFL_CH / 32, PFL_LS = 20;
__global__ __launch_bounds__(256) void k_pf_logits(tlm_hip_moe_desc d, WsLayout L, PfLayout P, uint8_t *ws) {
    __shared__ __align__(16) float s_x[PFL_TOK * 32 * PFL_LS];
    args_now(d.D, d.E, d.router_w, L.xb, L.logits, P.tok, P.tstride, P.T, ws);
    const int tid = threadIdx.x, hl = tid & 31;
    const int64_t D = d.D, e = (int64_t)blockIdx.x * PFL_ROWS + (tid >> 5);
    const int t0 = (int)blockIdx.y * PFL_TOK;
    const GAS float *wr = (const GAS float *)d.router_w + (e < d.E ? e : d.E - 1) * D + hl;
    /* staging: thread tid loads f32x4 q = tid % 128 (elements 4q..4q+3 of the
     * chunk) of tokens tid / 128 + 2 k, k = 0..7 */
    const int sq = tid & 127, st = tid >> 7;
    const GAS f32x4 *xrow[PFL_TOK / 2];
#pragma unroll
    for (int k = 0; k < PFL_TOK / 2; k++) {
        const int tt = t0 + st + 2 * k < P.T ? t0 + st + 2 * k : (int)P.T - 1;
        xrow[k] = (const GAS f32x4 *)(ws + P.tok + (size_t)tt * P.tstride + L.xb) + sq;
    }
    auto load_x = [&](int64_t c0, int ch, f32x4 (&xv)[PFL_TOK / 2]) {
#pragma unroll
        for (int k = 0; k < PFL_TOK / 2; k++) xv[k] = 4 * sq < ch ? xrow[k][c0 / 4] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    };
    auto load_w = [&](int64_t c0, int ch, float (&wv)[PFL_M]) {
#pragma unroll
        for (int m = 0; m < PFL_M; m++) wv[m] = 32 * m < ch ? wr[c0 + 32 * m] : 0.0f;
    };
    float acc[PFL_TOK];
#pragma unroll
    for (int t = 0; t < PFL_TOK; t++) acc[t] = 0.0f;
    f32x4 xv[PFL_TOK / 2];
    float wv[PFL_M], wn[PFL_M];
    int ch = D < PFL_CH ? (int)D : PFL_CH;          /* D is a multiple of 32 */
    load_x(0, ch, xv);
    load_w(0, ch, wv);
    for (int64_t c0 = 0; c0 < D; c0 += PFL_CH) {
        __syncthreads();                            /* the last chunk is consumed */
#pragma unroll
        for (int k = 0; k < PFL_TOK / 2; k++)
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = 4 * sq + u;           /* element c0 + i -> lane i % 32, m = i / 32 */
                s_x[((st + 2 * k) * 32 + (i & 31)) * PFL_LS + (i >> 5)] = xv[k][u];
            }
        __syncthreads();
        const int cur = ch;
        const int64_t c1 = c0 + PFL_CH;
        if (c1 < D) {
            ch = D - c1 < PFL_CH ? (int)(D - c1) : PFL_CH;
            load_x(c1, ch, xv);
            load_w(c1, ch, wn);
        }
        const LAS float *xl = (const LAS float *)s_x + hl * PFL_LS;
#pragma unroll
        for (int m4 = 0; m4 < PFL_M / 4; m4++) {
            if (32 * 4 * m4 >= cur) break;
#pragma unroll
            for (int t = 0; t < PFL_TOK; t++) {
                const f32x4 x4 = *(const LAS f32x4 *)(xl + t * 32 * PFL_LS + 4 * m4);
#pragma unroll
                for (int k = 0; k < 4; k++)
                    if (32 * (4 * m4 + k) < cur) acc[t] = fmaf(wv[4 * m4 + k], x4[k], acc[t]);
            }
        }
#pragma unroll
        for (int m = 0; m < PFL_M; m++) wv[m] = wn[m];
    }
#pragma unroll
    for (int t = 0; t < PFL_TOK; t++) {
        const float res = reduce32(acc[t]);
        if (hl == 0 && e < d.E && t0 + t < P.T)
            ((GAS float *)(ws + P.tok + (size_t)(t0 + t) * P.tstride + L.logits))[e] = res;
    }
}

__global__ __launch_bounds__(256) void k_pf_route(tlm_hip_moe_desc d, WsLayout L, PfLayout P, uint8_t *ws,
                                                  int32_t *ids_out, float *w_out) {
    __shared__ RouteLds s_route;
    args_now(d.E, d.k, d.router, d.routed_scale, d.mask, d.router_bias, L.logits, P.tok, P.tstride, P.pair_e,
             P.pair_w, ws, ids_out, w_out);
    ExpTabLanes tab;
    tab.load();
    const int t = blockIdx.x;
    const uint8_t *wst = ws + P.tok + (size_t)t * P.tstride;
    LAS RouteLds *R = (LAS RouteLds *)&s_route;
    route_group(d, (const GAS float *)(wst + L.logits), R, []() {}, tab);
    if ((int)threadIdx.x < d.k) {
        const int q = threadIdx.x;
        const size_t pr = (size_t)t * d.k + q;
        ((GAS int32_t *)(ws + P.pair_e))[pr] = R->ids[q];
        ((GAS float *)(ws + P.pair_w))[pr] = R->w[q];
        if (ids_out) ids_out[pr] = R->ids[q];
        if (w_out) w_out[pr] = R->w[q];
    }
}

/* Routing alone for one token (route(), src/lib/tlm_model.c:798-839) from the
 * logits the router launch left in the workspace: ids / w into the
 * workspace's route area (where the gate/up launch puts the same values) and,
 * when given, to ids_out / w_out. */
__global__ __launch_bounds__(256) void k_moe_route(tlm_hip_moe_desc d, WsLayout L, uint8_t *ws, int32_t *ids_out,
                                                   float *w_out) {
    __shared__ RouteLds s_route;
    args_now(d.E, d.k, d.router, d.routed_scale, d.mask, d.router_bias, L.logits, L.route, ws, ids_out, w_out);
    ExpTabLanes tab;
    tab.load();
    LAS RouteLds *R = (LAS RouteLds *)&s_route;
    route_group(d, (const GAS float *)(ws + L.logits), R, []() {}, tab);
    if ((int)threadIdx.x < d.k) {
        const int q = threadIdx.x;
        ws_ids(ws, L)[q] = R->ids[q];
        ws_w(ws, L)[q] = R->w[q];
        if (ids_out) ids_out[q] = R->ids[q];
        if (w_out) w_out[q] = R->w[q];
    }
}

/* The routing of several routers (group i: router i's logits in its
 * workspace) straight into a page-locked host area: ids int32[32] at 256 i,
 * w f32[32] at 256 i + 128, then the route's sequence word at seq_off + 4 i,
 * stored after a system-scope fence so that the host sees the routing first. */
struct RouteSet {
    tlm_hip_moe_desc d[MULTI_ROUTES];
    WsLayout L[MULTI_ROUTES];
    uint8_t *ws[MULTI_ROUTES];
};
__global__ __launch_bounds__(256) void k_moe_route_host(const RouteSet S, uint32_t *host, int seq_off, uint32_t seq,
                                                        const RouteDev rd) {
    __shared__ RouteLds s_route;
    __shared__ int s_bad;
    __shared__ int32_t s_row[MAXE];
    const int i = blockIdx.x;
    const tlm_hip_moe_desc &d = S.d[i];
    const int q = threadIdx.x;
    const bool dev = i == 0 && rd.tab != nullptr;   /* uniform over the group */
    if (q == 0) s_bad = 0;
    ExpTabLanes tab;
    tab.load();
    LAS RouteLds *R = (LAS RouteLds *)&s_route;
    /* the layer's row of the slot table (mapped host memory, system scope),
     * read while the logits arrive and the routing runs.  Safe that early:
     * this launch was queued after the host replayed the earlier layers (no
     * entry of this layer's experts can be cleared before its export), so an
     * entry read here is at worst a load that lands a moment later (-1),
     * which only hands the layer back */
    int32_t rowv = -1;
    int z;   /* 0, in a vector register: the loaded value stays per lane */
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    /* unconditional (a branch around it would make the routing wait for it);
     * without a table the word read is the export's own area */
    const int32_t *rp = dev ? rd.tab : (const int32_t *)host;
    route_group(d, (const GAS float *)(S.ws[i] + S.L[i].logits), R, []() {}, tab, true, [&]() {
        rowv = __hip_atomic_load(rp + (q < d.E ? q : 0) + z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    });
    if (dev) {
        if (q < d.E) s_row[q] = rowv;
        __syncthreads();
    }
    /* the routed experts' slots; any expert without a landed slot sends the
     * whole layer back to the caller */
    int32_t v = -1;
    if (dev && q < d.k) {
        v = s_row[R->ids[q]];
        if (v < 0 || v >= rd.n_slots) s_bad = 1;
    }
    if (q < 32) {
        const bool on = q < d.k;
        host[64 * i + q] = on ? (uint32_t)R->ids[q] : 0u;
        host[64 * i + 32 + q] = on ? __float_as_uint(R->w[q]) : 0u;
        if (on) {
            ws_ids(S.ws[i], S.L[i])[q] = R->ids[q];
            ws_w(S.ws[i], S.L[i])[q] = R->w[q];
        }
    }
    __syncthreads();
    if (dev) {
        const bool fast = s_bad == 0;
        if (q < d.k) rd.slot_out[q] = fast ? v : -1;
        if (q == 0) __hip_atomic_store(rd.report, fast ? 1u : 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    __threadfence_system();
    __syncthreads();
    if (q == 0) __hip_atomic_store(host + seq_off / 4 + i, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ __launch_bounds__(64) void k_publish_slot(int32_t *entry, int32_t v) {
    if (threadIdx.x == 0) __hip_atomic_store(entry, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

/* One group: slots grouped by expert (order within an expert is free - every
 * slot is computed on its own), and the tile table of 32-slot runs. */
__global__ __launch_bounds__(256) void k_pf_bucket(tlm_hip_moe_desc d, PfLayout P, uint8_t *ws) {
    __shared__ int s_cnt[MAXE], s_off[MAXE], s_toff[MAXE], s_wc[4], s_wt[4];
    args_now(d.E, d.k, P.T, P.MT, P.pair_e, P.pair_pos, P.slot_of, P.slot_tok, P.tiles, ws);
    const int tid = threadIdx.x, E = d.E;
    const int npair = (int)(P.T * d.k);
    const GAS int32_t *pe = (const GAS int32_t *)(ws + P.pair_e);
    GAS int32_t *ppos = (GAS int32_t *)(ws + P.pair_pos);
    if (tid < MAXE) s_cnt[tid] = 0;
    __syncthreads();
    /* 16 pairs per thread per batch: their loads in flight at once */
    constexpr int BP = 16;
    for (int p0 = 0; p0 < npair; p0 += 256 * BP) {
        int ev[BP];
#pragma unroll
        for (int q = 0; q < BP; q++) {
            const int p = p0 + tid + 256 * q;
            const int e = p < npair ? pe[p] : 0;
            ev[q] = (e < 0 || e >= E) ? 0 : e;
        }
#pragma unroll
        for (int q = 0; q < BP; q++) {
            const int p = p0 + tid + 256 * q;
            if (p < npair) ppos[p] = atomicAdd(&s_cnt[ev[q]], 1);
        }
    }
    __syncthreads();
    /* exclusive scans of slot counts and tile counts over the experts: wave
     * scans, then the wave totals */
    const int c = tid < E ? s_cnt[tid] : 0;
    const int nt = (c + tokmm::TM_TOK - 1) / tokmm::TM_TOK;
    const int lane = tid & 63, wave = tid >> 6;
    int ic = c, it = nt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int a = __shfl_up(ic, off, 64), b = __shfl_up(it, off, 64);
        if (lane >= off) { ic += a; it += b; }
    }
    if (lane == 63) { s_wc[wave] = ic; s_wt[wave] = it; }
    __syncthreads();
    int bc = 0, bt = 0;
    for (int w = 0; w < wave; w++) { bc += s_wc[w]; bt += s_wt[w]; }
    if (tid < E) {
        s_off[tid] = bc + ic - c;
        s_toff[tid] = bt + it - nt;
    }
    const int tiles_used = s_wt[0] + s_wt[1] + s_wt[2] + s_wt[3];
    __syncthreads();
    GAS int32_t *slot_of = (GAS int32_t *)(ws + P.slot_of);
    GAS int32_t *slot_tok = (GAS int32_t *)(ws + P.slot_tok);
    for (int p0 = 0; p0 < npair; p0 += 256 * BP) {
        int ev[BP], pv[BP];
#pragma unroll
        for (int q = 0; q < BP; q++) {
            const int p = p0 + tid + 256 * q;
            const int e = p < npair ? pe[p] : 0;
            ev[q] = (e < 0 || e >= E) ? 0 : e;
            pv[q] = p < npair ? ppos[p] : 0;
        }
#pragma unroll
        for (int q = 0; q < BP; q++) {
            const int p = p0 + tid + 256 * q;
            if (p < npair) {
                const int slot = s_off[ev[q]] + pv[q];
                slot_of[p] = slot;
                slot_tok[slot] = p / d.k;
            }
        }
    }
    GAS int32_t *tiles = (GAS int32_t *)(ws + P.tiles);
    if (tid < E) {
        for (int q = 0; q < nt; q++) {
            const int ti = s_toff[tid] + q;
            tiles[3 * ti] = tid;
            tiles[3 * ti + 1] = s_off[tid] + tokmm::TM_TOK * q;
            tiles[3 * ti + 2] = c - tokmm::TM_TOK * q < tokmm::TM_TOK ? c - tokmm::TM_TOK * q : tokmm::TM_TOK;
        }
    }
    for (int ti = tiles_used + tid; ti < P.MT; ti += 256) tiles[3 * ti] = -1;
}

/* Rows of gate and up: 64 rows per group over the tile's (up to 32) slots of
 * one expert - waves 0-1 stream gate rows, waves 2-3 the same rows of up -
 * then, through LDS, h = silu(g) * u per (slot, row) by all four waves. */
template <int DT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void k_pf_gateup(tlm_hip_moe_desc d, WsLayout L, PfLayout P, uint8_t *ws) {
    __shared__ __align__(16) uint8_t s_tile[tokmm::tile_lds_bytes<DT>()];
    static_assert(tokmm::tile_lds_bytes<DT>() >= 2 * 32 * 64 * 4, "g / u area");
    args_now(d.D, d.de, d.experts, L.xe, P.tok, P.tstride, P.tiles, P.slot_tok, P.hbuf, ws);
    const GAS int32_t *tl = (const GAS int32_t *)(ws + P.tiles) + 3 * blockIdx.y;
    const int e = tl[0];
    if (e < 0) return;
    const int s0 = tl[1], n = tl[2];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, half = lane >> 5, up = wave >> 1;
    const int64_t rows = d.de, row = (int64_t)blockIdx.x * 64 + (wave & 1) * 32 + (lane & 31);
    const int64_t rr = row < rows ? row : rows - 1;
    const int nb = (int)(d.D / 256);
    const int64_t units = (rows / TILE_ROWS) * nb * TILE_ROWS;
    const int64_t ubase = (rr / TILE_ROWS) * nb * TILE_ROWS + rr % TILE_ROWS;
    const int js = (int)threadIdx.x >> 3;                  /* the token this thread stages */
    const int slot = s0 + (js < n ? js : n - 1);
    const int tok = ((const GAS int32_t *)(ws + P.slot_tok))[slot];
    const GAS uint8_t *x = (const GAS uint8_t *)(ws + P.tok + (size_t)tok * P.tstride + L.xe);
    const GAS uint64_t *xt = (const GAS uint64_t *)d.experts;
    if (!xt[3 * e]) return;   /* an expert outside this pass (its matrices in no slot): uniform over the group */
    const tokmm::Chain ch = tokmm::chain_at<DT>((const uint8_t *)xt[3 * e + up], units, ubase);
    float acc[16];
    tokmm::tile_run<DT, true>(ch, nb, x, (LAS uint8_t *)s_tile, acc);
    /* the tile ended on a barrier: its LDS takes g and u of the group's 64
     * rows x 32 slots ([gate|up][slot][row]), then every thread forms 8 of
     * the h values (slots past the tile's last are skipped) */
    LAS float *gu = (LAS float *)s_tile;
    const int rl = (wave & 1) * 32 + (lane & 31);
#pragma unroll
    for (int v = 0; v < 16; v++) gu[(up * 32 + 8 * (v >> 2) + 4 * half + (v & 3)) * 64 + rl] = acc[v];
    __syncthreads();
    const int r2 = threadIdx.x & 63;
    const int64_t orow = (int64_t)blockIdx.x * 64 + r2;
    if (orow < rows) {
        GAS float *hb = (GAS float *)(ws + P.hbuf);
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int i = 4 * q + (threadIdx.x >> 6);
            if (i < n) {
                const float g = gu[i * 64 + r2], u = gu[(32 + i) * 64 + r2];
                hb[(size_t)(s0 + i) * rows + orow] = g / (1.0f + expf_ref(-g)) * u;
            }
        }
    }
}

/* Quantise h of every slot (src/lib/tlm_quant.c:458-478): one wave per block. */
__global__ __launch_bounds__(64) void k_pf_hquant(tlm_hip_moe_desc d, PfLayout P, uint8_t *ws) {
    args_now(d.de, P.hbuf, P.hq, P.hq_stride, ws);
    const int b = blockIdx.y, lane = threadIdx.x;
    const size_t slot = blockIdx.x;   /* T * k slots: the grid's x (y is capped at 65536) */
    const int nbd = (int)(d.de / 256);
    const f32x4 v = *(const GAS f32x4 *)((const GAS float *)(ws + P.hbuf) + slot * d.de + (size_t)b * 256 + 4 * lane);
    GAS uint8_t *q = (GAS uint8_t *)(ws + P.hq + slot * P.hq_stride);
    quant_block_to(DT_Q8_K, v, true, lane, (GAS uint32_t *)q, (GAS int16_t *)(q + nbd * 256),
                   (GAS float *)(q + nbd * 288), b);
}

/* Rows of down: 4 waves x 32 rows per group over the tile's slots of one
 * expert. */
template <int DT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void k_pf_down(tlm_hip_moe_desc d, PfLayout P, uint8_t *ws) {
    __shared__ __align__(16) uint8_t s_tile[tokmm::tile_lds_bytes<DT>()];
    args_now(d.D, d.de, d.experts, P.tiles, P.hq, P.hq_stride, P.out, ws);
    const GAS int32_t *tl = (const GAS int32_t *)(ws + P.tiles) + 3 * blockIdx.y;
    const int e = tl[0];
    if (e < 0) return;
    const int s0 = tl[1], n = tl[2];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, half = lane >> 5;
    const int64_t rows = d.D, row = (int64_t)blockIdx.x * 128 + wave * 32 + (lane & 31);
    const int64_t rr = row < rows ? row : rows - 1;
    const int nb = (int)(d.de / 256);
    const int64_t units = (rows / TILE_ROWS) * nb * TILE_ROWS;
    const int js = (int)threadIdx.x >> 3;
    const int slot = s0 + (js < n ? js : n - 1);
    const GAS uint8_t *x = (const GAS uint8_t *)(ws + P.hq + (size_t)slot * P.hq_stride);
    const uint8_t *wd = (const uint8_t *)((const GAS uint64_t *)d.experts)[3 * e + 2];
    if (!wd) return;   /* an expert outside this pass: uniform over the group */
    const tokmm::Chain ch = tokmm::chain_at<DT>(wd, units, (rr / TILE_ROWS) * nb * TILE_ROWS + rr % TILE_ROWS);
    float acc[16];
    tokmm::tile_run<DT, true>(ch, nb, x, (LAS uint8_t *)s_tile, acc);
    if (row < rows) {
        GAS float *out = (GAS float *)(ws + P.out);
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int i = 8 * (v >> 2) + 4 * half + (v & 3);
            if (i < n) out[(size_t)(s0 + i) * rows + row] = acc[v];
        }
    }
}

/* The shared expert's h = silu(g) * u per (token, row) (tlm_model.c:171, 927,
 * the decode gate/up tile's expression). */
__global__ __launch_bounds__(256) void k_pf_swiglu(const float *__restrict__ g, const float *__restrict__ u,
                                                   float *__restrict__ hs, int64_t n) {
    for (int64_t i = threadIdx.x + (int64_t)blockIdx.x * 256; i < n; i += (int64_t)gridDim.x * 256) {
        const float a = g[i];
        hs[i] = a / (1.0f + expf_ref(-a)) * u[i];
    }
}

/* The shared expert's gate per token (src/lib/tlm_model.c:1043-1046): the
 * sigmoid of the sequential float dot of shared_gate_inp with xb, or 1 -
 * the decode router launch's computation. */
__global__ __launch_bounds__(64) void k_pf_sgate(tlm_hip_moe_desc d, WsLayout L, PfLayout P, uint8_t *ws) {
    const int64_t t = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (t >= P.T) return;
    float g = 1.0f;
    if (d.shared_gate_inp) {
        const float *xb = (const float *)(ws + P.tok + (size_t)t * P.tstride + L.xb);
        const float *gi = (const float *)d.shared_gate_inp;
        float acc = 0.0f;
        for (int64_t i = 0; i < d.D; i++) acc += gi[i] * xb[i];
        g = 1.0f / (1.0f + expf_ref(-acc));
    }
    ((float *)(ws + P.sgate))[t] = g;
}

/* h[t] += sum_r w_r * out[slot(t, r)] in rank order, then + sgate * the
 * shared expert's output (src/lib/tlm_model.c:1029-1050). */
__global__ __launch_bounds__(256) void k_pf_combine(tlm_hip_moe_desc d, PfLayout P, float *__restrict__ h,
                                                    uint8_t *ws) {
    args_now(d.D, d.k, P.pair_w, P.slot_of, P.out, h, ws);
    /* four rows per thread (D is a multiple of 256), 16-byte loads */
    const int64_t r4 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int t = blockIdx.y;
    if (4 * r4 >= d.D) return;
    const GAS float *pw = (const GAS float *)(ws + P.pair_w) + (size_t)t * d.k;
    const GAS int32_t *so = (const GAS int32_t *)(ws + P.slot_of) + (size_t)t * d.k;
    const GAS float *out = (const GAS float *)(ws + P.out);
    f32x4 ev[MAXK];
    float wv[MAXK];
#pragma unroll
    for (int q = 0; q < MAXK; q++) {
        if (q < d.k) {
            wv[q] = pw[q];
            ev[q] = *(const GAS f32x4 *)(out + (size_t)so[q] * d.D + 4 * r4);
        }
    }
    GAS f32x4 *hp = (GAS f32x4 *)(h + (size_t)t * d.D) + r4;
    const f32x4 hv = *hp;
    f32x4 sv = {0.0f, 0.0f, 0.0f, 0.0f};
    float sg = 0.0f;
    if (d.ds > 0) {
        sv = *(const GAS f32x4 *)((const GAS float *)(ws + P.sout) + (size_t)t * d.D + 4 * r4);
        sg = ((const GAS float *)(ws + P.sgate))[t];
    }
    f32x4 o;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        float ffn = 0.0f;
#pragma unroll
        for (int q = 0; q < MAXK; q++) {
            if (q < d.k) {
                const float x = wv[q] * ev[q][c];
                ffn += x;
            }
        }
        if (d.ds > 0) ffn += sg * sv[c];
        o[c] = hv[c] + ffn;
    }
    *hp = o;
}

/* ---- instantiation table: [expert dtype][shared dtype or none] --------------- */
typedef void (*gateup_fn)(tlm_hip_moe_desc, WsLayout, int32_t *, float *, uint8_t *, const NoGiven);
typedef void (*down_fn)(tlm_hip_moe_desc, WsLayout, float *, uint8_t *, const NoGiven);
typedef void (*gateup_given_fn)(tlm_hip_moe_desc, WsLayout, int32_t *, float *, uint8_t *, const MoeGiven);
typedef void (*down_given_fn)(tlm_hip_moe_desc, WsLayout, float *, uint8_t *, const MoeGiven);
typedef void (*gateup_slots_fn)(tlm_hip_moe_desc, WsLayout, int32_t *, float *, uint8_t *, const MoeSlots);
typedef void (*down_slots_fn)(tlm_hip_moe_desc, WsLayout, float *, uint8_t *, const MoeSlots);

inline int dt_slot(int dt) { return dt == DT_Q6_K ? 0 : dt == DT_Q8_0 ? 1 : dt == DT_Q4_K ? 2 : dt == DT_Q5_K ? 3 : -1; }

#define ROW(K, E, G) {K<E, NONE, G>, K<E, DT_Q6_K, G>, K<E, DT_Q8_0, G>, K<E, DT_Q4_K, G>, K<E, DT_Q5_K, G>}
const gateup_fn GU[4][5] = {ROW(k_moe_gateup, DT_Q6_K, ROUTE), ROW(k_moe_gateup, DT_Q8_0, ROUTE),
                            ROW(k_moe_gateup, DT_Q4_K, ROUTE), ROW(k_moe_gateup, DT_Q5_K, ROUTE)};
const down_fn DN[4][5] = {ROW(k_moe_down, DT_Q6_K, ROUTE), ROW(k_moe_down, DT_Q8_0, ROUTE),
                          ROW(k_moe_down, DT_Q4_K, ROUTE), ROW(k_moe_down, DT_Q5_K, ROUTE)};
const gateup_given_fn GUG[4][5] = {ROW(k_moe_gateup, DT_Q6_K, GIVEN), ROW(k_moe_gateup, DT_Q8_0, GIVEN),
                                   ROW(k_moe_gateup, DT_Q4_K, GIVEN), ROW(k_moe_gateup, DT_Q5_K, GIVEN)};
const down_given_fn DNG[4][5] = {ROW(k_moe_down, DT_Q6_K, GIVEN), ROW(k_moe_down, DT_Q8_0, GIVEN),
                                 ROW(k_moe_down, DT_Q4_K, GIVEN), ROW(k_moe_down, DT_Q5_K, GIVEN)};
const gateup_slots_fn GUS[4][5] = {ROW(k_moe_gateup, DT_Q6_K, SLOTS), ROW(k_moe_gateup, DT_Q8_0, SLOTS),
                                   ROW(k_moe_gateup, DT_Q4_K, SLOTS), ROW(k_moe_gateup, DT_Q5_K, SLOTS)};
const down_slots_fn DNS[4][5] = {ROW(k_moe_down, DT_Q6_K, SLOTS), ROW(k_moe_down, DT_Q8_0, SLOTS),
                                 ROW(k_moe_down, DT_Q4_K, SLOTS), ROW(k_moe_down, DT_Q5_K, SLOTS)};
#undef ROW

}  // namespace

size_t moe_workspace_bytes(const tlm_hip_moe_desc *d) { return d ? ws_layout(*d).total : 0; }

static bool moe_dt_ok(int dt) { return dt_slot(dt) >= 0; }

int launch_moe_layer(const tlm_hip_moe_desc *d, float *h, int32_t *ids, float *w, void *ws, hipStream_t s) {
    return launch_moe_phase(d, 0, h, ids, w, ws, s);
}

size_t moe_route_offset(const tlm_hip_moe_desc *d) { return ws_layout(*d).route; }

static size_t x_area(int kind, int nb) { return (stage_bytes(kind, nb) + 15) & ~(size_t)15; }

/* descriptor checks shared by the decode and prefill launches; table: the
 * launch reads the expert table (not the routing-only launches, nor a block
 * whose routed matrices are given) */
static int moe_check(const tlm_hip_moe_desc *d, const float *h, const void *ws, bool table = true) {
    if (!d || !h || !ws) return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: NULL argument");
    if ((uintptr_t)ws & 255u) return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: workspace must be 256-byte aligned");
    if (d->E <= 0 || d->E > MAXE || d->k <= 0 || d->k > MAXK || d->k > d->E)
        return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: E=%d k=%d outside 1 <= k <= E <= %d, k <= %d", d->E, d->k, MAXE, MAXK);
    if (d->router < 0 || d->router > 2) return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: router kind %d", d->router);
    if (!moe_dt_ok(d->expert_dt) || (d->ds > 0 && !moe_dt_ok(d->shared_dt)))
        return tlmh_seterr(TLM_HIP_EUNSUP, "moe_layer: expert dtype %d / shared dtype %d not supported",
                           d->expert_dt, d->shared_dt);
    const int ebv = dt_block_values(d->expert_dt);
    if (d->D <= 0 || d->D % TILE_ROWS || d->D % ebv || d->de <= 0 || d->de % TILE_ROWS || d->de % ebv)
        return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: D=%lld de=%lld must be multiples of 16 and of the block",
                           (long long)d->D, (long long)d->de);
    if (d->ds < 0) return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: ds=%lld", (long long)d->ds);
    if (d->ds > 0) {
        const int sbv = dt_block_values(d->shared_dt);
        if (d->ds % TILE_ROWS || d->ds % sbv || d->D % sbv)
            return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: ds=%lld must be a multiple of 16 and of the block",
                               (long long)d->ds);
        if (!d->sg || !d->su || !d->sd) return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: shared matrices missing");
    }
    if (!d->ffn_norm || !d->router_w || (table && !d->experts))
        return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: NULL weights");
    if (((uintptr_t)h | (uintptr_t)d->ffn_norm) & 15u)
        return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: h and ffn_norm must be 16-byte aligned");
    if ((size_t)d->D * 8 > 64 * 1024)
        return tlmh_seterr(TLM_HIP_EUNSUP, "moe_layer: D=%lld exceeds the LDS staging limit", (long long)d->D);
    return TLM_HIP_OK;
}

/* phase 0 = all launches; 1 router, 2 gate/up, 3 down + combine; gv (may be
 * NULL): routing and matrices given by the caller; ms (may be NULL): the
 * routing in the workspace and the matrices in slots */
static int moe_phase(const tlm_hip_moe_desc *d, int phase, float *h, int32_t *ids, float *w, void *ws,
                     const MoeGiven *gvp, hipStream_t s, const MoeSlots *msp = nullptr) {
    if (phase < 0 || phase > 3) return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: phase %d", phase);
    if (int rc = moe_check(d, h, ws, gvp == nullptr && msp == nullptr && phase != 1)) return rc;
    const int ebv = dt_block_values(d->expert_dt);
    const int ek = dt_act_kind(d->expert_dt), sk = d->ds > 0 ? dt_act_kind(d->shared_dt) : ek;
    const int nbe = (int)(d->D / ebv), nbde = (int)(d->de / ebv);
    const int sbv = d->ds > 0 ? dt_block_values(d->shared_dt) : ebv;
    const int nbs = (int)(d->D / sbv), nbsd = d->ds > 0 ? (int)(d->ds / sbv) : 0;
    auto park2 = [](int nb) { int cb = nb < PARK_MAX / TILE_ROWS / 2 ? nb : PARK_MAX / TILE_ROWS / 2; return park_bytes(2 * cb * TILE_ROWS); };
    size_t lds1 = al256((size_t)d->D * 8);          /* x and the norm weights */
    size_t lds2e = NWAVE * x_area(ek, nbe) + park2(nbe);
    size_t lds2s = d->ds > 0 ? NWAVE * x_area(sk, nbs) + park2(nbs) : 0;
    /* K3: every rank's activation and parked rows, then the shared expert's */
    size_t lds3 = down_lds_part(ek, d->k * nbde) + (d->ds > 0 ? down_lds_part(sk, nbsd) : 0);
    size_t lds2 = lds2e > lds2s ? lds2e : lds2s;
    if (lds1 > 64 * 1024 || lds2 > 64 * 1024 || lds3 > 64 * 1024)
        return tlmh_seterr(TLM_HIP_EUNSUP, "moe_layer: D=%lld / k*de=%lld exceed the LDS staging limit",
                           (long long)d->D, (long long)(d->k * d->de));
    uint8_t *w8 = (uint8_t *)ws;
    const tlm_hip_moe_desc dv = *d;
    const WsLayout L = ws_layout(*d);
    const int es = dt_slot(d->expert_dt), ss = d->ds > 0 ? 1 + dt_slot(d->shared_dt) : 0;
    const gateup_fn gu = GU[es][ss];
    const down_fn dn = DN[es][ss];
    const unsigned g1 = (unsigned)router_groups(*d);
    const unsigned g2 = (unsigned)(d->k * (d->de / GUR) + (d->ds > 0 ? d->ds / TILE_ROWS : 0));
    const unsigned g3 = (unsigned)(d->D / DROWS);
    if (phase == 0 || phase == 1)
        hipLaunchKernelGGL(router_npre(d->D) == 8 ? k_moe_router<8> : k_moe_router<4>, dim3(g1), dim3(64), lds1, s,
                           dv, L, (const float *)h, w8, (size_t)0);
    if (msp) {
        const MoeSlots ms = *msp;
        if (phase == 0 || phase == 2)
            hipLaunchKernelGGL(GUS[es][ss], dim3(g2), dim3(64 * NWAVE), lds2, s, dv, L, ids, w, w8, ms);
        if (phase == 0 || phase == 3) hipLaunchKernelGGL(DNS[es][ss], dim3(g3), dim3(256), lds3, s, dv, L, h, w8, ms);
    } else if (gvp) {
        const MoeGiven gv = *gvp;
        if (phase == 0 || phase == 2)
            hipLaunchKernelGGL(GUG[es][ss], dim3(g2), dim3(64 * NWAVE), lds2, s, dv, L, ids, w, w8, gv);
        if (phase == 0 || phase == 3) hipLaunchKernelGGL(DNG[es][ss], dim3(g3), dim3(256), lds3, s, dv, L, h, w8, gv);
    } else {
        if (phase == 0 || phase == 2) hipLaunchKernelGGL(gu, dim3(g2), dim3(64 * NWAVE), lds2, s, dv, L, ids, w, w8,
                                                         NoGiven{});
        if (phase == 0 || phase == 3) hipLaunchKernelGGL(dn, dim3(g3), dim3(256), lds3, s, dv, L, h, w8, NoGiven{});
    }
    return tlmh_check(hipGetLastError(), "moe_layer launch");
}
int launch_moe_phase(const tlm_hip_moe_desc *d, int phase, float *h, int32_t *ids, float *w, void *ws,
                     hipStream_t s) {
    return moe_phase(d, phase, h, ids, w, ws, nullptr, s);
}
int launch_moe_phase_given(const tlm_hip_moe_desc *d, int phase, float *h, void *ws, const MoeGiven *gv,
                           hipStream_t s) {
    if (!gv || d->k > 32) return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: given routing");
    for (int r = 0; r < d->k; r++)
        for (int m = 0; m < 3; m++)
            if (!gv->p[3 * r + m] || ((uintptr_t)gv->p[3 * r + m] & 15u))
                return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: given matrix %d of rank %d", m, r);
    return moe_phase(d, phase, h, nullptr, nullptr, ws, gv, s);
}

int launch_moe_phase_slots(const tlm_hip_moe_desc *d, int phase, float *h, void *ws, const MoeSlots *ms,
                           hipStream_t s) {
    if (!ms || !ms->slot || !ms->arena || phase == 1 || phase == 0 || ((ms->slot_bytes | ms->off[0] | ms->off[1] |
                                                                         ms->off[2] | (uintptr_t)ms->arena) & 15u))
        return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: slot arena");
    return moe_phase(d, phase, h, nullptr, nullptr, ws, nullptr, s, ms);
}

/* The router launch, then routing alone: ids / w (k each) in the workspace's
 * route area (moe_route_offset: ids int32 at +0, w f32 at +128). */
int launch_moe_route(const tlm_hip_moe_desc *d, const float *h, int32_t *ids, float *w, void *ws, hipStream_t s) {
    if (int rc = launch_moe_phase(d, 1, (float *)h, nullptr, nullptr, ws, s)) return rc;
    hipLaunchKernelGGL(k_moe_route, dim3(1), dim3(256), 0, s, *d, ws_layout(*d), (uint8_t *)ws, ids, w);
    return tlmh_check(hipGetLastError(), "moe_route launch");
}

/* The routers of d[0..n) over the same residual h (one launch), then their
 * routing into the host area (one launch, see k_moe_route_host) */
int launch_moe_routes_host(const tlm_hip_moe_desc *const *d, void *const *ws, int n, const float *h,
                           uint32_t *host, int seq_off, uint32_t seq, hipStream_t s, const RouteDev *rd) {
    if (n < 1 || n > MULTI_ROUTES) return tlmh_seterr(TLM_HIP_EINVAL, "moe routes: %d routers", n);
    RouterSet rs{};
    RouteSet qs{};
    int g = 0;
    size_t lds = 0;
    for (int i = 0; i < n; i++) {
        if (int rc = moe_check(d[i], h, ws[i], false)) return rc;
        rs.d[i] = qs.d[i] = *d[i];
        rs.L[i] = qs.L[i] = ws_layout(*d[i]);
        rs.ws[i] = qs.ws[i] = (uint8_t *)ws[i];
        rs.groups[i] = router_groups(*d[i]);
        g = rs.groups[i] > g ? rs.groups[i] : g;
        lds = al256((size_t)d[i]->D * 8) > lds ? al256((size_t)d[i]->D * 8) : lds;
    }
    if (lds > 64 * 1024) return tlmh_seterr(TLM_HIP_EUNSUP, "moe routes: D exceeds the LDS staging limit");
    int64_t dmax = 0;
    for (int i = 0; i < n; i++) dmax = d[i]->D > dmax ? d[i]->D : dmax;
    hipLaunchKernelGGL(router_npre(dmax) == 8 ? k_moe_router_multi<8> : k_moe_router_multi<4>,
                       dim3((unsigned)g, (unsigned)n), dim3(64), lds, s, rs, h);
    RouteDev r{};
    if (rd) {
        if (!rd->tab || !rd->slot_out || !rd->report || rd->n_slots <= 0)
            return tlmh_seterr(TLM_HIP_EINVAL, "moe routes: slot resolution");
        r = *rd;
    }
    hipLaunchKernelGGL(k_moe_route_host, dim3((unsigned)n), dim3(256), 0, s, qs, host, seq_off, seq, r);
    return tlmh_check(hipGetLastError(), "moe routes launch");
}

int launch_publish_slot(int32_t *entry, int32_t v, hipStream_t s) {
    hipLaunchKernelGGL(k_publish_slot, dim3(1), dim3(64), 0, s, entry, v);
    return tlmh_check(hipGetLastError(), "store: publish slot");
}

size_t moe_prefill_workspace_bytes(const tlm_hip_moe_desc *d, int64_t T) {
    return (d && T > 0) ? pf_layout(*d, T).total : 0;
}

/* T tokens: norm + quantisation per token, batched router logits, routing per
 * token, bucketing, gate/up + SwiGLU,
 * h quantisation, down, combine. */
static int moe_prefill_check(const tlm_hip_moe_desc *d, const float *h, int64_t T, const void *ws, bool table) {
    if (int rc = moe_check(d, h, ws, table)) return rc;
    if (T <= 0 || T > 65536) return tlmh_seterr(TLM_HIP_EINVAL, "moe_prefill: T=%lld outside 1..65536", (long long)T);
    if ((d->expert_dt != DT_Q4_K && d->expert_dt != DT_Q5_K && d->expert_dt != DT_Q6_K) ||
        (d->ds > 0 && (!tokmm::tile_dt(d->shared_dt) || d->ds % 256 || d->D % 256)))
        return tlmh_seterr(TLM_HIP_EUNSUP, "moe_prefill: routed Q4_K / Q5_K / Q6_K experts, a shared expert of "
                           "Q4_K / Q5_K / Q6_K / Q8_0 and widths a multiple of 256 only (expert dtype %d, shared "
                           "dtype %d, ds %lld)", d->expert_dt, d->shared_dt, (long long)d->ds);
    if (pf_layout(*d, T).MT > 65536)   /* the tile grids' y */
        return tlmh_seterr(TLM_HIP_EINVAL, "moe_prefill: T=%lld x k=%d gives more than 65536 tiles", (long long)T,
                           d->k);
    return TLM_HIP_OK;
}

/* The prefill block in three stages, so that a caller whose experts come
 * through the slot cache can acquire them between the routing and the
 * expert work, and run the expert work in passes of the experts it holds:
 * route = norm, router logits, the shared expert, routing (ids / w per
 * (token, rank)), bucketing; experts = grouped gate/up, h quantisation,
 * grouped down for the tiles whose expert has matrices in d->experts (a
 * null entry skips the expert's tiles; every (token, rank) slot belongs to
 * one expert, so passes over disjoint expert sets fill disjoint slots);
 * combine = the rank-order sum into h. */
int launch_moe_prefill_route(const tlm_hip_moe_desc *d, float *h, int64_t T, int32_t *ids, float *w, void *ws,
                             hipStream_t s) {
    if (int rc = moe_prefill_check(d, h, T, ws, false)) return rc;
    const tlm_hip_moe_desc dv = *d;
    const WsLayout L = ws_layout(*d);
    const PfLayout P = pf_layout(*d, T);
    uint8_t *w8 = (uint8_t *)ws;
    hipLaunchKernelGGL(k_pf_norm, dim3((unsigned)(d->D / 256), (unsigned)T), dim3(64), 0, s, dv, L, P, (const float *)h,
                       w8);
    hipLaunchKernelGGL(k_pf_logits, dim3((unsigned)((d->E + PFL_ROWS - 1) / PFL_ROWS), (unsigned)((T + PFL_TOK - 1) / PFL_TOK)),
                       dim3(256), 0, s, dv, L, P, w8);
    if (d->ds > 0) {   /* the shared expert of every token: its gate / up, SwiGLU, down and gate */
        const int sk = dt_act_kind(d->shared_dt);
        float *G = (float *)(w8 + P.sg), *U = (float *)(w8 + P.su), *Hs = (float *)(w8 + P.sh);
        /* token rows of the activation as the token matmul reads them: act_bytes of the width */
        int rc = launch_tok_norm_act(sk, (const float *)(w8 + P.tok + L.xb), (int64_t)(P.tstride / 4), nullptr, 0.0f,
                                     d->D, T, w8 + P.sact, (int64_t)act_bytes(sk, d->D), s);
        const void *Wgu[2] = {d->sg, d->su};
        const int64_t Rgu[2] = {d->ds, d->ds};
        float *const Ygu[2] = {G, U};
        if (!rc) rc = launch_tokmm_segs(d->shared_dt, 2, Wgu, Rgu, d->D, w8 + P.sact, T, Ygu, s);
        if (!rc) {
            const int64_t n = T * d->ds;
            hipLaunchKernelGGL(k_pf_swiglu, dim3((unsigned)((n + 1023) / 1024)), dim3(256), 0, s, (const float *)G,
                               (const float *)U, Hs, n);
            rc = launch_tok_norm_act(sk, Hs, d->ds, nullptr, 0.0f, d->ds, T, w8 + P.sact, (int64_t)act_bytes(sk, d->ds),
                                     s);
        }
        if (!rc) rc = launch_tokmm(d->shared_dt, d->sd, d->D, d->ds, w8 + P.sact, T, (float *)(w8 + P.sout), s);
        if (rc) return rc;
        hipLaunchKernelGGL(k_pf_sgate, dim3((unsigned)((T + 63) / 64)), dim3(64), 0, s, dv, L, P, w8);
    }
    hipLaunchKernelGGL(k_pf_route, dim3((unsigned)T), dim3(256), 0, s, dv, L, P, w8, ids, w);
    hipLaunchKernelGGL(k_pf_bucket, dim3(1), dim3(256), 0, s, dv, P, w8);
    return tlmh_check(hipGetLastError(), "moe_prefill launch");
}

int launch_moe_prefill_experts(const tlm_hip_moe_desc *d, int64_t T, void *ws, hipStream_t s) {
    if (!d || !d->experts) return tlmh_seterr(TLM_HIP_EINVAL, "moe_prefill: no expert table");
    const tlm_hip_moe_desc dv = *d;
    const WsLayout L = ws_layout(*d);
    const PfLayout P = pf_layout(*d, T);
    uint8_t *w8 = (uint8_t *)ws;
    const dim3 ggu((unsigned)((d->de + 63) / 64), (unsigned)P.MT), gdn((unsigned)((d->D + 127) / 128), (unsigned)P.MT);
    switch (d->expert_dt) {
    case DT_Q4_K: hipLaunchKernelGGL(k_pf_gateup<DT_Q4_K>, ggu, dim3(256), 0, s, dv, L, P, w8); break;
    case DT_Q5_K: hipLaunchKernelGGL(k_pf_gateup<DT_Q5_K>, ggu, dim3(256), 0, s, dv, L, P, w8); break;
    default: hipLaunchKernelGGL(k_pf_gateup<DT_Q6_K>, ggu, dim3(256), 0, s, dv, L, P, w8); break;
    }
    hipLaunchKernelGGL(k_pf_hquant, dim3((unsigned)(T * d->k), (unsigned)(d->de / 256)), dim3(64), 0, s, dv, P, w8);
    switch (d->expert_dt) {
    case DT_Q4_K: hipLaunchKernelGGL(k_pf_down<DT_Q4_K>, gdn, dim3(256), 0, s, dv, P, w8); break;
    case DT_Q5_K: hipLaunchKernelGGL(k_pf_down<DT_Q5_K>, gdn, dim3(256), 0, s, dv, P, w8); break;
    default: hipLaunchKernelGGL(k_pf_down<DT_Q6_K>, gdn, dim3(256), 0, s, dv, P, w8); break;
    }
    return tlmh_check(hipGetLastError(), "moe_prefill launch");
}

int launch_moe_prefill_combine(const tlm_hip_moe_desc *d, float *h, int64_t T, void *ws, hipStream_t s) {
    const tlm_hip_moe_desc dv = *d;
    const PfLayout P = pf_layout(*d, T);
    hipLaunchKernelGGL(k_pf_combine, dim3((unsigned)((d->D + 1023) / 1024), (unsigned)T), dim3(256), 0, s, dv, P, h,
                       (uint8_t *)ws);
    return tlmh_check(hipGetLastError(), "moe_prefill launch");
}

int launch_moe_prefill(const tlm_hip_moe_desc *d, float *h, int64_t T, int32_t *ids, float *w, void *ws,
                       hipStream_t s) {
    if (int rc = moe_prefill_check(d, h, T, ws, true)) return rc;
    int rc = launch_moe_prefill_route(d, h, T, ids, w, ws, s);
    if (!rc) rc = launch_moe_prefill_experts(d, T, ws, s);
    if (!rc) rc = launch_moe_prefill_combine(d, h, T, ws, s);
    return rc;
}
