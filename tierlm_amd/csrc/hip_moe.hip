/* hip_moe.hip - one routed MoE block on device in three launches
 * (src/lib/tlm_model.c:940-1055, run_batch :900-938, route :798-839).
 *
 *   K1 moe_router   ceil(E/8) work-groups.  Each recomputes xb = rmsnorm(h)
 *                   (same tree, so the same bits in every group) and 8 router
 *                   rows in the reference's f32 lane order.  Group 0 also
 *                   publishes xb, quantises it for the experts and for the
 *                   shared expert, evaluates the shared sigmoid gate, and
 *                   clears the arrival counters used by K2 and K3.
 *   K2 moe_gateup   one group per (rank, 16-row tile) of gate and up, then the
 *                   shared expert's tiles.  Every group routes (softmax, top-k,
 *                   renormalise) from the logits itself - identical in all
 *                   groups - so routing needs no launch or counter of its own.
 *                   A group computes its 16 gate rows and 16 up rows,
 *                   h = silu(g) * u, and the last group to finish a
 *                   quantisation block of h (256 or 32 values) quantises it.
 *   K3 moe_down     one group per (rank, 16-row tile) of down, then shared.
 *                   The last group to finish a tile combines the tile's rows
 *                   in ascending rank order, adds the gated shared output and
 *                   updates the residual h.
 *
 * Integer sums, per-row fma chains, activation quantisation and the combine
 * order are the reference's; expf and rmsnorm's double sum of squares are
 * the device's (to about an ulp). */
#include "tlm_hip_internal.h"
#include "tlm_hip_items.h"

#include <math.h>

namespace {

constexpr int MAXK = 32;          /* top-k bound of this implementation */
constexpr int MAXE = 256;         /* expert-count bound (4 per lane of one wave) */

/* ---- workspace layout (256-byte aligned regions) ------------------------- */
struct WsLayout {
    size_t xb, xe, xs, logits, route, hh, hq, eo, so, cnt_h, cnt_t, total;
    int64_t nqe, nqs;             /* quantisation blocks of h per rank / for shared */
};

__host__ __device__ inline size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

__host__ __device__ inline WsLayout ws_layout(const tlm_hip_moe_desc &d) {
    WsLayout L;
    const int ek = dt_act_kind(d.expert_dt), sk = d.ds > 0 ? dt_act_kind(d.shared_dt) : DT_Q8_K;
    const int ebv = ek == DT_Q8_K ? 256 : 32, sbv = sk == DT_Q8_K ? 256 : 32;
    size_t o = 0;
    L.xb = o;     o += al256((size_t)d.D * 4);
    L.xe = o;     o += al256(act_bytes(ek, d.D));
    L.xs = o;     o += al256(act_bytes(sk, d.D));
    L.logits = o; o += al256((size_t)d.E * 4);
    L.route = o;  o += 512;                        /* ids[32] int32, w[32] f32, sgate, ... */
    L.hh = o;     o += al256((size_t)(d.k * d.de + d.ds) * 4);
    L.nqe = (d.de + ebv - 1) / ebv;
    L.nqs = d.ds > 0 ? (d.ds + sbv - 1) / sbv : 0;
    L.hq = o;     o += al256(act_bytes(ek, d.de) * (size_t)d.k + (d.ds > 0 ? act_bytes(sk, d.ds) : 0));
    L.eo = o;     o += al256((size_t)d.k * d.D * 4);
    L.so = o;     o += al256((size_t)d.D * 4);
    L.cnt_h = o;  o += al256((size_t)(d.k * L.nqe + L.nqs) * 4);
    L.cnt_t = o;  o += al256((size_t)((d.D + TILE_ROWS - 1) / TILE_ROWS) * 4);
    L.total = o;
    return L;
}

/* route region: ids at +0 (int32[32]), w at +128 (f32[32]), shared gate at +256 */
__device__ __forceinline__ int32_t *ws_ids(uint8_t *ws, const WsLayout &L) { return (int32_t *)(ws + L.route); }
__device__ __forceinline__ float *ws_w(uint8_t *ws, const WsLayout &L) { return (float *)(ws + L.route + 128); }
__device__ __forceinline__ float *ws_sgate(uint8_t *ws, const WsLayout &L) { return (float *)(ws + L.route + 256); }
/* quantised h of rank r (r == k: shared) */
__host__ __device__ __forceinline__ size_t hq_off(const tlm_hip_moe_desc &d, const WsLayout &L, int r) {
    return L.hq + act_bytes(dt_act_kind(d.expert_dt), d.de) * (size_t)r;
}

/* ---- block-wide helpers --------------------------------------------------- */
__device__ double block_sum_d(double v, double *scratch) {
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) scratch[wave] = v;
    __syncthreads();
    double s = 0.0;
    for (int i = 0; i < nw; i++) s += scratch[i];
    __syncthreads();
    return s;
}

/* xb = rmsnorm(h) * w into LDS (src/lib/tlm_model.c:164-169): sum of squares
 * in double (a fixed tree here), r = 1/sqrtf(mean + eps), (x * r) * w. */
__device__ void rmsnorm_lds(const float *__restrict__ h, const float *__restrict__ nw, int64_t D, float eps,
                            float *xb, double *scratch) {
    double ss = 0.0;
    for (int64_t i = threadIdx.x; i < D; i += blockDim.x) {
        double v = (double)h[i];
        ss += v * v;
    }
    ss = block_sum_d(ss, scratch);
    const float r = 1.0f / sqrtf((float)(ss / (double)D) + eps);
    for (int64_t i = threadIdx.x; i < D; i += blockDim.x) xb[i] = h[i] * r * nw[i];
    __syncthreads();
}

/* One activation block of `cnt` <= block values from `x` into the quantised
 * layout at dst, by one wave (rule of src/lib/tlm_quant.c:458-506). */
__device__ void quant_block_wave(int kind, const float *x, int cnt, uint8_t *dst) {
    const int lane = threadIdx.x & 63;
    const bool q8k = kind == DT_Q8_K;
    const int width = q8k ? 64 : 8;
    const bool mine = q8k || lane < 8;
    const int sub = q8k ? lane : (lane & 7);
    float v[4];
    bool ok[4];
    for (int j = 0; j < 4; j++) {
        int i = 4 * sub + j;
        ok[j] = mine && i < cnt;
        v[j] = ok[j] ? x[i] : 0.0f;
    }
    float amax = 0.0f;
    int nan = 0, inf = 0;
    for (int j = 0; j < 4; j++) {
        if (!ok[j]) continue;
        float a = fabsf(v[j]);
        if (a != a) nan = 1;
        else if (a == INFINITY) inf = 1;
        else if (a > amax) amax = a;
    }
    for (int m = 1; m < 64; m <<= 1) {
        if (m >= width) break;
        float o = __shfl_xor(amax, m, 64);
        amax = o > amax ? o : amax;
        nan |= __shfl_xor(nan, m, 64);
        inf |= __shfl_xor(inf, m, 64);
    }
    uint32_t codes = 0;
    float d;
    if (nan || inf) d = nan ? __uint_as_float(0x7FC00000u) : INFINITY;
    else if (!(amax > 0.0f)) d = 0.0f;
    else {
        d = amax / 127.0f;
        if (amax >= 0x1p-100f) {
            float id = 127.0f / amax;
            for (int j = 0; j < 4; j++)
                if (ok[j]) codes |= (uint32_t)(uint8_t)(int8_t)rne_clamp(v[j] * id, -127, 127) << (8 * j);
        } else {
            double id = 127.0 / (double)amax;
            for (int j = 0; j < 4; j++)
                if (ok[j]) codes |= (uint32_t)(uint8_t)(int8_t)rne_clamp((float)((double)v[j] * id), -127, 127) << (8 * j);
        }
    }
    if (mine) {
        if (sub == 0) *(float *)dst = d;
        *(uint32_t *)(dst + 4 + 4 * sub) = codes;
    }
    if (q8k) {
        int s = (int)(int8_t)(codes & 0xFF) + (int)(int8_t)((codes >> 8) & 0xFF) +
                (int)(int8_t)((codes >> 16) & 0xFF) + (int)(int8_t)(codes >> 24);
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        if ((lane & 3) == 0) *(int16_t *)(dst + 260 + 2 * (lane >> 2)) = (int16_t)s;
    }
}

/* ---- routing by one wave (src/lib/tlm_model.c:776-839) ------------------- */
/* larger value wins; equal values -> lower id; be < 0 means "none yet" */
__device__ __forceinline__ bool better(float v, int e, float bv, int be) {
    return be < 0 || v > bv || (v == bv && e < be);
}

/* ids[0..k) by repeated arg-max over unmasked, non-NaN, unused entries;
 * lane l owns experts l, l+64, l+128, l+192. */
__device__ void topk_wave(const float *v, const uint8_t *mask, int E, int k, int *ids) {
    const int lane = threadIdx.x & 63;
    uint32_t taken = 0;
    for (int r = 0; r < k; r++) {
        float bv = 0.0f;
        int be = -1;
        for (int j = 0; j < 4; j++) {
            int e = lane + 64 * j;
            if (e >= E || ((taken >> j) & 1u) || (mask && mask[e])) continue;
            float x = v[e];
            if (x != x) continue;
            if (better(x, e, bv, be)) { bv = x; be = e; }
        }
        for (int m = 32; m >= 1; m >>= 1) {
            float ov = __shfl_xor(bv, m, 64);
            int oe = __shfl_xor(be, m, 64);
            if (oe >= 0 && better(ov, oe, bv, be)) { bv = ov; be = oe; }
        }
        if (be < 0) {   /* nothing finite left: lowest unmasked unused id, else 0 */
            int cand = 1 << 30;
            for (int j = 0; j < 4; j++) {
                int e = lane + 64 * j;
                if (e >= E || ((taken >> j) & 1u) || (mask && mask[e])) continue;
                cand = e < cand ? e : cand;
            }
            for (int m = 32; m >= 1; m >>= 1) {
                int o = __shfl_xor(cand, m, 64);
                cand = o < cand ? o : cand;
            }
            be = cand == (1 << 30) ? 0 : cand;
        }
        if ((be & 63) == lane) taken |= 1u << (be >> 6);
        if (lane == 0) ids[r] = be;
    }
}

/* ids, w into LDS; p is LDS scratch of 2*MAXE floats. */
__device__ void route_wave(const tlm_hip_moe_desc &d, const float *logits, int *ids, float *w, float *p) {
    const int lane = threadIdx.x & 63, E = d.E, k = d.k;
    const uint8_t *mask = d.mask;
    if (d.router == 2) {   /* sigmoid; bias for selection only; renormalise; scale */
        for (int j = 0; j < 4; j++) {
            int e = lane + 64 * j;
            if (e < E) {
                float s = 1.0f / (1.0f + expf(-logits[e]));
                p[e] = s;
                p[MAXE + e] = s + (d.router_bias ? d.router_bias[e] : 0.0f);
            }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        topk_wave(p + MAXE, mask, E, k, ids);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (lane == 0) {
            double s = 0.0;
            for (int r = 0; r < k; r++) s += (double)p[ids[r]];
            float inv = (float)(1.0 / (s + 1e-20));
            for (int r = 0; r < k; r++) w[r] = p[ids[r]] * inv * d.routed_scale;
        }
        return;
    }
    /* softmax over routable experts, then top-k (router 0 renormalises) */
    float mx = -INFINITY;
    for (int j = 0; j < 4; j++) {
        int e = lane + 64 * j;
        if (e < E && !(mask && mask[e]) && logits[e] > mx) mx = logits[e];
    }
    for (int m = 32; m >= 1; m >>= 1) {
        float o = __shfl_xor(mx, m, 64);
        mx = o > mx ? o : mx;
    }
    double s = 0.0;
    float pv[4];
    for (int j = 0; j < 4; j++) {
        int e = lane + 64 * j;
        pv[j] = 0.0f;
        if (e < E) {
            float l = logits[e];
            bool off = (mask && mask[e]) || l != l || mx == -INFINITY;
            pv[j] = off ? 0.0f : expf(l - mx);
            s += (double)pv[j];
        }
    }
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
    const float inv = s > 0.0 ? (float)(1.0 / s) : 0.0f;
    for (int j = 0; j < 4; j++) {
        int e = lane + 64 * j;
        if (e < E) p[e] = pv[j] * inv;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    topk_wave(p, mask, E, k, ids);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane == 0) {
        for (int r = 0; r < k; r++) w[r] = p[ids[r]];
        if (d.router == 0) {
            double t = 0.0;
            for (int r = 0; r < k; r++) t += (double)w[r];
            if (t > 0.0) {
                float it = (float)(1.0 / t);
                for (int r = 0; r < k; r++) w[r] *= it;
            }
        }
        if (d.routed_scale != 1.0f)
            for (int r = 0; r < k; r++) w[r] *= d.routed_scale;
    }
}

/* ---- tile GEMV inside a fused kernel --------------------------------------
 * Items (b, i) of tile t of a packed matrix spread over the group's waves;
 * results parked in LDS arrays indexed b * 16 + i. */
template <int DT>
__device__ void tile_items(const uint8_t *Wp, int64_t rows, int nb, int64_t t, const XLds &X, int32_t *l_is,
                           int32_t *l_ms, float *l_da, float *l_dm) {
    using F = Packed<DT>;
    constexpr int LPI = F::LPI, IPW = 64 / LPI;
    constexpr bool AFF = DT == DT_Q4_K || DT == DT_Q5_K;
    const int64_t T = (rows + TILE_ROWS - 1) / TILE_ROWS, units = T * nb * TILE_ROWS;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    const int q = lane % LPI, slot = lane / LPI, nitems = nb * TILE_ROWS;
    for (int it = wave * IPW + slot; it - slot < nitems; it += nw * IPW) {
        if (it < nitems) {
            const int b = it / TILE_ROWS, i = it % TILE_ROWS;
            int32_t is, ms;
            float dA, dM;
            F::item(Wp, units, (t * nb + b) * TILE_ROWS + i, b, q, X, is, ms, dA, dM);
            if (q == 0) {
                l_is[it] = is;
                l_da[it] = dA;
                if (AFF) { l_ms[it] = ms; l_dm[it] = dM; }
            }
        }
    }
}

__device__ void tile_items_dt(int dt, const uint8_t *Wp, int64_t rows, int nb, int64_t t, const XLds &X,
                              int32_t *l_is, int32_t *l_ms, float *l_da, float *l_dm) {
    switch (dt) {
    case DT_Q6_K: tile_items<DT_Q6_K>(Wp, rows, nb, t, X, l_is, l_ms, l_da, l_dm); break;
    case DT_Q8_0: tile_items<DT_Q8_0>(Wp, rows, nb, t, X, l_is, l_ms, l_da, l_dm); break;
    case DT_Q4_K: tile_items<DT_Q4_K>(Wp, rows, nb, t, X, l_is, l_ms, l_da, l_dm); break;
    case DT_Q5_K: tile_items<DT_Q5_K>(Wp, rows, nb, t, X, l_is, l_ms, l_da, l_dm); break;
    default: break;
    }
}

/* Row i's float chain over the nb parked blocks, ascending. */
__device__ __forceinline__ float tile_chain(int dt, int nb, int i, const int32_t *l_is, const int32_t *l_ms,
                                            const float *l_da, const float *l_dm) {
    const bool aff = dt == DT_Q4_K || dt == DT_Q5_K;
    float acc = 0.0f;
    for (int b = 0; b < nb; b++) {
        acc = fmaf(l_da[b * TILE_ROWS + i], (float)l_is[b * TILE_ROWS + i], acc);
        if (aff) acc = fmaf(-l_dm[b * TILE_ROWS + i], (float)l_ms[b * TILE_ROWS + i], acc);
    }
    return acc;
}

/* LDS for one matrix's parked items */
__host__ __device__ inline size_t park_bytes(int nb) { return (size_t)nb * TILE_ROWS * 16; }

/* Arrival at a counter: returns true in every thread of the group for the
 * group that completes the count, which also re-arms the counter to 0 so the
 * launch can run again.  Release before the increment, acquire after. */
__device__ bool arrive_last(int32_t *cnt, int need, int *s_flag) {
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence();
        int old = atomicAdd(cnt, 1);
        int last = old == need - 1;
        if (last) atomicExch(cnt, 0);
        *s_flag = last;
    }
    __syncthreads();
    const bool last = *s_flag != 0;
    if (last) __threadfence();
    return last;
}

/* ======================================================================
 * K1: rmsnorm + router + activation quantisation + counter reset
 * ==================================================================== */
__global__ __launch_bounds__(256) void k_moe_router(tlm_hip_moe_desc d, const float *__restrict__ h, uint8_t *ws) {
    extern __shared__ __align__(16) uint8_t lds[];
    const WsLayout L = ws_layout(d);
    float *xb = (float *)lds;
    double *scratch = (double *)(lds + al256((size_t)d.D * 4));
    rmsnorm_lds(h, d.ffn_norm, d.D, d.eps, xb, scratch);

    /* router rows, 8 per group: lane i mod 32 + reduce32 (src/lib/tlm_quant.c:724-738) */
    const int hl = threadIdx.x & 31;
    const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    float r = 0.0f;
    if (row < d.E) {
        const float *wr = d.router_w + row * d.D;
        for (int64_t i = hl; i < d.D; i += 32) r = fmaf(wr[i], xb[i], r);
    }
    float s = r + __shfl_down(r, 16, 32);
    s = s + __shfl_down(s, 8, 32);
    s = s + __shfl_down(s, 4, 32);
    float a = s + __shfl_down(s, 2, 32);
    float res = a + __shfl_down(a, 1, 32);
    if (row < d.E && hl == 0) ((float *)(ws + L.logits))[row] = res;

    if (blockIdx.x != 0) return;
    float *gxb = (float *)(ws + L.xb);
    for (int64_t i = threadIdx.x; i < d.D; i += blockDim.x) gxb[i] = xb[i];
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int ek = dt_act_kind(d.expert_dt), ebv = ek == DT_Q8_K ? 256 : 32;
    for (int64_t b = wave; b < (d.D + ebv - 1) / ebv; b += nw) {
        int64_t rest = d.D - b * ebv;
        quant_block_wave(ek, xb + b * ebv, rest >= ebv ? ebv : (int)rest, ws + L.xe + b * (ebv == 256 ? 292 : 36));
    }
    if (d.ds > 0) {
        const int sk = dt_act_kind(d.shared_dt), sbv = sk == DT_Q8_K ? 256 : 32;
        for (int64_t b = wave; b < (d.D + sbv - 1) / sbv; b += nw) {
            int64_t rest = d.D - b * sbv;
            quant_block_wave(sk, xb + b * sbv, rest >= sbv ? sbv : (int)rest, ws + L.xs + b * (sbv == 256 ? 292 : 36));
        }
        if (threadIdx.x == 0) {
            float g = 1.0f;
            if (d.shared_gate_inp) {   /* sequential float dot (src/lib/tlm_model.c:1043-1046) */
                float acc = 0.0f;
                for (int64_t i = 0; i < d.D; i++) acc += d.shared_gate_inp[i] * xb[i];
                g = 1.0f / (1.0f + expf(-acc));
            }
            *ws_sgate(ws, L) = g;
        }
    }
    int32_t *ch = (int32_t *)(ws + L.cnt_h);
    for (int64_t i = threadIdx.x; i < d.k * L.nqe + L.nqs; i += blockDim.x) ch[i] = 0;
    int32_t *ct = (int32_t *)(ws + L.cnt_t);
    for (int64_t i = threadIdx.x; i < (d.D + TILE_ROWS - 1) / TILE_ROWS; i += blockDim.x) ct[i] = 0;
}

/* ======================================================================
 * K2: route + gate/up + SwiGLU + h quantisation
 * grid: k * de/16 expert tiles (rank-major), then ds/16 shared tiles
 * ==================================================================== */
__global__ __launch_bounds__(256) void k_moe_gateup(tlm_hip_moe_desc d, int32_t *ids_out, float *w_out, uint8_t *ws) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int s_ids[MAXK];
    __shared__ float s_w[MAXK];
    __shared__ float s_p[2 * MAXE];
    __shared__ int s_flag;
    const WsLayout L = ws_layout(d);

    const int64_t te = d.de / TILE_ROWS, nexp = (int64_t)d.k * te;
    const bool shared = (int64_t)blockIdx.x >= nexp;
    const int dt = shared ? d.shared_dt : d.expert_dt;
    const int kind = dt_act_kind(dt);
    const int64_t F = shared ? d.ds : d.de;
    const int r = shared ? d.k : (int)(blockIdx.x / te);
    const int64_t t = shared ? (int64_t)blockIdx.x - nexp : (int64_t)blockIdx.x % te;
    const int nb = (int)(d.D / dt_block_values(dt));

    const XLds X = stage_act(kind, ws + (shared ? L.xs : L.xe), nb, lds);
    const size_t off = (stage_bytes(kind, nb) + 15) & ~(size_t)15;
    int32_t *g_is = (int32_t *)(lds + off), *g_ms = g_is + nb * TILE_ROWS;
    float *g_da = (float *)(g_ms + nb * TILE_ROWS), *g_dm = g_da + nb * TILE_ROWS;
    int32_t *u_is = (int32_t *)(g_dm + nb * TILE_ROWS), *u_ms = u_is + nb * TILE_ROWS;
    float *u_da = (float *)(u_ms + nb * TILE_ROWS), *u_dm = u_da + nb * TILE_ROWS;

    if (!shared && threadIdx.x < 64) {
        route_wave(d, (const float *)(ws + L.logits), s_ids, s_w, s_p);
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            for (int q = 0; q < d.k; q++) {
                ws_ids(ws, L)[q] = s_ids[q];
                ws_w(ws, L)[q] = s_w[q];
                if (ids_out) ids_out[q] = s_ids[q];
                if (w_out) w_out[q] = s_w[q];
            }
        }
    }
    __syncthreads();

    const uint8_t *gW, *uW;
    if (shared) {
        gW = (const uint8_t *)d.sg;
        uW = (const uint8_t *)d.su;
    } else {
        const int e = s_ids[r];
        gW = (const uint8_t *)d.experts[3 * e + 0];
        uW = (const uint8_t *)d.experts[3 * e + 1];
    }
    tile_items_dt(dt, gW, F, nb, t, X, g_is, g_ms, g_da, g_dm);
    tile_items_dt(dt, uW, F, nb, t, X, u_is, u_ms, u_da, u_dm);
    __syncthreads();

    float *hh = (float *)(ws + L.hh) + (size_t)r * d.de;
    if (threadIdx.x < TILE_ROWS) {
        const int i = threadIdx.x;
        float g = tile_chain(dt, nb, i, g_is, g_ms, g_da, g_dm);
        float u = tile_chain(dt, nb, i, u_is, u_ms, u_da, u_dm);
        hh[t * TILE_ROWS + i] = g / (1.0f + expf(-g)) * u;   /* silu(g) * u (src/lib/tlm_model.c:171, 927) */
    }

    /* the group that completes a quantisation block of h quantises it */
    const int qbv = kind == DT_Q8_K ? 256 : 32;
    const int64_t qb = (t * TILE_ROWS) / qbv;
    const int64_t qend = (qb + 1) * qbv < F ? (qb + 1) * qbv : F;
    const int need = (int)((qend - qb * qbv + TILE_ROWS - 1) / TILE_ROWS);
    int32_t *cnt = (int32_t *)(ws + L.cnt_h) + (shared ? (int64_t)d.k * L.nqe : (int64_t)r * L.nqe) + qb;
    if (arrive_last(cnt, need, &s_flag) && threadIdx.x < 64)
        quant_block_wave(kind, hh + qb * qbv, (int)(qend - qb * qbv),
                         ws + hq_off(d, L, r) + (size_t)qb * (qbv == 256 ? 292 : 36));
}

/* ======================================================================
 * K3: down + rank-order combine + residual
 * grid: k * D/16 expert tiles (rank-major), then D/16 shared tiles
 * ==================================================================== */
__global__ __launch_bounds__(256) void k_moe_down(tlm_hip_moe_desc d, float *__restrict__ h, uint8_t *ws) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int s_flag;
    const WsLayout L = ws_layout(d);
    const int64_t TD = (d.D + TILE_ROWS - 1) / TILE_ROWS, nexp = (int64_t)d.k * TD;
    const bool shared = (int64_t)blockIdx.x >= nexp;
    const int dt = shared ? d.shared_dt : d.expert_dt;
    const int kind = dt_act_kind(dt);
    const int64_t F = shared ? d.ds : d.de;
    const int r = shared ? d.k : (int)(blockIdx.x / TD);
    const int64_t t = shared ? (int64_t)blockIdx.x - nexp : (int64_t)blockIdx.x % TD;
    const int nb = (int)(F / dt_block_values(dt));

    const XLds X = stage_act(kind, ws + hq_off(d, L, r), nb, lds);
    const size_t off = (stage_bytes(kind, nb) + 15) & ~(size_t)15;
    int32_t *l_is = (int32_t *)(lds + off), *l_ms = l_is + nb * TILE_ROWS;
    float *l_da = (float *)(l_ms + nb * TILE_ROWS), *l_dm = l_da + nb * TILE_ROWS;
    __syncthreads();

    int e = shared ? 0 : ws_ids(ws, L)[r];
    if (e < 0 || e >= d.E) e = 0;   /* only reachable if phase 3 runs before any phase 2 */
    const uint8_t *W = shared ? (const uint8_t *)d.sd : (const uint8_t *)d.experts[3 * e + 2];
    tile_items_dt(dt, W, d.D, nb, t, X, l_is, l_ms, l_da, l_dm);
    __syncthreads();
    float *out = shared ? (float *)(ws + L.so) : (float *)(ws + L.eo) + (size_t)r * d.D;
    if (threadIdx.x < TILE_ROWS) {
        const int64_t row = t * TILE_ROWS + threadIdx.x;
        float v = tile_chain(dt, nb, threadIdx.x, l_is, l_ms, l_da, l_dm);
        if (row < d.D) out[row] = v;
    }
    const int need = d.k + (d.ds > 0 ? 1 : 0);
    if (!arrive_last((int32_t *)(ws + L.cnt_t) + t, need, &s_flag) || threadIdx.x >= TILE_ROWS) return;

    /* combine in ascending rank order (src/lib/tlm_model.c:1029-1050) */
    const int64_t row = t * TILE_ROWS + threadIdx.x;
    if (row >= d.D) return;
    const float *eo = (const float *)(ws + L.eo);
    const float *w = ws_w(ws, L);
    float ffn = 0.0f;
    for (int q = 0; q < d.k; q++) {
        float c = w[q] * eo[(size_t)q * d.D + row];
        ffn += c;
    }
    if (d.ds > 0) ffn += *ws_sgate(ws, L) * ((const float *)(ws + L.so))[row];
    h[row] += ffn;
}

}  // namespace

size_t moe_workspace_bytes(const tlm_hip_moe_desc *d) { return d ? ws_layout(*d).total : 0; }

static bool moe_dt_ok(int dt) { return dt == DT_Q6_K || dt == DT_Q8_0 || dt == DT_Q4_K || dt == DT_Q5_K; }

int launch_moe_layer(const tlm_hip_moe_desc *d, float *h, int32_t *ids, float *w, void *ws, hipStream_t s) {
    return launch_moe_phase(d, 0, h, ids, w, ws, s);
}

/* phase 0 = all three launches */
int launch_moe_phase(const tlm_hip_moe_desc *d, int phase, float *h, int32_t *ids, float *w, void *ws,
                     hipStream_t s) {
    if (phase < 0 || phase > 3) return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: phase %d", phase);
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
    if (d->ds > 0) {
        const int sbv = dt_block_values(d->shared_dt);
        if (d->ds % TILE_ROWS || d->ds % sbv || d->D % sbv)
            return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: ds=%lld must be a multiple of 16 and of the block",
                               (long long)d->ds);
        if (!d->sg || !d->su || !d->sd) return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: shared matrices missing");
    }
    if (!d->ffn_norm || !d->router_w || !d->experts) return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer: NULL weights");
    const int ek = dt_act_kind(d->expert_dt), sk = d->ds > 0 ? dt_act_kind(d->shared_dt) : ek;
    const int nbe = (int)(d->D / ebv), nbde = (int)(d->de / ebv);
    const int nbs = d->ds > 0 ? (int)(d->D / dt_block_values(d->shared_dt)) : 0;
    const int nbsd = d->ds > 0 ? (int)(d->ds / dt_block_values(d->shared_dt)) : 0;
    size_t lds1 = al256((size_t)d->D * 4) + 64;
    size_t lds2e = ((stage_bytes(ek, nbe) + 15) & ~(size_t)15) + 2 * park_bytes(nbe);
    size_t lds2s = d->ds > 0 ? ((stage_bytes(sk, nbs) + 15) & ~(size_t)15) + 2 * park_bytes(nbs) : 0;
    size_t lds3e = ((stage_bytes(ek, nbde) + 15) & ~(size_t)15) + park_bytes(nbde);
    size_t lds3s = d->ds > 0 ? ((stage_bytes(sk, nbsd) + 15) & ~(size_t)15) + park_bytes(nbsd) : 0;
    size_t lds2 = lds2e > lds2s ? lds2e : lds2s, lds3 = lds3e > lds3s ? lds3e : lds3s;
    if (lds1 > 60 * 1024 || lds2 > 60 * 1024 || lds3 > 60 * 1024)
        return tlmh_seterr(TLM_HIP_EUNSUP, "moe_layer: D=%lld / de=%lld exceed the LDS staging limit",
                           (long long)d->D, (long long)d->de);
    uint8_t *w8 = (uint8_t *)ws;
    const tlm_hip_moe_desc dv = *d;
    const unsigned g1 = (unsigned)((d->E + 7) / 8);
    const unsigned g2 = (unsigned)(d->k * (d->de / TILE_ROWS) + (d->ds > 0 ? d->ds / TILE_ROWS : 0));
    const unsigned g3 = (unsigned)((d->k + (d->ds > 0 ? 1 : 0)) * (d->D / TILE_ROWS));
    if (phase == 0 || phase == 1)
        hipLaunchKernelGGL(k_moe_router, dim3(g1), dim3(256), lds1, s, dv, (const float *)h, w8);
    if (phase == 0 || phase == 2) hipLaunchKernelGGL(k_moe_gateup, dim3(g2), dim3(256), lds2, s, dv, ids, w, w8);
    if (phase == 0 || phase == 3) hipLaunchKernelGGL(k_moe_down, dim3(g3), dim3(256), lds3, s, dv, h, w8);
    return tlmh_check(hipGetLastError(), "moe_layer launch");
}
