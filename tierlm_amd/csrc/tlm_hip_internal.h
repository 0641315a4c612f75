/* tlm_hip_internal.h - shared device helpers and internal launch API of
 * libtlm_hip.so (gfx950).  Not installed; the public ABI is include/tlm_hip.h. */
#ifndef TLM_HIP_INTERNAL_H
#define TLM_HIP_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <functional>

#include "../../include/tlm_hip.h"

/* tlm_dtype codes (src/lib/tlm_quant.h:31-42) */
enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2, DT_Q8_0 = 8, DT_Q4_K = 12, DT_Q5_K = 13,
       DT_Q6_K = 14, DT_Q8_K = 15 };

/* Rows per tile of the packed layout: a wave covers one block column of one
 * tile with 4 lanes per (row, block) for the 256-value formats. */
#define TILE_ROWS 16

/* Threads per group of the streaming kernels: their launch bound and the size
 * they are always launched with.  A constant, because blockDim.x is read
 * through a vector memory load whose wait also waits for every load issued
 * before it. */
#define GROUP_THREADS 256

/* ---- host-side error plumbing (tlm_hip.cpp) ----------------------------- */
int tlmh_seterr(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int tlmh_check(hipError_t e, const char *what);
#define HIPCHK(call) do { hipError_t _e = (call); if (_e != hipSuccess) return tlmh_check(_e, #call); } while (0)

/* ---- format geometry (host + device) ------------------------------------ */
__host__ __device__ static inline int dt_block_values(int dt) {
    return dt == DT_F32 ? 1 : dt == DT_Q8_0 ? 32 : (dt == DT_Q4_K || dt == DT_Q5_K || dt == DT_Q6_K || dt == DT_Q8_K) ? 256 : 0;
}
__host__ __device__ static inline int dt_block_bytes(int dt) {
    return dt == DT_F32 ? 4 : dt == DT_Q8_0 ? 34 : dt == DT_Q4_K ? 144 : dt == DT_Q5_K ? 176
         : dt == DT_Q6_K ? 210 : dt == DT_Q8_K ? 292 : 0;
}
__host__ __device__ static inline int dt_act_kind(int dt) {
    return (dt == DT_Q4_K || dt == DT_Q5_K || dt == DT_Q6_K || dt == DT_Q8_K) ? DT_Q8_K
         : dt == DT_Q8_0 ? DT_Q8_0 : DT_F32;
}
__host__ __device__ static inline size_t act_bytes(int kind, int64_t n) {
    if (n < 0) return 0;
    return kind == DT_Q8_K ? (size_t)((n + 255) / 256) * 292
         : kind == DT_Q8_0 ? (size_t)((n + 31) / 32) * 36
         : kind == DT_F32 ? (size_t)n * 4 : 0;
}
static inline int dt_int_ok(int dt) {
    return dt == DT_Q8_0 || dt == DT_Q4_K || dt == DT_Q5_K || dt == DT_Q6_K || dt == DT_Q8_K;
}

/* ---- device helpers ----------------------------------------------------- */
/* binary16 -> binary32 built from the bit fields: exact for every code,
 * subnormals included, NaN payload kept and quieted (src/lib/tlm_quant.c:118-128). */
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    /* integer operations and selects only, so the compiler keeps it
     * branch-free and a kernel's items stay in one basic block; a subnormal
     * m * 2^-24 is normalised through its leading bit p: exponent p + 103,
     * mantissa the bits below p */
    const uint32_t s = (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    const uint32_t mnz = 0u - (uint32_t)(m != 0u), e31 = 0u - (uint32_t)(e == 31u), e0 = 0u - (uint32_t)(e == 0u);
    const uint32_t special = s | 0x7F800000u | (m << 13) | (mnz & 0x00400000u);
    const uint32_t p = 31u - (uint32_t)__clz((int)(m | 1u));
    const uint32_t sub = s | ((((p + 103u) << 23) | ((m << (23u - p)) & 0x7FFFFFu)) & mnz);
    const uint32_t norm = s | ((e + 112u) << 23) | (m << 13);
    return __uint_as_float((special & e31) | (sub & e0) | (norm & ~(e31 | e0)));
}

/* Round half to even via 1.5*2^23, clamp to [lo, hi], NaN -> 0
 * (src/lib/tlm_quant.c:233-243).  Built with -ffp-contract=off. */
__device__ __forceinline__ int rne_clamp(float v, int lo, int hi) {
    /* branch-free: the clamped bounds are integers, which the magic-number
     * rounding returns unchanged */
    const float t = v != v ? 0.0f : fminf(fmaxf(v, (float)lo), (float)hi);
    const float magic = 12582912.0f;
    return (int)((t + magic) - magic);
}

/* e^x as the reference computes it: libm's expf (src/lib/tlm_model.c:171-172,
 * 705, 806, 823), which on glibc 2.27+ is the published ARM optimized-routines
 * algorithm (Szabolcs Nagy, 2017): x * 32 / ln 2 = k + r with k rounded to the
 * nearest integer through the 1.5 * 2^52 shift, 2^(k/32) from a 32-entry table
 * of 2^(i/32) with the exponent of i/32 taken out, 2^(r/32) from a cubic, all
 * in double, rounded once to float.  The x86-64 FMA build fuses x * 32/ln 2 into
 * both the shift and r; the fused form is the one that reproduces that libm
 * bit for bit (every one of the 2^32 inputs, checked against glibc 2.35; the
 * polynomial's own fusions do not change any result).  Not correctly rounded:
 * about 8 in 10^5 results differ from exp in double rounded to float. */
#define TLM_EXP2_TAB                                                                                     \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,          \
     0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,          \
     0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,          \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,          \
     0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,          \
     0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,          \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,          \
     0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}
__device__ static const uint64_t tlm_exp2_tab[32] = TLM_EXP2_TAB;
/* tab(i) returns entry i of the table (i < 32) */
template <class Tab> __device__ __forceinline__ float expf_ref_with(float x, const Tab &tab) {
    /* branch-free: the main path for every input (out-of-range ones give
     * values that the selects below replace; the table index stays in range) */
    const double InvLn2N = 0x1.71547652b82fep+0 * 32.0, Shift = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / 32768.0, C1 = 0x1.ebfce50fac4f3p-3 / 1024.0,
                 C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = __builtin_fma(InvLn2N, xd, Shift);
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= Shift;
    const double r = __builtin_fma(InvLn2N, xd, -kd);
    const double s = __longlong_as_double((long long)(tab((int)(ki % 32)) + (ki << 47)));
    const double z = __builtin_fma(C0, r, C1), r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    float v = (float)(y * s);
    v = x > 0x1.62e42ep6f ? __builtin_inff() : v;   /* overflow */
    v = x < -0x1.9fe368p6f ? 0.0f : v;              /* underflow (and -inf) */
    return x != x ? x + x : v;
}
__device__ __forceinline__ float expf_ref(float x) {
    return expf_ref_with(x, [](int i) { return tlm_exp2_tab[i]; });
}
/* The same table held by a wave's lanes (lane l keeps entry l mod 32), for
 * kernels whose exponentials should not wait on a global read: a lookup is
 * two cross-lane reads.  Every lane of the wave must take part in a lookup. */
struct ExpTabLanes {
    uint32_t lo, hi;
    __device__ __forceinline__ void load() {
        const uint64_t v = tlm_exp2_tab[__lane_id() & 31];
        lo = (uint32_t)v;
        hi = (uint32_t)(v >> 32);
    }
    __device__ __forceinline__ uint64_t operator()(int i) const {
        return ((uint64_t)(uint32_t)__shfl((int)hi, i, 64) << 32) | (uint32_t)__shfl((int)lo, i, 64);
    }
};

/* Address-space qualified pointers.  Pointers that travel through structs,
 * tables or lambdas lose their address space and compile to flat_* accesses,
 * which count against both the vector-memory and the LDS wait counters; the
 * hot loops therefore name global (1) and LDS (3) explicitly. */
#define GAS __attribute__((address_space(1)))
#define LAS __attribute__((address_space(3)))
/* plain clang vectors: loadable through qualified pointers (HIP's uint4 is not) */
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

/* 4 x int8 dot with int32 accumulate (v_dot4_i32_i8): exact. */
__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

__device__ __forceinline__ int wave_lane() { return (int)__lane_id(); }

/* ---- wave reductions over DPP -------------------------------------------
 * Within each 16-lane row: xor-1 and xor-2 quad permutes, then the half-row
 * and row mirrors (lane i <-> 7-i, i <-> 15-i) pair whole quads and halves,
 * so every lane ends with its row's value; the four rows are then combined
 * from lanes 0, 16, 32, 48 through readlane, which leaves the result uniform.
 * A DPP move costs one VALU op, against an LDS round trip for a shuffle. */
enum { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140 };

template <int CTRL> __device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL> __device__ __forceinline__ float dpp_f32(float v) {
    return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(v)));
}
template <int CTRL> __device__ __forceinline__ double dpp_f64(double v) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const uint32_t lo = dpp_u32<CTRL>((uint32_t)b), hi = dpp_u32<CTRL>((uint32_t)(b >> 32));
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ float rdlane_f32(float v, int l) {
    return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), l));
}
__device__ __forceinline__ double rdlane_f64(double v, int l) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
/* max over the wave (no NaN inputs) */
__device__ __forceinline__ float wave_max_f32(float v) {
    float o;
    o = dpp_f32<DPP_XOR1>(v);        v = o > v ? o : v;
    o = dpp_f32<DPP_XOR2>(v);        v = o > v ? o : v;
    o = dpp_f32<DPP_HALF_MIRROR>(v); v = o > v ? o : v;
    o = dpp_f32<DPP_MIRROR>(v);      v = o > v ? o : v;
    const float a = rdlane_f32(v, 0), b = rdlane_f32(v, 16), c = rdlane_f32(v, 32), d = rdlane_f32(v, 48);
    const float ab = b > a ? b : a, cd = d > c ? d : c;
    return cd > ab ? cd : ab;
}
/* max / or over aligned groups of WIDTH lanes (2, 4, 8, 16 or 64), uniform in the group */
template <int WIDTH> __device__ __forceinline__ uint32_t group_max_u32(uint32_t v) {
    uint32_t o;
    if (WIDTH >= 2) { o = dpp_u32<DPP_XOR1>(v); v = o > v ? o : v; }
    if (WIDTH >= 4) { o = dpp_u32<DPP_XOR2>(v); v = o > v ? o : v; }
    if (WIDTH >= 8) { o = dpp_u32<DPP_HALF_MIRROR>(v); v = o > v ? o : v; }
    if (WIDTH >= 16) { o = dpp_u32<DPP_MIRROR>(v); v = o > v ? o : v; }
    if (WIDTH == 64) {
        const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
        const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
        const uint32_t ab = a > b ? a : b, cd = c > d ? c : d;
        v = ab > cd ? ab : cd;
    }
    return v;
}
template <int WIDTH> __device__ __forceinline__ uint32_t group_or_u32(uint32_t v) {
    if (WIDTH >= 2) v |= dpp_u32<DPP_XOR1>(v);
    if (WIDTH >= 4) v |= dpp_u32<DPP_XOR2>(v);
    if (WIDTH >= 8) v |= dpp_u32<DPP_HALF_MIRROR>(v);
    if (WIDTH >= 16) v |= dpp_u32<DPP_MIRROR>(v);
    if (WIDTH == 64)
        v = ((uint32_t)__builtin_amdgcn_readlane((int)v, 0) | (uint32_t)__builtin_amdgcn_readlane((int)v, 16)) |
            ((uint32_t)__builtin_amdgcn_readlane((int)v, 32) | (uint32_t)__builtin_amdgcn_readlane((int)v, 48));
    return v;
}

/* sum over the wave, fixed tree: ((row0 + row1) + (row2 + row3)) */
__device__ __forceinline__ double wave_sum_f64(double v) {
    v += dpp_f64<DPP_XOR1>(v);
    v += dpp_f64<DPP_XOR2>(v);
    v += dpp_f64<DPP_HALF_MIRROR>(v);
    v += dpp_f64<DPP_MIRROR>(v);
    return (rdlane_f64(v, 0) + rdlane_f64(v, 16)) + (rdlane_f64(v, 32) + rdlane_f64(v, 48));
}
/* ---- launchers (defined in the .hip files) ------------------------------ */
int launch_quantize_act(int kind, const float *x, int64_t n, void *dst, hipStream_t s);
int launch_expf(const float *x, float *y, int64_t n, hipStream_t s);
int launch_stream_read(const void *p, size_t bytes, uint32_t *sink, hipStream_t s);
int launch_matvec_plain(int dt, const void *W, size_t row_bytes, const void *act, float *y,
                        int64_t n, int64_t r0, int64_t r1, hipStream_t s);
int launch_nan_fill(float *y, int64_t count, hipStream_t s);
size_t packed_bytes(int dt, int64_t rows, int64_t n);
int launch_pack(int dt, const void *src, size_t row_bytes, int64_t rows, int64_t n, void *dst, hipStream_t s);
int launch_matvec_packed(int dt, const void *Wp, int64_t rows, int64_t n, const void *act, float *y,
                         hipStream_t s);
int launch_mv_job(const tlm_hip_seg *segs, int nseg, hipStream_t s);
/* ntok vectors of n floats (row stride xstride floats): rmsnorm with w (NULL:
 * none) then the activation quantiser of kind (Q8_0 = a8, or Q8_K), exactly
 * as the decode GEMV's prologue computes it, into the reference layout */
int launch_tok_norm_act(int kind, const float *x, int64_t xstride, const float *w, float eps, int64_t n,
                        int64_t ntok, void *out, int64_t ostride, hipStream_t s);
/* up to MV_SEGS packed matrices of one dtype and width n in one launch, one
 * shared activation; accum: y += W x.  With nx set, every group computes the
 * activation itself, quantising rmsnorm(nx) * nw (eps), or nx itself when nw
 * is null, instead of reading act; with
 * keys set (one segment), group t also stores the greedy key of its rows
 * (the maximum of argmax_key) at keys[t]. */
#define MV_SEGS 4
struct MvSegs {
    const uint8_t *W[MV_SEGS];
    int64_t rows[MV_SEGS], tile_end[MV_SEGS];
    float *y[MV_SEGS];
    const float *nx, *nw;
    unsigned long long *keys;
    float eps;
    int n, accum;
};
struct MvNorm {
    const float *x, *w;
    float eps;
};
int launch_mv_segs(int dt, int64_t n, const void *const *W, const int64_t *rows, float *const *y, int nseg, int accum,
                   const void *act, hipStream_t s, const MvNorm *norm = nullptr, unsigned long long *keys = nullptr);
/* greedy key of logit v at index i: larger value first, then lower index; 0
 * for NaN (skipped), so the maximum over a vector decodes to the reference's
 * argmax (first maximum, NaN skipped, 0 if none) - argmax_index */
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t i) {
    if (v != v) return 0ull;
    uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);   /* -0 == +0 */
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - i);
}
__host__ __device__ inline int argmax_index(unsigned long long key) {
    return key ? (int)(0xFFFFFFFFu - (uint32_t)key) : 0;
}
size_t moe_prefill_workspace_bytes(const tlm_hip_moe_desc *d, int64_t T);
int launch_moe_prefill(const tlm_hip_moe_desc *d, float *h, int64_t T, int32_t *ids, float *w, void *ws,
                       hipStream_t s);
int launch_moe_prefill_route(const tlm_hip_moe_desc *d, float *h, int64_t T, int32_t *ids, float *w, void *ws,
                             hipStream_t s);
int launch_moe_prefill_experts(const tlm_hip_moe_desc *d, int64_t T, void *ws, hipStream_t s);
int launch_moe_prefill_combine(const tlm_hip_moe_desc *d, float *h, int64_t T, void *ws, hipStream_t s);
int launch_tokmm(int dt, const void *Wp, int64_t rows, int64_t n, const void *act, int64_t ntok, float *Y,
                 hipStream_t s);
/* up to 4 matrices of one dtype and width n against the same ntok tokens in
 * one launch (the q / k / v of a prefill chunk) */
int launch_tokmm_segs(int dt, int nseg, const void *const *W, const int64_t *rows, int64_t n, const void *act,
                      int64_t ntok, float *const *Y, hipStream_t s);
size_t moe_workspace_bytes(const tlm_hip_moe_desc *d);
int launch_moe_layer(const tlm_hip_moe_desc *d, float *h, int32_t *ids, float *w, void *ws, hipStream_t s);
int launch_moe_phase(const tlm_hip_moe_desc *d, int phase, float *h, int32_t *ids, float *w, void *ws,
                     hipStream_t s);
int launch_moe_route(const tlm_hip_moe_desc *d, const float *h, int32_t *ids, float *w, void *ws, hipStream_t s);
size_t moe_route_offset(const tlm_hip_moe_desc *d);
/* The routing of a block and its routed experts' packed matrices, given by
 * the caller (the slot cache knows them before the block runs): rank r's
 * gate / up / down at p[3r], p[3r + 1], p[3r + 2].  on = 0: the block routes
 * itself and reads its expert table. */
struct MoeGiven {
    const uint8_t *p[3 * 32];
    float w[32];
    int32_t ids[32];
    int32_t on;
};
int launch_moe_phase_given(const tlm_hip_moe_desc *d, int phase, float *h, void *ws, const MoeGiven *gv,
                           hipStream_t s);
/* The routed experts sit in slots of one arena: rank r's slot index is
 * slot[r] (device memory, written by an earlier launch on the stream), its
 * gate / up / down at arena + slot[r] * slot_bytes + off[0 / 1 / 2].  The
 * routing (ids, weights) is already in the block's workspace. */
struct MoeSlots {
    const int32_t *slot;
    const uint8_t *arena;
    uint64_t slot_bytes;
    uint64_t off[3];
};
int launch_moe_phase_slots(const tlm_hip_moe_desc *d, int phase, float *h, void *ws, const MoeSlots *ms,
                           hipStream_t s);
/* The export launch's device-side slot resolution (tab == NULL: none):
 * after routing, the main route's group reads each routed expert's slot from
 * tab (the layer's row of the store's expert -> slot table, in mapped host
 * memory; -1 while the expert is not resident or its load has not landed).
 * All of them valid: it writes them to slot_out[0..k) and stores 1 at
 * report; otherwise slot_out[0..k) = -1 and report = 0 (the blocks reading
 * slot_out then do nothing, and the caller runs the layer itself).  The
 * report is stored before the export's sequence word.  Nothing waits. */
struct RouteDev {
    const int32_t *tab;
    int32_t *slot_out;
    uint32_t *report;
    int32_t n_slots;
};
int launch_moe_routes_host(const tlm_hip_moe_desc *const *d, void *const *ws, int n, const float *h,
                           uint32_t *host, int seq_off, uint32_t seq, hipStream_t s, const RouteDev *rd = nullptr);
/* one thread stores v at *entry (release, system scope): a load's last step */
int launch_publish_slot(int32_t *entry, int32_t v, hipStream_t s);
/* tlm_hip_moe_stack_store's loop (hip_store.hip); before(l), when given,
 * enqueues what precedes layer l's router (a model's attention) and returns 0
 * or an error; descs' expert tables are not used; descs[l] is the store's
 * layer layer0 + l (a model whose first layers are dense FFNs), o's per-layer
 * arrays start at descs[0]'s layer */
int moe_stack_run(const tlm_hip_moe_desc *descs, int n_layers, tlm_hip_store *s, float *h,
                  const tlm_hip_stack_opts *o, int32_t *ids_out, float *w_out, void *workspace, void *stream,
                  const std::function<int(int)> &before, int layer0);

#endif
