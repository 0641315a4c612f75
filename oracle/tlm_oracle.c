/* tlm_oracle.c - CPU restatement of the reference's quantised-MoE decode path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker of the HIP path (tests/, smoke(),
 * bench.py's cpu_baseline).  Never linked into tierlm_amd.
 *
 * Built with -ffp-contract=off and without fast-math: every float operation
 * below is one IEEE operation in the order written, exactly as the reference
 * is built (reference Makefile:32).
 *
 * How each part is pinned (a plausible slip must fail one of these):
 *   f16 <-> f32        exhaustive over all 65536 codes against the f16 layout
 *                      rules + KATs (tests/test_oracle_formats.py) and against
 *                      the compiled reference (tests/test_oracle_vs_ref.py).
 *   layouts, row bytes reference KATs (tests/test_quant.c:59-93 there).
 *   quantize_act       reference KATs (tests/test_quant.c:434-536 there) +
 *                      byte-equality with the compiled reference + golden
 *                      fixtures (tests/golden/).
 *   weight quantisers  no closed form: byte-equality with the compiled
 *                      reference on seeded rows + golden fixtures, and the
 *                      element-order KATs (tests/test_quant.c:396-425 there).
 *   dots / matvec      bit-equality with the compiled reference (scalar and
 *                      SIMD tiers) over the reference's edge-case generators,
 *                      + closed form: |dot - sum deq(w)*deq(x)| < 2e-6 sum|w x|
 *                      in double (tests/test_quant.c:540-583 there), + brute
 *                      force of the integer block sums on tiny inputs.
 *   rmsnorm/route/topk closed forms (softmax sums to 1, top-k order, ties to
 *                      the lowest id, NaN skipped, renormalisation) + a float64
 *                      numpy restatement; the reference keeps these static in
 *                      tlm_model.c, so no compiled entry point exists.
 *   moe_layer          composition of the above, checked against a numpy
 *                      float64 MoE on dequantised weights within the
 *                      quantisation error bound, and against the compiled
 *                      reference kernels driven by ref_moe.c (bit-exact).
 */
#include "tlm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#if defined(FLT_EVAL_METHOD) && FLT_EVAL_METHOD != 0
#error "the oracle needs FLT_EVAL_METHOD == 0"
#endif

/* ========================================================================
 * formats
 * ====================================================================== */
/* Block geometry: src/lib/tlm_quant.c:52-63. */
int orc_block_values(int dt) {
    switch (dt) {
    case ORC_F32: case ORC_F16: case ORC_BF16: return 1;
    case ORC_Q8_0: return 32;
    case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: case ORC_Q8_K: return 256;
    default: return 0;
    }
}

size_t orc_block_bytes(int dt) {
    switch (dt) {
    case ORC_F32: return 4;
    case ORC_F16: case ORC_BF16: return 2;
    case ORC_Q8_0: return 34;
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    case ORC_Q8_K: return 292;
    default: return 0;
    }
}

/* src/lib/tlm_quant.c:106-110 */
size_t orc_row_bytes(int dt, int64_t n) {
    int bv = orc_block_values(dt);
    if (bv == 0 || n < 0 || n % bv) return 0;
    return (size_t)(n / bv) * orc_block_bytes(dt);
}

/* src/lib/tlm_quant.c:689-697: partial blocks round up. */
size_t orc_qact_bytes(int kind, int64_t n) {
    if (n < 0) return 0;
    if (kind == ORC_Q8_K) return (size_t)((n + 255) / 256) * 292;
    if (kind == ORC_Q8_0) return (size_t)((n + 31) / 32) * 36;
    if (kind == ORC_F32) return (size_t)n * 4;
    return 0;
}

/* src/lib/tlm_quant.c:709-715 */
int orc_act_kind_for(int dt) {
    if (dt == ORC_Q4_K || dt == ORC_Q5_K || dt == ORC_Q6_K || dt == ORC_Q8_K) return ORC_Q8_K;
    if (dt == ORC_Q8_0) return ORC_Q8_0;
    return ORC_F32;
}

static inline uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float float_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline float rdf16(const uint8_t *p) { return orc_f16_to_f32(rd16(p)); }
static inline float rdf32(const uint8_t *p) { float f; memcpy(&f, p, 4); return f; }
static inline void wr16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* IEEE binary16 -> binary32, exact (src/lib/tlm_quant.c:118-128): NaN keeps
 * its payload and is made quiet; subnormals scale by 2^-24. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 31) return float_of(s | 0x7F800000u | (m << 13) | (m ? 0x00400000u : 0u));
    if (e == 0) return float_of(bits_of((float)m * 0x1p-24f) | s);
    return float_of(s | ((e + 127u - 15u) << 23) | (m << 13));
}

/* binary32 -> binary16, round to nearest even (src/lib/tlm_quant.c:130-151). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x = bits_of(f);
    uint16_t s = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t a = x & 0x7FFFFFFFu;
    if (a >= 0x7F800000u)                       /* inf, or NaN with payload kept quiet */
        return a == 0x7F800000u ? (uint16_t)(s | 0x7C00u) : (uint16_t)(s | 0x7E00u | ((a >> 13) & 0x3FFu));
    if (a >= 0x477FF000u) return (uint16_t)(s | 0x7C00u);   /* rounds past 65504 */
    if (a < 0x38800000u) {                      /* result is subnormal or zero */
        if (a <= 0x33000000u) return s;         /* at most half the smallest subnormal */
        uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;
        uint32_t sh = 126u - (a >> 23);         /* 14..24 */
        uint32_t q = mant >> sh, rest = mant & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        q += (rest > half) || (rest == half && (q & 1u));
        return (uint16_t)(s | q);
    }
    uint32_t r = a - ((127u - 15u) << 23);      /* rebias the exponent */
    uint32_t q = r >> 13, rest = r & 0x1FFFu;
    q += (rest > 0x1000u) || (rest == 0x1000u && (q & 1u));
    return (uint16_t)(s | q);
}

/* ========================================================================
 * quantisers
 * ====================================================================== */
/* Round half to even through the 1.5*2^23 magic constant, then clamp;
 * NaN gives 0 (src/lib/tlm_quant.c:233-243). */
static inline int rne_clamp(float v, int lo, int hi) {
    if (v != v) return 0;
    if (v <= (float)lo) return lo;
    if (v >= (float)hi) return hi;
    const float magic = 12582912.0f;
    return (int)((v + magic) - magic);
}

/* 12-byte 6-bit scale/min field -> sc[0..7], mn[0..7]
 * (src/lib/tlm_quant.c:253-261, layout at :246-252). */
static void kq_scales(const uint8_t *s12, uint8_t sc[8], uint8_t mn[8]) {
    for (int j = 0; j < 4; j++) {
        sc[j] = s12[j] & 63;
        mn[j] = s12[4 + j] & 63;
        sc[4 + j] = (uint8_t)((s12[8 + j] & 15) | ((s12[j] >> 6) << 4));
        mn[4 + j] = (uint8_t)((s12[8 + j] >> 4) | ((s12[4 + j] >> 6) << 4));
    }
}

/* src/lib/tlm_quant.c:263-269 */
static void kq_scales_pack(const uint8_t sc[8], const uint8_t mn[8], uint8_t *s12) {
    for (int j = 0; j < 4; j++) {
        s12[j] = (uint8_t)((sc[j] & 63) | ((sc[4 + j] >> 4) << 6));
        s12[4 + j] = (uint8_t)((mn[j] & 63) | ((mn[4 + j] >> 4) << 6));
        s12[8 + j] = (uint8_t)((sc[4 + j] & 15) | ((mn[4 + j] & 15) << 4));
    }
}

/* Q8_0 weights (src/lib/tlm_quant.c:276-287): d = amax/127 as f16, codes
 * from the unrounded reciprocal. */
static void q8_0_block(const float *x, uint8_t *blk) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) { float a = fabsf(x[i]); if (a > amax) amax = a; }
    float d = amax / 127.0f;
    if (d > 65504.0f) d = 65504.0f;
    float id = d > 0.0f ? 1.0f / d : 0.0f;
    wr16(blk, orc_f32_to_f16(d));
    for (int i = 0; i < 32; i++) blk[2 + i] = (uint8_t)(int8_t)rne_clamp(x[i] * id, -127, 127);
}

/* Affine fit x ~ a*L - m over L in [0, nmax], m >= 0: a start from the
 * min/max range, then 21 candidate inverse scales each solved by 2-parameter
 * least squares, lowest squared error wins (src/lib/tlm_quant.c:293-333).
 * The float expressions keep the reference's evaluation order. */
static float affine_fit(const float *x, int n, int nmax, float *m_out) {
    float lo = x[0], hi = x[0];
    for (int i = 1; i < n; i++) {
        if (x[i] < lo) lo = x[i];
        if (x[i] > hi) hi = x[i];
    }
    if (lo > 0.0f) lo = 0.0f;
    if (!(hi > lo)) { *m_out = -lo; return 0.0f; }
    float range = hi - lo, sx = 0.0f;
    for (int i = 0; i < n; i++) sx += x[i];
    float a_best = (float)nmax > 0 ? range / (float)nmax : 0.0f, b_best = lo, err_best = 0.0f;
    float inv0 = (float)nmax / range;
    for (int i = 0; i < n; i++) {
        int l = rne_clamp(inv0 * (x[i] - lo), 0, nmax);
        float e = a_best * (float)l + b_best - x[i];
        err_best += e * e;
    }
    for (int step = 0; step <= 20; step++) {
        float inv = ((float)nmax - 1.0f + 0.1f * (float)step) / range;
        float s1 = 0.0f, s2 = 0.0f, sxl = 0.0f;
        uint8_t codes[32];
        for (int i = 0; i < n; i++) {
            int l = rne_clamp(inv * (x[i] - lo), 0, nmax);
            codes[i] = (uint8_t)l;
            s1 += (float)l;
            s2 += (float)(l * l);
            sxl += (float)l * x[i];
        }
        float det = (float)n * s2 - s1 * s1;
        if (!(det > 0.0f)) continue;
        float a = ((float)n * sxl - s1 * sx) / det;
        float b = (s2 * sx - s1 * sxl) / det;
        if (b > 0.0f) { b = 0.0f; a = sxl / s2; }
        if (!(a > 0.0f)) continue;
        float err = 0.0f;
        for (int i = 0; i < n; i++) { float e = a * (float)codes[i] + b - x[i]; err += e * e; }
        if (err < err_best) { err_best = err; a_best = a; b_best = b; }
    }
    *m_out = -b_best;
    return a_best;
}

/* Q4_K (nmax 15) / Q5_K (nmax 31) super-block (src/lib/tlm_quant.c:340-381). */
static void kq_affine_block(const float *x, uint8_t *blk, int nmax) {
    float a[8], m[8], amax = 0.0f, mmax = 0.0f;
    for (int s = 0; s < 8; s++) a[s] = affine_fit(x + 32 * s, 32, nmax, &m[s]);
    for (int s = 0; s < 8; s++) {
        if (a[s] > amax) amax = a[s];
        if (m[s] > mmax) mmax = m[s];
    }
    float ia = amax > 0.0f ? 63.0f / amax : 0.0f;
    float im = mmax > 0.0f ? 63.0f / mmax : 0.0f;
    uint8_t sc[8], mn[8];
    for (int s = 0; s < 8; s++) {
        sc[s] = (uint8_t)rne_clamp(ia * a[s], 0, 63);
        mn[s] = (uint8_t)rne_clamp(im * m[s], 0, 63);
    }
    float dsup = amax / 63.0f, msup = mmax / 63.0f;
    if (dsup > 65504.0f) dsup = 65504.0f;
    if (msup > 65504.0f) msup = 65504.0f;
    wr16(blk, orc_f32_to_f16(dsup));
    wr16(blk + 2, orc_f32_to_f16(msup));
    kq_scales_pack(sc, mn, blk + 4);
    float d = rdf16(blk), dmin = rdf16(blk + 2);
    uint8_t L[256];
    for (int s = 0; s < 8; s++) {
        float ds = d * (float)sc[s], ms = dmin * (float)mn[s];
        for (int i = 0; i < 32; i++)
            L[32 * s + i] = (uint8_t)(ds > 0.0f ? rne_clamp((x[32 * s + i] + ms) / ds, 0, nmax) : 0);
    }
    /* element 64c+l -> low nibble of qs[32c+l], 64c+32+l -> high nibble;
     * Q5_K: bit 4 of sub-block element (s, l) is bit s of qh[l]. */
    uint8_t *qs = blk + (nmax == 15 ? 16 : 48);
    if (nmax == 31) memset(blk + 16, 0, 32);
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++) {
            uint8_t lo = L[64 * c + l], hi = L[64 * c + 32 + l];
            qs[32 * c + l] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
            if (nmax == 31) blk[16 + l] |= (uint8_t)(((lo >> 4) << (2 * c)) | ((hi >> 4) << (2 * c + 1)));
        }
}

/* Symmetric fit of 16 values to codes in [-32, 31]: 19 candidate inverse
 * scales around -32/x_extreme, keeping the one with the largest
 * (sum x*L)^2 / sum L^2 (src/lib/tlm_quant.c:387-404). */
static float symmetric_fit(const float *x) {
    float amax = 0.0f, ext = 0.0f;
    for (int i = 0; i < 16; i++) {
        float v = fabsf(x[i]);
        if (v > amax) { amax = v; ext = x[i]; }
    }
    if (!(amax > 1e-30f)) return 0.0f;
    float best = -1.0f, scale = 0.0f;
    for (int step = -9; step <= 9; step++) {
        float inv = -(32.0f + 0.1f * (float)step) / ext;
        float sxl = 0.0f, sll = 0.0f;
        for (int i = 0; i < 16; i++) {
            int l = rne_clamp(inv * x[i], -32, 31);
            sxl += x[i] * (float)l;
            sll += (float)(l * l);
        }
        if (!(sll > 0.0f)) continue;
        float score = sxl * sxl / sll;
        if (score > best) { best = score; scale = sxl / sll; }
    }
    return scale;
}

/* Q6_K element e of a super-block maps to (half h = e/128, quarter q =
 * (e%128)/32, l = e%32): low nibble of ql[64h + 32*(q&1) + l] for q < 2,
 * high nibble for q >= 2, and bits 2q..2q+1 of qh[32h + l] on top
 * (src/lib/tlm_quant.c:406-411, 442-450). */
static inline int q6_code(const uint8_t *blk, int e) {
    int h = e >> 7, q = (e >> 5) & 3, l = e & 31;
    uint8_t nib = blk[64 * h + 32 * (q & 1) + l];
    nib = (q & 2) ? (uint8_t)(nib >> 4) : (uint8_t)(nib & 15);
    int hi = (blk[128 + 32 * h + l] >> (2 * q)) & 3;
    return nib | (hi << 4);
}

/* Q6_K super-block (src/lib/tlm_quant.c:412-451). */
static void q6_k_block(const float *x, uint8_t *blk) {
    float gsc[16], big = 0.0f, big_signed = 0.0f;
    for (int g = 0; g < 16; g++) {
        gsc[g] = symmetric_fit(x + 16 * g);
        if (fabsf(gsc[g]) > big) { big = fabsf(gsc[g]); big_signed = gsc[g]; }
    }
    int8_t *sc = (int8_t *)(blk + 192);
    uint8_t U[256];
    if (!(big > 0.0f)) {
        memset(sc, 0, 16);
        wr16(blk + 208, orc_f32_to_f16(0.0f));
        memset(U, 32, sizeof U);
    } else {
        float inv = -128.0f / big_signed;
        float dsup = 1.0f / inv;
        if (dsup > 65504.0f) dsup = 65504.0f;
        if (dsup < -65504.0f) dsup = -65504.0f;
        wr16(blk + 208, orc_f32_to_f16(dsup));
        float d = rdf16(blk + 208);
        for (int g = 0; g < 16; g++) sc[g] = (int8_t)rne_clamp(inv * gsc[g], -128, 127);
        for (int g = 0; g < 16; g++) {
            float dg = d * (float)sc[g];
            for (int i = 0; i < 16; i++)
                U[16 * g + i] = (uint8_t)((dg != 0.0f ? rne_clamp(x[16 * g + i] / dg, -32, 31) : 0) + 32);
        }
    }
    memset(blk, 0, 192);
    for (int e = 0; e < 256; e++) {
        int h = e >> 7, q = (e >> 5) & 3, l = e & 31;
        int at = 64 * h + 32 * (q & 1) + l;
        blk[at] |= (uint8_t)((q & 2) ? (U[e] & 15) << 4 : (U[e] & 15));
        blk[128 + 32 * h + l] |= (uint8_t)((U[e] >> 4) << (2 * q));
    }
}

/* One activation block (src/lib/tlm_quant.c:458-478): d = amax/127 over the
 * nvalid real values, codes rne(x*127/amax) in [-127, 127], padding codes 0;
 * a NaN gives d = NaN, an infinity d = +inf, both with all-zero codes; a
 * block with amax < 2^-100 scales through double. */
static void act_block(const float *x, int nvalid, int qk, float *d, int8_t *q) {
    float amax = 0.0f;
    int nan = 0, inf = 0;
    for (int i = 0; i < nvalid; i++) {
        float a = fabsf(x[i]);
        if (a != a) nan = 1;
        else if (a == INFINITY) inf = 1;
        else if (a > amax) amax = a;
    }
    memset(q, 0, (size_t)qk);
    if (nan || inf) { *d = nan ? NAN : INFINITY; return; }
    if (!(amax > 0.0f)) { *d = 0.0f; return; }
    *d = amax / 127.0f;
    if (amax >= 0x1p-100f) {
        float id = 127.0f / amax;
        for (int i = 0; i < nvalid; i++) q[i] = (int8_t)rne_clamp(x[i] * id, -127, 127);
    } else {
        double id = 127.0 / (double)amax;
        for (int i = 0; i < nvalid; i++) q[i] = (int8_t)rne_clamp((float)((double)x[i] * id), -127, 127);
    }
}

/* Q8_K: 292-byte blocks, int16 code sums per 16 (src/lib/tlm_quant.c:483-498). */
static void q8_k_row(const float *x, int64_t n, uint8_t *out) {
    for (int64_t b = 0; b * 256 < n; b++) {
        int64_t rest = n - b * 256;
        float d;
        int8_t q[256];
        act_block(x + 256 * b, rest >= 256 ? 256 : (int)rest, 256, &d, q);
        uint8_t *blk = out + 292 * b;
        memcpy(blk, &d, 4);
        memcpy(blk + 4, q, 256);
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int i = 0; i < 16; i++) s += q[16 * g + i];
            wr16(blk + 260 + 2 * g, (uint16_t)(int16_t)s);
        }
    }
}

/* a8 activation blocks (src/lib/tlm_quant.c:500-506). */
static void a8_row(const float *x, int64_t n, uint8_t *out) {
    for (int64_t b = 0; b * 32 < n; b++) {
        int64_t rest = n - b * 32;
        float d;
        int8_t q[32];
        act_block(x + 32 * b, rest >= 32 ? 32 : (int)rest, 32, &d, q);
        memcpy(out + 36 * b, &d, 4);
        memcpy(out + 36 * b + 4, q, 32);
    }
}

/* src/lib/tlm_quant.c:563-587 (formats on this path only). */
int orc_quantize_row(int dt, const float *x, void *dst, int64_t n) {
    int bv = orc_block_values(dt);
    if (bv == 0 || n < 0 || n % bv) return -1;
    uint8_t *o = (uint8_t *)dst;
    int64_t nb = n / bv;
    switch (dt) {
    case ORC_F32: memcpy(o, x, (size_t)n * 4); return 0;
    case ORC_F16: for (int64_t i = 0; i < n; i++) wr16(o + 2 * i, orc_f32_to_f16(x[i])); return 0;
    case ORC_Q8_0: for (int64_t b = 0; b < nb; b++) q8_0_block(x + 32 * b, o + 34 * b); return 0;
    case ORC_Q4_K: for (int64_t b = 0; b < nb; b++) kq_affine_block(x + 256 * b, o + 144 * b, 15); return 0;
    case ORC_Q5_K: for (int64_t b = 0; b < nb; b++) kq_affine_block(x + 256 * b, o + 176 * b, 31); return 0;
    case ORC_Q6_K: for (int64_t b = 0; b < nb; b++) q6_k_block(x + 256 * b, o + 210 * b); return 0;
    case ORC_Q8_K: q8_k_row(x, n, o); return 0;
    default: return -1;
    }
}

/* src/lib/tlm_quant.c:592-675 */
int orc_dequantize_row(int dt, const void *src, float *y, int64_t n) {
    int bv = orc_block_values(dt);
    if (bv == 0 || n < 0 || n % bv) return -1;
    const uint8_t *s = (const uint8_t *)src;
    int64_t nb = n / bv;
    for (int64_t b = 0; b < nb; b++) {
        float *out = y + bv * b;
        if (dt == ORC_F32) { out[0] = rdf32(s + 4 * b); continue; }
        if (dt == ORC_F16) { out[0] = rdf16(s + 2 * b); continue; }
        if (dt == ORC_Q8_0) {
            const uint8_t *blk = s + 34 * b;
            float d = rdf16(blk);
            for (int i = 0; i < 32; i++) out[i] = d * (float)(int8_t)blk[2 + i];
        } else if (dt == ORC_Q8_K) {
            const uint8_t *blk = s + 292 * b;
            float d = rdf32(blk);
            for (int i = 0; i < 256; i++) out[i] = d * (float)(int8_t)blk[4 + i];
        } else if (dt == ORC_Q6_K) {
            const uint8_t *blk = s + 210 * b;
            float d = rdf16(blk + 208);
            for (int e = 0; e < 256; e++)
                out[e] = d * (float)(int8_t)blk[192 + e / 16] * (float)(q6_code(blk, e) - 32);
        } else {   /* Q4_K / Q5_K */
            int q5 = dt == ORC_Q5_K;
            const uint8_t *blk = s + (q5 ? 176 : 144) * b, *qs = blk + (q5 ? 48 : 16);
            uint8_t sc[8], mn[8];
            kq_scales(blk + 4, sc, mn);
            float d = rdf16(blk), dmin = rdf16(blk + 2);
            for (int e = 0; e < 256; e++) {
                int c = e >> 6, hi = (e >> 5) & 1, l = e & 31, sb = e >> 5;
                int code = hi ? qs[32 * c + l] >> 4 : qs[32 * c + l] & 15;
                if (q5) code |= ((blk[16 + l] >> (2 * c + hi)) & 1) << 4;
                out[e] = d * (float)sc[sb] * (float)code - dmin * (float)mn[sb];
            }
        }
    }
    return 0;
}

/* src/lib/tlm_quant.c:699-707 */
void orc_quantize_act(int kind, const float *x, int64_t n, void *dst) {
    if (n <= 0) return;
    if (kind == ORC_Q8_K) q8_k_row(x, n, (uint8_t *)dst);
    else if (kind == ORC_Q8_0) a8_row(x, n, (uint8_t *)dst);
    else if (kind == ORC_F32) memcpy(dst, x, (size_t)n * 4);
}

/* ========================================================================
 * dot products (the numerics contract, src/lib/tlm_quant.h:113-128)
 * ====================================================================== */
/* Integer sums of one weight block against its activation block.
 *   Q8_0 (src/lib/tlm_quant.c:778-792): isum = sum q_w * q_a.
 *   Q6_K (:856-882): isum = sum_g sc[g] * (sum_{16} u*x - 32 * bsums[g]).
 *   Q4_K/Q5_K (:814-842): isum = sum_s sc[s] * sum_{32} code*x,
 *                         msum = sum_s mn[s] * (bsums[2s] + bsums[2s+1]).
 *   Q8_K weight (:886-902): isum = sum q_w * q_a. */
void orc_block_isum(int dt, const void *wblock, const void *act_block, int32_t *isum, int32_t *msum) {
    const uint8_t *w = (const uint8_t *)wblock, *a = (const uint8_t *)act_block;
    int32_t is = 0, ms = 0;
    if (dt == ORC_Q8_0) {
        for (int i = 0; i < 32; i++) is += (int32_t)(int8_t)w[2 + i] * (int8_t)a[4 + i];
    } else if (dt == ORC_Q8_K) {
        for (int i = 0; i < 256; i++) is += (int32_t)(int8_t)w[4 + i] * (int8_t)a[4 + i];
    } else if (dt == ORC_Q6_K) {
        for (int g = 0; g < 16; g++) {
            int32_t gs = 0;
            for (int i = 0; i < 16; i++) gs += q6_code(w, 16 * g + i) * (int8_t)a[4 + 16 * g + i];
            int16_t bs = (int16_t)rd16(a + 260 + 2 * g);
            is += (int32_t)(int8_t)w[192 + g] * (gs - 32 * (int32_t)bs);
        }
    } else if (dt == ORC_Q4_K || dt == ORC_Q5_K) {
        int q5 = dt == ORC_Q5_K;
        const uint8_t *qs = w + (q5 ? 48 : 16);
        uint8_t sc[8], mn[8];
        kq_scales(w + 4, sc, mn);
        for (int sb = 0; sb < 8; sb++) {
            int c = sb >> 1, hi = sb & 1;
            int32_t s = 0;
            for (int l = 0; l < 32; l++) {
                int code = hi ? qs[32 * c + l] >> 4 : qs[32 * c + l] & 15;
                if (q5) code |= ((w[16 + l] >> (2 * c + hi)) & 1) << 4;
                s += code * (int8_t)a[4 + 32 * sb + l];
            }
            is += (int32_t)sc[sb] * s;
            int32_t pair = (int16_t)rd16(a + 260 + 4 * sb) + (int16_t)rd16(a + 262 + 4 * sb);
            ms += (int32_t)mn[sb] * pair;
        }
    }
    *isum = is;
    if (msum) *msum = ms;
}

/* f32 dot: element i feeds lane i mod 32 with fmaf, then the fixed tree
 * (src/lib/tlm_quant.c:721-738). */
static float dot_f32(const float *w, const float *x, int64_t n) {
    float lane[32] = { 0 };
    for (int64_t i = 0; i < n; i++) lane[i & 31] = fmaf(w[i], x[i], lane[i & 31]);
    float t16[16], t8[8], t4[4];
    for (int l = 0; l < 16; l++) t16[l] = lane[l] + lane[l + 16];
    for (int l = 0; l < 8; l++) t8[l] = t16[l] + t16[l + 8];
    for (int l = 0; l < 4; l++) t4[l] = t8[l] + t8[l + 4];
    return (t4[0] + t4[2]) + (t4[1] + t4[3]);
}

/* One row: per block, in ascending order from +0,
 *   acc = fmaf(d_w * d_a, (float)isum, acc)
 *   acc = fmaf(-(dmin_w * d_a), (float)msum, acc)   (Q4_K / Q5_K only). */
static float dot_row(int dt, const uint8_t *w, const uint8_t *a, int64_t n) {
    if (dt == ORC_F32) return dot_f32((const float *)(const void *)w, (const float *)(const void *)a, n);
    int bv = orc_block_values(dt);
    size_t wb = orc_block_bytes(dt), ab = bv == 32 ? 36 : 292;
    float acc = 0.0f;
    for (int64_t b = 0; b < n / bv; b++) {
        const uint8_t *wk = w + wb * b, *ak = a + ab * b;
        int32_t is, ms;
        orc_block_isum(dt, wk, ak, &is, &ms);
        float da = rdf32(ak);
        if (dt == ORC_Q6_K) acc = fmaf(rdf16(wk + 208) * da, (float)is, acc);
        else if (dt == ORC_Q8_K) acc = fmaf(rdf32(wk) * da, (float)is, acc);
        else if (dt == ORC_Q8_0) acc = fmaf(rdf16(wk) * da, (float)is, acc);
        else {
            float sa = rdf16(wk) * da, sm = rdf16(wk + 2) * da;
            acc = fmaf(sa, (float)is, acc);
            acc = fmaf(-sm, (float)ms, acc);
        }
    }
    return acc;
}

static int dot_dtype_ok(int dt) {
    return dt == ORC_F32 || dt == ORC_Q8_0 || dt == ORC_Q4_K || dt == ORC_Q5_K ||
           dt == ORC_Q6_K || dt == ORC_Q8_K;
}

/* src/lib/tlm_quant.c:1104-1112: NaN for a bad dtype or length. */
float orc_vec_dot(int dt, const void *wrow, const void *act, int64_t n) {
    if (!dot_dtype_ok(dt) || n < 0 || n % orc_block_values(dt)) return NAN;
    return dot_row(dt, (const uint8_t *)wrow, (const uint8_t *)act, n);
}

/* src/lib/tlm_quant.c:1119-1143: rows [r0, r1), absolute indexing into y;
 * a bad dtype or length NaN-fills the range. */
void orc_matvec_rows(int dt, const void *W, size_t row_bytes, const void *act,
                     float *y, int64_t n, int64_t r0, int64_t r1) {
    if (!dot_dtype_ok(dt) || n < 0 || n % orc_block_values(dt)) {
        for (int64_t r = r0; r < r1; r++) y[r] = NAN;
        return;
    }
    for (int64_t r = r0; r < r1; r++)
        y[r] = dot_row(dt, (const uint8_t *)W + (size_t)r * row_bytes, (const uint8_t *)act, n);
}

/* ========================================================================
 * decoder glue
 * ====================================================================== */
/* src/lib/tlm_model.c:164-169: sum of squares in double (ascending i),
 * r = 1/sqrtf(mean + eps), out = (x * r) * w. */
void orc_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps) {
    double ss = 0.0;
    for (int64_t i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
    float r = 1.0f / sqrtf((float)(ss / (double)n) + eps);
    for (int64_t i = 0; i < n; i++) out[i] = x[i] * r * w[i];
}

/* e^x as the reference evaluates it: libm's expf itself (src/lib/tlm_model.c:
 * 171-172, 705, 806, 823), over a vector */
void orc_expf_many(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = expf(x[i]);
}

/* The published algorithm behind glibc's expf (2.27+; ARM optimized-routines,
 * math/expf.c, Szabolcs Nagy 2017), restated from its description: x * N/ln 2
 * = k + r, k rounded to the nearest integer through the 1.5 * 2^52 shift, N =
 * 32; 2^(k/N) = 2^(floor(k/N)) * 2^((k mod N)/N) with the 32 values of
 * 2^(i/N) (correctly rounded doubles, exponent of i/N removed, computed by
 * tests/test_oracle_formats.py from exact arithmetic); 2^(r/N) from the cubic
 * C0 r^3 + C1 r^2 + C2 r + 1; everything in double, rounded once.  Overflow
 * above 0x1.62e42ep6, zero below -0x1.9fe368p6.  fused != 0 takes x * N/ln 2
 * into the shift and into r with fma, as the x86-64 FMA build of libm does.
 * The device's exponential is this algorithm with fused = 1. */
static const uint64_t exp2_tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

uint64_t orc_exp2_tab(int i) { return exp2_tab[i & 31]; }

float orc_expf_published(float x, int fused) {
    if (x != x) return x + x;
    if (x > 0x1.62e42ep6f) return INFINITY;
    if (x < -0x1.9fe368p6f) return 0.0f;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32768.0, c1 = 0x1.ebfce50fac4f3p-3 / 1024.0,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x, z = inv_ln2_n * xd;
    double kd = fused ? fma(inv_ln2_n, xd, shift) : z + shift;
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = fused ? fma(inv_ln2_n, xd, -kd) : z - kd;
    const uint64_t t = exp2_tab[ki % 32] + (ki << 47);
    double s;
    memcpy(&s, &t, 8);
    const double p = c0 * r + c1, r2 = r * r;
    double y = c2 * r + 1.0;
    y = p * r2 + y;
    return (float)(y * s);
}

void orc_expf_published_many(const float *x, float *y, int64_t n, int fused) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_expf_published(x[i], fused);
}

/* src/lib/tlm_model.c:171-172 */
float orc_silu(float x) { return x / (1.0f + expf(-x)); }
float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* Top-k by value over unmasked, non-NaN entries; ties keep the lowest id;
 * if nothing is left, the lowest unmasked unused id, else 0
 * (src/lib/tlm_model.c:776-795). */
void orc_topk(const float *v, const uint8_t *mask, int E, int k, int *ids) {
    for (int r = 0; r < k; r++) {
        int pick = -1;
        for (int pass = 0; pass < 2 && pick < 0; pass++) {
            for (int e = 0; e < E; e++) {
                if (mask && mask[e]) continue;
                int used = 0;
                for (int q = 0; q < r; q++) used |= ids[q] == e;
                if (used) continue;
                if (pass == 0) {
                    if (v[e] != v[e]) continue;
                    if (pick < 0 || v[e] > v[pick]) pick = e;
                } else { pick = e; break; }
            }
        }
        ids[r] = pick < 0 ? 0 : pick;
    }
}

/* src/lib/tlm_model.c:798-839 */
void orc_route(int router, const float *logits, const uint8_t *mask, const float *bias,
               int E, int k, float routed_scale, int *ids, float *w) {
    float *p = (float *)malloc(sizeof(float) * (size_t)E);
    float *v = (float *)malloc(sizeof(float) * (size_t)E);
    if (router == 2) {
        for (int e = 0; e < E; e++) {
            p[e] = orc_sigmoid(logits[e]);
            v[e] = p[e] + (bias ? bias[e] : 0.0f);
        }
        orc_topk(v, mask, E, k, ids);
        double s = 0.0;
        for (int r = 0; r < k; r++) s += (double)p[ids[r]];
        float inv = (float)(1.0 / (s + 1e-20));
        for (int r = 0; r < k; r++) w[r] = p[ids[r]] * inv * routed_scale;
        free(p); free(v);
        return;
    }
    float mx = -INFINITY;
    for (int e = 0; e < E; e++)
        if (!(mask && mask[e]) && logits[e] > mx) mx = logits[e];
    double s = 0.0;
    for (int e = 0; e < E; e++) {
        int off = (mask && mask[e]) || logits[e] != logits[e] || mx == -INFINITY;
        p[e] = off ? 0.0f : expf(logits[e] - mx);
        s += (double)p[e];
    }
    float inv = s > 0.0 ? (float)(1.0 / s) : 0.0f;
    for (int e = 0; e < E; e++) p[e] *= inv;
    orc_topk(p, mask, E, k, ids);
    for (int r = 0; r < k; r++) w[r] = p[ids[r]];
    if (router == 0) {
        double t = 0.0;
        for (int r = 0; r < k; r++) t += (double)w[r];
        if (t > 0.0) {
            float it = (float)(1.0 / t);
            for (int r = 0; r < k; r++) w[r] *= it;
        }
    }
    if (routed_scale != 1.0f)
        for (int r = 0; r < k; r++) w[r] *= routed_scale;
    free(p); free(v);
}

/* One SwiGLU FFN: g|u from `gate`/`up` on xb's activation, hh = silu(g)*u,
 * then `down` on hh's activation (src/lib/tlm_model.c:900-938). */
static void swiglu(int dt, const void *gate, const void *up, const void *down, int64_t D, int64_t F,
                   const uint8_t *xact, float *gu, float *hh, uint8_t *hq, float *out) {
    orc_matvec_rows(dt, gate, orc_row_bytes(dt, D), xact, gu, D, 0, F);
    orc_matvec_rows(dt, up, orc_row_bytes(dt, D), xact, gu + F, D, 0, F);
    for (int64_t i = 0; i < F; i++) hh[i] = orc_silu(gu[i]) * gu[F + i];
    int kind = orc_act_kind_for(dt);
    orc_quantize_act(kind, hh, F, hq);
    orc_matvec_rows(dt, down, orc_row_bytes(dt, F), kind == ORC_F32 ? (const void *)hh : hq, out, F, 0, D);
}

/* src/lib/tlm_model.c:940-1055 for a routed layer (no store: every expert is
 * resident, so the batching of run_batch cannot change a value). */
int orc_moe_layer(const orc_moe_desc *d, float *h, int *ids, float *w, orc_moe_trace *tr) {
    int64_t D = d->D, de = d->de, ds = d->ds;
    int k = d->k;
    float *xb = (float *)malloc(sizeof(float) * (size_t)D);
    float *logits = (float *)malloc(sizeof(float) * (size_t)d->E);
    float *ffn = (float *)malloc(sizeof(float) * (size_t)D);
    int64_t F = de > ds ? de : ds;
    float *gu = (float *)malloc(sizeof(float) * (size_t)(2 * F));
    float *hh = (float *)malloc(sizeof(float) * (size_t)F);
    float *eo = (float *)malloc(sizeof(float) * (size_t)D * (size_t)(k > 0 ? k : 1));
    float *s_out = (float *)malloc(sizeof(float) * (size_t)D);
    uint8_t *hq = (uint8_t *)malloc(orc_qact_bytes(ORC_Q8_0, F) + orc_qact_bytes(ORC_Q8_K, F) + 64);
    uint8_t *xe = (uint8_t *)malloc(orc_qact_bytes(ORC_Q8_K, D) + 64);
    uint8_t *xs = (uint8_t *)malloc(orc_qact_bytes(ORC_Q8_0, D) + orc_qact_bytes(ORC_Q8_K, D) + 64);

    orc_rmsnorm(xb, h, d->ffn_norm, D, d->eps);
    if (tr && tr->xb) memcpy(tr->xb, xb, sizeof(float) * (size_t)D);

    /* router on the raw normed vector when f32, else on its activation */
    int rk = orc_act_kind_for(d->router_dt);
    const void *ract = xb;
    if (rk != ORC_F32) { orc_quantize_act(rk, xb, D, xs); ract = xs; }
    orc_matvec_rows(d->router_dt, d->router_w, orc_row_bytes(d->router_dt, D), ract, logits, D, 0, d->E);
    if (tr && tr->logits) memcpy(tr->logits, logits, sizeof(float) * (size_t)d->E);
    orc_route(d->router, logits, d->mask, d->router_bias, d->E, k, d->routed_scale, ids, w);

    int ek = orc_act_kind_for(d->expert_dt);
    const uint8_t *xact = (const uint8_t *)xb;
    if (ek != ORC_F32) { orc_quantize_act(ek, xb, D, xe); xact = xe; }
    size_t hqb = orc_qact_bytes(ek, de);
    for (int r = 0; r < k; r++) {
        int e = ids[r];
        swiglu(d->expert_dt, d->gate[e], d->up[e], d->down[e], D, de, xact, gu, hh, hq, eo + (size_t)r * D);
        if (tr && tr->gu) memcpy(tr->gu + (size_t)r * 2 * de, gu, sizeof(float) * (size_t)(2 * de));
        if (tr && tr->hh) memcpy(tr->hh + (size_t)r * de, hh, sizeof(float) * (size_t)de);
        if (tr && tr->hq && ek != ORC_F32) memcpy(tr->hq + (size_t)r * hqb, hq, hqb);
    }
    if (tr && tr->eo) memcpy(tr->eo, eo, sizeof(float) * (size_t)D * (size_t)k);
    if (ds > 0) {
        int sk = orc_act_kind_for(d->shared_dt);
        const uint8_t *sact = (const uint8_t *)xb;
        if (sk != ORC_F32) { orc_quantize_act(sk, xb, D, xs); sact = xs; }
        swiglu(d->shared_dt, d->sg, d->su, d->sd, D, ds, sact, gu, hh, hq, s_out);
        if (tr && tr->s_out) memcpy(tr->s_out, s_out, sizeof(float) * (size_t)D);
    }

    /* rank-order combine (src/lib/tlm_model.c:1029-1051) */
    for (int64_t i = 0; i < D; i++) ffn[i] = 0.0f;
    for (int r = 0; r < k; r++)
        for (int64_t i = 0; i < D; i++) {
            float c = w[r] * eo[(size_t)r * D + i];
            ffn[i] += c;
        }
    if (ds > 0) {
        float gate = 1.0f;
        if (d->shared_gate_inp) {
            float s = 0.0f;
            for (int64_t i = 0; i < D; i++) s += d->shared_gate_inp[i] * xb[i];
            gate = orc_sigmoid(s);
        }
        for (int64_t i = 0; i < D; i++) ffn[i] += gate * s_out[i];
    }
    if (tr && tr->ffn) memcpy(tr->ffn, ffn, sizeof(float) * (size_t)D);
    for (int64_t i = 0; i < D; i++) h[i] += ffn[i];

    free(xb); free(logits); free(ffn); free(gu); free(hh); free(eo); free(s_out);
    free(hq); free(xe); free(xs);
    return 0;
}
