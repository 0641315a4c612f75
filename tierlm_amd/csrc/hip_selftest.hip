/* hip_selftest.hip - start-up self-test of the HIP kernels
 * (src/lib/tlm_quant.c:950-1056: fixed pseudo-random rows with finite scale
 * fields, 9 rows x 1024 values, two repetitions, bit-exact against the scalar
 * rule).  The host scalar rule below exists only to check the kernels; no
 * entry point ever computes a result with it.
 *
 * Checked: the device activation quantisers (bytes), the plain-layout matvec
 * and the packed-layout matvec (bits of every row) for F32, Q8_0, Q4_K, Q5_K,
 * Q6_K and Q8_K, and the exponential against this host's libm expf.  Returns
 * the number of failing kernels; bit dt of *mask is set for every dtype whose
 * kernels failed, bit 30 for the exponential. */
#include "tlm_hip_internal.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <vector>

namespace {

float h_f16(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u, u;
    if (e == 31u) u = s | 0x7F800000u | (m << 13) | (m ? 0x00400000u : 0u);
    else if (e == 0u) {
        float v = (float)m * 0x1p-24f;
        memcpy(&u, &v, 4);
        u |= s;
    } else u = s | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &u, 4);
    return f;
}
uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
float rdf(const uint8_t *p) { float f; memcpy(&f, p, 4); return f; }

int h_rne(float v, int lo, int hi) {
    if (v != v) return 0;
    if (v <= (float)lo) return lo;
    if (v >= (float)hi) return hi;
    volatile float t = v + 12582912.0f;
    return (int)(t - 12582912.0f);
}

/* activation rule, src/lib/tlm_quant.c:458-506 */
void h_act(int kind, const float *x, int64_t n, uint8_t *out) {
    const int qk = kind == DT_Q8_K ? 256 : 32, bb = kind == DT_Q8_K ? 292 : 36;
    for (int64_t b = 0; b * qk < n; b++) {
        int nv = (int)(n - b * qk < qk ? n - b * qk : qk);
        const float *v = x + b * qk;
        float amax = 0.0f, d;
        int nan = 0, inf = 0;
        int8_t q[256];
        memset(q, 0, sizeof q);
        for (int i = 0; i < nv; i++) {
            float a = fabsf(v[i]);
            if (a != a) nan = 1; else if (a == INFINITY) inf = 1; else if (a > amax) amax = a;
        }
        if (nan || inf) d = nan ? NAN : INFINITY;
        else if (!(amax > 0.0f)) d = 0.0f;
        else {
            d = amax / 127.0f;
            if (amax >= 0x1p-100f) {
                float id = 127.0f / amax;
                for (int i = 0; i < nv; i++) q[i] = (int8_t)h_rne(v[i] * id, -127, 127);
            } else {
                double id = 127.0 / (double)amax;
                for (int i = 0; i < nv; i++) q[i] = (int8_t)h_rne((float)((double)v[i] * id), -127, 127);
            }
        }
        uint8_t *o = out + b * bb;
        memcpy(o, &d, 4);
        memcpy(o + 4, q, (size_t)qk);
        if (kind == DT_Q8_K)
            for (int g = 0; g < 16; g++) {
                int s = 0;
                for (int i = 0; i < 16; i++) s += q[16 * g + i];
                int16_t s16 = (int16_t)s;
                memcpy(o + 260 + 2 * g, &s16, 2);
            }
    }
}

/* dot rule, src/lib/tlm_quant.c:721-902 */
float h_dot(int dt, const uint8_t *w, const uint8_t *a, int64_t n) {
    if (dt == DT_F32) {
        float r[32] = {0};
        for (int64_t i = 0; i < n; i++) r[i & 31] = fmaf(rdf(w + 4 * i), rdf(a + 4 * i), r[i & 31]);
        float s16[16], s8[8], s4[4];
        for (int l = 0; l < 16; l++) s16[l] = r[l] + r[l + 16];
        for (int l = 0; l < 8; l++) s8[l] = s16[l] + s16[l + 8];
        for (int l = 0; l < 4; l++) s4[l] = s8[l] + s8[l + 4];
        return (s4[0] + s4[2]) + (s4[1] + s4[3]);
    }
    const int bv = dt_block_values(dt), wb = dt_block_bytes(dt), ab = bv == 32 ? 36 : 292;
    float acc = 0.0f;
    for (int64_t b = 0; b < n / bv; b++) {
        const uint8_t *k = w + b * wb, *x = a + b * ab;
        const int8_t *xq = (const int8_t *)(x + 4);
        const float da = rdf(x);
        int32_t is = 0, ms = 0;
        if (dt == DT_Q8_0) {
            for (int i = 0; i < 32; i++) is += (int8_t)k[2 + i] * xq[i];
            acc = fmaf(h_f16(rd16(k)) * da, (float)is, acc);
        } else if (dt == DT_Q8_K) {
            for (int i = 0; i < 256; i++) is += (int8_t)k[4 + i] * xq[i];
            acc = fmaf(rdf(k) * da, (float)is, acc);
        } else if (dt == DT_Q6_K) {
            for (int g = 0; g < 16; g++) {
                int32_t gs = 0;
                for (int j = 0; j < 16; j++) {
                    int e = 16 * g + j, hh = e >> 7, q = (e >> 5) & 3, l = e & 31;
                    int nib = k[64 * hh + 32 * (q & 1) + l];
                    nib = (q & 2) ? nib >> 4 : nib & 15;
                    gs += (nib | (((k[128 + 32 * hh + l] >> (2 * q)) & 3) << 4)) * xq[e];
                }
                int16_t bs;
                memcpy(&bs, x + 260 + 2 * g, 2);
                is += (int8_t)k[192 + g] * (gs - 32 * bs);
            }
            acc = fmaf(h_f16(rd16(k + 208)) * da, (float)is, acc);
        } else {
            const bool q5 = dt == DT_Q5_K;
            const uint8_t *qs = k + (q5 ? 48 : 16), *s12 = k + 4;
            for (int sb = 0; sb < 8; sb++) {
                int c = sb >> 1, hb = sb & 1, sc, mn;
                if (sb < 4) { sc = s12[sb] & 63; mn = s12[4 + sb] & 63; }
                else { sc = (s12[sb + 4] & 15) | ((s12[sb - 4] >> 6) << 4); mn = (s12[sb + 4] >> 4) | ((s12[sb] >> 6) << 4); }
                int32_t s = 0;
                for (int l = 0; l < 32; l++) {
                    int code = hb ? qs[32 * c + l] >> 4 : qs[32 * c + l] & 15;
                    if (q5) code |= ((k[16 + l] >> (2 * c + hb)) & 1) << 4;
                    s += code * xq[32 * sb + l];
                }
                int16_t b0, b1;
                memcpy(&b0, x + 260 + 4 * sb, 2);
                memcpy(&b1, x + 262 + 4 * sb, 2);
                is += sc * s;
                ms += mn * (b0 + b1);
            }
            float sa = h_f16(rd16(k)) * da, sm = h_f16(rd16(k + 2)) * da;
            acc = fmaf(sa, (float)is, acc);
            acc = fmaf(-sm, (float)ms, acc);
        }
    }
    return acc;
}

uint32_t st_rng(uint32_t *s) { *s = *s * 1664525u + 1013904223u; return *s >> 8; }

/* half-precision scale in [-0.01, 0.01] as in the reference's self-test */
void put_scale(uint8_t *p, uint32_t *s) {
    float v = ((float)(st_rng(s) & 0xFFFF) / 65536.0f - 0.5f) * 0.02f;
    /* RNE f32 -> f16 for a normal-range value */
    uint32_t x;
    memcpy(&x, &v, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    uint16_t h;
    if (ax < 0x38800000u) {   /* |v| < 2^-14: f16 subnormal or zero */
        uint32_t e = ax >> 23, mant = (ax & 0x7FFFFFu) | 0x800000u;
        if (ax <= 0x33000000u) h = (uint16_t)sign;
        else {
            uint32_t sh = 126u - e, q = mant >> sh, rest = mant & ((1u << sh) - 1u), half = 1u << (sh - 1u);
            q += (rest > half) || (rest == half && (q & 1u));
            h = (uint16_t)(sign | q);
        }
    } else {
        uint32_t r = ax - 0x38000000u, q = r >> 13, rest = r & 0x1FFFu;
        q += (rest > 0x1000u) || (rest == 0x1000u && (q & 1u));
        h = (uint16_t)(sign | q);
    }
    p[0] = (uint8_t)h;
    p[1] = (uint8_t)(h >> 8);
}

void make_row(int dt, uint8_t *w, int64_t n, uint32_t *s) {
    const int bv = dt_block_values(dt), wb = dt_block_bytes(dt);
    const size_t bytes = (size_t)(n / bv) * wb;
    for (size_t i = 0; i < bytes; i++) w[i] = (uint8_t)st_rng(s);
    for (int64_t b = 0; b < n / bv; b++) {
        uint8_t *k = w + b * wb;
        if (dt == DT_F32) { float v = (float)(st_rng(s) & 0xFFFF) / 32768.0f - 1.0f; memcpy(k, &v, 4); }
        else if (dt == DT_Q8_0) put_scale(k, s);
        else if (dt == DT_Q4_K || dt == DT_Q5_K) { put_scale(k, s); put_scale(k + 2, s); }
        else if (dt == DT_Q6_K) put_scale(k + 208, s);
        else if (dt == DT_Q8_K) { float d = (float)(st_rng(s) & 0xFFFF) * 1e-7f; memcpy(k, &d, 4); }
    }
}

bool same(float a, float b) {
    if (a != a || b != b) return (a != a) && (b != b);
    uint32_t x, y;
    memcpy(&x, &a, 4);
    memcpy(&y, &b, 4);
    return x == y;
}

}  // namespace

int tlmh_selftest(int *failed_mask) {
    const int64_t N = 1024, NF = 1003;
    const int ROWS = 9;
    static const int dts[] = {DT_F32, DT_Q8_0, DT_Q4_K, DT_Q5_K, DT_Q6_K, DT_Q8_K};
    uint32_t s = 0x2545F491u;
    std::vector<float> xf(N);
    for (int64_t i = 0; i < N; i++) xf[i] = (float)(st_rng(&s) & 0xFFFF) / 32768.0f - 1.0f;
    xf[5] = 7.5f;
    xf[700] = -7.5f;
    std::vector<uint8_t> xk(act_bytes(DT_Q8_K, N)), xa(act_bytes(DT_Q8_0, N));
    h_act(DT_Q8_K, xf.data(), N, xk.data());
    h_act(DT_Q8_0, xf.data(), N, xa.data());

    uint8_t *dev = nullptr;
    const size_t wmax = (size_t)ROWS * N * 4, pmax = (size_t)16 * N * 4;
    size_t o_x = 0, o_xk = 8192, o_xa = 16384, o_w = 32768, o_p = o_w + wmax + 256, o_y = o_p + pmax + 256;
    size_t total = o_y + 4096;
    if (hipMalloc((void **)&dev, total) != hipSuccess) return tlmh_seterr(TLM_HIP_ENOMEM, "self-test: device memory");
    int fails = 0, mask = 0;
    std::vector<uint8_t> got(act_bytes(DT_Q8_K, N));
    std::vector<uint8_t> w(wmax);
    bool io_ok = hipMemcpy(dev + o_x, xf.data(), N * 4, hipMemcpyHostToDevice) == hipSuccess;
    /* activation quantisers */
    for (int kind : {DT_Q8_K, DT_Q8_0}) {
        size_t off = kind == DT_Q8_K ? o_xk : o_xa, nbytes = act_bytes(kind, N);
        bool ok = io_ok && launch_quantize_act(kind, (const float *)(dev + o_x), N, dev + off, nullptr) == TLM_HIP_OK &&
                  hipMemcpy(got.data(), dev + off, nbytes, hipMemcpyDeviceToHost) == hipSuccess &&
                  memcmp(got.data(), kind == DT_Q8_K ? xk.data() : xa.data(), nbytes) == 0;
        if (!ok) {
            fails++;
            mask |= 1 << kind;
        }
    }
    /* the activations the dots use are the host rule's bytes */
    io_ok = io_ok && hipMemcpy(dev + o_xk, xk.data(), xk.size(), hipMemcpyHostToDevice) == hipSuccess &&
            hipMemcpy(dev + o_xa, xa.data(), xa.size(), hipMemcpyHostToDevice) == hipSuccess;
    for (int dt : dts) {
        const int64_t n = dt == DT_F32 ? NF : N;
        const size_t rb = dt == DT_F32 ? (size_t)n * 4 : (size_t)(n / dt_block_values(dt)) * dt_block_bytes(dt);
        const int kind = dt_act_kind(dt);
        const uint8_t *hact = kind == DT_Q8_K ? xk.data() : kind == DT_Q8_0 ? xa.data() : (const uint8_t *)xf.data();
        const uint8_t *dact = dev + (kind == DT_Q8_K ? o_xk : kind == DT_Q8_0 ? o_xa : o_x);
        bool ok = io_ok;
        for (int rep = 0; rep < 2 && ok; rep++) {
            float ref[ROWS], y[ROWS];
            for (int r = 0; r < ROWS; r++) {
                make_row(dt, w.data() + rb * r, n, &s);
                ref[r] = h_dot(dt, w.data() + rb * r, hact, n);
            }
            ok = hipMemcpy(dev + o_w, w.data(), rb * ROWS, hipMemcpyHostToDevice) == hipSuccess;
            /* plain layout, rows [0, 9) then [2, 7) */
            ok = ok && launch_matvec_plain(dt, dev + o_w, rb, dact, (float *)(dev + o_y), n, 0, ROWS, nullptr) == 0 &&
                 hipMemcpy(y, dev + o_y, sizeof y, hipMemcpyDeviceToHost) == hipSuccess;
            for (int r = 0; ok && r < ROWS; r++) ok = same(ref[r], y[r]);
            /* packed layout */
            if (ok && dt != DT_F32) {
                ok = launch_pack(dt, dev + o_w, rb, ROWS, n, dev + o_p, nullptr) == 0 &&
                     launch_matvec_packed(dt, dev + o_p, ROWS, n, dact, (float *)(dev + o_y), nullptr) == 0 &&
                     hipMemcpy(y, dev + o_y, sizeof y, hipMemcpyDeviceToHost) == hipSuccess;
                for (int r = 0; ok && r < ROWS; r++) ok = same(ref[r], y[r]);
            }
        }
        if (!ok) {
            fails++;
            mask |= 1 << dt;
        }
    }
    /* the exponential against this host's libm expf (what the reference
     * calls): float bit patterns strided over the whole range, the overflow and
     * underflow edges and two inputs whose result needs the fused shift */
    {
        const int NE = 4096;
        std::vector<float> ex(NE), ey(NE), eg(NE);
        for (int i = 0; i < NE - 6; i++) {
            const uint32_t u = (uint32_t)i * 1048573u;
            memcpy(&ex[i], &u, 4);
        }
        const float edge[6] = {0x1.62e42ep6f, 0x1.62e430p6f, -0x1.9fe368p6f, -0x1.9fe366p6f, 0x1.04845ep+5f,
                               -0x1.f8cbb2p+5f};
        for (int i = 0; i < 6; i++) ex[NE - 6 + i] = edge[i];
        for (int i = 0; i < NE; i++) ey[i] = expf(ex[i]);
        float *dx = (float *)(dev + o_w), *dy = (float *)(dev + o_p);
        bool ok = hipMemcpy(dx, ex.data(), NE * 4, hipMemcpyHostToDevice) == hipSuccess &&
                  launch_expf(dx, dy, NE, nullptr) == TLM_HIP_OK &&
                  hipMemcpy(eg.data(), dy, NE * 4, hipMemcpyDeviceToHost) == hipSuccess;
        for (int i = 0; ok && i < NE; i++) ok = same(ey[i], eg[i]) || (ey[i] != ey[i] && eg[i] != eg[i]);
        if (!ok) {
            fails++;
            mask |= 1 << 30;
        }
    }
    (void)hipDeviceSynchronize();
    (void)hipFree(dev);
    *failed_mask = mask;
    return fails;
}
