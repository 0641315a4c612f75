/* hip_tokmm.hip - many tokens through one packed matrix with int8 MFMA.
 *
 * The reference has no GEMM: its prefill runs the decode step once per
 * token (src/lib/tlm_model.c:1105-1113), so every (token, row) output is the
 * decode dot - per super-block an exact int32 sum, then the row's fma chain
 * in ascending block order (src/lib/tlm_quant.c:853-882 for Q6_K).  Here the
 * weights stream once for up to 32 tokens and the int32 sums come from
 * v_mfma_i32_32x32x16_i8 (K = 16 = one Q6_K scale group); the chain is the
 * same, so the results are the decode kernel's bits.
 *
 * MFMA roles: srcA = activations (lane l: token l%32, codes 8*(l/32)..+7 of
 * the group), srcB = weights (lane l: weight row l%32, the same 8 positions),
 * D[token][row] in lane l, element v: token 8*(v/4) + 4*(l/32) + v%4, row
 * l%32.  Every accumulator of a lane belongs to one weight row, so the row's
 * group scale is one value per lane.
 *
 * Q6_K codes u in [0, 63] enter as u - 32 (int8): sum((u - 32) x) equals the
 * reference's gs - 32 * bsum exactly. */
#include "tlm_hip_internal.h"
#include "tlm_hip_items.h"

namespace {

typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int TM_ROWS = 32;      /* weight rows per wave */
constexpr int TM_TOK = 32;       /* tokens per wave */
constexpr int TM_WAVES = 4;      /* waves per group: 128 rows */

/* 4 Q6_K codes (ql nibbles + qh 2-bit fields, selected) -> 4 int8 of u - 32 */
__device__ __forceinline__ uint32_t q6_signed4(uint32_t ql, uint32_t qh, int nib, int sh) {
    const uint32_t u = ((ql >> (4 * nib)) & 0x0F0F0F0Fu) | (((qh >> sh) & 0x03030303u) << 4);
    const uint32_t t = u ^ 0x20202020u;            /* u - 32 for u >= 32; u + 32 otherwise */
    const uint32_t s = t & 0x20202020u;            /* sign bit 5 -> extend into bits 6, 7 */
    return t | (s << 1) | (s << 2);
}

/* One Q6_K block of one weight row, this lane's half (positions 8h..8h+7 of
 * every group): ql pieces [h][qq&1][g&1], qh pieces [h][g&1], scales, d. */
struct Q6Raw {
    u32x2 ql[8], qh[4];
    u32x4 sc;
    uint32_t dw;
};

__device__ __forceinline__ Q6Raw q6_load(const uint8_t *Wp, int64_t units, int64_t u, int half) {
    Q6Raw r;
    const GAS uint8_t *unit = (const GAS uint8_t *)Wp + u * 208;
#pragma unroll
    for (int p = 0; p < 8; p++) {          /* p = 4h + 2(qq&1) + gl */
        const int h = p >> 2, q1 = (p >> 1) & 1, gl = p & 1;
        r.ql[p] = *(const GAS u32x2 *)(unit + 64 * h + 32 * q1 + 16 * gl + 8 * half);
    }
#pragma unroll
    for (int p = 0; p < 4; p++) {          /* p = 2h + gl */
        const int h = p >> 1, gl = p & 1;
        r.qh[p] = *(const GAS u32x2 *)(unit + 128 + 32 * h + 16 * gl + 8 * half);
    }
    r.sc = *(const GAS u32x4 *)(unit + 192);
    r.dw = *(const GAS uint16_t *)((const GAS uint8_t *)Wp + units * 208 + u * 2);
    return r;
}

/* A operand of one Q8_K block of this lane's token: codes 16g + 8*half + 0..7
 * for g = 0..15, and the block's d. */
struct ActRaw {
    uint32_t c[32];
    float d;
};

__device__ __forceinline__ ActRaw act_load(const GAS uint8_t *blk, int half) {
    ActRaw a;
    const GAS uint32_t *q = (const GAS uint32_t *)(blk + 4);
#pragma unroll
    for (int g = 0; g < 16; g++) {
        a.c[2 * g] = q[4 * g + 2 * half];
        a.c[2 * g + 1] = q[4 * g + 2 * half + 1];
    }
    a.d = *(const GAS float *)blk;
    return a;
}

__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) {
    return (long)(((unsigned long long)hi << 32) | lo);
}

template <int DT>
__global__ __launch_bounds__(256) void k_tokmm(const uint8_t *__restrict__ Wp, int64_t rows, int nb,
                                               const uint8_t *__restrict__ act, int ntok, float *__restrict__ Y) {
    __shared__ float s_da[TM_WAVES][TM_TOK];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int j = lane & 31, half = lane >> 5;
    const int64_t row = (int64_t)blockIdx.x * (TM_ROWS * TM_WAVES) + wave * TM_ROWS + j;
    const int tok0 = blockIdx.y * TM_TOK;
    const bool rowok = row < rows;
    /* lanes past the last row / token read the last valid one and write nothing */
    const int64_t rr = rowok ? row : rows - 1;
    const int ta = tok0 + j < ntok ? tok0 + j : ntok - 1;
    const int64_t units = ((rows + TILE_ROWS - 1) / TILE_ROWS) * nb * TILE_ROWS;
    const int64_t ubase = (rr / TILE_ROWS) * nb * TILE_ROWS + rr % TILE_ROWS;
    const GAS uint8_t *arow = (const GAS uint8_t *)act + (int64_t)ta * nb * 292;
    LAS float *sda = (LAS float *)s_da[wave];

    float acc[16];
#pragma unroll
    for (int v = 0; v < 16; v++) acc[v] = 0.0f;

    Q6Raw w = q6_load(Wp, units, ubase, half);
    ActRaw a = act_load(arow, half);
    for (int b = 0; b < nb; b++) {
        /* next block's loads in flight while this one computes */
        Q6Raw wn = w;
        ActRaw an = a;
        if (b + 1 < nb) {
            wn = q6_load(Wp, units, ubase + (int64_t)(b + 1) * TILE_ROWS, half);
            an = act_load(arow + (int64_t)(b + 1) * 292, half);
        }
        int isum[16];
#pragma unroll
        for (int v = 0; v < 16; v++) isum[v] = 0;
        const uint32_t scw[4] = {w.sc.x, w.sc.y, w.sc.z, w.sc.w};
#pragma unroll
        for (int g = 0; g < 16; g++) {
            const int h = g >> 3, qq = (g >> 1) & 3, gl = g & 1;
            const u32x2 qlp = w.ql[4 * h + 2 * (qq & 1) + gl], qhp = w.qh[2 * h + gl];
            const long bw = pack2(q6_signed4(qlp.x, qhp.x, qq >> 1, 2 * qq), q6_signed4(qlp.y, qhp.y, qq >> 1, 2 * qq));
            const long aw = pack2(a.c[2 * g], a.c[2 * g + 1]);
            v16i p = {};
            p = __builtin_amdgcn_mfma_i32_32x32x16_i8(aw, bw, p, 0, 0, 0);
            const int s = (int)(int8_t)((scw[g >> 2] >> (8 * (g & 3))) & 0xFF);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                isum[v] += s * p[v];
                /* materialise the running sum here: otherwise the integer sums
                 * are reassociated across groups and all sixteen MFMA results
                 * stay live (and spill) */
                asm volatile("" : "+v"(isum[v]));
            }
        }
        /* the chain: acc = fmaf(d_w * d_a, (float)isum, acc), block order */
        if (half == 0) sda[j] = a.d;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const float dwf = f16_to_f32(w.dw);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const f32x4 da4 = *(const LAS f32x4 *)(sda + 8 * q + 4 * half);
#pragma unroll
            for (int t = 0; t < 4; t++) acc[4 * q + t] = fmaf(dwf * da4[t], (float)isum[4 * q + t], acc[4 * q + t]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        w = wn;
        a = an;
    }
    if (rowok) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int tok = tok0 + 8 * (v >> 2) + 4 * half + (v & 3);
            if (tok < ntok) Y[(int64_t)tok * rows + row] = acc[v];
        }
    }
}

}  // namespace

int launch_tokmm(int dt, const void *Wp, int64_t rows, int64_t n, const void *act, int64_t ntok, float *Y,
                 hipStream_t s) {
    if (!Wp || !act || !Y) return tlmh_seterr(TLM_HIP_EINVAL, "matmul_tokens: NULL argument");
    if (dt != DT_Q6_K) return tlmh_seterr(TLM_HIP_EUNSUP, "matmul_tokens: dtype %d not supported", dt);
    if (rows <= 0 || n <= 0 || n % 256 || ntok <= 0 || ntok > (int64_t)1 << 20)
        return tlmh_seterr(TLM_HIP_EINVAL, "matmul_tokens: rows=%lld n=%lld ntok=%lld", (long long)rows,
                           (long long)n, (long long)ntok);
    if ((uintptr_t)Wp & 15u || (uintptr_t)act & 3u)
        return tlmh_seterr(TLM_HIP_EINVAL, "matmul_tokens: packed weights must be 16-byte, activations 4-byte aligned");
    const int nb = (int)(n / 256);
    const dim3 grid((unsigned)((rows + TM_ROWS * TM_WAVES - 1) / (TM_ROWS * TM_WAVES)),
                    (unsigned)((ntok + TM_TOK - 1) / TM_TOK));
    hipLaunchKernelGGL(k_tokmm<DT_Q6_K>, grid, dim3(64 * TM_WAVES), 0, s, (const uint8_t *)Wp, rows, nb,
                       (const uint8_t *)act, (int)ntok, Y);
    return tlmh_check(hipGetLastError(), "matmul_tokens launch");
}
