/* hip_tokmm.hip - many tokens through one packed matrix (tlm_hip_matmul_tokens):
 * the int8 MFMA tile of tlm_hip_mfma.h over (128-row, 32-token) groups; K-quant
 * matrices take Q8_K activations, Q8_0 matrices a8 activations. */
#include "tlm_hip_internal.h"
#include "tlm_hip_items.h"
#include "tlm_hip_mfma.h"

namespace {

using tokmm::TM_ROWS;
using tokmm::TM_TOK;
constexpr int GROUP_ROWS = tokmm::TM_WAVES * TM_ROWS;

/* row group bx (GROUP_ROWS rows) of one matrix against the tile's 32 tokens */
template <int DT>
__device__ __forceinline__ void tokmm_group(const uint8_t *__restrict__ Wp, int64_t rows, int64_t bx, int nb,
                                            const uint8_t *__restrict__ act, int ntok, float *__restrict__ Y) {
    __shared__ __align__(16) uint8_t s_tile[tokmm::tile_lds_bytes<DT>()];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, half = lane >> 5;
    const int64_t row = bx * GROUP_ROWS + wave * TM_ROWS + (lane & 31);
    const int tok0 = blockIdx.y * TM_TOK;
    const int nbu = nb * tokmm::blocks_per_stage<DT>();   /* packed units per row */
    const int64_t units = ((rows + TILE_ROWS - 1) / TILE_ROWS) * nbu * TILE_ROWS;
    /* rows past the last one read the last valid row and write nothing;
     * tokens past the last one stage the last valid token */
    const int64_t rr = row < rows ? row : rows - 1;
    const tokmm::Chain ch = tokmm::chain_at<DT>(Wp, units, (rr / TILE_ROWS) * nbu * TILE_ROWS + rr % TILE_ROWS);
    const int ts = tok0 + ((int)threadIdx.x >> 3) < ntok ? tok0 + ((int)threadIdx.x >> 3) : ntok - 1;
    const int64_t astride = DT == DT_Q8_0 ? (int64_t)nb * 8 * 36 : (int64_t)nb * 292;   /* a8 / Q8_K bytes per token */
    float acc[16];
    tokmm::tile_run<DT, false>(ch, nb, (const GAS uint8_t *)act + (int64_t)ts * astride, (LAS uint8_t *)s_tile, acc);
    if (row < rows) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int tok = tok0 + 8 * (v >> 2) + 4 * half + (v & 3);
            if (tok < ntok) Y[(int64_t)tok * rows + row] = acc[v];
        }
    }
}

template <int DT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DT == DT_Q8_0 ? 2 : 3))) void k_tokmm(const uint8_t *__restrict__ Wp, int64_t rows, int nb,
                                               const uint8_t *__restrict__ act, int ntok, float *__restrict__ Y) {
    tokmm_group<DT>(Wp, rows, blockIdx.x, nb, act, ntok, Y);
}

/* up to TOK_SEGS matrices of one dtype and width against the same tokens in
 * one launch: segment s owns row groups [end[s-1], end[s]) */
constexpr int TOK_SEGS = 4;
struct TokSegs {
    const uint8_t *W[TOK_SEGS];
    int64_t rows[TOK_SEGS], end[TOK_SEGS];
    float *Y[TOK_SEGS];
    int n;
};
template <int DT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DT == DT_Q8_0 ? 2 : 3))) void k_tokmm_segs(const TokSegs sg, int nb,
                                               const uint8_t *__restrict__ act, int ntok) {
    int s = 0;
    while (s + 1 < sg.n && (int64_t)blockIdx.x >= sg.end[s]) s++;
    tokmm_group<DT>(sg.W[s], sg.rows[s], (int64_t)blockIdx.x - (s ? sg.end[s - 1] : 0), nb, act, ntok, sg.Y[s]);
}

}  // namespace

int launch_tokmm_segs(int dt, int nseg, const void *const *W, const int64_t *rows, int64_t n, const void *act,
                      int64_t ntok, float *const *Y, hipStream_t s) {
    if (nseg < 1 || nseg > TOK_SEGS || !W || !rows || !Y || !act)
        return tlmh_seterr(TLM_HIP_EINVAL, "matmul_tokens: %d segments", nseg);
    if (!tokmm::tile_dt(dt)) return tlmh_seterr(TLM_HIP_EUNSUP, "matmul_tokens: dtype %d not supported", dt);
    if (n <= 0 || n % 256 || ntok <= 0 || ntok > (int64_t)1 << 20 || ((uintptr_t)act & 3u))
        return tlmh_seterr(TLM_HIP_EINVAL, "matmul_tokens: n=%lld ntok=%lld", (long long)n, (long long)ntok);
    TokSegs sg{};
    sg.n = nseg;
    int64_t end = 0;
    for (int i = 0; i < nseg; i++) {
        if (!W[i] || !Y[i] || rows[i] <= 0 || ((uintptr_t)W[i] & 15u))
            return tlmh_seterr(TLM_HIP_EINVAL, "matmul_tokens: segment %d", i);
        sg.W[i] = (const uint8_t *)W[i];
        sg.rows[i] = rows[i];
        sg.Y[i] = Y[i];
        end += (rows[i] + GROUP_ROWS - 1) / GROUP_ROWS;
        sg.end[i] = end;
    }
    const int nb = (int)(n / 256);
    const dim3 grid((unsigned)end, (unsigned)((ntok + TM_TOK - 1) / TM_TOK));
    const uint8_t *a = (const uint8_t *)act;
    switch (dt) {
    case DT_Q4_K: hipLaunchKernelGGL(k_tokmm_segs<DT_Q4_K>, grid, dim3(256), 0, s, sg, nb, a, (int)ntok); break;
    case DT_Q5_K: hipLaunchKernelGGL(k_tokmm_segs<DT_Q5_K>, grid, dim3(256), 0, s, sg, nb, a, (int)ntok); break;
    case DT_Q8_0: hipLaunchKernelGGL(k_tokmm_segs<DT_Q8_0>, grid, dim3(256), 0, s, sg, nb, a, (int)ntok); break;
    default: hipLaunchKernelGGL(k_tokmm_segs<DT_Q6_K>, grid, dim3(256), 0, s, sg, nb, a, (int)ntok); break;
    }
    return tlmh_check(hipGetLastError(), "matmul_tokens launch");
}

int launch_tokmm(int dt, const void *Wp, int64_t rows, int64_t n, const void *act, int64_t ntok, float *Y,
                 hipStream_t s) {
    if (!Wp || !act || !Y) return tlmh_seterr(TLM_HIP_EINVAL, "matmul_tokens: NULL argument");
    if (!tokmm::tile_dt(dt)) return tlmh_seterr(TLM_HIP_EUNSUP, "matmul_tokens: dtype %d not supported", dt);
    if (rows <= 0 || n <= 0 || n % 256 || ntok <= 0 || ntok > (int64_t)1 << 20)
        return tlmh_seterr(TLM_HIP_EINVAL, "matmul_tokens: rows=%lld n=%lld ntok=%lld", (long long)rows,
                           (long long)n, (long long)ntok);
    if ((uintptr_t)Wp & 15u || (uintptr_t)act & 3u)
        return tlmh_seterr(TLM_HIP_EINVAL, "matmul_tokens: packed weights must be 16-byte, activations 4-byte aligned");
    const int nb = (int)(n / 256);
    const dim3 grid((unsigned)((rows + GROUP_ROWS - 1) / GROUP_ROWS), (unsigned)((ntok + TM_TOK - 1) / TM_TOK));
    const uint8_t *w = (const uint8_t *)Wp, *a = (const uint8_t *)act;
    switch (dt) {
    case DT_Q4_K: hipLaunchKernelGGL(k_tokmm<DT_Q4_K>, grid, dim3(256), 0, s, w, rows, nb, a, (int)ntok, Y); break;
    case DT_Q5_K: hipLaunchKernelGGL(k_tokmm<DT_Q5_K>, grid, dim3(256), 0, s, w, rows, nb, a, (int)ntok, Y); break;
    case DT_Q8_0: hipLaunchKernelGGL(k_tokmm<DT_Q8_0>, grid, dim3(256), 0, s, w, rows, nb, a, (int)ntok, Y); break;
    default: hipLaunchKernelGGL(k_tokmm<DT_Q6_K>, grid, dim3(256), 0, s, w, rows, nb, a, (int)ntok, Y); break;
    }
    return tlmh_check(hipGetLastError(), "matmul_tokens launch");
}
