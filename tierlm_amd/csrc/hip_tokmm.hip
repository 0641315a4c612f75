/* hip_tokmm.hip - many tokens through one packed matrix (tlm_hip_matmul_tokens):
 * the int8 MFMA tile of tlm_hip_mfma.h over (128-row, 32-token) groups. */
#include "tlm_hip_internal.h"
#include "tlm_hip_items.h"
#include "tlm_hip_mfma.h"

namespace {

constexpr int TM_WAVES = 4;      /* waves per group: 128 rows */
using tokmm::TM_ROWS;
using tokmm::TM_TOK;

__global__ __launch_bounds__(256) void k_tokmm_q6k(const uint8_t *__restrict__ Wp, int64_t rows, int nb,
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
    float acc[16];
    tokmm::tile_q6k<false>(Wp, units, ubase, nb, (const GAS uint8_t *)act + (int64_t)ta * nb * 292,
                    (LAS float *)s_da[wave], j, half, acc);
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
    hipLaunchKernelGGL(k_tokmm_q6k, grid, dim3(64 * TM_WAVES), 0, s, (const uint8_t *)Wp, rows, nb,
                       (const uint8_t *)act, (int)ntok, Y);
    return tlmh_check(hipGetLastError(), "matmul_tokens launch");
}
