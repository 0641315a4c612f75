/* tlm_hip_internal.h - shared device helpers and internal launch API of
 * libtlm_hip.so (gfx950).  Not installed; the public ABI is include/tlm_hip.h. */
#ifndef TLM_HIP_INTERNAL_H
#define TLM_HIP_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/tlm_hip.h"

/* tlm_dtype codes (src/lib/tlm_quant.h:31-42) */
enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2, DT_Q8_0 = 8, DT_Q4_K = 12, DT_Q5_K = 13,
       DT_Q6_K = 14, DT_Q8_K = 15 };

/* Rows per tile of the packed layout: a wave covers one block column of one
 * tile with 4 lanes per (row, block) for the 256-value formats. */
#define TILE_ROWS 16

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
    uint32_t s = (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 31u) return __uint_as_float(s | 0x7F800000u | (m << 13) | (m ? 0x00400000u : 0u));
    if (e == 0u) return __uint_as_float(__float_as_uint((float)m * 0x1p-24f) | s);
    return __uint_as_float(s | ((e + 112u) << 23) | (m << 13));
}

/* Round half to even via 1.5*2^23, clamp to [lo, hi], NaN -> 0
 * (src/lib/tlm_quant.c:233-243).  Built with -ffp-contract=off. */
__device__ __forceinline__ int rne_clamp(float v, int lo, int hi) {
    if (v != v) return 0;
    if (v <= (float)lo) return lo;
    if (v >= (float)hi) return hi;
    const float magic = 12582912.0f;
    return (int)((v + magic) - magic);
}

/* 4 x int8 dot with int32 accumulate (v_dot4_i32_i8): exact. */
__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

__device__ __forceinline__ int wave_lane() { return (int)__lane_id(); }

/* ---- launchers (defined in the .hip files) ------------------------------ */
int launch_quantize_act(int kind, const float *x, int64_t n, void *dst, hipStream_t s);
int launch_matvec_plain(int dt, const void *W, size_t row_bytes, const void *act, float *y,
                        int64_t n, int64_t r0, int64_t r1, hipStream_t s);
int launch_nan_fill(float *y, int64_t count, hipStream_t s);
size_t packed_bytes(int dt, int64_t rows, int64_t n);
int launch_pack(int dt, const void *src, size_t row_bytes, int64_t rows, int64_t n, void *dst, hipStream_t s);
int launch_matvec_packed(int dt, const void *Wp, int64_t rows, int64_t n, const void *act, float *y,
                         hipStream_t s);
int launch_mv_job(const tlm_hip_seg *segs, int nseg, hipStream_t s);
size_t moe_workspace_bytes(const tlm_hip_moe_desc *d);
int launch_moe_layer(const tlm_hip_moe_desc *d, float *h, int32_t *ids, float *w, void *ws, hipStream_t s);
int launch_moe_phase(const tlm_hip_moe_desc *d, int phase, float *h, int32_t *ids, float *w, void *ws,
                     hipStream_t s);

#endif
