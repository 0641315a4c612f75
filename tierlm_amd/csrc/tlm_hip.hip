/* tlm_hip.hip - the C ABI of libtlm_hip.so (include/tlm_hip.h): error
 * plumbing, device memory, dispatch to the kernels, the start-up self-test and
 * the host-pointer entries of the reference's kernel-tier table.
 *
 * No entry point falls back to CPU arithmetic: a kernel that fails its
 * self-test is refused (NaN results plus an error), never replaced. */
#include "tlm_hip_internal.h"

#include <math.h>
#include <mutex>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

/* host scalar rule used only by the self-test (hip_selftest.hip) */
int  tlmh_selftest(int *failed_mask);

/* ---- errors (thread-local message, like tlm_seterr) --------------------- */
static thread_local char g_err[512];

int tlmh_seterr(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int tlmh_check(hipError_t e, const char *what) {
    if (e == hipSuccess) return TLM_HIP_OK;
    int code = e == hipErrorOutOfMemory ? TLM_HIP_ENOMEM
             : (e == hipErrorNoDevice || e == hipErrorInvalidDevice) ? TLM_HIP_EUNSUP : TLM_HIP_EIO;
    return tlmh_seterr(code, "%s: %s", what, hipGetErrorString(e));
}

/* ---- state ---------------------------------------------------------------- */
static std::mutex g_mu;                 /* init + the staging area */
static int g_device = -1;
static int g_selftest_failures = 0;
static int g_failed_mask = 0;           /* bit dt set: that dtype failed its self-test */
static uint8_t *g_stage = nullptr;      /* device staging for host-pointer entries */
static size_t g_stage_bytes = 0;
static hipStream_t g_stage_stream = nullptr;

int tlmh_current_device(void) { return g_device; }

/* ---- the workspace of tlm_hip_moe_layer_noalloc ---------------------------
 * A file-scope device array: every GPU the library is initialised on holds its
 * own copy, TLM_HIP_MOE_NOALLOC_MAX_BYTES long, until the process ends.  In
 * host code the array's name is a host-side stand-in, not a device address:
 * its address on each device comes from hipGetSymbolAddress in tlm_hip_init
 * (that device current) and only that address ever reaches a kernel. */
static __device__ __align__(256) uint8_t scratch[TLM_HIP_MOE_NOALLOC_MAX_BYTES];
constexpr int SCRATCH_DEVICES = 64;
static void *g_scratch[SCRATCH_DEVICES];   /* per device; set once, under g_mu */

extern "C" {

const char *tlm_hip_errmsg(void) { return g_err; }

int tlm_hip_init(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_device == device && g_device >= 0) return TLM_HIP_OK;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) return tlmh_seterr(TLM_HIP_EUNSUP, "tlm_hip_init: no HIP device");
    if (device < 0 || device >= n) return tlmh_seterr(TLM_HIP_EINVAL, "tlm_hip_init: device %d of %d", device, n);
    HIPCHK(hipSetDevice(device));
    hipDeviceProp_t prop;
    HIPCHK(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return tlmh_seterr(TLM_HIP_EUNSUP, "tlm_hip_init: device %d is %s, this library is built for gfx950",
                           device, prop.gcnArchName);
    if (device < SCRATCH_DEVICES && !g_scratch[device]) {
        void *p = nullptr;
        HIPCHK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        g_scratch[device] = p;
    }
    if (g_stage) { (void)hipFree(g_stage); g_stage = nullptr; }
    if (g_stage_stream) { (void)hipStreamDestroy(g_stage_stream); g_stage_stream = nullptr; }
    g_stage_bytes = (size_t)64 << 20;
    HIPCHK(hipMalloc((void **)&g_stage, g_stage_bytes));
    HIPCHK(hipStreamCreateWithFlags(&g_stage_stream, hipStreamNonBlocking));
    g_device = device;
    int mask = 0;
    int rc = tlmh_selftest(&mask);
    if (rc < 0) { g_device = -1; return rc; }
    g_selftest_failures = rc;
    g_failed_mask = mask;
    return TLM_HIP_OK;
}

void tlm_hip_shutdown(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_stage) (void)hipFree(g_stage);
    if (g_stage_stream) (void)hipStreamDestroy(g_stage_stream);
    g_stage = nullptr;
    g_stage_stream = nullptr;
    g_stage_bytes = 0;
    g_device = -1;
}

const char *tlm_hip_tier(void) { return g_device >= 0 ? "hip" : "none"; }
int tlm_hip_selftest_failures(void) { return g_selftest_failures; }

/* ---- memory --------------------------------------------------------------- */
int tlm_hip_malloc(void **dptr, size_t bytes) {
    if (!dptr) return tlmh_seterr(TLM_HIP_EINVAL, "tlm_hip_malloc: NULL out pointer");
    *dptr = nullptr;
    if (bytes == 0) return TLM_HIP_OK;
    return tlmh_check(hipMalloc(dptr, bytes), "hipMalloc");
}
int tlm_hip_free(void *dptr) { return dptr ? tlmh_check(hipFree(dptr), "hipFree") : TLM_HIP_OK; }
int tlm_hip_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return TLM_HIP_OK;
    return tlmh_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream), "memcpy h2d");
}
int tlm_hip_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return TLM_HIP_OK;
    return tlmh_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream), "memcpy d2h");
}
int tlm_hip_sync(void *stream) { return tlmh_check(hipStreamSynchronize((hipStream_t)stream), "stream sync"); }

/* ---- compute -------------------------------------------------------------- */
size_t tlm_hip_qact_bytes(int kind, int64_t n) { return act_bytes(kind, n); }

int tlm_hip_quantize_act(int kind, const float *x, int64_t n, void *dst, void *stream) {
    return launch_quantize_act(kind, x, n, dst, (hipStream_t)stream);
}

int tlm_hip_stream_read(const void *p, size_t bytes, uint32_t *sink, void *stream) {
    return launch_stream_read(p, bytes, sink, (hipStream_t)stream);
}

int tlm_hip_expf(const float *x, float *y, int64_t n, void *stream) {
    return launch_expf(x, y, n, (hipStream_t)stream);
}

int tlm_hip_matvec_rows(int dt, const void *W, size_t row_bytes, const void *act, float *y, int64_t n, int64_t r0,
                        int64_t r1, void *stream) {
    return launch_matvec_plain(dt, W, row_bytes, act, y, n, r0, r1, (hipStream_t)stream);
}

size_t tlm_hip_packed_bytes(int dt, int64_t rows, int64_t n) { return packed_bytes(dt, rows, n); }

int tlm_hip_pack(int dt, const void *src, size_t row_bytes, int64_t rows, int64_t n, void *dst, void *stream) {
    return launch_pack(dt, src, row_bytes, rows, n, dst, (hipStream_t)stream);
}

int tlm_hip_matvec_packed(int dt, const void *Wp, int64_t rows, int64_t n, const void *act, float *y, void *stream) {
    return launch_matvec_packed(dt, Wp, rows, n, act, y, (hipStream_t)stream);
}

size_t tlm_hip_moe_prefill_workspace_bytes(const tlm_hip_moe_desc *d, int64_t T) {
    return moe_prefill_workspace_bytes(d, T);
}

int tlm_hip_moe_prefill(const tlm_hip_moe_desc *d, float *h, int64_t T, int32_t *ids, float *w, void *workspace,
                        void *stream) {
    return launch_moe_prefill(d, h, T, ids, w, workspace, (hipStream_t)stream);
}

int tlm_hip_matmul_tokens(int dt, const void *Wp, int64_t rows, int64_t n, const void *act, int64_t ntok,
                          float *Y, void *stream) {
    return launch_tokmm(dt, Wp, rows, n, act, ntok, Y, (hipStream_t)stream);
}

int tlm_hip_mv_job(const tlm_hip_seg *segs, int nseg, void *stream) {
    return launch_mv_job(segs, nseg, (hipStream_t)stream);
}

size_t tlm_hip_moe_workspace_bytes(const tlm_hip_moe_desc *d) { return moe_workspace_bytes(d); }

int tlm_hip_moe_layer(const tlm_hip_moe_desc *d, float *h, int32_t *ids, float *w, void *workspace, void *stream) {
    return launch_moe_layer(d, h, ids, w, workspace, (hipStream_t)stream);
}

int tlm_hip_moe_layer_noalloc(const tlm_hip_moe_desc *d, float *h, int32_t *ids, float *w, void *stream) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SCRATCH_DEVICES || !g_scratch[dev])
        return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer_noalloc: tlm_hip_init has not run on the current device");
    if (!d) return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer_noalloc: NULL descriptor");
    const size_t need = moe_workspace_bytes(d);
    if (need > TLM_HIP_MOE_NOALLOC_MAX_BYTES)
        return tlmh_seterr(TLM_HIP_ERANGE,
                           "moe_layer_noalloc: this block needs %zu bytes of workspace, more than the %u-byte "
                           "static scratch; use tlm_hip_moe_layer with a workspace",
                           need, (unsigned)TLM_HIP_MOE_NOALLOC_MAX_BYTES);
    return launch_moe_layer(d, h, ids, w, g_scratch[dev], (hipStream_t)stream);
}

int tlm_hip_moe_route(const tlm_hip_moe_desc *d, const float *h, int32_t *ids, float *w, void *workspace,
                      void *stream) {
    return launch_moe_route(d, h, ids, w, workspace, (hipStream_t)stream);
}

int tlm_hip_moe_layer_phase(const tlm_hip_moe_desc *d, int phase, float *h, int32_t *ids, float *w, void *workspace,
                            void *stream) {
    if (phase < 1 || phase > 3) return tlmh_seterr(TLM_HIP_EINVAL, "moe_layer_phase: phase %d not in 1..3", phase);
    return launch_moe_phase(d, phase, h, ids, w, workspace, (hipStream_t)stream);
}

}  // extern "C"

/* ---- host-pointer tier entries (src/lib/tlm_quant.h:156-166) --------------
 * Each call stages weights and activation through the device staging area
 * (rows in chunks that fit), runs the plain-layout kernel and copies y back.
 * Serialised by g_mu; a dtype that failed the self-test yields NaN. */
static size_t row_bytes_of(int dt, int64_t n) {
    int bv = dt_block_values(dt);
    return bv ? (size_t)(n / bv) * (size_t)dt_block_bytes(dt) : 0;
}

static void host_mv(int dt, const void *W, size_t row_bytes, const void *act, float *y, int64_t n, int64_t nrows) {
    std::lock_guard<std::mutex> lk(g_mu);
    const int kind = dt_act_kind(dt);
    const size_t ab = kind == DT_F32 ? (size_t)n * 4 : act_bytes(kind, n);
    const size_t tight = row_bytes_of(dt, n);
    bool ok = g_device >= 0 && !((g_failed_mask >> dt) & 1) && tight > 0 && row_bytes >= tight;
    const size_t a_off = 0, y_room = 4096 * 4, w_off = (ab + 255) & ~(size_t)255;
    int64_t chunk = ok && g_stage_bytes > w_off + y_room ? (int64_t)((g_stage_bytes - w_off - y_room) / tight) : 0;
    if (chunk > 4096) chunk = 4096;
    if (chunk <= 0) ok = false;
    hipStream_t s = g_stage_stream;
    if (ok && hipMemcpyAsync(g_stage + a_off, act, ab, hipMemcpyHostToDevice, s) != hipSuccess) ok = false;
    for (int64_t r0 = 0; ok && r0 < nrows; r0 += chunk) {
        int64_t m = nrows - r0 < chunk ? nrows - r0 : chunk;
        uint8_t *dW = g_stage + w_off;
        float *dy = (float *)(g_stage + g_stage_bytes - y_room);
        /* rows are copied tightly: the device kernel sees stride `tight` */
        const uint8_t *src = (const uint8_t *)W + (size_t)r0 * row_bytes;
        if (row_bytes == tight) {
            if (hipMemcpyAsync(dW, src, (size_t)m * tight, hipMemcpyHostToDevice, s) != hipSuccess) { ok = false; break; }
        } else if (hipMemcpy2DAsync(dW, tight, src, row_bytes, tight, (size_t)m, hipMemcpyHostToDevice, s) != hipSuccess) {
            ok = false;
            break;
        }
        if (launch_matvec_plain(dt, dW, tight, g_stage + a_off, dy, n, 0, m, s) != TLM_HIP_OK) { ok = false; break; }
        if (hipMemcpyAsync(y + r0, dy, (size_t)m * 4, hipMemcpyDeviceToHost, s) != hipSuccess) { ok = false; break; }
        if (hipStreamSynchronize(s) != hipSuccess) { ok = false; break; }
    }
    if (!ok) {
        for (int64_t r = 0; r < nrows; r++) y[r] = NAN;
        tlmh_seterr(TLM_HIP_EIO, "hip tier: dtype %d unavailable (not initialised, failed self-test, or copy error)", dt);
    }
}

#define HIP_TIER_ENTRY(NAME, DT)                                                                         \
    static float dot_##NAME(const void *w, const void *a, int64_t n, const float *aux) {                \
        (void)aux;                                                                                       \
        float y;                                                                                         \
        host_mv(DT, w, row_bytes_of(DT, n), a, &y, n, 1);                                                \
        return y;                                                                                        \
    }                                                                                                    \
    static void mv_##NAME(const void *W, size_t rb, const void *a, float *y, int64_t n, int64_t nrows) { \
        host_mv(DT, W, rb, a, y, n, nrows);                                                              \
    }
HIP_TIER_ENTRY(f32, DT_F32)
HIP_TIER_ENTRY(q8_0, DT_Q8_0)
HIP_TIER_ENTRY(q4_k, DT_Q4_K)
HIP_TIER_ENTRY(q5_k, DT_Q5_K)
HIP_TIER_ENTRY(q6_k, DT_Q6_K)
HIP_TIER_ENTRY(q8_k, DT_Q8_K)

/* table indices of src/lib/tlm_quant.h:152-155 */
enum { QK_F32 = 0, QK_Q8_0 = 3, QK_Q4_K = 4, QK_Q5_K = 5, QK_Q6_K = 6, QK_Q8_K = 9 };

extern "C" int tlm_kern_hip_fill(tlm_hip_quant_kernels *k) {
    if (!k || g_device < 0) return 0;
    k->dot[QK_F32] = dot_f32;   k->mv[QK_F32] = mv_f32;
    k->dot[QK_Q8_0] = dot_q8_0; k->mv[QK_Q8_0] = mv_q8_0;
    k->dot[QK_Q4_K] = dot_q4_k; k->mv[QK_Q4_K] = mv_q4_k;
    k->dot[QK_Q5_K] = dot_q5_k; k->mv[QK_Q5_K] = mv_q5_k;
    k->dot[QK_Q6_K] = dot_q6_k; k->mv[QK_Q6_K] = mv_q6_k;
    k->dot[QK_Q8_K] = dot_q8_k; k->mv[QK_Q8_K] = mv_q8_k;
    return 6;
}
