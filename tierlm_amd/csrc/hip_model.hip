/* hip_model.hip - the whole decode step on the device (tlm_hip_model_*):
 * src/lib/tlm_model.c:1058-1103 (tlm_model_step) with attention()
 * :730-763, attn_heads :683-719, the f32 KV cache :646-664, rmsnorm
 * :164-169, RoPE :721-728 with the tables of :529-545 and :1069-1073, the
 * MoE block of hip_moe.hip, the final norm + lm_head :1087-1095 and the
 * greedy sampler's argmax :1139-1146.  The model is loaded from a compiled
 * store (host_packet.cpp) into HBM: every weight packed once, every expert
 * resident.
 *
 * Numerics (against the reference's scalar C): the integer-format GEMVs,
 * router, routing, combine and quantisers are bit-exact (hip_gemv.hip,
 * hip_moe.hip); RoPE and the attention dot products, the softmax scaling and
 * the P.V sums run in the reference's order with separate roundings (one
 * thread per dot product, positions in ascending order).  What may differ in
 * the last bit: sums of squares and the softmax sum are double trees instead
 * of sequential double sums, and e^x is exp in double rounded to float; the
 * reference's greedy tokens are reproduced exactly. */
#include "tlm_hip_internal.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <vector>

int tlmh_current_device(void);

namespace {

constexpr int NT = 256;

/* ---- block reductions ------------------------------------------------------ */
__device__ double block_sum_f64(double v, double *red) {
    v = wave_sum_f64(v);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    double s = 0.0;
    for (int i = 0; i < nw; i++) s += red[i];
    return s;
}

/* max over non-NaN values (a NaN never compares greater), -inf if none */
__device__ float block_max_f32(float v, float *red) {
    for (int o = 32; o > 0; o >>= 1) {
        const float u = __shfl_xor(v, o);
        v = u > v ? u : v;
    }
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float m = -INFINITY;
    for (int i = 0; i < nw; i++) m = red[i] > m ? red[i] : m;
    return m;
}

/* ---- embedding row (tlm_dequantize_row, src/lib/tlm_quant.c:629-660) -------- */
/* The step's position and token live in device memory (st[0] = pos, seq[pos]
 * = the token), so one captured graph serves every position. */
__global__ __launch_bounds__(NT) void k_embed(const uint8_t *__restrict__ embd, size_t row_bytes, int dt,
                                              const int32_t *__restrict__ seq, const int32_t *__restrict__ st, int D,
                                              float *__restrict__ h) {
    const uint8_t *row = embd + (size_t)seq[st[0]] * row_bytes;
    for (int i = threadIdx.x + blockIdx.x * blockDim.x; i < D; i += blockDim.x * gridDim.x) {
        if (dt == DT_F32) {
            h[i] = ((const float *)row)[i];
        } else {   /* Q8_0: y = f16(d) * (float)q */
            const uint8_t *b = row + (size_t)(i >> 5) * 34;
            const float dd = f16_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
            h[i] = dd * (float)(int8_t)b[2 + (i & 31)];
        }
    }
}

/* ---- rmsnorm over one vector: out = x * r * w, r = 1 / sqrtf(mean(x^2) + eps) */
__global__ __launch_bounds__(NT) void k_rmsnorm(const float *__restrict__ x, const float *__restrict__ w, int n,
                                                float eps, float *__restrict__ out) {
    __shared__ double red[NT / 64];
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += NT) ss += (double)x[i] * (double)x[i];
    ss = block_sum_f64(ss, red);
    const float r = 1.0f / sqrtf((float)(ss / (double)n) + eps);
    for (int i = threadIdx.x; i < n; i += NT) out[i] = x[i] * r * w[i];
}

/* ---- per head: qk-norm, RoPE, KV append (src/lib/tlm_model.c:743-753) -------
 * One wave per head; blocks [0, H) take the query heads, [H, H + KV) the key
 * heads, which also store k (after RoPE) and v at position pos of this
 * layer's caches (head-major [KV][max_ctx][hd]). */
__global__ __launch_bounds__(64) void k_qk_rope(float *__restrict__ q, float *__restrict__ kx,
                                                const float *__restrict__ vx, const float *__restrict__ q_norm,
                                                const float *__restrict__ k_norm, const float *__restrict__ cs_all,
                                                const float *__restrict__ sn_all, float *__restrict__ kc,
                                                float *__restrict__ vc, int H, int hd, const int32_t *__restrict__ st,
                                                int max_ctx, float eps) {
    __shared__ float s_v[256];
    const int b = blockIdx.x, lane = threadIdx.x, half = hd >> 1, pos = st[0];
    const float *cs = cs_all + (size_t)pos * half, *sn = sn_all + (size_t)pos * half;
    const bool is_q = b < H;
    float *v = is_q ? q + (size_t)b * hd : kx + (size_t)(b - H) * hd;
    const float *nw = is_q ? q_norm : k_norm;
    float e[4];   /* hd <= 256 */
    for (int k = 0; k < 4; k++) e[k] = lane + 64 * k < hd ? v[lane + 64 * k] : 0.0f;
    if (nw) {   /* rmsnorm over the head, in place (tlm_model.c:743-746) */
        double ss = 0.0;
        for (int k = 0; k < 4; k++) ss += (double)e[k] * (double)e[k];
        ss = wave_sum_f64(ss);
        const float r = 1.0f / sqrtf((float)(ss / (double)hd) + eps);
        for (int k = 0; k < 4; k++)
            if (lane + 64 * k < hd) e[k] = e[k] * r * nw[lane + 64 * k];
    }
    for (int k = 0; k < 4; k++)
        if (lane + 64 * k < hd) s_v[lane + 64 * k] = e[k];
    __syncthreads();
    /* NeoX pairs (j, j + hd/2): a' = a cs - b sn, b' = b cs + a sn (rope(), :721-728) */
    for (int j = lane; j < half; j += 64) {
        const float a = s_v[j], c = s_v[j + half];
        const float x0 = a * cs[j] - c * sn[j], x1 = c * cs[j] + a * sn[j];
        v[j] = x0;
        v[j + half] = x1;
        if (!is_q) {
            float *kd = kc + ((size_t)(b - H) * max_ctx + pos) * hd;
            kd[j] = x0;
            kd[j + half] = x1;
        }
    }
    if (!is_q) {
        float *vd = vc + ((size_t)(b - H) * max_ctx + pos) * hd;
        for (int i = lane; i < hd; i += 64) vd[i] = vx[(size_t)(b - H) * hd + i];
    }
}

/* ---- attention core, one group per head (src/lib/tlm_model.c:683-719) --------
 * kc / vc: this layer's caches, head-major [KV][max_ctx][hd]; scores: H x
 * max_ctx floats of scratch.  The reference's order is kept: each score is
 * one thread's dot product in ascending i, and each output element one
 * thread's sum over positions in ascending t.  V goes through LDS in chunks
 * of ATT_TC positions (coalesced loads), so that ordered sum runs on LDS
 * reads instead of a global round trip per position. */
constexpr int ATT_TC = 32;

__global__ __launch_bounds__(NT) void k_attn(const float *__restrict__ q, const float *__restrict__ kc,
                                             const float *__restrict__ vc, float *__restrict__ scores,
                                             float *__restrict__ att, int H, int KV, int hd, int max_ctx,
                                             const int32_t *__restrict__ st) {
    __shared__ __align__(16) float s_q[256];
    __shared__ __align__(16) float s_v[ATT_TC * 256];
    __shared__ double s_red[NT / 64];
    __shared__ float s_redf[NT / 64];
    const int T = st[0] + 1;
    const int h = blockIdx.x, tid = threadIdx.x, kvh = h / (H / KV);
    const float *K = kc + (size_t)kvh * max_ctx * hd, *V = vc + (size_t)kvh * max_ctx * hd;
    float *s = scores + (size_t)h * max_ctx;
    for (int i = tid; i < hd; i += NT) s_q[i] = q[(size_t)h * hd + i];
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)hd);
    float mx = -INFINITY;
    for (int t = tid; t < T; t += NT) {
        const f32x4 *kt = (const f32x4 *)(K + (size_t)t * hd);   /* hd % 32 == 0: 16-byte rows */
        float d = 0.0f;
        for (int i4 = 0; i4 < hd / 4; i4++) {
            const f32x4 k4 = kt[i4];
            d += s_q[4 * i4] * k4.x;
            d += s_q[4 * i4 + 1] * k4.y;
            d += s_q[4 * i4 + 2] * k4.z;
            d += s_q[4 * i4 + 3] * k4.w;
        }
        d *= scale;   /* scale after the dot, before the max */
        s[t] = d;
        if (d > mx) mx = d;
    }
    mx = block_max_f32(mx, s_redf);
    double sum = 0.0;
    for (int t = tid; t < T; t += NT) {
        const float p = exp_rn(s[t] - mx);
        s[t] = p;
        sum += (double)p;
    }
    sum = block_sum_f64(sum, s_red);
    const float inv = (float)(1.0 / sum);
    __syncthreads();   /* every p stored */
    float o = 0.0f;
    for (int t0 = 0; t0 < T; t0 += ATT_TC) {
        const int tn = T - t0 < ATT_TC ? T - t0 : ATT_TC;
        const int n4 = tn * hd / 4;
        for (int e = tid; e < n4; e += NT) ((f32x4 *)s_v)[e] = ((const f32x4 *)(V + (size_t)t0 * hd))[e];
        __syncthreads();
        if (tid < hd)
            for (int t = 0; t < tn; t++) {
                const float p = s[t0 + t] * inv;
                o += p * s_v[t * hd + tid];
            }
        __syncthreads();   /* the chunk is read before the next one overwrites it */
    }
    if (tid < hd) att[(size_t)h * hd + tid] = o;
}

__global__ __launch_bounds__(NT) void k_add(float *__restrict__ h, const float *__restrict__ y, int n) {
    const int i = blockIdx.x * NT + threadIdx.x;
    if (i < n) h[i] += y[i];
}

/* greedy: the first maximum, NaN skipped, 0 if none (src/lib/tlm_model.c:1139-1146) */
__global__ __launch_bounds__(1024) void k_argmax(const float *__restrict__ l, int n, int32_t *__restrict__ seq,
                                                 const int32_t *__restrict__ st) {
    __shared__ float s_v[1024];
    __shared__ int s_i[1024];
    float bv = 0.0f;
    int bi = -1;
    for (int i = threadIdx.x; i < n; i += 1024) {
        const float v = l[i];
        if (v != v) continue;
        if (bi < 0 || v > bv) {
            bv = v;
            bi = i;
        }
    }
    s_v[threadIdx.x] = bv;
    s_i[threadIdx.x] = bi;
    __syncthreads();
    for (int w = 512; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) {
            const float ov = s_v[threadIdx.x + w];
            const int oi = s_i[threadIdx.x + w];
            const int mi = s_i[threadIdx.x];
            if (oi >= 0 && (mi < 0 || ov > s_v[threadIdx.x] || (ov == s_v[threadIdx.x] && oi < mi))) {
                s_v[threadIdx.x] = ov;
                s_i[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) seq[st[0] + 1] = s_i[0] < 0 ? 0 : s_i[0];   /* the next step's token */
}

__global__ void k_advance(int32_t *st) {
    if (threadIdx.x == 0) st[0] += 1;
}

struct DevMat {
    int dt = -1;
    int64_t rows = 0, n = 0;
    void *p = nullptr;   /* packed */
};

struct Layer {
    const float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    DevMat q, k, v, o;
    tlm_hip_moe_desc moe{};
};

}  // namespace

struct tlm_hip_model {
    tlm_hip_model_geom g{};
    int max_ctx = 0, kv_len = 0;
    hipStream_t stream = nullptr;
    std::vector<void *> allocs;
    std::vector<Layer> L;
    const uint8_t *embd = nullptr;
    int embd_dt = 0;
    size_t embd_row = 0;
    const float *out_norm = nullptr;
    DevMat lm_head;
    float *kc = nullptr, *vc = nullptr, *cs = nullptr, *sn = nullptr, *scores = nullptr;
    float *h = nullptr, *xb = nullptr, *xb2 = nullptr, *q = nullptr, *kx = nullptr, *vx = nullptr, *att = nullptr;
    float *logits = nullptr;
    uint8_t *act = nullptr, *act2 = nullptr, *moe_ws = nullptr;
    int32_t *st = nullptr, *seq = nullptr, *ids = nullptr;   /* st[0] = position; seq[max_ctx + 1] tokens */
    float *w = nullptr;
    int32_t *host_tok = nullptr;   /* pinned */
    hipGraphExec_t graph[2] = {nullptr, nullptr};   /* step without / with logits, captured at first use */
    bool graph_failed[2] = {false, false};

    void *dalloc(size_t n) {
        void *p = nullptr;
        if (hipMalloc(&p, n ? n : 16) != hipSuccess) return nullptr;
        allocs.push_back(p);
        return p;
    }
    ~tlm_hip_model() {
        if (stream) (void)hipStreamSynchronize(stream);
        for (hipGraphExec_t g : graph)
            if (g) (void)hipGraphExecDestroy(g);
        for (void *p : allocs) (void)hipFree(p);
        if (host_tok) (void)hipHostFree(host_tok);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

namespace {

int dev_upload(tlm_hip_model *M, const void *src, size_t n, void **out) {
    *out = M->dalloc(n);
    if (!*out) return tlmh_seterr(TLM_HIP_ENOMEM, "model: out of device memory (%zu bytes)", n);
    return tlmh_check(hipMemcpy(*out, src, n, hipMemcpyHostToDevice), "model: upload");
}

/* rows x n matrix of a payload in the reference's row layout -> packed on device */
int dev_matrix(tlm_hip_model *M, int dt, const uint8_t *rows_src, int64_t rows, int64_t n, DevMat *out) {
    const int bv = dt_block_values(dt);
    if (bv == 0 || !dt_int_ok(dt) || dt == DT_Q8_K || n % bv)
        return tlmh_seterr(TLM_HIP_EUNSUP, "model: matrix dtype %d, %lld columns", dt, (long long)n);
    const size_t rb = (size_t)(n / bv) * dt_block_bytes(dt), raw = rb * (size_t)rows;
    void *tmp = nullptr;
    if (hipMalloc(&tmp, raw) != hipSuccess) return tlmh_seterr(TLM_HIP_ENOMEM, "model: out of device memory");
    int rc = tlmh_check(hipMemcpy(tmp, rows_src, raw, hipMemcpyHostToDevice), "model: upload");
    out->dt = dt;
    out->rows = rows;
    out->n = n;
    out->p = rc ? nullptr : M->dalloc(packed_bytes(dt, rows, n));
    if (!rc && !out->p) rc = tlmh_seterr(TLM_HIP_ENOMEM, "model: out of device memory");
    if (!rc) rc = launch_pack(dt, tmp, rb, rows, n, out->p, M->stream);
    if (!rc) rc = tlmh_check(hipStreamSynchronize(M->stream), "model: pack");
    (void)hipFree(tmp);
    return rc;
}

struct Packet {
    std::vector<uint8_t> buf;
    uint64_t off = 0, len = 0;
    const uint8_t *payload() const { return buf.data() + off; }
};

int read_packet(tlm_hip_manifest *m, int type, int layer, uint32_t id, Packet &p) {
    const tlm_hip_packet_loc *loc = tlm_hip_manifest_find(m, type, layer, id);
    if (!loc) return tlmh_seterr(TLM_HIP_ENOTFOUND, "model: no packet type %d layer %d id %u", type, layer, id);
    p.buf.resize(loc->total_len);
    return tlm_hip_packet_read(m, loc, p.buf.data(), &p.off, &p.len);
}

/* tensor `name` of a directory payload as an f32 vector on device (NULL if
 * absent and not required) - dir_vec, src/lib/tlm_model.c:274-292 */
int dev_vec(tlm_hip_model *M, const Packet &pk, const char *name, int64_t n, bool required, const float **out) {
    *out = nullptr;
    tlm_hip_tensor_ref t;
    int rc = tlm_hip_dir_find(pk.payload(), pk.len, name, &t);
    if (rc == TLM_HIP_ENOTFOUND)
        return required ? tlmh_seterr(TLM_HIP_ENOTFOUND, "model: tensor '%s' missing", name) : TLM_HIP_OK;
    if (rc) return rc;
    if (t.dtype != DT_F32 || t.shape[0] * t.shape[1] != (uint64_t)n || t.nbytes != (uint64_t)n * 4)
        return tlmh_seterr(TLM_HIP_EUNSUP, "model: tensor '%s' is not an f32 vector of %lld", name, (long long)n);
    void *p;
    if ((rc = dev_upload(M, pk.payload() + t.offset, (size_t)t.nbytes, &p))) return rc;
    *out = (const float *)p;
    return TLM_HIP_OK;
}

/* dir_mat, src/lib/tlm_model.c:246-272 */
int dir_mat(tlm_hip_model *M, const Packet &pk, const char *name, int64_t rows, int64_t cols, DevMat *out) {
    tlm_hip_tensor_ref t;
    int rc = tlm_hip_dir_find(pk.payload(), pk.len, name, &t);
    if (rc == TLM_HIP_ENOTFOUND) return tlmh_seterr(TLM_HIP_ENOTFOUND, "model: tensor '%s' missing", name);
    if (rc) return rc;
    const int dt = (int)t.dtype, bv = dt_block_values(dt);
    if ((int64_t)t.shape[0] != rows || (int64_t)t.shape[1] != cols || bv == 0 || cols % bv)
        return tlmh_seterr(TLM_HIP_EFORMAT, "model: tensor '%s' shape [%llu, %llu], expected [%lld, %lld]", name,
                           (unsigned long long)t.shape[0], (unsigned long long)t.shape[1], (long long)rows,
                           (long long)cols);
    if (t.nbytes != (uint64_t)rows * (uint64_t)(cols / bv) * (uint64_t)dt_block_bytes(dt))
        return tlmh_seterr(TLM_HIP_EFORMAT, "model: tensor '%s' byte count", name);
    return dev_matrix(M, dt, pk.payload() + t.offset, rows, cols, out);
}

/* tlm_yarn_transform, src/lib/tlm_model.c:453-484 (HF YaRN, f32 ramp) */
int yarn(std::vector<float> &inv_freq, uint32_t head_dim, double theta, double factor, double beta_fast,
         double beta_slow, uint32_t orig_len, bool truncate, float *attn_factor) {
    const int half = (int)head_dim / 2;
    if (head_dim < 2 || (head_dim & 1) || !(theta > 0.0) || !(factor > 0.0) || !(beta_fast > 0.0) ||
        beta_fast < beta_slow || orig_len == 0)
        return tlmh_seterr(TLM_HIP_EINVAL, "model: invalid rope scaling parameters");
    const double two_pi = 6.283185307179586;
    double low = (double)head_dim * log((double)orig_len / (beta_fast * two_pi)) / (2.0 * log(theta));
    double high = (double)head_dim * log((double)orig_len / (beta_slow * two_pi)) / (2.0 * log(theta));
    if (truncate) {
        low = floor(low);
        high = ceil(high);
    }
    if (low < 0.0) low = 0.0;
    if (high > (double)head_dim - 1.0) high = (double)head_dim - 1.0;
    if (low == high) high += 0.001;
    const double af = factor > 1.0 ? 0.1 * log(factor) + 1.0 : 1.0;
    for (int j = 0; j < half; j++) {
        const float extrap = inv_freq[j];
        const float pos_freq = 1.0f / extrap;
        const float interp = 1.0f / ((float)factor * pos_freq);
        float ramp = ((float)j - (float)low) / (float)(high - low);
        if (ramp < 0.0f) ramp = 0.0f;
        if (ramp > 1.0f) ramp = 1.0f;
        inv_freq[j] = interp * ramp + extrap * (1.0f - ramp);
    }
    *attn_factor = (float)af;
    return TLM_HIP_OK;
}

int load(tlm_hip_model *M, tlm_hip_manifest *m, const tlm_hip_model_opts *o) {
    tlm_hip_model_geom &g = M->g;
    g = *tlm_hip_manifest_geom(m);
    /* tlm_model.c:490-498 */
    if (g.n_layers == 0 || g.d_model == 0 || g.n_heads == 0 || g.n_kv_heads == 0 || g.head_dim == 0 ||
        (g.head_dim & 1) || g.n_heads % g.n_kv_heads || g.vocab == 0 || g.top_k > g.n_experts ||
        (g.n_experts > 0 && g.top_k == 0) || g.router > 2 || g.rope_scale > 2)
        return tlmh_seterr(TLM_HIP_EFORMAT, "model: unsupported geometry");
    if (g.n_experts == 0 || g.head_dim > 256 || g.head_dim % 32 || g.top_k > 32)
        return tlmh_seterr(TLM_HIP_EUNSUP, "model: needs routed experts (top_k <= 32) and head_dim a multiple of 32 "
                           "up to 256");
    if (!(g.routed_scale > 0.0f)) g.routed_scale = 1.0f;   /* tlm_model.c:503-505 */
    if (!(g.norm_eps > 0.0f)) g.norm_eps = 1e-6f;
    if (!(g.rope_theta > 0.0f)) g.rope_theta = 10000.0f;
    /* tlm_kv_new, tlm_model.c:646-650 */
    int max_ctx = o && o->max_ctx > 0 ? o->max_ctx : 0;
    if (max_ctx <= 0) max_ctx = g.max_ctx > 0 ? (int)g.max_ctx : 4096;
    if (g.max_ctx > 0 && max_ctx > (int)g.max_ctx) max_ctx = (int)g.max_ctx;
    M->max_ctx = max_ctx;
    M->graph_failed[0] = M->graph_failed[1] = o && o->eager;
    const int64_t D = g.d_model, hd = g.head_dim, H = g.n_heads, KV = g.n_kv_heads, E = g.n_experts;
    const int64_t de = g.d_expert, ds = g.n_shared > 0 ? g.d_shared : 0;

    int rc = tlmh_check(hipStreamCreateWithFlags(&M->stream, hipStreamNonBlocking), "model: stream");
    if (rc) return rc;
    /* RoPE tables for every position, in double as tlm_model.c:535, 1069-1073 */
    {
        const int half = (int)hd / 2;
        std::vector<float> inv(half);
        for (int j = 0; j < half; j++) inv[j] = (float)pow((double)g.rope_theta, -2.0 * (double)j / (double)hd);
        float attn_scale = 1.0f;
        if (g.rope_scale != 0 &&
            (rc = yarn(inv, g.head_dim, g.rope_theta, g.rope_factor, g.rope_beta_fast, g.rope_beta_slow,
                       g.rope_orig_len, g.rope_scale == 1, &attn_scale)))
            return rc;
        std::vector<float> cs((size_t)max_ctx * half), sn((size_t)max_ctx * half);
        for (int p = 0; p < max_ctx; p++)
            for (int j = 0; j < half; j++) {
                const double a = (double)p * (double)inv[j];
                cs[(size_t)p * half + j] = (float)cos(a) * attn_scale;
                sn[(size_t)p * half + j] = (float)sin(a) * attn_scale;
            }
        void *a, *b;
        if ((rc = dev_upload(M, cs.data(), cs.size() * 4, &a)) || (rc = dev_upload(M, sn.data(), sn.size() * 4, &b)))
            return rc;
        M->cs = (float *)a;
        M->sn = (float *)b;
    }
    M->L.resize(g.n_layers);
    for (uint32_t l = 0; l < g.n_layers; l++) {   /* load_layer, tlm_model.c:294-341 */
        Packet pk;
        if ((rc = read_packet(m, TLM_HIP_PK_DENSE, (int)l, 0, pk))) return rc;
        Layer &Ly = M->L[l];
        tlm_hip_tensor_ref t;
        if (tlm_hip_dir_find(pk.payload(), pk.len, "ffn_gate", &t) == TLM_HIP_OK)
            return tlmh_seterr(TLM_HIP_EUNSUP, "model: layer %u has a dense FFN", l);
        if ((rc = dev_vec(M, pk, "attn_norm", D, true, &Ly.attn_norm)) ||
            (rc = dev_vec(M, pk, "ffn_norm", D, true, &Ly.ffn_norm)) ||
            (rc = dev_vec(M, pk, "q_norm", hd, false, &Ly.q_norm)) ||
            (rc = dev_vec(M, pk, "k_norm", hd, false, &Ly.k_norm)) ||
            (rc = dir_mat(M, pk, "attn_q", H * hd, D, &Ly.q)) || (rc = dir_mat(M, pk, "attn_k", KV * hd, D, &Ly.k)) ||
            (rc = dir_mat(M, pk, "attn_v", KV * hd, D, &Ly.v)) || (rc = dir_mat(M, pk, "attn_o", D, H * hd, &Ly.o)))
            return rc;
        if (dt_act_kind(Ly.q.dt) != dt_act_kind(Ly.k.dt) || dt_act_kind(Ly.q.dt) != dt_act_kind(Ly.v.dt))
            return tlmh_seterr(TLM_HIP_EUNSUP, "model: q / k / v of layer %u take different activation kinds", l);
        tlm_hip_moe_desc &d = Ly.moe;
        d.D = D;
        d.de = de;
        d.E = (int32_t)E;
        d.k = (int32_t)g.top_k;
        d.router = (int32_t)g.router;
        d.routed_scale = g.routed_scale;
        d.eps = g.norm_eps;
        d.ffn_norm = Ly.ffn_norm;
        if ((rc = tlm_hip_dir_find(pk.payload(), pk.len, "router", &t))) return rc;
        if (t.dtype != DT_F32 || t.shape[0] != (uint64_t)E || t.shape[1] != (uint64_t)D)
            return tlmh_seterr(TLM_HIP_EUNSUP, "model: router of layer %u is not f32 [%lld x %lld]", l, (long long)E,
                               (long long)D);
        void *p;
        if ((rc = dev_upload(M, pk.payload() + t.offset, (size_t)t.nbytes, &p))) return rc;
        d.router_w = (const float *)p;
        if ((rc = dev_vec(M, pk, "router_bias", E, false, &d.router_bias))) return rc;
        if (ds > 0) {
            DevMat sg, su, sd;
            if ((rc = dir_mat(M, pk, "shared_gate", ds, D, &sg)) || (rc = dir_mat(M, pk, "shared_up", ds, D, &su)) ||
                (rc = dir_mat(M, pk, "shared_down", D, ds, &sd)) ||
                (rc = dev_vec(M, pk, "shared_gate_inp", D, false, &d.shared_gate_inp)))
                return rc;
            if (sg.dt != su.dt || sg.dt != sd.dt)
                return tlmh_seterr(TLM_HIP_EUNSUP, "model: shared expert matrices of mixed dtypes");
            d.ds = ds;
            d.shared_dt = sg.dt;
            d.sg = sg.p;
            d.su = su.p;
            d.sd = sd.p;
        }
    }
    /* experts (load_experts, tlm_model.c:343-392): every one resident, packed */
    std::vector<std::vector<const void *>> tables(g.n_layers, std::vector<const void *>(3 * E, nullptr));
    std::vector<std::vector<uint8_t>> masks(g.n_layers, std::vector<uint8_t>(E, 1));
    std::vector<int> edt(g.n_layers, -1);
    for (int i = 0; i < tlm_hip_manifest_n_packets(m); i++) {
        const tlm_hip_packet_loc *loc = tlm_hip_manifest_packet(m, i);
        if (loc->type != TLM_HIP_PK_EXPERT) continue;
        if (loc->layer >= g.n_layers || loc->id >= E)
            return tlmh_seterr(TLM_HIP_EFORMAT, "model: EXPERT packet %u:%u out of range", loc->layer, loc->id);
        if (loc->flags & 2u) continue;   /* pruned: never routable */
        Packet pk;
        pk.buf.resize(loc->total_len);
        if ((rc = tlm_hip_packet_read(m, loc, pk.buf.data(), &pk.off, &pk.len))) return rc;
        uint32_t dt32, off[3];
        tlm_hip_packet_header(pk.buf.data(), &dt32, off);
        const int dt = (int)dt32;
        if (edt[loc->layer] >= 0 && edt[loc->layer] != dt)
            return tlmh_seterr(TLM_HIP_EUNSUP, "model: layer %u mixes expert dtypes", loc->layer);
        edt[loc->layer] = dt;
        const int64_t shapes[3][2] = {{de, D}, {de, D}, {D, de}};
        for (int k = 0; k < 3; k++) {
            const int bv = dt_block_values(dt);
            if (bv == 0 || shapes[k][1] % bv) return tlmh_seterr(TLM_HIP_EUNSUP, "model: expert dtype %d", dt);
            const uint64_t raw = (uint64_t)shapes[k][0] * (uint64_t)(shapes[k][1] / bv) * (uint64_t)dt_block_bytes(dt);
            if ((uint64_t)off[k] + raw > pk.len)
                return tlmh_seterr(TLM_HIP_EFORMAT, "model: expert %u:%u item %d overruns", loc->layer, loc->id, k);
            DevMat dm;
            if ((rc = dev_matrix(M, dt, pk.payload() + off[k], shapes[k][0], shapes[k][1], &dm))) return rc;
            tables[loc->layer][3 * loc->id + k] = dm.p;
        }
        masks[loc->layer][loc->id] = 0;
    }
    for (uint32_t l = 0; l < g.n_layers; l++) {
        int live = 0;
        for (int64_t e = 0; e < E; e++) live += !masks[l][e];
        if (live < (int)g.top_k)   /* tlm_model.c:597-600 */
            return tlmh_seterr(TLM_HIP_EFORMAT, "model: layer %u has %d routable experts, needs top_k=%u", l, live,
                               g.top_k);
        /* absent experts point at a present one: never routed (masked), never read */
        const void *any[3] = {nullptr, nullptr, nullptr};
        for (int64_t e = 0; e < E && !any[0]; e++)
            if (!masks[l][e])
                for (int k = 0; k < 3; k++) any[k] = tables[l][3 * e + k];
        for (int64_t e = 0; e < E; e++)
            if (masks[l][e])
                for (int k = 0; k < 3; k++) tables[l][3 * e + k] = any[k];
        void *tp, *mp;
        if ((rc = dev_upload(M, tables[l].data(), tables[l].size() * sizeof(void *), &tp)) ||
            (rc = dev_upload(M, masks[l].data(), masks[l].size(), &mp)))
            return rc;
        Layer &Ly = M->L[l];
        Ly.moe.experts = (const void *const *)tp;
        Ly.moe.mask = (const uint8_t *)mp;
        Ly.moe.expert_dt = edt[l];
    }
    {   /* META: output_norm + lm_head */
        Packet pk;
        if ((rc = read_packet(m, TLM_HIP_PK_META, TLM_HIP_LAYER_NONE, 0, pk)) ||
            (rc = dev_vec(M, pk, "output_norm", D, true, &M->out_norm)) ||
            (rc = dir_mat(M, pk, "lm_head", g.vocab, D, &M->lm_head)))
            return rc;
    }
    {   /* EMBED: tok_embd rows stay in the reference layout (gathered per token) */
        Packet pk;
        if ((rc = read_packet(m, TLM_HIP_PK_EMBED, TLM_HIP_LAYER_NONE, 0, pk))) return rc;
        tlm_hip_tensor_ref t;
        if ((rc = tlm_hip_dir_find(pk.payload(), pk.len, "tok_embd", &t))) return rc;
        const int dt = (int)t.dtype;
        if ((dt != DT_F32 && dt != DT_Q8_0) || t.shape[0] != g.vocab || t.shape[1] != (uint64_t)D || D % 32)
            return tlmh_seterr(TLM_HIP_EUNSUP, "model: embedding dtype %d", dt);
        M->embd_dt = dt;
        M->embd_row = dt == DT_F32 ? (size_t)D * 4 : (size_t)(D / 32) * 34;
        if (t.nbytes != (uint64_t)M->embd_row * g.vocab) return tlmh_seterr(TLM_HIP_EFORMAT, "model: embedding bytes");
        void *p;
        if ((rc = dev_upload(M, pk.payload() + t.offset, (size_t)t.nbytes, &p))) return rc;
        M->embd = (const uint8_t *)p;
    }
    /* KV cache, scratch (alloc_scratch, tlm_model.c:402-446) */
    const size_t per = (size_t)g.n_layers * KV * (size_t)max_ctx * hd;
    M->kc = (float *)M->dalloc(per * 4);
    M->vc = (float *)M->dalloc(per * 4);
    M->scores = (float *)M->dalloc((size_t)H * max_ctx * 4);
    M->h = (float *)M->dalloc((size_t)D * 4);
    M->xb = (float *)M->dalloc((size_t)D * 4);
    M->xb2 = (float *)M->dalloc((size_t)D * 4);
    M->q = (float *)M->dalloc((size_t)H * hd * 4);
    M->kx = (float *)M->dalloc((size_t)KV * hd * 4);
    M->vx = (float *)M->dalloc((size_t)KV * hd * 4);
    M->att = (float *)M->dalloc((size_t)H * hd * 4);
    M->logits = (float *)M->dalloc((size_t)g.vocab * 4);
    const int64_t amax = D > H * hd ? D : H * hd;
    M->act = (uint8_t *)M->dalloc(act_bytes(DT_Q8_K, amax) + act_bytes(DT_Q8_0, amax) + 64);
    M->act2 = (uint8_t *)M->dalloc(act_bytes(DT_Q8_K, amax) + act_bytes(DT_Q8_0, amax) + 64);
    size_t ws = 0;
    for (const Layer &Ly : M->L) ws = std::max(ws, tlm_hip_moe_workspace_bytes(&Ly.moe));
    M->moe_ws = (uint8_t *)M->dalloc(ws + 256);
    M->st = (int32_t *)M->dalloc(16);
    M->seq = (int32_t *)M->dalloc(((size_t)max_ctx + 1) * 4);
    M->ids = (int32_t *)M->dalloc(32 * 4);
    M->w = (float *)M->dalloc(32 * 4);
    for (void *p : {(void *)M->kc, (void *)M->vc, (void *)M->scores, (void *)M->h, (void *)M->xb, (void *)M->xb2,
                    (void *)M->q, (void *)M->kx, (void *)M->vx, (void *)M->att, (void *)M->logits, (void *)M->act,
                    (void *)M->act2, (void *)M->moe_ws, (void *)M->st, (void *)M->seq, (void *)M->ids,
                    (void *)M->w})
        if (!p) return tlmh_seterr(TLM_HIP_ENOMEM, "model: out of device memory for the KV cache / scratch");
    if ((rc = tlmh_check(hipHostMalloc((void **)&M->host_tok, 64, hipHostMallocDefault), "model: pinned scratch")))
        return rc;
    if ((rc = tlmh_check(hipMemset(M->st, 0, 16), "model: position"))) return rc;
    return tlmh_check(hipStreamSynchronize(M->stream), "model: load");
}

/* one matrix-vector job with the activation of x quantised for the matrix's kind */
int matvec(tlm_hip_model *M, const DevMat &W, const float *x, uint8_t *act, float *y) {
    int rc = launch_quantize_act(dt_act_kind(W.dt), x, W.n, act, M->stream);
    if (!rc) rc = launch_matvec_packed(W.dt, W.p, W.rows, W.n, act, y, M->stream);
    return rc;
}

/* tlm_model_step, src/lib/tlm_model.c:1058-1103, enqueued: the token is
 * seq[pos], pos = st[0]; with logits, the greedy next token goes to
 * seq[pos + 1]; st[0] advances.  Every argument is the same at every position
 * (the step is captured once as a graph). */
int enqueue_step(tlm_hip_model *M, bool want_logits) {
    const tlm_hip_model_geom &g = M->g;
    const int D = (int)g.d_model, hd = (int)g.head_dim, H = (int)g.n_heads, KV = (int)g.n_kv_heads;
    hipStream_t s = M->stream;
    hipLaunchKernelGGL(k_embed, dim3((D + NT - 1) / NT), dim3(NT), 0, s, M->embd, M->embd_row, M->embd_dt,
                       (const int32_t *)M->seq, (const int32_t *)M->st, D, M->h);
    int rc = tlmh_check(hipGetLastError(), "model: embed");
    for (uint32_t l = 0; l < g.n_layers && !rc; l++) {
        const Layer &Ly = M->L[l];
        /* attention(), tlm_model.c:730-763 */
        hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(NT), 0, s, (const float *)M->h, Ly.attn_norm, D, g.norm_eps,
                           M->xb);
        rc = launch_quantize_act(dt_act_kind(Ly.q.dt), M->xb, D, M->act, s);
        if (!rc) rc = launch_matvec_packed(Ly.q.dt, Ly.q.p, Ly.q.rows, Ly.q.n, M->act, M->q, s);
        if (!rc) rc = launch_matvec_packed(Ly.k.dt, Ly.k.p, Ly.k.rows, Ly.k.n, M->act, M->kx, s);
        if (!rc) rc = launch_matvec_packed(Ly.v.dt, Ly.v.p, Ly.v.rows, Ly.v.n, M->act, M->vx, s);
        if (rc) break;
        const size_t lbase = (size_t)l * KV * M->max_ctx * hd;
        hipLaunchKernelGGL(k_qk_rope, dim3(H + KV), dim3(64), 0, s, M->q, M->kx, (const float *)M->vx, Ly.q_norm,
                           Ly.k_norm, (const float *)M->cs, (const float *)M->sn, M->kc + lbase, M->vc + lbase, H,
                           hd, (const int32_t *)M->st, M->max_ctx, g.norm_eps);
        hipLaunchKernelGGL(k_attn, dim3(H), dim3(NT), 0, s, (const float *)M->q, (const float *)(M->kc + lbase),
                           (const float *)(M->vc + lbase), M->scores, M->att, H, KV, hd, M->max_ctx,
                           (const int32_t *)M->st);
        rc = tlmh_check(hipGetLastError(), "model: attention");
        if (!rc) rc = matvec(M, Ly.o, M->att, M->act2, M->xb2);
        if (rc) break;
        hipLaunchKernelGGL(k_add, dim3((D + NT - 1) / NT), dim3(NT), 0, s, M->h, (const float *)M->xb2, D);
        /* moe(), tlm_model.c:940-1055 */
        rc = launch_moe_layer(&Ly.moe, M->h, M->ids, M->w, M->moe_ws, s);
    }
    if (rc) return rc;
    if (want_logits) {   /* tlm_model.c:1087-1095, then the greedy argmax */
        hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(NT), 0, s, (const float *)M->h, M->out_norm, D, g.norm_eps,
                           M->xb);
        rc = matvec(M, M->lm_head, M->xb, M->act, M->logits);
        if (rc) return rc;
        hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, s, (const float *)M->logits, (int)g.vocab, M->seq,
                           (const int32_t *)M->st);
    }
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, s, M->st);
    return tlmh_check(hipGetLastError(), "model: step");
}

/* One step (the caller checked the context): the captured graph of the kind,
 * captured at first use; eager launches if capture is unavailable. */
int step(tlm_hip_model *M, bool want_logits) {
    const int k = want_logits ? 1 : 0;
    if (!M->graph[k] && !M->graph_failed[k]) {
        hipGraph_t gr = nullptr;
        int rc = tlmh_check(hipStreamBeginCapture(M->stream, hipStreamCaptureModeThreadLocal), "model: capture");
        if (!rc) {
            const int rc_enq = enqueue_step(M, want_logits);
            rc = tlmh_check(hipStreamEndCapture(M->stream, &gr), "model: capture");
            if (!rc) rc = rc_enq;
        }
        if (!rc) rc = tlmh_check(hipGraphInstantiate(&M->graph[k], gr, nullptr, nullptr, 0), "model: instantiate");
        if (gr) (void)hipGraphDestroy(gr);
        if (rc) {
            M->graph[k] = nullptr;
            M->graph_failed[k] = true;
            (void)hipGetLastError();
        }
    }
    int rc = M->graph[k] ? tlmh_check(hipGraphLaunch(M->graph[k], M->stream), "model: step graph")
                         : enqueue_step(M, want_logits);
    if (!rc) M->kv_len++;
    return rc;
}

}  // namespace

extern "C" {

int tlm_hip_model_open(const char *manifest_path, const tlm_hip_model_opts *o, tlm_hip_model **out) {
    if (!manifest_path || !out) return tlmh_seterr(TLM_HIP_EINVAL, "model open: NULL argument");
    *out = nullptr;
    if (tlmh_current_device() < 0) return tlmh_seterr(TLM_HIP_EUNSUP, "model open: tlm_hip_init has not run");
    tlm_hip_manifest *m = nullptr;
    int rc = tlm_hip_manifest_load(manifest_path, &m);
    if (rc) return rc;
    tlm_hip_model *M = new tlm_hip_model;
    rc = load(M, m, o);
    tlm_hip_manifest_free(m);
    if (rc) {
        delete M;
        return rc;
    }
    *out = M;
    return TLM_HIP_OK;
}

void tlm_hip_model_close(tlm_hip_model *M) { delete M; }

const tlm_hip_model_geom *tlm_hip_model_geom_of(const tlm_hip_model *M) { return M ? &M->g : nullptr; }
int tlm_hip_model_kv_len(const tlm_hip_model *M) { return M ? M->kv_len : 0; }
int tlm_hip_model_kv_capacity(const tlm_hip_model *M) { return M ? M->max_ctx : 0; }
void tlm_hip_model_reset(tlm_hip_model *M) {
    if (!M) return;
    M->kv_len = 0;
    M->host_tok[2] = 0;
    (void)hipMemcpyAsync(M->st, M->host_tok + 2, 4, hipMemcpyHostToDevice, M->stream);
    (void)hipStreamSynchronize(M->stream);
}

/* tlm_model_step: one token; logits (host, vocab floats) and the greedy next
 * token (argmax) when asked for. */
int tlm_hip_model_step(tlm_hip_model *M, int token, float *logits, int32_t *next) {
    if (!M) return tlmh_seterr(TLM_HIP_EINVAL, "model step: NULL");
    if (token < 0 || (uint32_t)token >= M->g.vocab) return tlmh_seterr(TLM_HIP_EINVAL, "token %d out of range", token);
    if (M->kv_len >= M->max_ctx) return tlmh_seterr(TLM_HIP_ERANGE, "context full (%d tokens)", M->max_ctx);
    const int pos = M->kv_len;
    M->host_tok[0] = token;
    int rc = tlmh_check(hipMemcpyAsync(M->seq + pos, M->host_tok, 4, hipMemcpyHostToDevice, M->stream), "model: token");
    if (!rc) rc = step(M, logits || next);
    if (!rc && logits)
        rc = tlmh_check(hipMemcpyAsync(logits, M->logits, (size_t)M->g.vocab * 4, hipMemcpyDeviceToHost, M->stream),
                        "model: logits");
    if (!rc && next)
        rc = tlmh_check(hipMemcpyAsync(M->host_tok + 1, M->seq + pos + 1, 4, hipMemcpyDeviceToHost, M->stream),
                        "model: next token");
    if (!rc) rc = tlmh_check(hipStreamSynchronize(M->stream), "model: step");
    if (!rc && next) *next = M->host_tok[1];
    return rc;
}

/* tlm_model_prefill (src/lib/tlm_model.c:1105-1113) then n_gen greedy tokens
 * (tierlm bench's loop, src/bin/tierlm.c:720-729): the prompt is written to
 * the device once, each step's token is read there and each greedy token is
 * written there by the previous step; out receives the n_gen tokens. */
int tlm_hip_model_generate(tlm_hip_model *M, const int32_t *prompt, int n_prompt, int n_gen, int32_t *out) {
    if (!M || !prompt || n_prompt <= 0 || n_gen < 0 || (n_gen > 0 && !out))
        return tlmh_seterr(TLM_HIP_EINVAL, "model generate: bad arguments");
    const int pos0 = M->kv_len;
    if ((int64_t)pos0 + n_prompt + (n_gen > 0 ? n_gen - 1 : 0) > M->max_ctx)
        return tlmh_seterr(TLM_HIP_ERANGE, "model generate: %d + %d tokens exceed the context (%d)", n_prompt, n_gen,
                           M->max_ctx);
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || (uint32_t)prompt[i] >= M->g.vocab)
            return tlmh_seterr(TLM_HIP_EINVAL, "token %d out of range", prompt[i]);
    int rc = tlmh_check(hipMemcpy(M->seq + pos0, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice), "model: prompt");
    for (int i = 0; i < n_prompt && !rc; i++) rc = step(M, i == n_prompt - 1);
    for (int gi = 1; gi < n_gen && !rc; gi++) rc = step(M, true);
    if (!rc && n_gen > 0)
        rc = tlmh_check(hipMemcpyAsync(out, M->seq + pos0 + n_prompt, (size_t)n_gen * 4, hipMemcpyDeviceToHost,
                                       M->stream), "model: out");
    if (!rc) rc = tlmh_check(hipStreamSynchronize(M->stream), "model: generate");
    return rc;
}

}  // extern "C"
