/* tlm_oracle.h - CPU restatement of the reference's quantised-MoE decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * of the HIP path, never as the thing measured or shipped.
 *
 * Every function follows a reference function, cited as file:line against
 * the reference tree (src/lib/...).  The dtype codes are the reference's
 * tlm_dtype values (src/lib/tlm_quant.h:31-42).
 *
 * Byte layouts (little endian, values per block in brackets):
 *   Q8_0 weight [32]  34 B : f16 d, int8 q[32]
 *   Q4_K        [256] 144 B: f16 d, f16 dmin, u8 scales[12], u8 qs[128]
 *   Q5_K        [256] 176 B: f16 d, f16 dmin, u8 scales[12], u8 qh[32], u8 qs[128]
 *   Q6_K        [256] 210 B: u8 ql[128], u8 qh[64], int8 sc[16], f16 d
 *   Q8_K        [256] 292 B: f32 d, int8 q[256], int16 bsums[16]   (activation)
 *   a8 (Q8_0 activation) [32] 36 B: f32 d, int8 q[32]
 *
 * Pinning status of each function (how a mistake in it would be caught) is
 * listed in the header of tlm_oracle.c.
 */
#ifndef TLM_ORACLE_H
#define TLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2, ORC_Q8_0 = 8, ORC_Q4_K = 12,
    ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_Q8_K = 15
};

/* ---- formats (src/lib/tlm_quant.c:52-63, 106-110, 689-715) ---------------- */
int      orc_block_values(int dt);
size_t   orc_block_bytes(int dt);
size_t   orc_row_bytes(int dt, int64_t n);          /* 0: bad dtype or n */
size_t   orc_qact_bytes(int kind, int64_t n);
int      orc_act_kind_for(int dt);
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

/* ---- quantisers (src/lib/tlm_quant.c:275-506, 563-587, 699-707) --------- */
int  orc_quantize_row(int dt, const float *x, void *dst, int64_t n);   /* 0 or -1 */
int  orc_dequantize_row(int dt, const void *src, float *y, int64_t n);
void orc_quantize_act(int kind, const float *x, int64_t n, void *dst);

/* ---- dot / matvec (src/lib/tlm_quant.c:721-902, 1104-1143) ---------------- */
float orc_vec_dot(int dt, const void *wrow, const void *act, int64_t n);   /* NaN on bad args */
void  orc_matvec_rows(int dt, const void *W, size_t row_bytes, const void *act,
                      float *y, int64_t n, int64_t r0, int64_t r1);
/* Integer part of one block of a row dot: the exact int32 the fma chain
 * consumes (isum), and for Q4_K / Q5_K the min sum (msum). */
void  orc_block_isum(int dt, const void *wblock, const void *act_block,
                     int32_t *isum, int32_t *msum);

/* ---- decoder glue (src/lib/tlm_model.c:164-172, 776-839) ------------------ */
void  orc_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps);
void orc_expf_many(const float *x, float *y, int64_t n);
uint64_t orc_exp2_tab(int i);
float orc_expf_published(float x, int fused);
void orc_expf_published_many(const float *x, float *y, int64_t n, int fused);
float orc_silu(float x);
float orc_sigmoid(float x);
void  orc_topk(const float *v, const uint8_t *mask, int E, int k, int *ids);
/* router: 0 softmax + renormalise, 1 softmax, 2 sigmoid + bias (selection only).
 * `logits` is read only (the reference scribbles on its copy). */
void  orc_route(int router, const float *logits, const uint8_t *mask, const float *bias,
                int E, int k, float routed_scale, int *ids, float *w);

/* ---- one MoE block (src/lib/tlm_model.c:900-1055) ------------------------- */
typedef struct {
    int64_t D, de, ds;          /* d_model, expert width, shared width (0 = none) */
    int     E, k, router;       /* experts, top-k, router kind as orc_route */
    float   routed_scale, eps;
    const float   *ffn_norm;    /* [D] */
    int            router_dt;   /* ORC_F32 in every compiled model */
    const void    *router_w;    /* [E x D], row stride orc_row_bytes(router_dt, D) */
    const float   *router_bias; /* [E] or NULL (router 2) */
    const uint8_t *mask;        /* [E] 1 = pruned, or NULL */
    int            expert_dt;
    const void *const *gate;    /* [E] rows de x D */
    const void *const *up;      /* [E] rows de x D */
    const void *const *down;    /* [E] rows D x de */
    int            shared_dt;
    const void    *sg, *su, *sd;       /* ds x D, ds x D, D x ds  (ds > 0) */
    const float   *shared_gate_inp;    /* [D] or NULL (sigmoid gate) */
} orc_moe_desc;

/* Optional intermediates; any pointer may be NULL. */
typedef struct {
    float   *xb;        /* [D] normed input */
    float   *logits;    /* [E] */
    float   *gu;        /* [k][2*de] gate | up */
    float   *hh;        /* [k][de] silu(g)*u */
    uint8_t *hq;        /* [k][orc_qact_bytes(kind, de)] quantised hh */
    float   *eo;        /* [k][D] down outputs */
    float   *s_out;     /* [D] shared expert output */
    float   *ffn;       /* [D] combined FFN output */
} orc_moe_trace;

/* h[D] += MoE(h).  ids[k], w[k] receive the routing.  Returns 0. */
int orc_moe_layer(const orc_moe_desc *d, float *h, int *ids, float *w, orc_moe_trace *tr);

#ifdef __cplusplus
}
#endif
#endif
