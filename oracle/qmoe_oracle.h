/*
 * qmoe_oracle.h -- CPU restatement of the reference MoE FFN layer semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it.  The product library (libqmoe) never links, loads or calls it.
 *
 * What it restates (reference citations are into rye-001/Qwenium):
 *   - the op order of MoELayer::build, src/layers/moe.cpp:55-177
 *     (router mul_mat :72, argsort DESC + view :77-82, get_rows + soft_max
 *     :88-94, 3x mul_mat_id :105-127, silu*up :117, weight + k-ordered sum
 *     :134-151, shared expert + sigmoid gate :161-174);
 *   - the top-k + softmax oracle of tests/unit/test_moe.cpp:31-50;
 *   - the tensor roles and shapes of src/core/model.h:110-119;
 *   - RMSNorm of src/layers/norm.cpp:15-26 (ggml_rms_norm + mul);
 *   - the Q8_0 block layout read by src/cli/tensor_tracer.h:57-73.
 * The arithmetic itself lives in ggml (llama.cpp tag b8390, fetched at
 * configure time by CMakeLists.txt:50-55 and absent offline).  Its published
 * semantics are restated here:
 *   - Q4_0 / Q8_0 block formats (ggml-common.h): 18 / 34 bytes per 32 values;
 *   - quantize_row_q4_0_ref / quantize_row_q8_0_ref (ggml-quants.c) for weights;
 *   - quantize_row_q8_0 of the x86 AVX2 CPU backend for activations
 *     (d = amax/127 stored as fp16, q = round-to-nearest-even(x * 127/amax));
 *   - vec_dot_q4_0_q8_0 / vec_dot_q8_0_q8_0: per block fp32(d_w)*fp32(d_x)*isum.
 *
 * Deliberate choices where ggml's result depends on its SIMD summation order
 * (unverifiable offline):
 *   - router logits are the correctly rounded f32 of the exact dot product
 *     (f64 accumulation of exact f32*f32 products);
 *   - quantized dots are the correctly rounded f32 of the exact block sum
 *     (every block term d_w*d_x*isum is exact in f64 and the 64-block sum is
 *     exact in f64 for the scale ranges of these layers);
 *   - exp() used by silu / sigmoid / softmax is qo_exp_det(): a fixed sequence
 *     of IEEE f64 operations (Cody-Waite reduction + degree-13 Taylor) so the
 *     value is reproducible on any IEEE machine; it agrees with libm exp to
 *     ~1 ulp (pinned by tests/test_oracle_kat.py).
 * ggml's own f32 accumulation differs from these exact values by ~1e-6
 * relative, far inside the layer tolerance (2e-3 x output RMS).
 *
 * The Gemma 4 GeGLU variant (Gemma4ForwardPass::build_moe_geglu,
 * src/models/gemma4.cpp:367-445, inputs prepared at :549-564):
 *   - gelu is ggml's CPU ggml_vec_gelu_f32 with GGML_GELU_FP16 (vec.h of the
 *     same ggml tag; the reference's tests/unit/test_ffn.cpp:172-175 notes the
 *     f16 table): x <= -10 -> 0, x >= 10 -> x, else the entry of a table
 *     indexed by fp16(x) that holds fp16(gelu_f32(x16)), with
 *     gelu_f32(x) = 0.5f*x*(1 + tanhf(0.7978845608f*x*(1 + 0.044715f*x*x)))
 *     in f32 (libm tanhf); then gelu(g)*u in f32 (ggml_mul, :423);
 *   - gate and up are the two halves of one [n_embd, 2*ffn, E] tensor
 *     (views at :403-409: gate rows 0..F-1, up rows F..2F-1 of each expert);
 *   - the router reads its own input (:380): router_in =
 *     ((rms_norm(x) * (1/sqrtf(n_embd))) * ffn_gate_inp.scale), three f32
 *     roundings (ggml_rms_norm, ggml_scale, ggml_mul, :561-563), while the
 *     experts read rms_norm(x) * pre_ffw_norm_2 (:555-557).
 */
#ifndef QMOE_ORACLE_H
#define QMOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids as stored in GGUF (gguf_loader.cpp:490 reads them). */
enum { QO_TYPE_F32 = 0, QO_TYPE_Q4_0 = 2, QO_TYPE_Q8_0 = 8 };

/* ---- scalar helpers -------------------------------------------------- */
uint16_t qo_fp32_to_fp16(float f);           /* IEEE binary16, round to nearest even */
float    qo_fp16_to_fp32(uint16_t h);
double   qo_exp_det(double x);               /* deterministic exp */
double   qo_log_det(double x);               /* deterministic log, x > 0 */
double   qo_cospi2_det(double u);            /* deterministic cos(2*pi*u), u in [0,1) */

/* ---- seeded synthetic data (portable counter-based RNG) ---------------- */
uint64_t qo_hash3(uint64_t seed, uint64_t stream, uint64_t ctr);
double   qo_normal(uint64_t seed, uint64_t stream, uint64_t idx);   /* N(0,1) */
void     qo_gen_normal_f32(uint64_t seed, uint64_t stream, double mean, double sigma,
                           float* out, int64_t n);

/* ---- block formats ---------------------------------------------------- */
size_t qo_type_block_bytes(int type);        /* 18 (Q4_0), 34 (Q8_0), 4 (F32 per value) */
size_t qo_row_bytes(int type, int64_t n);    /* bytes of a row of n values */
void   qo_quantize_q4_0(const float* x, void* dst, int64_t n);      /* ggml ref */
void   qo_quantize_q8_0(const float* x, void* dst, int64_t n);      /* ggml ref */
void   qo_quantize_q8_0_act(const float* x, void* dst, int64_t n);  /* ggml x86 SIMD */
void   qo_dequantize(int type, const void* src, float* dst, int64_t n);
/* quantized row . Q8_0 activation row (n values): correctly rounded exact value */
float  qo_vec_dot(int wtype, const void* wrow, const void* xq8, int64_t n);
/* the same dot, returned as the exact f64 value before rounding */
double qo_vec_dot_f64(int wtype, const void* wrow, const void* xq8, int64_t n);

/* ---- layer pieces ----------------------------------------------------- */
float qo_dot_f32_exact(const float* a, const float* b, int64_t n);
void  qo_router_logits(const float* w_router /*[E][H]*/, const float* x /*[T][H]*/,
                       int T, int H, int E, float* logits /*[T][E]*/);
void  qo_topk_softmax(const float* logits, int T, int E, int k,
                      int32_t* idx /*[T][k]*/, float* w /*[T][k]*/);
/* Per-expert lists in ggml mul_mat_id order: ascending (token, slot).
 * offsets[E+1] exclusive prefix of counts; rows[T*k] holds t*k+j;
 * pos[T*k] is the inverse map (position of assignment t*k+j). */
void  qo_sort_assignments(const int32_t* idx, int T, int E, int k,
                          int32_t* offsets, int32_t* rows, int32_t* pos);
float qo_silu_mul(float g, float u);         /* silu(g)*u via qo_exp_det */
float qo_gelu_f16(float x);                  /* ggml CPU gelu (fp16 table semantics) */
float qo_geglu_mul(float g, float u);        /* qo_gelu_f16(g)*u in f32 */
float qo_sigmoid(float g);
void  qo_rms_norm(const float* x, const float* w, int T, int H, float eps, float* y);
/* The RMSNorm sum of squares in pieces of 32 columns, in the library's fixed
 * order (no reference counterpart: ggml_rms_norm, norm.cpp:15-26, sums inside
 * the op): run r = f64(f32(x[4r]^2)) + ... + f64(f32(x[4r+3]^2)) in column
 * order (columns >= H skipped), entry c = ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7))
 * over runs 8c .. 8c+7.  out[T][ceil(H/32)]. */
void  qo_rms_partials(const float* x, int T, int H, double* out);
/* Gemma 4 MoE inputs from one residual row (gemma4.cpp:555-563):
 * expert_in = (x*scale)*w_pre, router_in = ((x*scale)*(1/sqrtf(H)))*w_rs. */
void  qo_gemma4_moe_inputs(const float* x, const float* w_pre, const float* w_rs, int T, int H, float eps,
                           float* expert_in, float* router_in);

/* ---- whole layer ------------------------------------------------------ */
typedef struct qo_layer {
    int n_embd, n_experts, top_k, ffn_dim, has_shared_expert;
    int expert_type;                 /* Q4_0 or Q8_0 for all expert + shared matrices */
    const float* w_router;           /* [E][H] f32 */
    const void*  w_gate;             /* E x F rows of H values */
    const void*  w_up;               /* E x F rows of H values */
    const void*  w_down;             /* E x H rows of F values */
    const void*  w_sh_gate;          /* F rows of H values */
    const void*  w_sh_up;            /* F rows of H values */
    const void*  w_sh_down;          /* H rows of F values */
    const float* w_sh_norm;          /* [H] f32 shared-expert gate vector */
    int act;                         /* QO_ACT_SILU (SwiGLU) or QO_ACT_GELU_TANH (GeGLU) */
    int gate_up_fused;               /* 1: w_gate holds E x 2F rows (gate rows, then up rows, per expert) */
} qo_layer;

enum { QO_ACT_SILU = 0, QO_ACT_GELU_TANH = 1 };

typedef struct qo_debug {            /* every pointer optional (NULL) */
    float*   logits;                 /* [T][E] */
    int32_t* topk_idx;               /* [T][k] */
    float*   topk_w;                 /* [T][k] */
    float*   sh_gate;                /* [T] sigmoid(w_sh . x) */
    int32_t* offsets;                /* [E+1] */
    int32_t* rows;                   /* [T*k] */
    float*   h;                      /* [T*k][F] SwiGLU activations, (t,j) order */
    float*   y;                      /* [T*k][H] down outputs before weighting, (t,j) order */
    float*   sh_out;                 /* [T][H] shared down output before gating */
    float*   sh_h;                   /* [T][F] shared expert's h = act(g)*u (before its Q8_0) */
} qo_debug;

/* y[T][H] = MoE(x[T][H]).  nthreads <= 0 selects the OpenMP default.
 * Returns 0 on success, nonzero on invalid arguments. */
int qo_moe_forward(const qo_layer* L, const float* x, int T, float* y,
                   qo_debug* dbg, int nthreads);
/* The same with the router reading xr[T][H] (x feeds the experts). */
int qo_moe_forward_routed(const qo_layer* L, const float* x, const float* xr, int T, float* y,
                          qo_debug* dbg, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
