/*
 * qmoe.h -- C ABI of the MI355X-native MoE FFN layer (libqmoe.so).
 *
 * Drop-in for the reference's MoE layer module (rye-001/Qwenium):
 *   MoELayer::Hparams          src/layers/moe.h:34-39
 *   MoELayer::MoELayer(...)    src/layers/moe.h:44-53, src/layers/moe.cpp:27-53
 *   MoELayer::build(...)       src/layers/moe.h:58-63, src/layers/moe.cpp:55-177
 *   build_rms_norm(...)        src/layers/norm.h:10-15, src/layers/norm.cpp:15-26
 * Weight roles/shapes follow TransformerBlock's MoE slots,
 * src/core/model.h:110-119, in GGUF block layout (ggml ne/nb conventions).
 *
 * Conventions
 *   - All tensor data and activation pointers are DEVICE pointers.
 *   - Every call returns QMOE_OK (0) or a QMOE_ERR_* code; the message of the
 *     last failure on the calling thread is qmoe_last_error().  Messages name
 *     the slot/parameter, the expected value and the actual value, in that
 *     order (the reference's fail-loud contract, src/qinf_error.h:1-29).
 *   - Work is enqueued on the caller's HIP stream; no host synchronisation
 *     happens inside qmoe_layer_forward.
 *   - A layer (and a workspace) is not thread-safe; calls that share a
 *     workspace must be ordered on one stream.
 */
#ifndef QMOE_H
#define QMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids, as stored in GGUF (read at gguf_loader.cpp:490). */
enum qmoe_type {
    QMOE_TYPE_F32  = 0,
    QMOE_TYPE_Q4_0 = 2,
    QMOE_TYPE_Q8_0 = 8
};

enum qmoe_status {
    QMOE_OK           = 0,
    QMOE_ERR_NULL     = 1,  /* required pointer was NULL */
    QMOE_ERR_SHAPE    = 2,  /* ne/nb/dimension mismatch */
    QMOE_ERR_TYPE     = 3,  /* unsupported or mismatched ggml type */
    QMOE_ERR_VALUE    = 4,  /* bad hparam / argument value */
    QMOE_ERR_CAPACITY = 5,  /* n_tokens above the workspace capacity */
    QMOE_ERR_HIP      = 6,  /* a HIP runtime call failed */
    QMOE_ERR_SYNC     = 7   /* reserved: no kernel waits on another workgroup, so
                               no forward returns it */
};

/* A borrowed ggml tensor view: device data + ggml type + ne/nb (ne[0] contiguous).
 * Replaces the ggml_tensor* slots of MoELayer::MoELayer (moe.h:44-53). */
typedef struct qmoe_tensor {
    const void* data;
    int32_t     type;      /* enum qmoe_type */
    int32_t     n_dims;    /* 1..3 */
    int64_t     ne[4];
    uint64_t    nb[4];     /* byte strides */
} qmoe_tensor;

/* Mirrors MoELayer::Hparams (moe.h:34-39). */
typedef struct qmoe_hparams {
    int32_t n_experts;
    int32_t top_k;
    int32_t ffn_dim;
    int32_t has_shared_expert;
} qmoe_hparams;

/* Optional device-side copies of the intermediates that the reference names
 * moe_logits / moe_idx / moe_weights (moe.cpp:73,83,95) plus the per-expert
 * row lists that ggml_mul_mat_id builds internally.  Any pointer may be NULL. */
typedef struct qmoe_debug {
    float*   logits;    /* [T][n_experts] router logits */
    int32_t* topk_idx;  /* [T][top_k] expert ids, descending logit, ties -> lowest id */
    float*   topk_w;    /* [T][top_k] softmax over the selected logits */
    float*   sh_gate;   /* [T] sigmoid(w_sh_norm . x); only with a shared expert */
    int32_t* offsets;   /* [n_experts+1] exclusive prefix of per-expert counts */
    int32_t* rows;      /* [T*top_k] assignment t*top_k+j, grouped by expert,
                           ascending (token, slot) inside each group */
    /* Batched-router internals, written only when the forward routed through
     * the bf16-MFMA router (large token counts): its approximate logits and a
     * bound with |router_approx - logits| <= router_bound elementwise.  No
     * counterpart in the reference. */
    float*   router_approx; /* [T][n_experts] */
    float*   router_bound;  /* [T][n_experts] */
    /* The Q8_0 of h = silu(gate) * up (GeGLU: gelu(gate) * up) as the down
     * projection reads it: the reference's moe_exp_act (moe.cpp:117-118),
     * which ggml's mul_mat_id quantizes for the down GEMM (:127), and the
     * shared expert's sh_act (:163-164).  Rows: assignment t*top_k + j, then
     * with a shared expert one row per token (row T*top_k + t).  Written on
     * every path. */
    int8_t*  h_qs;      /* [T*top_k + S*T][ffn_dim] quants */
    float*   h_d;       /* [T*top_k + S*T][ffn_dim/32] block scales (fp16 values) */
    /* [1] h blocks whose f32 rounding the large-token-count (f16-MFMA) path
     * could not settle and recomputed exactly; 0 on the other paths.  No
     * counterpart in the reference. */
    int32_t* h_fixed;
    /* [T*top_k + S*T][n_embd] the unweighted expert rows, the reference's
     * moe_exp_down (moe.cpp:127-128) and moe_shared_out (:165), same row
     * order as h.  Written only where the forward materializes them (the
     * f16-MFMA path and the streaming path without the fused combine); at
     * decode sizes the combine consumes them in registers and this buffer is
     * left as it was. */
    float*   exp_down;
} qmoe_debug;

typedef struct qmoe_layer qmoe_layer;
typedef struct qmoe_workspace qmoe_workspace;

/* Thread-local text of the last failure ("" if none). */
const char* qmoe_last_error(void);

/* Replaces MoELayer::MoELayer (moe.h:44-53, moe.cpp:27-53).  Slots in the
 * reference's order.  w_router [n_embd, n_experts] F32; w_exp_gate/up
 * [n_embd, ffn_dim, n_experts] and w_exp_down [ffn_dim, n_embd, n_experts]
 * Q4_0 or Q8_0; w_sh_gate/up [n_embd, ffn_dim], w_sh_down [ffn_dim, n_embd]
 * (same types as the routed gate/up and down); w_sh_norm [n_embd] F32.
 * w_sh_* must be non-NULL iff hp->has_shared_expert.  Weights are borrowed:
 * they must outlive the layer.  The layer is bound to the current device.
 * n_embd and ffn_dim: multiples of 32 (whole Q4_0/Q8_0 blocks) up to 4096.
 * When n_embd is not a multiple of 256 or ffn_dim not of 64, the layer keeps
 * zero-padded copies of the weights at those widths (made here, one more copy
 * of the weights, any byte strides accepted) and every forward pads its rows
 * into the workspace and writes back the caller's width; results are those of
 * the unpadded layer (zero columns add exact zeros). */
int qmoe_layer_create(const qmoe_tensor* w_router,
                      const qmoe_tensor* w_exp_gate,
                      const qmoe_tensor* w_exp_up,
                      const qmoe_tensor* w_exp_down,
                      const qmoe_tensor* w_sh_gate,
                      const qmoe_tensor* w_sh_up,
                      const qmoe_tensor* w_sh_down,
                      const qmoe_tensor* w_sh_norm,
                      const qmoe_hparams* hp,
                      qmoe_layer** out);
int qmoe_layer_destroy(qmoe_layer* layer);
/* n_embd of a created layer (ne[0] of w_router). */
int qmoe_layer_n_embd(const qmoe_layer* layer);
/* Reads the layer's expert tensors now (their data must be in place) and keeps
 * chunk-major copies of them for the prefill GEMMs (block pairs of one k chunk
 * of consecutive rows side by side), which then load a few cache lines per wave
 * instead of one per lane.  Costs one more copy of the expert weights in device
 * memory, freed by qmoe_layer_destroy; a layer without it works the same, its
 * prefill GEMMs reading the GGUF rows.  Idempotent.  No counterpart in the
 * reference (ggml's mul_mat_id reads the rows as stored). */
int qmoe_layer_build_prefill_copies(qmoe_layer* layer);

/* Scratch for routing tables, quantized activations and per-row outputs,
 * sized for up to max_tokens tokens of layers no larger than `like`.  One
 * workspace may serve every layer of a model on one stream. */
int qmoe_workspace_create(const qmoe_layer* like, int32_t max_tokens, qmoe_workspace** out);
int qmoe_workspace_destroy(qmoe_workspace* ws);
int32_t qmoe_workspace_capacity(const qmoe_workspace* ws);
/* Synchronizes the device (a device error surfaces as QMOE_ERR_HIP) and
 * reports, in *fault, whether a forward on this workspace failed a
 * cross-workgroup wait: always 0, since no kernel waits on another workgroup
 * (every dependency is a launch boundary or a last-workgroup counter).  No
 * counterpart in the reference (ggml runs ops one after another). */
int qmoe_workspace_check(qmoe_workspace* ws, int32_t* fault);

/* Replaces MoELayer::build (moe.h:58-63, moe.cpp:55-177):
 *   y[T][n_embd] = MoE(x[T][n_embd])  (+ residual[T][n_embd] when non-NULL,
 *   the caller's ggml_add(cur, ffn_inp) of qwen36.cpp:304).
 * x, y, residual: device f32, token-major (ggml [n_embd, n_tokens]).  y may
 * alias residual but not x.  ws == NULL uses a workspace owned by the layer,
 * allocated on first use and grown when n_tokens exceeds it; growing it
 * synchronises the device, and on a stream that is being captured into a HIP
 * graph it fails with QMOE_ERR_CAPACITY instead (pass a workspace there).
 * n_tokens == 0 is a no-op.  dbg may be NULL. */
int qmoe_layer_forward(qmoe_layer* layer, qmoe_workspace* ws,
                       const float* x, int32_t n_tokens, float* y,
                       const float* residual, const qmoe_debug* dbg,
                       void* hip_stream);

/* Allocation-free forward.  No counterpart in the reference: for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same result as
 * qmoe_layer_forward(layer, ws, x, n_tokens, y, residual, NULL, stream) on a
 * workspace of its own, but the scratch is a file-scope device array of
 * QMOE_STATIC_SCRATCH_BYTES per GPU (held until the process ends), so no call
 * allocates or frees.  Its first call on a GPU (with that GPU current) looks
 * the array up; its signalling area (counters the routing returns to zero
 * after each use) is zero when the library loads, and a first call on a
 * stream that is not being captured also clears it and waits for that clear
 * (the one synchronisation this entry point performs).  Sizes whose
 * scratch exceeds the maximum (at the 35B-A3B shape: above about 100 tokens)
 * fail with QMOE_ERR_CAPACITY.  Every call on one GPU shares that GPU's
 * array: calls that overlap in time on one GPU (other streams, other threads)
 * race and must not be issued; calls ordered on one stream are fine. */
#define QMOE_STATIC_SCRATCH_BYTES (16u << 20)
int qmoe_layer_forward_static(qmoe_layer* layer, const float* x, int32_t n_tokens, float* y,
                              const float* residual, void* hip_stream);

/* Optional per-phase timing for benchmarks and profilers.  events points to
 * QMOE_N_PHASE_EVENTS hipEvent_t created by the caller (or is NULL to disable).
 * While set, each qmoe_layer_forward records them on its stream: [0] before
 * routing, [1] and [2] at the start and end of the gate/up expert kernel
 * (recorded by that launch itself), [3] after the down expert kernel, [4]
 * after the combine (at decode sizes the combine runs inside the down kernel).
 * No counterpart in the reference (ggml schedules the graph itself). */
#define QMOE_N_PHASE_EVENTS 5
int qmoe_layer_set_phase_events(qmoe_layer* layer, void* const* events);

/* ---------------------------------------------------------------------------
 * Expert-dispatch telemetry.  The reference's tracker (src/layers/
 * moe_residency.h) has no caller in its forward pass; here the layer feeds it.
 * ------------------------------------------------------------------------- */
/* Optional device histogram: while set, every forward of `layer` adds its
 * per-expert dispatch counts (the routing's count sort; T*top_k in total) to
 * device_counts[n_experts] (u64, zeroed by the caller), stream-ordered, no host
 * sync.  NULL stops it. */
int qmoe_layer_set_expert_counts(qmoe_layer* layer, uint64_t* device_counts);

/* Replaces MoEMetrics (src/telemetry/metrics.h:13-17). */
typedef struct qmoe_moe_metrics {
    uint64_t cold_dispatch_count;  /* dispatches to an expert outside the resident set */
} qmoe_moe_metrics;

/* Replaces MoEResidencyTracker (src/layers/moe_residency.{h,cpp}): per-expert
 * dispatch frequencies, the resident set (top resident_k experts by frequency,
 * frequency > 0, descending; equal frequencies ordered as the reference's
 * std::partial_sort over ascending ids orders them) and the cold counter
 * (incremented when the dispatched expert was not resident at dispatch time).
 * resident_k is clamped to n_experts; n_experts <= 0, resident_k <= 0 and ids
 * outside [0, n_experts) fail with the reference's messages.  Host-only. */
typedef struct qmoe_residency qmoe_residency;
int qmoe_residency_create(int32_t n_experts, int32_t resident_k, qmoe_residency** out);
void qmoe_residency_destroy(qmoe_residency* tracker);
/* record_dispatch for each id in turn (e.g. a forward's topk_idx, token-major). */
int qmoe_residency_record(qmoe_residency* tracker, const int32_t* expert_ids, int64_t n);
/* One batch from a dispatch histogram (counts[n_experts], e.g. copied from the
 * qmoe_layer_set_expert_counts buffer): the batch is cold by the resident set
 * at its start, then the set is refreshed once.  No counterpart in the
 * reference; for single-dispatch batches it equals qmoe_residency_record. */
int qmoe_residency_record_counts(qmoe_residency* tracker, const uint64_t* counts, int32_t n);
int qmoe_residency_is_resident(const qmoe_residency* tracker, int32_t expert_id);
int qmoe_residency_metrics(const qmoe_residency* tracker, qmoe_moe_metrics* out);
/* Writes up to cap ids of the resident set (descending frequency); returns its size. */
int32_t qmoe_residency_resident_set(const qmoe_residency* tracker, int32_t* out, int32_t cap);
int qmoe_residency_frequencies(const qmoe_residency* tracker, uint64_t* out, int32_t cap);
void qmoe_residency_reset(qmoe_residency* tracker);

/* The caller slice of the reference's block (qwen36.cpp:297-304 and 427-432)
 * in one call: y = x + MoE(RMSNorm(x) * norm_w), RMSNorm as qmoe_rms_norm.
 * At decode sizes (n_tokens <= 16, n_embd <= 2048) the routing normalizes x as
 * it loads it (no RMSNorm launch); otherwise the normalized rows go to the
 * workspace.  The residual add is the combine epilogue.  Bits equal
 * qmoe_rms_norm followed by qmoe_layer_forward(residual = x).  No counterpart
 * as one call in the reference; for callers that own the whole block. */
int qmoe_layer_forward_norm(qmoe_layer* layer, qmoe_workspace* ws, const float* x, const float* norm_w,
                            float eps, int32_t n_tokens, float* y, const qmoe_debug* dbg, void* hip_stream);

/* qmoe_layer_forward_norm for a chain of blocks (qwen36.cpp:297-304 and
 * 427-432 over the layers, x <- x + MoE_l(RMSNorm(x) * w_l)), carrying each
 * block's RMSNorm sum of squares to the next:
 *   x_ssq: NULL, or [n_tokens][ceil(n_embd/32)] doubles, the partial sums of x
 *          as qmoe_rms_partials defines them (a previous call's y_ssq);
 *   y_ssq: NULL, or receives y's partial sums in that layout.
 * Entry c of a row is the sum of squares of columns 32c .. 32c+31 in
 * qmoe_rms_norm's order (runs of four, then the pairwise tree), so the tree
 * over a row's entries is the row's sum: with or without x_ssq the bits equal
 * qmoe_layer_forward_norm's.  Where the decode routing normalizes on the fly
 * it finishes the tree from x_ssq instead of summing x (elsewhere x_ssq is not
 * read: n_tokens <= 16 and n_embd <= 2048); at decode sizes the down+combine
 * epilogue writes y_ssq, otherwise one more launch does (a caller at prefill
 * sizes gains nothing from the pair and passes NULL for both).  x_ssq and
 * y_ssq may be the same buffer.  16-byte aligned.
 * No counterpart in the reference; for callers that run the whole stack. */
int qmoe_layer_forward_norm_chain(qmoe_layer* layer, qmoe_workspace* ws, const float* x, const double* x_ssq,
                                  const float* norm_w, float eps, int32_t n_tokens, float* y, double* y_ssq,
                                  const qmoe_debug* dbg, void* hip_stream);

/* ---------------------------------------------------------------------------
 * Gemma 4 GeGLU MoE (replaces Gemma4ForwardPass::build_moe_geglu,
 * src/models/gemma4.cpp:367-445).  The same router, top-k, softmax, count
 * sort, grouped expert GEMMs and combine as the Qwen layer, with:
 *   - gate and up in one tensor ffn_gate_up_exps [n_embd, 2*ffn_dim,
 *     n_experts] (gate = rows 0..ffn_dim-1, up = the next ffn_dim rows of each
 *     expert, the views at :403-409), Q4_0 or Q8_0;
 *   - h = gelu(gate) * up (:423) with ggml's CPU gelu: the tanh form through
 *     its fp16 table (|g| >= 10 passes g or 0 through);
 *   - no shared expert (hp->has_shared_expert must be 0);
 *   - the router reading its own input (:380).
 * w_router is ffn_gate_inp.weight [n_embd, n_experts] F32; w_down_exps is
 * ffn_down_exps.weight [ffn_dim, n_embd, n_experts].  The layer is destroyed
 * with qmoe_layer_destroy; qmoe_layer_forward routes on x itself.
 * ------------------------------------------------------------------------- */
int qmoe_geglu_layer_create(const qmoe_tensor* w_router, const qmoe_tensor* w_gate_up_exps,
                            const qmoe_tensor* w_down_exps, const qmoe_hparams* hp, qmoe_layer** out);

/* y = MoE(expert_in) with the routing computed from router_in ([n_tokens][n_embd]
 * each; build_moe_geglu's expert_in / router_in).  Works for every layer; a
 * shared expert's sigmoid gate also reads router_in. */
int qmoe_layer_forward_routed(qmoe_layer* layer, qmoe_workspace* ws, const float* expert_in, const float* router_in,
                              int32_t n_tokens, float* y, const qmoe_debug* dbg, void* hip_stream);

/* The Gemma 4 MoE branch from the residual rows x (gemma4.cpp:555-565):
 *   expert_in = rms_norm(x) * pre_norm_w            (blk.N.pre_ffw_norm_2)
 *   router_in = (rms_norm(x) * (1/sqrtf(n_embd))) * router_scale_w  (ffn_gate_inp.scale)
 *   y = build_moe_geglu(expert_in, router_in)
 * both inputs from one pass over x, into the workspace.  y is the routed sum
 * (the caller's post_ffw_norm_2 follows, :566). */
int qmoe_layer_forward_gemma4(qmoe_layer* layer, qmoe_workspace* ws, const float* x, const float* pre_norm_w,
                              const float* router_scale_w, float eps, int32_t n_tokens, float* y,
                              const qmoe_debug* dbg, void* hip_stream);
/* The two inputs alone (n_embd <= 4096), into caller buffers. */
int qmoe_gemma4_moe_inputs(const float* x, const float* pre_norm_w, const float* router_scale_w, float eps,
                           int32_t n_tokens, int32_t n_embd, float* expert_in, float* router_in, void* hip_stream);
/* Host: the 65536-entry fp16 gelu table the GeGLU kernels read (entry i =
 * fp16(gelu(fp16 value i)); the inf and NaN codes map to themselves). */
int qmoe_gelu_f16_table(uint16_t* out);

/* Replaces build_rms_norm (norm.cpp:15-26): y = x / sqrt(mean(x^2) + eps) * w,
 * per token (ggml_rms_norm followed by ggml_mul).  w may be NULL (no scale).
 * The sum of squares is f64 of the f32 squares, in one fixed order (runs of four
 * columns, then a pairwise tree: ggml adds the columns in turn, which rounds
 * differently only where the sum lies within a few f64 ulps of an f32
 * rounding boundary of the mean).  n_embd up to 65536 (QMOE_ERR_VALUE above). */
int qmoe_rms_norm(const float* x, const float* w, int32_t n_tokens, int32_t n_embd,
                  float eps, float* y, void* hip_stream);
/* out[n_tokens][ceil(n_embd/32)]: qmoe_rms_norm's sum of squares of each row in
 * pieces of 32 columns -- entry c is the subtree over runs 8c .. 8c+7 (run r:
 * f64(x[4r]^2) + ... + f64(x[4r+3]^2) in column order, columns past n_embd
 * skipped), i.e. ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)).  No counterpart in the
 * reference (it sums inside ggml_rms_norm); the input of forward_norm_chain. */
int qmoe_rms_partials(const float* x, int32_t n_tokens, int32_t n_embd, double* out, void* hip_stream);

/* Seeded synthetic data for tests and benchmarks, generated on the device.
 * Value i of a stream is N(mean, sigma) from a counter-based hash of
 * (seed, stream, i) and a Box-Muller transform made of fixed IEEE operations,
 * so the bytes equal those of a CPU implementation of the same recipe.
 *   qmoe_synth_f32:   dst[i] = (float)(mean + sigma * z_i), i < n
 *   qmoe_synth_quant: n_rows rows of row_len values (value index row*row_len+col)
 *                     quantized to `type` with ggml's reference quantizers
 *                     (quantize_row_q4_0_ref / quantize_row_q8_0_ref). */
int qmoe_synth_f32(float* dst, int64_t n, uint64_t seed, uint64_t stream,
                   double mean, double sigma, void* hip_stream);
int qmoe_synth_quant(void* dst, int32_t type, int64_t n_rows, int64_t row_len,
                     uint64_t seed, uint64_t stream, double sigma, void* hip_stream);

/* ---------------------------------------------------------------------------
 * GGUF ingestion: replaces GGUFLoader (src/loader/gguf_loader.cpp) for the
 * tensors of the MoE path.  The file is memory-mapped; tensor bytes are copied
 * unchanged, since the GGUF block layout is the layer's input layout.
 * ------------------------------------------------------------------------- */
typedef struct qmoe_gguf qmoe_gguf;

/* One inventory entry (gguf_loader.cpp:474-497): ggml type id, shape (ggml ne
 * order, unused dims 1), absolute file offset of its data (data start aligned
 * as at gguf_loader.cpp:84-85 + the entry's offset) and byte size
 * (type size * elements / block size, gguf_loader.cpp:213). */
typedef struct qmoe_gguf_tensor {
    int32_t  type;
    int32_t  n_dims;
    int64_t  ne[4];
    uint64_t file_offset;
    uint64_t nbytes;
} qmoe_gguf_tensor;

/* Replaces GGUFLoader::load_model (gguf_loader.cpp:46-91): maps `path`, checks
 * the magic ("GGUF") and version (2 or 3), parses the key/value metadata (arrays
 * are skipped, as the reference does for every key it does not consume) and the
 * tensor inventory.  Errors name what was expected and what was found. */
int qmoe_gguf_open(const char* path, qmoe_gguf** out);
void qmoe_gguf_close(qmoe_gguf* gguf);
/* Header facts: version, inventory size, metadata size, data start offset. */
int qmoe_gguf_info(const qmoe_gguf* gguf, uint32_t* version, int64_t* n_tensors, int64_t* n_kv,
                   uint64_t* data_offset);
/* Scalar metadata (the raw_kv lookups of the model recipes, e.g.
 * "qwen35moe.expert_count", qwen36.cpp:23-25).  The key must hold that type. */
int qmoe_gguf_get_u32(const qmoe_gguf* gguf, const char* key, uint32_t* out);
int qmoe_gguf_get_f32(const qmoe_gguf* gguf, const char* key, float* out);
/* *out points into the handle; valid until qmoe_gguf_close. */
int qmoe_gguf_get_str(const qmoe_gguf* gguf, const char* key, const char** out);
/* Inventory order access and lookup by name (GGUFLoader::get_tensor_metadata). */
int qmoe_gguf_tensor_name(const qmoe_gguf* gguf, int64_t index, const char** out);
int qmoe_gguf_find(const qmoe_gguf* gguf, const char* name, qmoe_gguf_tensor* out);
/* Replaces get_tensor_data + ggml_backend_tensor_set (gguf_loader.cpp:621-639):
 * copies the tensor's bytes to host memory / to device memory (stream-ordered,
 * returns once the file mapping has been read).  dst must hold nbytes. */
int qmoe_gguf_read(const qmoe_gguf* gguf, const char* name, void* dst, uint64_t dst_bytes);
int qmoe_gguf_upload(const qmoe_gguf* gguf, const char* name, void* dst_device, uint64_t dst_bytes,
                     void* hip_stream);
/* The contiguous ggml view of an uploaded tensor: data = device_data, nb from
 * the type's block geometry (nb[0] = block bytes, nb[1] = row bytes, ...). */
int qmoe_gguf_tensor_view(const qmoe_gguf_tensor* t, const void* device_data, qmoe_tensor* out);

#ifdef __cplusplus
}
#endif
#endif /* QMOE_H */
