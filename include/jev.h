/*
 * jev.h -- C ABI of libjev, the MI355X token loop behind Jevstral's managed API.
 *
 * The managed host (GgufFile, JevstralDecider, SystemPromptCache) keeps its API
 * and calls these entry points over [LibraryImport("jev")].  Every array in a
 * signature is a plain pointer owned by the caller and only read or written
 * during the call.  A context owns its device weights, KV arena, scratch and
 * HIP stream; it is not thread-safe (like MinistralModel, MinistralModel.cs:21-22):
 * use one context per concurrent request.  Only jev_cancel may be called from
 * another thread.
 *
 * Status codes map onto the reference's exceptions:
 *   JEV_EINVAL    ArgumentException        (QuantMatMul.cs:77-80, MinistralModel.cs:306, :202-207)
 *   JEV_EDATA     InvalidDataException     (ModelConfig.cs:108-110, MinistralModel.cs:110-123)
 *   JEV_ECANCELED OperationCanceledException (ParallelOptions.CancellationToken)
 *   JEV_ENOMEM / JEV_EDEVICE               HIP allocation / runtime failures
 *   JEV_ESTATE    InvalidOperationException (call order, e.g. forward before finalize)
 * jev_last_error() returns the thread's last message.
 */
#ifndef JEV_H
#define JEV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JEV_OK 0
#define JEV_EINVAL 1
#define JEV_EDATA 2
#define JEV_ENOMEM 3
#define JEV_EDEVICE 4
#define JEV_ECANCELED 5
#define JEV_ESTATE 6

/* GGML type ids (src/Jevstral/Gguf/GgmlType.cs:12-18). */
#define JEV_TYPE_F32 0
#define JEV_TYPE_F16 1
#define JEV_TYPE_Q4_0 2
#define JEV_TYPE_Q5_1 7
#define JEV_TYPE_Q8_0 8

/* Tensor slots: the tensors MinistralModel binds (MinistralModel.cs:74-96). */
#define JEV_SLOT_TOKEN_EMBD 0  /* token_embd.weight                    */
#define JEV_SLOT_OUTPUT_NORM 1 /* output_norm.weight                   */
#define JEV_SLOT_OUTPUT 2      /* output.weight (optional; tied if absent) */
#define JEV_SLOT_ATTN_NORM 3   /* blk.{l}.attn_norm.weight             */
#define JEV_SLOT_Q 4           /* blk.{l}.attn_q.weight                */
#define JEV_SLOT_K 5           /* blk.{l}.attn_k.weight                */
#define JEV_SLOT_V 6           /* blk.{l}.attn_v.weight                */
#define JEV_SLOT_O 7           /* blk.{l}.attn_output.weight           */
#define JEV_SLOT_FFN_NORM 8    /* blk.{l}.ffn_norm.weight              */
#define JEV_SLOT_GATE 9        /* blk.{l}.ffn_gate.weight              */
#define JEV_SLOT_UP 10         /* blk.{l}.ffn_up.weight                */
#define JEV_SLOT_DOWN 11       /* blk.{l}.ffn_down.weight              */

/* Output modes of the private ForwardAsync (MinistralModel.cs:301-425). */
#define JEV_OUT_NONE 0      /* PrefillAsync: KV state only (:148-149)                       */
#define JEV_OUT_LAST_FULL 1 /* computeLogits: full vocabulary at the last token (:411-424)  */
#define JEV_OUT_SELECTED 2  /* selectedRows at every output token (:386-410)               */
#define JEV_OUT_FULL 3      /* full vocabulary at every output token (:362-385)            */

/* ModelConfig (ModelConfig.cs:12-118): filled by the managed side from the GGUF
 * metadata it already parses (ModelConfig.FromGguf). */
typedef struct jev_config {
    int32_t n_layers;       /* {arch}.block_count                          */
    int32_t hidden;         /* {arch}.embedding_length                     */
    int32_t n_heads;        /* {arch}.attention.head_count                 */
    int32_t n_kv_heads;     /* {arch}.attention.head_count_kv              */
    int32_t head_dim;       /* {arch}.attention.key_length (must be 128)   */
    int32_t ffn;            /* {arch}.feed_forward_length                  */
    int32_t vocab;          /* tokenizer.ggml.tokens length                */
    float rms_eps;          /* {arch}.attention.layer_norm_rms_epsilon     */
    float rope_freq_base;   /* {arch}.rope.freq_base                       */
    int32_t rope_dim;       /* {arch}.rope.dimension_count                 */
    float rope_scale_factor;/* {arch}.rope.scaling.factor                  */
    int32_t rope_scaling_yarn; /* {arch}.rope.scaling.type == "yarn"       */
    int32_t rope_original_context;
    float yarn_beta_fast, yarn_beta_slow, yarn_ext_factor, yarn_mscale, yarn_mscale_all_dim;
    float rope_attn_factor;
    float attention_temperature_scale;
    int32_t initial_kv_capacity; /* MinistralModel(path, initialCacheCapacity) */
} jev_config;

/* TokenLayout (MinistralModel.cs:703-781): token t is written to cache slot
 * slot[t], rotated as position[t], and attends to slots [shared_lo[t],
 * shared_hi[t]) and to its own segment [segment[t], slot[t]].  The reference's
 * layouts are shared_lo = 0 and shared_hi = Shared; a nonzero shared_lo lets
 * independent decisions keep their own trunks in one cache.  outputs lists the
 * tokens whose logits are returned; end is one past the highest slot written. */
typedef struct jev_layout {
    const int32_t *slot;
    const int32_t *position;
    const int32_t *shared_lo;
    const int32_t *shared_hi;
    const int32_t *segment;
    const int32_t *outputs;
    int32_t n_outputs;
    int32_t end;
} jev_layout;

typedef struct jev_ctx jev_ctx;

const char *jev_last_error(void);

/* new MinistralModel(...) minus the GGUF parse: validates the config and
 * allocates the KV arena (KvCache ctor, KvCache.cs:25-33) on `device`. */
int jev_create(const jev_config *cfg, int device, jev_ctx **out);
void jev_destroy(jev_ctx *ctx);

/* WeightMatrix.From / VectorParameter.From (WeightMatrix.cs:53-90): copies one
 * GGUF tensor (rows = Shape[1], cols = Shape[0]; bytes = GgufFile.GetTensorPointer)
 * into HBM, repacked for the kernels.  `layer` is ignored for global slots. */
int jev_bind_tensor(jev_ctx *ctx, int slot, int layer, int ggml_type, int64_t rows, int64_t cols,
                    const void *bytes, size_t nbytes);
/* MinistralModel.ValidateShapes (MinistralModel.cs:110-123) plus the
 * every-tensor-present check of its constructor. */
int jev_finalize(jev_ctx *ctx);

/* KvCache (KvCache.cs). */
int jev_kv_length(jev_ctx *ctx, int32_t *length);
int jev_kv_capacity(jev_ctx *ctx, int32_t *capacity);
int jev_kv_reserve(jev_ctx *ctx, int32_t required);              /* EnsureCapacity :48-70 */
int jev_kv_truncate(jev_ctx *ctx, int32_t length);               /* Truncate :46          */
int jev_kv_reset(jev_ctx *ctx);                                  /* Reset :43             */
int jev_kv_snapshot(jev_ctx *ctx, int32_t length, float *out, size_t n_floats); /* Snapshot :94-112 */
int jev_kv_restore(jev_ctx *ctx, const float *in, size_t n_floats, int32_t length); /* Restore :115-136 */

/* The same snapshot kept in HBM (KvCache.Snapshot/Restore, KvCache.cs:94-136, as
 * JevstralDecider's question-snapshot LRU and the system-prompt snapshot use it,
 * JevstralDecider.cs:259-266, :348-354): taking and restoring one is a copy
 * inside device memory, never through the host.  The handle owns its HBM
 * (2 x layers x kv heads x length x head_dim floats) until destroyed; it can
 * be restored into any context of the same geometry on the same device.
 * jev_snapshot_read copies it out in jev_kv_snapshot's flat layout (SHKV files). */
typedef struct jev_snapshot jev_snapshot;
int jev_kv_snapshot_device(jev_ctx *ctx, int32_t length, jev_snapshot **out);
int jev_kv_restore_device(jev_ctx *ctx, const jev_snapshot *snapshot);
int jev_snapshot_length(const jev_snapshot *snapshot, int32_t *length);
int jev_snapshot_read(const jev_snapshot *snapshot, float *out, size_t n_floats);
void jev_snapshot_destroy(jev_snapshot *snapshot);

/* The private ForwardAsync (MinistralModel.cs:301-435).  layout NULL = plain
 * causal append after the cached tokens.  out receives (by mode): nothing;
 * vocab floats; n_outputs * n_rows floats; n_outputs * vocab floats, where
 * n_outputs is 1 without a layout. */
int jev_forward(jev_ctx *ctx, const int32_t *tokens, int32_t n_tokens, const jev_layout *layout, int mode,
                const int32_t *rows, int32_t n_rows, float *out, size_t out_len);

/* IActivationSink.Observe (MinistralModel.cs:787-790): one named tensor of
 * rows x columns floats, valid only during the call. */
typedef void (*jev_sink)(void *user, const char *name, const float *values, int32_t rows, int32_t columns);

/* The public ForwardAsync(tokens, capture, options) (MinistralModel.cs:157-160
 * -> :301-435): appends `tokens` causally, writes the last token's vocab
 * logits to `logits`, and calls `sink` once per tensor the reference observes,
 * in its order and with its names -- "embeddings"; per layer l
 * "blk.{l}.attn_norm", "q_rope", "k_rope", "v", "attn_weighted", "attn_out",
 * "post_attn", "ffn_norm", "ffn_out", "output"; then "final_norm" and
 * "logits" (MinistralModel.cs:331-357, :418-422, AttentionAsync :459-549).
 * The sink runs on the calling thread after the pass has finished.  A
 * debugging path: the device synchronises at every tap. */
int jev_capture(jev_ctx *ctx, const int32_t *tokens, int32_t n_tokens, jev_sink sink, void *user, float *logits,
                size_t out_len);

/* ForwardTreeAsync (MinistralModel.cs:198-219): the trunk appended causally,
 * then every branch continuing from its end; branch_tokens holds the branches
 * back to back.  out = n_branches * n_rows verdict-row logits. */
int jev_forward_tree(jev_ctx *ctx, const int32_t *trunk, int32_t n_trunk, const int32_t *branch_tokens,
                     const int32_t *branch_lens, int32_t n_branches, const int32_t *rows, int32_t n_rows,
                     float *out, size_t out_len);

/* Greedy decode (Benchmark.cs:411-422 / ReasoningDecider.cs:157-178): feeds
 * `first`, then n_steps - 1 argmax tokens, one ForwardAsync([next]) each;
 * tokens_out (room for tokens_out_len ids) receives the n_steps argmax ids
 * (Kernels.ArgMax, lowest index on ties).  A tokens_out shorter than n_steps
 * is refused with JEV_EINVAL before any work, as the reference refuses a
 * destination span that is too short (MinistralModel.cs:306). */
int jev_decode_greedy(jev_ctx *ctx, int32_t first, int32_t n_steps, int32_t *tokens_out, size_t tokens_out_len);

/* ReasoningDecider's batched greedy loop (ReasoningDecider.cs:157-178, each step
 * a ForwardRowsAsync of one token per row, MinistralModel.cs:272-294, with the
 * rows layout TokenLayout.Rows :758-780): n_rows rows over `shared` shared
 * positions, row r's slots from row_base[r] with row_length[r] tokens cached;
 * every step feeds each row's last token (first[r] at step 0) and takes each
 * row's argmax over the full vocabulary (lowest index on ties) as its next
 * token.  The step runs as a replayed HIP graph with the per-row state on the
 * device; tokens_out (room for tokens_out_len ids; fewer than n_steps x
 * n_rows is JEV_EINVAL before any work) receives n_steps x n_rows ids,
 * [step][row].  Every row
 * runs all n_steps: the caller ends a row at its stop token by discarding
 * what follows (rows are independent and the kernels batch-invariant, so a
 * row's tokens do not depend on which other rows run, as long as two or more
 * rows run -- a lone row takes the one-token path, QuantMatMul.cs:84).  The
 * rows' slots over the whole run must stay clear of the shared prefix and of
 * each other (JEV_EINVAL otherwise). */
int jev_decode_rows_greedy(jev_ctx *ctx, int32_t shared, int32_t n_rows, const int32_t *row_base,
                           const int32_t *row_length, const int32_t *first, int32_t n_steps, int32_t *tokens_out,
                           size_t tokens_out_len);

/* JevstralDecider.DecideAsync margins (:306-308) and softmax(z/T) (:310-313):
 * verdicts is n_options x (n_yes + n_no). */
int jev_margins(const float *verdicts, int32_t n_options, int32_t n_yes, int32_t n_no, float temperature,
                float *margins, float *probs);

/* ParallelOptions.CancellationToken (MinistralModel.cs:301-304, KernelTests.cs:206-219):
 * cancels the call in flight on ctx -- jev_forward, jev_forward_tree,
 * jev_decode_greedy, jev_capture -- which then returns JEV_ECANCELED with the
 * cache length unchanged (greedy decoding: advanced by the steps that ran).
 * Those calls keep at most two groups of layers (decode: two steps) enqueued
 * ahead of the device and check between layers, so the work stops within that
 * many; a group is about 2e11 FLOPs of linear work (one layer from a few
 * thousand tokens, a few layers at a few hundred, half the model for one
 * token).  A cancel that lands after the last layer was enqueued still
 * cancels the call.  A cancel aimed at no call (none in flight) does nothing, so it
 * never reaches a later call.  The only entry point safe from another thread. */
void jev_cancel(jev_ctx *ctx);

/* Timing support: device-resident variant of jev_forward for a fixed plan.
 * d_tokens / d_out are device pointers; the call only enqueues work on the
 * context's stream (no host synchronisation); jev_sync waits for it.  A
 * cancel is honoured only while it enqueues (between layers). */
int jev_forward_device(jev_ctx *ctx, const int32_t *d_tokens, int32_t n_tokens, const jev_layout *layout, int mode,
                       const int32_t *rows, int32_t n_rows, float *d_out);
int jev_sync(jev_ctx *ctx);
/* The context's HIP stream (hipStream_t), for event timing by the caller. */
void *jev_stream(jev_ctx *ctx);

/* Kernel timing: with profiling enabled (mode 1), the context records a HIP
 * event pair around every launch of the listed kernel classes on its own
 * stream, and accumulates launches, device time and algorithmic work (FLOPs of
 * the product, bytes of the weights and activations it must move); the greedy
 * decodes then launch kernel by kernel instead of replaying a graph.  Mode 2
 * instead stamps only the step boundaries of the greedy decodes (graphs kept):
 * jev_profile_steps returns the last decode's per-step device time in ms, the
 * per-token latency Benchmark.cs:411-422 samples.  Mode 0 turns both off.
 * Enabling clears the counters; reading synchronises the stream. */
#define JEV_PROF_GEMM 0 /* MFMA prefill GEMM                     */
#define JEV_PROF_ATTN 1 /* tree attention (prefill)              */
#define JEV_PROF_GEMV 2 /* one-token quantized GEMV              */
#define JEV_PROF_DECODE_ATTN 3 /* decode attention (chunks)      */
#define JEV_PROF_CLASSES 4
int jev_profile_enable(jev_ctx *ctx, int enable);
int jev_profile_read(jev_ctx *ctx, int kernel_class, int64_t *launches, double *total_ms, double *flops,
                     double *bytes);
int jev_profile_steps(jev_ctx *ctx, float *ms, int32_t n, int32_t *n_steps);

/* ---- A single quantized weight resident in HBM ---- */

/* The narrower seam QuantMatMul.ForwardAsync(WeightMatrix, x, tokens, y)
 * (QuantMatMul.cs:66-121) over a weight uploaded once (WeightMatrix.From,
 * WeightMatrix.cs:53-65: rows = Shape[1], cols = Shape[0], GGUF bytes read
 * only during the call).  The weight owns its stream and scratch. */
typedef struct jev_weight jev_weight;
int jev_weight_create(int ggml_type, int64_t rows, int64_t cols, const void *bytes, size_t nbytes, int device,
                      jev_weight **out);
void jev_weight_destroy(jev_weight *w);
/* y = x . W^T with x [tokens][cols] and y [tokens][rows], both fp32 device
 * pointers; tokens >= 2 take the MFMA GEMM, 1 token the GEMV (the dispatch of
 * QuantMatMul.cs:84-101).  Only enqueues on the weight's stream.  Any float
 * alignment; at 16 bytes the fp16-pair split of x and the K-split sum into y
 * move 16 bytes per access (the result bits are the same). */
int jev_matmul_device(jev_weight *w, const float *x, int32_t tokens, float *y);
/* jev_matmul_device without any allocation.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory during the call (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same kernels and the same result bits as jev_matmul_device;
 * the call's scratch (fp16 pair of x, Q5_1 block sums, K-split partials, or
 * the integer strategy's quantized activations) comes from one static 16 MiB
 * device array per GPU, held until the process ends.  A call whose scratch
 * would exceed 16 MiB fails with JEV_EINVAL (256 tokens x 3072 x 3072 fits).
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (on different weights' streams, or from several threads) race. */
int jev_matmul_device_noalloc(jev_weight *w, const float *x, int32_t tokens, float *y);
int jev_weight_sync(jev_weight *w);
/* The weight's HIP stream (hipStream_t): the caller may capture calls on it
 * into a HIP graph (jev_matmul_device_noalloc allocates nothing, so it can be
 * captured) or time them with events. */
void *jev_weight_stream(jev_weight *w);

/* QuantMatMul.Strategy (QuantMatMul.cs:10-41), process-wide, read by every
 * jev_matmul_device / jev_matmul_q call.  AUTO and FLOAT take the float path
 * above (exact quants, fp16-pair activations on the fp16 matrix cores: the
 * numerics the model was validated with); INTEGER is the opt-in integer path
 * (QuantMatMul.cs:186-287, IntegerDot.cs): activations quantized to Q8_0
 * blocks, IntegerDot's block dots on the int8 matrix cores.  The model
 * forward always takes the float path.  JEV_EINVAL for an unknown value. */
enum { JEV_MATMUL_AUTO = 0, JEV_MATMUL_FLOAT = 1, JEV_MATMUL_INTEGER = 2 };
int jev_set_matmul_strategy(int strategy);
int jev_get_matmul_strategy(void);

/* ---- Test hooks (no managed counterpart) ---- */

/* The Rope ctor's tables (Rope.cs:33-106): the n = rope_dim / 2 pair
 * frequencies (YaRN-ramped when ModelConfig.YarnActive, ModelConfig.cs:54-56)
 * and the magnitude scale folded into cos / sin (ComputeMagnitudeScale,
 * Rope.cs:78-88) -- the tables jev_create uploads.  Host only: no device. */
int jev_rope_table(const jev_config *cfg, float *freqs, int32_t n, float *mscale);

/* Dequantizer.Dequantize (Dequantizer.cs:45-93) run on the device:
 * `count` elements from GGUF blocks to float32. */
int jev_dequantize(int ggml_type, const void *src, size_t nbytes, float *dst, int64_t count);
/* QuantMatMul.ForwardAsync (QuantMatMul.cs:66-121) run on the device: tokens >= 2
 * take the MFMA GEMM, 1 token the GEMV.  y = tokens x rows. */
int jev_matmul_q(int ggml_type, const void *w, int64_t rows, int64_t cols, const float *x, int32_t tokens, float *y);
/* IntegerDot.QuantizeActivations (IntegerDot.cs:60-96) run on the device:
 * `count` floats (a multiple of 32) to count / 32 Q8_0 blocks of 34 bytes
 * (Half scale max|x| / 127, quants rounded half away from zero and clamped to
 * +-127); block_sums (optional, count / 32 floats) gets d * sum(q) with the
 * float d, as QuantMatMul's integer path computes them (QuantMatMul.cs:223-234). */
int jev_quantize_activations(const float *x, int64_t count, void *out, size_t out_bytes, float *block_sums);

/* ---- Synthetic-model tool (replaces the converter for offline runs) ---- */

/* ggml reference quantizers (quantize_row_q8_0/q4_0/q5_1_ref) over `count`
 * floats into GGUF blocks. */
int jev_quantize(int ggml_type, const float *src, int64_t count, void *dst, size_t nbytes);
/* Fills a rows x cols tensor with N(0, stddev) draws from a counter-based
 * generator keyed by (seed, stream), quantized to ggml_type (F32 writes floats).
 * The bytes depend only on (seed, stream, shape, type), not on `threads`. */
int jev_synth_tensor(uint64_t seed, uint64_t stream, int ggml_type, int64_t rows, int64_t cols, float stddev,
                     void *dst, size_t nbytes, int threads);

#ifdef __cplusplus
}
#endif
#endif
