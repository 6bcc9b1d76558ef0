/*
 * CPU oracle for the Jevstral token loop -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's managed `Float` path
 * (QuantMatMul.Strategy = Float, PanelGemm, AttendHead, Kernels, Rope,
 * KvCache, TokenLayout).  It is the checker for the HIP library: only the
 * tests, the smoke check and the bench's CPU-baseline leg load it.  Nothing
 * in the product links against it.
 *
 * Every function cites the reference file:line it follows.
 */
#ifndef JEV_ORACLE_H
#define JEV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids, src/Jevstral/Gguf/GgmlType.cs:12-18. */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q5_1 = 7, ORC_Q8_0 = 8 };

/* Output modes of the private ForwardAsync (MinistralModel.cs:301-425). */
enum {
    ORC_OUT_NONE = 0,      /* PrefillAsync: KV only                          */
    ORC_OUT_LAST_FULL = 1, /* computeLogits: full vocab at the last token     */
    ORC_OUT_SELECTED = 2,  /* selectedRows at each output (verdict rows)      */
    ORC_OUT_FULL = 3       /* full vocab at each output (ForwardTreeLogits)   */
};

int orc_block_size(int type);            /* GgmlType.cs:55-64  */
int orc_type_size(int type);             /* GgmlType.cs:67-82  */
int64_t orc_row_bytes(int type, int64_t cols); /* GgmlType.cs:112-120 */

/* Dequantizer.Dequantize (Dequantizer.cs:45-93) for F32/F16/Q4_0/Q5_1/Q8_0.
 * Returns 0, or -1 for an unsupported type / a count that is not whole blocks. */
int orc_dequantize(int type, const void *src, float *dst, int64_t count);

/* QuantMatMul.ForwardAsync with Strategy = Float (QuantMatMul.cs:66-121):
 * y[t*rows + r] = dot(x[t*cols ...], W[r, :]).  tokens >= 2 and a panel-able
 * shape take the PanelGemm chain (PanelGemm.cs:87-318); otherwise the
 * row-wise float dot (QuantMatMul.cs:140-176). */
void orc_matmul(int type, const void *w, int rows, int cols, const float *x, int tokens, float *y);

/* MatMulStrategy.Integer (QuantMatMul.cs:186-287, IntegerDot.cs): Q8_0
 * activation blocks (34 bytes: Half scale + 32 int8) and the integer matmul.
 * Both return 0, or -1 for an unsupported type or a count not in whole blocks. */
int orc_quantize_activations(const float *x, int64_t count, uint8_t *out, float *sums);
int orc_matmul_integer(int type, const void *w, int rows, int cols, const float *x, int tokens, float *y);

/* Individual kernels (Kernels.cs). */
void orc_rmsnorm(const float *x, const float *w, float eps, int n, float *y); /* :25-60  */
void orc_softmax(float *x, int n);                                            /* :102-121 */
void orc_swiglu(const float *gate, float *up, float *dst, int n);             /* :82-89  */
float orc_dot(const float *a, const float *b, int n);                         /* :68     */

/* Attention for one query head against one KV head (AttendHead,
 * MinistralModel.cs:564-636 with AttentionKernels.Scores/WeightedSum):
 * visible logical keys i in [0, limit) with limit = n_sh + (slot - segment + 1),
 * physical p = i < n_sh ? shared_lo + i : segment + (i - n_sh).  keys/values
 * are [slot][head_dim] rows.  scores must hold `limit` floats. */
void orc_attend(const float *q, const float *keys, const float *values, int head_dim,
                int shared_lo, int shared_hi, int segment, int slot, float scale,
                float *scores, float *out);

/* Model config: the fields ModelConfig.FromGguf reads (ModelConfig.cs:62-112). */
typedef struct orc_config {
    int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab;
    float rms_eps;
    float rope_freq_base;
    int32_t rope_dim;
    float rope_scale_factor;
    int32_t rope_scaling_yarn; /* RopeScalingType == "yarn" */
    int32_t rope_original_context;
    float yarn_beta_fast, yarn_beta_slow, yarn_ext_factor, yarn_mscale, yarn_mscale_all_dim;
    float rope_attn_factor, attention_temperature_scale;
    int32_t initial_kv_capacity;
} orc_config;

/* TokenLayout (MinistralModel.cs:703-781), with the shared range
 * generalised to [shared_lo, shared_hi); the reference's layouts have
 * shared_lo = 0.  NULL arrays in a layout are not allowed; pass a NULL
 * layout for a plain causal append. */
typedef struct orc_layout {
    const int32_t *slot, *position, *shared_lo, *shared_hi, *segment;
    const int32_t *outputs;
    int32_t n_outputs;
    int32_t end;
} orc_layout;

/* Tensor slots bound into a model (MinistralModel.cs:74-96). */
enum {
    ORC_SLOT_TOKEN_EMBD = 0, ORC_SLOT_OUTPUT_NORM = 1, ORC_SLOT_OUTPUT = 2,
    ORC_SLOT_ATTN_NORM = 3, ORC_SLOT_Q = 4, ORC_SLOT_K = 5, ORC_SLOT_V = 6, ORC_SLOT_O = 7,
    ORC_SLOT_FFN_NORM = 8, ORC_SLOT_GATE = 9, ORC_SLOT_UP = 10, ORC_SLOT_DOWN = 11
};

typedef struct orc_model orc_model;

orc_model *orc_model_create(const orc_config *cfg);
void orc_model_destroy(orc_model *m);
/* Binds a tensor by pointer (not copied: the reference reads the mmap). */
int orc_model_bind(orc_model *m, int slot, int layer, int type, int rows, int cols, const void *bytes);
int orc_forward(orc_model *m, const int32_t *tokens, int n, const orc_layout *layout, int mode,
                const int32_t *rows, int n_rows, float *out, size_t out_len);
/* IActivationSink.Observe (MinistralModel.cs:787-790). */
typedef void (*orc_sink)(void *user, const char *name, const float *values, int rows, int columns);
/* The public ForwardAsync(tokens, capture, options) (MinistralModel.cs:157-160
 * -> :301-435): causal append with full-vocabulary logits at the last token,
 * calling `sink` for every tap the reference observes, in its order. */
int orc_forward_capture(orc_model *m, const int32_t *tokens, int n, orc_sink sink, void *user, float *out,
                        size_t out_len);
/* ForwardTreeAsync (MinistralModel.cs:198-219): out = n_branches x n_rows. */
int orc_forward_tree(orc_model *m, const int32_t *trunk, int n_trunk, const int32_t *branch_tokens,
                     const int32_t *branch_lens, int n_branches, const int32_t *rows, int n_rows,
                     float *out, size_t out_len);
int orc_kv_length(const orc_model *m);
void orc_kv_truncate(orc_model *m, int length); /* KvCache.cs:46 */
void orc_kv_reset(orc_model *m);                /* KvCache.cs:43 */
int orc_kv_snapshot(const orc_model *m, int length, float *out, size_t n); /* KvCache.cs:94-112 */
int orc_kv_restore(orc_model *m, const float *in, size_t n, int length);  /* KvCache.cs:115-136 */
/* Cache access for tests: pointer to key/value row (layer, kv head, slot). */
const float *orc_kv_key(const orc_model *m, int layer, int head, int slot);
const float *orc_kv_value(const orc_model *m, int layer, int head, int slot);

/* RoPE table (Rope.cs:33-66) and rotation (Rope.cs:112-135). */
int orc_rope_freqs(const orc_config *cfg, float *freqs, float *mscale);
void orc_rope_apply(const float *freqs, int half, float mscale, float *data, int heads, int head_dim, int position);

/* TokenLayout.Tree (MinistralModel.cs:720-745) into caller arrays of
 * `tokens` entries; outputs has n_branches entries.  Returns End. */
int orc_layout_tree(int start_pos, int trunk, const int32_t *offsets, int n_branches, int tokens,
                    int32_t *slot, int32_t *pos, int32_t *shared, int32_t *seg, int32_t *outputs);
/* TokenLayout.Rows (MinistralModel.cs:758-780). */
int orc_layout_rows(int shared, const int32_t *row_base, const int32_t *row_length, const int32_t *row_tokens,
                    int n_rows, int32_t *slot, int32_t *pos, int32_t *sh, int32_t *seg, int32_t *outputs);

/* JevstralDecider margins and probabilities (JevstralDecider.cs:306-313). */
void orc_margins(const float *verdicts, int n_options, int n_yes, int n_no, float temperature,
                 float *margins, float *probs);

void orc_set_threads(int n);
int orc_get_threads(void);
/* PanelGemm.VectorBits (PanelGemm.cs:50-63): 512 or 256 forces a tile width,
 * 0 picks 512 when the host has AVX-512F.  Both widths give the same bits. */
void orc_set_vector_bits(int bits);
int orc_get_vector_bits(void);

#ifdef __cplusplus
}
#endif
#endif
