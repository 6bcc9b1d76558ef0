// Internal interfaces of libjev: device weight layout, kernel launchers and
// the host-side quantizer / repack helpers.  Not part of the C ABI.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

namespace jev {

// GGML type ids (GgmlType.cs:12-18).
enum : int { kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ5_1 = 7, kQ8_0 = 8 };

int block_size(int type);           // elements per block (GgmlType.cs:55-64)
int type_size(int type);            // bytes per block    (GgmlType.cs:67-82)
int64_t row_bytes(int type, int64_t cols);

// ---------------------------------------------------------------- layout
//
// A quantized 2-D weight in HBM as "MFMA tiles": rows in groups of 16 and K
// in pairs of quant blocks (64 elements).  A tile is, in lane order, exactly
// the B operand of two v_mfma_f32_16x16x32_f16 (one per block): lane
// l = 16 g + r of a wave owns row r and k = 8 g .. 8 g + 7 of each block, so
// one wave-wide load of a tile is a single contiguous access.  Tiles are
// ordered [row group][block pair]; rows pad to a multiple of 16 and blocks to
// an even count with zero quants and scales.  Per tile:
//   qs  Q8_0       1024 B: lane l's 16 bytes at 16 l -- 8 quants of block 0, then 8 of block 1,
//                          each stored biased as the byte q + 128
//       Q4_0/Q5_1   512 B: lane l's 8 bytes at 8 l -- 4 of block 0, then 4 of block 1; byte i
//                          of a block's four = element 8g+i (low nibble) | element 8g+i+4 (high)
//   d   fp16         64 B: row r's two block scales at 4 r (Q8_0, Q4_0)
//       Q5_1        128 B: row r's two scales then its two mins at 8 r, so a
//                          lane's scales and mins are one 8-byte load
//                          (QWeight::m points at the first min)
//   qh  (Q5_1)      128 B: lane l's fifth bits at 2 l + block, bit i = element 8 g + i
//   qb  (Q5_1)     1024 B: the same quants again as whole bytes q in [0, 31], in
//                          Q8_0's order (lane l's 16 bytes at 16 l), for the
//                          kernels of two or more tokens: one byte permute and
//                          one packed subtraction per two weights instead of the
//                          nibble and fifth-bit assembly (the one-token GEMV keeps
//                          the 5-bit fields, whose bytes it streams)
constexpr int kTileRows = 16, kTileK = 64;
struct QWeight {
    int type = -1;
    int rows = 0, cols = 0;
    const uint8_t *qs = nullptr;
    const uint16_t *d = nullptr;
    const uint16_t *m = nullptr;
    const uint8_t *qh = nullptr;
    const uint8_t *qb = nullptr; // Q5_1 quants as bytes (see qb above)
    void *base = nullptr; // owning allocation
    size_t bytes = 0;
};
// Tile counts of a weight: row groups and block pairs.
__host__ __device__ inline int tile_rows(int rows) { return (rows + kTileRows - 1) / kTileRows; }
__host__ __device__ inline int tile_kpairs(int cols) { return ((cols >> 5) + 1) >> 1; }
__host__ __device__ inline int tile_qs_bytes(int type) { return type == kQ8_0 ? 1024 : 512; }
// Bytes of scales (and Q5_1 mins) per tile.
__host__ __device__ inline int tile_d_bytes(int type) { return type == kQ5_1 ? 128 : 64; }

// Byte offsets of the fields inside one allocation of the layout above.
struct QLayout {
    size_t qs, d, m, qh, qb, total;
};
QLayout qlayout(int type, int64_t rows, int64_t cols);

// Host: GGUF blocks (rows x cols) -> the tiled layout in `dst`
// (qlayout(type, rows, cols).total bytes).  Returns false on a bad type/shape.
bool repack_host(int type, int64_t rows, int64_t cols, const void *gguf, void *dst, int threads);

// Host scalar helpers.
float half_to_float(uint16_t h);
uint16_t float_to_half(float f); // round to nearest even

// ---------------------------------------------------------------- kernels

// Dequantize `rows` full rows of a weight into fp32 [rows][cols].
hipError_t launch_dequant(const QWeight &w, float *dst, hipStream_t s);

// Embedding gather: h[t] = decode(row ids[t]).
hipError_t launch_gather(const QWeight &w, const int32_t *ids, int n, float *h, hipStream_t s);

// GEMM y = x . W^T with x given as an fp16 hi/lo pair (x ~= hi + lo) in the
// operand-tile layout (xt_index in jev_dev.h; rows padded to 16) and W
// quantized.  Every output is computed in an order that does not depend on M.
enum GemmMode : int {
    kGemmStore = 0,  // y fp32 [M][ldy]   (ldy = total columns of all segments)
    kGemmSwiGlu = 1, // seg 0 = gate, seg 1 = up: out = silu(g)*u as fp16 hi/lo [M][N_gate]
};
struct GemmArgs {
    int M = 0, K = 0;
    const uint16_t *xt = nullptr;                  // fp16 pair, operand-tile layout
    const float *xsum = nullptr;                   // Q5_1 only: per-32 block sums [M][K/32]
    int nseg = 1;
    QWeight seg[3];
    int ldy = 0;
    float *y = nullptr;
    int ksplit = 1;                      // store mode: K in ksplit ranges, partial z at y + z*M*ldy
    // fold (store mode, ksplit > 1, batches of kGemmFoldMinRows rows or more): one
    // workgroup walks the ksplit ranges of its tile in order, each from zero,
    // and stores their sum taken in split order ((p0 + p1) + p2) + ... at y --
    // the value a consumer forms from the partials, so the same bits in one
    // buffer
    int fold = 0;
    uint16_t *ot = nullptr;              // SwiGLU output pair, operand-tile layout, K = seg[0].rows
    float *osum = nullptr;               // SwiGLU at M <= 16: per-32 block sums of ot [M][seg[0].rows / 32], or null
    int mode = kGemmStore;
    hipEvent_t ev_start = nullptr, ev_stop = nullptr; // optional dispatch-stamped timing
};
hipError_t launch_gemm(const GemmArgs &a, hipStream_t s);

// Integer strategy (IntegerDot): activations x [T][K] fp32 quantized to Q8_0
// blocks -- int8 quants in int8 MFMA operand tiles (T16 x K bytes), and per
// (block, token) block-major [K/32][T16]: the Half-rounded scale as float, the
// integer sum of the quants, and d * sum with the float d.
struct QuantActArgs {
    const float *x = nullptr;
    int T = 0, K = 0, T16 = 0;
    int8_t *xq = nullptr;
    float *xd = nullptr;
    int *xqs = nullptr;
    float *xs = nullptr;
};
hipError_t launch_quant_act(const QuantActArgs &a, hipStream_t s);
// y [T][ldy] = integer matmul of the quantized activations against w.
struct GemmI8Args {
    QWeight w;
    const int8_t *xq = nullptr;
    const float *xd = nullptr;
    const int *xqs = nullptr;
    const float *xs = nullptr;
    int T = 0, T16 = 0;
    float *y = nullptr;
    int ldy = 0;
};
hipError_t launch_gemm_i8(const GemmI8Args &a, hipStream_t s);
// Quant blocks per K split: an even count (whole 64-wide stages), the last
// split takes the remainder.  Depends on K and the split count only, so a
// row's partials are the same whatever M is.
__host__ __device__ inline int gemm_split_blocks(int nblk, int ksplit)
{
    return (((nblk + ksplit - 1) / ksplit) + 1) & ~1;
}
// Batches from this many rows take the store-mode GEMMs with their K-split
// partials summed inside the GEMM (GemmArgs::fold): there the partial
// buffers' HBM round trip through the consumer costs more than the GEMM's
// own extra accumulator set.  Q5_1 keeps the partials (its large-batch tile
// has no registers to spare).
constexpr int kGemmFoldMinRows = 8192;
inline bool gemm_fold(int type, int M, int ksplit) { return ksplit > 1 && M >= kGemmFoldMinRows && type != kQ5_1; }
// K-split count of a store-mode GEMM with N outputs and K inputs: up to 4
// splits of at least 8 blocks, so that narrow projections of small batches
// still fill the GPU.  A function of the weight shape only.
inline int gemm_choose_split(int N, int K)
{
    const int nblk = K >> 5;
    int s = N > 0 ? 12288 / N : 1;
    s = s < 1 ? 1 : (s > 4 ? 4 : s);
    while (s > 1 && (nblk / s < 8 || gemm_split_blocks(nblk, s) * (s - 1) >= nblk)) s--;
    return s;
}
// y[m][n] = sum_z partial[z][m][n] (+ res[m][n] if res), z ascending.
hipError_t launch_reduce_partials(const float *partial, int ksplit, int M, int N, float *y, hipStream_t s);

// One token's decode attention before its chunks are combined: per-chunk
// partials (max, sum, o[128]) of every head, [heads][max_chunks][130], and
// what fixes the token's visible-key count -- the layout arrays (entry 0) or
// the causal start (read from start_dev when set).
struct DecodeChunks {
    const float *part = nullptr;
    int max_chunks = 0;
    const int32_t *slot = nullptr, *shared_lo = nullptr, *shared_hi = nullptr, *segment = nullptr;
    int start = 0;
    const int32_t *start_dev = nullptr;
};

// GEMV for one token: y[r] = dot(x, W[r]) with fp32 x.  Up to 3 segments
// (outputs concatenated), or a gate/up pair with SwiGLU fused (y = silu(g)*u).
struct GemvArgs {
    int K = 0;
    const float *x = nullptr;
    int nseg = 1;
    QWeight seg[3];
    float *y = nullptr;
    int swiglu = 0;
    int ksplit = 1; // K in ksplit ranges (gemm_split_blocks), partial z at y + z * rows
    // x_up > 0: x holds a gate row and, x_up floats later, an up row; the
    // input is Kernels.SwiGlu of the pair (silu(g) * u), formed while staging
    int x_up = 0;
    // attn.part set: x is unused; the input is the decode attention output,
    // its chunks merged in ascending order while staging
    DecodeChunks attn;
    hipEvent_t ev_start = nullptr, ev_stop = nullptr; // optional dispatch-stamped timing
};
hipError_t launch_gemv(const GemvArgs &a, hipStream_t s);
// GEMV shape rules, functions of the weight shape only.  Many rows: each wave
// takes 16 rows over the whole K.  Otherwise the four waves of a workgroup
// share 16 rows, and narrow outputs split K over up to 4 workgroups as well.
inline bool gemv_rows_mode(int rows) { return (rows + 15) / 16 >= 2048; }
inline int gemv_choose_split(int rows, int K)
{
    if (gemv_rows_mode(rows)) return 1;
    const int groups = (rows + 15) / 16, nb = K >> 5;
    int s = 1;
    while (s < 4 && groups * 4 * s < 2048 && nb / (2 * s * 4) >= 4) s *= 2;
    return s;
}

// Row kernels.
//  rmsnorm: if add != nullptr, h[t] += add[t] first (stored back).  Output is
//  fp32 (out32) and/or an fp16 pair in the operand-tile layout (ot); xsum
//  (optional) receives per-32 block sums of the normalised row.
struct NormArgs {
    int T = 0, D = 0;
    float *h = nullptr;
    const float *add = nullptr;    // nadd K-split partials, add_stride floats apart
    int nadd = 1;
    size_t add_stride = 0;
    bool store_h = true;           // write h + add back into h
    const float *w = nullptr;
    float eps = 1e-5f;
    const int32_t *rows = nullptr; // optional row indices into h (output rows)
    float *out32 = nullptr;
    uint16_t *ot = nullptr;
    float *xsum = nullptr;
};
hipError_t launch_rmsnorm(const NormArgs &a, hipStream_t s);

// x [T][D] fp32 -> fp16 pair in the operand-tile layout.
hipError_t launch_split(const float *x, int T, int D, uint16_t *xt, hipStream_t s);

// Per-32 block sums of an operand-tile activation (Q5_1 offset term).
hipError_t launch_block_sums(const uint16_t *xt, int T, int D, float *xsum, hipStream_t s);

// RoPE + KV store: y is [T][qdim + 2*kvdim] (q | k | v) or separate pointers.
struct RopeArgs {
    int T = 0, n_heads = 0, n_kv = 0, hd = 128, half = 64;
    const float *q_in = nullptr, *k_in = nullptr, *v_in = nullptr;
    int ld_in = 0;
    int nin = 1;            // K-split partials of the inputs, in_stride floats apart
    size_t in_stride = 0;
    float *q_out = nullptr; // [T][qdim]
    float *kc = nullptr, *vc = nullptr; // layer base: [kvh][cap][hd]
    uint16_t *kp = nullptr, *vp = nullptr; // pair shadows, layer base: [kvh][cap][hi, lo][hd]
    int cap = 0;
    const int32_t *pos = nullptr, *slot = nullptr;
    int start = 0; // used when pos/slot are null (causal append)
    const int32_t *start_dev = nullptr; // if set, the causal start is read from device memory
    const float *freqs = nullptr;
    float mscale = 1.f;
    int orig_ctx = 0;
    float temp_scale = 0.f;
};
hipError_t launch_rope_store(const RopeArgs &a, hipStream_t s);

// Tree-masked attention tiles: consecutive tokens sharing (shared_lo,
// shared_hi, segment) with consecutive slots, at most kAttnTileTokens per tile
// (the query columns of one 32 x 32 MFMA).
constexpr int kAttnTileTokens = 32;
struct AttnTile {
    int32_t t0, n, shared_lo, shared_hi, segment, slot0, pad0, pad1;
};
struct AttnArgs {
    int n_tiles = 0, n_heads = 0, group = 4, hd = 128;
    const AttnTile *tiles = nullptr;
    const float *q = nullptr; // [T][qdim]
    const uint16_t *kp = nullptr, *vp = nullptr; // pair shadows, layer base [kvh][cap][hi, lo][hd]
    int cap = 0;
    float scale = 0.f;
    uint16_t *ot = nullptr; // context pair, operand-tile layout, K = qdim
    hipEvent_t ev_start = nullptr, ev_stop = nullptr; // optional dispatch-stamped timing
};
hipError_t launch_attn_tree(const AttnArgs &a, hipStream_t s);

// Decode attention: one query token per entry, split over kDecodeKeys-key
// chunks; leaves per-chunk partials for the consumer (GemvArgs::attn).
constexpr int kDecodeKeys = 64;
// A pass whose attention tiles are all single tokens (rows of one token each)
// always takes the decode attention; its tokens are served in launch groups
// whose chunk partials (tokens x chunks of them) stay within this many, so the
// partials buffer stays bounded at any context.  The group size changes no
// token's arithmetic.
constexpr int kSingleRowsChunks = 4096;
struct DecodeAttnArgs {
    int T = 0, n_heads = 0, group = 4, hd = 128, max_chunks = 0;
    int t0 = 0; // first token of this launch: token t0 + blockIdx.x, partials at blockIdx.x
    const float *q = nullptr;
    const float *kc = nullptr, *vc = nullptr;
    int cap = 0;
    const int32_t *slot = nullptr, *shared_lo = nullptr, *shared_hi = nullptr, *segment = nullptr;
    int start = 0; // causal append when the arrays are null
    const int32_t *start_dev = nullptr; // if set, the causal start is read from device memory
    float scale = 0.f;
    float *part = nullptr;   // [T][heads][max_chunks][hd + 2], token t0 first
    // (T >= 2 needs the per-token arrays and q already rotated: rope_fused 0.)
    // One token (T = 1) with rope_fused: RoPE and the KV store happen here --
    // q from the projection partials of `rope` (q_in / k_in / v_in, nin,
    // in_stride, the frequency and scaling fields), the new key and value
    // written to kc / vc / kp / vp by the workgroup of the chunk that holds
    // them -- instead of in rope_store_kernel; `q` is then unused.
    int rope_fused = 0;
    RopeArgs rope;
    hipEvent_t ev_start = nullptr, ev_stop = nullptr; // optional dispatch-stamped timing
};
hipError_t launch_attn_decode(const DecodeAttnArgs &a, hipStream_t s);

// Several one-token queries (a pass whose attention tiles are all single
// tokens: the reasoning decider's rows) through the decode attention: each
// token's chunk partials merged in ascending chunk order -- the arithmetic of
// the one-token O GEMV's merge -- and written as the fp16 pair in the
// operand-tile layout the O projection's GEMM reads.
struct AttnCombineArgs {
    int T = 0, n_heads = 0, max_chunks = 0;
    int t0 = 0;                  // first token of this launch (as DecodeAttnArgs::t0)
    const float *part = nullptr; // [T][heads][max_chunks][130], indexed from t0
    const int32_t *slot = nullptr, *shared_lo = nullptr, *shared_hi = nullptr, *segment = nullptr;
    uint16_t *ot = nullptr; // [T16][heads * 128] pair tiles
    float *xsum = nullptr;  // [T][heads * 4] block sums of ot (Q5_1 projections), or null
    hipEvent_t ev_start = nullptr, ev_stop = nullptr;
};
hipError_t launch_attn_combine(const AttnCombineArgs &a, hipStream_t s);

// Verdict-row head: for each output b, logits[b][i] = dot(norm(h[outputs[b]]), W[rows[i]]).
struct HeadRowsArgs {
    int n_out = 0, n_rows = 0, D = 0;
    const float *xn = nullptr; // normalised output rows [n_out][D]
    QWeight table;
    const int32_t *rows = nullptr;
    float *out = nullptr;
};
hipError_t launch_head_rows(const HeadRowsArgs &a, hipStream_t s);

// Lowest index of the maximum of x[0..n).
// Greedy decode step: the argmax of x (ties to the lower index) becomes the
// next token: state[2] = token, out[state[1]] = token, then the step
// (state[1]) and the cache length (state[0]) advance by one.
hipError_t launch_argmax_decode(const float *x, int n, float *sv, int32_t *si, int32_t *state, int32_t *out,
                                hipStream_t s);
hipError_t launch_argmax(const float *x, int n, int32_t *result, float *scratch_val, int32_t *scratch_idx,
                         hipStream_t s);
// Greedy step of the rows layout: per row, argmax(logits[r]) -> tokens[r] and
// out[rowstep[r] * n_rows + r]; slot[r], pos[r] and rowstep[r] advance by one.
hipError_t launch_rows_step(const float *logits, int vocab, int n_rows, int32_t *tokens, int32_t *slot, int32_t *pos,
                            int32_t *rowstep, int32_t *out, hipStream_t s);

// KV copy for capacity growth: [L*kvh] heads of `len` rows from stride old_cap to new_cap.
// Pair shadow of a fp32 cache: [heads_total][cap][hd] -> [heads_total][cap][hi, lo][hd]
// for positions [0, len).
hipError_t launch_kv_split(const float *src, uint16_t *dst, int heads_total, int cap, int len, int hd, hipStream_t s);
hipError_t launch_kv_copy(const float *src, float *dst, int heads_total, int old_cap, int new_cap, int len, int hd,
                          hipStream_t s);

} // namespace jev
