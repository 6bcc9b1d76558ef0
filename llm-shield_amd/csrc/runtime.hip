// libjev host runtime: the C ABI of include/jev.h.
//
// Mirrors MinistralModel (MinistralModel.cs) behind the managed API: weights are
// bound once into HBM, the KV cache is a device arena laid out like KvCache
// ([layer][kv head][capacity][128] fp32, KvCache.cs:18-19, :75), and the
// private ForwardAsync (:301-435) becomes one enqueue of HIP kernels on the
// context's stream.  Calls of two or more tokens take the MFMA path (GEMM +
// tree attention), one-token calls the GEMV path (decode), as the reference
// switches between PanelGemm and the row-wise float dot at PanelMinTokens = 2
// (QuantMatMul.cs:51, :84).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/jev.h"
#include "jev_dev.h"
#include "jev_internal.h"

using namespace jev;

namespace {

thread_local std::string g_error;

int fail(int code, const char *fmt, ...)
{
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

#define HIP_TRY(expr)                                                                                          \
    do {                                                                                                       \
        hipError_t e_ = (expr);                                                                                \
        if (e_ != hipSuccess) return fail(JEV_EDEVICE, "%s failed: %s", #expr, hipGetErrorString(e_));         \
    } while (0)

int host_threads()
{
    unsigned n = std::thread::hardware_concurrency();
    return n == 0 ? 4 : (int)std::min(16u, n);
}

// A device buffer that only grows.
template <typename T>
struct DevBuf {
    T *p = nullptr;
    size_t n = 0;
    hipError_t ensure(size_t need)
    {
        if (need <= n) return hipSuccess;
        if (p) {
            // work queued on any stream may still read the old buffer
            hipError_t e = hipDeviceSynchronize();
            if (e != hipSuccess) return e;
            e = hipFree(p);
            if (e != hipSuccess) return e;
            p = nullptr;
            n = 0;
        }
        hipError_t e = hipMalloc((void **)&p, std::max<size_t>(need, 1) * sizeof(T));
        if (e == hipSuccess) n = need;
        return e;
    }
    void release()
    {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
};

struct Layer {
    float *attn_norm = nullptr, *ffn_norm = nullptr;
    int64_t attn_norm_n = 0, ffn_norm_n = 0; // elements bound
    QWeight q, k, v, o, gate, up, down;
};

bool is_quant(int type) { return type == kQ8_0 || type == kQ4_0 || type == kQ5_1; }

void free_weight(QWeight &w)
{
    if (w.base) (void)hipFree(w.base);
    w = QWeight();
}

} // namespace

struct jev_ctx {
    jev_config cfg{};
    int device = 0;
    hipStream_t stream = nullptr;
    QWeight embd, output;
    float *out_norm = nullptr;
    int64_t out_norm_n = 0;
    std::vector<Layer> layers;
    float *freqs = nullptr;
    int half = 0;
    float mscale = 1.f;
    bool finalized = false;
    // Cancellation (ParallelOptions.CancellationToken): `active` is the id of
    // the call in flight (0 when idle); jev_cancel marks that id, so a cancel
    // never outlives the call it was aimed at.
    std::atomic<uint64_t> active{0}, cancel_id{0};
    uint64_t calls = 0;
    // One event per group of layers (a forward pass) or per step (a greedy
    // decode) in flight: the host stays at most kLeadLayers groups or steps
    // ahead of the device, so that a cancel stops the work within that many.
    static constexpr int kLayerEvents = 4, kLeadLayers = 2;
    hipEvent_t layer_ev[kLayerEvents] = {};

    // KV arena: fp32 K and V (the cache's contents) and their fp16-pair
    // shadows (same byte size; [layer][kv head][cap][hi, lo][hd]) that the
    // prefill/tree attention stages from
    float *kc = nullptr, *vc = nullptr;
    uint16_t *kp = nullptr, *vp = nullptr;
    int cap = 0, len = 0;

    // workspace
    DevBuf<float> h, y, yo, ydown, q, x32, f32, xn, logits, part, xsum, cap32;
    DevBuf<uint16_t> xt, ft; // fp16 pairs in the GEMM operand-tile layout
    DevBuf<int32_t> ints, dec_state;
    DevBuf<AttnTile> tiles;
    DevBuf<float> amax_v;
    DevBuf<int32_t> amax_i;
    std::vector<int32_t> host_ints;
    std::vector<AttnTile> host_tiles;
    // Pinned staging for the per-call metadata upload; `copied` marks when the
    // previous upload has left it.
    int32_t *pin_ints = nullptr;
    size_t pin_ints_n = 0;
    AttnTile *pin_tiles = nullptr;
    size_t pin_tiles_n = 0;
    hipEvent_t copied = nullptr;
    // Pinned landing buffer of the outputs a call returns to the host: a
    // device-to-pageable copy of the 512 KiB logits cost ~80 us more than a
    // copy to pinned memory plus a host memcpy.  Every call that uses it
    // drains the stream before returning, so it is free between calls.
    float *pin_out = nullptr;
    size_t pin_out_n = 0;

    // Kernel timing (jev_profile_enable).
    struct ProfRec {
        int cls;
        hipEvent_t a, b;
        double flops, bytes;
    };
    bool profiling = false;
    bool capturing = false; // a graph capture is open on the stream (no event records)
    // Step stamps (jev_profile_enable mode 2): the greedy decodes keep their
    // graphs and record a timing event at every step boundary.
    bool step_stamps = false;
    std::vector<hipEvent_t> step_ev;
    std::vector<float> step_ms; // the last greedy decode's per-step device times
    std::vector<hipEvent_t> ev_pool;
    size_t ev_used = 0;
    std::vector<ProfRec> prof;

    int qdim() const { return cfg.n_heads * cfg.head_dim; }
    int kvdim() const { return cfg.n_kv_heads * cfg.head_dim; }
    const QWeight &table() const { return output.base ? output : embd; }
    // K-split counts of the store-mode projections for a call of T tokens
    // (GEMM for two or more, GEMV for one); the partials are summed by the
    // kernel that consumes the output.
    static int split(int T, int N, int K) { return T >= 2 ? gemm_choose_split(N, K) : gemv_choose_split(N, K); }
    int split_qkv(int T) const { return split(T, qdim() + 2 * kvdim(), cfg.hidden); }
    int split_o(int T) const { return split(T, cfg.hidden, qdim()); }
    int split_down(int T) const { return split(T, cfg.hidden, cfg.ffn); }
    size_t layer_stride() const { return (size_t)cfg.n_kv_heads * cap * cfg.head_dim; }
};

// ---------------------------------------------------------------- helpers

namespace {

// Rope ctor (Rope.cs:33-66) on the host: the frequency table both the
// prefill and the decode path rotate with.
int rope_table(const jev_config &c, std::vector<float> &freqs, float &mscale)
{
    int half = c.rope_dim / 2;
    freqs.assign(half, 0.f);
    float freq_scale = 1.0f / c.rope_scale_factor;
    bool yarn = c.rope_scaling_yarn && c.rope_original_context > 0 && c.yarn_ext_factor != 0.0f &&
                c.rope_scale_factor > 1.0f; // ModelConfig.YarnActive (ModelConfig.cs:54-56)
    if (!yarn) {
        for (int i = 0; i < half; i++)
            freqs[i] = freq_scale / powf(c.rope_freq_base, 2.0f * (float)i / (float)c.rope_dim);
        mscale = c.rope_attn_factor;
        return half;
    }
    float low, high;
    if (c.yarn_beta_fast == 0.0f && c.yarn_beta_slow == 0.0f) { // YarnCorrectionDims (Rope.cs:91-106)
        low = 3.402823466e+38f;
        high = (float)c.rope_dim / 2.0f - 1.0f;
    } else {
        const float pi = 3.14159265358979323846f;
        float dims = (float)c.rope_dim, base = c.rope_freq_base;
        auto corr = [&](float rot) { return dims * logf((float)c.rope_original_context / (rot * 2.0f * pi)) / (2.0f * logf(base)); };
        low = fmaxf(0.0f, floorf(corr(c.yarn_beta_fast)));
        high = fminf(dims / 2.0f - 1.0f, ceilf(corr(c.yarn_beta_slow)));
    }
    for (int i = 0; i < half; i++) {
        float extrapolated = 1.0f / powf(c.rope_freq_base, 2.0f * (float)i / (float)c.rope_dim);
        float interpolated = freq_scale * extrapolated;
        float yv = ((float)i - low) / fmaxf(0.001f, high - low);
        float cl = std::min(1.0f, std::max(0.0f, yv));
        float mix = (1.0f - cl) * c.yarn_ext_factor;
        float a = interpolated * (1.0f - mix);
        float b = extrapolated * mix;
        freqs[i] = a + b;
    }
    auto ms = [](float scale, float m) { return scale <= 1.0f ? 1.0f : 0.1f * m * logf(scale) + 1.0f; };
    float factor = c.rope_scale_factor; // ComputeMagnitudeScale (Rope.cs:78-88)
    float m = c.yarn_mscale != 0.0f ? c.yarn_mscale : 1.0f;
    float ratio = c.yarn_mscale_all_dim != 0.0f ? ms(factor, m) / ms(factor, c.yarn_mscale_all_dim) : ms(factor, 1.0f);
    mscale = ratio * c.rope_attn_factor;
    return half;
}

// Event pair around one launch when profiling (no-op otherwise).
struct ProfScope {
    jev_ctx *c;
    int cls;
    double flops, bytes;
    hipEvent_t a = nullptr, z = nullptr;
    bool stamped = false;
    // stamped: the caller's one kernel launch stamps a and z itself
    // (hipExtLaunchKernelGGL, GemmArgs::ev_start / ev_stop), so the time is the
    // kernel's alone; otherwise event markers bracket everything in the scope.
    ProfScope(jev_ctx *ctx, int k, double f, double b, bool by_launch = false)
        : c(ctx), cls(k), flops(f), bytes(b)
    {
        if (!c->profiling || c->capturing) return;
        a = next_event();
        if (by_launch) {
            z = next_event();
            stamped = true;
            return;
        }
        (void)hipEventRecord(a, c->stream);
    }
    ~ProfScope()
    {
        if (!a) return;
        if (!stamped) {
            z = next_event();
            (void)hipEventRecord(z, c->stream);
        }
        c->prof.push_back({cls, a, z, flops, bytes});
    }
    hipEvent_t next_event()
    {
        if (c->ev_used == c->ev_pool.size()) {
            hipEvent_t e = nullptr;
            if (hipEventCreate(&e) != hipSuccess) return nullptr;
            c->ev_pool.push_back(e);
        }
        return c->ev_pool[c->ev_used++];
    }
};

// Marks one cancellable call in flight on a context.
struct CallScope {
    jev_ctx *c;
    uint64_t id;
    explicit CallScope(jev_ctx *ctx) : c(ctx), id(++ctx->calls) { c->active.store(id); }
    ~CallScope() { c->active.store(0); }
    bool cancelled() const { return c->cancel_id.load() == id; }
};

// Timing events for the step boundaries of a greedy decode of n steps.
int step_events(jev_ctx *c, int n)
{
    while ((int)c->step_ev.size() < n + 1) {
        hipEvent_t e = nullptr;
        HIP_TRY(hipEventCreate(&e));
        c->step_ev.push_back(e);
    }
    c->step_ms.clear();
    return JEV_OK;
}

// After the stream has drained: the device time of each of the `launched` steps.
void read_step_times(jev_ctx *c, int launched)
{
    c->step_ms.assign(launched, 0.f);
    for (int i = 0; i < launched; i++)
        if (hipEventElapsedTime(&c->step_ms[i], c->step_ev[i], c->step_ev[i + 1]) != hipSuccess) c->step_ms[i] = -1.f;
}

double weight_bytes(const QWeight &w) { return (double)row_bytes(w.type, w.cols) * w.rows; }

// Uploads GGUF rows into a field-split HBM weight.
int upload_weight(int type, int64_t rows, int64_t cols, const void *bytes, QWeight &w)
{
    QLayout L = qlayout(type, rows, cols);
    std::vector<uint8_t> staging(L.total);
    if (!repack_host(type, rows, cols, bytes, staging.data(), host_threads()))
        return fail(JEV_EINVAL, "cannot repack a %lld x %lld tensor of type %d", (long long)rows, (long long)cols, type);
    void *base = nullptr;
    hipError_t e = hipMalloc(&base, L.total);
    if (e != hipSuccess) return fail(JEV_ENOMEM, "hipMalloc(%zu) for a weight failed: %s", L.total, hipGetErrorString(e));
    e = hipMemcpy(base, staging.data(), L.total, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(base);
        return fail(JEV_EDEVICE, "weight upload failed: %s", hipGetErrorString(e));
    }
    w.type = type;
    w.rows = (int)rows;
    w.cols = (int)cols;
    w.base = base;
    w.bytes = L.total;
    uint8_t *b8 = (uint8_t *)base;
    w.qs = b8 + L.qs;
    w.d = (const uint16_t *)(b8 + L.d);
    w.m = type == kQ5_1 ? (const uint16_t *)(b8 + L.m) : nullptr;
    w.qh = type == kQ5_1 ? b8 + L.qh : nullptr;
    w.qb = type == kQ5_1 ? b8 + L.qb : nullptr;
    return JEV_OK;
}

int upload_vector(int type, int64_t count, const void *bytes, float **dst)
{
    std::vector<float> v((size_t)count);
    if (type == kF32) {
        std::memcpy(v.data(), bytes, (size_t)count * 4);
    } else if (type == kF16) {
        const uint16_t *hp = (const uint16_t *)bytes;
        for (int64_t i = 0; i < count; i++) {
            uint16_t hv;
            std::memcpy(&hv, hp + i, 2);
            v[(size_t)i] = half_to_float(hv);
        }
    } else {
        return fail(JEV_EDATA, "a 1-D parameter must be F32 or F16, got type %d", type);
    }
    if (*dst) (void)hipFree(*dst);
    *dst = nullptr;
    HIP_TRY(hipMalloc((void **)dst, (size_t)count * sizeof(float)));
    HIP_TRY(hipMemcpy(*dst, v.data(), (size_t)count * sizeof(float), hipMemcpyHostToDevice));
    return JEV_OK;
}

// KvCache.EnsureCapacity (KvCache.cs:48-70): doubles until it fits and copies
// the populated prefix of every head.
int kv_ensure(jev_ctx *c, int required)
{
    if (required <= c->cap) return JEV_OK;
    int cap = std::max(1, c->cap);
    while (cap < required) cap *= 2;
    size_t heads = (size_t)c->cfg.n_layers * c->cfg.n_kv_heads;
    size_t bytes = heads * cap * c->cfg.head_dim * sizeof(float);
    void *buf[4] = {nullptr, nullptr, nullptr, nullptr};
    hipError_t e = hipSuccess;
    for (int i = 0; i < 4 && e == hipSuccess; i++) e = hipMalloc(&buf[i], bytes);
    if (e != hipSuccess) {
        for (void *b : buf)
            if (b) (void)hipFree(b);
        return fail(JEV_ENOMEM, "KV cache growth to %d positions (%zu bytes x 4) failed: %s", cap, bytes,
                    hipGetErrorString(e));
    }
    float *k = (float *)buf[0], *v = (float *)buf[1];
    uint16_t *kp = (uint16_t *)buf[2], *vp = (uint16_t *)buf[3];
    if (c->kc && c->len > 0) {
        // a pair row is as long as a fp32 row: the shadows move as 4-byte words
        HIP_TRY(launch_kv_copy(c->kc, k, (int)heads, c->cap, cap, c->len, c->cfg.head_dim, c->stream));
        HIP_TRY(launch_kv_copy(c->vc, v, (int)heads, c->cap, cap, c->len, c->cfg.head_dim, c->stream));
        HIP_TRY(launch_kv_copy((const float *)c->kp, (float *)kp, (int)heads, c->cap, cap, c->len, c->cfg.head_dim,
                               c->stream));
        HIP_TRY(launch_kv_copy((const float *)c->vp, (float *)vp, (int)heads, c->cap, cap, c->len, c->cfg.head_dim,
                               c->stream));
    }
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (c->kc) (void)hipFree(c->kc);
    if (c->vc) (void)hipFree(c->vc);
    if (c->kp) (void)hipFree(c->kp);
    if (c->vp) (void)hipFree(c->vp);
    c->kc = k;
    c->vc = v;
    c->kp = kp;
    c->vp = vp;
    c->cap = cap;
    return JEV_OK;
}

bool same_type3(const QWeight &a, const QWeight &b, const QWeight &c) { return a.type == b.type && b.type == c.type; }

// One linear step y = x . W^T over up to three weights sharing x, as
// `ksplit` K-split partials T * ldy floats apart.  T >= 2: MFMA GEMM on the
// fp16 pair in the operand-tile layout; T == 1: GEMV on fp32 x.
// x_up (one token): x32 holds gate | up rows and the GEMV's input is their SwiGLU.
// attn (one token): the GEMV's input is the decode attention output, combined
// from its chunk partials while staging (x32 unused).
int linear(jev_ctx *c, int T, const QWeight *const *ws, int nw, const uint16_t *xt, const float *xsum,
           const float *x32, float *y, int ldy, int ksplit, int x_up = 0, const DecodeChunks *attn = nullptr)
{
    double nrows = 0, wbytes = 0;
    for (int i = 0; i < nw; i++) {
        nrows += ws[i]->rows;
        wbytes += weight_bytes(*ws[i]);
    }
    const double K = ws[0]->cols;
    if (T == 1) {
        GemvArgs g;
        g.K = ws[0]->cols;
        g.x = x32;
        g.nseg = nw;
        for (int i = 0; i < nw; i++) g.seg[i] = *ws[i];
        g.y = y;
        g.ksplit = ksplit;
        g.x_up = x_up;
        if (attn) g.attn = *attn;
        ProfScope ps(c, JEV_PROF_GEMV, 2.0 * nrows * K, wbytes + 4.0 * (K + nrows), true);
        g.ev_start = ps.a;
        g.ev_stop = ps.z;
        HIP_TRY(launch_gemv(g, c->stream));
        return JEV_OK;
    }
    ProfScope ps(c, JEV_PROF_GEMM, 2.0 * T * nrows * K, wbytes + T * (4.0 * K + 4.0 * nrows), true);
    GemmArgs g;
    g.M = T;
    g.K = ws[0]->cols;
    g.xt = xt;
    g.xsum = xsum;
    g.nseg = nw;
    for (int i = 0; i < nw; i++) g.seg[i] = *ws[i];
    g.ldy = ldy;
    g.y = y;
    g.ksplit = ksplit;
    g.fold = gemm_fold(ws[0]->type, T, ksplit) ? 1 : 0; // one buffer: stored_parts() is 1
    g.ev_start = ps.a;
    g.ev_stop = ps.z;
    HIP_TRY(launch_gemm(g, c->stream));
    return JEV_OK;
}

// Tokens per decode-attention launch of a single-token-rows pass: the chunk
// partials of one launch stay within kSingleRowsChunks.
int single_rows_group(int T, int max_chunks) { return std::max(1, std::min(T, kSingleRowsChunks / std::max(1, max_chunks))); }

// K-split partials a store-mode projection of T tokens leaves for its
// consumer: its split count, or one buffer when the GEMM sums them itself
// (gemm_fold); the GEMV path (T == 1) always leaves its partials.
int stored_parts(int T, const QWeight &w, int ksplit) { return T >= 2 && gemm_fold(w.type, T, ksplit) ? 1 : ksplit; }

int ensure_workspace(jev_ctx *c, int T, int n_out, int mode, int max_chunks, bool single_rows = false)
{
    const jev_config &f = c->cfg;
    size_t qkv = (size_t)c->qdim() + 2 * c->kvdim();
    size_t wide = std::max<size_t>({(size_t)f.hidden, (size_t)c->qdim(), (size_t)f.ffn});
    HIP_TRY(c->h.ensure((size_t)T * f.hidden));
    HIP_TRY(c->y.ensure((size_t)T * qkv * c->split_qkv(T)));
    HIP_TRY(c->yo.ensure((size_t)T * f.hidden * c->split_o(T)));
    HIP_TRY(c->ydown.ensure((size_t)T * f.hidden * c->split_down(T)));
    HIP_TRY(c->q.ensure((size_t)T * c->qdim()));
    // [0, T * wide / 32): the block sums a GEMM reads; past it, the SwiGLU
    // output's, written by the small-batch SwiGLU GEMM while it still reads
    // its own input's
    HIP_TRY(c->xsum.ensure((size_t)std::max(T, n_out) * wide / 32 + (T <= 16 ? (size_t)T * f.ffn / 32 : 0) + 1));
    if (T == 1) {
        HIP_TRY(c->x32.ensure((size_t)std::max<size_t>(f.hidden, 1)));
        HIP_TRY(c->f32.ensure((size_t)2 * f.ffn));
        HIP_TRY(c->part.ensure((size_t)f.n_heads * std::max(1, max_chunks) * 130));
    } else {
        if (single_rows)
            HIP_TRY(c->part.ensure((size_t)single_rows_group(T, max_chunks) * f.n_heads * std::max(1, max_chunks) * 130));
        size_t T16 = ((size_t)T + 15) & ~(size_t)15;
        HIP_TRY(c->xt.ensure(T16 * std::max(f.hidden, c->qdim()) * 2));
        HIP_TRY(c->ft.ensure(T16 * f.ffn * 2));
    }
    size_t nx = std::max(1, n_out);
    HIP_TRY(c->xn.ensure(nx * f.hidden));
    if (mode == JEV_OUT_FULL || mode == JEV_OUT_LAST_FULL) {
        HIP_TRY(c->logits.ensure(nx * (size_t)f.vocab));
        if (nx >= 2) HIP_TRY(c->xt.ensure(std::max(c->xt.n, ((nx + 15) & ~(size_t)15) * f.hidden * 2)));
    }
    HIP_TRY(c->amax_v.ensure(512));
    HIP_TRY(c->amax_i.ensure(512));
    return JEV_OK;
}

struct Plan {
    int T = 0;
    int start = 0;
    int end = 0;
    bool has_layout = false;
    int n_out = 1;
    int max_chunks = 0;
    // device pointers into ctx->ints
    const int32_t *d_tokens = nullptr, *d_slot = nullptr, *d_pos = nullptr, *d_slo = nullptr, *d_shi = nullptr,
                  *d_seg = nullptr, *d_out = nullptr, *d_rows = nullptr;
    int n_tiles = 0;
    // every attention tile a single token (rows of one token each): the
    // decode attention serves them, its chunks combined per token
    bool single_rows = false;
    // ... and no token sees another's key from this pass (rows: each sees the
    // cached prefix and its own row): each token's RoPE and KV store can run
    // inside its own decode attention, as for one token
    bool rows_independent = false;
    double visible_pairs = 0; // sum over tokens of visible keys
    double kv_rows = 0;       // distinct cache rows a layer's attention reads
};

// Validates a layout the way the reference's own checks would fail
// (MinistralModel.cs:306, :202-207) plus what keeps every kernel in bounds.
int check_layout(const jev_ctx *c, int T, const jev_layout *L)
{
    if (!L->slot || !L->position || !L->shared_lo || !L->shared_hi || !L->segment)
        return fail(JEV_EINVAL, "layout arrays must not be null");
    if (L->end <= 0 || L->end > (1 << 28)) return fail(JEV_EINVAL, "layout end %d is out of range", L->end);
    for (int t = 0; t < T; t++) {
        int s = L->slot[t], lo = L->shared_lo[t], hi = L->shared_hi[t], seg = L->segment[t];
        if (s < 0 || s >= L->end) return fail(JEV_EINVAL, "token %d: slot %d outside [0, end=%d)", t, s, L->end);
        if (lo < 0 || hi < lo || hi > L->end) return fail(JEV_EINVAL, "token %d: shared range [%d, %d) is invalid", t, lo, hi);
        if (seg < 0 || seg > s) return fail(JEV_EINVAL, "token %d: segment %d is after its slot %d", t, seg, s);
        if (L->position[t] < 0) return fail(JEV_EINVAL, "token %d: negative position", t);
    }
    if (L->n_outputs < 0 || (L->n_outputs > 0 && !L->outputs)) return fail(JEV_EINVAL, "bad outputs list");
    for (int b = 0; b < L->n_outputs; b++)
        if (L->outputs[b] < 0 || L->outputs[b] >= T) return fail(JEV_EINVAL, "output %d names token %d of %d", b, L->outputs[b], T);
    return JEV_OK;
}

// Uploads tokens (unless already on the device), layout arrays, outputs,
// selected rows and the attention tiles.
int build_plan(jev_ctx *c, const int32_t *tokens, bool tokens_on_device, int T, const jev_layout *L, int mode,
               const int32_t *rows, int n_rows, Plan &p)
{
    p.T = T;
    p.start = c->len;
    p.has_layout = L != nullptr;
    p.end = L ? L->end : c->len + T;
    p.n_out = L ? L->n_outputs : 1;
    if (mode == JEV_OUT_LAST_FULL) p.n_out = 1;

    std::vector<int32_t> &H = c->host_ints;
    H.clear();
    auto push = [&](const int32_t *src, int n) {
        size_t off = H.size();
        if (src) H.insert(H.end(), src, src + n);
        else H.resize(H.size() + n, 0);
        return off;
    };
    size_t o_tok = push(tokens_on_device ? nullptr : tokens, T);
    size_t o_slot = 0, o_pos = 0, o_slo = 0, o_shi = 0, o_seg = 0;
    if (L) {
        o_slot = push(L->slot, T);
        o_pos = push(L->position, T);
        o_slo = push(L->shared_lo, T);
        o_shi = push(L->shared_hi, T);
        o_seg = push(L->segment, T);
    }
    std::vector<int32_t> outs;
    if (mode == JEV_OUT_LAST_FULL || !L) outs.push_back(T - 1);
    else outs.assign(L->outputs, L->outputs + L->n_outputs);
    size_t o_out = push(outs.data(), (int)outs.size());
    size_t o_rows = push(rows, rows ? n_rows : 0);

    // Attention tiles (T >= 2) and decode chunks (T == 1).
    std::vector<AttnTile> &tiles = c->host_tiles;
    tiles.clear();
    int max_limit = 0;
    for (int t = 0; t < T;) {
        auto at = [&](int i, int &slot, int &lo, int &hi, int &seg) {
            if (L) {
                slot = L->slot[i];
                lo = L->shared_lo[i];
                hi = L->shared_hi[i];
                seg = L->segment[i];
            } else {
                slot = p.start + i;
                lo = 0;
                hi = p.start;
                seg = p.start;
            }
        };
        int s0, lo0, hi0, seg0;
        at(t, s0, lo0, hi0, seg0);
        int n = 1;
        while (n < kAttnTileTokens && t + n < T) {
            int s, lo, hi, seg;
            at(t + n, s, lo, hi, seg);
            if (lo != lo0 || hi != hi0 || seg != seg0 || s != s0 + n) break;
            n++;
        }
        AttnTile tile{t, n, lo0, hi0, seg0, s0, 0, 0};
        tiles.push_back(tile);
        for (int i = 0; i < n; i++) p.visible_pairs += (double)(hi0 - lo0) + (s0 + i - seg0 + 1);
        max_limit = std::max(max_limit, (hi0 - lo0) + (s0 + n - 1 - seg0 + 1));
        t += n;
    }
    p.n_tiles = (int)tiles.size();
    p.kv_rows = std::min<double>(p.end, max_limit + (double)T);
    p.max_chunks = (max_limit + kDecodeKeys - 1) / kDecodeKeys;
    // a function of the layout's shape alone -- not of the context length or
    // of how many rows run -- so a rows step takes the same attention kernel
    // whether it is replayed from a graph or run step by step
    p.single_rows = L && T >= 2 && p.n_tiles == T;
    if (p.single_rows) {
        std::vector<int32_t> fresh(L->slot, L->slot + T);
        std::sort(fresh.begin(), fresh.end());
        auto any_in = [&](int a, int b) { // a slot of this pass in [a, b)
            return a < b && std::lower_bound(fresh.begin(), fresh.end(), b) - std::lower_bound(fresh.begin(), fresh.end(), a) > 0;
        };
        bool ok = true;
        for (int t = 0; t < T && ok; t++)
            ok = !any_in(L->shared_lo[t], L->shared_hi[t]) && !any_in(L->segment[t], L->slot[t]);
        p.rows_independent = ok;
    }

    HIP_TRY(c->ints.ensure(H.size() + 1));
    HIP_TRY(c->tiles.ensure(tiles.size() + 1));
    // Stage through pinned memory; wait until the previous upload has read it.
    HIP_TRY(hipEventSynchronize(c->copied));
    if (c->pin_ints_n < H.size() + 1) {
        if (c->pin_ints) HIP_TRY(hipHostFree(c->pin_ints));
        c->pin_ints = nullptr;
        c->pin_ints_n = 0;
        HIP_TRY(hipHostMalloc((void **)&c->pin_ints, (H.size() + 1) * sizeof(int32_t), hipHostMallocDefault));
        c->pin_ints_n = H.size() + 1;
    }
    if (c->pin_tiles_n < tiles.size() + 1) {
        if (c->pin_tiles) HIP_TRY(hipHostFree(c->pin_tiles));
        c->pin_tiles = nullptr;
        c->pin_tiles_n = 0;
        HIP_TRY(hipHostMalloc((void **)&c->pin_tiles, (tiles.size() + 1) * sizeof(AttnTile), hipHostMallocDefault));
        c->pin_tiles_n = tiles.size() + 1;
    }
    std::memcpy(c->pin_ints, H.data(), H.size() * sizeof(int32_t));
    std::memcpy(c->pin_tiles, tiles.data(), tiles.size() * sizeof(AttnTile));
    HIP_TRY(hipMemcpyAsync(c->ints.p, c->pin_ints, H.size() * sizeof(int32_t), hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(c->tiles.p, c->pin_tiles, tiles.size() * sizeof(AttnTile), hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipEventRecord(c->copied, c->stream));
    int32_t *base = c->ints.p;
    p.d_tokens = tokens_on_device ? tokens : base + o_tok;
    if (L) {
        p.d_slot = base + o_slot;
        p.d_pos = base + o_pos;
        p.d_slo = base + o_slo;
        p.d_shi = base + o_shi;
        p.d_seg = base + o_seg;
    }
    p.d_out = base + o_out;
    p.d_rows = rows ? base + o_rows : nullptr;
    return JEV_OK;
}

// Enqueues the whole forward pass; the head output lands in `dout`
// (device) or in ctx->logits / ctx->xn scratch.
// ---- Activation capture (IActivationSink, MinistralModel.cs:787-790).
//
// jev_capture records every tensor the reference observes in ForwardAsync
// (MinistralModel.cs:331-357, :418-422; AttentionAsync's q_rope, k_rope, v,
// attn_weighted) as the device holds it: the stream is synchronised at each
// tap and the tensor copied to the host.  K-split partials are summed in
// split order (as their consumer sums them); k_rope and v are read back from
// the cache rows the pass wrote; attn_weighted is rebuilt from the attention
// output the O projection reads (the fp16 pair hi + lo, or, for one token,
// the decode attention's chunks merged in ascending order).
struct Capture {
    struct Tap {
        std::string name;
        int rows, cols;
        std::vector<float> v;
    };
    std::vector<Tap> taps;
};

int cap_add(jev_ctx *c, Capture *cap, std::string name, const float *d, int rows, int cols)
{
    Capture::Tap t{std::move(name), rows, cols, std::vector<float>((size_t)rows * cols)};
    HIP_TRY(hipMemcpyAsync(t.v.data(), d, t.v.size() * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    cap->taps.push_back(std::move(t));
    return JEV_OK;
}

// K-split partials (nsplit of them, rows * cols floats apart) summed in split order.
int cap_partials(jev_ctx *c, Capture *cap, std::string name, const float *part, int nsplit, int rows, int cols)
{
    HIP_TRY(launch_reduce_partials(part, nsplit, rows, cols, c->cap32.p, c->stream));
    return cap_add(c, cap, std::move(name), c->cap32.p, rows, cols);
}

// Rows [start, start + T) of every KV head of one layer's cache as [T][kv heads * hd].
int cap_kv(jev_ctx *c, Capture *cap, std::string name, const float *layer, int start, int T)
{
    const int hd = c->cfg.head_dim, kvh = c->cfg.n_kv_heads;
    Capture::Tap t{std::move(name), T, kvh * hd, std::vector<float>((size_t)T * kvh * hd)};
    for (int h = 0; h < kvh; h++)
        HIP_TRY(hipMemcpy2DAsync(t.v.data() + (size_t)h * hd, (size_t)kvh * hd * sizeof(float),
                                 layer + ((size_t)h * c->cap + start) * hd, (size_t)hd * sizeof(float),
                                 (size_t)hd * sizeof(float), T, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    cap->taps.push_back(std::move(t));
    return JEV_OK;
}

// The attention output of T >= 2 tokens from its fp16 pair in the operand-tile layout.
int cap_pair(jev_ctx *c, Capture *cap, std::string name, const uint16_t *xt, int T, int K)
{
    const size_t T16 = ((size_t)T + 15) & ~(size_t)15;
    std::vector<uint16_t> raw(T16 * K * 2);
    HIP_TRY(hipMemcpyAsync(raw.data(), xt, raw.size() * sizeof(uint16_t), hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    Capture::Tap t{std::move(name), T, K, std::vector<float>((size_t)T * K)};
    const int nblk = K >> 5;
    for (int r = 0; r < T; r++)
        for (int k = 0; k < K; k++)
            t.v[(size_t)r * K + k] = half_to_float(raw[xt_index(r, k, nblk, 0)]) + half_to_float(raw[xt_index(r, k, nblk, 1)]);
    cap->taps.push_back(std::move(t));
    return JEV_OK;
}

// The one-token decode attention output from its per-chunk (max, sum, o[hd])
// partials, merged in ascending chunk order with a running max, as the O
// projection's GEMV merges them.
int cap_chunks(jev_ctx *c, Capture *cap, std::string name, const float *part, int max_chunks, int nch)
{
    const int heads = c->cfg.n_heads, hd = c->cfg.head_dim, w = hd + 2;
    std::vector<float> raw((size_t)heads * max_chunks * w);
    HIP_TRY(hipMemcpyAsync(raw.data(), part, raw.size() * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    Capture::Tap t{std::move(name), 1, heads * hd, std::vector<float>((size_t)heads * hd)};
    for (int h = 0; h < heads; h++) {
        float M = -INFINITY, L = 0.f;
        float *o = t.v.data() + (size_t)h * hd;
        for (int ch = 0; ch < nch; ch++) {
            const float *pc = raw.data() + ((size_t)h * max_chunks + ch) * w;
            const float Mn = std::max(M, pc[0]), fo = expf(M - Mn), fc = expf(pc[0] - Mn);
            L = fmaf(pc[1], fc, L * fo);
            for (int d = 0; d < hd; d++) o[d] = fmaf(pc[2 + d], fc, o[d] * fo);
            M = Mn;
        }
        const float inv = 1.0f / L; // as the O projection's staging normalises
        for (int d = 0; d < hd; d++) o[d] = o[d] * inv;
    }
    cap->taps.push_back(std::move(t));
    return JEV_OK;
}

std::string layer_tap(int l, const char *tap)
{
    char b[64];
    snprintf(b, sizeof b, "blk.%d.%s", l, tap);
    return b;
}

// Layers per throttle group of a pass of T tokens: about kThrottleGroupFlops
// of linear work (~0.5 ms at the GEMMs' large-batch rate) per group, at most
// half the layers.  Each event marker in the stream costs the device several
// microseconds (one per layer added 3 % to a 256-token prefill), so short
// passes record a few per pass; passes of thousands of tokens keep one per
// layer.
constexpr double kThrottleGroupFlops = 2.0e11;
int throttle_group(const jev_ctx *c, int T)
{
    const jev_config &f = c->cfg;
    const double params = (double)f.hidden * (c->qdim() + 2 * c->kvdim()) + (double)c->qdim() * f.hidden +
                          3.0 * f.ffn * f.hidden;
    const double k = std::ceil(kThrottleGroupFlops / std::max(2.0 * T * params, 1.0));
    return (int)std::max(1.0, std::min(k, (double)std::max(1, f.n_layers / 2)));
}

// `call` (optional) is the cancellable call this pass belongs to: its cancel
// flag is checked before every layer; with `throttle` the host also waits,
// before each group of throttle_group layers, until the device has finished
// the group kLeadLayers back, so a cancel stops the pass within that many
// groups.
// With `cap` (a causal call of jev_capture) every tap is recorded as the pass
// produces it; the one-token pass then runs RoPE before the decode attention
// instead of inside it, so the rotated queries exist in memory.
int enqueue_forward(jev_ctx *c, const Plan &p, int mode, int n_rows, float *dout, const int32_t *dpos = nullptr,
                    const CallScope *call = nullptr, bool throttle = false, Capture *cap = nullptr)
{
#define CAP_TRY(expr)                                                                                           \
    do {                                                                                                        \
        if (cap) {                                                                                              \
            int rc_ = (expr);                                                                                   \
            if (rc_) return rc_;                                                                                \
        }                                                                                                       \
    } while (0)
    const jev_config &f = c->cfg;
    const int T = p.T, D = f.hidden, qdim = c->qdim(), kvdim = c->kvdim();
    const int group = f.n_heads / f.n_kv_heads;
    const float scale = 1.0f / sqrtf((float)f.head_dim);
    const bool q51 = c->layers[0].q.type == kQ5_1; // per-weight below
    (void)q51;
    hipStream_t s = c->stream;

    const int s_o = c->split_o(T), s_down = c->split_down(T);
    const size_t stride_d = (size_t)T * D; // floats between partials of yo / ydown
    HIP_TRY(launch_gather(c->embd, p.d_tokens, T, c->h.p, s));
    CAP_TRY(cap_add(c, cap, "embeddings", c->h.p, T, D));
    const int tg = throttle ? throttle_group(c, T) : 1;
    for (int l = 0; l < f.n_layers; l++) {
        if (call && throttle && l % tg == 0 && l / tg >= jev_ctx::kLeadLayers)
            HIP_TRY(hipEventSynchronize(c->layer_ev[(l / tg - jev_ctx::kLeadLayers) % jev_ctx::kLayerEvents]));
        if (call && call->cancelled()) return fail(JEV_ECANCELED, "the forward pass was cancelled at layer %d", l);
        const Layer &L = c->layers[l];
        float *kc = c->kc + (size_t)l * c->layer_stride();
        float *vc = c->vc + (size_t)l * c->layer_stride();
        uint16_t *kp = c->kp + 2 * (size_t)l * c->layer_stride();
        uint16_t *vp = c->vp + 2 * (size_t)l * c->layer_stride();

        // attention norm (+ the previous layer's FFN residual)
        NormArgs na;
        na.T = T;
        na.D = D;
        na.h = c->h.p;
        na.add = l > 0 ? c->ydown.p : nullptr;
        na.nadd = l > 0 ? stored_parts(T, c->layers[l - 1].down, s_down) : 1;
        na.add_stride = stride_d;
        na.w = L.attn_norm;
        na.eps = f.rms_eps;
        if (T == 1) na.out32 = c->x32.p;
        else {
            na.ot = c->xt.p;
            if (L.q.type == kQ5_1) na.xsum = c->xsum.p;
            if (cap) na.out32 = c->cap32.p;
        }
        HIP_TRY(launch_rmsnorm(na, s));
        if (l > 0) CAP_TRY(cap_add(c, cap, layer_tap(l - 1, "output"), c->h.p, T, D)); // h + the FFN residual
        CAP_TRY(cap_add(c, cap, layer_tap(l, "attn_norm"), na.out32, T, D));

        // Q | K | V
        const int ldqkv = qdim + 2 * kvdim;
        bool fuse = same_type3(L.q, L.k, L.v) && (T == 1 || (qdim % 128 == 0 && kvdim % 128 == 0));
        // separate projections share y's columns, so they are not split
        const int s_qkv = fuse ? c->split_qkv(T) : 1;
        if (fuse) {
            const QWeight *ws[3] = {&L.q, &L.k, &L.v};
            int rc = linear(c, T, ws, 3, c->xt.p, c->xsum.p, c->x32.p, c->y.p, ldqkv, s_qkv);
            if (rc) return rc;
        } else {
            const QWeight *wq[1] = {&L.q}, *wk[1] = {&L.k}, *wv[1] = {&L.v};
            float *yq = c->y.p, *yk = c->y.p + qdim, *yv = c->y.p + qdim + kvdim;
            int rc = linear(c, T, wq, 1, c->xt.p, c->xsum.p, c->x32.p, yq, ldqkv, 1);
            if (!rc) rc = linear(c, T, wk, 1, c->xt.p, c->xsum.p, c->x32.p, yk, ldqkv, 1);
            if (!rc) rc = linear(c, T, wv, 1, c->xt.p, c->xsum.p, c->x32.p, yv, ldqkv, 1);
            if (rc) return rc;
        }
        if (T == 1 && !fuse) {
            // GEMV writes rows contiguously; the three outputs of one token are
            // already at their column offsets.
        }

        RopeArgs ra;
        ra.T = T;
        ra.n_heads = f.n_heads;
        ra.n_kv = f.n_kv_heads;
        ra.hd = f.head_dim;
        ra.half = c->half;
        ra.q_in = c->y.p;
        ra.k_in = c->y.p + qdim;
        ra.v_in = c->y.p + qdim + kvdim;
        ra.ld_in = ldqkv;
        ra.nin = stored_parts(T, L.q, s_qkv);
        ra.in_stride = (size_t)T * ldqkv;
        ra.q_out = c->q.p;
        ra.kc = kc;
        ra.kp = kp;
        ra.vp = vp;
        ra.vc = vc;
        ra.cap = c->cap;
        ra.pos = p.d_pos;
        ra.slot = p.d_slot;
        ra.start = p.start;
        ra.start_dev = dpos;
        ra.freqs = c->freqs;
        ra.mscale = c->mscale;
        ra.orig_ctx = f.rope_original_context;
        ra.temp_scale = f.attention_temperature_scale;
        // one token, or rows of one token that see none of each other's keys:
        // RoPE and the KV store run inside the decode attention kernel
        const bool rows_fused = p.single_rows && p.rows_independent && !cap;
        if ((T != 1 && !rows_fused) || cap) HIP_TRY(launch_rope_store(ra, s));
        CAP_TRY(cap_add(c, cap, layer_tap(l, "q_rope"), c->q.p, T, qdim));
        CAP_TRY(cap_kv(c, cap, layer_tap(l, "k_rope"), kc, p.start, T));
        CAP_TRY(cap_kv(c, cap, layer_tap(l, "v"), vc, p.start, T));
        DecodeChunks dchunks;

        if (T == 1) {
            DecodeAttnArgs da;
            da.T = 1;
            da.n_heads = f.n_heads;
            da.group = group;
            da.hd = f.head_dim;
            da.max_chunks = p.max_chunks;
            da.q = c->q.p;
            da.kc = kc;
            da.vc = vc;
            da.cap = c->cap;
            da.slot = p.d_slot;
            da.shared_lo = p.d_slo;
            da.shared_hi = p.d_shi;
            da.segment = p.d_seg;
            da.start = p.start;
            da.start_dev = dpos;
            da.scale = scale;
            da.part = c->part.p;
            da.rope_fused = cap ? 0 : 1;
            da.rope = ra;
            // the O GEMV merges the chunks while staging its input
            dchunks.part = da.part;
            dchunks.max_chunks = da.max_chunks;
            dchunks.slot = da.slot;
            dchunks.shared_lo = da.shared_lo;
            dchunks.shared_hi = da.shared_hi;
            dchunks.segment = da.segment;
            dchunks.start = da.start;
            dchunks.start_dev = da.start_dev;
            ProfScope ps(c, JEV_PROF_DECODE_ATTN, 4.0 * f.head_dim * f.n_heads * p.visible_pairs,
                         8.0 * f.head_dim * f.n_kv_heads * p.visible_pairs, true);
            da.ev_start = ps.a;
            da.ev_stop = ps.z;
            HIP_TRY(launch_attn_decode(da, s));
            CAP_TRY(cap_chunks(c, cap, layer_tap(l, "attn_weighted"), c->part.p, p.max_chunks,
                               (p.start + 1 + kDecodeKeys - 1) / kDecodeKeys));
        } else if (p.single_rows) {
            // rows of one token: the decode attention per token (RoPE and the
            // KV store inside it, or by rope_store_kernel above when tokens
            // see each other's keys or taps are captured), then its chunks
            // combined into the O projection's pair input
            DecodeAttnArgs da;
            da.T = T;
            da.n_heads = f.n_heads;
            da.group = group;
            da.hd = f.head_dim;
            da.max_chunks = p.max_chunks;
            da.q = c->q.p;
            da.kc = kc;
            da.vc = vc;
            da.cap = c->cap;
            da.slot = p.d_slot;
            da.shared_lo = p.d_slo;
            da.shared_hi = p.d_shi;
            da.segment = p.d_seg;
            da.start = p.start;
            da.scale = scale;
            da.part = c->part.p;
            da.rope_fused = rows_fused ? 1 : 0;
            da.rope = ra;
            AttnCombineArgs ca;
            ca.n_heads = f.n_heads;
            ca.max_chunks = p.max_chunks;
            ca.part = c->part.p;
            ca.slot = p.d_slot;
            ca.shared_lo = p.d_slo;
            ca.shared_hi = p.d_shi;
            ca.segment = p.d_seg;
            ca.ot = c->xt.p;
            ca.xsum = L.o.type == kQ5_1 ? c->xsum.p : nullptr;
            // token groups share the partials buffer, one after the other
            const int G = single_rows_group(T, p.max_chunks);
            for (int t0 = 0; t0 < T; t0 += G) {
                da.t0 = ca.t0 = t0;
                da.T = ca.T = std::min(G, T - t0);
                {
                    ProfScope ps(c, JEV_PROF_DECODE_ATTN, 4.0 * f.head_dim * f.n_heads * p.visible_pairs * da.T / T,
                                 8.0 * f.head_dim * f.n_kv_heads * p.visible_pairs * da.T / T, true);
                    da.ev_start = ps.a;
                    da.ev_stop = ps.z;
                    HIP_TRY(launch_attn_decode(da, s));
                }
                HIP_TRY(launch_attn_combine(ca, s));
            }
            CAP_TRY(cap_pair(c, cap, layer_tap(l, "attn_weighted"), c->xt.p, T, qdim));
        } else {
            AttnArgs aa;
            aa.n_tiles = p.n_tiles;
            aa.n_heads = f.n_heads;
            aa.group = group;
            aa.hd = f.head_dim;
            aa.tiles = c->tiles.p;
            aa.q = c->q.p;
            aa.kp = kp;
            aa.vp = vp;
            aa.cap = c->cap;
            aa.scale = scale;
            aa.ot = c->xt.p;
            {
                ProfScope ps(c, JEV_PROF_ATTN, 4.0 * f.head_dim * f.n_heads * p.visible_pairs,
                             8.0 * f.head_dim * f.n_kv_heads * p.kv_rows + 8.0 * T * qdim, true);
                aa.ev_start = ps.a;
                aa.ev_stop = ps.z;
                HIP_TRY(launch_attn_tree(aa, s));
            }
            CAP_TRY(cap_pair(c, cap, layer_tap(l, "attn_weighted"), c->xt.p, T, qdim));
            if (L.o.type == kQ5_1) HIP_TRY(launch_block_sums(c->xt.p, T, qdim, c->xsum.p, s));
        }
        {
            const QWeight *wo[1] = {&L.o};
            int rc = linear(c, T, wo, 1, c->xt.p, c->xsum.p, nullptr, c->yo.p, D, s_o, 0,
                            T == 1 ? &dchunks : nullptr);
            if (rc) return rc;
        }
        CAP_TRY(cap_partials(c, cap, layer_tap(l, "attn_out"), c->yo.p, stored_parts(T, L.o, s_o), T, D));

        // FFN norm (+ attention residual)
        NormArgs nf = na;
        nf.add = c->yo.p;
        nf.nadd = stored_parts(T, L.o, s_o);
        nf.w = L.ffn_norm;
        nf.xsum = (T > 1 && L.gate.type == kQ5_1) ? c->xsum.p : nullptr;
        HIP_TRY(launch_rmsnorm(nf, s));
        CAP_TRY(cap_add(c, cap, layer_tap(l, "post_attn"), c->h.p, T, D));
        CAP_TRY(cap_add(c, cap, layer_tap(l, "ffn_norm"), nf.out32, T, D));

        const bool gu_rows = T == 1 && L.gate.type == L.up.type && f.ffn % 16 == 0;
        const float *down_sums = c->xsum.p;
        if (gu_rows) {
            // one token: gate and up rows as one GEMV of 2 x ffn rows (twice the
            // workgroups of the fused SwiGLU GEMV, so the GPU fills evenly); the
            // down GEMV forms silu(g) * u while staging its input
            const QWeight *wgu[2] = {&L.gate, &L.up};
            int rc = linear(c, T, wgu, 2, nullptr, nullptr, c->x32.p, c->f32.p, 2 * f.ffn, 1);
            if (rc) return rc;
        } else if (T == 1) {
            GemvArgs g;
            g.K = D;
            g.x = c->x32.p;
            g.nseg = 2;
            g.seg[0] = L.gate;
            g.seg[1] = L.up;
            g.y = c->f32.p;
            g.swiglu = 1;
            ProfScope ps(c, JEV_PROF_GEMV, 4.0 * f.ffn * D, weight_bytes(L.gate) + weight_bytes(L.up) + 4.0 * (D + f.ffn),
                         true);
            g.ev_start = ps.a;
            g.ev_stop = ps.z;
            HIP_TRY(launch_gemv(g, s));
        } else {
            GemmArgs g;
            g.M = T;
            g.K = D;
            g.xt = c->xt.p;
            g.xsum = c->xsum.p;
            g.nseg = 2;
            g.seg[0] = L.gate;
            g.seg[1] = L.up;
            g.mode = kGemmSwiGlu;
            g.ot = c->ft.p;
            // up to 16 tokens the SwiGLU GEMM also forms the down projection's
            // Q5_1 block sums
            if (L.down.type == kQ5_1 && T <= 16)
                g.osum = c->xsum.p + (size_t)T * std::max<size_t>({(size_t)f.hidden, (size_t)c->qdim(), (size_t)f.ffn}) / 32;
            {
                ProfScope ps(c, JEV_PROF_GEMM, 4.0 * T * f.ffn * D,
                             weight_bytes(L.gate) + weight_bytes(L.up) + T * (4.0 * D + 4.0 * f.ffn), true);
                g.ev_start = ps.a;
                g.ev_stop = ps.z;
                HIP_TRY(launch_gemm(g, s));
            }
            if (L.down.type == kQ5_1 && !g.osum) HIP_TRY(launch_block_sums(c->ft.p, T, f.ffn, c->xsum.p, s));
            down_sums = g.osum ? g.osum : c->xsum.p;
        }
        {
            const QWeight *wd[1] = {&L.down};
            int rc = linear(c, T, wd, 1, c->ft.p, down_sums, c->f32.p, c->ydown.p, D, s_down, gu_rows ? f.ffn : 0);
            if (rc) return rc;
        }
        CAP_TRY(cap_partials(c, cap, layer_tap(l, "ffn_out"), c->ydown.p, stored_parts(T, L.down, s_down), T, D));
        if (cap && l == f.n_layers - 1) {
            // the last layer's residual is folded into the final norm of the
            // output rows; h + ffn_out is that same single fp32 add
            const std::vector<float> &hp = cap->taps[cap->taps.size() - 3].v; // post_attn
            Capture::Tap o{layer_tap(l, "output"), T, D, cap->taps.back().v};
            for (size_t i = 0; i < o.v.size(); i++) o.v[i] = hp[i] + o.v[i];
            cap->taps.push_back(std::move(o));
        }
        if (call && throttle && (l % tg == tg - 1 || l == f.n_layers - 1))
            HIP_TRY(hipEventRecord(c->layer_ev[(l / tg) % jev_ctx::kLayerEvents], s));
    }

    // Heads.  The last layer's FFN residual is folded into the final norm of
    // the output rows (h itself is not needed after the last layer).
    if (mode == JEV_OUT_NONE) return JEV_OK;
    const QWeight &tab = c->table();
    NormArgs fn;
    fn.T = p.n_out;
    fn.D = D;
    fn.h = c->h.p;
    fn.add = c->ydown.p;
    fn.nadd = stored_parts(T, c->layers[f.n_layers - 1].down, s_down);
    fn.add_stride = stride_d;
    fn.store_h = false;
    fn.w = c->out_norm;
    fn.eps = f.rms_eps;
    fn.rows = p.d_out;
    if (mode == JEV_OUT_SELECTED) {
        fn.out32 = c->xn.p;
        HIP_TRY(launch_rmsnorm(fn, s));
        HeadRowsArgs hr;
        hr.n_out = p.n_out;
        hr.n_rows = n_rows;
        hr.D = D;
        hr.xn = c->xn.p;
        hr.table = tab;
        hr.rows = p.d_rows;
        hr.out = dout;
        HIP_TRY(launch_head_rows(hr, s));
        return JEV_OK;
    }
    // full vocabulary
    if (p.n_out == 1) {
        fn.out32 = c->xn.p;
        HIP_TRY(launch_rmsnorm(fn, s));
        CAP_TRY(cap_add(c, cap, "final_norm", c->xn.p, 1, D));
        GemvArgs g;
        g.K = D;
        g.x = c->xn.p;
        g.nseg = 1;
        g.seg[0] = tab;
        g.y = dout;
        {
            ProfScope ps(c, JEV_PROF_GEMV, 2.0 * tab.rows * D, weight_bytes(tab) + 4.0 * (D + tab.rows), true);
            g.ev_start = ps.a;
            g.ev_stop = ps.z;
            HIP_TRY(launch_gemv(g, s));
        }
        CAP_TRY(cap_add(c, cap, "logits", dout, 1, tab.rows));
    } else {
        fn.ot = c->xt.p;
        fn.xsum = tab.type == kQ5_1 ? c->xsum.p : nullptr;
        HIP_TRY(launch_rmsnorm(fn, s));
        GemmArgs g;
        g.M = p.n_out;
        g.K = D;
        g.xt = c->xt.p;
        g.xsum = c->xsum.p;
        g.nseg = 1;
        g.seg[0] = tab;
        g.ldy = tab.rows;
        g.y = dout;
        ProfScope ps(c, JEV_PROF_GEMM, 2.0 * p.n_out * tab.rows * D, weight_bytes(tab) + p.n_out * 4.0 * (D + tab.rows),
                     true);
        g.ev_start = ps.a;
        g.ev_stop = ps.z;
        HIP_TRY(launch_gemm(g, s));
    }
    return JEV_OK;
#undef CAP_TRY
}

size_t out_floats(const jev_ctx *c, int mode, int n_out, int n_rows)
{
    switch (mode) {
    case JEV_OUT_NONE: return 0;
    case JEV_OUT_LAST_FULL: return (size_t)c->cfg.vocab;
    case JEV_OUT_SELECTED: return (size_t)n_out * n_rows;
    case JEV_OUT_FULL: return (size_t)n_out * c->cfg.vocab;
    default: return 0;
    }
}

int check_ready(jev_ctx *c)
{
    if (!c) return fail(JEV_EINVAL, "null context");
    if (!c->finalized) return fail(JEV_ESTATE, "jev_finalize has not succeeded on this context");
    HIP_TRY(hipSetDevice(c->device));
    return JEV_OK;
}

// Copies n floats of device output to the caller's host buffer through the
// pinned landing buffer, draining the stream (the call's synchronisation).
int copy_out(jev_ctx *c, float *host, const float *dev, size_t n)
{
    if (n > c->pin_out_n) {
        if (c->pin_out) HIP_TRY(hipHostFree(c->pin_out));
        c->pin_out = nullptr;
        c->pin_out_n = 0;
        HIP_TRY(hipHostMalloc((void **)&c->pin_out, n * sizeof(float), hipHostMallocDefault));
        c->pin_out_n = n;
    }
    if (n) HIP_TRY(hipMemcpyAsync(c->pin_out, dev, n * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (n) std::memcpy(host, c->pin_out, n * sizeof(float));
    return JEV_OK;
}

// Common front half of jev_forward / jev_forward_device.
int prepare(jev_ctx *c, const int32_t *tokens, bool on_device, int T, const jev_layout *layout, int mode,
            const int32_t *rows, int n_rows, Plan &p)
{
    if (T <= 0) return fail(JEV_EINVAL, "No tokens to forward.");
    if (!tokens) return fail(JEV_EINVAL, "tokens is null");
    if (mode < JEV_OUT_NONE || mode > JEV_OUT_FULL) return fail(JEV_EINVAL, "unknown output mode %d", mode);
    if (mode == JEV_OUT_SELECTED) {
        if (!rows || n_rows <= 0) return fail(JEV_EINVAL, "selected-rows mode needs rows");
        for (int i = 0; i < n_rows; i++)
            if (rows[i] < 0 || rows[i] >= c->table().rows)
                return fail(JEV_EINVAL, "vocabulary row %d is outside the %d-row head", rows[i], c->table().rows);
    }
    if (!on_device)
        for (int t = 0; t < T; t++)
            if (tokens[t] < 0 || tokens[t] >= c->embd.rows) // QuantMatMul.GatherRows (QuantMatMul.cs:300-302)
                return fail(JEV_EINVAL, "Token id %d is outside the %d-entry embedding table.", tokens[t], c->embd.rows);
    if (layout) {
        int rc = check_layout(c, T, layout);
        if (rc) return rc;
        if (mode == JEV_OUT_SELECTED || mode == JEV_OUT_FULL)
            if (layout->n_outputs <= 0) return fail(JEV_EINVAL, "the layout lists no outputs");
    }
    int end = layout ? layout->end : c->len + T;
    int rc = kv_ensure(c, end);
    if (rc) return rc;
    rc = build_plan(c, tokens, on_device, T, layout, mode, rows, n_rows, p);
    if (rc) return rc;
    return ensure_workspace(c, T, p.n_out, mode, p.max_chunks, p.single_rows);
}

} // namespace

// ================================================================ C ABI

// QuantMatMul.Strategy (QuantMatMul.cs:41): process-wide, read at each call.
static std::atomic<int> g_matmul_strategy{JEV_MATMUL_AUTO};

extern "C" {

const char *jev_last_error(void) { return g_error.c_str(); }

int jev_create(const jev_config *cfg, int device, jev_ctx **out)
{
    if (!cfg || !out) return fail(JEV_EINVAL, "null argument");
    *out = nullptr;
    const jev_config &f = *cfg;
    if (f.n_layers <= 0 || f.hidden <= 0 || f.n_heads <= 0 || f.n_kv_heads <= 0 || f.ffn <= 0 || f.vocab <= 0)
        return fail(JEV_EINVAL, "model dimensions must be positive");
    if (f.n_heads % f.n_kv_heads != 0) // ModelConfig.FromGguf (ModelConfig.cs:108-110)
        return fail(JEV_EDATA, "%d attention heads do not divide into %d KV heads.", f.n_heads, f.n_kv_heads);
    if (f.head_dim != 128) return fail(JEV_EINVAL, "head_dim %d: the kernels are built for 128-wide heads", f.head_dim);
    if (f.hidden % 32 != 0 || f.ffn % 64 != 0) return fail(JEV_EINVAL, "hidden must be a multiple of 32 and ffn of 64");
    if (f.rope_dim <= 0 || f.rope_dim > f.head_dim || f.rope_dim % 2 != 0)
        return fail(JEV_EINVAL, "rope_dim %d must be even and at most head_dim", f.rope_dim);
    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess || ndev == 0) return fail(JEV_EDEVICE, "no HIP device: %s", hipGetErrorString(e));
    if (device < 0 || device >= ndev) return fail(JEV_EINVAL, "device %d of %d", device, ndev);
    HIP_TRY(hipSetDevice(device));
    jev_ctx *c = new jev_ctx();
    c->cfg = f;
    c->device = device;
    c->layers.resize(f.n_layers);
    e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        return fail(JEV_EDEVICE, "hipStreamCreate: %s", hipGetErrorString(e));
    }
    e = hipEventCreateWithFlags(&c->copied, hipEventDisableTiming);
    for (int i = 0; i < jev_ctx::kLayerEvents && e == hipSuccess; i++)
        e = hipEventCreateWithFlags(&c->layer_ev[i], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(c->copied, c->stream);
    if (e != hipSuccess) {
        jev_destroy(c);
        return fail(JEV_EDEVICE, "hipEventCreate: %s", hipGetErrorString(e));
    }
    std::vector<float> freqs;
    c->half = rope_table(f, freqs, c->mscale);
    e = hipMalloc((void **)&c->freqs, freqs.size() * sizeof(float));
    if (e == hipSuccess) e = hipMemcpy(c->freqs, freqs.data(), freqs.size() * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        jev_destroy(c);
        return fail(JEV_EDEVICE, "rope table: %s", hipGetErrorString(e));
    }
    int rc = kv_ensure(c, std::max(1, f.initial_kv_capacity));
    if (rc) {
        std::string msg = g_error;
        jev_destroy(c);
        return fail(rc, "%s", msg.c_str());
    }
    *out = c;
    return JEV_OK;
}

void jev_destroy(jev_ctx *c)
{
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    free_weight(c->embd);
    free_weight(c->output);
    if (c->out_norm) (void)hipFree(c->out_norm);
    for (auto &L : c->layers) {
        if (L.attn_norm) (void)hipFree(L.attn_norm);
        if (L.ffn_norm) (void)hipFree(L.ffn_norm);
        free_weight(L.q); free_weight(L.k); free_weight(L.v); free_weight(L.o);
        free_weight(L.gate); free_weight(L.up); free_weight(L.down);
    }
    if (c->freqs) (void)hipFree(c->freqs);
    if (c->kc) (void)hipFree(c->kc);
    if (c->vc) (void)hipFree(c->vc);
    if (c->kp) (void)hipFree(c->kp);
    if (c->vp) (void)hipFree(c->vp);
    c->h.release(); c->y.release(); c->yo.release(); c->ydown.release(); c->q.release();
    c->x32.release(); c->f32.release(); c->xn.release(); c->logits.release();
    c->part.release(); c->xsum.release(); c->cap32.release(); c->xt.release(); c->ft.release(); c->ints.release(); c->dec_state.release(); c->tiles.release(); c->amax_v.release(); c->amax_i.release();
    if (c->pin_ints) (void)hipHostFree(c->pin_ints);
    if (c->pin_tiles) (void)hipHostFree(c->pin_tiles);
    if (c->pin_out) (void)hipHostFree(c->pin_out);
    if (c->copied) (void)hipEventDestroy(c->copied);
    for (auto e : c->layer_ev)
        if (e) (void)hipEventDestroy(e);
    for (auto e : c->ev_pool) (void)hipEventDestroy(e);
    for (auto e : c->step_ev) (void)hipEventDestroy(e);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

int jev_bind_tensor(jev_ctx *c, int slot, int layer, int type, int64_t rows, int64_t cols, const void *bytes,
                    size_t nbytes)
{
    if (!c || !bytes) return fail(JEV_EINVAL, "null argument");
    HIP_TRY(hipSetDevice(c->device));
    if (slot < JEV_SLOT_TOKEN_EMBD || slot > JEV_SLOT_DOWN) return fail(JEV_EINVAL, "unknown tensor slot %d", slot);
    if (slot >= JEV_SLOT_ATTN_NORM && (layer < 0 || layer >= c->cfg.n_layers))
        return fail(JEV_EINVAL, "layer %d of %d", layer, c->cfg.n_layers);
    if (rows <= 0 || cols <= 0 || rows > INT32_MAX || cols > INT32_MAX) return fail(JEV_EINVAL, "bad shape");
    int bs = block_size(type);
    if (bs == 0) return fail(JEV_EDATA, "GGML type %d is not supported by this runtime", type);
    if (cols % bs != 0) return fail(JEV_EDATA, "%lld columns are not whole blocks of %d", (long long)cols, bs);
    size_t need = (size_t)row_bytes(type, cols) * (size_t)rows;
    if (nbytes < need) // GgufFile.ThrowIfTruncated's concern, per tensor
        return fail(JEV_EDATA, "tensor bytes are truncated: %zu of %zu", nbytes, need);
    c->finalized = false;
    bool vec = slot == JEV_SLOT_OUTPUT_NORM || slot == JEV_SLOT_ATTN_NORM || slot == JEV_SLOT_FFN_NORM;
    if (vec) {
        if (rows != 1) return fail(JEV_EDATA, "a norm weight must be 1-D");
        float **dst = slot == JEV_SLOT_OUTPUT_NORM ? &c->out_norm
                    : slot == JEV_SLOT_ATTN_NORM ? &c->layers[layer].attn_norm : &c->layers[layer].ffn_norm;
        int64_t *dn = slot == JEV_SLOT_OUTPUT_NORM ? &c->out_norm_n
                    : slot == JEV_SLOT_ATTN_NORM ? &c->layers[layer].attn_norm_n : &c->layers[layer].ffn_norm_n;
        *dn = 0;
        int rc = upload_vector(type, cols, bytes, dst);
        if (rc == JEV_OK) *dn = cols;
        return rc;
    }
    if (!is_quant(type)) return fail(JEV_EDATA, "weight matrices must be Q8_0, Q5_1 or Q4_0 (type %d)", type);
    QWeight *w = nullptr;
    switch (slot) {
    case JEV_SLOT_TOKEN_EMBD: w = &c->embd; break;
    case JEV_SLOT_OUTPUT: w = &c->output; break;
    case JEV_SLOT_Q: w = &c->layers[layer].q; break;
    case JEV_SLOT_K: w = &c->layers[layer].k; break;
    case JEV_SLOT_V: w = &c->layers[layer].v; break;
    case JEV_SLOT_O: w = &c->layers[layer].o; break;
    case JEV_SLOT_GATE: w = &c->layers[layer].gate; break;
    case JEV_SLOT_UP: w = &c->layers[layer].up; break;
    case JEV_SLOT_DOWN: w = &c->layers[layer].down; break;
    default: return fail(JEV_EINVAL, "slot %d", slot);
    }
    free_weight(*w);
    return upload_weight(type, rows, cols, bytes, *w);
}

int jev_finalize(jev_ctx *c)
{
    if (!c) return fail(JEV_EINVAL, "null context");
    const jev_config &f = c->cfg;
    int qdim = c->qdim(), kvdim = c->kvdim();
    if (!c->embd.base) return fail(JEV_EDATA, "missing tensor 'token_embd.weight'.");
    if (!c->out_norm) return fail(JEV_EDATA, "missing tensor 'output_norm.weight'.");
    // MinistralModel.ValidateShapes (MinistralModel.cs:110-123) and the rest of the shapes.
    if (c->embd.cols != f.hidden)
        return fail(JEV_EDATA, "token_embd is %d wide but the model's hidden size is %d.", c->embd.cols, f.hidden);
    if (c->table().rows != f.vocab || c->table().cols != f.hidden)
        return fail(JEV_EDATA, "the LM head is %d x %d; expected %d x %d", c->table().rows, c->table().cols, f.vocab, f.hidden);
    // Greedy decoding feeds argmax ids (< vocab) back into the embedding
    // gather on the device, so the table must hold every vocabulary row.
    if (c->embd.rows < f.vocab)
        return fail(JEV_EDATA, "token_embd has %d rows but the vocabulary has %d entries.", c->embd.rows, f.vocab);
    // The norm kernels read `hidden` weights (Kernels.RmsNorm, Kernels.cs:25-60).
    if (c->out_norm_n != f.hidden)
        return fail(JEV_EDATA, "output_norm.weight has %lld elements; expected %d.", (long long)c->out_norm_n, f.hidden);
    for (int l = 0; l < f.n_layers; l++) {
        Layer &L = c->layers[l];
        const char *missing = !L.attn_norm ? "attn_norm" : !L.ffn_norm ? "ffn_norm" : !L.q.base ? "attn_q"
                            : !L.k.base ? "attn_k" : !L.v.base ? "attn_v" : !L.o.base ? "attn_output"
                            : !L.gate.base ? "ffn_gate" : !L.up.base ? "ffn_up" : !L.down.base ? "ffn_down" : nullptr;
        if (missing) return fail(JEV_EDATA, "missing tensor 'blk.%d.%s.weight'.", l, missing);
        if (L.attn_norm_n != f.hidden || L.ffn_norm_n != f.hidden)
            return fail(JEV_EDATA, "blk.%d.%s.weight has %lld elements; expected %d.", l,
                        L.attn_norm_n != f.hidden ? "attn_norm" : "ffn_norm",
                        (long long)(L.attn_norm_n != f.hidden ? L.attn_norm_n : L.ffn_norm_n), f.hidden);
        struct { const QWeight *w; int r, c; const char *n; } chk[] = {
            {&L.q, qdim, f.hidden, "attn_q"}, {&L.k, kvdim, f.hidden, "attn_k"}, {&L.v, kvdim, f.hidden, "attn_v"},
            {&L.o, f.hidden, qdim, "attn_output"}, {&L.gate, f.ffn, f.hidden, "ffn_gate"},
            {&L.up, f.ffn, f.hidden, "ffn_up"}, {&L.down, f.hidden, f.ffn, "ffn_down"}};
        for (auto &k : chk)
            if (k.w->rows != k.r || k.w->cols != k.c)
                return fail(JEV_EDATA, "blk.%d.%s is %d x %d; expected %d x %d.", l, k.n, k.w->rows, k.w->cols, k.r, k.c);
        if (L.gate.type != L.up.type) return fail(JEV_EDATA, "blk.%d: ffn_gate and ffn_up must share a type", l);
    }
    c->finalized = true;
    return JEV_OK;
}

int jev_kv_length(jev_ctx *c, int32_t *length)
{
    if (!c || !length) return fail(JEV_EINVAL, "null argument");
    *length = c->len;
    return JEV_OK;
}

int jev_kv_capacity(jev_ctx *c, int32_t *capacity)
{
    if (!c || !capacity) return fail(JEV_EINVAL, "null argument");
    *capacity = c->cap;
    return JEV_OK;
}

int jev_kv_reserve(jev_ctx *c, int32_t required)
{
    if (!c) return fail(JEV_EINVAL, "null context");
    HIP_TRY(hipSetDevice(c->device));
    return kv_ensure(c, required);
}

int jev_kv_truncate(jev_ctx *c, int32_t length)
{
    if (!c) return fail(JEV_EINVAL, "null context");
    c->len = std::min(std::max(length, 0), c->len); // KvCache.Truncate (KvCache.cs:46)
    return JEV_OK;
}

int jev_kv_reset(jev_ctx *c)
{
    if (!c) return fail(JEV_EINVAL, "null context");
    c->len = 0;
    return JEV_OK;
}

// Copies positions [0, length) of every [layer][kv head] of the cache's K and V
// between the arena (rows `cap` positions apart) and a flat buffer in
// KvCache.Snapshot's order (KvCache.cs:94-112): keys [l][h][0..length)[hd],
// then values.  One pitched copy per array.
static int kv_flat_copy(jev_ctx *c, int32_t length, float *flat, bool to_flat, hipMemcpyKind kind)
{
    const jev_config &f = c->cfg;
    const size_t heads = (size_t)f.n_layers * f.n_kv_heads, row = (size_t)length * f.head_dim * sizeof(float);
    const size_t pitch = (size_t)c->cap * f.head_dim * sizeof(float);
    if (length == 0) return JEV_OK;
    for (int pass = 0; pass < 2; pass++) {
        float *arena = pass ? c->vc : c->kc;
        float *dense = flat + (size_t)pass * heads * length * f.head_dim;
        if (to_flat) HIP_TRY(hipMemcpy2DAsync(dense, row, arena, pitch, row, heads, kind, c->stream));
        else HIP_TRY(hipMemcpy2DAsync(arena, pitch, dense, row, row, heads, kind, c->stream));
    }
    return JEV_OK;
}

// KvCache.Snapshot (KvCache.cs:94-112): keys of every [layer][head], then values.
int jev_kv_snapshot(jev_ctx *c, int32_t length, float *out, size_t n)
{
    if (!c || !out) return fail(JEV_EINVAL, "null argument");
    if (length < 0 || length > c->len) return fail(JEV_EINVAL, "Only %d positions are cached.", c->len);
    const jev_config &f = c->cfg;
    size_t per = (size_t)f.n_layers * f.n_kv_heads * length * f.head_dim;
    if (n != per * 2) return fail(JEV_EINVAL, "Snapshot needs %zu floats; got %zu.", per * 2, n);
    HIP_TRY(hipSetDevice(c->device));
    int rc = kv_flat_copy(c, length, out, true, hipMemcpyDeviceToHost);
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize(c->stream));
    return JEV_OK;
}

// Leaves the cache holding exactly `length` positions from a flat K / V
// buffer already in the arena (KvCache.Restore's end state): the fp16-pair
// shadows the prefill attention reads are rebuilt from the fp32 rows.
static int kv_finish_restore(jev_ctx *c, int32_t length)
{
    const jev_config &f = c->cfg;
    const int heads = f.n_layers * f.n_kv_heads;
    HIP_TRY(launch_kv_split(c->kc, c->kp, heads, c->cap, length, f.head_dim, c->stream));
    HIP_TRY(launch_kv_split(c->vc, c->vp, heads, c->cap, length, f.head_dim, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    c->len = length;
    return JEV_OK;
}

// KvCache.Restore (KvCache.cs:115-136): leaves the cache holding exactly that prefix.
int jev_kv_restore(jev_ctx *c, const float *in, size_t n, int32_t length)
{
    if (!c || !in) return fail(JEV_EINVAL, "null argument");
    const jev_config &f = c->cfg;
    if (length < 0) return fail(JEV_EINVAL, "negative length");
    size_t per = (size_t)f.n_layers * f.n_kv_heads * length * f.head_dim;
    if (n != per * 2) return fail(JEV_EINVAL, "Snapshot holds %zu floats; %d positions need %zu.", n, length, per * 2);
    HIP_TRY(hipSetDevice(c->device));
    int rc = kv_ensure(c, length);
    if (rc) return rc;
    rc = kv_flat_copy(c, length, const_cast<float *>(in), false, hipMemcpyHostToDevice);
    if (rc) return rc;
    return kv_finish_restore(c, length);
}

// A snapshot kept in HBM: the same flat layout as jev_kv_snapshot's output.
struct jev_snapshot {
    int device = 0;
    int32_t layers = 0, kv_heads = 0, head_dim = 0, length = 0;
    float *data = nullptr; // keys then values, KvCache.Snapshot order
    size_t floats = 0;
};

int jev_kv_snapshot_device(jev_ctx *c, int32_t length, jev_snapshot **out)
{
    if (!c || !out) return fail(JEV_EINVAL, "null argument");
    *out = nullptr;
    if (length < 0 || length > c->len) return fail(JEV_EINVAL, "Only %d positions are cached.", c->len);
    const jev_config &f = c->cfg;
    HIP_TRY(hipSetDevice(c->device));
    jev_snapshot *sn = new jev_snapshot;
    sn->device = c->device;
    sn->layers = f.n_layers;
    sn->kv_heads = f.n_kv_heads;
    sn->head_dim = f.head_dim;
    sn->length = length;
    sn->floats = 2 * (size_t)f.n_layers * f.n_kv_heads * length * f.head_dim;
    hipError_t e = hipMalloc((void **)&sn->data, std::max<size_t>(sn->floats, 1) * sizeof(float));
    if (e != hipSuccess) {
        const size_t bytes = sn->floats * sizeof(float);
        delete sn;
        return fail(JEV_ENOMEM, "device snapshot of %d positions (%zu bytes): %s", length, bytes, hipGetErrorString(e));
    }
    int rc = kv_flat_copy(c, length, sn->data, true, hipMemcpyDeviceToDevice);
    if (!rc && (e = hipStreamSynchronize(c->stream)) != hipSuccess) rc = fail(JEV_EDEVICE, "snapshot: %s", hipGetErrorString(e));
    if (rc) {
        jev_snapshot_destroy(sn);
        return rc;
    }
    *out = sn;
    return JEV_OK;
}

int jev_kv_restore_device(jev_ctx *c, const jev_snapshot *sn)
{
    if (!c || !sn) return fail(JEV_EINVAL, "null argument");
    const jev_config &f = c->cfg;
    if (sn->layers != f.n_layers || sn->kv_heads != f.n_kv_heads || sn->head_dim != f.head_dim)
        return fail(JEV_EINVAL, "The snapshot was taken for %d layers x %d KV heads x %d; this model has %d x %d x %d.",
                    sn->layers, sn->kv_heads, sn->head_dim, f.n_layers, f.n_kv_heads, f.head_dim);
    if (sn->device != c->device) return fail(JEV_EINVAL, "the snapshot lives on device %d, the model on %d", sn->device, c->device);
    HIP_TRY(hipSetDevice(c->device));
    int rc = kv_ensure(c, sn->length);
    if (rc) return rc;
    rc = kv_flat_copy(c, sn->length, sn->data, false, hipMemcpyDeviceToDevice);
    if (rc) return rc;
    return kv_finish_restore(c, sn->length);
}

int jev_snapshot_length(const jev_snapshot *sn, int32_t *length)
{
    if (!sn || !length) return fail(JEV_EINVAL, "null argument");
    *length = sn->length;
    return JEV_OK;
}

int jev_snapshot_read(const jev_snapshot *sn, float *out, size_t n)
{
    if (!sn || !out) return fail(JEV_EINVAL, "null argument");
    if (n != sn->floats) return fail(JEV_EINVAL, "Snapshot needs %zu floats; got %zu.", sn->floats, n);
    HIP_TRY(hipSetDevice(sn->device));
    if (n) HIP_TRY(hipMemcpy(out, sn->data, n * sizeof(float), hipMemcpyDeviceToHost));
    return JEV_OK;
}

void jev_snapshot_destroy(jev_snapshot *sn)
{
    if (!sn) return;
    (void)hipSetDevice(sn->device);
    if (sn->data) (void)hipFree(sn->data);
    delete sn;
}

int jev_forward(jev_ctx *c, const int32_t *tokens, int32_t T, const jev_layout *layout, int mode,
                const int32_t *rows, int32_t n_rows, float *out, size_t out_len)
{
    int rc = check_ready(c);
    if (rc) return rc;
    CallScope call(c);
    Plan p;
    rc = prepare(c, tokens, false, T, layout, mode, rows, n_rows, p);
    if (rc) return rc;
    size_t need = out_floats(c, mode, p.n_out, n_rows);
    if (need && (!out || out_len < need)) return fail(JEV_EINVAL, "Expected room for %zu outputs, got %zu.", need, out_len);
    float *dout = nullptr;
    if (need) {
        HIP_TRY(c->logits.ensure(std::max(c->logits.n, need)));
        dout = c->logits.p;
    }
    rc = enqueue_forward(c, p, mode, n_rows, dout, nullptr, &call, true);
    if (rc) {
        (void)hipStreamSynchronize(c->stream);
        return rc;
    }
    rc = copy_out(c, out, dout, need);
    if (rc) return rc;
    // a cancel that landed after the last layer was enqueued still cancels
    // this call: the cache length stays where it was (KvCache.Advance is skipped)
    if (call.cancelled()) return fail(JEV_ECANCELED, "the forward pass was cancelled");
    c->len = std::max(c->len, p.end); // KvCache.Advance (MinistralModel.cs:360)
    return JEV_OK;
}

int jev_capture(jev_ctx *c, const int32_t *tokens, int32_t T, jev_sink sink, void *user, float *logits,
                size_t out_len)
{
    int rc = check_ready(c);
    if (rc) return rc;
    if (!sink) return fail(JEV_EINVAL, "sink is null");
    if (!logits || out_len < (size_t)c->cfg.vocab)
        return fail(JEV_EINVAL, "Expected room for %d logits, got %zu.", c->cfg.vocab, out_len);
    CallScope call(c);
    Plan p;
    rc = prepare(c, tokens, false, T, nullptr, JEV_OUT_LAST_FULL, nullptr, 0, p);
    if (rc) return rc;
    HIP_TRY(c->cap32.ensure((size_t)T * std::max(c->cfg.hidden, c->qdim())));
    HIP_TRY(c->logits.ensure(std::max(c->logits.n, (size_t)c->cfg.vocab)));
    Capture cap;
    rc = enqueue_forward(c, p, JEV_OUT_LAST_FULL, 0, c->logits.p, nullptr, &call, false, &cap);
    if (rc) {
        (void)hipStreamSynchronize(c->stream);
        return rc;
    }
    rc = copy_out(c, logits, c->logits.p, (size_t)c->cfg.vocab);
    if (rc) return rc;
    if (call.cancelled()) return fail(JEV_ECANCELED, "the forward pass was cancelled");
    c->len = std::max(c->len, p.end); // KvCache.Advance (MinistralModel.cs:360)
    for (const Capture::Tap &t : cap.taps) sink(user, t.name.c_str(), t.v.data(), t.rows, t.cols);
    return JEV_OK;
}

int jev_forward_device(jev_ctx *c, const int32_t *d_tokens, int32_t T, const jev_layout *layout, int mode,
                       const int32_t *rows, int32_t n_rows, float *d_out)
{
    int rc = check_ready(c);
    if (rc) return rc;
    CallScope call(c);
    Plan p;
    rc = prepare(c, d_tokens, true, T, layout, mode, rows, n_rows, p);
    if (rc) return rc;
    if (out_floats(c, mode, p.n_out, n_rows) && !d_out) return fail(JEV_EINVAL, "d_out is null");
    rc = enqueue_forward(c, p, mode, n_rows, d_out, nullptr, &call, false);
    if (rc) return rc;
    c->len = std::max(c->len, p.end);
    return JEV_OK;
}

int jev_sync(jev_ctx *c)
{
    if (!c) return fail(JEV_EINVAL, "null context");
    HIP_TRY(hipStreamSynchronize(c->stream));
    return JEV_OK;
}

void *jev_stream(jev_ctx *c) { return c ? (void *)c->stream : nullptr; }

// ForwardTreeAsync (MinistralModel.cs:198-219) with TokenLayout.Tree (:720-745).
int jev_forward_tree(jev_ctx *c, const int32_t *trunk, int32_t n_trunk, const int32_t *btok, const int32_t *blen,
                     int32_t nb, const int32_t *rows, int32_t n_rows, float *out, size_t out_len)
{
    if (!c) return fail(JEV_EINVAL, "null context");
    if (nb <= 0 || !blen || !btok) return fail(JEV_EINVAL, "No branches to forward.");
    if (n_trunk < 0 || (n_trunk > 0 && !trunk)) return fail(JEV_EINVAL, "bad trunk");
    std::vector<int32_t> offsets(nb);
    int total = n_trunk;
    for (int b = 0; b < nb; b++) {
        if (blen[b] <= 0) return fail(JEV_EINVAL, "Branch %d is empty.", b);
        offsets[b] = total;
        total += blen[b];
    }
    std::vector<int32_t> tokens(total), slot(total), pos(total), lo(total, 0), sh(total), seg(total), outs(nb);
    std::copy(trunk, trunk + n_trunk, tokens.begin());
    std::copy(btok, btok + (total - n_trunk), tokens.begin() + n_trunk);
    int start = c->len, branch = -1;
    for (int t = 0; t < total; t++) {
        slot[t] = start + t;
        while (branch + 1 < nb && t >= offsets[branch + 1]) branch++;
        if (t < n_trunk || branch < 0) {
            pos[t] = start + t;
            sh[t] = start;
            seg[t] = start;
        } else {
            pos[t] = start + n_trunk + (t - offsets[branch]);
            sh[t] = start + n_trunk;
            seg[t] = start + offsets[branch];
        }
    }
    for (int b = 0; b < nb; b++) outs[b] = (b + 1 < nb ? offsets[b + 1] : total) - 1;
    jev_layout L{slot.data(), pos.data(), lo.data(), sh.data(), seg.data(), outs.data(), nb, start + total};
    return jev_forward(c, tokens.data(), total, &L, JEV_OUT_SELECTED, rows, n_rows, out, out_len);
}

int jev_decode_greedy(jev_ctx *c, int32_t first, int32_t n_steps, int32_t *tokens_out, size_t tokens_out_len)
{
    // the destination is checked before anything else, as the reference
    // checks its spans on entry (MinistralModel.cs:306)
    if (n_steps <= 0 || !tokens_out) return fail(JEV_EINVAL, "bad arguments");
    if (tokens_out_len < (size_t)n_steps)
        return fail(JEV_EINVAL, "tokens_out holds %zu ids; %d steps need %d.", tokens_out_len, n_steps, n_steps);
    int rc = check_ready(c);
    if (rc) return rc;
    if (first < 0 || first >= c->embd.rows) return fail(JEV_EINVAL, "Token id %d is outside the embedding table.", first);
    CallScope call(c);
    // Every step is the same launch sequence: the token, the cache length and
    // the output index live in device memory (state = {length, step, token})
    // and the argmax kernel advances them.  The step is captured once as a
    // HIP graph and replayed; with the per-kernel profiler on it is launched
    // directly instead so every kernel is timed.
    const int start = c->len, end = start + n_steps;
    rc = kv_ensure(c, end);
    if (rc) return rc;
    HIP_TRY(c->dec_state.ensure((size_t)n_steps + 3));
    int32_t *state = c->dec_state.p, *out = c->dec_state.p + 3;
    const int32_t init[3] = {start, 0, first};
    HIP_TRY(hipMemcpy(state, init, sizeof(init), hipMemcpyHostToDevice));
    Plan p;
    rc = prepare(c, state + 2, true, 1, nullptr, JEV_OUT_LAST_FULL, nullptr, 0, p);
    if (rc) return rc;
    p.max_chunks = (end + kDecodeKeys - 1) / kDecodeKeys; // grid for the longest step; shorter ones exit early
    rc = ensure_workspace(c, 1, p.n_out, JEV_OUT_LAST_FULL, p.max_chunks);
    if (!rc && c->logits.ensure(std::max(c->logits.n, (size_t)c->cfg.vocab)) != hipSuccess) rc = fail(JEV_ENOMEM, "logits");
    if (rc) return rc;
    auto step = [&]() -> int {
        int r = enqueue_forward(c, p, JEV_OUT_LAST_FULL, 0, c->logits.p, state);
        if (r) return r;
        hipError_t e = launch_argmax_decode(c->logits.p, c->cfg.vocab, c->amax_v.p, c->amax_i.p, state, out, c->stream);
        return e == hipSuccess ? JEV_OK : fail(JEV_EDEVICE, "argmax: %s", hipGetErrorString(e));
    };
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    if (!c->profiling) {
        HIP_TRY(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
        c->capturing = true;
        rc = step();
        c->capturing = false;
        hipError_t e = hipStreamEndCapture(c->stream, &graph);
        if (!rc && e != hipSuccess) rc = fail(JEV_EDEVICE, "graph capture: %s", hipGetErrorString(e));
        if (!rc && (e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0)) != hipSuccess)
            rc = fail(JEV_EDEVICE, "graph instantiate: %s", hipGetErrorString(e));
    }
    // Steps are enqueued at most kLeadLayers ahead of the device (one event
    // per step), so a cancel stops the loop within that many steps.
    const bool stamps = c->step_stamps && !c->profiling;
    if (!rc && stamps) rc = step_events(c, n_steps);
    if (!rc && stamps) {
        hipError_t e = hipEventRecord(c->step_ev[0], c->stream);
        if (e != hipSuccess) rc = fail(JEV_EDEVICE, "decode: %s", hipGetErrorString(e));
    }
    int launched = 0;
    while (!rc && launched < n_steps) {
        if (launched >= jev_ctx::kLeadLayers) {
            hipError_t e = hipEventSynchronize(c->layer_ev[(launched - jev_ctx::kLeadLayers) % jev_ctx::kLayerEvents]);
            if (e != hipSuccess) {
                rc = fail(JEV_EDEVICE, "decode: %s", hipGetErrorString(e));
                break;
            }
        }
        if (call.cancelled()) {
            rc = fail(JEV_ECANCELED, "greedy decoding was cancelled after %d steps", launched);
            break;
        }
        if (exec) {
            hipError_t e = hipGraphLaunch(exec, c->stream);
            if (e != hipSuccess) {
                rc = fail(JEV_EDEVICE, "graph launch: %s", hipGetErrorString(e));
                break;
            }
        } else {
            rc = step();
            if (rc) break;
        }
        launched++;
        hipError_t e = hipEventRecord(c->layer_ev[(launched - 1) % jev_ctx::kLayerEvents], c->stream);
        if (e == hipSuccess && stamps) e = hipEventRecord(c->step_ev[launched], c->stream);
        if (e != hipSuccess) rc = fail(JEV_EDEVICE, "decode: %s", hipGetErrorString(e));
    }
    hipError_t e = hipStreamSynchronize(c->stream);
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (!rc && e != hipSuccess) rc = fail(JEV_EDEVICE, "decode: %s", hipGetErrorString(e));
    if (!rc && stamps) read_step_times(c, launched);
    if (!rc && call.cancelled()) rc = fail(JEV_ECANCELED, "greedy decoding was cancelled after %d steps", launched);
    // every launched step ran to the end and advanced the cache by one token
    if (!rc || rc == JEV_ECANCELED) c->len = std::max(c->len, start + launched);
    if (!rc) {
        e = hipMemcpy(tokens_out, out, sizeof(int32_t) * n_steps, hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = fail(JEV_EDEVICE, "decode: %s", hipGetErrorString(e));
    }
    return rc;
}

// ReasoningDecider's batched greedy loop (ReasoningDecider.cs:157-178 through
// ForwardRowsAsync, MinistralModel.cs:272-294): the rows-layout step captured
// as a HIP graph and replayed.  The per-row tokens, slots and positions live
// in the plan's device buffers and rows_step_kernel advances them, so nothing
// returns to the host between steps.
int jev_decode_rows_greedy(jev_ctx *c, int32_t shared, int32_t n_rows, const int32_t *row_base,
                           const int32_t *row_length, const int32_t *first, int32_t n_steps, int32_t *tokens_out,
                           size_t tokens_out_len)
{
    if (n_rows <= 0 || n_steps <= 0 || shared < 0 || !row_base || !row_length || !first || !tokens_out)
        return fail(JEV_EINVAL, "bad arguments");
    if (tokens_out_len < (size_t)n_steps * (size_t)n_rows)
        return fail(JEV_EINVAL, "tokens_out holds %zu ids; %d steps of %d rows need %zu.", tokens_out_len, n_steps,
                    n_rows, (size_t)n_steps * (size_t)n_rows);
    int rc = check_ready(c);
    if (rc) return rc;
    // every row's slots over the whole run, [base, base + length + steps),
    // clear of the shared prefix and of each other
    std::vector<std::pair<int64_t, int64_t>> span(n_rows);
    int64_t end_max = shared;
    for (int r = 0; r < n_rows; r++) {
        if (row_length[r] < 0 || row_base[r] < 0) return fail(JEV_EINVAL, "row %d: negative base or length", r);
        if (first[r] < 0 || first[r] >= c->embd.rows)
            return fail(JEV_EINVAL, "Token id %d is outside the %d-entry embedding table.", first[r], c->embd.rows);
        span[r] = {row_base[r], (int64_t)row_base[r] + row_length[r] + n_steps};
        end_max = std::max(end_max, span[r].second);
        if (span[r].first < shared) return fail(JEV_EINVAL, "row %d starts at slot %d, inside the %d shared slots", r, row_base[r], shared);
    }
    if (end_max > (1 << 28)) return fail(JEV_EINVAL, "the rows reach slot %lld", (long long)end_max);
    {
        std::vector<std::pair<int64_t, int64_t>> sorted = span;
        std::sort(sorted.begin(), sorted.end());
        for (int r = 1; r < n_rows; r++)
            if (sorted[r].first < sorted[r - 1].second)
                return fail(JEV_EINVAL, "two rows' slots overlap within %d steps", n_steps);
    }
    CallScope call(c);
    std::vector<int32_t> slot(n_rows), pos(n_rows), lo(n_rows, 0), hi(n_rows, shared), seg(n_rows), outs(n_rows);
    int32_t end0 = shared;
    for (int r = 0; r < n_rows; r++) {
        slot[r] = row_base[r] + row_length[r];
        pos[r] = shared + row_length[r];
        seg[r] = row_base[r];
        outs[r] = r;
        end0 = std::max(end0, slot[r] + 1);
    }
    jev_layout lay{slot.data(), pos.data(), lo.data(), hi.data(), seg.data(), outs.data(), n_rows, end0};
    rc = kv_ensure(c, (int)end_max);
    if (rc) return rc;
    Plan p;
    rc = prepare(c, first, false, n_rows, &lay, JEV_OUT_FULL, nullptr, 0, p);
    if (rc) return rc;
    int max_limit = 0;
    for (int r = 0; r < n_rows; r++) max_limit = std::max(max_limit, shared + row_length[r] + n_steps);
    p.max_chunks = (max_limit + kDecodeKeys - 1) / kDecodeKeys; // grid for the longest step
    rc = ensure_workspace(c, n_rows, p.n_out, JEV_OUT_FULL, p.max_chunks, p.single_rows);
    if (rc) return rc;
    HIP_TRY(c->logits.ensure(std::max(c->logits.n, (size_t)n_rows * c->cfg.vocab)));
    HIP_TRY(c->dec_state.ensure((size_t)n_rows * (n_steps + 1)));
    int32_t *rowstep = c->dec_state.p, *out = c->dec_state.p + n_rows;
    HIP_TRY(hipMemsetAsync(rowstep, 0, (size_t)n_rows * sizeof(int32_t), c->stream));
    // two or more rows: every row is its own attention tile (the rows' slots
    // never meet), so the step takes the decode attention per token, whose
    // layout arrays rows_step_kernel advances; no attention tile is replayed
    if (n_rows >= 2 && !p.single_rows) return fail(JEV_EINVAL, "the rows do not form one-token attention tiles");
    auto step = [&]() -> int {
        int r = enqueue_forward(c, p, JEV_OUT_FULL, 0, c->logits.p);
        if (r) return r;
        hipError_t e = launch_rows_step(c->logits.p, c->cfg.vocab, n_rows, const_cast<int32_t *>(p.d_tokens),
                                        const_cast<int32_t *>(p.d_slot), const_cast<int32_t *>(p.d_pos), rowstep, out,
                                        c->stream);
        return e == hipSuccess ? JEV_OK : fail(JEV_EDEVICE, "rows step: %s", hipGetErrorString(e));
    };
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    if (!c->profiling) {
        HIP_TRY(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
        c->capturing = true;
        rc = step();
        c->capturing = false;
        hipError_t e = hipStreamEndCapture(c->stream, &graph);
        if (!rc && e != hipSuccess) rc = fail(JEV_EDEVICE, "graph capture: %s", hipGetErrorString(e));
        if (!rc && (e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0)) != hipSuccess)
            rc = fail(JEV_EDEVICE, "graph instantiate: %s", hipGetErrorString(e));
    }
    const bool stamps = c->step_stamps && !c->profiling;
    if (!rc && stamps) rc = step_events(c, n_steps);
    if (!rc && stamps) {
        hipError_t e = hipEventRecord(c->step_ev[0], c->stream);
        if (e != hipSuccess) rc = fail(JEV_EDEVICE, "rows decode: %s", hipGetErrorString(e));
    }
    int launched = 0;
    while (!rc && launched < n_steps) {
        if (launched >= jev_ctx::kLeadLayers) {
            hipError_t e = hipEventSynchronize(c->layer_ev[(launched - jev_ctx::kLeadLayers) % jev_ctx::kLayerEvents]);
            if (e != hipSuccess) {
                rc = fail(JEV_EDEVICE, "rows decode: %s", hipGetErrorString(e));
                break;
            }
        }
        if (call.cancelled()) {
            rc = fail(JEV_ECANCELED, "rows decoding was cancelled after %d steps", launched);
            break;
        }
        if (exec) {
            hipError_t e = hipGraphLaunch(exec, c->stream);
            if (e != hipSuccess) {
                rc = fail(JEV_EDEVICE, "graph launch: %s", hipGetErrorString(e));
                break;
            }
        } else {
            rc = step();
            if (rc) break;
        }
        launched++;
        hipError_t e = hipEventRecord(c->layer_ev[(launched - 1) % jev_ctx::kLayerEvents], c->stream);
        if (e == hipSuccess && stamps) e = hipEventRecord(c->step_ev[launched], c->stream);
        if (e != hipSuccess) rc = fail(JEV_EDEVICE, "rows decode: %s", hipGetErrorString(e));
    }
    hipError_t e = hipStreamSynchronize(c->stream);
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (!rc && e != hipSuccess) rc = fail(JEV_EDEVICE, "rows decode: %s", hipGetErrorString(e));
    if (!rc && stamps) read_step_times(c, launched);
    if (!rc && call.cancelled()) rc = fail(JEV_ECANCELED, "rows decoding was cancelled after %d steps", launched);
    if (!rc || rc == JEV_ECANCELED) {
        int32_t end = shared; // KvCache.Advance to the highest slot written
        for (int r = 0; r < n_rows; r++) end = std::max(end, row_base[r] + row_length[r] + launched);
        if (launched > 0) c->len = std::max(c->len, end);
    }
    if (!rc) {
        e = hipMemcpy(tokens_out, out, sizeof(int32_t) * (size_t)n_steps * n_rows, hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = fail(JEV_EDEVICE, "rows decode: %s", hipGetErrorString(e));
    }
    return rc;
}

int jev_margins(const float *v, int32_t n_options, int32_t n_yes, int32_t n_no, float temperature, float *margins,
                float *probs)
{
    if (!v || !margins || !probs || n_options <= 0 || n_yes <= 0 || n_no <= 0)
        return fail(JEV_EINVAL, "bad arguments");
    int nr = n_yes + n_no;
    for (int i = 0; i < n_options; i++) {
        const float *r = v + (size_t)i * nr;
        float by = r[0], bn = r[n_yes];
        for (int j = 1; j < n_yes; j++) by = std::max(by, r[j]);
        for (int j = 1; j < n_no; j++) bn = std::max(bn, r[n_yes + j]);
        margins[i] = by - bn;
        probs[i] = margins[i] / temperature;
    }
    // Kernels.Softmax (Kernels.cs:102-121)
    float mx = probs[0];
    for (int i = 1; i < n_options; i++) mx = std::max(mx, probs[i]);
    if (!std::isfinite(mx)) {
        for (int i = 0; i < n_options; i++) probs[i] = 1.0f / (float)n_options;
        return JEV_OK;
    }
    float sum = 0.f;
    for (int i = 0; i < n_options; i++) {
        probs[i] = expf(probs[i] - mx);
        sum += probs[i];
    }
    for (int i = 0; i < n_options; i++) probs[i] = probs[i] / sum;
    return JEV_OK;
}

int jev_profile_enable(jev_ctx *c, int enable)
{
    if (!c) return fail(JEV_EINVAL, "null context");
    if (enable < 0 || enable > 2) return fail(JEV_EINVAL, "profiling mode %d is not 0, 1 or 2", enable);
    HIP_TRY(hipStreamSynchronize(c->stream));
    c->prof.clear();
    c->ev_used = 0;
    c->profiling = enable == 1;
    c->step_stamps = enable == 2;
    c->step_ms.clear();
    return JEV_OK;
}

int jev_profile_steps(jev_ctx *c, float *ms, int32_t n, int32_t *n_steps)
{
    if (!c || !n_steps || n < 0 || (n > 0 && !ms)) return fail(JEV_EINVAL, "bad arguments");
    *n_steps = (int32_t)c->step_ms.size();
    std::copy_n(c->step_ms.begin(), std::min<size_t>((size_t)n, c->step_ms.size()), ms);
    return JEV_OK;
}

int jev_profile_read(jev_ctx *c, int cls, int64_t *launches, double *total_ms, double *flops, double *bytes)
{
    if (!c || cls < 0 || cls >= JEV_PROF_CLASSES) return fail(JEV_EINVAL, "bad arguments");
    HIP_TRY(hipStreamSynchronize(c->stream));
    int64_t n = 0;
    double ms = 0, fl = 0, by = 0;
    for (auto &r : c->prof) {
        if (r.cls != cls || !r.a || !r.b) continue;
        float e = 0.f;
        HIP_TRY(hipEventElapsedTime(&e, r.a, r.b));
        n++;
        ms += e;
        fl += r.flops;
        by += r.bytes;
    }
    if (launches) *launches = n;
    if (total_ms) *total_ms = ms;
    if (flops) *flops = fl;
    if (bytes) *bytes = by;
    return JEV_OK;
}

void jev_cancel(jev_ctx *c)
{
    if (!c) return;
    const uint64_t a = c->active.load();
    if (a) c->cancel_id.store(a); // aimed at the call in flight; none in flight: nothing to cancel
}

// ---------------------------------------------------------------- test hooks

int jev_set_matmul_strategy(int strategy)
{
    if (strategy != JEV_MATMUL_AUTO && strategy != JEV_MATMUL_FLOAT && strategy != JEV_MATMUL_INTEGER)
        return fail(JEV_EINVAL, "unknown matmul strategy %d", strategy);
    g_matmul_strategy.store(strategy);
    return JEV_OK;
}

int jev_get_matmul_strategy(void) { return g_matmul_strategy.load(); }

int jev_quantize_activations(const float *x, int64_t count, void *out, size_t out_bytes, float *block_sums)
{
    if (!x || !out || count <= 0 || count % 32 != 0) return fail(JEV_EINVAL, "count must be a positive multiple of 32");
    if (count > (int64_t)1 << 30) return fail(JEV_EINVAL, "count too large");
    const int64_t nb = count / 32;
    if (out_bytes < (size_t)nb * 34) return fail(JEV_EINVAL, "output holds %zu bytes, %lld needed", out_bytes,
                                                 (long long)(nb * 34));
    // one token of `count` values: the operand tiles hold it in row 0 of a 16-row group
    float *dx = nullptr, *dd = nullptr, *ds = nullptr;
    int8_t *dq = nullptr;
    int *dqs = nullptr;
    hipError_t e = hipMalloc((void **)&dx, (size_t)count * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&dq, (size_t)count * 16);
    if (e == hipSuccess) e = hipMalloc((void **)&dd, (size_t)nb * 16 * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&ds, (size_t)nb * 16 * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&dqs, (size_t)nb * 16 * sizeof(int));
    if (e == hipSuccess) e = hipMemcpy(dx, x, (size_t)count * sizeof(float), hipMemcpyHostToDevice);
    std::vector<int8_t> q((size_t)count * 16);
    std::vector<float> d((size_t)nb * 16), sums((size_t)nb * 16);
    if (e == hipSuccess) {
        QuantActArgs a;
        a.x = dx;
        a.T = 1;
        a.K = (int)count;
        a.T16 = 16;
        a.xq = dq;
        a.xd = dd;
        a.xqs = dqs;
        a.xs = ds;
        e = launch_quant_act(a, nullptr);
    }
    if (e == hipSuccess) e = hipMemcpy(q.data(), dq, q.size(), hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(d.data(), dd, d.size() * sizeof(float), hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(sums.data(), ds, sums.size() * sizeof(float), hipMemcpyDeviceToHost);
    for (void *p : {(void *)dx, (void *)dq, (void *)dd, (void *)ds, (void *)dqs})
        if (p) (void)hipFree(p);
    if (e != hipSuccess) return fail(JEV_EDEVICE, "quantize activations: %s", hipGetErrorString(e));
    // reassemble GGUF Q8_0 blocks: Half scale, then the 32 quants of token 0
    uint8_t *o = (uint8_t *)out;
    for (int64_t b = 0; b < nb; b++) {
        const uint16_t h = float_to_half(d[(size_t)b * 16]); // exact: the value is a Half already
        o[34 * b] = (uint8_t)(h & 0xff);
        o[34 * b + 1] = (uint8_t)(h >> 8);
        for (int i = 0; i < 32; i++) {
            const int k = (int)(32 * b + i), kk = k & 31;
            o[34 * b + 2 + i] = (uint8_t)q[(((size_t)b * 64) + (kk >> 3) * 16) * 8 + (kk & 7)];
        }
        if (block_sums) block_sums[b] = sums[(size_t)b * 16];
    }
    return JEV_OK;
}

int jev_rope_table(const jev_config *cfg, float *freqs, int32_t n, float *mscale)
{
    if (!cfg || !freqs || !mscale) return fail(JEV_EINVAL, "null argument");
    if (cfg->rope_dim <= 0 || cfg->rope_dim % 2 != 0) return fail(JEV_EINVAL, "rope_dim %d must be even and positive", cfg->rope_dim);
    if (n != cfg->rope_dim / 2) return fail(JEV_EINVAL, "the table has %d entries; %d given", cfg->rope_dim / 2, n);
    std::vector<float> f;
    float m = 1.f;
    rope_table(*cfg, f, m);
    std::copy(f.begin(), f.end(), freqs);
    *mscale = m;
    return JEV_OK;
}

int jev_dequantize(int type, const void *src, size_t nbytes, float *dst, int64_t count)
{
    if (!src || !dst || count <= 0) return fail(JEV_EINVAL, "bad arguments");
    if (!is_quant(type)) return fail(JEV_EINVAL, "type %d is not a block type", type);
    if (count % 32 != 0) return fail(JEV_EINVAL, "%d decodes whole blocks of 32; asked for %lld elements.", type, (long long)count);
    if ((int64_t)nbytes < row_bytes(type, count)) return fail(JEV_EINVAL, "need %lld bytes", (long long)row_bytes(type, count));
    QWeight w;
    int rc = upload_weight(type, 1, count, src, w);
    if (rc) return rc;
    float *d = nullptr;
    hipError_t e = hipMalloc((void **)&d, (size_t)count * sizeof(float));
    if (e == hipSuccess) e = launch_dequant(w, d, nullptr);
    if (e == hipSuccess) e = hipMemcpy(dst, d, (size_t)count * sizeof(float), hipMemcpyDeviceToHost);
    if (d) (void)hipFree(d);
    free_weight(w);
    if (e != hipSuccess) return fail(JEV_EDEVICE, "dequantize: %s", hipGetErrorString(e));
    return JEV_OK;
}

struct jev_weight {
    int device = 0;
    hipStream_t stream = nullptr;
    QWeight w;
    DevBuf<uint16_t> xt;
    DevBuf<float> xsum, part;
    DevBuf<int8_t> xq; // integer strategy: quantized activations and their block data
    DevBuf<float> xd, xs;
    DevBuf<int> xqs;
};

// Device buffers one matmul call works in (besides x and y).
struct MatmulBufs {
    uint16_t *xt = nullptr; // fp16 pair of x, operand-tile layout (tokens >= 2)
    float *xsum = nullptr;  // Q5_1: per-32 block sums of x
    float *part = nullptr;  // K-split partials (ksplit > 1)
    int8_t *xq = nullptr;   // integer strategy: quantized activations and their block data
    float *xd = nullptr, *xs = nullptr;
    int *xqs = nullptr;
};
// Bytes of each buffer a call of `tokens` rows needs, in MatmulBufs order.
struct MatmulNeeds {
    size_t xt = 0, xsum = 0, part = 0, xq = 0, xd = 0, xs = 0, xqs = 0;
    int ksplit = 1;
    bool fold = false; // the GEMM sums its K splits itself (gemm_fold): no partials buffer
    bool integer = false;
};
static MatmulNeeds matmul_needs(const QWeight &w, int tokens, bool integer)
{
    MatmulNeeds n;
    const size_t t16 = ((size_t)tokens + 15) & ~(size_t)15, nb = (size_t)w.cols / 32;
    n.integer = integer;
    if (integer) {
        n.xq = t16 * w.cols;
        n.xd = n.xs = n.xqs = nb * t16 * 4;
        return n;
    }
    n.ksplit = jev_ctx::split(tokens, w.rows, w.cols);
    n.fold = tokens >= 2 && gemm_fold(w.type, tokens, n.ksplit);
    if (n.ksplit > 1 && !n.fold) n.part = (size_t)tokens * w.rows * n.ksplit * sizeof(float);
    if (tokens >= 2) {
        n.xt = t16 * w.cols * 2 * sizeof(uint16_t);
        if (w.type == kQ5_1) n.xsum = ((size_t)tokens * nb + 1) * sizeof(float);
    }
    return n;
}

// The Integer strategy on the device: quantize x [tokens][cols] (fp32, device)
// to Q8_0 blocks, then the int8-MFMA block dots into y [tokens][rows].
static hipError_t matmul_integer(const QWeight &w, const float *x, int tokens, float *y, const MatmulBufs &b,
                                 hipStream_t s)
{
    const int t16 = (tokens + 15) & ~15;
    QuantActArgs q;
    q.x = x;
    q.T = tokens;
    q.K = w.cols;
    q.T16 = t16;
    q.xq = b.xq;
    q.xd = b.xd;
    q.xqs = b.xqs;
    q.xs = b.xs;
    hipError_t e = launch_quant_act(q, s);
    if (e != hipSuccess) return e;
    GemmI8Args g;
    g.w = w;
    g.xq = b.xq;
    g.xd = b.xd;
    g.xqs = b.xqs;
    g.xs = b.xs;
    g.T = tokens;
    g.T16 = t16;
    g.y = y;
    g.ldy = w.rows;
    return launch_gemm_i8(g, s);
}

// y = x . W^T on the device in the given buffers (QuantMatMul.ForwardAsync's
// dispatch, QuantMatMul.cs:84-101): the integer strategy, else the MFMA GEMM
// for two or more tokens and the GEMV for one, K-split partials summed after.
static hipError_t matmul_run(const QWeight &w, const float *x, int tokens, float *y, const MatmulNeeds &n,
                             const MatmulBufs &b, hipStream_t s)
{
    if (n.integer) return matmul_integer(w, x, tokens, y, b, s);
    const int rows = w.rows, cols = w.cols;
    const bool partials = n.ksplit > 1 && !n.fold;
    float *dst = partials ? b.part : y;
    hipError_t e = hipSuccess;
    if (tokens >= 2) {
        e = launch_split(x, tokens, cols, b.xt, s);
        if (e == hipSuccess && w.type == kQ5_1) e = launch_block_sums(b.xt, tokens, cols, b.xsum, s);
        if (e == hipSuccess) {
            GemmArgs g;
            g.M = tokens;
            g.K = cols;
            g.xt = b.xt;
            g.xsum = b.xsum;
            g.seg[0] = w;
            g.ldy = rows;
            g.y = dst;
            g.ksplit = n.ksplit;
            g.fold = n.fold ? 1 : 0;
            e = launch_gemm(g, s);
        }
    } else {
        GemvArgs g;
        g.K = cols;
        g.x = x;
        g.seg[0] = w;
        g.y = dst;
        g.ksplit = n.ksplit;
        e = launch_gemv(g, s);
    }
    if (e == hipSuccess && partials) e = launch_reduce_partials(dst, n.ksplit, tokens, rows, y, s);
    return e;
}

int jev_weight_create(int type, int64_t rows, int64_t cols, const void *bytes, size_t nbytes, int device,
                      jev_weight **out)
{
    if (!out) return fail(JEV_EINVAL, "out is null");
    *out = nullptr;
    if (!bytes || rows <= 0 || cols <= 0) return fail(JEV_EINVAL, "bad arguments");
    if (!is_quant(type) || cols % 32 != 0) return fail(JEV_EINVAL, "unsupported type %d or shape %lld x %lld", type,
                                                       (long long)rows, (long long)cols);
    if (nbytes < (size_t)row_bytes(type, cols) * (size_t)rows)
        return fail(JEV_EDATA, "%zu bytes are too few for a %lld x %lld tensor", nbytes, (long long)rows, (long long)cols);
    HIP_TRY(hipSetDevice(device));
    jev_weight *h = new jev_weight;
    h->device = device;
    hipError_t e = hipStreamCreate(&h->stream);
    if (e != hipSuccess) {
        delete h;
        return fail(JEV_EDEVICE, "stream: %s", hipGetErrorString(e));
    }
    int rc = upload_weight(type, rows, cols, bytes, h->w);
    if (rc) {
        (void)hipStreamDestroy(h->stream);
        delete h;
        return rc;
    }
    *out = h;
    return JEV_OK;
}

void jev_weight_destroy(jev_weight *h)
{
    if (!h) return;
    (void)hipSetDevice(h->device);
    (void)hipStreamSynchronize(h->stream);
    free_weight(h->w);
    h->xt.release();
    h->xsum.release();
    h->part.release();
    h->xq.release();
    h->xd.release();
    h->xs.release();
    h->xqs.release();
    (void)hipStreamDestroy(h->stream);
    delete h;
}

int jev_matmul_device(jev_weight *h, const float *x, int32_t tokens, float *y)
{
    if (!h || !x || !y || tokens <= 0) return fail(JEV_EINVAL, "bad arguments");
    HIP_TRY(hipSetDevice(h->device));
    const MatmulNeeds n = matmul_needs(h->w, tokens, g_matmul_strategy.load() == JEV_MATMUL_INTEGER);
    MatmulBufs b;
    if (n.xt) HIP_TRY(h->xt.ensure(n.xt / sizeof(uint16_t)));
    if (n.xsum) HIP_TRY(h->xsum.ensure(n.xsum / sizeof(float)));
    if (n.part) HIP_TRY(h->part.ensure(n.part / sizeof(float)));
    if (n.xq) HIP_TRY(h->xq.ensure(n.xq));
    if (n.xd) HIP_TRY(h->xd.ensure(n.xd / sizeof(float)));
    if (n.xs) HIP_TRY(h->xs.ensure(n.xs / sizeof(float)));
    if (n.xqs) HIP_TRY(h->xqs.ensure(n.xqs / sizeof(int)));
    b.xt = h->xt.p;
    b.xsum = h->xsum.p;
    b.part = h->part.p;
    b.xq = h->xq.p;
    b.xd = h->xd.p;
    b.xs = h->xs.p;
    b.xqs = h->xqs.p;
    HIP_TRY(matmul_run(h->w, x, tokens, y, n, b, h->stream));
    return JEV_OK;
}

// ---- The same matmul without allocation (jev_matmul_device_noalloc).
//
// Its buffers (the fp16 pair of x, Q5_1 block sums, K-split partials, or the
// integer strategy's quantized activations) are carved from `scratch`, one
// static device array per GPU that lives until the process ends.  Host code
// never passes `scratch` itself to a kernel (that name is a host-side stand-in,
// not a device address): the device address comes from hipGetSymbolAddress,
// fetched once per device with that device current, and only that pointer is
// used.  Nothing in it has to start at zero: every element a call reads was
// written earlier in the same call (padding rows of the operand tiles feed
// only padding outputs, which are never stored).
} // extern "C"

static constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch_dev[kMaxDevices] = {};

// The device address of this device's `scratch` (the current device must be `device`).
int scratch_for(int device, uint8_t **out)
{
    if (device < 0 || device >= kMaxDevices) return fail(JEV_EINVAL, "device %d is out of range", device);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[device]) {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(JEV_EDEVICE, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
        g_scratch_dev[device] = (uint8_t *)p;
    }
    *out = g_scratch_dev[device];
    return JEV_OK;
}
} // namespace

extern "C" {

int jev_matmul_device_noalloc(jev_weight *h, const float *x, int32_t tokens, float *y)
{
    if (!h || !x || !y || tokens <= 0) return fail(JEV_EINVAL, "bad arguments");
    HIP_TRY(hipSetDevice(h->device));
    const MatmulNeeds n = matmul_needs(h->w, tokens, g_matmul_strategy.load() == JEV_MATMUL_INTEGER);
    // carve 256-byte aligned pieces in MatmulBufs order
    const size_t sizes[7] = {n.xt, n.xsum, n.part, n.xq, n.xd, n.xs, n.xqs};
    size_t off[7], total = 0;
    for (int i = 0; i < 7; i++) {
        off[i] = total;
        total += (sizes[i] + 255) & ~(size_t)255;
    }
    if (total > kNoAllocScratchBytes)
        return fail(JEV_EINVAL,
                    "a %d-token matmul over a %d x %d weight needs %zu bytes of scratch; the no-allocation entry point "
                    "has %zu (use jev_matmul_device)",
                    tokens, h->w.rows, h->w.cols, total, kNoAllocScratchBytes);
    uint8_t *base = nullptr;
    int rc = scratch_for(h->device, &base);
    if (rc) return rc;
    MatmulBufs b;
    b.xt = n.xt ? (uint16_t *)(base + off[0]) : nullptr;
    b.xsum = n.xsum ? (float *)(base + off[1]) : nullptr;
    b.part = n.part ? (float *)(base + off[2]) : nullptr;
    b.xq = n.xq ? (int8_t *)(base + off[3]) : nullptr;
    b.xd = n.xd ? (float *)(base + off[4]) : nullptr;
    b.xs = n.xs ? (float *)(base + off[5]) : nullptr;
    b.xqs = n.xqs ? (int *)(base + off[6]) : nullptr;
    HIP_TRY(matmul_run(h->w, x, tokens, y, n, b, h->stream));
    return JEV_OK;
}

void *jev_weight_stream(jev_weight *h) { return h ? (void *)h->stream : nullptr; }

int jev_weight_sync(jev_weight *h)
{
    if (!h) return fail(JEV_EINVAL, "null weight");
    hipError_t e = hipStreamSynchronize(h->stream);
    if (e != hipSuccess) return fail(JEV_EDEVICE, "matmul: %s", hipGetErrorString(e));
    return JEV_OK;
}

int jev_matmul_q(int type, const void *wbytes, int64_t rows, int64_t cols, const float *x, int32_t tokens, float *y)
{
    if (!wbytes || !x || !y || tokens <= 0 || rows <= 0 || cols <= 0) return fail(JEV_EINVAL, "bad arguments");
    if (!is_quant(type) || cols % 32 != 0) return fail(JEV_EINVAL, "unsupported type or shape");
    QWeight w;
    int rc = upload_weight(type, rows, cols, wbytes, w);
    if (rc) return rc;
    size_t nx = (size_t)tokens * cols, ny = (size_t)tokens * rows;
    float *dx = nullptr, *dy = nullptr, *dsum = nullptr;
    uint16_t *xt = nullptr;
    hipError_t e = hipMalloc((void **)&dx, nx * sizeof(float));
    const int ksplit = jev_ctx::split(tokens, (int)rows, (int)cols);
    if (e == hipSuccess) e = hipMalloc((void **)&dy, ny * ksplit * sizeof(float));
    if (e == hipSuccess) e = hipMemcpy(dx, x, nx * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess && g_matmul_strategy.load() == JEV_MATMUL_INTEGER) {
        const MatmulNeeds n = matmul_needs(w, tokens, true);
        DevBuf<int8_t> xq;
        DevBuf<float> xd, xs;
        DevBuf<int> xqs;
        e = xq.ensure(n.xq);
        if (e == hipSuccess) e = xd.ensure(n.xd / sizeof(float));
        if (e == hipSuccess) e = xs.ensure(n.xs / sizeof(float));
        if (e == hipSuccess) e = xqs.ensure(n.xqs / sizeof(int));
        MatmulBufs b;
        b.xq = xq.p;
        b.xd = xd.p;
        b.xs = xs.p;
        b.xqs = xqs.p;
        if (e == hipSuccess) e = matmul_integer(w, dx, tokens, dy, b, nullptr);
        if (e == hipSuccess) e = hipDeviceSynchronize();
        xq.release();
        xd.release();
        xs.release();
        xqs.release();
    } else if (e == hipSuccess && tokens >= 2) {
        size_t t16 = ((size_t)tokens + 15) & ~(size_t)15;
        e = hipMalloc((void **)&xt, t16 * cols * 2 * sizeof(uint16_t));
        if (e == hipSuccess) e = hipMalloc((void **)&dsum, (nx / 32 + 1) * sizeof(float));
        if (e == hipSuccess) e = launch_split(dx, tokens, (int)cols, xt, nullptr);
        if (e == hipSuccess && type == kQ5_1) e = launch_block_sums(xt, tokens, (int)cols, dsum, nullptr);
        if (e == hipSuccess) {
            GemmArgs g;
            g.M = tokens;
            g.K = (int)cols;
            g.xt = xt;
            g.xsum = dsum;
            g.seg[0] = w;
            g.ldy = (int)rows;
            g.y = dy;
            g.ksplit = ksplit;
            e = launch_gemm(g, nullptr);
            if (e == hipSuccess && ksplit > 1) e = launch_reduce_partials(dy, ksplit, tokens, (int)rows, dy, nullptr);
        }
    } else if (e == hipSuccess) {
        GemvArgs g;
        g.K = (int)cols;
        g.x = dx;
        g.seg[0] = w;
        g.y = dy;
        g.ksplit = ksplit;
        e = launch_gemv(g, nullptr);
        if (e == hipSuccess && ksplit > 1) e = launch_reduce_partials(dy, ksplit, 1, (int)rows, dy, nullptr);
    }
    if (e == hipSuccess) e = hipMemcpy(y, dy, ny * sizeof(float), hipMemcpyDeviceToHost);
    for (void *pp : {(void *)dx, (void *)dy, (void *)dsum, (void *)xt})
        if (pp) (void)hipFree(pp);
    free_weight(w);
    if (e != hipSuccess) return fail(JEV_EDEVICE, "matmul: %s", hipGetErrorString(e));
    return JEV_OK;
}

} // extern "C"
