/*
 * CPU oracle for the Jevstral token loop -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates the reference's managed Float path in plain C so the HIP library
 * can be checked against it.  Only tests/, the smoke check and the bench's
 * cpu_baseline leg load this library.  Arithmetic follows the reference
 * operation by operation; where the reference delegates to
 * System.Numerics.Tensors (TensorPrimitives.Dot/Sum/Exp, Vector.Sum), whose
 * reduction order is vector-width dependent and not pinned by its tests, a
 * fixed order is used and stated at the function.
 *
 * Build with -ffp-contract=off: every fused multiply-add below is an explicit
 * fmaf(), matching Vector512.FusedMultiplyAdd / MathF.FusedMultiplyAdd in the
 * reference; every other a*b+c is two roundings, as C# does not contract.
 */
#include "jev_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 0;
static int g_vector_bits = 0; /* 0: 512 when the host has AVX-512F, else 256 */

void orc_set_threads(int n) { g_threads = n; }
void orc_set_vector_bits(int bits) { g_vector_bits = bits; }
int orc_get_vector_bits(void)
{
#if defined(__x86_64__)
    if (g_vector_bits == 512 || g_vector_bits == 256) return g_vector_bits;
    return __builtin_cpu_supports("avx512f") ? 512 : 256;
#else
    return 256;
#endif
}
int orc_get_threads(void)
{
#ifdef _OPENMP
    return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------ geometry */

int orc_block_size(int type)
{
    switch (type) {
    case ORC_F32: case ORC_F16: return 1;
    case ORC_Q4_0: case ORC_Q5_1: case ORC_Q8_0: return 32;
    default: return 0;
    }
}

int orc_type_size(int type)
{
    switch (type) {
    case ORC_F32: return 4;
    case ORC_F16: return 2;
    case ORC_Q4_0: return 2 + 16;         /* d, 32 x 4 bit           GgmlType.cs:78 */
    case ORC_Q5_1: return 2 + 2 + 4 + 16; /* d, m, qh, 32 x 4 bit    GgmlType.cs:81 */
    case ORC_Q8_0: return 2 + 32;         /* d, 32 x 8 bit           GgmlType.cs:82 */
    default: return 0;
    }
}

int64_t orc_row_bytes(int type, int64_t cols)
{
    int bs = orc_block_size(type);
    if (bs == 0) return -1;
    return cols / bs * orc_type_size(type);
}

/* IEEE binary16 -> binary32, exact (what (float)Half does). */
static float h2f(uint16_t h)
{
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff, f;
    if (e == 0) {
        if (m == 0) {
            f = s;
        } else { /* subnormal: renormalise */
            int32_t ee = 127 - 15 + 1;
            while (!(m & 0x400)) { m <<= 1; ee--; }
            m &= 0x3ff;
            f = s | ((uint32_t)ee << 23) | (m << 13);
        }
    } else if (e == 31) {
        f = s | 0x7f800000u | (m << 13);
    } else {
        f = s | ((e - 15 + 127) << 23) | (m << 13);
    }
    float r;
    memcpy(&r, &f, 4);
    return r;
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }

/* ------------------------------------------------------------ dequant */

/* Dequantizer.Q4_0 (Dequantizer.cs:155-182): d * ((qs[j] & 15) - 8) for
 * element j, d * ((qs[j] >> 4) - 8) for element 16 + j.  One multiply. */
static void deq_q4_0(const uint8_t *src, float *dst, int64_t n)
{
    for (int64_t b = 0; b < n / 32; b++, src += 18, dst += 32) {
        float d = h2f(rd16(src));
        const uint8_t *qs = src + 2;
        for (int j = 0; j < 16; j++) {
            dst[j] = d * (float)((qs[j] & 0x0F) - 8);
            dst[16 + j] = d * (float)((qs[j] >> 4) - 8);
        }
    }
}

/* Dequantizer.Q5_1 (Dequantizer.cs:240-268): d * q + m with
 * q = nibble | ((qh >> j) & 1) << 4 (element j) and
 * q = (qs[j] >> 4) | ((qh >> (j + 16)) & 1) << 4 (element 16 + j).
 * d * q is exact in float, so the result rounds once at "+ m". */
static void deq_q5_1(const uint8_t *src, float *dst, int64_t n)
{
    for (int64_t b = 0; b < n / 32; b++, src += 24, dst += 32) {
        float d = h2f(rd16(src));
        float m = h2f(rd16(src + 2));
        uint32_t qh = rd32(src + 4);
        const uint8_t *qs = src + 8;
        for (int j = 0; j < 16; j++) {
            int lo = (qs[j] & 0x0F) | (int)(((qh >> j) & 1) << 4);
            int hi = (qs[j] >> 4) | (int)(((qh >> (j + 16)) & 1) << 4);
            float a = d * (float)lo;
            float c = d * (float)hi;
            dst[j] = a + m;
            dst[16 + j] = c + m;
        }
    }
}

/* Dequantizer.Q8_0 (Dequantizer.cs:270-305): q * d. */
static void deq_q8_0(const uint8_t *src, float *dst, int64_t n)
{
    for (int64_t b = 0; b < n / 32; b++, src += 34, dst += 32) {
        float d = h2f(rd16(src));
        const int8_t *qs = (const int8_t *)(src + 2);
        for (int j = 0; j < 32; j++) dst[j] = (float)qs[j] * d;
    }
}

int orc_dequantize(int type, const void *src, float *dst, int64_t count)
{
    int bs = orc_block_size(type);
    if (bs == 0 || count % bs != 0) return -1; /* Dequantizer.cs:47-50 */
    const uint8_t *s = (const uint8_t *)src;
    switch (type) {
    case ORC_F32: memcpy(dst, s, (size_t)count * 4); return 0;
    case ORC_F16: for (int64_t i = 0; i < count; i++) dst[i] = h2f(rd16(s + 2 * i)); return 0;
    case ORC_Q4_0: deq_q4_0(s, dst, count); return 0;
    case ORC_Q5_1: deq_q5_1(s, dst, count); return 0;
    case ORC_Q8_0: deq_q8_0(s, dst, count); return 0;
    default: return -1;
    }
}

/* ------------------------------------------------------------ dot / sums */

/* TensorPrimitives.Dot (used by Kernels.Dot, Kernels.cs:68, and the 1-token
 * row path, QuantMatMul.cs:167).  Its order is implementation-defined; the
 * oracle uses 16 lanes of fused chains (lane = i mod 16) summed in lane order,
 * then the scalar tail as a fused chain. */
float orc_dot(const float *a, const float *b, int n)
{
    float lane[16] = {0};
    int i = 0;
    for (; i + 16 <= n; i += 16)
        for (int j = 0; j < 16; j++) lane[j] = fmaf(a[i + j], b[i + j], lane[j]);
    float s = 0.f;
    for (int j = 0; j < 16; j++) s += lane[j];
    for (; i < n; i++) s = fmaf(a[i], b[i], s);
    return s;
}

/* TensorPrimitives.Sum (Kernels.cs:120) with the same lane scheme. */
static float sum_f(const float *a, int n)
{
    float lane[16] = {0};
    int i = 0;
    for (; i + 16 <= n; i += 16)
        for (int j = 0; j < 16; j++) lane[j] += a[i + j];
    float s = 0.f;
    for (int j = 0; j < 16; j++) s += lane[j];
    for (; i < n; i++) s += a[i];
    return s;
}

/* ------------------------------------------------------------ elementwise */

/* Kernels.RmsNorm (Kernels.cs:25-60).  Vector<float> is 8 lanes on x64 (the
 * JIT keeps it 256 bits wide even with AVX-512): two accumulators over
 * 16-element strides, each summed lane by lane (Vector.Sum's order is not
 * specified; lane order here), widened to double; the scalar tail in double;
 * scale = 1 / sqrt((float)(sum / n) + eps); y = (x * scale) * w. */
void orc_rmsnorm(const float *x, const float *w, float eps, int n, float *y)
{
    double sum = 0;
    int i = 0;
    const int width = 8;
    if (n >= 2 * width) {
        float even[8] = {0}, odd[8] = {0};
        for (; i + 2 * width <= n; i += 2 * width)
            for (int j = 0; j < width; j++) {
                float a = x[i + j], b = x[i + width + j];
                float aa = a * a, bb = b * b;
                even[j] = even[j] + aa;
                odd[j] = odd[j] + bb;
            }
        float se = 0.f, so = 0.f;
        for (int j = 0; j < width; j++) { se += even[j]; so += odd[j]; }
        sum = (double)se + (double)so;
    }
    for (; i < n; i++) sum += (double)x[i] * (double)x[i];
    float scale = 1.0f / sqrtf((float)(sum / n) + eps);
    for (i = 0; i < n; i++) {
        float v = x[i] * scale;
        y[i] = v * w[i];
    }
}

/* Kernels.Softmax (Kernels.cs:102-121): max-shifted; a row whose max is not
 * finite becomes uniform.  exp is libm's expf (TensorPrimitives.Exp is a
 * vectorised approximation; parity at tolerance). */
void orc_softmax(float *x, int n)
{
    if (n == 0) return;
    float mx = x[0];
    for (int i = 1; i < n; i++) if (x[i] > mx) mx = x[i];
    if (!isfinite(mx)) {
        for (int i = 0; i < n; i++) x[i] = 1.0f / (float)n;
        return;
    }
    for (int i = 0; i < n; i++) x[i] = expf(x[i] - mx);
    float s = sum_f(x, n);
    for (int i = 0; i < n; i++) x[i] = x[i] / s;
}

/* Kernels.SwiGlu (Kernels.cs:82-89): up <- gate*up; dst <- sigmoid(gate);
 * dst <- dst*up; sigmoid(v) = 1 / (1 + exp(-v)). */
void orc_swiglu(const float *gate, float *up, float *dst, int n)
{
    for (int i = 0; i < n; i++) {
        float gu = gate[i] * up[i];
        float e = expf(-gate[i]);
        float s = 1.0f / (1.0f + e);
        up[i] = gu;
        dst[i] = s * gu;
    }
}

/* ------------------------------------------------------------ matmul */

#define PANEL 64    /* PanelGemm.PanelWidth, PanelGemm.cs:36 */
#define KBLOCK 2048 /* PanelGemm.KBlock, PanelGemm.cs:43     */
#define ROWBLK 6    /* PanelGemm.RowBlock, PanelGemm.cs:45   */

static int panel_supports(int type, int rows, int cols)
{
    int bs = orc_block_size(type);
    /* PanelGemm.Supports, PanelGemm.cs:68-70 */
    return rows % PANEL == 0 && cols % bs == 0 && (cols <= KBLOCK || KBLOCK % bs == 0);
}

/* PanelGemm's 512-bit tiles (Tile512x6 / Tile512x1, PanelGemm.cs:245-318):
 * the 64 outputs of a panel as four 16-float vectors per token, six tokens at
 * a time in 24 accumulator registers.  Every output is the same fused chain
 * over k ascending as the portable loops below (the 256-bit path), so both
 * give the same bits; PanelGemm picks 512 bits when the JIT accelerates them
 * (VectorBits, :50-63), and so does the oracle (orc_get_vector_bits). */
#if defined(__x86_64__)
#include <immintrin.h>
__attribute__((target("avx512f"))) static void tile6_512(const float *x, int64_t ldx, const float *p, int kc,
                                                         float *y, int64_t ldy, int acc)
{
    __m512 c[ROWBLK][4];
    for (int i = 0; i < ROWBLK; i++)
        for (int j = 0; j < 4; j++) c[i][j] = acc ? _mm512_loadu_ps(y + i * ldy + 16 * j) : _mm512_setzero_ps();
    for (int k = 0; k < kc; k++) {
        const float *w = p + (int64_t)k * PANEL;
        const __m512 b0 = _mm512_loadu_ps(w), b1 = _mm512_loadu_ps(w + 16), b2 = _mm512_loadu_ps(w + 32),
                     b3 = _mm512_loadu_ps(w + 48);
        for (int i = 0; i < ROWBLK; i++) {
            const __m512 sv = _mm512_set1_ps(x[i * ldx + k]);
            c[i][0] = _mm512_fmadd_ps(sv, b0, c[i][0]);
            c[i][1] = _mm512_fmadd_ps(sv, b1, c[i][1]);
            c[i][2] = _mm512_fmadd_ps(sv, b2, c[i][2]);
            c[i][3] = _mm512_fmadd_ps(sv, b3, c[i][3]);
        }
    }
    for (int i = 0; i < ROWBLK; i++)
        for (int j = 0; j < 4; j++) _mm512_storeu_ps(y + i * ldy + 16 * j, c[i][j]);
}

__attribute__((target("avx512f"))) static void tile1_512(const float *x, const float *p, int kc, float *y, int acc)
{
    __m512 c0 = acc ? _mm512_loadu_ps(y) : _mm512_setzero_ps(), c1 = acc ? _mm512_loadu_ps(y + 16) : _mm512_setzero_ps(),
           c2 = acc ? _mm512_loadu_ps(y + 32) : _mm512_setzero_ps(), c3 = acc ? _mm512_loadu_ps(y + 48) : _mm512_setzero_ps();
    for (int k = 0; k < kc; k++) {
        const float *w = p + (int64_t)k * PANEL;
        const __m512 sv = _mm512_set1_ps(x[k]);
        c0 = _mm512_fmadd_ps(sv, _mm512_loadu_ps(w), c0);
        c1 = _mm512_fmadd_ps(sv, _mm512_loadu_ps(w + 16), c1);
        c2 = _mm512_fmadd_ps(sv, _mm512_loadu_ps(w + 32), c2);
        c3 = _mm512_fmadd_ps(sv, _mm512_loadu_ps(w + 48), c3);
    }
    _mm512_storeu_ps(y, c0);
    _mm512_storeu_ps(y + 16, c1);
    _mm512_storeu_ps(y + 32, c2);
    _mm512_storeu_ps(y + 48, c3);
}
#endif

/* PanelGemm.RunPanel (PanelGemm.cs:87-135) for one 64-row panel: decode the
 * panel's K block into packed[k][64] (Pack, :144-164), then every token's
 * output is one fused chain over k ascending (Tile512x6 / Tile512x1,
 * :245-318); the store/reload at a K-block boundary is exact, so the chain is
 * one chain over all of k. */
static void run_panel(int type, const uint8_t *w, int rows, int cols, const float *x, int tokens,
                      float *y, int panel, float *packed, float *rowbuf)
{
    int r0 = panel * PANEL;
    int64_t rb = orc_row_bytes(type, cols);
    for (int k0 = 0; k0 < cols; k0 += KBLOCK) {
        int kc = cols - k0 < KBLOCK ? cols - k0 : KBLOCK;
        int64_t off = orc_row_bytes(type, k0);
        for (int j = 0; j < PANEL; j++) {
            orc_dequantize(type, w + (int64_t)(r0 + j) * rb + off, rowbuf, kc);
            for (int k = 0; k < kc; k++) packed[(int64_t)k * PANEL + j] = rowbuf[k];
        }
        int acc = k0 != 0;
        int t = 0;
#if defined(__x86_64__)
        if (orc_get_vector_bits() == 512) {
            for (; t + ROWBLK <= tokens; t += ROWBLK)
                tile6_512(x + (int64_t)t * cols + k0, cols, packed, kc, y + (int64_t)t * rows + r0, rows, acc);
            for (; t < tokens; t++) tile1_512(x + (int64_t)t * cols + k0, packed, kc, y + (int64_t)t * rows + r0, acc);
        }
#endif
        for (; t + ROWBLK <= tokens; t += ROWBLK) {
            float c[ROWBLK][PANEL];
            for (int i = 0; i < ROWBLK; i++)
                for (int j = 0; j < PANEL; j++)
                    c[i][j] = acc ? y[(int64_t)(t + i) * rows + r0 + j] : 0.f;
            for (int k = 0; k < kc; k++) {
                const float *p = packed + (int64_t)k * PANEL;
                for (int i = 0; i < ROWBLK; i++) {
                    float s = x[(int64_t)(t + i) * cols + k0 + k];
                    for (int j = 0; j < PANEL; j++) c[i][j] = fmaf(s, p[j], c[i][j]);
                }
            }
            for (int i = 0; i < ROWBLK; i++)
                for (int j = 0; j < PANEL; j++) y[(int64_t)(t + i) * rows + r0 + j] = c[i][j];
        }
        for (; t < tokens; t++) {
            float c[PANEL];
            for (int j = 0; j < PANEL; j++) c[j] = acc ? y[(int64_t)t * rows + r0 + j] : 0.f;
            const float *xt = x + (int64_t)t * cols + k0;
            for (int k = 0; k < kc; k++) {
                const float *p = packed + (int64_t)k * PANEL;
                float s = xt[k];
                for (int j = 0; j < PANEL; j++) c[j] = fmaf(s, p[j], c[j]);
            }
            for (int j = 0; j < PANEL; j++) y[(int64_t)t * rows + r0 + j] = c[j];
        }
    }
}

void orc_matmul(int type, const void *wv, int rows, int cols, const float *x, int tokens, float *y)
{
    const uint8_t *w = (const uint8_t *)wv;
    int nt = orc_get_threads();
    if (tokens >= 2 && panel_supports(type, rows, cols)) { /* QuantMatMul.cs:84-88 */
        int panels = rows / PANEL;
        int kmax = cols < KBLOCK ? cols : KBLOCK;
#pragma omp parallel num_threads(nt)
        {
            float *packed = (float *)malloc(sizeof(float) * (size_t)kmax * PANEL);
            float *rowbuf = (float *)malloc(sizeof(float) * (size_t)kmax);
#pragma omp for schedule(dynamic)
            for (int p = 0; p < panels; p++) run_panel(type, w, rows, cols, x, tokens, y, p, packed, rowbuf);
            free(packed);
            free(rowbuf);
        }
        return;
    }
    /* RunRowsFloat (QuantMatMul.cs:140-176): decode each row once, dot every
     * token against it. */
    int64_t rb = orc_row_bytes(type, cols);
#pragma omp parallel num_threads(nt)
    {
        float *row = (float *)malloc(sizeof(float) * (size_t)cols);
#pragma omp for schedule(static)
        for (int r = 0; r < rows; r++) {
            orc_dequantize(type, w + (int64_t)r * rb, row, cols);
            for (int t = 0; t < tokens; t++) y[(int64_t)t * rows + r] = orc_dot(x + (int64_t)t * cols, row, cols);
        }
        free(row);
    }
}

/* ------------------------------------------------------------ integer strategy */

/* binary32 -> binary16, round to nearest even (what the (Half)f conversion
 * does); used for the stored activation scale. */
static uint16_t f2h(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds past 65504 */
    if (ax < 0x38800000u) {                                    /* fp16 subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign;           /* below half the smallest subnormal */
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int)(ax >> 23);               /* to units of 2^-24 */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((ax >> 23) - 112) << 10 | ((ax >> 13) & 0x3ffu);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

/* IntegerDot.QuantizeActivations (IntegerDot.cs:60-96), count a multiple of
 * 32: per block d = max|x| / 127, inverse = d != 0 ? 1 / d : 0, stored scale
 * (Half)d, q = clamp(round-half-away-from-zero(x * inverse), -127, 127), 34
 * bytes per block.  `sums` (optional) gets d * sum(q) with the float d, as
 * QuantMatMul's integer path feeds the Q5_1 offsets (QuantMatMul.cs:223-234). */
int orc_quantize_activations(const float *x, int64_t count, uint8_t *out, float *sums)
{
    if (count % 32 != 0) return -1;
    for (int64_t b = 0; b < count / 32; b++) {
        const float *xb = x + 32 * b;
        uint8_t *o = out + 34 * b;
        float mx = 0.0f;
        for (int i = 0; i < 32; i++) {
            const float a = fabsf(xb[i]);
            if (a > mx) mx = a;
        }
        const float d = mx / 127.0f;
        const float inverse = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t h = f2h(d);
        o[0] = (uint8_t)(h & 0xff);
        o[1] = (uint8_t)(h >> 8);
        int sum = 0;
        for (int i = 0; i < 32; i++) {
            const float scaled = xb[i] * inverse;
            int v = (int)roundf(scaled);
            v = v < -127 ? -127 : (v > 127 ? 127 : v);
            o[2 + i] = (uint8_t)(int8_t)v;
            sum += v;
        }
        if (sums) sums[b] = d * (float)sum;
    }
    return 0;
}

/* IntegerDot.UnpackRow (IntegerDot.cs:113-204) for Q8_0 / Q4_0 / Q5_1: plain
 * int8 values, per-block scales and (Q5_1) offsets. */
static void unpack_row(int type, const uint8_t *w, int8_t *v, float *scales, float *offsets, int blocks)
{
    for (int b = 0; b < blocks; b++) {
        if (type == ORC_Q8_0) {
            const uint8_t *blk = w + 34 * b;
            scales[b] = h2f(rd16(blk));
            memcpy(v + 32 * b, blk + 2, 32);
        } else if (type == ORC_Q4_0) {
            const uint8_t *blk = w + 18 * b, *qs = blk + 2;
            scales[b] = h2f(rd16(blk));
            for (int j = 0; j < 16; j++) {
                v[32 * b + j] = (int8_t)((qs[j] & 0x0F) - 8);
                v[32 * b + 16 + j] = (int8_t)((qs[j] >> 4) - 8);
            }
        } else { /* Q5_1 */
            const uint8_t *blk = w + 24 * b, *qs = blk + 8;
            scales[b] = h2f(rd16(blk));
            offsets[b] = h2f(rd16(blk + 2));
            const uint32_t qh = rd32(blk + 4);
            for (int j = 0; j < 16; j++) {
                v[32 * b + j] = (int8_t)((qs[j] & 0x0F) | (int)(((qh >> j) & 1) << 4));
                v[32 * b + 16 + j] = (int8_t)((qs[j] >> 4) | (int)(((qh >> (j + 16)) & 1) << 4));
            }
        }
    }
}

/* QuantMatMul.ForwardAsync with Strategy = Integer (QuantMatMul.cs:84-100,
 * ForwardIntegerAsync :186-221, RunRowsInteger :236-287): activations
 * quantized per token, then per (row, token) the block dots of
 * IntegerDot.DotPackedQ8_0 / DotUnpacked (IntegerDot.cs:206-272) in their
 * scalar form -- total += (w_scale * x_scale) * sum(w_i * q_i), blocks
 * ascending -- plus, for Q5_1, OffsetContribution (:274-279): sum over blocks
 * of offset * (d * sum(q)), added after the dot.  The AVX2 branches of those
 * dots keep eight lane partials instead; their order is not pinned by the
 * reference's tests (IntegerDotTests.cs:56-101 bound the path against the
 * float one at 1 % relative L2). */
int orc_matmul_integer(int type, const void *wv, int rows, int cols, const float *x, int tokens, float *y)
{
    if ((type != ORC_Q8_0 && type != ORC_Q4_0 && type != ORC_Q5_1) || cols % 32 != 0) return -1;
    const uint8_t *w = (const uint8_t *)wv;
    const int blocks = cols / 32;
    const int64_t rb = orc_row_bytes(type, cols), qrb = (int64_t)blocks * 34;
    uint8_t *act = (uint8_t *)malloc((size_t)(qrb * tokens));
    float *sums = (float *)malloc(sizeof(float) * (size_t)blocks * tokens);
    for (int t = 0; t < tokens; t++) orc_quantize_activations(x + (int64_t)t * cols, cols, act + t * qrb, sums + (int64_t)t * blocks);
    int nt = orc_get_threads();
#pragma omp parallel num_threads(nt)
    {
        int8_t *v = (int8_t *)malloc((size_t)cols);
        float *sc = (float *)malloc(sizeof(float) * blocks), *of = (float *)malloc(sizeof(float) * blocks);
#pragma omp for schedule(static)
        for (int r = 0; r < rows; r++) {
            unpack_row(type, w + (int64_t)r * rb, v, sc, of, blocks);
            for (int t = 0; t < tokens; t++) {
                const uint8_t *a = act + t * qrb;
                float total = 0.0f;
                for (int b = 0; b < blocks; b++) {
                    const int8_t *q = (const int8_t *)(a + 34 * b + 2);
                    int sumi = 0;
                    for (int i = 0; i < 32; i++) sumi += (int)v[32 * b + i] * (int)q[i];
                    const float s = sc[b] * h2f(rd16(a + 34 * b));
                    total = total + s * (float)sumi;
                }
                if (type == ORC_Q5_1) {
                    float off = 0.0f;
                    for (int b = 0; b < blocks; b++) off = off + of[b] * sums[(int64_t)t * blocks + b];
                    total = total + off;
                }
                y[(int64_t)t * rows + r] = total;
            }
        }
        free(v);
        free(sc);
        free(of);
    }
    free(act);
    free(sums);
    return 0;
}

/* ------------------------------------------------------------ attention */

/* One query against its visible keys: AttentionKernels.Scores (:44-78) gives
 * each key a fused chain over d ascending, then * scale; Kernels.Softmax over
 * exactly the visible keys; AttentionKernels.WeightedSum (:85-105) a fused
 * chain over the visible keys in logical order for every output dim. */
void orc_attend(const float *q, const float *keys, const float *values, int hd,
                int shared_lo, int shared_hi, int segment, int slot, float scale,
                float *scores, float *out)
{
    int n_sh = shared_hi - shared_lo;
    int limit = n_sh + (slot - segment + 1);
    for (int i = 0; i < limit; i++) {
        int p = i < n_sh ? shared_lo + i : segment + (i - n_sh);
        const float *k = keys + (int64_t)p * hd;
        float a = 0.f;
        for (int d = 0; d < hd; d++) a = fmaf(q[d], k[d], a);
        scores[i] = a * scale;
    }
    orc_softmax(scores, limit);
    for (int d = 0; d < hd; d++) out[d] = 0.f;
    for (int i = 0; i < limit; i++) {
        int p = i < n_sh ? shared_lo + i : segment + (i - n_sh);
        const float *v = values + (int64_t)p * hd;
        float wgt = scores[i];
        for (int d = 0; d < hd; d++) out[d] = fmaf(wgt, v[d], out[d]);
    }
}

/* ------------------------------------------------------------ RoPE */

static float mscale_of(float scale, float m) { return scale <= 1.0f ? 1.0f : 0.1f * m * logf(scale) + 1.0f; }

/* Rope ctor (Rope.cs:33-66) with ComputeMagnitudeScale (:78-88) and
 * YarnCorrectionDims (:91-106).  Returns the number of pairs. */
int orc_rope_freqs(const orc_config *c, float *freqs, float *mscale)
{
    int half = c->rope_dim / 2;
    float freq_scale = 1.0f / c->rope_scale_factor;
    int yarn = c->rope_scaling_yarn && c->rope_original_context > 0 && c->yarn_ext_factor != 0.0f &&
               c->rope_scale_factor > 1.0f; /* ModelConfig.YarnActive, ModelConfig.cs:54-56 */
    if (!yarn) {
        for (int i = 0; i < half; i++)
            freqs[i] = freq_scale / powf(c->rope_freq_base, 2.0f * (float)i / (float)c->rope_dim);
        *mscale = c->rope_attn_factor;
        return half;
    }
    float low, high;
    if (c->yarn_beta_fast == 0.0f && c->yarn_beta_slow == 0.0f) {
        low = 3.402823466e+38f;
        high = (float)c->rope_dim / 2.0f - 1.0f;
    } else {
        const float pi = 3.14159265358979323846f;
        float dims = (float)c->rope_dim, base = c->rope_freq_base;
        float cd_fast = dims * logf((float)c->rope_original_context / (c->yarn_beta_fast * 2.0f * pi)) / (2.0f * logf(base));
        float cd_slow = dims * logf((float)c->rope_original_context / (c->yarn_beta_slow * 2.0f * pi)) / (2.0f * logf(base));
        low = fmaxf(0.0f, floorf(cd_fast));
        high = fminf(dims / 2.0f - 1.0f, ceilf(cd_slow));
    }
    for (int i = 0; i < half; i++) {
        float extrapolated = 1.0f / powf(c->rope_freq_base, 2.0f * (float)i / (float)c->rope_dim);
        float interpolated = freq_scale * extrapolated;
        float yv = ((float)i - low) / fmaxf(0.001f, high - low);
        float cl = yv < 0.0f ? 0.0f : (yv > 1.0f ? 1.0f : yv);
        float mix = (1.0f - cl) * c->yarn_ext_factor;
        float a = interpolated * (1.0f - mix);
        float b = extrapolated * mix;
        freqs[i] = a + b;
    }
    float factor = c->rope_scale_factor;
    float m = c->yarn_mscale != 0.0f ? c->yarn_mscale : 1.0f;
    float ratio = c->yarn_mscale_all_dim != 0.0f ? mscale_of(factor, m) / mscale_of(factor, c->yarn_mscale_all_dim)
                                                 : mscale_of(factor, 1.0f);
    *mscale = ratio * c->rope_attn_factor;
    return half;
}

/* Rope.Apply (Rope.cs:112-135): cos/sin of position * freq in float times
 * mscale; adjacent pairs rotated with separate multiplies. */
void orc_rope_apply(const float *freqs, int half, float mscale, float *data, int heads, int hd, int position)
{
    float cs[512], sn[512];
    for (int i = 0; i < half; i++) {
        float theta = (float)position * freqs[i];
        cs[i] = cosf(theta) * mscale;
        sn[i] = sinf(theta) * mscale;
    }
    for (int h = 0; h < heads; h++) {
        float *v = data + (int64_t)h * hd;
        for (int i = 0; i < half; i++) {
            float x0 = v[2 * i], x1 = v[2 * i + 1];
            float a = x0 * cs[i], b = x1 * sn[i];
            float c = x0 * sn[i], d = x1 * cs[i];
            v[2 * i] = a - b;
            v[2 * i + 1] = c + d;
        }
    }
}

/* ------------------------------------------------------------ layouts */

int orc_layout_tree(int start_pos, int trunk, const int32_t *offsets, int nb, int tokens,
                    int32_t *slot, int32_t *pos, int32_t *shared, int32_t *seg, int32_t *outputs)
{
    int branch = -1;
    for (int t = 0; t < tokens; t++) {
        slot[t] = start_pos + t;
        while (branch + 1 < nb && t >= offsets[branch + 1]) branch++;
        if (t < trunk || branch < 0) {
            pos[t] = start_pos + t; shared[t] = start_pos; seg[t] = start_pos;
        } else {
            pos[t] = start_pos + trunk + (t - offsets[branch]);
            shared[t] = start_pos + trunk;
            seg[t] = start_pos + offsets[branch];
        }
    }
    for (int b = 0; b < nb; b++) outputs[b] = (b + 1 < nb ? offsets[b + 1] : tokens) - 1;
    return start_pos + tokens;
}

int orc_layout_rows(int shared, const int32_t *row_base, const int32_t *row_length, const int32_t *row_tokens,
                    int nr, int32_t *slot, int32_t *pos, int32_t *sh, int32_t *seg, int32_t *outputs)
{
    int t = 0, end = shared;
    for (int r = 0; r < nr; r++) {
        for (int i = 0; i < row_tokens[r]; i++, t++) {
            slot[t] = row_base[r] + row_length[r] + i;
            pos[t] = shared + row_length[r] + i;
            sh[t] = shared;
            seg[t] = row_base[r];
            if (slot[t] + 1 > end) end = slot[t] + 1;
        }
        outputs[r] = t - 1;
    }
    return end;
}

/* ------------------------------------------------------------ model */

typedef struct { int type, rows, cols; const uint8_t *data; } tensor_t;

struct orc_model {
    orc_config c;
    tensor_t embd, out_norm_t, output;
    float *out_norm;
    tensor_t *q, *k, *v, *o, *gate, *up, *down;
    float **attn_norm, **ffn_norm;
    float freqs[512];
    int half;
    float mscale;
    /* KvCache (KvCache.cs:12-140): [layer][head][capacity][hd] */
    float **keys, **values;
    int capacity, length;
    /* the capture of the call in flight (orc_forward_capture), else NULL */
    orc_sink sink;
    void *sink_user;
};

/* capture?.Observe(name, values, rows, columns) */
static void observe(const orc_model *m, const char *name, const float *v, int rows, int cols)
{
    if (m->sink) m->sink(m->sink_user, name, v, rows, cols);
}

static void observe_layer(const orc_model *m, int l, const char *tap, const float *v, int rows, int cols)
{
    char name[64];
    if (!m->sink) return;
    snprintf(name, sizeof name, "blk.%d.%s", l, tap);
    m->sink(m->sink_user, name, v, rows, cols);
}

static float **kv_alloc(const orc_model *m, int cap)
{
    float **a = (float **)calloc((size_t)m->c.n_layers, sizeof(float *));
    for (int l = 0; l < m->c.n_layers; l++)
        a[l] = (float *)calloc((size_t)m->c.n_kv_heads * cap * m->c.head_dim, sizeof(float));
    return a;
}

static void kv_free(const orc_model *m, float **a)
{
    if (!a) return;
    for (int l = 0; l < m->c.n_layers; l++) free(a[l]);
    free(a);
}

/* KvCache.EnsureCapacity (KvCache.cs:48-70): double until it fits, copy the
 * populated prefix of every head. */
static void kv_ensure(orc_model *m, int required)
{
    if (required <= m->capacity) return;
    int cap = m->capacity;
    while (cap < required) cap *= 2;
    float **k = kv_alloc(m, cap), **v = kv_alloc(m, cap);
    int hd = m->c.head_dim;
    for (int l = 0; l < m->c.n_layers; l++)
        for (int h = 0; h < m->c.n_kv_heads; h++) {
            memcpy(k[l] + (int64_t)h * cap * hd, m->keys[l] + (int64_t)h * m->capacity * hd, sizeof(float) * (size_t)m->length * hd);
            memcpy(v[l] + (int64_t)h * cap * hd, m->values[l] + (int64_t)h * m->capacity * hd, sizeof(float) * (size_t)m->length * hd);
        }
    kv_free(m, m->keys);
    kv_free(m, m->values);
    m->keys = k;
    m->values = v;
    m->capacity = cap;
}

static float *kv_row(float **a, const orc_model *m, int layer, int head, int slot)
{
    return a[layer] + ((int64_t)head * m->capacity + slot) * m->c.head_dim;
}

const float *orc_kv_key(const orc_model *m, int layer, int head, int slot) { return kv_row(m->keys, m, layer, head, slot); }
const float *orc_kv_value(const orc_model *m, int layer, int head, int slot) { return kv_row(m->values, m, layer, head, slot); }

orc_model *orc_model_create(const orc_config *cfg)
{
    if (cfg->n_heads % cfg->n_kv_heads != 0 || cfg->rope_dim > 1024) return NULL;
    orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
    m->c = *cfg;
    int L = cfg->n_layers;
    m->q = (tensor_t *)calloc((size_t)L, sizeof(tensor_t));
    m->k = (tensor_t *)calloc((size_t)L, sizeof(tensor_t));
    m->v = (tensor_t *)calloc((size_t)L, sizeof(tensor_t));
    m->o = (tensor_t *)calloc((size_t)L, sizeof(tensor_t));
    m->gate = (tensor_t *)calloc((size_t)L, sizeof(tensor_t));
    m->up = (tensor_t *)calloc((size_t)L, sizeof(tensor_t));
    m->down = (tensor_t *)calloc((size_t)L, sizeof(tensor_t));
    m->attn_norm = (float **)calloc((size_t)L, sizeof(float *));
    m->ffn_norm = (float **)calloc((size_t)L, sizeof(float *));
    m->half = orc_rope_freqs(cfg, m->freqs, &m->mscale);
    m->capacity = cfg->initial_kv_capacity > 1 ? cfg->initial_kv_capacity : 1;
    m->keys = kv_alloc(m, m->capacity);
    m->values = kv_alloc(m, m->capacity);
    return m;
}

void orc_model_destroy(orc_model *m)
{
    if (!m) return;
    for (int l = 0; l < m->c.n_layers; l++) { free(m->attn_norm[l]); free(m->ffn_norm[l]); }
    free(m->q); free(m->k); free(m->v); free(m->o); free(m->gate); free(m->up); free(m->down);
    free(m->attn_norm); free(m->ffn_norm); free(m->out_norm);
    kv_free(m, m->keys);
    kv_free(m, m->values);
    free(m);
}

static float *decode_vector(int type, const void *bytes, int n)
{
    float *v = (float *)malloc(sizeof(float) * (size_t)n);
    orc_dequantize(type, bytes, v, n); /* VectorParameter.From, WeightMatrix.cs:76-90 */
    return v;
}

int orc_model_bind(orc_model *m, int slot, int layer, int type, int rows, int cols, const void *bytes)
{
    if (orc_block_size(type) == 0) return -1;
    tensor_t t = {type, rows, cols, (const uint8_t *)bytes};
    if (slot >= ORC_SLOT_ATTN_NORM && (layer < 0 || layer >= m->c.n_layers)) return -1;
    switch (slot) {
    case ORC_SLOT_TOKEN_EMBD: m->embd = t; return 0;
    case ORC_SLOT_OUTPUT_NORM: free(m->out_norm); m->out_norm = decode_vector(type, bytes, cols); return 0;
    case ORC_SLOT_OUTPUT: m->output = t; return 0;
    case ORC_SLOT_ATTN_NORM: free(m->attn_norm[layer]); m->attn_norm[layer] = decode_vector(type, bytes, cols); return 0;
    case ORC_SLOT_FFN_NORM: free(m->ffn_norm[layer]); m->ffn_norm[layer] = decode_vector(type, bytes, cols); return 0;
    case ORC_SLOT_Q: m->q[layer] = t; return 0;
    case ORC_SLOT_K: m->k[layer] = t; return 0;
    case ORC_SLOT_V: m->v[layer] = t; return 0;
    case ORC_SLOT_O: m->o[layer] = t; return 0;
    case ORC_SLOT_GATE: m->gate[layer] = t; return 0;
    case ORC_SLOT_UP: m->up[layer] = t; return 0;
    case ORC_SLOT_DOWN: m->down[layer] = t; return 0;
    default: return -1;
    }
}

static void mm(const tensor_t *w, const float *x, int tokens, float *y)
{
    orc_matmul(w->type, w->data, w->rows, w->cols, x, tokens, y);
}

/* MinistralModel.ApplyPositionScale (MinistralModel.cs:676-682). */
static void position_scale(const orc_model *m, float *q, int n, int position)
{
    if (m->c.rope_original_context <= 0 || m->c.attention_temperature_scale == 0.0f) return;
    float interval = floorf((float)position / (float)m->c.rope_original_context);
    if (interval == 0.0f) return;
    float s = 1.0f + m->c.attention_temperature_scale * logf(1.0f + interval);
    for (int i = 0; i < n; i++) q[i] = q[i] * s;
}

/* The private ForwardAsync (MinistralModel.cs:301-435) with AttentionAsync
 * (:446-557) and the AttendHead arithmetic (:564-636). */
int orc_forward(orc_model *m, const int32_t *tokens, int seq, const orc_layout *lay, int mode,
                const int32_t *rows, int n_rows, float *out, size_t out_len)
{
    const orc_config *c = &m->c;
    if (seq <= 0) return -1;
    int hidden = c->hidden, ff = c->ffn, hd = c->head_dim;
    int heads = c->n_heads, kvh = c->n_kv_heads, group = heads / kvh;
    int qdim = heads * hd, kvdim = kvh * hd;
    int start = m->length;
    int end = lay ? lay->end : start + seq;
    int n_out = lay ? lay->n_outputs : 1;
    size_t need = mode == ORC_OUT_NONE ? 0 : mode == ORC_OUT_LAST_FULL ? (size_t)c->vocab
                 : mode == ORC_OUT_SELECTED ? (size_t)n_out * n_rows : (size_t)n_out * c->vocab;
    if (out_len < need) return -1;
    for (int t = 0; t < seq; t++)
        if (tokens[t] < 0 || tokens[t] >= m->embd.rows) return -1; /* GatherRows, QuantMatMul.cs:300-302 */
    kv_ensure(m, end);

    float *h = (float *)malloc(sizeof(float) * (size_t)seq * hidden);
    float *norm = (float *)malloc(sizeof(float) * (size_t)seq * hidden);
    float *scratch = (float *)malloc(sizeof(float) * (size_t)seq * hidden);
    float *q = (float *)malloc(sizeof(float) * (size_t)seq * qdim);
    float *ctx = (float *)malloc(sizeof(float) * (size_t)seq * qdim);
    float *kv = (float *)malloc(sizeof(float) * (size_t)seq * kvdim);
    float *g = (float *)malloc(sizeof(float) * (size_t)seq * ff);
    float *u = (float *)malloc(sizeof(float) * (size_t)seq * ff);
    int64_t erb = orc_row_bytes(m->embd.type, hidden);

    for (int t = 0; t < seq; t++) /* QuantMatMul.GatherRows, QuantMatMul.cs:294-305 */
        orc_dequantize(m->embd.type, m->embd.data + (int64_t)tokens[t] * erb, h + (int64_t)t * hidden, hidden);
    observe(m, "embeddings", h, seq, hidden);

    float scale = 1.0f / sqrtf((float)hd);
    int nt = orc_get_threads();
    for (int l = 0; l < c->n_layers; l++) {
        for (int t = 0; t < seq; t++)
            orc_rmsnorm(h + (int64_t)t * hidden, m->attn_norm[l], c->rms_eps, hidden, norm + (int64_t)t * hidden);
        observe_layer(m, l, "attn_norm", norm, seq, hidden);
        /* AttentionAsync: Q, RotateQueries (:638-647) */
        mm(&m->q[l], norm, seq, q);
        for (int t = 0; t < seq; t++) {
            int p = lay ? lay->position[t] : start + t;
            orc_rope_apply(m->freqs, m->half, m->mscale, q + (int64_t)t * qdim, heads, hd, p);
            position_scale(m, q + (int64_t)t * qdim, qdim, p);
        }
        observe_layer(m, l, "q_rope", q, seq, qdim);
        /* K -> StoreKeys (:649-660), V -> StoreValues (:662-669) */
        mm(&m->k[l], norm, seq, kv);
        for (int t = 0; t < seq; t++) {
            float *row = kv + (int64_t)t * kvdim;
            orc_rope_apply(m->freqs, m->half, m->mscale, row, kvh, hd, lay ? lay->position[t] : start + t);
            int s = lay ? lay->slot[t] : start + t;
            for (int kh = 0; kh < kvh; kh++) memcpy(kv_row(m->keys, m, l, kh, s), row + kh * hd, sizeof(float) * hd);
        }
        observe_layer(m, l, "k_rope", kv, seq, kvdim);
        mm(&m->v[l], norm, seq, kv);
        observe_layer(m, l, "v", kv, seq, kvdim);
        for (int t = 0; t < seq; t++) {
            int s = lay ? lay->slot[t] : start + t;
            for (int kh = 0; kh < kvh; kh++) memcpy(kv_row(m->values, m, l, kh, s), kv + (int64_t)t * kvdim + kh * hd, sizeof(float) * hd);
        }
        /* Grouped-query attention, heads in parallel (:498-503). */
#pragma omp parallel num_threads(nt)
        {
            float *scores = (float *)malloc(sizeof(float) * (size_t)end);
#pragma omp for schedule(dynamic)
            for (int head = 0; head < heads; head++) {
                int kvhead = head / group;
                const float *keys = kv_row(m->keys, m, l, kvhead, 0);
                const float *vals = kv_row(m->values, m, l, kvhead, 0);
                for (int t = 0; t < seq; t++) {
                    int slot = lay ? lay->slot[t] : start + t;
                    int slo = lay ? lay->shared_lo[t] : 0;
                    int shi = lay ? lay->shared_hi[t] : start;
                    int segm = lay ? lay->segment[t] : start;
                    orc_attend(q + (int64_t)t * qdim + head * hd, keys, vals, hd, slo, shi, segm, slot, scale,
                               scores, ctx + (int64_t)t * qdim + head * hd);
                }
            }
            free(scores);
        }
        observe_layer(m, l, "attn_weighted", ctx, seq, qdim);
        mm(&m->o[l], ctx, seq, scratch);
        observe_layer(m, l, "attn_out", scratch, seq, hidden);
        for (int i = 0; i < seq * hidden; i++) h[i] = h[i] + scratch[i]; /* Kernels.Add */
        observe_layer(m, l, "post_attn", h, seq, hidden);
        for (int t = 0; t < seq; t++)
            orc_rmsnorm(h + (int64_t)t * hidden, m->ffn_norm[l], c->rms_eps, hidden, norm + (int64_t)t * hidden);
        observe_layer(m, l, "ffn_norm", norm, seq, hidden);
        mm(&m->gate[l], norm, seq, g);
        mm(&m->up[l], norm, seq, u);
        orc_swiglu(g, u, g, seq * ff);
        mm(&m->down[l], g, seq, scratch);
        observe_layer(m, l, "ffn_out", scratch, seq, hidden);
        for (int i = 0; i < seq * hidden; i++) h[i] = h[i] + scratch[i];
        observe_layer(m, l, "output", h, seq, hidden);
    }
    if (end > m->length) m->length = end; /* KvCache.Advance (:360) */

    const tensor_t *table = m->output.data ? &m->output : &m->embd;
    int64_t trb = orc_row_bytes(table->type, hidden);
    if (mode == ORC_OUT_FULL) { /* :362-385 */
        float *rowsbuf = (float *)malloc(sizeof(float) * (size_t)n_out * hidden);
        for (int b = 0; b < n_out; b++) {
            int tok = lay ? lay->outputs[b] : seq - 1;
            orc_rmsnorm(h + (int64_t)tok * hidden, m->out_norm, c->rms_eps, hidden, rowsbuf + (int64_t)b * hidden);
        }
        mm(table, rowsbuf, n_out, out);
        free(rowsbuf);
    } else if (mode == ORC_OUT_SELECTED) { /* :386-410 */
        float *row = (float *)malloc(sizeof(float) * (size_t)hidden);
        for (int b = 0; b < n_out; b++) {
            int tok = lay ? lay->outputs[b] : seq - 1;
            orc_rmsnorm(h + (int64_t)tok * hidden, m->out_norm, c->rms_eps, hidden, norm);
            for (int i = 0; i < n_rows; i++) {
                orc_dequantize(table->type, table->data + (int64_t)rows[i] * trb, row, hidden);
                out[(size_t)b * n_rows + i] = orc_dot(norm, row, hidden);
            }
        }
        free(row);
    } else if (mode == ORC_OUT_LAST_FULL) { /* :411-424 */
        orc_rmsnorm(h + (int64_t)(seq - 1) * hidden, m->out_norm, c->rms_eps, hidden, norm);
        observe(m, "final_norm", norm, 1, hidden);
        mm(table, norm, 1, out);
        observe(m, "logits", out, 1, c->vocab);
    }
    free(h); free(norm); free(scratch); free(q); free(ctx); free(kv); free(g); free(u);
    return 0;
}

int orc_forward_capture(orc_model *m, const int32_t *tokens, int n, orc_sink sink, void *user, float *out,
                        size_t out_len)
{
    m->sink = sink;
    m->sink_user = user;
    int rc = orc_forward(m, tokens, n, NULL, ORC_OUT_LAST_FULL, NULL, 0, out, out_len);
    m->sink = NULL;
    m->sink_user = NULL;
    return rc;
}

int orc_forward_tree(orc_model *m, const int32_t *trunk, int n_trunk, const int32_t *btok,
                     const int32_t *blen, int nb, const int32_t *rows, int n_rows, float *out, size_t out_len)
{
    if (nb <= 0) return -1;
    int total = n_trunk;
    int32_t *offsets = (int32_t *)malloc(sizeof(int32_t) * (size_t)nb);
    for (int b = 0; b < nb; b++) {
        if (blen[b] <= 0) { free(offsets); return -1; }
        offsets[b] = total;
        total += blen[b];
    }
    int32_t *tokens = (int32_t *)malloc(sizeof(int32_t) * (size_t)total);
    memcpy(tokens, trunk, sizeof(int32_t) * (size_t)n_trunk);
    memcpy(tokens + n_trunk, btok, sizeof(int32_t) * (size_t)(total - n_trunk));
    int32_t *slot = (int32_t *)malloc(sizeof(int32_t) * (size_t)total * 5);
    int32_t *pos = slot + total, *sh = slot + 2 * total, *seg = slot + 3 * total, *lo = slot + 4 * total;
    int32_t *outs = (int32_t *)malloc(sizeof(int32_t) * (size_t)nb);
    int endp = orc_layout_tree(m->length, n_trunk, offsets, nb, total, slot, pos, sh, seg, outs);
    for (int t = 0; t < total; t++) lo[t] = 0;
    orc_layout lay = {slot, pos, lo, sh, seg, outs, nb, endp};
    int rc = orc_forward(m, tokens, total, &lay, ORC_OUT_SELECTED, rows, n_rows, out, out_len);
    free(offsets); free(tokens); free(slot); free(outs);
    return rc;
}

int orc_kv_length(const orc_model *m) { return m->length; }
void orc_kv_truncate(orc_model *m, int length) { m->length = length < 0 ? 0 : (length > m->length ? m->length : length); }
void orc_kv_reset(orc_model *m) { m->length = 0; }

int orc_kv_snapshot(const orc_model *m, int length, float *out, size_t n)
{
    int hd = m->c.head_dim;
    size_t per = (size_t)m->c.n_layers * m->c.n_kv_heads * length * hd;
    if (length > m->length || n != per * 2) return -1;
    size_t cur = 0;
    for (int pass = 0; pass < 2; pass++)
        for (int l = 0; l < m->c.n_layers; l++)
            for (int h = 0; h < m->c.n_kv_heads; h++) {
                memcpy(out + cur, kv_row(pass ? m->values : m->keys, m, l, h, 0), sizeof(float) * (size_t)length * hd);
                cur += (size_t)length * hd;
            }
    return 0;
}

int orc_kv_restore(orc_model *m, const float *in, size_t n, int length)
{
    int hd = m->c.head_dim;
    size_t per = (size_t)m->c.n_layers * m->c.n_kv_heads * length * hd;
    if (n != per * 2) return -1;
    kv_ensure(m, length);
    size_t cur = 0;
    for (int pass = 0; pass < 2; pass++)
        for (int l = 0; l < m->c.n_layers; l++)
            for (int h = 0; h < m->c.n_kv_heads; h++) {
                memcpy(kv_row(pass ? m->values : m->keys, m, l, h, 0), in + cur, sizeof(float) * (size_t)length * hd);
                cur += (size_t)length * hd;
            }
    m->length = length;
    return 0;
}

/* JevstralDecider.DecideAsync margins (:306-308, Best = max over the listed
 * rows) and probabilities softmax(z / T) (:310-313). */
void orc_margins(const float *v, int n_options, int n_yes, int n_no, float temperature, float *margins, float *probs)
{
    int nr = n_yes + n_no;
    for (int i = 0; i < n_options; i++) {
        const float *r = v + (size_t)i * nr;
        float by = r[0], bn = r[n_yes];
        for (int j = 1; j < n_yes; j++) if (r[j] > by) by = r[j];
        for (int j = 1; j < n_no; j++) if (r[n_yes + j] > bn) bn = r[n_yes + j];
        margins[i] = by - bn;
        probs[i] = margins[i] / temperature;
    }
    orc_softmax(probs, n_options);
}
