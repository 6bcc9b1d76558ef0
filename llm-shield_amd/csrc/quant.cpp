// Host-side block formats: GGML geometry, fp16 conversion, the field-split
// repack that feeds HBM, the ggml reference quantizers and the synthetic
// weight generator.  Built with -ffp-contract=off: the quantizers' rounding
// must follow the published scalar algorithms exactly (no fused multiply-add).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <thread>
#include <vector>

#include "../../include/jev.h"
#include "jev_internal.h"

namespace jev {

int block_size(int type)
{
    switch (type) {
    case kF32: case kF16: return 1;
    case kQ4_0: case kQ5_1: case kQ8_0: return 32;
    default: return 0;
    }
}

int type_size(int type)
{
    switch (type) {
    case kF32: return 4;
    case kF16: return 2;
    case kQ4_0: return 18;
    case kQ5_1: return 24;
    case kQ8_0: return 34;
    default: return 0;
    }
}

int64_t row_bytes(int type, int64_t cols)
{
    int bs = block_size(type);
    return bs ? cols / bs * type_size(type) : -1;
}

float half_to_float(uint16_t h)
{
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff, f;
    if (e == 0) {
        if (m == 0) {
            f = s;
        } else {
            int ee = 127 - 15 + 1;
            while (!(m & 0x400)) {
                m <<= 1;
                ee--;
            }
            m &= 0x3ff;
            f = s | ((uint32_t)ee << 23) | (m << 13);
        }
    } else if (e == 31) {
        f = s | 0x7f800000u | (m << 13);
    } else {
        f = s | ((e - 15 + 127) << 23) | (m << 13);
    }
    float r;
    std::memcpy(&r, &f, 4);
    return r;
}

// IEEE binary32 -> binary16, round to nearest even (what F16C's vcvtps2ph with
// imm 0, numpy's astype(float16) and GGML_FP32_TO_FP16 all do).
uint16_t float_to_half(float f)
{
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u)); // inf / nan
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); // rounds to >= 65520 -> inf
    if (ax < 0x38800000u) { // subnormal half (or zero)
        if (ax < 0x33000000u) return (uint16_t)sign; // < 2^-25 rounds to zero (ties to even at 2^-25 -> 0)
        uint32_t e = ax >> 23;
        uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
        int shift = 126 - (int)e; // 14 + (113 - e)... value = mant * 2^(e-150); half unit = 2^-24
        // result = mant * 2^(e - 150 + 24) = mant >> (126 - e)
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 127 + 15;
    uint32_t mant = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

QLayout qlayout(int type, int64_t rows, int64_t cols)
{
    QLayout l{0, 0, 0, 0, 0, 0};
    const size_t tiles = (size_t)tile_rows((int)rows) * (size_t)tile_kpairs((int)cols);
    l.qs = 0;
    l.d = align256(tiles * tile_qs_bytes(type));
    size_t end = l.d + tiles * tile_d_bytes(type);
    if (type == kQ5_1) {
        l.m = l.d + 4; // interleaved with the scales: row r's mins at 8 r + 4
        l.qh = align256(end);
        end = l.qh + tiles * 128;
        l.qb = align256(end);
        end = l.qb + tiles * 1024;
    }
    l.total = align256(end);
    return l;
}

static void parallel_rows(int64_t rows, int threads, const std::function<void(int64_t, int64_t)> &fn);

// GGUF blocks -> tiles.  Element (r, k) of a block pair goes to lane
// l = 16 (k % 32 / 8) + r % 16; see the layout description in jev_internal.h.
bool repack_host(int type, int64_t rows, int64_t cols, const void *gguf, void *dst, int threads)
{
    if ((type != kQ8_0 && type != kQ4_0 && type != kQ5_1) || cols % 32 != 0 || rows <= 0) return false;
    QLayout L = qlayout(type, rows, cols);
    const uint8_t *src = (const uint8_t *)gguf;
    uint8_t *out = (uint8_t *)dst;
    const int64_t nb = cols / 32, ts = type_size(type);
    const int64_t KP = tile_kpairs((int)cols), RG = tile_rows((int)rows);
    const size_t TQ = tile_qs_bytes(type);
    // zero padding (rows past the weight, the odd last block) and alignment gaps
    parallel_rows(RG, threads, [&](int64_t g0, int64_t g1) {
        auto clear = [&](size_t off, size_t per_tile) { std::memset(out + off + g0 * KP * per_tile, 0, (g1 - g0) * KP * per_tile); };
        clear(L.qs, TQ);
        clear(L.d, (size_t)tile_d_bytes(type));
        if (type == kQ5_1) {
            clear(L.qh, 128);
            clear(L.qb, 1024);
        }
    });
    parallel_rows(rows, threads, [&](int64_t r0, int64_t r1) {
        for (int64_t row = r0; row < r1; row++) {
            const uint8_t *rowp = src + row * nb * ts;
            const int64_t rg = row / 16, r = row % 16;
            for (int64_t b = 0; b < nb; b++) {
                const uint8_t *blk = rowp + b * ts;
                const size_t tile = (size_t)(rg * KP + b / 2);
                const int bb = (int)(b & 1);
                const size_t dstride = (size_t)tile_d_bytes(type), drow = type == kQ5_1 ? 8 : 4;
                std::memcpy(out + L.d + tile * dstride + drow * r + 2 * bb, blk, 2);
                if (type == kQ8_0) {
                    // stored biased, q + 128 (the sign bit flipped): the decoders
                    // place the byte under an fp16 exponent as it is
                    for (int g = 0; g < 4; g++) {
                        uint8_t *dq = out + L.qs + tile * TQ + 16 * (16 * g + r) + 8 * bb;
                        for (int i = 0; i < 8; i++) dq[i] = (uint8_t)(blk[2 + 8 * g + i] ^ 0x80u);
                    }
                    continue;
                }
                // element j of the block: low nibble of byte j (j < 16), high nibble of byte j - 16
                const uint8_t *qs = blk + (type == kQ4_0 ? 2 : 8);
                uint32_t qh = 0;
                if (type == kQ5_1) {
                    std::memcpy(out + L.d + tile * dstride + drow * r + 4 + 2 * bb, blk + 2, 2);
                    std::memcpy(&qh, blk + 4, 4);
                }
                for (int g = 0; g < 4; g++) {
                    uint8_t *dq = out + L.qs + tile * TQ + 8 * (16 * g + r) + 4 * bb;
                    for (int i = 0; i < 4; i++) {
                        auto nib = [&](int j) { return j < 16 ? (qs[j] & 15) : (qs[j - 16] >> 4); };
                        dq[i] = (uint8_t)(nib(8 * g + i) | (nib(8 * g + i + 4) << 4));
                    }
                    if (type == kQ5_1) {
                        out[L.qh + tile * 128 + 2 * (16 * g + r) + bb] = (uint8_t)((qh >> (8 * g)) & 0xffu);
                        // the byte copy: element 8 g + i at byte 8 bb + i of lane 16 g + r
                        uint8_t *db = out + L.qb + tile * 1024 + 16 * (16 * g + r) + 8 * bb;
                        for (int i = 0; i < 8; i++) {
                            const int j = 8 * g + i;
                            const int nibj = j < 16 ? (qs[j] & 15) : (qs[j - 16] >> 4);
                            db[i] = (uint8_t)(nibj | (((qh >> j) & 1u) << 4));
                        }
                    }
                }
            }
        }
    });
    return true;
}

static void parallel_rows(int64_t rows, int threads, const std::function<void(int64_t, int64_t)> &fn)
{
    if (threads <= 1 || rows < 64) {
        fn(0, rows);
        return;
    }
    int n = (int)std::min<int64_t>(threads, rows);
    std::vector<std::thread> pool;
    int64_t per = (rows + n - 1) / n;
    for (int i = 0; i < n; i++) {
        int64_t a = i * per, b = std::min(rows, a + per);
        if (a >= b) break;
        pool.emplace_back(fn, a, b);
    }
    for (auto &t : pool) t.join();
}

// ------------------------------------------------------------ quantizers
//
// The ggml reference quantizers (ggml-quants.c quantize_row_q8_0_ref,
// quantize_row_q4_0_ref, quantize_row_q5_1_ref), the algorithms the `gguf`
// package restates bit for bit and the reference's fixtures were made with.

static void quant_q8_0(const float *x, uint8_t *y)
{
    float amax = 0.f;
    for (int j = 0; j < 32; j++) amax = std::max(amax, std::fabs(x[j]));
    float d = amax / 127.0f;
    float id = d != 0.f ? 1.0f / d : 0.0f;
    uint16_t dh = float_to_half(d);
    std::memcpy(y, &dh, 2);
    for (int j = 0; j < 32; j++) {
        float v = x[j] * id;
        y[2 + j] = (uint8_t)(int8_t)std::roundf(v);
    }
}

static void quant_q4_0(const float *x, uint8_t *y)
{
    float amax = 0.f, mx = 0.f;
    for (int j = 0; j < 32; j++) {
        float v = x[j];
        if (amax < std::fabs(v)) {
            amax = std::fabs(v);
            mx = v;
        }
    }
    float d = mx / -8.0f;
    float id = d != 0.f ? 1.0f / d : 0.0f;
    uint16_t dh = float_to_half(d);
    std::memcpy(y, &dh, 2);
    for (int j = 0; j < 16; j++) {
        float x0 = x[j] * id, x1 = x[16 + j] * id;
        float a0 = x0 + 8.5f, a1 = x1 + 8.5f;
        int xi0 = std::min(15, (int)(int8_t)a0);
        int xi1 = std::min(15, (int)(int8_t)a1);
        y[2 + j] = (uint8_t)(xi0 | (xi1 << 4));
    }
}

static void quant_q5_1(const float *x, uint8_t *y)
{
    float mn = 3.402823466e+38f, mx = -3.402823466e+38f;
    for (int j = 0; j < 32; j++) {
        if (x[j] < mn) mn = x[j];
        if (x[j] > mx) mx = x[j];
    }
    float d = (mx - mn) / 31.0f;
    float id = d != 0.f ? 1.0f / d : 0.0f;
    uint16_t dh = float_to_half(d), mh = float_to_half(mn);
    std::memcpy(y, &dh, 2);
    std::memcpy(y + 2, &mh, 2);
    uint32_t qh = 0;
    for (int j = 0; j < 16; j++) {
        float x0 = (x[j] - mn) * id, x1 = (x[16 + j] - mn) * id;
        float a0 = x0 + 0.5f, a1 = x1 + 0.5f;
        uint8_t xi0 = (uint8_t)a0, xi1 = (uint8_t)a1;
        y[8 + j] = (uint8_t)((xi0 & 0x0f) | ((xi1 & 0x0f) << 4));
        qh |= ((uint32_t)(xi0 & 0x10u) >> 4) << j;
        qh |= ((uint32_t)(xi1 & 0x10u) >> 4) << (j + 16);
    }
    std::memcpy(y + 4, &qh, 4);
}

static bool quantize_row(int type, const float *x, int64_t count, uint8_t *dst)
{
    int64_t nb = count / 32;
    switch (type) {
    case kF32: std::memcpy(dst, x, (size_t)count * 4); return true;
    case kF16:
        for (int64_t i = 0; i < count; i++) {
            uint16_t hh = float_to_half(x[i]);
            std::memcpy(dst + 2 * i, &hh, 2);
        }
        return true;
    case kQ8_0: for (int64_t b = 0; b < nb; b++) quant_q8_0(x + 32 * b, dst + 34 * b); return true;
    case kQ4_0: for (int64_t b = 0; b < nb; b++) quant_q4_0(x + 32 * b, dst + 18 * b); return true;
    case kQ5_1: for (int64_t b = 0; b < nb; b++) quant_q5_1(x + 32 * b, dst + 24 * b); return true;
    default: return false;
    }
}

// ------------------------------------------------------------ synthetic weights

static inline uint64_t splitmix64(uint64_t z)
{
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// Elements 2p and 2p+1 of the stream: pair p draws one 64-bit counter hash,
// Box-Muller in double; the even element takes the cosine branch.
static inline void normal_pair(uint64_t key, uint64_t p, float &even, float &odd)
{
    uint64_t z = splitmix64(key ^ splitmix64(p));
    double u1 = ((double)(z >> 11) + 0.5) * (1.0 / 9007199254740992.0); // (0,1)
    uint64_t z2 = splitmix64(z);
    double u2 = (double)(z2 >> 11) * (1.0 / 9007199254740992.0);
    double r = std::sqrt(-2.0 * std::log(u1));
    double a = 6.283185307179586 * u2;
    even = (float)(r * std::cos(a));
    odd = (float)(r * std::sin(a));
}

} // namespace jev

using namespace jev;

extern "C" int jev_quantize(int ggml_type, const float *src, int64_t count, void *dst, size_t nbytes)
{
    int bs = block_size(ggml_type);
    if (bs == 0 || count < 0 || count % bs != 0 || !src || !dst) return JEV_EINVAL;
    if ((int64_t)nbytes < row_bytes(ggml_type, count)) return JEV_EINVAL;
    return quantize_row(ggml_type, src, count, (uint8_t *)dst) ? JEV_OK : JEV_EINVAL;
}

extern "C" int jev_synth_tensor(uint64_t seed, uint64_t stream, int ggml_type, int64_t rows, int64_t cols,
                                float stddev, void *dst, size_t nbytes, int threads)
{
    int bs = block_size(ggml_type);
    if (bs == 0 || rows <= 0 || cols <= 0 || cols % bs != 0 || !dst) return JEV_EINVAL;
    int64_t rb = row_bytes(ggml_type, cols);
    if ((int64_t)nbytes < rb * rows) return JEV_EINVAL;
    uint64_t key = splitmix64(seed * 0x100000001b3ull ^ splitmix64(stream + 0x51ed270b27ull));
    uint8_t *out = (uint8_t *)dst;
    parallel_rows(rows, threads, [&](int64_t r0, int64_t r1) {
        std::vector<float> buf((size_t)cols);
        for (int64_t r = r0; r < r1; r++) {
            // cols is a multiple of the block size, so rows hold whole pairs
            // whenever cols is even; an odd F32 row draws its pairs unaligned.
            for (int64_t c = 0; c < cols; c++) {
                uint64_t i = (uint64_t)(r * cols + c);
                float e, o;
                normal_pair(key, i >> 1, e, o);
                if ((i & 1) == 0 && c + 1 < cols) {
                    buf[(size_t)c] = e * stddev;
                    buf[(size_t)c + 1] = o * stddev;
                    c++;
                } else {
                    buf[(size_t)c] = ((i & 1) ? o : e) * stddev;
                }
            }
            quantize_row(ggml_type, buf.data(), cols, out + r * rb);
        }
    });
    return JEV_OK;
}
