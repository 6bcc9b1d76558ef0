// One-token GEMV against GGUF-quantized weights: y[r] = dot(x, W[r]).
//
// Replaces QuantMatMul.RunRowsFloat (QuantMatMul.cs:140-176), the path a
// one-token call (decode, the last-position LM head) takes.  The kernel is
// bound by streaming the weights from HBM once, so the design goal is bytes in
// flight, not arithmetic: every lane loads 16 bytes of quants per step
// (coalesced 1 KiB per wave instruction), decodes them in registers and keeps
// fp32 FMA chains; x (fp32) is staged once per workgroup in LDS in a
// lane-interleaved order so the fragment reads are bank-conflict free.
//
// A lane owns one "unit" per step: 16 elements (half a Q8_0 block) or 32 (a
// whole Q4_0 / Q5_1 block).  Its partial dot with the integer quants is scaled
// by the block's d in fp32 (and Q5_1 adds m * sum(x) over the block), then the
// wave reduces with a fixed butterfly.  x is fp32 throughout: the decode path
// carries no fp16 rounding.
#include "jev_dev.h"

namespace jev {

namespace {

constexpr int kRowsPerWave = 4;
constexpr int kWaves = 4;
constexpr int kRowsPerBlock = kRowsPerWave * kWaves;

template <int TYPE>
struct Unit {
    static constexpr int E = TYPE == kQ8_0 ? 16 : 32; // elements per lane-step
    static constexpr int G = E / 4;                   // float4 groups
};

struct alignas(16) u32x4 {
    uint32_t x, y, z, w;
};

// Dot of one unit of row r with the lane's x fragment.
template <int TYPE>
__device__ __forceinline__ float unit_dot(const QWeight &w, int r, int u, const float4 *xf, float xsum)
{
    const int nb = w.cols >> 5;
    if (TYPE == kQ8_0) {
        const u32x4 q = *(const u32x4 *)(w.qs + (size_t)r * w.cols + (size_t)u * 16);
        float d = h2f(w.d[(size_t)r * nb + (u >> 1)]);
        uint32_t wd[4] = {q.x, q.y, q.z, q.w};
        float p = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            float4 xv = xf[g];
            p = fmaf(xv.x, (float)(int8_t)(wd[g]), p);
            p = fmaf(xv.y, (float)(int8_t)(wd[g] >> 8), p);
            p = fmaf(xv.z, (float)(int8_t)(wd[g] >> 16), p);
            p = fmaf(xv.w, (float)(int8_t)(wd[g] >> 24), p);
        }
        return d * p;
    } else {
        const u32x4 q = *(const u32x4 *)(w.qs + (size_t)r * (w.cols >> 1) + (size_t)u * 16);
        size_t blk = (size_t)r * nb + u;
        float d = h2f(w.d[blk]);
        uint32_t wd[4] = {q.x, q.y, q.z, q.w};
        uint32_t qh = TYPE == kQ5_1 ? w.qh[blk] : 0u;
        float p = 0.f;
        // elements 0..15: low nibbles; 16..31: high nibbles.  xf[g] holds
        // elements 4g..4g+3.
#pragma unroll
        for (int g = 0; g < 8; g++) {
            float4 xv = xf[g];
            uint32_t word = wd[g & 3];
            uint32_t nib = g < 4 ? (word & 0x0f0f0f0fu) : ((word >> 4) & 0x0f0f0f0fu);
            if (TYPE == kQ5_1) {
                // bits 4g..4g+3 of qh -> bit 4 of each byte
                uint32_t hb = (qh >> (4 * g)) & 15u;
                uint32_t spread = (hb * 0x00204081u) & 0x01010101u;
                nib |= spread << 4;
            }
            float q0 = (float)(nib & 0xff), q1 = (float)((nib >> 8) & 0xff);
            float q2 = (float)((nib >> 16) & 0xff), q3 = (float)(nib >> 24);
            if (TYPE == kQ4_0) {
                q0 -= 8.f;
                q1 -= 8.f;
                q2 -= 8.f;
                q3 -= 8.f;
            }
            p = fmaf(xv.x, q0, p);
            p = fmaf(xv.y, q1, p);
            p = fmaf(xv.z, q2, p);
            p = fmaf(xv.w, q3, p);
        }
        float r0 = d * p;
        if (TYPE == kQ5_1) r0 = fmaf(h2f(w.m[blk]), xsum, r0);
        return r0;
    }
}

} // namespace

// LDS x layout: unit u = 64 c + l of lane l, group g, element i of the group
// lives at ((c * G + g) * 64 + l) * 4 + i.
template <int TYPE>
__global__ __launch_bounds__(256) void gemv_q_kernel(GemvArgs a, int nrows_total)
{
    extern __shared__ float smem[];
    constexpr int E = Unit<TYPE>::E, G = Unit<TYPE>::G;
    const int K = a.K;
    const int U = K / E;
    const int chunks = (U + 63) / 64;
    float *xs = smem;                       // chunks * G * 64 * 4 floats
    float *bsum = smem + chunks * G * 256;  // Q5_1 block sums, U floats
    for (int i = threadIdx.x; i < K; i += 256) {
        int u = i / E, e = i % E;
        int c = u >> 6, l = u & 63, g = e >> 2, k = e & 3;
        xs[((c * G + g) * 64 + l) * 4 + k] = a.x[i];
    }
    if (TYPE == kQ5_1) {
        __syncthreads();
        for (int u = threadIdx.x; u < U; u += 256) {
            int c = u >> 6, l = u & 63;
            float s = 0.f;
            for (int g = 0; g < G; g++)
                for (int k = 0; k < 4; k++) s += xs[((c * G + g) * 64 + l) * 4 + k];
            bsum[u] = s;
        }
    }
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = blockIdx.x * kRowsPerBlock + wave * kRowsPerWave;
    for (int i = 0; i < kRowsPerWave; i++) {
        int gr = row0 + i; // row over the concatenated outputs
        if (gr >= nrows_total) break;
        // resolve segment
        int s = 0, r = gr;
        if (!a.swiglu) {
            while (s + 1 < a.nseg && r >= a.seg[s].rows) {
                r -= a.seg[s].rows;
                s++;
            }
        }
        float acc = 0.f, acc2 = 0.f;
        for (int c = 0; c < chunks; c++) {
            int u = c * 64 + lane;
            if (u >= U) break;
            const float4 *xf = (const float4 *)(xs + (size_t)(c * G) * 256) + lane;
            float4 xv[G];
#pragma unroll
            for (int g = 0; g < G; g++) xv[g] = xf[g * 64];
            float xsum = TYPE == kQ5_1 ? bsum[u] : 0.f;
            acc += unit_dot<TYPE>(a.seg[s], r, u, xv, xsum);
            if (a.swiglu) acc2 += unit_dot<TYPE>(a.seg[1], r, u, xv, xsum);
        }
        acc = warp_sum(acc);
        if (a.swiglu) {
            acc2 = warp_sum(acc2);
            if (lane == 0) {
                // Kernels.SwiGlu (Kernels.cs:82-89)
                float gu = acc * acc2;
                float e = expf(-acc);
                float sg = 1.0f / (1.0f + e);
                a.y[gr] = sg * gu;
            }
        } else if (lane == 0) {
            a.y[gr] = acc;
        }
    }
}

template <int TYPE>
static hipError_t launch_gemv_typed(const GemvArgs &a, hipStream_t s)
{
    constexpr int E = Unit<TYPE>::E, G = Unit<TYPE>::G;
    int U = a.K / E;
    int chunks = (U + 63) / 64;
    size_t lds = sizeof(float) * ((size_t)chunks * G * 256 + (TYPE == kQ5_1 ? U : 0));
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    int rows = 0;
    if (a.swiglu) rows = a.seg[0].rows;
    else
        for (int i = 0; i < a.nseg; i++) rows += a.seg[i].rows;
    int blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
    hipLaunchKernelGGL(gemv_q_kernel<TYPE>, dim3(blocks), dim3(256), lds, s, a, rows);
    return hipGetLastError();
}

hipError_t launch_gemv(const GemvArgs &a, hipStream_t s)
{
    if (a.K % 32 != 0) return hipErrorInvalidValue;
    for (int i = 0; i < a.nseg; i++)
        if (a.seg[i].type != a.seg[0].type || a.seg[i].cols != a.K) return hipErrorInvalidValue;
    if (a.swiglu && (a.nseg != 2 || a.seg[0].rows != a.seg[1].rows)) return hipErrorInvalidValue;
    switch (a.seg[0].type) {
    case kQ8_0: return launch_gemv_typed<kQ8_0>(a, s);
    case kQ4_0: return launch_gemv_typed<kQ4_0>(a, s);
    case kQ5_1: return launch_gemv_typed<kQ5_1>(a, s);
    default: return hipErrorInvalidValue;
    }
}

} // namespace jev
