// Opt-in integer matmul: the reference's MatMulStrategy.Integer.
//
// Replaces QuantMatMul.ForwardIntegerAsync / RunRowsInteger
// (QuantMatMul.cs:186-287) and IntegerDot (IntegerDot.cs).  Activations are
// quantized per token and 32-block to Q8_0 exactly as
// IntegerDot.QuantizeActivations (IntegerDot.cs:60-96) does; the weights keep
// their quants as 8-bit integers; each block's integer dot runs on the int8
// matrix cores (v_mfma_i32_16x16x32_i8, one quant block per instruction, exact
// int32 sums) and is scaled on the vector ALU in the order of IntegerDot's
// scalar dots (IntegerDot.cs:206-272):
//   total = total + (w_scale * x_scale) * sum_i(w_i * q_i),  blocks ascending,
// and for Q5_1 the offset term of OffsetContribution (:274-279),
// sum_b m_b * (d_b * sum_i q_i), added after the dot.  No K split: one lane
// owns an output for the whole K, so the float order is fixed.
//
// Weight quants come from the tiled layout: Q8_0 bytes (stored biased) get
// their sign bit flipped back; Q4_0 nibbles enter as 0..15 and the integer
// sum is corrected by 8 * sum(q) (exact); Q5_1's 0..31 enter as they are.
#include "jev_dev.h"

namespace jev {

namespace {

typedef int int4v __attribute__((ext_vector_type(4)));

// Operand tiles of the int8 16x16x32 MFMA: row group rg (16 tokens) and block
// b hold 64 lanes x 8 bytes; lane 16 g + r carries token 16 rg + r at
// k = 32 b + 8 g .. + 7.
__device__ __forceinline__ size_t xq_index(int t, int k, int nb)
{
    const int rg = t >> 4, r = t & 15, b = k >> 5, kk = k & 31;
    return (((size_t)rg * nb + b) * 64 + (kk >> 3) * 16 + r) * 8 + (kk & 7);
}

} // namespace

// One 32-lane half-wave per (token, block).  Per-block results are stored
// block-major ([b][t16]) so a lane reads its four output rows with one load.
__global__ __launch_bounds__(256) void quant_act_kernel(QuantActArgs a)
{
    const int nb = a.K >> 5;
    const int id = blockIdx.x * 8 + (threadIdx.x >> 5), i = threadIdx.x & 31;
    if (id >= a.T * nb) return; // whole half-waves; the shuffles stay inside 32 lanes
    const int t = id / nb, b = id % nb;
    const float v = a.x[(size_t)t * a.K + 32 * b + i];
    float mx = fabsf(v);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 32));
    const float d = mx / 127.0f;
    const float inverse = d != 0.0f ? 1.0f / d : 0.0f;
    const float scaled = v * inverse;
    const int q = min(127, max(-127, (int)roundf(scaled))); // roundf: half away from zero
    int s = q;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) s += __shfl_xor(s, o, 32);
    a.xq[xq_index(t, 32 * b + i, nb)] = (int8_t)q;
    if (i == 0) {
        const size_t bi = (size_t)b * a.T16 + t;
        a.xd[bi] = (float)(_Float16)d; // the stored Half scale
        a.xqs[bi] = s;
        a.xs[bi] = d * (float)s; // QuantMatMul's block sums use the float d
    }
}

hipError_t launch_quant_act(const QuantActArgs &a, hipStream_t s)
{
    if (a.T <= 0) return hipSuccess;
    if (a.K <= 0 || a.K % 32 != 0 || a.T16 < ((a.T + 15) & ~15)) return hipErrorInvalidValue;
    const long long halves = (long long)a.T * (a.K >> 5);
    hipLaunchKernelGGL(quant_act_kernel, dim3((unsigned)((halves + 7) / 8)), dim3(256), 0, s, a);
    return hipGetLastError();
}

// Wave w of workgroup (x, y) owns weight row group 4 x + w (16 output
// columns) and the TM token groups from TM y.  No LDS, no barriers.
template <int TYPE, int TM>
__global__ __launch_bounds__(256) void gemm_i8_kernel(GemmI8Args a)
{
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, rl = lane & 15;
    const QWeight &w = a.w;
    const int rgw = blockIdx.x * 4 + wave;
    if (rgw * 16 >= w.rows) return; // wave-uniform
    const int nb = w.cols >> 5, KP = tile_kpairs(w.cols);
    const int tg0 = blockIdx.y * TM;
    const size_t tile0 = (size_t)rgw * KP;

    float acc[TM][4], off[TM][4];
#pragma unroll
    for (int mi = 0; mi < TM; mi++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[mi][r] = off[mi][r] = 0.0f;

    for (int kp = 0; kp < KP; kp++) {
        const size_t tile = tile0 + kp;
        uint32_t wq[2][2]; // [block][dword]: the lane's 8 quants of each block
        float dw[2], mw[2] = {0.0f, 0.0f};
        if (TYPE == kQ8_0) {
            const uint4 q = *(const uint4 *)(w.qs + tile * 1024 + 16 * lane);
            wq[0][0] = q.x ^ 0x80808080u;
            wq[0][1] = q.y ^ 0x80808080u;
            wq[1][0] = q.z ^ 0x80808080u;
            wq[1][1] = q.w ^ 0x80808080u;
        } else {
            const uint2 q = *(const uint2 *)(w.qs + tile * 512 + 8 * lane);
            const uint32_t qh = TYPE == kQ5_1 ? *(const uint16_t *)(w.qh + tile * 128 + 2 * lane) : 0u;
#pragma unroll
            for (int bb = 0; bb < 2; bb++) {
                const uint32_t v = bb ? q.y : q.x;
                uint32_t n0 = v & 0x0f0f0f0fu, n1 = (v >> 4) & 0x0f0f0f0fu;
                if (TYPE == kQ5_1) {
                    const uint32_t hb = (qh >> (8 * bb)) & 0xffu;
                    n0 |= (((hb & 15u) * 0x00204081u) & 0x01010101u) << 4;
                    n1 |= (((hb >> 4) * 0x00204081u) & 0x01010101u) << 4;
                }
                wq[bb][0] = n0;
                wq[bb][1] = n1;
            }
        }
#pragma unroll
        for (int bb = 0; bb < 2; bb++) {
            dw[bb] = h2f(TYPE == kQ5_1 ? w.d[tile * 64 + 4 * rl + bb] : w.d[tile * 32 + 2 * rl + bb]);
            if (TYPE == kQ5_1) mw[bb] = h2f(w.d[tile * 64 + 4 * rl + 2 + bb]);
        }
#pragma unroll
        for (int bb = 0; bb < 2; bb++) {
            const int kb = 2 * kp + bb;
            if (kb >= nb) break; // an odd block count's padding block does not exist
            const long bf = (long)(((uint64_t)wq[bb][1] << 32) | wq[bb][0]);
#pragma unroll
            for (int mi = 0; mi < TM; mi++) {
                const int tg = tg0 + mi;
                const long af = *(const long *)(a.xq + (((size_t)tg * nb + kb) * 64 + lane) * 8);
                const int4v p = __builtin_amdgcn_mfma_i32_16x16x32_i8(af, bf, int4v{0, 0, 0, 0}, 0, 0, 0);
                // this lane's outputs: tokens 16 tg + 4 g + r, column rl
                const size_t bi = (size_t)kb * a.T16 + 16 * tg + 4 * g;
                const float4 xd = *(const float4 *)(a.xd + bi);
                const float xdv[4] = {xd.x, xd.y, xd.z, xd.w};
                int4v xqs = {0, 0, 0, 0};
                if (TYPE == kQ4_0) xqs = *(const int4v *)(a.xqs + bi);
                float4 xs = make_float4(0.f, 0.f, 0.f, 0.f);
                if (TYPE == kQ5_1) xs = *(const float4 *)(a.xs + bi);
                const float xsv[4] = {xs.x, xs.y, xs.z, xs.w};
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int sumi = TYPE == kQ4_0 ? p[r] - 8 * xqs[r] : p[r];
                    const float sc = dw[bb] * xdv[r];
                    acc[mi][r] = acc[mi][r] + sc * (float)sumi;
                    if (TYPE == kQ5_1) off[mi][r] = off[mi][r] + mw[bb] * xsv[r];
                }
            }
        }
    }

    const int col = rgw * 16 + rl;
    if (col >= w.rows) return;
#pragma unroll
    for (int mi = 0; mi < TM; mi++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int t = 16 * (tg0 + mi) + 4 * g + r;
            if (t < a.T) a.y[(size_t)t * a.ldy + col] = TYPE == kQ5_1 ? acc[mi][r] + off[mi][r] : acc[mi][r];
        }
}

template <int TYPE, int TM>
static hipError_t launch_i8_cfg(const GemmI8Args &a, hipStream_t s)
{
    const int groups = (a.T + 15) / 16;
    dim3 grid((a.w.rows + 63) / 64, (groups + TM - 1) / TM);
    hipLaunchKernelGGL((gemm_i8_kernel<TYPE, TM>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int TYPE>
static hipError_t launch_i8_typed(const GemmI8Args &a, hipStream_t s)
{
    // token groups per wave: a divisor of the group count (the padded
    // activation tiles a wave reads always exist), as many as keep at least
    // 1024 workgroups (four waves per SIMD) in flight
    const int groups = (a.T + 15) / 16, cols = (a.w.rows + 63) / 64;
    if (groups % 4 == 0 && cols * (groups / 4) >= 1024) return launch_i8_cfg<TYPE, 4>(a, s);
    if (groups % 2 == 0 && cols * (groups / 2) >= 1024) return launch_i8_cfg<TYPE, 2>(a, s);
    return launch_i8_cfg<TYPE, 1>(a, s);
}

hipError_t launch_gemm_i8(const GemmI8Args &a, hipStream_t s)
{
    if (a.T <= 0) return hipSuccess;
    if (a.w.cols % 32 != 0 || a.T16 < ((a.T + 15) & ~15) || a.ldy < a.w.rows) return hipErrorInvalidValue;
    switch (a.w.type) {
    case kQ8_0: return launch_i8_typed<kQ8_0>(a, s);
    case kQ4_0: return launch_i8_typed<kQ4_0>(a, s);
    case kQ5_1: return launch_i8_typed<kQ5_1>(a, s);
    default: return hipErrorInvalidValue;
    }
}

} // namespace jev
