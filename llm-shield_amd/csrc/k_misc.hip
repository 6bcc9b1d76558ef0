// Row-wise and small kernels of the token loop: dequantize, embedding gather,
// fused residual-add + RMSNorm, RoPE + KV store, verdict-row head, argmax,
// split-K reduction and KV-arena growth.  All HBM-bound; every reduction has
// a fixed order so results are reproducible bit for bit.
#include "jev_dev.h"

namespace jev {

// ------------------------------------------------------------ dequant / gather

__global__ void dequant_kernel(QWeight w, float *dst)
{
    int r = blockIdx.x;
    for (int k = threadIdx.x; k < w.cols; k += blockDim.x) dst[(size_t)r * w.cols + k] = decode_elem(w, r, k);
}

hipError_t launch_dequant(const QWeight &w, float *dst, hipStream_t s)
{
    if (w.rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(dequant_kernel, dim3(w.rows), dim3(256), 0, s, w, dst);
    return hipGetLastError();
}

// QuantMatMul.GatherRows (QuantMatMul.cs:294-305): ids are validated on the host.
__global__ void gather_kernel(QWeight w, const int32_t *ids, float *h)
{
    int t = blockIdx.x;
    int r = ids[t];
    for (int k = threadIdx.x; k < w.cols; k += blockDim.x) h[(size_t)t * w.cols + k] = decode_elem(w, r, k);
}

hipError_t launch_gather(const QWeight &w, const int32_t *ids, int n, float *h, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(gather_kernel, dim3(n), dim3(256), 0, s, w, ids, h);
    return hipGetLastError();
}

// ------------------------------------------------------------ RMSNorm

// Kernels.RmsNorm (Kernels.cs:25-60) with one wave per row.  Lane l holds
// the 8-element groups g = l + 64 i of the row in registers, so the row is
// read once and every operand-tile store is 16 bytes.  Each lane sums its
// squares in fp32 in group order, a fixed butterfly adds the lanes; then
// scale = 1 / sqrt(sum / n + eps) and y = (x * scale) * w.  With `add`, the
// residual step h += add (Kernels.Add) comes first, where add is the sum of
// `nadd` K-split partials taken in split order.
constexpr int kNormGroups = 16; // groups of 8 per lane: D <= 8192

__global__ __launch_bounds__(64) void rmsnorm_kernel(NormArgs a)
{
    const int t = blockIdx.x, lane = threadIdx.x;
    const int row = a.rows ? a.rows[t] : t;
    const int ng = a.D >> 3, nblk = a.D >> 5;
    float *h = a.h + (size_t)row * a.D;
    const float *add = a.add ? a.add + (size_t)row * a.D : nullptr;
    float x[kNormGroups][8];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kNormGroups; i++) {
        const int g = lane + 64 * i;
        if (64 * i >= ng) break; // uniform: no lane has a group this far
        if (g < ng) {
            float4 v0 = *(const float4 *)(h + 8 * g), v1 = *(const float4 *)(h + 8 * g + 4);
            float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            if (add) {
                float4 p0 = *(const float4 *)(add + 8 * g), p1 = *(const float4 *)(add + 8 * g + 4);
                float s8[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
                for (int z = 1; z < a.nadd; z++) {
                    const float *pz = add + (size_t)z * a.add_stride + 8 * g;
                    float4 q0 = *(const float4 *)pz, q1 = *(const float4 *)(pz + 4);
                    s8[0] = s8[0] + q0.x; s8[1] = s8[1] + q0.y; s8[2] = s8[2] + q0.z; s8[3] = s8[3] + q0.w;
                    s8[4] = s8[4] + q1.x; s8[5] = s8[5] + q1.y; s8[6] = s8[6] + q1.z; s8[7] = s8[7] + q1.w;
                }
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = v[j] + s8[j];
                if (a.store_h) {
                    *(float4 *)(h + 8 * g) = make_float4(v[0], v[1], v[2], v[3]);
                    *(float4 *)(h + 8 * g + 4) = make_float4(v[4], v[5], v[6], v[7]);
                }
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                x[i][j] = v[j];
                float sq = v[j] * v[j];
                ss = ss + sq;
            }
        }
    }
    ss = warp_sum(ss);
    const float scale = 1.0f / sqrtf(ss / (float)a.D + a.eps);
#pragma unroll
    for (int i = 0; i < kNormGroups; i++) {
        const int g = lane + 64 * i;
        if (64 * i >= ng) break;
        float y[8];
        float bsum = 0.f;
        if (g < ng) {
            float4 w0 = *(const float4 *)(a.w + 8 * g), w1 = *(const float4 *)(a.w + 8 * g + 4);
            float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                float v = x[i][j] * scale;
                y[j] = v * w[j];
            }
            if (a.out32) {
                float *o = a.out32 + (size_t)t * a.D + 8 * g;
                *(float4 *)o = make_float4(y[0], y[1], y[2], y[3]);
                *(float4 *)(o + 4) = make_float4(y[4], y[5], y[6], y[7]);
            }
            if (a.ot) {
                uint32_t hv[4], lv[4];
#pragma unroll
                for (int j = 0; j < 8; j += 2) {
                    uint16_t h0, l0, h1, l1;
                    split_f16(y[j], h0, l0);
                    split_f16(y[j + 1], h1, l1);
                    hv[j >> 1] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                    lv[j >> 1] = (uint32_t)l0 | ((uint32_t)l1 << 16);
                    bsum += (h2f(h0) + h2f(l0)) + (h2f(h1) + h2f(l1));
                }
                *(uint4 *)(a.ot + xt_index(t, 8 * g, nblk, 0)) = make_uint4(hv[0], hv[1], hv[2], hv[3]);
                *(uint4 *)(a.ot + xt_index(t, 8 * g, nblk, 1)) = make_uint4(lv[0], lv[1], lv[2], lv[3]);
            }
        }
        if (a.xsum) {
            // per-32 block sums of the (hi + lo) values the GEMM sees: the
            // block's four groups sit on four neighbouring lanes
            bsum = bsum + __shfl_xor(bsum, 1, 64);
            bsum = bsum + __shfl_xor(bsum, 2, 64);
            if (g < ng && (lane & 3) == 0) a.xsum[(size_t)t * nblk + (g >> 2)] = bsum;
        }
    }
}

hipError_t launch_rmsnorm(const NormArgs &a, hipStream_t s)
{
    if (a.T <= 0) return hipSuccess;
    if (a.D % 32 != 0 || a.D > 8 * 64 * kNormGroups || a.nadd < 1) return hipErrorInvalidValue;
    if (a.xsum && !a.ot) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(a.T), dim3(64), 0, s, a);
    return hipGetLastError();
}

__global__ void block_sums_kernel(const uint16_t *xt, int D, float *xsum)
{
    int t = blockIdx.x;
    int nb = D >> 5;
    for (int b = threadIdx.x; b < nb; b += blockDim.x) {
        float s = 0.f;
        for (int j = 0; j < 32; j++) {
            int k = b * 32 + j;
            s += h2f(xt[xt_index(t, k, nb, 0)]) + h2f(xt[xt_index(t, k, nb, 1)]);
        }
        xsum[(size_t)t * nb + b] = s;
    }
}

hipError_t launch_block_sums(const uint16_t *xt, int T, int D, float *xsum, hipStream_t s)
{
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(block_sums_kernel, dim3(T), dim3(128), 0, s, xt, D, xsum);
    return hipGetLastError();
}

// ------------------------------------------------------------ RoPE + KV store

// Rope.Apply (Rope.cs:112-135) for q and k of one token, then
// ApplyPositionScale on q (MinistralModel.cs:676-682); k and v land in their
// cache slots (StoreKeys / StoreValues, :649-669).  cos/sin are computed in
// float from position * freq with the accurate library functions.
__global__ __launch_bounds__(256) void rope_store_kernel(RopeArgs a)
{
    __shared__ float cs[512], sn[512];
    int t = blockIdx.x;
    int pos = a.pos ? a.pos[t] : a.start + t;
    int slot = a.slot ? a.slot[t] : a.start + t;
    for (int i = threadIdx.x; i < a.half; i += 256) {
        float theta = (float)pos * a.freqs[i];
        cs[i] = cosf(theta) * a.mscale;
        sn[i] = sinf(theta) * a.mscale;
    }
    __syncthreads();
    float qscale = 1.f;
    bool scaled = false;
    if (a.orig_ctx > 0 && a.temp_scale != 0.f) {
        float interval = floorf((float)pos / (float)a.orig_ctx);
        if (interval != 0.f) {
            qscale = 1.f + a.temp_scale * logf(1.f + interval);
            scaled = true;
        }
    }
    int qdim = a.n_heads * a.hd, kvdim = a.n_kv * a.hd;
    const float *qi = a.q_in + (size_t)t * a.ld_in;
    const float *ki = a.k_in + (size_t)t * a.ld_in;
    const float *vi = a.v_in + (size_t)t * a.ld_in;
    // K-split partials of the projection, summed in split order
    auto in2 = [&](const float *p, int k, float &x0, float &x1) {
        float2 v = *(const float2 *)(p + k);
        for (int z = 1; z < a.nin; z++) {
            float2 u = *(const float2 *)(p + (size_t)z * a.in_stride + k);
            v.x = v.x + u.x;
            v.y = v.y + u.y;
        }
        x0 = v.x;
        x1 = v.y;
    };
    float *qo = a.q_out + (size_t)t * qdim;
    int hpairs = a.hd >> 1;
    for (int p = threadIdx.x; p < (qdim >> 1); p += 256) {
        int i = p % hpairs;
        float x0, x1;
        in2(qi, 2 * p, x0, x1);
        float o0 = x0, o1 = x1;
        if (i < a.half) {
            float c = cs[i], sv = sn[i];
            float m0 = x0 * c, m1 = x1 * sv, m2 = x0 * sv, m3 = x1 * c;
            o0 = m0 - m1;
            o1 = m2 + m3;
        }
        if (scaled) {
            o0 = o0 * qscale;
            o1 = o1 * qscale;
        }
        qo[2 * p] = o0;
        qo[2 * p + 1] = o1;
    }
    for (int p = threadIdx.x; p < (kvdim >> 1); p += 256) {
        int i = p % hpairs;
        int h = (2 * p) / a.hd, d = (2 * p) % a.hd;
        float x0, x1;
        in2(ki, 2 * p, x0, x1);
        float o0 = x0, o1 = x1;
        if (i < a.half) {
            float c = cs[i], sv = sn[i];
            float m0 = x0 * c, m1 = x1 * sv, m2 = x0 * sv, m3 = x1 * c;
            o0 = m0 - m1;
            o1 = m2 + m3;
        }
        float *kd = a.kc + ((size_t)h * a.cap + slot) * a.hd + d;
        kd[0] = o0;
        kd[1] = o1;
        float *vd = a.vc + ((size_t)h * a.cap + slot) * a.hd + d;
        float v0, v1;
        in2(vi, 2 * p, v0, v1);
        vd[0] = v0;
        vd[1] = v1;
    }
}

hipError_t launch_rope_store(const RopeArgs &a, hipStream_t s)
{
    if (a.T <= 0) return hipSuccess;
    hipLaunchKernelGGL(rope_store_kernel, dim3(a.T), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ------------------------------------------------------------ verdict-row head

// One wave per (output, selected row): the decoded row dotted with the
// normalised output state (MinistralModel.cs:386-410), lane-strided fp32 FMA
// chains reduced by a fixed butterfly.
__global__ __launch_bounds__(64) void head_rows_kernel(HeadRowsArgs a)
{
    int b = blockIdx.x, i = blockIdx.y;
    int r = a.rows[i];
    const float *x = a.xn + (size_t)b * a.D;
    float acc = 0.f;
    for (int k = threadIdx.x; k < a.D; k += 64) acc = fmaf(x[k], decode_elem(a.table, r, k), acc);
    acc = warp_sum(acc);
    if (threadIdx.x == 0) a.out[(size_t)b * a.n_rows + i] = acc;
}

hipError_t launch_head_rows(const HeadRowsArgs &a, hipStream_t s)
{
    if (a.n_out <= 0 || a.n_rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(head_rows_kernel, dim3(a.n_out, a.n_rows), dim3(64), 0, s, a);
    return hipGetLastError();
}

// ------------------------------------------------------------ argmax

// Kernels.ArgMax (Kernels.cs:146): index of the largest element, lowest index
// on ties.  Pass 1: one (value, index) per block; pass 2: one block over those.
__device__ __forceinline__ void better(float &v, int &i, float v2, int i2)
{
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

// xi == nullptr: candidates are x[k] at index k; otherwise (x[k], xi[k]) pairs
// from the first pass.
__global__ __launch_bounds__(256) void argmax_kernel(const float *x, const int32_t *xi, int n, float *ov, int32_t *oi)
{
    __shared__ float sv[256];
    __shared__ int si[256];
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int k = blockIdx.x * 256 + threadIdx.x; k < n; k += gridDim.x * 256) better(v, idx, x[k], xi ? xi[k] : k);
    sv[threadIdx.x] = v;
    si[threadIdx.x] = idx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o) {
            float v2 = sv[threadIdx.x + o];
            int i2 = si[threadIdx.x + o];
            float v1 = sv[threadIdx.x];
            int i1 = si[threadIdx.x];
            better(v1, i1, v2, i2);
            sv[threadIdx.x] = v1;
            si[threadIdx.x] = i1;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        ov[blockIdx.x] = sv[0];
        oi[blockIdx.x] = si[0];
    }
}

hipError_t launch_argmax(const float *x, int n, int32_t *result, float *sv, int32_t *si, hipStream_t s)
{
    const int blocks = 256;
    hipLaunchKernelGGL(argmax_kernel, dim3(blocks), dim3(256), 0, s, x, (const int32_t *)nullptr, n, sv, si);
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(256), 0, s, (const float *)sv, (const int32_t *)si, blocks,
                       sv + blocks, si + blocks);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return hipMemcpyAsync(result, si + blocks, sizeof(int32_t), hipMemcpyDeviceToDevice, s);
}

// ------------------------------------------------------------ fp32 -> fp16 pair

__global__ void split_kernel(const float *x, int T, int D, uint16_t *xt)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)T * D) return;
    int t = (int)(i / D), k = (int)(i % D);
    uint16_t a, b;
    split_f16(x[i], a, b);
    xt[xt_index(t, k, D >> 5, 0)] = a;
    xt[xt_index(t, k, D >> 5, 1)] = b;
}

hipError_t launch_split(const float *x, int T, int D, uint16_t *xt, hipStream_t s)
{
    size_t n = (size_t)T * D;
    if (n == 0) return hipSuccess;
    if (D % 32 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(split_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, T, D, xt);
    return hipGetLastError();
}

// ------------------------------------------------------------ split-K reduce

__global__ void reduce_partials_kernel(const float *p, int ksplit, size_t mn, float *y)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= mn) return;
    float s = p[i];
    for (int z = 1; z < ksplit; z++) s = s + p[(size_t)z * mn + i];
    y[i] = s;
}

hipError_t launch_reduce_partials(const float *partial, int ksplit, int M, int N, float *y, hipStream_t s)
{
    size_t mn = (size_t)M * N;
    if (mn == 0) return hipSuccess;
    hipLaunchKernelGGL(reduce_partials_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, partial, ksplit, mn, y);
    return hipGetLastError();
}

// ------------------------------------------------------------ KV growth

__global__ void kv_copy_kernel(const float *src, float *dst, int old_cap, int new_cap, int len, int hd)
{
    int h = blockIdx.y;
    size_t n = (size_t)len * hd;
    const float *s = src + (size_t)h * old_cap * hd;
    float *d = dst + (size_t)h * new_cap * hd;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) d[i] = s[i];
}

hipError_t launch_kv_copy(const float *src, float *dst, int heads_total, int old_cap, int new_cap, int len, int hd,
                          hipStream_t s)
{
    if (len <= 0 || heads_total <= 0) return hipSuccess;
    hipLaunchKernelGGL(kv_copy_kernel, dim3(64, heads_total), dim3(256), 0, s, src, dst, old_cap, new_cap, len, hd);
    return hipGetLastError();
}

} // namespace jev
