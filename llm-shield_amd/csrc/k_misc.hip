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
// A thread decodes 8 consecutive elements -- one lane slot of a tile, so one
// load of their quants and one of the block scale -- with decode_elem's
// arithmetic per element.
__global__ __launch_bounds__(256) void gather_kernel(QWeight w, const int32_t *ids, float *h)
{
    const int t = blockIdx.x, row = ids[t];
    const int rg = row >> 4, r = row & 15, kp = tile_kpairs(w.cols), ng = w.cols >> 3;
    for (int j = threadIdx.x; j < ng; j += 256) {
        const int k = 8 * j, b = k >> 5, bb = b & 1, l = 16 * ((k & 31) >> 3) + r;
        const size_t tile = (size_t)rg * kp + (b >> 1);
        float v[8];
        if (w.type == kQ8_0) {
            const float d = h2f(w.d[tile * 32 + 2 * r + bb]);
            const uint2 q = *(const uint2 *)(w.qs + tile * 1024 + 16 * l + 8 * bb);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int qi = (int)(((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xffu) - 128; // stored biased
                v[i] = (float)qi * d;
            }
        } else {
            const uint32_t q = *(const uint32_t *)(w.qs + tile * 512 + 8 * l + 4 * bb);
            if (w.type == kQ4_0) {
                const float d = h2f(w.d[tile * 32 + 2 * r + bb]);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const int nib = (int)((q >> (8 * (i & 3) + (i < 4 ? 0 : 4))) & 15u);
                    v[i] = d * (float)(nib - 8);
                }
            } else {
                const float d = h2f(w.d[tile * 64 + 4 * r + bb]), m = h2f(w.d[tile * 64 + 4 * r + 2 + bb]);
                const uint32_t qh = w.qh[tile * 128 + 2 * l + bb];
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const int nib = (int)((q >> (8 * (i & 3) + (i < 4 ? 0 : 4))) & 15u);
                    const int qi = nib | (int)(((qh >> i) & 1u) << 4);
                    const float dq = d * (float)qi;
                    v[i] = dq + m;
                }
            }
        }
        float4 *o = (float4 *)(h + (size_t)t * w.cols + k);
        o[0] = make_float4(v[0], v[1], v[2], v[3]);
        o[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

hipError_t launch_gather(const QWeight &w, const int32_t *ids, int n, float *h, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(gather_kernel, dim3(n), dim3(256), 0, s, w, ids, h);
    return hipGetLastError();
}

// ------------------------------------------------------------ RMSNorm

// Kernels.RmsNorm (Kernels.cs:25-60), one workgroup per row.  Thread t
// owns the float4 groups g = t + 256 i of the row; every load of the row (h
// and the K-split partials of `add`) is issued before the first use, so a row
// costs one memory round trip.  Squares are summed per thread in group order,
// then by a fixed butterfly per wave and the four wave sums in order;
// scale = 1 / sqrt(sum / n + eps) and y = (x * scale) * w.  With `add`, the
// residual step h += add (Kernels.Add) comes first, where add is the sum of
// `nadd` partials taken in split order.
constexpr int kNormIters = 8;   // float4 groups per thread: D <= 8192
constexpr int kNormParts = 4;   // K-split partials

// NI: float4 groups per thread for this D (the registers of the loads in
// flight are sized for it; 3 for D = 3072).
// Row of workgroup L: workgroups go to the eight XCDs round robin (L % 8),
// and the 16 rows of an operand tile share its cache lines, so within each
// full 128 rows the 16 rows of a tile are given to workgroups of one XCD
// (its L2 then holds whole lines); rows past the last full 128 map to
// themselves.
__device__ __forceinline__ int norm_row(int L, int T)
{
    if (L >= (T & ~127)) return L;
    const int x = L & 7, j = L >> 3;
    return (j & 15) + 16 * ((j >> 4) * 8 + x);
}

template <int NI, int NT = 256>
__global__ __launch_bounds__(NT) void rmsnorm_kernel(NormArgs a)
{
    constexpr int kNormIters = NI;
    __shared__ float wsum[NT / 64];
    const int t = norm_row(blockIdx.x, a.T), tid = threadIdx.x;
    const int row = a.rows ? a.rows[t] : t;
    const int ng = a.D >> 2, nblk = a.D >> 5;
    float4 *h4 = (float4 *)(a.h + (size_t)row * a.D);
    const float4 *add4 = a.add ? (const float4 *)(a.add + (size_t)row * a.D) : nullptr;
    float4 x[kNormIters], wv[kNormIters];
    const float4 *w4 = (const float4 *)a.w;
#pragma unroll
    for (int i = 0; i < kNormIters; i++) {
        if (NT * i >= ng) break;
        wv[i] = w4[min(tid + NT * i, ng - 1)]; // clamped: out-of-row lanes load and drop
    }
    const float scale = row_rms_scale<kNormIters, kNormParts, NT>(h4, add4, a.nadd, a.add_stride >> 2, a.D, a.eps, x, wsum);
    if (add4 && a.store_h) {
#pragma unroll
        for (int i = 0; i < kNormIters; i++) {
            if (NT * i >= ng) break;
            if (tid + NT * i < ng) h4[tid + NT * i] = x[i];
        }
    }
#pragma unroll
    for (int i = 0; i < kNormIters; i++) {
        if (NT * i >= ng) break;
        const int g = tid + NT * i;
        const bool own = g < ng;
        const float4 w = wv[i];
        float y[4] = {(x[i].x * scale) * w.x, (x[i].y * scale) * w.y, (x[i].z * scale) * w.z, (x[i].w * scale) * w.w};
        if (a.out32 && own) *(float4 *)(a.out32 + (size_t)t * a.D + 4 * g) = make_float4(y[0], y[1], y[2], y[3]);
        if (a.ot) {
            uint16_t hh[4], ll[4];
            float bsum = 0.f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                split_f16(y[j], hh[j], ll[j]);
                bsum += h2f(hh[j]) + h2f(ll[j]);
            }
            if (own) {
                *(uint2 *)(a.ot + xt_index(t, 4 * g, nblk, 0)) =
                    make_uint2((uint32_t)hh[0] | ((uint32_t)hh[1] << 16), (uint32_t)hh[2] | ((uint32_t)hh[3] << 16));
                *(uint2 *)(a.ot + xt_index(t, 4 * g, nblk, 1)) =
                    make_uint2((uint32_t)ll[0] | ((uint32_t)ll[1] << 16), (uint32_t)ll[2] | ((uint32_t)ll[3] << 16));
            }
            if (a.xsum) {
                // per-32 block sums of the (hi + lo) values the GEMM sees: a
                // block's eight groups sit on eight neighbouring lanes
                bsum = bsum + __shfl_xor(bsum, 1, 64);
                bsum = bsum + __shfl_xor(bsum, 2, 64);
                bsum = bsum + __shfl_xor(bsum, 4, 64);
                if (own && (tid & 7) == 0) a.xsum[(size_t)t * nblk + (g >> 3)] = bsum;
            }
        }
    }
}

hipError_t launch_rmsnorm(const NormArgs &a, hipStream_t s)
{
    if (a.T <= 0) return hipSuccess;
    if (a.D % 32 != 0 || a.D > 4 * 256 * kNormIters || a.nadd < 1 || a.nadd > kNormParts) return hipErrorInvalidValue;
    if (a.xsum && !a.ot) return hipErrorInvalidValue;
    // The per-layer norms of a one-token pass (one row, no row list, no
    // operand tiles: the one-token GEMV reads fp32): 1024 threads, a quarter
    // of the serial work per thread on the latency path.  Their reduction
    // order is their own; a single token already takes the one-token GEMV
    // rather than the batched arithmetic.  The head norm (a row list) keeps
    // one order for any number of outputs, so a tree's verdicts still equal
    // its branches run alone bit for bit.
    if (a.T == 1 && !a.rows && !a.ot && a.D <= 4 * 1024) {
        hipLaunchKernelGGL((rmsnorm_kernel<1, 1024>), dim3(1), dim3(1024), 0, s, a);
        return hipGetLastError();
    }
    switch ((a.D / 4 + 255) / 256) {
    case 1: hipLaunchKernelGGL(rmsnorm_kernel<1>, dim3(a.T), dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL(rmsnorm_kernel<2>, dim3(a.T), dim3(256), 0, s, a); break;
    case 3: hipLaunchKernelGGL(rmsnorm_kernel<3>, dim3(a.T), dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL(rmsnorm_kernel<4>, dim3(a.T), dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(rmsnorm_kernel<kNormIters>, dim3(a.T), dim3(256), 0, s, a); break;
    }
    return hipGetLastError();
}

// Q5_1 block sums of an operand tile buffer: per row t and 32-block b, the
// sum of (hi + lo) over the block's 32 values in ascending k -- the term the
// Q5_1 min multiplies.  One thread per (row, block); the block's hi and lo
// parts are four 16-byte slots each (slot q holds k = 8 q .. 8 q + 7), and the
// 16 rows of a row group are neighbouring threads, so each slot load is a
// contiguous 256 bytes across them.
__global__ __launch_bounds__(256) void block_sums_kernel(const uint16_t *xt, int T, int nb, float *xsum)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int r = i & 15, gb = i >> 4; // gb = row group * nb + block
    const int rg = gb / nb, b = gb - rg * nb;
    const int t = rg * 16 + r;
    if (t >= T) return;
    const uint4 *base = (const uint4 *)xt + (size_t)gb * 2 * 64 + r;
    uint4 h[4], l[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        h[q] = base[16 * q];
        l[q] = base[64 + 16 * q];
    }
    float sum = 0.f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint32_t hw[4] = {h[q].x, h[q].y, h[q].z, h[q].w}, lw[4] = {l[q].x, l[q].y, l[q].z, l[q].w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint16_t hv = (uint16_t)(hw[e >> 1] >> (16 * (e & 1))), lv = (uint16_t)(lw[e >> 1] >> (16 * (e & 1)));
            sum += h2f(hv) + h2f(lv);
        }
    }
    xsum[(size_t)t * nb + b] = sum;
}

hipError_t launch_block_sums(const uint16_t *xt, int T, int D, float *xsum, hipStream_t s)
{
    if (T <= 0) return hipSuccess;
    if (D % 32 != 0) return hipErrorInvalidValue;
    const int nb = D >> 5;
    const long threads = (long)((T + 15) / 16) * nb * 16;
    hipLaunchKernelGGL(block_sums_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, xt, T, nb, xsum);
    return hipGetLastError();
}

// ------------------------------------------------------------ RoPE + KV store

// Rope.Apply (Rope.cs:112-135) for q and k of one token, then
// ApplyPositionScale on q (MinistralModel.cs:676-682); k and v land in their
// cache slots (StoreKeys / StoreValues, :649-669).  cos/sin are computed in
// float from position * freq with the accurate library functions.  A token's
// pairs are shared by gridDim.y workgroups when there are few tokens (every
// element is independent, so the split changes no result).
constexpr int kRopeIters = 16; // q pairs per thread: q dims <= 8192
constexpr int kRopeKv = 4;     // k / v pairs per thread: kv dims <= 2048
constexpr int kRopeParts = 4;  // K-split partials of the projection

__global__ __launch_bounds__(256) void rope_store_kernel(RopeArgs a)
{
    __shared__ float cs[512], sn[512];
    const int t = blockIdx.x, tid = threadIdx.x;
    const int start = a.start_dev ? *a.start_dev : a.start;
    const int pos = a.pos ? a.pos[t] : start + t;
    const int slot = a.slot ? a.slot[t] : start + t;
    const int qdim = a.n_heads * a.hd, kvdim = a.n_kv * a.hd;
    const int nq_all = qdim >> 1, nkv_all = kvdim >> 1, hpairs = a.hd >> 1;
    // this workgroup's share of the token's q pairs [q0, q0 + nq) and k / v
    // pairs [k0, k0 + nkv) (gridDim.y workgroups per token)
    const int qper = (nq_all + gridDim.y - 1) / gridDim.y, kper = (nkv_all + gridDim.y - 1) / gridDim.y;
    const int q0 = min(nq_all, (int)blockIdx.y * qper), k0 = min(nkv_all, (int)blockIdx.y * kper);
    const int nq = min(nq_all - q0, qper), nkv = min(nkv_all - k0, kper);
    const float2 *qi = (const float2 *)(a.q_in + (size_t)t * a.ld_in) + q0;
    const float2 *ki = (const float2 *)(a.k_in + (size_t)t * a.ld_in) + k0;
    const float2 *vi = (const float2 *)(a.v_in + (size_t)t * a.ld_in) + k0;
    const size_t zs = a.in_stride >> 1;
    // every load first (clamped indices; lanes past the end drop their value),
    // the K-split partials summed in split order afterwards
    float2 qv[kRopeIters], kv[kRopeKv], vv[kRopeKv];
#pragma unroll
    for (int i = 0; i < kRopeIters; i++) {
        if (256 * i >= nq) continue;
        qv[i] = qi[min(tid + 256 * i, nq - 1)];
    }
#pragma unroll
    for (int i = 0; i < kRopeKv; i++) {
        if (256 * i >= nkv) continue;
        kv[i] = ki[min(tid + 256 * i, nkv - 1)];
        vv[i] = vi[min(tid + 256 * i, nkv - 1)];
    }
#pragma unroll
    for (int z = 1; z < kRopeParts; z++) {
        if (z >= a.nin) continue;
        float2 uq[kRopeIters], uk[kRopeKv], uv[kRopeKv];
#pragma unroll
        for (int i = 0; i < kRopeIters; i++) {
            if (256 * i >= nq) continue;
            uq[i] = qi[z * zs + min(tid + 256 * i, nq - 1)];
        }
#pragma unroll
        for (int i = 0; i < kRopeKv; i++) {
            if (256 * i >= nkv) continue;
            uk[i] = ki[z * zs + min(tid + 256 * i, nkv - 1)];
            uv[i] = vi[z * zs + min(tid + 256 * i, nkv - 1)];
        }
#pragma unroll
        for (int i = 0; i < kRopeIters; i++) {
            if (256 * i >= nq) continue;
            qv[i].x = qv[i].x + uq[i].x;
            qv[i].y = qv[i].y + uq[i].y;
        }
#pragma unroll
        for (int i = 0; i < kRopeKv; i++) {
            if (256 * i >= nkv) continue;
            kv[i].x = kv[i].x + uk[i].x;
            kv[i].y = kv[i].y + uk[i].y;
            vv[i].x = vv[i].x + uv[i].x;
            vv[i].y = vv[i].y + uv[i].y;
        }
    }
    for (int i = tid; i < a.half; i += 256) {
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
    float2 *qo = (float2 *)(a.q_out + (size_t)t * qdim) + q0;
#pragma unroll
    for (int it = 0; it < kRopeIters; it++) {
        if (256 * it >= nq) continue;
        const int p = tid + 256 * it;  // within the share
        const int i = (q0 + p) % hpairs;
        float x0 = qv[it].x, x1 = qv[it].y;
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
        if (p < nq) qo[p] = make_float2(o0, o1);
    }
#pragma unroll
    for (int it = 0; it < kRopeKv; it++) {
        if (256 * it >= nkv) continue;
        const int p = tid + 256 * it; // within the share
        if (p < nkv) {
        const int pg = k0 + p;
        const int i = pg % hpairs;
        const int h = (2 * pg) / a.hd, d = (2 * pg) % a.hd;
        float x0 = kv[it].x, x1 = kv[it].y;
        float o0 = x0, o1 = x1;
        if (i < a.half) {
            float c = cs[i], sv = sn[i];
            float m0 = x0 * c, m1 = x1 * sv, m2 = x0 * sv, m3 = x1 * c;
            o0 = m0 - m1;
            o1 = m2 + m3;
        }
        const size_t row = (size_t)h * a.cap + slot;
        *(float2 *)(a.kc + row * a.hd + d) = make_float2(o0, o1);
        *(float2 *)(a.vc + row * a.hd + d) = vv[it];
        // the pair shadows the attention kernel stages from
        uint32_t hv, lv;
        split2_rtz(o0, o1, hv, lv);
        *(uint32_t *)(a.kp + (row * 2 + 0) * a.hd + d) = hv;
        *(uint32_t *)(a.kp + (row * 2 + 1) * a.hd + d) = lv;
        split2_rtz(vv[it].x, vv[it].y, hv, lv);
        *(uint32_t *)(a.vp + (row * 2 + 0) * a.hd + d) = hv;
        *(uint32_t *)(a.vp + (row * 2 + 1) * a.hd + d) = lv;
        }
    }
}

hipError_t launch_rope_store(const RopeArgs &a, hipStream_t s)
{
    if (a.T <= 0) return hipSuccess;
    if (a.n_heads * a.hd > 512 * kRopeIters || a.n_kv * a.hd > 512 * kRopeKv || a.nin < 1 || a.nin > kRopeParts ||
        a.half > 512 || a.hd % 2 != 0 || !a.kp || !a.vp)
        return hipErrorInvalidValue;
    // few tokens: several workgroups per token share its heads, ~512
    // workgroups in all (measured at 256 tokens: 2 per token ahead of 1, 4, 8)
    const int split = a.T >= 512 ? 1 : std::min(8, 512 / a.T);
    hipLaunchKernelGGL(rope_store_kernel, dim3(a.T, split), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ------------------------------------------------------------ verdict-row head

// One wave per (output, selected row): the decoded row dotted with the
// normalised output state (MinistralModel.cs:386-410), lane-strided fp32 FMA
// chains reduced by a fixed butterfly.  Each lane's elements are taken eight
// at a time, their loads (the state and the weight element's quant and scale)
// all issued before the eight FMAs, which run in the chain's order.
template <int TYPE>
__global__ __launch_bounds__(64) void head_rows_kernel(HeadRowsArgs a)
{
    int b = blockIdx.x, i = blockIdx.y;
    int r = a.rows[i];
    const float *x = a.xn + (size_t)b * a.D;
    float acc = 0.f;
    constexpr int B = 8;
    for (int k0 = threadIdx.x; k0 < a.D; k0 += 64 * B) {
        float xv[B], wv[B];
#pragma unroll
        for (int j = 0; j < B; j++) {
            const int k = min(k0 + 64 * j, a.D - 1); // clamped: unused copies
            xv[j] = x[k];
            wv[j] = decode_elem<TYPE>(a.table, r, k);
        }
#pragma unroll
        for (int j = 0; j < B; j++)
            if (k0 + 64 * j < a.D) acc = fmaf(xv[j], wv[j], acc);
    }
    acc = warp_sum(acc);
    if (threadIdx.x == 0) a.out[(size_t)b * a.n_rows + i] = acc;
}

hipError_t launch_head_rows(const HeadRowsArgs &a, hipStream_t s)
{
    if (a.n_out <= 0 || a.n_rows <= 0) return hipSuccess;
    const dim3 grid(a.n_out, a.n_rows);
    switch (a.table.type) {
    case kQ8_0: hipLaunchKernelGGL(head_rows_kernel<kQ8_0>, grid, dim3(64), 0, s, a); break;
    case kQ4_0: hipLaunchKernelGGL(head_rows_kernel<kQ4_0>, grid, dim3(64), 0, s, a); break;
    case kQ5_1: hipLaunchKernelGGL(head_rows_kernel<kQ5_1>, grid, dim3(64), 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ------------------------------------------------------------ argmax

// Kernels.ArgMax (Kernels.cs:146) is TensorPrimitives.IndexOfMax: the first
// NaN if there is one, else the largest element with +0 above -0, lowest
// index on ties.  better() is that order as a reduction step, so any
// reduction tree gives the same index, and the index is always in range.
// Pass 1: one (value, index) per block; pass 2: one block over those.
__device__ __forceinline__ void better(float &v, int &i, float v2, int i2)
{
    bool take;
    if (v2 != v2) take = v == v || i2 < i;
    else if (v != v) take = false;
    else if (v2 != v) take = v2 > v;
    else if (v2 == 0.f && signbit(v2) != signbit(v)) take = !signbit(v2);
    else take = i2 < i;
    if (take) {
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
    // four candidates' loads in flight per thread, then their comparisons
    // (better() is a total order: the order taken does not change the result)
    const int stride = gridDim.x * 256;
    for (int k0 = blockIdx.x * 256 + threadIdx.x; k0 < n; k0 += 4 * stride) {
        float cv[4];
        int ci[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int k = min(k0 + j * stride, n - 1); // clamped: unused copies
            cv[j] = x[k];
            ci[j] = xi ? xi[k] : k;
        }
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (k0 + j * stride < n) better(v, idx, cv[j], ci[j]);
    }
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

__global__ __launch_bounds__(256) void argmax_decode_kernel(const float *sv, const int32_t *si, int n, int32_t *state,
                                                            int32_t *out)
{
    __shared__ float bv[256];
    __shared__ int bi[256];
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int k = threadIdx.x; k < n; k += 256) better(v, idx, sv[k], si[k]);
    bv[threadIdx.x] = v;
    bi[threadIdx.x] = idx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o) {
            float v1 = bv[threadIdx.x];
            int i1 = bi[threadIdx.x];
            better(v1, i1, bv[threadIdx.x + o], bi[threadIdx.x + o]);
            bv[threadIdx.x] = v1;
            bi[threadIdx.x] = i1;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int tok = bi[0];
        out[state[1]] = tok;
        state[2] = tok;
        state[1] = state[1] + 1;
        state[0] = state[0] + 1;
    }
}

hipError_t launch_argmax_decode(const float *x, int n, float *sv, int32_t *si, int32_t *state, int32_t *out,
                                hipStream_t s)
{
    const int blocks = 256;
    hipLaunchKernelGGL(argmax_kernel, dim3(blocks), dim3(256), 0, s, x, (const int32_t *)nullptr, n, sv, si);
    hipLaunchKernelGGL(argmax_decode_kernel, dim3(1), dim3(256), 0, s, (const float *)sv, (const int32_t *)si, blocks,
                       state, out);
    return hipGetLastError();
}

// One greedy step of the rows layout (ReasoningDecider.cs:157-178): row r's
// argmax over its logits (lowest index on ties, Kernels.ArgMax) becomes its
// next input token and is recorded at out[rowstep[r] * n_rows + r]; the
// row's cache slot and position advance by one.  Each workgroup owns one row,
// so no two touch the same state.
__global__ __launch_bounds__(256) void rows_step_kernel(const float *logits, int vocab, int n_rows, int32_t *tokens,
                                                       int32_t *slot, int32_t *pos, int32_t *rowstep, int32_t *out)
{
    __shared__ float bv[256];
    __shared__ int bi[256];
    const int r = blockIdx.x;
    const float *x = logits + (size_t)r * vocab;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    // eight 16-byte loads in flight per thread, then their elements in
    // turn (one row per workgroup: a load-then-compare chain per element
    // would wait on memory once per element); better() is a total order, so
    // the order elements are taken in does not change the result
    const int n4 = vocab % 4 == 0 && ((uintptr_t)x & 15) == 0 ? vocab / 4 : 0;
    const float4 *x4 = (const float4 *)x;
    constexpr int B = 8;
    for (int base = 0; base < n4; base += 256 * B) {
        float4 c[B];
#pragma unroll
        for (int j = 0; j < B; j++) c[j] = x4[min(base + 256 * j + (int)threadIdx.x, n4 - 1)]; // clamped: unused copies
#pragma unroll
        for (int j = 0; j < B; j++) {
            const int e = base + 256 * j + threadIdx.x;
            if (e < n4) {
                better(v, idx, c[j].x, 4 * e);
                better(v, idx, c[j].y, 4 * e + 1);
                better(v, idx, c[j].z, 4 * e + 2);
                better(v, idx, c[j].w, 4 * e + 3);
            }
        }
    }
    for (int k = 4 * n4 + threadIdx.x; k < vocab; k += 256) better(v, idx, x[k], k);
    bv[threadIdx.x] = v;
    bi[threadIdx.x] = idx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o) {
            float v1 = bv[threadIdx.x];
            int i1 = bi[threadIdx.x];
            better(v1, i1, bv[threadIdx.x + o], bi[threadIdx.x + o]);
            bv[threadIdx.x] = v1;
            bi[threadIdx.x] = i1;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int tok = bi[0];
        tokens[r] = tok;
        out[(size_t)rowstep[r] * n_rows + r] = tok;
        rowstep[r] = rowstep[r] + 1;
        slot[r] = slot[r] + 1;
        pos[r] = pos[r] + 1;
    }
}

hipError_t launch_rows_step(const float *logits, int vocab, int n_rows, int32_t *tokens, int32_t *slot, int32_t *pos,
                            int32_t *rowstep, int32_t *out, hipStream_t s)
{
    if (n_rows <= 0 || vocab <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rows_step_kernel, dim3(n_rows), dim3(256), 0, s, logits, vocab, n_rows, tokens, slot, pos, rowstep,
                       out);
    return hipGetLastError();
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

// The same split in the tiles' lane order: one wave per (16-row group, quant
// block) tile, lane l taking row l % 16 and k = 8 (l / 16) .. + 7 -- two
// 16-byte loads, and one contiguous 1 KiB store per part for the wave.  Rows
// past T (the tile's padding) are written as zeros.  x 16-byte aligned.
__global__ __launch_bounds__(256) void split_tile_kernel(const float *x, int T, int D, uint16_t *xt)
{
    const int nblk = D >> 5, lane = threadIdx.x & 63;
    const int tile = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (tile >= ((T + 15) >> 4) * nblk) return;
    const int t = (tile / nblk) * 16 + (lane & 15), k = (tile % nblk) * 32 + 8 * (lane >> 4);
    float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
    if (t < T) {
        const float4 *xp = (const float4 *)(x + (size_t)t * D + k);
        v0 = xp[0];
        v1 = xp[1];
    }
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        uint16_t h0, l0, h1, l1;
        split_f16(v[j], h0, l0);
        split_f16(v[j + 1], h1, l1);
        hw[j >> 1] = (uint32_t)h0 | ((uint32_t)h1 << 16);
        lw[j >> 1] = (uint32_t)l0 | ((uint32_t)l1 << 16);
    }
    uint16_t *o = xt + (size_t)tile * 1024 + 8 * lane; // xt_index(t, k, nblk, 0)
    *(uint4 *)o = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    *(uint4 *)(o + 512) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
}

hipError_t launch_split(const float *x, int T, int D, uint16_t *xt, hipStream_t s)
{
    size_t n = (size_t)T * D;
    if (n == 0) return hipSuccess;
    if (D % 32 != 0) return hipErrorInvalidValue;
    if ((uintptr_t)x % 16 == 0) {
        const size_t tiles = (size_t)((T + 15) / 16) * (D / 32);
        hipLaunchKernelGGL(split_tile_kernel, dim3((unsigned)((tiles + 3) / 4)), dim3(256), 0, s, x, T, D, xt);
    } else {
        hipLaunchKernelGGL(split_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, T, D, xt);
    }
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

// Four outputs per thread, the partials added in the same order (mn % 4 == 0,
// p and y 16-byte aligned); every partial's load issued before the first add.
template <int KS>
__global__ __launch_bounds__(256) void reduce_partials4_kernel(const float *p, size_t mn, float *y)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (4 * i >= mn) return;
    float4 v[KS];
#pragma unroll
    for (int z = 0; z < KS; z++) v[z] = ((const float4 *)(p + (size_t)z * mn))[i];
    float4 s = v[0];
#pragma unroll
    for (int z = 1; z < KS; z++) {
        s.x = s.x + v[z].x;
        s.y = s.y + v[z].y;
        s.z = s.z + v[z].z;
        s.w = s.w + v[z].w;
    }
    ((float4 *)y)[i] = s;
}

hipError_t launch_reduce_partials(const float *partial, int ksplit, int M, int N, float *y, hipStream_t s)
{
    size_t mn = (size_t)M * N;
    if (mn == 0) return hipSuccess;
    if (mn % 4 == 0 && (uintptr_t)partial % 16 == 0 && (uintptr_t)y % 16 == 0 && ksplit >= 2 && ksplit <= 4) {
        const dim3 grid((unsigned)((mn / 4 + 255) / 256));
        if (ksplit == 2) hipLaunchKernelGGL(reduce_partials4_kernel<2>, grid, dim3(256), 0, s, partial, mn, y);
        else if (ksplit == 3) hipLaunchKernelGGL(reduce_partials4_kernel<3>, grid, dim3(256), 0, s, partial, mn, y);
        else hipLaunchKernelGGL(reduce_partials4_kernel<4>, grid, dim3(256), 0, s, partial, mn, y);
        return hipGetLastError();
    }
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

__global__ void kv_split_kernel(const float *src, uint16_t *dst, int cap, int len, int hd)
{
    const int h = blockIdx.y;
    const size_t n = (size_t)len * hd / 2;
    const float2 *s = (const float2 *)(src + (size_t)h * cap * hd);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const size_t pos = 2 * i / hd, d = 2 * i % hd, row = (size_t)h * cap + pos;
        uint32_t hv, lv;
        split2_rtz(s[i].x, s[i].y, hv, lv);
        *(uint32_t *)(dst + (row * 2 + 0) * hd + d) = hv;
        *(uint32_t *)(dst + (row * 2 + 1) * hd + d) = lv;
    }
}

hipError_t launch_kv_split(const float *src, uint16_t *dst, int heads_total, int cap, int len, int hd, hipStream_t s)
{
    if (len <= 0 || heads_total <= 0) return hipSuccess;
    if (hd % 2 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(kv_split_kernel, dim3(64, heads_total), dim3(256), 0, s, src, dst, cap, len, hd);
    return hipGetLastError();
}

hipError_t launch_kv_copy(const float *src, float *dst, int heads_total, int old_cap, int new_cap, int len, int hd,
                          hipStream_t s)
{
    if (len <= 0 || heads_total <= 0) return hipSuccess;
    hipLaunchKernelGGL(kv_copy_kernel, dim3(64, heads_total), dim3(256), 0, s, src, dst, old_cap, new_cap, len, hd);
    return hipGetLastError();
}

} // namespace jev
