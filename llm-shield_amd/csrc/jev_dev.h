// Device helpers shared by the kernels: fp16 conversions and block decoding
// of the field-split weight layout (see QWeight in jev_internal.h).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jev_internal.h"

namespace jev {

// Kernel launch with optional timing events (a profiled pass): given both,
// the dispatch itself stamps them (hipExtLaunchKernelGGL), so their elapsed
// time is this kernel's alone rather than a marker's on either side of it.
template <typename Kernel, typename... Args>
inline void launch_stamped(hipEvent_t e0, hipEvent_t e1, Kernel k, dim3 grid, dim3 block, uint32_t lds, hipStream_t s,
                           Args... args)
{
    if (e0 && e1)
        hipExtLaunchKernelGGL(k, grid, block, lds, s, e0, e1, 0, args...);
    else
        hipLaunchKernelGGL(k, grid, block, lds, s, args...);
}

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

// x ~= hi + lo with both halves fp16 (round to nearest even each time).
__device__ __forceinline__ void split_f16(float x, uint16_t &hi, uint16_t &lo)
{
    _Float16 h = (_Float16)x;
    _Float16 l = (_Float16)(x - (float)h);
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, l);
}

// Two floats as fp16 pairs x = hi + lo, each half rounded toward zero (one
// v_cvt_pkrtz per part): |x - hi - lo| < 2^-20 |x| for normal fp16 hi.
__device__ __forceinline__ void split2_rtz(float x0, float x1, uint32_t &hi, uint32_t &lo)
{
    typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));
    const fp16x2 h = __builtin_amdgcn_cvt_pkrtz(x0, x1);
    const fp16x2 l = __builtin_amdgcn_cvt_pkrtz(x0 - (float)h[0], x1 - (float)h[1]);
    hi = __builtin_bit_cast(uint32_t, h);
    lo = __builtin_bit_cast(uint32_t, l);
}

// One weight element of the tiled layout, decoded exactly as Dequantizer
// does (Dequantizer.cs: Q4_0 :155-182, Q5_1 :240-268, Q8_0 :270-305).  d*q is
// exact in fp32, so the Q5_1 "+ m" rounds once whether or not it is fused.
// TYPE >= 0: the weight's type known at compile time (no branches around the
// loads, so a caller's loads of several elements can all be in flight).
template <int TYPE = -1>
__device__ __forceinline__ float decode_elem(const QWeight &w, int row, int k)
{
    const int type = TYPE >= 0 ? TYPE : w.type;
    const int rg = row >> 4, r = row & 15, b = k >> 5, kk = k & 31, g = kk >> 3, i = kk & 7, bb = b & 1;
    const int l = 16 * g + r;
    const size_t tile = (size_t)rg * tile_kpairs(w.cols) + (b >> 1);
    const float d = h2f(type == kQ5_1 ? w.d[tile * 64 + 4 * r + bb] : w.d[tile * 32 + 2 * r + bb]);
    if (type == kQ8_0) {
        const int q = (int)w.qs[tile * 1024 + 16 * l + 8 * bb + i] - 128; // stored biased
        return (float)q * d;
    }
    const uint8_t byte = w.qs[tile * 512 + 8 * l + 4 * bb + (i & 3)];
    const int nib = i < 4 ? (byte & 15) : (byte >> 4);
    if (type == kQ4_0) return d * (float)(nib - 8);
    const int q = nib | (((w.qh[tile * 128 + 2 * l + bb] >> i) & 1) << 4);
    const float m = h2f(w.d[tile * 64 + 4 * r + 2 + bb]);
    const float dq = d * (float)q;
    return dq + m;
}

// GEMM activation layout ("operand tiles"): an fp16 pair x ~= hi + lo for
// rows grouped by 16 and K by 32.  Each (row group, K block, part) is one
// 16 x 32 MFMA A-operand tile stored in lane order -- lane 16*(k%32 / 8) +
// row%16 holds 8 consecutive k -- so a wave fetches its fragment with one
// contiguous 1 KiB load.  part 0 = hi, 1 = lo.  Rows are padded to 16.
__host__ __device__ __forceinline__ size_t xt_index(int row, int k, int nblk, int part)
{
    int rg = row >> 4, r = row & 15, b = k >> 5, kk = k & 31;
    return ((((size_t)rg * nblk + b) * 2 + part) * 64 + ((kk >> 3) * 16 + r)) * 8 + (kk & 7);
}

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw buffer resource over [p, p + bytes): offsets past the end read zeros.
__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

// Integer quants to fp16 without float conversions: a byte u placed under
// the exponent byte 0x64 is the fp16 value 1024 + u (exact, ulp 1 in
// [1024, 2048)); one packed fp16 subtraction of the bias then leaves the
// integer.  Four values cost one byte permute per pair plus one v_pk_add_f16
// per pair.
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t biased_pair(uint32_t bytes, uint32_t sel)
{
    return __builtin_amdgcn_perm(0x64646464u, bytes, sel);
}

__device__ __forceinline__ uint32_t sub_bias(uint32_t v, _Float16 bias)
{
    half2_t h = __builtin_bit_cast(half2_t, v) - half2_t{bias, bias};
    return __builtin_bit_cast(uint32_t, h);
}

// Four biased bytes -> two fp16 pairs (elements 0,1 and 2,3).
__device__ __forceinline__ void bytes_to_f16(uint32_t bytes, _Float16 bias, uint32_t &p01, uint32_t &p23)
{
    p01 = sub_bias(biased_pair(bytes, 0x04010400u), bias);
    p23 = sub_bias(biased_pair(bytes, 0x04030402u), bias);
}

__device__ __forceinline__ float warp_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float warp_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Kernels.RmsNorm's statistics (Kernels.cs:25-60) for one row of D floats in
// a workgroup of NT threads: thread t owns the float4 groups g = t + NT i
// (i < NI), x[i] = h + the sum of the `nadd` K-split partials taken in split
// order (Kernels.Add first), squares summed per thread in group order, then by
// a fixed butterfly per wave and the NT / 64 wave sums in order.  Returns
// 1 / sqrt(sum / D + eps).  `wsum` is NT / 64 floats of LDS.  Groups a thread
// does not own (g >= D / 4) load a clamped neighbour and are left out of the
// sum.  The order is a function of NT: every caller of one width gets the
// same bits.
template <int NI, int NP, int NT = 256>
__device__ __forceinline__ float row_rms_scale(const float4 *h4, const float4 *add4, int nadd, size_t pstride, int D,
                                               float eps, float4 (&x)[NI], float *wsum)
{
    const int tid = threadIdx.x, ng = D >> 2;
    float4 p[NP][NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        if (NT * i >= ng) break;
        x[i] = h4[min(tid + NT * i, ng - 1)];
    }
    if (add4) {
#pragma unroll
        for (int z = 0; z < NP; z++) {
            if (z >= nadd) break;
#pragma unroll
            for (int i = 0; i < NI; i++) {
                if (NT * i >= ng) break;
                p[z][i] = add4[z * pstride + min(tid + NT * i, ng - 1)];
            }
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        if (NT * i >= ng) break;
        float4 v = x[i];
        if (add4) {
            float4 s4 = p[0][i];
#pragma unroll
            for (int z = 1; z < NP; z++) {
                if (z >= nadd) break;
                s4.x = s4.x + p[z][i].x;
                s4.y = s4.y + p[z][i].y;
                s4.z = s4.z + p[z][i].z;
                s4.w = s4.w + p[z][i].w;
            }
            v.x = v.x + s4.x;
            v.y = v.y + s4.y;
            v.z = v.z + s4.z;
            v.w = v.w + s4.w;
        }
        x[i] = v;
        if (tid + NT * i < ng) {
            float q0 = v.x * v.x, q1 = v.y * v.y, q2 = v.z * v.z, q3 = v.w * v.w;
            ss = ss + q0;
            ss = ss + q1;
            ss = ss + q2;
            ss = ss + q3;
        }
    }
    ss = warp_sum(ss);
    if ((tid & 63) == 0) wsum[tid >> 6] = ss;
    __syncthreads();
    float sum = wsum[0];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) sum = sum + wsum[w];
    return 1.0f / sqrtf(sum / (float)D + eps);
}

} // namespace jev
