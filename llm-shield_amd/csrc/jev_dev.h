// Device helpers shared by the kernels: fp16 conversions and block decoding
// of the field-split weight layout (see QWeight in jev_internal.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jev_internal.h"

namespace jev {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// x ~= hi + lo with both halves fp16 (round to nearest even each time).
__device__ __forceinline__ void split_f16(float x, uint16_t &hi, uint16_t &lo)
{
    _Float16 h = (_Float16)x;
    _Float16 l = (_Float16)(x - (float)h);
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, l);
}

// One weight element, decoded exactly as Dequantizer does (Dequantizer.cs:
// Q4_0 :155-182, Q5_1 :240-268, Q8_0 :270-305).  d*q is exact in fp32, so
// the Q5_1 "+ m" rounds once whether or not it is fused.
__device__ __forceinline__ float decode_elem(const QWeight &w, int r, int k)
{
    int nb = w.cols >> 5;
    int b = k >> 5, j = k & 31;
    float d = h2f(w.d[(size_t)r * nb + b]);
    if (w.type == kQ8_0) {
        int8_t q = (int8_t)w.qs[(size_t)r * w.cols + k];
        return (float)q * d;
    }
    uint8_t byte = w.qs[(size_t)r * (w.cols >> 1) + b * 16 + (j & 15)];
    int nib = j < 16 ? (byte & 15) : (byte >> 4);
    if (w.type == kQ4_0) return d * (float)(nib - 8);
    uint32_t qh = w.qh[(size_t)r * nb + b];
    int q = nib | (int)(((qh >> j) & 1u) << 4);
    float m = h2f(w.m[(size_t)r * nb + b]);
    float dq = d * (float)q;
    return dq + m;
}

// GEMM activation layout ("operand tiles"): an fp16 pair x ~= hi + lo for
// rows grouped by 16 and K by 32.  Each (row group, K block, part) is one
// 16 x 32 MFMA A-operand tile stored in lane order -- lane 16*(k%32 / 8) +
// row%16 holds 8 consecutive k -- so a wave fetches its fragment with one
// contiguous 1 KiB load.  part 0 = hi, 1 = lo.  Rows are padded to 16.
__device__ __forceinline__ size_t xt_index(int row, int k, int nblk, int part)
{
    int rg = row >> 4, r = row & 15, b = k >> 5, kk = k & 31;
    return ((((size_t)rg * nblk + b) * 2 + part) * 64 + ((kk >> 3) * 16 + r)) * 8 + (kk & 7);
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

} // namespace jev
