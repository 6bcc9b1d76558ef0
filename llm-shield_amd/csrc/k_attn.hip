// Tree-masked grouped-query attention over the HBM-resident fp32 KV cache.
//
// Replaces AttentionAsync / AttendHead (MinistralModel.cs:446-636) and
// AttentionKernels (AttentionKernels.cs).  A query token t of head h (KV head
// h / group) sees the logical keys i in [0, limit) with
//   n_sh  = shared_hi - shared_lo
//   limit = n_sh + (slot - segment + 1)
//   p(i)  = i < n_sh ? shared_lo + i : segment + (i - n_sh)
// (MinistralModel.cs:518-527, with the shared range generalised to start at
// shared_lo).  Scores are q.k * 1/sqrt(head_dim), softmax runs over exactly the
// visible keys, and the context is the weighted sum of their values.
//
// Prefill / tree kernel (attn_tree_kernel): flash-style online softmax over
// blocks of 64 *logical* keys on the fp16 MFMA cores.  A block's shape
// depends only on the query's own visible range, never on which other queries
// share its tile, so a branch scores exactly as it would alone: the tree pass
// is bit-identical to running the branches one at a time.  Each tile is up to
// 64 consecutive tokens with one (shared_lo, shared_hi, segment) and
// consecutive slots; 4 waves take 16 queries each.
//
// Operands are fp16 pairs (x = hi + lo, ~22 bits): every product is three
// v_mfma_f32_16x16x32_f16 (hi.hi + hi.lo + lo.hi), which keeps fp32-grade
// scores at a fraction of the fp32-MFMA cost.  The KV cache stays fp32; K and V
// blocks are split into pairs while being staged in LDS, K as [key][dim] and V
// transposed to [dim][key] so both operand fragments are vector reads.
//
//   S^T (16 keys x 16 queries) = K (16 x 128) . Q^T      12 MFMAs per 16 keys
//   O^T (128 x 16) += V^T (128 x 64) . P^T (64 x 16)      48 MFMAs per 64 keys,
//                     keys taken in the order the S^T fragments hold them
//
// Decode kernel (attn_decode_kernel): one query per token, split over chunks
// of 64 logical keys (one wave each: lane = key for the scores, lane = two
// dims for the weighted sum), chunks combined in ascending order.
#include "jev_dev.h"

namespace jev {

namespace {
constexpr int KB = 64;          // keys per block
constexpr int KROW = 128 + 8;   // K pair LDS row, halves (padded: conflict-free fragment reads)
constexpr int VROW = KB + 8;    // transposed V pair LDS row, halves

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void split4(float4 v, uint2 &hi, uint2 &lo)
{
    uint16_t h0, l0, h1, l1, h2, l2, h3, l3;
    split_f16(v.x, h0, l0);
    split_f16(v.y, h1, l1);
    split_f16(v.z, h2, l2);
    split_f16(v.w, h3, l3);
    hi = make_uint2((uint32_t)h0 | ((uint32_t)h1 << 16), (uint32_t)h2 | ((uint32_t)h3 << 16));
    lo = make_uint2((uint32_t)l0 | ((uint32_t)l1 << 16), (uint32_t)l2 | ((uint32_t)l3 << 16));
}

__device__ __forceinline__ half8_t cat4(uint2 a, uint2 b)
{
    uint4 u = make_uint4(a.x, a.y, b.x, b.y);
    return __builtin_bit_cast(half8_t, u);
}
} // namespace

__global__ __launch_bounds__(256, 2) void attn_tree_kernel(AttnArgs a)
{
    __shared__ __attribute__((aligned(16))) uint16_t Kh[KB * KROW], Kl[KB * KROW];
    __shared__ __attribute__((aligned(16))) uint16_t Vh[128 * VROW], Vl[128 * VROW];

    const AttnTile tile = a.tiles[blockIdx.x];
    const int head = blockIdx.y;
    const int kvh = head / a.group;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4;
    const int qdim = a.n_heads * 128;
    const float *kbase = a.kc + (size_t)kvh * a.cap * 128;
    const float *vbase = a.vc + (size_t)kvh * a.cap * 128;

    const int n_sh = tile.shared_hi - tile.shared_lo;
    // This lane's query (column of S^T / O^T).
    const int qi = 16 * wave + (lane & 15);
    const bool q_ok = qi < tile.n;
    const int my_limit = q_ok ? n_sh + (tile.slot0 + qi - tile.segment + 1) : 1;
    const int max_limit = n_sh + (tile.slot0 + tile.n - 1 - tile.segment + 1);
    const int nblocks = (max_limit + KB - 1) / KB;

    // Q^T fragments: dims 32 c + 8 g .. + 7 of this lane's query, as pairs.
    half8_t qh[4], ql[4];
    {
        const float *qp = a.q + (size_t)(tile.t0 + (q_ok ? qi : 0)) * qdim + head * 128 + 8 * g;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float4 v0 = q_ok ? *(const float4 *)(qp + 32 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
            float4 v1 = q_ok ? *(const float4 *)(qp + 32 * c + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
            uint2 h0, l0, h1, l1;
            split4(v0, h0, l0);
            split4(v1, h1, l1);
            qh[c] = cat4(h0, h1);
            ql[c] = cat4(l0, l1);
        }
    }

    floatx4 o[8];
#pragma unroll
    for (int j = 0; j < 8; j++) o[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;

    for (int b = 0; b < nblocks; b++) {
        __syncthreads();
        // Stage K: thread -> (key, quarter row) as pairs in [key][dim].
        {
            int key = tid >> 2, part = tid & 3;
            int kl = b * KB + key;
            uint2 hv[8], lv[8];
            if (kl < max_limit) {
                int p = kl < n_sh ? tile.shared_lo + kl : tile.segment + (kl - n_sh);
                const float4 *ks = (const float4 *)(kbase + (size_t)p * 128 + part * 32);
#pragma unroll
                for (int i = 0; i < 8; i++) split4(ks[i], hv[i], lv[i]);
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) hv[i] = lv[i] = make_uint2(0u, 0u);
            }
            uint4 *kh4 = (uint4 *)(Kh + key * KROW + part * 32);
            uint4 *kl4 = (uint4 *)(Kl + key * KROW + part * 32);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                kh4[i] = make_uint4(hv[2 * i].x, hv[2 * i].y, hv[2 * i + 1].x, hv[2 * i + 1].y);
                kl4[i] = make_uint4(lv[2 * i].x, lv[2 * i].y, lv[2 * i + 1].x, lv[2 * i + 1].y);
            }
        }
        // Stage V transposed: thread -> 4 keys x 8 dims, written as [dim][key].
        {
            int kg = tid >> 4, dg = tid & 15;
            float vv[4][8];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                int kl = b * KB + 4 * kg + kk;
                if (kl < max_limit) {
                    int p = kl < n_sh ? tile.shared_lo + kl : tile.segment + (kl - n_sh);
                    const float4 *vs = (const float4 *)(vbase + (size_t)p * 128 + 8 * dg);
                    float4 v0 = vs[0], v1 = vs[1];
                    vv[kk][0] = v0.x; vv[kk][1] = v0.y; vv[kk][2] = v0.z; vv[kk][3] = v0.w;
                    vv[kk][4] = v1.x; vv[kk][5] = v1.y; vv[kk][6] = v1.z; vv[kk][7] = v1.w;
                } else {
#pragma unroll
                    for (int i = 0; i < 8; i++) vv[kk][i] = 0.f;
                }
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                uint2 hv, lv;
                split4(make_float4(vv[0][i], vv[1][i], vv[2][i], vv[3][i]), hv, lv);
                *(uint2 *)(Vh + (8 * dg + i) * VROW + 4 * kg) = hv;
                *(uint2 *)(Vl + (8 * dg + i) * VROW + 4 * kg) = lv;
            }
        }
        __syncthreads();

        // S^T for 4 sub-blocks of 16 keys.
        floatx4 sc[4];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            floatx4 c = floatx4{0.f, 0.f, 0.f, 0.f};
            const int row = (16 * s + (lane & 15)) * KROW + 8 * g;
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                half8_t kh = *(const half8_t *)(Kh + row + 32 * cc);
                half8_t kl = *(const half8_t *)(Kl + row + 32 * cc);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[cc], c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[cc], c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[cc], c, 0, 0, 0);
            }
            sc[s] = c;
        }
        // Scale, mask (by the logical key index), block max.
        float bmax = -INFINITY;
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                int kl = b * KB + 16 * s + 4 * g + r;
                float v = sc[s][r] * a.scale;
                v = kl < my_limit ? v : -INFINITY;
                sc[s][r] = v;
                bmax = fmaxf(bmax, v);
            }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 16, 64));
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
        float m_new = fmaxf(m_run, bmax);
        float alpha = expf(m_run - m_new);
        float psum = 0.f;
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float p = expf(sc[s][r] - m_new);
                sc[s][r] = p;
                psum += p;
            }
        psum += __shfl_xor(psum, 16, 64);
        psum += __shfl_xor(psum, 32, 64);
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int j = 0; j < 8; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) o[j][r] = o[j][r] * alpha;

        // O^T += V^T P^T over two 32-key chunks; k slot (g, i) <-> key
        // 16 (2 c + i / 4) + 4 g + i % 4, the keys this lane's P values hold.
#pragma unroll
        for (int c = 0; c < 2; c++) {
            uint2 ph0, pl0, ph1, pl1;
            split4(make_float4(sc[2 * c][0], sc[2 * c][1], sc[2 * c][2], sc[2 * c][3]), ph0, pl0);
            split4(make_float4(sc[2 * c + 1][0], sc[2 * c + 1][1], sc[2 * c + 1][2], sc[2 * c + 1][3]), ph1, pl1);
            half8_t bh = cat4(ph0, ph1), bl = cat4(pl0, pl1);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int row = (16 * j + (lane & 15)) * VROW + 32 * c + 4 * g;
                half8_t vh = cat4(*(const uint2 *)(Vh + row), *(const uint2 *)(Vh + row + 16));
                half8_t vl = cat4(*(const uint2 *)(Vl + row), *(const uint2 *)(Vl + row + 16));
                o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, bh, o[j], 0, 0, 0);
                o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, bl, o[j], 0, 0, 0);
                o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, bh, o[j], 0, 0, 0);
            }
        }
    }

    if (q_ok) {
        // dims 16 j + 4 (lane/16) + r: four consecutive k, one 8-byte store per part
        float inv = 1.0f / l_run;
        const int t = tile.t0 + qi, nblk = qdim >> 5;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            int k = head * 128 + 16 * j + 4 * g;
            uint2 hv, lv;
            split4(make_float4(o[j][0] * inv, o[j][1] * inv, o[j][2] * inv, o[j][3] * inv), hv, lv);
            *(uint2 *)(a.ot + xt_index(t, k, nblk, 0)) = hv;
            *(uint2 *)(a.ot + xt_index(t, k, nblk, 1)) = lv;
        }
    }
}

hipError_t launch_attn_tree(const AttnArgs &a, hipStream_t s)
{
    if (a.n_tiles <= 0) return hipSuccess;
    if (a.hd != 128) return hipErrorInvalidValue;
    hipLaunchKernelGGL(attn_tree_kernel, dim3(a.n_tiles, a.n_heads), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ------------------------------------------------------------ decode

__global__ __launch_bounds__(64) void attn_decode_kernel(DecodeAttnArgs a)
{
    __shared__ float qs[128];
    __shared__ float ps[64];
    const int t = blockIdx.x, head = blockIdx.y, c = blockIdx.z;
    const int lane = threadIdx.x;
    const int kvh = head / a.group;
    const int qdim = a.n_heads * 128;
    const int slot = a.slot ? a.slot[t] : a.start + t;
    const int slo = a.shared_lo ? a.shared_lo[t] : 0;
    const int shi = a.shared_hi ? a.shared_hi[t] : a.start;
    const int seg = a.segment ? a.segment[t] : a.start;
    const int n_sh = shi - slo;
    const int limit = n_sh + (slot - seg + 1);
    float *part = a.part + (((size_t)t * a.n_heads + head) * a.max_chunks + c) * 130;

    if (c * 64 >= limit) {
        if (lane == 0) {
            part[0] = -INFINITY;
            part[1] = 0.f;
        }
        for (int d = lane; d < 128; d += 64) part[2 + d] = 0.f;
        return;
    }
    const float *q = a.q + (size_t)t * qdim + head * 128;
    qs[lane] = q[lane];
    qs[lane + 64] = q[lane + 64];
    __syncthreads();

    const float *kbase = a.kc + (size_t)kvh * a.cap * 128;
    const float *vbase = a.vc + (size_t)kvh * a.cap * 128;
    int kl = c * 64 + lane;
    float sc = -INFINITY;
    if (kl < limit) {
        int p = kl < n_sh ? slo + kl : seg + (kl - n_sh);
        const float4 *kr = (const float4 *)(kbase + (size_t)p * 128);
        float acc = 0.f;
#pragma unroll 8
        for (int i = 0; i < 32; i++) {
            float4 kv = kr[i];
            acc = fmaf(qs[4 * i], kv.x, acc);
            acc = fmaf(qs[4 * i + 1], kv.y, acc);
            acc = fmaf(qs[4 * i + 2], kv.z, acc);
            acc = fmaf(qs[4 * i + 3], kv.w, acc);
        }
        sc = acc * a.scale;
    }
    float mx = warp_max(sc);
    float p = kl < limit ? expf(sc - mx) : 0.f;
    float sum = warp_sum(p);
    ps[lane] = p;
    __syncthreads();
    float o0 = 0.f, o1 = 0.f;
    int nk = min(64, limit - c * 64);
    for (int k = 0; k < nk; k++) {
        int kk = c * 64 + k;
        int pp = kk < n_sh ? slo + kk : seg + (kk - n_sh);
        float2 vv = *(const float2 *)(vbase + (size_t)pp * 128 + 2 * lane);
        float w = ps[k];
        o0 = fmaf(w, vv.x, o0);
        o1 = fmaf(w, vv.y, o1);
    }
    if (lane == 0) {
        part[0] = mx;
        part[1] = sum;
    }
    part[2 + 2 * lane] = o0;
    part[3 + 2 * lane] = o1;
}

__global__ __launch_bounds__(128) void attn_combine_kernel(DecodeAttnArgs a)
{
    const int t = blockIdx.x, head = blockIdx.y, d = threadIdx.x;
    const float *part = a.part + ((size_t)t * a.n_heads + head) * a.max_chunks * 130;
    float M = -INFINITY;
    for (int c = 0; c < a.max_chunks; c++) M = fmaxf(M, part[c * 130]);
    float L = 0.f, O = 0.f;
    for (int c = 0; c < a.max_chunks; c++) {
        float mc = part[c * 130];
        float f = mc == -INFINITY ? 0.f : expf(mc - M);
        L = fmaf(part[c * 130 + 1], f, L);
        O = fmaf(part[c * 130 + 2 + d], f, O);
    }
    a.ctx[(size_t)t * a.n_heads * 128 + head * 128 + d] = O / L;
}

hipError_t launch_attn_decode(const DecodeAttnArgs &a, hipStream_t s)
{
    if (a.T <= 0) return hipSuccess;
    if (a.hd != 128) return hipErrorInvalidValue;
    hipLaunchKernelGGL(attn_decode_kernel, dim3(a.T, a.n_heads, a.max_chunks), dim3(64), 0, s, a);
    hipLaunchKernelGGL(attn_combine_kernel, dim3(a.T, a.n_heads), dim3(128), 0, s, a);
    return hipGetLastError();
}

} // namespace jev
