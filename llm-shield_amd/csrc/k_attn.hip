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
// Prefill / tree kernel (attn_tree_kernel): fp32 MFMA (v_mfma_f32_16x16x4_f32),
// flash-style online softmax over blocks of 64 *logical* keys.  A block's
// shape depends only on the query's own visible range, never on which other
// queries share its tile, so a branch scores exactly as it would alone:
// the tree pass is bit-identical to running the branches one at a time.
// Each tile is up to 64 consecutive tokens with one (shared_lo, shared_hi,
// segment) and consecutive slots; 4 waves take 16 queries each.  K and V
// blocks are staged in LDS (rows padded to 132 floats: the fragment reads of a
// wave fall two lanes per bank).
//
//   S^T (16 keys x 16 queries) = K (16 x 128) . Q^T   32 MFMAs per 16 keys
//   O^T (128 x 16) += V^T (128 x 64) . P^T (64 x 16)  keys taken in the order
//                                                     the S^T layout holds them
//
// Decode kernel (attn_decode_kernel): one query per token, split over chunks
// of 64 logical keys (one wave each: lane = key for the scores, lane = two
// dims for the weighted sum), chunks combined in ascending order.
#include "jev_dev.h"

namespace jev {

namespace {
constexpr int KB = 64;        // keys per block
constexpr int KROW = 132;     // padded LDS row (floats)
} // namespace

__global__ __launch_bounds__(256) void attn_tree_kernel(AttnArgs a)
{
    __shared__ __attribute__((aligned(16))) float Ks[KB * KROW];
    __shared__ __attribute__((aligned(16))) float Vs[KB * KROW];

    const AttnTile tile = a.tiles[blockIdx.x];
    const int head = blockIdx.y;
    const int kvh = head / a.group;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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

    // Q^T fragments: qreg[t] = Q[query][4t + lane/16].
    float qreg[32];
    {
        const float *qp = a.q + (size_t)(tile.t0 + (q_ok ? qi : 0)) * qdim + head * 128 + (lane >> 4);
#pragma unroll
        for (int t = 0; t < 32; t++) qreg[t] = q_ok ? qp[4 * t] : 0.f;
    }

    floatx4 o[8];
#pragma unroll
    for (int j = 0; j < 8; j++) o[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;

    for (int b = 0; b < nblocks; b++) {
        __syncthreads();
        // Stage 64 keys (and values) of logical block b: thread -> (key, quarter row).
        {
            int key = tid >> 2, part = tid & 3;
            int kl = b * KB + key;
            float4 *kd = (float4 *)(Ks + key * KROW + part * 32);
            float4 *vd = (float4 *)(Vs + key * KROW + part * 32);
            if (kl < max_limit) {
                int p = kl < n_sh ? tile.shared_lo + kl : tile.segment + (kl - n_sh);
                const float4 *ks = (const float4 *)(kbase + (size_t)p * 128 + part * 32);
                const float4 *vs = (const float4 *)(vbase + (size_t)p * 128 + part * 32);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    kd[i] = ks[i];
                    vd[i] = vs[i];
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    kd[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                    vd[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
        }
        __syncthreads();

        // S^T for 4 sub-blocks of 16 keys.
        floatx4 sc[4];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            floatx4 c = floatx4{0.f, 0.f, 0.f, 0.f};
            const float *kr = Ks + (16 * s + (lane & 15)) * KROW + (lane >> 4);
#pragma unroll
            for (int t = 0; t < 32; t++) c = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[4 * t], qreg[t], c, 0, 0, 0);
            sc[s] = c;
        }
        // Scale, mask (by the logical key index), block max.
        float bmax = -INFINITY;
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                int kl = b * KB + 16 * s + 4 * (lane >> 4) + r;
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

        // O^T += V^T P^T, k-index kk = lane/16 <-> key 16 s + 4 kk + r.
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float *vr = Vs + (16 * s + 4 * (lane >> 4) + r) * KROW + (lane & 15);
#pragma unroll
                for (int j = 0; j < 8; j++) o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[16 * j], sc[s][r], o[j], 0, 0, 0);
            }
    }

    if (q_ok) {
        // dims 16 j + 4 (lane/16) + r: four consecutive k, one 8-byte store per part
        float inv = 1.0f / l_run;
        const int t = tile.t0 + qi, nblk = qdim >> 5;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            int k = head * 128 + 16 * j + 4 * (lane >> 4);
            uint16_t hi[4], lo[4];
#pragma unroll
            for (int r = 0; r < 4; r++) split_f16(o[j][r] * inv, hi[r], lo[r]);
            *(uint2 *)(a.ot + xt_index(t, k, nblk, 0)) =
                make_uint2((uint32_t)hi[0] | ((uint32_t)hi[1] << 16), (uint32_t)hi[2] | ((uint32_t)hi[3] << 16));
            *(uint2 *)(a.ot + xt_index(t, k, nblk, 1)) =
                make_uint2((uint32_t)lo[0] | ((uint32_t)lo[1] << 16), (uint32_t)lo[2] | ((uint32_t)lo[3] << 16));
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
