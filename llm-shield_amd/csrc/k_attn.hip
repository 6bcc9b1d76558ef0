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
// Decode kernel (attn_decode_kernel): few tokens, one query per head, split
// over chunks of 64 logical keys per KV head; chunks combined in ascending
// order by the last workgroup to finish.
#include "jev_dev.h"

namespace jev {

namespace {
constexpr int KB = 64;          // keys per block
constexpr int KROW = 128 + 8;   // K pair LDS row, halves (padded: conflict-free fragment reads)
constexpr int VROW = KB + 8;    // transposed V pair LDS row, halves

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

// x = hi + lo as fp16 pairs: hi rounded toward zero (two per v_cvt_pkrtz),
// lo the remainder rounded the same way; |x - hi - lo| < 2^-20 |x| for normal fp16 hi.
__device__ __forceinline__ void split4(float4 v, uint2 &hi, uint2 &lo)
{
    typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));
    const fp16x2 h01 = __builtin_amdgcn_cvt_pkrtz(v.x, v.y), h23 = __builtin_amdgcn_cvt_pkrtz(v.z, v.w);
    const float r0 = v.x - (float)h01[0], r1 = v.y - (float)h01[1];
    const float r2 = v.z - (float)h23[0], r3 = v.w - (float)h23[1];
    const fp16x2 l01 = __builtin_amdgcn_cvt_pkrtz(r0, r1), l23 = __builtin_amdgcn_cvt_pkrtz(r2, r3);
    hi = make_uint2(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23));
    lo = make_uint2(__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23));
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

    // Staging.  K: thread -> (key tid / 4, quarter row) as pairs in
    // [key][dim].  V transposed to [dim][key]: thread -> 4 keys (4 (tid % 16)
    // ..) x 8 dims (8 (tid / 16) ..), so a wave's stores spread over the
    // banks.  The next block's rows are loaded into registers while the
    // current block is on the matrix cores; loads are unconditional (the key
    // clamped, the value zeroed past the end when stored).
    const int kkey = tid >> 2, kpart = tid & 3;
    const int vkq = tid & 15, vdq = tid >> 4;
    float4 kr[8], vr[4][2];
    auto slot_of = [&](int kl) { return kl < n_sh ? tile.shared_lo + kl : tile.segment + (kl - n_sh); };
    auto load_kv = [&](int b) __attribute__((always_inline)) {
        const int kl = min(b * KB + kkey, max_limit - 1);
        const float4 *ks = (const float4 *)(kbase + (size_t)slot_of(kl) * 128 + kpart * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) kr[i] = ks[i];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const int vl = min(b * KB + 4 * vkq + kk, max_limit - 1);
            const float4 *vs = (const float4 *)(vbase + (size_t)slot_of(vl) * 128 + 8 * vdq);
            vr[kk][0] = vs[0];
            vr[kk][1] = vs[1];
        }
    };
    auto store_kv = [&](int b) __attribute__((always_inline)) {
        {
            const bool ok = b * KB + kkey < max_limit;
            uint2 *kh2 = (uint2 *)(Kh + kkey * KROW + kpart * 32);
            uint2 *kl2 = (uint2 *)(Kl + kkey * KROW + kpart * 32);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                uint2 hv, lv;
                split4(kr[i], hv, lv);
                kh2[i] = make_uint2(ok ? hv.x : 0u, ok ? hv.y : 0u);
                kl2[i] = make_uint2(ok ? lv.x : 0u, ok ? lv.y : 0u);
            }
        }
        {
            float vv[4][8];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const bool ok = b * KB + 4 * vkq + kk < max_limit;
                const float4 v0 = vr[kk][0], v1 = vr[kk][1];
                vv[kk][0] = ok ? v0.x : 0.f; vv[kk][1] = ok ? v0.y : 0.f;
                vv[kk][2] = ok ? v0.z : 0.f; vv[kk][3] = ok ? v0.w : 0.f;
                vv[kk][4] = ok ? v1.x : 0.f; vv[kk][5] = ok ? v1.y : 0.f;
                vv[kk][6] = ok ? v1.z : 0.f; vv[kk][7] = ok ? v1.w : 0.f;
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                uint2 hv, lv;
                split4(make_float4(vv[0][i], vv[1][i], vv[2][i], vv[3][i]), hv, lv);
                *(uint2 *)(Vh + (8 * vdq + i) * VROW + 4 * vkq) = hv;
                *(uint2 *)(Vl + (8 * vdq + i) * VROW + 4 * vkq) = lv;
            }
        }
    };

    load_kv(0);
    for (int b = 0; b < nblocks; b++) {
        __syncthreads(); // the previous block's fragments have been read
        store_kv(b);
        __syncthreads();
        load_kv(min(b + 1, nblocks - 1)); // in flight during this block's math

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
        float alpha = __expf(m_run - m_new);
        float psum = 0.f;
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float p = __expf(sc[s][r] - m_new);
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

// One workgroup per (token, KV head, chunk of 64 logical keys): the chunk's K
// and V rows are staged in LDS once with coalesced loads and serve the
// group's query heads (wave w takes heads w, w + 4, ...).  Scores: lane =
// key, fp32 dot over 128 dims; weighted sum: lane = two dims.  Each chunk
// leaves (max, sum, o[128]) per head; the last workgroup of a (token, KV
// head) to finish -- counted with an atomic that it resets -- combines the
// chunks in ascending order, so the result does not depend on timing.
constexpr int kDecKeys = 64;
constexpr int kDecRow = 132; // padded K row, floats

__global__ __launch_bounds__(256) void attn_decode_kernel(DecodeAttnArgs a)
{
    __shared__ __attribute__((aligned(16))) float Ks[kDecKeys * kDecRow];
    __shared__ __attribute__((aligned(16))) float Vs[kDecKeys * 128];
    __shared__ __attribute__((aligned(16))) float qs[4][128];
    __shared__ float ps[4][kDecKeys];
    __shared__ int last;
    const int t = blockIdx.x, kvh = blockIdx.y, c = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int qdim = a.n_heads * 128;
    const int start = a.start_dev ? *a.start_dev : a.start;
    const int slot = a.slot ? a.slot[t] : start + t;
    const int slo = a.shared_lo ? a.shared_lo[t] : 0;
    const int shi = a.shared_hi ? a.shared_hi[t] : start;
    const int seg = a.segment ? a.segment[t] : start;
    const int n_sh = shi - slo;
    const int limit = n_sh + (slot - seg + 1);
    const int nchunks = (limit + kDecKeys - 1) / kDecKeys;
    if (c >= nchunks) return; // this token sees fewer keys

    // ---- stage the chunk's K and V rows (logical key -> cache slot)
    const float *kbase = a.kc + (size_t)kvh * a.cap * 128;
    const float *vbase = a.vc + (size_t)kvh * a.cap * 128;
    const int nk = min(kDecKeys, limit - c * kDecKeys);
    {
        // unconditional (clamped) loads, all in flight before the first store
        float4 kv[8], vv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int e = tid + 256 * i; // float4 index in the 64 x 32 chunk
            const int key = min(e >> 5, nk - 1), d4 = e & 31;
            const int kl = c * kDecKeys + key;
            const int p = kl < n_sh ? slo + kl : seg + (kl - n_sh);
            kv[i] = *(const float4 *)(kbase + (size_t)p * 128 + 4 * d4);
            vv[i] = *(const float4 *)(vbase + (size_t)p * 128 + 4 * d4);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int e = tid + 256 * i;
            const int key = e >> 5, d4 = e & 31;
            const bool ok = key < nk;
            const float4 k4 = kv[i], v4 = vv[i];
            *(float4 *)(Ks + key * kDecRow + 4 * d4) =
                make_float4(ok ? k4.x : 0.f, ok ? k4.y : 0.f, ok ? k4.z : 0.f, ok ? k4.w : 0.f);
            *(float4 *)(Vs + key * 128 + 4 * d4) =
                make_float4(ok ? v4.x : 0.f, ok ? v4.y : 0.f, ok ? v4.z : 0.f, ok ? v4.w : 0.f);
        }
    }
    float *part_base = a.part + ((size_t)t * a.n_heads) * a.max_chunks * 130;
    for (int h0 = 0; h0 < a.group; h0 += 4) { // every wave takes every barrier
        const int h = h0 + wave;
        const bool active = h < a.group;
        const int head = kvh * a.group + min(h, a.group - 1);
        __syncthreads(); // K/V staged; the previous head's qs/ps consumed
        const float *q = a.q + (size_t)t * qdim + head * 128;
        qs[wave][lane] = q[lane];
        qs[wave][lane + 64] = q[lane + 64];
        __syncthreads();
        // scores: lane = key
        float sc = -INFINITY;
        if (lane < nk) {
            float acc = 0.f;
            const float4 *kr = (const float4 *)(Ks + lane * kDecRow);
            const float4 *qr = (const float4 *)qs[wave];
#pragma unroll 8
            for (int i = 0; i < 32; i++) {
                const float4 kv = kr[i], qv = qr[i];
                acc = fmaf(qv.x, kv.x, acc);
                acc = fmaf(qv.y, kv.y, acc);
                acc = fmaf(qv.z, kv.z, acc);
                acc = fmaf(qv.w, kv.w, acc);
            }
            sc = acc * a.scale;
        }
        const float mx = warp_max(sc);
        const float p = lane < nk ? __expf(sc - mx) : 0.f;
        const float sum = warp_sum(p);
        ps[wave][lane] = p;
        __syncthreads();
        // weighted sum: lane = dims 2 lane, 2 lane + 1
        float o0 = 0.f, o1 = 0.f;
#pragma unroll 8
        for (int k = 0; k < nk; k++) {
            const float w = ps[wave][k];
            const float2 vv = *(const float2 *)(Vs + k * 128 + 2 * lane);
            o0 = fmaf(w, vv.x, o0);
            o1 = fmaf(w, vv.y, o1);
        }
        if (active) {
            float *part = part_base + ((size_t)head * a.max_chunks + c) * 130;
            if (lane == 0) {
                part[0] = mx;
                part[1] = sum;
            }
            *(float2 *)(part + 2 + 2 * lane) = make_float2(o0, o1);
        }
    }

    // ---- the last chunk of this (token, KV head) to finish combines
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        int *ctr = a.counters + (size_t)t * (a.n_heads / a.group) + kvh;
        const int done = atomicAdd(ctr, 1);
        last = done == nchunks - 1;
        if (last) *ctr = 0; // ready for the next call
    }
    __syncthreads();
    if (!last) return;
    __threadfence(); // acquire: the other chunks' partials are visible
    for (int h = wave; h < a.group; h += 4) {
        const int head = kvh * a.group + h;
        const float *part = part_base + (size_t)head * a.max_chunks * 130;
        // chunks in ascending order, eight loads in flight at a time
        float M = -INFINITY;
        for (int c0 = 0; c0 < nchunks; c0 += 8) {
            float mv[8];
#pragma unroll
            for (int j = 0; j < 8; j++) mv[j] = part[min(c0 + j, nchunks - 1) * 130];
#pragma unroll
            for (int j = 0; j < 8; j++) M = fmaxf(M, mv[j]);
        }
        float L = 0.f, O0 = 0.f, O1 = 0.f;
        for (int c0 = 0; c0 < nchunks; c0 += 8) {
            float mv[8], lv[8];
            float2 ov[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float *pc = part + min(c0 + j, nchunks - 1) * 130;
                mv[j] = pc[0];
                lv[j] = pc[1];
                ov[j] = *(const float2 *)(pc + 2 + 2 * lane);
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                if (c0 + j < nchunks) {
                    const float f = __expf(mv[j] - M);
                    L = fmaf(lv[j], f, L);
                    O0 = fmaf(ov[j].x, f, O0);
                    O1 = fmaf(ov[j].y, f, O1);
                }
            }
        }
        float *ctx = a.ctx + (size_t)t * qdim + head * 128;
        *(float2 *)(ctx + 2 * lane) = make_float2(O0 / L, O1 / L);
    }
}

hipError_t launch_attn_decode(const DecodeAttnArgs &a, hipStream_t s)
{
    if (a.T <= 0) return hipSuccess;
    if (a.hd != 128 || a.group < 1 || a.n_heads % a.group != 0 || !a.counters) return hipErrorInvalidValue;
    hipLaunchKernelGGL(attn_decode_kernel, dim3(a.T, a.n_heads / a.group, a.max_chunks), dim3(256), 0, s, a);
    return hipGetLastError();
}

} // namespace jev
