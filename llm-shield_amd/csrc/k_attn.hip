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
// 32 consecutive tokens with one (shared_lo, shared_hi, segment) and
// consecutive slots; a workgroup takes one tile and one KV head, and its four
// waves are four query heads of that KV head, so every staged K/V block
// serves 4 x 32 query rows.
//
// Operands are fp16 pairs (x = hi + lo, ~22 bits): every product is three
// v_mfma_f32_32x32x16_f16 (hi.hi + hi.lo + lo.hi), which keeps fp32-grade
// scores at a fraction of the fp32-MFMA cost.  The KV cache stays fp32 and
// carries fp16-pair shadows of every row ([hi, lo][dim], written with the
// row); the kernel stages those shadows straight into LDS, where K fragments
// are plain reads and V^T fragments transposing reads (ds_read_b64_tr_b16).
//
//   S^T (32 keys x 32 queries) = K (32 x 128) . Q^T      24 MFMAs per 32 keys
//   O^T (128 x 32) += V^T (128 x 64) . P^T (64 x 32)      48 MFMAs per 64 keys,
//                     keys taken in the order the S^T fragments hold them
//
// Decode kernel (attn_decode_kernel): one query per head, split over chunks
// of 64 logical keys per KV head; the chunks are combined in ascending order
// by the consumer, the O projection's GEMV, while it stages its input.
#include "jev_dev.h"

#include <type_traits>

namespace jev {

namespace {
constexpr int KB = 64;      // keys per block
constexpr int KCH = KB * 32; // 16-byte chunks of a staged K or V block: [key][hi, lo][16]

// Chunk swizzle of a staged key row: 16 consecutive keys, and 4 aligned keys
// x 4 chunks, land on distinct 16-byte bank groups.
__device__ __forceinline__ int swz(int key) { return ((key & 3) << 2) | ((key >> 2) & 3); }

typedef short short4_t __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16 over a 16-lane group: lane 4 a + e receives element e of
// the 8 bytes addressed by lanes a, a + 4, a + 8, a + 12 (in that order).
__device__ __forceinline__ uint2 read_tr(uint32_t lds_byte)
{
    const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t *)(size_t)lds_byte);
    return __builtin_bit_cast(uint2, v);
}

// x - (float)h for h the low (hi_half = false) or high fp16 of `h2`, by one
// v_fma_mix_f32 (h * -1 + x, the f16 source converted exactly): the same
// bits as converting h and subtracting, fp16 denormals included.
__device__ __forceinline__ float pair_rem(uint32_t h2, float x, bool hi_half)
{
    float r;
    if (hi_half)
        asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(x));
    else
        asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(x));
    return r;
}

// LDS byte address of a __shared__ object, and a 16-byte read at one.
__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
    return (uint32_t)(size_t)(const __attribute__((address_space(3))) char *)p;
}
__device__ __forceinline__ half8_t lds_load8h(uint32_t lds_byte)
{
    return *(const __attribute__((address_space(3))) half8_t *)(size_t)lds_byte;
}

typedef float floatx16 __attribute__((ext_vector_type(16)));

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

// DS = 2 or 4 (grids smaller than the GPU): DS workgroups per tile and KV
// head (blockIdx.z); each stages the blocks and computes the scores and
// softmax (the same instructions on the same data) and accumulates 128 / DS
// of the output dims.  Every output is the same chain of MFMAs either way.
//
// Schedule (one wave per SIMD: the workgroup's 128 KiB of LDS fills the CU):
// a wave's matrix-core work and its softmax overlap only if its instruction
// stream interleaves them, so each block is two regions of independent work:
//   A(b): S(b) = K(b) Q^T on the matrix cores, beside the second half of block
//         b - 1's softmax (row sum, P pairs, o *= alpha) on the vector ALU;
//   B(b): O^T += V^T P^T of block b - 1 on the matrix cores, beside the first
//         half of block b's softmax (mask, running max, exponentials).
// The operations and their order per output are those of the plain sequence
// S(b), P V(b - 1), softmax(b), rescale, so the bits do not depend on it.
template <int DS>
__global__ __launch_bounds__(256, 1) void attn_tree_kernel(AttnArgs a)
{
    constexpr int ND = 4 / DS; // 32-dim output tiles per wave
    // Double-buffered K and V blocks as fp16 pairs: [key][hi, lo][16 chunks of
    // 8 dims], chunks swizzled per key (chunk ^ swz(key)) so that both the
    // K fragment reads and the V transpose reads hit distinct banks.  One
    // array, K0 K1 V0 V1: a K read reaches its buffer through the LDS
    // instruction's 16-bit offset, a V read from a base of 64 KiB held in
    // its address register.
    __shared__ __attribute__((aligned(16))) uint4 lds[4 * KCH];
    uint4 *const Ks0 = lds, *const Ks1 = lds + KCH, *const Vs0 = lds + 2 * KCH, *const Vs1 = lds + 3 * KCH;
    constexpr uint32_t KBUF = KCH * 16; // bytes per buffer

    // Longest tiles first: the plan lists tiles in token order, and later
    // tokens see more keys.
    const AttnTile tile = a.tiles[a.n_tiles - 1 - (int)blockIdx.y];
    const int hsets = (a.group + 3) >> 2;
    const int kvh = blockIdx.x / hsets;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int dh = DS > 1 ? (int)blockIdx.z : 0; // output dims 128 / DS * dh ..
    const int g = lane >> 5, col = lane & 31;
    const int hl = (blockIdx.x % hsets) * 4 + wave; // query head within the group
    const bool head_ok = hl < a.group;              // wave-uniform
    const int head = kvh * a.group + min(hl, a.group - 1);
    const int qdim = a.n_heads * 128;

    const int n_sh = tile.shared_hi - tile.shared_lo;
    // This lane's query is column `col` of S^T / O^T; lanes col and col + 32
    // hold the two row halves of it.
    const bool q_ok = head_ok && col < tile.n;
    const int my_limit = q_ok ? n_sh + (tile.slot0 + col - tile.segment + 1) : 1;
    const int min_limit = n_sh + (tile.slot0 - tile.segment + 1); // the tile's first query
    const int max_limit = n_sh + (tile.slot0 + tile.n - 1 - tile.segment + 1);
    const int nblocks = (max_limit + KB - 1) / KB;
    auto slot_of = [&](int kl) { return kl < n_sh ? tile.shared_lo + kl : tile.segment + (kl - n_sh); };

    // Staging: wave w's load i moves LDS chunks (8 w + i) * 64 + lane, i.e.
    // key 16 w + 2 i + lane / 32, part (lane / 16) % 2, stored chunk lane % 16;
    // the lane fetches the logical chunk that position holds.  Keys past the
    // tile's last visible key are clamped to it: every staged row is a
    // written cache row (finite), masked for every query, and enters the
    // context only as 0 * v.
    int skey[8];
    uint32_t soff[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        skey[i] = 16 * wave + 2 * i + (lane >> 5);
        soff[i] = skey[i] * 512 + ((lane >> 4) & 1) * 256 + ((lane & 15) ^ swz(skey[i])) * 16;
    }
    // One block of 64 logical keys from `src` (the KV head's pair rows) into
    // `dst`.  A block inside one contiguous range below the last visible key
    // has slot = base + key: a uniform offset plus the lane's constant one.
    // Buffer loads straight to LDS: as loads they count on the vector-memory
    // counter alone, so the LDS reads after them wait for exactly the reads
    // they need.
    auto stage = [&](int b, rsrc_t src, uint4 *dst) __attribute__((always_inline)) {
        const int k0 = b * KB;
        const bool in_shared = k0 + KB <= n_sh, in_seg = k0 >= n_sh;
        if (k0 + KB <= max_limit && (in_shared || in_seg)) {
            const int base = (in_shared ? tile.shared_lo + k0 : tile.segment + (k0 - n_sh));
#pragma unroll
            for (int i = 0; i < 8; i++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(src, (__attribute__((address_space(3))) void *)&dst[(8 * wave + i) * 64], 16,
                                                         soff[i], base * 512, 0, 0);
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int kl = min(k0 + skey[i], max_limit - 1);
                const uint32_t off = (uint32_t)slot_of(kl) * 512 + (soff[i] - skey[i] * 512);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(src, (__attribute__((address_space(3))) void *)&dst[(8 * wave + i) * 64], 16,
                                                         off, 0, 0, 0);
            }
        }
    };
    const rsrc_t kpb = make_rsrc(a.kp + (size_t)kvh * a.cap * 256, (uint32_t)a.cap * 512);
    const rsrc_t vpb = make_rsrc(a.vp + (size_t)kvh * a.cap * 256, (uint32_t)a.cap * 512);
    stage(0, kpb, Ks0); // in flight while Q is read

    // Q^T fragments: dims 16 c + 8 g .. + 7 of this lane's query, scaled by
    // 1/sqrt(head_dim) * log2 e (scores come out in log2 units), as pairs.
    half8_t qh[8], ql[8];
    {
        const float sl2 = a.scale * 1.44269504088896340736f;
        const float *qp = a.q + (size_t)(tile.t0 + (q_ok ? col : 0)) * qdim + head * 128 + 8 * g;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            float4 v0 = q_ok ? *(const float4 *)(qp + 16 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
            float4 v1 = q_ok ? *(const float4 *)(qp + 16 * c + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
            v0 = make_float4(v0.x * sl2, v0.y * sl2, v0.z * sl2, v0.w * sl2);
            v1 = make_float4(v1.x * sl2, v1.y * sl2, v1.z * sl2, v1.w * sl2);
            uint2 h0, l0, h1, l1;
            split4(v0, h0, l0);
            split4(v1, h1, l1);
            qh[c] = cat4(h0, h1);
            ql[c] = cat4(l0, l1);
            // The Q fragments are only ever MFMA B operands: accumulation
            // registers, leaving the vector registers to the softmax and P V.
            asm volatile("" : "+a"(qh[c]), "+a"(ql[c]));
        }
    }

    // K fragment of S^T half t, dim chunk c: key 32 t + col, logical chunk
    // 2 c + g.  swz(32 t + col) = swz(col).
    uint32_t koff[8];
#pragma unroll
    for (int c = 0; c < 8; c++) koff[c] = lds_addr(Ks0) + col * 512 + ((2 * c + g) ^ swz(col)) * 16;
    // V^T fragment (transpose reads): lane (G = lane / 16, s = lane % 16)
    // supplies key 16 c + 8 r + 4 (G / 2) + s / 4 at dims 32 d + 16 (G % 2) +
    // 4 (s % 4); it receives dim 32 d + lane % 32 of the four keys
    // 16 c + 8 r + 4 (G / 2) + j.  Addresses for c = 0, hi part, buffer V0; c
    // adds 16 keys.  Kept opaque so the V0 base stays in the register.
    uint32_t vadr[2][4];
    {
        const int s16 = lane & 15, G = lane >> 4, gp = G >> 1;
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int d = 0; d < 4; d++) {
                const int key = 8 * r + 4 * gp + (s16 >> 2);
                const int lc = 4 * d + 2 * (G & 1) + ((s16 & 3) >> 1);
                vadr[r][d] = lds_addr(Vs0) + key * 512 + ((lc ^ swz(key)) * 16) + 8 * (s16 & 1);
                asm volatile("" : "+v"(vadr[r][d]));
            }
    }

    floatx16 o[ND]; // output dims 32 (ND dh + d) ..
#pragma unroll
    for (int d = 0; d < ND; d++)
#pragma unroll
        for (int j = 0; j < 16; j++) o[d][j] = 0.f;
    float m_run = -INFINITY, l_run = 0.f; // running max in log2 units
    float alpha = 0.f;                    // exp2(previous max - new max) of the block in ex
    floatx16 sc[2];                       // S^T of the block being scored
    floatx16 ex[2];                       // exp2(s - max) of the block in the softmax
    half8_t pbh[4], pbl[4];               // its P as pairs: chunk c's B fragments

    // S^T for the block in K buffer kb (byte offset 0 or KBUF), two 32-key
    // halves.  Each K fragment of dim chunk c + 1 is read as soon as the last
    // MFMA of chunk c that uses its register has issued.  slot(k) runs after
    // the k-th of the 48 MFMAs, in a scheduling region of its own: the order
    // written here is the order issued.
    auto scores = [&](uint32_t kb, auto &&slot) __attribute__((always_inline)) {
        half8_t kf[4]; // [2 t + part]
        auto kread = [&](int c, int i) __attribute__((always_inline)) {
            kf[i] = lds_load8h(koff[c] + kb + (i >> 1) * (32 * 512) + (i & 1) * 256);
        };
#pragma unroll
        for (int i = 0; i < 4; i++) kread(0, i);
#pragma unroll
        for (int c = 0; c < 8; c++) {
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const floatx16 acc = c == 0 ? floatx16{} : sc[t];
                sc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[2 * t], qh[c], acc, 0, 0, 0);
                slot(6 * c + 3 * t);
                __builtin_amdgcn_sched_barrier(0);
                sc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[2 * t], ql[c], sc[t], 0, 0, 0);
                if (c + 1 < 8) kread(c + 1, 2 * t);
                slot(6 * c + 3 * t + 1);
                __builtin_amdgcn_sched_barrier(0);
                sc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[2 * t + 1], qh[c], sc[t], 0, 0, 0);
                if (c + 1 < 8) kread(c + 1, 2 * t + 1);
                slot(6 * c + 3 * t + 2);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    // O^T += V^T P^T for the block in V buffer vb over four 16-key chunks,
    // 4 ND steps (chunk c, dim tile d); the V^T fragments of the step after
    // next are read while this step's three MFMAs run.  Chunk c's k slot
    // 8 g + i is key 16 c + 8 (i / 4) + 4 g + i % 4: the P values
    // ex[c / 2][8 (c % 2) + i] of this lane, as pbh / pbl.  slot(k) as above,
    // after the k-th of the 12 ND MFMAs.
    auto pv = [&](uint32_t vb, auto &&slot) __attribute__((always_inline)) {
        constexpr int NST = 4 * ND;
        // [step % 2][hi pair (two reads), lo pair]; a pair for step st + 2 is
        // read as soon as step st's last MFMA using its registers has issued
        uint2 vf[2][4];
        auto vread = [&](int st, int half) __attribute__((always_inline)) {
            const int c = st / ND, d = ND * dh + st % ND;
            const uint32_t v0 = vadr[0][d] + vb + c * (16 * 512) + half * 256, v1 = vadr[1][d] + vb + c * (16 * 512) + half * 256;
            vf[st & 1][2 * half] = read_tr(v0);
            vf[st & 1][2 * half + 1] = read_tr(v1);
        };
        vread(0, 0);
        vread(0, 1);
        if (NST > 1) {
            vread(1, 0);
            vread(1, 1);
        }
#pragma unroll
        for (int st = 0; st < NST; st++) {
            const int c = st / ND, d = st % ND;
            const uint2(&f)[4] = vf[st & 1];
            const half8_t vh = cat4(f[0], f[1]), vl = cat4(f[2], f[3]);
            o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, pbh[c], o[d], 0, 0, 0);
            slot(3 * st);
            __builtin_amdgcn_sched_barrier(0);
            o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, pbl[c], o[d], 0, 0, 0);
            if (st + 2 < NST) vread(st + 2, 0);
            slot(3 * st + 1);
            __builtin_amdgcn_sched_barrier(0);
            o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vl, pbh[c], o[d], 0, 0, 0);
            if (st + 2 < NST) vread(st + 2, 1);
            slot(3 * st + 2);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Softmax of block b, first half, in the NS1 = 12 ND slots of P V: the
    // mask (where the block reaches past the tile's first query, by logical
    // key index), the running max, the exponentials.  sc[t][j] holds key
    // 32 t + 8 (j / 4) + 4 g + j % 4.  PER slots' worth of work per slot.
    constexpr int NS1 = 12 * ND, PER = 48 / NS1;
    constexpr int MAX_SLOTS = 8 / PER, BPERM = MAX_SLOTS, MNEW = MAX_SLOTS + 1 + (PER == 1), EXP0 = MNEW + 1;
    float bmax = -INFINITY, bmax_o = -INFINITY, m_new = 0.f;
    auto soft1 = [&](int k, int b, auto masked) __attribute__((always_inline)) {
        if (k < MAX_SLOTS) {
            if (k == 0) bmax = -INFINITY;
#pragma unroll
            for (int u = 4 * PER * k; u < 4 * PER * (k + 1); u++) {
                const int t = u >> 4, j = u & 15;
                if constexpr (decltype(masked)::value) {
                    const int kl = b * KB + 32 * t + 8 * (j >> 2) + 4 * g + (j & 3);
                    sc[t][j] = kl < my_limit ? sc[t][j] : -INFINITY;
                }
                bmax = fmaxf(bmax, sc[t][j]);
            }
        }
        if (k == BPERM) bmax_o = __shfl_xor(bmax, 32, 64);
        if (k == MNEW) {
            m_new = fmaxf(m_run, fmaxf(bmax, bmax_o));
            alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
        }
        if (k >= EXP0 && k < EXP0 + 32 / PER) {
#pragma unroll
            for (int u = PER * (k - EXP0); u < PER * (k - EXP0 + 1); u++)
                ex[u >> 4][u & 15] = __builtin_amdgcn_exp2f(sc[u >> 4][u & 15] - m_new);
        }
    };
    // Second half, in the 48 slots of the next block's S: the row sum (in key
    // order), the P pairs, and the rescale of the output accumulated so far
    // (o * 1 is o, so it runs unconditionally).  Per three slots: one pair of
    // P values split (over two slots), three row-sum terms, 4 ND / 4 output
    // multiplies (two in the third slot): at most four vector instructions
    // beside each MFMA, about what one wave issues while its MFMA runs.
    float psum = 0.f, psum_o = 0.f;
    uint32_t p_hi = 0; // the pair in flight: its hi half
    auto soft2 = [&](int k) __attribute__((always_inline)) {
        typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));
        const int u = 2 * (k / 3), t = u >> 4, j = u & 15, c = u >> 3, part = (u >> 1) & 3;
        if (k == 0) psum = 0.f;
        if (k < 32) psum += ex[k >> 4][k & 15];
        if (k % 3 == 0) {
            p_hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(ex[t][j], ex[t][j + 1]));
            uint4 hv = __builtin_bit_cast(uint4, pbh[c]);
            (&hv.x)[part] = p_hi;
            pbh[c] = __builtin_bit_cast(half8_t, hv);
        }
        if (k % 3 == 1) {
            // lo = the remainders x - hi (exact), rounded toward zero as hi was
            const fp16x2 l = __builtin_amdgcn_cvt_pkrtz(pair_rem(p_hi, ex[t][j], false), pair_rem(p_hi, ex[t][j + 1], true));
            uint4 lv = __builtin_bit_cast(uint4, pbl[c]);
            (&lv.x)[part] = __builtin_bit_cast(uint32_t, l);
            pbl[c] = __builtin_bit_cast(half8_t, lv);
        }
        if (k == 33) psum_o = __shfl_xor(psum, 32, 64);
        if (k == 36) l_run = l_run * alpha + (psum + psum_o);
        // output multiplies: weights 1, 1, 2 per three slots, 16 ND in all
        auto mark = [](int kk) { return (16 * ND * (4 * (kk / 3) + (kk % 3))) / 64; };
#pragma unroll
        for (int e = mark(k); e < mark(k + 1); e++) o[e >> 4][e & 15] *= alpha;
    };
    auto none = [](int) {};
    using Plain = std::integral_constant<bool, false>;
    using Masked = std::integral_constant<bool, true>;
    // block b reaches past the tile's first query: its scores need the mask
    auto tail = [&](int b) { return (b + 1) * KB > min_limit; };

    // Block 0: staged K(1) and V(0), S(0) and its softmax's first half.
    __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0): this thread's K(0) has landed
    __syncthreads();                    // everyone's
    if (nblocks > 1) stage(1, kpb, Ks1);
    stage(0, vpb, Vs0);
    // A wave past the group's last head (group not a multiple of 4) computes
    // its clamped head's rows like the others and stores nothing: no branch
    // around the block loop, so every block keeps o, sc and ex in place.
    scores(0, none);
    if (tail(0)) {
#pragma unroll
        for (int k = 0; k < NS1; k++) soft1(k, 0, Masked{});
    } else {
#pragma unroll
        for (int k = 0; k < NS1; k++) soft1(k, 0, Plain{});
    }
    // Block b >= 1: K(b) in buffer b % 2, V(b - 1) in the other; K(b + 1) and
    // V(b) are staged while A(b) and B(b) run.
    auto step = [&](int b, uint32_t kb, uint32_t vb, uint4 *Kn, uint4 *Vn, auto masked) __attribute__((always_inline)) {
        __builtin_amdgcn_s_waitcnt(0x0F70); // this thread's K(b) and V(b - 1) have landed
        __syncthreads();                    // everyone's; K(b - 1) and V(b - 2) are free again
        if (b + 1 < nblocks) stage(b + 1, kpb, Kn);
        stage(b, vpb, Vn);
        __builtin_amdgcn_sched_barrier(0);
        scores(kb, soft2);
        pv(vb, [&](int k) __attribute__((always_inline)) { soft1(k, b, masked); });
    };
    for (int b = 1; b < nblocks; b += 2) {
        if (tail(b))
            step(b, KBUF, 0, Ks0, Vs1, Masked{});
        else
            step(b, KBUF, 0, Ks0, Vs1, Plain{});
        if (b + 1 < nblocks) {
            if (tail(b + 1))
                step(b + 1, 0, KBUF, Ks1, Vs0, Masked{});
            else
                step(b + 1, 0, KBUF, Ks1, Vs0, Plain{});
        }
    }
    // The last block's second softmax half and P V.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 48; k++) soft2(k);
    pv(((nblocks - 1) & 1) ? KBUF : 0, none);

    if (q_ok) {
        // o[d][j] is dim 32 (ND dh + d) + 8 (j / 4) + 4 g + j % 4: four
        // consecutive k, one 8-byte store per part
        const float inv = 1.0f / l_run;
        const int t = tile.t0 + col, nblk = qdim >> 5;
#pragma unroll
        for (int d = 0; d < ND; d++)
#pragma unroll
            for (int jq = 0; jq < 4; jq++) {
                const int k = head * 128 + 32 * (ND * dh + d) + 8 * jq + 4 * g;
                uint2 hv, lv;
                split4(make_float4(o[d][4 * jq] * inv, o[d][4 * jq + 1] * inv, o[d][4 * jq + 2] * inv,
                                   o[d][4 * jq + 3] * inv), hv, lv);
                *(uint2 *)(a.ot + xt_index(t, k, nblk, 0)) = hv;
                *(uint2 *)(a.ot + xt_index(t, k, nblk, 1)) = lv;
            }
    }
}

hipError_t launch_attn_tree(const AttnArgs &a, hipStream_t s)
{
    if (a.n_tiles <= 0) return hipSuccess;
    // cap * 512 bytes per KV head is a buffer resource's 32-bit extent (2^32
    // itself would wrap to an empty resource)
    if (a.hd != 128 || a.group < 1 || a.n_tiles > 65535 || !a.kp || !a.vp || a.cap <= 0 || a.cap >= (1 << 23))
        return hipErrorInvalidValue;
    const int n_kv = a.n_heads / a.group, hsets = (a.group + 3) / 4;
    const dim3 grid(n_kv * hsets, a.n_tiles);
    // fewer workgroups than compute units: the output dims split over two or four
    const long wgs = (long)grid.x * grid.y;
    if (wgs <= 64)
        launch_stamped(a.ev_start, a.ev_stop, attn_tree_kernel<4>, dim3(grid.x, grid.y, 4), dim3(256), 0, s, a);
    else if (wgs < 256)
        launch_stamped(a.ev_start, a.ev_stop, attn_tree_kernel<2>, dim3(grid.x, grid.y, 2), dim3(256), 0, s, a);
    else
        launch_stamped(a.ev_start, a.ev_stop, attn_tree_kernel<1>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

// ------------------------------------------------------------ decode

// One workgroup per (token, KV head, chunk of 64 logical keys): the chunk's K
// and V rows are staged in LDS once with coalesced loads and serve the
// group's query heads (wave w takes heads w, w + 4, ...).  Scores: lane =
// key, fp32 dot over 128 dims; weighted sum: lane = two dims.  Each chunk
// leaves (max, sum, o[128]) per head.  The GEMV of the O projection merges
// the chunks in ascending order while staging its input (the kernel boundary
// makes the partials visible; a last-to-finish merge here would need a
// device-scope fence per workgroup, an L2 write-back and invalidate on this
// multi-XCD part), so the result does not depend on timing.
constexpr int kDecKeys = kDecodeKeys;
constexpr int kDecRow = 132; // padded K row, floats
constexpr int kDecLoads = kDecKeys * 32 / 256; // float4 loads of K (and of V) per thread

__global__ __launch_bounds__(256) void attn_decode_kernel(DecodeAttnArgs a)
{
    __shared__ __attribute__((aligned(16))) float Ks[kDecKeys * kDecRow];
    __shared__ __attribute__((aligned(16))) float Vs[kDecKeys * 128];
    __shared__ __attribute__((aligned(16))) float qs[4][128];
    __shared__ float ps[4][kDecKeys];
    __shared__ float cs[64], sn[64]; // fused RoPE: cos / sin (times mscale) of the token's position
    const int tl = blockIdx.x, t = a.t0 + tl, kvh = blockIdx.y, c = blockIdx.z;
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

    // ---- loads, all in flight before the first use and issued in the order
    // they are needed (the vector-memory counter retires loads in order, so
    // waiting on one waits on every older one): the RoPE frequency, the first
    // query head's projection partials, the chunk's K and V rows (logical key
    // -> cache slot), then the new key's and value's partials.  The hoisted
    // loads are unconditional with in-range addresses (the projection and
    // frequency buffers are set whether or not RoPE is fused here) and feed
    // nothing where unused.
    const RopeArgs &r = a.rope;
    const size_t zs = r.in_stride;
    constexpr int kHoist = 2; // projection K-split partials loaded up front
    const bool hoisted = r.nin <= kHoist;
    const int head0 = kvh * a.group + min(wave, a.group - 1);
    const float fr = r.freqs[min(tid, max(r.half, 1) - 1)];
    __builtin_amdgcn_sched_barrier(0); // keep the issue order
    float qx[kHoist][2];
#pragma unroll
    for (int z = 0; z < kHoist; z++) {
        const float *qi = r.q_in + min(z, r.nin - 1) * zs + (size_t)t * r.ld_in + head0 * 128;
        qx[z][0] = qi[lane];
        qx[z][1] = qi[lane + 64];
    }
    __builtin_amdgcn_sched_barrier(0);
    const float *kbase = a.kc + (size_t)kvh * a.cap * 128;
    const float *vbase = a.vc + (size_t)kvh * a.cap * 128;
    const int nk = min(kDecKeys, limit - c * kDecKeys);
    float4 kv[kDecLoads], vv[kDecLoads];
#pragma unroll
    for (int i = 0; i < kDecLoads; i++) {
        const int e = tid + 256 * i; // float4 index in the kDecKeys x 32 chunk
        const int key = min(e >> 5, nk - 1), d4 = e & 31;
        const int kl = c * kDecKeys + key;
        const int p = kl < n_sh ? slo + kl : seg + (kl - n_sh);
        kv[i] = *(const float4 *)(kbase + (size_t)p * 128 + 4 * d4);
        vv[i] = *(const float4 *)(vbase + (size_t)p * 128 + 4 * d4);
    }
    // the new key's and value's column 4 (tid % 32) .. + 3 (every thread loads
    // one; the threads holding the new key's row use theirs)
    float4 kxz[kHoist], vxz[kHoist];
#pragma unroll
    for (int z = 0; z < kHoist; z++) {
        const size_t off = min(z, r.nin - 1) * zs + (size_t)t * r.ld_in + kvh * 128 + 4 * (tid & 31);
        kxz[z] = *(const float4 *)(r.k_in + off);
        vxz[z] = *(const float4 *)(r.v_in + off);
    }
    // Fused RoPE + KV store (Rope.Apply, Rope.cs:112-135; ApplyPositionScale,
    // MinistralModel.cs:676-682; StoreKeys / StoreValues :649-669), the same
    // operations in the same order as rope_store_kernel: the projection's
    // K-split partials summed in split order, pairs (2i, 2i + 1) rotated by
    // cos / sin(pos * freq_i) * mscale with separate products, q scaled.
    const int pos = a.rope_fused ? (r.pos ? r.pos[t] : start + t) : 0;
    float qscale = 1.f;
    bool qscaled = false;
    if (a.rope_fused) {
        if (tid < r.half) {
            const float theta = (float)pos * fr;
            cs[tid] = cosf(theta) * r.mscale;
            sn[tid] = sinf(theta) * r.mscale;
        }
        if (r.orig_ctx > 0 && r.temp_scale != 0.f) {
            const float interval = floorf((float)pos / (float)r.orig_ctx);
            if (interval != 0.f) {
                qscale = 1.f + r.temp_scale * logf(1.f + interval);
                qscaled = true;
            }
        }
        __syncthreads();
    }
    // rotated q of one head: this lane holds dims `lane` and `lane + 64`; the
    // pair partner of dim d is d ^ 1, held by lane ^ 1.  first: the wave's
    // first head, whose partials were loaded up front.
    auto rope_q = [&](int head, float &o0, float &o1, bool first) __attribute__((always_inline)) {
        const float *qi = r.q_in + (size_t)t * r.ld_in + head * 128;
        float x[2];
        if (first && hoisted) {
            x[0] = qx[0][0];
            x[1] = qx[0][1];
#pragma unroll
            for (int z = 1; z < kHoist; z++) {
                if (z >= r.nin) break;
                x[0] = x[0] + qx[z][0];
                x[1] = x[1] + qx[z][1];
            }
        } else {
            x[0] = qi[lane];
            x[1] = qi[lane + 64];
            for (int z = 1; z < r.nin; z++) {
                x[0] = x[0] + qi[z * zs + lane];
                x[1] = x[1] + qi[z * zs + lane + 64];
            }
        }
        float o[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const float y = __shfl_xor(x[j], 1, 64);
            const int d = lane + 64 * j, i = d >> 1;
            const float x0 = (d & 1) ? y : x[j], x1 = (d & 1) ? x[j] : y;
            float v = x[j];
            if (i < r.half) {
                const float cc = cs[i], sv = sn[i];
                const float m0 = x0 * cc, m1 = x1 * sv, m2 = x0 * sv, m3 = x1 * cc;
                v = (d & 1) ? m2 + m3 : m0 - m1;
            }
            if (qscaled) v = v * qscale;
            o[j] = v;
        }
        o0 = o[0];
        o1 = o[1];
    };
    float q0, q1;
    if (a.rope_fused) {
        rope_q(head0, q0, q1, true);
    } else {
        const float *q = a.q + (size_t)t * qdim + (kvh * a.group + min(wave, a.group - 1)) * 128;
        q0 = q[lane];
        q1 = q[lane + 64];
    }
    // the token's own key (logical limit - 1) is in the last chunk: that
    // workgroup forms it from the partials and stores it to the cache
    const bool own_chunk = a.rope_fused && c == nchunks - 1;
    {
#pragma unroll
        for (int i = 0; i < kDecLoads; i++) {
            const int e = tid + 256 * i;
            const int key = e >> 5, d4 = e & 31;
            const bool ok = key < nk;
            float4 k4 = kv[i], v4 = vv[i];
            if (own_chunk && key == nk - 1) {
                // the new key and value: partials summed, k rotated, stored
                const size_t off = (size_t)t * r.ld_in + kvh * 128 + 4 * d4;
                float4 kx, vx;
                if (hoisted) {
                    // d4 == tid % 32: this thread's up-front loads
                    kx = kxz[0];
                    vx = vxz[0];
#pragma unroll
                    for (int z = 1; z < kHoist; z++) {
                        if (z >= r.nin) break;
                        const float4 ku = kxz[z], vu = vxz[z];
                        kx = make_float4(kx.x + ku.x, kx.y + ku.y, kx.z + ku.z, kx.w + ku.w);
                        vx = make_float4(vx.x + vu.x, vx.y + vu.y, vx.z + vu.z, vx.w + vu.w);
                    }
                } else {
                    kx = *(const float4 *)(r.k_in + off);
                    vx = *(const float4 *)(r.v_in + off);
                    for (int z = 1; z < r.nin; z++) {
                        const float4 ku = *(const float4 *)(r.k_in + z * zs + off), vu = *(const float4 *)(r.v_in + z * zs + off);
                        kx = make_float4(kx.x + ku.x, kx.y + ku.y, kx.z + ku.z, kx.w + ku.w);
                        vx = make_float4(vx.x + vu.x, vx.y + vu.y, vx.z + vu.z, vx.w + vu.w);
                    }
                }
                float kr[4] = {kx.x, kx.y, kx.z, kx.w};
#pragma unroll
                for (int pp = 0; pp < 2; pp++) {
                    const int ip = 2 * d4 + pp;
                    if (ip < r.half) {
                        const float x0 = kr[2 * pp], x1 = kr[2 * pp + 1], cc = cs[ip], sv = sn[ip];
                        const float m0 = x0 * cc, m1 = x1 * sv, m2 = x0 * sv, m3 = x1 * cc;
                        kr[2 * pp] = m0 - m1;
                        kr[2 * pp + 1] = m2 + m3;
                    }
                }
                k4 = make_float4(kr[0], kr[1], kr[2], kr[3]);
                v4 = vx;
                const size_t row = (size_t)kvh * r.cap + slot;
                *(float4 *)(r.kc + row * 128 + 4 * d4) = k4;
                *(float4 *)(r.vc + row * 128 + 4 * d4) = v4;
                uint32_t kh0, kl0, kh1, kl1, vh0, vl0, vh1, vl1;
                split2_rtz(k4.x, k4.y, kh0, kl0);
                split2_rtz(k4.z, k4.w, kh1, kl1);
                split2_rtz(v4.x, v4.y, vh0, vl0);
                split2_rtz(v4.z, v4.w, vh1, vl1);
                *(uint2 *)(r.kp + (row * 2 + 0) * 128 + 4 * d4) = make_uint2(kh0, kh1);
                *(uint2 *)(r.kp + (row * 2 + 1) * 128 + 4 * d4) = make_uint2(kl0, kl1);
                *(uint2 *)(r.vp + (row * 2 + 0) * 128 + 4 * d4) = make_uint2(vh0, vh1);
                *(uint2 *)(r.vp + (row * 2 + 1) * 128 + 4 * d4) = make_uint2(vl0, vl1);
            }
            *(float4 *)(Ks + key * kDecRow + 4 * d4) =
                make_float4(ok ? k4.x : 0.f, ok ? k4.y : 0.f, ok ? k4.z : 0.f, ok ? k4.w : 0.f);
            *(float4 *)(Vs + key * 128 + 4 * d4) =
                make_float4(ok ? v4.x : 0.f, ok ? v4.y : 0.f, ok ? v4.z : 0.f, ok ? v4.w : 0.f);
        }
    }
    float *part_base = a.part + ((size_t)tl * a.n_heads) * a.max_chunks * 130;
    for (int h0 = 0; h0 < a.group; h0 += 4) { // every wave takes every barrier
        const int h = h0 + wave;
        const bool active = h < a.group;
        const int head = kvh * a.group + min(h, a.group - 1);
        __syncthreads(); // K/V staged; the previous head's qs/ps consumed
        if (h0 > 0) {
            if (a.rope_fused) {
                rope_q(head, q0, q1, false);
            } else {
                const float *q = a.q + (size_t)t * qdim + head * 128;
                q0 = q[lane];
                q1 = q[lane + 64];
            }
        }
        qs[wave][lane] = q0;
        qs[wave][lane + 64] = q1;
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
        if (lane < kDecKeys) ps[wave][lane] = p;
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
}

hipError_t launch_attn_decode(const DecodeAttnArgs &a, hipStream_t s)
{
    if (a.T <= 0) return hipSuccess;
    // several tokens (or a later group of them): each its own layout entry
    // (and position, when RoPE is fused: the caller guarantees no token sees
    // another's new key)
    if ((a.T > 1 || a.t0 > 0) && (!a.slot || !a.shared_lo || !a.shared_hi || !a.segment || (a.rope_fused && !a.rope.pos)))
        return hipErrorInvalidValue;
    if (a.t0 < 0) return hipErrorInvalidValue;
    if (a.hd != 128 || a.group < 1 || a.n_heads % a.group != 0) return hipErrorInvalidValue;
    if (!a.rope.q_in || !a.rope.k_in || !a.rope.v_in || !a.rope.freqs || a.rope.nin < 1) return hipErrorInvalidValue;
    if (a.rope_fused && (a.rope.hd != 128 || a.rope.half > 64 || a.rope.nin < 1 || !a.rope.q_in ||
                         !a.rope.k_in || !a.rope.v_in || !a.rope.kc || !a.rope.vc || !a.rope.kp || !a.rope.vp ||
                         !a.rope.freqs || a.rope.kc != a.kc || a.rope.vc != a.vc))
        return hipErrorInvalidValue;
    launch_stamped(a.ev_start, a.ev_stop, attn_decode_kernel, dim3(a.T, a.n_heads / a.group, a.max_chunks), dim3(256), 0, s,
                   a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return hipGetLastError();
}

// One workgroup of 64 lanes per (token, head): lane l merges dims 2 l and
// 2 l + 1 over the token's chunks in ascending order with a running max
// (each step rescales what came before by exp(old max - new max)), the same
// operations as the one-token O GEMV's staging, then writes the normalised
// context as the fp16 pair (hi rounded to nearest, lo the remainder).
__global__ __launch_bounds__(64) void attn_combine_kernel(AttnCombineArgs a)
{
    const int tl = blockIdx.x, t = a.t0 + tl, h = blockIdx.y, lane = threadIdx.x;
    const int slot = a.slot[t], slo = a.shared_lo[t], shi = a.shared_hi[t], seg = a.segment[t];
    const int limit = (shi - slo) + (slot - seg + 1);
    const int nch = min((limit + kDecodeKeys - 1) / kDecodeKeys, a.max_chunks);
    const float *pp = a.part + ((size_t)tl * a.n_heads + h) * a.max_chunks * 130;
    float M = -INFINITY, L = 0.f, v0 = 0.f, v1 = 0.f;
    for (int c0 = 0; c0 < nch; c0 += 8) {
        float mv[8], lv[8];
        float2 ov[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float *pc = pp + min(c0 + j, nch - 1) * 130; // clamped reloads are unused
            mv[j] = pc[0];
            lv[j] = pc[1];
            ov[j] = *(const float2 *)(pc + 2 + 2 * lane);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (c0 + j < nch) {
                const float Mn = fmaxf(M, mv[j]);
                const float fo = __expf(M - Mn), fc = __expf(mv[j] - Mn);
                L = fmaf(lv[j], fc, L * fo);
                v0 = fmaf(ov[j].x, fc, v0 * fo);
                v1 = fmaf(ov[j].y, fc, v1 * fo);
                M = Mn;
            }
        }
    }
    const float inv = 1.0f / L;
    v0 = v0 * inv;
    v1 = v1 * inv;
    uint16_t h0, l0, h1, l1;
    split_f16(v0, h0, l0);
    split_f16(v1, h1, l1);
    const int k = h * 128 + 2 * lane, nblk = a.n_heads * 4;
    // k and k + 1 are neighbours in the layout (k even)
    *(uint32_t *)(a.ot + xt_index(t, k, nblk, 0)) = (uint32_t)h0 | ((uint32_t)h1 << 16);
    *(uint32_t *)(a.ot + xt_index(t, k, nblk, 1)) = (uint32_t)l0 | ((uint32_t)l1 << 16);
    if (a.xsum) {
        // the Q5_1 block sums of these pairs, in the order the block-sum
        // kernel adds an operand tile's values (ascending k, hi + lo per
        // element): block q of the head is lanes 16 q .. 16 q + 15
        const float e0 = h2f(h0) + h2f(l0), e1 = h2f(h1) + h2f(l1);
        const int q0 = lane & 48;
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            sum += __shfl(e0, q0 + i, 64);
            sum += __shfl(e1, q0 + i, 64);
        }
        if ((lane & 15) == 0) a.xsum[(size_t)t * nblk + h * 4 + (lane >> 4)] = sum;
    }
}

hipError_t launch_attn_combine(const AttnCombineArgs &a, hipStream_t s)
{
    if (a.T <= 0) return hipSuccess;
    if (a.t0 < 0 || a.n_heads < 1 || a.max_chunks < 1 || !a.part || !a.ot || !a.slot || !a.shared_lo || !a.shared_hi ||
        !a.segment)
        return hipErrorInvalidValue;
    launch_stamped(a.ev_start, a.ev_stop, attn_combine_kernel, dim3(a.T, a.n_heads), dim3(64), 0, s, a);
    return hipGetLastError();
}

} // namespace jev
