// Prefill GEMM against GGUF-quantized weights: y = x . W^T on the MFMA cores.
//
// Replaces PanelGemm (PanelGemm.cs:87-318) for calls of two or more tokens.
//
// Numerics.  The weight quants are small integers (Q8_0 q in [-127,127],
// Q4_0 q-8 in [-8,7], Q5_1 q in [0,31]) and therefore exact in fp16; only the
// per-32 block scale d (and Q5_1's min m) is not.  One MFMA of 16x16x32 covers
// exactly one quant block, so each block's dot of x with the integer quants
// comes out of the matrix core unscaled and the fp32 scale is applied on the
// vector ALU:  acc += d * (x . q)  (+ m * sum(x) for Q5_1).  The activation x
// enters as an fp16 pair hi + lo (two MFMAs into the same partial), ~22
// significant bits; a single fp16 or bf16 operand measured 4e-3 / 2e-2
// relative error on the 26-layer logits, the pair 3e-5.
//
// Determinism.  Each output is the same sequence of MFMAs and FMAs over its K
// blocks whatever M is and whichever tile shape or position its row lands in,
// so a token's result does not depend on the batch around it (the reference's
// batch invariance, PanelGemm.cs:28-31); that is what keeps a tree pass
// bit-identical to running its branches one at a time.  Tile shapes may
// therefore be chosen by M without changing a single bit.
//
// Pipeline.  K advances 64 (two quant blocks) per stage.  Weights stream from
// HBM as raw quant bytes into registers two stages ahead, are decoded to fp16
// integers into a double-buffered LDS tile one stage ahead ("dequant in LDS":
// each decoded weight feeds every row of the tile), and the activation
// fragments are loaded straight from global memory (L2-resident) into the
// MFMA operand registers one stage ahead.  One barrier per stage.
//
// Outputs.  Store-mode results (and K-split partials) are written with
// nontemporal stores: their consumer runs on whichever XCD its workgroup lands
// on, so they must reach memory anyway.  Streamed out during the kernel rather
// than written back from L2 after it, the 256-row projections launched back
// to back took 1-6 % less time (QKV 25.4 -> 24.8 us, O 18.7 -> 17.8, down
// 34.9 -> 34.3); in the model, between other kernels, under 0.5 %.
//
// Tiles.  4 waves.  This dequant-in-LDS kernel serves segment lists the
// B-direct kernel below cannot split (64 x 64 tiles at small M, 128 x 128 at
// large M); the B-direct kernel takes everything else.  Workgroup ids are remapped so each XCD (ids round-robin over 8) works on a
// contiguous run of a grouped tile order: neighbouring tiles on one XCD share
// weight and activation tiles in its L2.  LDS rows are padded to 72 halves
// (144 B) so 16-byte fragment reads of 8 lanes hit distinct banks.
#include "jev_dev.h"

#include <type_traits>

namespace jev {

namespace {

constexpr int BK = 64;           // K per stage (two quant blocks)
constexpr int LROW = BK + 8;     // padded LDS row, halves

struct alignas(16) u32x4 {
    uint32_t x, y, z, w;
};


// One loader chunk: a lane slot of a weight tile -- the quants of one row
// at k = 8g .. 8g + 7 of both blocks of the stage -- and that row's scales.
struct BChunk {
    uint4 q;       // bytes (Q8_0, Q5_1's byte copy): 16; nibbles (Q4_0, Q5_1's fields): 8 in .x, .y
    uint32_t d, m; // two fp16 each (block 0 low half)
    uint32_t qh;   // Q5_1 from its 5-bit fields: the lane's fifth bits (block 0 low byte)
};

// Segment and local row of tile column rr (epilogue).
template <int MODE, int BN>
__device__ __forceinline__ void map_row(const GemmArgs &a, int tile_n, int rr, int &seg, int &row)
{
    if (MODE == kGemmSwiGlu) {
        int sub = rr >> 4;
        seg = sub & 1;
        row = tile_n * (BN / 2) + (sub >> 1) * 16 + (rr & 15);
    } else {
        int n0 = tile_n * BN;
        int s = 0, start = 0;
        while (s + 1 < a.nseg && n0 >= start + a.seg[s].rows) {
            start += a.seg[s].rows;
            s++;
        }
        seg = s;
        row = n0 - start + rr;
    }
}

// Loads are unconditional with clamped addresses: a row past the weight's end
// or a block past K only feeds outputs that are never stored, and keeping the
// loop free of divergent loads lets the compiler count outstanding loads
// exactly instead of draining the queue every stage.

// Quants as these kernels read them.  BQ (byte quants): whole bytes, 1 KiB
// per tile -- Q8_0's (QWeight::qs, stored biased as q + 128) or Q5_1's byte
// copy (QWeight::qb, q itself).  Otherwise 512 B of nibbles per tile (QWeight::qs:
// Q4_0, or Q5_1's low four bits with the fifth bits in QWeight::qh).  Q8_0
// is always bytes, Q4_0 always nibbles; Q5_1 is bytes wherever the kernel's
// registers allow the 16-byte chunk (all but the 64 x 256 tile): one byte
// permute and one packed subtraction per two weights instead of the nibble
// and fifth-bit assembly.  The decoded integers are the same either way.
template <int TYPE, bool BQ>
__device__ __forceinline__ rsrc_t quant_rsrc(const QWeight &w, uint32_t tiles)
{
    return make_rsrc(TYPE == kQ5_1 && BQ ? w.qb : w.qs, tiles * (BQ ? 1024u : 512u));
}

// Four quants of a block as two fp16 pairs of exact integers: a byte b placed
// under the exponent byte is 1024 + b; the bias subtracts 1024 and, for Q8_0's
// biased bytes or Q4_0's offset 8, that too.
template <int TYPE, bool BQ>
__device__ __forceinline__ void decode4(const BChunk &c, int bb, int half, uint32_t &pa, uint32_t &pb)
{
    if (BQ) {
        const uint32_t w = bb ? (half ? c.q.w : c.q.z) : (half ? c.q.y : c.q.x);
        bytes_to_f16(w, TYPE == kQ8_0 ? (_Float16)1152.0f : (_Float16)1024.0f, pa, pb);
    } else {
        // byte i = element i (low nibble) | element i + 4 (high nibble)
        const uint32_t w = bb ? c.q.y : c.q.x;
        uint32_t n = half ? (w >> 4) & 0x0f0f0f0fu : w & 0x0f0f0f0fu;
        _Float16 bias = (_Float16)1032.0f;
        if (TYPE == kQ5_1) {
            // fifth bits: spread 4 bits to bit 4 of each byte
            const uint32_t hb = (c.qh >> (8 * bb)) & 0xffu;
            n |= ((((half ? hb >> 4 : hb & 15u)) * 0x00204081u) & 0x01010101u) << 4;
            bias = (_Float16)1024.0f;
        }
        bytes_to_f16(n, bias, pa, pb);
    }
}

// B fragment of block bb of a loaded chunk: 8 fp16 integers for the lane's
// row at k = 8g .. 8g + 7.
template <int TYPE, bool BQ>
__device__ __forceinline__ half8_t decode_b_frag(const BChunk &c, int bb)
{
    uint32_t o0, o1, o2, o3;
    decode4<TYPE, BQ>(c, bb, 0, o0, o1);
    decode4<TYPE, BQ>(c, bb, 1, o2, o3);
    return __builtin_bit_cast(half8_t, make_uint4(o0, o1, o2, o3));
}

// Decoded quants of one chunk as fp16 integers: block 0 to dst[0..8),
// block 1 to dst[32..40) (the LDS row of the chunk's weight row).
template <int TYPE, bool BQ>
__device__ __forceinline__ void store_chunk(const BChunk &c, uint16_t *dst)
{
#pragma unroll
    for (int bb = 0; bb < 2; bb++) {
        uint32_t o0, o1, o2, o3;
        decode4<TYPE, BQ>(c, bb, 0, o0, o1);
        decode4<TYPE, BQ>(c, bb, 1, o2, o3);
        *(u32x4 *)(dst + 32 * bb) = u32x4{o0, o1, o2, o3};
    }
}

// A fragments of one stage: [mi][kb2] hi and lo.
template <int TM>
struct AFrag {
    half8_t hi[TM][2], lo[TM][2];
    floatx4 s[TM][2]; // Q5_1 block sums of the lane's 4 C rows
};

} // namespace

// KS: quant blocks whose partials are in flight together (1 or 2); OCC:
// waves per SIMD the register budget is cut for.
template <int TYPE, int MODE, int WM, int WN, int TM, int TN, int PD, int KS, int OCC>
__global__ __launch_bounds__(256, OCC) void gemm_q_kernel(GemmArgs a, int mt, int nt, int gm)
{
    constexpr int BM = WM * TM * 16, BN = WN * TN * 16;
    constexpr int CHUNKS = BN * 4; // 64 lane slots per 16-row weight tile
    constexpr int CPT = (CHUNKS + 255) / 256;
    constexpr int NG = TN < 4 ? TN : 4; // N tiles per partial group
    // One spare chunk / scale slot past each tile: loaders with nothing to
    // store write there, so no store (and no wait on its load) is conditional.
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LROW + 40];
    __shared__ float Ds[2][BN * 2 + 2];
    __shared__ float Ms[2][TYPE == kQ5_1 ? BN * 2 + 2 : 1];

    // ---- tile of this workgroup: contiguous per-XCD runs of a grouped order
    const int total = gridDim.x;
    const int per_xcd = total >> 3;
    const int L = blockIdx.x;
    int Lp = (L & 7) * per_xcd + (L >> 3);
    // K split z (partials of store-mode GEMMs): whole runs of the tile order
    const int tiles8 = total / a.ksplit;
    const int z = Lp / tiles8;
    Lp -= z * tiles8;
    const int group = gm * nt;
    const int first_m = (Lp / group) * gm;
    const int gsz = min(mt - first_m, gm);
    if (gsz <= 0) return;
    const int tile_m = first_m + (Lp % group) % gsz;
    const int tile_n = (Lp % group) / gsz;
    if (tile_m >= mt || tile_n >= nt) return;

    // wave-uniform in a scalar register (a vector value can turn the loads'
    // scalar offsets into per-lane loops)
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int M = a.M, K = a.K, nblk = K >> 5;
    // this split's K blocks: [kb_begin, kb_begin + nb)
    const int nb_per = gemm_split_blocks(nblk, a.ksplit);
    const int kb_begin = z * nb_per;
    const int nb = min(nblk - kb_begin, nb_per);
    const int nstage = (nb + 1) >> 1;
    const int m0 = tile_m * BM;

    // ---- loader role (B): chunk c = tid + 256 j is lane slot c % 64 of the
    // tile row c / 64 of the workgroup's BN weight rows -- one tile per wave,
    // so its weight (segment) is uniform.  Every load is a buffer load: a
    // scalar resource, a per-lane offset fixed for the loop and a scalar
    // per-stage offset; no per-stage vector address arithmetic.
    rsrc_t rq[CPT], rd[CPT];
    int btile0[CPT]; // first tile of the chunk's row group (uniform)
    int b_lds[CPT], b_ds[CPT];
    const int slot = tid & 63, sg = slot >> 4, sr = slot & 15;
    constexpr bool BQ = TYPE != kQ4_0; // byte quants (see quant_rsrc)
    const uint32_t vq = (uint32_t)slot * (BQ ? 16 : 8), vd = 4 * sr;
    const int kp_begin = kb_begin >> 1; // kb_begin is even
#pragma unroll
    for (int j = 0; j < CPT; j++) {
        const int t = wave + 4 * j; // tile row within the workgroup
        const bool own = 16 * t < BN; // waves past the tile load a duplicate and store it in the spare slot
        int seg, rgw;
        if (MODE == kGemmSwiGlu) {
            // 16-row groups alternate gate (segment 0) and up (segment 1)
            seg = t & 1;
            rgw = tile_n * (BN / 32) + (t >> 1);
        } else {
            int s0 = 0, start = 0, n0 = tile_n * BN;
            while (s0 + 1 < a.nseg && n0 >= start + a.seg[s0].rows) {
                start += a.seg[s0].rows;
                s0++;
            }
            seg = s0;
            rgw = (n0 - start) / 16 + t; // segments but the last are whole tiles
        }
        seg = __builtin_amdgcn_readfirstlane(seg);
        const QWeight &w = a.seg[seg];
        const int KP = tile_kpairs(w.cols), RG = tile_rows(w.rows);
        const uint32_t tiles = (uint32_t)RG * KP;
        rq[j] = quant_rsrc<TYPE, BQ>(w, tiles);
        rd[j] = make_rsrc(w.d, tiles * tile_d_bytes(TYPE));
        // row groups past the weight feed unstored columns
        btile0[j] = __builtin_amdgcn_readfirstlane(min(rgw, RG - 1) * KP + kp_begin);
        b_lds[j] = own ? (16 * t + sr) * LROW + 8 * sg : BN * LROW;
        // lanes of the first k group store the row's two scales, the rest the spare slot
        b_ds[j] = own && sg == 0 ? (16 * t + sr) * 2 : BN * 2;
    }
    // A stage past the end reloads the last one.  An odd block count leaves
    // the last stage's second block to the tile padding (zero quants and
    // scales) or to the next split's first block; either way it only feeds
    // the skipped second half.
    auto load_b = [&](int st, BChunk (&br)[CPT]) {
        st = min(st, nstage - 1);
#pragma unroll
        for (int j = 0; j < CPT; j++) {
            const int tile = btile0[j] + st;
            if (BQ) {
                br[j].q = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq[j], vq, tile * 1024, 0));
            } else {
                uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rq[j], vq, tile * 512, 0));
                br[j].q = make_uint4(v.x, v.y, 0u, 0u);
            }
            if (TYPE == kQ5_1) {
                // the row's scales and mins in one load
                const uint2 dm = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rd[j], 2 * vd, tile * 128, 0));
                br[j].d = dm.x;
                br[j].m = dm.y;
            } else {
                br[j].d = __builtin_amdgcn_raw_buffer_load_b32(rd[j], vd, tile * 64, 0);
            }
        }
    };
    auto store_b = [&](int buf, const BChunk (&br)[CPT]) {
#pragma unroll
        for (int j = 0; j < CPT; j++) {
            store_chunk<TYPE, BQ>(br[j], &Bs[buf][b_lds[j]]);
            Ds[buf][b_ds[j]] = h2f((uint16_t)br[j].d);
            Ds[buf][b_ds[j] + 1] = h2f((uint16_t)(br[j].d >> 16));
            if (TYPE == kQ5_1) {
                Ms[buf][b_ds[j]] = h2f((uint16_t)br[j].m);
                Ms[buf][b_ds[j] + 1] = h2f((uint16_t)(br[j].m >> 16));
            }
        }
    };

    // ---- A fragments straight from global memory: each is one contiguous
    // 1 KiB operand tile (xt_index layout), one 16-byte load per lane.
    const int rg0 = (m0 >> 4) + wm * TM;
    const int frag_k = 8 * (lane >> 4); // k offset of this lane's B fragment within a block
    const int rg_last = (M - 1) >> 4; // groups past M feed unstored rows
    const rsrc_t ra = make_rsrc(a.xt, (uint32_t)(rg_last + 1) * nblk * 2048);
    uint32_t va[TM];
#pragma unroll
    for (int mi = 0; mi < TM; mi++) va[mi] = ((uint32_t)min(rg0 + mi, rg_last) * nblk * 1024 + lane * 8) * 2;
    rsrc_t rs;
    uint32_t vs[TM];
    if (TYPE == kQ5_1) {
        rs = make_rsrc(a.xsum, (uint32_t)M * nblk * 4);
#pragma unroll
        for (int mi = 0; mi < TM; mi++) vs[mi] = (uint32_t)(m0 + wm * TM * 16 + mi * 16 + 4 * (lane >> 4)) * nblk * 4;
    }
    auto load_a = [&](int st, AFrag<TM> &f) {
        st = min(st, nstage - 1);
#pragma unroll
        for (int mi = 0; mi < TM; mi++) {
#pragma unroll
            for (int kb2 = 0; kb2 < 2; kb2++) {
                const int kblk = kb_begin + min(2 * st + kb2, nb - 1);
                f.hi[mi][kb2] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(ra, va[mi], kblk * 2048, 0));
                f.lo[mi][kb2] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(ra, va[mi] + 1024, kblk * 2048, 0));
                if (TYPE == kQ5_1) {
                    // rows past M read zeros (outside the buffer) and are never stored
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        f.s[mi][kb2][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, vs[mi] + r * nblk * 4, kblk * 4, 0));
                }
            }
        }
    };

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // Per block: p = x_hi . q, p += x_lo . q (MFMA), acc = fma(d, p, acc)
    // (+ m * sum(x)).  KS blocks' partials are in flight together so each MFMA
    // result is consumed several MFMAs after it issues; the FMAs still apply
    // block 0 before block 1 for every output.
    static_assert(KS == 1 || KS == 2, "one or two blocks in flight");
    auto compute = [&](int st, int buf, const AFrag<TM> &f) {
        const bool second = 2 * st + 1 < nb;
#pragma unroll
        for (int k0 = 0; k0 < 2; k0 += KS) {
#pragma unroll
            for (int g = 0; g < TN / NG; g++) {
                half8_t fb[KS][NG];
                float dsc[KS][NG], mn[KS][NG];
                floatx4 p[KS][TM][NG];
#pragma unroll
                for (int kk = 0; kk < KS; kk++)
#pragma unroll
                    for (int n = 0; n < NG; n++) {
                        int c = wn * TN * 16 + (g * NG + n) * 16 + (lane & 15);
                        fb[kk][n] = *(const half8_t *)(&Bs[buf][c * LROW + (k0 + kk) * 32 + frag_k]);
                        dsc[kk][n] = Ds[buf][c * 2 + k0 + kk];
                        if (TYPE == kQ5_1) mn[kk][n] = Ms[buf][c * 2 + k0 + kk];
                    }
#pragma unroll
                for (int kk = 0; kk < KS; kk++)
#pragma unroll
                    for (int mi = 0; mi < TM; mi++)
#pragma unroll
                        for (int n = 0; n < NG; n++)
                            p[kk][mi][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.hi[mi][k0 + kk], fb[kk][n],
                                                                                   floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int kk = 0; kk < KS; kk++)
#pragma unroll
                    for (int mi = 0; mi < TM; mi++)
#pragma unroll
                        for (int n = 0; n < NG; n++)
                            p[kk][mi][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.lo[mi][k0 + kk], fb[kk][n],
                                                                                   p[kk][mi][n], 0, 0, 0);
#pragma unroll
                for (int kk = 0; kk < KS; kk++) {
                    // an odd block count's missing second block adds 0 * p (p is finite):
                    // no branch inside the stage's straight-line code
                    const bool live = k0 + kk == 0 || second;
#pragma unroll
                    for (int mi = 0; mi < TM; mi++)
#pragma unroll
                        for (int n = 0; n < NG; n++)
#pragma unroll
                            for (int r = 0; r < 4; r++) {
                                float v = fmaf(live ? dsc[kk][n] : 0.f, p[kk][mi][n][r], acc[mi][g * NG + n][r]);
                                if (TYPE == kQ5_1) v = fmaf(live ? mn[kk][n] : 0.f, f.s[mi][k0 + kk][r], v);
                                acc[mi][g * NG + n][r] = v;
                            }
                }
            }
        }
    };

    // ---- software pipeline.  Ring of U = PD + 1 register slots: A fragments
    // are loaded PD stages ahead, raw weight chunks PD + 1 stages ahead (they
    // are decoded into LDS one stage before use).  The loop is unrolled by U
    // so every ring index is a compile-time constant.
    constexpr int U = PD + 1;
    BChunk br[U][CPT];
    AFrag<TM> fa[U];
#pragma unroll
    for (int j = 0; j < PD; j++) load_a(j, fa[j]);
#pragma unroll
    for (int j = 0; j <= PD; j++) load_b(j, br[j]);
    store_b(0, br[0]);
    __syncthreads();

    // Stage s: compute it (LDS buffer s & 1, A slot s % U), decode stage
    // s + 1 into the other buffer, refill the freed slots.  The loop runs
    // whole groups of U stages only and the remainder follows it: a loop with
    // exits inside its body would merge a half-advanced ring into the loop
    // header, where the compiler would then drain every outstanding load.
    auto stage = [&](auto jc, int s) {
        constexpr int j = decltype(jc)::value;
        load_a(s + PD, fa[(j + PD) % U]);
        compute(s, s & 1, fa[j]);
        store_b((s + 1) & 1, br[(j + 1) % U]);
        load_b(s + PD + 1, br[j]);
        __syncthreads();
    };
    const int ngroups = nstage / U;
    int s0 = 0;
    for (int g = 0; g < ngroups; g++, s0 += U) {
        stage(std::integral_constant<int, 0>{}, s0);
        if constexpr (U > 1) stage(std::integral_constant<int, 1 % U>{}, s0 + 1);
        if constexpr (U > 2) stage(std::integral_constant<int, 2 % U>{}, s0 + 2);
        if constexpr (U > 3) stage(std::integral_constant<int, 3 % U>{}, s0 + 3);
        static_assert(U <= 4, "ring deeper than the unrolled group");
    }
    {
        const int rem = nstage - s0;
        if constexpr (U > 1) if (rem > 0) stage(std::integral_constant<int, 0>{}, s0);
        if constexpr (U > 2) if (rem > 1) stage(std::integral_constant<int, 1 % U>{}, s0 + 1);
        if constexpr (U > 3) if (rem > 2) stage(std::integral_constant<int, 2 % U>{}, s0 + 2);
    }

    // ---- epilogue.  Lane holds C[4*(lane/16) + r][lane % 16] of each 16x16 tile.
    const int row_base = m0 + wm * TM * 16 + 4 * (lane >> 4);
    if (MODE == kGemmStore) {
        float *y = a.y + (size_t)z * M * a.ldy;
        int seg, r0;
        map_row<MODE, BN>(a, tile_n, 0, seg, r0); // segment and local row of the tile's first column
        const QWeight &ws = a.seg[seg];
        const int col0 = tile_n * BN;
#pragma unroll
        for (int j = 0; j < TN; j++) {
            int off = wn * TN * 16 + j * 16 + (lane & 15);
            if (r0 + off >= ws.rows) continue;
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    int row = row_base + 16 * i + r;
                    if (row < M) __builtin_nontemporal_store(acc[i][j][r], &y[(size_t)row * a.ldy + col0 + off]);
                }
        }
    } else {
        const int ld = a.seg[0].rows;
        const int cbase = tile_n * (BN / 2);
#pragma unroll
        for (int pp = 0; pp < TN / 2; pp++) {
            // N tiles 2pp (gate) and 2pp+1 (up) of this wave cover the same outputs
            int col = cbase + ((wn * TN + 2 * pp) >> 1) * 16 + (lane & 15);
            if (col >= ld) continue;
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    int row = row_base + 16 * i + r;
                    if (row >= M) continue;
                    // Kernels.SwiGlu (Kernels.cs:82-89): (g*u) * sigmoid(g).
                    float g = acc[i][2 * pp][r], u = acc[i][2 * pp + 1][r];
                    float gu = g * u;
                    float e = expf(-g);
                    float sg = 1.0f / (1.0f + e);
                    float v = sg * gu;
                    uint16_t hi, lo;
                    split_f16(v, hi, lo);
                    a.ot[xt_index(row, col, ld >> 5, 0)] = hi;
                    a.ot[xt_index(row, col, ld >> 5, 1)] = lo;
                }
        }
    }
}

// ---------------------------------------------------------------------------
// B-direct variant: the four waves sit side by side along N, each owning TN
// weight tiles (16 rows each) that it streams from HBM straight into
// registers and decodes there -- a tile slot is exactly the lane's B fragment
// -- while the BM x 64 activation tile of a stage is loaded once per
// workgroup into LDS and read by all four waves.  Per MFMA this moves half
// the bytes through the vector-memory path and the LDS of the variant above
// (whose B tile goes through LDS and whose A fragments come per wave from
// L2).  The arithmetic per output is the same sequence of MFMAs and FMAs, so
// the two variants agree bit for bit and either may serve any M.
//
// FOLD: the workgroup walks every K-split range of its tile in order (the
// grid has no split dimension), each range's chain from zero as a split
// workgroup would run it, and keeps the ranges' sum in split order in a
// second accumulator set; it stores that sum once instead of ksplit partials.
//
// NW: waves per workgroup, side by side along N (BN = 16 TN NW).  Twelve
// waves share one activation tile three times as wide as four do: a third of
// the activation loads and LDS stores per MFMA.  At 256 rows of the 3B
// projections that gives 256 workgroups of 12 waves, one per CU and the same
// three waves per SIMD as 768 workgroups of four (QKV 27.4 -> 26.2 us, O 20.0
// -> 19.2, down 39.1 -> 36.2; cold weights).
template <int TYPE, int MODE, int TM, int TN, int PD, int OCC, bool FOLD = false, int NW = 4>
__global__ __launch_bounds__(64 * NW, OCC) void gemm_bd_kernel(GemmArgs a, int mt, int nt, int gm)
{
    constexpr int BM = 16 * TM, BN = 16 * TN * NW;
    constexpr int U = PD + 1; // weight register ring
    static_assert(!FOLD || MODE == kGemmStore, "folded K splits are a store-mode form");
    static_assert(NW % 4 == 0, "whole groups of four waves");
    __shared__ __attribute__((aligned(16))) uint16_t As[2][TM * 4 * 512]; // [mi][block][part] operand tiles

    // ---- tile of this workgroup (same order and K splits as gemm_q_kernel)
    const int total = gridDim.x;
    const int per_xcd = total >> 3;
    const int L = blockIdx.x;
    int Lp = (L & 7) * per_xcd + (L >> 3);
    const int tiles8 = FOLD ? total : total / a.ksplit;
    const int z = FOLD ? 0 : Lp / tiles8;
    Lp -= z * tiles8;
    const int group = gm * nt;
    const int first_m = (Lp / group) * gm;
    const int gsz = min(mt - first_m, gm);
    if (gsz <= 0) return;
    const int tile_m = first_m + (Lp % group) % gsz;
    const int tile_n = (Lp % group) / gsz;
    if (tile_m >= mt || tile_n >= nt) return;

    // wave-uniform in a scalar register: the activation loads' scalar offset
    // depends on it, and a vector one would make the compiler wrap each load in
    // a one-pass loop that drains every outstanding load at the next wait
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = a.M, K = a.K, nblk = K >> 5;
    const int nb_per = gemm_split_blocks(nblk, a.ksplit);
    const int kb_begin = z * nb_per;
    const int nb = FOLD ? nblk : min(nblk - kb_begin, nb_per); // blocks this workgroup walks
    const int nstage = (nb + 1) >> 1;
    const int m0 = tile_m * BM;

    // ---- activation loader: the stage's TM * 4 fragments (row group mi,
    // block f >> 1, part f & 1 for fragment 4 mi + f) of 1 KiB go to the waves
    // round robin, wave w taking fragments w, w + NW, ...; each lane loads its
    // 16-byte slot.  With four waves, wave w takes fragment f = w of every row
    // group.  Past the last fragment a wave repeats it (the same bytes to the
    // same LDS slot).
    const int rg_last = (M - 1) >> 4; // groups past M feed unstored rows
    const rsrc_t ra = make_rsrc(a.xt, (uint32_t)(rg_last + 1) * nblk * 2048);
    constexpr int NCH = TM * 4, AL = (NCH + NW - 1) / NW;
    int ach[AL], abb[AL];
    uint32_t va[AL];
#pragma unroll
    for (int j = 0; j < AL; j++) {
        // four waves: fragment `wave` of row group j (block and part are the wave's for every j)
        const int ch = NW == 4 ? 4 * j + wave : min(wave + NW * j, NCH - 1);
        const int mi = NW == 4 ? j : ch >> 2, part = NW == 4 ? wave & 1 : ch & 1;
        ach[j] = ch;
        abb[j] = NW == 4 ? wave >> 1 : (ch >> 1) & 1;
        va[j] = (((uint32_t)min((m0 >> 4) + mi, rg_last) * nblk * 2 + part) * 512 + lane * 8) * 2;
    }
    // Q5_1 block sums of the stage's BM rows x 2 blocks, one per thread of the
    // first 2 * BM, staged through LDS with the activations.  The block index
    // rides in the per-thread offset so the scalar offset stays uniform; the
    // other threads read past the buffer (zeros).  A missing odd last block
    // reads a finite neighbour that its zero min cancels.
    __shared__ __attribute__((aligned(16))) float Xs[2][TYPE == kQ5_1 ? 64 * NW : 4]; // [bb * BM + row], the rest unused
    rsrc_t rs;
    uint32_t vx = 0;
    if (TYPE == kQ5_1) {
        rs = make_rsrc(a.xsum, (uint32_t)M * nblk * 4);
        vx = tid < 2 * BM ? ((uint32_t)(m0 + tid % BM) * nblk + tid / BM) * 4 : 0x40000000u;
    }
    struct AStage {
        uint4 v[AL];
        float xs;
    };
    auto load_a = [&](int st, AStage &r) __attribute__((always_inline)) {
        st = min(st, nstage - 1);
#pragma unroll
        for (int j = 0; j < AL; j++) {
            const int kblk = kb_begin + min(2 * st + (NW == 4 ? abb[0] : abb[j]), nb - 1);
            r.v[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ra, va[j], kblk * 2048, 0));
        }
        if (TYPE == kQ5_1) r.xs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, vx, (kb_begin + 2 * st) * 4, 0));
    };
    auto store_a = [&](int buf, const AStage &r) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < AL; j++) *(uint4 *)&As[buf][(NW == 4 ? j * 4 + wave : ach[j]) * 512 + lane * 8] = r.v[j];
        if (TYPE == kQ5_1) Xs[buf][tid] = r.xs;
    };

    // ---- weight loader: tile n of this wave is tile row wave * TN + n of the workgroup
    // byte quants (see quant_rsrc), Q5_1 but in the 64 x 256 tile
    constexpr bool BQ = TYPE == kQ8_0 || (TYPE == kQ5_1 && TM * TN < 16);
    rsrc_t rq[TN], rd[TN], rh[TN];
    int btile0[TN];
    const uint32_t vq = (uint32_t)lane * (BQ ? 16 : 8), vd = 4 * (lane & 15), vh = 2 * lane;
#pragma unroll
    for (int n = 0; n < TN; n++) {
        const int t = wave * TN + n;
        int seg, rgw;
        if (MODE == kGemmSwiGlu) {
            seg = t & 1; // 16-row groups alternate gate and up
            rgw = tile_n * (BN / 32) + (t >> 1);
        } else {
            // the segment of the workgroup's tile (four waves: a tile never
            // straddles two) or of this wave's 16 TN rows (which never do)
            int s0 = 0, start = 0;
            const int r0 = tile_n * BN + (NW == 4 ? 0 : 16 * t);
            while (s0 + 1 < a.nseg && r0 >= start + a.seg[s0].rows) {
                start += a.seg[s0].rows;
                s0++;
            }
            seg = s0;
            rgw = (r0 - start) / 16 + (NW == 4 ? t : 0);
        }
        seg = __builtin_amdgcn_readfirstlane(seg);
        const QWeight &w = a.seg[seg];
        const int KP = tile_kpairs(w.cols), RG = tile_rows(w.rows);
        const uint32_t tiles = (uint32_t)RG * KP;
        rq[n] = quant_rsrc<TYPE, BQ>(w, tiles);
        rd[n] = make_rsrc(w.d, tiles * tile_d_bytes(TYPE));
        if (TYPE == kQ5_1 && !BQ) rh[n] = make_rsrc(w.qh, tiles * 128);
        btile0[n] = __builtin_amdgcn_readfirstlane(min(rgw, RG - 1) * KP + (kb_begin >> 1));
    }
    auto load_b = [&](int st, BChunk (&br)[TN]) __attribute__((always_inline)) {
        st = min(st, nstage - 1);
#pragma unroll
        for (int n = 0; n < TN; n++) {
            const int tile = btile0[n] + st;
            if (BQ) {
                br[n].q = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq[n], vq, tile * 1024, 0));
            } else {
                uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rq[n], vq, tile * 512, 0));
                br[n].q = make_uint4(v.x, v.y, 0u, 0u);
            }
            if (TYPE == kQ5_1) {
                const uint2 dm = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rd[n], 2 * vd, tile * 128, 0));
                br[n].d = dm.x;
                br[n].m = dm.y;
                if (!BQ) br[n].qh = __builtin_amdgcn_raw_buffer_load_b16(rh[n], vh, tile * 128, 0);
            } else {
                br[n].d = __builtin_amdgcn_raw_buffer_load_b32(rd[n], vd, tile * 64, 0);
            }
        }
    };

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    // FOLD: the finished ranges' sum in split order; a range of spr stages ends
    // after stage done - 1 when done is a multiple of spr
    floatx4 tot[FOLD ? TM : 1][FOLD ? TN : 1];
    const int spr = nb_per >> 1;
    auto fold_range = [&](int done) __attribute__((always_inline)) {
        if constexpr (FOLD) {
            if (done % spr != 0 || done >= nstage) return;
            const bool first = done == spr;
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
#pragma unroll
                    for (int r = 0; r < 4; r++) tot[i][j][r] = first ? acc[i][j][r] : tot[i][j][r] + acc[i][j][r];
                    acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
                }
        }
    };

    // Large tiles: the scale FMAs of a tile trail its MFMA pair by two pairs
    // (the result is ready by then, so the vector ALU works beside the matrix
    // core instead of waiting on it; 2-4 % at 4528 rows, nothing at 256).
    // Each accumulator still takes its blocks' FMAs in block order, so the
    // arithmetic is that of the plain order.
    auto compute = [&](int st, int buf, const BChunk (&br)[TN]) __attribute__((always_inline)) {
        const bool second = 2 * st + 1 < nb;
        constexpr int LAG = TM * TN >= 16 ? 2 : 0, NQ = 2 * TM * TN;
        floatx4 pq[LAG > 0 ? LAG : 1], xq[LAG > 0 ? LAG : 1];
        float dq[LAG > 0 ? LAG : 1], mq[LAG > 0 ? LAG : 1];
        auto apply = [&](int t) __attribute__((always_inline)) {
            const int mt_ = (t / TN) % TM, nt_ = t % TN, k = LAG > 0 ? t % LAG : 0;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float v = fmaf(dq[k], pq[k][r], acc[mt_][nt_][r]);
                if (TYPE == kQ5_1) v = fmaf(mq[k], xq[k][r], v);
                acc[mt_][nt_][r] = v;
            }
        };
#pragma unroll
        for (int bb = 0; bb < 2; bb++) {
            // an odd block count's missing second block adds 0 * p (p is finite)
            // (a mask rather than a select: the compiler turns a select on a
            // uniform condition into branches around the conversions)
            const uint32_t live = bb == 0 || second ? ~0u : 0u;
            half8_t bf[TN];
            float dv[TN], mv[TN];
#pragma unroll
            for (int n = 0; n < TN; n++) {
                bf[n] = decode_b_frag<TYPE, BQ>(br[n], bb);
                dv[n] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, h2f((uint16_t)(bb ? br[n].d >> 16 : br[n].d))) & live);
                if (TYPE == kQ5_1)
                    mv[n] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, h2f((uint16_t)(bb ? br[n].m >> 16 : br[n].m))) & live);
            }
#pragma unroll
            for (int mi = 0; mi < TM; mi++) {
                const half8_t ah = *(const half8_t *)&As[buf][(mi * 4 + bb * 2 + 0) * 512 + lane * 8];
                const half8_t al = *(const half8_t *)&As[buf][(mi * 4 + bb * 2 + 1) * 512 + lane * 8];
                floatx4 xs4; // block sums of the lane's four C rows
                if (TYPE == kQ5_1) xs4 = *(const floatx4 *)&Xs[buf][bb * BM + mi * 16 + 4 * (lane >> 4)];
#pragma unroll
                for (int n = 0; n < TN; n++) {
                    floatx4 p = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bf[n], floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bf[n], p, 0, 0, 0);
                    if constexpr (LAG == 0) {
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            float v = fmaf(dv[n], p[r], acc[mi][n][r]);
                            if (TYPE == kQ5_1) v = fmaf(mv[n], xs4[r], v);
                            acc[mi][n][r] = v;
                        }
                    } else {
                        const int q = (bb * TM + mi) * TN + n;
                        if (q >= LAG) apply(q - LAG);
                        pq[q % LAG] = p;
                        dq[q % LAG] = dv[n];
                        if (TYPE == kQ5_1) {
                            xq[q % LAG] = xs4;
                            mq[q % LAG] = mv[n];
                        }
                        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0); // the pair's MFMAs
                        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0); // then vector work
                    }
                }
            }
        }
        if constexpr (LAG > 0) {
#pragma unroll
            for (int t = NQ - LAG; t < NQ; t++) apply(t);
        }
    };

    // ---- pipeline: weights U stages ahead in a register ring; activations
    // loaded UA stages ahead into a register ring (stage t in slot t % UA)
    // and copied to LDS (double buffered) by the stage before their own.
    // Whole groups of U stages in the loop, the remainder after it (see
    // gemm_q_kernel).  The prologue issues its loads in the loop's order
    // (activations of stage t + 1, then weights of stage t) so the compiler's
    // wait counts at the loop head, merged over entry and back edge, stay
    // those of the loop.
    // Tall tiles (TM = 4) keep one activation slot: a second would cost the
    // registers of a third resident workgroup.
    constexpr int UA = TM >= 4 ? 1 : U;
    BChunk br[U][TN];
    AStage araw[UA], a0;
    load_a(0, a0);
#pragma unroll
    for (int t = 0; t < U; t++) {
        if (t < UA) load_a(t + 1, araw[(t + 1) % UA]);
        load_b(t, br[t]);
        __builtin_amdgcn_sched_barrier(0);
    }
    store_a(0, a0);
    __syncthreads();
    auto stage = [&](auto jc, int s) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        compute(s, s & 1, br[j]);
        fold_range(s + 1);
        store_a((s + 1) & 1, araw[(j + 1) % UA]);
        load_a(s + 1 + UA, araw[(j + 1) % UA]);
        load_b(s + U, br[j]);
        __syncthreads();
        // keep the next stage's decode below the barrier: hoisted above it,
        // it would wait on the weights loaded one stage ago
        __builtin_amdgcn_sched_barrier(0);
    };
    const int ngroups = nstage / U;
    int s0 = 0;
    for (int g = 0; g < ngroups; g++, s0 += U) {
        stage(std::integral_constant<int, 0>{}, s0);
        if constexpr (U > 1) stage(std::integral_constant<int, 1 % U>{}, s0 + 1);
        if constexpr (U > 2) stage(std::integral_constant<int, 2 % U>{}, s0 + 2);
        if constexpr (U > 3) stage(std::integral_constant<int, 3 % U>{}, s0 + 3);
        static_assert(U <= 4, "ring deeper than the unrolled group");
    }
    {
        const int rem = nstage - s0;
        if constexpr (U > 1) if (rem > 0) stage(std::integral_constant<int, 0>{}, s0);
        if constexpr (U > 2) if (rem > 1) stage(std::integral_constant<int, 1 % U>{}, s0 + 1);
        if constexpr (U > 3) if (rem > 2) stage(std::integral_constant<int, 2 % U>{}, s0 + 2);
    }

    if constexpr (FOLD) {
        if (nstage > spr) {
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[i][j][r] = tot[i][j][r] + acc[i][j][r];
        }
    }

    // ---- epilogue.  Lane holds C[4*(lane/16) + r][lane % 16] of each 16x16 tile.
    const int row_base = m0 + 4 * (lane >> 4);
    if (MODE == kGemmStore) {
        // columns are the segments' rows concatenated; only the last segment
        // may end inside a tile
        float *y = a.y + (size_t)z * M * a.ldy;
        const int n0 = tile_n * BN;
        int seg = 0, start = 0, end = 0;
        if constexpr (NW == 4) {
            // a four-wave tile lies in one segment
            while (seg + 1 < a.nseg && n0 >= start + a.seg[seg].rows) {
                start += a.seg[seg].rows;
                seg++;
            }
            end = start + a.seg[seg].rows;
        } else {
            for (int i = 0; i < a.nseg; i++) end += a.seg[i].rows;
        }
#pragma unroll
        for (int n = 0; n < TN; n++) {
            const int col = n0 + (wave * TN + n) * 16 + (lane & 15);
            if (col >= end) continue;
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = row_base + 16 * i + r;
                    if (row < M) __builtin_nontemporal_store(acc[i][n][r], &y[(size_t)row * a.ldy + col]);
                }
        }
    } else {
        const int ld = a.seg[0].rows;
#pragma unroll
        for (int pp = 0; pp < TN / 2; pp++) {
            // tiles 2pp (gate) and 2pp+1 (up) of this wave cover the same outputs
            const int col = tile_n * (BN / 2) + ((wave * TN + 2 * pp) >> 1) * 16 + (lane & 15);
            if (col >= ld) continue;
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = row_base + 16 * i + r;
                    if (row >= M) continue;
                    // Kernels.SwiGlu (Kernels.cs:82-89): (g*u) * sigmoid(g).
                    const float g = acc[i][2 * pp][r], u = acc[i][2 * pp + 1][r];
                    const float gu = g * u;
                    const float e = expf(-g);
                    const float sg = 1.0f / (1.0f + e);
                    const float v = sg * gu;
                    uint16_t hi, lo;
                    split_f16(v, hi, lo);
                    a.ot[xt_index(row, col, ld >> 5, 0)] = hi;
                    a.ot[xt_index(row, col, ld >> 5, 1)] = lo;
                }
        }
    }
}

// Skinny variant for M <= 16 (one row group: the reasoning decider's rows,
// short branches).  The B-direct grid at such M is N / 128 x splits
// workgroups -- 96 for a 3072-row projection split 4 -- and leaves most of the
// chip's load bandwidth idle.  Here each wave owns one 16-row weight group
// (SwiGLU: the gate and the up group of the same outputs) and the workgroup's
// four waves one K split, 8x the waves of B-direct.  Each wave streams its
// weights through its own U-stage register ring; the activation fragments
// (and Q5_1 block sums), the same for all four waves, are staged into LDS
// once per workgroup in chunks of CH stages, double buffered, with one
// barrier per chunk: loaded into registers at the top of the chunk before,
// written to LDS at its end.  (Direct-to-LDS loads would save the registers,
// but the compiler then drains every outstanding load before the first LDS
// read after them, the weight ring included, once per chunk.)  Per output it issues exactly
// gemm_bd_kernel's sequence: per block p = mfma(x_hi, q); p = mfma(x_lo, q,
// p); acc = fma(d, p, acc) (+ fma(m, sum x, acc)), blocks ascending within the
// split, the same clamped operands for an odd last block -- so its results
// are the same bits.
template <int TYPE, int MODE, int U, int CH>
__global__ __launch_bounds__(256, 2) void gemm_skinny_kernel(GemmArgs a, int ngroups, int nq)
{
    constexpr int TN = MODE == kGemmSwiGlu ? 2 : 1;
    constexpr int NB = 2 * TN; // weight loads per stage
    static_assert(CH % U == 0, "ring slots restart at every chunk");
    static_assert(CH * NB + CH + 1 <= 63, "outstanding loads beyond the vmcnt range");
    __shared__ __attribute__((aligned(16))) uint4 As[2][CH * 4 * 64]; // [stage][block][part][lane]
    __shared__ __attribute__((aligned(16))) float Xs[2][TYPE == kQ5_1 ? CH * 2 * 16 : 4]; // [block][row]

    // Every index below is wave-uniform and kept in scalar registers: the
    // integer divisions are vector-ALU sequences, and left as vector values
    // their results would drag all the per-stage address arithmetic onto the
    // vector ALU with the decode and the scale FMAs.
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int z = __builtin_amdgcn_readfirstlane((int)blockIdx.x / nq), q = blockIdx.x - z * nq;
    const int g = q * 4 + wave;              // this wave's row group; past ngroups: loads only
    const int gl = min(g, ngroups - 1);
    const int M = a.M, K = a.K, nblk = K >> 5;
    const int nb_per = __builtin_amdgcn_readfirstlane(gemm_split_blocks(nblk, a.ksplit));
    const int kb_begin = z * nb_per;
    const int nb = min(nblk - kb_begin, nb_per);
    const int nstage = (nb + 1) >> 1;
    const int nchunk = __builtin_amdgcn_readfirstlane((nstage + CH - 1) / CH);

    const rsrc_t ra = make_rsrc(a.xt, (uint32_t)nblk * 2048); // row group 0 of the operand tiles
    rsrc_t rs;
    if (TYPE == kQ5_1) rs = make_rsrc(a.xsum, (uint32_t)M * nblk * 4);

    // weights: tile n of this wave
    constexpr bool BQ = TYPE != kQ4_0; // byte quants (see quant_rsrc)
    rsrc_t rq[TN], rd[TN];
    int btile0[TN];
    int seg_store = 0, start_store = 0;
    const uint32_t vq = (uint32_t)lane * (BQ ? 16 : 8), vd = 4 * (lane & 15);
#pragma unroll
    for (int n = 0; n < TN; n++) {
        int seg, rgw;
        if (MODE == kGemmSwiGlu) {
            seg = n;
            rgw = gl;
        } else {
            int s0 = 0, start = 0;
            while (s0 + 1 < a.nseg && gl * 16 >= start + a.seg[s0].rows) {
                start += a.seg[s0].rows;
                s0++;
            }
            seg = s0;
            rgw = (gl * 16 - start) / 16;
            seg_store = s0;
            start_store = start;
        }
        seg = __builtin_amdgcn_readfirstlane(seg);
        const QWeight &wt = a.seg[seg];
        const int KP = tile_kpairs(wt.cols), RG = tile_rows(wt.rows);
        const uint32_t tiles = (uint32_t)RG * KP;
        rq[n] = quant_rsrc<TYPE, BQ>(wt, tiles);
        rd[n] = make_rsrc(wt.d, tiles * tile_d_bytes(TYPE));
        btile0[n] = __builtin_amdgcn_readfirstlane(min(rgw, RG - 1) * KP + (kb_begin >> 1));
    }
    auto load_b = [&](int st, BChunk (&br)[TN]) __attribute__((always_inline)) {
        st = min(st, nstage - 1);
#pragma unroll
        for (int n = 0; n < TN; n++) {
            const int tile = __builtin_amdgcn_readfirstlane(btile0[n] + st);
            if (BQ) {
                br[n].q = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq[n], vq, tile * 1024, 0));
            } else {
                uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rq[n], vq, tile * 512, 0));
                br[n].q = make_uint4(v.x, v.y, 0u, 0u);
            }
            if (TYPE == kQ5_1) {
                const uint2 dm = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rd[n], 2 * vd, tile * 128, 0));
                br[n].d = dm.x;
                br[n].m = dm.y;
            } else {
                br[n].d = __builtin_amdgcn_raw_buffer_load_b32(rd[n], vd, tile * 64, 0);
            }
        }
    };
    // Chunk c's activation fragments: this wave's CH of the chunk's 4 * CH,
    // fragment f = stage * 4 + block * 2 + part, one KiB each.
    auto load_a = [&](int c, uint4 (&ar)[CH]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int f = wave * CH + i;
            const int st = min(c * CH + (f >> 2), nstage - 1);
            const int kblk = kb_begin + min(2 * st + ((f >> 1) & 1), nb - 1);
            // the offset is wave-uniform; as a vector value it would cost a one-pass loop per load
            const int soff = __builtin_amdgcn_readfirstlane((kblk * 2 + (f & 1)) * 1024);
            ar[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ra, lane * 16, soff, 0));
        }
    };
    auto store_a = [&](int buf, const uint4 (&ar)[CH]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < CH; i++) As[buf][(wave * CH + i) * 64 + lane] = ar[i];
    };
    // Chunk c's block sums, thread t: block t / 16 of the chunk, row t % 16
    // (the address gemm_bd_kernel reads for that row and block).
    auto load_xs = [&](int c) __attribute__((always_inline)) -> float {
        if (TYPE != kQ5_1) return 0.f;
        // every thread loads (threads past CH * 32 a clamped entry nobody
        // stores): a branch around the load would cost the compiler its count
        // of the loads in flight, and a full drain at each chunk's first stage
        const int e = min(tid, CH * 32 - 1);
        const int bl = e >> 4, st = min(c * CH + (bl >> 1), nstage - 1);
        const uint32_t off = ((uint32_t)(e & 15) * nblk + kb_begin + 2 * st + (bl & 1)) * 4;
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
    };

    floatx4 acc[TN];
#pragma unroll
    for (int n = 0; n < TN; n++) acc[n] = floatx4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int st, int buf, int sl, const BChunk (&br)[TN]) __attribute__((always_inline)) {
        const bool second = 2 * st + 1 < nb;
#pragma unroll
        for (int bb = 0; bb < 2; bb++) {
            const uint32_t live = bb == 0 || second ? ~0u : 0u;
            const half8_t ah = __builtin_bit_cast(half8_t, As[buf][(sl * 4 + bb * 2 + 0) * 64 + lane]);
            const half8_t al = __builtin_bit_cast(half8_t, As[buf][(sl * 4 + bb * 2 + 1) * 64 + lane]);
            floatx4 xs4;
            if (TYPE == kQ5_1) xs4 = *(const floatx4 *)&Xs[buf][(sl * 2 + bb) * 16 + 4 * (lane >> 4)];
#pragma unroll
            for (int n = 0; n < TN; n++) {
                const half8_t bf = decode_b_frag<TYPE, BQ>(br[n], bb);
                const float dv = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, h2f((uint16_t)(bb ? br[n].d >> 16 : br[n].d))) & live);
                float mv = 0.f;
                if (TYPE == kQ5_1)
                    mv = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, h2f((uint16_t)(bb ? br[n].m >> 16 : br[n].m))) & live);
                floatx4 p = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bf, floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                p = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bf, p, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float v = fmaf(dv, p[r], acc[n][r]);
                    if (TYPE == kQ5_1) v = fmaf(mv, xs4[r], v);
                    acc[n][r] = v;
                }
            }
        }
    };

    // ---- pipeline.  Issue order per chunk c: the activations and block sums
    // of chunk c + 1 (registers, written to the other LDS buffer at the end of
    // chunk c), then one weight stage per stage of chunk c, U stages ahead.
    BChunk br[U][TN];
    uint4 ar[CH];
    float xr = load_xs(0);
    load_a(0, ar);
#pragma unroll
    for (int t = 0; t < U; t++) load_b(t, br[t]);
    store_a(0, ar);
    if (TYPE == kQ5_1 && tid < CH * 32) Xs[0][tid] = xr;
    // Unconditional, so every chunk issues the same loads (the last one
    // re-reads clamped stages into a buffer nobody reads): with a branch
    // around them the compiler's wait counts at the chunk top assume the
    // shorter path and wait on the activation loads just issued.
    for (int c = 0; c < nchunk; c++) {
        const int buf = c & 1;
        __syncthreads(); // chunk c staged by everyone; chunk c - 1's buffers are free
        xr = load_xs(c + 1);
        load_a(c + 1, ar);
#pragma unroll
        for (int j = 0; j < CH; j++) {
            const int st = c * CH + j;
            if (st < nstage) compute(st, buf, j, br[j % U]);
            load_b(st + U, br[j % U]);
        }
        store_a(buf ^ 1, ar);
        if (TYPE == kQ5_1 && tid < CH * 32) Xs[buf ^ 1][tid] = xr;
    }

    // ---- epilogue.  Lane holds C[4*(lane/16) + r][lane % 16].
    const int row_base = 4 * (lane >> 4);
    if (MODE == kGemmStore) {
        if (g >= ngroups) return;
        const QWeight &ws = a.seg[seg_store];
        if (g * 16 - start_store + (lane & 15) >= ws.rows) return;
        float *y = a.y + (size_t)z * M * a.ldy + g * 16 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (row_base + r < M) __builtin_nontemporal_store(acc[0][r], &y[(size_t)(row_base + r) * a.ldy]);
    } else {
        const int ld = a.seg[0].rows;
        const int col = g * 16 + (lane & 15);
        const bool live = g < ngroups && col < ld;
        __shared__ float es[16 * 64]; // [row][column of the workgroup's 64]: hi + lo of each output
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = row_base + r;
            // Kernels.SwiGlu (Kernels.cs:82-89): (g*u) * sigmoid(g).
            const float gv = acc[0][r], u = acc[1][r];
            const float gu = gv * u;
            const float e = expf(-gv);
            const float sg = 1.0f / (1.0f + e);
            const float v = sg * gu;
            uint16_t hi, lo;
            split_f16(v, hi, lo);
            if (live && row < M) {
                a.ot[xt_index(row, col, ld >> 5, 0)] = hi;
                a.ot[xt_index(row, col, ld >> 5, 1)] = lo;
            }
            if (a.osum) es[row * 64 + wave * 16 + (lane & 15)] = h2f(hi) + h2f(lo);
        }
        if (a.osum) {
            // the Q5_1 block sums of these outputs for the down projection: the
            // workgroup's four row groups are 64 consecutive columns, two whole
            // blocks (ld is a multiple of 32), each summed in ascending column
            // order as the block-sum kernel sums an operand tile
            __syncthreads();
            const int row = tid & 15, blk = tid >> 4, c0 = q * 64 + 32 * blk;
            if (tid < 32 && row < M && c0 < ld) {
                float sum = 0.f;
                for (int j = 0; j < 32; j++) sum += es[row * 64 + 32 * blk + j];
                a.osum[(size_t)row * (ld >> 5) + (c0 >> 5)] = sum;
            }
        }
    }
}

template <int TYPE, int MODE, int U, int CH>
static hipError_t launch_skinny(const GemmArgs &a, hipStream_t s)
{
    int ngroups;
    if (MODE == kGemmSwiGlu) {
        ngroups = a.seg[0].rows / 16;
    } else {
        // every segment but the last is a whole number of 16-row groups
        int ntot = 0;
        for (int i = 0; i < a.nseg; i++) ntot += a.seg[i].rows;
        ngroups = (ntot + 15) / 16;
    }
    const int nq = (ngroups + 3) / 4;
    launch_stamped(a.ev_start, a.ev_stop, gemm_skinny_kernel<TYPE, MODE, U, CH>, dim3(nq * a.ksplit), dim3(256), 0, s, a,
                   ngroups, nq);
    return hipGetLastError();
}

// gm_cap: M tiles per group of the tile order (the tiles of a group that share
// an N column run on one XCD, so its L2 serves their common weight tile).
template <int TYPE, int MODE, int TM, int TN, int PD, int OCC, bool FOLD = false, int NW = 4>
static hipError_t launch_bd(const GemmArgs &a, hipStream_t s, int gm_cap = 8)
{
    constexpr int BM = 16 * TM, BN = 16 * TN * NW;
    static_assert(MODE != kGemmSwiGlu || TN % 2 == 0, "SwiGLU pairs tiles within a wave");
    int mt = (a.M + BM - 1) / BM;
    int ncols;
    if (MODE == kGemmSwiGlu) {
        ncols = (a.seg[0].rows + BN / 2 - 1) / (BN / 2);
    } else {
        int ntot = 0;
        for (int i = 0; i < a.nseg; i++) ntot += a.seg[i].rows;
        ncols = (ntot + BN - 1) / BN;
    }
    int gm = mt <= gm_cap ? mt : gm_cap;
    int tiles = mt * ncols;
    int grid = ((tiles + 7) & ~7) * (FOLD ? 1 : a.ksplit);
    launch_stamped(a.ev_start, a.ev_stop, gemm_bd_kernel<TYPE, MODE, TM, TN, PD, OCC, FOLD, NW>, dim3(grid), dim3(64 * NW), 0, s,
                   a, mt, ncols, gm);
    return hipGetLastError();
}

template <int TYPE, int MODE, int WM, int WN, int TM, int TN, int PD, int KS, int OCC>
static hipError_t launch_cfg(const GemmArgs &a, hipStream_t s)
{
    constexpr int BM = WM * TM * 16, BN = WN * TN * 16;
    int mt = (a.M + BM - 1) / BM;
    int ncols;
    if (MODE == kGemmSwiGlu) {
        ncols = (a.seg[0].rows + BN / 2 - 1) / (BN / 2);
    } else {
        int ntot = 0;
        for (int i = 0; i < a.nseg; i++) ntot += a.seg[i].rows;
        ncols = (ntot + BN - 1) / BN;
    }
    int gm = mt <= 8 ? mt : 8;
    int tiles = mt * ncols;
    int grid = ((tiles + 7) & ~7) * a.ksplit;
    launch_stamped(a.ev_start, a.ev_stop, gemm_q_kernel<TYPE, MODE, WM, WN, TM, TN, PD, KS, OCC>, dim3(grid), dim3(256), 0,
                   s, a, mt, ncols, gm);
    return hipGetLastError();
}

template <int TYPE, int MODE>
static hipError_t launch_mode(const GemmArgs &a, hipStream_t s)
{
    // Shape choice by M only changes which rows share a tile, never a result bit.
    // Measured on MI355X (3B shapes, Q8_0): small batches take B-direct
    // 32 x 128 tiles (4-5 % ahead of dequant-in-LDS 64 x 64 tiles on the
    // store shapes), large batches B-direct 64 x 256 tiles.  B-direct needs
    // the store-mode segments to split on 256-row boundaries.
    bool bd_ok = true;
    for (int i = 0; i + 1 < a.nseg; i++) bd_ok = bd_ok && a.seg[i].rows % 256 == 0;
    // One row group (the reasoning decider's rows, short branches): one wave
    // per weight row group, 1.5-2x the B-direct kernel there (12 rows of the
    // Q5_1 3B shape: 2.1 against 3.6 ms of GEMM per step)
    if (a.M <= 16) return launch_skinny<TYPE, MODE, 4, 8>(a, s);
    if (a.M <= 512) {
        // SwiGLU (9216 rows at 256 tokens: 1152 workgroups): built for five
        // resident workgroups per CU (80 VGPRs, six fit) so they all run in
        // one round -- 3 % ahead alone, 0.15 % of a prefill step in the
        // model; the store shapes lose 4-5 % that way.  Groups of 4 M tiles
        // in the tile order: 8 % faster than 8 at 256 tokens (the store
        // shapes are indifferent)
        if (MODE == kGemmSwiGlu) return launch_bd<TYPE, MODE, 2, 2, 1, 5>(a, s, 4);
        // 225..256 rows: 12-wave workgroups (one per CU at the 3B projection
        // shapes, three waves per SIMD), 4-8 % ahead of 4-wave ones.  Fewer
        // rows would leave CUs idle, more would need a second round.
        if constexpr (MODE == kGemmStore)
            if (bd_ok && a.M > 224 && a.M <= 256) return launch_bd<TYPE, MODE, 2, 2, 1, 1, false, 12>(a, s);
        if (bd_ok) return launch_bd<TYPE, MODE, 2, 2, 1, 4>(a, s);
        return launch_cfg<TYPE, MODE, 4, 1, 1, 4, 2, 2, 2>(a, s);
    }
    if (bd_ok) {
        if constexpr (MODE == kGemmStore && TYPE != kQ5_1)
            if (a.fold) return launch_bd<TYPE, MODE, 4, 4, 1, 2, true>(a, s);
        return launch_bd<TYPE, MODE, 4, 4, 1, 2>(a, s);
    }
    return launch_cfg<TYPE, MODE, 4, 1, 2, 8, 1, 1, 2>(a, s);
}

template <int TYPE>
static hipError_t launch_typed(const GemmArgs &a, hipStream_t s)
{
    if (a.mode == kGemmSwiGlu) return launch_mode<TYPE, kGemmSwiGlu>(a, s);
    return launch_mode<TYPE, kGemmStore>(a, s);
}

hipError_t launch_gemm(const GemmArgs &a, hipStream_t s)
{
    if (a.M <= 0) return hipSuccess;
    if (a.K % 32 != 0 || a.ksplit < 1 || a.ksplit > 8) return hipErrorInvalidValue;
    if (a.ksplit > 1 && (a.mode != kGemmStore || gemm_split_blocks(a.K >> 5, a.ksplit) * (a.ksplit - 1) >= (a.K >> 5)))
        return hipErrorInvalidValue; // every split non-empty; SwiGLU needs whole sums
    for (int i = 0; i < a.nseg; i++) {
        if (a.seg[i].type != a.seg[0].type || a.seg[i].cols != a.K) return hipErrorInvalidValue;
        // every segment but the last must tile exactly (both tile widths divide 64)
        if (a.mode == kGemmStore && i + 1 < a.nseg && a.seg[i].rows % 128 != 0) return hipErrorInvalidValue;
    }
    if (a.mode == kGemmSwiGlu && (a.nseg != 2 || a.seg[0].rows != a.seg[1].rows || a.seg[0].rows % 32 != 0))
        return hipErrorInvalidValue;
    if (a.osum && (a.mode != kGemmSwiGlu || a.M > 16)) return hipErrorInvalidValue; // written by the skinny kernel only
    // the folded form exists for the large-batch store tiles (the caller asks
    // for it exactly when gemm_fold says so)
    if (a.fold && (a.mode != kGemmStore || !gemm_fold(a.seg[0].type, a.M, a.ksplit))) return hipErrorInvalidValue;
    for (int i = 0; a.fold && i + 1 < a.nseg; i++)
        if (a.seg[i].rows % 256 != 0) return hipErrorInvalidValue;
    switch (a.seg[0].type) {
    case kQ8_0: return launch_typed<kQ8_0>(a, s);
    case kQ4_0: return launch_typed<kQ4_0>(a, s);
    case kQ5_1: return launch_typed<kQ5_1>(a, s);
    default: return hipErrorInvalidValue;
    }
}

} // namespace jev
