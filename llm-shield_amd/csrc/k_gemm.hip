// Prefill GEMM against GGUF-quantized weights: y = x . W^T on the MFMA cores.
//
// Replaces PanelGemm (PanelGemm.cs:87-318) for calls of two or more tokens.
//
// Numerics.  The weight quants are small integers (Q8_0 q in [-127,127],
// Q4_0 q-8 in [-8,7], Q5_1 q in [0,31]) and therefore exact in fp16; only the
// per-32 block scale d (and Q5_1's min m) is not.  One MFMA of 16x16x32 covers
// exactly one quant block, so each block's partial dot of x with the integer
// quants comes out of the matrix core exactly-scaled-free and the fp32 scale is
// applied on the vector ALU:  acc += d * (x . q)  (+ m * sum(x) for Q5_1).
// The activation x enters as an fp16 pair hi + lo (two MFMAs into the same
// partial), which carries ~22 significant bits; a single fp16 or bf16 operand
// measured 4e-3 / 2e-2 relative error on the 26-layer logits, the pair 3e-5.
//
// Determinism.  Each output is the same sequence of MFMAs and FMAs over its K
// blocks whatever M is and whichever tile its row lands in, so a token's
// result does not depend on the batch around it (the reference's batch
// invariance, PanelGemm.cs:28-31); that is what keeps a tree pass bit-identical
// to running its branches one at a time.
//
// Tiling.  256 threads = 4 waves as 2 x 2; workgroup tile 128 x 128, wave tile
// 64 x 64 = 4 x 4 MFMA tiles; one quant block (K = 32) per pipeline step,
// double-buffered in LDS.  The loader decodes quants to fp16 on their way into
// LDS ("dequant in LDS"), so each decoded weight feeds all 128 rows of the
// tile.  LDS rows are padded to 40 halves (80 bytes) so the 16-byte fragment
// reads of 8 consecutive lanes fall on distinct banks.
#include "jev_dev.h"

namespace jev {

namespace {

constexpr int BM = 128, BN = 128, LDS_ROW = 40;

struct alignas(16) u32x4 {
    uint32_t x, y, z, w;
};

__device__ __forceinline__ uint16_t h16(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }
__device__ __forceinline__ uint32_t pack2(float a, float b) { return (uint32_t)h16(a) | ((uint32_t)h16(b) << 16); }

template <int TYPE>
struct BRaw {
    u32x4 q;      // 16 bytes of quants
    uint32_t qh;  // Q5_1 fifth bits
    float d, m;   // scale, min
    bool valid;
};

// Source row of the B tile's LDS row rr.
struct RowMap {
    const QWeight *w;
    int row;
};

template <int MODE>
__device__ __forceinline__ void map_row(const GemmArgs &a, int tile_n, int rr, int &seg, int &row, int &col_base)
{
    if (MODE == kGemmSwiGlu) {
        int sub = rr >> 4;
        seg = sub & 1;
        row = tile_n * 64 + (sub >> 1) * 16 + (rr & 15);
        col_base = tile_n * 64;
    } else {
        int n0 = tile_n * BN;
        int s = 0, start = 0;
        while (s + 1 < a.nseg && n0 >= start + a.seg[s].rows) {
            start += a.seg[s].rows;
            s++;
        }
        seg = s;
        row = n0 - start + rr;
        col_base = n0;
    }
}

template <int TYPE>
__device__ __forceinline__ void load_b(const QWeight &w, int row, int kb, int h, BRaw<TYPE> &b)
{
    b.valid = row < w.rows;
    if (!b.valid) return;
    int nb = w.cols >> 5;
    size_t blk = (size_t)row * nb + kb;
    if (TYPE == kQ8_0) {
        b.q = *(const u32x4 *)(w.qs + (size_t)row * w.cols + (size_t)kb * 32 + 16 * h);
    } else {
        b.q = *(const u32x4 *)(w.qs + (size_t)row * (w.cols >> 1) + (size_t)kb * 16);
    }
    b.d = h2f(w.d[blk]);
    if (TYPE == kQ5_1) {
        b.m = h2f(w.m[blk]);
        b.qh = w.qh[blk] >> (16 * h);
    }
}

// The 16 quants of this thread's half block as fp16 integers, into LDS.
template <int TYPE>
__device__ __forceinline__ void store_b(const BRaw<TYPE> &b, int h, uint16_t *dst)
{
    uint32_t out[8];
    if (!b.valid) {
#pragma unroll
        for (int i = 0; i < 8; i++) out[i] = 0;
    } else {
        uint32_t wds[4] = {b.q.x, b.q.y, b.q.z, b.q.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            // elements 2i and 2i+1 of this half block
            int e0 = 2 * i, e1 = 2 * i + 1;
            float v0, v1;
            if (TYPE == kQ8_0) {
                v0 = (float)(int8_t)(wds[e0 >> 2] >> (8 * (e0 & 3)));
                v1 = (float)(int8_t)(wds[e1 >> 2] >> (8 * (e1 & 3)));
            } else {
                uint32_t b0 = (wds[e0 >> 2] >> (8 * (e0 & 3))) & 0xff;
                uint32_t b1 = (wds[e1 >> 2] >> (8 * (e1 & 3))) & 0xff;
                int n0 = h ? (int)(b0 >> 4) : (int)(b0 & 15);
                int n1 = h ? (int)(b1 >> 4) : (int)(b1 & 15);
                if (TYPE == kQ4_0) {
                    v0 = (float)(n0 - 8);
                    v1 = (float)(n1 - 8);
                } else {
                    v0 = (float)(n0 | (int)(((b.qh >> e0) & 1u) << 4));
                    v1 = (float)(n1 | (int)(((b.qh >> e1) & 1u) << 4));
                }
            }
            out[i] = pack2(v0, v1);
        }
    }
    u32x4 *d4 = (u32x4 *)dst;
    d4[0] = u32x4{out[0], out[1], out[2], out[3]};
    d4[1] = u32x4{out[4], out[5], out[6], out[7]};
}

} // namespace

template <int TYPE, int MODE>
__global__ __launch_bounds__(256, 2) void gemm_q_kernel(GemmArgs a)
{
    __shared__ __attribute__((aligned(16))) uint16_t As_hi[2][BM * LDS_ROW];
    __shared__ __attribute__((aligned(16))) uint16_t As_lo[2][BM * LDS_ROW];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDS_ROW];
    __shared__ float Ds[2][BN];
    __shared__ float Msh[2][TYPE == kQ5_1 ? BN : 1];
    __shared__ __attribute__((aligned(16))) float Ss[2][TYPE == kQ5_1 ? BM : 4];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int tile_n = blockIdx.x, tile_m = blockIdx.y, z = blockIdx.z;
    const int m0 = tile_m * BM;
    const int M = a.M, K = a.K, nblk = K >> 5;
    const int per = (nblk + a.ksplit - 1) / a.ksplit;
    const int kb0 = z * per;
    const int kb1 = min(nblk, kb0 + per);

    // Loader role: LDS row rr, half block h.
    const int rr = tid >> 1, h = tid & 1;
    int seg, wrow, col_base;
    map_row<MODE>(a, tile_n, rr, seg, wrow, col_base);
    const QWeight &w = a.seg[seg];
    const int am = m0 + rr;
    const bool a_ok = am < M;

    u32x4 ahi[2], alo[2];
    BRaw<TYPE> braw;
    float s_next = 0.f;

    auto load = [&](int kb) {
        if (a_ok) {
            const u32x4 *ph = (const u32x4 *)(a.xhi + (size_t)am * K + (size_t)kb * 32 + 16 * h);
            const u32x4 *pl = (const u32x4 *)(a.xlo + (size_t)am * K + (size_t)kb * 32 + 16 * h);
            ahi[0] = ph[0];
            ahi[1] = ph[1];
            alo[0] = pl[0];
            alo[1] = pl[1];
            if (TYPE == kQ5_1) s_next = a.xsum[(size_t)am * nblk + kb];
        } else {
            ahi[0] = ahi[1] = alo[0] = alo[1] = u32x4{0, 0, 0, 0};
            s_next = 0.f;
        }
        load_b<TYPE>(w, wrow, kb, h, braw);
    };
    auto store = [&](int st) {
        u32x4 *dh = (u32x4 *)(&As_hi[st][rr * LDS_ROW + 16 * h]);
        u32x4 *dl = (u32x4 *)(&As_lo[st][rr * LDS_ROW + 16 * h]);
        dh[0] = ahi[0];
        dh[1] = ahi[1];
        dl[0] = alo[0];
        dl[1] = alo[1];
        store_b<TYPE>(braw, h, &Bs[st][rr * LDS_ROW + 16 * h]);
        if (h == 0) {
            Ds[st][rr] = braw.valid ? braw.d : 0.f;
            if (TYPE == kQ5_1) {
                Msh[st][rr] = braw.valid ? braw.m : 0.f;
                Ss[st][rr] = s_next;
            }
        }
    };

    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    if (kb0 < kb1) {
        load(kb0);
        store(0);
    }
    __syncthreads();

    const int frag_row = lane & 15, frag_k = 8 * (lane >> 4);
    for (int kb = kb0; kb < kb1; kb++) {
        const int st = (kb - kb0) & 1;
        if (kb + 1 < kb1) load(kb + 1);

        half8_t fa_hi[4], fa_lo[4], fb[4];
        float dsc[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int r = 64 * wm + 16 * i + frag_row;
            fa_hi[i] = *(const half8_t *)(&As_hi[st][r * LDS_ROW + frag_k]);
            fa_lo[i] = *(const half8_t *)(&As_lo[st][r * LDS_ROW + frag_k]);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int c = 64 * wn + 16 * j + frag_row;
            fb[j] = *(const half8_t *)(&Bs[st][c * LDS_ROW + frag_k]);
            dsc[j] = Ds[st][c];
        }
        floatx4 p[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                p[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa_hi[i], fb[j], floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) p[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa_lo[i], fb[j], p[i][j], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[i][j][r] = fmaf(dsc[j], p[i][j][r], acc[i][j][r]);
        if (TYPE == kQ5_1) {
            float mn[4];
#pragma unroll
            for (int j = 0; j < 4; j++) mn[j] = Msh[st][64 * wn + 16 * j + frag_row];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                floatx4 sv = *(const floatx4 *)(&Ss[st][64 * wm + 16 * i + 4 * (lane >> 4)]);
#pragma unroll
                for (int j = 0; j < 4; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[i][j][r] = fmaf(mn[j], sv[r], acc[i][j][r]);
            }
        }
        if (kb + 1 < kb1) store(st ^ 1);
        __syncthreads();
    }

    // Epilogue.  Lane holds C[4*(lane/16) + r][lane % 16] of each 16x16 tile.
    const int row_base = m0 + 64 * wm + 4 * (lane >> 4);
    if (MODE == kGemmStore) {
        float *y = a.y + (size_t)z * M * a.ldy;
        const QWeight &ws = a.seg[seg]; // segment of this workgroup's columns
        int seg_start = col_base;       // global column of the tile's first row
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                int col = seg_start + 64 * wn + 16 * j + frag_row;
                int local = wrow - rr + 64 * wn + 16 * j + frag_row; // row within the segment
                if (local >= ws.rows) continue;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    int row = row_base + 16 * i + r;
                    if (row < M) y[(size_t)row * a.ldy + col] = acc[i][j][r];
                }
            }
    } else {
        const int ld = a.seg[0].rows;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int pp = 0; pp < 2; pp++) {
                int col = col_base + (2 * wn + pp) * 16 + frag_row;
                if (col >= ld) continue;
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
                    a.ohi[(size_t)row * ld + col] = hi;
                    a.olo[(size_t)row * ld + col] = lo;
                }
            }
    }
}

template <int TYPE>
static hipError_t launch_typed(const GemmArgs &a, hipStream_t s)
{
    int mt = (a.M + BM - 1) / BM;
    if (a.mode == kGemmSwiGlu) {
        int nt = (a.seg[0].rows + 63) / 64;
        hipLaunchKernelGGL((gemm_q_kernel<TYPE, kGemmSwiGlu>), dim3(nt, mt, 1), dim3(256), 0, s, a);
    } else {
        int ntot = 0;
        for (int i = 0; i < a.nseg; i++) ntot += a.seg[i].rows;
        int nt = (ntot + BN - 1) / BN;
        hipLaunchKernelGGL((gemm_q_kernel<TYPE, kGemmStore>), dim3(nt, mt, a.ksplit), dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmArgs &a, hipStream_t s)
{
    if (a.M <= 0) return hipSuccess;
    if (a.K % 32 != 0 || a.ksplit < 1) return hipErrorInvalidValue;
    for (int i = 0; i < a.nseg; i++) {
        if (a.seg[i].type != a.seg[0].type || a.seg[i].cols != a.K) return hipErrorInvalidValue;
        // every segment but the last must tile exactly into 128-row tiles
        if (a.mode == kGemmStore && i + 1 < a.nseg && a.seg[i].rows % BN != 0) return hipErrorInvalidValue;
    }
    if (a.mode == kGemmSwiGlu && (a.nseg != 2 || a.seg[0].rows != a.seg[1].rows || a.ksplit != 1))
        return hipErrorInvalidValue;
    switch (a.seg[0].type) {
    case kQ8_0: return launch_typed<kQ8_0>(a, s);
    case kQ4_0: return launch_typed<kQ4_0>(a, s);
    case kQ5_1: return launch_typed<kQ5_1>(a, s);
    default: return hipErrorInvalidValue;
    }
}

} // namespace jev
