// One-token GEMV against GGUF-quantized weights: y[r] = dot(x, W[r]).
//
// Replaces QuantMatMul.RunRowsFloat (QuantMatMul.cs:140-176), the path a
// one-token call (decode, the last-position LM head) takes.  The kernel is
// bound by streaming the weights from HBM once; the design goal is bytes in
// flight and few vector instructions per weight byte, so the dot products run
// on the matrix cores:
//
//  * x (fp32) is split once per workgroup into an fp16 pair x = hi + lo
//    (~22 significant bits) and staged in LDS.  It is the MFMA A operand:
//    row 0 holds hi, row 1 holds lo, rows 2..15 read a zero slot.
//  * A wave owns 16 weight rows, one tile row of the tiled weight layout.
//    Per tile (two quant blocks) a lane loads its slot -- the quants of its
//    row (l % 16) at k = 8 (l / 16) .. + 7 of both blocks, exactly its B
//    fragments -- as one piece of a contiguous wave-wide load, and decodes
//    them to exact fp16 integers in registers.
//  * One v_mfma_f32_16x16x32_f16 per block then yields x_hi . q and x_lo . q
//    for the 16 rows; the fp32 scale is applied on the vector ALU:
//    acc += d * (p_hi + p_lo)  (+ m * sum(x) over the block for Q5_1).
//
// Narrow projections split K over the workgroup's four waves and, for more
// parallelism, over `ksplit` workgroups whose partials land ksplit * N floats
// apart (summed in split order by the consumer).  The LM head (many rows)
// gives each wave its own 16 rows over the whole K instead.  Loads are buffer
// loads with clamped, branch-free addressing and run a stage of two or four
// tiles ahead of the matrix work.
#include "jev_dev.h"

namespace jev {

namespace {


// One lane's share of a tile: its quants for both blocks, the two scales /
// mins of its row and its fifth bits.
struct RawTile {
    uint4 q;       // Q8_0: 16 bytes; Q4_0 / Q5_1: 8 bytes in .x, .y
    uint32_t d, m; // two fp16 each (block 0 low half)
    uint32_t qh;   // Q5_1: two bytes (block 0 low byte)
};

// Bit i of a 4-bit value x << 4 to bit 8 i + 4 (masked by the caller):
// (x << 4) * 0x204081 (both fit 24 bits) on the full-rate 24-bit multiplier
// (the compiler picks the quarter-rate 32-bit one for the plain product).
__device__ __forceinline__ uint32_t spread4(uint32_t x)
{
    uint32_t r;
    asm("v_mul_u32_u24 %0, %1, %2" : "=v"(r) : "v"(x), "v"(0x00204081u));
    return r;
}

// B fragment of block bb of the tile: 8 fp16 integers for k = 8g .. 8g + 7.
template <int TYPE>
__device__ __forceinline__ half8_t decode_frag(const RawTile &t, int bb)
{
    uint32_t o0, o1, o2, o3;
    if (TYPE == kQ8_0) {
        const uint32_t w0 = bb ? t.q.z : t.q.x, w1 = bb ? t.q.w : t.q.y;
        bytes_to_f16(w0, (_Float16)1152.0f, o0, o1);
        bytes_to_f16(w1, (_Float16)1152.0f, o2, o3);
    } else {
        const uint32_t w = bb ? t.q.y : t.q.x;
        uint32_t n0 = w & 0x0f0f0f0fu, n1 = (w >> 4) & 0x0f0f0f0fu;
        _Float16 bias = (_Float16)1032.0f;
        if (TYPE == kQ5_1) {
            const uint32_t hb = (t.qh >> (8 * bb)) & 0xffu;
            n0 |= spread4((hb & 15u) << 4) & 0x10101010u;
            n1 |= spread4(hb & 0xf0u) & 0x10101010u;
            bias = (_Float16)1024.0f;
        }
        bytes_to_f16(n0, bias, o0, o1);
        bytes_to_f16(n1, bias, o2, o3);
    }
    return __builtin_bit_cast(half8_t, make_uint4(o0, o1, o2, o3));
}

__device__ __forceinline__ float half_of(uint32_t v, int hi) { return h2f((uint16_t)(hi ? v >> 16 : v)); }

// Per-lane loader of one weight's 16-row group: scalar resources and
// per-lane offsets fixed for the loop, a scalar offset per tile.
template <int TYPE>
struct TileLoader {
    rsrc_t rq, rd, rh;
    uint32_t vq, vd, vh;
    int tile0; // first tile of the row group

    __device__ void init(const QWeight &w, int rg, int lane)
    {
        const int KP = tile_kpairs(w.cols), RG = tile_rows(w.rows);
        const uint32_t tiles = (uint32_t)RG * KP;
        rq = make_rsrc(w.qs, tiles * tile_qs_bytes(TYPE));
        rd = make_rsrc(w.d, tiles * tile_d_bytes(TYPE));
        if (TYPE == kQ5_1) rh = make_rsrc(w.qh, tiles * 128);
        vq = (uint32_t)lane * (TYPE == kQ8_0 ? 16 : 8);
        vd = 4 * (lane & 15);
        vh = 2 * lane;
        tile0 = min(rg, RG - 1) * KP; // groups past the weight feed unstored outputs
    }

    // ok false: a tile past the wave's range -- its lane offsets point past
    // every buffer, so the loads return zeros (quants, scales and mins) and
    // the tile adds 0 * p without a mask
    __device__ RawTile load(int kp, bool ok) const
    {
        RawTile t;
        const int tile = tile0 + kp;
        const uint32_t past = ok ? 0u : 0x80000000u;
        if (TYPE == kQ8_0) {
            t.q = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, vq + past, tile * 1024, 0));
        } else {
            uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rq, vq + past, tile * 512, 0));
            t.q = make_uint4(v.x, v.y, 0u, 0u);
        }
        if (TYPE == kQ5_1) {
            // the row's scales and mins in one load
            const uint2 dm = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rd, 2 * vd + past, tile * 128, 0));
            t.d = dm.x;
            t.m = dm.y;
            t.qh = __builtin_amdgcn_raw_buffer_load_b16(rh, vh + past, tile * 128, 0);
        } else {
            t.d = __builtin_amdgcn_raw_buffer_load_b32(rd, vd + past, tile * 64, 0);
        }
        return t;
    }
};

} // namespace

// WR: waves along rows (4: each wave its own 16 rows over the whole range;
// 1: the four waves share 16 rows and split the range).  Grid: (row groups /
// WR, ksplit).  nbz: quant blocks per K split (even).  DEPTH: tiles (block
// pairs) per pipeline stage, chosen per shape so that a wave's last stage
// carries few clamped reloads.
// ATTN: the input is the decode attention output (GemvArgs::attn).
// XUP: the input is the SwiGLU of a gate and an up row (GemvArgs::x_up).
template <int TYPE, int WR, bool SWIGLU, int DEPTH, bool ATTN, bool XUP>
__global__ __launch_bounds__(256, 2) void gemv_q_kernel(GemvArgs a, int nrows, int nbz)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int NW = SWIGLU ? 2 : 1; // weights per row (gate and up)
    // wave-uniform in a scalar register: the loads' scalar offsets depend on
    // it, and a vector value would wrap each load in a one-pass loop
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, rl = lane & 15;
    const int nb = a.K >> 5;
    const int z = blockIdx.y;
    const int kb0 = z * nbz, nbw = min(nb - kb0, nbz); // this workgroup's blocks
    const int ntw = (nbw + 1) >> 1;                     // ... and tiles (the odd last block pads)

    // ---- this wave's row group and tiles
    const int rg = WR == 4 ? blockIdx.x * 4 + wave : blockIdx.x;
    const int per = WR == 4 ? ntw : (ntw + 3) / 4;
    const int t0 = WR == 4 ? 0 : min(ntw, wave * per);
    const int ntiles = min(ntw, t0 + per) - t0;
    const int kp0 = (kb0 >> 1) + t0; // first block pair (kb0 is even)

    TileLoader<TYPE> ld[NW];
    {
        int g0 = rg, seg = 0;
        if (!SWIGLU)
            while (seg + 1 < a.nseg && g0 >= a.seg[seg].rows / 16) {
                g0 -= a.seg[seg].rows / 16;
                seg++;
            }
        seg = __builtin_amdgcn_readfirstlane(seg);
        g0 = __builtin_amdgcn_readfirstlane(g0);
#pragma unroll
        for (int w = 0; w < NW; w++) ld[w].init(a.seg[SWIGLU ? w : seg], g0, lane);
    }
    auto load_stage = [&](int st, RawTile (&r)[NW][DEPTH]) {
#pragma unroll
        for (int j = 0; j < DEPTH; j++) {
            const int tl = st * DEPTH + j;
            const int kp = kp0 + max(0, min(tl, ntiles - 1)); // in range; past the wave's tiles the loads read zeros
#pragma unroll
            for (int w = 0; w < NW; w++) r[w][j] = ld[w].load(kp, tl < ntiles);
        }
    };
    // x of the first kPre groups of 256 is loaded before the first stage's
    // weights, which are in flight while x is staged: the staging then waits
    // on x alone (the vector-memory counter retires loads in order, so a load
    // issued after the weights would wait for them too)
    constexpr int kPre = 2;
    const int nst = (ntiles + DEPTH - 1) / DEPTH;
    RawTile r0[NW][DEPTH], r1[NW][DEPTH];
    // (clamped, unconditional loads: the buffer loads of a wave without
    // tiles stay inside the weight and feed nothing; branches here would make
    // the compiler drain every outstanding load where they join)
    float4 px[kPre][2], pu[kPre][2];
    if (!ATTN) {
#pragma unroll
        for (int it = 0; it < kPre; it++) {
            const int i = min(256 * it + tid, nbw * 4 - 1);
            const float4 *xp = (const float4 *)(a.x + (size_t)kb0 * 32 + 8 * i);
            px[it][0] = xp[0];
            px[it][1] = xp[1];
            if (XUP) {
                pu[it][0] = xp[a.x_up / 4];
                pu[it][1] = xp[a.x_up / 4 + 1];
            }
        }
    }
    load_stage(0, r0);

    // ---- x pair of the workgroup's K range (zero past K), a zero slot, Q5_1 block sums
    uint16_t *xh = (uint16_t *)smem, *xl = xh + nbz * 32, *zero = xl + nbz * 32;
    float *xsum = (float *)(zero + 8);
    float *red = xsum + nbz; // [4][NW][16] wave partials
    // decode attention input: the token's chunk count, as the attention
    // kernel computes it
    int nch = 0;
    if (ATTN) {
        const DecodeChunks &d = a.attn;
        const int start = d.start_dev ? *d.start_dev : d.start;
        const int slot = d.slot ? d.slot[0] : start;
        const int slo = d.shared_lo ? d.shared_lo[0] : 0;
        const int shi = d.shared_hi ? d.shared_hi[0] : start;
        const int seg = d.segment ? d.segment[0] : start;
        const int limit = (shi - slo) + (slot - seg + 1);
        nch = min((limit + kDecodeKeys - 1) / kDecodeKeys, d.max_chunks);
    }
    // thread -> 8 consecutive elements; a block's four groups are neighbouring lanes
    auto stage_group = [&](int i0, auto prec) __attribute__((always_inline)) {
        constexpr int PRE = decltype(prec)::value; // prefetched group index, or -1
        const int i = i0 + tid;
        float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (ATTN && i < nbw * 4) {
            // the decode attention output for these 8 dims of one head: the
            // chunks' (max, sum, o) merged in ascending chunk order with a
            // running max (each step rescales what came before by
            // exp(old max - new max)), eight chunks' loads in flight at a time
            const int k = kb0 * 32 + 8 * i, d = k & 127;
            const float *pp = a.attn.part + (size_t)(k >> 7) * a.attn.max_chunks * 130;
            float M = -INFINITY, L = 0.f;
            for (int c0 = 0; c0 < nch; c0 += 8) {
                float mv[8], lv[8];
                float2 ov[8][4];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float *pc = pp + min(c0 + j, nch - 1) * 130; // clamped reloads are unused
                    mv[j] = pc[0];
                    lv[j] = pc[1];
#pragma unroll
                    for (int e = 0; e < 4; e++) ov[j][e] = *(const float2 *)(pc + 2 + d + 2 * e);
                }
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    if (c0 + j < nch) {
                        const float Mn = fmaxf(M, mv[j]);
                        const float fo = __expf(M - Mn), fc = __expf(mv[j] - Mn);
                        L = fmaf(lv[j], fc, L * fo);
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            v[2 * e] = fmaf(ov[j][e].x, fc, v[2 * e] * fo);
                            v[2 * e + 1] = fmaf(ov[j][e].y, fc, v[2 * e + 1] * fo);
                        }
                        M = Mn;
                    }
                }
            }
            const float inv = 1.0f / L; // one division, eight products
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = v[e] * inv;
        } else if (PRE >= 0 || i < nbw * 4) {
            // a prefetched group selects rather than branches (its lanes past
            // the range hold clamped copies and stage zeros)
            const bool valid = i < nbw * 4;
            const float4 *xp = (const float4 *)(a.x + (size_t)kb0 * 32 + 8 * i);
            const float4 v0 = PRE >= 0 ? px[PRE < 0 ? 0 : PRE][0] : xp[0];
            const float4 v1 = PRE >= 0 ? px[PRE < 0 ? 0 : PRE][1] : xp[1];
            v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w;
            v[4] = v1.x; v[5] = v1.y; v[6] = v1.z; v[7] = v1.w;
            if (XUP) {
                // Kernels.SwiGlu (Kernels.cs:82-89): (g*u) * sigmoid(g).  Every
                // workgroup of the down projection forms the inputs of its K
                // range (192 row groups each redo them), so the sigmoid is the
                // hardware exp2 and reciprocal (a few ulp, as TensorPrimitives'
                // vectorised Sigmoid is not libm either) rather than the
                // library's exact expf and IEEE division.
                const float4 u0 = PRE >= 0 ? pu[PRE < 0 ? 0 : PRE][0] : xp[a.x_up / 4];
                const float4 u1 = PRE >= 0 ? pu[PRE < 0 ? 0 : PRE][1] : xp[a.x_up / 4 + 1];
                const float u[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float gu = v[j] * u[j];
                    const float e = __builtin_amdgcn_exp2f(-v[j] * 1.44269504088896340736f);
                    const float sg = __builtin_amdgcn_rcpf(1.0f + e);
                    v[j] = sg * gu;
                }
            }
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = valid ? v[j] : 0.f;
        }
        uint32_t hw[4], lw[4];
        float bs = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            uint16_t h0, l0, h1, l1;
            split_f16(v[j], h0, l0);
            split_f16(v[j + 1], h1, l1);
            hw[j >> 1] = (uint32_t)h0 | ((uint32_t)h1 << 16);
            lw[j >> 1] = (uint32_t)l0 | ((uint32_t)l1 << 16);
            bs += (h2f(h0) + h2f(l0)) + (h2f(h1) + h2f(l1));
        }
        if (i < 2 * ntw * 4) {
            *(uint4 *)(xh + 8 * i) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
            *(uint4 *)(xl + 8 * i) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        }
        if (TYPE == kQ5_1) {
            bs = bs + __shfl_xor(bs, 1, 64);
            bs = bs + __shfl_xor(bs, 2, 64);
            if (i < 2 * ntw * 4 && (i & 3) == 0) xsum[i >> 2] = bs;
        }
    };
    // the prefetched groups in straight-line code, any further ones in a loop
    stage_group(0, std::integral_constant<int, ATTN ? -1 : 0>{});
    if (256 < 2 * ntw * 4) stage_group(256, std::integral_constant<int, ATTN ? -1 : 1>{});
    for (int i0 = 256 * kPre; i0 < 2 * ntw * 4; i0 += 256) stage_group(i0, std::integral_constant<int, -1>{});
    if (tid < 8) zero[tid] = 0;
    __syncthreads();

    // A fragment address: row 0 -> hi, row 1 -> lo, rows 2..15 -> the zero slot
    const uint16_t *abase = rl == 0 ? xh + 8 * g : rl == 1 ? xl + 8 * g : zero;
    const int astep = rl <= 1 ? 32 : 0;

    float acc[NW];
#pragma unroll
    for (int w = 0; w < NW; w++) acc[w] = 0.f;

    auto compute_stage = [&](int st, const RawTile (&r)[NW][DEPTH]) {
#pragma unroll
        for (int j = 0; j < DEPTH; j++) {
            const int tl = st * DEPTH + j; // tile within the wave's range
            const int lt = t0 + min(tl, ntiles - 1); // tile within the workgroup's range
#pragma unroll
            for (int bb = 0; bb < 2; bb++) {
                const half8_t af = *(const half8_t *)(abase + astep * (2 * lt + bb));
#pragma unroll
                for (int w = 0; w < NW; w++) {
                    const half8_t bf = decode_frag<TYPE>(r[w][j], bb);
                    floatx4 p = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf, floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    const float dv = half_of(r[w][j].d, bb); // 0 past the range
                    const float v = p[0] + p[1];
                    acc[w] = fmaf(dv, v, acc[w]);
                    if (TYPE == kQ5_1) {
                        const float mv = half_of(r[w][j].m, bb);
                        acc[w] = fmaf(mv, xsum[2 * lt + bb], acc[w]);
                    }
                }
            }
        }
    };

    // Two register stages; whole pairs in the loop, the odd stage after it.
    if (nst > 0) {
        int st = 0;
        // sched_barriers at the stage boundaries: the scheduler would hoist
        // parts of the next stage's decode into this stage's compute, where
        // they wait on loads issued moments before
        for (; st + 2 <= nst; st += 2) {
            load_stage(st + 1, r1);
            __builtin_amdgcn_sched_barrier(0);
            compute_stage(st, r0);
            __builtin_amdgcn_sched_barrier(0);
            load_stage(st + 2, r0);
            __builtin_amdgcn_sched_barrier(0);
            compute_stage(st + 1, r1);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (st < nst) compute_stage(st, r0);
    }

    // ---- outputs: lane l < 16 holds row rg * 16 + l
    const int row = rg * 16 + rl;
    if (WR == 4) {
        if (g == 0 && row < nrows) a.y[(size_t)z * nrows + row] = acc[0];
    } else {
        if (g == 0) {
#pragma unroll
            for (int w = 0; w < NW; w++) red[(wave * NW + w) * 16 + rl] = acc[w];
        }
        __syncthreads();
        if (wave == 0 && g == 0 && row < nrows) {
            float s[NW];
#pragma unroll
            for (int w = 0; w < NW; w++)
                s[w] = ((red[(0 * NW + w) * 16 + rl] + red[(1 * NW + w) * 16 + rl]) + red[(2 * NW + w) * 16 + rl]) +
                       red[(3 * NW + w) * 16 + rl];
            if (SWIGLU) {
                // Kernels.SwiGlu (Kernels.cs:82-89): (g*u) * sigmoid(g)
                float gu = s[0] * s[NW - 1];
                float e = expf(-s[0]);
                float sg = 1.0f / (1.0f + e);
                a.y[row] = sg * gu;
            } else {
                a.y[(size_t)z * nrows + row] = s[0];
            }
        }
    }
}

template <int TYPE, int WR, bool SWIGLU, bool ATTN = false, bool XUP = false>
static hipError_t launch_gemv_cfg(const GemvArgs &a, int rows, hipStream_t s)
{
    const int nb = a.K >> 5;
    const int nbz = gemm_split_blocks(nb, a.ksplit);
    const int groups = (rows + 15) / 16;
    size_t lds = (size_t)nbz * 32 * 2 * 2 + 16 + (size_t)nbz * 4 + 4 * 2 * 16 * 4; // nbz is even
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    dim3 grid(WR == 4 ? (groups + 3) / 4 : groups, a.ksplit);
    // tiles of one wave, and the stage depth that pads them least (4 on a tie)
    const int ntw = nbz / 2, per = WR == 4 ? ntw : (ntw + 3) / 4;
    const int pad4 = (per + 3) / 4 * 4 - per, pad2 = (per + 1) / 2 * 2 - per;
    if (pad2 < pad4)
        launch_stamped(a.ev_start, a.ev_stop, gemv_q_kernel<TYPE, WR, SWIGLU, 2, ATTN, XUP>, grid, dim3(256), (uint32_t)lds, s, a,
                       rows, nbz);
    else
        launch_stamped(a.ev_start, a.ev_stop, gemv_q_kernel<TYPE, WR, SWIGLU, 4, ATTN, XUP>, grid, dim3(256), (uint32_t)lds, s, a,
                       rows, nbz);
    return hipGetLastError();
}

template <int TYPE>
static hipError_t launch_gemv_typed(const GemvArgs &a, hipStream_t s)
{
    if (a.swiglu) return launch_gemv_cfg<TYPE, 1, true>(a, a.seg[0].rows, s);
    int rows = 0;
    for (int i = 0; i < a.nseg; i++) rows += a.seg[i].rows;
    if (a.attn.part) {
        if (gemv_rows_mode(rows)) return launch_gemv_cfg<TYPE, 4, false, true>(a, rows, s);
        return launch_gemv_cfg<TYPE, 1, false, true>(a, rows, s);
    }
    if (a.x_up > 0) {
        if (gemv_rows_mode(rows)) return hipErrorInvalidValue; // the SwiGLU input is a narrow projection's
        return launch_gemv_cfg<TYPE, 1, false, false, true>(a, rows, s);
    }
    if (gemv_rows_mode(rows)) return launch_gemv_cfg<TYPE, 4, false>(a, rows, s);
    return launch_gemv_cfg<TYPE, 1, false>(a, rows, s);
}

hipError_t launch_gemv(const GemvArgs &a, hipStream_t s)
{
    if (a.K % 32 != 0 || a.K <= 0 || a.ksplit < 1 || a.x_up < 0 || a.x_up % 4 != 0) return hipErrorInvalidValue;
    // the attention input: 128-dim heads, one weight, no other input transform
    if (a.attn.part && (a.K % 128 != 0 || a.x_up || a.swiglu || a.nseg != 1 || a.attn.max_chunks < 1))
        return hipErrorInvalidValue;
    const int nb = a.K >> 5;
    if (a.ksplit > 1 && (a.swiglu || gemm_split_blocks(nb, a.ksplit) * (a.ksplit - 1) >= nb)) return hipErrorInvalidValue;
    for (int i = 0; i < a.nseg; i++) {
        if (a.seg[i].type != a.seg[0].type || a.seg[i].cols != a.K) return hipErrorInvalidValue;
        // a 16-row group (tile row) never straddles two segments
        if (!a.swiglu && i + 1 < a.nseg && a.seg[i].rows % 16 != 0) return hipErrorInvalidValue;
    }
    if (a.swiglu && (a.nseg != 2 || a.seg[0].rows != a.seg[1].rows)) return hipErrorInvalidValue;
    switch (a.seg[0].type) {
    case kQ8_0: return launch_gemv_typed<kQ8_0>(a, s);
    case kQ4_0: return launch_gemv_typed<kQ4_0>(a, s);
    case kQ5_1: return launch_gemv_typed<kQ5_1>(a, s);
    default: return hipErrorInvalidValue;
    }
}

} // namespace jev
