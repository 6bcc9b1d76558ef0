// Opt-in integer matmul: the reference's MatMulStrategy.Integer.
//
// Replaces QuantMatMul.ForwardIntegerAsync / RunRowsInteger
// (QuantMatMul.cs:186-287) and IntegerDot (IntegerDot.cs).  Activations are
// quantized per token and 32-block to Q8_0 exactly as
// IntegerDot.QuantizeActivations (IntegerDot.cs:60-96) does; the weights keep
// their quants as 8-bit integers; each block's integer dot runs on the int8
// matrix cores (v_mfma_i32_16x16x32_i8, one quant block per instruction, exact
// int32 sums) and is scaled on the vector ALU in the order of IntegerDot's
// scalar dots (IntegerDot.cs:206-272):
//   total = total + (w_scale * x_scale) * sum_i(w_i * q_i),  blocks ascending,
// and for Q5_1 the offset term of OffsetContribution (:274-279),
// sum_b m_b * (d_b * sum_i q_i), added after the dot.  No K split: one lane
// owns an output for the whole K, so the float order is fixed.
//
// Weight quants come from the tiled layout: Q8_0 bytes (stored biased) get
// their sign bit flipped back; Q4_0 nibbles enter as 0..15 and the integer
// sum is corrected by 8 * sum(q) (exact); Q5_1's 0..31 enter as they are.
#include "jev_dev.h"

#include <type_traits>

namespace jev {

namespace {

typedef int int4v __attribute__((ext_vector_type(4)));

// Operand tiles of the int8 16x16x32 MFMA: row group rg (16 tokens) and block
// b hold 64 lanes x 8 bytes; lane 16 g + r carries token 16 rg + r at
// k = 32 b + 8 g .. + 7.
__device__ __forceinline__ size_t xq_index(int t, int k, int nb)
{
    const int rg = t >> 4, r = t & 15, b = k >> 5, kk = k & 31;
    return (((size_t)rg * nb + b) * 64 + (kk >> 3) * 16 + r) * 8 + (kk & 7);
}

} // namespace

// Eight lanes per (token, block), four consecutive elements each (one
// 16-byte load, one 4-byte store of quants).  The block's max |x| and its
// integer quant sum are order-free, so any reduction tree gives the same
// result.  Per-block results are stored block-major ([b][t16]) so a lane of
// the GEMM reads its four output rows with one load.
__global__ __launch_bounds__(256) void quant_act_kernel(QuantActArgs a)
{
    const int nb = a.K >> 5;
    const int id = blockIdx.x * 32 + (threadIdx.x >> 3), i = threadIdx.x & 7;
    if (id >= a.T * nb) return; // whole groups of eight; the shuffles stay inside them
    const int t = id / nb, b = id % nb;
    const float4 v = *(const float4 *)(a.x + (size_t)t * a.K + 32 * b + 4 * i);
    float mx = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int o = 4; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 8));
    const float d = mx / 127.0f;
    const float inverse = d != 0.0f ? 1.0f / d : 0.0f;
    const float vv[4] = {v.x, v.y, v.z, v.w};
    int q[4], s = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float scaled = vv[j] * inverse;
        q[j] = min(127, max(-127, (int)roundf(scaled))); // roundf: half away from zero
        s += q[j];
    }
#pragma unroll
    for (int o = 4; o > 0; o >>= 1) s += __shfl_xor(s, o, 8);
    // four consecutive k of one lane of the operand tile: contiguous bytes
    *(uint32_t *)(a.xq + xq_index(t, 32 * b + 4 * i, nb)) =
        (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) | ((uint32_t)(uint8_t)q[2] << 16) | ((uint32_t)(uint8_t)q[3] << 24);
    if (i == 0) {
        const size_t bi = (size_t)b * a.T16 + t;
        a.xd[bi] = (float)(_Float16)d; // the stored Half scale
        a.xqs[bi] = s;
        a.xs[bi] = d * (float)s; // QuantMatMul's block sums use the float d
    }
}

// x not 16-byte aligned: one lane per element, the same arithmetic.
__global__ __launch_bounds__(256) void quant_act1_kernel(QuantActArgs a)
{
    const int nb = a.K >> 5;
    const int id = blockIdx.x * 8 + (threadIdx.x >> 5), i = threadIdx.x & 31;
    if (id >= a.T * nb) return; // whole half-waves; the shuffles stay inside 32 lanes
    const int t = id / nb, b = id % nb;
    const float v = a.x[(size_t)t * a.K + 32 * b + i];
    float mx = fabsf(v);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 32));
    const float d = mx / 127.0f;
    const float inverse = d != 0.0f ? 1.0f / d : 0.0f;
    const float scaled = v * inverse;
    const int q = min(127, max(-127, (int)roundf(scaled))); // roundf: half away from zero
    int s = q;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) s += __shfl_xor(s, o, 32);
    a.xq[xq_index(t, 32 * b + i, nb)] = (int8_t)q;
    if (i == 0) {
        const size_t bi = (size_t)b * a.T16 + t;
        a.xd[bi] = (float)(_Float16)d;
        a.xqs[bi] = s;
        a.xs[bi] = d * (float)s;
    }
}

hipError_t launch_quant_act(const QuantActArgs &a, hipStream_t s)
{
    if (a.T <= 0) return hipSuccess;
    if (a.K <= 0 || a.K % 32 != 0 || a.T16 < ((a.T + 15) & ~15)) return hipErrorInvalidValue;
    const long long blocks = (long long)a.T * (a.K >> 5);
    if (((uintptr_t)a.x & 15) == 0) // eight lanes per block, 32 blocks per workgroup
        hipLaunchKernelGGL(quant_act_kernel, dim3((unsigned)((blocks + 31) / 32)), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(quant_act1_kernel, dim3((unsigned)((blocks + 7) / 8)), dim3(256), 0, s, a);
    return hipGetLastError();
}

// Wave w of workgroup (x, y) owns weight row group 4 x + w (16 output
// columns) and the TM token groups from TM y.  The activation side of a tile
// pair (two quant blocks) -- the token groups' int8 fragments and their
// per-block scale terms -- is the same for the workgroup's four waves, so it
// is staged in LDS once per workgroup, CH pairs at a time, double buffered
// with one barrier per chunk: loaded into registers a chunk ahead, written to
// the free buffer at the end of the chunk.  Each wave streams its own weight
// slots through a register ring DEPTH pairs ahead (buffer loads, the pair in
// the scalar offset).  Loads past the last pair are clamped; the last chunk
// discards what lies past the last block by selects, so each output takes its
// blocks ascending, one IntegerDot step each.
template <int TYPE, int TM>
__global__ __launch_bounds__(256, 2) void gemm_i8_kernel(GemmI8Args a)
{
    constexpr int CH = 8 / TM;             // tile pairs per staged chunk
    constexpr int DEPTH = CH < 4 ? CH : 4; // weight ring (divides CH)
    constexpr int NB = 2 * CH;             // blocks per chunk
    constexpr bool AUX = TYPE != kQ8_0;    // Q4_0: quant sums; Q5_1: d * sum(q)
    __shared__ __attribute__((aligned(16))) uint8_t sa[2][TM][NB][512]; // int8 fragments
    __shared__ __attribute__((aligned(16))) float sd[2][TM][NB][16];    // x scales
    __shared__ __attribute__((aligned(16))) float sx[2][TM][AUX ? NB : 1][16];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, rl = lane & 15;
    const QWeight &w = a.w;
    const int nb = w.cols >> 5, KP = tile_kpairs(w.cols), RG = tile_rows(w.rows);
    const int tg0 = blockIdx.y * TM;
    // waves past the weight's rows keep loading a clamped row group (their
    // outputs are not stored): every wave reaches every barrier
    const int rgw = blockIdx.x * 4 + wave;
    const int tile0 = __builtin_amdgcn_readfirstlane(min(rgw, RG - 1) * KP);
    const uint32_t tiles = (uint32_t)RG * KP;
    constexpr bool BYTES = TYPE == kQ8_0;
    const rsrc_t rq = make_rsrc(w.qs, tiles * (BYTES ? 1024u : 512u));
    const rsrc_t rd = make_rsrc(w.d, tiles * (uint32_t)tile_d_bytes(TYPE));
    rsrc_t rh;
    if (TYPE == kQ5_1) rh = make_rsrc(w.qh, tiles * 128u);
    const rsrc_t rx = make_rsrc(a.xq, (uint32_t)a.T16 * nb * 32u);
    const rsrc_t rxd = make_rsrc(a.xd, (uint32_t)a.T16 * nb * 4u);
    rsrc_t raux;
    if (TYPE == kQ4_0) raux = make_rsrc(a.xqs, (uint32_t)a.T16 * nb * 4u);
    if (TYPE == kQ5_1) raux = make_rsrc(a.xs, (uint32_t)a.T16 * nb * 4u);
    const int nchunk = (KP + CH - 1) / CH;

    // ---- activation chunk c: per token group, NB fragments of 512 B (16
    // bytes per thread per pair of fragments) and NB x 16 scale terms (one
    // float per thread per group of 16 blocks)
    constexpr int AQ = TM * NB * 512 / 16 / 256; // 16-byte loads per thread
    constexpr int AS = (TM * NB * 16 + 255) / 256; // scale floats per thread
    struct AChunk {
        uint4 q[AQ];
        float d[AS], x[AS];
    };
    auto load_a = [&](int c, AChunk &r) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < AQ; i++) {
            const int e = i * 256 + tid;             // 16-byte element of the chunk
            const int tm = e / (NB * 32), rem = e % (NB * 32);
            const int lb = rem >> 5, part = rem & 31;  // block of the chunk, 16 bytes of its 512
            const int kb = min(c * NB + lb, nb - 1);
            const int tg = tg0 + tm;
            // (the block varies per lane: all of it in the lane offset)
            r.q[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, ((uint32_t)(tg * nb + kb) * 32 + part) * 16, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < AS; i++) {
            const int e = min(i * 256 + tid, TM * NB * 16 - 1);
            const int tm = e / (NB * 16), rem = e % (NB * 16);
            const int lb = rem >> 4, t = rem & 15;
            const int kb = min(c * NB + lb, nb - 1);
            const uint32_t off = ((uint32_t)kb * a.T16 + 16 * (tg0 + tm) + t) * 4;
            r.d[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rxd, off, 0, 0));
            if (AUX) r.x[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(raux, off, 0, 0));
        }
    };
    auto store_a = [&](int buf, const AChunk &r) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < AQ; i++) {
            const int e = i * 256 + tid;
            const int tm = e / (NB * 32), rem = e % (NB * 32);
            *(uint4 *)&sa[buf][tm][rem >> 5][16 * (rem & 31)] = r.q[i];
        }
#pragma unroll
        for (int i = 0; i < AS; i++) {
            const int e = i * 256 + tid;
            if (e < TM * NB * 16) {
                const int tm = e / (NB * 16), rem = e % (NB * 16);
                sd[buf][tm][rem >> 4][rem & 15] = r.d[i];
                if (AUX) sx[buf][tm][rem >> 4][rem & 15] = r.x[i];
            }
        }
    };

    // ---- weight slot of tile pair kp (clamped past the last)
    struct WStage {
        uint4 q;     // Q8_0 16 bytes, nibbles 8 in .x, .y
        uint32_t qh; // Q5_1 fifth bits (block 0 low byte)
        uint2 dm;    // two scales (.x; Q5_1: mins in .y)
    };
    auto load_w = [&](WStage &s, int kp) __attribute__((always_inline)) {
        kp = min(kp, KP - 1);
        const int tile = tile0 + kp;
        if (BYTES) {
            s.q = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, 16 * lane, tile * 1024, 0));
        } else {
            const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rq, 8 * lane, tile * 512, 0));
            s.q = make_uint4(v.x, v.y, 0u, 0u);
        }
        if (TYPE == kQ5_1) {
            s.qh = __builtin_amdgcn_raw_buffer_load_b16(rh, 2 * lane, tile * 128, 0);
            s.dm = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rd, 8 * rl, tile * 128, 0));
        } else {
            s.dm.x = __builtin_amdgcn_raw_buffer_load_b32(rd, 4 * rl, tile * 64, 0);
        }
    };

    float acc[TM][4], off[TM][4];
#pragma unroll
    for (int mi = 0; mi < TM; mi++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[mi][r] = off[mi][r] = 0.0f;

    // pair kp from LDS buffer buf (its blocks at lb0, lb0 + 1 of the chunk);
    // CHECK: the pair may be the last (an odd block count's missing second
    // block) or past it -- every earlier pair is whole and takes no selects
    auto compute = [&](const WStage &s, int kp, int buf, int lb0, auto check) __attribute__((always_inline)) {
        constexpr bool CHECK = decltype(check)::value;
        uint32_t wq[2][2]; // [block][dword]: the lane's 8 quants of each block
        if (TYPE == kQ8_0) {
            wq[0][0] = s.q.x ^ 0x80808080u;
            wq[0][1] = s.q.y ^ 0x80808080u;
            wq[1][0] = s.q.z ^ 0x80808080u;
            wq[1][1] = s.q.w ^ 0x80808080u;
        } else {
#pragma unroll
            for (int bb = 0; bb < 2; bb++) {
                const uint32_t v = bb ? s.q.y : s.q.x;
                uint32_t n0 = v & 0x0f0f0f0fu, n1 = (v >> 4) & 0x0f0f0f0fu;
                if (TYPE == kQ5_1) {
                    const uint32_t hb = (s.qh >> (8 * bb)) & 0xffu;
                    n0 |= (((hb & 15u) * 0x00204081u) & 0x01010101u) << 4;
                    n1 |= (((hb >> 4) * 0x00204081u) & 0x01010101u) << 4;
                }
                wq[bb][0] = n0;
                wq[bb][1] = n1;
            }
        }
#pragma unroll
        for (int bb = 0; bb < 2; bb++) {
            const bool valid = !CHECK || 2 * kp + bb < nb; // past the last block: the select keeps the sums
            const float dw = h2f((uint16_t)(bb ? s.dm.x >> 16 : s.dm.x));
            const float mw = TYPE == kQ5_1 ? h2f((uint16_t)(bb ? s.dm.y >> 16 : s.dm.y)) : 0.0f;
            const long bf = (long)(((uint64_t)wq[bb][1] << 32) | wq[bb][0]);
#pragma unroll
            for (int mi = 0; mi < TM; mi++) {
                const long af = *(const long *)&sa[buf][mi][lb0 + bb][8 * lane];
                const int4v p = __builtin_amdgcn_mfma_i32_16x16x32_i8(af, bf, int4v{0, 0, 0, 0}, 0, 0, 0);
                // this lane's outputs: tokens 16 tg + 4 g + r, column rl
                const float4 xd = *(const float4 *)&sd[buf][mi][lb0 + bb][4 * g];
                float4 xa = make_float4(0.f, 0.f, 0.f, 0.f);
                if (AUX) xa = *(const float4 *)&sx[buf][mi][lb0 + bb][4 * g];
                const float xdv[4] = {xd.x, xd.y, xd.z, xd.w};
                const float xav[4] = {xa.x, xa.y, xa.z, xa.w};
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int sumi = TYPE == kQ4_0 ? p[r] - 8 * __builtin_bit_cast(int, xav[r]) : p[r];
                    const float sc = dw * xdv[r];
                    const float v = acc[mi][r] + sc * (float)sumi;
                    acc[mi][r] = CHECK ? (valid ? v : acc[mi][r]) : v;
                    if (TYPE == kQ5_1) {
                        const float o = off[mi][r] + mw * xav[r];
                        off[mi][r] = CHECK ? (valid ? o : off[mi][r]) : o;
                    }
                }
            }
        }
    };

    // ---- pipeline
    AChunk ar;
    WStage ring[DEPTH];
    load_a(0, ar);
#pragma unroll
    for (int d = 0; d < DEPTH; d++) load_w(ring[d], d);
    store_a(0, ar);
    auto chunk = [&](int c, auto check) __attribute__((always_inline)) {
        constexpr bool CHECK = decltype(check)::value;
        const int buf = c & 1;
        __syncthreads(); // chunk c staged by every wave; the other buffer is free
        load_a(c + 1, ar); // past the last chunk: clamped reloads nobody reads
#pragma unroll
        for (int j = 0; j < CH; j++) {
            const int kp = c * CH + j;
            if (!CHECK || kp < KP) compute(ring[j % DEPTH], kp, buf, 2 * j, check);
            load_w(ring[j % DEPTH], kp + DEPTH);
            // one pair at a time: the sums are taken here (left to the end of
            // the chunk, every pair's products and scale terms stay live)
#pragma unroll
            for (int mi = 0; mi < TM; mi++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    asm volatile("" : "+v"(acc[mi][r]));
                    if (TYPE == kQ5_1) asm volatile("" : "+v"(off[mi][r]));
                }
            __builtin_amdgcn_sched_barrier(0);
        }
        store_a(buf ^ 1, ar);
    };
    for (int c = 0; c + 1 < nchunk; c++) chunk(c, std::false_type{});
    chunk(nchunk - 1, std::true_type{});

    const int col = rgw * 16 + rl;
    if (col >= w.rows) return;
#pragma unroll
    for (int mi = 0; mi < TM; mi++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int t = 16 * (tg0 + mi) + 4 * g + r;
            if (t < a.T) a.y[(size_t)t * a.ldy + col] = TYPE == kQ5_1 ? acc[mi][r] + off[mi][r] : acc[mi][r];
        }
}

template <int TYPE, int TM>
static hipError_t launch_i8_cfg(const GemmI8Args &a, hipStream_t s)
{
    const int groups = (a.T + 15) / 16;
    dim3 grid((a.w.rows + 63) / 64, (groups + TM - 1) / TM);
    hipLaunchKernelGGL((gemm_i8_kernel<TYPE, TM>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int TYPE>
static hipError_t launch_i8_typed(const GemmI8Args &a, hipStream_t s)
{
    // token groups per wave: a divisor of the group count (the padded
    // activation tiles a wave reads always exist), as many as keep at least
    // 1024 workgroups (four waves per SIMD) in flight
    const int groups = (a.T + 15) / 16, cols = (a.w.rows + 63) / 64;
    if (groups % 4 == 0 && cols * (groups / 4) >= 1024) return launch_i8_cfg<TYPE, 4>(a, s);
    if (groups % 2 == 0 && cols * (groups / 2) >= 1024) return launch_i8_cfg<TYPE, 2>(a, s);
    return launch_i8_cfg<TYPE, 1>(a, s);
}

hipError_t launch_gemm_i8(const GemmI8Args &a, hipStream_t s)
{
    if (a.T <= 0) return hipSuccess;
    if (a.w.cols % 32 != 0 || a.T16 < ((a.T + 15) & ~15) || a.ldy < a.w.rows) return hipErrorInvalidValue;
    switch (a.w.type) {
    case kQ8_0: return launch_i8_typed<kQ8_0>(a, s);
    case kQ4_0: return launch_i8_typed<kQ4_0>(a, s);
    case kQ5_1: return launch_i8_typed<kQ5_1>(a, s);
    default: return hipErrorInvalidValue;
    }
}

} // namespace jev
