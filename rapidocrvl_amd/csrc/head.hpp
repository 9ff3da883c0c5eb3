// head.hpp — the greedy LM head (MatVecArgmaxQ*, internal/tensor/
// argmax_quant.go:11-433) on the matrix cores, for 1 to kHeadMaxVec
// activation vectors at once.
//
// Each vector is written as three int8 digit planes under one power-of-two
// scale S ≥ max|y|/127 over its columns (y = x, or x·w under RMSNorm with the
// factor fastRsqrt(Σx²/n + eps) applied to the score, ops.go:1015-1037):
//   y = S·(d0 + d1/2⁷ + d2/2¹⁴) + e,   |e| ≤ S/2¹⁵,
// the planes of vector v are columns 3v, 3v+1, 3v+2 of the B operand of
// v_mfma_i32_16x16x64_i8, and the weight codes enter as stored (Q4 nibbles
// u = code + 8, Q6 fields u = code + 32, Q8 bytes): a row's three plane sums
// are exact int32, the code offset leaves as IBIAS·Σd, and only the final
// combination is f32.  One MFMA per 64 columns serves every vector; the
// weight unpack costs 0–2 VALU operations per 8 codes, where a VALU dot
// product of the same precision costs 7.
//
// Launch: a workgroup owns kHeadRB blocks of 16 rows; its four waves split
// the columns in quarters, request all their weight bytes before the
// digitizing prologue, sum their exact partials through LDS, and wave w
// finishes blocks w, w + 4, …: scores, the optional score rows, the argmax key
// (order-preserving score bits · 2³² + ~row: ties go to the lowest row,
// argmax_quant.go:255-262) folded into the vector's argmax slot.
#pragma once

#include "gemm.hpp"

namespace pocr {

constexpr int kHeadMaxVec = 4;  // vectors per launch (two per 16-column B tile)
#ifndef POCR_HEAD_RB
#define POCR_HEAD_RB 4
#endif
constexpr int kHeadRB = POCR_HEAD_RB;  // row blocks (16 rows) per workgroup, a multiple of kWaves
static_assert(kHeadRB % kWaves == 0, "wave w finishes blocks w, w + 4, …");

struct HeadParams {
    DevMat m;
    int rows;
    const float *x;        // vector v at x + v·x_stride (cols floats)
    int x_stride;
    const float *norm_w;   // null → the scores use x as given
    float eps;
    float *out;            // optional: scores of vector v at out + v·out_stride
    int out_stride;
    StepState *st[kHeadMaxVec];  // argmax slots of vector v
};

// The shape of the work.  Every load instruction of a wave reads 8 weight
// rows × one 128-byte line: lane (lr, lg) reads the 16 bytes at
// 64·(lr/8) + 16·lg of its row's line (row lr % 8 of the row group).  In the
// MFMA, A-row lr < 8 thus carries the first half of the line and A-row
// lr + 8 the second half of the same weight row; the two halves are
// separate B columns (6 per vector: half hb, plane pl → 6v + 3hb + pl), and
// a row's partial sums are C[lr][3hb+pl] with lr/8 = hb, added afterwards.
// Q4: a 16-byte piece is 32 codes, two MFMA steps of 8 bytes; Q8: one step.
template <int QT>
constexpr int head_steps_per_load() { return QT == QT_Q4 ? 2 : 1; }
// first column (relative to the wave's quarter) of step h of line ℓ, half hb,
// lane group lg: 16 columns in the MFMA K order (digit_pos16)
template <int QT>
__device__ __forceinline__ int head_col(int l, int hb, int lg, int h) {
    if constexpr (QT == QT_Q4) return 256 * l + 128 * hb + 32 * lg + 16 * h;
    else return 128 * l + 64 * hb + 16 * lg;
}

template <int CTL>
__device__ __forceinline__ unsigned long long key_max_dpp(unsigned long long k) {
    const uint32_t hi = (uint32_t)(k >> 32), lo = (uint32_t)k;
    const uint32_t oh = __builtin_amdgcn_update_dpp(0u, hi, CTL, 0xF, 0xF, false);
    const uint32_t ol = __builtin_amdgcn_update_dpp(0u, lo, CTL, 0xF, 0xF, false);
    const unsigned long long o = ((unsigned long long)oh << 32) | ol;
    return o > k ? o : k;
}

// NS: cols = 256·NS; a wave's quarter of the columns is LINES 128-byte lines
// of every row.  NV vectors need ⌈6·NV/16⌉ B tiles (two vectors per tile).
template <int QT, int NS, int NV>
__global__ void __launch_bounds__(kThreads) k_head_mfma(HeadParams p) {
    static_assert(QT == QT_Q4 || QT == QT_Q8, "Q6 rows do not fall on 128-byte lines");
    static_assert(NV == 1 || NV == 2 || NV == 4, "vectors per launch");
    constexpr int COLS = 256 * NS;
    constexpr int LINES = (QT == QT_Q4 ? 32 * NS : 64 * NS) / 128;  // per row, per wave
    constexpr int SPL = head_steps_per_load<QT>();
    constexpr int T = (NV + 1) / 2;  // B tiles
    constexpr int RB = kHeadRB;
    constexpr int PER_T = COLS / kThreads;  // prologue columns per thread
    static_assert(PER_T == 4 || PER_T == 8, "prologue handles 4 or 8 columns per thread");
    static_assert(LINES >= 1, "a wave's quarter is a whole number of lines");
    constexpr int IB = DigitTraits<QT>::IBIAS;
    __shared__ __attribute__((aligned(16))) int8_t xdig[3][NV][COLS];
    // partial plane sums: [wave][row block][row 0..15][vector][half][plane]
    __shared__ int part[kWaves][RB][16][NV][2][3];
    __shared__ float redf[2][NV][kWaves];
    __shared__ int redi[3][NV][kWaves];
    __shared__ unsigned long long kred[NV][kWaves];
    // every kernel argument live up front: one kernel-argument round trip
    asm volatile("" ::"s"(p.m.data), "s"(p.m.scale), "s"(p.x), "s"(p.norm_w), "s"(p.out), "s"(p.rows),
                 "s"(p.m.row_bytes), "s"(p.x_stride), "s"(p.out_stride), "s"(p.eps));

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int rows = p.rows;
    const int rb0 = blockIdx.x * RB;
    const int kbeg = wave * (COLS / kWaves);

    // 1. activations first (a few KB, cached), so that the prologue waits for
    // them and not for the weights: thread t digitizes columns PER_T·t ..
    const int cb = PER_T * (int)threadIdx.x;
    const bool norm = p.norm_w != nullptr;
    float xr[NV][PER_T];
    float nw[PER_T];
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int i = 0; i < PER_T; i += 4) {
            const float4 x4 = *reinterpret_cast<const float4 *>(p.x + (size_t)v * p.x_stride + cb + i);
            xr[v][i] = x4.x;
            xr[v][i + 1] = x4.y;
            xr[v][i + 2] = x4.z;
            xr[v][i + 3] = x4.w;
        }
#pragma unroll
    for (int i = 0; i < PER_T; i += 4) {
        const float4 w4 = norm ? *reinterpret_cast<const float4 *>(p.norm_w + cb + i) : make_float4(1, 1, 1, 1);
        nw[i] = w4.x;
        nw[i + 1] = w4.y;
        nw[i + 2] = w4.z;
        nw[i + 3] = w4.w;
    }

    // 2. this wave's weight lines: row block rb, row group g (8 rows), line l
    typedef unsigned u4v __attribute__((ext_vector_type(4)));
    u4v raw[RB][2][LINES];
    {
        const int qbyte = QT == QT_Q4 ? kbeg / 2 : kbeg;
        const int lb = 64 * (lr >> 3) + 16 * lg;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                const int r = min(16 * (rb0 + rb) + 8 * g + (lr & 7), rows - 1);  // past the end: loaded, never scored
                const uint8_t *row = p.m.data + (size_t)r * p.m.row_bytes + qbyte + lb;
#pragma unroll
                for (int l = 0; l < LINES; ++l)
                    raw[rb][g][l] = __builtin_nontemporal_load(reinterpret_cast<const u4v *>(row + 128 * l));
            }
    }

    // 3. prologue: digits of every vector
    float y[NV][PER_T];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        float ss = 0.0f, mx = 0.0f;
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            ss = fmaf(xr[v][i], xr[v][i], ss);
            y[v][i] = norm ? xr[v][i] * nw[i] : xr[v][i];  // a lone product: nothing to contract
            mx = fmaxf(mx, fabsf(y[v][i]));
        }
        ss = wave_sum(ss);
        mx = wave_max(mx);
        if (lane == 0) {
            redf[0][v][wave] = mx;
            redf[1][v][wave] = ss;
        }
    }
    __syncthreads();
    int ex[NV];
    float sx[NV];  // S·(RMSNorm factor): the vector's score scale
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        float m = redf[0][v][0], tot = redf[1][v][0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) {
            m = fmaxf(m, redf[0][v][w]);
            tot += redf[1][v][w];
        }
        ex[v] = 0;
        (void)frexpf(m * (1.0f / 127.0f), &ex[v]);  // m/127 < 2^ex; m = 0 → ex = 0
        const float S = m > 0.0f ? ldexpf(1.0f, ex[v]) : 1.0f;
        sx[v] = norm ? S * fast_rsqrt_ref(tot / (float)COLS + p.eps) : S;
        int sd[3] = {0, 0, 0};
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const int c = cb + i;
            const float t = ldexpf(y[v][i], -ex[v]);  // exact
            const float a = rintf(t);
            const float t1 = (t - a) * 128.0f;        // exact: |t − a| ≤ 1/2
            const float b = rintf(t1);
            const int d2 = (int)rintf((t1 - b) * 128.0f);
            const int pos = 16 * (c / 16) + digit_pos16<QT>(c % 16);  // the MFMA K order
            xdig[0][v][pos] = (int8_t)(int)a;
            xdig[1][v][pos] = (int8_t)(int)b;
            xdig[2][v][pos] = (int8_t)d2;
            sd[0] += (int)a;
            sd[1] += (int)b;
            sd[2] += d2;
        }
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) {
            const int s = (int)wave_sum((float)sd[pl]);  // |Σ| ≤ 512·127: exact in f32
            if (lane == 0) redi[pl][v][wave] = s;
        }
    }
    __syncthreads();

    // 4. B operands: tile t, column lr = vector 2t + lr/6, half (lr%6)/3, plane lr%3
    v4i b[LINES][SPL][T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int v = 2 * t + lr / 6, hb = (lr % 6) / 3, pl = lr % 3;
        const bool col = lr < 12 && v < NV;
#pragma unroll
        for (int l = 0; l < LINES; ++l)
#pragma unroll
            for (int h = 0; h < SPL; ++h)
                b[l][h][t] = col ? *reinterpret_cast<const v4i *>(&xdig[pl][min(v, NV - 1)][kbeg + head_col<QT>(l, hb, lg, h)])
                                 : v4i{0, 0, 0, 0};
    }

    // 5. the MFMAs: exact int32 partial sums of this wave's columns; lane
    // (lr, lg) ends with C[4lg + i][lr]: row 4lg+i of the block's row group
    // when (4lg + i)/8 is the half of B column lr
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            v4i acc[T];
#pragma unroll
            for (int t = 0; t < T; ++t) acc[t] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int l = 0; l < LINES; ++l)
#pragma unroll
                for (int h = 0; h < SPL; ++h) {
                    RawCodes<QT> rc;
                    if constexpr (QT == QT_Q4) {
                        rc.d[0] = raw[rb][g][l][2 * h];
                        rc.d[1] = raw[rb][g][l][2 * h + 1];
                    } else {
#pragma unroll
                        for (int w = 0; w < 4; ++w) rc.d[w] = raw[rb][g][l][w];
                    }
                    const v4i a = unpack_codes16<QT>(rc);
#pragma unroll
                    for (int t = 0; t < T; ++t) acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[l][h][t], acc[t], 0, 0, 0);
                }
            // keep C[i][col] where i/8 is col's half: rows of lane group lg
            // are 4lg..4lg+3, half (lg ≥ 2)
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int v = 2 * t + lr / 6, hb = (lr % 6) / 3, pl = lr % 3;
                if (lr < 12 && v < NV && hb == (lg >> 1)) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) part[wave][rb][8 * g + ((4 * lg + i) & 7)][v][hb][pl] = acc[t][i];
                }
            }
        }
    __syncthreads();

    // 6. wave w finishes blocks w, w + 4, …: lane (row lr, vector lg) adds the
    // halves and the waves' quarters of its three plane sums
    constexpr int FIN = RB / kWaves;
    const int v = lg;  // lanes of vectors past NV idle
    int b0 = 0, b1 = 0, b2 = 0;
    float sv = sx[0];
    if (v < NV) {
        b0 = IB * (redi[0][v][0] + redi[0][v][1] + redi[0][v][2] + redi[0][v][3]);
        b1 = IB * (redi[1][v][0] + redi[1][v][1] + redi[1][v][2] + redi[1][v][3]);
        b2 = IB * (redi[2][v][0] + redi[2][v][1] + redi[2][v][2] + redi[2][v][3]);
#pragma unroll
        for (int u = 1; u < NV; ++u) sv = v == u ? sx[u] : sv;
    }
    unsigned long long key = 0ull;
#pragma unroll
    for (int f = 0; f < FIN; ++f) {
        const int rb = wave + kWaves * f;
        const int r = 16 * (rb0 + rb) + lr;
        const float rsc = p.m.scale[min(r, rows - 1)];
        if (v < NV) {
            int c0 = 0, c1 = 0, c2 = 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w)
#pragma unroll
                for (int hb = 0; hb < 2; ++hb) {
                    c0 += part[w][rb][lr][v][hb][0];
                    c1 += part[w][rb][lr][v][hb][1];
                    c2 += part[w][rb][lr][v][hb][2];
                }
            // |Σ u·d| < 2^24 per plane (cols ≤ 2048): exact converts
            const float f0 = (float)(c0 - b0);
            const float f1 = (float)(c1 - b1);
            const float f2 = (float)(c2 - b2);
            const float s = fmaf(f2, 1.0f / 16384.0f, fmaf(f1, 1.0f / 128.0f, f0)) * sv * rsc;
            if (r < rows) {
                if (p.out) p.out[(size_t)v * p.out_stride + r] = s;
                const unsigned long long k = argmax_key(s, r);
                key = k > key ? k : key;
            }
        }
    }
    // the best key of each vector over its 16 lanes (one DPP row: quad xor 1,
    // quad xor 2, half-row mirror, row mirror)
    key = key_max_dpp<0xB1>(key);
    key = key_max_dpp<0x4E>(key);
    key = key_max_dpp<0x141>(key);
    key = key_max_dpp<0x140>(key);
    if (lr == 0 && v < NV) kred[v][wave] = key;
    __syncthreads();
    if (threadIdx.x < NV) {
        const int vv = threadIdx.x;
        unsigned long long m = kred[vv][0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) m = kred[vv][w] > m ? kred[vv][w] : m;
        StepState *st = p.st[0];
#pragma unroll
        for (int u = 1; u < NV; ++u) st = vv == u ? p.st[u] : st;
        if (m) atomicMax(&st->argmax_slot[(blockIdx.x % kArgSlots) * kSlotPitch], m);
    }
}

}  // namespace pocr
