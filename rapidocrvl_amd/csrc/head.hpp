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
// 12 bytes on a 4-byte boundary: one global_load_dwordx3
typedef uint32_t U3v __attribute__((ext_vector_type(3), aligned(4)));

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
    StepState *st[kHeadMaxVec];  // argmax slots of vector v (null: scores only)
};

// The shape of the work.  Every load instruction of a wave reads 8 weight
// rows × one 128-byte line: lane (lr, lg) reads the 16 bytes at
// 64·(lr/8) + 16·lg of its row's line (row lr % 8 of the row group).  In the
// MFMA, A-row lr < 8 thus carries the first half of the line and A-row
// lr + 8 the second half of the same weight row; the two halves are
// separate B columns (6 per vector: half hb, plane pl → 6v + 3hb + pl), and
// a row's partial sums are C[lr][3hb+pl] with lr/8 = hb, added afterwards.
// Q4: a 16-byte piece is 32 codes, two MFMA steps of 8 bytes; Q8: one step.
//
// Q6 rows (3 bytes per 4 codes) do not fall on 128-byte lines, so Q6 reads
// 4 rows × 192 contiguous bytes (256 codes) per load instruction: lane
// (lr, lg) reads the 12 bytes (16 codes) at 48·(lr/4) + 12·lg of row lr % 4's
// 192-byte unit. A-row lr thus carries part lr/4 of row lr % 4, and B
// columns are (part, plane) → 3·part + pl (12 per vector, one vector per B
// tile); a row's partial sums are C[lr][3·(lr/4) + pl], added afterwards.
// One MFMA step per load; a wave's quarter of the columns is NS/4 units.
template <int QT>
constexpr int head_steps_per_load() { return QT == QT_Q4 ? 2 : 1; }
// A-rows per weight row within one load instruction: halves (Q4, Q8) or
// parts (Q6)
template <int QT>
constexpr int head_parts() { return QT == QT_Q6 ? 4 : 2; }
// Q6 head image.  The 12-byte pieces of a 192-byte unit straddle 128-byte
// lines (a wave's unit shares lines with its neighbours'), which streams at
// about 0.9 of whole lines.  So Q6 matrices of LM-head size also keep their
// rows in the load order of the heads: unit (b, w, g, l) — block b of 16
// rows, column quarter w, row group g (rows 16b + 4g … + 3), unit l of the
// quarter — is 768 consecutive bytes at ((4b + w)·4 + g)·LINES + l times 768,
// slot L (= lr + 16·lg) holding what lane L of k_head_mfma loads: the 12
// bytes at w·row_bytes/4 + 192·l + 48·(lr/4) + 12·lg of row 16b + 4g + lr%4
// (rows past the end: the last row).  nblk = ⌈rows/16⌉ blocks, nblk·16 rows
// of bytes in all.
__device__ __forceinline__ size_t head_img_unit_q6(int b, int w, int g, int l, int lines) {
    return ((((size_t)b * kWaves + w) * 4 + g) * lines + l) * 768;
}

// one thread per (unit, slot): 3 dwords
static __global__ void __launch_bounds__(kThreads) k_head_image_q6(const uint8_t *src, int row_bytes, int rows,
                                                                 int nblk, uint8_t *dst) {
    const int lines = row_bytes / 768;
    const size_t id = (size_t)blockIdx.x * kThreads + threadIdx.x;
    const size_t units = (size_t)nblk * 16 * lines;
    if (id >= units * 64) return;
    const int L = (int)(id % 64);
    const size_t u = id / 64;
    const int l = (int)(u % lines), g = (int)(u / lines % 4), w = (int)(u / lines / 4 % kWaves);
    const int b = (int)(u / lines / 4 / kWaves);
    const int lr = L & 15, lg = L >> 4;
    const int r = min(16 * b + 4 * g + (lr & 3), rows - 1);
    const uint32_t *s = reinterpret_cast<const uint32_t *>(src + (size_t)r * row_bytes + w * (row_bytes / 4) + 192 * l +
                                                           48 * (lr >> 2) + 12 * lg);
    uint32_t *d = reinterpret_cast<uint32_t *>(dst + head_img_unit_q6(b, w, g, l, lines) + 12 * L);
    d[0] = s[0];
    d[1] = s[1];
    d[2] = s[2];
}

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
    static_assert(QT != QT_Q6 || NS % 4 == 0, "Q6: whole 192-byte units per wave quarter");
    static_assert(NV == 1 || NV == 2 || NV == 4, "vectors per launch");
    constexpr bool Q6 = QT == QT_Q6;
    constexpr int COLS = 256 * NS;
    // loads per row group and wave: 128-byte lines (Q4, Q8) or 192-byte
    // units (Q6) of the wave's quarter of every row
    constexpr int LINES = Q6 ? NS / 4 : (QT == QT_Q4 ? 32 * NS : 64 * NS) / 128;
    constexpr int SPL = head_steps_per_load<QT>();
    constexpr int NP = head_parts<QT>();
    constexpr int G = NP;            // row groups of 16/NP rows per block of 16
    constexpr int T = Q6 ? NV : (NV + 1) / 2;  // B tiles
    constexpr int RB = kHeadRB;
    constexpr int PER_T = COLS / kThreads;  // prologue columns per thread
    static_assert(PER_T == 4 || PER_T == 8, "prologue handles 4 or 8 columns per thread");
    static_assert(LINES >= 1, "a wave's quarter is a whole number of lines");
    constexpr int IB = DigitTraits<QT>::IBIAS;
    __shared__ __attribute__((aligned(16))) int8_t xdig[3][NV][COLS];
    // partial plane sums: [wave][row block][row 0..15][vector][half/part][plane]
    __shared__ int part[kWaves][RB][16][NV][NP][3];
    __shared__ float redf[2][NV][kWaves];
    __shared__ int redi[3][NV][kWaves];
    __shared__ unsigned long long kred[NV][kWaves];
    // every kernel argument live up front: one kernel-argument round trip
    asm volatile("" ::"s"(p.m.data), "s"(p.m.scale), "s"(p.x), "s"(p.norm_w), "s"(p.out), "s"(p.rows),
                 "s"(p.m.row_bytes), "s"(p.x_stride), "s"(p.out_stride), "s"(p.eps));
    if constexpr (QT == QT_Q6) asm volatile("" ::"s"(p.m.head_img));

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

    // 2. this wave's weight lines: row block rb, row group g (16/NP rows),
    // line or unit l
    typedef unsigned u4v __attribute__((ext_vector_type(4)));
    // Q6 pieces: 12 bytes on 4-byte boundaries, one global_load_dwordx3 each
    // (a 3-vector of dword alignment: 12 bytes read, none past the piece)
    struct U3 {
        uint32_t d[3];
        __device__ __forceinline__ uint32_t operator[](int i) const { return d[i]; }
    };
    using RawT = std::conditional_t<Q6, U3, u4v>;
    RawT raw[RB][G][LINES];
    {
        constexpr int RPG = 16 / NP;  // rows per load instruction
        const int qbyte = Q6 ? kbeg / 4 * 3 : (QT == QT_Q4 ? kbeg / 2 : kbeg);
        const int lb = Q6 ? 48 * (lr >> 2) + 12 * lg : 64 * (lr >> 3) + 16 * lg;
        constexpr int STRIDE = Q6 ? 192 : 128;
        const int nblk = (rows + 15) / 16;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int g = 0; g < G; ++g) {
                // past the end: loaded, never scored
                const int r = min(16 * (rb0 + rb) + RPG * g + (lr % RPG), rows - 1);
                const uint8_t *row = p.m.data + (size_t)r * p.m.row_bytes + qbyte + lb;
#pragma unroll
                for (int l = 0; l < LINES; ++l) {
                    if constexpr (Q6) {
                        // the same 12 bytes from the head image when there is one
                        const uint8_t *src =
                            p.m.head_img ? p.m.head_img + head_img_unit_q6(min(rb0 + rb, nblk - 1), wave, g, l, LINES) +
                                               12 * lane
                                         : row + STRIDE * l;
                        const U3v q = __builtin_nontemporal_load(reinterpret_cast<const U3v *>(src));
                        raw[rb][g][l].d[0] = q.x;
                        raw[rb][g][l].d[1] = q.y;
                        raw[rb][g][l].d[2] = q.z;
                    } else {
                        raw[rb][g][l] = __builtin_nontemporal_load(reinterpret_cast<const u4v *>(row + STRIDE * l));
                    }
                }
            }
    }

    // the row scales the finish needs, requested with the weights (a load at
    // the finish would add a memory round trip to every workgroup's tail)
    constexpr int FIN = RB / kWaves;
    float rsc[FIN];
#pragma unroll
    for (int f = 0; f < FIN; ++f) rsc[f] = p.m.scale[min(16 * (rb0 + wave + kWaves * f) + lr, rows - 1)];

    // 3. prologue: digits of every vector.  Only the scale S (the largest
    // |y|) stands between the activations and the MFMAs; the thread's Σx² and
    // plane sums wait in registers and are reduced after the MFMAs, in the
    // same order, before the finish's barrier.
    float y[NV][PER_T];
    float ssk[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        float ss = 0.0f, mx = 0.0f;
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            ss = fmaf(xr[v][i], xr[v][i], ss);
            y[v][i] = norm ? xr[v][i] * nw[i] : xr[v][i];  // a lone product: nothing to contract
            mx = fmaxf(mx, fabsf(y[v][i]));
        }
        ssk[v] = ss;
        mx = wave_max(mx);
        if (lane == 0) redf[0][v][wave] = mx;
    }
    __syncthreads();
    float sx[NV];  // S, and after the finish's barrier S·(RMSNorm factor): the vector's score scale
    int sdk[NV][3];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        float m = redf[0][v][0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) m = fmaxf(m, redf[0][v][w]);
        int ex = 0;
        (void)frexpf(m * (1.0f / 127.0f), &ex);  // m/127 < 2^ex; m = 0 → ex = 0
        sx[v] = m > 0.0f ? ldexpf(1.0f, ex) : 1.0f;
        int sd[3] = {0, 0, 0};
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const int c = cb + i;
            const float t = ldexpf(y[v][i], -ex);  // exact
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
        for (int pl = 0; pl < 3; ++pl) sdk[v][pl] = sd[pl];
    }
    __syncthreads();

    // 4. B operands: Q4/Q8 tile t, column lr = vector 2t + lr/6, half
    // (lr%6)/3, plane lr%3; Q6 tile t = vector t, column lr = part lr/3,
    // plane lr%3 (unit l of the quarter: columns 256·l + 64·part + 16·lg)
    v4i b[LINES][SPL][T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int v = Q6 ? t : 2 * t + lr / 6, hb = Q6 ? lr / 3 : (lr % 6) / 3, pl = lr % 3;
        const bool col = lr < 12 && v < NV;
#pragma unroll
        for (int l = 0; l < LINES; ++l)
#pragma unroll
            for (int h = 0; h < SPL; ++h) {
                const int c = Q6 ? 256 * l + 64 * hb + 16 * lg : head_col<QT>(l, hb, lg, h);
                b[l][h][t] = col ? *reinterpret_cast<const v4i *>(&xdig[pl][min(v, NV - 1)][kbeg + c])
                                 : v4i{0, 0, 0, 0};
            }
    }

    // 5. the MFMAs: exact int32 partial sums of this wave's columns; lane
    // (lr, lg) ends with C[4lg + i][lr]: row 4lg+i of the block's row group
    // when (4lg + i)/8 is the half of B column lr (Q6: row i of the group
    // when lg is the part of B column lr)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int g = 0; g < G; ++g) {
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
                    } else if constexpr (Q6) {
#pragma unroll
                        for (int w = 0; w < 3; ++w) rc.d[w] = raw[rb][g][l][w];
                    } else {
#pragma unroll
                        for (int w = 0; w < 4; ++w) rc.d[w] = raw[rb][g][l][w];
                    }
                    const v4i a = unpack_codes16<QT>(rc);
#pragma unroll
                    for (int t = 0; t < T; ++t) acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[l][h][t], acc[t], 0, 0, 0);
                }
            // keep C[i][col] where i/8 is col's half: rows of lane group lg
            // are 4lg..4lg+3, half (lg ≥ 2); Q6: A-rows 4lg..4lg+3 are part
            // lg of the group's rows 0..3
#pragma unroll
            for (int t = 0; t < T; ++t) {
                if constexpr (Q6) {
                    const int v = t, pt = lr / 3, pl = lr % 3;
                    if (lr < 12 && pt == lg) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) part[wave][rb][4 * g + i][v][pt][pl] = acc[t][i];
                    }
                } else {
                    const int v = 2 * t + lr / 6, hb = (lr % 6) / 3, pl = lr % 3;
                    if (lr < 12 && v < NV && hb == (lg >> 1)) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) part[wave][rb][8 * g + ((4 * lg + i) & 7)][v][hb][pl] = acc[t][i];
                    }
                }
            }
        }
    // the deferred sums: each vector's plane sums (|Σ| ≤ 512·127: exact in
    // f32) and Σx², per wave
#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) {
            const int s = (int)wave_sum((float)sdk[v][pl]);
            if (lane == 0) redi[pl][v][wave] = s;
        }
        const float ss = wave_sum(ssk[v]);
        if (lane == 0) redf[1][v][wave] = ss;
    }
    __syncthreads();
    if (norm) {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            float tot = redf[1][v][0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) tot += redf[1][v][w];
            sx[v] *= fast_rsqrt_ref(tot / (float)COLS + p.eps);
        }
    }

    // 6. wave w finishes blocks w, w + 4, …: lane (row lr, vector lg) adds the
    // halves and the waves' quarters of its three plane sums
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
        if (v < NV) {
            int c0 = 0, c1 = 0, c2 = 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w)
#pragma unroll
                for (int hb = 0; hb < NP; ++hb) {
                    c0 += part[w][rb][lr][v][hb][0];
                    c1 += part[w][rb][lr][v][hb][1];
                    c2 += part[w][rb][lr][v][hb][2];
                }
            // |Σ u·d| < 2^24 per plane (cols ≤ 2048): exact converts
            const float f0 = (float)(c0 - b0);
            const float f1 = (float)(c1 - b1);
            const float f2 = (float)(c2 - b2);
            const float s = fmaf(f2, 1.0f / 16384.0f, fmaf(f1, 1.0f / 128.0f, f0)) * sv * rsc[f];
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
        if (m && st) atomicMax(&st->argmax_slot[(blockIdx.x % kArgSlots) * kSlotPitch], m);
    }
}

// ---------------------------------------------------------------------------
// The same head for 2 to 16 vectors (the batched decode's greedy members, or
// M rows of scores), in two launches.
//
// k_head_digits (one workgroup per vector) writes each vector's three digit
// planes, its score scale and its plane biases exactly as k_head_mfma makes
// them (same thread → column map and reduction order), so a vector's scores
// are bit-identical to that kernel's: a row's three plane sums are exact.
// The planes land in the order the head's B operands are read, 16 bytes per
// (step, plane, lane group, vector), so a B read is 64 consecutive 16-byte
// pieces in LDS and the head copies only the live vectors' pieces.
//
// k_head_wide: one B tile per digit plane holds all 16 vectors (column =
// vector), so every MFMA column is used and the A operand is 16 distinct
// weight rows.  Weights are read as whole 128-byte lines (8 rows per load
// instruction; a 16-rows × 64-byte pattern streams at two thirds of the
// rate on MI355X) and one DPP rotate per dword forms the A operands.  A wave
// owns R blocks of 16 rows over all the columns (no cross-wave sums) and
// requests every weight byte of its rows at once (R·row bytes/4 per lane,
// 512 at most), right behind the digit planes.
// ---------------------------------------------------------------------------
constexpr int kHeadWideVec = 16;
#ifndef POCR_HEAD_WIDE_LANE_BYTES
#define POCR_HEAD_WIDE_LANE_BYTES 512  // weight bytes a lane requests at once
#endif

// LB: weight bytes a lane requests at once (R row blocks of 16 rows per wave)
template <int QT, int NS, int LB = POCR_HEAD_WIDE_LANE_BYTES>
struct HeadWideShape {
    static constexpr int COLS = 256 * NS;
    static constexpr int ROW_BYTES = QT == QT_Q4 ? COLS / 2 : (QT == QT_Q6 ? COLS / 4 * 3 : COLS);
    static constexpr int LINES = ROW_BYTES / 128;  // 128-byte lines per row (Q4, Q8)
    static constexpr int CP = QT == QT_Q4 ? 32 : 16;  // codes per 16-byte piece
    static constexpr int SPL = head_steps_per_load<QT>();
    // MFMA steps of 64 columns
    static constexpr int STEPS = QT == QT_Q6 ? COLS / 64 : LINES * 2 * SPL;
    static constexpr int PLANE_BYTES = STEPS * 3 * 4 * kHeadWideVec * 16;
    static constexpr int R0 = LB * 4 / ROW_BYTES;
    static constexpr int R = R0 > 1 ? R0 : 1;  // row blocks per wave
    static constexpr int ROWS_PER_WG = 16 * R * kWaves;
};

// byte offset of column c's digit (plane pl, vector v) in the planes buffer:
// step (line ln, piece parity par, half h), lane group g of K slice
// 8·CP·ln + 2·CP·g + CP·par + 16·h, digit_pos16 order inside the 16 columns
template <int QT, int NS>
__device__ __forceinline__ int head_plane_off(int c, int pl, int v) {
    using SH = HeadWideShape<QT, NS>;
    if constexpr (QT == QT_Q6) {
        // k_head_wide_q6: step c/64, lane group (c%64)/16, natural order
        return (((c / 64) * 3 + pl) * 4 + (c % 64) / 16) * 256 + v * 16 + c % 16;
    }
    const int ln = c / (8 * SH::CP), rem = c % (8 * SH::CP);
    const int g = rem / (2 * SH::CP), rem2 = rem % (2 * SH::CP);
    const int par = rem2 / SH::CP, h = (rem2 % SH::CP) / 16;
    const int st = (ln * 2 + par) * SH::SPL + h;
    return ((st * 3 + pl) * 4 + g) * 256 + v * 16 + digit_pos16<QT>(c % 16);
}

struct HeadDigitParams {
    const float *x;        // vector v at x + v·x_stride (cols floats)
    int x_stride;
    const float *norm_w;   // null → the scores use x as given
    float eps;
    int8_t *planes;        // HeadWideShape::PLANE_BYTES
    float *vscale;         // [16] S·(RMSNorm factor)
    int *vbias;            // [16][3] IBIAS·Σd per plane
};

template <int QT, int NS>
__global__ void __launch_bounds__(kThreads) k_head_digits(HeadDigitParams p) {
    constexpr int COLS = 256 * NS;
    constexpr int PER_T = COLS / kThreads;
    constexpr int IB = DigitTraits<QT>::IBIAS;
    __shared__ float redf[2][kWaves];
    __shared__ int redi[3][kWaves];
    const int v = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int cb = PER_T * (int)threadIdx.x;
    const bool norm = p.norm_w != nullptr;
    float xr[PER_T], y[PER_T];
    float ss = 0.0f, mx = 0.0f;
#pragma unroll
    for (int i = 0; i < PER_T; i += 4) {
        const float4 x4 = *reinterpret_cast<const float4 *>(p.x + (size_t)v * p.x_stride + cb + i);
        const float4 w4 = norm ? *reinterpret_cast<const float4 *>(p.norm_w + cb + i) : make_float4(1, 1, 1, 1);
        xr[i] = x4.x;
        xr[i + 1] = x4.y;
        xr[i + 2] = x4.z;
        xr[i + 3] = x4.w;
        y[i] = norm ? x4.x * w4.x : x4.x;  // a lone product: nothing to contract
        y[i + 1] = norm ? x4.y * w4.y : x4.y;
        y[i + 2] = norm ? x4.z * w4.z : x4.z;
        y[i + 3] = norm ? x4.w * w4.w : x4.w;
    }
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
        ss = fmaf(xr[i], xr[i], ss);
        mx = fmaxf(mx, fabsf(y[i]));
    }
    ss = wave_sum(ss);
    mx = wave_max(mx);
    if (lane == 0) {
        redf[0][wave] = mx;
        redf[1][wave] = ss;
    }
    __syncthreads();
    float m = redf[0][0], tot = redf[1][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
        m = fmaxf(m, redf[0][w]);
        tot += redf[1][w];
    }
    int ex = 0;
    (void)frexpf(m * (1.0f / 127.0f), &ex);  // m/127 < 2^ex; m = 0 → ex = 0
    const float S = m > 0.0f ? ldexpf(1.0f, ex) : 1.0f;
    int sd[3] = {0, 0, 0};
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
        const int c = cb + i;
        const float t = ldexpf(y[i], -ex);  // exact
        const float a = rintf(t);
        const float t1 = (t - a) * 128.0f;  // exact: |t − a| ≤ 1/2
        const float b = rintf(t1);
        const int d0 = (int)a, d1 = (int)b, d2 = (int)rintf((t1 - b) * 128.0f);
        p.planes[head_plane_off<QT, NS>(c, 0, v)] = (int8_t)d0;
        p.planes[head_plane_off<QT, NS>(c, 1, v)] = (int8_t)d1;
        p.planes[head_plane_off<QT, NS>(c, 2, v)] = (int8_t)d2;
        sd[0] += d0;
        sd[1] += d1;
        sd[2] += d2;
    }
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) {
        const int s = (int)wave_sum((float)sd[pl]);  // |Σ| ≤ 512·127: exact in f32
        if (lane == 0) redi[pl][wave] = s;
    }
    __syncthreads();
    if (threadIdx.x < 3) {
        const int pl = threadIdx.x;
        p.vbias[v * 3 + pl] = IB * (redi[pl][0] + redi[pl][1] + redi[pl][2] + redi[pl][3]);
    }
    if (threadIdx.x == 3) p.vscale[v] = norm ? S * fast_rsqrt_ref(tot / (float)COLS + p.eps) : S;
}

struct HeadWideParams {
    DevMat m;
    int rows;
    int nvec;              // 1..16; B columns of other vectors are never read into C
    const int8_t *planes;  // k_head_digits' output
    const float *vscale;
    const int *vbias;
    float *out;            // optional: scores of vector v at out + v·out_stride
    int out_stride;
    int out_vec4;          // out 16-byte aligned, out_stride % 4 == 0, rows % 16 == 0
    StepState *st[kHeadWideVec];  // argmax slots of vector v (null: no argmax)
};

// PK (up to 5 vectors): one B tile holds every (vector, plane) pair, column
// 3v + pl, so one MFMA per A operand instead of one per plane; the lane of
// column 3v gathers planes 1 and 2 from its two neighbours for the finish.
// Row blocks per wave: with few vectors the finish is short, so the Q4 head of
// 1024 columns takes 2 blocks per wave (twice the workgroups; M = 3-5 on the
// 103424-row head 19.1-19.4 -> 18.1-18.5 us), and 4 otherwise (M = 16: 22.5
// against 23.2 us with 2).
template <int QT, int NS, bool PK>
constexpr int head_wide_lane_bytes() {
    return (PK && QT == QT_Q4 && NS == 4) ? POCR_HEAD_WIDE_LANE_BYTES / 2 : POCR_HEAD_WIDE_LANE_BYTES;
}
template <int QT, int NS, bool PK>
using HeadWideShapeK = HeadWideShape<QT, NS, head_wide_lane_bytes<QT, NS, PK>()>;

template <int QT, int NS, bool PK>
__global__ void __launch_bounds__(kThreads, 2) k_head_wide(HeadWideParams p) {
    static_assert(QT == QT_Q4 || QT == QT_Q8, "codes in 16-byte pieces of 16 or 32 columns");
    using SH = HeadWideShapeK<QT, NS, PK>;
    constexpr int LINES = SH::LINES, R = SH::R, CP = SH::CP, SPL = SH::SPL;
    constexpr int NV = kHeadWideVec;
    static_assert(R >= 1 && LINES >= 1, "rows of whole 128-byte lines");
    static_assert(SH::PLANE_BYTES % (16 * NV) == 0, "planes in 16-vector groups of 16 bytes");
    __shared__ __attribute__((aligned(16))) int8_t xdig[SH::PLANE_BYTES];
    __shared__ unsigned long long kred[NV][kWaves];
    asm volatile("" ::"s"(p.m.data), "s"(p.m.scale), "s"(p.planes), "s"(p.vscale), "s"(p.vbias), "s"(p.out),
                 "s"(p.rows), "s"(p.m.row_bytes), "s"(p.out_stride), "s"(p.nvec), "s"(p.out_vec4));

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int rows = p.rows;
    const int nvec = p.nvec;
    const int r0 = (blockIdx.x * kWaves + wave) * 16 * R;  // this wave's first row

    // 1. the live vectors' digit pieces (16 bytes each), requested first so
    // that filling LDS waits for them alone
    constexpr int GROUPS = SH::PLANE_BYTES / (16 * NV);  // (step, plane, lane group) groups
    constexpr int MAXK = (GROUPS * NV + kThreads - 1) / kThreads;
    const int npieces = GROUPS * nvec;
    v4i piece[MAXK];
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
        const int id = (int)threadIdx.x + k * kThreads;
        if (id < npieces) {
            const int off = (id / nvec) * 256 + (id % nvec) * 16;
            piece[k] = *reinterpret_cast<const v4i *>(p.planes + off);
        }
    }
    asm volatile("" ::: "memory");  // the weight requests stay behind the pieces

    // 2. every weight byte of the wave's rows (past the end: the last row,
    // loaded and never scored), in the order the MFMAs consume them.  A load
    // instruction reads 8 rows × one 128-byte line: lane L takes the 16
    // bytes at 16·(L/8) of row 8·hf + L%8 of its block (half hf), so each
    // piece k = L/8 of a line holds CP codes.
    typedef unsigned u4v __attribute__((ext_vector_type(4)));
    u4v raw[R][2][LINES];
    const uint8_t *wrow[R][2];
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
            wrow[rb][hf] = p.m.data + (size_t)min(r0 + 16 * rb + 8 * hf + (lane & 7), rows - 1) * p.m.row_bytes +
                           16 * (lane >> 3);
#pragma unroll
    for (int ln = 0; ln < LINES; ++ln)
#pragma unroll
        for (int rb = 0; rb < R; ++rb)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
                raw[rb][hf][ln] = __builtin_nontemporal_load(reinterpret_cast<const u4v *>(wrow[rb][hf] + 128 * ln));
    // LDS gets the pieces; every thread then passes the barrier
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
        const int id = (int)threadIdx.x + k * kThreads;
        if (id < npieces) {
            const int off = (id / nvec) * 256 + (id % nvec) * 16;
            *reinterpret_cast<v4i *>(xdig + off) = piece[k];
        }
    }
    float rsc[R][4];  // row scales, first used after the MFMAs
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) rsc[rb][i] = p.m.scale[min(r0 + 16 * rb + 4 * lg + i, rows - 1)];
    __syncthreads();

    // 3. the MFMAs.  The A operand wants lane L = (lr, lg) to hold row lr's
    // K slice lg.  Of a line, the even pieces 2g of rows 0..7 sit in lanes
    // with L%16 < 8 of half 0, those of rows 8..15 in lanes L ^ 8 of half 1
    // (one DPP row rotate away); odd pieces 2g + 1 the other way round.  So
    // set par (0: even, 1: odd) is own data where bit 3 of L equals par and
    // the rotated other half elsewhere, and K slice lg of set par is piece
    // 2·lg + par: columns 8·CP·ln + 2·CP·lg + CP·par + 16·h for step h.
    // B column lr = vector lr.
    constexpr int NA = PK ? 1 : 3;  // accumulators (B tiles) per row block
    v4i acc[R][NA];
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
#pragma unroll
        for (int pl = 0; pl < NA; ++pl) acc[rb][pl] = v4i{0, 0, 0, 0};
    const int bit3 = (lane >> 3) & 1;
    // PK: column lr = vector lr/3, plane lr%3 (column 15 repeats column 14 and
    // is never read into a score)
    const int pk_off = ((min(lr, 14) % 3) * 4 + lg) * 256 + (min(lr, 14) / 3) * 16;
#pragma unroll
    for (int ln = 0; ln < LINES; ++ln)
#pragma unroll
        for (int par = 0; par < 2; ++par) {
            u4v aset[R];
#pragma unroll
            for (int rb = 0; rb < R; ++rb) {
                const u4v own = raw[rb][par][ln];
                const u4v far = raw[rb][1 - par][ln];
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const unsigned rot = (unsigned)__builtin_amdgcn_update_dpp(0, (int)far[w], 0x128, 0xF, 0xF, false);
                    aset[rb][w] = bit3 == par ? own[w] : rot;
                }
            }
#pragma unroll
            for (int h = 0; h < SPL; ++h) {
                const int st = (ln * 2 + par) * SPL + h;
                v4i b[NA];  // lane (lr, lg): vector lr's K slice lg, 16 consecutive bytes per lane
                if constexpr (PK) {
                    b[0] = *reinterpret_cast<const v4i *>(xdig + st * 3 * 1024 + pk_off);
                } else {
#pragma unroll
                    for (int pl = 0; pl < 3; ++pl)
                        b[pl] = *reinterpret_cast<const v4i *>(xdig + (st * 3 + pl) * 1024 + 16 * lane);
                }
#pragma unroll
                for (int rb = 0; rb < R; ++rb) {
                    RawCodes<QT> rc;
                    if constexpr (QT == QT_Q4) {
                        rc.d[0] = aset[rb][2 * h];
                        rc.d[1] = aset[rb][2 * h + 1];
                    } else {
#pragma unroll
                        for (int w = 0; w < 4; ++w) rc.d[w] = aset[rb][w];
                    }
                    const v4i a = unpack_codes16<QT>(rc);
#pragma unroll
                    for (int pl = 0; pl < NA; ++pl)
                        acc[rb][pl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[pl], acc[rb][pl], 0, 0, 0);
                }
            }
        }

    // 4. lane (lr, lg) holds C[4lg + i][lr]: rows r0 + 16rb + 4lg + i of
    // vector lr (PK: of vector lr/3, plane lr%3; the lane of plane 0 takes
    // planes 1 and 2 from lanes lane + 1 and lane + 2).  Scores as k_head_mfma
    // forms them.
    int pls[R][3][4];
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (PK) {
                pls[rb][0][i] = acc[rb][0][i];
                pls[rb][1][i] = __shfl(acc[rb][0][i], min(lane + 1, 63), 64);
                pls[rb][2][i] = __shfl(acc[rb][0][i], min(lane + 2, 63), 64);
            } else {
#pragma unroll
                for (int pl = 0; pl < 3; ++pl) pls[rb][pl][i] = acc[rb][pl < NA ? pl : 0][i];
            }
        }
    const int v = PK ? lr / 3 : lr;
    const bool live = v < nvec && (!PK || (lr % 3 == 0 && lr < 15));
    int b0 = 0, b1 = 0, b2 = 0;
    float my_sx = 1.0f;
    if (live) {
        b0 = p.vbias[v * 3];
        b1 = p.vbias[v * 3 + 1];
        b2 = p.vbias[v * 3 + 2];
        my_sx = p.vscale[v];
    }
    unsigned long long key = 0ull;
#pragma unroll
    for (int rb = 0; rb < R; ++rb) {
        const int rr = r0 + 16 * rb + 4 * lg;
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // |Σ u·d| < 2^24 per plane (cols ≤ 2048): exact converts
            const float f0 = (float)(pls[rb][0][i] - b0);
            const float f1 = (float)(pls[rb][1][i] - b1);
            const float f2 = (float)(pls[rb][2][i] - b2);
            sc[i] = fmaf(f2, 1.0f / 16384.0f, fmaf(f1, 1.0f / 128.0f, f0)) * my_sx * rsc[rb][i];
            if (live && rr + i < rows) {
                const unsigned long long k = argmax_key(sc[i], rr + i);
                key = k > key ? k : key;
            }
        }
        if (p.out && live) {
            float *o = p.out + (size_t)v * p.out_stride + rr;
            if (p.out_vec4) {
                if (rr < rows) *reinterpret_cast<float4 *>(o) = make_float4(sc[0], sc[1], sc[2], sc[3]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (rr + i < rows) o[i] = sc[i];
            }
        }
    }
    // the best key of vector lr over the four lane groups, then the waves
    {
        const unsigned long long o16 = shfl_xor_u64(key, 16);
        key = o16 > key ? o16 : key;
        const unsigned long long o32 = shfl_xor_u64(key, 32);
        key = o32 > key ? o32 : key;
    }
    if (lg == 0 && (!PK || (lr % 3 == 0 && lr < 15))) kred[v][wave] = key;
    __syncthreads();
    if ((int)threadIdx.x < nvec) {
        const int vv = threadIdx.x;
        unsigned long long m = kred[vv][0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) m = kred[vv][w] > m ? kred[vv][w] : m;
        StepState *st = p.st[0];
#pragma unroll
        for (int u = 1; u < NV; ++u) st = vv == u ? p.st[u] : st;
        if (m && st) atomicMax(&st->argmax_slot[(blockIdx.x % kArgSlots) * kSlotPitch], m);
    }
}

// ---------------------------------------------------------------------------
// k_head_wide_q6: the 2-to-16-vector head for Q6 rows.  Q6 rows (3 bytes per
// 4 codes) do not fall on 128-byte lines.  Every load instruction reads 4 rows
// × 192 contiguous bytes (a unit: 256 codes): lane L takes the 12 bytes (16
// codes) at 12·(L%16) of row L/16 of its row group.  The MFMA wants lane
// (lr, lg) to hold row lr's 16 codes of K slice lg instead, so each wave
// passes its units through a wave-private LDS tile (rows padded to 49 dwords
// against bank conflicts; a wave's LDS accesses stay in order, so no barrier)
// and reads A back as row lr, piece 4k + lg for MFMA step k of the unit.
// Loading 16 rows × 48 bytes per instruction, which is the A operand as
// loaded, streamed at half the rate.
// B column lr = vector lr (one tile per digit plane), or with PK (up to 5
// vectors) column 3v + pl in one tile, as in k_head_wide; a wave owns R blocks
// of 16 rows over all the columns, so no cross-wave sums.  Scores, argmax and
// digit planes (k_head_digits, Q6 plane order: step c/64, K slice (c%64)/16)
// as k_head_wide.
// ---------------------------------------------------------------------------
template <int NS, bool PK>
__global__ void __launch_bounds__(kThreads, 2) k_head_wide_q6(HeadWideParams p) {
    using SH = HeadWideShape<QT_Q6, NS>;
    constexpr int STEPS = SH::STEPS, R = SH::R;
    constexpr int UNITS = STEPS / 4;  // 192-byte units per row
    constexpr int TRW = 49;           // dwords per row of the transpose tile (48 + 1 pad)
    constexpr int NV = kHeadWideVec;
    static_assert(R >= 1, "at least one block of 16 rows per wave");
    static_assert(STEPS % 16 == 0, "whole 192-byte units in every column quarter");
    static_assert(SH::PLANE_BYTES % (16 * NV) == 0, "planes in 16-vector groups of 16 bytes");
    __shared__ __attribute__((aligned(16))) int8_t xdig[SH::PLANE_BYTES];
    __shared__ uint32_t tr[kWaves][R][16][TRW];
    __shared__ unsigned long long kred[NV][kWaves];
    asm volatile("" ::"s"(p.m.data), "s"(p.m.scale), "s"(p.planes), "s"(p.vscale), "s"(p.vbias), "s"(p.out),
                 "s"(p.rows), "s"(p.m.row_bytes), "s"(p.out_stride), "s"(p.nvec), "s"(p.out_vec4));

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int rows = p.rows;
    const int nvec = p.nvec;
    const int r0 = (blockIdx.x * kWaves + wave) * 16 * R;  // this wave's first row

    // 1. the live vectors' digit pieces, requested first
    constexpr int GROUPS = SH::PLANE_BYTES / (16 * NV);
    constexpr int MAXK = (GROUPS * NV + kThreads - 1) / kThreads;
    const int npieces = GROUPS * nvec;
    v4i piece[MAXK];
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
        const int id = (int)threadIdx.x + k * kThreads;
        if (id < npieces) {
            const int off = (id / nvec) * 256 + (id % nvec) * 16;
            piece[k] = *reinterpret_cast<const v4i *>(p.planes + off);
        }
    }
    asm volatile("" ::: "memory");  // the weight requests stay behind the pieces

    // 2. every weight byte of the wave's rows (past the end: the last row,
    // loaded and never scored), unit by unit in the order the MFMAs consume
    // them: row group g of block rb is rows 16rb + 4g + L/16.  With a head
    // image, lane L's piece L%16 of row L/16 sits in slot 4·(k/4) + L/16 +
    // 16·(k%4), k = L%16, of the unit (k_head_mfma's lane order)
    uint32_t raw[UNITS][R][4][3];
    const uint8_t *wrow[R][4];
    const bool img = p.m.head_img != nullptr;  // uniform
    constexpr int LINES = UNITS / 4;           // units per column quarter
    const int nblk = (rows + 15) / 16;
    const int slot = 4 * ((lane & 15) >> 2) + (lane >> 4) + 16 * (lane & 3);
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            wrow[rb][g] = p.m.data + (size_t)min(r0 + 16 * rb + 4 * g + (lane >> 4), rows - 1) * p.m.row_bytes +
                          12 * (lane & 15);
#pragma unroll
    for (int u = 0; u < UNITS; ++u)
#pragma unroll
        for (int rb = 0; rb < R; ++rb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint8_t *src =
                    img ? p.m.head_img + head_img_unit_q6(min(r0 / 16 + rb, nblk - 1), u / LINES, g, u % LINES, LINES) +
                              12 * slot
                        : wrow[rb][g] + 192 * u;
                const U3v q = __builtin_nontemporal_load(reinterpret_cast<const U3v *>(src));
                raw[u][rb][g][0] = q.x;
                raw[u][rb][g][1] = q.y;
                raw[u][rb][g][2] = q.z;
            }
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
        const int id = (int)threadIdx.x + k * kThreads;
        if (id < npieces) {
            const int off = (id / nvec) * 256 + (id % nvec) * 16;
            *reinterpret_cast<v4i *>(xdig + off) = piece[k];
        }
    }
    float rsc[R][4];  // row scales, first used after the MFMAs
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) rsc[rb][i] = p.m.scale[min(r0 + 16 * rb + 4 * lg + i, rows - 1)];
    __syncthreads();

    // 3. the MFMAs: A = row lr's codes of step st, K slice lg; B column lr =
    // vector lr's digits of the same 16 columns
    constexpr int NA = PK ? 1 : 3;  // accumulators (B tiles) per row block, as in k_head_wide
    v4i acc[R][NA];
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
#pragma unroll
        for (int pl = 0; pl < NA; ++pl) acc[rb][pl] = v4i{0, 0, 0, 0};
    const int pk_off = ((min(lr, 14) % 3) * 4 + lg) * 256 + (min(lr, 14) / 3) * 16;
#pragma unroll
    for (int u = 0; u < UNITS; ++u) {
        // this unit of the wave's rows into its LDS tile: row 4g + L/16,
        // piece L%16 (the previous unit's reads have all been consumed)
#pragma unroll
        for (int rb = 0; rb < R; ++rb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                uint32_t *d = &tr[wave][rb][4 * g + (lane >> 4)][3 * (lane & 15)];
#pragma unroll
                for (int w = 0; w < 3; ++w) d[w] = raw[u][rb][g][w];
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int st = 4 * u + k;
            v4i b[NA];
            if constexpr (PK) {
                b[0] = *reinterpret_cast<const v4i *>(xdig + st * 3 * 1024 + pk_off);
            } else {
#pragma unroll
                for (int pl = 0; pl < 3; ++pl)
                    b[pl] = *reinterpret_cast<const v4i *>(xdig + (st * 3 + pl) * 1024 + 16 * lane);
            }
#pragma unroll
            for (int rb = 0; rb < R; ++rb) {
                // row lr, piece 4k + lg: columns 64·st + 16·lg .. +15
                const uint32_t *a3 = &tr[wave][rb][lr][12 * k + 3 * lg];
                RawCodes<QT_Q6> rc;
#pragma unroll
                for (int w = 0; w < 3; ++w) rc.d[w] = a3[w];
                const v4i a = unpack_codes16<QT_Q6>(rc);
#pragma unroll
                for (int pl = 0; pl < NA; ++pl)
                    acc[rb][pl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[pl], acc[rb][pl], 0, 0, 0);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // 4. lane (lr, lg) holds C[4lg + i][lr]: rows r0 + 16rb + 4lg + i of
    // vector lr (PK: vector lr/3, plane lr%3, gathered as in k_head_wide).
    // Scores as k_head_mfma forms them.
    int pls[R][3][4];
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (PK) {
                pls[rb][0][i] = acc[rb][0][i];
                pls[rb][1][i] = __shfl(acc[rb][0][i], min(lane + 1, 63), 64);
                pls[rb][2][i] = __shfl(acc[rb][0][i], min(lane + 2, 63), 64);
            } else {
#pragma unroll
                for (int pl = 0; pl < 3; ++pl) pls[rb][pl][i] = acc[rb][pl < NA ? pl : 0][i];
            }
        }
    const int v = PK ? lr / 3 : lr;
    const bool live = v < nvec && (!PK || (lr % 3 == 0 && lr < 15));
    int b0 = 0, b1 = 0, b2 = 0;
    float my_sx = 1.0f;
    if (live) {
        b0 = p.vbias[v * 3];
        b1 = p.vbias[v * 3 + 1];
        b2 = p.vbias[v * 3 + 2];
        my_sx = p.vscale[v];
    }
    unsigned long long key = 0ull;
#pragma unroll
    for (int rb = 0; rb < R; ++rb) {
        const int rr = r0 + 16 * rb + 4 * lg;
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // |Σ u·d| < 2^24 per plane (cols ≤ 2048): exact converts
            const float f0 = (float)(pls[rb][0][i] - b0);
            const float f1 = (float)(pls[rb][1][i] - b1);
            const float f2 = (float)(pls[rb][2][i] - b2);
            sc[i] = fmaf(f2, 1.0f / 16384.0f, fmaf(f1, 1.0f / 128.0f, f0)) * my_sx * rsc[rb][i];
            if (live && rr + i < rows) {
                const unsigned long long k = argmax_key(sc[i], rr + i);
                key = k > key ? k : key;
            }
        }
        if (p.out && live) {
            float *o = p.out + (size_t)v * p.out_stride + rr;
            if (p.out_vec4) {
                if (rr < rows) *reinterpret_cast<float4 *>(o) = make_float4(sc[0], sc[1], sc[2], sc[3]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (rr + i < rows) o[i] = sc[i];
            }
        }
    }
    {
        const unsigned long long o16 = shfl_xor_u64(key, 16);
        key = o16 > key ? o16 : key;
        const unsigned long long o32 = shfl_xor_u64(key, 32);
        key = o32 > key ? o32 : key;
    }
    if (lg == 0 && (!PK || (lr % 3 == 0 && lr < 15))) kred[v][wave] = key;
    __syncthreads();
    if ((int)threadIdx.x < nvec) {
        const int vv = threadIdx.x;
        unsigned long long m = kred[vv][0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) m = kred[vv][w] > m ? kred[vv][w] : m;
        StepState *st = p.st[0];
#pragma unroll
        for (int u = 1; u < NV; ++u) st = vv == u ? p.st[u] : st;
        if (m && st) atomicMax(&st->argmax_slot[(blockIdx.x % kArgSlots) * kSlotPitch], m);
    }
}

}  // namespace pocr
