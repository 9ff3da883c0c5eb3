// gemm.hpp — batched (M > 1) decoder kernels on the matrix cores: prompt
// prefill and the batched GEMV.
//
// Prefill runs the same step as the decode kernels (forwardEmbeddingForSampling,
// internal/model/model.go:3475-3643) for N prompt tokens at once, with the
// per-token semantics of the token-by-token loop (model.go:1514-1536): token n
// sees cache rows [0, clen0+n], the Q4/Q6 residual behaviour depends on its own
// cache length, and its K/V rows land at clen0+n.
//
// Quantized products use int8 MFMA (v_mfma_i32_16x16x64_i8).  Activations are
// written per token as three int8 digit planes with one power-of-two scale S_n:
//   x = S_n·(d0 + d1/2^7 + d2/2^14) + e,  |e| ≤ S_n/2^15,
// so a whole row of K products accumulates exactly in int32 (|Σ| < 2^26) and
// the f32 result differs from the reference's f32 accumulation by rounding
// only.  Weight codes enter the MFMA as stored: Q8 bytes, Q4 nibbles u ∈ [0,15]
// (code = u − 8), Q6 fields u ∈ [0,63] (code = u − 32); the offset is removed
// exactly as IBIAS·Σ_k d_k per token and plane.
#pragma once

#include "kernels.hpp"

namespace pocr {

constexpr int kGemmK = 64;       // K per MFMA step
constexpr int kGemmWaveRows = 64;  // rows per wave (4 blocks of 16)
constexpr int kGemmRows = kGemmWaveRows * kWaves;  // rows per workgroup

// ---------------------------------------------------------------------------
// Activation digitizer: one workgroup per token row.  y = x (or x·w with the
// RMSNorm factor fastRsqrt(Σx²/K + eps) carried in the row scale, ops.go:
// 1015-1037), S = 2^e ≥ max|y|/127, planes [3][npad][K] int8 in the K order
// above, row scale S·factor, bias sums Σd per plane.
// ---------------------------------------------------------------------------
struct DigitizeParams {
    const float *x;        // [n][x_stride]
    int x_stride;
    const float *norm_w;   // null → no RMSNorm
    float eps;
    int K;                 // multiple of 16, ≤ 8192
    int8_t *xd;            // planes [3][npad][K], or the tile layout below
    size_t plane_stride;   // npad·K
    float *xs;             // [n] row scale
    int *xb;               // [n][4] Σd per plane (4th unused); VNNI: [n][4] with Σq first
    int tiled;             // 1: the prefill GEMM's tile layout (K a multiple of 128)
    int vnni;              // 1: one plane of VNNI activation bytes (k_digitize_vnni, tile layout only)
};

// Byte offset of the 16-column group at column c0 (a multiple of 16) of token
// n, digit plane pl.  Plane layout: [pl][npad][K].  Tile layout (the operand
// order of k_gemm_lds, so each of its loads reads 1 KB of consecutive bytes),
// with NPL planes (3, or 1 in the VNNI mode):
// [token tile n/32][stage c0/128][chunk j][lane][16 B], where in stage u the
// MFMA step s, plane pl and token block tb form chunk j = (NPL·s + pl)·2 + tb
// and lane lr + 16·lg holds token 16tb + lr, columns 128u + 32lg + 16s .. +15.
__device__ __forceinline__ size_t digit_off(const DigitizeParams &p, int pl, int n, int c0) {
    if (!p.tiled) return pl * p.plane_stride + (size_t)n * p.K + c0;
    const int npl = p.vnni ? 1 : 3;
    const int g = c0 >> 4, u = g >> 3, gi = g & 7;
    const int tl = n & 31, j = ((gi & 1) * npl + pl) * 2 + (tl >> 4), lane = (tl & 15) + 16 * (gi >> 1);
    return ((size_t)((n >> 5) * (p.K >> 7) + u) * 4 * npl + j) * 1024 + lane * 16;
}

template <int QT, int G>
static __global__ void __launch_bounds__(kThreads) k_digitize(DigitizeParams p) {
    // G 16-column groups per thread: K ≤ 4096·G
    __shared__ float red[kWaves];
    __shared__ int redi[3][kWaves];
    const int n = blockIdx.x;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    float y[G][16];
    bool valid[G];
    int c0[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        c0[g] = 16 * (t + g * kThreads);  // this thread's 16-column groups
        valid[g] = c0[g] < p.K;
        const int cl = valid[g] ? c0[g] : p.K - 16;  // clamped, never written
        const float *xr = p.x + (size_t)n * p.x_stride + cl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = reinterpret_cast<const float4 *>(xr)[i];
            y[g][4 * i] = v.x;
            y[g][4 * i + 1] = v.y;
            y[g][4 * i + 2] = v.z;
            y[g][4 * i + 3] = v.w;
        }
    }
    float factor = 1.0f;
    if (p.norm_w) {
        float ss = 0.0f;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float sg = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) sg = fmaf(y[g][i], y[g][i], sg);
            ss += valid[g] ? sg : 0.0f;
        }
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        float tot = red[0];
#pragma unroll
        for (int k = 1; k < kWaves; ++k) tot += red[k];
        factor = fast_rsqrt_ref(tot / (float)p.K + p.eps);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int cl = valid[g] ? c0[g] : p.K - 16;
            float w[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = reinterpret_cast<const float4 *>(p.norm_w + cl)[i];
                w[4 * i] = v.x;
                w[4 * i + 1] = v.y;
                w[4 * i + 2] = v.z;
                w[4 * i + 3] = v.w;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) y[g][i] = y[g][i] * w[i];  // a lone product: nothing to contract
        }
        __syncthreads();  // red is reused below
    }
    float m = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < 16; ++i) m = valid[g] ? fmaxf(m, fabsf(y[g][i])) : m;
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int k = 1; k < kWaves; ++k) m = fmaxf(m, red[k]);
    int ex = 0;
    (void)frexpf(m * (1.0f / 127.0f), &ex);  // m/127 < 2^ex; m = 0 → ex = 0
    const float S = m > 0.0f ? ldexpf(1.0f, ex) : 1.0f;
    int sd[3] = {0, 0, 0};
#pragma unroll
    for (int g = 0; g < G; ++g) {
        int d[3][16];  // digit of K position pos (the group's shared order)
        int sg[3] = {0, 0, 0};
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            const float tt = ldexpf(y[g][c], -ex);  // exact (no overflow of 2^-ex for tiny rows)
            const float a = rintf(tt);
            const float t1 = (tt - a) * 128.0f;
            const float b = rintf(t1);
            const int d2 = (int)rintf((t1 - b) * 128.0f);
            const int pos = digit_pos16<QT>(c);
            d[0][pos] = (int)a;
            d[1][pos] = (int)b;
            d[2][pos] = d2;
            sg[0] += (int)a;
            sg[1] += (int)b;
            sg[2] += d2;
        }
        if (valid[g]) {
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) {
                *reinterpret_cast<int4 *>(p.xd + digit_off(p, pl, n, c0[g])) =
                    make_int4(pack4(d[pl][0], d[pl][1], d[pl][2], d[pl][3]),
                              pack4(d[pl][4], d[pl][5], d[pl][6], d[pl][7]),
                              pack4(d[pl][8], d[pl][9], d[pl][10], d[pl][11]),
                              pack4(d[pl][12], d[pl][13], d[pl][14], d[pl][15]));
                sd[pl] += sg[pl];
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) {
        const int s = (int)wave_sum((float)sd[pl]);  // |Σ| ≤ 8192·127: exact in f32
        if (lane == 0) redi[pl][wave] = s;
    }
    __syncthreads();
    if (t < 3) {
        int s = 0;
#pragma unroll
        for (int k = 0; k < kWaves; ++k) s += redi[t][k];
        p.xb[n * 4 + t] = s;
    }
    if (t == 0) p.xs[n] = S * factor;
}

// The same digit planes with one wave per token (four tokens per workgroup)
// for K ≤ 1024·J: lane l of the token's wave takes the 16-column groups
// 64j + l, j < ⌈K/1024⌉, which k_digitize gives thread 64j + l, and reduces
// each j's partials with the same wave sum before adding them in j order, so
// Σx², the maximum, the digits and the plane sums are bit-identical to
// k_digitize's.  No barrier: at K = 1024, k_digitize keeps three of its four
// waves idle through three workgroup barriers per token.
template <int QT, int J>
static __global__ void __launch_bounds__(kThreads) k_digitize_w(DigitizeParams p, int ntok) {
    static_assert(J >= 1 && J <= 4, "1024-column slices, K ≤ 1024·J ≤ 4096");
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (n >= ntok) return;  // wave-uniform; no barrier below
    float y[J][16];
    bool valid[J];
    int c0[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        c0[j] = 16 * (64 * j + lane);
        valid[j] = c0[j] < p.K;
        const int cl = valid[j] ? c0[j] : p.K - 16;  // clamped, never written
        const float *xr = p.x + (size_t)n * p.x_stride + cl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = reinterpret_cast<const float4 *>(xr)[i];
            y[j][4 * i] = v.x;
            y[j][4 * i + 1] = v.y;
            y[j][4 * i + 2] = v.z;
            y[j][4 * i + 3] = v.w;
        }
    }
    float factor = 1.0f;
    if (p.norm_w) {
        // k_digitize adds its idle waves' zero partials after these: +0
        // changes nothing
        float tot = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            float sg = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) sg = fmaf(y[j][i], y[j][i], sg);
            const float pj = wave_sum(valid[j] ? sg : 0.0f);
            tot = j == 0 ? pj : tot + pj;
        }
        factor = fast_rsqrt_ref(tot / (float)p.K + p.eps);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int cl = valid[j] ? c0[j] : p.K - 16;
            float w[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = reinterpret_cast<const float4 *>(p.norm_w + cl)[i];
                w[4 * i] = v.x;
                w[4 * i + 1] = v.y;
                w[4 * i + 2] = v.z;
                w[4 * i + 3] = v.w;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) y[j][i] = y[j][i] * w[i];  // a lone product: nothing to contract
        }
    }
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) m = valid[j] ? fmaxf(m, fabsf(y[j][i])) : m;
    m = wave_max(m);
    int ex = 0;
    (void)frexpf(m * (1.0f / 127.0f), &ex);  // m/127 < 2^ex; m = 0 → ex = 0
    const float S = m > 0.0f ? ldexpf(1.0f, ex) : 1.0f;
    int sd[3] = {0, 0, 0};
#pragma unroll
    for (int j = 0; j < J; ++j) {
        int d[3][16];
        int sg[3] = {0, 0, 0};
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            const float tt = ldexpf(y[j][c], -ex);  // exact (no overflow of 2^-ex for tiny rows)
            const float a = rintf(tt);
            const float t1 = (tt - a) * 128.0f;
            const float b = rintf(t1);
            const int d2 = (int)rintf((t1 - b) * 128.0f);
            const int pos = digit_pos16<QT>(c);
            d[0][pos] = (int)a;
            d[1][pos] = (int)b;
            d[2][pos] = d2;
            sg[0] += (int)a;
            sg[1] += (int)b;
            sg[2] += d2;
        }
        if (valid[j]) {
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) {
                *reinterpret_cast<int4 *>(p.xd + digit_off(p, pl, n, c0[j])) =
                    make_int4(pack4(d[pl][0], d[pl][1], d[pl][2], d[pl][3]),
                              pack4(d[pl][4], d[pl][5], d[pl][6], d[pl][7]),
                              pack4(d[pl][8], d[pl][9], d[pl][10], d[pl][11]),
                              pack4(d[pl][12], d[pl][13], d[pl][14], d[pl][15]));
                sd[pl] += sg[pl];
            }
        }
    }
    int tot[3];
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) tot[pl] = (int)wave_sum((float)sd[pl]);  // |Σ| ≤ 4096·127: exact in f32
    if (lane < 3) p.xb[n * 4 + lane] = lane == 0 ? tot[0] : (lane == 1 ? tot[1] : tot[2]);
    if (lane == 0) p.xs[n] = S * factor;
}

// The VNNI mode's activation bytes (quantizeXForVNNI, internal/tensor/
// quant.go:2087-2115; dot_amd64.go:228-252), one wave per token, as the VNNI
// GEMV's prologue forms them for one vector, so each token's bytes are the
// token step's:
// * with norm_w, RMSNorm first: Σx² in sumSquaresScalar's order (ops.go:
//   1039-1058; K a multiple of 8: eight running sums over the columns ≡ j mod
//   8, lanes 0-7, then ((s0+s1)+(s2+s3))+((s4+s5)+(s6+s7))), factor =
//   fastRsqrt(Σ/K + eps), y = (x·factor)·w;
// * m = max|y|, sx = m/127 (1 for m = 0), inv = 1/sx, q = clamp(RNE(y·inv) +
//   128, 0, 255), every q = 128 for m = 0.
// The tile layout's one plane holds d = q − 128 (the GEMM's B operand) in the
// weight codes' order; xs = sx, xb[0] = Σq.
template <int QT, int J>
static __global__ void __launch_bounds__(kThreads) k_digitize_vnni(DigitizeParams p, int ntok) {
#pragma clang fp contract(off)
    static_assert(J >= 1 && J <= 4, "1024-column slices, K ≤ 1024·J ≤ 4096");
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (n >= ntok) return;  // wave-uniform; no barrier below
    const float *xr = p.x + (size_t)n * p.x_stride;
    float y[J][16];
    bool valid[J];
    int c0[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        c0[j] = 16 * (64 * j + lane);
        valid[j] = c0[j] < p.K;
        const int cl = valid[j] ? c0[j] : p.K - 16;  // clamped, never written
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = reinterpret_cast<const float4 *>(xr + cl)[i];
            y[j][4 * i] = v.x;
            y[j][4 * i + 1] = v.y;
            y[j][4 * i + 2] = v.z;
            y[j][4 * i + 3] = v.w;
        }
    }
    if (p.norm_w) {
        float s = 0.0f;
        if (lane < 8) {  // running sum `lane`: columns lane, lane + 8, … in order, 16 reads in flight
            int i = lane;
            for (; i + 8 * 15 < p.K; i += 8 * 16) {
                float v[16];
#pragma unroll
                for (int k = 0; k < 16; ++k) v[k] = xr[i + 8 * k];
#pragma unroll
                for (int k = 0; k < 16; ++k) s = s + v[k] * v[k];
            }
            for (; i < p.K; i += 8) s = s + xr[i] * xr[i];
        }
        float r[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) r[k] = __shfl(s, k, 64);
        const float ss = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        const float factor = fast_rsqrt_ref(ss / (float)p.K + p.eps);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int cl = valid[j] ? c0[j] : p.K - 16;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 w = reinterpret_cast<const float4 *>(p.norm_w + cl)[i];
                y[j][4 * i] = y[j][4 * i] * factor * w.x;
                y[j][4 * i + 1] = y[j][4 * i + 1] * factor * w.y;
                y[j][4 * i + 2] = y[j][4 * i + 2] * factor * w.z;
                y[j][4 * i + 3] = y[j][4 * i + 3] * factor * w.w;
            }
        }
    }
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) m = valid[j] ? fmaxf(m, fabsf(y[j][i])) : m;
    m = wave_max(m);
    const float sx = m == 0.0f ? 1.0f : m / 127.0f;
    const float inv = 1.0f / sx;
    int sq = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        int d[16];
        int sg = 0;
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            int q = 128;
            if (m != 0.0f) {
                float v = rintf(y[j][c] * inv) + 128.0f;
                v = fminf(fmaxf(v, 0.0f), 255.0f);
                q = (int)v;
            }
            d[digit_pos16<QT>(c)] = q - 128;
            sg += q;
        }
        if (valid[j]) {
            *reinterpret_cast<int4 *>(p.xd + digit_off(p, 0, n, c0[j])) =
                make_int4(pack4(d[0], d[1], d[2], d[3]), pack4(d[4], d[5], d[6], d[7]),
                          pack4(d[8], d[9], d[10], d[11]), pack4(d[12], d[13], d[14], d[15]));
            sq += sg;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off, 64);
    if (lane == 0) {
        p.xb[n * 4] = sq;
        p.xs[n] = sx;
    }
}

// Σ of the stored codes of each row (Q4 nibbles, Q6 fields; cols a multiple of
// 16), one wave per row: the VNNI mode's row sum is Σu − IBIAS·cols.
template <int QT>
static __global__ void __launch_bounds__(kThreads) k_row_usum(const uint8_t *data, int row_bytes, int rows, int cols,
                                                              int *out) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (r >= rows) return;
    const uint8_t *row = data + (size_t)r * row_bytes;
    int u = 0;
    if constexpr (QT == QT_Q4) {
        for (int b = 4 * lane; b < cols / 2; b += 4 * 64) {
            const uint32_t w = *reinterpret_cast<const uint32_t *>(row + b);
            u += (int)((w & 15u) + ((w >> 4) & 15u) + ((w >> 8) & 15u) + ((w >> 12) & 15u) +
                                                ((w >> 16) & 15u) + ((w >> 20) & 15u) + ((w >> 24) & 15u) + (w >> 28));
        }
    } else {
        for (int c = lane; c < cols / 16; c += 64) {
            const uint32_t *q = reinterpret_cast<const uint32_t *>(row + 12 * (size_t)c);
            const uint32_t w0 = q[0], w1 = q[1], w2 = q[2];
            const uint32_t g[4] = {w0 & 0xFFFFFFu, (w0 >> 24) | ((w1 & 0xFFFFu) << 8), (w1 >> 16) | ((w2 & 0xFFu) << 16),
                                   w2 >> 8};
#pragma unroll
            for (int k = 0; k < 4; ++k)
                u += (int)((g[k] & 63u) + ((g[k] >> 6) & 63u) + ((g[k] >> 12) & 63u) + (g[k] >> 18));
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) u += __shfl_xor(u, off, 64);
    if (lane == 0) out[r] = u;
}

// ---------------------------------------------------------------------------
// MFMA GEMM: Y[n][r] = epilogue(scale[r]·xs[n]·(D0 + D1/2^7 + D2/2^14)),
// D_p = Σ_k u[r][k]·d_p[n][k] − IBIAS·Σ_k d_p[n][k].  Workgroup: 256 rows ×
// 16·TN tokens; wave w owns rows r0+64w.. (4 blocks of 16) for all its tokens.
// Rows come from up to three matrices (segments, as the fused QKV GEMV) or,
// with NMAT = 2, from two matrices side by side (gate and up).
// ---------------------------------------------------------------------------
enum : int { G_PLAIN = 0, G_SWIGLU = 1, G_OPROJ = 2, G_DOWN = 3, G_BIAS = 4, G_BIAS_GELU = 5 };

struct GemmParams {
    DevMat m[3];
    int seg_end[3];
    int rows;              // multiple of 64
    int K;                 // multiple of 64
    const int8_t *xd;      // planes [3][npad][K]
    size_t plane_stride;
    const float *xs;       // [n]
    const int *xb;         // [n][4]
    int ntok;
    float *out;            // PLAIN / SWIGLU: [n][out_stride]
    int out_stride;
    float *h;              // OPROJ / DOWN residual rows [n][rows]
    float *vbuf;           // [n][rows]
    int quirk;             // OPROJ: Q4/Q6 residual behaviour
    int clen0;             // cache rows before token 0 (one sequence's rows)
    StepState *const *rst; // [n] step state of row n (batched decode: rows are sequences), or null
    int last;              // DOWN: last layer → vbuf = h + y (h untouched)
    const float *bias;     // BIAS / BIAS_GELU: [rows]
    int vnni;              // one plane of VNNI bytes (xs = scaleX, xb[0] = Σq): the VNNI finalize
};

// 16 weight codes of row `row` at columns k..k+15 (k multiple of 16) as the
// MFMA A operand, in the shared K order
template <int QT>
__device__ __forceinline__ v4i load_codes16(const uint8_t *rowp, int k) {
    v4i a;
    if constexpr (QT == QT_Q8) {
        const uint4 v = *reinterpret_cast<const uint4 *>(rowp + k);
        a = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
    } else if constexpr (QT == QT_Q4) {
        const uint2 v = *reinterpret_cast<const uint2 *>(rowp + k / 2);
        a = v4i{(int)(v.x & 0x0F0F0F0Fu), (int)(v.y & 0x0F0F0F0Fu), (int)((v.x >> 4) & 0x0F0F0F0Fu),
                (int)((v.y >> 4) & 0x0F0F0F0Fu)};
    } else {
        const uint8_t *q = rowp + (k / 16) * 12;
        const uint32_t d0 = *reinterpret_cast<const uint32_t *>(q);
        const uint32_t d1 = *reinterpret_cast<const uint32_t *>(q + 4);
        const uint32_t d2 = *reinterpret_cast<const uint32_t *>(q + 8);
        a = v4i{spread6(d0), spread6(__builtin_amdgcn_alignbit(d1, d0, 24)),
                spread6(__builtin_amdgcn_alignbit(d2, d1, 16)), spread6(d2 >> 8)};
    }
    return a;
}

__device__ __forceinline__ bool prefill_in_place(const GemmParams &p, int n) {
    // model.go:3895-3902, 4051-4057: Q4/Q6 take the OutOnly variant at cache
    // length 0 and ≥ 6; row n is token clen0 + n of one sequence, or the
    // current token of sequence n in a batched decode step
    const int clen = p.rst ? p.rst[n]->clen : p.clen0 + n;
    return !(p.quirk && (clen == 0 || clen >= 6));
}

// Store of rows rr..rr+3 for token n, given their f32 values y (one set per
// matrix; SwiGLU pairs gate and up).
template <int NMAT>
__device__ __forceinline__ void gemm_store_y(const GemmParams &p, int epi, int n, int rr, const float (&y)[NMAT][4]) {
    if (epi == G_PLAIN) {
        *reinterpret_cast<float4 *>(p.out + (size_t)n * p.out_stride + rr) = make_float4(y[0][0], y[0][1], y[0][2], y[0][3]);
    } else if (epi == G_BIAS || epi == G_BIAS_GELU) {
        // matVecQ8BiasSerial (quant.go:1469-1472): y·scale + bias, then
        // GELUTanhInPlace over the row (ops.go:1166-1177) for the first
        // projector matrix
        const float4 bv = *reinterpret_cast<const float4 *>(p.bias + rr);
        float o[4];
        {
#pragma clang fp contract(off)
            o[0] = y[0][0] + bv.x;
            o[1] = y[0][1] + bv.y;
            o[2] = y[0][2] + bv.z;
            o[3] = y[0][3] + bv.w;
        }
        if (epi == G_BIAS_GELU) {
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = gelu_tanh_ref(o[i]);
        }
        *reinterpret_cast<float4 *>(p.out + (size_t)n * p.out_stride + rr) = make_float4(o[0], o[1], o[2], o[3]);
    } else if (epi == G_SWIGLU) {
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma clang fp contract(off)
            o[i] = silu_ref(y[0][i]) * y[NMAT - 1][i];
        }
        *reinterpret_cast<float4 *>(p.out + (size_t)n * p.out_stride + rr) = make_float4(o[0], o[1], o[2], o[3]);
    } else {
        float4 *hp = reinterpret_cast<float4 *>(p.h + (size_t)n * p.rows + rr);
        const float4 hv = *hp;
        float4 v;
        {
#pragma clang fp contract(off)
            v = make_float4(hv.x + y[0][0], hv.y + y[0][1], hv.z + y[0][2], hv.w + y[0][3]);
        }
        float4 *vp = reinterpret_cast<float4 *>(p.vbuf + (size_t)n * p.rows + rr);
        if (epi == G_OPROJ) {
            *vp = v;
            if (prefill_in_place(p, n)) *hp = v;
        } else if (p.last) {
            *vp = v;
        } else {
            *hp = v;
        }
    }
}

// Epilogue of rows rr..rr+3 for token n, given the int32 accumulators of the
// three digit planes: y = scale[r]·xs[n]·(D0 + D1/2^7 + D2/2^14).
template <int QT, int NMAT>
__device__ __forceinline__ void gemm_store(const GemmParams &p, int epi, int n, int rr, const float *const (&scl)[2],
                                           const v4i (&a)[NMAT][3]) {
    constexpr int IB = DigitTraits<QT>::IBIAS;
    const float sx = p.xs[n];
    const int4 bs = *reinterpret_cast<const int4 *>(p.xb + 4 * n);
    float y[NMAT][4];
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi) {
        const float *sc = scl[mi];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float f0 = (float)(a[mi][0][i] - IB * bs.x);
            const float f1 = (float)(a[mi][1][i] - IB * bs.y);
            const float f2 = (float)(a[mi][2][i] - IB * bs.z);
            y[mi][i] = fmaf(f2, 1.0f / 16384.0f, fmaf(f1, 1.0f / 128.0f, f0)) * sx * sc[i];
        }
    }
    gemm_store_y<NMAT>(p, epi, n, rr, y);
}

// The VNNI mode's epilogue of rows rr..rr+3 for token n from the int32 Σu·d of
// each row (u the stored code, d = q − 128), as the VNNI GEMV finishes a row
// (finalizeDotQ8VNNI, dot_vnni_amd64.s:1043-1080; rows in whole 16-row blocks):
//   dot = Σu·d + 128·Σu − IBIAS·Σq = Σ code·q,  rowSum = Σu − IBIAS·K,
//   y = ((f32(dot) − f32(rowSum)·128)·scaleX)·scale[r].
template <int QT, int NMAT>
__device__ __forceinline__ void gemm_store_vnni(const GemmParams &p, int epi, int n, int rr,
                                                const float *const (&scl)[2], const int *const (&us)[2],
                                                const v4i (&a)[NMAT]) {
#pragma clang fp contract(off)
    constexpr int IB = DigitTraits<QT>::IBIAS;
    const float sx = p.xs[n];
    const int sq = p.xb[4 * n];
    float y[NMAT][4];
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int u = us[mi][i];
            const int dot = a[mi][i] + 128 * u - IB * sq;
            const int rowsum = u - IB * p.K;
            const float v = (float)dot - (float)rowsum * 128.0f;
            y[mi][i] = v * sx * scl[mi][i];
        }
    }
    gemm_store_y<NMAT>(p, epi, n, rr, y);
}

// the wave's rows lie in one segment (segment ends are multiples of 16 rows
// for the small kernel, of 64 for the prefill one)
struct GemmSeg {
    const uint8_t *base[2];
    const uint8_t *tiled[2];
    const float *scale[2];
    const int *usum[2];
    int start;
};
template <int NMAT>
__device__ __forceinline__ GemmSeg gemm_seg(const GemmParams &p, int r0) {
    GemmSeg g;
    g.base[1] = nullptr;
    g.tiled[1] = nullptr;
    g.scale[1] = nullptr;
    g.usum[1] = nullptr;
    g.start = 0;
    const int i = NMAT == 2 ? 0 : (r0 >= p.seg_end[1] ? 2 : (r0 >= p.seg_end[0] ? 1 : 0));
    g.base[0] = p.m[i].data;
    g.tiled[0] = p.m[i].tiled;
    g.scale[0] = p.m[i].scale;
    g.usum[0] = p.m[i].usum;
    if (NMAT == 2) {
        g.base[1] = p.m[1].data;
        g.tiled[1] = p.m[1].tiled;
        g.scale[1] = p.m[1].scale;
        g.usum[1] = p.m[1].usum;
    } else if (i > 0) {
        g.start = p.seg_end[i - 1];
    }
    return g;
}

template <int QT, int NMAT, int TN>
static __global__ void __launch_bounds__(kThreads) k_gemm(GemmParams p, int epi) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r0 = blockIdx.x * kGemmRows + wave * kGemmWaveRows;
    if (r0 >= p.rows) return;  // rows are a multiple of 64: whole waves only
    const int n0 = blockIdx.y * 16 * TN;
    const int lr = lane & 15, lg = lane >> 4;

    // the wave's 64 rows lie in one segment (segment ends are multiples of 64)
    const uint8_t *base0;
    const uint8_t *base1 = nullptr;
    const float *scale0;
    const float *scale1 = nullptr;
    int start = 0;
    if (NMAT == 2) {
        base0 = p.m[0].data;
        base1 = p.m[1].data;
        scale0 = p.m[0].scale;
        scale1 = p.m[1].scale;
    } else if (r0 >= p.seg_end[1]) {
        base0 = p.m[2].data;
        scale0 = p.m[2].scale;
        start = p.seg_end[1];
    } else if (r0 >= p.seg_end[0]) {
        base0 = p.m[1].data;
        scale0 = p.m[1].scale;
        start = p.seg_end[0];
    } else {
        base0 = p.m[0].data;
        scale0 = p.m[0].scale;
    }
    const int row_bytes = p.m[0].row_bytes;
    const uint8_t *arow[NMAT][4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        const size_t off = (size_t)(r0 + 16 * rb + lr - start) * row_bytes;
        arow[0][rb] = base0 + off;
        if (NMAT == 2) arow[NMAT - 1][rb] = base1 + off;
    }
    const int8_t *brow[TN];
#pragma unroll
    for (int tb = 0; tb < TN; ++tb) brow[tb] = p.xd + (size_t)(n0 + 16 * tb + lr) * p.K + 16 * lg;

    v4i acc[NMAT][4][TN][3];
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int tb = 0; tb < TN; ++tb)
#pragma unroll
                for (int pl = 0; pl < 3; ++pl) acc[mi][rb][tb][pl] = v4i{0, 0, 0, 0};

    v4i a[NMAT][4], b[TN][3];
    auto load = [&](int k0, v4i (&aa)[NMAT][4], v4i (&bb)[TN][3]) {
        const int k = k0 + 16 * lg;
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) aa[mi][rb] = load_codes16<QT>(arow[mi][rb], k);
#pragma unroll
        for (int tb = 0; tb < TN; ++tb)
#pragma unroll
            for (int pl = 0; pl < 3; ++pl)
                bb[tb][pl] = *reinterpret_cast<const v4i *>(brow[tb] + pl * p.plane_stride + k0);
    };
    load(0, a, b);
    for (int k0 = 0; k0 < p.K; k0 += kGemmK) {
        v4i an[NMAT][4], bn[TN][3];
        const bool more = k0 + kGemmK < p.K;  // uniform
        if (more) load(k0 + kGemmK, an, bn);
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int tb = 0; tb < TN; ++tb)
#pragma unroll
                    for (int pl = 0; pl < 3; ++pl)
                        acc[mi][rb][tb][pl] =
                            __builtin_amdgcn_mfma_i32_16x16x64_i8(a[mi][rb], b[tb][pl], acc[mi][rb][tb][pl], 0, 0, 0);
        if (more) {
#pragma unroll
            for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) a[mi][rb] = an[mi][rb];
#pragma unroll
            for (int tb = 0; tb < TN; ++tb)
#pragma unroll
                for (int pl = 0; pl < 3; ++pl) b[tb][pl] = bn[tb][pl];
        }
    }

    // epilogue: lane holds token n0+16tb+lr, rows r0+16rb+4lg+i (i < 4)
#pragma unroll
    for (int tb = 0; tb < TN; ++tb) {
        const int n = n0 + 16 * tb + lr;
        if (n >= p.ntok) continue;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            const int rr = r0 + 16 * rb + 4 * lg;  // 4 consecutive rows
            const float *const scl[2] = {scale0 + (rr - start), NMAT == 2 ? scale1 + (rr - start) : nullptr};
            v4i a3[NMAT][3];
#pragma unroll
            for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
                for (int pl = 0; pl < 3; ++pl) a3[mi][pl] = acc[mi][rb][tb][pl];
            gemm_store<QT, NMAT>(p, epi, n, rr, scl, a3);
        }
    }
}

// raw code bytes of 16 columns (Q8 16 B, Q4 8 B, Q6 12 B)
template <int QT>
struct RawCodes {
    uint32_t d[QT == QT_Q8 ? 4 : (QT == QT_Q4 ? 2 : 3)];
};

// the MFMA A operand of 16 raw columns, unpacked as load_codes16 does
template <int QT>
__device__ __forceinline__ v4i unpack_codes16(const RawCodes<QT> &r) {
    if constexpr (QT == QT_Q8) {
        return v4i{(int)r.d[0], (int)r.d[1], (int)r.d[2], (int)r.d[3]};
    } else if constexpr (QT == QT_Q4) {
        return v4i{(int)(r.d[0] & 0x0F0F0F0Fu), (int)(r.d[1] & 0x0F0F0F0Fu), (int)((r.d[0] >> 4) & 0x0F0F0F0Fu),
                   (int)((r.d[1] >> 4) & 0x0F0F0F0Fu)};
    } else {
        return v4i{spread6(r.d[0]), spread6(__builtin_amdgcn_alignbit(r.d[1], r.d[0], 24)),
                   spread6(__builtin_amdgcn_alignbit(r.d[2], r.d[1], 16)), spread6(r.d[2] >> 8)};
    }
}

// XCD-aware tile order: workgroups are dispatched round-robin over the 8 XCDs
// (XCD = linear id mod 8), so XCD j is given the j-th contiguous run of tiles
// in token-major order: its L2 keeps a few token tiles' digit planes and the
// weight rows they meet, instead of every XCD streaming every tile.
__device__ __forceinline__ int2 xcd_tile() {
    const int gx = gridDim.x;
    const int L = blockIdx.x + gx * blockIdx.y;
    const int W = gx * gridDim.y, q = W >> 3, r = W & 7, j = L & 7;
    const int logical = j * q + min(j, r) + (L >> 3);
    return make_int2(logical % gx, logical / gx);
}

// ---------------------------------------------------------------------------
// Prefill GEMM with both operands streamed into LDS by direct loads
// (global_load_lds: HBM → LDS with no staging registers) through a ring of
// NST stages of 128 columns.  Workgroup: 4 waves along the rows × 32 tokens;
// a wave owns RB blocks of 16 rows of each of its NMAT matrices (gate and up
// side by side) × 32 tokens: NMAT·RB·2·3 MFMAs (row blocks × 2 token blocks ×
// 3 digit planes) per 64 columns.
//
// K order of the MFMA operands: in stage u, MFMA step s, lane group lg takes
// columns 128u + 32lg + 16s .. +15 (A and B alike; inside a 16-column group
// the digit planes follow the weight codes' own order).  So a lane's weight
// bytes for a stage are contiguous (Q4 16 B, Q8 32 B, Q6 24 B of its row):
// each lane loads exactly the A operand it will use, and the LDS ring only
// decouples the loads from the MFMAs (no register cost for the prefetch).
// The digit planes are shared by the 4 waves.
//
// Both operands are read from HBM images in this load order (the digitizer's
// tile layout, digit_off; the weight image, k_tile_weight), so each direct
// load reads 64 lanes × 16 (or 12) consecutive bytes.  From the row-major
// weights and [pl][n][K] planes a load touched 16 rows × 64 B, half of each
// 128-byte line, and the loads took 2.5× as long.
//
// Per stage and wave: B 3 loads (1 KB each: 12 per workgroup), A NMAT·RB
// (Q4) or 2·NMAT·RB (Q8, Q6) loads.  One barrier per stage: at its top every wave has waited
// for its own loads of this stage, and every wave has finished the previous
// stage, whose slot is then refilled NST−1 stages ahead.
// ---------------------------------------------------------------------------
constexpr int kStageCols = 128;

template <int QT>
struct ALds {
    static constexpr int chunks = QT == QT_Q4 ? 1 : 2;       // loads per (matrix, row block) and stage
    static constexpr int bytes = QT == QT_Q6 ? 12 : 16;      // bytes per lane and load
    static constexpr int lane_words = QT == QT_Q4 ? 4 : (QT == QT_Q8 ? 8 : 6);
    static constexpr int stage_row = QT == QT_Q4 ? 64 : (QT == QT_Q8 ? 128 : 96);  // row bytes per stage
    static constexpr int block_stage = chunks * 64 * bytes;  // image bytes per 16-row block and stage (16·stage_row)
};

// Weight image of the prefill GEMM: for 16-row block rb, stage u, load c and
// lane lr + 16·lg, the `bytes` that row 16rb + lr holds at stage_row·u +
// lg·stage_row/4 + c·bytes, stored at (((rb·nst + u)·chunks + c)·64 + lane)·
// bytes.  A permutation of the row-major bytes (rows a multiple of 16, K of
// 128); one thread per lane-load.
template <int QT>
static __global__ void __launch_bounds__(kThreads) k_tile_weight(const uint8_t *src, int row_bytes, int rows, int nst,
                                                                 uint8_t *dst) {
    using A = ALds<QT>;
    const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    const size_t total = (size_t)(rows / 16) * nst * A::chunks * 64;
    if (i >= total) return;
    const int lane = (int)(i % 64);
    const size_t t = i / 64;
    const int c = (int)(t % A::chunks);
    const int u = (int)((t / A::chunks) % nst);
    const size_t rb = t / A::chunks / nst;
    const uint32_t *sp = reinterpret_cast<const uint32_t *>(
        src + (16 * rb + (lane & 15)) * (size_t)row_bytes + A::stage_row * u + (lane >> 4) * (A::stage_row / 4) + c * A::bytes);
    uint32_t *dp = reinterpret_cast<uint32_t *>(dst + i * A::bytes);
#pragma unroll
    for (int w = 0; w < A::bytes / 4; ++w) dp[w] = sp[w];
}
// the direct load places lane i's bytes at 16·i for 12- and 16-byte loads alike
constexpr int kLdsLaneStride = 16;

template <int QT, int NMAT, int NST, int RB_, int NPL = 3>
struct GemmLdsLayout {
    static constexpr int RB = RB_;
    static constexpr int b_bytes = 2 * NPL * 2 * 64 * 16;                                     // [s][pl][tb][lane]
    static constexpr int a_wave = NMAT * RB * ALds<QT>::chunks * 64 * kLdsLaneStride;        // [mi][rb][c][lane]
    static constexpr int stage = b_bytes + kWaves * a_wave;
    static constexpr int total = NST * stage;
};

// HBM → LDS load of BYTES (16 or 12) per lane: lane i's bytes land at
// lds + 16·i.  Written as inline asm so the compiler's wait-count pass does
// not see an LDS write it cannot place (it would wait for every load in flight
// before each LDS read); the kernel orders these loads itself with wait_vm and
// lds_barrier.
template <int BYTES>
__device__ __forceinline__ void lds_load(const void *g, void *lds) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)lds);
    if constexpr (BYTES == 16)
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(base)
                     : "m0");
    else
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx3 %0, off" ::"v"(g), "s"(base)
                     : "m0");
}

// s_waitcnt vmcnt(N): at most N of this wave's vector-memory loads in flight
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// workgroup barrier that keeps LDS reads and loads on their side of it
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_barrier" ::: "memory");
}

template <int QT, int NMAT, int NST, int RB, int NPL = 3>
static __global__ void __launch_bounds__(kThreads) k_gemm_lds(GemmParams p, int epi) {
    static_assert(NST == 2 || NST == 3, "the main loop is unrolled over two or three slots");
    static_assert(NMAT * RB <= 4, "at most four row blocks per wave");
    static_assert(NPL == 3 || (NPL == 1 && QT != QT_Q8), "three digit planes, or one plane of VNNI bytes (Q4, Q6)");
    using Lay = GemmLdsLayout<QT, NMAT, NST, RB, NPL>;
    constexpr int WR = 16 * RB;                 // rows per matrix and wave
    constexpr int TB = 2;
    constexpr int CH = ALds<QT>::chunks, AB = ALds<QT>::bytes;
    constexpr int LPS = NPL + NMAT * RB * CH;   // loads per stage and wave
    __shared__ __attribute__((aligned(16))) uint8_t slot0[Lay::stage];
    __shared__ __attribute__((aligned(16))) uint8_t slot1[Lay::stage];
    __shared__ __attribute__((aligned(16))) uint8_t slot2[NST == 3 ? Lay::stage : 16];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int2 tile = xcd_tile();
    const int n0 = tile.y * 16 * TB;
    const int r0 = tile.x * (WR * kWaves) + wave * WR;
    const bool on = r0 < p.rows;              // uniform; rows are a multiple of WR
    const int rc = on ? r0 : p.rows - WR;     // loads stay in bounds for idle waves
    const int nst = p.K / kStageCols;

    const GemmSeg sg = gemm_seg<NMAT>(p, rc);
    constexpr int BS = ALds<QT>::block_stage;
    // this lane's A source in the weight image: 16-row block (rc − start)/16 + rb, stage 0, load 0
    const uint8_t *asrc[NMAT][RB];
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
            asrc[mi][rb] = sg.tiled[mi] + (size_t)((rc - sg.start) / 16 + rb) * nst * BS + lane * AB;
    // this wave's NPL B loads: chunks j = NPL·wave + i of the token tile's stages (digit_off)
    const int8_t *bsrc[NPL];
    int boff[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const int j = NPL * wave + i;
        bsrc[i] = p.xd + ((size_t)tile.y * nst * 4 * NPL + j) * 1024 + lane * 16;
        boff[i] = j * 1024;
    }
    const int aoff = Lay::b_bytes + wave * Lay::a_wave;

    auto issue = [&](int u, uint8_t *st) {
#pragma unroll
        for (int i = 0; i < NPL; ++i) lds_load<16>(bsrc[i] + (size_t)4 * NPL * 1024 * u, st + boff[i]);
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int c = 0; c < CH; ++c)
                    lds_load<AB>(asrc[mi][rb] + (size_t)BS * u + c * 64 * AB,
                                 st + aoff + ((mi * RB + rb) * CH + c) * 64 * kLdsLaneStride);
    };

    v4i acc[NMAT][RB][TB][NPL];
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                for (int pl = 0; pl < NPL; ++pl) acc[mi][rb][tb][pl] = v4i{0, 0, 0, 0};

    auto compute = [&](const uint8_t *st) {
        const v4i *bl = reinterpret_cast<const v4i *>(st);
        uint32_t raw[NMAT][RB][ALds<QT>::lane_words];  // the stage's weight bytes of this lane
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int c = 0; c < CH; ++c) {
                    const uint8_t *q = st + aoff + (((mi * RB + rb) * CH + c) * 64 + lane) * kLdsLaneStride;
                    if constexpr (AB == 16) {
                        const uint4 v = *reinterpret_cast<const uint4 *>(q);
                        raw[mi][rb][4 * c] = v.x; raw[mi][rb][4 * c + 1] = v.y;
                        raw[mi][rb][4 * c + 2] = v.z; raw[mi][rb][4 * c + 3] = v.w;
                    } else {
                        const uint32_t *w = reinterpret_cast<const uint32_t *>(q);
                        raw[mi][rb][3 * c] = w[0]; raw[mi][rb][3 * c + 1] = w[1]; raw[mi][rb][3 * c + 2] = w[2];
                    }
                }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            v4i b[TB][NPL];
#pragma unroll
            for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                for (int pl = 0; pl < NPL; ++pl) b[tb][pl] = bl[((s * NPL + pl) * TB + tb) * 64 + lane];
#pragma unroll
            for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
                    RawCodes<QT> rcd;
                    constexpr int W = QT == QT_Q8 ? 4 : (QT == QT_Q4 ? 2 : 3);
#pragma unroll
                    for (int w = 0; w < W; ++w) rcd.d[w] = raw[mi][rb][W * s + w];
                    const v4i av = unpack_codes16<QT>(rcd);
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                        for (int pl = 0; pl < NPL; ++pl)
                            acc[mi][rb][tb][pl] =
                                __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b[tb][pl], acc[mi][rb][tb][pl], 0, 0, 0);
                }
        }
    };
    // stage u: wait for this wave's loads of u (stage u+1 may stay in flight),
    // barrier (every wave's loads of u have landed; every wave is done with
    // u−1, whose slot takes stage u+2), then the MFMAs of u
    auto body = [&](int u, const uint8_t *cur, uint8_t *refill) {
        if (u + 1 < nst) wait_vm<LPS>();
        else wait_vm<0>();
        lds_barrier();
        if (u + 2 < nst) issue(u + 2, refill);
        if (on) compute(cur);
    };

    if constexpr (NST == 3) {
        issue(0, slot0);
        if (nst > 1) issue(1, slot1);
        for (int u = 0; u < nst; u += 3) {
            body(u, slot0, slot2);
            if (u + 1 < nst) body(u + 1, slot1, slot0);
            if (u + 2 < nst) body(u + 2, slot2, slot1);
        }
    } else {
        // two slots: stage u+1 is requested after the barrier of stage u
        // (every wave is done with u−1, whose slot it takes) and lands while
        // u is computed; the smaller ring lets two workgroups share a CU
        auto body2 = [&](int u, const uint8_t *cur, uint8_t *next) {
            wait_vm<0>();
            lds_barrier();
            if (u + 1 < nst) issue(u + 1, next);
            if (on) compute(cur);
        };
        issue(0, slot0);
        for (int u = 0; u < nst; u += 2) {
            body2(u, slot0, slot1);
            if (u + 1 < nst) body2(u + 1, slot1, slot0);
        }
    }
    if (!on) return;

    // epilogue: lane holds token n0+16tb+lr, rows r0+16rb+4lg+i (i < 4)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
        const int n = n0 + 16 * tb + lr;
        if (n >= p.ntok) continue;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int rr = r0 + 16 * rb + 4 * lg;
            const float *const scl[2] = {sg.scale[0] + (rr - sg.start),
                                         NMAT == 2 ? sg.scale[1] + (rr - sg.start) : nullptr};
            if constexpr (NPL == 1) {
                const int *const us[2] = {sg.usum[0] + (rr - sg.start),
                                          NMAT == 2 ? sg.usum[1] + (rr - sg.start) : nullptr};
                v4i a1[NMAT];
#pragma unroll
                for (int mi = 0; mi < NMAT; ++mi) a1[mi] = acc[mi][rb][tb][0];
                gemm_store_vnni<QT, NMAT>(p, epi, n, rr, scl, us, a1);
            } else {
                v4i a3[NMAT][3];
#pragma unroll
                for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
                    for (int pl = 0; pl < 3; ++pl) a3[mi][pl] = acc[mi][rb][tb][pl];
                gemm_store<QT, NMAT>(p, epi, n, rr, scl, a3);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Small-M MFMA GEMM (M ≤ 16 tokens, the batched GEMV): a workgroup owns 16
// rows (of each matrix with NMAT = 2) and all tokens; its 4 waves split K in
// quarters, request their K-steps in double-buffered batches of four (a wave
// waits on memory once or twice, not once per step), and their exact int32
// partials are summed through LDS before wave 0 applies the epilogue.
// ---------------------------------------------------------------------------
constexpr int kSmallBatch = 4;  // K-steps per request batch

template <int QT, int NMAT>
static __global__ void __launch_bounds__(kThreads) k_gemm_small(GemmParams p, int epi) {
    __shared__ v4i part[kWaves - 1][NMAT][3][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r0 = blockIdx.x * 16;
    const int lr = lane & 15, lg = lane >> 4;
    const GemmSeg sg = gemm_seg<NMAT>(p, r0);
    const int row_bytes = p.m[0].row_bytes;
    const uint8_t *arow[NMAT];
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi) arow[mi] = sg.base[mi] + (size_t)(r0 + lr - sg.start) * row_bytes;
    const int8_t *brow = p.xd + (size_t)lr * p.K + 16 * lg;
    const int kq = p.K / kWaves;  // this wave's K range [wave·kq, (wave+1)·kq), a multiple of 64
    const int kbeg = wave * kq;
    const int nsteps = kq / kGemmK;

    v4i acc[NMAT][3];
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) acc[mi][pl] = v4i{0, 0, 0, 0};
    v4i a[kSmallBatch][NMAT], b[kSmallBatch][3];
    auto load = [&](int s0, v4i (&aa)[kSmallBatch][NMAT], v4i (&bb)[kSmallBatch][3]) {
#pragma unroll
        for (int j = 0; j < kSmallBatch; ++j) {
            const int k0 = kbeg + kGemmK * min(s0 + j, nsteps - 1);  // clamped: loaded, not used
            const int k = k0 + 16 * lg;
#pragma unroll
            for (int mi = 0; mi < NMAT; ++mi) aa[j][mi] = load_codes16<QT>(arow[mi], k);
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) bb[j][pl] = *reinterpret_cast<const v4i *>(brow + pl * p.plane_stride + k0);
        }
    };
    load(0, a, b);
    for (int s0 = 0; s0 < nsteps; s0 += kSmallBatch) {
        v4i an[kSmallBatch][NMAT], bn[kSmallBatch][3];
        const bool more = s0 + kSmallBatch < nsteps;  // uniform
        if (more) load(s0 + kSmallBatch, an, bn);
#pragma unroll
        for (int j = 0; j < kSmallBatch; ++j) {
            if (s0 + j >= nsteps) break;  // uniform
#pragma unroll
            for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
                for (int pl = 0; pl < 3; ++pl)
                    acc[mi][pl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[j][mi], b[j][pl], acc[mi][pl], 0, 0, 0);
        }
        if (more) {
#pragma unroll
            for (int j = 0; j < kSmallBatch; ++j) {
#pragma unroll
                for (int mi = 0; mi < NMAT; ++mi) a[j][mi] = an[j][mi];
#pragma unroll
                for (int pl = 0; pl < 3; ++pl) b[j][pl] = bn[j][pl];
            }
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) part[wave - 1][mi][pl][lane] = acc[mi][pl];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < kWaves - 1; ++w)
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) acc[mi][pl] += part[w][mi][pl][lane];
    const int n = lr;  // token (column)
    if (n >= p.ntok) return;
    const int rr = r0 + 4 * lg;
    const float *const scl[2] = {sg.scale[0] + (rr - sg.start), NMAT == 2 ? sg.scale[1] + (rr - sg.start) : nullptr};
    gemm_store<QT, NMAT>(p, epi, n, rr, scl, acc);
}

// ---------------------------------------------------------------------------
// Per-token RoPE of q and k (table from the token's (T,H,W) position in f64,
// buildMRoPETable, model.go:7318-7357) and the K/V append of token n at cache
// row clen0+n (kvCache.append, model.go:5593-5612).  qkv rows are
// [q heads | k heads | v heads] of head_dim floats; q is rotated in place.
// ---------------------------------------------------------------------------
static __global__ void __launch_bounds__(kThreads) k_rope_append(float *qkv, int stride, const int32_t *pos3,
                                                            const double *freq, const uint8_t *axis, int heads,
                                                            int kvh, int head_dim, float *kc, float *vc,
                                                            int clen0) {
    __shared__ float cs[kMaxHalf], sn[kMaxHalf];
    const int n = blockIdx.x;
    const int half = head_dim / 2;
    for (int i = threadIdx.x; i < half; i += kThreads) {
        const int a = axis[i];
        const double ang = (double)pos3[3 * n + a] * freq[i];
        cs[i] = (float)cos(ang);
        sn[i] = (float)sin(ang);
    }
    __syncthreads();
    float *row = qkv + (size_t)n * stride;
    const int kvd = kvh * head_dim;
    const int t = clen0 + n;
    for (int i = threadIdx.x; i < (heads + kvh) * half; i += kThreads) {
        const int h = i / half, j = i % half;
        float *x = row + (size_t)h * head_dim;  // k heads follow the q heads
        float a = x[j], b = x[j + half];
        rope_pair(a, b, cs[j], sn[j]);
        if (h < heads) {
            x[j] = a;
            x[j + half] = b;
        } else {
            float *kd = kc + (size_t)t * kvd + (h - heads) * head_dim;
            kd[j] = a;
            kd[j + half] = b;
        }
    }
    const float *v = row + (size_t)(heads + kvh) * head_dim;
    for (int i = threadIdx.x; i < kvd; i += kThreads) vc[(size_t)t * kvd + i] = v[i];
}

// ---------------------------------------------------------------------------
// Causal prefill attention on bf16 MFMA (v_mfma_f32_16x16x32_bf16) with split
// operands: every fp32 operand x is carried as hi = bf16(x), lo = bf16(x − hi)
// (x = hi + lo to 2^-17 relative) and a product as hi·hi + hi·lo + lo·hi,
// accumulated in fp32 (the dropped lo·lo term is below 2^-16 relative).
//
// k_kv_blocks first writes, per KV head and 32-key block, the block's LDS
// image (32 KB): K as [hi/lo][key][16 chunks of 8 dims] with chunk j of key r
// at position j ^ (r & 15), and V transposed as [hi/lo][dim][8 quads of 4 keys]
// with quad q of dim d at position q ^ ((d >> 1) & 7).  The XOR swizzles make
// the attention kernel's operand reads bank-conflict free with unpadded rows.
//
// k_attn_prefill — workgroup: one KV head, 4 query heads of its group (one per
// wave) and two 16-token tiles, i and NT−1−i, so every workgroup meets the
// same number of key blocks under the causal mask.  Both tiles go in one pass
// over the longer one's key blocks: each block image is loaded once for both
// (HBM → LDS by direct loads, two slots of two blocks); per block and tile
// each wave runs
//   Sᵀ (keys × tokens) = K · Qᵀ     2 key tiles × 4 dim chunks × 3 MFMAs
//   online softmax per token column (the column's keys sit in 4 lane groups)
//   Oᵀ (dims × tokens) += Vᵀ · Pᵀ   8 dim tiles × 3 MFMAs, K index = keys
// Pᵀ feeds the second product straight from the first one's accumulators: MFMA
// step element e of lane group lg is key 4lg+e (e < 4) or 16+4lg+(e−4), the
// rows that lane already holds, and Vᵀ is read in the same key order.
// Online softmax per token (max, Σexp) with exp_hw; token n attends cache
// rows [0, clen0+n]; scores dot·f32(1/√128) (model.go:4623-4795, 7391).
// ---------------------------------------------------------------------------
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
constexpr int kPfTok = 16;                  // query tokens per tile
constexpr int kPfKeys = 32;                 // keys per block
constexpr int kPfKPlane = kPfKeys * kHD;    // bf16 per K plane of a block image
constexpr int kPfImage = 4 * kPfKPlane * 2; // bytes per block image (K and Vᵀ, hi and lo): 32 KB

// e^x from the hardware base-2 exponential (v_exp_f32, about 1 ulp), for the
// prefill attention's weights, rescales and parity merge: the weights enter
// split-bf16 products (2^-16 relative), so FastExpF32's own ~1e-7 departure
// from e^x is far below what the products keep, and the hardware form costs
// 3 VALU issues against about 20 for the restated polynomial, which made this
// kernel VALU-bound (57.1 → 50.3 µs per layer at 1,345 tokens)
__device__ __forceinline__ float exp_hw(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

__device__ __forceinline__ void split_bf16(float x, __bf16 &hi, __bf16 &lo) {
    hi = (__bf16)x;
    lo = (__bf16)(x - (float)hi);
}

// image offsets (bf16 elements) of K chunk (plane, key r, chunk j) and Vᵀ quad
// (plane, dim d, quad q)
__device__ __forceinline__ int pf_k_at(int plane, int r, int j) {
    return plane * kPfKPlane + r * kHD + 8 * (j ^ (r & 15));
}
__device__ __forceinline__ int pf_v_at(int plane, int d, int q) {
    return 2 * kPfKPlane + plane * kPfKPlane + d * kPfKeys + 4 * (q ^ ((d >> 1) & 7));
}

// grid (blocks, kvh): block images of cache rows [0, rows) (rows past the end
// repeat the last one; the attention masks them)
static __global__ void __launch_bounds__(kThreads) k_kv_blocks(const float *kc, const float *vc, int kvh, int rows,
                                                          int nblk, uint8_t *img) {
    const int b = blockIdx.x, g = blockIdx.y, t = threadIdx.x;
    const int kvd = kvh * kHD;
    __bf16 *im = reinterpret_cast<__bf16 *>(img + ((size_t)g * nblk + b) * kPfImage);
    {   // K: key r = t/8, chunks 2·(t%8), 2·(t%8)+1
        const int r = t >> 3, j0 = 2 * (t & 7);
        const float4 *src = reinterpret_cast<const float4 *>(kc + (size_t)min(b * kPfKeys + r, rows - 1) * kvd +
                                                             g * kHD + 8 * j0);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const float4 x0 = src[2 * c], x1 = src[2 * c + 1];
            const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            v8bf h, l;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                __bf16 a, bb;
                split_bf16(x[e], a, bb);
                h[e] = a;
                l[e] = bb;
            }
            *reinterpret_cast<v8bf *>(im + pf_k_at(0, r, j0 + c)) = h;
            *reinterpret_cast<v8bf *>(im + pf_k_at(1, r, j0 + c)) = l;
        }
    }
    {   // Vᵀ: dim d = t/2, quads 4·(t%2) .. +3
        const int d = t >> 1, qb = 4 * (t & 1);
#pragma unroll
        for (int q = qb; q < qb + 4; ++q) {
            v4bf h, l;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float x = vc[(size_t)min(b * kPfKeys + 4 * q + i, rows - 1) * kvd + g * kHD + d];
                __bf16 a, bb;
                split_bf16(x, a, bb);
                h[i] = a;
                l[i] = bb;
            }
            *reinterpret_cast<v4bf *>(im + pf_v_at(0, d, q)) = h;
            *reinterpret_cast<v4bf *>(im + pf_v_at(1, d, q)) = l;
        }
    }
}

// max / sum over the lanes l, l^16, l^32, l^48 (the 4 lane groups of an MFMA
// column) with VALU lane swaps: swap(x, x) leaves {x[l], x[l^16]} (resp.
// l^32) in the two results of every lane
__device__ __forceinline__ float groups4_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float groups4_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

constexpr int kPfThreads = 512;   // 8 waves: 4 query heads × 2 key-block parities

static __global__ void __launch_bounds__(kPfThreads) k_attn_prefill(const float *qkv, int stride, const uint8_t *img,
                                                               int nblk_img, int heads, int kvh, int ntok,
                                                               int clen0, float scale, float *out, int out_stride) {
    // two stages of two block images (blocks 2s, 2s+1): 128 KB
    __shared__ __attribute__((aligned(16))) uint8_t stage0[2 * kPfImage];
    __shared__ __attribute__((aligned(16))) uint8_t stage1[2 * kPfImage];
    constexpr int kW = kPfThreads / 64;
    constexpr int LPS = 2 * kPfImage / 1024 / kW;  // direct loads per stage and wave (8)
    const int group = heads / kvh;
    const int quads = (group + 3) / 4;
    const int g = blockIdx.x / quads, quad = blockIdx.x % quads;
    const int t = threadIdx.x, l = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int par = wave >> 2;                    // key-block parity of this wave
    const int lr = l & 15, lg = l >> 4;
    const int hl = 4 * quad + (wave & 3);         // head within the group
    const bool wave_on = hl < group;              // uniform
    const int hh = g * group + min(hl, group - 1);
    const int nt = (ntok + kPfTok - 1) / kPfTok;
    const uint8_t *gimg = img + (size_t)g * nblk_img * kPfImage + (size_t)wave * LPS * 1024 + 16 * l;
    auto issue = [&](int s, int nblk, uint8_t *st) {
        // blocks 2s, 2s+1 are contiguous in the image; a missing 2s+1 is not loaded
        const uint8_t *src = gimg + (size_t)(2 * s) * kPfImage;
        const bool two = 2 * s + 1 < nblk;
#pragma unroll
        for (int i = 0; i < LPS; ++i) {
            const int chunk = wave * LPS + i;  // 1 KB chunk of the stage
            if (two || chunk < kPfImage / 1024) lds_load<16>(src + 1024 * i, st + chunk * 1024);
        }
    };

    // the causal pair: tile 0 = blockIdx.y (the shorter), tile 1 = nt − 1 −
    // blockIdx.y, both in one pass over the longer one's key blocks, so each
    // block is loaded once and its operands are read from LDS once for both
    const int tq0 = (int)blockIdx.y, tq1 = nt - 1 - (int)blockIdx.y;
    const bool pair = tq1 > tq0;                  // uniform; the middle tile of an odd count is alone
    int q0[2], my_last[2], nblk[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        q0[u] = (u == 0 ? tq0 : tq1) * kPfTok;
        const int tq = min(q0[u] + lr, ntok - 1);  // this lane's token (clamped; stored only if < ntok)
        my_last[u] = clen0 + tq;
        nblk[u] = (clen0 + min(q0[u] + kPfTok, ntok) - 1) / kPfKeys + 1;
    }
    const int nblk_all = pair ? nblk[1] : nblk[0];
    const int nstage = (nblk_all + 1) / 2;

    // Qᵀ operands of the first product: token lr, dims 32c + 8lg + e
    v8bf qh[2][4], ql[2][4];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const float *qs = qkv + (size_t)min(q0[u] + lr, ntok - 1) * stride + (size_t)hh * kHD + 8 * lg;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float4 a4 = *reinterpret_cast<const float4 *>(qs + 32 * c);
            const float4 b4 = *reinterpret_cast<const float4 *>(qs + 32 * c + 4);
            const float x[8] = {a4.x, a4.y, a4.z, a4.w, b4.x, b4.y, b4.z, b4.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                __bf16 h, lo;
                split_bf16(x[e], h, lo);
                qh[u][c][e] = h;
                ql[u][c][e] = lo;
            }
        }
    }
    v4f o[2][8];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[u][dt] = v4f{0.f, 0.f, 0.f, 0.f};
    float m[2] = {-INFINITY, -INFINITY}, lsum[2] = {0.0f, 0.0f};

    // block b for tile U (a compile-time index, so the tile's registers stay
    // registers): Sᵀ, the online softmax of token column lr, Oᵀ += Vᵀ·Pᵀ
    auto compute = [&](int b, const uint8_t *slot, auto tile) {
        // scores are rounded (s·scale) before the max is subtracted
#pragma clang fp contract(off)
        constexpr int U = decltype(tile)::value;
        const __bf16 *im = reinterpret_cast<const __bf16 *>(slot);
        const int k0 = b * kPfKeys;
        v4f sT[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            sT[kt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const v8bf kh = *reinterpret_cast<const v8bf *>(im + pf_k_at(0, 16 * kt + lr, 4 * c + lg));
                const v8bf kl = *reinterpret_cast<const v8bf *>(im + pf_k_at(1, 16 * kt + lr, 4 * c + lg));
                sT[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, qh[U][c], sT[kt], 0, 0, 0);
                sT[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, ql[U][c], sT[kt], 0, 0, 0);
                sT[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, qh[U][c], sT[kt], 0, 0, 0);
            }
        }
        // online softmax of token column lr (branch-free: masked keys get
        // p = 0 by selection after an exp of a clamped argument)
        float sv[8];
        bool vis[8];
        float mb = m[U];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                vis[4 * kt + i] = k0 + 16 * kt + 4 * lg + i <= my_last[U];
                sv[4 * kt + i] = vis[4 * kt + i] ? sT[kt][i] * scale : -INFINITY;
                mb = fmaxf(mb, sv[4 * kt + i]);
            }
        mb = groups4_max(mb);
        // a column may have seen no visible key yet on this parity (mb = −∞):
        // its p are all 0 and its running sums stay 0
        const float mx = mb == -INFINITY ? 0.0f : mb;
        float ps = 0.0f;
        v8bf ph, pl;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float ex = exp_hw(sv[e] - mx);
            const float p = vis[e] ? ex : 0.0f;
            ps += p;
            __bf16 a, c;
            split_bf16(p, a, c);
            ph[e] = a;
            pl[e] = c;
        }
        ps = groups4_sum(ps);
        // rescale only when a column's maximum moved (exp_hw(0) is exactly
        // 1, so skipping is exact)
        if (__builtin_amdgcn_ballot_w64(mb != m[U])) {
            const float fe = exp_hw(m[U] - mx);
            const float f = m[U] == -INFINITY ? 0.0f : fe;
            lsum[U] *= f;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) o[U][dt] *= f;
        }
        lsum[U] += ps;
        m[U] = mb;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const int d = 16 * dt + lr;
            const v4bf ah0 = *reinterpret_cast<const v4bf *>(im + pf_v_at(0, d, lg));
            const v4bf ah1 = *reinterpret_cast<const v4bf *>(im + pf_v_at(0, d, 4 + lg));
            const v4bf al0 = *reinterpret_cast<const v4bf *>(im + pf_v_at(1, d, lg));
            const v4bf al1 = *reinterpret_cast<const v4bf *>(im + pf_v_at(1, d, 4 + lg));
            const v8bf vh = __builtin_shufflevector(ah0, ah1, 0, 1, 2, 3, 4, 5, 6, 7);
            const v8bf vl = __builtin_shufflevector(al0, al1, 0, 1, 2, 3, 4, 5, 6, 7);
            o[U][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, ph, o[U][dt], 0, 0, 0);
            o[U][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, pl, o[U][dt], 0, 0, 0);
            o[U][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl, ph, o[U][dt], 0, 0, 0);
        }
    };
    // stage s: wait for this wave's loads of s, barrier (every wave's loads
    // of s have landed; every wave is done with s−1, whose buffer takes
    // s+1), then this wave's block 2s + parity
    auto body = [&](int s, const uint8_t *cur, uint8_t *next) {
        wait_vm<0>();
        lds_barrier();
        if (s + 1 < nstage) issue(s + 1, nblk_all, next);
        const int b = 2 * s + par;
        if (!wave_on || b >= nblk_all) return;
        const uint8_t *slot = cur + par * kPfImage;
        // the shorter tile's keys end at block nblk[0]; the middle tile of an
        // odd count is tile 0 alone
        if (b < nblk[0]) compute(b, slot, std::integral_constant<int, 0>{});
        if (pair) compute(b, slot, std::integral_constant<int, 1>{});
    };
    issue(0, nblk_all, stage0);
    for (int s = 0; s < nstage; s += 2) {
        body(s, stage0, stage1);
        if (s + 1 < nstage) body(s + 1, stage1, stage0);
    }

    // merge the two parities of each head through LDS, tile u in stage u
    // (free after the barrier: no loads are in flight)
    lds_barrier();
    if (par == 1) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            float *mrg = reinterpret_cast<float *>(u == 0 ? stage0 : stage1) + (size_t)((wave & 3) * 64 + l) * 34;
            mrg[0] = m[u];
            mrg[1] = lsum[u];
#pragma unroll
            for (int dt = 0; dt < 8; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i) mrg[2 + 4 * dt + i] = o[u][dt][i];
        }
    }
    lds_barrier();
    if (par == 0 && wave_on) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if ((u == 1 && !pair) || q0[u] + lr >= ntok) continue;
            const float *mrg = reinterpret_cast<const float *>(u == 0 ? stage0 : stage1) + (size_t)((wave & 3) * 64 + l) * 34;
            const float m1 = mrg[0], l1 = mrg[1];
            const float M = fmaxf(m[u], m1);  // finite: key 0 is in block 0
            const float f0 = m[u] == -INFINITY ? 0.0f : exp_hw(m[u] - M);
            const float f1 = m1 == -INFINITY ? 0.0f : exp_hw(m1 - M);
            const float inv = 1.0f / (lsum[u] * f0 + l1 * f1);
            float *dst = out + (size_t)(q0[u] + lr) * out_stride + (size_t)hh * kHD + 4 * lg;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) {
                float r[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) r[i] = (o[u][dt][i] * f0 + mrg[2 + 4 * dt + i] * f1) * inv;
                *reinterpret_cast<float4 *>(dst + 16 * dt) = make_float4(r[0], r[1], r[2], r[3]);
            }
        }
    }
}


// Greedy choice over rows of logits (the batched LM head): workgroup (x, i)
// scans its slice of row i and folds the best (score, index) key into argmax
// slot x of sequence i's state, as the GEMV argmax epilogue does: key =
// ordered score bits · 2^32 + (2^32 − 1 − index), so the maximum key is the
// highest score and, among equal scores, the lowest index; NaN and −inf are
// never chosen.
static __global__ void __launch_bounds__(kThreads) k_argmax_rows(const float *logits, int ld, int cols, int slice,
                                                               StepState *const *rst) {
    const int i = blockIdx.y;
    const int c0 = blockIdx.x * slice, c1 = min(cols, c0 + slice);
    const float *row = logits + (size_t)i * ld;
    unsigned long long best = 0ull;
    for (int c = c0 + (int)threadIdx.x; c < c1; c += kThreads) {
        const float v = row[c];
        if (v > -INFINITY) {
            const unsigned long long k =
                ((unsigned long long)ordered_bits(v) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)c);
            best = k > best ? k : best;
        }
    }
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) {
        const unsigned long long o = ((unsigned long long)__shfl_xor((unsigned)(best >> 32), m, 64) << 32) |
                                     (unsigned)__shfl_xor((unsigned)best, m, 64);
        best = o > best ? o : best;
    }
    __shared__ unsigned long long wb[kWaves];
    if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long m = wb[0];
        for (int w = 1; w < kWaves; ++w) m = wb[w] > m ? wb[w] : m;
        if (m) atomicMax(&rst[i]->argmax_slot[(blockIdx.x % kArgSlots) * kSlotPitch], m);
    }
}
}  // namespace pocr
