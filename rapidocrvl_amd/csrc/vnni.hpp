// vnni.hpp — the reference's VNNI activation mode for Q4/Q6 matrices.
//
// On an amd64 host with AVX512-VNNI the reference's CPU path does not
// multiply the f32 activation by the codes.  It quantizes the activation once
// per matvec to unsigned bytes (quantizeXForVNNI, internal/tensor/
// quant.go:2087-2115; quantizeXForVNNIAVX2, dot_amd64.go:228-252;
// quantizeXForVNNIAsm, dot_vnni_amd64.s:434-500):
//   m = max|x|;  m = 0 → every byte 128, scaleX = 1;
//   scaleX = m/127,  inv = 1/scaleX,  xq[c] = clamp(RNE(x[c]·inv) + 128, 0, 255)
// takes the exact int32 dot of the signed codes with those bytes (VPDPBUSD,
// dotQ8VNNI dot_amd64.go:150-167) and finishes a row as
//   out[r] = ((f32(dot) − f32(rowSum)·128)·scaleX)·scale[r]
// (finalizeDotQ8VNNI, dot_vnni_amd64.s:1043-1080), rowSum = Σ code of the row.
// Q8 matrices keep the plain f32 mode (they carry no row sums), and so do
// inputs of fewer than 32 columns.
//
// Here every step of that is exact or a single IEEE operation, so the scores
// are bit-identical to the reference's:
// * the maximum is order-free; the two divisions are correctly rounded;
// * the row's integer sums come from v_dot4_i32_i8 on the stored unsigned
//   codes u = code + IBIAS (Q4 nibbles, Q6 fields) against d = xq − 128:
//     Σ code·xq = Σ u·d + 128·Σu − IBIAS·Σxq,   rowSum = Σu − IBIAS·cols,
//   all int32 (|Σ u·d| ≤ 63·128·8192 < 2³¹);
// * only the finalize is f32, in the reference's order.
// RMSNorm prologues form the normalised vector first (x·factor·w, as
// RMSNorm does, ops.go:1015-1037, with Σx² in sumSquaresScalar's order,
// ops.go:1039-1058) and quantize that.
//
// A matvec is bit-identical to the reference's VNNI matvec for the same x.
// Around the matvecs the mode keeps the portable scalar orders (RMSNorm's
// sumSquaresScalar, dotF32's eight running sums, the scalar Softmax). An
// x86-64 AVX512-VNNI host runs those ops through its FMA/AVX kernels instead
// (useDotFMA is fixed true there, dot_amd64.go:11: sumSquaresF32FMA,
// mulScaleFMA, dotF32AVX, expScaledVecFMA), whose accumulation orders are not
// restated here. Whole steps and streams are therefore bit-identical to the
// CPU port's VNNI mode, and agree with such a host to rounding only.
#pragma once

#include "kernels.hpp"

namespace pocr {

constexpr int kVnniMaxCols = 8192;  // f32 copy + one byte per column in LDS
constexpr int kVnniMaxGrid = 2048;

// byte position of column c's d in LDS.  Q4 (fast rows): a 32-column chunk
// is 8 dwords, dword 2k holding columns 8k+0,2,4,6 (the low nibbles of the
// row's dword k) and dword 2k+1 columns 8k+1,3,5,7.  Q6 and the any-shape
// rows: natural order.
template <int QT, bool FAST>
__device__ __forceinline__ int vnni_pos(int c) {
    if constexpr (QT == QT_Q4 && FAST) {
        const int w = c & 31, k = 2 * (w >> 3) + (w & 1), m = (w & 7) >> 1;
        return (c & ~31) + 4 * k + m;
    } else {
        return c;
    }
}

__device__ __forceinline__ int half_wave_sum_i(int v) {
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// The row's Σ u·d and Σ u over this lane's chunks (FAST shapes): Q4 chunks of
// 16 bytes (32 codes), Q6 chunks of 12 bytes (16 codes); 32 lanes per row.
template <int QT>
__device__ __forceinline__ void vnni_row_fast(const uint8_t *row, const int *dq, int nchunks, int l32, int &a,
                                              int &u) {
    constexpr int ONES = 0x01010101;
    for (int c = l32; c < nchunks; c += 32) {
        if constexpr (QT == QT_Q4) {
            const uint4 w = *reinterpret_cast<const uint4 *>(row + 16 * (size_t)c);
            const int4 d0 = *reinterpret_cast<const int4 *>(dq + 8 * c);
            const int4 d1 = *reinterpret_cast<const int4 *>(dq + 8 * c + 4);
            const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
            const int dd[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int lo = (int)(wd[k] & 0x0F0F0F0Fu), hi = (int)((wd[k] >> 4) & 0x0F0F0F0Fu);
                a = __builtin_amdgcn_sdot4(lo, dd[2 * k], a, false);
                a = __builtin_amdgcn_sdot4(hi, dd[2 * k + 1], a, false);
                u = __builtin_amdgcn_sdot4(lo, ONES, u, false);
                u = __builtin_amdgcn_sdot4(hi, ONES, u, false);
            }
        } else {
            const uint32_t *p = reinterpret_cast<const uint32_t *>(row + 12 * (size_t)c);
            const uint32_t w0 = p[0], w1 = p[1], w2 = p[2];
            const int4 d = *reinterpret_cast<const int4 *>(dq + 4 * c);
            const int g[4] = {spread6(w0 & 0xFFFFFFu), spread6((w0 >> 24) | ((w1 & 0xFFFFu) << 8)),
                              spread6((w1 >> 16) | ((w2 & 0xFFu) << 16)), spread6(w2 >> 8)};
            const int dd[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                a = __builtin_amdgcn_sdot4(g[k], dd[k], a, false);
                u = __builtin_amdgcn_sdot4(g[k], ONES, u, false);
            }
        }
    }
}

// The same sums for any shape: codes one at a time (signed code c = u − IBIAS
// is folded back to u so both paths produce the same integers).
__device__ __forceinline__ void vnni_row_any(const DevMat &M, const uint8_t *row, const int8_t *dq, int cols,
                                             int l32, int ibias, int &a, int &u) {
    for (int c = l32; c < cols; c += 32) {
        const int uc = decode_code(M, row, c) + ibias;
        a += uc * (int)dq[c];
        u += uc;
    }
}

// x → LDS, RMSNorm'ed with Σx² in sumSquaresScalar's order (ops.go:1039-1058:
// eight running sums over the columns ≡ j mod 8, added as a tree, the tail
// one by one), so that the normalised vector, and with it every byte, is the
// reference's: an activation byte that moves moves a whole row's score by
// one step of the weights.  red holds at least 8 floats.
__device__ __forceinline__ void stage_x_rms_ordered(float *xs, const float *x, const float *w, int n, float eps,
                                                    float *red) {
#pragma clang fp contract(off)
    for (int i = threadIdx.x; i < n; i += kThreads) xs[i] = x[i];
    __syncthreads();
    const int n8 = n & ~7;
    if (threadIdx.x < 8) {  // sum j: columns j, j + 8, … in order, 16 reads in flight
        float s = 0.0f;
        int i = threadIdx.x;
        for (; i + 8 * 15 < n8; i += 8 * 16) {
            float v[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) v[k] = xs[i + 8 * k];
#pragma unroll
            for (int k = 0; k < 16; ++k) s = s + v[k] * v[k];
        }
        for (; i < n8; i += 8) s = s + xs[i] * xs[i];
        red[threadIdx.x] = s;
    }
    __syncthreads();
    float ss = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
    for (int i = n8; i < n; ++i) ss = ss + xs[i] * xs[i];
    const float scale = fast_rsqrt_ref(ss / (float)n + eps);
    __syncthreads();  // every thread has read red
    for (int i = threadIdx.x; i < n; i += kThreads) xs[i] = xs[i] * scale * w[i];
    __syncthreads();
}

// LDS: xs f32[cols], then d = xq − 128 as int8 [cols rounded up to 16].
template <int QT, int NMAT, bool FAST>
__global__ void __launch_bounds__(kThreads) k_gemv_vnni(GemvParams p, int pro, int epi) {
    if (p.st && p.st->err) return;
    extern __shared__ float xs[];
    __shared__ float red[2 * kWaves];
    __shared__ int redi[kWaves];
    static_assert(2 * kWaves >= 8, "the ordered sum of squares keeps eight partial sums");
    const int cols = p.cols;
    if (pro == PRO_RMSNORM) stage_x_rms_ordered(xs, p.x, p.norm_w, cols, p.eps, red);
    else stage_x<PRO_COPY>(xs, p.x, p.norm_w, cols, p.eps, red);
    int8_t *dq = reinterpret_cast<int8_t *>(xs + cols);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

    // 1. scaleX and the bytes (quantizeXForVNNI)
    float mx = 0.0f;
    for (int i = threadIdx.x; i < cols; i += kThreads) mx = fmaxf(mx, fabsf(xs[i]));
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) m = fmaxf(m, red[w]);
    const float sx = m == 0.0f ? 1.0f : m / 127.0f;
    const float inv = 1.0f / sx;
    int sq = 0;
    for (int i = threadIdx.x; i < cols; i += kThreads) {
        int q = 128;
        if (m != 0.0f) {
            float v = rintf(xs[i] * inv) + 128.0f;
            v = fminf(fmaxf(v, 0.0f), 255.0f);
            q = (int)v;
        }
        dq[vnni_pos<QT, FAST>(i)] = (int8_t)(q - 128);
        sq += q;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off, 64);
    if (lane == 0) redi[wave] = sq;
    __syncthreads();
    int sum_xq = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) sum_xq += redi[w];
    constexpr int IB = DigitTraits<QT>::IBIAS;

    // 2. rows: 32 lanes per row, two rows per wave and pass
    const int half = lane >> 5, l32 = lane & 31;
    const int nchunks = cols / QTraits<QT>::W;
    const bool in_place = epi == EPI_OPROJ ? oproj_in_place(p, p.st) : false;
    float best_v = -INFINITY;
    int best_r = 0x7FFFFFFF;
    constexpr int RPB = 2 * kWaves;
    for (int r0 = blockIdx.x * RPB; r0 < p.rows; r0 += gridDim.x * RPB) {
        const int r = r0 + 2 * wave + half;
        const bool valid = r < p.rows;
        const int rc = valid ? r : p.rows - 1;
        int sg = 0, lr = rc;
        if (NMAT == 1) {
            sg = (rc >= p.seg_end[0]) + (rc >= p.seg_end[1]);
            lr = rc - (sg == 0 ? 0 : (sg == 1 ? p.seg_end[0] : p.seg_end[1]));
        }
        float s[NMAT];
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi) {
            const DevMat M = seg_mat(p, NMAT == 1 ? sg : mi);
            const uint8_t *row = M.data + (size_t)lr * M.row_bytes;
            int a = 0, u = 0;
            if constexpr (FAST) vnni_row_fast<QT>(row, reinterpret_cast<const int *>(dq), nchunks, l32, a, u);
            else vnni_row_any(M, row, dq, cols, l32, IB, a, u);
            a = half_wave_sum_i(a);
            u = half_wave_sum_i(u);
            const int dot = a + 128 * u - IB * sum_xq;  // Σ code·xq
            const int rowsum = u - IB * cols;           // Σ code
            {
#pragma clang fp contract(off)
                const float v = (float)dot - (float)rowsum * 128.0f;
                s[mi] = v * sx * M.scale[lr];
            }
        }
        if (l32 == 0 && valid)
            gemv_epilogue(p, epi, r, r, s, epi_reads_residual(epi) ? p.residual[r] : 0.0f, in_place, best_v, best_r);
    }
    if (epi == EPI_ARGMAX) argmax_finish(p.st, best_v, best_r, red);
}

// ---------------------------------------------------------------------------
// Decode attention in the reference's summation order (attendHead over the
// f32 cache, internal/model/model.go:4603-5590; Softmax ops.go:1199-1363;
// weightedCacheValueSum128 5479-5515), for the VNNI mode: there an ulp of
// difference in one attention output can move an activation byte of o_proj
// and with it a whole row, so the split-K kernel's reassociated sums would
// not keep the reference's tokens.  Every sum here is the reference's:
// * score t = dotF32 (eight running sums over dims ≡ j mod 8, tree-added,
//   ops.go:626-645) of the rotated q and cached k, times 1/√dim;
// * Softmax: two rows by the closed pair form, 3–8 rows by its fixed trees,
//   more rows by one running sum in row order; weights = e·(1/sum);
// * out[d] = p0·v0[d], then out[d] += p_t·v_t[d] in row order.
// One workgroup per q head; the previous kernel (the split attention) has
// appended this step's rotated K/V row.  Scores live in LDS (len floats, at
// most kOrdMaxRows).

// One q head over len ≥ 2 cache rows in that order; the whole workgroup
// calls it.  qs (LDS) holds the rotated q, kc / vc point at the KV head's
// columns of row 0 (row stride kvd), sc is LDS of len floats.
__device__ __forceinline__ void attn_ordered_head(const float *qs, const float *kc, const float *vc, size_t kvd,
                                                  int len, float scale, float *out, float *sc, float *red,
                                                  float *s_inv) {
#pragma clang fp contract(off)
    for (int t = threadIdx.x; t < len; t += kThreads) {
        const float *k = kc + (size_t)t * kvd;
        float s[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        for (int i = 0; i < 128; i += 8) {
            const float4 k0 = *reinterpret_cast<const float4 *>(k + i);
            const float4 k1 = *reinterpret_cast<const float4 *>(k + i + 4);
            s[0] = s[0] + qs[i] * k0.x;
            s[1] = s[1] + qs[i + 1] * k0.y;
            s[2] = s[2] + qs[i + 2] * k0.z;
            s[3] = s[3] + qs[i + 3] * k0.w;
            s[4] = s[4] + qs[i + 4] * k1.x;
            s[5] = s[5] + qs[i + 5] * k1.y;
            s[6] = s[6] + qs[i + 6] * k1.z;
            s[7] = s[7] + qs[i + 7] * k1.w;
        }
        sc[t] = (((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]))) * scale;
    }
    __syncthreads();
    // the maximum (order-free)
    float mx = -INFINITY;
    for (int t = threadIdx.x; t < len; t += kThreads) mx = fmaxf(mx, sc[t]);
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) m = fmaxf(m, red[w]);
    if (len == 2) {
        if (threadIdx.x == 0) {
            const float x0 = sc[0], x1 = sc[1];
            const float e = x0 >= x1 ? fast_exp_wrap(x1 - x0) : fast_exp_wrap(x0 - x1);
            const float inv = 1.0f / (1.0f + e);
            sc[0] = x0 >= x1 ? inv : e * inv;
            sc[1] = x0 >= x1 ? e * inv : inv;
        }
    } else {
        for (int t = threadIdx.x; t < len; t += kThreads) sc[t] = fast_exp_wrap(sc[t] - m);
        __syncthreads();
        if (threadIdx.x == 0) {
            float sum;
            if (len <= 8) {
                sum = sc[0] + sc[1];
                if (len == 3) sum = sum + sc[2];
                if (len >= 4) sum = sum + (sc[2] + sc[3]);
                if (len == 5) sum = sum + sc[4];
                if (len >= 6) sum = sum + (sc[4] + sc[5]);
                if (len == 7) sum = sum + sc[6];
                if (len == 8) sum = sum + (sc[6] + sc[7]);
            } else {  // one running sum in row order, 16 reads in flight
                sum = 0.0f;
                int t = 0;
                for (; t + 16 <= len; t += 16) {
                    float v[16];
#pragma unroll
                    for (int k = 0; k < 16; ++k) v[k] = sc[t + k];
#pragma unroll
                    for (int k = 0; k < 16; ++k) sum = sum + v[k];
                }
                for (; t < len; ++t) sum = sum + sc[t];
            }
            *s_inv = 1.0f / sum;
        }
        __syncthreads();
        const float inv = *s_inv;
        for (int t = threadIdx.x; t < len; t += kThreads) sc[t] = sc[t] * inv;
    }
    __syncthreads();
    if (threadIdx.x < 128) {
        const int d = threadIdx.x;
        float acc = sc[0] * vc[d];
        int t = 1;
        for (; t + 32 <= len; t += 32) {  // 32 value rows in flight, added in row order
            float v[32];
#pragma unroll
            for (int k = 0; k < 32; ++k) v[k] = vc[(size_t)(t + k) * kvd + d];
#pragma unroll
            for (int k = 0; k < 32; ++k) acc = acc + sc[t + k] * v[k];
        }
        for (; t < len; ++t) acc = acc + sc[t] * vc[(size_t)t * kvd + d];
        out[d] = acc;
    }
}

static __global__ void __launch_bounds__(kThreads) k_attn_ordered(AttnParams a) {
#pragma clang fp contract(off)
    const StepState *st = a.st;
    if (st->err) return;
    extern __shared__ float sc[];
    __shared__ float qs[128];
    __shared__ float red[kWaves];
    __shared__ float s_inv;
    const int len = st->len;
    const int h = blockIdx.x, kvh = h / (a.heads / a.kvh);
    const size_t kvd = (size_t)a.kvh * 128;
    const float *kc = a.kc + (size_t)kvh * 128, *vc = a.vc + (size_t)kvh * 128;
    float *out = a.head_out + (size_t)h * 128;
    if (len == 1) {  // attendHead's single row: V itself
        if (threadIdx.x < 128) out[threadIdx.x] = vc[threadIdx.x];
        return;
    }
    if (threadIdx.x < 64) {  // applyRoPE's pairs (i, 64 + i)
        const int i = threadIdx.x;
        const float q0 = a.q[(size_t)h * 128 + i], q1 = a.q[(size_t)h * 128 + 64 + i];
        if (st->has_rope) {
            const float cs = st->cos_t[i], sn = st->sin_t[i];
            qs[i] = q0 * cs - q1 * sn;
            qs[64 + i] = q1 * cs + q0 * sn;
        } else {
            qs[i] = q0;
            qs[64 + i] = q1;
        }
    }
    __syncthreads();
    attn_ordered_head(qs, kc, vc, kvd, len, a.scale, out, sc, red, &s_inv);
}

// The same for the rows of a batched prompt.  Workgroup (KV head g, head
// group hg, token i) takes HPW q heads of g's group for token i over cache rows
// [0, len), len = clen0 + i + 1, with token i's q already rotated in the qkv
// rows (k_rope_append, the token step's pair formula).  Each K and V row is
// read once for the HPW heads; every (head, token) result is formed exactly as
// attn_ordered_head forms it:
// * score t: dotF32's eight running sums over the dims in order (s_k over
//   dims ≡ k mod 8), the tree, times the scale;
// * the maximum (order-free), FastExp of s − max (the wrapped form), the pair
//   form for two rows; Σ by the fixed trees up to 8 rows, else one running
//   sum in row order (one thread per head); weights e·(1/Σ);
// * out[d] = p0·v0[d], then + p_t·v_t[d] in row order (one chain per head and
//   dim; a thread keeps HPW/2 chains of one dim, one V load for all of them).
// LDS: the HPW rotated q rows and HPW·len scores (dynamic).
template <int HPW>
static __global__ void __launch_bounds__(kThreads) k_attn_ordered_rows(const float *qkv, int stride, const float *kc,
                                                                       const float *vc, int heads, int kvh, int clen0,
                                                                       float scale, float *out, int out_stride) {
#pragma clang fp contract(off)
    static_assert(HPW == 1 || HPW == 2 || HPW == 4 || HPW == 8, "q heads per workgroup");
    extern __shared__ float sc_all[];
    __shared__ float qs[HPW][128];
    __shared__ float red[kWaves][HPW];
    __shared__ float s_inv[HPW];
    const int group = heads / kvh;
    const int ngrp = group / HPW;
    const int g = blockIdx.x / ngrp, h0 = g * group + (blockIdx.x % ngrp) * HPW;
    const int i = blockIdx.y;
    const int len = clen0 + i + 1;
    const size_t kvd = (size_t)kvh * 128;
    const float *kh = kc + (size_t)g * 128, *vh = vc + (size_t)g * 128;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (len == 1) {  // attendHead's single row: V itself
        for (int e = tid; e < HPW * 128; e += kThreads)
            out[(size_t)i * out_stride + (size_t)(h0 + e / 128) * 128 + e % 128] = vh[e % 128];
        return;
    }
    for (int e = tid; e < HPW * 128; e += kThreads)
        qs[e / 128][e % 128] = qkv[(size_t)i * stride + (size_t)(h0 + e / 128) * 128 + e % 128];
    __syncthreads();
    // scores: thread → rows t, the row's dims 8 at a time for all HPW heads
    for (int t = tid; t < len; t += kThreads) {
        const float *k = kh + (size_t)t * kvd;
        float s[HPW][8];
#pragma unroll
        for (int h = 0; h < HPW; ++h)
#pragma unroll
            for (int c = 0; c < 8; ++c) s[h][c] = 0.0f;
        for (int d = 0; d < 128; d += 8) {
            const float4 k0 = *reinterpret_cast<const float4 *>(k + d);
            const float4 k1 = *reinterpret_cast<const float4 *>(k + d + 4);
            const float kv[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
#pragma unroll
            for (int h = 0; h < HPW; ++h)
#pragma unroll
                for (int c = 0; c < 8; ++c) s[h][c] = s[h][c] + qs[h][d + c] * kv[c];
        }
#pragma unroll
        for (int h = 0; h < HPW; ++h)
            sc_all[(size_t)h * len + t] =
                (((s[h][0] + s[h][1]) + (s[h][2] + s[h][3])) + ((s[h][4] + s[h][5]) + (s[h][6] + s[h][7]))) * scale;
    }
    __syncthreads();
    // the maxima (order-free)
    {
        float mx[HPW];
#pragma unroll
        for (int h = 0; h < HPW; ++h) {
            mx[h] = -INFINITY;
            for (int t = tid; t < len; t += kThreads) mx[h] = fmaxf(mx[h], sc_all[(size_t)h * len + t]);
            mx[h] = wave_max(mx[h]);
        }
        if (lane == 0) {
#pragma unroll
            for (int h = 0; h < HPW; ++h) red[wave][h] = mx[h];
        }
    }
    __syncthreads();
    if (len == 2) {
        if (tid < HPW) {
            float *sc = sc_all + (size_t)tid * len;
            const float x0 = sc[0], x1 = sc[1];
            const float e = x0 >= x1 ? fast_exp_wrap(x1 - x0) : fast_exp_wrap(x0 - x1);
            const float inv = 1.0f / (1.0f + e);
            sc[0] = x0 >= x1 ? inv : e * inv;
            sc[1] = x0 >= x1 ? e * inv : inv;
        }
    } else {
        float m[HPW];
#pragma unroll
        for (int h = 0; h < HPW; ++h) {
            m[h] = red[0][h];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) m[h] = fmaxf(m[h], red[w][h]);
        }
#pragma unroll
        for (int h = 0; h < HPW; ++h)
            for (int t = tid; t < len; t += kThreads) {
                float *e = sc_all + (size_t)h * len + t;
                *e = fast_exp_wrap(*e - m[h]);
            }
        __syncthreads();
        if (tid < HPW) {  // thread h: head h's sum, in Softmax's order
            const float *sc = sc_all + (size_t)tid * len;
            float sum;
            if (len <= 8) {
                sum = sc[0] + sc[1];
                if (len == 3) sum = sum + sc[2];
                if (len >= 4) sum = sum + (sc[2] + sc[3]);
                if (len == 5) sum = sum + sc[4];
                if (len >= 6) sum = sum + (sc[4] + sc[5]);
                if (len == 7) sum = sum + sc[6];
                if (len == 8) sum = sum + (sc[6] + sc[7]);
            } else {
                sum = 0.0f;
                int t = 0;
                for (; t + 16 <= len; t += 16) {
                    float v[16];
#pragma unroll
                    for (int k = 0; k < 16; ++k) v[k] = sc[t + k];
#pragma unroll
                    for (int k = 0; k < 16; ++k) sum = sum + v[k];
                }
                for (; t < len; ++t) sum = sum + sc[t];
            }
            s_inv[tid] = 1.0f / sum;
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < HPW; ++h) {
            const float inv = s_inv[h];
            for (int t = tid; t < len; t += kThreads) {
                float *e = sc_all + (size_t)h * len + t;
                *e = *e * inv;
            }
        }
    }
    __syncthreads();
    // Σ p·V: thread (dim d, half hf) keeps the chains of heads hf, hf + 2, …
    constexpr int CH = HPW >= 2 ? HPW / 2 : 1;
    const int d = tid & 127, hf = tid >> 7;
    if (HPW >= 2 || hf == 0) {
        float acc[CH];
        const float v0 = vh[d];
#pragma unroll
        for (int c = 0; c < CH; ++c) acc[c] = sc_all[(size_t)(hf + 2 * c) * len] * v0;
        int t = 1;
        for (; t + 32 <= len; t += 32) {  // 32 value rows in flight, added in row order
            float v[32];
#pragma unroll
            for (int k = 0; k < 32; ++k) v[k] = vh[(size_t)(t + k) * kvd + d];
#pragma unroll
            for (int k = 0; k < 32; ++k)
#pragma unroll
                for (int c = 0; c < CH; ++c) acc[c] = acc[c] + sc_all[(size_t)(hf + 2 * c) * len + t + k] * v[k];
        }
        for (; t < len; ++t) {
            const float v = vh[(size_t)t * kvd + d];
#pragma unroll
            for (int c = 0; c < CH; ++c) acc[c] = acc[c] + sc_all[(size_t)(hf + 2 * c) * len + t] * v;
        }
#pragma unroll
        for (int c = 0; c < CH; ++c) out[(size_t)i * out_stride + (size_t)(h0 + hf + 2 * c) * 128 + d] = acc[c];
    }
}

}  // namespace pocr
