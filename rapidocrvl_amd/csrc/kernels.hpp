// kernels.hpp — gfx950 HIP kernels of the ERNIE text-decoder step.
//
// Weights stay in the GGUF Q*_ROW row layout (internal/gguf/gguf.go:446-558):
// per tensor an f32 scale per row and the packed rows, row-major.  One
// wavefront streams LPR×16-byte chunks of a row with coalesced 128-bit (Q6:
// 96-bit) loads, decodes the codes in registers against an activation slice it
// keeps in VGPRs for all rows, and reduces the row across its LPR lanes with
// DPP/swizzle shuffles.  Row r's result is (Σ code·x)·scale[r], the plain
// fp32-activation semantics of MatVecQ{8,4,6} (internal/tensor/quant.go:443-561).
#pragma once

#include <cstddef>

#include <hip/hip_runtime.h>
#include <type_traits>
#include <stdint.h>

namespace pocr {

enum : int { QT_Q8 = 1000, QT_Q4 = 1001, QT_Q6 = 1002 };

constexpr int kThreads = 256;  // 4 wavefronts per workgroup
constexpr int kWaves = kThreads / 64;
constexpr int kMaxHalf = 128;  // head_dim/2 upper bound for RoPE tables
constexpr int kMaxCols = 4096; // widest input of the streaming GEMV kernel

struct DevMat {
    const float *scale;    // [rows]
    const uint8_t *data;   // rows * row_bytes, 256-byte aligned base
    const uint8_t *tiled;  // the same bytes in the prefill GEMM's operand order (k_tile_weight), or null
    const int *usum;       // Q4/Q6 with a tile image: Σ of the row's stored codes (k_row_usum), else null
    const uint8_t *head_img;  // Q6 LM-head-sized rows in the greedy head's load order (k_head_image_q6), or null
    int rows;
    int cols;
    int row_bytes;
    int qtype;
};

// Per-sequence step state kept in HBM so one captured graph can be replayed
// token after token.
constexpr int kArgSlots = 64;
constexpr int kSlotPitch = 16;  // u64 per slot: 128 bytes
constexpr int kMaxEos = 16;     // EOS ids held in the step state itself
constexpr int kMaxEosIds = 1024;  // maxEOSTokenIDs (internal/model/model.go:432)
// err value of a decode loop that took an EOS token: not a failure, but like
// one every later kernel of the sequence returns at once (nothing appended)
constexpr int kErrStopped = -1;

struct StepState {
    int32_t len;       // cache rows after this step's append
    int32_t clen;      // cache rows before the append (= token index)
    int32_t cap;       // cache capacity
    int32_t err;       // nonzero → every kernel returns immediately
    int32_t pos[3];    // (T,H,W) position of this token
    int32_t next_pos;  // decode position counter
    int32_t n_out;     // tokens emitted by the device decode loop
    int32_t has_rope;
    int32_t half;
    int32_t n_eos;     // decode loop: a taken token equal to eos[i < n_eos] stops it
    int32_t eos[kMaxEos];
    // longer lists: bit t of this vocabulary bitmap set ⇔ token t is an EOS
    // id (the sequence's own buffer; null when the list fits eos[])
    const uint32_t *eos_bits;
    alignas(16) float cos_t[kMaxHalf];
    float sin_t[kMaxHalf];
    // greedy argmax: workgroup b of the LM head folds its best (score, row)
    // key into slot b % kArgSlots with atomicMax; slots sit one 128-byte line
    // apart so the atomics spread over memory channels.  The consumer takes
    // the max over the slots (0 = no candidate).
    alignas(128) unsigned long long argmax_slot[kArgSlots * kSlotPitch];
};
// kernels read len, clen, cap and err as one 16-byte load
static_assert(offsetof(StepState, len) == 0 && offsetof(StepState, clen) == 4 && offsetof(StepState, err) == 12,
              "step state header layout");
static_assert(offsetof(StepState, eos) % 16 == 0 && kMaxEos % 4 == 0, "the step prologue reads eos[] as int4");
static_assert(kMaxHalf <= kThreads && kArgSlots <= 64, "the step prologue: one table entry per thread, slots in wave 0");

// ---------------------------------------------------------------------------
// reference numerics (internal/tensor/ops.go)
// ---------------------------------------------------------------------------

// FastExpF32 exactly as the reference computes it (ops.go:1099-1112),
// including the exponent add that wraps below about −88.7 (the result's bits
// then carry into the sign: −90 gives −9.5e37). Pointwise uses (SiLU,
// low-temperature draws, the reference-order softmax of the VNNI mode) take
// this form so their results equal the reference's there too.
__device__ __forceinline__ float fast_exp_wrap(float x) {
#pragma clang fp contract(off)
    const float log2e = 1.4426950408889634f;
    const float magic = 12582912.0f;
    const float t = x * log2e;
    const int32_t n = (int32_t)((t + magic) - magic);
    const float f = t - (float)n;
    const float f2 = f * f;
    const float poly = (1.0f + 0.6931471824645996f * f) +
                       f2 * (0.24022650718688965f + 0.05550410971045494f * f +
                             f2 * (0.009618128649890423f + 0.0013352063251659274f * f));
    return __uint_as_float(__float_as_uint(poly) + ((uint32_t)n << 23));
}

// FastExpF32 with its input clamped at −87, where exp() is below FLT_MIN.
// The split softmaxes (decode and prefill attention, their merges) take this
// form: they rescale partial sums by exp(m_split − m) terms that the
// reference's one-pass softmax never forms, so no choice of theirs could
// reproduce its wrapped weights for score gaps beyond 88; the clamp keeps
// those rows at weight ≈ 0, the mathematical softmax.
__device__ __forceinline__ float fast_exp_ref(float x) {
#pragma clang fp contract(off)
    x = fmaxf(x, -87.0f);
    const float log2e = 1.4426950408889634f;
    const float magic = 12582912.0f;
    float t = x * log2e;
    int32_t n = (int32_t)((t + magic) - magic);
    float f = t - (float)n;
    float f2 = f * f;
    float poly = (1.0f + 0.6931471824645996f * f) +
                 f2 * (0.24022650718688965f + 0.05550410971045494f * f +
                       f2 * (0.009618128649890423f + 0.0013352063251659274f * f));
    return __uint_as_float(__float_as_uint(poly) + ((uint32_t)n << 23));
}

// fastRsqrtF32 (ops.go:1374-1381)
__device__ __forceinline__ float fast_rsqrt_ref(float x) {
#pragma clang fp contract(off)
    float half = x * 0.5f;
    float y = __uint_as_float(0x5f3759dfu - (__float_as_uint(x) >> 1));
    y = y * (1.5f - half * y * y);
    return y * (1.5f - half * y * y);
}

// SiLU (ops.go:1092-1094), FastExp's wrap included: a gate above ≈ 88.7
// gives x / (1 + (negative huge)) ≈ −0, as in the reference
__device__ __forceinline__ float silu_ref(float x) {
#pragma clang fp contract(off)
    return x / (1.0f + fast_exp_wrap(-x));
}

// fastExpF32T (ops.go:1152-1164): 2^x for x already scaled by log2(e); the
// exponent add wraps outside about ±127 exactly as in the reference
__device__ __forceinline__ float fast_exp2_wrap(float x) {
#pragma clang fp contract(off)
    const float magic = 12582912.0f;
    const int32_t n = (int32_t)((x + magic) - magic);
    const float f = x - (float)n;
    const float f2 = f * f;
    const float poly = (1.0f + 0.6931471824645996f * f) +
                       f2 * (0.24022650718688965f + 0.05550410971045494f * f +
                             f2 * (0.009618128649890423f + 0.0013352063251659274f * f));
    return __uint_as_float(__float_as_uint(poly) + ((uint32_t)n << 23));
}

// GELUTanh (ops.go:1140-1150): 0.5·x·(1 + tanh(√(2/π)(x + 0.044715x³))) with
// tanh = (e−1)/(e+1), e = 2^(x·2c·log2e + x³·2ck·log2e); the two constants
// are the reference's exact products rounded once to f32
__device__ __forceinline__ float gelu_tanh_ref(float x) {
#pragma clang fp contract(off)
    const float c1 = 0x1.26aec2p+1f;  // 2·0.7978845608028654·1.4426950408889634
    const float c3 = 0x1.a5a7dp-4f;   // 2·0.7978845608028654·0.044715·1.4426950408889634
    const float x3 = x * (x * x);
    const float e = fast_exp2_wrap(c1 * x + c3 * x3);
    const float th = (e - 1.0f) / (e + 1.0f);
    return 0.5f * x * (1.0f + th);
}

// ---------------------------------------------------------------------------
// code decode: chunk of packed bytes → Σ u·x with unsigned codes u; the signed
// value is u − BIAS, folded as −BIAS·Σx once per lane.
// ---------------------------------------------------------------------------
template <int QT> struct QTraits;
template <> struct QTraits<QT_Q4> {  // 16 B = 32 nibbles, value = nib − 8 (quant.go:2356)
    static constexpr int CB = 16, W = 32;
    static constexpr float BIAS = 8.0f;
};
template <> struct QTraits<QT_Q8> {  // 16 B = 16 int8; u = b ^ 0x80 = b + 128
    static constexpr int CB = 16, W = 16;
    static constexpr float BIAS = 128.0f;
};
template <> struct QTraits<QT_Q6> {  // 12 B = 16 six-bit codes, value = code − 32 (quant.go:2592)
    static constexpr int CB = 12, W = 16;
    static constexpr float BIAS = 32.0f;
};

struct Chunk {
    uint32_t d[4];
};

typedef int v4i __attribute__((ext_vector_type(4)));

// Within each 16-column group the K order of an int8 MFMA is a permutation
// shared by the weights and the activation digits: Q4 puts the group's even
// columns first (the low nibbles of its 8 packed bytes), then the odd ones;
// Q8/Q6 keep the natural order.
template <int QT>
__host__ __device__ constexpr int digit_pos16(int c) {
    return QT == QT_Q4 ? ((c & 1) ? 8 + (c >> 1) : (c >> 1)) : c;
}

// Weights stream once per launch: non-temporal loads (global_load … nt).
template <int QT>
__device__ __forceinline__ Chunk load_chunk(const uint8_t *p) {
    Chunk c;
    if constexpr (QT == QT_Q6) {
        const uint32_t *q = reinterpret_cast<const uint32_t *>(p);  // 4-byte aligned 12-byte chunk
        c.d[0] = __builtin_nontemporal_load(q);
        c.d[1] = __builtin_nontemporal_load(q + 1);
        c.d[2] = __builtin_nontemporal_load(q + 2);
        c.d[3] = 0;
    } else {
        typedef unsigned u4v __attribute__((ext_vector_type(4)));
        const u4v v = __builtin_nontemporal_load(reinterpret_cast<const u4v *>(p));
        c.d[0] = v[0];
        c.d[1] = v[1];
        c.d[2] = v[2];
        c.d[3] = v[3];
    }
    return c;
}

// v_cvt_f32_ubyte{0..3}: one VALU op per code (the compiler otherwise emits a
// bit-field extract before each convert once it knows the bytes are nibbles)
__device__ __forceinline__ float ubyte(uint32_t v, int i) {
    float r;
    switch (i) {
    case 0: asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v)); break;
    case 1: asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v)); break;
    case 2: asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v)); break;
    default: asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v)); break;
    }
    return r;
}

template <int QT>
__device__ __forceinline__ float chunk_dot(const Chunk &c, const float *x) {
    float a0 = 0.0f, a1 = 0.0f;
    if constexpr (QT == QT_Q4) {
        // byte j holds col 2j (low nibble) and col 2j+1 (high nibble) (quant.go:322-353)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t lo = c.d[k] & 0x0F0F0F0Fu;
            uint32_t hi = (c.d[k] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                a0 = fmaf(ubyte(lo, m), x[8 * k + 2 * m], a0);
                a1 = fmaf(ubyte(hi, m), x[8 * k + 2 * m + 1], a1);
            }
        }
    } else if constexpr (QT == QT_Q8) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t u = c.d[k] ^ 0x80808080u;
            a0 = fmaf(ubyte(u, 0), x[4 * k + 0], a0);
            a1 = fmaf(ubyte(u, 1), x[4 * k + 1], a1);
            a0 = fmaf(ubyte(u, 2), x[4 * k + 2], a0);
            a1 = fmaf(ubyte(u, 3), x[4 * k + 3], a1);
        }
    } else {
        // little-endian 6-bit stream, col i at bits [6i, 6i+6) (quant.go:2886-2906)
        const uint32_t d0 = c.d[0], d1 = c.d[1], d2 = c.d[2];
        uint32_t u[16];
#pragma unroll
        for (int i = 0; i < 5; ++i) u[i] = __builtin_amdgcn_ubfe(d0, 6 * i, 6);
        u[5] = __builtin_amdgcn_alignbit(d1, d0, 30) & 63u;
#pragma unroll
        for (int i = 6; i < 10; ++i) u[i] = __builtin_amdgcn_ubfe(d1, 6 * i - 32, 6);
        u[10] = __builtin_amdgcn_alignbit(d2, d1, 28) & 63u;
#pragma unroll
        for (int i = 11; i < 16; ++i) u[i] = __builtin_amdgcn_ubfe(d2, 6 * i - 64, 6);
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            a0 = fmaf((float)u[i], x[i], a0);
            a1 = fmaf((float)u[i + 1], x[i + 1], a1);
        }
    }
    return a0 + a1;
}

template <int LPR>
__device__ __forceinline__ float lane_group_sum(float v) {
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// ---------------------------------------------------------------------------
// Integer inner product.  Each lane turns its activation slice once into
// three int8 digit planes: with S a power of two ≥ max|x|/127,
//   x = S·(d0 + d1/2^7 + d2/2^14) + e,  |e| ≤ S/2^15  (≈ 2^-22·max|x|),
// d0 ∈ [-127,127], d1,d2 ∈ [-64,64].  A row's dot product is then three exact
// int32 accumulations of v_dot4 (4 code×digit products per instruction),
// combined to f32 once per row.  Unsigned codes (Q4 nibble, Q6 field) are
// fed as their raw value u and the offset is removed exactly as
// BIAS·Σd_k per digit plane.
// ---------------------------------------------------------------------------
template <int QT>
struct DigitTraits {
    static constexpr int NDW = QT == QT_Q4 ? 8 : 4;  // digit dwords per chunk
    static constexpr int IBIAS = QT == QT_Q4 ? 8 : (QT == QT_Q6 ? 32 : 0);
};

__device__ __forceinline__ int pack4(int a, int b, int c, int d) {
    return (a & 0xFF) | ((b & 0xFF) << 8) | ((c & 0xFF) << 16) | ((d & 0xFF) << 24);
}

template <int QT, int CPL>
struct XDigits {
    int d[CPL][DigitTraits<QT>::NDW][3];
    int bias[CPL][3];
    float scale[CPL];
    // Q4: the planes' int32 sums are combined in integer before one convert
    // (bias and scale of the combination below)
    int bias_comb[CPL];
    float scale_comb[CPL];
};

template <int QT, int CPL, int NPL>
using XDig = XDigits<QT, CPL>;

// column (within a chunk) of byte m of digit dword k: Q4 dword 2k' holds the
// low nibbles of chunk dword k' (cols 8k'+0,2,4,6), dword 2k'+1 the high ones
// (cols 8k'+1,3,5,7); Q8/Q6 dword k holds cols 4k..4k+3.
template <int QT>
__device__ __forceinline__ int digit_col(int k, int m) {
    if constexpr (QT == QT_Q4) return 8 * (k >> 1) + 2 * m + (k & 1);
    else return 4 * k + m;
}

// LDS layout after the activation prologue: one record of RS ints per chunk
// c (W columns): its digit dwords dig[k][plane] (k < NDW, plane < 3), then
// the three bias sums IBIAS·Σd of the planes, then the chunk scale (a power
// of two ≥ max|x|/127 over the chunk's columns, as float bits).  RS·4 is a
// multiple of 16, so a lane reads its records with 16-byte LDS loads.
template <int QT>
struct DigitRec {
    static constexpr int NDW = DigitTraits<QT>::NDW;
    static constexpr int RS = NDW * 3 + 4;
    static constexpr int TPC = QTraits<QT>::W / 8;  // prologue threads per chunk (8 columns each)
    static_assert((RS * 4) % 16 == 0, "record must be 16-byte aligned");
};
template <int QT>
__host__ __device__ constexpr size_t gemv_lds_bytes(int cols) {
    return (size_t)(cols / QTraits<QT>::W) * DigitRec<QT>::RS * 4;
}

// code4 · digits of the first NPL planes (NPL = 3: x to 2^-15 of the chunk
// scale; NPL = 2: to 2^-8)
template <int NPL>
__device__ __forceinline__ void dotp(int code4, const int (&x)[3], int (&a)[3]) {
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl) a[pl] = __builtin_amdgcn_sdot4(code4, x[pl], a[pl], false);
}

// six-bit fields of one 24-bit group spread into the four bytes of a dword
__device__ __forceinline__ int spread6(uint32_t g) {
    // fields 0-1 stay in bits 0-11, fields 2-3 move to bits 16-27; then each
    // 12-bit pair splits into two bytes
    const uint32_t t = (g & 0xFFFu) | ((g << 4) & 0xFFF0000u);
    return (int)((t & 0x3F003Fu) | ((t << 2) & 0x3F003F00u));
}

template <int QT, int CPL, int NPL = 3>
__device__ __forceinline__ float row_dot_bytes(const Chunk (&w)[CPL], const XDigits<QT, CPL> &xd) {
    float r = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        int a[3] = {0, 0, 0};
        if constexpr (QT == QT_Q8) {
#pragma unroll
            for (int k = 0; k < 4; ++k) dotp<NPL>((int)w[j].d[k], xd.d[j][k], a);
        } else if constexpr (QT == QT_Q4) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                dotp<NPL>((int)(w[j].d[k] & 0x0F0F0F0Fu), xd.d[j][2 * k], a);
                dotp<NPL>((int)((w[j].d[k] >> 4) & 0x0F0F0F0Fu), xd.d[j][2 * k + 1], a);
            }
        } else {
            const uint32_t d0 = w[j].d[0], d1 = w[j].d[1], d2 = w[j].d[2];
            dotp<NPL>(spread6(d0), xd.d[j][0], a);
            dotp<NPL>(spread6(__builtin_amdgcn_alignbit(d1, d0, 24)), xd.d[j][1], a);
            dotp<NPL>(spread6(__builtin_amdgcn_alignbit(d2, d1, 16)), xd.d[j][2], a);
            dotp<NPL>(spread6(d2 >> 8), xd.d[j][3], a);
        }
        if constexpr (QT == QT_Q4) {
            // |a0| ≤ 32·15·127 < 2^16: a0·2^14 + a1·2^7 + a2 stays inside int32
            const int comb = NPL == 3 ? a[0] * 16384 + a[1] * 128 + a[2] : a[0] * 128 + a[1];
            r = fmaf(xd.scale_comb[j], (float)(comb - xd.bias_comb[j]), r);
        } else {
            const float f0 = (float)(a[0] - xd.bias[j][0]);
            const float f1 = (float)(a[1] - xd.bias[j][1]);
            const float f = NPL == 3 ? fmaf((float)(a[2] - xd.bias[j][2]), 1.0f / 16384.0f, fmaf(f1, 1.0f / 128.0f, f0))
                                     : fmaf(f1, 1.0f / 128.0f, f0);
            r = fmaf(xd.scale[j], f, r);
        }
    }
    return r;
}

template <int QT, int CPL, int NPL = 3>
__device__ __forceinline__ float row_dot(const Chunk (&w)[CPL], const XDig<QT, CPL, NPL> &xd) {
    return row_dot_bytes<QT, CPL, NPL>(w, xd);
}

// Cross-lane exchanges used by the reduce-scatter.  Each pairs every lane with
// a partner that differs in one chosen lane bit (and agrees on all higher
// ones): xor 32, xor 16 (ds_swizzle), mirror within 16 (DPP row_mirror,
// bit 3), mirror within 8 (DPP row_half_mirror, bit 2), xor 2 and xor 1 (DPP
// quad_perm).
enum : int { XS32 = 0, XS16 = 1, XM16 = 2, XM8 = 3, XQ2 = 4, XQ1 = 5 };
template <int S>
__device__ __forceinline__ float xchg(float v) {
    const int i = __float_as_int(v);
    if constexpr (S == XS32) return __shfl_xor(v, 32, 64);
    else if constexpr (S == XS16) return __int_as_float(__builtin_amdgcn_ds_swizzle(i, 0x401F));
    else if constexpr (S == XM16) return __int_as_float(__builtin_amdgcn_update_dpp(0, i, 0x140, 0xF, 0xF, false));
    else if constexpr (S == XM8) return __int_as_float(__builtin_amdgcn_update_dpp(0, i, 0x141, 0xF, 0xF, false));
    else if constexpr (S == XQ2) return __int_as_float(__builtin_amdgcn_update_dpp(0, i, 0x4E, 0xF, 0xF, false));
    else return __int_as_float(__builtin_amdgcn_update_dpp(0, i, 0xB1, 0xF, 0xF, false));
}

// One reduce-scatter step over N entries of NM floats: lanes whose step bit
// is set keep the upper half (and receive it from the partner); with one
// entry left the step is a butterfly add.
template <int N, int NM, int S, int BIT, int CAP>
__device__ __forceinline__ void rs_step(float (&v)[CAP][NM], int lane) {
    if constexpr (N > 1) {
        const bool hi = (lane & BIT) != 0;
#pragma unroll
        for (int i = 0; i < N / 2; ++i)
#pragma unroll
            for (int k = 0; k < NM; ++k) {
                const float keep = hi ? v[N / 2 + i][k] : v[i][k];
                const float send = hi ? v[i][k] : v[N / 2 + i][k];
                v[i][k] = keep + xchg<S>(send);
            }
    } else {
#pragma unroll
        for (int k = 0; k < NM; ++k) v[0][k] += xchg<S>(v[0][k]);
    }
}

// Sums U entries (of NM floats) over the LPR lanes of a row group.  Lane
// u·(LPR/U) ends up with the full sum of entry u in v[0].
template <int LPR, int U, int NM, int CAP>
__device__ __forceinline__ void reduce_scatter(float (&v)[CAP][NM], int lane) {
    static_assert(U <= CAP && U <= LPR, "entries exceed the array or the lanes");
    constexpr int N1 = U, N2 = N1 > 1 ? N1 / 2 : 1, N3 = N2 > 1 ? N2 / 2 : 1, N4 = N3 > 1 ? N3 / 2 : 1;
    if constexpr (LPR == 64) {
        constexpr int N5 = N4 > 1 ? N4 / 2 : 1, N6 = N5 > 1 ? N5 / 2 : 1;
        rs_step<N1, NM, XS32, 32>(v, lane);
        rs_step<N2, NM, XS16, 16>(v, lane);
        rs_step<N3, NM, XM16, 8>(v, lane);
        rs_step<N4, NM, XM8, 4>(v, lane);
        rs_step<N5, NM, XQ2, 2>(v, lane);
        rs_step<N6, NM, XQ1, 1>(v, lane);
    } else {
        constexpr int N5 = N4 > 1 ? N4 / 2 : 1;
        rs_step<N1, NM, XS16, 16>(v, lane);
        rs_step<N2, NM, XM16, 8>(v, lane);
        rs_step<N3, NM, XM8, 4>(v, lane);
        rs_step<N4, NM, XQ2, 2>(v, lane);
        rs_step<N5, NM, XQ1, 1>(v, lane);
    }
}

// Sum over the 64 lanes of a wave, the same value in every lane (DPP within
// rows of 16, then swizzle and bpermute across them).
// 64-bit lane exchange
__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long v, int m) {
    const unsigned lo = __shfl_xor((unsigned)v, m, 64);
    const unsigned hi = __shfl_xor((unsigned)(v >> 32), m, 64);
    return ((unsigned long long)hi << 32) | lo;
}

__device__ __forceinline__ float wave_sum(float v) {
    v += xchg<XQ1>(v);
    v += xchg<XQ2>(v);
    v += xchg<XM8>(v);
    v += xchg<XM16>(v);
    v += xchg<XS16>(v);
    v += xchg<XS32>(v);
    return v;
}

// Maximum over the 64 lanes of a wave, the same value in every lane.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, xchg<XQ1>(v));
    v = fmaxf(v, xchg<XQ2>(v));
    v = fmaxf(v, xchg<XM8>(v));
    v = fmaxf(v, xchg<XM16>(v));
    v = fmaxf(v, xchg<XS16>(v));
    v = fmaxf(v, xchg<XS32>(v));
    return v;
}


// ---------------------------------------------------------------------------
// Activation prologue.  Thread t owns 8 consecutive columns per pass (2048
// columns a pass); the TPC threads of a chunk are adjacent lanes.  Each turns
// its columns into its two digit dwords of the three planes and writes them
// to the chunk's LDS record; lane 0 of the chunk adds the bias sums and the
// scale.  Columns past cols are clamped loads, never written.
// ---------------------------------------------------------------------------
constexpr int kXPass = 8 * kThreads;              // columns per prologue pass
constexpr int kXPasses = kMaxCols / kXPass;       // 2

struct XRegs {
    float4 x[kXPasses][2];
    float4 w[kXPasses][2];
};

// Requests the activation (and RMSNorm weight) columns of this thread.
__device__ __forceinline__ void x_load(const float *x, const float *nw, bool norm, int cols, XRegs &r) {
#pragma unroll
    for (int pp = 0; pp < kXPasses; ++pp) {
        if (pp * kXPass >= cols) break;  // uniform
        const int cb = min((pp * kThreads + (int)threadIdx.x) * 8, cols - 8);
        const float4 *xp = reinterpret_cast<const float4 *>(x + cb);
        r.x[pp][0] = xp[0];
        r.x[pp][1] = xp[1];
        if (norm) {
            const float4 *wp = reinterpret_cast<const float4 *>(nw + cb);
            r.w[pp][0] = wp[0];
            r.w[pp][1] = wp[1];
        }
    }
}

// PRO_OPART's activation, staged through LDS: thread t sums 4 columns
// (4t..4t+3: every thread takes part, 1024 columns at most) of the residual
// and up to kMaxOparts partial rows, each added in row order; the loads are
// requested together (branch-free: rows past nparts re-read the last one and
// are not added).
constexpr int kMaxOparts = 16;
struct OpartRegs {
    float4 p[kMaxOparts];
    float4 h;
};
__device__ __forceinline__ void opart_issue(const float *part, int nparts, const float *resid, int cols,
                                            OpartRegs &r) {
    const int c = min(4 * (int)threadIdx.x, cols - 4);
#pragma unroll
    for (int k = 0; k < kMaxOparts; ++k)
        r.p[k] = *reinterpret_cast<const float4 *>(part + (size_t)min(k, nparts - 1) * cols + c);
    r.h = *reinterpret_cast<const float4 *>(resid + c);
}
// the sum into LDS (stage[cols]) and, for vbuf != null, into vbuf
__device__ __forceinline__ void opart_stage(const OpartRegs &r, int nparts, int cols, float *stage, float *vbuf) {
    float4 o = r.p[0];
#pragma unroll
    for (int k = 1; k < kMaxOparts; ++k)
        if (k < nparts)  // uniform
            o = make_float4(o.x + r.p[k].x, o.y + r.p[k].y, o.z + r.p[k].z, o.w + r.p[k].w);
    const float4 v = make_float4(r.h.x + o.x, r.h.y + o.y, r.h.z + o.z, r.h.w + o.w);
    const int c = 4 * (int)threadIdx.x;
    if (c < cols) {
        *reinterpret_cast<float4 *>(stage + c) = v;
        if (vbuf) *reinterpret_cast<float4 *>(vbuf + c) = v;
    }
}

// Digit planes of the thread's columns → LDS records, and the wave's Σx²
// into red[wave] (with the norm on, the digits encode x·w and the row sums
// are scaled by fastRsqrt(Σx²/n + eps) afterwards: x_norm_factor after the
// workgroup barrier).
template <int QT>
__device__ __forceinline__ void x_digits(const XRegs &r, const XRegs &rw, bool norm, int cols, int *lds, float *red) {
    constexpr int NDW = DigitRec<QT>::NDW, RS = DigitRec<QT>::RS, TPC = DigitRec<QT>::TPC;
    const int lane = threadIdx.x & 63;
    float ss = 0.0f;
#pragma unroll
    for (int pp = 0; pp < kXPasses; ++pp) {
        if (pp * kXPass >= cols) break;  // uniform
        const int G = pp * kThreads + (int)threadIdx.x;  // 8-column group
        const bool valid = G * 8 < cols;
        float y[8] = {r.x[pp][0].x, r.x[pp][0].y, r.x[pp][0].z, r.x[pp][0].w,
                      r.x[pp][1].x, r.x[pp][1].y, r.x[pp][1].z, r.x[pp][1].w};
        if (norm) {
            const float wv[8] = {rw.w[pp][0].x, rw.w[pp][0].y, rw.w[pp][0].z, rw.w[pp][0].w,
                                 rw.w[pp][1].x, rw.w[pp][1].y, rw.w[pp][1].z, rw.w[pp][1].w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                ss = valid ? fmaf(y[i], y[i], ss) : ss;
                y[i] = y[i] * wv[i];  // a lone product: nothing to contract
            }
        }
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(y[i]));
        m = fmaxf(m, xchg<XQ1>(m));
        if constexpr (TPC == 4) m = fmaxf(m, xchg<XQ2>(m));
        int ex = 0;
        (void)frexpf(m * (1.0f / 127.0f), &ex);  // m/127 < 2^ex; m = 0 → ex = 0
        int d0[8], d1[8], d2[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float t = ldexpf(y[i], -ex);  // exact (no overflow of 2^-ex for tiny chunks)
            const float a = rintf(t);
            const float t1 = (t - a) * 128.0f;
            const float b = rintf(t1);
            d0[i] = (int)a;
            d1[i] = (int)b;
            d2[i] = (int)rintf((t1 - b) * 128.0f);
        }
        // digit dwords: Q4 → even columns, then odd ones (low / high nibbles);
        // Q8/Q6 → columns 0..3, then 4..7
        int lo[3], hi[3];
        if constexpr (QT == QT_Q4) {
            lo[0] = pack4(d0[0], d0[2], d0[4], d0[6]);
            hi[0] = pack4(d0[1], d0[3], d0[5], d0[7]);
            lo[1] = pack4(d1[0], d1[2], d1[4], d1[6]);
            hi[1] = pack4(d1[1], d1[3], d1[5], d1[7]);
            lo[2] = pack4(d2[0], d2[2], d2[4], d2[6]);
            hi[2] = pack4(d2[1], d2[3], d2[5], d2[7]);
        } else {
            lo[0] = pack4(d0[0], d0[1], d0[2], d0[3]);
            hi[0] = pack4(d0[4], d0[5], d0[6], d0[7]);
            lo[1] = pack4(d1[0], d1[1], d1[2], d1[3]);
            hi[1] = pack4(d1[4], d1[5], d1[6], d1[7]);
            lo[2] = pack4(d2[0], d2[1], d2[2], d2[3]);
            hi[2] = pack4(d2[4], d2[5], d2[6], d2[7]);
        }
        float bs[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const int b2 = __builtin_amdgcn_sdot4(hi[k], 0x01010101, __builtin_amdgcn_sdot4(lo[k], 0x01010101, 0, false),
                                                  false);
            bs[k] = (float)b2;  // |Σ| ≤ 32·127: exact in f32
            bs[k] += xchg<XQ1>(bs[k]);
            if constexpr (TPC == 4) bs[k] += xchg<XQ2>(bs[k]);
        }
        if (valid) {
            const int c = G / TPC, q = G % TPC;
            int *rec = lds + c * RS;
            int2 *dp = reinterpret_cast<int2 *>(rec + 2 * q * 3);  // dwords 2q, 2q+1: 6 ints
            dp[0] = make_int2(lo[0], lo[1]);
            dp[1] = make_int2(lo[2], hi[0]);
            dp[2] = make_int2(hi[1], hi[2]);
            if (q == 0) {
                const float sc = m > 0.0f ? ldexpf(1.0f, ex) : 1.0f;
                *reinterpret_cast<int4 *>(rec + NDW * 3) =
                    make_int4(DigitTraits<QT>::IBIAS * (int)bs[0], DigitTraits<QT>::IBIAS * (int)bs[1],
                              DigitTraits<QT>::IBIAS * (int)bs[2], __float_as_int(sc));
            }
        }
    }
    if (norm) {
        ss = wave_sum(ss);
        if (lane == 0) red[threadIdx.x >> 6] = ss;
    }
}

// RMSNorm (ops.go:1015-1037): x·fastRsqrt(Σx²/n + eps)·w — the factor from
// the waves' Σx² (after the barrier that follows x_digits)
__device__ __forceinline__ float x_norm_factor(bool norm, int cols, float eps, const float *red) {
    if (!norm) return 1.0f;
    float tot = red[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) tot += red[w];
    return fast_rsqrt_ref(tot / (float)cols + eps);
}

// The lane's CPL chunk records (chunks l + j·LPR) → registers.
template <int QT, int LPR, int CPL, int NPL = 3>
__device__ __forceinline__ void load_digits(const int *lds, int l, XDig<QT, CPL, NPL> &xd) {
    constexpr int NDW = DigitRec<QT>::NDW, RS = DigitRec<QT>::RS;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int4 *rec = reinterpret_cast<const int4 *>(lds + (l + j * LPR) * RS);
        int v[RS];
#pragma unroll
        for (int i = 0; i < RS / 4; ++i) {
            const int4 t = rec[i];
            v[4 * i] = t.x;
            v[4 * i + 1] = t.y;
            v[4 * i + 2] = t.z;
            v[4 * i + 3] = t.w;
        }
#pragma unroll
        for (int k = 0; k < NDW; ++k)
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) xd.d[j][k][pl] = v[k * 3 + pl];
        xd.bias[j][0] = v[NDW * 3];
        xd.bias[j][1] = v[NDW * 3 + 1];
        xd.bias[j][2] = v[NDW * 3 + 2];
        xd.scale[j] = __int_as_float(v[NDW * 3 + 3]);
        if constexpr (NPL == 3) {
            xd.bias_comb[j] = xd.bias[j][0] * 16384 + xd.bias[j][1] * 128 + xd.bias[j][2];
            xd.scale_comb[j] = xd.scale[j] * (1.0f / 16384.0f);  // exact: powers of two
        } else {
            xd.bias_comb[j] = xd.bias[j][0] * 128 + xd.bias[j][1];
            xd.scale_comb[j] = xd.scale[j] * (1.0f / 128.0f);
        }
    }
}

// ---------------------------------------------------------------------------
// GEMV family
// ---------------------------------------------------------------------------
// PRO_OPART: x = residual + (((x[0·cols..] + x[1·cols..]) + …) + x[(flag−1)·cols..])
// (the o_proj partials of k_attn_merge_oproj), then RMSNorm as PRO_RMSNORM;
// workgroup 0 also writes that x (residual + attention) to vbuf, where the
// down GEMV (EPI_DOWNV) takes it as its residual when the o_proj runs in place.
enum : int { PRO_COPY = 0, PRO_RMSNORM = 1, PRO_OPART = 2 };
enum : int {
    EPI_PLAIN = 0,   // out[r] = s
    EPI_SWIGLU = 1,  // out[r] = SiLU(s_gate)·s_up            (NMAT = 2)
    EPI_OPROJ = 2,   // v = residual + s; vbuf = v; residual = v if in place
    EPI_DOWN = 3,    // residual += s, or vbuf = residual + s on the last layer
    EPI_ARGMAX = 4,  // greedy LM head (+ optional logits)
    EPI_ADDV = 5,    // vbuf = residual + s (op-level AddRMSNorm, norm in a 2nd kernel)
    EPI_DOWNV = 6,   // EPI_DOWN over residual = (o_proj in place ? vbuf : residual), after PRO_OPART
};

struct GemvParams {
    DevMat m[3];
    int seg_end[3];  // NMAT == 1: rows [seg_end[i-1], seg_end[i]) come from m[i]
    int rows;
    int cols;
    const float *x;
    const float *norm_w;
    float eps;
    float *out;
    float *residual;
    float *vbuf;
    StepState *st;  // may be null (op level)
    int flag;       // EPI_OPROJ: in-place when st==null; EPI_DOWN: last layer
    int quirk;      // EPI_OPROJ: Q4/Q6 residual behaviour on
};
// NV > 1 activation vectors (a separate kernel argument, so single-vector
// launches keep their argument block): vector v reads x + v·x_stride and
// writes out/residual/vbuf + v·o_stride; its step state is stv[v−1] (v ≥ 1)
struct GemvNV {
    int x_stride;
    int o_stride;
    StepState *stv[3];
};
constexpr int kMaxNV = 4;
constexpr int kMaxBatch = 16;  // sequences of one batched decode step

__device__ __forceinline__ unsigned long long argmax_key(float v, int row) {
    uint32_t b = __float_as_uint(v);
    uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)row);
}

// Block-wide sum in a fixed order (deterministic).
__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s += red[w];
    return s;
}

// x → LDS, optionally RMSNorm'ed: out = x·fastRsqrt(Σx²/n + eps)·w (ops.go:1015-1037)
template <int PRO>
__device__ __forceinline__ void stage_x(float *xs, const float *x, const float *w, int n, float eps,
                                        float *red) {
    if constexpr (PRO == PRO_COPY) {
        for (int i = threadIdx.x; i < n; i += kThreads) xs[i] = x[i];
        __syncthreads();
    } else {
        float ss = 0.0f;
        for (int i = threadIdx.x; i < n; i += kThreads) {
            float v = x[i];
            xs[i] = v;
            ss = fmaf(v, v, ss);
        }
        ss = block_sum(ss, red);
        const float scale = fast_rsqrt_ref(ss / (float)n + eps);
        for (int i = threadIdx.x; i < n; i += kThreads) {
#pragma clang fp contract(off)
            xs[i] = xs[i] * scale * w[i];
        }
        __syncthreads();
    }
}

// resid = residual[r], read by the caller ahead of time (EPI_OPROJ/DOWN/ADDV)
// row r of activation vector v (memory index o = v·o_stride + r)
__device__ __forceinline__ void gemv_epilogue(const GemvParams &p, int epi, int r, int o, const float *s, float resid,
                                              bool in_place, float &best_v, int &best_r) {
#pragma clang fp contract(off)
    switch (epi) {
    case EPI_PLAIN: p.out[o] = s[0]; break;
    case EPI_SWIGLU: p.out[o] = silu_ref(s[0]) * s[1]; break;
    case EPI_OPROJ: {
        const float v = resid + s[0];
        p.vbuf[o] = v;
        if (in_place) p.residual[o] = v;
        break;
    }
    case EPI_DOWN: {
        const float v = resid + s[0];
        if (p.flag) p.vbuf[o] = v;
        else p.residual[o] = v;
        break;
    }
    case EPI_ADDV: p.vbuf[o] = resid + s[0]; break;
    case EPI_DOWNV: {  // resid was picked from vbuf or residual by the o_proj rule
        const float v = resid + s[0];
        if (p.flag) p.vbuf[o] = v;
        else p.residual[o] = v;
        break;
    }
    default:  // EPI_ARGMAX
        if (p.out) p.out[o] = s[0];
        if (s[0] > best_v || (s[0] == best_v && r < best_r)) {
            best_v = s[0];
            best_r = r;
        }
    }
}

__device__ __forceinline__ bool epi_reads_residual(int epi) {
    return epi == EPI_OPROJ || epi == EPI_DOWN || epi == EPI_ADDV || epi == EPI_DOWNV;
}

__device__ __forceinline__ StepState *st_of(const GemvParams &p, const GemvNV &q, int v) {
    return v == 0 ? p.st : (v == 1 ? q.stv[0] : (v == 2 ? q.stv[1] : q.stv[2]));
}

__device__ __forceinline__ bool oproj_in_place(const GemvParams &p, const StepState *st) {
    if (!st) return p.flag != 0;
    // model.go:3895-3902 (first token) and 4051-4057 (len > 6): Q4/Q6 use the
    // OutOnly variant; positions 1..5 go through matVecOutAddRMSNormCPU (in place).
    const int clen = st->clen;
    return !(p.quirk && (clen == 0 || clen >= 6));
}

__device__ __forceinline__ uint32_t ordered_bits(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// unsigned max / signed min over the 64 lanes of a wave (DPP and swizzle
// exchanges of the bit pattern), the same value in every lane
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, __float_as_uint(xchg<XQ1>(__uint_as_float(v))));
    v = max(v, __float_as_uint(xchg<XQ2>(__uint_as_float(v))));
    v = max(v, __float_as_uint(xchg<XM8>(__uint_as_float(v))));
    v = max(v, __float_as_uint(xchg<XM16>(__uint_as_float(v))));
    v = max(v, __float_as_uint(xchg<XS16>(__uint_as_float(v))));
    v = max(v, __float_as_uint(xchg<XS32>(__uint_as_float(v))));
    return v;
}
__device__ __forceinline__ int wave_min_i32(int v) {
    v = min(v, __float_as_int(xchg<XQ1>(__int_as_float(v))));
    v = min(v, __float_as_int(xchg<XQ2>(__int_as_float(v))));
    v = min(v, __float_as_int(xchg<XM8>(__int_as_float(v))));
    v = min(v, __float_as_int(xchg<XM16>(__int_as_float(v))));
    v = min(v, __float_as_int(xchg<XS16>(__int_as_float(v))));
    v = min(v, __float_as_int(xchg<XS32>(__int_as_float(v))));
    return v;
}

// Greedy argmax of the workgroup's rows into its slot: the largest score
// (compared as order-preserving bits, like the 64-bit key), then the lowest
// row holding it (argmax_quant.go:255-262: ties keep the first index).
__device__ __forceinline__ void argmax_finish(StepState *st, float best_v, int best_r, float *red) {
    const bool has = best_r != 0x7FFFFFFF;
    const uint32_t ob = wave_max_u32(has ? ordered_bits(best_v) : 0u);
    const int rmin = wave_min_i32(has && ordered_bits(best_v) == ob ? best_r : 0x7FFFFFFF);
    unsigned long long *kred = reinterpret_cast<unsigned long long *>(red);
    const int wave = threadIdx.x >> 6;
    __syncthreads();  // red may still be read by the prologue's reductions
    if ((threadIdx.x & 63) == 0)
        kred[wave] = rmin == 0x7FFFFFFF ? 0ull
                                        : (((unsigned long long)ob << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)rmin));
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long m = kred[0];
        for (int w = 1; w < kWaves; ++w) m = kred[w] > m ? kred[w] : m;
        if (m) atomicMax(&st->argmax_slot[(blockIdx.x % kArgSlots) * kSlotPitch], m);
    }
}

// row → (segment, row within the segment's matrix), by selects (no dynamic
// indexing of the kernel-argument array)
__device__ __forceinline__ DevMat seg_mat(const GemvParams &p, int sg) {
    return sg == 0 ? p.m[0] : (sg == 1 ? p.m[1] : p.m[2]);
}

// A wave's row group never straddles a segment boundary (the host checks
// that segment sizes are multiples of the group size), so the segment is
// chosen once per group from wave-uniform values: scalar branches over the
// kernel-argument pointers.
struct SegSel {
    const uint8_t *data0, *data1;  // matrix (NMAT==1) or gate/up (NMAT==2)
    const float *scale0, *scale1;
    int start;  // first global row of the segment
};

template <int NMAT>
__device__ __forceinline__ SegSel seg_select(const GemvParams &p, int r0) {
    SegSel s;
    if (NMAT == 2) {
        s.data0 = p.m[0].data;
        s.data1 = p.m[1].data;
        s.scale0 = p.m[0].scale;
        s.scale1 = p.m[1].scale;
        s.start = 0;
    } else if (r0 >= p.seg_end[1]) {
        s.data0 = s.data1 = p.m[2].data;
        s.scale0 = s.scale1 = p.m[2].scale;
        s.start = p.seg_end[1];
    } else if (r0 >= p.seg_end[0]) {
        s.data0 = s.data1 = p.m[1].data;
        s.scale0 = s.scale1 = p.m[1].scale;
        s.start = p.seg_end[0];
    } else {
        s.data0 = s.data1 = p.m[0].data;
        s.scale0 = s.scale1 = p.m[0].scale;
        s.start = 0;
    }
    return s;
}

// Requests one group's chunks.  Rows past the end are clamped to the last
// row (loaded, never written back), so every lane issues the same number of
// loads and the wait counts stay static.
template <int QT, int LPR, int CPL, int U, int NMAT>
__device__ __forceinline__ void load_group(const SegSel &sel, int row_bytes, int rows, int g, int sub, int l,
                                           Chunk (&w)[U][NMAT][CPL]) {
    using T = QTraits<QT>;
    constexpr int RPW = 64 / LPR;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int lr = min((g * U + u) * RPW + sub, rows - 1) - sel.start;
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi) {
            const uint8_t *row = (mi == 0 ? sel.data0 : sel.data1) + (size_t)lr * row_bytes;
#pragma unroll
            for (int j = 0; j < CPL; ++j) w[u][mi][j] = load_chunk<QT>(row + (l + j * LPR) * T::CB);
        }
    }
}

// LPR lanes share one row; each lane owns CPL chunks (lane + j·LPR) of every
// row, so its x slice (CPL·W floats) stays in VGPRs across rows.  A wave
// handles groups of U·RPW rows (RPW = 64/LPR side by side): the first group's
// weights are requested before the activation prologue, and each group's
// successor is requested before the group is computed, so a wave always has
// U·CPL·NMAT 16-byte loads in flight.  The U row sums are reduced together
// with one reduce-scatter, leaving row u's sum in lane u·(LPR/U).
// TAG only separates instances for profiling (TAG=1: the timing entry point).
// ONE: the grid gives every wave at most one group (no row loop, no prefetch
// registers), for the large single-matrix launch.
// NPL: byte digit planes of the activation (3: x to 2^-22 of each chunk's
// maximum; the greedy heads of the shapes head.hpp does not take use 3 too).
// NV: activation vectors sharing each weight pass (batched decode, M = NV):
// every chunk is dotted against each vector's digits (read from LDS per
// group), and the reduce-scatter runs over U·NV entries e = u·NV + v.
template <int QT, int LPR, int CPL, int U, int NMAT, int TAG, bool ONE, int NPL, int NV>
__device__ __forceinline__ void gemv_body(GemvParams p, int pro, int epi, const GemvNV &q) {
    // No step-state check up front: a GEMV writes only step scratch (the
    // residual stream, q/k/v, gate) and never indexes by the step state, so a
    // failed step needs no guard here and the first loads wait for nothing.
    extern __shared__ int4 lds4[];
    int *lds = reinterpret_cast<int *>(lds4);
    __shared__ float red[2 * kWaves * NV];
    constexpr int RPW = 64 / LPR;
    constexpr int RG = RPW * U;
    constexpr int E = U * NV;  // reduce-scatter entries
    static_assert(E <= LPR && (E & (E - 1)) == 0, "entries: a power of two within the row's lanes");
    // Every kernel argument is made live here, so their scalar loads issue as
    // one batch: one kernel-argument round trip instead of one per branch.
    asm volatile("" ::"s"(p.m[0].data), "s"(p.m[0].scale), "s"(p.m[1].data), "s"(p.m[1].scale), "s"(p.m[2].data),
                 "s"(p.m[2].scale));
    asm volatile("" ::"s"(p.x), "s"(p.norm_w), "s"(p.out), "s"(p.residual), "s"(p.vbuf), "s"(p.st));
    asm volatile("" ::"s"(p.seg_end[0]), "s"(p.seg_end[1]), "s"(p.rows), "s"(p.cols), "s"(p.m[0].row_bytes),
                 "s"(p.eps), "s"(p.flag), "s"(p.quirk), "s"(pro), "s"(epi));
    if constexpr (NV > 1) asm volatile("" ::"s"(q.x_stride), "s"(q.o_stride), "s"(q.stv[0]), "s"(q.stv[1]), "s"(q.stv[2]));

    const int rows = p.rows;
    const int row_bytes = p.m[0].row_bytes;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sub = lane / LPR;
    const int l = lane % LPR;
    const int ngroups = (rows + RG - 1) / RG;
    const int gstride = gridDim.x * kWaves;
    int g = blockIdx.x * kWaves + wave;
    constexpr int SPAN = LPR / E;  // lanes per entry after the reduce-scatter
    const int my_e = l / SPAN;
    const int my_u = my_e / NV, my_v = my_e % NV;
    const bool writer = (l % SPAN) == 0;
    const bool need_resid = epi_reads_residual(epi);
    const int my_o = NV > 1 ? my_v * q.o_stride : 0;  // the writer's vector in out/residual/vbuf

    // activations first, so that waiting for them does not wait for weights
    const int cols = p.cols;
    const bool norm = pro == PRO_RMSNORM || pro == PRO_OPART;
    XRegs xr[NV];
    OpartRegs opr;
    const bool opart = NV == 1 && pro == PRO_OPART;  // uniform
    if (opart) {
        opart_issue(p.x, p.flag, p.residual, cols, opr);
#pragma unroll
        for (int pp = 0; pp < kXPasses; ++pp) {  // the norm weight; x itself comes from LDS below
            if (pp * kXPass >= cols) break;      // uniform
            const float4 *wp =
                reinterpret_cast<const float4 *>(p.norm_w + min((pp * kThreads + (int)threadIdx.x) * 8, cols - 8));
            xr[0].w[pp][0] = wp[0];
            xr[0].w[pp][1] = wp[1];
        }
    } else {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const float *xv = p.x + (NV > 1 ? v * q.x_stride : 0);
            x_load(xv, p.norm_w, norm && v == 0, cols, xr[v]);
        }
    }
    // first group: weights, then the writer lane's epilogue operands (row
    // scale, residual), all requested before the prologue's first wait
    Chunk w[U][NMAT][CPL];
    float scl[NMAT], resid, residv;
    {
        const int gc = min(g, ngroups - 1);
        const SegSel sel = seg_select<NMAT>(p, gc * RG);
        load_group<QT, LPR, CPL, U, NMAT>(sel, row_bytes, rows, gc, sub, l, w);
        const int rc = min((gc * U + my_u) * RPW + sub, rows - 1);
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi) scl[mi] = (mi == 0 ? sel.scale0 : sel.scale1)[rc - sel.start];
        resid = need_resid ? p.residual[my_o + rc] : 0.0f;
        residv = epi == EPI_DOWNV ? p.vbuf[rc] : 0.0f;
    }
    const int recs = QT == QT_Q4 ? (cols / 32) * DigitRec<QT>::RS : (cols / 16) * DigitRec<QT>::RS;
    if (opart) {
        // residual + Σ partials → LDS after the digit records (and, in
        // workgroup 0, to vbuf for the down GEMV), then each prologue thread
        // takes its 8 columns as x_load would have
        float *stage = reinterpret_cast<float *>(lds + recs);
        opart_stage(opr, p.flag, cols, stage, blockIdx.x == 0 ? p.vbuf : nullptr);
        __syncthreads();
#pragma unroll
        for (int pp = 0; pp < kXPasses; ++pp) {
            if (pp * kXPass >= cols) break;  // uniform
            const int cb = min((pp * kThreads + (int)threadIdx.x) * 8, cols - 8);
            xr[0].x[pp][0] = *reinterpret_cast<const float4 *>(stage + cb);
            xr[0].x[pp][1] = *reinterpret_cast<const float4 *>(stage + cb + 4);
        }
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        // the norm weight was loaded once, with vector 0
        x_digits<QT>(xr[v], xr[0], norm, cols, lds + v * recs, red + v * kWaves);
    }
    __syncthreads();
    float xscale = x_norm_factor(norm, cols, p.eps, red);
#pragma unroll
    for (int v = 1; v < NV; ++v) {
        const float f = x_norm_factor(norm, cols, p.eps, red + v * kWaves);
        xscale = my_v == v ? f : xscale;
    }
    XDig<QT, CPL, NPL> xd;  // NV = 1: the vector's digits stay in registers across groups
    if constexpr (NV == 1) load_digits<QT, LPR, CPL, NPL>(lds, l, xd);
    const bool in_place = (epi == EPI_OPROJ || epi == EPI_DOWNV) ? oproj_in_place(p, st_of(p, q, my_v)) : false;
    const bool use_v = epi == EPI_DOWNV && in_place;  // the residual includes this layer's attention
    float best_v = -INFINITY;
    int best_r = 0x7FFFFFFF;

    // one group: row sums, reduce-scatter, epilogue by the writer lanes
    auto compute = [&](int gg, const Chunk (&wc)[U][NMAT][CPL], const float (&sc)[NMAT], float rs) {
        const int r = (gg * U + my_u) * RPW + sub;
        float acc[E > 8 ? E : 8][NMAT];
        if constexpr (NV == 1) {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int mi = 0; mi < NMAT; ++mi) acc[u][mi] = row_dot<QT, CPL, NPL>(wc[u][mi], xd);
        } else {
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                XDig<QT, CPL, NPL> xv;
                load_digits<QT, LPR, CPL, NPL>(lds + v * recs, l, xv);
#pragma unroll
                for (int u = 0; u < U; ++u)
#pragma unroll
                    for (int mi = 0; mi < NMAT; ++mi) acc[u * NV + v][mi] = row_dot<QT, CPL, NPL>(wc[u][mi], xv);
                // one vector's digits live at a time: keep the next vector's
                // LDS reads below this point
                asm volatile("" ::: "memory");
            }
        }
        reduce_scatter<LPR, E, NMAT>(acc, lane);
        if (writer && r < rows) {
            float sv[NMAT];
#pragma unroll
            for (int mi = 0; mi < NMAT; ++mi) sv[mi] = acc[0][mi] * xscale * sc[mi];
            gemv_epilogue(p, epi, r, my_o + r, sv, rs, in_place, best_v, best_r);
        }
    };
    // Every group but a wave's last requests its successor's weights and
    // epilogue operands before it is computed (software pipeline of depth
    // one); the last one is peeled off, so no wave requests rows it does not
    // use and every path keeps static wait counts.
    if constexpr (!ONE) for (; g + gstride < ngroups; g += gstride) {
        Chunk wn[U][NMAT][CPL];
        float scln[NMAT], residn, residvn;
        {
            const int gn = g + gstride;
            const SegSel seln = seg_select<NMAT>(p, gn * RG);
            load_group<QT, LPR, CPL, U, NMAT>(seln, row_bytes, rows, gn, sub, l, wn);
            const int rn = min((gn * U + my_u) * RPW + sub, rows - 1);
#pragma unroll
            for (int mi = 0; mi < NMAT; ++mi) scln[mi] = (mi == 0 ? seln.scale0 : seln.scale1)[rn - seln.start];
            residn = need_resid ? p.residual[my_o + rn] : 0.0f;
            residvn = epi == EPI_DOWNV ? p.vbuf[rn] : 0.0f;
        }
        compute(g, w, scl, use_v ? residv : resid);
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
                for (int j = 0; j < CPL; ++j) w[u][mi][j] = wn[u][mi][j];
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi) scl[mi] = scln[mi];
        resid = residn;
        residv = residvn;
    }
    if (g < ngroups) compute(g, w, scl, use_v ? residv : resid);
    if (epi == EPI_ARGMAX) {
#pragma unroll
        for (int v = 0; v < NV; ++v)
            argmax_finish(st_of(p, q, v), my_v == v ? best_v : -INFINITY, my_v == v ? best_r : 0x7FFFFFFF, red);
    }
}

template <int QT, int LPR, int CPL, int U, int NMAT, int TAG = 0, int NPL = 3>
__global__ void __launch_bounds__(kThreads) k_gemv(GemvParams p, int pro, int epi) {
    gemv_body<QT, LPR, CPL, U, NMAT, TAG, false, NPL, 1>(p, pro, epi, GemvNV{});
}

// One row group per wave (no row loop, no prefetch registers).
template <int QT, int LPR, int CPL, int U, int NMAT, int TAG = 0, int NPL = 3>
__global__ void __launch_bounds__(kThreads) k_gemv_one(GemvParams p, int pro, int epi) {
    gemv_body<QT, LPR, CPL, U, NMAT, TAG, true, NPL, 1>(p, pro, epi, GemvNV{});
}

// NV activation vectors per weight pass (batched decode, M = NV)
template <int QT, int LPR, int CPL, int U, int NMAT, int NPL, int NV, bool ONE>
__global__ void __launch_bounds__(kThreads) k_gemv_nv(GemvParams p, int pro, int epi, GemvNV q) {
    gemv_body<QT, LPR, CPL, U, NMAT, 0, ONE, NPL, NV>(p, pro, epi, q);
}

// Any shape (tiny test matrices, odd column counts): one wavefront per row,
// lanes stride over columns and decode one code at a time.
__device__ __forceinline__ int decode_code(const DevMat &M, const uint8_t *row, int c) {
    if (M.qtype == QT_Q8) return (int)(int8_t)row[c];
    if (M.qtype == QT_Q4) {
        const uint8_t b = row[c >> 1];
        return (int)((c & 1) ? (b >> 4) : (b & 15)) - 8;
    }
    const int bit = c * 6, idx = bit >> 3, sh = bit & 7;
    uint32_t v = row[idx];
    if (idx + 1 < M.row_bytes) v |= (uint32_t)row[idx + 1] << 8;
    return (int)((v >> sh) & 63u) - 32;
}

template <int NMAT>
__global__ void __launch_bounds__(kThreads) k_gemv_any(GemvParams p, int pro, int epi) {
    if (p.st && p.st->err) return;
    extern __shared__ float xs[];
    __shared__ float red[2 * kWaves];
    if (pro == PRO_RMSNORM) stage_x<PRO_RMSNORM>(xs, p.x, p.norm_w, p.cols, p.eps, red);
    else stage_x<PRO_COPY>(xs, p.x, p.norm_w, p.cols, p.eps, red);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const bool in_place = epi == EPI_OPROJ ? oproj_in_place(p, p.st) : false;
    float best_v = -INFINITY;
    int best_r = 0x7FFFFFFF;
    const int nw = gridDim.x * kWaves;
    const int iters = (p.rows + nw - 1) / nw;
    for (int it = 0; it < iters; ++it) {
        const int r = it * nw + blockIdx.x * kWaves + wave;
        const bool valid = r < p.rows;
        int sg = 0, lr = r;
        if (NMAT == 1) {
            sg = (r >= p.seg_end[0]) + (r >= p.seg_end[1]);
            lr = r - (sg == 0 ? 0 : (sg == 1 ? p.seg_end[0] : p.seg_end[1]));
        }
        float s[NMAT];
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi) {
            const DevMat M = seg_mat(p, NMAT == 1 ? sg : mi);
            float acc = 0.0f;
            if (valid) {
                const uint8_t *row = M.data + (size_t)lr * M.row_bytes;
                for (int c = lane; c < p.cols; c += 64) acc = fmaf((float)decode_code(M, row, c), xs[c], acc);
            }
            s[mi] = lane_group_sum<64>(acc);
            if (valid) {
#pragma clang fp contract(off)
                s[mi] = s[mi] * M.scale[lr];
            }
        }
        if (lane == 0 && valid)
            gemv_epilogue(p, epi, r, r, s, epi_reads_residual(epi) ? p.residual[r] : 0.0f, in_place, best_v, best_r);
    }
    if (epi == EPI_ARGMAX) argmax_finish(p.st, best_v, best_r, red);
}

// ---------------------------------------------------------------------------
// small vector kernels
// ---------------------------------------------------------------------------

// out = RMSNorm(x)·w (single workgroup)
static __global__ void __launch_bounds__(kThreads) k_rmsnorm(const float *x, const float *w, int n, float eps,
                                                        float *out) {
    __shared__ float red[2 * kWaves];
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += kThreads) ss = fmaf(x[i], x[i], ss);
    ss = block_sum(ss, red);
    const float scale = fast_rsqrt_ref(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += kThreads) {
#pragma clang fp contract(off)
        out[i] = x[i] * scale * w[i];
    }
}

// AddRMSNorm (ops.go:913-935) / AddRMSNormOutOnly (fused_matvec2.go:11-33):
// v = dst + add into v_out, out = v·fastRsqrt(Σv²/n + eps)·w (one workgroup)
static __global__ void __launch_bounds__(kThreads) k_add_rmsnorm(const float *dst, const float *add, const float *w,
                                                            int n, float eps, float *v_out, float *out) {
    __shared__ float red[2 * kWaves];
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += kThreads) {
        float v;
        {
#pragma clang fp contract(off)
            v = dst[i] + add[i];
        }
        v_out[i] = v;
        ss = fmaf(v, v, ss);
    }
    ss = block_sum(ss, red);
    const float scale = fast_rsqrt_ref(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += kThreads) {  // each thread reads back its own v
#pragma clang fp contract(off)
        out[i] = v_out[i] * scale * w[i];
    }
}

// ApplyMRoPETable (internal/tensor/weighted_sum.go:231-250) on q and k in place
__device__ __forceinline__ void rope_pair(float &a, float &b, float cs, float sn) {
#pragma clang fp contract(off)
    const float na = a * cs - b * sn;
    const float nb = b * cs + a * sn;
    a = na;
    b = nb;
}

static __global__ void __launch_bounds__(kThreads) k_rope(float *q, float *k, const float *cos_t, const float *sin_t,
                                                     int q_heads, int kv_heads, int dim) {
    const int half = dim / 2;
    const int total = (q_heads + kv_heads) * half;
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < total; i += gridDim.x * kThreads) {
        const int h = i / half, j = i % half;
        float *base = h < q_heads ? q + (size_t)h * dim : k + (size_t)(h - q_heads) * dim;
        rope_pair(base[j], base[j + half], cos_t[j], sin_t[j]);
    }
}

// Step prologue: token/position bookkeeping, RoPE table (buildMRoPETable,
// model.go:7318-7357: f64 angle, f64 cos/sin rounded to f32), embedding row.
// mode 0: h and pos were written by the host.  mode 1: greedy decode — the
// token is the previous step's argmax, its embedding row is copied into h and
// the position is next_pos (decode position len(out)-1+ropeDelta, model.go:1695).
// Everything that does not wait for the chosen token is requested at entry in
// one round trip (the argmax slots, thread 0's state fields, the position),
// and the table entry is computed while the slots are reduced; the token's
// embedding row is requested while thread 0 settles the state.  Results are
// stored only once the step is known to go ahead.
constexpr int kStepEmb = 4;  // embedding floats a thread holds across the state barrier
__device__ __forceinline__ void step_begin_body(StepState *st, const float *embed, float *h, int hidden, int vocab,
                                                const double *freq, const uint8_t *axis, int mode, int32_t *tokens,
                                                int max_tokens) {
    __shared__ int s_err;
    __shared__ unsigned long long s_key;
    const int t = threadIdx.x;
    unsigned long long k = 0ull;
    if (t < kArgSlots) k = st->argmax_slot[t * kSlotPitch];
    int4 hdr = make_int4(0, 0, 0, 0);  // len, clen, cap, err
    int n_out = 0, n_eos = 0;
    const uint32_t *bits = nullptr;
    int4 eos4[kMaxEos / 4];
    if (t == 0) {
        hdr = *reinterpret_cast<const int4 *>(st);
        n_out = st->n_out;
        n_eos = st->n_eos;
        bits = st->eos_bits;
#pragma unroll
        for (int i = 0; i < kMaxEos / 4; ++i) eos4[i] = reinterpret_cast<const int4 *>(st->eos)[i];
    }
    // this step's position: the decode counter (mode 1) or the host's (mode 0)
    int pos[3];
    if (mode == 1) {
        pos[0] = pos[1] = pos[2] = st->next_pos;
    } else {
        pos[0] = st->pos[0];
        pos[1] = st->pos[1];
        pos[2] = st->pos[2];
    }
    const int half = st->half;  // ≤ kMaxHalf ≤ kThreads: one table entry per thread
    float ct = 0.0f, sn = 0.0f;
    if (t < half) {
        const int a = axis[t];
        const int p = a == 0 ? pos[0] : (a == 1 ? pos[1] : pos[2]);
        const double ang = (double)p * freq[t];
        ct = (float)cos(ang);
        sn = (float)sin(ang);
    }
    if (t < kArgSlots) {  // wave 0: max over the argmax slots
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const unsigned long long o = __shfl_xor(k, off, 64);
            k = o > k ? o : k;
        }
        if (t == 0) s_key = k;
    }
    __syncthreads();
    const unsigned long long key = s_key;
    const int tok = (int)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
    const bool take = mode == 1 && key != 0ull && tok >= 0 && tok < vocab;
    float e[kStepEmb];
    if (take) {
        const float *src = embed + (size_t)tok * hidden;
#pragma unroll
        for (int j = 0; j < kStepEmb; ++j) {
            const int i = t + j * kThreads;
            e[j] = i < hidden ? src[i] : 0.0f;
        }
    }
    if (t == 0) {
        int err = hdr.w;
        if (!err && hdr.x >= hdr.z) err = 1;  // len ≥ cap
        if (!err && mode == 1) {
            if (key == 0ull) err = 2;
            if (tok < 0 || tok >= vocab) err = 3;
            if (!err && n_out >= max_tokens) err = 4;
            if (!err) {
                tokens[n_out] = tok;
                st->n_out = n_out + 1;
                st->next_pos = pos[0] + 1;
                st->pos[0] = st->pos[1] = st->pos[2] = pos[0];
                // the generation loop stops at an EOS token once it is in the
                // output, before any step for it (model.go:1545-1548)
                if (bits) {
                    if ((bits[tok >> 5] >> (tok & 31)) & 1u) err = kErrStopped;
                } else {
                    const int ne = min(n_eos, kMaxEos);
                    const int *ev = reinterpret_cast<const int *>(eos4);
#pragma unroll
                    for (int i = 0; i < kMaxEos; ++i)
                        if (i < ne && ev[i] == tok) err = kErrStopped;
                }
            }
        }
        if (!err) {
            st->clen = hdr.x;
            st->len = hdr.x + 1;
            st->has_rope = (pos[0] != 0 || pos[1] != 0 || pos[2] != 0) ? 1 : 0;
        }
        st->err = err;
        s_err = err;
    }
    __syncthreads();
    if (!s_err && t < kArgSlots) st->argmax_slot[t * kSlotPitch] = 0ull;
    if (s_err) return;
    if (t < half) {
        st->cos_t[t] = ct;
        st->sin_t[t] = sn;
    }
    if (mode == 1) {
#pragma unroll
        for (int j = 0; j < kStepEmb; ++j) {
            const int i = t + j * kThreads;
            if (i < hidden) h[i] = e[j];
        }
        const float *src = embed + (size_t)tok * hidden;
        for (int i = t + kStepEmb * kThreads; i < hidden; i += kThreads) h[i] = src[i];
    }
}

static __global__ void __launch_bounds__(kThreads) k_step_begin(StepState *st, const float *embed, float *h, int hidden,
                                                           int vocab, const double *freq, const uint8_t *axis,
                                                           int mode, int32_t *tokens, int max_tokens) {
    step_begin_body(st, embed, h, hidden, vocab, freq, axis, mode, tokens, max_tokens);
}

// Greedy decode of several sequences in one step: workgroup b runs sequence
// b's prologue (mode 1) and writes its embedding row to h + b·hidden.
struct StepBatch {
    StepState *st[kMaxBatch];
    int32_t *tokens[kMaxBatch];
    int max_tokens[kMaxBatch];
};
// b is the kernel's first argument (offset 0 of the argument segment): entry
// blockIdx.x is read in place with scalar loads.  The argument segment exists
// in the device pass only.
typedef __attribute__((address_space(4))) const StepBatch KernargStepBatch;
static __global__ void __launch_bounds__(kThreads) k_step_begin_multi(StepBatch b, const float *embed, float *h,
                                                                 int hidden, int vocab, const double *freq,
                                                                 const uint8_t *axis) {
    (void)b;
#if defined(__HIP_DEVICE_COMPILE__)
    const KernargStepBatch *kb = (KernargStepBatch *)__builtin_amdgcn_kernarg_segment_ptr();
    const int i = blockIdx.x;
    step_begin_body(kb->st[i], embed, h + (size_t)i * hidden, hidden, vocab, freq, axis, 1, kb->tokens[i],
                    kb->max_tokens[i]);
#endif
}

// ---------------------------------------------------------------------------
// GQA decode attention, head_dim 128, split over cache rows.
//
// Workgroup (g, s) owns kv head g and cache rows [s·chunk, (s+1)·chunk),
// chunk ≤ 4·RPW; wave w of it owns the RPW rows from s·chunk + RPW·w and is
// a softmax split of its own.  RPW (8 or 16 rows per wave) trades workgroups
// in flight against split records to merge: the host picks it from the cache
// capacity.  Every request (the q heads of the group and the RoPE table
// entries first, the new K/V row, the wave's K rows by score pass, then its V
// rows) is issued before the step state is read, in one memory round trip;
// scores start as soon as their K rows have arrived.  The group's q is
// rotated once per workgroup (each thread holds a RoPE pair (d, d+64) in its
// own registers) and shared through LDS.  Scores for all GROUP q heads share
// each K row (16 lanes × 8 dims per row, reduced by a DPP reduce-scatter);
// the wave's softmax uses lane exchanges only, its probabilities reach the
// P·V lanes through a wave-private LDS slot, and one barrier combines the
// four waves into the split's record (max, Σexp, Σexp·V), which
// k_attn_merge combines across splits.  The owner wave of the
// newest row appends it (kvCache.append, model.go:5593-5612: row t at
// t·kvDim + g·128).  Scores: dot(q,k)·f32(1/√128) (model.go:4623-4795, 7391);
// softmax with FastExp (ops.go:1199-1363); out = Σ p·V (model.go:5201-5590).
// ---------------------------------------------------------------------------
constexpr int kHD = 128;
constexpr int kMaxGroup = 8;
constexpr int kOrdMaxRows = 8192;  // cache rows of the VNNI mode's ordered attention (scores in LDS)
constexpr int kMaxChunk = 64;  // cache rows per workgroup (RPW 16)
constexpr int kRec = kHD + 4;  // partial record per head: m, l, 2 pad, acc[128] (16-byte aligned)

struct AttnParams {
    const float *q;        // [heads*128] (unrotated if rope)
    const float *k_new;    // [kvh*128] new row (unrotated if rope) or null
    const float *v_new;    // [kvh*128] or null
    float *kc;             // layer cache base [cap][kvh*128]
    float *vc;
    StepState *st;         // null → op level (len/rope from fields below)
    int len;               // op level: rows in cache (no append)
    int has_rope;          // op level
    const float *cos_t;    // op level tables (null: no RoPE)
    const float *sin_t;
    float *part;           // [kvh][nsplit][GROUP][kRec]
    float *head_out;       // [heads*128]
    int heads, kvh, nsplit;
    int rows_cap;          // rows the splits are cut from (cache capacity)
    float scale;
    int chunk;             // rows per split, attn_chunk(rows_cap, nsplit, 4·RPW)
};

// rows per split: the capacity's share rounded up to 16, at most max_chunk
__host__ __device__ constexpr int attn_chunk(int rows_cap, int nsplit, int max_chunk) {
    return ((rows_cap + nsplit - 1) / nsplit + 15) / 16 * 16 < max_chunk
               ? ((rows_cap + nsplit - 1) / nsplit + 15) / 16 * 16
               : max_chunk;
}

// reduce-scatter of 8 per-head partial dots over the 16 lanes of a row:
// lanes 2h and 2h+1 end with head h's full sum
__device__ __forceinline__ float rs16_heads(float (&v)[8][1], int lane) {
    rs_step<8, 1, XM16, 8>(v, lane);
    rs_step<4, 1, XM8, 4>(v, lane);
    rs_step<2, 1, XQ2, 2>(v, lane);
    rs_step<1, 1, XQ1, 1>(v, lane);
    return v[0][0];
}

// Kernel arguments made live at entry: one batch of scalar loads instead of
// one argument round trip at each field's first use.  Input operands only:
// an in/out operand would hide the pointers' provenance, turning every load
// through them into a flat load (tracked by the 4-bit LGKM counter too, so
// the loads would drain in rounds of 15).
__device__ __forceinline__ void pin_args(const AttnParams &p) {
    asm volatile("" ::"s"(p.q), "s"(p.k_new), "s"(p.v_new), "s"(p.kc), "s"(p.vc), "s"(p.st), "s"(p.part),
                 "s"(p.head_out));
    asm volatile("" ::"s"(p.cos_t), "s"(p.sin_t), "s"(p.heads), "s"(p.kvh), "s"(p.nsplit), "s"(p.rows_cap));
    asm volatile("" ::"s"(p.len), "s"(p.has_rope), "s"(p.chunk));
}

// in-lane RoPE of pairs (a = dim d, b = dim d + 64): a' = a·cos − b·sin,
// b' = b·cos + a·sin, products rounded before the add
__device__ __forceinline__ void rope_pair4(float4 &a, float4 &b, const float4 &c, const float4 &s) {
#pragma clang fp contract(off)
    const float4 a0 = a, b0 = b;
    a = make_float4(a0.x * c.x - b0.x * s.x, a0.y * c.y - b0.y * s.y, a0.z * c.z - b0.z * s.z, a0.w * c.w - b0.w * s.w);
    b = make_float4(b0.x * c.x + a0.x * s.x, b0.y * c.y + a0.y * s.y, b0.z * c.z + a0.z * s.z, b0.w * c.w + a0.w * s.w);
}
__device__ __forceinline__ void rope_pair2(float2 &a, float2 &b, const float2 &c, const float2 &s) {
#pragma clang fp contract(off)
    const float2 a0 = a, b0 = b;
    a = make_float2(a0.x * c.x - b0.x * s.x, a0.y * c.y - b0.y * s.y);
    b = make_float2(b0.x * c.x + a0.x * s.x, b0.y * c.y + a0.y * s.y);
}

// Lane layouts.  Scores: a 16-lane row (rg = lane / 16) takes one K row per
// pass, lane l16 holding dims 4·l16..4·l16+3 and their RoPE partners 64 + the
// same (two 16-byte loads that together read the row's 512 bytes as two
// contiguous 256-byte halves).  P·V: lanes 0-31 and 32-63 take alternate rows,
// lane holding dims 4·(lane & 31)..+3 (one 16-byte load per lane per two rows).
template <int RPW>
__device__ __forceinline__ void attn_decode_body(AttnParams p) {
    // products round before any later add (scores: s·scale, then s − max, as
    // the reference does); the fused steps are written as fmaf
#pragma clang fp contract(off)
    static_assert(RPW == 8 || RPW == 16, "rows per wave");
    constexpr int NJ = RPW / 4;  // score passes of 4 rows
    constexpr int NV = RPW / 2;  // P·V loads: two rows each
    StepState *st = p.st;
    __shared__ float4 q_lds[kMaxGroup][kHD / 4];          // the group's rotated q
    __shared__ __align__(16) float e_lds[kWaves][kMaxGroup][2][NV];  // wave-private probabilities [head][row parity][row / 2]
    __shared__ float w_m[kWaves][kMaxGroup], w_l[kWaves][kMaxGroup];
    __shared__ float4 w_acc[kWaves][kMaxGroup][2][kHD / 4];

    const int g = blockIdx.x;  // kv head
    const int split = blockIdx.y;
    const int group = p.heads / p.kvh;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, rg = lane >> 4;
    const int half = lane >> 5, l32 = lane & 31;
    const float *cos_t = st ? st->cos_t : p.cos_t;
    const float *sin_t = st ? st->sin_t : p.sin_t;
    const int kvd = p.kvh * kHD;

    // Splits are cut from the row capacity (a launch constant), so every
    // request below is issued before the step state has arrived.
    const int chunk = p.chunk;
    const int t0 = split * chunk;
    const int wr0 = t0 + RPW * wave;  // first row of this wave
    const int tmax = p.rows_cap - 1;

    // ---- 1. requests, oldest first, in the order they are used: the step
    // state's header (len, clen, cap, err) and RoPE flag; this thread's q pair
    // (head tid / 32, dims 2i, 2i+1 and 64 + the same) with its cos/sin; the
    // new K/V row and its cos/sin (score layout); then K by score pass, then
    // V.  Without a step state, RoPE table or new row the loads read q (a
    // readable stand-in, replaced at use); heads past the group re-read the
    // group's last head; rows past the capacity are clamped to the last row
    // (loaded, masked below).  Every lane issues the same loads.
    int4 st4 = *reinterpret_cast<const int4 *>(st ? reinterpret_cast<const float *>(st) : p.q);
    int st_rope = *(st ? &st->has_rope : reinterpret_cast<const int *>(p.q));
    asm volatile("" ::: "memory");
    const int qh = tid >> 5, qi = tid & 31;
    float2 qa, qb, qc, qs;
    {
        const float *qp = p.q + (size_t)(g * group + min(qh, group - 1)) * kHD + 2 * qi;
        qa = *reinterpret_cast<const float2 *>(qp);
        qb = *reinterpret_cast<const float2 *>(qp + kHD / 2);
        qc = *reinterpret_cast<const float2 *>((cos_t ? cos_t : p.q) + 2 * qi);
        qs = *reinterpret_cast<const float2 *>((cos_t ? sin_t : p.q) + 2 * qi);
    }
    float4 kc4, ks4, kn0, kn1, vn;
    {
        kc4 = *reinterpret_cast<const float4 *>((cos_t ? cos_t : p.q) + 4 * l16);
        ks4 = *reinterpret_cast<const float4 *>((cos_t ? sin_t : p.q) + 4 * l16);
        const float *kb = p.k_new ? p.k_new : p.q;
        const float *vb = p.k_new ? p.v_new : p.q;
        kn0 = *reinterpret_cast<const float4 *>(kb + (size_t)g * kHD + 4 * l16);
        kn1 = *reinterpret_cast<const float4 *>(kb + (size_t)g * kHD + kHD / 2 + 4 * l16);
        vn = *reinterpret_cast<const float4 *>(vb + (size_t)g * kHD + 4 * l32);
    }
    asm volatile("" ::: "memory");
    float4 ka[NJ][2];  // K: pass j → row wr0 + 4j + rg
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int t = min(wr0 + 4 * j + rg, tmax);
        const float *src = p.kc + (size_t)t * kvd + g * kHD + 4 * l16;
        ka[j][0] = *reinterpret_cast<const float4 *>(src);
        ka[j][1] = *reinterpret_cast<const float4 *>(src + kHD / 2);
    }
    float4 va[NV];  // V: load k → row wr0 + 2k + half
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int t = min(wr0 + 2 * k + half, tmax);
        va[k] = *reinterpret_cast<const float4 *>(p.vc + (size_t)t * kvd + g * kHD + 4 * l32);
    }

    // every request above is issued before the step state is examined: the
    // memory clobber keeps the loads above this point (the exits below would
    // otherwise let the compiler sink them past), and passing the step
    // state's values through it keeps their first use (and the wait for
    // them) below it
    asm volatile("" : "+v"(st4.x), "+v"(st4.y), "+v"(st4.z), "+v"(st4.w), "+v"(st_rope)::"memory");

    // ---- 2. step state
    if (st && st4.w) return;  // err: a failed step appends nothing
    const int L = st ? st4.x : p.len;
    const int newest = st ? st4.y : -1;  // row appended by this step (clen)
    const bool rope = (st ? st_rope : p.has_rope) && cos_t;
    const int t1 = min(L, t0 + chunk);
    if (t1 <= t0) return;  // split past the step's rows (uniform): the merge skips it

    // ---- 3. the group's q, rotated once per workgroup (thread → one head's
    // pairs 2i, 2i+1) and shared through LDS; the owner wave rotates and
    // appends the newest row
    if (qh < group) {
        if (rope) rope_pair2(qa, qb, qc, qs);
        float *qrow = reinterpret_cast<float *>(&q_lds[qh][0]);
        *reinterpret_cast<float2 *>(qrow + 2 * qi) = qa;
        *reinterpret_cast<float2 *>(qrow + kHD / 2 + 2 * qi) = qb;
    }
    // the newest row's place in this wave (ni = -1: not here); its loaded
    // K/V registers are replaced where they are used, so that no wave waits
    // for its rows before the barrier below
    const int ni = newest >= wr0 && newest < wr0 + RPW && newest < t1 ? newest - wr0 : -1;  // uniform per wave
    if (ni >= 0) {
        if (rope) rope_pair4(kn0, kn1, kc4, ks4);
        if (rg == 0) {
            float *kd = p.kc + (size_t)newest * kvd + g * kHD + 4 * l16;
            *reinterpret_cast<float4 *>(kd) = kn0;
            *reinterpret_cast<float4 *>(kd + kHD / 2) = kn1;
        }
        if (half == 0) *reinterpret_cast<float4 *>(p.vc + (size_t)newest * kvd + g * kHD + 4 * l32) = vn;
    }
    __syncthreads();
    float4 q[kMaxGroup][2];  // score layout
#pragma unroll
    for (int h = 0; h < kMaxGroup; ++h) {
        const int hh = min(h, group - 1);
        q[h][0] = q_lds[hh][l16];
        q[h][1] = q_lds[hh][kHD / 8 + l16];
    }

    // ---- 4. scores; lanes 2h, 2h+1 of each 16-lane row hold head h's score
    const int hs = l16 >> 1;  // this lane's head after the reduce-scatter
    const int jn = ni >= 0 && rg == (ni & 3) ? ni >> 2 : -1;  // pass holding the newest row in this lane
    float sj[NJ];
    bool ok[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        // the newest row's K: a per-lane select (an indexed store would send
        // ka to scratch memory)
        const bool r = jn == j;
        const float4 k0 = make_float4(r ? kn0.x : ka[j][0].x, r ? kn0.y : ka[j][0].y, r ? kn0.z : ka[j][0].z,
                                      r ? kn0.w : ka[j][0].w);
        const float4 k1 = make_float4(r ? kn1.x : ka[j][1].x, r ? kn1.y : ka[j][1].y, r ? kn1.z : ka[j][1].z,
                                      r ? kn1.w : ka[j][1].w);
        float part[8][1];
#pragma unroll
        for (int h = 0; h < kMaxGroup; ++h) {
            float a = 0.0f;
            a = fmaf(q[h][0].x, k0.x, a);
            a = fmaf(q[h][0].y, k0.y, a);
            a = fmaf(q[h][0].z, k0.z, a);
            a = fmaf(q[h][0].w, k0.w, a);
            a = fmaf(q[h][1].x, k1.x, a);
            a = fmaf(q[h][1].y, k1.y, a);
            a = fmaf(q[h][1].z, k1.z, a);
            a = fmaf(q[h][1].w, k1.w, a);
            part[h][0] = a;
        }
        const float sdot = rs16_heads(part, lane);
        ok[j] = wr0 + 4 * j + rg < t1;
        sj[j] = sdot * p.scale;
    }

    // ---- 5. the wave's softmax per head (rows of head hs: NJ passes × 4 lane rows)
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NJ; ++j) m = ok[j] ? fmaxf(m, sj[j]) : m;
    m = fmaxf(m, xchg<XS16>(m));
    m = fmaxf(m, xchg<XS32>(m));
    float ej[NJ], lsum = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        ej[j] = ok[j] ? fast_exp_ref(sj[j] - m) : 0.0f;
        lsum += ej[j];
    }
    lsum += xchg<XS16>(lsum);
    lsum += xchg<XS32>(lsum);
    if ((l16 & 1) == 0 && hs < group) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int r = 4 * j + rg;  // row within the wave
            e_lds[wave][hs][r & 1][r >> 1] = ej[j];
        }
        if (rg == 0) {
            w_m[wave][hs] = m;
            w_l[wave][hs] = lsum;
        }
    }
    // the wave reads back what its own lanes wrote: LDS keeps a wave's
    // accesses in order, the fence keeps the compiler from reordering them
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");

    // ---- 6. Σ e·V for every head over this lane's half of the wave's rows;
    // every head's probabilities are read before the first product
    float4 ev[kMaxGroup][NV / 4];
#pragma unroll
    for (int h = 0; h < kMaxGroup; ++h)
#pragma unroll
        for (int k = 0; k < NV / 4; ++k)
            ev[h][k] = reinterpret_cast<const float4 *>(&e_lds[wave][min(h, group - 1)][half][0])[k];
    asm volatile("" ::: "memory");  // all of them issued here, not one per head
    {
        // the newest row's V: a per-lane select on each register (an
        // indexed store would send va to scratch memory)
        const int nk = ni >= 0 && half == (ni & 1) ? ni >> 1 : -1;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const bool r = nk == k;
            va[k] = make_float4(r ? vn.x : va[k].x, r ? vn.y : va[k].y, r ? vn.z : va[k].z, r ? vn.w : va[k].w);
        }
    }
#pragma unroll
    for (int h = 0; h < kMaxGroup; ++h) {
        if (h >= group) break;
        float e[NV];
#pragma unroll
        for (int k = 0; k < NV / 4; ++k) {
            e[4 * k] = ev[h][k].x;
            e[4 * k + 1] = ev[h][k].y;
            e[4 * k + 2] = ev[h][k].z;
            e[4 * k + 3] = ev[h][k].w;
        }
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            a.x = fmaf(e[k], va[k].x, a.x);
            a.y = fmaf(e[k], va[k].y, a.y);
            a.z = fmaf(e[k], va[k].z, a.z);
            a.w = fmaf(e[k], va[k].w, a.w);
        }
        w_acc[wave][h][half][l32] = a;
    }
    __syncthreads();

    // ---- 7. combine the four waves (two row halves each) → the split's record per head
    const int h = tid >> 5;     // head
    const int d4 = tid & 31;    // dims 4·d4..4·d4+3
    if (h < group) {
        float M = w_m[0][h];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) M = fmaxf(M, w_m[w][h]);  // finite: wave 0 holds row t0
        float lt = 0.0f;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float mw = w_m[w][h];
            const float f = mw == -INFINITY ? 0.0f : fast_exp_ref(mw - M);
            lt = fmaf(f, w_l[w][h], lt);
            const float4 a = w_acc[w][h][0][d4];
            const float4 b = w_acc[w][h][1][d4];
            o.x = fmaf(f, a.x + b.x, o.x);
            o.y = fmaf(f, a.y + b.y, o.y);
            o.z = fmaf(f, a.z + b.z, o.z);
            o.w = fmaf(f, a.w + b.w, o.w);
        }
        float *rh = p.part + ((size_t)(g * p.nsplit + split) * kMaxGroup + h) * kRec;
        if (d4 == 0) *reinterpret_cast<float2 *>(rh) = make_float2(M, lt);
        *reinterpret_cast<float4 *>(rh + 4 + 4 * d4) = o;
    }
}

// Merge of the per-split records, one workgroup per q head (four waves):
// M = max m_s, out = Σ e_s·acc_s / Σ e_s·l_s with e_s = FastExp(m_s − M).
// Wave 0 computes the split weights lane-parallel (lane = split) and hands
// them over in LDS; the 256 threads are 8 split groups × 32 lanes of 4 dims,
// group k summing splits k, k+8, … with 16-byte loads, and the groups' sums
// are added in group order.  A separate launch: the kernel boundary orders
// the record writes before these reads on every XCD.  The first records are
// requested before the step state is read; splits at or past the step's
// length hold stale records and are skipped.
constexpr int kMaxSplits = 1024;  // cache capacity ≤ 65536 rows
constexpr int kMergeThreads = 256;
constexpr int kMergeGroups = kMergeThreads / 32;

// Returns false when the step has failed (nothing written).  The merged head
// (128 floats, 16-byte aligned) goes to dst, by default its head_out slot.
// B: acc vectors each split group requests up front, 8 (splits < 64 in one
// round trip) or 16 (< 128; the host picks 16 above 64 splits)
template <int B = 8>
__device__ __forceinline__ bool attn_merge_body(AttnParams p, float *dst = nullptr) {
    static_assert(B == 8 || B == 16, "8 or 16 acc vectors per split group");
    __shared__ float e_lds[kMaxSplits];
    __shared__ float4 o_lds[kMergeGroups][32];
    __shared__ float l_lds;
    const int hq = blockIdx.x;  // q head
    const int group = p.heads / p.kvh;
    const int g = hq / group, h = hq % group;
    const int t = threadIdx.x, lane = t & 63;
    const int sg = t >> 5, j = t & 31;  // split group, dims 4j..4j+3
    const bool wave0 = t < 64;
    const float *base = p.part + ((size_t)g * p.nsplit * kMaxGroup + h) * kRec;
    constexpr size_t RS = (size_t)kMaxGroup * kRec;  // split stride
    auto acc = [&](int sidx) { return *reinterpret_cast<const float4 *>(base + sidx * RS + 4 + 4 * j); };
    // the step state's header first (len, clen, cap, err; without a step
    // state a readable stand-in), so waiting for it waits for nothing else
    int4 st4 = *reinterpret_cast<const int4 *>(p.st ? reinterpret_cast<const float *>(p.st) : p.part);
    // then (max, Σexp) of split lane (and lane + 64 with B = 16; every wave
    // loads them, only wave 0 uses them: no load inside a branch), then the
    // acc vectors of splits sg + 8b, b < B: with B = 16 every record of up to
    // 128 splits (8,192 rows at 64 rows per split) arrives in one round trip
    const float2 ml = *reinterpret_cast<const float2 *>(base + min(lane, p.nsplit - 1) * RS);
    float2 ml2 = ml;
    if constexpr (B == 16) ml2 = *reinterpret_cast<const float2 *>(base + min(lane + 64, p.nsplit - 1) * RS);
    asm volatile("" ::: "memory");
    float4 av[B];
#pragma unroll
    for (int b = 0; b < B; ++b) av[b] = acc(min(sg + kMergeGroups * b, p.nsplit - 1));
    asm volatile("" : "+v"(st4.x), "+v"(st4.y), "+v"(st4.z), "+v"(st4.w)::"memory");  // requests above, uses below
    if (p.st && st4.w) return false;  // err
    const int L = p.st ? st4.x : p.len;
    const int used = min(p.nsplit, (L + p.chunk - 1) / p.chunk);  // ≥ 1 for L ≥ 1
    if (wave0) {  // split weights, lane s + 64k ↔ split
        // (m, l) of split s: the registers for s < 128, else a load
        constexpr int HELD = B == 16 ? 128 : 64;  // splits whose (m, l) arrived with the requests above
        auto ms_of = [&](int s) { return s < 64 ? ml.x : (s < HELD ? ml2.x : base[s * RS]); };
        auto ls_of = [&](int s) { return s < 64 ? ml.y : (s < HELD ? ml2.y : base[s * RS + 1]); };
        float M = lane < used ? ml.x : -INFINITY;
        for (int s = 64 + lane; s - lane < used; s += 64) M = fmaxf(M, s < used ? ms_of(s) : -INFINITY);
        M = wave_max(M);
        float ls = 0.0f;
        for (int s = lane; s - lane < used; s += 64) {
            float e = 0.0f, lv = 0.0f;
            if (s < used) {
                const float ms = ms_of(s);
                lv = ls_of(s);
                e = fast_exp_ref(ms - M);
                e_lds[s] = e;
            }
            ls = fmaf(e, lv, ls);
        }
        ls = wave_sum(ls);
        if (lane == 0) l_lds = ls;
    }
    __syncthreads();
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    auto add = [&](int s, const float4 &a) {
        const float e = e_lds[s];
        o.x = fmaf(e, a.x, o.x);
        o.y = fmaf(e, a.y, o.y);
        o.z = fmaf(e, a.z, o.z);
        o.w = fmaf(e, a.w, o.w);
    };
#pragma unroll
    for (int b = 0; b < B; ++b)
        if (sg + kMergeGroups * b < used) add(sg + kMergeGroups * b, av[b]);
#pragma unroll 4
    for (int s = sg + kMergeGroups * B; s < used; s += kMergeGroups) add(s, acc(s));
    o_lds[sg][j] = o;
    __syncthreads();
    if (t < 32) {
        float4 r = o_lds[0][t];
#pragma unroll
        for (int k = 1; k < kMergeGroups; ++k) {
            const float4 a = o_lds[k][t];
            r.x += a.x;
            r.y += a.y;
            r.z += a.z;
            r.w += a.w;
        }
        const float inv = 1.0f / l_lds;
        float *o = dst ? dst : p.head_out + (size_t)hq * kHD;
        *reinterpret_cast<float4 *>(o + 4 * t) = make_float4(r.x * inv, r.y * inv, r.z * inv, r.w * inv);
    }
    return true;
}

template <int RPW>
__global__ void __launch_bounds__(kThreads) k_attn_decode(AttnParams args) {
    AttnParams p = args;
    pin_args(p);
    attn_decode_body<RPW>(p);
}
template <int B>
__global__ void __launch_bounds__(kMergeThreads) k_attn_merge(AttnParams args) {
    AttnParams p = args;
    pin_args(p);
    attn_merge_body<B>(p);
}
// acc vectors per split group requested up front for nsplit splits
__host__ __device__ constexpr int merge_prefetch(int nsplit) { return nsplit > 64 ? 16 : 8; }

// ---------------------------------------------------------------------------
// The merge with o_proj folded in, as a split over heads.  Workgroup (q head
// h, row slice s) merges head h exactly as k_attn_merge does, writes its 128
// values as the o_proj GEMV's digit records (x_digits over the head's
// columns: the GEMV's chunks never straddle a head), and multiplies them by
// W_o's columns of head h for its rows:
//   part[h][r] = (Σ over the head's chunks of the GEMV's chunk value)·scale[r].
// The consumer (the gate/up GEMV prologue, PRO_OPART) forms
//   v = h_res + (((part[0] + part[1]) + …) + part[heads−1])
// and RMSNorm(v).  So one launch per layer goes: the o_proj GEMV's.
// ---------------------------------------------------------------------------
constexpr int kOprojSlices = 16;  // row slices per head: heads × 16 workgroups

struct OprojParts {
    DevMat w;      // W_o [rows][heads·128]
    float *part;   // [heads][rows]
};

template <int QT, int B>
__global__ void __launch_bounds__(kMergeThreads) k_attn_merge_oproj(AttnParams args, OprojParts op) {
    constexpr int LPROW = 128 / QTraits<QT>::W;  // lanes per row: one chunk each (Q4 4, Q8/Q6 8)
    constexpr int ROWS_PASS = kMergeThreads / LPROW;
    constexpr int RS = DigitRec<QT>::RS;
    constexpr int MAXP = 4;  // passes of ROWS_PASS rows: up to 4·64 (Q4) / 4·32 rows per slice
    static_assert(kMergeThreads == kThreads, "x_digits runs on kThreads threads");
    __shared__ __attribute__((aligned(16))) float merged[kHD];
    __shared__ __attribute__((aligned(16))) int recs[LPROW * RS];
    __shared__ float red[kWaves];
    AttnParams p = args;
    pin_args(p);
    asm volatile("" ::"s"(op.w.data), "s"(op.w.scale), "s"(op.w.row_bytes), "s"(op.w.rows), "s"(op.part));
    const int hq = blockIdx.x;
    const int t = threadIdx.x;
    const int rows = op.w.rows;
    const int per_slice = (rows + kOprojSlices - 1) / kOprojSlices;
    const int r_begin = blockIdx.y * per_slice;
    const int j = t % LPROW;  // this lane's chunk of the head
    // the weight chunks and row scales of this workgroup's rows, requested
    // before the merge waits for its records (rows past the slice: the last
    // row, loaded and never written)
    Chunk w[MAXP];
    float sc[MAXP];
#pragma unroll
    for (int ps = 0; ps < MAXP; ++ps) {
        if (ps * ROWS_PASS >= per_slice) break;  // uniform
        const int rr = r_begin + ps * ROWS_PASS + t / LPROW;
        const int r = min(rr, rows - 1);
        w[ps] = load_chunk<QT>(op.w.data + (size_t)r * op.w.row_bytes +
                               (size_t)(hq * LPROW + j) * QTraits<QT>::CB);
        sc[ps] = op.w.scale[r];
    }
    if (!attn_merge_body<B>(p, merged)) return;
    __syncthreads();
    // digit records of the head's 128 values (threads 0..15 hold 8 columns each)
    XRegs xr;
    {
        const float4 *mp = reinterpret_cast<const float4 *>(merged);
        const int g = min(t, kHD / 8 - 1);
        xr.x[0][0] = mp[2 * g];
        xr.x[0][1] = mp[2 * g + 1];
#pragma unroll
        for (int pp = 1; pp < kXPasses; ++pp) xr.x[pp][0] = xr.x[pp][1] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    x_digits<QT>(xr, xr, false, kHD, recs, red);
    __syncthreads();
    XDig<QT, 1, 3> xd;
    load_digits<QT, LPROW, 1, 3>(recs, j, xd);
#pragma unroll
    for (int ps = 0; ps < MAXP; ++ps) {
        const int rr = r_begin + ps * ROWS_PASS + t / LPROW;
        if (ps * ROWS_PASS >= per_slice) break;  // uniform
        Chunk wc[1] = {w[ps]};
        const float v = row_dot<QT, 1, 3>(wc, xd);
        // the head's chunk values in chunk order, on the row's first lane
        float acc = 0.0f;
        const int base = (t & 63) - j;
#pragma unroll
        for (int k = 0; k < LPROW; ++k) {
            const float vk = __shfl(v, base + k, 64);
            acc = k == 0 ? vk : acc + vk;
        }
        if (j == 0 && rr < min(rows, r_begin + per_slice)) op.part[(size_t)hq * rows + rr] = acc * sc[ps];
    }
}

// Several sequences in one launch (batched decode): blockIdx.z picks the
// sequence's parameters (its cache, step state, partials, q and output rows);
// splits past a sequence's own count exit at once.
struct AttnMulti {
    AttnParams a[kMaxBatch];
};
static_assert(sizeof(AttnMulti) <= 4096, "kernel arguments of the batched attention");
// b is the kernel's only argument (offset 0 of the argument segment): entry
// blockIdx.z is read in place with scalar loads (a select over the array
// would copy it to scratch).  The argument segment exists in the device pass.
typedef __attribute__((address_space(4))) const AttnParams KernargAttn;
template <int RPW>
__global__ void __launch_bounds__(kThreads) k_attn_decode_multi(AttnMulti b) {
    (void)b;
#if defined(__HIP_DEVICE_COMPILE__)
    const AttnParams p = ((KernargAttn *)__builtin_amdgcn_kernarg_segment_ptr())[blockIdx.z];
    if ((int)blockIdx.y >= p.nsplit) return;  // uniform
    attn_decode_body<RPW>(p);
#endif
}
template <int B>
__global__ void __launch_bounds__(kMergeThreads) k_attn_merge_multi(AttnMulti b) {
    (void)b;
#if defined(__HIP_DEVICE_COMPILE__)
    attn_merge_body<B>(((KernargAttn *)__builtin_amdgcn_kernarg_segment_ptr())[blockIdx.z]);
#endif
}

// Attention for head dims other than 128 (small test shapes): one workgroup
// per q head, serial over rows, same math.
static __global__ void __launch_bounds__(kThreads) k_attn_small(const float *q, const float *kc, const float *vc, int len,
                                                          int heads, int kvh, int dim, float scale, float *out) {
    extern __shared__ float sc_dyn[];
    __shared__ float red[2 * kWaves];
    const int h = blockIdx.x;
    const int g = h / (heads / kvh);
    const int kvd = kvh * dim;
    const float *qh = q + (size_t)h * dim;
    for (int t = threadIdx.x; t < len; t += kThreads) {
        float a = 0.0f;
        for (int d = 0; d < dim; ++d) a = fmaf(qh[d], kc[(size_t)t * kvd + g * dim + d], a);
        sc_dyn[t] = a * scale;
    }
    __syncthreads();
    float m = -INFINITY;
    for (int t = threadIdx.x; t < len; t += kThreads) m = fmaxf(m, sc_dyn[t]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float s = 0.0f;
    for (int t = threadIdx.x; t < len; t += kThreads) {
        const float e = fast_exp_ref(sc_dyn[t] - m);
        sc_dyn[t] = e;
        s += e;
    }
    s = block_sum(s, red + kWaves);
    const float inv = 1.0f / s;
    for (int d = threadIdx.x; d < dim; d += kThreads) {
        float a = 0.0f;
        for (int t = 0; t < len; ++t) a = fmaf(sc_dyn[t], vc[(size_t)t * kvd + g * dim + d], a);
        out[(size_t)h * dim + d] = a * inv;
    }
}

}  // namespace pocr
