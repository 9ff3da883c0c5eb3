// Wide sampling on the device: draws over every LM-head score (top_k 0 or
// >= vocab) and over more than 64 candidates.
//
// Full vocabulary — sampleFullLogitsScratch (internal/model/model.go:
// 2215-2307) with ExpScaledVec's portable loop (weighted_sum.go:314-329,
// dot_other.go:398-411) and CumulativeSum (internal/tensor/cumsum.go:9-58):
//   k_full_weights   one workgroup: the maximum (tensor.Max), then every
//                    weight w_i = FastExpF32(x_i·s + b) with its exponent wrap;
//   k_chain          the running f32 sums the draw reads, exactly in the
//                    reference's order (one workgroup per sum): the total
//                    Σ w_i from index 0, and CumulativeSum's four block sums
//                    (from 4096 entries on), each summed from zero;
//   k_full_pick      pick = float32(Float64()) · total and the binary search
//                    of pickCumulativeFloat32 (model.go:2326-2340) over the
//                    cumulative sums, block b ≥ 1 shifted by the running
//                    block totals as CumulativeSum shifts them.
// Wide candidate sets (64 < top_k < vocab) — matVecTopKMaybeCPU (model.go:
// 7202-7235) returns the k best scores sorted (topKSelectWithWork,
// topk.go:322-345), then sampleCandidateScoresScratch (model.go:1950-1990):
//   k_sort_*         bitonic sort of every (score, row) key, descending;
//   k_cand_weights   the k weights (temperature 1: FastExp(s − max); else
//                    FastExp(s·(1/T) − max·(1/T)));
//   k_chain          their running sum: f32 at temperature 1
//                    (pickWeightedRawFloat32, 2418-2456), f64 otherwise
//                    (pickWeightedFloat32, 2342-2416);
//   k_cand_pick      the first candidate whose running sum reaches the pick.
// Floating-point addition is not associative, so the running sums are
// evaluated in the reference's order, one add after another, by one lane;
// the workgroup's other waves stream the weights into LDS ahead of it and
// the sums back out.
#pragma once

#include "sample.hpp"

namespace pocr {

constexpr int kWideThreads = 1024;
constexpr int kSortTile = 2048;    // keys per workgroup in the LDS bitonic stages
constexpr int kChainChunk = 2048;  // weights per LDS stage of a running sum
constexpr int kChainThreads = 1024;  // threads of a one-by-one running-sum workgroup

// device buffers of the wide sampler (one allocation)
struct WideBufs {
    unsigned long long *keys;  // [N] sorted candidate keys (N = next power of two ≥ n)
    float *w;                  // [n] weights
    float *pre32;              // [n] f32 running sums
    double *pre64;             // [n] f64 running sums
    double *totals;            // [4]
    int *checks;               // [4] check-mode difference counts
    float *bmax;               // [ceil(n / kFullSpan)] workgroup maxima
    double *tsum;              // [ntiles_max]
    int *tbad;                 // [ntiles_max]
    int *tcnt;                 // [2][ntiles_max][2]
    unsigned long long *trs;   // [2][ntiles_max]
    int *cls;                  // [2][n]
    unsigned long long *rr;    // [2][n]
    uint8_t *ev;               // [4] event workspaces
    size_t ev_stride;
};

// ---------------------------------------------------------------------------
// bitonic sort, descending: keys[i] = cand_key(score, row) (0 past n)
// ---------------------------------------------------------------------------

__device__ __forceinline__ void bitonic_pair(unsigned long long *s, int i, int l, bool desc) {
    const unsigned long long a = s[i], b = s[l];
    if (desc ? a < b : a > b) {
        s[i] = b;
        s[l] = a;
    }
}

// tile sort: every workgroup sorts its len = min(N, 2048) keys into the
// bitonic order of the network (tile t descending where bit 2048 of its
// global index is clear), loading them from the scores
static __global__ void __launch_bounds__(kWideThreads) k_sort_tile(const float *scores, int n,
                                                                   unsigned long long *keys, int N,
                                                                   const StepState *st) {
    __shared__ unsigned long long s[kSortTile];
    if (st && st->err) return;
    const int tid = threadIdx.x;
    const int len = N < kSortTile ? N : kSortTile;
    const int base = blockIdx.x * kSortTile;
    for (int i = tid; i < len; i += kWideThreads) {
        const int g = base + i;
        s[i] = g < n ? cand_key(scores[g], g) : 0ull;
    }
    for (int size = 2; size <= len; size <<= 1)
        for (int j = size >> 1; j > 0; j >>= 1) {
            __syncthreads();
            if (tid < len / 2) {
                const int i = 2 * j * (tid / j) + (tid % j);
                bitonic_pair(s, i, i + j, ((base + i) & size) == 0);
            }
        }
    __syncthreads();
    for (int i = tid; i < len; i += kWideThreads) keys[base + i] = s[i];
}

// one compare-exchange stage of distance j ≥ 2048 across the whole array
static __global__ void __launch_bounds__(kWideThreads) k_sort_stage(unsigned long long *keys, int N, int size, int j,
                                                                    const StepState *st) {
    if (st && st->err) return;
    const int t = blockIdx.x * kWideThreads + threadIdx.x;
    if (t >= N / 2) return;
    const int i = 2 * j * (t / j) + (t % j);
    bitonic_pair(keys, i, i + j, (i & size) == 0);
}

// the stages j = 1024 … 1 of a merge of the given size, in LDS per tile
static __global__ void __launch_bounds__(kWideThreads) k_sort_merge(unsigned long long *keys, int N, int size,
                                                                    const StepState *st) {
    __shared__ unsigned long long s[kSortTile];
    if (st && st->err) return;
    const int tid = threadIdx.x;
    const int base = blockIdx.x * kSortTile;
    for (int i = tid; i < kSortTile; i += kWideThreads) s[i] = keys[base + i];
    for (int j = kSortTile / 2; j > 0; j >>= 1) {
        __syncthreads();
        const int i = 2 * j * (tid / j) + (tid % j);
        bitonic_pair(s, i, i + j, ((base + i) & size) == 0);
    }
    __syncthreads();
    for (int i = tid; i < kSortTile; i += kWideThreads) keys[base + i] = s[i];
}

// ---------------------------------------------------------------------------
// chain sets: a weight array in segments and tiles
// ---------------------------------------------------------------------------

constexpr int kCThreads = 1024;            // threads of a chain-set workgroup
constexpr int kCK = 2;                     // consecutive entries per thread
constexpr int kCTile = kCThreads * kCK;    // entries per tile
constexpr int kClsSerial = -0x7FFF;  // class of an entry the walk adds itself

// n weights in nseg consecutive segments of seg_len entries (the last one
// shorter), each cut into tiles of kCTile from its own start.  Sum 0 runs
// over the whole array from index 0 and writes its sums below pre_lim0;
// with nseg = 4 sum q >= 1 runs over segment q from zero (CumulativeSum's
// blocks) and writes that segment's sums.  Per entry and per tile the
// arrays hold two slots: slot 0 for sum 0, slot 1 for the entry's segment
// sum.
struct ChainSet {
    float *w;
    int n, nseg, seg_len, seg_tiles, ntiles;
    int pre_lim0;
    float *pre32;              // f32 sums
    double *pre64;             // f64 sums
    double *totals;            // [4] each sum's last value
    double *tsum;              // [ntiles] f64 sums of the tiles' weights
    int *tbad;                 // [ntiles] a weight negative, infinite or NaN
    int *tcnt;                 // [2][ntiles][2] events starting, SERIAL entries
    unsigned long long *trs;   // [2][ntiles] Σr of REG entries
    int *cls;                  // [2][n] classes
    unsigned long long *rr;    // [2][n] r
    uint8_t *ev;               // [4] event workspaces of ev_stride bytes
    size_t ev_stride;
    int *check;                // [4] check-mode difference counts
};

__device__ __forceinline__ int cs_tb(const ChainSet &S, int t) {
    return (t / S.seg_tiles) * S.seg_len + (t % S.seg_tiles) * kCTile;
}
__device__ __forceinline__ int cs_te(const ChainSet &S, int t) {
    const int q = t / S.seg_tiles;
    const int se = (q + 1) * S.seg_len < S.n ? (q + 1) * S.seg_len : S.n;
    const int e = cs_tb(S, t) + kCTile;
    return e < se ? e : se;
}
// sum q's first tile, its tile count, first entry and entry count
__device__ __forceinline__ int cs_jt0(const ChainSet &S, int q) { return q * S.seg_tiles; }
__device__ __forceinline__ int cs_jtn(const ChainSet &S, int q) {
    if (q == 0) return S.ntiles;
    const int e = q + 1 == S.nseg ? S.ntiles : (q + 1) * S.seg_tiles;
    return e - q * S.seg_tiles;
}
__device__ __forceinline__ int cs_j0(const ChainSet &S, int q) { return q * S.seg_len; }
__device__ __forceinline__ int cs_jm(const ChainSet &S, int q) {
    if (q == 0) return S.n;
    const int e = (q + 1) * S.seg_len < S.n ? (q + 1) * S.seg_len : S.n;
    return e - q * S.seg_len;
}
__device__ __forceinline__ int cs_prelim(const ChainSet &S, int q) { return q == 0 ? S.pre_lim0 : cs_jm(S, q); }

// ---------------------------------------------------------------------------
// workgroup helpers (kCThreads threads)
// ---------------------------------------------------------------------------

struct WgLds {
    double d[kCThreads / 64];
    unsigned long long u[kCThreads / 64];
    int i0[kCThreads / 64], i1[kCThreads / 64];
    int edge[kCThreads / 64];  // each wave's last class
    int flag;
};

// wave sum by butterfly (every lane gets the sum)
template <typename V> __device__ __forceinline__ V wave_sum(V v) {
    for (int off = 32; off > 0; off >>= 1) v = v + __shfl_xor(v, off, 64);
    return v;
}

// workgroup sum of v, the same order in every workgroup
__device__ double wg_sum_f64(double v, WgLds &L) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) L.d[wid] = v;
    __syncthreads();
    return wave_sum(lane < kCThreads / 64 ? L.d[lane] : 0.0);
}

// inclusive workgroup scans in thread order of (a, b, c), with totals
__device__ void wg_scan3(int &a, int &b, unsigned long long &c, WgLds &L, int *ta, int *tb,
                         unsigned long long *tc) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    for (int off = 1; off < 64; off <<= 1) {
        const int oa = __shfl_up(a, off, 64), ob = __shfl_up(b, off, 64);
        const unsigned long long oc = __shfl_up(c, off, 64);
        if (lane >= off) {
            a += oa;
            b += ob;
            c += oc;
        }
    }
    __syncthreads();
    if (lane == 63) {
        L.i0[wid] = a;
        L.i1[wid] = b;
        L.u[wid] = c;
    }
    __syncthreads();
    const bool in = lane < kCThreads / 64, lo = lane < wid;
    const int pa = in ? L.i0[lane] : 0, pb = in ? L.i1[lane] : 0;
    const unsigned long long pc = in ? L.u[lane] : 0ull;
    *ta = wave_sum(pa);
    *tb = wave_sum(pb);
    *tc = wave_sum(pc);
    a += wave_sum(lo ? pa : 0);
    b += wave_sum(lo ? pb : 0);
    c += wave_sum(lo ? pc : 0ull);
}

// exclusive f64 scan in thread order, adds only
__device__ double wg_exscan_f64(double v, WgLds &L) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    double inc = v;
    for (int off = 1; off < 64; off <<= 1) {
        const double o = __shfl_up(inc, off, 64);
        if (lane >= off) inc = inc + o;
    }
    double ex = __shfl_up(inc, 1, 64);
    if (lane == 0) ex = 0.0;
    __syncthreads();
    if (lane == 63) L.d[wid] = inc;
    __syncthreads();
    const double part = lane < kCThreads / 64 ? L.d[lane] : 0.0;
    return wave_sum(lane < wid ? part : 0.0) + ex;
}

// the class of the previous thread's entry (kClsSerial for thread 0)
__device__ int wg_prev_cls(int c, WgLds &L) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    int p = __shfl_up(c, 1, 64);
    __syncthreads();
    if (lane == 63) L.edge[wid] = c;
    __syncthreads();
    if (lane == 0) p = wid > 0 ? L.edge[wid - 1] : kClsSerial;
    return p;
}

// any thread's flag
__device__ bool wg_any(int f, WgLds &L) {
    __syncthreads();
    if (threadIdx.x == 0) L.flag = 0;
    __syncthreads();
    if (f) L.flag = 1;
    __syncthreads();
    return L.flag != 0;
}

// ---------------------------------------------------------------------------
// weights (one tile per workgroup), with each tile's f64 sum and bad flag
// ---------------------------------------------------------------------------

__device__ void tile_sum_out(const ChainSet &S, double ls, int bad, WgLds &L) {
    const double t = wg_sum_f64(ls, L);
    const bool b = wg_any(bad, L);
    if (threadIdx.x == 0) {
        S.tsum[blockIdx.x] = t;
        S.tbad[blockIdx.x] = b;
    }
}

__device__ __forceinline__ int bad_weight(float v) { return !(v >= 0.0f && v <= 3.4028234663852886e38f); }

// sampleFullLogitsScratch's weights: the workgroup maxima of x[1..n) in
// spans of kFullSpan (entries compared with v > m, so NaN entries drop out),
// then per tile the maximum — x[0] first, as tensor.Max takes it, NaN if
// x[0] is — and the weights: T = float32(temperature); T == 1:
// v = x·1 + (−m); otherwise v = x·(1/T) + (−(m·(1/T))); w = FastExpF32(v)
constexpr int kFullThreads = 256;
constexpr int kFullSpan = 1024;

static __global__ void __launch_bounds__(kFullThreads) k_full_max(const float *x, int n, float *bmax,
                                                                  const StepState *st) {
    __shared__ float red[kFullThreads / 64];
    if (st && st->err) return;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int base = blockIdx.x * kFullSpan;
    float m = -__builtin_inff();
    for (int i = tid; i < kFullSpan; i += kFullThreads) {
        const int j = base + i;
        if (j >= 1 && j < n) {
            const float v = x[j];
            m = v > m ? v : m;
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    if (lane == 0) red[wid] = m;
    __syncthreads();
    if (tid == 0) {
        float r = red[0];
        for (int i = 1; i < kFullThreads / 64; ++i) r = red[i] > r ? red[i] : r;
        bmax[blockIdx.x] = r;
    }
}

static __global__ void __launch_bounds__(kCThreads) k_full_weights(const float *x, const float *bmax, int nb,
                                                                   const SampleState *ss, ChainSet S,
                                                                   const StepState *st) {
#pragma clang fp contract(off)
    __shared__ WgLds L;
    if (st && st->err) return;
    // every wave reduces the workgroup maxima itself
    float m = -__builtin_inff();
    for (int i = threadIdx.x & 63; i < nb; i += 64) {
        const float v = bmax[i];
        m = v > m ? v : m;
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    const float first = x[0];
    m = first != first ? first : (first > m ? first : m);
    const float T = (float)ss->temperature;
    float scale = 1.0f, bias = -m;
    if (T != 1.0f) {
        scale = 1.0f / T;
        bias = -(m * scale);
    }
    const int j0 = cs_tb(S, blockIdx.x) + (int)threadIdx.x * kCK, te = cs_te(S, blockIdx.x);
    double ls = 0.0;
    int bad = 0;
#pragma unroll
    for (int e = 0; e < kCK; ++e)
        if (j0 + e < te) {
            const float v = fast_exp_wrap(x[j0 + e] * scale + bias);
            S.w[j0 + e] = v;
            ls = ls + (double)v;
            bad |= bad_weight(v);
        }
    tile_sum_out(S, ls, bad, L);
}

__device__ __forceinline__ float key_score(unsigned long long k) { return score_of((uint32_t)(k >> 32)); }
__device__ __forceinline__ int key_row(unsigned long long k) { return (int)(0xFFFFFFFFu - (uint32_t)k); }

// sampleCandidateScoresScratch's weights over the k (> 4) best keys, sorted
// by score: the maximum the reference takes over them (max32Local in
// candidate order) is the first one's score
static __global__ void __launch_bounds__(kCThreads) k_cand_weights(const unsigned long long *keys,
                                                                   const SampleState *ss, ChainSet S,
                                                                   const StepState *st) {
#pragma clang fp contract(off)
    __shared__ WgLds L;
    if (st && st->err) return;
    const float m = key_score(keys[0]);
    const double temp = ss->temperature;
    const float inv = (float)(1.0 / temp);
    const int j0 = cs_tb(S, blockIdx.x) + (int)threadIdx.x * kCK, te = cs_te(S, blockIdx.x);
    double ls = 0.0;
    int bad = 0;
#pragma unroll
    for (int e = 0; e < kCK; ++e)
        if (j0 + e < te) {
            const float sc = key_score(keys[j0 + e]);
            const float v = temp == 1.0 ? fast_exp_wrap(sc - m) : fast_exp_wrap(sc * inv - m * inv);
            S.w[j0 + e] = v;
            ls = ls + (double)v;
            bad |= bad_weight(v);
        }
    tile_sum_out(S, ls, bad, L);
}

// ---------------------------------------------------------------------------
// running sums
// ---------------------------------------------------------------------------

// stage weights [base, base + cnt) into LDS, zero-padded to a multiple of 4
// (adding +0 leaves every running sum as it is: the sums start at +0)
__device__ __forceinline__ void chain_stage(const float *w, int base, int cnt, float *dst, int t0, int nt) {
    const int cnt4 = (cnt + 3) & ~3;
    for (int i = t0; i < cnt4; i += nt) dst[i] = i < cnt ? w[base + i] : 0.0f;
}

template <typename T>
__device__ __forceinline__ void chain_flush(const T *src, int base, int cnt, int lim, T *pre, int t0, int nt) {
    if (!pre) return;
    const int e = lim - base < cnt ? lim - base : cnt;
    for (int i = t0; i < e; i += nt) pre[base + i] = src[i];
}

// c_{j+1} = c_j + w_j from c_0 = 0, one add after another by thread 0 while
// waves 1.. stage the next chunk in and the previous chunk's sums out;
// pre[j] = c_{j+1} for j < pre_lim, *total = c_m
template <typename T>
__device__ void chain_serial(const float *w, int m, T *pre, int pre_lim, double *total, float (*in)[kChainChunk],
                             T (*out)[kChainChunk]) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x;
    const int nch = (m + kChainChunk - 1) / kChainChunk;
    T c = 0;
    if (nch > 0) chain_stage(w, 0, m < kChainChunk ? m : kChainChunk, in[0], tid, kChainThreads);
    __syncthreads();
    for (int k = 0; k < nch; ++k) {
        const int cur = k & 1;
        const int base = k * kChainChunk;
        const int cnt = m - base < kChainChunk ? m - base : kChainChunk;
        if (tid == 0) {
            const float4 *src = reinterpret_cast<const float4 *>(in[cur]);
            T *o = out[cur];
            const int n4 = (cnt + 3) >> 2;
#pragma unroll 4
            for (int q = 0; q < n4; ++q) {
                const float4 v = src[q];
                c = c + (T)v.x;
                o[4 * q] = c;
                c = c + (T)v.y;
                o[4 * q + 1] = c;
                c = c + (T)v.z;
                o[4 * q + 2] = c;
                c = c + (T)v.w;
                o[4 * q + 3] = c;
            }
        } else if (tid >= 64) {
            if (k + 1 < nch) {
                const int nb = base + kChainChunk;
                chain_stage(w, nb, m - nb < kChainChunk ? m - nb : kChainChunk, in[cur ^ 1], tid - 64,
                            kChainThreads - 64);
            }
            if (k > 0) chain_flush<T>(out[cur ^ 1], base - kChainChunk, kChainChunk, pre_lim, pre, tid - 64,
                                      kChainThreads - 64);
        }
        __syncthreads();
    }
    if (nch > 0) {
        const int base = (nch - 1) * kChainChunk;
        chain_flush<T>(out[(nch - 1) & 1], base, m - base, pre_lim, pre, tid, kChainThreads);
    }
    if (tid == 0) *total = (double)c;
    __syncthreads();
}

// The same sums in parallel.  While a running sum c stays in one binade
// [2^E, 2^(E+1)), every add lands on the grid u = 2^(E−P) (P = 23 for f32,
// 52 for f64): c + x rounds to c + u·rint(x/u) unless x/u is a tie.  A run of
// adds in one binade is therefore an integer prefix sum of r = rint(x/u),
// independent of where the run starts.  Each entry is classed from the
// exact-arithmetic prefix P_j (f64): REG(E) when c_j and c_j + x_j sit well
// inside binade E of P_j, SERIAL near a binade edge, at a tie, or near the
// subnormal range.  Consecutive entries of one class in one tile form an
// event.  One wave then walks a sum's events in order: a REG run whose start
// c lies in binade E and whose end M = c/u + Σr stays below 2^(P+1) is exact
// by induction (every partial sum is a grid point of binade E, every exact
// sum is below 2^(E+1) − u/2, so hardware rounding picks the same point);
// a run failing that check, and every SERIAL entry, is added one by one.
// Launches: k_chain_cls (classes, per tile), k_chain_compact (events, per
// tile), k_chain_walk (one workgroup per sum), k_chain_fin (every entry's
// sum, per tile).  Weights that are negative, infinite or NaN (FastExp's
// wrap), or totals near the top of the range, take chain_serial in the walk.


template <typename T> struct ChainFmt;
template <> struct ChainFmt<float> {
    static constexpr int P = 23;
    static constexpr double lo_lim = 0x1p-124;  // smallest classed prefix (grids stay normal)
    static constexpr double hi_lim = 0x1p126;   // largest total taken in parallel
    static constexpr double eps = 0x1p-24;
    static constexpr double tol0 = 0x1p-20;
};
template <> struct ChainFmt<double> {
    static constexpr int P = 52;
    static constexpr double lo_lim = 0x1p-1020;
    static constexpr double hi_lim = 0x1p1022;
    static constexpr double eps = 0x1p-53;
    static constexpr double tol0 = 0x1p-48;
};

// per-sum event workspace (device memory), carved by chain_work
struct ChainWork {
    int *ev_a, *ev_kind, *ev_len;          // event start (within the sum), class, length
    unsigned long long *ev_r0, *ev_rs;     // Σr before the event, Σr over it
    double *ev_c0;                         // the sum at a run's start (−1: the walk added the run itself)
    float *sw;                             // SERIAL entries' weights, in order
    double *spre;                          // their sums
    double *chk;                           // check mode: the one-by-one sums
};

__host__ __device__ inline size_t chain_align(size_t b) { return (b + 255) & ~(size_t)255; }
__host__ __device__ inline size_t chain_work_bytes(int m) {
    const size_t ne = (size_t)m + 8;
    return 3 * chain_align(ne * 4) + 3 * chain_align(ne * 8) + chain_align((size_t)m * 4) +
           2 * chain_align((size_t)m * 8);
}
__device__ inline ChainWork chain_work(uint8_t *p, int m) {
    const size_t ne = (size_t)m + 8;
    ChainWork W;
    W.ev_a = reinterpret_cast<int *>(p);
    p += chain_align(ne * 4);
    W.ev_kind = reinterpret_cast<int *>(p);
    p += chain_align(ne * 4);
    W.ev_len = reinterpret_cast<int *>(p);
    p += chain_align(ne * 4);
    W.ev_r0 = reinterpret_cast<unsigned long long *>(p);
    p += chain_align(ne * 8);
    W.ev_rs = reinterpret_cast<unsigned long long *>(p);
    p += chain_align(ne * 8);
    W.ev_c0 = reinterpret_cast<double *>(p);
    p += chain_align(ne * 8);
    W.sw = reinterpret_cast<float *>(p);
    p += chain_align((size_t)m * 4);
    W.spre = reinterpret_cast<double *>(p);
    p += chain_align((size_t)m * 8);
    W.chk = reinterpret_cast<double *>(p);
    return W;
}

// class of an entry (weight x, exact-arithmetic prefix P ≈ c_j, relative
// tolerance tol for |c_j − P|): the binade E with r = rint(x / 2^(E−P)), or
// kClsSerial.  A guess only: the walk checks every run before it trusts one.
__device__ __forceinline__ int dexp(double v) { return (int)((__double_as_longlong(v) >> 52) & 0x7FF) - 1023; }
__device__ __forceinline__ double dpow2(int e) { return __longlong_as_double((long long)(e + 1023) << 52); }

template <typename T>
__device__ __forceinline__ int chain_cls(double P, float x, double tol, unsigned long long &r) {
    using F = ChainFmt<T>;
    const double lo = P * (1.0 - tol);
    if (!(lo >= F::lo_lim)) return kClsSerial;
    const double hi = (P + (double)x) * (1.0 + tol);
    const int E = dexp(lo);
    if (dexp(hi) != E) return kClsSerial;
    if (sizeof(T) == 4 && E > -100) {
        // x·2^(23−E) < 2^24: exact in f32 (an underflow only drops bits far
        // below ½, which leaves r = 0 and no tie)
        const float q = x * __int_as_float((150 - E) << 23);
        const unsigned fq = (unsigned)q;
        const float fr = q - (float)fq;
        if (fr == 0.5f) return kClsSerial;
        r = fq + (fr > 0.5f);
    } else {
        const double q = (double)x * dpow2(F::P - E);  // < 2^53, exact
        const unsigned long long fq = (unsigned long long)q;
        const double fr = q - (double)fq;
        if (fr == 0.5) return kClsSerial;
        r = fq + (fr > 0.5);
    }
    return E;
}

// the tolerance of a thread's entries (up to index j1)
template <typename T> __device__ __forceinline__ double chain_tol(int j1) {
    using F = ChainFmt<T>;
    return F::tol0 + 32.0 * F::eps * sqrt((double)j1 + 1.0);
}

__device__ __forceinline__ int rl_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ float rl_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ unsigned long long rl_u64(unsigned long long v, int l) {
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)v, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(v >> 32), l);
    return ((unsigned long long)hi << 32) | lo;
}

// wave 0: c + w[a] + … + w[a+len−1] one by one (the whole wave in step,
// lane i keeping the i-th sum of each 64-entry chunk), sums into pre
template <typename T>
__device__ T wave_add_run(const float *w, int a, int len, T c, T *pre, int pre_lim) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    for (int base = a; base < a + len; base += 64) {
        const int cnt = a + len - base < 64 ? a + len - base : 64;
        const float v = lane < cnt ? w[base + lane] : 0.0f;
        T o = 0;
        for (int i = 0; i < cnt; ++i) {
            c = c + (T)rl_f(v, i);
            if (lane == i) o = c;
        }
        if (lane < cnt && base + lane < pre_lim) pre[base + lane] = o;
    }
    return c;
}

__device__ __forceinline__ bool same_bits(float a, float b) { return __float_as_uint(a) == __float_as_uint(b); }
__device__ __forceinline__ bool same_bits(double a, double b) {
    return __double_as_longlong(a) == __double_as_longlong(b);
}

// sums as integers on their binade's grid: c = M·2^(E−P), 2^P <= M < 2^(P+1)
template <typename T> __device__ __forceinline__ unsigned long long bits_of(T c);
template <> __device__ __forceinline__ unsigned long long bits_of<float>(float c) { return __float_as_uint(c); }
template <> __device__ __forceinline__ unsigned long long bits_of<double>(double c) {
    return (unsigned long long)__double_as_longlong(c);
}
// the significand M of c (bits b, c >= 0) when c lies in binade E, else 0
template <typename T> __device__ __forceinline__ unsigned long long significand_bits(unsigned long long b, int E) {
    using F = ChainFmt<T>;
    constexpr int bias = sizeof(T) == 4 ? 127 : 1023;
    const unsigned long long one = 1ull << F::P;
    return (b >> F::P) == (unsigned long long)(E + bias) ? (b & (one - 1)) | one : 0ull;
}
template <typename T> __device__ __forceinline__ unsigned long long significand_in(T c, int E) {
    return significand_bits<T>(bits_of<T>(c), E);
}
template <typename T> __device__ __forceinline__ T from_bits(unsigned long long b);
template <> __device__ __forceinline__ float from_bits<float>(unsigned long long b) { return __uint_as_float((unsigned)b); }
template <> __device__ __forceinline__ double from_bits<double>(unsigned long long b) {
    return __longlong_as_double((long long)b);
}
__device__ __forceinline__ unsigned long long uniform_u64(unsigned long long b) {
    const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)b);
    const unsigned hi = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)(b >> 32));
    return ((unsigned long long)hi << 32) | lo;
}
// bits of a value every lane of the wave holds, as a wave-uniform value
template <typename T> __device__ __forceinline__ unsigned long long uniform_bits(T c) {
    const unsigned long long b = bits_of<T>(c);
    const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)b);
    if (sizeof(T) == 4) return lo;
    const unsigned hi = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)(b >> 32));
    return ((unsigned long long)hi << 32) | lo;
}
// the bits of M·2^(E−P) for 2^P <= M < 2^(P+1)
template <typename T> __device__ __forceinline__ unsigned long long bits_with_significand(int E, unsigned long long M) {
    using F = ChainFmt<T>;
    constexpr int bias = sizeof(T) == 4 ? 127 : 1023;
    return ((unsigned long long)(E + bias) << F::P) | (M & ((1ull << F::P) - 1));
}
template <typename T> __device__ __forceinline__ T with_significand(int E, unsigned long long M) {
    return from_bits<T>(bits_with_significand<T>(E, M));
}

// f64 sums when `by_temperature` and the sampler's temperature is not 1
__device__ __forceinline__ bool chain_f64(const SampleState *ss, int by_temperature) {
    return by_temperature && ss->temperature != 1.0;
}

// the sum a (tile, slot) block works on, or −1; sums on chain_serial are
// skipped here (mode 1, or a bad weight anywhere in the sum)
__device__ int chain_block_sum(const ChainSet &S, int mode, WgLds &L) {
    const int t = blockIdx.x, slot = blockIdx.y;
    const int seg = t / S.seg_tiles;
    if (slot == 1 && seg == 0) return -1;
    const int q = slot == 0 ? 0 : seg;
    if (mode == 1) return -1;
    const int t0 = cs_jt0(S, q), tn = cs_jtn(S, q);
    int bad = 0;
    for (int u = threadIdx.x; u < tn; u += kCThreads) bad |= S.tbad[t0 + u];
    return wg_any(bad, L) ? -1 : q;
}

// Σ over the sum's tiles before this one: tile sums (f64), events, SERIAL
// entries and Σr of slot `slot`
__device__ void chain_before(const ChainSet &S, int q, int slot, WgLds &L, double *P0, int *E0, int *S0,
                             unsigned long long *R0) {
    const int t0 = cs_jt0(S, q), t = blockIdx.x;
    double p = 0.0;
    int e = 0, sn = 0;
    unsigned long long r = 0;
    for (int u = t0 + (int)threadIdx.x; u < t; u += kCThreads) {
        p = p + S.tsum[u];
        e += S.tcnt[(slot * S.ntiles + u) * 2];
        sn += S.tcnt[(slot * S.ntiles + u) * 2 + 1];
        r += S.trs[slot * S.ntiles + u];
    }
    *P0 = wg_sum_f64(p, L);
    int te, ts;
    unsigned long long tr;
    wg_scan3(e, sn, r, L, &te, &ts, &tr);
    *E0 = te;
    *S0 = ts;
    *R0 = tr;
}

// this thread's kCK consecutive entries of the tile
__device__ __forceinline__ void chain_rows(const ChainSet &S, int *j0, int *cnt) {
    const int t = blockIdx.x;
    *j0 = cs_tb(S, t) + (int)threadIdx.x * kCK;
    const int c = cs_te(S, t) - *j0;
    *cnt = c < 0 ? 0 : (c < kCK ? c : kCK);
}

template <typename T>
__device__ void chain_cls_tile(const ChainSet &S, int q, WgLds &L) {
    const int slot = blockIdx.y, t = blockIdx.x;
    double P0;
    int E0, S0;
    unsigned long long R0;
    chain_before(S, q, slot, L, &P0, &E0, &S0, &R0);
    int j0, cnt;
    chain_rows(S, &j0, &cnt);
    float x[kCK];
    double ls = 0.0;
#pragma unroll
    for (int e = 0; e < kCK; ++e) {
        x[e] = e < cnt ? S.w[j0 + e] : 0.0f;
        ls = ls + (double)x[e];
    }
    double P = P0 + wg_exscan_f64(ls, L);
    const double tol = chain_tol<T>(j0 + cnt - cs_j0(S, q));
    int c[kCK];
    unsigned long long r[kCK];
#pragma unroll
    for (int e = 0; e < kCK; ++e) {
        r[e] = 0;
        c[e] = kClsSerial;
        if (e < cnt) {
            c[e] = chain_cls<T>(P, x[e], tol, r[e]);
            P = P + (double)x[e];
        }
    }
    int last = kClsSerial;
#pragma unroll
    for (int e = 0; e < kCK; ++e)
        if (e < cnt) last = c[e];
    const int pc = wg_prev_cls(last, L);
    int nev = 0, nser = 0;
    unsigned long long rs = 0;
#pragma unroll
    for (int e = 0; e < kCK; ++e)
        if (e < cnt) {
            nev += e == 0 ? (threadIdx.x == 0 || c[0] != pc) : c[e] != c[e - 1];
            if (c[e] == kClsSerial) ++nser;
            else rs += r[e];
            S.cls[(size_t)slot * S.n + j0 + e] = c[e];
            S.rr[(size_t)slot * S.n + j0 + e] = r[e];
        }
    int te, ts;
    unsigned long long tr;
    wg_scan3(nev, nser, rs, L, &te, &ts, &tr);
    if (threadIdx.x == 0) {
        S.tcnt[(slot * S.ntiles + t) * 2] = te;
        S.tcnt[(slot * S.ntiles + t) * 2 + 1] = ts;
        S.trs[slot * S.ntiles + t] = tr;
    }
}

// classes: grid (ntiles, nseg > 1 ? 2 : 1)
static __global__ void __launch_bounds__(kCThreads) k_chain_cls(ChainSet S, const SampleState *ss, int by_temperature,
                                                                int mode, const StepState *st) {
    __shared__ WgLds L;
    if (st && st->err) return;
    const int q = chain_block_sum(S, mode, L);
    if (q < 0) return;
    if (chain_f64(ss, by_temperature)) chain_cls_tile<double>(S, q, L);
    else chain_cls_tile<float>(S, q, L);
}

// a thread's entries with their classes, r and event starts, and what came
// before them in the sum: the event of the entry before the first (ev0),
// SERIAL entries (s0) and Σr (r0)
struct TileRows {
    int j0, cnt;
    int c[kCK];
    unsigned long long r[kCK];
    bool st[kCK];
    int ev0, s0;
    unsigned long long r0;
};

__device__ __forceinline__ TileRows chain_scan_tile(const ChainSet &S, int q, WgLds &L) {
    const int slot = blockIdx.y;
    TileRows z;
    double P0;
    int E0, S0;
    unsigned long long R0;
    chain_before(S, q, slot, L, &P0, &E0, &S0, &R0);
    chain_rows(S, &z.j0, &z.cnt);
#pragma unroll
    for (int e = 0; e < kCK; ++e) {
        z.c[e] = e < z.cnt ? S.cls[(size_t)slot * S.n + z.j0 + e] : kClsSerial;
        z.r[e] = e < z.cnt ? S.rr[(size_t)slot * S.n + z.j0 + e] : 0ull;
    }
    int last = kClsSerial;
#pragma unroll
    for (int e = 0; e < kCK; ++e)
        if (e < z.cnt) last = z.c[e];
    const int pc = wg_prev_cls(last, L);
    int nev = 0, nser = 0;
    unsigned long long rs = 0;
#pragma unroll
    for (int e = 0; e < kCK; ++e) {
        z.st[e] = e < z.cnt && (e == 0 ? (threadIdx.x == 0 || z.c[0] != pc) : z.c[e] != z.c[e - 1]);
        nev += z.st[e];
        if (e < z.cnt) {
            if (z.c[e] == kClsSerial) ++nser;
            else rs += z.r[e];
        }
    }
    int ie = nev, is = nser;
    unsigned long long ir = rs;
    int te, ts;
    unsigned long long tr;
    wg_scan3(ie, is, ir, L, &te, &ts, &tr);
    z.ev0 = E0 + ie - nev - 1;
    z.s0 = S0 + is - nser;
    z.r0 = R0 + ir - rs;
    return z;
}

// events and SERIAL weights in entry order
static __global__ void __launch_bounds__(kCThreads) k_chain_compact(ChainSet S, int mode, const StepState *st) {
    __shared__ WgLds L;
    if (st && st->err) return;
    const int q = chain_block_sum(S, mode, L);
    if (q < 0) return;
    const TileRows z = chain_scan_tile(S, q, L);
    ChainWork W = chain_work(S.ev + (size_t)q * S.ev_stride, cs_jm(S, q));
    const int js = cs_j0(S, q);
    int idx = z.ev0, sidx = z.s0;
    unsigned long long R = z.r0;
#pragma unroll
    for (int e = 0; e < kCK; ++e)
        if (e < z.cnt) {
            if (z.st[e]) {
                ++idx;
                W.ev_a[idx] = z.j0 + e - js;
                W.ev_kind[idx] = z.c[e];
                W.ev_r0[idx] = R;
            }
            if (z.c[e] == kClsSerial) W.sw[sidx++] = S.w[z.j0 + e];
            else R += z.r[e];
        }
}

template <typename T>
__device__ void chain_walk(const ChainSet &S, int q, T *pre, float (*in)[kChainChunk], T (*out)[kChainChunk],
                           bool serial, WgLds &L) {
#pragma clang fp contract(off)
    using F = ChainFmt<T>;
    const int m = cs_jm(S, q), pre_lim = cs_prelim(S, q);
    const float *w = S.w + cs_j0(S, q);
    double *total = S.totals + q;
    if (serial) {
        chain_serial<T>(w, m, pre, pre_lim, total, in, out);
        return;
    }
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    ChainWork W = chain_work(S.ev + (size_t)q * S.ev_stride, m);
    const int slot = q == 0 ? 0 : 1, t0 = cs_jt0(S, q), tn = cs_jtn(S, q);
    int e = 0, sn = 0;
    unsigned long long r = 0;
    for (int u = tid; u < tn; u += kCThreads) {
        e += S.tcnt[(slot * S.ntiles + t0 + u) * 2];
        sn += S.tcnt[(slot * S.ntiles + t0 + u) * 2 + 1];
        r += S.trs[slot * S.ntiles + t0 + u];
    }
    int NE, NS;
    unsigned long long RT;
    wg_scan3(e, sn, r, L, &NE, &NS, &RT);
    if (tid == 0) {
        W.ev_a[NE] = m;
        W.ev_r0[NE] = RT;
    }
    __syncthreads();
    for (int k = tid; k < NE; k += kCThreads) {
        W.ev_len[k] = W.ev_a[k + 1] - W.ev_a[k];
        W.ev_rs[k] = W.ev_r0[k + 1] - W.ev_r0[k];
    }
    __syncthreads();
    if (wid != 0) return;
    NE = __builtin_amdgcn_readfirstlane(NE);  // equal in every lane: let the loops run on scalars
    NS = __builtin_amdgcn_readfirstlane(NS);
    // The wave keeps the running sum as uniform bits (scalar registers): the
    // run steps are integer work on them, and each one-by-one add goes
    // through the vector unit and back.
    unsigned long long cb = 0;
    int scur = 0, sb = 0;
    float sv = lane < NS ? W.sw[lane] : 0.0f;
    T so = 0;
    for (int e0 = 0; e0 < NE; e0 += 64) {
        const int k = e0 + lane;
        int a_l = 0, k_l = kClsSerial, n_l = 0;
        unsigned long long rs_l = 0;
        if (k < NE) {
            a_l = W.ev_a[k];
            k_l = W.ev_kind[k];
            n_l = W.ev_len[k];
            rs_l = W.ev_rs[k];
        }
        double c0_l = -1.0;  // lane i: the sum at event e0 + i's start if it is a checked run
        const int ne = NE - e0 < 64 ? NE - e0 : 64;
        for (int i = 0; i < ne; ++i) {
            const int kind = rl_i(k_l, i), len = rl_i(n_l, i);
            if (kind == kClsSerial) {
                for (int h = 0; h < len; ++h) {
                    const int sl = scur - sb;
                    const T c = from_bits<T>(cb) + (T)rl_f(sv, sl);
                    if (lane == sl) so = c;
                    cb = uniform_bits<T>(c);
                    if (++scur - sb == 64) {
                        W.spre[sb + lane] = (double)so;
                        sb += 64;
                        sv = sb + lane < NS ? W.sw[sb + lane] : 0.0f;
                    }
                }
            } else {
                // c in binade E (c >= 0 here): its exponent field is E + bias and
                // c = M·2^(E−P) with M its significand; the run moves M by Σr
                const int E = kind;
                const unsigned long long M = significand_bits<T>(cb, E), Mb = M + rl_u64(rs_l, i);
                if (M != 0ull && Mb < (1ull << (F::P + 1))) {
                    c0_l = lane == i ? (double)from_bits<T>(cb) : c0_l;
                    cb = bits_with_significand<T>(E, Mb);
                } else {
                    const T c = wave_add_run<T>(w, rl_i(a_l, i), len, from_bits<T>(cb), pre, pre_lim);
                    cb = uniform_bits<T>(c);
                }
            }
            cb = uniform_u64(cb);
        }
        if (k < NE) W.ev_c0[k] = c0_l;
    }
    if (lane < scur - sb) W.spre[sb + lane] = (double)so;
    if (lane == 0) *total = (double)from_bits<T>(cb);
}

// one workgroup per sum
static __global__ void __launch_bounds__(kCThreads) k_chain_walk(ChainSet S, const SampleState *ss, int by_temperature,
                                                              int mode, const StepState *st) {
    __shared__ __align__(16) float in[2][kChainChunk];
    __shared__ __align__(16) double out[2][kChainChunk];
    __shared__ WgLds L;
    if (st && st->err) return;
    const int q = blockIdx.x;
    const int t0 = cs_jt0(S, q), tn = cs_jtn(S, q);
    int bad = 0;
    for (int u = threadIdx.x; u < tn; u += kCThreads) bad |= S.tbad[t0 + u];
    const bool serial = mode == 1 || wg_any(bad, L);
    const int j0 = cs_j0(S, q);
    if (chain_f64(ss, by_temperature)) {
        chain_walk<double>(S, q, S.pre64 + j0, in, out, serial, L);
    } else {
        chain_walk<float>(S, q, S.pre32 + j0, in, reinterpret_cast<float(*)[kChainChunk]>(out), serial, L);
    }
}

template <typename T>
__device__ void chain_fin_tile(const ChainSet &S, int q, T *pre, WgLds &L) {
    const TileRows z = chain_scan_tile(S, q, L);
    ChainWork W = chain_work(S.ev + (size_t)q * S.ev_stride, cs_jm(S, q));
    const int js = cs_j0(S, q), lim = cs_prelim(S, q);
    int idx = z.ev0, sidx = z.s0;
    unsigned long long R = z.r0, Ra = 0;
    double c0 = -1.0;
    if (z.cnt > 0 && !z.st[0] && z.c[0] != kClsSerial) {
        c0 = W.ev_c0[idx];
        Ra = W.ev_r0[idx];
    }
#pragma unroll
    for (int e = 0; e < kCK; ++e)
        if (e < z.cnt) {
            const int jj = z.j0 + e - js;
            if (z.st[e]) {
                ++idx;
                if (z.c[e] != kClsSerial) {
                    c0 = W.ev_c0[idx];
                    Ra = W.ev_r0[idx];
                }
            }
            if (z.c[e] == kClsSerial) {
                if (jj < lim) pre[jj] = (T)W.spre[sidx];
                ++sidx;
            } else {
                R += z.r[e];
                // c0 < 0: the walk added this run itself
                if (c0 >= 0.0 && jj < lim)
                    pre[jj] = with_significand<T>(z.c[e], significand_in<T>((T)c0, z.c[e]) + (R - Ra));
            }
        }
}

// every entry's sum
static __global__ void __launch_bounds__(kCThreads) k_chain_fin(ChainSet S, const SampleState *ss, int by_temperature,
                                                                int mode, const StepState *st) {
    __shared__ WgLds L;
    if (st && st->err) return;
    const int q = chain_block_sum(S, mode, L);
    if (q < 0) return;
    const int j0 = cs_j0(S, q);
    if (chain_f64(ss, by_temperature)) chain_fin_tile<double>(S, q, S.pre64 + j0, L);
    else chain_fin_tile<float>(S, q, S.pre32 + j0, L);
}

// check mode: every sum again one add after another, differences counted
template <typename T>
__device__ void chain_check_sum(const ChainSet &S, int q, const T *pre, float (*in)[kChainChunk],
                                T (*out)[kChainChunk]) {
    __shared__ double tchk;
    const int m = cs_jm(S, q), pre_lim = cs_prelim(S, q);
    ChainWork W = chain_work(S.ev + (size_t)q * S.ev_stride, m);
    T *chk = reinterpret_cast<T *>(W.chk);
    chain_serial<T>(S.w + cs_j0(S, q), m, chk, m, &tchk, in, out);
    int diff = 0;
    for (int j = threadIdx.x; j < pre_lim; j += kCThreads) diff += !same_bits(pre[j], chk[j]);
    if (threadIdx.x == 0) diff += !same_bits(S.totals[q], tchk);
    if (diff) atomicAdd(S.check + q, diff);
}

static __global__ void __launch_bounds__(kCThreads) k_chain_check(ChainSet S, const SampleState *ss, int by_temperature,
                                                               const StepState *st) {
    __shared__ __align__(16) float in[2][kChainChunk];
    __shared__ __align__(16) double out[2][kChainChunk];
    if (st && st->err) return;
    const int q = blockIdx.x, j0 = cs_j0(S, q);
    if (chain_f64(ss, by_temperature))
        chain_check_sum<double>(S, q, S.pre64 + j0, in, out);
    else
        chain_check_sum<float>(S, q, S.pre32 + j0, in, reinterpret_cast<float(*)[kChainChunk]>(out));
}

// ---------------------------------------------------------------------------
// draws
// ---------------------------------------------------------------------------

__device__ __forceinline__ void write_draw(SampleState *ss, StepState *st, unsigned long long rng, int tok) {
    ss->rng = rng;
    ss->token = tok;
    if (st) st->argmax_slot[0] = (1ull << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)tok);
}

// sampleTwoLogits (model.go:2309-2324)
__device__ int sample_two_dev(float s0, float s1, float inv, unsigned long long &rng) {
#pragma clang fp contract(off)
    if (s0 >= s1) {
        const double w1 = (double)fast_exp_wrap((s1 - s0) * inv);
        return rng_float64(rng) * (1 + w1) <= 1 ? 0 : 1;
    }
    const double w0 = (double)fast_exp_wrap((s0 - s1) * inv);
    return rng_float64(rng) * (w0 + 1) <= w0 ? 0 : 1;
}

// pick over CumulativeSum(w), one wave.  The binary search probes exactly
// the reference's midpoints; six levels at a time, every lane loads the
// cumulative entry at one node of the next six levels' probe tree, then the
// levels are walked with those values.
static __global__ void __launch_bounds__(64) k_full_pick(const float *x, int n, const float *pre,
                                                         const double *totals, SampleState *ss, StepState *st) {
#pragma clang fp contract(off)
    if (st && st->err) return;
    const int lane = threadIdx.x;
    unsigned long long rng = ss->rng;
    int idx;
    if (n == 2) {
        idx = sample_two_dev(x[0], x[1], 1.0f / (float)ss->temperature, rng);
    } else {
        const float sum = (float)totals[0];
        const int bs = (n + 3) / 4;
        const bool blocks = n >= 4096;
        float off1 = 0.0f, off2 = 0.0f, off3 = 0.0f;
        if (blocks) {
            off1 = pre[bs - 1];
            off2 = off1 + (float)totals[1];
            off3 = off2 + (float)totals[2];
        }
        const float pick = (float)rng_float64(rng) * sum;
        int lo = 0, hi = n;
        while (lo < hi) {
            // this lane's node of the next six levels (heap order 1..63: the
            // bits of the node below its leading one are the left/right turns)
            float v = 0.0f;
            if (lane >= 1) {
                int a = lo, b = hi;
                const int lvl = 31 - __clz(lane);
                for (int k = lvl - 1; k >= 0 && a < b; --k) {
                    const int mid = (int)((unsigned)(a + b) >> 1);
                    if ((lane >> k) & 1) a = mid + 1;
                    else b = mid;
                }
                if (a < b) {
                    const int mid = (int)((unsigned)(a + b) >> 1);
                    v = pre[mid];
                    if (blocks && mid >= bs) v = v + (mid >= 3 * bs ? off3 : mid >= 2 * bs ? off2 : off1);
                }
            }
            int node = 1;
            for (int k = 0; k < 6 && lo < hi; ++k) {
                const int mid = (int)((unsigned)(lo + hi) >> 1);
                const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), node));
                if (pick <= c) {
                    hi = mid;
                    node = 2 * node;
                } else {
                    lo = mid + 1;
                    node = 2 * node + 1;
                }
            }
        }
        idx = lo < n ? lo : n - 1;
    }
    if (lane == 0) write_draw(ss, st, rng, idx);
}

// the first candidate whose running sum reaches the pick (k - 1 if none)
static __global__ void __launch_bounds__(kWideThreads) k_cand_pick(const unsigned long long *keys, int k,
                                                                   const float *pre32, const double *pre64,
                                                                   const double *totals, SampleState *ss,
                                                                   StepState *st) {
#pragma clang fp contract(off)
    __shared__ int red[kWideThreads / 64];
    if (st && st->err) return;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    unsigned long long rng = ss->rng;
    const double u = rng_float64(rng);
    const bool f32 = ss->temperature == 1.0;
    const float pick32 = (float)u * (float)totals[0];
    const double pick64 = u * totals[0];
    int first = k;
    for (int i = tid; i < k; i += kWideThreads)
        if (f32 ? pick32 <= pre32[i] : pick64 <= pre64[i]) {
            first = i;
            break;
        }
    for (int off = 32; off > 0; off >>= 1) {
        const int o = __shfl_xor(first, off, 64);
        first = o < first ? o : first;
    }
    if (lane == 0) red[wid] = first;
    __syncthreads();
    if (tid == 0) {
        int f = red[0];
        for (int i = 1; i < kWideThreads / 64; ++i) f = red[i] < f ? red[i] : f;
        const int idx = f < k ? f : k - 1;
        write_draw(ss, st, rng, key_row(keys[idx]));
    }
}

}  // namespace pocr
