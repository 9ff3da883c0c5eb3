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
constexpr int kChainJobs = 4;

// one running sum c_0 = 0, c_{j+1} = c_j + w_j (f32 or f64 adds): pre[j] =
// c_{j+1} for j < pre_lim, *total = c_m
struct ChainJob {
    const float *w;
    int m;
    int pre_lim;
    float *pre32;   // f32 sums
    double *pre64;  // f64 sums
    double *total;
};
struct ChainJobs {
    ChainJob j[kChainJobs];
};

// device buffers of the wide sampler (one allocation)
struct WideBufs {
    unsigned long long *keys;  // [N] sorted candidate keys (N = next power of two ≥ n)
    float *w;                  // [n] weights
    float *pre32;              // [n] f32 running sums
    double *pre64;             // [n] f64 running sums
    double *totals;            // [kChainJobs]
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
// workgroup reductions
// ---------------------------------------------------------------------------

// the reference's maximum (x[0], then v > m): NaN entries are skipped unless
// x[0] is NaN, which the maximum then stays
__device__ __forceinline__ float wg_max(float m, float first, float *red) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    if (lane == 0) red[wid] = m;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < kWideThreads / 64; ++i) r = red[i] > r ? red[i] : r;
    __syncthreads();
    return first != first ? first : (first > r ? first : r);
}

// ---------------------------------------------------------------------------
// weights
// ---------------------------------------------------------------------------

// sampleFullLogitsScratch's weights: T = float32(temperature); T == 1:
// v = x·1 + (−m); otherwise v = x·(1/T) + (−(m·(1/T))); w = FastExpF32(v)
static __global__ void __launch_bounds__(kWideThreads) k_full_weights(const float *x, int n, const SampleState *ss,
                                                                      float *w, const StepState *st) {
#pragma clang fp contract(off)
    __shared__ float red[kWideThreads / 64];
    if (st && st->err) return;
    const int tid = threadIdx.x;
    float m = -__builtin_inff();
    for (int i = tid + 1; i < n; i += kWideThreads) {
        const float v = x[i];
        m = v > m ? v : m;
    }
    m = wg_max(m, x[0], red);  // x[0] enters first
    const float T = (float)ss->temperature;
    float scale = 1.0f, bias = -m;
    if (T != 1.0f) {
        scale = 1.0f / T;
        bias = -(m * scale);
    }
    for (int i = tid; i < n; i += kWideThreads) w[i] = fast_exp_wrap(x[i] * scale + bias);
}

__device__ __forceinline__ float key_score(unsigned long long k) { return score_of((uint32_t)(k >> 32)); }
__device__ __forceinline__ int key_row(unsigned long long k) { return (int)(0xFFFFFFFFu - (uint32_t)k); }

// sampleCandidateScoresScratch's weights over the k best keys (k > 4)
static __global__ void __launch_bounds__(kWideThreads) k_cand_weights(const unsigned long long *keys, int k,
                                                                      const SampleState *ss, float *w,
                                                                      const StepState *st) {
#pragma clang fp contract(off)
    __shared__ float red[kWideThreads / 64];
    if (st && st->err) return;
    const int tid = threadIdx.x;
    float m = -__builtin_inff();
    for (int i = tid + 1; i < k; i += kWideThreads) {
        const float v = key_score(keys[i]);
        m = v > m ? v : m;
    }
    m = wg_max(m, key_score(keys[0]), red);
    const double temp = ss->temperature;
    if (temp == 1.0) {
        for (int i = tid; i < k; i += kWideThreads) w[i] = fast_exp_wrap(key_score(keys[i]) - m);
    } else {
        const float inv = (float)(1.0 / temp);
        const float mx = m * inv;
        for (int i = tid; i < k; i += kWideThreads) w[i] = fast_exp_wrap(key_score(keys[i]) * inv - mx);
    }
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
// waves 1.. stage the next chunk in and the previous chunk's sums out
template <typename T>
__device__ void chain_serial(const ChainJob &J, float (*in)[kChainChunk], T (*out)[kChainChunk], T *pre) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x;
    const int m = J.m;
    const int nch = (m + kChainChunk - 1) / kChainChunk;
    T c = 0;
    if (nch > 0) chain_stage(J.w, 0, m < kChainChunk ? m : kChainChunk, in[0], tid, kWideThreads);
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
                chain_stage(J.w, nb, m - nb < kChainChunk ? m - nb : kChainChunk, in[cur ^ 1], tid - 64,
                            kWideThreads - 64);
            }
            if (k > 0) chain_flush<T>(out[cur ^ 1], base - kChainChunk, kChainChunk, J.pre_lim, pre, tid - 64,
                                      kWideThreads - 64);
        }
        __syncthreads();
    }
    if (nch > 0) {
        const int base = (nch - 1) * kChainChunk;
        chain_flush<T>(out[(nch - 1) & 1], base, m - base, J.pre_lim, pre, tid, kWideThreads);
    }
    if (tid == 0) *J.total = (double)c;
}

// one workgroup per job; f64 sums when `by_temperature` and the sampler's
// temperature is not 1, f32 sums otherwise
static __global__ void __launch_bounds__(kWideThreads) k_chain(ChainJobs jobs, const SampleState *ss,
                                                               int by_temperature, const StepState *st) {
    __shared__ __align__(16) float in[2][kChainChunk];
    __shared__ __align__(16) double out[2][kChainChunk];
    if (st && st->err) return;
    ChainJob J = jobs.j[0];
#pragma unroll
    for (int q = 1; q < kChainJobs; ++q)
        if ((int)blockIdx.x == q) J = jobs.j[q];
    if (by_temperature && ss->temperature != 1.0)
        chain_serial<double>(J, in, out, J.pre64);
    else
        chain_serial<float>(J, in, reinterpret_cast<float(*)[kChainChunk]>(out), J.pre32);
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

// pick over CumulativeSum(w): one thread (launch one wave)
static __global__ void __launch_bounds__(64) k_full_pick(const float *x, int n, const float *pre,
                                                         const double *totals, SampleState *ss, StepState *st) {
#pragma clang fp contract(off)
    if (threadIdx.x != 0 || (st && st->err)) return;
    unsigned long long rng = ss->rng;
    int idx;
    if (n == 2) {
        idx = sample_two_dev(x[0], x[1], 1.0f / (float)ss->temperature, rng);
    } else {
        const float sum = (float)totals[0];
        const int bs = (n + 3) / 4;
        float off[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const bool blocks = n >= 4096;
        if (blocks) {
            off[1] = pre[bs - 1];
            off[2] = off[1] + (float)totals[1];
            off[3] = off[2] + (float)totals[2];
        }
        const float pick = (float)rng_float64(rng) * sum;
        int lo = 0, hi = n;
        while (lo < hi) {
            const int mid = (int)((unsigned)(lo + hi) >> 1);
            float c = pre[mid];
            if (blocks && mid >= bs) c = c + off[mid / bs];
            if (pick <= c) hi = mid;
            else lo = mid + 1;
        }
        idx = lo < n ? lo : n - 1;
    }
    write_draw(ss, st, rng, idx);
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
