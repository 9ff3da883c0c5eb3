// Sampling LM head on the device: the top-k candidates of the LM-head scores
// (MatVecTopKQ*WithWork + topKSelectWithWork, internal/tensor/topk.go:200-345;
// VulkanMatVecTopKQ*, internal/backend/vulkan_exec_stub.go:194-328) and the
// draw among them (sampleCandidateScoresScratch, internal/model/model.go:
// 1950-1990, with fastRNG 1829-1840).
//
// A candidate is the 64-bit key (order-preserving score bits << 32 | ~row):
// keys are unique, a larger key is a higher score or, for equal scores, the
// lower row — the reference's order.  Selection is two launches:
//   k_topk_partial   one workgroup per 2,048-row slice: the slice's k largest
//                    keys by an LDS radix select (8-bit digits from the top,
//                    stopping as soon as a digit's bin holds exactly the keys
//                    still needed), written unordered;
//   k_topk_final     one workgroup: the k largest of the partials the same
//                    way, sorted in one wave (bitonic, one key per lane),
//                    written as (id, score) and, when sampling, drawn from by
//                    lane 0 with the reference's arithmetic (f32 or f64 sums
//                    in candidate order, FastExp with its exponent wrap).
// The drawn token goes to argmax slot 0 of the step state, where the next
// step's prologue takes it like a greedy argmax.
#pragma once

#include "kernels.hpp"

namespace pocr {

constexpr int kTopKMax = 64;       // candidates: one per lane of the final sort
constexpr int kTopKThreads = 256;
constexpr int kTopKPer = 8;        // keys per thread of a partial
constexpr int kTopKSlice = kTopKThreads * kTopKPer;
constexpr int kTopKMaxParts = 64;  // rows ≤ 131,072
constexpr int kTopKFinalPer = kTopKMaxParts * kTopKMax / kTopKThreads;

// per sequence (and per context for the op-level calls), in device memory
struct SampleState {
    unsigned long long rng;  // fastRNG state
    double temperature;
    int32_t top_k;
    int32_t n;      // candidates written by the last selection
    int32_t token;  // the last draw
    int32_t pad;
    int32_t ids[kTopKMax];  // score descending, equal scores by lower id
    float scores[kTopKMax];
};

// order-preserving bits of a score; −0 is taken as +0 (the reference compares
// floats, for which they are equal)
__device__ __forceinline__ uint32_t score_order(float s) {
    uint32_t b = __float_as_uint(s);
    b = b == 0x80000000u ? 0u : b;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float score_of(uint32_t o) {
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}
__device__ __forceinline__ unsigned long long cand_key(float s, int row) {
    return ((unsigned long long)score_order(s) << 32) | (0xFFFFFFFFu - (uint32_t)row);
}

// The threshold T such that this workgroup's nonzero keys ≥ T are its `want`
// largest (all of them when fewer: T = 1; 0 is "no key").  hist: 256 LDS
// counters, pick: 3 LDS ints.
template <int E>
__device__ unsigned long long radix_select(const unsigned long long (&key)[E], int want, unsigned *hist, int *pick) {
    const int tid = threadIdx.x, lane = tid & 63;
    // nonzero keys in the workgroup
    int mine = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) mine += key[e] != 0ull;
    for (int off = 32; off > 0; off >>= 1) mine += __shfl_xor(mine, off, 64);
    if (tid == 0) pick[0] = 0;
    __syncthreads();
    if (lane == 0) atomicAdd(&pick[0], mine);
    __syncthreads();
    const int valid = pick[0];
    __syncthreads();
    if (valid <= want) return 1ull;
    unsigned long long prefix = 0ull, pmask = 0ull;
    int need = want;
    for (int shift = 56; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += kTopKThreads) hist[i] = 0u;
        __syncthreads();
#pragma unroll
        for (int e = 0; e < E; ++e)
            if (key[e] != 0ull && (key[e] & pmask) == prefix) atomicAdd(&hist[(uint32_t)(key[e] >> shift) & 255u], 1u);
        __syncthreads();
        if (tid < 64) {
            // lane l holds digits 4l..4l+3; the digit whose bin contains the
            // need-th largest remaining key is unique
            const unsigned h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2],
                           h3 = hist[4 * lane + 3];
            const unsigned tot = h0 + h1 + h2 + h3;
            unsigned suf = tot;  // this lane and the lanes above it
            for (int off = 1; off < 64; off <<= 1) {
                const unsigned o = __shfl_down(suf, off, 64);
                suf += lane + off < 64 ? o : 0u;
            }
            const unsigned a3 = suf - tot, a2 = a3 + h3, a1 = a2 + h2, a0 = a1 + h1;
            const unsigned n = (unsigned)need;
            int d = -1;
            unsigned ab = 0u, hc = 0u;
            if (a3 < n && n <= a3 + h3) d = 4 * lane + 3, ab = a3, hc = h3;
            else if (a2 < n && n <= a2 + h2) d = 4 * lane + 2, ab = a2, hc = h2;
            else if (a1 < n && n <= a1 + h1) d = 4 * lane + 1, ab = a1, hc = h1;
            else if (a0 < n && n <= a0 + h0) d = 4 * lane, ab = a0, hc = h0;
            if (d >= 0) {
                pick[0] = d;
                pick[1] = (int)ab;
                pick[2] = (int)hc;
            }
        }
        __syncthreads();
        const int d = pick[0], above = pick[1], in_bin = pick[2];
        __syncthreads();  // hist and pick are rewritten by the next digit
        prefix |= (unsigned long long)d << shift;
        pmask |= 0xFFull << shift;
        need -= above;
        if (in_bin == need) break;  // every key of this bin is taken
    }
    return prefix;
}

static __global__ void __launch_bounds__(kTopKThreads) k_topk_partial(const float *scores, int rows, int k,
                                                              unsigned long long *part) {
    __shared__ unsigned hist[256];
    __shared__ int pick[3];
    __shared__ int count;
    const int tid = threadIdx.x;
    const int lo = blockIdx.x * kTopKSlice;
    unsigned long long key[kTopKPer];
#pragma unroll
    for (int e = 0; e < kTopKPer; ++e) {
        const int r = lo + e * kTopKThreads + tid;
        key[e] = r < rows ? cand_key(scores[r], r) : 0ull;
    }
    if (tid == 0) count = 0;
    const unsigned long long T = radix_select<kTopKPer>(key, k, hist, pick);
    unsigned long long *out = part + (size_t)blockIdx.x * k;
#pragma unroll
    for (int e = 0; e < kTopKPer; ++e)
        if (key[e] != 0ull && key[e] >= T) out[atomicAdd(&count, 1)] = key[e];
    __syncthreads();
    for (int j = count + tid; j < k; j += kTopKThreads) out[j] = 0ull;
}

// FastExpF32 with its wrap (fast_exp_wrap, kernels.hpp): low-temperature
// draws reach the wrap, and the reference's picks depend on it

// fastRNG.Float64 (model.go:1833-1840)
__device__ __forceinline__ double rng_float64(unsigned long long &s) {
    s += 0x9e3779b97f4a7c15ull;
    unsigned long long z = s;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

// sampleCandidateScoresScratch (model.go:1950-1990) over n ≥ 2 candidates
// sorted as above; returns the candidate index.  One thread; for n > 4, w
// holds the weights FastExp(s − max) (temperature 1) or FastExp(s·(1/T) −
// max·(1/T)) (otherwise), computed lane-parallel by the caller.
static __device__ int draw_candidate(const float *sc, const float *w, int n, double temp, unsigned long long &rng) {
#pragma clang fp contract(off)
    if (temp == 1.0) {
        float mx = sc[0];
        for (int i = 1; i < n; ++i) mx = sc[i] > mx ? sc[i] : mx;
        if (n == 2) {  // sampleCandidateScoresTemp1Small, model.go:2145-2158
            const float s0 = sc[0], s1 = sc[1];
            if (s0 >= s1) {
                const double w1 = (double)fast_exp_wrap(s1 - s0);
                return rng_float64(rng) * (1 + w1) <= 1 ? 0 : 1;
            }
            const double w0 = (double)fast_exp_wrap(s0 - s1);
            return rng_float64(rng) * (w0 + 1) <= w0 ? 0 : 1;
        }
        if (n <= 4) {  // model.go:2159-2199
            const float w0 = fast_exp_wrap(sc[0] - mx), w1 = fast_exp_wrap(sc[1] - mx), w2 = fast_exp_wrap(sc[2] - mx);
            if (n == 3) {
                const float pick = (float)rng_float64(rng) * ((w0 + w1) + w2);
                if (pick <= w0) return 0;
                if (pick <= w0 + w1) return 1;
                return 2;
            }
            const float w3 = fast_exp_wrap(sc[3] - mx);
            const float pick = (float)rng_float64(rng) * ((w0 + w1) + (w2 + w3));
            float acc = w0;
            if (pick <= acc) return 0;
            acc += w1;
            if (pick <= acc) return 1;
            acc += w2;
            if (pick <= acc) return 2;
            return 3;
        }
        // sampleCandidateScoresTemp1Scratch (model.go:2040-2063): f32 weights
        // and sum, pickWeightedRawFloat32 (2418-2456)
        float sum = 0.0f;
        for (int i = 0; i < n; ++i) sum += w[i];
        const float pick = (float)rng_float64(rng) * sum;
        float acc = 0.0f;
        for (int i = 0; i < n; ++i) {
            acc += w[i];
            if (pick <= acc) return i;
        }
        return n - 1;
    }
    const float inv = (float)(1.0 / temp);
    float mxr = sc[0];
    for (int i = 1; i < n; ++i) mxr = sc[i] > mxr ? sc[i] : mxr;
    const float mx = mxr * inv;
    if (n == 2) {  // sampleCandidateScoresSmall, model.go:1997-2011
        const float s0 = sc[0] * inv, s1 = sc[1] * inv;
        if (s0 >= s1) {
            const double w1 = (double)fast_exp_wrap(s1 - s0);
            return rng_float64(rng) * (1 + w1) <= 1 ? 0 : 1;
        }
        const double w0 = (double)fast_exp_wrap(s0 - s1);
        return rng_float64(rng) * (w0 + 1) <= w0 ? 0 : 1;
    }
    if (n <= 4) {  // model.go:2012-2037
        const double w0 = (double)fast_exp_wrap(sc[0] * inv - mx), w1 = (double)fast_exp_wrap(sc[1] * inv - mx),
                     w2 = (double)fast_exp_wrap(sc[2] * inv - mx);
        if (n == 3) {
            const double pick = rng_float64(rng) * ((w0 + w1) + w2);
            double acc = w0;
            if (pick <= acc) return 0;
            acc += w1;
            if (pick <= acc) return 1;
            return 2;
        }
        const double w3 = (double)fast_exp_wrap(sc[3] * inv - mx);
        const double pick = rng_float64(rng) * ((w0 + w1) + (w2 + w3));
        double acc = w0;
        if (pick <= acc) return 0;
        acc += w1;
        if (pick <= acc) return 1;
        acc += w2;
        if (pick <= acc) return 2;
        return 3;
    }
    // model.go:1971-1989: f64 sum of the weights, the f32-stored weights
    // summed again in f64 by pickWeightedFloat32 (2342-2416)
    double sum = 0.0;
    for (int i = 0; i < n; ++i) sum += (double)w[i];
    const double pick = rng_float64(rng) * sum;
    double acc = 0.0;
    for (int i = 0; i < n; ++i) {
        acc += (double)w[i];
        if (pick <= acc) return i;
    }
    return n - 1;
}

// The k best of the partials → ss->ids/scores (sorted); with `sample`, one
// draw (k ≥ 2) into ss->token, ss->rng and argmax slot 0 of st (if any).
static __global__ void __launch_bounds__(kTopKThreads) k_topk_final(const unsigned long long *part, int nparts, int k,
                                                            SampleState *ss, StepState *st, int sample) {
    __shared__ unsigned hist[256];
    __shared__ int pick[3];
    __shared__ int count;
    __shared__ unsigned long long sel[kTopKMax];
    __shared__ float csc[kTopKMax];
    __shared__ float cw[kTopKMax];
    __shared__ int cid[kTopKMax];
    const int tid = threadIdx.x, lane = tid & 63;
    if (st && st->err) return;  // a failed step draws nothing (uniform)
    const int N = nparts * k;
    unsigned long long key[kTopKFinalPer];
#pragma unroll
    for (int e = 0; e < kTopKFinalPer; ++e) {
        const int i = e * kTopKThreads + tid;
        key[e] = i < N ? part[i] : 0ull;
    }
    if (tid == 0) count = 0;
    const unsigned long long T = radix_select<kTopKFinalPer>(key, k, hist, pick);
#pragma unroll
    for (int e = 0; e < kTopKFinalPer; ++e)
        if (key[e] != 0ull && key[e] >= T) sel[atomicAdd(&count, 1)] = key[e];
    __syncthreads();
    if (tid >= 64) return;
    const int n = count;
    unsigned long long v = lane < n ? sel[lane] : 0ull;
    // bitonic sort, descending across the 64 lanes
    for (int size = 2; size <= 64; size <<= 1)
        for (int j = size >> 1; j > 0; j >>= 1) {
            const unsigned long long o = shfl_xor_u64(v, j);
            const unsigned long long hi = v > o ? v : o, lo = v > o ? o : v;
            v = (((lane & j) == 0) == ((lane & size) == 0)) ? hi : lo;
        }
    const float score = score_of((uint32_t)(v >> 32));
    const int id = (int)(0xFFFFFFFFu - (uint32_t)v);
    if (lane < n) {
        ss->ids[lane] = id;
        ss->scores[lane] = score;
        csc[lane] = score;
        cid[lane] = id;
    }
    if (lane == 0) ss->n = n;
    if (!sample) return;
    {
        // the draw's weights, one per lane (the maximum is lane 0's score)
#pragma clang fp contract(off)
        const double temp = ss->temperature;
        const float mx0 = __shfl(score, 0, 64);
        float wgt;
        if (temp == 1.0) {
            wgt = fast_exp_wrap(score - mx0);
        } else {
            const float inv = (float)(1.0 / temp);
            wgt = fast_exp_wrap(score * inv - mx0 * inv);
        }
        if (lane < n) cw[lane] = wgt;
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // csc, cw, cid written by the wave's lanes
    if (lane == 0) {
        unsigned long long rng = ss->rng;
        const int c = n >= 2 ? draw_candidate(csc, cw, n, ss->temperature, rng) : 0;
        const int tok = cid[c];
        ss->rng = rng;
        ss->token = tok;
        if (st) st->argmax_slot[0] = (1ull << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)tok);
    }
}

}  // namespace pocr
