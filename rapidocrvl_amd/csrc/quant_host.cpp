// quant_host.cpp — host-side Q8/Q4/Q6 row encoders, unpackers and multimodal
// positions of the C ABI (product code; the converter/loader side of the path).
//
// Encoders follow internal/tensor/quant.go: QuantizeQ8RowBytesInto (96-137),
// QuantizeQ4RowInto (291-354), QuantizeQ6RowInto (201-270) with quantInt8 /
// q4Nib / quantByte6 (139-147, 357-365, 272-280) and roundToInt (436-441).
// scale = maxAbs/{127,7,31} in f32; inv = 1/scale; code = clamp(round(w·inv)).
// An all-zero row encodes as zero bytes with scale 1 (so Q4 decodes to -8 and
// Q6 to -32, the reference's behaviour).
#include <cmath>
#include <cstdint>
#include <cstring>

#include "../../include/pocr_hip.h"

#ifdef __clang__
#pragma clang fp contract(off)
#endif

namespace {

int round_half_away(float x) { return x >= 0.0f ? (int)(x + 0.5f) : (int)(x - 0.5f); }
int round_even(float x) { return (int)std::nearbyint(x); }
int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

float max_abs(const float *x, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float a = std::fabs(x[i]);
        if (a > m) m = a;
    }
    return m;
}

// putQ6 (quant.go:2886-2895)
void put_q6(uint8_t *row, size_t row_len, int col, uint8_t v) {
    const int bit = col * 6, idx = bit / 8, shift = bit % 8;
    const uint16_t x = (uint16_t)((v & 0x3F) << shift);
    row[idx] |= (uint8_t)x;
    if ((size_t)idx + 1 < row_len) row[idx + 1] |= (uint8_t)(x >> 8);
}

float quantize_row(int qtype, int tie, const float *w, int cols, uint8_t *out) {
    const size_t nb = pocr_row_bytes(qtype, cols);
    const float m = max_abs(w, cols);
    if (m == 0.0f) {
        std::memset(out, 0, nb);
        return 1.0f;
    }
    const float qmax = qtype == POCR_Q8 ? 127.0f : (qtype == POCR_Q4 ? 7.0f : 31.0f);
    const int lim = (int)qmax;
    const float scale = m / qmax;
    const float inv = 1.0f / scale;
    if (qtype == POCR_Q8) {
        // the converter's byte encoder has no AVX2 branch: half-away always
        for (int i = 0; i < cols; ++i) out[i] = (uint8_t)(int8_t)clampi(round_half_away(w[i] * inv), -127, 127);
        return scale;
    }
    std::memset(out, 0, nb);
    if (qtype == POCR_Q4) {
        const bool rne = tie == POCR_TIE_AMD64 && cols >= 8;
        for (int i = 0; i < cols; ++i) {
            const float v = w[i] * inv;
            const uint8_t nib = (uint8_t)(clampi(rne ? round_even(v) : round_half_away(v), -lim, lim) + 8);
            out[i / 2] |= (i & 1) ? (uint8_t)(nib << 4) : nib;
        }
        return scale;
    }
    // Q6: the amd64 converter rounds the floor(cols/8)*8 prefix with AVX2 (RNE)
    // and the tail with quantByte6 (half away), quant.go:208-232
    const int prefix = (tie == POCR_TIE_AMD64 && cols >= 8) ? (cols / 8) * 8 : 0;
    for (int i = 0; i < cols; ++i) {
        const float v = w[i] * inv;
        const int r = i < prefix ? round_even(v) : round_half_away(v);
        put_q6(out, nb, i, (uint8_t)(clampi(r, -lim, lim) + 32));
    }
    return scale;
}

}  // namespace

extern "C" size_t pocr_row_bytes(int qtype, int cols) {
    if (cols < 0) return 0;
    switch (qtype) {
    case POCR_Q8: return (size_t)cols;
    case POCR_Q4: return ((size_t)cols + 1) / 2;
    case POCR_Q6: return ((size_t)cols * 6 + 7) / 8;
    case POCR_F32: return (size_t)cols * 4;
    }
    return 0;
}

extern "C" int pocr_quantize_rows(int qtype, int tie_mode, const float *w, int rows, int cols, float *scales,
                                  uint8_t *packed) {
    if ((qtype != POCR_Q8 && qtype != POCR_Q4 && qtype != POCR_Q6) || rows < 0 || cols <= 0 || !w || !scales ||
        !packed)
        return POCR_ERR_ARG;
    const size_t rb = pocr_row_bytes(qtype, cols);
    for (int r = 0; r < rows; ++r)
        scales[r] = quantize_row(qtype, tie_mode, w + (size_t)r * cols, cols, packed + (size_t)r * rb);
    return POCR_OK;
}

extern "C" int pocr_unpack_rows(int qtype, const uint8_t *packed, int rows, int cols, int8_t *out) {
    if ((qtype != POCR_Q8 && qtype != POCR_Q4 && qtype != POCR_Q6) || rows < 0 || cols <= 0 || !packed || !out)
        return POCR_ERR_ARG;
    const size_t rb = pocr_row_bytes(qtype, cols);
    for (int r = 0; r < rows; ++r) {
        const uint8_t *row = packed + (size_t)r * rb;
        int8_t *dst = out + (size_t)r * cols;
        for (int c = 0; c < cols; ++c) {
            if (qtype == POCR_Q8) {
                dst[c] = (int8_t)row[c];
            } else if (qtype == POCR_Q4) {
                const uint8_t b = row[c / 2];
                dst[c] = (int8_t)(((c & 1) ? (b >> 4) : (b & 0x0F)) - 8);  // q4Int8Table
            } else {
                // getQ6 (quant.go:2897-2906) then q6Int8Table (code − 32)
                const int bit = c * 6, idx = bit / 8, shift = bit % 8;
                uint16_t x = row[idx];
                if ((size_t)idx + 1 < rb) x |= (uint16_t)row[idx + 1] << 8;
                dst[c] = (int8_t)(((x >> shift) & 0x3F) - 32);
            }
        }
    }
    return POCR_OK;
}

// multimodalPositionsInto (internal/model/model.go:1717-1783)
extern "C" int pocr_mm_positions(const int32_t *ids, int n, int32_t image_token_id, const int32_t grid[3],
                                 int32_t merge, int32_t *pos3, int32_t *rope_delta) {
    if (!ids || n < 0 || !pos3 || !rope_delta || merge <= 0 || !grid) return POCR_ERR_ARG;
    int pi = 0, st = 0, next_pos = 0;
    for (;;) {
        int ed = -1;
        for (int i = st; i < n; ++i)
            if (ids[i] == image_token_id) {
                ed = i;
                break;
            }
        if (ed < 0) break;
        const int st_idx = next_pos;
        for (int i = 0; i < ed - st; ++i) {
            const int p = st_idx + i;
            pos3[3 * pi] = pos3[3 * pi + 1] = pos3[3 * pi + 2] = p;
            ++pi;
        }
        const int text_len = ed - st;
        int max_pos = st_idx + text_len - 1;
        const int gt = grid[0], gh = grid[1] / merge, gw = grid[2] / merge;
        if (gt <= 0 || gh <= 0 || gw <= 0) return POCR_ERR_ARG;
        for (int t = 0; t < gt; ++t)
            for (int h = 0; h < gh; ++h)
                for (int w = 0; w < gw; ++w) {
                    if (pi >= n) return POCR_ERR_ARG;  // grid larger than the placeholder run
                    const int pt = text_len + st_idx + t, ph = text_len + st_idx + h, pw = text_len + st_idx + w;
                    pos3[3 * pi] = pt;
                    pos3[3 * pi + 1] = ph;
                    pos3[3 * pi + 2] = pw;
                    ++pi;
                    if (pt > max_pos) max_pos = pt;
                    if (ph > max_pos) max_pos = ph;
                    if (pw > max_pos) max_pos = pw;
                }
        next_pos = max_pos + 1;
        st = ed + gt * gh * gw;
    }
    if (st < n) {
        const int st_idx = next_pos;
        for (int i = 0; i < n - st; ++i) {
            const int p = st_idx + i;
            pos3[3 * pi] = pos3[3 * pi + 1] = pos3[3 * pi + 2] = p;
            ++pi;
        }
        next_pos = st_idx + n - st;
    }
    *rope_delta = pi == 0 ? 0 : next_pos - n;
    return pi;
}
