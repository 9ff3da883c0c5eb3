// prefill.hip — prompt prefill and batched (M>1) GEMV.
#include "internal.hpp"

void prefill_free(PrefillBufs &b) {
    for (void *p : {(void *)b.x, (void *)b.y, (void *)b.h, (void *)b.v, (void *)b.pos, (void *)b.tabs})
        if (p) (void)hipFree(p);
    b = PrefillBufs{};
}

namespace pocr {

// M rows of activations against one weight stream
int batched_gemv(hipStream_t s, const DevMat &w, const float *x, int m, float *out) {
    for (int i = 0; i < m; ++i) {
        GemvParams p{};
        p.m[0] = p.m[1] = p.m[2] = w;
        p.seg_end[0] = p.seg_end[1] = p.seg_end[2] = w.rows;
        p.rows = w.rows;
        p.cols = w.cols;
        p.x = x + (size_t)i * w.cols;
        p.out = out + (size_t)i * w.rows;
        RC(gemv_launch(s, p, 1, PRO_COPY, EPI_PLAIN, kBigGrid));
    }
    return POCR_OK;
}

// token-by-token prefill (model.go:1514-1536): same semantics as n steps
int prefill_locked(pocr_seq *s, int n, const float *emb, const int32_t *pos3, float *logits, int32_t *token) {
    const int H = s->m->cfg.hidden;
    for (int i = 0; i < n; ++i) {
        const bool last = i == n - 1;
        RC(step_locked(s, emb + (size_t)i * H, pos3 + 3 * i, last ? 1 : 0, last ? logits : nullptr,
                       last ? token : nullptr));
    }
    return POCR_OK;
}

}  // namespace pocr
