// prefill.hip — prompt prefill and batched (M>1) GEMV on the matrix cores.
#include "gemm.hpp"
#include "internal.hpp"

using namespace pocr;

void prefill_free(PrefillBufs &b) {
    for (void *p : {(void *)b.h, (void *)b.v, (void *)b.qkv, (void *)b.ho, (void *)b.g, (void *)b.xd, (void *)b.xs,
                    (void *)b.xb, (void *)b.pos, (void *)b.kvimg})
        if (p) (void)hipFree(p);
    b = PrefillBufs{};
}

namespace {

int round_up(int x, int m) { return (x + m - 1) / m * m; }

// the MFMA GEMM takes rows in whole 64-row wave tiles and K in 64-column steps
bool gemm_shape_ok(int rows, int K) { return rows % kGemmWaveRows == 0 && K % kGemmK == 0 && K <= kMaxCols; }

template <int G>
int launch_digitize_g(hipStream_t s, int qtype, const DigitizeParams &p, int n) {
    switch (qtype) {
    case QT_Q8: hipLaunchKernelGGL((k_digitize<QT_Q8, G>), dim3(n), dim3(kThreads), 0, s, p); break;
    case QT_Q4: hipLaunchKernelGGL((k_digitize<QT_Q4, G>), dim3(n), dim3(kThreads), 0, s, p); break;
    case QT_Q6: hipLaunchKernelGGL((k_digitize<QT_Q6, G>), dim3(n), dim3(kThreads), 0, s, p); break;
    default: return fail(POCR_ERR_UNSUPPORTED, "digitize: qtype %d", qtype);
    }
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

template <int J>
int launch_digitize_w(hipStream_t s, int qtype, const DigitizeParams &p, int n) {
    const dim3 grid((n + kWaves - 1) / kWaves);
    switch (qtype) {
    case QT_Q8: hipLaunchKernelGGL((k_digitize_w<QT_Q8, J>), grid, dim3(kThreads), 0, s, p, n); break;
    case QT_Q4: hipLaunchKernelGGL((k_digitize_w<QT_Q4, J>), grid, dim3(kThreads), 0, s, p, n); break;
    case QT_Q6: hipLaunchKernelGGL((k_digitize_w<QT_Q6, J>), grid, dim3(kThreads), 0, s, p, n); break;
    default: return fail(POCR_ERR_UNSUPPORTED, "digitize: qtype %d", qtype);
    }
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

template <int J>
int launch_digitize_vnni_j(hipStream_t s, int qtype, const DigitizeParams &p, int n) {
    const dim3 grid((n + kWaves - 1) / kWaves);
    switch (qtype) {
    case QT_Q4: hipLaunchKernelGGL((k_digitize_vnni<QT_Q4, J>), grid, dim3(kThreads), 0, s, p, n); break;
    case QT_Q6: hipLaunchKernelGGL((k_digitize_vnni<QT_Q6, J>), grid, dim3(kThreads), 0, s, p, n); break;
    default: return fail(POCR_ERR_UNSUPPORTED, "VNNI digitize: qtype %d", qtype);
    }
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

// the VNNI mode's bytes: tile layout only, K a multiple of 128 up to 4096
int launch_digitize_vnni(hipStream_t s, int qtype, const DigitizeParams &p, int n) {
    if (!p.tiled || p.K % kStageCols || p.K > 4096) return fail(POCR_ERR_UNSUPPORTED, "VNNI digitize: K %d", p.K);
    if (p.K <= 1024) return launch_digitize_vnni_j<1>(s, qtype, p, n);
    if (p.K <= 2048) return launch_digitize_vnni_j<2>(s, qtype, p, n);
    if (p.K <= 3072) return launch_digitize_vnni_j<3>(s, qtype, p, n);
    return launch_digitize_vnni_j<4>(s, qtype, p, n);
}

int launch_digitize(hipStream_t s, int qtype, const DigitizeParams &p, int n) {
    if (p.vnni) return launch_digitize_vnni(s, qtype, p, n);
    if (p.K % 16 || p.K > 2 * 16 * kThreads) return fail(POCR_ERR_UNSUPPORTED, "digitize: K %d", p.K);
    if (p.K > 16 * kThreads) return launch_digitize_g<2>(s, qtype, p, n);
    // up to 3072 columns: one wave per token, the same bytes (1345 tokens of
    // 1024 / 2048 / 3072 columns, planes in the tile layout: 6.9 / 7.6 / 10.2
    // µs; a workgroup per token with three barriers took 14 µs at 3072)
    if (p.K <= 1024) return launch_digitize_w<1>(s, qtype, p, n);
    if (p.K <= 2048) return launch_digitize_w<2>(s, qtype, p, n);
    if (p.K <= 3072) return launch_digitize_w<3>(s, qtype, p, n);
    return launch_digitize_g<1>(s, qtype, p, n);
}

template <int NMAT, int TN>
int launch_gemm_t(hipStream_t s, int qtype, const GemmParams &p, int epi, int npad) {
    const dim3 grid((p.rows + kGemmRows - 1) / kGemmRows, npad / (16 * TN));
    switch (qtype) {
    case QT_Q8: hipLaunchKernelGGL((k_gemm<QT_Q8, NMAT, TN>), grid, dim3(kThreads), 0, s, p, epi); break;
    case QT_Q4: hipLaunchKernelGGL((k_gemm<QT_Q4, NMAT, TN>), grid, dim3(kThreads), 0, s, p, epi); break;
    case QT_Q6: hipLaunchKernelGGL((k_gemm<QT_Q6, NMAT, TN>), grid, dim3(kThreads), 0, s, p, epi); break;
    default: return fail(POCR_ERR_UNSUPPORTED, "gemm: qtype %d", qtype);
    }
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

// small M (≤ 16 tokens): 16-row workgroups whose waves split K
template <int NMAT>
int launch_gemm_small_t(hipStream_t s, int qtype, const GemmParams &p, int epi) {
    const dim3 grid(p.rows / 16);
    switch (qtype) {
    case QT_Q8: hipLaunchKernelGGL((k_gemm_small<QT_Q8, NMAT>), grid, dim3(kThreads), 0, s, p, epi); break;
    case QT_Q4: hipLaunchKernelGGL((k_gemm_small<QT_Q4, NMAT>), grid, dim3(kThreads), 0, s, p, epi); break;
    case QT_Q6: hipLaunchKernelGGL((k_gemm_small<QT_Q6, NMAT>), grid, dim3(kThreads), 0, s, p, epi); break;
    default: return fail(POCR_ERR_UNSUPPORTED, "gemm: qtype %d", qtype);
    }
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

bool small_shape_ok(int rows, int K) { return rows % 16 == 0 && K % (kGemmK * kWaves) == 0 && K <= kMaxCols; }

// One, two or four 16-row blocks per wave (64, 128 or 256 rows of each matrix
// per workgroup), two-slot ring.  These kernels are latency-bound: the more
// workgroups share a CU, the better their loads and barriers overlap, so the
// row tile shrinks until the grid holds about three workgroups per CU.
// Measured on the MI355X at 1,345 tokens (Q4, µs; 256 / 128 / 64-row tiles):
// QKV 2560×1024 15.3 / 14.1 / 15.2; o_proj 1024×2048 16.5 / 13.5 / 12.3;
// down 1024×3072 22.0 / 18.5 / 16.4; gate/up 2×3072×1024 – / 28.0 / 23.0.
template <int NMAT, int RB>
int launch_gemm_lds_rb(hipStream_t s, int qtype, const GemmParams &p, int epi, int npad) {
    const dim3 grid((p.rows + 64 * RB - 1) / (64 * RB), npad / 32);
    if (p.vnni) {  // one plane of VNNI bytes (Q4, Q6)
        switch (qtype) {
        case QT_Q4: hipLaunchKernelGGL((k_gemm_lds<QT_Q4, NMAT, 2, RB, 1>), grid, dim3(kThreads), 0, s, p, epi); break;
        case QT_Q6: hipLaunchKernelGGL((k_gemm_lds<QT_Q6, NMAT, 2, RB, 1>), grid, dim3(kThreads), 0, s, p, epi); break;
        default: return fail(POCR_ERR_UNSUPPORTED, "VNNI gemm: qtype %d", qtype);
        }
        HIP_TRY(hipGetLastError());
        return POCR_OK;
    }
    switch (qtype) {
    case QT_Q8: hipLaunchKernelGGL((k_gemm_lds<QT_Q8, NMAT, 2, RB>), grid, dim3(kThreads), 0, s, p, epi); break;
    case QT_Q4: hipLaunchKernelGGL((k_gemm_lds<QT_Q4, NMAT, 2, RB>), grid, dim3(kThreads), 0, s, p, epi); break;
    case QT_Q6: hipLaunchKernelGGL((k_gemm_lds<QT_Q6, NMAT, 2, RB>), grid, dim3(kThreads), 0, s, p, epi); break;
    default: return fail(POCR_ERR_UNSUPPORTED, "gemm: qtype %d", qtype);
    }
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

constexpr int kGemmTargetGroups = 768;  // about three workgroups per CU

template <int NMAT>
int launch_gemm_lds_t(hipStream_t s, int qtype, const GemmParams &p, int epi, int npad) {
    if (NMAT == 1 && p.rows % 128 == 0 && (p.rows / 128) * (npad / 32) >= kGemmTargetGroups)
        return launch_gemm_lds_rb<1, 2>(s, qtype, p, epi, npad);
    return launch_gemm_lds_rb<NMAT, 1>(s, qtype, p, epi, npad);
}

}  // namespace

// the LDS-ring kernel takes K in whole 128-column stages; its digit planes
// are written in the tile layout
bool pocr::gemm_tiled(int K) {
    const char *env = getenv("POCR_PREFILL_GEMM");
    return K % kStageCols == 0 && !(env && env[0] == 'd');
}

bool pocr::weight_tiles_ok(int rows, int cols) { return rows % 16 == 0 && cols % kStageCols == 0; }

int pocr::tile_weight(hipStream_t s, int qtype, const uint8_t *src, int row_bytes, int rows, int cols, uint8_t *dst) {
    const int nst = cols / kStageCols;
    const size_t loads = (size_t)(rows / 16) * nst * 64 * (qtype == QT_Q4 ? 1 : 2);
    const dim3 grid((unsigned)((loads + kThreads - 1) / kThreads));
    switch (qtype) {
    case QT_Q8: hipLaunchKernelGGL(k_tile_weight<QT_Q8>, grid, dim3(kThreads), 0, s, src, row_bytes, rows, nst, dst); break;
    case QT_Q4: hipLaunchKernelGGL(k_tile_weight<QT_Q4>, grid, dim3(kThreads), 0, s, src, row_bytes, rows, nst, dst); break;
    case QT_Q6: hipLaunchKernelGGL(k_tile_weight<QT_Q6>, grid, dim3(kThreads), 0, s, src, row_bytes, rows, nst, dst); break;
    default: return fail(POCR_ERR_UNSUPPORTED, "tile_weight: qtype %d", qtype);
    }
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

int pocr::row_usum(hipStream_t s, int qtype, const uint8_t *src, int row_bytes, int rows, int cols, int *dst) {
    if (cols % 16) return fail(POCR_ERR_UNSUPPORTED, "row_usum: %d columns", cols);
    const dim3 grid((rows + kWaves - 1) / kWaves);
    switch (qtype) {
    case QT_Q4: hipLaunchKernelGGL(k_row_usum<QT_Q4>, grid, dim3(kThreads), 0, s, src, row_bytes, rows, cols, dst); break;
    case QT_Q6: hipLaunchKernelGGL(k_row_usum<QT_Q6>, grid, dim3(kThreads), 0, s, src, row_bytes, rows, cols, dst); break;
    default: return fail(POCR_ERR_UNSUPPORTED, "row_usum: qtype %d", qtype);
    }
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

namespace {

// npad: token rows of the digit planes, a multiple of 32
int launch_gemm(hipStream_t s, int qtype, int nmat, const GemmParams &p, int epi, int npad) {
    if (p.vnni && !gemm_tiled(p.K)) return fail(POCR_ERR_UNSUPPORTED, "VNNI gemm: K %d", p.K);
    if (gemm_tiled(p.K)) {
        for (int i = 0; i < (nmat == 2 ? 2 : 3); ++i) {
            if (!p.m[i].tiled) return fail(POCR_ERR_UNSUPPORTED, "gemm: %dx%d weight has no tile image", p.m[i].rows, p.K);
            if (p.vnni && !p.m[i].usum) return fail(POCR_ERR_UNSUPPORTED, "VNNI gemm: %dx%d weight has no row sums", p.m[i].rows, p.K);
        }
        if (nmat == 2) return launch_gemm_lds_t<2>(s, qtype, p, epi, npad);
        return launch_gemm_lds_t<1>(s, qtype, p, epi, npad);
    }
    if (nmat == 2) return launch_gemm_t<2, 1>(s, qtype, p, epi, npad);
    return launch_gemm_t<1, 2>(s, qtype, p, epi, npad);
}

GemmParams gemm_params_1(const pocr_weight *w) {
    GemmParams p{};
    p.m[0] = p.m[1] = p.m[2] = dev_mat(w);
    p.seg_end[0] = p.seg_end[1] = p.seg_end[2] = w->rows;
    p.rows = w->rows;
    p.K = w->cols;
    return p;
}

template <class T>
int grow(T *&p, size_t count) {
    if (p) (void)hipFree(p);
    p = nullptr;
    HIP_TRY(hipMalloc(&p, std::max<size_t>(count, 64) * sizeof(T)));
    return POCR_OK;
}

int ensure_bufs(pocr_seq *s, int rows) {
    PrefillBufs &b = s->pf;
    const int img_blocks = (s->cap + kPfKeys - 1) / kPfKeys;
    if (rows <= b.cap_rows && img_blocks <= b.img_blocks) return POCR_OK;
    rows = std::max(rows, b.cap_rows);
    const pocr_config &c = s->m->cfg;
    const size_t H = c.hidden, Q = (size_t)c.heads * c.head_dim, KV = (size_t)c.kv_heads * c.head_dim;
    const size_t kmax = std::max({H, Q, (size_t)c.intermediate});
    prefill_free(b);
    RC(grow(b.h, rows * H));
    RC(grow(b.v, rows * H));
    RC(grow(b.qkv, rows * (Q + 2 * KV)));
    RC(grow(b.ho, rows * Q));
    RC(grow(b.g, rows * (size_t)c.intermediate));
    RC(grow(b.xd, 3 * rows * kmax));
    RC(grow(b.xs, (size_t)rows));
    RC(grow(b.xb, (size_t)rows * 4));
    RC(grow(b.pos, (size_t)rows * 4));  // positions [rows][3], then the prompt ids
    RC(grow(b.kvimg, (size_t)c.kv_heads * img_blocks * kPfImage));
    b.cap_rows = rows;
    b.img_blocks = img_blocks;
    return POCR_OK;
}

// every shape the batched layer needs, else the token-by-token path runs
bool prefill_supported(const pocr_model *m) {
    const pocr_config &c = m->cfg;
    const int Q = c.heads * c.head_dim, KV = c.kv_heads * c.head_dim;
    if (c.head_dim != kHD || c.heads % c.kv_heads || c.heads / c.kv_heads > kMaxGroup) return false;
    if (c.hidden % 16 || Q % 16 || c.intermediate % 16) return false;
    for (int li = 0; li < c.layers; ++li) {
        const LayerW &L = m->layers[li];
        const int qt = L.w[POCR_W_Q]->qtype;
        for (int r = 0; r < 7; ++r)
            if (L.w[r]->qtype != qt) return false;
        if (L.w[POCR_W_GATE]->qtype != L.w[POCR_W_UP]->qtype) return false;
        if (Q % kGemmWaveRows || KV % kGemmWaveRows) return false;
        if (!gemm_shape_ok(Q + 2 * KV, c.hidden) || !gemm_shape_ok(c.hidden, Q) ||
            !gemm_shape_ok(c.intermediate, c.hidden) || !gemm_shape_ok(c.hidden, c.intermediate))
            return false;
    }
    return true;
}

// token-by-token prefill (model.go:1514-1536): n sequential steps
int prefill_tokenwise(pocr_seq *s, int n, const float *emb, const int32_t *pos3, float *logits, int32_t *token) {
    const int H = s->m->cfg.hidden;
    for (int i = 0; i < n; ++i) {
        const bool last = i == n - 1;
        RC(step_locked(s, emb + (size_t)i * H, pos3 + 3 * i, last ? 1 : 0, last ? logits : nullptr,
                       last ? token : nullptr));
    }
    return POCR_OK;
}

}  // namespace

namespace pocr {

// M rows of activations against one weight stream: digit planes per row, then
// the MFMA GEMM; shapes it does not take run M launches of the GEMV
int batched_gemv(pocr_ctx *ctx, const DevMat &w, const float *x, int m, float *out) {
    hipStream_t s = ctx->stream;
    if (!gemm_shape_ok(w.rows, w.cols)) {
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
    const bool small = m <= 16 && small_shape_ok(w.rows, w.cols);
    const int npad = small ? 16 : round_up(m, 32);
    RC(ctx->gxd.ensure((size_t)3 * npad * w.cols));
    RC(ctx->gxs.ensure((size_t)npad * 4));
    RC(ctx->gxb.ensure((size_t)npad * 16));
    DigitizeParams d{};
    d.x = x;
    d.x_stride = w.cols;
    d.K = w.cols;
    d.xd = ctx->gxd.as<int8_t>();
    d.plane_stride = (size_t)npad * w.cols;
    d.xs = ctx->gxs.as<float>();
    d.xb = ctx->gxb.as<int>();
    d.tiled = !small && gemm_tiled(w.cols);
    RC(launch_digitize(s, w.qtype, d, m));
    GemmParams p{};
    p.m[0] = p.m[1] = p.m[2] = w;
    p.seg_end[0] = p.seg_end[1] = p.seg_end[2] = w.rows;
    p.rows = w.rows;
    p.K = w.cols;
    p.xd = d.xd;
    p.plane_stride = d.plane_stride;
    p.xs = d.xs;
    p.xb = d.xb;
    p.ntok = m;
    p.out = out;
    p.out_stride = w.rows;
    if (small) return launch_gemm_small_t<1>(s, w.qtype, p, G_PLAIN);
    return launch_gemm(s, w.qtype, 1, p, G_PLAIN, npad);
}

// Batched prefill: every layer runs once over the n prompt tokens (digit
// planes → MFMA GEMMs with the step's epilogues, per-token RoPE + K/V append,
// causal attention), then the LM head on the last token.  Per-token semantics
// match n sequential steps (model.go:1514-1536, 3475-3643).
namespace {

// The VNNI mode's batched prompt (vnni.hpp): Q4/Q6 layers (Q8 keeps plain
// matvecs in that mode), every GEMM on the tile layout with K ≤ 4096 (one
// wave per token forms the bytes), and the ordered attention's row limit.
bool vnni_prefill_ok(const pocr_seq *s) {
    const pocr_model *m = s->m;
    const pocr_config &c = m->cfg;
    if (m->layers[0].w[POCR_W_Q]->qtype == POCR_Q8) return false;
    for (const int K : {c.hidden, c.heads * c.head_dim, c.intermediate})
        if (!gemm_tiled(K) || K > 4096) return false;
    return c.head_dim == kHD && s->cap <= kOrdMaxRows;
}

bool batched_prefill_on(const pocr_seq *s) {
    const char *env = getenv("POCR_BATCHED_PREFILL");
    if ((env && env[0] == '0') || !prefill_supported(s->m)) return false;
    return !s->m->vnni || vnni_prefill_ok(s);
}

// text rows of the prompt from the device embedding table; image rows
// (id == image_token) are left as uploaded
__global__ void k_embed_rows(const int32_t *ids, int n, int32_t image_token, const float *embed, int H, float *h) {
    const int i = blockIdx.x;
    if (i >= n || ids[i] == image_token) return;
    const float4 *src = reinterpret_cast<const float4 *>(embed + (size_t)ids[i] * H);
    float4 *dst = reinterpret_cast<float4 *>(h + (size_t)i * H);
    for (int c = threadIdx.x; c < H / 4; c += blockDim.x) dst[c] = src[c];
}

// the layers over b.h (the n embedding rows) and the LM head on the last row
int prefill_run(pocr_seq *s, int n, const int32_t *pos3, float *logits, int32_t *token);

}  // namespace

int prefill_locked(pocr_seq *s, int n, const float *emb, const int32_t *pos3, float *logits, int32_t *token) {
    if (!batched_prefill_on(s)) return prefill_tokenwise(s, n, emb, pos3, logits, token);
    if (s->len + n > s->cap) return fail(POCR_ERR_ARG, "prefill: %d rows exceed capacity", n);
    RC(ensure_bufs(s, round_up(n, 32)));
    RC(upload_staged(s->m->ctx, s->pf.h, emb, (size_t)n * s->m->cfg.hidden * 4));
    return prefill_run(s, n, pos3, logits, token);
}

int prefill_ids_locked(pocr_seq *s, const int32_t *ids, int n, const float *image, int32_t image_token,
                       const int32_t *pos3, float *logits, int32_t *token, bool image_on_device) {
    pocr_model *m = s->m;
    if (!batched_prefill_on(s) || m->cfg.hidden % 4) return POCR_ERR_UNSUPPORTED;
    if (s->len + n > s->cap) return fail(POCR_ERR_ARG, "prefill: %d rows exceed capacity", n);
    const int H = m->cfg.hidden;
    RC(ensure_bufs(s, round_up(n, 32)));
    PrefillBufs &b = s->pf;
    // runs of image placeholders: their rows straight from the caller's buffer
    int img = 0;
    for (int i = 0; i < n;) {
        if (!image || ids[i] != image_token) {
            ++i;
            continue;
        }
        int j = i;
        while (j < n && ids[j] == image_token) ++j;
        if (image_on_device)
            HIP_TRY(hipMemcpyAsync(b.h + (size_t)i * H, image + (size_t)img * H, (size_t)(j - i) * H * 4,
                                   hipMemcpyDeviceToDevice, m->ctx->stream));
        else
            RC(upload_staged(m->ctx, b.h + (size_t)i * H, image + (size_t)img * H, (size_t)(j - i) * H * 4));
        img += j - i;
        i = j;
    }
    // ids ride in the position buffer's tail (rows·3 int32 + n)
    HIP_TRY(hipMemcpyAsync(b.pos + (size_t)3 * b.cap_rows, ids, (size_t)n * 4, hipMemcpyHostToDevice,
                           m->ctx->stream));
    hipLaunchKernelGGL(k_embed_rows, dim3(n), dim3(kThreads), 0, m->ctx->stream, b.pos + (size_t)3 * b.cap_rows, n,
                       image ? image_token : -1, m->embed, H, b.h);
    HIP_TRY(hipGetLastError());
    return prefill_run(s, n, pos3, logits, token);
}

namespace {

int prefill_run(pocr_seq *s, int n, const int32_t *pos3, float *logits, int32_t *token) {
    pocr_model *m = s->m;
    const pocr_config &c = m->cfg;
    hipStream_t st = m->ctx->stream;
    const int H = c.hidden, Q = c.heads * c.head_dim, KV = c.kv_heads * c.head_dim, F = c.intermediate;
    const int QKV = Q + 2 * KV;
    const int clen0 = s->len;
    const int npad = round_up(n, 32);
    PrefillBufs &b = s->pf;
    HIP_TRY(hipMemcpyAsync(b.pos, pos3, (size_t)n * 12, hipMemcpyHostToDevice, st));
    const float eps = c.rms_norm_eps;
    const float scale = (float)(1.0 / std::sqrt((double)c.head_dim));
    const int qt = m->layers[0].w[POCR_W_Q]->qtype;
    // VNNI mode (vnni.hpp): one plane of activation bytes per token and the
    // mode's integer finish in every GEMM, the ordered attention per (head,
    // token); every step is exact or in the token step's order, so the rows
    // are the token steps' to the bit
    const int vnni = m->vnni ? 1 : 0;

    auto digitize = [&](const float *x, int stride, const float *norm_w, int K) {
        DigitizeParams d{};
        d.x = x;
        d.x_stride = stride;
        d.norm_w = norm_w;
        d.eps = eps;
        d.K = K;
        d.xd = b.xd;
        d.plane_stride = (size_t)npad * K;
        d.xs = b.xs;
        d.xb = b.xb;
        d.tiled = gemm_tiled(K);
        d.vnni = vnni;
        return launch_digitize(st, qt, d, n);
    };
    auto gemm_in = [&](GemmParams &p) {
        p.xd = b.xd;
        p.plane_stride = (size_t)npad * p.K;
        p.xs = b.xs;
        p.xb = b.xb;
        p.ntok = n;
        p.clen0 = clen0;
        p.vnni = vnni;
    };

    for (int li = 0; li < c.layers; ++li) {
        const LayerW &L = m->layers[li];
        const bool last = li + 1 == c.layers;
        // 1. RMSNorm(h)·ln1 → q|k|v
        RC(digitize(b.h, H, L.ln1, H));
        GemmParams g{};
        g.m[0] = dev_mat(L.w[POCR_W_Q]);
        g.m[1] = dev_mat(L.w[POCR_W_K]);
        g.m[2] = dev_mat(L.w[POCR_W_V]);
        g.seg_end[0] = Q;
        g.seg_end[1] = Q + KV;
        g.seg_end[2] = QKV;
        g.rows = QKV;
        g.K = H;
        gemm_in(g);
        g.out = b.qkv;
        g.out_stride = QKV;
        RC(launch_gemm(st, qt, 1, g, G_PLAIN, npad));
        // 2. per-token RoPE, K/V append at rows clen0.., causal attention
        hipLaunchKernelGGL(k_rope_append, dim3(n), dim3(kThreads), 0, st, b.qkv, QKV, b.pos, m->freq, m->axis,
                           c.heads, c.kv_heads, c.head_dim, layer_k(s, li), layer_v(s, li), clen0);
        if (vnni) {
            HIP_TRY(hipGetLastError());
            RC(launch_attn_ordered_rows(st, b.qkv, QKV, layer_k(s, li), layer_v(s, li), c.heads, c.kv_heads, n, clen0,
                                        scale, b.ho, Q));
        } else {
            const int ntiles = (n + kPfTok - 1) / kPfTok, quads = (c.heads / c.kv_heads + 3) / 4;
            const int nblk = (clen0 + n + kPfKeys - 1) / kPfKeys;
            hipLaunchKernelGGL(k_kv_blocks, dim3(nblk, c.kv_heads), dim3(kThreads), 0, st, layer_k(s, li),
                               layer_v(s, li), c.kv_heads, clen0 + n, nblk, b.kvimg);
            hipLaunchKernelGGL(k_attn_prefill, dim3(c.kv_heads * quads, (ntiles + 1) / 2), dim3(kPfThreads), 0, st,
                               b.qkv, QKV, b.kvimg, nblk, c.heads, c.kv_heads, n, clen0, scale, b.ho, Q);
            HIP_TRY(hipGetLastError());
        }
        // 3. o_proj + residual (+ the Q4/Q6 behaviour per token) → v; h if in place
        RC(digitize(b.ho, Q, nullptr, Q));
        GemmParams o = gemm_params_1(L.w[POCR_W_O]);
        gemm_in(o);
        o.h = b.h;
        o.vbuf = b.v;
        o.quirk = (m->quirk && (qt == POCR_Q4 || qt == POCR_Q6)) ? 1 : 0;
        RC(launch_gemm(st, qt, 1, o, G_OPROJ, npad));
        // 4. RMSNorm(v)·ln2 → SiLU(gate)·up
        RC(digitize(b.v, H, L.ln2, H));
        GemmParams gu = gemm_params_1(L.w[POCR_W_GATE]);
        gu.m[1] = dev_mat(L.w[POCR_W_UP]);
        gemm_in(gu);
        gu.out = b.g;
        gu.out_stride = F;
        RC(launch_gemm(st, qt, 2, gu, G_SWIGLU, npad));
        // 5. down + residual; last layer: v = h + down
        RC(digitize(b.g, F, nullptr, F));
        GemmParams d = gemm_params_1(L.w[POCR_W_DOWN]);
        gemm_in(d);
        d.h = b.h;
        d.vbuf = b.v;
        d.last = last ? 1 : 0;
        RC(launch_gemm(st, qt, 1, d, G_DOWN, npad));
    }

    // step state after the last prompt token, then the LM head on its row
    StepState hs{};
    hs.len = clen0 + n;
    hs.clen = clen0 + n - 1;
    hs.cap = s->cap;
    hs.half = c.head_dim / 2;
    hs.pos[0] = pos3[3 * (n - 1)];
    hs.pos[1] = pos3[3 * (n - 1) + 1];
    hs.pos[2] = pos3[3 * (n - 1) + 2];
    HIP_TRY(hipMemcpyAsync(s->st, &hs, sizeof(hs), hipMemcpyHostToDevice, st));
    HIP_TRY(hipStreamSynchronize(st));  // hs is a stack object
    RC(enqueue_lm_head(s, b.v + (size_t)(n - 1) * H, logits != nullptr));
    StepState out;
    RC(read_state(s, &out));
    s->len = clen0 + n;
    if (token) {
        const unsigned long long key = argmax_of(out);
        if (key == 0ull) return fail(POCR_ERR_DEVICE, "prefill: no finite logit");
        *token = (int32_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
    }
    if (logits) HIP_TRY(hipMemcpy(logits, s->logits, (size_t)c.vocab * 4, hipMemcpyDeviceToHost));
    return POCR_OK;
}

}  // namespace

int digitize_rows(hipStream_t s, int qtype, const DigitizeParams &p, int n) { return launch_digitize(s, qtype, p, n); }
int gemm_rows(hipStream_t s, int qtype, int nmat, const GemmParams &p, int epi, int npad) {
    return launch_gemm(s, qtype, nmat, p, epi, npad);
}
bool gemm_small_ok(int rows, int K) { return small_shape_ok(rows, K); }
int gemm_small_rows(hipStream_t s, int qtype, int nmat, const GemmParams &p, int epi) {
    if (p.ntok > 16 || !small_shape_ok(p.rows, p.K) || p.plane_stride != (size_t)16 * p.K)
        return fail(POCR_ERR_UNSUPPORTED, "gemm: %d tokens of %dx%d outside the small kernel", p.ntok, p.rows, p.K);
    return nmat == 2 ? launch_gemm_small_t<2>(s, qtype, p, epi) : launch_gemm_small_t<1>(s, qtype, p, epi);
}

}  // namespace pocr
