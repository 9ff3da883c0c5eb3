// projector.hip — the vision projector (mlp_AR) on the device: the step that
// turns vision-encoder rows into the decoder's image embeddings
// ((*Runtime).projectImage / projectImageRows, internal/model/vision.go:
// 1029-1108; VulkanProjectImageF32, internal/backend/vulkan_exec_stub.go:122).
//
// For merged row b (frame t, block (by, bx) of the 2×2 patch grid):
//   m_b  = [LN(x[base]) | LN(x[base+1]) | LN(x[base+W]) | LN(x[base+W+1])]
//   h_b  = GELUTanh(W1·m_b + b1)          W1: [4·vd][4·vd]
//   out_b = W2·h_b + b2                    W2: [td][4·vd]
// with LN(x) = ((x − mean)·fastRsqrt(var/n + eps))·w + b (ops.go:1060-1097)
// and both matrices quantized to Q8 rows once, as cacheVisionWeights does
// (vision.go:286-302; the runtime then multiplies with matVecQ8BiasSerial,
// quant.go:1443-1473).
//
// Device plan: one LayerNorm workgroup per vision row writes straight into
// its merged row's quarter; the merged rows become int8 digit planes and run
// through the int8-MFMA GEMM with a bias+GELU epilogue, digitize again, and
// a second GEMM with a bias epilogue writes the embeddings — for
// pocr_generate_vision straight into the prompt's image rows in HBM.
#include "gemm.hpp"
#include "internal.hpp"

using namespace pocr;

struct pocr_projector {
    pocr_ctx *ctx = nullptr;
    int vd = 0, td = 0;
    float eps = 0.0f;
    float *norm_w = nullptr, *norm_b = nullptr, *b1 = nullptr, *b2 = nullptr;
    pocr_weight *w1 = nullptr, *w2 = nullptr;
    // per-call buffers, grown on demand
    float *x = nullptr;       // [vision rows][vd]
    float *merged = nullptr;  // [rows][4·vd]
    float *hidden = nullptr;  // [rows][4·vd]
    float *out = nullptr;     // [rows][td]
    int8_t *xd = nullptr;     // [3][cap_rows][4·vd]
    float *xs = nullptr;
    int *xb = nullptr;
    int cap_rows = 0, cap_vis = 0;
    ~pocr_projector();
};

namespace {

void dfree(void *p) {
    if (p) (void)hipFree(p);
}

// LayerNorm of vision row i (ops.go:1060-1097) into quarter q of merged row
// b (projectImageRows' block walk, vision.go:1070-1106).  Sums are tree
// reductions (the reference's 8-lane partial sums differ in rounding order).
__global__ void __launch_bounds__(kThreads) k_ln_merge(const float *x, int vd, int H, int W, const float *w,
                                                      const float *bias, float eps, float *merged) {
#pragma clang fp contract(off)
    __shared__ float red[kWaves];
    const int i = blockIdx.x;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int hw = H * W;
    const int f = i / hw, rem = i - f * hw, yy = rem / W, xx = rem - yy * W;
    const int bh = H / 2, bw = W / 2;
    if (yy / 2 >= bh || xx / 2 >= bw) return;  // odd edge rows belong to no block (uniform)
    const int b = f * bh * bw + (yy / 2) * bw + xx / 2;
    const int q = (yy & 1) * 2 + (xx & 1);
    const float *xr = x + (size_t)i * vd;
    float *out = merged + (size_t)b * 4 * vd + (size_t)q * vd;
    float s = 0.0f;
    for (int c = t; c < vd; c += kThreads) s += xr[c];
    s = wave_sum(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    float sum = red[0];
#pragma unroll
    for (int k = 1; k < kWaves; ++k) sum += red[k];
    const float mean = sum / (float)vd;
    __syncthreads();
    float v = 0.0f;
    for (int c = t; c < vd; c += kThreads) {
        const float d = xr[c] - mean;
        v += d * d;
    }
    v = wave_sum(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float var = red[0];
#pragma unroll
    for (int k = 1; k < kWaves; ++k) var += red[k];
    const float scale = fast_rsqrt_ref(var / (float)vd + eps);
    for (int c = t; c < vd; c += kThreads) out[c] = (xr[c] - mean) * scale * w[c] + bias[c];
}

int round32(int x) { return (x + 31) / 32 * 32; }

int grow(pocr_projector *p, int vis_rows, int rows) {
    const int K = 4 * p->vd;
    if (vis_rows > p->cap_vis) {
        dfree(p->x);
        p->x = nullptr;
        p->cap_vis = 0;
        HIP_TRY(hipMalloc(&p->x, (size_t)vis_rows * p->vd * 4));
        p->cap_vis = vis_rows;
    }
    const int cap = round32(rows);
    if (cap > p->cap_rows) {
        for (void *q : {(void *)p->merged, (void *)p->hidden, (void *)p->out, (void *)p->xd, (void *)p->xs,
                        (void *)p->xb})
            dfree(q);
        p->merged = p->hidden = p->out = p->xs = nullptr;
        p->xd = nullptr;
        p->xb = nullptr;
        p->cap_rows = 0;
        HIP_TRY(hipMalloc(&p->merged, (size_t)cap * K * 4));
        HIP_TRY(hipMalloc(&p->hidden, (size_t)cap * K * 4));
        HIP_TRY(hipMalloc(&p->out, (size_t)cap * p->td * 4));
        HIP_TRY(hipMalloc(&p->xd, (size_t)3 * cap * K));
        HIP_TRY(hipMalloc(&p->xs, (size_t)cap * 4));
        HIP_TRY(hipMalloc(&p->xb, (size_t)cap * 16));
        // padding token rows of the digit planes are read by the GEMM tiles
        // (never stored): keep them defined
        HIP_TRY(hipMemset(p->xd, 0, (size_t)3 * cap * K));
        HIP_TRY(hipMemset(p->xs, 0, (size_t)cap * 4));
        HIP_TRY(hipMemset(p->xb, 0, (size_t)cap * 16));
        p->cap_rows = cap;
    }
    return POCR_OK;
}

GemmParams proj_gemm(const pocr_projector *p, const pocr_weight *w, const float *bias, float *out, int n, int npad) {
    GemmParams g{};
    g.m[0] = g.m[1] = g.m[2] = dev_mat(w);
    g.seg_end[0] = g.seg_end[1] = g.seg_end[2] = w->rows;
    g.rows = w->rows;
    g.K = w->cols;
    g.xd = p->xd;
    g.plane_stride = (size_t)npad * w->cols;
    g.xs = p->xs;
    g.xb = p->xb;
    g.ntok = n;
    g.out = out;
    g.out_stride = w->rows;
    g.bias = bias;
    return g;
}

int digitize(const pocr_projector *p, const float *x, int n, int npad) {
    DigitizeParams d{};
    d.x = x;
    d.x_stride = 4 * p->vd;
    d.norm_w = nullptr;
    d.K = 4 * p->vd;
    d.xd = p->xd;
    d.plane_stride = (size_t)npad * d.K;
    d.xs = p->xs;
    d.xb = p->xb;
    d.tiled = gemm_tiled(d.K);
    return digitize_rows(p->ctx->stream, QT_Q8, d, n);
}

}  // namespace

pocr_projector::~pocr_projector() {
    for (void *q : {(void *)norm_w, (void *)norm_b, (void *)b1, (void *)b2, (void *)x, (void *)merged,
                    (void *)hidden, (void *)out, (void *)xd, (void *)xs, (void *)xb})
        dfree(q);
    if (w1) weight_release(w1);
    if (w2) weight_release(w2);
    if (ctx) ctx_release(ctx);
}

// Vision rows already on the device (p->x) → p->out on the context stream;
// caller holds the context lock.  Returns the merged row count via *rows.
int pocr::project_locked(pocr_projector *p, int grid_t, int grid_h, int grid_w, int *rows_out) {
    hipStream_t st = p->ctx->stream;
    const int rows = grid_t * (grid_h / 2) * (grid_w / 2);
    *rows_out = rows;
    if (rows == 0) return POCR_OK;
    const int npad = round32(rows);
    hipLaunchKernelGGL(k_ln_merge, dim3(grid_t * grid_h * grid_w), dim3(kThreads), 0, st, p->x, p->vd, grid_h, grid_w,
                       p->norm_w, p->norm_b, p->eps, p->merged);
    HIP_TRY(hipGetLastError());
    RC(digitize(p, p->merged, rows, npad));
    GemmParams g1 = proj_gemm(p, p->w1, p->b1, p->hidden, rows, npad);
    RC(gemm_rows(st, QT_Q8, 1, g1, G_BIAS_GELU, npad));
    RC(digitize(p, p->hidden, rows, npad));
    GemmParams g2 = proj_gemm(p, p->w2, p->b2, p->out, rows, npad);
    return gemm_rows(st, QT_Q8, 1, g2, G_BIAS, npad);
}

int pocr::project_upload_locked(pocr_projector *p, const float *vision_rows, int grid_t, int grid_h, int grid_w,
                                const float **out_dev, int *rows) {
    const int n_vis = grid_t * grid_h * grid_w;
    RC(grow(p, n_vis, grid_t * (grid_h / 2) * (grid_w / 2)));
    RC(upload_staged(p->ctx, p->x, vision_rows, (size_t)n_vis * p->vd * 4));
    RC(project_locked(p, grid_t, grid_h, grid_w, rows));
    *out_dev = p->out;
    return POCR_OK;
}

extern "C" int pocr_projector_create(pocr_ctx *ctx, int vision_dim, int text_dim, const float *norm_w,
                                     const float *norm_b, const float *w1, const float *b1, const float *w2,
                                     const float *b2, float eps, pocr_projector **out) {
    if (!ctx || !out || !norm_w || !norm_b || !w1 || !b1 || !w2 || !b2 || vision_dim <= 0 || text_dim <= 0)
        return fail(POCR_ERR_ARG, "pocr_projector_create: bad arguments");
    *out = nullptr;
    const int K = 4 * vision_dim;
    // the MFMA GEMM takes K in 128-column stages and rows in 64-row tiles
    if (K % kStageCols || K > 2 * 16 * kThreads || text_dim % kGemmWaveRows)
        return fail(POCR_ERR_UNSUPPORTED, "projector: vision_dim %d (4·vd a multiple of 128, <= 8192), text_dim %d "
                    "(multiple of 64)", vision_dim, text_dim);
    CHECK_INJECT("projector");
    // quantize like cacheVisionWeights (QuantizeQ8Row, round half away)
    std::vector<float> s1(K), s2(text_dim);
    std::vector<uint8_t> q1((size_t)K * K), q2((size_t)text_dim * K);
    RC(pocr_quantize_rows(POCR_Q8, 0, w1, K, K, s1.data(), q1.data()));
    RC(pocr_quantize_rows(POCR_Q8, 0, w2, text_dim, K, s2.data(), q2.data()));
    pocr_projector *p = new pocr_projector();
    int rc = pocr_weight_upload(ctx, POCR_Q8, K, K, s1.data(), q1.data(), &p->w1);
    if (rc == POCR_OK) rc = pocr_weight_upload(ctx, POCR_Q8, text_dim, K, s2.data(), q2.data(), &p->w2);
    if (rc != POCR_OK) {
        delete p;
        return rc;
    }
    ctx->refs.fetch_add(1);
    p->ctx = ctx;
    p->vd = vision_dim;
    p->td = text_dim;
    p->eps = eps;
    std::lock_guard<std::mutex> lk(ctx->mu);
    hipError_t e = hipSetDevice(ctx->device);
    const size_t vb = (size_t)vision_dim * 4;
    if (e == hipSuccess) e = hipMalloc(&p->norm_w, vb);
    if (e == hipSuccess) e = hipMalloc(&p->norm_b, vb);
    if (e == hipSuccess) e = hipMalloc(&p->b1, (size_t)K * 4);
    if (e == hipSuccess) e = hipMalloc(&p->b2, (size_t)text_dim * 4);
    if (e == hipSuccess) e = hipMemcpy(p->norm_w, norm_w, vb, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(p->norm_b, norm_b, vb, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(p->b1, b1, (size_t)K * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(p->b2, b2, (size_t)text_dim * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        delete p;
        return fail(POCR_ERR_NOMEM, "pocr_projector_create: %s", hipGetErrorString(e));
    }
    *out = p;
    return POCR_OK;
}

extern "C" void pocr_projector_destroy(pocr_projector *p) {
    if (!p) return;
    pocr_ctx *ctx = p->ctx;
    if (ctx) {
        std::lock_guard<std::mutex> lk(ctx->mu);
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
    }
    delete p;
}

extern "C" int pocr_project_image(pocr_projector *p, const float *vision_rows, int grid_t, int grid_h, int grid_w,
                                  float *out) {
    if (!p || !vision_rows || !out || grid_t <= 0 || grid_h <= 0 || grid_w <= 0)
        return fail(POCR_ERR_ARG, "pocr_project_image: bad arguments");
    CHECK_INJECT("project_image");
    std::lock_guard<std::mutex> lk(p->ctx->mu);
    HIP_TRY(hipSetDevice(p->ctx->device));
    const float *dev = nullptr;
    int rows = 0;
    RC(project_upload_locked(p, vision_rows, grid_t, grid_h, grid_w, &dev, &rows));
    if (rows == 0) return 0;
    HIP_TRY(hipMemcpyAsync(out, dev, (size_t)rows * p->td * 4, hipMemcpyDeviceToHost, p->ctx->stream));
    HIP_TRY(hipStreamSynchronize(p->ctx->stream));
    return rows;
}

extern "C" int pocr_time_project(pocr_projector *p, int grid_t, int grid_h, int grid_w, int iters, float *avg_us) {
    if (!p || grid_t <= 0 || grid_h <= 1 || grid_w <= 1 || iters <= 0 || !avg_us)
        return fail(POCR_ERR_ARG, "pocr_time_project: bad arguments");
    CHECK_INJECT("time_project");
    std::lock_guard<std::mutex> lk(p->ctx->mu);
    HIP_TRY(hipSetDevice(p->ctx->device));
    hipStream_t st = p->ctx->stream;
    const int n_vis = grid_t * grid_h * grid_w;
    RC(grow(p, n_vis, grid_t * (grid_h / 2) * (grid_w / 2)));
    // vision rows hold 1/128 (the values do not change the work)
    HIP_TRY(hipMemsetD32Async((hipDeviceptr_t)p->x, 0x3C000000, (size_t)n_vis * p->vd, st));
    int rows = 0;
    RC(project_locked(p, grid_t, grid_h, grid_w, &rows));
    hipEvent_t e0, e1;
    HIP_TRY(hipEventCreate(&e0));
    HIP_TRY(hipEventCreate(&e1));
    HIP_TRY(hipEventRecord(e0, st));
    for (int i = 0; i < iters; ++i) RC(project_locked(p, grid_t, grid_h, grid_w, &rows));
    HIP_TRY(hipEventRecord(e1, st));
    HIP_TRY(hipEventSynchronize(e1));
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *avg_us = ms * 1000.0f / (float)iters;
    return POCR_OK;
}

int pocr::projector_text_dim(const pocr_projector *p) { return p->td; }
pocr_ctx *pocr::projector_ctx(const pocr_projector *p) { return p->ctx; }
