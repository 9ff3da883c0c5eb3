// pocr_runtime.hip — host runtime of the C ABI in include/pocr_hip.h.
//
// One context per device owns a HIP stream (default priority) and a mutex;
// weights are uploaded once in their Q*_ROW layout; a sequence owns its
// per-layer fp32 K/V cache in HBM, its step state and its scratch vectors, and
// a captured HIP graph of the whole greedy decode step that is replayed token
// after token without host round trips.
#include <cmath>

#include "gemm.hpp"
#include "vnni.hpp"
#include "head.hpp"
#include "internal.hpp"

namespace pocr {

// POCR_HIP_FAIL_OP=<op>[,<op>...] makes the named ops return POCR_ERR_INJECTED
// before touching the device, so a caller's CPU fallback can be exercised
// (the reference disables a failing op and uses the CPU kernel,
// internal/model/model.go:7240-7258).
bool injected(const char *op) {
    const char *env = getenv("POCR_HIP_FAIL_OP");
    if (!env || !*env) return false;
    std::string s(env);
    size_t start = 0;
    while (start <= s.size()) {
        size_t end = s.find(',', start);
        if (end == std::string::npos) end = s.size();
        if (s.compare(start, end - start, op) == 0 || s.compare(start, end - start, "all") == 0) return true;
        start = end + 1;
    }
    return false;
}

}  // namespace pocr

using namespace pocr;

extern "C" int pocr_abi_version(void) { return POCR_ABI_VERSION; }

extern "C" int pocr_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

static void free_dev(void *p) {
    if (p) (void)hipFree(p);
}

static void drop_decode_graphs(pocr_seq *s) {
    if (s->decode_exec) (void)hipGraphExecDestroy(s->decode_exec);
    if (s->decode_graph) (void)hipGraphDestroy(s->decode_graph);
    if (s->decode_exec_n) (void)hipGraphExecDestroy(s->decode_exec_n);
    if (s->decode_graph_n) (void)hipGraphDestroy(s->decode_graph_n);
    s->decode_exec = s->decode_exec_n = nullptr;
    s->decode_graph = s->decode_graph_n = nullptr;
}

pocr_seq::~pocr_seq() {
    drop_decode_graphs(this);
    free_dev(kv);
    free_dev(h);
    free_dev(qkv);
    free_dev(head_out);
    free_dev(opart);
    free_dev(vbuf);
    free_dev(g);
    free_dev(logits);
    free_dev(part);
    free_dev(st);
    free_dev(tokens);
    free_dev(eos_bits);
    free_dev(samp);
    free_dev(topk_part);
    prefill_free(pf);
}

// ---------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------
// Split records of pocr_text_attention_noalloc: a fixed device array (each
// GPU holds its own copy until the process ends), so that entry allocates
// nothing.  Host code never passes the array's name to a kernel: its device
// address is taken once per device (scratch_setup) and kept in the context.
constexpr int kNoAllocSplitRecs = 512;  // kv heads × splits
constexpr size_t kNoAllocScratchFloats = (size_t)kNoAllocSplitRecs * kMaxGroup * kRec;
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

static std::mutex g_scratch_mu;
static float *g_scratch[64];  // per device, set once

// the current device's scratch address (the device must be current)
static int scratch_setup(int device, float **out) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (device < 0 || device >= 64) return fail(POCR_ERR_UNSUPPORTED, "device %d: at most 64 devices", device);
    if (!g_scratch[device]) {
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(POCR_ERR_DEVICE, "device %d: scratch address: %s", device, hipGetErrorString(e));
        g_scratch[device] = static_cast<float *>(ptr);
    }
    *out = g_scratch[device];
    return POCR_OK;
}

extern "C" int pocr_ctx_create(int device, pocr_ctx **out) {
    if (!out) return fail(POCR_ERR_ARG, "pocr_ctx_create: null out");
    *out = nullptr;
    CHECK_INJECT("ctx");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(POCR_ERR_DEVICE, "no HIP device visible");
    if (device < 0 || device >= n) return fail(POCR_ERR_ARG, "device %d out of range [0,%d)", device, n);
    HIP_TRY(hipSetDevice(device));
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(POCR_ERR_UNSUPPORTED, "device %d is %s; this library is built for gfx950", device, prop.gcnArchName);
    float *scr = nullptr;
    RC(scratch_setup(device, &scr));
    pocr_ctx *c = new pocr_ctx();
    c->device = device;
    c->scratch = scr;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return fail(POCR_ERR_DEVICE, "hipStreamCreate failed");
    }
    *out = c;
    return POCR_OK;
}

void pocr::ctx_release(pocr_ctx *ctx) {
    if (!ctx || ctx->refs.fetch_sub(1) != 1) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) {
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipStreamDestroy(ctx->stream);
    }
    for (hipEvent_t &e : ctx->pin_ev)
        if (e) (void)hipEventDestroy(e);
    if (ctx->pin) (void)hipHostFree(ctx->pin);
    if (ctx->readback) (void)hipHostFree(ctx->readback);
    delete ctx;
}

// Chunks of at most pin_half bytes alternate between the two pinned halves:
// the host copy into a half waits only for that half's previous transfer, so
// the memcpy of one chunk overlaps the DMA of the one before.
int pocr::upload_staged(pocr_ctx *ctx, void *dst, const void *src, size_t bytes) {
    constexpr size_t kHalf = 2u << 20;
    if (!ctx->pin) {
        HIP_TRY(hipHostMalloc((void **)&ctx->pin, 2 * kHalf, hipHostMallocDefault));
        ctx->pin_half = kHalf;
        for (hipEvent_t &e : ctx->pin_ev) HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    }
    const uint8_t *s8 = static_cast<const uint8_t *>(src);
    uint8_t *d8 = static_cast<uint8_t *>(dst);
    for (size_t off = 0, c = 0; off < bytes; off += ctx->pin_half, ++c) {
        const size_t len = std::min(ctx->pin_half, bytes - off);
        uint8_t *half = ctx->pin + (c & 1) * ctx->pin_half;
        HIP_TRY(hipEventSynchronize(ctx->pin_ev[c & 1]));
        std::memcpy(half, s8 + off, len);
        HIP_TRY(hipMemcpyAsync(d8 + off, half, len, hipMemcpyHostToDevice, ctx->stream));
        HIP_TRY(hipEventRecord(ctx->pin_ev[c & 1], ctx->stream));
    }
    return POCR_OK;
}

extern "C" void pocr_ctx_destroy(pocr_ctx *ctx) { ctx_release(ctx); }

// ---------------------------------------------------------------------------
// weights
// ---------------------------------------------------------------------------
static bool valid_qtype(int q) { return q == POCR_Q8 || q == POCR_Q4 || q == POCR_Q6; }

// Q6 matrices of LM-head size (the shapes the greedy heads take) also keep
// their rows in the heads' load order (head.hpp, k_head_image_q6);
// POCR_HEAD_IMAGE=0 at upload leaves a weight without it (the heads then read
// the rows)
static bool head_image_ok(int qtype, int rows, int cols) {
    const char *env = getenv("POCR_HEAD_IMAGE");
    if (env && env[0] == '0') return false;
    return qtype == POCR_Q6 && (cols == 1024 || cols == 2048) && rows >= kHeadWideMinRows;
}
static size_t head_image_bytes(int rows, size_t row_bytes) { return (size_t)(rows + 15) / 16 * 16 * row_bytes; }
static int head_image_q6(hipStream_t s, const uint8_t *src, int row_bytes, int rows, uint8_t *dst) {
    const int nblk = (rows + 15) / 16;
    const size_t threads = (size_t)nblk * 16 * (row_bytes / 768) * 64;
    hipLaunchKernelGGL(k_head_image_q6, dim3((unsigned)((threads + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, src,
                       row_bytes, rows, nblk, dst);
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

extern "C" int pocr_weight_upload(pocr_ctx *ctx, int qtype, int rows, int cols, const float *scales,
                                  const uint8_t *packed, pocr_weight **out) {
    if (!ctx || !out || !scales || !packed) return fail(POCR_ERR_ARG, "pocr_weight_upload: null argument");
    *out = nullptr;
    if (!valid_qtype(qtype)) return fail(POCR_ERR_ARG, "pocr_weight_upload: unsupported type %d", qtype);
    if (rows <= 0 || cols <= 0) return fail(POCR_ERR_ARG, "pocr_weight_upload: bad shape %dx%d", rows, cols);
    CHECK_INJECT("weight_upload");
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    const size_t rb = pocr_row_bytes(qtype, cols);
    const size_t scale_bytes = (((size_t)rows * 4) + 255) & ~(size_t)255;  // keep rows 256-B aligned
    const size_t data_bytes = rb * (size_t)rows;
    void *base = nullptr;
    HIP_TRY(hipMalloc(&base, scale_bytes + data_bytes + 64));  // +64: tail chunk over-read guard
    hipError_t e = hipMemcpy(base, scales, (size_t)rows * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy((uint8_t *)base + scale_bytes, packed, data_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset((uint8_t *)base + scale_bytes + data_bytes, 0, 64);
    if (e != hipSuccess) {
        (void)hipFree(base);
        return fail(POCR_ERR_DEVICE, "weight upload copy: %s", hipGetErrorString(e));
    }
    // the prefill GEMM's image of the same bytes (k_tile_weight), and for Q4/Q6
    // the rows' code sums of its VNNI mode
    uint8_t *tiled = nullptr, *head_img = nullptr;
    int *usum = nullptr;
    // the image is an optional copy: without room for it the heads read the rows
    if (head_image_ok(qtype, rows, cols) && hipMalloc(&head_img, head_image_bytes(rows, rb)) != hipSuccess) {
        (void)hipGetLastError();
        head_img = nullptr;
    }
    if (head_img) {
        int rc = head_image_q6(ctx->stream, (const uint8_t *)base + scale_bytes, (int)rb, rows, head_img);
        if (rc == POCR_OK && (e = hipStreamSynchronize(ctx->stream)) != hipSuccess)
            rc = fail(POCR_ERR_DEVICE, "weight head image: %s", hipGetErrorString(e));
        if (rc != POCR_OK) {
            free_dev(head_img);
            (void)hipFree(base);
            return rc;
        }
    }
    if (weight_tiles_ok(rows, cols)) {
        const uint8_t *src = (const uint8_t *)base + scale_bytes;
        e = hipMalloc(&tiled, data_bytes);
        if (e == hipSuccess && qtype != POCR_Q8) e = hipMalloc(&usum, (size_t)rows * sizeof(int));
        int rc = e == hipSuccess ? POCR_OK : fail(POCR_ERR_DEVICE, "weight tile image: %s", hipGetErrorString(e));
        if (rc == POCR_OK) rc = tile_weight(ctx->stream, qtype, src, (int)rb, rows, cols, tiled);
        if (rc == POCR_OK && usum) rc = row_usum(ctx->stream, qtype, src, (int)rb, rows, cols, usum);
        if (rc == POCR_OK && (e = hipStreamSynchronize(ctx->stream)) != hipSuccess)
            rc = fail(POCR_ERR_DEVICE, "weight tile image: %s", hipGetErrorString(e));
        if (rc != POCR_OK) {
            free_dev(usum);
            free_dev(tiled);
            free_dev(head_img);
            (void)hipFree(base);
            return rc;
        }
    }
    pocr_weight *w = new pocr_weight();
    ctx->refs.fetch_add(1);
    w->ctx = ctx;
    w->qtype = qtype;
    w->rows = rows;
    w->cols = cols;
    w->row_bytes = rb;
    w->base = base;
    w->scale = (const float *)base;
    w->data = (const uint8_t *)base + scale_bytes;
    w->tiled = tiled;
    w->usum = usum;
    w->head_img = head_img;
    *out = w;
    return POCR_OK;
}

void pocr::weight_retain(const pocr_weight *w) {
    if (w) const_cast<pocr_weight *>(w)->refs.fetch_add(1);
}

void pocr::weight_release(const pocr_weight *cw) {
    pocr_weight *w = const_cast<pocr_weight *>(cw);
    if (!w || w->refs.fetch_sub(1) != 1) return;
    pocr_ctx *ctx = w->ctx;
    {
        std::lock_guard<std::mutex> lk(ctx->mu);
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        free_dev(w->base);
        free_dev(w->tiled);
        free_dev(w->usum);
        free_dev(w->head_img);
    }
    delete w;
    ctx_release(ctx);
}

extern "C" void pocr_weight_free(pocr_weight *w) { weight_release(w); }

DevMat pocr::dev_mat(const pocr_weight *w) {
    DevMat m;
    m.scale = w->scale;
    m.data = w->data;
    m.tiled = w->tiled;
    m.usum = w->usum;
    m.head_img = w->head_img;
    m.rows = w->rows;
    m.cols = w->cols;
    m.row_bytes = (int)w->row_bytes;
    m.qtype = w->qtype;
    return m;
}

// ---------------------------------------------------------------------------
// GEMV dispatch
// ---------------------------------------------------------------------------
template <int QT, int L, int C, int U, int NMAT, int TAG, bool ONE, int NPL, int NV>
static const void *gemv_fn() {
    if constexpr (NV > 1) return reinterpret_cast<const void *>(&k_gemv_nv<QT, L, C, U, NMAT, NPL, NV, ONE>);
    else if constexpr (ONE) return reinterpret_cast<const void *>(&k_gemv_one<QT, L, C, U, NMAT, TAG, NPL>);
    else return reinterpret_cast<const void *>(&k_gemv<QT, L, C, U, NMAT, TAG, NPL>);
}

template <int QT, int NMAT, int U, int TAG = 0, bool ONE = false, int NPL = 3, int NV = 1>
static bool gemv_fast_kernel(int lpr, int cpl, const void **fn) {
#define POCR_K(L, C)                                            \
    if (lpr == L && cpl == C) {                                 \
        *fn = gemv_fn<QT, L, C, U, NMAT, TAG, ONE, NPL, NV>();  \
        return true;                                            \
    }
    if constexpr (U > 2) {  // the large single-matrix shape: one chunk per lane
        POCR_K(64, 1)
        POCR_K(32, 1)
    } else {
        POCR_K(64, 1)
        POCR_K(64, 2)
        POCR_K(64, 3)
        POCR_K(64, 4)
        POCR_K(32, 1)
        POCR_K(32, 2)
        POCR_K(32, 3)
    }
#undef POCR_K
    return false;
}

// Launch shape of the large single-matrix GEMV (the LM head): rows per lane
// group and step, and the workgroup cap (rows loop inside the kernel).
#ifndef POCR_BIG_U
#define POCR_BIG_U 8
#endif
#ifndef POCR_BIG_GRID
#define POCR_BIG_GRID 4096  // enough for one group per wave up to 262144 rows
#endif
constexpr int kBigU = POCR_BIG_U;
// one: every wave gets at most one row group (the big launch covers them all)
template <int QT>
static bool pick_big(int tag, bool one, int lpr, int cpl, const void **fn) {
    if (one)
        return tag == 1 ? gemv_fast_kernel<QT, 1, kBigU, 1, true>(lpr, cpl, fn)
                        : gemv_fast_kernel<QT, 1, kBigU, 0, true>(lpr, cpl, fn);
    return tag == 1 ? gemv_fast_kernel<QT, 1, kBigU, 1, false>(lpr, cpl, fn)
                    : gemv_fast_kernel<QT, 1, kBigU, 0, false>(lpr, cpl, fn);
}

// NV activation vectors per weight pass (batched decode): the big launch keeps
// kBigU rows per lane group (U·NV ≤ 32 reduce-scatter entries, the workgroup
// count and its activation prologues as for one vector) and gives every wave
// one group
template <int QT, int NV>
static bool pick_nv(int nmat, int u, int lpr, int cpl, const void **fn) {
    if (nmat == 2) return gemv_fast_kernel<QT, 2, 2, 0, false, 3, NV>(lpr, cpl, fn);
    if (u == kBigU) return gemv_fast_kernel<QT, 1, kBigU, 0, true, 3, NV>(lpr, cpl, fn);
    if (u == 1) {  // only the down projection's shape takes one row per lane group here
        if (lpr != 32 || cpl != 3) return false;
        *fn = gemv_fn<QT, 32, 3, 1, 1, 0, false, 3, NV>();
        return true;
    }
    return gemv_fast_kernel<QT, 1, 2, 0, false, 3, NV>(lpr, cpl, fn);
}

template <int QT>
static bool pick_fast(int nmat, int u, int tag, int lpr, int cpl, bool one, int nv, const void **fn) {
    if (nv == 2) return pick_nv<QT, 2>(nmat, u, lpr, cpl, fn);
    if (nv == 4) return pick_nv<QT, 4>(nmat, u, lpr, cpl, fn);
    if (nmat == 2) return gemv_fast_kernel<QT, 2, 2>(lpr, cpl, fn);
    if (u == kBigU) return pick_big<QT>(tag, one, lpr, cpl, fn);
    if (u == 1) return tag == 1 ? gemv_fast_kernel<QT, 1, 1, 1>(lpr, cpl, fn) : gemv_fast_kernel<QT, 1, 1>(lpr, cpl, fn);
    return tag == 1 ? gemv_fast_kernel<QT, 1, 2, 1>(lpr, cpl, fn) : gemv_fast_kernel<QT, 1, 2>(lpr, cpl, fn);
}

struct GemvPlan {
    const void *fn = nullptr;
    int grid = 1;
    size_t lds = 0;
    int nv = 1;  // > 1: the kernel takes a GemvNV argument
};

// Choose the kernel for `rows` outputs of matrices with `cols` columns.
// max_grid caps the workgroup count (rows loop inside the kernel).
static int plan_gemv(int qtype, int nmat, int rows, int cols, const DevMat *mats, int nm, int max_grid,
                     GemvPlan *plan, int tag, const int *seg_end, int epi, int nv = 1) {
    if (nv != 1 && nv != 2 && nv != 4) return fail(POCR_ERR_UNSUPPORTED, "gemv: %d vectors per pass", nv);
    if (cols > 16384) return fail(POCR_ERR_UNSUPPORTED, "gemv: cols %d > 16384", cols);
    plan->lds = (size_t)cols * 4;
    int W = qtype == POCR_Q4 ? 32 : 16;
    int CB = qtype == POCR_Q6 ? 12 : 16;
    bool fast = cols % W == 0 && cols <= kMaxCols;
    int C = cols / W;
    for (int i = 0; i < nm && fast; ++i) {
        if (mats[i].row_bytes != C * CB) fast = false;
        if (((uintptr_t)mats[i].data) % 16 != 0) fast = false;
        if (mats[i].qtype != qtype || mats[i].cols != cols) fast = false;
    }
    int lpr = 0, cpl = 0;
    if (fast) {
        if (C % 64 == 0) lpr = 64;
        else if (C % 32 == 0) lpr = 32;
        else fast = false;
        if (fast) {
            cpl = C / lpr;
            if (cpl > 4 || (lpr == 32 && cpl > 3)) fast = false;
        }
    }
    bool ok = false;
    // big row counts: 8 rows per lane group and step (more bytes in flight)
    const bool big = fast && nmat == 1 && cpl == 1 && rows >= 8192;
    // one row per lane group and step when two would leave fewer than 128
    // workgroups (the down projection's 1024 rows of 3072 columns): the
    // shorter rows of work per wave beat the longer pipeline there
    int u = big ? kBigU : 2;
    if (fast && !big && nmat == 1 && (nv == 1 || (lpr == 32 && cpl == 3))) {
        const int groups2 = (rows + (64 / lpr) * 2 - 1) / ((64 / lpr) * 2);
        if ((groups2 + kWaves - 1) / kWaves < 128) u = 1;
    }
    if (big) max_grid = nv > 1 ? 1 << 30 : std::max(max_grid, POCR_BIG_GRID);
    // row groups must not straddle segments
    if (fast && nmat == 1 && seg_end) {
        const int rg = (64 / lpr) * u;
        for (int i = 0; i < 2; ++i)
            if (seg_end[i] % rg != 0) fast = false;
    }
    int grid = 1;
    bool one = false;
    if (fast) {
        const int rows_per_group = (64 / lpr) * u;
        const int groups = (rows + rows_per_group - 1) / rows_per_group;
        const int want = (groups + kWaves - 1) / kWaves;
        grid = std::max(1, std::min(want, max_grid));
        one = big && grid == want;
        if (qtype == POCR_Q4) ok = pick_fast<QT_Q4>(nmat, u, tag, lpr, cpl, one, nv, &plan->fn);
        if (qtype == POCR_Q8) ok = pick_fast<QT_Q8>(nmat, u, tag, lpr, cpl, one, nv, &plan->fn);
        if (qtype == POCR_Q6) ok = pick_fast<QT_Q6>(nmat, u, tag, lpr, cpl, one, nv, &plan->fn);
    }
    if (ok) {
        plan->lds = (size_t)nv * (qtype == POCR_Q4 ? gemv_lds_bytes<QT_Q4>(cols)
                                                   : (qtype == POCR_Q8 ? gemv_lds_bytes<QT_Q8>(cols)
                                                                       : gemv_lds_bytes<QT_Q6>(cols)));
        plan->grid = grid;
        plan->nv = nv;
    } else if (nv > 1) {
        return fail(POCR_ERR_UNSUPPORTED, "gemv: %d vectors need the fast kernel shapes", nv);
    } else {
        plan->fn = nmat == 1 ? reinterpret_cast<const void *>(&k_gemv_any<1>)
                             : reinterpret_cast<const void *>(&k_gemv_any<2>);
        plan->grid = std::max(1, std::min((rows + kWaves - 1) / kWaves, max_grid));
    }
    return POCR_OK;
}

static int launch_gemv(hipStream_t s, const GemvPlan &plan, GemvParams p, int pro, int epi, GemvNV q = {}) {
    void *args[] = {&p, &pro, &epi, &q};
    if (plan.nv == 1) args[3] = nullptr;
    HIP_TRY(hipLaunchKernel(plan.fn, dim3(plan.grid), dim3(kThreads), args, plan.lds, s));
    return POCR_OK;
}

GemvParams pocr::gemv_params_1(const pocr_weight *w) {
    GemvParams p{};
    p.m[0] = p.m[1] = p.m[2] = dev_mat(w);
    p.seg_end[0] = p.seg_end[1] = p.seg_end[2] = w->rows;
    p.rows = w->rows;
    p.cols = w->cols;
    return p;
}

// The greedy head on the matrix cores (head.hpp) for the shapes it takes:
// one Q4, Q8 or Q6 matrix of 1024 or 2048 columns whose rows are 16-byte
// aligned, 1, 2 or 4 vectors.
template <int QT>
static const void *head_fn(int ns, int nv) {
#define POCR_H(NS, NV) \
    if (ns == NS && nv == NV) return reinterpret_cast<const void *>(&k_head_mfma<QT, NS, NV>);
    POCR_H(4, 1) POCR_H(4, 2) POCR_H(4, 4) POCR_H(8, 1) POCR_H(8, 2) POCR_H(8, 4)
#undef POCR_H
    return nullptr;
}

static const void *plan_head(const GemvParams &p, int nmat, int nv) {
    const DevMat &m = p.m[0];
    if (nmat != 1 || p.seg_end[0] != p.rows || m.cols != p.cols) return nullptr;
    if (p.cols != 1024 && p.cols != 2048) return nullptr;
    if (((uintptr_t)m.data) % 16 != 0 || m.row_bytes % 16 != 0) return nullptr;
    const int ns = p.cols / 256;
    if (m.qtype == POCR_Q4) return head_fn<QT_Q4>(ns, nv);
    if (m.qtype == POCR_Q8) return head_fn<QT_Q8>(ns, nv);
    if (m.qtype == POCR_Q6) return head_fn<QT_Q6>(ns, nv);
    return nullptr;
}

// argmax: fold each vector's best (score, row) into its step state's slots;
// otherwise only the scores are written (a sampling head's logits: the slots
// then carry the drawn token and must not be touched)
static int launch_head(hipStream_t s, const void *fn, const GemvParams &p, int pro, int nv, const GemvNV *q,
                       bool argmax) {
    HeadParams h{};
    h.m = p.m[0];
    h.rows = p.rows;
    h.x = p.x;
    h.x_stride = nv > 1 ? q->x_stride : 0;
    h.norm_w = pro == PRO_RMSNORM ? p.norm_w : nullptr;
    h.eps = p.eps;
    h.out = p.out;
    h.out_stride = nv > 1 ? q->o_stride : 0;
    for (int v = 0; v < kHeadMaxVec; ++v)
        h.st[v] = !argmax ? nullptr : (v == 0 ? p.st : (v < nv ? q->stv[v - 1] : p.st));
    const int blocks = (p.rows + 15) / 16;
    void *args[] = {&h};
    HIP_TRY(hipLaunchKernel(fn, dim3((blocks + kHeadRB - 1) / kHeadRB), dim3(kThreads), args, 0, s));
    return POCR_OK;
}

// The head for 2 to 16 vectors (head.hpp: k_head_digits, then k_head_wide,
// or k_head_wide_q6 for Q6 rows): rows of 1024 or 2048 columns on 16-byte
// boundaries.
struct HeadWidePlan {
    const void *digits = nullptr, *head = nullptr;
    const void *head_few = nullptr;  // up to kHeadPackedVec vectors: one B tile for all planes
    int rows_per_wg = 0, rows_per_wg_few = 0, plane_bytes = 0;
};
constexpr int kHeadPackedVec = 5;  // (vector, plane) pairs in one 16-column B tile

template <int QT, int NS>
static HeadWidePlan head_wide_plan() {
    HeadWidePlan h;
    h.digits = reinterpret_cast<const void *>(&k_head_digits<QT, NS>);
    if constexpr (QT == QT_Q6) {
        h.head = reinterpret_cast<const void *>(&k_head_wide_q6<NS, false>);
        h.head_few = reinterpret_cast<const void *>(&k_head_wide_q6<NS, true>);
    } else {
        h.head = reinterpret_cast<const void *>(&k_head_wide<QT, NS, false>);
        h.head_few = reinterpret_cast<const void *>(&k_head_wide<QT, NS, true>);
    }
    if constexpr (QT == QT_Q6) {
        h.rows_per_wg = h.rows_per_wg_few = HeadWideShape<QT, NS>::ROWS_PER_WG;
    } else {
        h.rows_per_wg = HeadWideShapeK<QT, NS, false>::ROWS_PER_WG;
        h.rows_per_wg_few = HeadWideShapeK<QT, NS, true>::ROWS_PER_WG;
    }
    h.plane_bytes = HeadWideShape<QT, NS>::PLANE_BYTES;
    return h;
}

static bool plan_head_wide(const DevMat &m, HeadWidePlan *h) {
    if (m.cols != 1024 && m.cols != 2048) return false;
    if (((uintptr_t)m.data) % 16 != 0 || m.row_bytes % 16 != 0) return false;
    const bool ns4 = m.cols == 1024;
    if (m.qtype == POCR_Q4) *h = ns4 ? head_wide_plan<QT_Q4, 4>() : head_wide_plan<QT_Q4, 8>();
    else if (m.qtype == POCR_Q8) *h = ns4 ? head_wide_plan<QT_Q8, 4>() : head_wide_plan<QT_Q8, 8>();
    else if (m.qtype == POCR_Q6) *h = ns4 ? head_wide_plan<QT_Q6, 4>() : head_wide_plan<QT_Q6, 8>();
    else return false;
    return true;
}

bool pocr::head_wide_ok(const pocr_weight *w) {
    HeadWidePlan h;
    return plan_head_wide(dev_mat(w), &h);
}

size_t pocr::head_wide_plane_bytes(const pocr_weight *w) {
    HeadWidePlan h;
    return plan_head_wide(dev_mat(w), &h) ? (size_t)h.plane_bytes : 0;
}

// nvec (≤ 16) vectors at x + v·x_stride against w: optional scores at out +
// v·out_stride, optional argmax into st[v] (null entries: none).  planes
// (head_wide_plane_bytes), vscale (16 floats) and vbias (48 ints) are the
// caller's device scratch.
int pocr::launch_head_wide(hipStream_t s, const pocr_weight *w, const float *x, int x_stride, int nvec,
                           const float *norm_w, float eps, float *out, int out_stride, StepState *const *st,
                           int8_t *planes, float *vscale, int *vbias) {
    if (nvec < 1 || nvec > kHeadWideVec) return fail(POCR_ERR_ARG, "head: %d vectors", nvec);
    const DevMat m = dev_mat(w);
    HeadWidePlan plan;
    if (!plan_head_wide(m, &plan)) return fail(POCR_ERR_UNSUPPORTED, "head: %d columns of qtype %d", m.cols, m.qtype);
    HeadDigitParams d{};
    d.x = x;
    d.x_stride = x_stride;
    d.norm_w = norm_w;
    d.eps = eps;
    d.planes = planes;
    d.vscale = vscale;
    d.vbias = vbias;
    void *dargs[] = {&d};
    HIP_TRY(hipLaunchKernel(plan.digits, dim3(nvec), dim3(kThreads), dargs, 0, s));
    HeadWideParams h{};
    h.m = m;
    h.rows = m.rows;
    h.nvec = nvec;
    h.planes = planes;
    h.vscale = vscale;
    h.vbias = vbias;
    h.out = out;
    h.out_stride = out_stride;
    h.out_vec4 = out && ((uintptr_t)out % 16 == 0) && out_stride % 4 == 0 && h.rows % 16 == 0;
    for (int v = 0; v < kHeadWideVec; ++v) h.st[v] = (st && v < nvec) ? st[v] : nullptr;
    void *args[] = {&h};
    const bool few = nvec <= kHeadPackedVec;
    const int rows_per_wg = few ? plan.rows_per_wg_few : plan.rows_per_wg;
    HIP_TRY(hipLaunchKernel(few ? plan.head_few : plan.head, dim3((h.rows + rows_per_wg - 1) / rows_per_wg),
                            dim3(kThreads), args, 0, s));
    return POCR_OK;
}

int pocr::gemv_launch(hipStream_t s, GemvParams p, int nmat, int pro, int epi, int max_grid, int nv,
                      const GemvNV *q) {
    if (nv > 1 && !q) return fail(POCR_ERR_ARG, "gemv: %d vectors need their strides", nv);
    if (epi == EPI_ARGMAX && p.st) {
        if (const void *fn = plan_head(p, nmat, nv)) return launch_head(s, fn, p, pro, nv, q, true);
    }
    // every score of an LM-head-sized matrix (the sampling head's logits, a
    // one-row pocr_matvec): the same kernel with the argmax off
    if (epi == EPI_PLAIN && nv == 1 && p.out && p.rows >= kHeadWideMinRows && !p.residual) {
        if (const void *fn = plan_head(p, nmat, nv)) return launch_head(s, fn, p, pro, nv, q, false);
    }
    GemvPlan plan;
    const int nm = nmat == 2 ? 2 : (p.seg_end[0] == p.rows ? 1 : (p.seg_end[1] == p.rows ? 2 : 3));
    int rc = plan_gemv(p.m[0].qtype, nmat, p.rows, p.cols, p.m, nm, max_grid, &plan, 0, p.seg_end, epi, nv);
    if (rc) return rc;
    if ((pro == PRO_OPART || epi == EPI_DOWNV) && (plan.fn == reinterpret_cast<const void *>(&k_gemv_any<1>) ||
                                                   plan.fn == reinterpret_cast<const void *>(&k_gemv_any<2>)))
        return fail(POCR_ERR_UNSUPPORTED, "gemv: the partial-sum prologue needs the streaming kernel's shapes");
    if (pro == PRO_OPART) {
        if (nv != 1 || p.cols > 4 * kThreads || p.cols % 8 != 0 || p.flag < 1 || p.flag > kMaxOparts)
            return fail(POCR_ERR_UNSUPPORTED, "gemv: partial-sum prologue for %d columns, %d rows", p.cols, p.flag);
        plan.lds += (size_t)p.cols * 4;  // the staged activation after the digit records
    }
    if (nv > 1 && !q) return fail(POCR_ERR_ARG, "gemv: %d vectors need their strides", nv);
    return launch_gemv(s, plan, p, pro, epi, nv > 1 ? *q : GemvNV{});
}

// VNNI mode: rows on 16-byte (Q4) or 4-byte (Q6) boundaries in whole chunks
// take the chunked row loop, anything else the code-at-a-time one.
static bool vnni_fast_shape(const DevMat &m) {
    if (m.qtype == POCR_Q4)
        return m.cols % 32 == 0 && m.row_bytes == m.cols / 2 && ((uintptr_t)m.data) % 16 == 0;
    return m.cols % 16 == 0 && m.row_bytes == m.cols / 16 * 12 && ((uintptr_t)m.data) % 4 == 0;
}

template <int QT>
static const void *vnni_fn(int nmat, bool fast) {
    if (nmat == 2)
        return fast ? reinterpret_cast<const void *>(&k_gemv_vnni<QT, 2, true>)
                    : reinterpret_cast<const void *>(&k_gemv_vnni<QT, 2, false>);
    return fast ? reinterpret_cast<const void *>(&k_gemv_vnni<QT, 1, true>)
                : reinterpret_cast<const void *>(&k_gemv_vnni<QT, 1, false>);
}

int pocr::gemv_launch_vnni(hipStream_t s, const GemvParams &p, int nmat, int pro, int epi, int max_grid) {
    const int qt = p.m[0].qtype;
    // Q8 and inputs under 32 columns stay in plain mode (quant.go:2087-2115)
    if (qt == POCR_Q8 || p.cols < 32) return gemv_launch(s, p, nmat, pro, epi, max_grid);
    if (pro == PRO_OPART || epi == EPI_DOWNV)
        return fail(POCR_ERR_UNSUPPORTED, "gemv (VNNI mode): the partial-sum prologue is plain-mode only");
    if (p.cols > kVnniMaxCols) return fail(POCR_ERR_UNSUPPORTED, "gemv (VNNI mode): cols %d > %d", p.cols, kVnniMaxCols);
    const int nm = nmat == 2 ? 2 : (p.seg_end[0] == p.rows ? 1 : (p.seg_end[1] == p.rows ? 2 : 3));
    bool fast = true;
    for (int i = 0; i < nm; ++i) {
        if (p.m[i].qtype != qt || p.m[i].cols != p.cols)
            return fail(POCR_ERR_ARG, "gemv (VNNI mode): matrices of one launch differ in type or columns");
        fast = fast && vnni_fast_shape(p.m[i]);
    }
    const void *fn = qt == POCR_Q4 ? vnni_fn<QT_Q4>(nmat, fast) : vnni_fn<QT_Q6>(nmat, fast);
    const int grid = std::max(1, std::min({(p.rows + 2 * kWaves - 1) / (2 * kWaves), kVnniMaxGrid, max_grid}));
    const size_t lds = (size_t)p.cols * 4 + (((size_t)p.cols + 15) & ~(size_t)15);
    GemvParams a = p;
    void *args[] = {&a, &pro, &epi};
    HIP_TRY(hipLaunchKernel(fn, dim3(grid), dim3(kThreads), args, lds, s));
    return POCR_OK;
}


// ---------------------------------------------------------------------------
// op level
// ---------------------------------------------------------------------------
#define CTX_GUARD(ctx)                                    \
    std::lock_guard<std::mutex> lk_((ctx)->mu);           \
    HIP_TRY(hipSetDevice((ctx)->device))

static int h2d(hipStream_t s, void *dst, const void *src, size_t n) {
    HIP_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, s));
    return POCR_OK;
}
static int d2h(hipStream_t s, void *dst, const void *src, size_t n) {
    HIP_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, s));
    return POCR_OK;
}
static int sync(hipStream_t s) {
    HIP_TRY(hipStreamSynchronize(s));
    return POCR_OK;
}
// M rows of activations (device, row-major) against one weight: M ≤ 4 share
// each weight pass in the GEMV (2 or 4 vectors per launch), larger M take the
// digit-plane MFMA GEMM; shapes the vector kernel does not take fall back too.
static int matvec_rows(pocr_ctx *ctx, const pocr_weight *w, const float *x, int m, float *out) {
    hipStream_t s = ctx->stream;
    // LM-head-sized matrices: up to 16 rows of x per weight pass on the matrix
    // cores (one power-of-two digit scale per row of x)
    // two rows: the 2-vector head (103424x1024 Q4 13.2 us against 19.3 on the
    // 16-vector kernel; at 4 rows the two tie)
    if (m == 2 && w->rows >= kHeadWideMinRows) {
        GemvParams p = gemv_params_1(w);
        p.x = x;
        p.out = out;
        GemvNV q{};
        q.x_stride = w->cols;
        q.o_stride = w->rows;
        if (const void *fn = plan_head(p, 1, m)) return launch_head(s, fn, p, PRO_COPY, m, &q, false);
    }
    if (m > 1 && w->rows >= kHeadWideMinRows && head_wide_ok(w)) {
        RC(ctx->gxd.ensure(head_wide_plane_bytes(w)));
        RC(ctx->gxs.ensure(kHeadWideVec * sizeof(float)));
        RC(ctx->gxb.ensure(3 * kHeadWideVec * sizeof(int)));
        for (int r0 = 0; r0 < m; r0 += kHeadWideVec) {
            const int nv = std::min(kHeadWideVec, m - r0);
            if (nv > 1) {
                RC(launch_head_wide(s, w, x + (size_t)r0 * w->cols, w->cols, nv, nullptr, 0.0f,
                                    out + (size_t)r0 * w->rows, w->rows, nullptr, ctx->gxd.as<int8_t>(),
                                    ctx->gxs.as<float>(), ctx->gxb.as<int>()));
                continue;
            }
            GemvParams p = gemv_params_1(w);
            p.x = x + (size_t)r0 * w->cols;
            p.out = out + (size_t)r0 * w->rows;
            RC(gemv_launch(s, p, 1, PRO_COPY, EPI_PLAIN, kBigGrid));
        }
        return POCR_OK;
    }
    if (m <= 4) {
        for (int r0 = 0; r0 < m;) {
            const int nv = m - r0 >= 4 ? 4 : (m - r0 >= 2 ? 2 : 1);
            GemvParams p = gemv_params_1(w);
            p.x = x + (size_t)r0 * w->cols;
            p.out = out + (size_t)r0 * w->rows;
            GemvNV q{};
            q.x_stride = w->cols;
            q.o_stride = w->rows;
            const int rc = gemv_launch(s, p, 1, PRO_COPY, EPI_PLAIN, kBigGrid, nv, &q);
            if (rc == POCR_ERR_UNSUPPORTED && nv > 1) return batched_gemv(ctx, dev_mat(w), x, m, out);
            RC(rc);
            r0 += nv;
        }
        return POCR_OK;
    }
    return batched_gemv(ctx, dev_mat(w), x, m, out);
}

extern "C" int pocr_matvec(pocr_ctx *ctx, const pocr_weight *w, const float *x, int m, float *out) {
    if (!ctx || !w || !x || !out || m <= 0) return fail(POCR_ERR_ARG, "pocr_matvec: bad arguments");
    if (w->ctx != ctx) return fail(POCR_ERR_ARG, "pocr_matvec: weight from another context");
    CHECK_INJECT("matvec");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    RC(ctx->x.ensure((size_t)m * w->cols * 4));
    RC(ctx->out.ensure((size_t)m * w->rows * 4));
    RC(h2d(s, ctx->x.p, x, (size_t)m * w->cols * 4));
    RC(matvec_rows(ctx, w, ctx->x.as<float>(), m, ctx->out.as<float>()));
    RC(d2h(s, out, ctx->out.p, (size_t)m * w->rows * 4));
    return sync(s);
}

// m rows of x against one weight in the VNNI activation mode (Q8: plain)
extern "C" int pocr_matvec_vnni(pocr_ctx *ctx, const pocr_weight *w, const float *x, int m, float *out) {
    if (!ctx || !w || !x || !out || m <= 0) return fail(POCR_ERR_ARG, "pocr_matvec_vnni: bad arguments");
    if (w->ctx != ctx) return fail(POCR_ERR_ARG, "pocr_matvec_vnni: weight from another context");
    CHECK_INJECT("matvec_vnni");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    RC(ctx->x.ensure((size_t)m * w->cols * 4));
    RC(ctx->out.ensure((size_t)m * w->rows * 4));
    RC(h2d(s, ctx->x.p, x, (size_t)m * w->cols * 4));
    for (int r = 0; r < m; ++r) {
        GemvParams p = gemv_params_1(w);
        p.x = ctx->x.as<float>() + (size_t)r * w->cols;
        p.out = ctx->out.as<float>() + (size_t)r * w->rows;
        RC(gemv_launch_vnni(s, p, 1, PRO_COPY, EPI_PLAIN, kBigGrid));
    }
    RC(d2h(s, out, ctx->out.p, (size_t)m * w->rows * 4));
    return sync(s);
}

// greedy argmax key of a step state: the max over the LM head's slots
unsigned long long pocr::argmax_of(const StepState &s) {
    unsigned long long k = 0;
    for (int i = 0; i < kArgSlots; ++i) k = std::max(k, s.argmax_slot[i * kSlotPitch]);
    return k;
}

static float key_value(unsigned long long key) {
    uint32_t ord = (uint32_t)(key >> 32);
    uint32_t b = (ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord;
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

extern "C" int pocr_matvec_argmax(pocr_ctx *ctx, const pocr_weight *w, const float *x, int32_t *index,
                                  float *score) {
    if (!ctx || !w || !x || !index) return fail(POCR_ERR_ARG, "pocr_matvec_argmax: bad arguments");
    CHECK_INJECT("matvec_argmax");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    RC(ctx->x.ensure((size_t)w->cols * 4));
    RC(ctx->state.ensure(sizeof(StepState)));
    RC(h2d(s, ctx->x.p, x, (size_t)w->cols * 4));
    HIP_TRY(hipMemsetAsync(ctx->state.p, 0, sizeof(StepState), s));
    GemvParams p = gemv_params_1(w);
    p.x = ctx->x.as<float>();
    p.st = ctx->state.as<StepState>();
    RC(gemv_launch(s, p, 1, PRO_COPY, EPI_ARGMAX, kBigGrid));
    StepState hst;
    RC(d2h(s, &hst, ctx->state.p, sizeof(StepState)));
    RC(sync(s));
    if (hst.err) return fail(POCR_ERR_DEVICE, "matvec_argmax: device error %d", hst.err);
    const unsigned long long key = argmax_of(hst);
    if (key == 0ull) return fail(POCR_ERR_DEVICE, "matvec_argmax: no finite score");
    *index = (int32_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
    if (score) *score = key_value(key);
    return POCR_OK;
}

// top-k of `rows` scores into ss (and, with sample, one draw into ss and
// argmax slot 0 of st)
static int enqueue_topk(hipStream_t s, const float *scores, int rows, int k, unsigned long long *part,
                        SampleState *ss, StepState *st, int sample) {
    const int nparts = (rows + kTopKSlice - 1) / kTopKSlice;
    if (k < 1 || k > kTopKMax || k > rows || nparts > kTopKMaxParts)
        return fail(POCR_ERR_UNSUPPORTED, "top-k: k=%d over %d rows (k <= 64, rows <= %d)", k, rows,
                    kTopKMaxParts * kTopKSlice);
    hipLaunchKernelGGL(k_topk_partial, dim3(nparts), dim3(kTopKThreads), 0, s, scores, rows, k, part);
    hipLaunchKernelGGL(k_topk_final, dim3(1), dim3(kTopKThreads), 0, s, part, nparts, k, ss, st, sample);
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

// ---- wide sampler: every score (top_k 0 or >= rows) or more than 64 candidates

static int pow2_at_least(int n) {
    int N = 2;
    while (N < n) N <<= 1;
    return N;
}

static size_t align16(size_t b) { return (b + 15) & ~(size_t)15; }

static int wide_tiles(int n) { return n / kCTile + 8; }

static size_t wide_bytes(int n) {
    const size_t nt = (size_t)wide_tiles(n);
    return align16((size_t)pow2_at_least(n) * 8) + align16((size_t)n * 8) + 2 * align16((size_t)n * 4) +
           align16(4 * 8) + align16(4 * 4) + align16((size_t)(n / kFullSpan + 1) * 4) + align16(nt * 8) +
           align16(nt * 4) + align16(nt * 16) + align16(nt * 16) + align16((size_t)n * 8) + align16((size_t)n * 16) +
           4 * chain_work_bytes(n) + 512;
}

// POCR_CHAIN=serial: running sums one add after another; =check: both ways,
// differences counted (op-level calls fail on any)
static int chain_mode() {
    const char *e = getenv("POCR_CHAIN");
    if (!e) return 0;
    if (!strcmp(e, "serial")) return 1;
    if (!strcmp(e, "check")) return 2;
    return 0;
}

// the buffers for n scores, carved from buf (grown as needed)
static int wide_bufs(DevBuf &buf, int n, WideBufs *b) {
    RC(buf.ensure(wide_bytes(n)));
    uint8_t *p = buf.as<uint8_t>();
    b->keys = reinterpret_cast<unsigned long long *>(p);
    p += align16((size_t)pow2_at_least(n) * 8);
    b->pre64 = reinterpret_cast<double *>(p);
    p += align16((size_t)n * 8);
    b->w = reinterpret_cast<float *>(p);
    p += align16((size_t)n * 4);
    b->pre32 = reinterpret_cast<float *>(p);
    p += align16((size_t)n * 4);
    b->totals = reinterpret_cast<double *>(p);
    p += align16(4 * 8);
    b->checks = reinterpret_cast<int *>(p);
    p += align16(4 * 4);
    b->bmax = reinterpret_cast<float *>(p);
    p += align16((size_t)(n / kFullSpan + 1) * 4);
    const size_t nt = (size_t)wide_tiles(n);
    b->tsum = reinterpret_cast<double *>(p);
    p += align16(nt * 8);
    b->tbad = reinterpret_cast<int *>(p);
    p += align16(nt * 4);
    b->tcnt = reinterpret_cast<int *>(p);
    p += align16(nt * 16);
    b->trs = reinterpret_cast<unsigned long long *>(p);
    p += align16(nt * 16);
    b->cls = reinterpret_cast<int *>(p);
    p += align16((size_t)n * 8);
    b->rr = reinterpret_cast<unsigned long long *>(p);
    p += align16((size_t)n * 16);
    b->ev = reinterpret_cast<uint8_t *>(((uintptr_t)p + 255) & ~(uintptr_t)255);
    b->ev_stride = chain_work_bytes(n);
    return POCR_OK;
}

// n weights in b.w as one sum (nseg 1, sums below pre_lim0) or as
// CumulativeSum's four blocks plus the sum from index 0 (nseg 4)
static ChainSet chain_set(const WideBufs &b, int n, int nseg, int pre_lim0) {
    ChainSet S{};
    S.w = b.w;
    S.n = n;
    S.nseg = nseg;
    S.seg_len = nseg == 1 ? n : (n + 3) / 4;
    S.seg_tiles = (S.seg_len + kCTile - 1) / kCTile;
    S.ntiles = nseg == 1 ? S.seg_tiles : 3 * S.seg_tiles + (n - 3 * S.seg_len + kCTile - 1) / kCTile;
    S.pre_lim0 = pre_lim0;
    S.pre32 = b.pre32;
    S.pre64 = b.pre64;
    S.totals = b.totals;
    S.tsum = b.tsum;
    S.tbad = b.tbad;
    S.tcnt = b.tcnt;
    S.trs = b.trs;
    S.cls = b.cls;
    S.rr = b.rr;
    S.ev = b.ev;
    S.ev_stride = b.ev_stride;
    S.check = b.checks;
    return S;
}

// the running sums of a chain set whose weights (and tile sums) are written
static int enqueue_chain(hipStream_t s, const ChainSet &S, SampleState *ss, int by_temperature, StepState *st) {
    const int mode = chain_mode();
    const dim3 grid(S.ntiles, S.nseg > 1 ? 2 : 1);
    const SampleState *cs = ss;
    const StepState *cst = st;
    hipLaunchKernelGGL(k_chain_cls, grid, dim3(kCThreads), 0, s, S, cs, by_temperature, mode, cst);
    hipLaunchKernelGGL(k_chain_compact, grid, dim3(kCThreads), 0, s, S, mode, cst);
    hipLaunchKernelGGL(k_chain_walk, dim3(S.nseg), dim3(kCThreads), 0, s, S, cs, by_temperature, mode, cst);
    hipLaunchKernelGGL(k_chain_fin, grid, dim3(kCThreads), 0, s, S, cs, by_temperature, mode, cst);
    if (mode == 2) hipLaunchKernelGGL(k_chain_check, dim3(S.nseg), dim3(kCThreads), 0, s, S, cs, by_temperature, cst);
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

// every (score, row) key of scores[0..n) sorted descending into b.keys
static int enqueue_sort(hipStream_t s, const float *scores, int n, const WideBufs &b, StepState *st) {
    const int N = pow2_at_least(n);
    const int tiles = N > kSortTile ? N / kSortTile : 1;
    hipLaunchKernelGGL(k_sort_tile, dim3(tiles), dim3(kWideThreads), 0, s, scores, n, b.keys, N, st);
    for (int size = 2 * kSortTile; size <= N; size <<= 1) {
        for (int j = size / 2; j >= kSortTile; j >>= 1)
            hipLaunchKernelGGL(k_sort_stage, dim3(N / 2 / kWideThreads), dim3(kWideThreads), 0, s, b.keys, N, size,
                               j, st);
        hipLaunchKernelGGL(k_sort_merge, dim3(tiles), dim3(kWideThreads), 0, s, b.keys, N, size, st);
    }
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

// sampleFullLogitsScratch over scores[0..n): one draw into ss and argmax
// slot 0 of st
static int enqueue_sample_full(hipStream_t s, const float *x, int n, const WideBufs &b, SampleState *ss,
                               StepState *st) {
    if (n > 2) {
        const int nb = (n + kFullSpan - 1) / kFullSpan;
        hipLaunchKernelGGL(k_full_max, dim3(nb), dim3(kFullThreads), 0, s, x, n, b.bmax, (const StepState *)st);
        // the sum from index 0 (its first block is CumulativeSum's block 0)
        // and, from 4096 entries on, the blocks 1..3 from zero
        const ChainSet S = n < 4096 ? chain_set(b, n, 1, n) : chain_set(b, n, 4, (n + 3) / 4);
        hipLaunchKernelGGL(k_full_weights, dim3(S.ntiles), dim3(kCThreads), 0, s, x, (const float *)b.bmax, nb,
                           (const SampleState *)ss, S, (const StepState *)st);
        RC(enqueue_chain(s, S, ss, 0, st));
    }
    hipLaunchKernelGGL(k_full_pick, dim3(1), dim3(64), 0, s, x, n, b.pre32, b.totals, ss, st);
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

// the k (> 4) best of scores[0..n) sorted into b.keys, then, with sample,
// sampleCandidateScoresScratch's draw among them into ss and st
static int enqueue_sample_sorted(hipStream_t s, const float *x, int n, int k, const WideBufs &b, SampleState *ss,
                                 StepState *st, int sample) {
    RC(enqueue_sort(s, x, n, b, st));
    if (!sample) return POCR_OK;
    const ChainSet S = chain_set(b, k, 1, k);
    hipLaunchKernelGGL(k_cand_weights, dim3(S.ntiles), dim3(kCThreads), 0, s, (const unsigned long long *)b.keys,
                       (const SampleState *)ss, S, (const StepState *)st);
    RC(enqueue_chain(s, S, ss, 1, st));
    hipLaunchKernelGGL(k_cand_pick, dim3(1), dim3(kWideThreads), 0, s, (const unsigned long long *)b.keys, k,
                       (const float *)b.pre32, (const double *)b.pre64, (const double *)b.totals, ss, st);
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

// synchronize; in check mode, fail when the parallel running sums differed
// from the one-by-one sums anywhere
static int chain_checked(hipStream_t s, const WideBufs &b) {
    int chk[4] = {0, 0, 0, 0};
    if (chain_mode() == 2) RC(d2h(s, chk, b.checks, sizeof(chk)));
    RC(sync(s));
    const int d = chk[0] + chk[1] + chk[2] + chk[3];
    if (d) return fail(POCR_ERR_DEVICE, "running sums: %d differ from the one-by-one sums", d);
    return POCR_OK;
}

// ids and scores of the first k sorted keys (host)
static void keys_to_host(const std::vector<unsigned long long> &keys, int k, int32_t *ids, float *scores) {
    for (int i = 0; i < k; ++i) {
        const unsigned long long key = keys[i];
        if (ids) ids[i] = (int32_t)(0xFFFFFFFFu - (uint32_t)key);
        if (scores) {
            uint32_t o = (uint32_t)(key >> 32);
            o = (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
            std::memcpy(&scores[i], &o, 4);
        }
    }
}

// top-k of `rows` device scores in ctx->out through ctx's sampler state;
// returns the state read back
static int ctx_topk(pocr_ctx *ctx, int rows, int k, int sample, const SampleState &in, SampleState *out) {
    hipStream_t s = ctx->stream;
    RC(ctx->topk_part.ensure((size_t)kTopKMaxParts * kTopKMax * 8));
    RC(ctx->samp.ensure(sizeof(SampleState)));
    RC(h2d(s, ctx->samp.p, &in, sizeof(SampleState)));
    RC(enqueue_topk(s, ctx->out.as<float>(), rows, k, ctx->topk_part.as<unsigned long long>(),
                    ctx->samp.as<SampleState>(), nullptr, sample));
    RC(d2h(s, out, ctx->samp.p, sizeof(SampleState)));
    return sync(s);
}

extern "C" int pocr_matvec_topk(pocr_ctx *ctx, const pocr_weight *w, const float *x, int k, int32_t *ids,
                                float *scores) {
    if (!ctx || !w || !x || !ids || k < 1) return fail(POCR_ERR_ARG, "pocr_matvec_topk: bad arguments");
    if (k > w->rows) return fail(POCR_ERR_ARG, "pocr_matvec_topk: k %d > rows %d", k, w->rows);
    CHECK_INJECT("matvec_topk");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    RC(ctx->x.ensure((size_t)w->cols * 4));
    RC(ctx->out.ensure((size_t)w->rows * 4));
    RC(h2d(s, ctx->x.p, x, (size_t)w->cols * 4));
    GemvParams p = gemv_params_1(w);
    p.x = ctx->x.as<float>();
    p.out = ctx->out.as<float>();
    RC(gemv_launch(s, p, 1, PRO_COPY, EPI_PLAIN, kBigGrid));
    if (k > kTopKMax) {
        WideBufs b;
        RC(wide_bufs(ctx->wide, w->rows, &b));
        RC(enqueue_sample_sorted(s, ctx->out.as<float>(), w->rows, k, b, nullptr, nullptr, 0));
        std::vector<unsigned long long> keys((size_t)k);
        RC(d2h(s, keys.data(), b.keys, (size_t)k * 8));
        RC(sync(s));
        keys_to_host(keys, k, ids, scores);
        return k;
    }
    SampleState in{}, out;
    RC(ctx_topk(ctx, w->rows, k, 0, in, &out));
    for (int i = 0; i < out.n; ++i) {
        ids[i] = out.ids[i];
        if (scores) scores[i] = out.scores[i];
    }
    return out.n;
}

extern "C" int pocr_sample_topk(pocr_ctx *ctx, const float *logits, int n, int k, double temperature,
                                uint64_t *rng_state, int32_t *token, int32_t *ids, float *scores) {
    if (!ctx || !logits || !rng_state || !token || n <= 0) return fail(POCR_ERR_ARG, "pocr_sample_topk: bad arguments");
    if (!(temperature > 0.0) || std::isinf(temperature) || k < 2 || k >= n)
        return fail(POCR_ERR_ARG, "pocr_sample_topk: needs temperature > 0 and 1 < k < n");
    CHECK_INJECT("sample_topk");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    RC(ctx->out.ensure((size_t)n * 4));
    RC(h2d(s, ctx->out.p, logits, (size_t)n * 4));
    SampleState in{}, out;
    in.rng = *rng_state;
    in.temperature = temperature;
    in.top_k = k;
    if (k > kTopKMax) {
        WideBufs b;
        RC(wide_bufs(ctx->wide, n, &b));
        RC(ctx->samp.ensure(sizeof(SampleState)));
        RC(h2d(s, ctx->samp.p, &in, sizeof(SampleState)));
        HIP_TRY(hipMemsetAsync(b.checks, 0, 4 * 4, s));
        RC(enqueue_sample_sorted(s, ctx->out.as<float>(), n, k, b, ctx->samp.as<SampleState>(), nullptr, 1));
        std::vector<unsigned long long> keys((size_t)k);
        RC(d2h(s, keys.data(), b.keys, (size_t)k * 8));
        RC(d2h(s, &out, ctx->samp.p, sizeof(SampleState)));
        RC(chain_checked(s, b));
        keys_to_host(keys, k, ids, scores);
        *rng_state = out.rng;
        *token = out.token;
        return POCR_OK;
    }
    RC(ctx_topk(ctx, n, k, 1, in, &out));
    *rng_state = out.rng;
    *token = out.token;
    for (int i = 0; i < out.n; ++i) {
        if (ids) ids[i] = out.ids[i];
        if (scores) scores[i] = out.scores[i];
    }
    return POCR_OK;
}

extern "C" int pocr_sample_full(pocr_ctx *ctx, const float *logits, int n, double temperature, uint64_t *rng_state,
                                int32_t *token) {
    if (!ctx || !logits || !rng_state || !token || n <= 0) return fail(POCR_ERR_ARG, "pocr_sample_full: bad arguments");
    if (!(temperature > 0.0) || std::isinf(temperature))
        return fail(POCR_ERR_ARG, "pocr_sample_full: needs a finite temperature > 0");
    CHECK_INJECT("sample_full");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    RC(ctx->out.ensure((size_t)n * 4));
    RC(h2d(s, ctx->out.p, logits, (size_t)n * 4));
    SampleState in{}, out;
    in.rng = *rng_state;
    in.temperature = temperature;
    WideBufs b;
    RC(wide_bufs(ctx->wide, n, &b));
    RC(ctx->samp.ensure(sizeof(SampleState)));
    RC(h2d(s, ctx->samp.p, &in, sizeof(SampleState)));
    HIP_TRY(hipMemsetAsync(b.checks, 0, 4 * 4, s));
    RC(enqueue_sample_full(s, ctx->out.as<float>(), n, b, ctx->samp.as<SampleState>(), nullptr));
    RC(d2h(s, &out, ctx->samp.p, sizeof(SampleState)));
    RC(chain_checked(s, b));
    *rng_state = out.rng;
    *token = out.token;
    return POCR_OK;
}

static int fused3(pocr_ctx *ctx, const pocr_weight *a, const pocr_weight *b, const pocr_weight *c,
                  const float *x) {
    hipStream_t s = ctx->stream;
    const int rows = a->rows + b->rows + c->rows;
    RC(ctx->x.ensure((size_t)a->cols * 4));
    RC(ctx->out.ensure((size_t)rows * 4));
    RC(h2d(s, ctx->x.p, x, (size_t)a->cols * 4));
    GemvParams p{};
    p.m[0] = dev_mat(a);
    p.m[1] = dev_mat(b);
    p.m[2] = dev_mat(c);
    p.seg_end[0] = a->rows;
    p.seg_end[1] = a->rows + b->rows;
    p.seg_end[2] = rows;
    p.rows = rows;
    p.cols = a->cols;
    p.x = ctx->x.as<float>();
    p.out = ctx->out.as<float>();
    return gemv_launch(s, p, 1, PRO_COPY, EPI_PLAIN, kBigGrid);
}

static int check3(const pocr_weight *a, const pocr_weight *b, const pocr_weight *c) {
    if (!a || !b || !c) return fail(POCR_ERR_ARG, "fused_matvec3: null weight");
    if (a->qtype != b->qtype || b->qtype != c->qtype || a->cols != b->cols || b->cols != c->cols)
        return fail(POCR_ERR_ARG, "fused_matvec3: weights differ in type or columns");
    if (a->ctx != b->ctx || b->ctx != c->ctx) return fail(POCR_ERR_ARG, "fused_matvec3: mixed contexts");
    return POCR_OK;
}

extern "C" int pocr_fused_matvec3(pocr_ctx *ctx, const pocr_weight *a, const pocr_weight *b, const pocr_weight *c,
                                  const float *x, float *out_a, float *out_b, float *out_c) {
    if (!ctx || !x || !out_a || !out_b || !out_c) return fail(POCR_ERR_ARG, "pocr_fused_matvec3: null argument");
    RC(check3(a, b, c));
    CHECK_INJECT("fused_matvec3");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    RC(fused3(ctx, a, b, c, x));
    float *o = ctx->out.as<float>();
    RC(d2h(s, out_a, o, (size_t)a->rows * 4));
    RC(d2h(s, out_b, o + a->rows, (size_t)b->rows * 4));
    RC(d2h(s, out_c, o + a->rows + b->rows, (size_t)c->rows * 4));
    return sync(s);
}

extern "C" int pocr_fused_matvec3_mrope(pocr_ctx *ctx, const pocr_weight *a, const pocr_weight *b,
                                        const pocr_weight *c, const float *x, const float *cos_t,
                                        const float *sin_t, int q_heads, int kv_heads, int head_dim,
                                        float *out_a, float *out_b, float *out_c) {
    if (!ctx || !x || !cos_t || !sin_t || !out_a || !out_b || !out_c)
        return fail(POCR_ERR_ARG, "pocr_fused_matvec3_mrope: null argument");
    RC(check3(a, b, c));
    if (head_dim <= 0 || head_dim % 2 || q_heads * head_dim != a->rows || kv_heads * head_dim != b->rows)
        return fail(POCR_ERR_ARG, "pocr_fused_matvec3_mrope: heads/head_dim do not match rows");
    CHECK_INJECT("fused_matvec3_mrope");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    RC(fused3(ctx, a, b, c, x));
    const int half = head_dim / 2;
    RC(ctx->tabs.ensure((size_t)half * 8));
    RC(h2d(s, ctx->tabs.p, cos_t, (size_t)half * 4));
    RC(h2d(s, ctx->tabs.as<float>() + half, sin_t, (size_t)half * 4));
    float *o = ctx->out.as<float>();
    const int total = (q_heads + kv_heads) * half;
    hipLaunchKernelGGL(k_rope, dim3((total + kThreads - 1) / kThreads), dim3(kThreads), 0, s, o, o + a->rows,
                       ctx->tabs.as<float>(), ctx->tabs.as<float>() + half, q_heads, kv_heads, head_dim);
    HIP_TRY(hipGetLastError());
    RC(d2h(s, out_a, o, (size_t)a->rows * 4));
    RC(d2h(s, out_b, o + a->rows, (size_t)b->rows * 4));
    RC(d2h(s, out_c, o + a->rows + b->rows, (size_t)c->rows * 4));
    return sync(s);
}

extern "C" int pocr_swiglu_gate_up(pocr_ctx *ctx, const pocr_weight *gate, const pocr_weight *up, const float *x,
                                   float *out) {
    if (!ctx || !gate || !up || !x || !out) return fail(POCR_ERR_ARG, "pocr_swiglu_gate_up: null argument");
    if (gate->rows != up->rows || gate->cols != up->cols || gate->qtype != up->qtype)
        return fail(POCR_ERR_ARG, "pocr_swiglu_gate_up: gate/up shapes differ");
    CHECK_INJECT("swiglu_gate_up");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    RC(ctx->x.ensure((size_t)gate->cols * 4));
    RC(ctx->out.ensure((size_t)gate->rows * 4));
    RC(h2d(s, ctx->x.p, x, (size_t)gate->cols * 4));
    GemvParams p = gemv_params_1(gate);
    p.m[1] = dev_mat(up);
    p.x = ctx->x.as<float>();
    p.out = ctx->out.as<float>();
    RC(gemv_launch(s, p, 2, PRO_COPY, EPI_SWIGLU, kBigGrid));
    RC(d2h(s, out, ctx->out.p, (size_t)gate->rows * 4));
    return sync(s);
}

// v = residual + W·x_dev (x already on the device), norm_out = RMSNorm(v)·norm_w,
// residual = v iff in_place; host residual/norm_w/norm_out, synchronous
static int matvec_add_rmsnorm_dev(pocr_ctx *ctx, const pocr_weight *w, const float *x_dev, float *residual,
                                  const float *norm_w, float eps, int in_place, float *norm_out) {
    hipStream_t s = ctx->stream;
    const int n = w->rows;
    RC(ctx->res.ensure((size_t)n * 4 * 2));
    RC(ctx->vbuf.ensure((size_t)n * 4));
    RC(ctx->out3.ensure((size_t)n * 4));
    RC(h2d(s, ctx->res.p, residual, (size_t)n * 4));
    RC(h2d(s, ctx->res.as<float>() + n, norm_w, (size_t)n * 4));
    GemvParams p = gemv_params_1(w);
    p.x = x_dev;
    p.residual = ctx->res.as<float>();
    p.vbuf = ctx->vbuf.as<float>();
    RC(gemv_launch(s, p, 1, PRO_COPY, EPI_ADDV, kBigGrid));
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(kThreads), 0, s, ctx->vbuf.as<float>(), ctx->res.as<float>() + n, n,
                       eps, ctx->out3.as<float>());
    HIP_TRY(hipGetLastError());
    RC(d2h(s, norm_out, ctx->out3.p, (size_t)n * 4));
    if (in_place) RC(d2h(s, residual, ctx->vbuf.p, (size_t)n * 4));
    return sync(s);
}

extern "C" int pocr_matvec_add_rmsnorm(pocr_ctx *ctx, const pocr_weight *w, const float *x, float *residual,
                                       const float *norm_w, float eps, int in_place, float *norm_out) {
    if (!ctx || !w || !x || !residual || !norm_w || !norm_out)
        return fail(POCR_ERR_ARG, "pocr_matvec_add_rmsnorm: null argument");
    CHECK_INJECT("matvec_add_rmsnorm");
    CTX_GUARD(ctx);
    RC(ctx->x.ensure((size_t)w->cols * 4));
    RC(h2d(ctx->stream, ctx->x.p, x, (size_t)w->cols * 4));
    return matvec_add_rmsnorm_dev(ctx, w, ctx->x.as<float>(), residual, norm_w, eps, in_place, norm_out);
}

// SiLU(G·x)·(U·x) of host x into ctx->out (device), for the SwiGLU-down ops
static int swiglu_dev(pocr_ctx *ctx, const pocr_weight *gate, const pocr_weight *up, const float *x) {
    hipStream_t s = ctx->stream;
    RC(ctx->x.ensure((size_t)gate->cols * 4));
    RC(ctx->out.ensure((size_t)gate->rows * 4));
    RC(h2d(s, ctx->x.p, x, (size_t)gate->cols * 4));
    GemvParams p = gemv_params_1(gate);
    p.m[1] = dev_mat(up);
    p.x = ctx->x.as<float>();
    p.out = ctx->out.as<float>();
    return gemv_launch(s, p, 2, PRO_COPY, EPI_SWIGLU, kBigGrid);
}

static int swiglu_down_args(const pocr_weight *gate, const pocr_weight *up, const pocr_weight *down, const char *op) {
    if (gate->rows != up->rows || gate->cols != up->cols || gate->qtype != up->qtype)
        return fail(POCR_ERR_ARG, "%s: gate/up shapes differ", op);
    if (down->cols != gate->rows) return fail(POCR_ERR_ARG, "%s: down takes %d columns, gate gives %d", op, down->cols,
                                              gate->rows);
    return POCR_OK;
}

extern "C" int pocr_swiglu_down(pocr_ctx *ctx, const pocr_weight *gate, const pocr_weight *up, const pocr_weight *down,
                                const float *x, float *out) {
    if (!ctx || !gate || !up || !down || !x || !out) return fail(POCR_ERR_ARG, "pocr_swiglu_down: null argument");
    RC(swiglu_down_args(gate, up, down, "pocr_swiglu_down"));
    CHECK_INJECT("swiglu_down");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    RC(swiglu_dev(ctx, gate, up, x));
    RC(ctx->out2.ensure((size_t)down->rows * 4));
    GemvParams p = gemv_params_1(down);
    p.x = ctx->out.as<float>();
    p.out = ctx->out2.as<float>();
    RC(gemv_launch(s, p, 1, PRO_COPY, EPI_PLAIN, kBigGrid));
    RC(d2h(s, out, ctx->out2.p, (size_t)down->rows * 4));
    return sync(s);
}

extern "C" int pocr_swiglu_down_add_rmsnorm(pocr_ctx *ctx, const pocr_weight *gate, const pocr_weight *up,
                                            const pocr_weight *down, const float *x, float *residual,
                                            const float *norm_w, float eps, int in_place, float *norm_out) {
    if (!ctx || !gate || !up || !down || !x || !residual || !norm_w || !norm_out)
        return fail(POCR_ERR_ARG, "pocr_swiglu_down_add_rmsnorm: null argument");
    RC(swiglu_down_args(gate, up, down, "pocr_swiglu_down_add_rmsnorm"));
    CHECK_INJECT("swiglu_down_add_rmsnorm");
    CTX_GUARD(ctx);
    RC(swiglu_dev(ctx, gate, up, x));
    return matvec_add_rmsnorm_dev(ctx, down, ctx->out.as<float>(), residual, norm_w, eps, in_place, norm_out);
}

extern "C" int pocr_add_rmsnorm(pocr_ctx *ctx, float *dst, const float *add, const float *w, int n, float eps,
                                int in_place, float *out) {
    if (!ctx || !dst || !add || !w || !out || n <= 0) return fail(POCR_ERR_ARG, "pocr_add_rmsnorm: bad arguments");
    CHECK_INJECT("add_rmsnorm");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    RC(ctx->x.ensure((size_t)n * 12));
    RC(ctx->vbuf.ensure((size_t)n * 4));
    RC(ctx->out.ensure((size_t)n * 4));
    float *xd = ctx->x.as<float>();
    RC(h2d(s, xd, dst, (size_t)n * 4));
    RC(h2d(s, xd + n, add, (size_t)n * 4));
    RC(h2d(s, xd + 2 * n, w, (size_t)n * 4));
    hipLaunchKernelGGL(k_add_rmsnorm, dim3(1), dim3(kThreads), 0, s, xd, xd + n, xd + 2 * n, n, eps,
                       ctx->vbuf.as<float>(), ctx->out.as<float>());
    HIP_TRY(hipGetLastError());
    RC(d2h(s, out, ctx->out.p, (size_t)n * 4));
    if (in_place) RC(d2h(s, dst, ctx->vbuf.p, (size_t)n * 4));
    return sync(s);
}

extern "C" int pocr_mrope(pocr_ctx *ctx, float *x, const float *cos_t, const float *sin_t, int heads, int head_dim) {
    if (!ctx || !x || !cos_t || !sin_t || head_dim <= 0 || head_dim % 2 || heads <= 0)
        return fail(POCR_ERR_ARG, "pocr_mrope: bad arguments");
    CHECK_INJECT("mrope");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    const int half = head_dim / 2;
    const size_t nx = (size_t)heads * head_dim;
    RC(ctx->x.ensure(nx * 4));
    RC(ctx->tabs.ensure((size_t)half * 8));
    RC(h2d(s, ctx->x.p, x, nx * 4));
    RC(h2d(s, ctx->tabs.p, cos_t, (size_t)half * 4));
    RC(h2d(s, ctx->tabs.as<float>() + half, sin_t, (size_t)half * 4));
    const int total = heads * half;
    hipLaunchKernelGGL(k_rope, dim3((total + kThreads - 1) / kThreads), dim3(kThreads), 0, s, ctx->x.as<float>(),
                       ctx->x.as<float>(), ctx->tabs.as<float>(), ctx->tabs.as<float>() + half, heads, 0, head_dim);
    HIP_TRY(hipGetLastError());
    RC(d2h(s, x, ctx->x.p, nx * 4));
    return sync(s);
}

extern "C" int pocr_rmsnorm(pocr_ctx *ctx, const float *x, const float *w, int n, float eps, float *out) {
    if (!ctx || !x || !w || !out || n <= 0) return fail(POCR_ERR_ARG, "pocr_rmsnorm: bad arguments");
    CHECK_INJECT("rmsnorm");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    RC(ctx->x.ensure((size_t)n * 8));
    RC(ctx->out.ensure((size_t)n * 4));
    RC(h2d(s, ctx->x.p, x, (size_t)n * 4));
    RC(h2d(s, ctx->x.as<float>() + n, w, (size_t)n * 4));
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(kThreads), 0, s, ctx->x.as<float>(), ctx->x.as<float>() + n, n, eps,
                       ctx->out.as<float>());
    HIP_TRY(hipGetLastError());
    RC(d2h(s, out, ctx->out.p, (size_t)n * 4));
    return sync(s);
}

extern "C" int pocr_mrope_pair(pocr_ctx *ctx, float *q, float *k, const float *cos_t, const float *sin_t,
                               int q_heads, int kv_heads, int head_dim) {
    if (!ctx || !q || !k || !cos_t || !sin_t || head_dim <= 0 || head_dim % 2 || q_heads <= 0 || kv_heads <= 0)
        return fail(POCR_ERR_ARG, "pocr_mrope_pair: bad arguments");
    CHECK_INJECT("mrope_pair");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    const int half = head_dim / 2;
    const size_t nq = (size_t)q_heads * head_dim, nk = (size_t)kv_heads * head_dim;
    RC(ctx->x.ensure((nq + nk) * 4));
    RC(ctx->tabs.ensure((size_t)half * 8));
    RC(h2d(s, ctx->x.p, q, nq * 4));
    RC(h2d(s, ctx->x.as<float>() + nq, k, nk * 4));
    RC(h2d(s, ctx->tabs.p, cos_t, (size_t)half * 4));
    RC(h2d(s, ctx->tabs.as<float>() + half, sin_t, (size_t)half * 4));
    const int total = (q_heads + kv_heads) * half;
    hipLaunchKernelGGL(k_rope, dim3((total + kThreads - 1) / kThreads), dim3(kThreads), 0, s, ctx->x.as<float>(),
                       ctx->x.as<float>() + nq, ctx->tabs.as<float>(), ctx->tabs.as<float>() + half, q_heads,
                       kv_heads, head_dim);
    HIP_TRY(hipGetLastError());
    RC(d2h(s, q, ctx->x.p, nq * 4));
    RC(d2h(s, k, ctx->x.as<float>() + nq, nk * 4));
    return sync(s);
}

// Rows per wave of the decode attention for a cache capacity: short caches
// take 32-row splits (more workgroups in flight), longer ones 64-row splits
// (half the records to merge); the split count stays ≤ kMaxSplits.  On
// MI355X (18 layers, 16 q / 2 kv heads; attention + merge back to back) 8
// rows per wave lead up to ~2k rows of capacity; at 4096 rows 16 per wave
// are ahead (8.7 against 9.3 µs) and at 8192 they tie the attention while
// halving the records to merge.
static int attn_rpw(int cap) { return cap <= 2048 ? 8 : 16; }
// one split per 4·rpw rows of capacity
static int attn_nsplit(int cap, int rpw) { return std::max(1, (cap + 4 * rpw - 1) / (4 * rpw)); }

// the launch shape of one decode attention: rows per wave, splits, rows per split
static void attn_shape(AttnParams &a, int cap, int rpw) {
    a.rows_cap = cap;
    a.nsplit = attn_nsplit(cap, rpw);
    a.chunk = attn_chunk(cap, a.nsplit, 4 * rpw);
}

// the split merge with its records requested in one round trip for up to
// 64 (or, above 64 splits, 128) splits
static void launch_attn_merge(hipStream_t s, dim3 grid, const AttnParams &a) {
    if (merge_prefetch(a.nsplit) == 16) hipLaunchKernelGGL(k_attn_merge<16>, grid, dim3(kMergeThreads), 0, s, a);
    else hipLaunchKernelGGL(k_attn_merge<8>, grid, dim3(kMergeThreads), 0, s, a);
}
static void launch_attn_merge_multi(hipStream_t s, dim3 grid, int max_split, const AttnMulti &am) {
    if (merge_prefetch(max_split) == 16) hipLaunchKernelGGL(k_attn_merge_multi<16>, grid, dim3(kMergeThreads), 0, s, am);
    else hipLaunchKernelGGL(k_attn_merge_multi<8>, grid, dim3(kMergeThreads), 0, s, am);
}

static void launch_attn_decode(hipStream_t s, int rpw, dim3 grid, const AttnParams &a) {
    if (rpw == 8) hipLaunchKernelGGL(k_attn_decode<8>, grid, dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL(k_attn_decode<16>, grid, dim3(kThreads), 0, s, a);
}

// GQA attention of host q over host caches into ctx->out (device, heads·dim)
static int text_attention_dev(pocr_ctx *ctx, const float *q, const float *k_cache, const float *v_cache, int cache_len,
                              int heads, int kv_heads, int head_dim) {
    hipStream_t s = ctx->stream;
    const size_t kvd = (size_t)kv_heads * head_dim;
    const size_t nq = (size_t)heads * head_dim;
    RC(ctx->x.ensure(nq * 4));
    RC(ctx->kc.ensure(kvd * cache_len * 4));
    RC(ctx->vc.ensure(kvd * cache_len * 4));
    RC(ctx->out.ensure(nq * 4));
    RC(h2d(s, ctx->x.p, q, nq * 4));
    RC(h2d(s, ctx->kc.p, k_cache, kvd * cache_len * 4));
    RC(h2d(s, ctx->vc.p, v_cache, kvd * cache_len * 4));
    const float scale = (float)(1.0 / std::sqrt((double)head_dim));  // invSqrt, model.go:7391
    const int group = heads / kv_heads;
    if (head_dim == kHD && group <= kMaxGroup) {
        const int rpw = attn_rpw(cache_len);
        const int nsplit = attn_nsplit(cache_len, rpw);
        if (nsplit > kMaxSplits) return fail(POCR_ERR_UNSUPPORTED, "text_attention: cache above %d rows", kMaxSplits * kMaxChunk);
        RC(ctx->part.ensure((size_t)kv_heads * nsplit * kMaxGroup * kRec * 4));
        AttnParams p{};
        p.q = ctx->x.as<float>();
        p.kc = ctx->kc.as<float>();
        p.vc = ctx->vc.as<float>();
        p.st = nullptr;
        p.len = cache_len;
        p.has_rope = 0;
        p.part = ctx->part.as<float>();
        p.head_out = ctx->out.as<float>();
        p.heads = heads;
        p.kvh = kv_heads;
        attn_shape(p, cache_len, rpw);
        p.scale = scale;
        launch_attn_decode(s, rpw, dim3(kv_heads, nsplit), p);
        launch_attn_merge(s, dim3(heads), p);
    } else {
        if ((size_t)cache_len * 4 > 60 * 1024) return fail(POCR_ERR_UNSUPPORTED, "text_attention: cache too long");
        hipLaunchKernelGGL(k_attn_small, dim3(heads), dim3(kThreads), (size_t)cache_len * 4, s, ctx->x.as<float>(),
                           ctx->kc.as<float>(), ctx->vc.as<float>(), cache_len, heads, kv_heads, head_dim, scale,
                           ctx->out.as<float>());
    }
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

static bool attention_args_ok(const void *q, const void *kc, const void *vc, int cache_len, int heads, int kv_heads,
                              int head_dim) {
    return q && kc && vc && cache_len > 0 && heads > 0 && kv_heads > 0 && head_dim > 0 && heads % kv_heads == 0;
}

extern "C" int pocr_text_attention(pocr_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                                   int cache_len, int heads, int kv_heads, int head_dim, float *out) {
    if (!ctx || !out || !attention_args_ok(q, k_cache, v_cache, cache_len, heads, kv_heads, head_dim))
        return fail(POCR_ERR_ARG, "pocr_text_attention: bad arguments");
    CHECK_INJECT("text_attention");
    CTX_GUARD(ctx);
    RC(text_attention_dev(ctx, q, k_cache, v_cache, cache_len, heads, kv_heads, head_dim));
    RC(d2h(ctx->stream, out, ctx->out.p, (size_t)heads * head_dim * 4));
    return sync(ctx->stream);
}

static int attention_out_args(const pocr_weight *wo, int heads, int head_dim, const char *op) {
    if (!wo) return fail(POCR_ERR_ARG, "%s: null weight", op);
    if (wo->cols != heads * head_dim)
        return fail(POCR_ERR_ARG, "%s: o_proj takes %d columns, attention gives %d", op, wo->cols, heads * head_dim);
    return POCR_OK;
}

extern "C" int pocr_text_attention_out(pocr_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                                       int cache_len, int heads, int kv_heads, int head_dim, const pocr_weight *wo,
                                       float *out) {
    if (!ctx || !out || !attention_args_ok(q, k_cache, v_cache, cache_len, heads, kv_heads, head_dim))
        return fail(POCR_ERR_ARG, "pocr_text_attention_out: bad arguments");
    RC(attention_out_args(wo, heads, head_dim, "pocr_text_attention_out"));
    CHECK_INJECT("text_attention_out");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    RC(text_attention_dev(ctx, q, k_cache, v_cache, cache_len, heads, kv_heads, head_dim));
    RC(ctx->out2.ensure((size_t)wo->rows * 4));
    GemvParams p = gemv_params_1(wo);
    p.x = ctx->out.as<float>();
    p.out = ctx->out2.as<float>();
    RC(gemv_launch(s, p, 1, PRO_COPY, EPI_PLAIN, kBigGrid));
    RC(d2h(s, out, ctx->out2.p, (size_t)wo->rows * 4));
    return sync(s);
}

extern "C" int pocr_text_attention_out_add_rmsnorm(pocr_ctx *ctx, const float *q, const float *k_cache,
                                                   const float *v_cache, int cache_len, int heads, int kv_heads,
                                                   int head_dim, const pocr_weight *wo, float *residual,
                                                   const float *norm_w, float eps, int in_place, float *norm_out) {
    if (!ctx || !residual || !norm_w || !norm_out ||
        !attention_args_ok(q, k_cache, v_cache, cache_len, heads, kv_heads, head_dim))
        return fail(POCR_ERR_ARG, "pocr_text_attention_out_add_rmsnorm: bad arguments");
    RC(attention_out_args(wo, heads, head_dim, "pocr_text_attention_out_add_rmsnorm"));
    CHECK_INJECT("text_attention_out_add_rmsnorm");
    CTX_GUARD(ctx);
    RC(text_attention_dev(ctx, q, k_cache, v_cache, cache_len, heads, kv_heads, head_dim));
    return matvec_add_rmsnorm_dev(ctx, wo, ctx->out.as<float>(), residual, norm_w, eps, in_place, norm_out);
}

extern "C" int pocr_first_token_value_out_add_rmsnorm(pocr_ctx *ctx, const float *k_cache, const float *v_cache,
                                                      int heads, int kv_heads, int head_dim, const pocr_weight *wo,
                                                      float *residual, const float *norm_w, float eps, int in_place,
                                                      float *norm_out) {
    const std::vector<float> q((size_t)std::max(heads, 1) * std::max(head_dim, 1), 0.0f);
    if (!ctx || !residual || !norm_w || !norm_out ||
        !attention_args_ok(q.data(), k_cache, v_cache, 1, heads, kv_heads, head_dim))
        return fail(POCR_ERR_ARG, "pocr_first_token_value_out_add_rmsnorm: bad arguments");
    RC(attention_out_args(wo, heads, head_dim, "pocr_first_token_value_out_add_rmsnorm"));
    CHECK_INJECT("first_token_value_out_add_rmsnorm");
    CTX_GUARD(ctx);
    // attention over the one cached row is that row's V, exactly (each head's
    // single weight is FastExp(0)/FastExp(0) = 1): expandValueHeads
    // (model.go:4603-4621) on the device, whatever q is
    RC(text_attention_dev(ctx, q.data(), k_cache, v_cache, 1, heads, kv_heads, head_dim));
    return matvec_add_rmsnorm_dev(ctx, wo, ctx->out.as<float>(), residual, norm_w, eps, in_place, norm_out);
}

// The computation of pocr_text_attention over device buffers the caller owns,
// allocating nothing: the split records go to this device's scratch array,
// which limits kv_heads × splits to kNoAllocSplitRecs.  Calls that overlap on
// one GPU race on the array (every call rewrites the records it reads; none
// needs them zeroed).
extern "C" int pocr_text_attention_noalloc(pocr_ctx *ctx, const float *q_dev, const float *k_cache_dev,
                                           const float *v_cache_dev, int cache_len, int heads, int kv_heads,
                                           int head_dim, float *out_dev) {
    if (!ctx || !q_dev || !k_cache_dev || !v_cache_dev || !out_dev || cache_len <= 0 || heads <= 0 || kv_heads <= 0 ||
        head_dim <= 0 || heads % kv_heads)
        return fail(POCR_ERR_ARG, "pocr_text_attention_noalloc: bad arguments");
    CHECK_INJECT("text_attention_noalloc");
    CTX_GUARD(ctx);
    if (!ctx->scratch) return fail(POCR_ERR_DEVICE, "pocr_text_attention_noalloc: no scratch array");
    hipStream_t s = ctx->stream;
    const float scale = (float)(1.0 / std::sqrt((double)head_dim));  // invSqrt, model.go:7391
    const int group = heads / kv_heads;
    if (head_dim == kHD && group <= kMaxGroup) {
        const int rpw = attn_rpw(cache_len);
        const int nsplit = attn_nsplit(cache_len, rpw);
        if ((long long)kv_heads * nsplit > kNoAllocSplitRecs)
            return fail(POCR_ERR_ARG,
                        "pocr_text_attention_noalloc: %d kv heads x %d splits (%d cache rows) exceed the %d split "
                        "records of the fixed scratch array",
                        kv_heads, nsplit, cache_len, kNoAllocSplitRecs);
        AttnParams p{};
        p.q = q_dev;
        p.kc = const_cast<float *>(k_cache_dev);  // read only: no append without a step state
        p.vc = const_cast<float *>(v_cache_dev);
        p.st = nullptr;
        p.len = cache_len;
        p.has_rope = 0;
        p.part = ctx->scratch;
        p.head_out = out_dev;
        p.heads = heads;
        p.kvh = kv_heads;
        attn_shape(p, cache_len, rpw);
        p.scale = scale;
        launch_attn_decode(s, rpw, dim3(kv_heads, nsplit), p);
        launch_attn_merge(s, dim3(heads), p);
    } else {
        if ((size_t)cache_len * 4 > 60 * 1024)
            return fail(POCR_ERR_UNSUPPORTED, "pocr_text_attention_noalloc: cache too long for this head shape");
        hipLaunchKernelGGL(k_attn_small, dim3(heads), dim3(kThreads), (size_t)cache_len * 4, s, q_dev, k_cache_dev,
                           v_cache_dev, cache_len, heads, kv_heads, head_dim, scale, out_dev);
    }
    HIP_TRY(hipGetLastError());
    return sync(s);
}

// ---------------------------------------------------------------------------
// model
// ---------------------------------------------------------------------------
extern "C" int pocr_model_create(pocr_ctx *ctx, const pocr_config *cfg, pocr_model **out) {
    if (!ctx || !cfg || !out) return fail(POCR_ERR_ARG, "pocr_model_create: null argument");
    *out = nullptr;
    const pocr_config &c = *cfg;
    if (c.hidden <= 0 || c.intermediate <= 0 || c.layers <= 0 || c.heads <= 0 || c.kv_heads <= 0 ||
        c.head_dim <= 0 || c.vocab <= 0 || c.heads % c.kv_heads || c.head_dim % 2)
        return fail(POCR_ERR_ARG, "pocr_model_create: invalid config");
    if (c.head_dim != kHD || c.heads / c.kv_heads > kMaxGroup)
        return fail(POCR_ERR_UNSUPPORTED, "pocr_model_create: step path needs head_dim 128 and group <= 8");
    if (c.hidden > 16384 || c.intermediate > 16384 || c.heads * c.head_dim > 16384)
        return fail(POCR_ERR_UNSUPPORTED, "pocr_model_create: width > 16384");
    CHECK_INJECT("model");
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    pocr_model *m = new pocr_model();
    ctx->refs.fetch_add(1);
    m->ctx = ctx;
    m->cfg = c;
    m->layers.resize(c.layers);
    // initTextRoPE (model.go:877-902): freq_i = theta^(-2i/d) in f64, axis from
    // the mrope sections (default 16,24,24), clamped to 2
    const int half = c.head_dim / 2;
    int sec[3] = {c.mrope_section[0], c.mrope_section[1], c.mrope_section[2]};
    if (sec[0] == 0 && sec[1] == 0 && sec[2] == 0) {
        sec[0] = 16;
        sec[1] = 24;
        sec[2] = 24;
    }
    m->h_freq.resize(half);
    m->h_axis.resize(half);
    int section_end = sec[0], ax = 0;
    for (int i = 0; i < half; ++i) {
        while (ax + 1 < 3 && i >= section_end) {
            ++ax;
            section_end += sec[ax];
        }
        m->h_axis[i] = (uint8_t)std::min(ax, 2);
        m->h_freq[i] = std::pow(c.rope_theta, -(double)(2 * i) / (double)c.head_dim);
    }
    hipError_t e = hipMalloc(&m->freq, half * sizeof(double));
    if (e == hipSuccess) e = hipMalloc(&m->axis, half);
    if (e == hipSuccess) e = hipMemcpy(m->freq, m->h_freq.data(), half * sizeof(double), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(m->axis, m->h_axis.data(), half, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        free_dev(m->freq);
        free_dev(m->axis);
        delete m;
        ctx->refs.fetch_sub(1);
        return fail(POCR_ERR_DEVICE, "model tables: %s", hipGetErrorString(e));
    }
    *out = m;
    return POCR_OK;
}

void pocr::model_release(pocr_model *m) {
    if (!m || m->refs.fetch_sub(1) != 1) return;
    pocr_ctx *ctx = m->ctx;
    {
        std::lock_guard<std::mutex> lk(ctx->mu);
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        for (auto &l : m->layers) {
            free_dev(l.ln1);
            free_dev(l.ln2);
        }
        free_dev(m->final_norm);
        free_dev(m->embed);
        free_dev(m->freq);
        free_dev(m->axis);
    }
    for (auto &l : m->layers)
        for (const pocr_weight *w : l.w) weight_release(w);
    weight_release(m->lm);
    delete m;
    ctx_release(ctx);
}

extern "C" void pocr_model_destroy(pocr_model *m) { model_release(m); }

// Matrices are fixed once the model has sequences: their captured decode
// graphs hold the weights' device addresses (a replaced weight may be freed).
extern "C" int pocr_model_set_weight(pocr_model *m, int layer, int role, const pocr_weight *w) {
    if (!m || !w) return fail(POCR_ERR_ARG, "pocr_model_set_weight: null argument");
    if (w->ctx != m->ctx) return fail(POCR_ERR_ARG, "pocr_model_set_weight: weight from another context");
    if (m->refs.load() != 1)
        return fail(POCR_ERR_ARG, "pocr_model_set_weight: set the weights before creating sequences");
    const pocr_config &c = m->cfg;
    const int q_rows = c.heads * c.head_dim, kv_rows = c.kv_heads * c.head_dim;
    if (layer == -1 && role == POCR_W_LM_HEAD) {
        if (w->rows != c.vocab || w->cols != c.hidden) return fail(POCR_ERR_ARG, "lm_head shape mismatch");
        weight_retain(w);
        weight_release(m->lm);
        m->lm = w;
        return POCR_OK;
    }
    if (layer < 0 || layer >= c.layers || role < 0 || role > POCR_W_DOWN)
        return fail(POCR_ERR_ARG, "pocr_model_set_weight: bad layer/role %d/%d", layer, role);
    static const char *names[] = {"q", "k", "v", "o", "gate", "up", "down"};
    const int want_rows[] = {q_rows, kv_rows, kv_rows, c.hidden, c.intermediate, c.intermediate, c.hidden};
    const int want_cols[] = {c.hidden, c.hidden, c.hidden, q_rows, c.hidden, c.hidden, c.intermediate};
    if (w->rows != want_rows[role] || w->cols != want_cols[role])
        return fail(POCR_ERR_ARG, "layer %d %s: shape %dx%d, want %dx%d", layer, names[role], w->rows, w->cols,
                    want_rows[role], want_cols[role]);
    weight_retain(w);
    weight_release(m->layers[layer].w[role]);
    m->layers[layer].w[role] = w;
    return POCR_OK;
}

static int upload_floats(pocr_ctx *ctx, float **dst, const float *src, size_t n) {
    if (!*dst) HIP_TRY(hipMalloc(dst, n * 4));
    HIP_TRY(hipMemcpy(*dst, src, n * 4, hipMemcpyHostToDevice));
    (void)ctx;
    return POCR_OK;
}

extern "C" int pocr_model_set_norm(pocr_model *m, int layer, int role, const float *w) {
    if (!m || !w) return fail(POCR_ERR_ARG, "pocr_model_set_norm: null argument");
    std::lock_guard<std::mutex> lk(m->ctx->mu);
    HIP_TRY(hipSetDevice(m->ctx->device));
    const size_t n = m->cfg.hidden;
    if (layer == -1 && role == POCR_N_FINAL) return upload_floats(m->ctx, &m->final_norm, w, n);
    if (layer < 0 || layer >= m->cfg.layers || (role != POCR_N_LN1 && role != POCR_N_LN2))
        return fail(POCR_ERR_ARG, "pocr_model_set_norm: bad layer/role %d/%d", layer, role);
    return upload_floats(m->ctx, role == POCR_N_LN1 ? &m->layers[layer].ln1 : &m->layers[layer].ln2, w, n);
}

extern "C" int pocr_model_set_embed(pocr_model *m, const float *embed) {
    if (!m || !embed) return fail(POCR_ERR_ARG, "pocr_model_set_embed: null argument");
    std::lock_guard<std::mutex> lk(m->ctx->mu);
    HIP_TRY(hipSetDevice(m->ctx->device));
    return upload_floats(m->ctx, &m->embed, embed, (size_t)m->cfg.vocab * m->cfg.hidden);
}

// A decoder model straight from a checkpoint: the tensors preloadTextWeights
// reads by name (model.go:2861-2885) out of a GGUF file (gguf.Open,
// internal/gguf/gguf.go:110-243); the config comes from config.json as in the
// reference (internal/config/config.go:51).  Matrices must be Q*_ROW, norms
// and embeddings F32.
extern "C" int pocr_model_load_gguf(pocr_ctx *ctx, const pocr_config *cfg, const char *path, pocr_model **out) {
    if (!ctx || !cfg || !path || !out) return fail(POCR_ERR_ARG, "pocr_model_load_gguf: null argument");
    *out = nullptr;
    CHECK_INJECT("model_load_gguf");
    pocr_gguf *g = nullptr;
    RC(pocr_gguf_open(path, &g));
    pocr_model *m = nullptr;
    int rc = pocr_model_create(ctx, cfg, &m);
    std::vector<uint8_t> buf;
    auto matrix = [&](const std::string &name, int layer, int role) -> int {
        const int i = pocr_gguf_find(g, name.c_str());
        if (i < 0) return i;
        uint32_t type = 0;
        int nd = 0;
        int64_t dims[8], bytes = 0;
        RC(pocr_gguf_tensor_info(g, i, nullptr, &type, &nd, dims, &bytes));
        if (type != POCR_Q8 && type != POCR_Q4 && type != POCR_Q6)
            return fail(POCR_ERR_UNSUPPORTED, "gguf: %s has type %u (Q8_ROW/Q4_ROW/Q6_ROW only)", name.c_str(), type);
        if (nd != 2 || dims[0] > INT32_MAX || dims[1] > INT32_MAX)
            return fail(POCR_ERR_ARG, "gguf: %s is not a 2-D matrix", name.c_str());
        const int rows = (int)dims[0], cols = (int)dims[1];
        buf.resize((size_t)bytes);
        RC(pocr_gguf_read(g, i, buf.data(), bytes));
        pocr_weight *w = nullptr;
        RC(pocr_weight_upload(ctx, (int)type, rows, cols, reinterpret_cast<const float *>(buf.data()),
                              buf.data() + (size_t)rows * 4, &w));
        const int r = pocr_model_set_weight(m, layer, role, w);  // checks the shape, retains w
        pocr_weight_free(w);
        return r;
    };
    auto floats = [&](const std::string &name, int64_t n) -> int {
        const int i = pocr_gguf_find(g, name.c_str());
        if (i < 0) return i;
        uint32_t type = 0;
        int64_t bytes = 0;
        RC(pocr_gguf_tensor_info(g, i, nullptr, &type, nullptr, nullptr, &bytes));
        if (type != 0 || bytes != n * 4)
            return fail(POCR_ERR_ARG, "gguf: %s must be F32 with %lld values", name.c_str(), (long long)n);
        buf.resize((size_t)bytes);
        return pocr_gguf_read(g, i, buf.data(), bytes);
    };
    const float *fbuf = nullptr;
    if (rc == POCR_OK) rc = floats("model.embed_tokens.weight", (int64_t)cfg->vocab * cfg->hidden);
    fbuf = reinterpret_cast<const float *>(buf.data());
    if (rc == POCR_OK) rc = pocr_model_set_embed(m, fbuf);
    if (rc == POCR_OK) rc = floats("model.norm.weight", cfg->hidden);
    if (rc == POCR_OK) rc = pocr_model_set_norm(m, -1, POCR_N_FINAL, reinterpret_cast<const float *>(buf.data()));
    if (rc == POCR_OK) rc = matrix("lm_head.weight", -1, POCR_W_LM_HEAD);
    static const char *roles[] = {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                                  "self_attn.o_proj.weight", "mlp.gate_proj.weight",    "mlp.up_proj.weight",
                                  "mlp.down_proj.weight"};
    for (int li = 0; li < cfg->layers && rc == POCR_OK; ++li) {
        const std::string pre = "model.layers." + std::to_string(li) + ".";
        rc = floats(pre + "input_layernorm.weight", cfg->hidden);
        if (rc == POCR_OK) rc = pocr_model_set_norm(m, li, POCR_N_LN1, reinterpret_cast<const float *>(buf.data()));
        if (rc == POCR_OK) rc = floats(pre + "post_attention_layernorm.weight", cfg->hidden);
        if (rc == POCR_OK) rc = pocr_model_set_norm(m, li, POCR_N_LN2, reinterpret_cast<const float *>(buf.data()));
        for (int role = 0; role <= POCR_W_DOWN && rc == POCR_OK; ++role) rc = matrix(pre + roles[role], li, role);
    }
    pocr_gguf_close(g);
    if (rc != POCR_OK) {
        if (m) pocr_model_destroy(m);
        return rc;
    }
    *out = m;
    return POCR_OK;
}

// Fixed once the model has sequences, like the activation mode: their
// captured decode graphs hold the o_proj epilogue's residual rule.
extern "C" int pocr_model_set_residual_quirk(pocr_model *m, int on) {
    if (!m) return fail(POCR_ERR_ARG, "pocr_model_set_residual_quirk: null model");
    const int q = on ? 1 : 0;
    if (q != m->quirk && m->refs.load() != 1)
        return fail(POCR_ERR_ARG, "pocr_model_set_residual_quirk: set the behaviour before creating sequences");
    m->quirk = q;
    return POCR_OK;
}

// The activation mode is fixed before the model's first sequence: captured
// decode graphs hold the mode's kernels.
extern "C" int pocr_model_set_vnni(pocr_model *m, int on) {
    if (!m) return fail(POCR_ERR_ARG, "pocr_model_set_vnni: null model");
    if (m->refs.load() != 1) return fail(POCR_ERR_ARG, "pocr_model_set_vnni: set the mode before creating sequences");
    m->vnni = on ? 1 : 0;
    return POCR_OK;
}

static int model_ready(const pocr_model *m) {
    for (int l = 0; l < m->cfg.layers; ++l) {
        for (int r = 0; r < 7; ++r)
            if (!m->layers[l].w[r]) return fail(POCR_ERR_ARG, "layer %d weight %d not set", l, r);
        if (!m->layers[l].ln1 || !m->layers[l].ln2) return fail(POCR_ERR_ARG, "layer %d norms not set", l);
        const int qt = m->layers[l].w[0]->qtype;
        for (int r = 1; r < 3; ++r)
            if (m->layers[l].w[r]->qtype != qt) return fail(POCR_ERR_ARG, "layer %d q/k/v types differ", l);
        if (m->layers[l].w[4]->qtype != m->layers[l].w[5]->qtype)
            return fail(POCR_ERR_ARG, "layer %d gate/up types differ", l);
    }
    if (!m->lm || !m->final_norm || !m->embed) return fail(POCR_ERR_ARG, "lm_head/final norm/embedding not set");
    return POCR_OK;
}

// ---------------------------------------------------------------------------
// sequences
// ---------------------------------------------------------------------------
extern "C" int pocr_seq_create(pocr_model *m, int capacity, pocr_seq **out) {
    if (!m || !out || capacity <= 0) return fail(POCR_ERR_ARG, "pocr_seq_create: bad arguments");
    *out = nullptr;
    CHECK_INJECT("seq");
    std::lock_guard<std::mutex> lk(m->ctx->mu);
    HIP_TRY(hipSetDevice(m->ctx->device));
    const pocr_config &c = m->cfg;
    pocr_seq *s = new pocr_seq();
    m->refs.fetch_add(1);
    s->m = m;
    s->cap = capacity;
    s->rpw = attn_rpw(capacity);
    s->nsplit = attn_nsplit(capacity, s->rpw);
    if (s->nsplit > kMaxSplits) {
        delete s;
        m->refs.fetch_sub(1);
        return fail(POCR_ERR_UNSUPPORTED, "pocr_seq_create: capacity %d above %d rows", capacity,
                    kMaxSplits * kMaxChunk);
    }
    s->max_tokens = capacity + 1;
    const size_t kvd = (size_t)c.kv_heads * c.head_dim;
    const size_t q_rows = (size_t)c.heads * c.head_dim;
    const size_t qkv = q_rows + 2 * kvd;
    hipError_t e = hipMalloc(&s->kv, (size_t)c.layers * 2 * capacity * kvd * 4);
    if (e == hipSuccess) e = hipMalloc(&s->h, (size_t)c.hidden * 4);
    if (e == hipSuccess) e = hipMalloc(&s->qkv, qkv * 4);
    if (e == hipSuccess) e = hipMalloc(&s->head_out, q_rows * 4);
    if (e == hipSuccess) e = hipMalloc(&s->opart, (size_t)c.heads * c.hidden * 4);
    if (e == hipSuccess) e = hipMalloc(&s->vbuf, (size_t)c.hidden * 4);
    if (e == hipSuccess) e = hipMalloc(&s->g, (size_t)c.intermediate * 4);
    if (e == hipSuccess) e = hipMalloc(&s->logits, (size_t)c.vocab * 4);
    if (e == hipSuccess) e = hipMalloc(&s->part, (size_t)c.kv_heads * s->nsplit * kMaxGroup * kRec * 4);
    if (e == hipSuccess) e = hipMalloc(&s->st, sizeof(StepState));
    if (e == hipSuccess) e = hipMalloc(&s->tokens, (size_t)s->max_tokens * 4);
    if (e == hipSuccess) e = hipMalloc(&s->samp, sizeof(SampleState));
    if (e == hipSuccess) e = hipMalloc(&s->topk_part, (size_t)kTopKMaxParts * kTopKMax * 8);
    if (e == hipSuccess) e = hipMemset(s->samp, 0, sizeof(SampleState));
    if (e == hipSuccess) e = hipMemset(s->kv, 0, (size_t)c.layers * 2 * capacity * kvd * 4);
    if (e != hipSuccess) {
        delete s;
        m->refs.fetch_sub(1);
        return fail(POCR_ERR_NOMEM, "pocr_seq_create(%d): %s", capacity, hipGetErrorString(e));
    }
    StepState st{};
    st.cap = capacity;
    st.half = c.head_dim / 2;
    e = hipMemcpy(s->st, &st, sizeof(st), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        delete s;
        m->refs.fetch_sub(1);
        return fail(POCR_ERR_DEVICE, "pocr_seq_create: %s", hipGetErrorString(e));
    }
    *out = s;
    return POCR_OK;
}

static void batch_forget(pocr_batch *b, const pocr_seq *s);

extern "C" void pocr_seq_destroy(pocr_seq *s) {
    if (!s) return;
    pocr_model *m = s->m;
    {
        std::lock_guard<std::mutex> lk(m->ctx->mu);
        (void)hipSetDevice(m->ctx->device);
        (void)hipStreamSynchronize(m->ctx->stream);
        if (s->batch) batch_forget(s->batch, s);
        delete s;
    }
    model_release(m);
}

int pocr::seq_idle(const pocr_seq *s, const char *op) {
    return s->batch ? fail(POCR_ERR_ARG, "%s: the sequence is in a decode batch", op) : POCR_OK;
}

float *pocr::layer_k(const pocr_seq *s, int layer) {
    const pocr_config &c = s->m->cfg;
    return s->kv + (size_t)layer * 2 * s->cap * c.kv_heads * c.head_dim;
}
float *pocr::layer_v(const pocr_seq *s, int layer) {
    const pocr_config &c = s->m->cfg;
    return layer_k(s, layer) + (size_t)s->cap * c.kv_heads * c.head_dim;
}

int pocr::seq_set_state(pocr_seq *s, int len) {
    StepState st{};
    st.len = len;
    st.cap = s->cap;
    st.half = s->m->cfg.head_dim / 2;
    HIP_TRY(hipMemcpyAsync(s->st, &st, sizeof(st), hipMemcpyHostToDevice, s->m->ctx->stream));
    HIP_TRY(hipStreamSynchronize(s->m->ctx->stream));
    s->len = len;
    return POCR_OK;
}

extern "C" int pocr_seq_reset(pocr_seq *s) {
    if (!s) return fail(POCR_ERR_ARG, "pocr_seq_reset: null");
    std::lock_guard<std::mutex> lk(s->m->ctx->mu);
    RC(seq_idle(s, "pocr_seq_reset"));
    HIP_TRY(hipSetDevice(s->m->ctx->device));
    return seq_set_state(s, 0);
}

extern "C" int pocr_seq_len(const pocr_seq *s) { return s ? s->len : POCR_ERR_ARG; }

extern "C" int pocr_seq_device_tokens(const pocr_seq *s) { return s ? s->device_tokens : POCR_ERR_ARG; }

// the generator at its seed (samplingRNGInto, model.go:1846-1852)
static int seed_sampler(pocr_seq *s) {
    hipStream_t st = s->m->ctx->stream;
    HIP_TRY(hipMemcpyAsync(&s->samp->rng, &s->seed, 8, hipMemcpyHostToDevice, st));
    HIP_TRY(hipStreamSynchronize(st));  // s->seed may change once the lock is released
    return POCR_OK;
}

extern "C" int pocr_seq_set_sampling(pocr_seq *s, double temperature, int top_k, uint64_t seed) {
    if (!s) return fail(POCR_ERR_ARG, "pocr_seq_set_sampling: null");
    // ValidateGenerateOptions (model.go:450-470)
    if (!(temperature >= 0.0) || std::isinf(temperature)) return fail(POCR_ERR_ARG, "temperature must be finite and >= 0");
    if (top_k < 0) return fail(POCR_ERR_ARG, "top_k must be >= 0");
    // generationUsesArgmaxSampling (model.go:1858-1860) → greedy; otherwise
    // the candidates path (1866-1868) for 1 < top_k < vocab, and every score
    // (sampleTokenScratch → sampleFullLogitsScratch, 1877-1879) for top_k 0
    // or >= vocab, kept here as top_k 0
    const bool greedy = temperature <= 0.0 || top_k == 1;
    if (!greedy && top_k >= s->m->cfg.vocab) top_k = 0;
    std::lock_guard<std::mutex> lk(s->m->ctx->mu);
    RC(seq_idle(s, "pocr_seq_set_sampling"));
    HIP_TRY(hipSetDevice(s->m->ctx->device));
    HIP_TRY(hipStreamSynchronize(s->m->ctx->stream));
    if (!greedy && (top_k == 0 || top_k > kTopKMax)) {
        WideBufs b;
        RC(wide_bufs(s->wide, s->m->cfg.vocab, &b));  // allocated before any capture
    }
    if (s->sampling != !greedy || (!greedy && s->top_k != top_k)) {
        // the captured step ends in the other LM head: capture again
        drop_decode_graphs(s);
    }
    s->sampling = !greedy;
    s->temperature = temperature;
    s->top_k = greedy ? 0 : top_k;
    s->seed = seed;
    SampleState h{};
    h.rng = seed;
    h.temperature = temperature;
    h.top_k = s->top_k;
    HIP_TRY(hipMemcpy(s->samp, &h, sizeof(h), hipMemcpyHostToDevice));
    return POCR_OK;
}

extern "C" int pocr_seq_read_kv(pocr_seq *s, int layer, float *k, float *v) {
    if (!s || !k || !v || layer < 0 || layer >= s->m->cfg.layers) return fail(POCR_ERR_ARG, "pocr_seq_read_kv");
    std::lock_guard<std::mutex> lk(s->m->ctx->mu);
    HIP_TRY(hipSetDevice(s->m->ctx->device));
    const size_t n = (size_t)s->len * s->m->cfg.kv_heads * s->m->cfg.head_dim * 4;
    if (n == 0) return POCR_OK;
    HIP_TRY(hipMemcpy(k, layer_k(s, layer), n, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(v, layer_v(s, layer), n, hipMemcpyDeviceToHost));
    return POCR_OK;
}

extern "C" int pocr_seq_write_kv(pocr_seq *s, int layer, const float *k, const float *v, int len) {
    if (!s || !k || !v || layer < 0 || layer >= s->m->cfg.layers || len < 0 || len > s->cap)
        return fail(POCR_ERR_ARG, "pocr_seq_write_kv: bad arguments");
    std::lock_guard<std::mutex> lk(s->m->ctx->mu);
    RC(seq_idle(s, "pocr_seq_write_kv"));
    HIP_TRY(hipSetDevice(s->m->ctx->device));
    const size_t n = (size_t)len * s->m->cfg.kv_heads * s->m->cfg.head_dim * 4;
    if (n) {
        HIP_TRY(hipMemcpy(layer_k(s, layer), k, n, hipMemcpyHostToDevice));
        HIP_TRY(hipMemcpy(layer_v(s, layer), v, n, hipMemcpyHostToDevice));
    }
    return seq_set_state(s, len);
}

extern "C" int pocr_seq_truncate(pocr_seq *s, int len) {
    if (!s || len < 0 || len > s->len) return fail(POCR_ERR_ARG, "pocr_seq_truncate: bad length");
    std::lock_guard<std::mutex> lk(s->m->ctx->mu);
    RC(seq_idle(s, "pocr_seq_truncate"));
    HIP_TRY(hipSetDevice(s->m->ctx->device));
    return seq_set_state(s, len);
}

static int time_matvec_impl(pocr_ctx *ctx, const pocr_weight *const *weights, int n_weights, const float *x,
                            int iters, float *avg_us, bool argmax, const char *name) {
    if (!ctx || !weights || n_weights <= 0 || !x || iters <= 0 || !avg_us)
        return fail(POCR_ERR_ARG, "%s: bad arguments", name);
    for (int i = 0; i < n_weights; ++i)
        if (!weights[i] || weights[i]->rows != weights[0]->rows || weights[i]->cols != weights[0]->cols ||
            weights[i]->qtype != weights[0]->qtype || weights[i]->ctx != ctx)
            return fail(POCR_ERR_ARG, "%s: weights differ in shape/type/context", name);
    CHECK_INJECT(name + 5);  // the op name without "pocr_"
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    const pocr_weight *w0 = weights[0];
    const int epi = argmax ? EPI_ARGMAX : EPI_PLAIN;
    RC(ctx->x.ensure((size_t)w0->cols * 4));
    RC(ctx->out.ensure((size_t)w0->rows * 4));
    RC(ctx->state.ensure(sizeof(StepState)));
    RC(h2d(s, ctx->x.p, x, (size_t)w0->cols * 4));
    HIP_TRY(hipMemsetAsync(ctx->state.p, 0, sizeof(StepState), s));
    GemvPlan plan;
    DevMat dm = dev_mat(w0);
    RC(plan_gemv(w0->qtype, 1, w0->rows, w0->cols, &dm, 1, kBigGrid, &plan, 1, nullptr, epi));
    auto params = [&](int i) {
        GemvParams p = gemv_params_1(weights[i]);
        p.x = ctx->x.as<float>();
        p.out = argmax ? nullptr : ctx->out.as<float>();
        p.st = ctx->state.as<StepState>();  // argmax slots (the key only grows: no reset needed)
        return p;
    };
    // the kernel pocr_matvec / the decode run: the MFMA head for the greedy
    // argmax and for every score of an LM-head-sized matrix, where the shape
    // allows it
    const void *hfn = (argmax || w0->rows >= kHeadWideMinRows) ? plan_head(params(0), 1, 1) : nullptr;
    auto launch = [&](int i) {
        return hfn ? launch_head(s, hfn, params(i), PRO_COPY, 1, nullptr, argmax)
                   : launch_gemv(s, plan, params(i), PRO_COPY, epi);
    };
    hipEvent_t e0, e1;
    HIP_TRY(hipEventCreate(&e0));
    HIP_TRY(hipEventCreate(&e1));
    for (int i = 0; i < n_weights; ++i) RC(launch(i));  // warm-up pass
    HIP_TRY(hipEventRecord(e0, s));
    for (int it = 0; it < iters; ++it) RC(launch(it % n_weights));
    HIP_TRY(hipEventRecord(e1, s));
    HIP_TRY(hipEventSynchronize(e1));
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *avg_us = ms * 1000.0f / (float)iters;
    return POCR_OK;
}

extern "C" int pocr_time_matvec(pocr_ctx *ctx, const pocr_weight *const *weights, int n_weights, const float *x,
                                int iters, float *avg_us) {
    return time_matvec_impl(ctx, weights, n_weights, x, iters, avg_us, false, "pocr_time_matvec");
}

extern "C" int pocr_time_matvec_argmax(pocr_ctx *ctx, const pocr_weight *const *weights, int n_weights,
                                       const float *x, int iters, float *avg_us) {
    return time_matvec_impl(ctx, weights, n_weights, x, iters, avg_us, true, "pocr_time_matvec_argmax");
}

extern "C" int pocr_time_matvec_batched(pocr_ctx *ctx, const pocr_weight *const *weights, int n_weights,
                                        const float *x, int m, int iters, float *avg_us) {
    if (!ctx || !weights || n_weights <= 0 || !x || m <= 0 || iters <= 0 || !avg_us)
        return fail(POCR_ERR_ARG, "pocr_time_matvec_batched: bad arguments");
    for (int i = 0; i < n_weights; ++i)
        if (!weights[i] || weights[i]->rows != weights[0]->rows || weights[i]->cols != weights[0]->cols ||
            weights[i]->qtype != weights[0]->qtype || weights[i]->ctx != ctx)
            return fail(POCR_ERR_ARG, "pocr_time_matvec_batched: weights differ in shape/type/context");
    CHECK_INJECT("time_matvec_batched");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    const pocr_weight *w0 = weights[0];
    RC(ctx->x.ensure((size_t)m * w0->cols * 4));
    RC(ctx->out.ensure((size_t)m * w0->rows * 4));
    RC(h2d(s, ctx->x.p, x, (size_t)m * w0->cols * 4));
    // the launches pocr_matvec makes for m rows: the vector GEMV with 2 or 4
    // vectors per pass up to m = 4, the digit-plane MFMA GEMM above
    for (int i = 0; i < n_weights; ++i)  // warm-up pass (allocates the digit buffers)
        RC(matvec_rows(ctx, weights[i], ctx->x.as<float>(), m, ctx->out.as<float>()));
    hipEvent_t e0, e1;
    HIP_TRY(hipEventCreate(&e0));
    HIP_TRY(hipEventCreate(&e1));
    HIP_TRY(hipEventRecord(e0, s));
    for (int it = 0; it < iters; ++it)
        RC(matvec_rows(ctx, weights[it % n_weights], ctx->x.as<float>(), m, ctx->out.as<float>()));
    HIP_TRY(hipEventRecord(e1, s));
    HIP_TRY(hipEventSynchronize(e1));
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *avg_us = ms * 1000.0f / (float)iters;
    return POCR_OK;
}

extern "C" int pocr_time_attention(pocr_ctx *ctx, int heads, int kv_heads, int head_dim, int cache_len, int n_layers,
                                   int iters, float *avg_us) {
    if (!ctx || heads <= 0 || kv_heads <= 0 || heads % kv_heads || cache_len <= 0 || n_layers <= 0 || iters <= 0 ||
        !avg_us)
        return fail(POCR_ERR_ARG, "pocr_time_attention: bad arguments");
    if (head_dim != kHD || heads / kv_heads > kMaxGroup)
        return fail(POCR_ERR_UNSUPPORTED, "pocr_time_attention: head_dim 128 and GQA group <= 8 only");
    const int rpw = attn_rpw(cache_len);
    const int nsplit = attn_nsplit(cache_len, rpw);
    if (nsplit > kMaxSplits) return fail(POCR_ERR_UNSUPPORTED, "pocr_time_attention: cache above %d rows",
                                         kMaxSplits * kMaxChunk);
    CHECK_INJECT("time_attention");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    const size_t kvd = (size_t)kv_heads * kHD;
    const size_t layer_floats = 2 * (size_t)cache_len * kvd;
    RC(ctx->kc.ensure(layer_floats * n_layers * 4));
    RC(ctx->x.ensure((size_t)(heads + 2 * kv_heads) * kHD * 4));
    RC(ctx->out.ensure((size_t)heads * kHD * 4));
    RC(ctx->part.ensure((size_t)kv_heads * nsplit * kMaxGroup * kRec * 4));
    RC(ctx->state.ensure(sizeof(StepState)));
    // cache rows and q/k/v hold 1/128 (the values do not change the work)
    HIP_TRY(hipMemsetD32Async((hipDeviceptr_t)ctx->kc.p, 0x3C000000, layer_floats * n_layers, s));
    HIP_TRY(hipMemsetD32Async((hipDeviceptr_t)ctx->x.p, 0x3C000000, (size_t)(heads + 2 * kv_heads) * kHD, s));
    StepState hs{};
    hs.len = cache_len;
    hs.clen = cache_len - 1;  // each launch re-appends the last row
    hs.cap = cache_len;
    hs.half = kHD / 2;
    hs.has_rope = 1;
    for (int i = 0; i < kHD / 2; ++i) {
        hs.cos_t[i] = 1.0f;
        hs.sin_t[i] = 0.0f;
    }
    HIP_TRY(hipMemcpyAsync(ctx->state.p, &hs, sizeof(hs), hipMemcpyHostToDevice, s));
    HIP_TRY(hipStreamSynchronize(s));  // hs is a stack object
    AttnParams a{};
    a.q = ctx->x.as<float>();
    a.k_new = a.q + (size_t)heads * kHD;
    a.v_new = a.k_new + kvd;
    a.st = ctx->state.as<StepState>();
    a.part = ctx->part.as<float>();
    a.head_out = ctx->out.as<float>();
    a.heads = heads;
    a.kvh = kv_heads;
    attn_shape(a, cache_len, rpw);
    a.scale = (float)(1.0 / std::sqrt((double)kHD));
    auto launch = [&](int layer) {
        a.kc = ctx->kc.as<float>() + layer * layer_floats;
        a.vc = a.kc + (size_t)cache_len * kvd;
        launch_attn_decode(s, rpw, dim3(kv_heads, nsplit), a);
        launch_attn_merge(s, dim3(heads), a);
    };
    for (int l = 0; l < n_layers; ++l) launch(l);
    HIP_TRY(hipGetLastError());
    hipEvent_t e0, e1;
    HIP_TRY(hipEventCreate(&e0));
    HIP_TRY(hipEventCreate(&e1));
    HIP_TRY(hipEventRecord(e0, s));
    for (int it = 0; it < iters; ++it) launch(it % n_layers);
    HIP_TRY(hipEventRecord(e1, s));
    HIP_TRY(hipEventSynchronize(e1));
    HIP_TRY(hipGetLastError());
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *avg_us = ms * 1000.0f / (float)iters;
    return POCR_OK;
}

// The read ceiling a weight-streaming kernel is measured against: every
// workgroup reads 16-byte nontemporal chunks of one buffer in a grid-stride
// loop (4 in flight per lane) and folds them into one xor per lane, stored
// only if it equals a constant (never, for the filled buffers), so the reads
// stay and nothing else costs time.  (An earlier form reduced the xors
// through LDS with one thread per workgroup: that tail cost about 2 µs of a
// 53 MB launch and made the ceiling look 20 % lower than it is.)
static __global__ void __launch_bounds__(kThreads) k_stream_read(const uint4 *p, size_t n16, unsigned *out) {
    constexpr int U = 4;
    typedef unsigned u4v __attribute__((ext_vector_type(4)));
    const u4v *q = reinterpret_cast<const u4v *>(p);
    const size_t stride = (size_t)gridDim.x * kThreads * U;
    size_t i = (size_t)blockIdx.x * kThreads * U + threadIdx.x;
    unsigned acc = 0;
    for (; i + (U - 1) * kThreads < n16; i += stride) {
        u4v v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(q + i + u * kThreads);
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += kThreads) acc ^= q[i].x ^ q[i].y ^ q[i].z ^ q[i].w;
    if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;
}

extern "C" int pocr_time_stream_read(pocr_ctx *ctx, int64_t bytes, int n_buffers, int iters, float *avg_us) {
    if (!ctx || bytes < 16 || bytes % 16 || n_buffers <= 0 || n_buffers > 64 || iters <= 0 || !avg_us)
        return fail(POCR_ERR_ARG, "pocr_time_stream_read: bad arguments");
    CHECK_INJECT("time_stream_read");
    CTX_GUARD(ctx);
    hipStream_t s = ctx->stream;
    constexpr int kGrid = 2048;
    std::vector<void *> bufs(n_buffers, nullptr);
    unsigned *out = nullptr;
    auto release = [&] {
        (void)hipStreamSynchronize(s);
        for (void *b : bufs)
            if (b) (void)hipFree(b);
        if (out) (void)hipFree(out);
    };
    hipError_t e = hipMalloc(&out, kGrid * sizeof(unsigned));
    for (int i = 0; i < n_buffers && e == hipSuccess; ++i) {
        e = hipMalloc(&bufs[i], (size_t)bytes);
        if (e == hipSuccess) e = hipMemsetAsync(bufs[i], 1, (size_t)bytes, s);
    }
    if (e != hipSuccess) {
        release();
        return fail(POCR_ERR_NOMEM, "pocr_time_stream_read: %s", hipGetErrorString(e));
    }
    const size_t n16 = (size_t)bytes / 16;
    auto launch = [&](int i) {
        hipLaunchKernelGGL(k_stream_read, dim3(kGrid), dim3(kThreads), 0, s,
                           static_cast<const uint4 *>(bufs[i % n_buffers]), n16, out);
    };
    for (int i = 0; i < n_buffers; ++i) launch(i);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0.0f;
    e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = hipEventRecord(e0, s);
    if (e == hipSuccess) {
        for (int it = 0; it < iters; ++it) launch(it);
        e = hipEventRecord(e1, s);
    }
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipGetLastError();
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    release();
    if (e != hipSuccess) return fail(POCR_ERR_DEVICE, "pocr_time_stream_read: %s", hipGetErrorString(e));
    *avg_us = ms * 1000.0f / (float)iters;
    return POCR_OK;
}

// ---------------------------------------------------------------------------
// the decoder step on the device
// ---------------------------------------------------------------------------

// One layer (model.go:3492-3603 with attentionWithNorm 3850-4066 and
// mlpDownAddRMSNormCPU 5714-5800).  last/kv_only select the final-layer
// variants.
// The o_proj folded into the attention merge (k_attn_merge_oproj, the
// consumers' PRO_OPART / EPI_DOWNV): head_dim 128, o_proj columns = heads·128,
// and gate/up/down on the streaming GEMV's shapes (their prologue and
// epilogue carry the partial sums).  POCR_FUSED_OPROJ=0 keeps the separate
// merge and o_proj launches.
static bool gemv_fast_shape(const DevMat &m) {
    const int W = m.qtype == POCR_Q4 ? 32 : 16, CB = m.qtype == POCR_Q6 ? 12 : 16;
    if (m.cols % W != 0 || m.cols > kMaxCols || ((uintptr_t)m.data) % 16 != 0) return false;
    const int C = m.cols / W;
    if (m.row_bytes != C * CB) return false;
    const int lpr = C % 64 == 0 ? 64 : (C % 32 == 0 ? 32 : 0);
    return lpr != 0 && !(C / lpr > 4 || (lpr == 32 && C / lpr > 3));
}

static bool fused_oproj(const pocr_model *m, const LayerW &L) {
    const char *env = getenv("POCR_FUSED_OPROJ");
    if (env && env[0] == '0') return false;
    const pocr_config &c = m->cfg;
    const DevMat o = dev_mat(L.w[POCR_W_O]);
    if (c.head_dim != kHD || o.cols != c.heads * kHD || o.rows != c.hidden || c.heads > kMaxOparts ||
        c.hidden > 4 * kThreads || c.hidden % 8 != 0)
        return false;
    if (((uintptr_t)o.data) % 16 != 0 || o.row_bytes % 4 != 0) return false;
    if (o.qtype == POCR_Q6 ? o.row_bytes != o.cols / 16 * 12 : o.row_bytes != o.cols * (o.qtype == POCR_Q4 ? 1 : 2) / 2)
        return false;
    return gemv_fast_shape(dev_mat(L.w[POCR_W_GATE])) && gemv_fast_shape(dev_mat(L.w[POCR_W_UP])) &&
           gemv_fast_shape(dev_mat(L.w[POCR_W_DOWN]));
}

static int launch_merge_oproj(hipStream_t st, const AttnParams &a, const pocr_weight *wo, float *part, int heads) {
    OprojParts op{dev_mat(wo), part};
    const dim3 grid(heads, kOprojSlices);
    const bool wide = merge_prefetch(a.nsplit) == 16;
    switch (wo->qtype) {
    case POCR_Q4:
        if (wide) hipLaunchKernelGGL((k_attn_merge_oproj<QT_Q4, 16>), grid, dim3(kMergeThreads), 0, st, a, op);
        else hipLaunchKernelGGL((k_attn_merge_oproj<QT_Q4, 8>), grid, dim3(kMergeThreads), 0, st, a, op);
        break;
    case POCR_Q8:
        if (wide) hipLaunchKernelGGL((k_attn_merge_oproj<QT_Q8, 16>), grid, dim3(kMergeThreads), 0, st, a, op);
        else hipLaunchKernelGGL((k_attn_merge_oproj<QT_Q8, 8>), grid, dim3(kMergeThreads), 0, st, a, op);
        break;
    default:
        if (wide) hipLaunchKernelGGL((k_attn_merge_oproj<QT_Q6, 16>), grid, dim3(kMergeThreads), 0, st, a, op);
        else hipLaunchKernelGGL((k_attn_merge_oproj<QT_Q6, 8>), grid, dim3(kMergeThreads), 0, st, a, op);
        break;
    }
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

// the model's GEMV: plain mode, or the VNNI activation mode (vnni.hpp)
static int model_gemv(const pocr_model *m, hipStream_t st, const GemvParams &p, int nmat, int pro, int epi) {
    return m->vnni ? gemv_launch_vnni(st, p, nmat, pro, epi, kBigGrid) : gemv_launch(st, p, nmat, pro, epi, kBigGrid);
}

static int enqueue_layer(pocr_seq *s, int li, bool last, bool kv_only) {
    pocr_model *m = s->m;
    const pocr_config &c = m->cfg;
    hipStream_t st = m->ctx->stream;
    const LayerW &L = m->layers[li];
    if (m->vnni && (c.head_dim != kHD || s->cap > kOrdMaxRows))
        return fail(POCR_ERR_UNSUPPORTED, "VNNI mode: head_dim %d, capacity %d (128 and at most %d)", c.head_dim,
                    s->cap, kOrdMaxRows);
    const int q_rows = c.heads * c.head_dim, kv_rows = c.kv_heads * c.head_dim;
    const float eps = c.rms_norm_eps;

    // 1. x = RMSNorm(h)·ln1 (recomputed per workgroup) → q|k|v
    GemvParams p{};
    p.m[0] = dev_mat(L.w[POCR_W_Q]);
    p.m[1] = dev_mat(L.w[POCR_W_K]);
    p.m[2] = dev_mat(L.w[POCR_W_V]);
    p.seg_end[0] = q_rows;
    p.seg_end[1] = q_rows + kv_rows;
    p.seg_end[2] = q_rows + 2 * kv_rows;
    p.rows = q_rows + 2 * kv_rows;
    p.cols = c.hidden;
    p.x = s->h;
    p.norm_w = L.ln1;
    p.eps = eps;
    p.out = s->qkv;
    p.st = s->st;
    RC(model_gemv(m, st, p, 1, PRO_RMSNORM, EPI_PLAIN));

    // 2. RoPE + KV append + split-K attention → head_out
    AttnParams a{};
    a.q = s->qkv;
    a.k_new = s->qkv + q_rows;
    a.v_new = s->qkv + q_rows + kv_rows;
    a.kc = layer_k(s, li);
    a.vc = layer_v(s, li);
    a.st = s->st;
    a.part = s->part;
    a.head_out = s->head_out;
    a.heads = c.heads;
    a.kvh = c.kv_heads;
    attn_shape(a, s->cap, s->rpw);
    a.scale = (float)(1.0 / std::sqrt((double)c.head_dim));
    launch_attn_decode(st, s->rpw, dim3(c.kv_heads, s->nsplit), a);
    const pocr_weight *wo = L.w[POCR_W_O];
    const int quirk = (m->quirk && (wo->qtype == POCR_Q4 || wo->qtype == POCR_Q6)) ? 1 : 0;
    if (!kv_only && !m->vnni && fused_oproj(m, L)) {
        // 2'. merge + o_proj partials per head; gate/up sums them with the
        // residual (PRO_OPART), down takes residual + attention when in place
        RC(launch_merge_oproj(st, a, wo, s->opart, c.heads));
        GemvParams gu = gemv_params_1(L.w[POCR_W_GATE]);
        gu.m[1] = dev_mat(L.w[POCR_W_UP]);
        gu.x = s->opart;
        gu.flag = c.heads;  // partial rows
        gu.residual = s->h;
        gu.vbuf = s->vbuf;
        gu.norm_w = L.ln2;
        gu.eps = eps;
        gu.out = s->g;
        gu.st = s->st;
        RC(gemv_launch(st, gu, 2, PRO_OPART, EPI_SWIGLU, kBigGrid));
        GemvParams d = gemv_params_1(L.w[POCR_W_DOWN]);
        d.x = s->g;
        d.residual = s->h;
        d.vbuf = s->vbuf;
        d.st = s->st;
        d.flag = last ? 1 : 0;
        d.quirk = quirk;
        return gemv_launch(st, d, 1, PRO_COPY, EPI_DOWNV, kBigGrid);
    }
    if (m->vnni) {
        // the reference's summation order (vnni.hpp): the split records are unused
        if (!kv_only) hipLaunchKernelGGL(k_attn_ordered, dim3(c.heads), dim3(kThreads), (size_t)s->cap * 4, st, a);
    } else {
        launch_attn_merge(st, dim3(c.heads), a);
    }
    HIP_TRY(hipGetLastError());
    if (kv_only) return POCR_OK;

    // 3. o_proj + residual (+quirk) → vbuf (= h + attn), h updated if in place
    GemvParams o = gemv_params_1(wo);
    o.x = s->head_out;
    o.residual = s->h;
    o.vbuf = s->vbuf;
    o.st = s->st;
    o.quirk = quirk;
    RC(model_gemv(m, st, o, 1, PRO_COPY, EPI_OPROJ));

    // 4. RMSNorm(vbuf)·ln2 → gate/up → SiLU(g)·u
    GemvParams gu = gemv_params_1(L.w[POCR_W_GATE]);
    gu.m[1] = dev_mat(L.w[POCR_W_UP]);
    gu.x = s->vbuf;
    gu.norm_w = L.ln2;
    gu.eps = eps;
    gu.out = s->g;
    gu.st = s->st;
    RC(model_gemv(m, st, gu, 2, PRO_RMSNORM, EPI_SWIGLU));

    // 5. down + residual: h += W_down·g (in place); last layer: vbuf = h + down (OutOnly)
    GemvParams d = gemv_params_1(L.w[POCR_W_DOWN]);
    d.x = s->g;
    d.residual = s->h;
    d.vbuf = s->vbuf;
    d.st = s->st;
    d.flag = last ? 1 : 0;
    RC(model_gemv(m, st, d, 1, PRO_COPY, EPI_DOWN));
    return POCR_OK;
}

int pocr::launch_attn_ordered_rows(hipStream_t s, const float *qkv, int stride, const float *kc, const float *vc,
                                   int heads, int kvh, int n, int clen0, float scale, float *out, int out_stride) {
    const int rows = clen0 + n, group = heads / kvh;
    if (rows > kOrdMaxRows) return fail(POCR_ERR_UNSUPPORTED, "ordered attention: %d rows", rows);
    // q heads per workgroup: as many of the group as keep the scores within
    // 56 KB of LDS (with the q rows under 64 KB; two workgroups per CU or more)
    int hpw = 1;
    for (const int c : {8, 4, 2})
        if (group % c == 0 && (size_t)c * rows * 4 <= 56 * 1024) {
            hpw = c;
            break;
        }
    const dim3 grid(kvh * (group / hpw), n);
    const size_t lds = (size_t)hpw * rows * 4;
    switch (hpw) {
    case 8: hipLaunchKernelGGL(k_attn_ordered_rows<8>, grid, dim3(kThreads), lds, s, qkv, stride, kc, vc, heads, kvh, clen0, scale, out, out_stride); break;
    case 4: hipLaunchKernelGGL(k_attn_ordered_rows<4>, grid, dim3(kThreads), lds, s, qkv, stride, kc, vc, heads, kvh, clen0, scale, out, out_stride); break;
    case 2: hipLaunchKernelGGL(k_attn_ordered_rows<2>, grid, dim3(kThreads), lds, s, qkv, stride, kc, vc, heads, kvh, clen0, scale, out, out_stride); break;
    default: hipLaunchKernelGGL(k_attn_ordered_rows<1>, grid, dim3(kThreads), lds, s, qkv, stride, kc, vc, heads, kvh, clen0, scale, out, out_stride);
    }
    HIP_TRY(hipGetLastError());
    return POCR_OK;
}

int pocr::enqueue_lm_head(pocr_seq *s, const float *x, bool want_logits) {
    pocr_model *m = s->m;
    hipStream_t st = m->ctx->stream;
    GemvParams p = gemv_params_1(m->lm);
    p.x = x;
    p.norm_w = m->final_norm;
    p.eps = m->cfg.rms_norm_eps;
    p.st = s->st;
    if (!s->sampling) {
        p.out = want_logits ? s->logits : nullptr;
        return model_gemv(m, st, p, 1, PRO_RMSNORM, EPI_ARGMAX);
    }
    // matVecTopKMaybeCPU (model.go:7202-7235): every score, then the top-k
    // and the draw (sampleCandidateScoresScratch, 1950-1990)
    p.out = s->logits;
    RC(model_gemv(m, st, p, 1, PRO_RMSNORM, EPI_PLAIN));
    const int vocab = m->cfg.vocab;
    if (s->top_k >= 2 && s->top_k <= kTopKMax)
        return enqueue_topk(st, s->logits, vocab, s->top_k, s->topk_part, s->samp, s->st, 1);
    WideBufs b;
    RC(wide_bufs(s->wide, vocab, &b));
    // top_k 0: every score through sampleTokenScratch (model.go:1877-1879)
    if (s->top_k == 0) return enqueue_sample_full(st, s->logits, vocab, b, s->samp, s->st);
    return enqueue_sample_sorted(st, s->logits, vocab, s->top_k, b, s->samp, s->st, 1);
}

static int enqueue_step(pocr_seq *s, int mode, bool need_logits, bool want_logits) {
    pocr_model *m = s->m;
    const pocr_config &c = m->cfg;
    hipStream_t st = m->ctx->stream;
    hipLaunchKernelGGL(k_step_begin, dim3(1), dim3(kThreads), 0, st, s->st, m->embed, s->h, c.hidden, c.vocab,
                       m->freq, m->axis, mode, s->tokens, s->max_tokens);
    HIP_TRY(hipGetLastError());
    for (int li = 0; li < c.layers; ++li) {
        const bool last = li + 1 == c.layers;
        RC(enqueue_layer(s, li, last, last && !need_logits));
    }
    if (need_logits) RC(enqueue_lm_head(s, s->vbuf, want_logits));
    return POCR_OK;
}

int pocr::read_state(pocr_seq *s, StepState *out) {
    HIP_TRY(hipMemcpyAsync(out, s->st, sizeof(StepState), hipMemcpyDeviceToHost, s->m->ctx->stream));
    HIP_TRY(hipStreamSynchronize(s->m->ctx->stream));
    return POCR_OK;
}

int pocr::step_locked(pocr_seq *s, const float *emb, const int32_t pos3[3], int need_logits, float *logits,
                       int32_t *token) {
    pocr_model *m = s->m;
    hipStream_t st = m->ctx->stream;
    if (s->len >= s->cap) return fail(POCR_ERR_ARG, "pocr_step: cache full (%d rows)", s->cap);
    RC(h2d(st, s->h, emb, (size_t)m->cfg.hidden * 4));
    RC(h2d(st, &s->st->pos, pos3, 12));
    RC(enqueue_step(s, 0, need_logits != 0, logits != nullptr));
    StepState hs;
    RC(read_state(s, &hs));
    if (hs.err) return fail(POCR_ERR_DEVICE, "step: device state error %d", hs.err);
    s->len = hs.len;
    if (need_logits) {
        if (token) {
            const unsigned long long key = argmax_of(hs);
            if (key == 0ull) return fail(POCR_ERR_DEVICE, "step: no finite logit");
            *token = (int32_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
        }
        if (logits) {
            HIP_TRY(hipMemcpy(logits, s->logits, (size_t)m->cfg.vocab * 4, hipMemcpyDeviceToHost));
        }
    }
    return POCR_OK;
}

extern "C" int pocr_step(pocr_seq *s, const float *emb, const int32_t pos3[3], int need_logits, float *logits,
                         int32_t *token) {
    if (!s || !emb || !pos3) return fail(POCR_ERR_ARG, "pocr_step: null argument");
    RC(model_ready(s->m));
    CHECK_INJECT("step");
    std::lock_guard<std::mutex> lk(s->m->ctx->mu);
    RC(seq_idle(s, "pocr_step"));
    HIP_TRY(hipSetDevice(s->m->ctx->device));
    return step_locked(s, emb, pos3, need_logits, logits, token);
}

// `steps` decode steps (mode 1) captured as one graph
static int capture_decode_steps(pocr_seq *s, int steps, hipGraph_t *graph_out, hipGraphExec_t *exec_out) {
    hipStream_t st = s->m->ctx->stream;
    HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    int rc = POCR_OK;
    for (int i = 0; i < steps && rc == POCR_OK; ++i) rc = enqueue_step(s, 1, true, false);
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(st, &graph);
    if (rc != POCR_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    if (e != hipSuccess) return fail(POCR_ERR_DEVICE, "graph capture: %s", hipGetErrorString(e));
    e = hipGraphInstantiate(exec_out, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return fail(POCR_ERR_DEVICE, "graph instantiate: %s", hipGetErrorString(e));
    }
    *graph_out = graph;
    return POCR_OK;
}

static int build_decode_graph(pocr_seq *s) {
    if (s->decode_exec) return POCR_OK;
    return capture_decode_steps(s, 1, &s->decode_graph, &s->decode_exec);
}

// The decode loop replays kDecodeGraphSteps steps per graph launch: each
// launch costs about 5 µs on the device beyond its kernels, against 390 µs
// per step (capture and instantiation take about 0.25 ms per step, once per
// sequence).
static int build_decode_graph_n(pocr_seq *s) {
    RC(build_decode_graph(s));
    if (s->decode_exec_n) return POCR_OK;
    return capture_decode_steps(s, kDecodeGraphSteps, &s->decode_graph_n, &s->decode_exec_n);
}

static bool is_eos(int32_t t, const int32_t *eos, int n) {
    for (int i = 0; i < n; ++i)
        if (eos[i] == t) return true;
    return false;
}

// The decode loop's EOS ids in the step state. Up to kMaxEos ids sit in the
// state itself; a longer list (up to maxEOSTokenIDs) becomes a bitmap over the
// vocabulary in the sequence's own buffer, which the step prologue tests with
// one load. Ids at or past the vocabulary can never be taken and are left out.
// The caller uploads hs and synchronizes the stream before the bitmap's host
// copy could change.
static int set_state_eos(pocr_seq *s, StepState &hs, const int32_t *eos, int n_eos) {
    hs.eos_bits = nullptr;
    if (n_eos <= kMaxEos) {
        hs.n_eos = n_eos;
        for (int i = 0; i < kMaxEos; ++i) hs.eos[i] = i < n_eos ? eos[i] : 0;
        return POCR_OK;
    }
    const int vocab = s->m->cfg.vocab;
    const size_t words = ((size_t)vocab + 31) / 32;
    if (!s->eos_bits) HIP_TRY(hipMalloc((void **)&s->eos_bits, words * 4));
    std::vector<uint32_t> bits(words, 0u);
    for (int i = 0; i < n_eos; ++i)
        if (eos[i] < vocab) bits[(size_t)eos[i] >> 5] |= 1u << (eos[i] & 31);
    HIP_TRY(hipMemcpyAsync(s->eos_bits, bits.data(), words * 4, hipMemcpyHostToDevice, s->m->ctx->stream));
    HIP_TRY(hipStreamSynchronize(s->m->ctx->stream));
    hs.n_eos = 0;
    for (int i = 0; i < kMaxEos; ++i) hs.eos[i] = 0;
    hs.eos_bits = s->eos_bits;
    return POCR_OK;
}

// ValidateGenerateOptions (internal/model/model.go:461-467): at most
// maxEOSTokenIDs ids, none negative
static int check_eos(const char *fn, const int32_t *eos, int n_eos) {
    if (n_eos < 0 || (n_eos > 0 && !eos)) return fail(POCR_ERR_ARG, "%s: bad EOS list", fn);
    if (n_eos > kMaxEosIds)
        return fail(POCR_ERR_ARG, "%s: eos_token_ids length %d exceeds limit %d", fn, n_eos, kMaxEosIds);
    for (int i = 0; i < n_eos; ++i)
        if (eos[i] < 0) return fail(POCR_ERR_ARG, "%s: eos_token_ids must not contain negative ids", fn);
    return POCR_OK;
}

static bool state_failed(const StepState &hs) { return hs.err != 0 && hs.err != kErrStopped; }

// The generation loop ended at an EOS token, output index `index` (the first
// token is index 0): the reference ran no step for it, so the cache holds the
// rows of tokens 0..index-1 (model.go:1538-1548).  Rows later steps of the
// chunk appended are dropped and the state is cleared (a stopped state would
// turn the sequence's next step into a no-op).
static int end_at_eos(pocr_seq *s, int start_len, int index) { return seq_set_state(s, start_len + index); }

// Greedy decode loop (model.go:1538-1568) with the step graph replayed on the
// device.  The step prologue stops the loop at an EOS token (later replays of
// the chunk do nothing); the host reads the tokens every `batch` steps.
static int decode_locked(pocr_seq *s, int32_t first_token, int32_t first_pos, int max_new, const int32_t *eos,
                         int n_eos, int32_t *out_tokens) {
    pocr_model *m = s->m;
    hipStream_t st = m->ctx->stream;
    if (max_new <= 0) return 0;
    if (first_token < 0 || first_token >= m->cfg.vocab) return fail(POCR_ERR_ARG, "decode: token out of vocab");
    const int steps_needed = max_new - 1;  // the last token needs no step
    if (s->len + steps_needed > s->cap)
        return fail(POCR_ERR_ARG, "decode: %d steps exceed capacity (%d of %d rows used)", steps_needed, s->len,
                    s->cap);
    // POCR_HIP_GRAPH=0 replays the same kernel sequence with direct launches
    // (profilers that cannot follow graph launches)
    const char *g_env = getenv("POCR_HIP_GRAPH");
    const bool use_graph = !(g_env && g_env[0] == '0');
    if (use_graph) RC(build_decode_graph_n(s));
    pocr_ctx *ctx = m->ctx;
    if (!ctx->readback)
        HIP_TRY(hipHostMalloc((void **)&ctx->readback, sizeof(StepState) + kDecodeSyncSteps * 4, hipHostMallocDefault));
    StepState hs;
    RC(read_state(s, &hs));
    const int start_len = hs.len;
    hs.err = 0;
    hs.n_out = 0;
    hs.next_pos = first_pos;
    RC(set_state_eos(s, hs, eos, n_eos));
    for (int i = 0; i < kArgSlots; ++i) hs.argmax_slot[i * kSlotPitch] = 0ull;
    hs.argmax_slot[0] = (1ull << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)first_token);
    HIP_TRY(hipMemcpyAsync(s->st, &hs, sizeof(hs), hipMemcpyHostToDevice, st));
    HIP_TRY(hipStreamSynchronize(st));  // hs is reused as a read-back target below
    int produced = 0;  // tokens known on the host
    int launched = 0;
    s->device_tokens = 0;
    StepState *rb_state = reinterpret_cast<StepState *>(ctx->readback);
    int32_t *rb_tok = reinterpret_cast<int32_t *>(ctx->readback + sizeof(StepState));
    while (launched < steps_needed) {
        const int n = std::min(kDecodeSyncSteps, steps_needed - launched);
        int i = 0;
        if (use_graph) {
            for (; i + kDecodeGraphSteps <= n; i += kDecodeGraphSteps) HIP_TRY(hipGraphLaunch(s->decode_exec_n, st));
            for (; i < n; ++i) HIP_TRY(hipGraphLaunch(s->decode_exec, st));
        } else {
            for (; i < n; ++i) RC(enqueue_step(s, 1, true, false));
        }
        launched += n;
        // the state and the tokens this batch can have taken (step j takes
        // token j at most: tokens [produced, launched)), one synchronization
        const int span = std::min(launched, s->max_tokens) - produced;
        if (span > kDecodeSyncSteps) return fail(POCR_ERR_DEVICE, "decode: %d tokens pending", span);
        HIP_TRY(hipMemcpyAsync(rb_state, s->st, sizeof(StepState), hipMemcpyDeviceToHost, st));
        if (span > 0)
            HIP_TRY(hipMemcpyAsync(rb_tok, s->tokens + produced, (size_t)span * 4, hipMemcpyDeviceToHost, st));
        HIP_TRY(hipStreamSynchronize(st));
        std::memcpy(&hs, rb_state, sizeof(StepState));
        s->device_tokens = hs.n_out;
        if (state_failed(hs)) return fail(POCR_ERR_DEVICE, "decode: device state error %d", hs.err);
        if (hs.n_out - produced > span) return fail(POCR_ERR_DEVICE, "decode: %d tokens after %d steps", hs.n_out, launched);
        for (int j = 0; produced < hs.n_out; ++produced, ++j) {
            out_tokens[produced] = rb_tok[j];
            if (is_eos(rb_tok[j], eos, n_eos)) {
                RC(end_at_eos(s, start_len, produced));
                return produced + 1;
            }
        }
    }
    // the token chosen by the last step
    out_tokens[produced] = (int32_t)(0xFFFFFFFFu - (uint32_t)(argmax_of(hs) & 0xFFFFFFFFull));
    ++produced;
    s->len = hs.len;
    return produced;
}

extern "C" int pocr_decode_greedy(pocr_seq *s, int32_t first_token, int32_t first_pos, int max_new,
                                  const int32_t *eos, int n_eos, int32_t *out_tokens) {
    if (!s || !out_tokens || (n_eos > 0 && !eos)) return fail(POCR_ERR_ARG, "pocr_decode_greedy: null argument");
    RC(check_eos("pocr_decode_greedy", eos, n_eos));
    RC(model_ready(s->m));
    CHECK_INJECT("decode");
    std::lock_guard<std::mutex> lk(s->m->ctx->mu);
    RC(seq_idle(s, "pocr_decode_greedy"));
    HIP_TRY(hipSetDevice(s->m->ctx->device));
    return decode_locked(s, first_token, first_pos, max_new, eos, n_eos, out_tokens);
}

// ---------------------------------------------------------------------------
// Batched greedy decode: up to kMaxBatch sequences of one model advance together.
// Every layer GEMV streams its weights once for all of them (NV activation
// vectors per pass, padded to 2 or 4), attention and its merge run in one
// launch each with the sequence in blockIdx.z, and each sequence keeps its own
// KV cache, step state and token buffer.  One step is captured into a HIP
// graph and replayed; the host reads the states back every 16 steps.
// ---------------------------------------------------------------------------
namespace {

// greedy sequences from which the LM head takes the digit-plane launch and the
// 16-vector head (k_head_digits + k_head_wide) instead of a 4-vector pass
constexpr int kBatchWideHeadMin = 3;

struct DecodeBatch {
    pocr_model *m = nullptr;
    int n = 0;    // sequences: the ng greedy ones first, then the sampling ones
    int ng = 0;
    int nv = 1;   // vectors per GEMV pass (n ≤ 4: n padded to 1, 2 or 4)
    int cap = 0;  // vector rows the buffers hold (≥ nv; kMaxBatch for the wide step)
    pocr_seq *seq[kMaxBatch] = {};
    float *h = nullptr, *v = nullptr, *qkv = nullptr, *ho = nullptr, *g = nullptr;
    StepState *pad = nullptr;  // step state of the padding vectors
    // digit planes of 16 rows, row scales and sums (the wide step, n > 4, and
    // the wide LM head from kBatchWideHeadMin rows), and the wide step's row
    // step states (the o_proj epilogue reads each sequence's clen)
    int8_t *xd = nullptr;
    float *xs = nullptr;
    int *xb = nullptr;
    StepState **rst = nullptr;
    float *logits = nullptr;  // [16][vocab] greedy rows of the MFMA LM head (vocab a multiple of 16)
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool owns = true;  // false: the vector buffers belong to a continuous batch
    ~DecodeBatch() {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        if (owns)
            for (void *p : {(void *)h, (void *)v, (void *)qkv, (void *)ho, (void *)g, (void *)pad, (void *)xd,
                            (void *)xs, (void *)xb, (void *)rst, (void *)logits})
                if (p) (void)hipFree(p);
    }
    StepState *st(int i) const { return i < n ? seq[i]->st : pad; }
};

// states of the vectors base .. base+3 of a GEMV pass; vectors at or past lim
// (padding, or rows outside the pass) take the dummy state
GemvNV batch_nv(const DecodeBatch &b, int x_stride, int o_stride, int base = 0, int lim = kMaxBatch) {
    GemvNV q{};
    q.x_stride = x_stride;
    q.o_stride = o_stride;
    for (int i = 1; i < kMaxNV; ++i) q.stv[i - 1] = base + i < lim ? b.st(base + i) : b.pad;
    return q;
}

// the batch's sequences in step order: greedy ones first (their LM head runs
// as 4-vector argmax passes over consecutive rows), then the sampling ones
void batch_order(DecodeBatch &b, pocr_seq *const *seqs, int n) {
    b.n = b.ng = 0;
    for (int i = 0; i < n; ++i)
        if (!seqs[i]->sampling) b.seq[b.n++] = seqs[i];
    b.ng = b.n;
    for (int i = 0; i < n; ++i)
        if (seqs[i]->sampling) b.seq[b.n++] = seqs[i];
}

// Sequences a batch step can take: up to 4 on the GEMV passes, up to 16 when
// every layer matrix fits the small MFMA GEMM (rows a multiple of 16, K a
// multiple of 256).
int batch_limit(const pocr_model *m) {
    const pocr_config &c = m->cfg;
    const int Q = c.heads * c.head_dim, KV = c.kv_heads * c.head_dim;
    const bool wide = gemm_small_ok(Q + 2 * KV, c.hidden) && Q % 16 == 0 && KV % 16 == 0 &&
                      gemm_small_ok(c.hidden, Q) && gemm_small_ok(c.intermediate, c.hidden) &&
                      gemm_small_ok(c.hidden, c.intermediate);
    return wide ? kMaxBatch : kMaxNV;
}

// digit planes of the batch's n rows of x (RMSNorm·norm_w first if norm_w)
int batch_digitize(const DecodeBatch &b, int qtype, const float *x, int K, const float *norm_w) {
    DigitizeParams d{};
    d.x = x;
    d.x_stride = K;
    d.norm_w = norm_w;
    d.eps = b.m->cfg.rms_norm_eps;
    d.K = K;
    d.xd = b.xd;
    d.plane_stride = (size_t)16 * K;
    d.xs = b.xs;
    d.xb = b.xb;
    return digitize_rows(b.m->ctx->stream, qtype, d, b.n);
}

GemmParams batch_gemm(const DecodeBatch &b, const pocr_weight *w, int K) {
    GemmParams p{};
    p.m[0] = p.m[1] = p.m[2] = dev_mat(w);
    p.seg_end[0] = p.seg_end[1] = p.seg_end[2] = w->rows;
    p.rows = w->rows;
    p.K = K;
    p.xd = b.xd;
    p.plane_stride = (size_t)16 * K;
    p.xs = b.xs;
    p.xb = b.xb;
    p.ntok = b.n;
    p.rst = b.rst;
    return p;
}

// One layer of the wide step (5..16 sequences): digit planes of the rows,
// then the small MFMA GEMM with the prefill epilogues (each row a sequence);
// attention and its merge as in the narrow step.
int batch_layer_wide(DecodeBatch &b, const LayerW &L, int li, bool last, int rpw, int max_split) {
    pocr_model *m = b.m;
    const pocr_config &c = m->cfg;
    hipStream_t st = m->ctx->stream;
    const int H = c.hidden, Q = c.heads * c.head_dim, KV = c.kv_heads * c.head_dim, F = c.intermediate;
    const int QKV = Q + 2 * KV;
    const int qt = L.w[POCR_W_Q]->qtype;
    // 1. RMSNorm(h)·ln1 → q|k|v
    RC(batch_digitize(b, qt, b.h, H, L.ln1));
    GemmParams g = batch_gemm(b, L.w[POCR_W_Q], H);
    g.m[1] = dev_mat(L.w[POCR_W_K]);
    g.m[2] = dev_mat(L.w[POCR_W_V]);
    g.seg_end[0] = Q;
    g.seg_end[1] = Q + KV;
    g.seg_end[2] = QKV;
    g.rows = QKV;
    g.out = b.qkv;
    g.out_stride = QKV;
    RC(gemm_small_rows(st, qt, 1, g, G_PLAIN));
    // 2. RoPE + KV append + split attention, then the merge
    AttnMulti am{};
    for (int i = 0; i < b.n; ++i) {
        pocr_seq *s = b.seq[i];
        AttnParams &a = am.a[i];
        a.q = b.qkv + (size_t)i * QKV;
        a.k_new = a.q + Q;
        a.v_new = a.q + Q + KV;
        a.kc = layer_k(s, li);
        a.vc = layer_v(s, li);
        a.st = s->st;
        a.part = s->part;
        a.head_out = b.ho + (size_t)i * Q;
        a.heads = c.heads;
        a.kvh = c.kv_heads;
        attn_shape(a, s->cap, rpw);
        a.scale = (float)(1.0 / std::sqrt((double)c.head_dim));
    }
    const dim3 ag(c.kv_heads, max_split, b.n);
    if (rpw == 8) hipLaunchKernelGGL(k_attn_decode_multi<8>, ag, dim3(kThreads), 0, st, am);
    else hipLaunchKernelGGL(k_attn_decode_multi<16>, ag, dim3(kThreads), 0, st, am);
    launch_attn_merge_multi(st, dim3(c.heads, 1, b.n), max_split, am);
    HIP_TRY(hipGetLastError());
    // 3. o_proj + residual (+ the Q4/Q6 behaviour by each sequence's clen)
    const pocr_weight *wo = L.w[POCR_W_O];
    RC(batch_digitize(b, wo->qtype, b.ho, Q, nullptr));
    GemmParams o = batch_gemm(b, wo, Q);
    o.h = b.h;
    o.vbuf = b.v;
    o.quirk = (m->quirk && (wo->qtype == POCR_Q4 || wo->qtype == POCR_Q6)) ? 1 : 0;
    RC(gemm_small_rows(st, wo->qtype, 1, o, G_OPROJ));
    // 4. RMSNorm(v)·ln2 → gate/up → SiLU(g)·u
    const pocr_weight *wg = L.w[POCR_W_GATE];
    RC(batch_digitize(b, wg->qtype, b.v, H, L.ln2));
    GemmParams gu = batch_gemm(b, wg, H);
    gu.m[1] = dev_mat(L.w[POCR_W_UP]);
    gu.out = b.g;
    gu.out_stride = F;
    RC(gemm_small_rows(st, wg->qtype, 2, gu, G_SWIGLU));
    // 5. down + residual; last layer: v = h + down
    const pocr_weight *wd = L.w[POCR_W_DOWN];
    RC(batch_digitize(b, wd->qtype, b.g, F, nullptr));
    GemmParams d = batch_gemm(b, wd, F);
    d.h = b.h;
    d.vbuf = b.v;
    d.last = last ? 1 : 0;
    return gemm_small_rows(st, wd->qtype, 1, d, G_DOWN);
}

int enqueue_batch_step(DecodeBatch &b) {
    pocr_model *m = b.m;
    const pocr_config &c = m->cfg;
    hipStream_t st = m->ctx->stream;
    const int H = c.hidden, Q = c.heads * c.head_dim, KV = c.kv_heads * c.head_dim, F = c.intermediate;
    const int QKV = Q + 2 * KV;
    const float eps = c.rms_norm_eps;
    StepBatch sb{};
    for (int i = 0; i < b.n; ++i) {
        sb.st[i] = b.seq[i]->st;
        sb.tokens[i] = b.seq[i]->tokens;
        sb.max_tokens[i] = b.seq[i]->max_tokens;
    }
    hipLaunchKernelGGL(k_step_begin_multi, dim3(b.n), dim3(kThreads), 0, st, sb, m->embed, b.h, H, c.vocab, m->freq,
                       m->axis);
    HIP_TRY(hipGetLastError());
    // one rows-per-wave for all: the largest the sequences' capacities pick
    // (no more splits than any sequence's records were sized for)
    int rpw = 8, max_split = 1;
    for (int i = 0; i < b.n; ++i) rpw = std::max(rpw, b.seq[i]->rpw);
    for (int i = 0; i < b.n; ++i) max_split = std::max(max_split, attn_nsplit(b.seq[i]->cap, rpw));
    const bool wide = b.n > kMaxNV;
    for (int li = 0; li < c.layers; ++li) {
        const LayerW &L = m->layers[li];
        const bool last = li + 1 == c.layers;
        if (wide) {
            RC(batch_layer_wide(b, L, li, last, rpw, max_split));
            continue;
        }
        // 1. RMSNorm(h)·ln1 → q|k|v for every sequence
        GemvParams p{};
        p.m[0] = dev_mat(L.w[POCR_W_Q]);
        p.m[1] = dev_mat(L.w[POCR_W_K]);
        p.m[2] = dev_mat(L.w[POCR_W_V]);
        p.seg_end[0] = Q;
        p.seg_end[1] = Q + KV;
        p.seg_end[2] = QKV;
        p.rows = QKV;
        p.cols = H;
        p.x = b.h;
        p.norm_w = L.ln1;
        p.eps = eps;
        p.out = b.qkv;
        p.st = b.st(0);
        GemvNV q = batch_nv(b, H, QKV);
        RC(gemv_launch(st, p, 1, PRO_RMSNORM, EPI_PLAIN, kBigGrid, b.nv, &q));
        // 2. per sequence: RoPE + KV append + split attention, then the merge
        AttnMulti am{};
        for (int i = 0; i < b.n; ++i) {
            pocr_seq *s = b.seq[i];
            AttnParams &a = am.a[i];
            a.q = b.qkv + (size_t)i * QKV;
            a.k_new = a.q + Q;
            a.v_new = a.q + Q + KV;
            a.kc = layer_k(s, li);
            a.vc = layer_v(s, li);
            a.st = s->st;
            a.part = s->part;
            a.head_out = b.ho + (size_t)i * Q;
            a.heads = c.heads;
            a.kvh = c.kv_heads;
            attn_shape(a, s->cap, rpw);
            a.scale = (float)(1.0 / std::sqrt((double)c.head_dim));
        }
        const dim3 ag(c.kv_heads, max_split, b.n);
        if (rpw == 8) hipLaunchKernelGGL(k_attn_decode_multi<8>, ag, dim3(kThreads), 0, st, am);
        else hipLaunchKernelGGL(k_attn_decode_multi<16>, ag, dim3(kThreads), 0, st, am);
        launch_attn_merge_multi(st, dim3(c.heads, 1, b.n), max_split, am);
        HIP_TRY(hipGetLastError());
        // 3. o_proj + residual (+ the Q4/Q6 behaviour per sequence)
        const pocr_weight *wo = L.w[POCR_W_O];
        GemvParams o = gemv_params_1(wo);
        o.x = b.ho;
        o.residual = b.h;
        o.vbuf = b.v;
        o.st = b.st(0);
        o.quirk = (m->quirk && (wo->qtype == POCR_Q4 || wo->qtype == POCR_Q6)) ? 1 : 0;
        q = batch_nv(b, Q, H);
        RC(gemv_launch(st, o, 1, PRO_COPY, EPI_OPROJ, kBigGrid, b.nv, &q));
        // 4. RMSNorm(v)·ln2 → gate/up → SiLU(g)·u
        GemvParams gu = gemv_params_1(L.w[POCR_W_GATE]);
        gu.m[1] = dev_mat(L.w[POCR_W_UP]);
        gu.x = b.v;
        gu.norm_w = L.ln2;
        gu.eps = eps;
        gu.out = b.g;
        gu.st = b.st(0);
        q = batch_nv(b, H, F);
        RC(gemv_launch(st, gu, 2, PRO_RMSNORM, EPI_SWIGLU, kBigGrid, b.nv, &q));
        // 5. down + residual; last layer: v = h + down
        GemvParams d = gemv_params_1(L.w[POCR_W_DOWN]);
        d.x = b.g;
        d.residual = b.h;
        d.vbuf = b.v;
        d.st = b.st(0);
        d.flag = last ? 1 : 0;
        q = batch_nv(b, F, H);
        RC(gemv_launch(st, d, 1, PRO_COPY, EPI_DOWN, kBigGrid, b.nv, &q));
    }
    // LM head on RMSNorm(v)·final_norm.  Greedy sequences: argmax into each
    // one's state — from kBatchWideHeadMin of them and a head the wide kernels
    // take: one digit-plane launch and one 16-vector head for all; more than 4
    // of them otherwise (and a vocabulary in 16-row blocks): digit planes, the
    // small MFMA GEMM into logits rows and a per-row argmax; otherwise one GEMV
    // pass per 4 of them (the last pass padded to 1, 2 or 4 vectors).
    // Sampling sequences: each its own logits, top-k and draw (the draw lands
    // in argmax slot 0, where the next step reads it).
    const bool head_wide = b.ng >= kBatchWideHeadMin && b.xd && head_wide_ok(m->lm);
    if (head_wide) {
        // one launch for every greedy sequence (rows 0..ng-1 of v)
        StepState *sts[kHeadWideVec];
        for (int i = 0; i < b.ng; ++i) sts[i] = b.seq[i]->st;
        RC(launch_head_wide(st, m->lm, b.v, H, b.ng, m->final_norm, eps, nullptr, 0, sts, b.xd, b.xs, b.xb));
    } else if (wide && b.ng > kMaxNV && b.logits) {
        const int V = c.vocab;
        RC(batch_digitize(b, m->lm->qtype, b.v, H, m->final_norm));
        GemmParams lp = batch_gemm(b, m->lm, H);
        lp.ntok = b.ng;
        lp.out = b.logits;
        lp.out_stride = V;
        RC(gemm_small_rows(st, m->lm->qtype, 1, lp, G_PLAIN));
        constexpr int kSlice = 2048;
        hipLaunchKernelGGL(k_argmax_rows, dim3((V + kSlice - 1) / kSlice, b.ng), dim3(kThreads), 0, st, b.logits, V, V,
                           kSlice, b.rst);
        HIP_TRY(hipGetLastError());
    }
    for (int base = 0; base < b.ng && !head_wide && !(wide && b.ng > kMaxNV && b.logits); base += kMaxNV) {
        const int left = b.ng - base;
        const int nv = left == 1 ? 1 : (left == 2 ? 2 : 4);
        GemvParams lm = gemv_params_1(m->lm);
        lm.x = b.v + (size_t)base * H;
        lm.norm_w = m->final_norm;
        lm.eps = eps;
        lm.st = b.st(base);
        GemvNV q = batch_nv(b, H, 0, base, b.ng);
        RC(gemv_launch(st, lm, 1, PRO_RMSNORM, EPI_ARGMAX, kBigGrid, nv, &q));
    }
    for (int i = b.ng; i < b.n; ++i) RC(enqueue_lm_head(b.seq[i], b.v + (size_t)i * H, false));
    return POCR_OK;
}

// the first token of a batched decode sits in the argmax slots as if the
// previous step had chosen it (the step prologue reads it from there)
int seed_first_token(pocr_seq *s, int32_t first_token, int32_t first_pos, const int32_t *eos, int n_eos,
                     StepState &hs) {
    RC(read_state(s, &hs));
    hs.err = 0;
    hs.n_out = 0;
    hs.next_pos = first_pos;
    RC(set_state_eos(s, hs, eos, n_eos));
    for (int k = 0; k < kArgSlots; ++k) hs.argmax_slot[k * kSlotPitch] = 0ull;
    hs.argmax_slot[0] = (1ull << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)first_token);
    HIP_TRY(hipMemcpyAsync(s->st, &hs, sizeof(StepState), hipMemcpyHostToDevice, s->m->ctx->stream));
    HIP_TRY(hipStreamSynchronize(s->m->ctx->stream));
    return POCR_OK;
}

int32_t pending_token(const StepState &hs) {
    return (int32_t)(0xFFFFFFFFu - (uint32_t)(argmax_of(hs) & 0xFFFFFFFFull));
}

// vector buffers for b.cap rows; from kBatchWideHeadMin rows also digit planes
// (16 rows of the widest input), with cap > 4 the wide step's row-state table
int batch_alloc(DecodeBatch &b) {
    const pocr_config &c = b.m->cfg;
    const size_t H = c.hidden, Q = (size_t)c.heads * c.head_dim, KV = (size_t)c.kv_heads * c.head_dim;
    const size_t rows = std::max(b.cap, b.nv);
    hipStream_t s = b.m->ctx->stream;
    for (auto pr : {std::make_pair(&b.h, H), std::make_pair(&b.v, H), std::make_pair(&b.qkv, Q + 2 * KV),
                    std::make_pair(&b.ho, Q), std::make_pair(&b.g, (size_t)c.intermediate)}) {
        HIP_TRY(hipMalloc(pr.first, rows * pr.second * 4));
        // padding rows stay finite zeros (their results are never read)
        HIP_TRY(hipMemsetAsync(*pr.first, 0, rows * pr.second * 4, s));
    }
    HIP_TRY(hipMalloc(&b.pad, sizeof(StepState)));
    HIP_TRY(hipMemsetAsync(b.pad, 0, sizeof(StepState), s));
    if (rows >= (size_t)kBatchWideHeadMin) {
        const size_t kmax = std::max(std::max(H, Q), (size_t)c.intermediate);
        HIP_TRY(hipMalloc(&b.xd, 3 * 16 * kmax));
        HIP_TRY(hipMemsetAsync(b.xd, 0, 3 * 16 * kmax, s));
        HIP_TRY(hipMalloc(&b.xs, 16 * sizeof(float)));
        HIP_TRY(hipMalloc(&b.xb, 16 * 4 * sizeof(int)));
    }
    if (rows > (size_t)kMaxNV) {
        HIP_TRY(hipMalloc(&b.rst, kMaxBatch * sizeof(StepState *)));
        if (gemm_small_ok(c.vocab, c.hidden)) HIP_TRY(hipMalloc(&b.logits, (size_t)16 * c.vocab * 4));
    }
    return POCR_OK;
}

// the row-state table of a wide step (rows = sequences), before its capture
int batch_set_rows(DecodeBatch &b) {
    if (b.n <= kMaxNV) return POCR_OK;
    StepState *h[kMaxBatch] = {};
    for (int i = 0; i < b.n; ++i) h[i] = b.seq[i]->st;
    HIP_TRY(hipMemcpy(b.rst, h, sizeof(h), hipMemcpyHostToDevice));
    return POCR_OK;
}

}  // namespace

extern "C" int pocr_decode_batch(pocr_seq *const *seqs, int n_seq, const int32_t *first_tokens,
                                 const int32_t *first_positions, int max_new, const int32_t *eos, int n_eos,
                                 int32_t *out_tokens, int32_t *out_counts) {
    if (!seqs || n_seq <= 0 || n_seq > kMaxBatch || !first_tokens || !first_positions || !out_tokens || !out_counts ||
        (n_eos > 0 && !eos))
        return fail(POCR_ERR_ARG, "pocr_decode_batch: bad arguments (1..%d sequences)", kMaxBatch);
    RC(check_eos("pocr_decode_batch", eos, n_eos));
    pocr_model *m = seqs[0] ? seqs[0]->m : nullptr;
    for (int i = 0; i < n_seq; ++i) {
        if (!seqs[i] || seqs[i]->m != m) return fail(POCR_ERR_ARG, "pocr_decode_batch: sequences of one model");
        for (int j = 0; j < i; ++j)
            if (seqs[j] == seqs[i]) return fail(POCR_ERR_ARG, "pocr_decode_batch: sequence %d repeated", i);
        if (first_tokens[i] < 0 || first_tokens[i] >= m->cfg.vocab)
            return fail(POCR_ERR_ARG, "pocr_decode_batch: token out of vocab");
    }
    for (int i = 0; i < n_seq; ++i) out_counts[i] = 0;
    if (max_new <= 0) return POCR_OK;
    RC(model_ready(m));
    CHECK_INJECT("decode_batch");
    std::lock_guard<std::mutex> lk(m->ctx->mu);
    for (int i = 0; i < n_seq; ++i) RC(seq_idle(seqs[i], "pocr_decode_batch"));
    HIP_TRY(hipSetDevice(m->ctx->device));
    hipStream_t st = m->ctx->stream;
    const int steps_needed = max_new - 1;
    for (int i = 0; i < n_seq; ++i)
        if (seqs[i]->len + steps_needed > seqs[i]->cap || max_new > seqs[i]->max_tokens)
            return fail(POCR_ERR_ARG, "pocr_decode_batch: sequence %d: %d steps exceed capacity", i, steps_needed);
    // VNNI mode: each member runs its own decode loop of the mode's
    // single-sequence step (the members are independent, so their streams
    // are what decoding each alone gives, as the reference's server computes
    // them: one request per goroutine)
    if (m->vnni) {
        for (int i = 0; i < n_seq; ++i) {
            const int n = decode_locked(seqs[i], first_tokens[i], first_positions[i], max_new, eos, n_eos,
                                        out_tokens + (size_t)i * max_new);
            if (n < 0) return n;
            out_counts[i] = n;
        }
        return POCR_OK;
    }
    DecodeBatch b;
    b.m = m;
    b.n = n_seq;
    if (n_seq > batch_limit(m))
        return fail(POCR_ERR_UNSUPPORTED, "pocr_decode_batch: %d sequences need layer shapes the small GEMM takes", n_seq);
    b.nv = n_seq == 1 ? 1 : (n_seq == 2 ? 2 : 4);
    b.cap = n_seq;
    batch_order(b, seqs, n_seq);
    RC(batch_alloc(b));
    RC(batch_set_rows(b));
    // per-sequence state: the first token sits in the argmax slots as if the
    // previous step had chosen it (the step prologue reads it from there)
    std::vector<StepState> hs(n_seq);
    std::vector<int> start_len(n_seq);
    for (int i = 0; i < n_seq; ++i) {
        start_len[i] = seqs[i]->len;
        RC(seed_first_token(seqs[i], first_tokens[i], first_positions[i], eos, n_eos, hs[i]));
    }
    const char *g_env = getenv("POCR_HIP_GRAPH");
    const bool use_graph = !(g_env && g_env[0] == '0');
    if (use_graph) {
        HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        const int rc = enqueue_batch_step(b);
        const hipError_t e = hipStreamEndCapture(st, &b.graph);
        if (rc != POCR_OK) return rc;
        if (e != hipSuccess) return fail(POCR_ERR_DEVICE, "graph capture: %s", hipGetErrorString(e));
        HIP_TRY(hipGraphInstantiate(&b.exec, b.graph, nullptr, nullptr, 0));
    }
    std::vector<int> produced(n_seq, 0);
    std::vector<char> done(n_seq, 0);
    std::vector<int32_t> tok;
    int launched = 0;
    const int batch = 16;
    while (launched < steps_needed) {
        const int k = std::min(batch, steps_needed - launched);
        for (int i = 0; i < k; ++i) {
            if (use_graph) HIP_TRY(hipGraphLaunch(b.exec, st));
            else RC(enqueue_batch_step(b));
        }
        launched += k;
        bool all_done = true;
        for (int i = 0; i < n_seq; ++i) {
            RC(read_state(seqs[i], &hs[i]));
            if (done[i]) continue;
            if (state_failed(hs[i]))
                return fail(POCR_ERR_DEVICE, "decode_batch: sequence %d: device state error %d", i, hs[i].err);
            tok.resize(hs[i].n_out);
            HIP_TRY(hipMemcpy(tok.data(), seqs[i]->tokens, (size_t)hs[i].n_out * 4, hipMemcpyDeviceToHost));
            for (; produced[i] < hs[i].n_out && !done[i]; ++produced[i]) {
                out_tokens[(size_t)i * max_new + produced[i]] = tok[produced[i]];
                if (is_eos(tok[produced[i]], eos, n_eos)) done[i] = 1;
            }
            all_done = all_done && done[i];
        }
        if (all_done) break;
    }
    for (int i = 0; i < n_seq; ++i) {
        seqs[i]->device_tokens = hs[i].n_out;
        if (!done[i]) {  // the token chosen by the last step
            out_tokens[(size_t)i * max_new + produced[i]] = pending_token(hs[i]);
            ++produced[i];
            seqs[i]->len = hs[i].len;
        } else {
            RC(end_at_eos(seqs[i], start_len[i], produced[i] - 1));
        }
        out_counts[i] = produced[i];
    }
    return POCR_OK;
}

// ---------------------------------------------------------------------------
// Continuous batching: members join and leave between token steps.  The
// device set (members still decoding) is captured into one batched step graph,
// captured again whenever the set changes; the vector buffers are allocated
// once for the batch's limit of vectors.  A member decodes from its seeded first token until
// an EOS id or its token budget; steps are issued in chunks no longer than any
// member's remaining budget, so no cache grows past what its join checked.
// ---------------------------------------------------------------------------
struct pocr_batch {
    struct Member {
        pocr_seq *s = nullptr;
        int max_new = 0;
        int steps = 0;                // device steps run
        std::vector<int32_t> eos;
        std::vector<int32_t> out;     // tokens produced, first token first
        int start_len = 0;            // cache rows at the join
        bool finished = false;
    };
    pocr_model *m = nullptr;
    std::vector<Member> members;      // join order
    DecodeBatch bufs;                 // owns the vector buffers (limit rows)
    int limit = kMaxNV;               // members decoding at once
    std::unique_ptr<DecodeBatch> cur; // the captured device set, null when stale
    bool use_graph = true;
};

static void batch_forget(pocr_batch *b, const pocr_seq *s) {
    for (size_t i = 0; i < b->members.size(); ++i)
        if (b->members[i].s == s) {
            if (!b->members[i].finished) b->cur.reset();
            b->members.erase(b->members.begin() + (long)i);
            break;
        }
    const_cast<pocr_seq *>(s)->batch = nullptr;
}

extern "C" int pocr_batch_create(pocr_model *m, pocr_batch **out) {
    if (!m || !out) return fail(POCR_ERR_ARG, "pocr_batch_create: null argument");
    *out = nullptr;
    CHECK_INJECT("batch");
    std::lock_guard<std::mutex> lk(m->ctx->mu);
    HIP_TRY(hipSetDevice(m->ctx->device));
    pocr_batch *b = new pocr_batch();
    b->m = m;
    b->bufs.m = m;
    b->limit = batch_limit(m);
    b->bufs.nv = kMaxNV;
    b->bufs.cap = b->limit;
    const int rc = batch_alloc(b->bufs);
    if (rc == POCR_OK) {
        const hipError_t e = hipStreamSynchronize(m->ctx->stream);
        if (e != hipSuccess) {
            delete b;
            return fail(POCR_ERR_DEVICE, "pocr_batch_create: %s", hipGetErrorString(e));
        }
    }
    if (rc != POCR_OK) {
        delete b;
        return rc;
    }
    const char *g_env = getenv("POCR_HIP_GRAPH");
    b->use_graph = !(g_env && g_env[0] == '0');
    m->refs.fetch_add(1);
    *out = b;
    return POCR_OK;
}

extern "C" void pocr_batch_destroy(pocr_batch *b) {
    if (!b) return;
    pocr_model *m = b->m;
    {
        std::lock_guard<std::mutex> lk(m->ctx->mu);
        (void)hipSetDevice(m->ctx->device);
        (void)hipStreamSynchronize(m->ctx->stream);
        for (auto &mb : b->members) mb.s->batch = nullptr;
        delete b;
    }
    model_release(m);
}

extern "C" int pocr_batch_join(pocr_batch *b, pocr_seq *s, int32_t first_token, int32_t first_pos, int max_new,
                               const int32_t *eos, int n_eos) {
    if (!b || !s || max_new <= 0 || n_eos < 0 || (n_eos > 0 && !eos))
        return fail(POCR_ERR_ARG, "pocr_batch_join: bad arguments");
    RC(check_eos("pocr_batch_join", eos, n_eos));
    if (s->m != b->m) return fail(POCR_ERR_ARG, "pocr_batch_join: the sequence belongs to another model");
    if (first_token < 0 || first_token >= b->m->cfg.vocab) return fail(POCR_ERR_ARG, "pocr_batch_join: token out of vocab");
    RC(model_ready(b->m));
    CHECK_INJECT("batch_join");
    std::lock_guard<std::mutex> lk(b->m->ctx->mu);
    HIP_TRY(hipSetDevice(b->m->ctx->device));
    if (s->batch) return fail(POCR_ERR_ARG, "pocr_batch_join: the sequence is already in a decode batch");
    int decoding = 0;
    for (const auto &mb : b->members) decoding += mb.finished ? 0 : 1;
    if (decoding >= b->limit) return fail(POCR_ERR_ARG, "pocr_batch_join: %d members are decoding", b->limit);
    if (s->len + max_new - 1 > s->cap || max_new > s->max_tokens)
        return fail(POCR_ERR_ARG, "pocr_batch_join: %d tokens exceed the capacity", max_new);
    pocr_batch::Member mb;
    mb.s = s;
    mb.max_new = max_new;
    mb.eos.assign(eos, eos + n_eos);
    mb.start_len = s->len;
    if (max_new == 1 || is_eos(first_token, eos, n_eos)) {
        mb.out.push_back(first_token);  // done before any device step
        mb.finished = true;
    } else {
        StepState hs;
        RC(seed_first_token(s, first_token, first_pos, eos, n_eos, hs));
        b->cur.reset();
    }
    s->batch = b;
    b->members.push_back(std::move(mb));
    return POCR_OK;
}

static int batch_capture(pocr_batch *b) {
    auto d = std::make_unique<DecodeBatch>();
    d->m = b->m;
    d->owns = false;
    pocr_seq *dec[kMaxBatch];
    int nd = 0;
    for (auto &mb : b->members)
        if (!mb.finished) dec[nd++] = mb.s;
    batch_order(*d, dec, nd);
    d->nv = d->n == 1 ? 1 : (d->n == 2 ? 2 : 4);
    d->cap = b->bufs.cap;
    d->h = b->bufs.h;
    d->v = b->bufs.v;
    d->qkv = b->bufs.qkv;
    d->ho = b->bufs.ho;
    d->g = b->bufs.g;
    d->pad = b->bufs.pad;
    d->xd = b->bufs.xd;
    d->xs = b->bufs.xs;
    d->xb = b->bufs.xb;
    d->rst = b->bufs.rst;
    d->logits = b->bufs.logits;
    RC(batch_set_rows(*d));
    if (b->use_graph) {
        hipStream_t st = b->m->ctx->stream;
        HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        const int rc = enqueue_batch_step(*d);
        const hipError_t e = hipStreamEndCapture(st, &d->graph);
        if (rc != POCR_OK) return rc;
        if (e != hipSuccess) return fail(POCR_ERR_DEVICE, "graph capture: %s", hipGetErrorString(e));
        HIP_TRY(hipGraphInstantiate(&d->exec, d->graph, nullptr, nullptr, 0));
    }
    b->cur = std::move(d);
    return POCR_OK;
}

extern "C" int pocr_batch_step(pocr_batch *b, int max_steps) {
    if (!b || max_steps <= 0) return fail(POCR_ERR_ARG, "pocr_batch_step: bad arguments");
    CHECK_INJECT("batch_step");
    std::lock_guard<std::mutex> lk(b->m->ctx->mu);
    HIP_TRY(hipSetDevice(b->m->ctx->device));
    int k = max_steps, decoding = 0;
    for (const auto &mb : b->members)
        if (!mb.finished) {
            k = std::min(k, mb.max_new - 1 - mb.steps);  // >= 1: a member at its budget has finished
            ++decoding;
        }
    if (decoding == 0) return 0;
    hipStream_t st = b->m->ctx->stream;
    if (b->m->vnni) {
        // VNNI mode: every decoding member takes k steps of the mode's
        // single-sequence step graph (its state and token list advance as
        // under the batched step)
        for (auto &mb : b->members) {
            if (mb.finished) continue;
            if (b->use_graph) RC(build_decode_graph(mb.s));
            for (int i = 0; i < k; ++i) {
                if (b->use_graph) HIP_TRY(hipGraphLaunch(mb.s->decode_exec, st));
                else RC(enqueue_step(mb.s, 1, true, false));
            }
        }
    } else {
        if (!b->cur) RC(batch_capture(b));
        for (int i = 0; i < k; ++i) {
            if (b->use_graph) HIP_TRY(hipGraphLaunch(b->cur->exec, st));
            else RC(enqueue_batch_step(*b->cur));
        }
    }
    StepState hs;
    std::vector<int32_t> tok;
    decoding = 0;
    for (auto &mb : b->members) {
        if (mb.finished) continue;
        RC(read_state(mb.s, &hs));
        if (state_failed(hs)) return fail(POCR_ERR_DEVICE, "pocr_batch_step: device state error %d", hs.err);
        mb.s->len = hs.len;
        mb.steps += k;
        // tokens the steps appended (the first one is the seeded first token)
        tok.resize(hs.n_out);
        if (hs.n_out > (int)mb.out.size())
            HIP_TRY(hipMemcpy(tok.data(), mb.s->tokens, (size_t)hs.n_out * 4, hipMemcpyDeviceToHost));
        for (int t = (int)mb.out.size(); t < hs.n_out && !mb.finished; ++t) {
            mb.out.push_back(tok[t]);
            mb.finished = is_eos(tok[t], mb.eos.data(), (int)mb.eos.size());
            if (mb.finished) RC(end_at_eos(mb.s, mb.start_len, t));
        }
        // the token the last step chose ends the member at its budget or an EOS
        if (!mb.finished) {
            const int32_t next = pending_token(hs);
            if (mb.steps == mb.max_new - 1 || is_eos(next, mb.eos.data(), (int)mb.eos.size())) {
                mb.out.push_back(next);
                mb.finished = true;
            }
        }
        if (mb.finished) b->cur.reset();
        else ++decoding;
    }
    return decoding;
}

extern "C" int pocr_batch_poll(pocr_batch *b, const pocr_seq *s, int *finished) {
    if (!b || !s) return fail(POCR_ERR_ARG, "pocr_batch_poll: null argument");
    std::lock_guard<std::mutex> lk(b->m->ctx->mu);
    for (const auto &mb : b->members)
        if (mb.s == s) {
            if (finished) *finished = mb.finished ? 1 : 0;
            return (int)mb.out.size();
        }
    return fail(POCR_ERR_ARG, "pocr_batch_poll: the sequence is not in this batch");
}

extern "C" int pocr_batch_leave(pocr_batch *b, pocr_seq *s, int32_t *out_tokens, int cap) {
    if (!b || !s || cap < 0 || (cap > 0 && !out_tokens)) return fail(POCR_ERR_ARG, "pocr_batch_leave: bad arguments");
    std::lock_guard<std::mutex> lk(b->m->ctx->mu);
    for (const auto &mb : b->members)
        if (mb.s == s) {
            const int n = (int)mb.out.size();
            std::copy(mb.out.begin(), mb.out.begin() + std::min(n, cap), out_tokens);
            batch_forget(b, s);
            return n;
        }
    return fail(POCR_ERR_ARG, "pocr_batch_leave: the sequence is not in this batch");
}

extern "C" int pocr_prefill(pocr_seq *s, int n, const float *emb, const int32_t *pos3, float *logits,
                            int32_t *token) {
    if (!s || !emb || !pos3 || n <= 0) return fail(POCR_ERR_ARG, "pocr_prefill: bad arguments");
    RC(model_ready(s->m));
    CHECK_INJECT("prefill");
    std::lock_guard<std::mutex> lk(s->m->ctx->mu);
    RC(seq_idle(s, "pocr_prefill"));
    HIP_TRY(hipSetDevice(s->m->ctx->device));
    if (s->len + n > s->cap) return fail(POCR_ERR_ARG, "pocr_prefill: %d rows exceed capacity", n);
    return prefill_locked(s, n, emb, pos3, logits, token);
}

extern "C" int pocr_generate(pocr_seq *s, const int32_t *ids, int n_ids, const float *image_embeds, int n_image,
                             int32_t image_token_id, const int32_t grid[3], int32_t merge, int max_new,
                             const int32_t *eos, int n_eos, int use_prefill, int32_t *out_tokens) {
    if (!s || !ids || n_ids <= 0 || !out_tokens || (n_image > 0 && (!image_embeds || !grid)))
        return fail(POCR_ERR_ARG, "pocr_generate: bad arguments");
    RC(check_eos("pocr_generate", eos, n_eos));
    if (max_new <= 0) return 0;
    RC(model_ready(s->m));
    CHECK_INJECT("generate");
    std::lock_guard<std::mutex> lk(s->m->ctx->mu);
    RC(seq_idle(s, "pocr_generate"));
    HIP_TRY(hipSetDevice(s->m->ctx->device));
    return generate_locked(s, ids, n_ids, image_embeds, false, n_image, image_token_id, grid, merge, max_new, eos,
                           n_eos, use_prefill, out_tokens);
}

int pocr::generate_locked(pocr_seq *s, const int32_t *ids, int n_ids, const float *image_embeds, bool image_dev,
                          int n_image, int32_t image_token_id, const int32_t grid[3], int32_t merge, int max_new,
                          const int32_t *eos, int n_eos, int use_prefill, int32_t *out_tokens) {
    pocr_model *m = s->m;
    const int H = m->cfg.hidden;
    // positions (model.go:1717-1783) and embeddings (tokenEmbeddingInto 3251 /
    // image rows substituted for placeholders 1646-1652)
    std::vector<int32_t> pos((size_t)n_ids * 3);
    int32_t rope_delta = 0;
    if (n_image > 0) {
        int np = pocr_mm_positions(ids, n_ids, image_token_id, grid, merge, pos.data(), &rope_delta);
        if (np != n_ids) return fail(POCR_ERR_ARG, "pocr_generate: image grid does not match placeholders");
    } else {
        for (int i = 0; i < n_ids; ++i) pos[3 * i] = pos[3 * i + 1] = pos[3 * i + 2] = i;
    }
    int n_placeholders = 0;
    for (int i = 0; i < n_ids; ++i) {
        if (n_image > 0 && ids[i] == image_token_id) ++n_placeholders;
        else if (ids[i] < 0 || ids[i] >= m->cfg.vocab) return fail(POCR_ERR_ARG, "token id %d outside vocab", ids[i]);
    }
    if (n_placeholders != n_image)
        return fail(POCR_ERR_ARG, "image placeholder tokens: got %d need %d", n_placeholders, n_image);
    RC(seq_set_state(s, 0));
    if (n_ids + max_new - 1 > s->cap) return fail(POCR_ERR_ARG, "pocr_generate: capacity %d too small", s->cap);
    if (s->sampling) RC(seed_sampler(s));  // one generator per generation call
    int32_t next = -1;
    if (use_prefill) {
        const int rc = prefill_ids_locked(s, ids, n_ids, n_image > 0 ? image_embeds : nullptr,
                                          n_image > 0 ? image_token_id : -1, pos.data(), nullptr, &next, image_dev);
        if (rc == POCR_OK) return decode_locked(s, next, n_ids + rope_delta, max_new, eos, n_eos, out_tokens);
        if (rc != POCR_ERR_UNSUPPORTED) return rc;
    }
    // token-by-token or host-assembled prompt: image rows on the host
    std::vector<float> host_img;
    if (image_dev && n_image > 0) {
        host_img.resize((size_t)n_image * H);
        HIP_TRY(hipMemcpyAsync(host_img.data(), image_embeds, host_img.size() * 4, hipMemcpyDeviceToHost,
                               m->ctx->stream));
        HIP_TRY(hipStreamSynchronize(m->ctx->stream));
        image_embeds = host_img.data();
    }
    std::vector<float> emb((size_t)n_ids * H);
    int img = 0;
    for (int i = 0; i < n_ids; ++i) {
        if (n_image > 0 && ids[i] == image_token_id) {
            if (img >= n_image) return fail(POCR_ERR_ARG, "too many image placeholder tokens");
            std::memcpy(&emb[(size_t)i * H], image_embeds + (size_t)img * H, (size_t)H * 4);
            ++img;
        } else {
            HIP_TRY(hipMemcpy(&emb[(size_t)i * H], m->embed + (size_t)ids[i] * H, (size_t)H * 4,
                              hipMemcpyDeviceToHost));
        }
    }
    if (use_prefill) {
        RC(prefill_locked(s, n_ids, emb.data(), pos.data(), nullptr, &next));
    } else {
        for (int i = 0; i < n_ids; ++i)
            RC(step_locked(s, &emb[(size_t)i * H], &pos[3 * i], i == n_ids - 1, nullptr,
                           i == n_ids - 1 ? &next : nullptr));
    }
    // first decode token sits at position len(out)-1+ropeDelta = n_ids+rope_delta
    return decode_locked(s, next, n_ids + rope_delta, max_new, eos, n_eos, out_tokens);
}

extern "C" int pocr_generate_vision(pocr_seq *s, pocr_projector *proj, const int32_t *ids, int n_ids,
                                    const float *vision_rows, int32_t image_token_id, const int32_t grid[3],
                                    int max_new, const int32_t *eos, int n_eos, int32_t *out_tokens) {
    if (!s || !proj || !ids || n_ids <= 0 || !out_tokens || !vision_rows || !grid || grid[0] <= 0 || grid[1] <= 0 ||
        grid[2] <= 0)
        return fail(POCR_ERR_ARG, "pocr_generate_vision: bad arguments");
    RC(check_eos("pocr_generate_vision", eos, n_eos));
    if (projector_ctx(proj) != s->m->ctx) return fail(POCR_ERR_ARG, "pocr_generate_vision: projector of another context");
    if (projector_text_dim(proj) != s->m->cfg.hidden)
        return fail(POCR_ERR_ARG, "pocr_generate_vision: projector width %d, model hidden %d",
                    projector_text_dim(proj), s->m->cfg.hidden);
    if (max_new <= 0) return 0;
    RC(model_ready(s->m));
    CHECK_INJECT("generate");
    std::lock_guard<std::mutex> lk(s->m->ctx->mu);
    RC(seq_idle(s, "pocr_generate_vision"));
    HIP_TRY(hipSetDevice(s->m->ctx->device));
    const float *rows_dev = nullptr;
    int n_image = 0;
    RC(project_upload_locked(proj, vision_rows, grid[0], grid[1], grid[2], &rows_dev, &n_image));
    return generate_locked(s, ids, n_ids, rows_dev, true, n_image, image_token_id, grid, 2, max_new, eos, n_eos, 1,
                           out_tokens);
}
