// internal.hpp — shared host-side definitions of the C ABI implementation.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/pocr_hip.h"
#include "kernels.hpp"
#include "sample.hpp"
#include "sample_wide.hpp"

namespace pocr {
int fail(int code, const char *fmt, ...);
bool injected(const char *op);
// greedy decode loop: steps per graph replay, and steps between the host's
// reads of the step state and tokens (a multiple of the former)
constexpr int kDecodeGraphSteps = 4;
constexpr int kDecodeSyncSteps = 16;
static_assert(kDecodeSyncSteps % kDecodeGraphSteps == 0, "whole graph replays per read-back");
}  // namespace pocr

#define HIP_TRY(expr)                                                                                     \
    do {                                                                                                  \
        hipError_t e_ = (expr);                                                                           \
        if (e_ != hipSuccess) return pocr::fail(POCR_ERR_DEVICE, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

#define CHECK_INJECT(op) \
    if (pocr::injected(op)) return pocr::fail(POCR_ERR_INJECTED, "%s: injected failure (POCR_HIP_FAIL_OP)", op)

#define RC(expr)                        \
    do {                                \
        int rc_ = (expr);               \
        if (rc_ != POCR_OK) return rc_; \
    } while (0)

struct DevBuf {
    void *p = nullptr;
    size_t n = 0;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    int ensure(size_t bytes) {
        if (bytes <= n) return POCR_OK;
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
        const size_t sz = std::max<size_t>(bytes, 256);
        HIP_TRY(hipMalloc(&p, sz));
        n = sz;
        return POCR_OK;
    }
    template <class T> T *as() const { return reinterpret_cast<T *>(p); }
};

// Lifetimes: every object holds a reference on its parent (weight→ctx,
// model→ctx and its weights, seq→model), and the public destroy/free calls
// drop the caller's reference.  Native memory is released child-before-parent
// whatever order a caller (or a garbage collector) destroys handles in.
struct pocr_ctx {
    std::atomic<int> refs{1};
    int device = 0;
    hipStream_t stream = nullptr;
    float *scratch = nullptr;  // this device's copy of the allocation-free entry's split records
    std::mutex mu;
    // op-level staging
    DevBuf x, out, out2, out3, res, vbuf, kc, vc, part, tabs, state;
    DevBuf gxd, gxs, gxb;  // batched GEMV activation digits
    DevBuf topk_part, samp;  // top-k partial keys, sampler state
    DevBuf wide;             // wide sampler buffers (pocr::WideBufs)
    // pinned host staging for large host→device uploads: two halves, each
    // reused once the copy recorded on its event has finished
    uint8_t *pin = nullptr;
    size_t pin_half = 0;
    hipEvent_t pin_ev[2] = {nullptr, nullptr};
    // pinned host read-back of the greedy decode loop: the step state and the
    // tokens of one batch of steps, fetched with one synchronization
    uint8_t *readback = nullptr;
};

struct pocr_weight {
    std::atomic<int> refs{1};
    pocr_ctx *ctx = nullptr;
    int qtype = 0, rows = 0, cols = 0;
    size_t row_bytes = 0;
    void *base = nullptr;
    const float *scale = nullptr;
    const uint8_t *data = nullptr;
    uint8_t *tiled = nullptr;  // the prefill GEMM's copy in its load order, when weight_tiles_ok
    int *usum = nullptr;       // Q4/Q6 with a tile image: Σ of each row's stored codes (row_usum)
    uint8_t *head_img = nullptr;  // Q6 heads: the rows in the head kernels' load order, when head_image_ok
};

struct LayerW {
    const pocr_weight *w[7] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    float *ln1 = nullptr, *ln2 = nullptr;
};

struct pocr_model {
    std::atomic<int> refs{1};
    pocr_ctx *ctx = nullptr;
    pocr_config cfg{};
    std::vector<LayerW> layers;
    const pocr_weight *lm = nullptr;
    float *final_norm = nullptr;
    float *embed = nullptr;
    double *freq = nullptr;
    uint8_t *axis = nullptr;
    std::vector<double> h_freq;
    std::vector<uint8_t> h_axis;
    int quirk = 1;
    int vnni = 0;  // Q4/Q6 matvecs in the reference's VNNI activation mode (vnni.hpp)
};


// prefill / batched GEMV (prefill.hip)
struct PrefillBufs {
    float *h = nullptr;      // [rows][hidden] residual rows
    float *v = nullptr;      // [rows][hidden] residual + attention rows
    float *qkv = nullptr;    // [rows][q_rows + 2·kv_rows]
    float *ho = nullptr;     // [rows][q_rows] attention output
    float *g = nullptr;      // [rows][inter] SwiGLU output
    int8_t *xd = nullptr;    // activation digit planes [3][rows][max K]
    float *xs = nullptr;     // [rows] digit row scales
    int *xb = nullptr;       // [rows][4] digit sums
    int32_t *pos = nullptr;  // [rows][3]
    uint8_t *kvimg = nullptr;  // one layer's attention block images [kv head][block][32 KB]
    int cap_rows = 0;        // rows allocated (a multiple of 32)
    int img_blocks = 0;      // key blocks per kv head in kvimg
};
void prefill_free(PrefillBufs &b);

struct pocr_seq {
    pocr_model *m = nullptr;
    int cap = 0;
    int len = 0;  // host mirror
    float *kv = nullptr;  // [layers][2][cap][kvd]
    float *h = nullptr, *qkv = nullptr, *head_out = nullptr, *vbuf = nullptr, *g = nullptr, *logits = nullptr;
    float *opart = nullptr;  // [heads][hidden] o_proj partials of the fused merge (k_attn_merge_oproj)
    float *part = nullptr;
    pocr::StepState *st = nullptr;
    int32_t *tokens = nullptr;
    int max_tokens = 0;
    uint32_t *eos_bits = nullptr;  // [ceil(vocab/32)] EOS bitmap for lists over kMaxEos ids
    int device_tokens = 0;         // tokens the device decode loop took in the last greedy decode
    int nsplit = 32;  // attention splits for rpw rows per wave
    int rpw = 16;
    pocr_batch *batch = nullptr;  // the continuous batch this sequence decodes in (ctx lock)
    // sampling head (temperature > 0, top_k != 1); greedy otherwise
    bool sampling = false;
    double temperature = 0.0;
    int top_k = 0;  // 0: every score (top_k 0 or >= vocab)
    uint64_t seed = 0;
    pocr::SampleState *samp = nullptr;
    unsigned long long *topk_part = nullptr;  // [kTopKMaxParts][kTopKMax] keys
    DevBuf wide;                              // wide sampler buffers (top_k 0 or > 64)
    hipGraphExec_t decode_exec = nullptr;    // one greedy (or sampled) decode step
    hipGraph_t decode_graph = nullptr;
    hipGraphExec_t decode_exec_n = nullptr;  // pocr::kDecodeGraphSteps of them in one replay
    hipGraph_t decode_graph_n = nullptr;
    PrefillBufs pf;
    ~pocr_seq();
};

namespace pocr {
void ctx_release(pocr_ctx *c);
void weight_retain(const pocr_weight *w);
void weight_release(const pocr_weight *w);
void model_release(pocr_model *m);
DevMat dev_mat(const pocr_weight *w);
int gemv_launch(hipStream_t s, GemvParams p, int nmat, int pro, int epi, int max_grid, int nv = 1,
                const GemvNV *q = nullptr);
GemvParams gemv_params_1(const pocr_weight *w);
// the same GEMV in the reference's VNNI activation mode for Q4/Q6 matrices of
// at least 32 columns (vnni.hpp); other matrices take gemv_launch
int gemv_launch_vnni(hipStream_t s, const GemvParams &p, int nmat, int pro, int epi, int max_grid);
int step_locked(pocr_seq *s, const float *emb, const int32_t pos3[3], int need_logits, float *logits,
                int32_t *token);
int prefill_locked(pocr_seq *s, int n, const float *emb, const int32_t *pos3, float *logits, int32_t *token);
// prefill from token ids: image rows uploaded straight into the device rows,
// text rows gathered from the device embedding table; POCR_ERR_UNSUPPORTED
// (no error recorded) when the model's shapes need the token-by-token path
int prefill_ids_locked(pocr_seq *s, const int32_t *ids, int n, const float *image, int32_t image_token,
                       const int32_t *pos3, float *logits, int32_t *token, bool image_on_device = false);
// host → device copy through the context's pinned staging (stream-ordered)
int upload_staged(pocr_ctx *ctx, void *dst, const void *src, size_t bytes);
int batched_gemv(pocr_ctx *ctx, const DevMat &w, const float *x, int m, float *out);
int read_state(pocr_seq *s, StepState *out);
unsigned long long argmax_of(const StepState &s);
float *layer_k(const pocr_seq *s, int layer);
float *layer_v(const pocr_seq *s, int layer);
int seq_set_state(pocr_seq *s, int len);
// POCR_ERR_ARG while the sequence is a member of a continuous batch (ctx lock held)
int seq_idle(const pocr_seq *s, const char *op);
// LM head on RMSNorm(x)·final_norm: greedy argmax into the step state, or the
// sampling head (logits, top-k, one draw into argmax slot 0) when the
// sequence samples
int enqueue_lm_head(pocr_seq *s, const float *x, bool want_logits);
// the VNNI mode's ordered attention for the n rows of a batched prompt
// (k_attn_ordered_rows): workgroups of up to 8 q heads of one KV head × n
// tokens, token i over cache rows [0, clen0 + i]
int launch_attn_ordered_rows(hipStream_t s, const float *qkv, int stride, const float *kc, const float *vc,
                             int heads, int kvh, int n, int clen0, float scale, float *out, int out_stride);
// the matrix-core head for 2 to 16 vectors (head.hpp, k_head_wide)
constexpr int kHeadWideMinRows = 16384;  // plain scores of fewer rows stay on the GEMV
bool head_wide_ok(const pocr_weight *w);
size_t head_wide_plane_bytes(const pocr_weight *w);
int launch_head_wide(hipStream_t s, const pocr_weight *w, const float *x, int x_stride, int nvec, const float *norm_w,
                     float eps, float *out, int out_stride, StepState *const *st, int8_t *planes, float *vscale,
                     int *vbias);
// batched building blocks (prefill.hip): digit planes of n rows, and the
// MFMA GEMM over them (npad = n rounded up to 32 tokens)
struct DigitizeParams;
struct GemmParams;
int digitize_rows(hipStream_t s, int qtype, const DigitizeParams &p, int n);
int gemm_rows(hipStream_t s, int qtype, int nmat, const GemmParams &p, int epi, int npad);
// gemm_rows over K columns reads digit planes in the tile layout
// (DigitizeParams::tiled) and the weights' tile images
bool gemm_tiled(int K);
// weights of this shape get a tile image at upload (k_tile_weight)
bool weight_tiles_ok(int rows, int cols);
int tile_weight(hipStream_t s, int qtype, const uint8_t *src, int row_bytes, int rows, int cols, uint8_t *dst);
// Σ of each row's stored codes (Q4, Q6), for the VNNI-mode GEMM epilogue
int row_usum(hipStream_t s, int qtype, const uint8_t *src, int row_bytes, int rows, int cols, int *dst);
// the small MFMA GEMM over at most 16 rows (digit planes of 16 rows)
bool gemm_small_ok(int rows, int K);
int gemm_small_rows(hipStream_t s, int qtype, int nmat, const GemmParams &p, int epi);
// vision projector (projector.hip); callers hold the context lock
int project_locked(pocr_projector *p, int grid_t, int grid_h, int grid_w, int *rows);
int project_upload_locked(pocr_projector *p, const float *vision_rows, int grid_t, int grid_h, int grid_w,
                          const float **out_dev, int *rows);
int projector_text_dim(const pocr_projector *p);
pocr_ctx *projector_ctx(const pocr_projector *p);
// pocr_generate under the context lock, image rows from the host or (image_dev) the device
int generate_locked(pocr_seq *s, const int32_t *ids, int n_ids, const float *image, bool image_dev, int n_image,
                    int32_t image_token_id, const int32_t grid[3], int32_t merge, int max_new, const int32_t *eos,
                    int n_eos, int use_prefill, int32_t *out_tokens);
constexpr int kBigGrid = 1024;
}  // namespace pocr
