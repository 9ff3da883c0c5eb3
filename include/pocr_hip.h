/*
 * pocr_hip.h — C ABI of the MI355X (gfx950) ERNIE text-decoder step.
 *
 * This is the drop-in boundary a `hip` implementation of RapidOCRvl's
 * internal/backend package binds through cgo.  Plain pointers and sizes only.
 *
 * Conventions (mirroring internal/backend/vulkan_exec_stub.go:14-328):
 *  - Every call returns an int status.  POCR_OK (0) on success.
 *    POCR_ERR_ARG: shape/length/handle problem detected BEFORE any device work;
 *      the Go caller must return the error without disabling the op
 *      (internal/model/vulkan_fallback_test.go:167-290).
 *    POCR_ERR_DEVICE / POCR_ERR_NOMEM / POCR_ERR_INJECTED: device-side failure;
 *      the Go caller disables the op and falls back to the CPU kernels
 *      (internal/model/model.go:7240-7258 disableVulkanOp).
 *  - pocr_last_error() returns the calling thread's last message.
 *  - Op-level calls borrow host slices for the duration of the call and are
 *    synchronous, like the backend.Vulkan* functions.
 *  - Weights are uploaded once, in the GGUF Q*_ROW row layout
 *    (internal/gguf/gguf.go:446-464,506-520,544-558): rows × f32 scale, then
 *    rows × packed row bytes.  Handles replace the Vulkan backend's
 *    host-pointer fingerprint cache (internal/backend/vulkan_cache_windows.go:7-98).
 *  - Thread safety: a context serialises device work on its own stream; a
 *    sequence must not be used by two threads at once.
 */
#ifndef POCR_HIP_H
#define POCR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define POCR_ABI_VERSION 1

#define POCR_OK 0
#define POCR_ERR_ARG (-1)
#define POCR_ERR_DEVICE (-2)
#define POCR_ERR_NOMEM (-3)
#define POCR_ERR_UNSUPPORTED (-4)
#define POCR_ERR_INJECTED (-5)

/* tensor types = GGUF type ids (internal/gguf/gguf.go:19-22) */
#define POCR_F32 0
#define POCR_Q8 1000
#define POCR_Q4 1001
#define POCR_Q6 1002

/* row encoder tie modes */
#define POCR_TIE_HALF_AWAY 0 /* roundToInt, internal/tensor/quant.go:436-441 */
#define POCR_TIE_AMD64 1     /* RNE where the amd64 converter rounds with AVX2 */

/* matrix roles for pocr_model_set_weight (internal/model text layer fields) */
#define POCR_W_Q 0
#define POCR_W_K 1
#define POCR_W_V 2
#define POCR_W_O 3
#define POCR_W_GATE 4
#define POCR_W_UP 5
#define POCR_W_DOWN 6
#define POCR_W_LM_HEAD 7
/* norm roles for pocr_model_set_norm */
#define POCR_N_LN1 0
#define POCR_N_LN2 1
#define POCR_N_FINAL 2

typedef struct pocr_ctx pocr_ctx;
typedef struct pocr_weight pocr_weight;
typedef struct pocr_model pocr_model;
typedef struct pocr_seq pocr_seq;
typedef struct pocr_projector pocr_projector;
typedef struct pocr_gguf pocr_gguf;
typedef struct pocr_batch pocr_batch;

/* decoder hyper-parameters (internal/config/config.go:31-49).  Unlike the
 * reference loader (internal/model/model.go:647-653) heads*head_dim may
 * differ from hidden. */
typedef struct {
    int32_t hidden;
    int32_t intermediate;
    int32_t layers;
    int32_t heads;
    int32_t kv_heads;
    int32_t head_dim;
    int32_t vocab;
    float rms_norm_eps;
    double rope_theta;
    int32_t mrope_section[3]; /* zeros → default {16,24,24} (model.go:882) */
} pocr_config;

/* ---------------- library / context ---------------- */
int pocr_abi_version(void);
const char *pocr_last_error(void);
/* replaces backend.Select("hip") device bring-up (internal/backend/backend.go:85-111) */
int pocr_ctx_create(int device, pocr_ctx **out);
void pocr_ctx_destroy(pocr_ctx *ctx);
/* number of HIP devices visible (0 when none); never fails */
int pocr_device_count(void);

/* ---------------- formats (host) ---------------- */
/* row bytes of one packed row: Q8 cols, Q4 (cols+1)/2, Q6 PackedQ6Cols
 * (internal/tensor/quant.go:2882) */
size_t pocr_row_bytes(int qtype, int cols);
/* QuantizeQ8RowBytesInto / QuantizeQ4RowInto / QuantizeQ6RowInto
 * (internal/tensor/quant.go:96-137, 291-354, 201-270) over rows. */
int pocr_quantize_rows(int qtype, int tie_mode, const float *w, int rows, int cols, float *scales,
                       uint8_t *packed);
/* UnpackQ4Matrix / UnpackQ6Matrix / q8ValueTable (internal/tensor/quant.go:2325-2368,
 * 2605-2656, 2314-2320): packed rows → int8 codes */
int pocr_unpack_rows(int qtype, const uint8_t *packed, int rows, int cols, int8_t *out);

/* ---------------- weights ---------------- */
/* upload one Q*_ROW tensor (scales f32[rows] + packed rows) into HBM.  A
 * tensor of rows a multiple of 16 and cols a multiple of 128 also gets the
 * prefill GEMM's tile image of the same bytes (and, for Q4/Q6, each row's sum
 * of stored codes for the VNNI mode), built on the device here: its HBM
 * footprint is then about twice the packed bytes. */
int pocr_weight_upload(pocr_ctx *ctx, int qtype, int rows, int cols, const float *scales,
                       const uint8_t *packed, pocr_weight **out);
void pocr_weight_free(pocr_weight *w);

/* ---------------- op level (host buffers, synchronous) ---------------- */
/* VulkanMatVecQ{8,6,4} (vulkan_exec_stub.go:186,234,282): out[m][rows] = W·x[m].
 * m > 1 is the batched GEMV (M rows of activations sharing one weight stream). */
int pocr_matvec(pocr_ctx *ctx, const pocr_weight *w, const float *x, int m, float *out);
/* MatVecQ4/MatVecQ6 as the reference's CPU path computes them on an
 * AVX512-VNNI host (quantizeXForVNNI internal/tensor/quant.go:2087-2115,
 * quantizeXForVNNIAVX2 dot_amd64.go:228-252, dotQ8VNNI dot_amd64.go:150-167,
 * finalizeDotQ8VNNI dot_vnni_amd64.s:1043-1080): each row of x quantized to
 * u8 with one scale, exact int32 dots, out = ((dot - 128*rowSum)*scaleX)*scale[r].
 * Bit-identical to that matvec for the same x.  Q8 matrices and inputs of
 * fewer than 32 columns are computed in plain mode, as there. */
int pocr_matvec_vnni(pocr_ctx *ctx, const pocr_weight *w, const float *x, int m, float *out);
/* VulkanMatVecArgmaxQ* (vulkan_exec_stub.go:190,238,286): greedy LM head,
 * ties → lowest index (internal/tensor/argmax_quant.go:255-262) */
int pocr_matvec_argmax(pocr_ctx *ctx, const pocr_weight *w, const float *x, int32_t *index,
                       float *score);
/* VulkanMatVecTopKQ{8,4,6} (vulkan_exec_stub.go:194,242,290; CPU
 * MatVecTopKQ*WithWork, internal/tensor/topk.go:200-275): the k best rows of
 * W·x, score descending, equal scores by lower row (topKSelectWithWork,
 * topk.go:322-345).  1 <= k <= rows; k > 64 (past the reference's GPU
 * limit, model.go:7143, where its CPU path takes over) sorts every score on
 * the device.  Writes k ids (and scores if non-null), returns k. */
int pocr_matvec_topk(pocr_ctx *ctx, const pocr_weight *w, const float *x, int k, int32_t *ids,
                     float *scores);
/* one draw from the top k of n host logits — the candidates path of a
 * sampled token (matVecTopKMaybeCPU, internal/model/model.go:7202-7235, then
 * sampleCandidateScoresScratch 1950-1990) — with the fastRNG state *rng_state
 * (model.go:1829-1840), which is advanced.  temperature > 0, 1 < k < n.
 * Writes the token and, if non-null, the k candidates. */
int pocr_sample_topk(pocr_ctx *ctx, const float *logits, int n, int k, double temperature,
                     uint64_t *rng_state, int32_t *token, int32_t *ids, float *scores);
/* one draw over all n host logits — sampleFullLogitsScratch (internal/model/
 * model.go:2215-2307), which sampleTokenScratch (1870-1879) takes for top_k
 * 0 or >= n: FastExpF32 weights of x·(1/T) − max·(1/T) (x − max at T = 1,
 * T = float32(temperature)), their running f32 sum, CumulativeSum
 * (internal/tensor/cumsum.go:9-58) and pickCumulativeFloat32 (model.go:
 * 2326-2340); two logits take sampleTwoLogits (2309-2324).  *rng_state is
 * the fastRNG state, advanced by one draw.  temperature > 0. */
int pocr_sample_full(pocr_ctx *ctx, const float *logits, int n, double temperature, uint64_t *rng_state,
                     int32_t *token);
/* VulkanFusedMatVec3Q* (vulkan_exec_stub.go:202,250,298) */
int pocr_fused_matvec3(pocr_ctx *ctx, const pocr_weight *a, const pocr_weight *b, const pocr_weight *c,
                       const float *x, float *out_a, float *out_b, float *out_c);
/* VulkanFusedMatVec3MRoPEQ* (vulkan_exec_stub.go:214,262,310): Q,K,V then
 * rotate-half RoPE on out_a (q_heads) and out_b (kv_heads) */
int pocr_fused_matvec3_mrope(pocr_ctx *ctx, const pocr_weight *a, const pocr_weight *b,
                             const pocr_weight *c, const float *x, const float *cos_t,
                             const float *sin_t, int q_heads, int kv_heads, int head_dim,
                             float *out_a, float *out_b, float *out_c);
/* VulkanSwiGLUGateUpQ* (vulkan_exec_stub.go:222,270,318): out = SiLU(G·x)·(U·x) */
int pocr_swiglu_gate_up(pocr_ctx *ctx, const pocr_weight *gate, const pocr_weight *up, const float *x,
                        float *out);
/* VulkanMatVecAddRMSNormQ* (vulkan_exec_stub.go:198,246,294) and the OutOnly
 * CPU variants (internal/tensor/fused_matvec2.go:339-1623):
 * v = residual + W·x; norm_out = RMSNorm(v)·norm_w; residual = v iff in_place */
int pocr_matvec_add_rmsnorm(pocr_ctx *ctx, const pocr_weight *w, const float *x, float *residual,
                            const float *norm_w, float eps, int in_place, float *norm_out);
/* VulkanRMSNormF32 (vulkan_exec_stub.go:26) */
int pocr_rmsnorm(pocr_ctx *ctx, const float *x, const float *w, int n, float eps, float *out);
/* VulkanMRoPEPairF32 (vulkan_exec_stub.go:42), in place */
int pocr_mrope_pair(pocr_ctx *ctx, float *q, float *k, const float *cos_t, const float *sin_t,
                    int q_heads, int kv_heads, int head_dim);
/* VulkanSwiGLUDownQ{8,4,6} (vulkan_exec_stub.go:218,266,314):
 * out = Down·(SiLU(G·x)·(U·x)); the SwiGLU vector stays on the device */
int pocr_swiglu_down(pocr_ctx *ctx, const pocr_weight *gate, const pocr_weight *up, const pocr_weight *down,
                     const float *x, float *out);
/* VulkanSwiGLUDownAddRMSNormQ{8,4,6} (vulkan_exec_stub.go:226,274,322;
 * in_place = 1) and ...OutOnly (230,278,326; in_place = 0), the MLP half of
 * mlpDownAddRMSNormCPU (internal/model/model.go:5714-5800):
 * v = residual + Down·SwiGLU(x); norm_out = RMSNorm(v)·norm_w; residual = v
 * iff in_place.  The Vulkan functions assume eps 1e-6 (model.go:6869). */
int pocr_swiglu_down_add_rmsnorm(pocr_ctx *ctx, const pocr_weight *gate, const pocr_weight *up,
                                 const pocr_weight *down, const float *x, float *residual, const float *norm_w,
                                 float eps, int in_place, float *norm_out);
/* VulkanAddRMSNormF32 (vulkan_exec_stub.go:30; in_place = 1: dst += add,
 * AddRMSNorm ops.go:913-935) and VulkanAddRMSNormF32OutOnly (34; in_place = 0,
 * fused_matvec2.go:11-33): out = RMSNorm(dst + add)·w */
int pocr_add_rmsnorm(pocr_ctx *ctx, float *dst, const float *add, const float *w, int n, float eps, int in_place,
                     float *out);
/* VulkanMRoPEF32 (vulkan_exec_stub.go:38; ApplyMRoPETable,
 * internal/tensor/weighted_sum.go:231-250): rotate-half RoPE of x[heads*dim]
 * in place */
int pocr_mrope(pocr_ctx *ctx, float *x, const float *cos_t, const float *sin_t, int heads, int head_dim);
/* VulkanTextAttentionF32 (vulkan_exec_stub.go:134): GQA decode attention of
 * q[heads*dim] over cache_len rows of kv_heads*dim fp32 K/V */
int pocr_text_attention(pocr_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                        int cache_len, int heads, int kv_heads, int head_dim, float *out);
/* VulkanTextAttentionOutQ{8,6,4} (vulkan_exec_stub.go:162,170,178): the
 * attention above, then out = Wo·attention (wo: rows × heads·dim) */
int pocr_text_attention_out(pocr_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                            int cache_len, int heads, int kv_heads, int head_dim, const pocr_weight *wo,
                            float *out);
/* VulkanTextAttentionOutAddRMSNormQ{8,6,4} (vulkan_exec_stub.go:166,174,182),
 * the general branch of attentionWithNorm (internal/model/model.go:4040-4066):
 * v = residual + Wo·attention; norm_out = RMSNorm(v)·norm_w; residual = v iff
 * in_place (0 for the Q4/Q6 OutOnly behaviour, model.go:4051-4057) */
int pocr_text_attention_out_add_rmsnorm(pocr_ctx *ctx, const float *q, const float *k_cache,
                                        const float *v_cache, int cache_len, int heads, int kv_heads, int head_dim,
                                        const pocr_weight *wo, float *residual, const float *norm_w, float eps,
                                        int in_place, float *norm_out);
/* VulkanTextFirstTokenValueOutAddRMSNormQ{8,6,4} (vulkan_exec_stub.go:150,
 * 154,158), the first-token branch of attentionWithNorm (model.go:3857-3902):
 * with one cached row the attention output is its V row per q head
 * (expandValueHeads, model.go:4603-4621; k_cache is not read for the result),
 * then v = residual + Wo·that; norm_out = RMSNorm(v)·norm_w; residual = v iff
 * in_place (0 for the Q4/Q6 OutOnly branch, model.go:3895-3902) */
int pocr_first_token_value_out_add_rmsnorm(pocr_ctx *ctx, const float *k_cache, const float *v_cache, int heads,
                                           int kv_heads, int head_dim, const pocr_weight *wo, float *residual,
                                           const float *norm_w, float eps, int in_place, float *norm_out);
/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops).  The
 * computation of pocr_text_attention over device buffers the caller owns
 * (q_dev, the caches, out_dev), allocating nothing: its split records live in
 * a fixed per-device array of 512 (kv head, split) records, so kv_heads x
 * splits above 512 (2 kv heads: above 16384 cache rows) is POCR_ERR_ARG.
 * Synchronous on the context's stream.  Calls that overlap on one GPU race
 * on the array. */
int pocr_text_attention_noalloc(pocr_ctx *ctx, const float *q_dev, const float *k_cache_dev,
                                const float *v_cache_dev, int cache_len, int heads, int kv_heads, int head_dim,
                                float *out_dev);

/* Average device time (microseconds, HIP events on the context stream) of the
 * M=1 GEMV kernel over `iters` launches that rotate through n_weights copies of
 * one shape, so the working set can exceed the 256 MB Infinity Cache.  Runs a
 * separately named instance of the same kernel so profiles can attribute it.
 * Measurement counterpart of internal/tensor/model_dims_bench_test.go. */
int pocr_time_matvec(pocr_ctx *ctx, const pocr_weight *const *weights, int n_weights, const float *x, int iters,
                     float *avg_us);

/* The same for the greedy LM-head launch (MatVecArgmaxQ*, argmax_quant.go:
 * 11-433): the argmax kernel the device decode loop runs, no logits written. */
int pocr_time_matvec_argmax(pocr_ctx *ctx, const pocr_weight *const *weights, int n_weights, const float *x,
                            int iters, float *avg_us);

/* The same for the batched GEMV: m rows of x (m*cols floats) per launch pair
 * (digit planes + MFMA GEMM).  Measurement counterpart of the reference's
 * M-row benchmarks (internal/tensor/model_dims_bench_test.go). */
int pocr_time_matvec_batched(pocr_ctx *ctx, const pocr_weight *const *weights, int n_weights, const float *x, int m,
                             int iters, float *avg_us);

/* Average device time (microseconds) of one decode-attention call — RoPE,
 * K/V append and GQA attention of one token over cache_len fp32 rows, the
 * work of cacheAttentionScores + weightedCacheValueSum
 * (internal/model/model.go:4623-4795, 5201-5590) — rotating over n_layers
 * separate caches so the working set can exceed the Infinity Cache. */
int pocr_time_attention(pocr_ctx *ctx, int heads, int kv_heads, int head_dim, int cache_len, int n_layers, int iters,
                        float *avg_us);

/* Average device time (microseconds) of a plain streaming read of `bytes`
 * (a multiple of 16) from one of n_buffers device buffers, rotating so the
 * working set can exceed the Infinity Cache: the read ceiling a
 * weight-streaming kernel of the same size is compared with.  No counterpart
 * in the reference (a measurement aid); allocates and frees its buffers. */
int pocr_time_stream_read(pocr_ctx *ctx, int64_t bytes, int n_buffers, int iters, float *avg_us);

/* ---------------- model / step level (device-resident) ---------------- */
int pocr_model_create(pocr_ctx *ctx, const pocr_config *cfg, pocr_model **out);
void pocr_model_destroy(pocr_model *m);
/* borrow an uploaded weight; layer -1 with POCR_W_LM_HEAD for the head.
 * Set the matrices before the model's first sequence: while sequences exist
 * this returns POCR_ERR_ARG (their captured decode graphs hold the weights'
 * device addresses).  Norms and the embedding table may be rewritten any time
 * (in place). */
int pocr_model_set_weight(pocr_model *m, int layer, int role, const pocr_weight *w);
/* copies hidden floats to HBM; layer -1 with POCR_N_FINAL for the final norm */
int pocr_model_set_norm(pocr_model *m, int layer, int role, const float *w);
/* copies the f32 embed_tokens table [vocab][hidden] to HBM */
int pocr_model_set_embed(pocr_model *m, const float *embed);
/* reproduce the reference's Q4/Q6 attention-residual behaviour
 * (internal/model/model.go:3895-3902, 4051-4057); default on.  Set it before
 * the model's first sequence: changing it while sequences exist returns
 * POCR_ERR_ARG (their captured decode graphs hold the rule). */
int pocr_model_set_residual_quirk(pocr_model *m, int on);
/* Every Q4/Q6 matvec of the model's decode steps and LM head in the VNNI
 * activation mode above, as the reference's CPU path runs on an
 * AVX512-VNNI host (dot_amd64.go:12 selects it; UnpackQ4Matrix/Q6 keep the
 * row sums it needs, quant.go:2325); default off (plain mode).  Set it before
 * the model's first sequence (POCR_ERR_ARG after).  In this mode prompts run
 * token by token (pocr_prefill and pocr_generate take their rows as token
 * steps), and the batched decode (pocr_decode_batch, the continuous batch)
 * steps each member with the mode's single-sequence step: every member's
 * stream is what decoding it alone gives.  The ops around
 * the matvecs keep the portable scalar accumulation orders
 * (sumSquaresScalar, dotF32's running sums); an x86-64 host takes its
 * FMA/AVX kernels for those (dot_amd64.go:11), so steps are bit-identical to
 * the scalar-order restatement of the mode and agree with such a host to
 * rounding. */
int pocr_model_set_vnni(pocr_model *m, int on);

/* per-sequence state: per-layer fp32 K/V in HBM preallocated for `capacity`
 * tokens (getKVCaches, internal/model/model.go:3286-3327) */
int pocr_seq_create(pocr_model *m, int capacity, pocr_seq **out);
void pocr_seq_destroy(pocr_seq *s);
int pocr_seq_reset(pocr_seq *s);
int pocr_seq_len(const pocr_seq *s);
/* Tokens the device decode loop took in the sequence's last greedy decode
 * (pocr_decode_greedy, pocr_generate, pocr_generate_vision,
 * pocr_decode_batch): each step prologue takes the previous step's token.
 * A loop that met an EOS id took it and ran no step after it
 * (model.go:1545-1548), so this is the EOS's output index + 1 there, where a
 * loop that kept stepping would show its whole chunk of steps.  No reference
 * counterpart: accounting for callers and tests. */
int pocr_seq_device_tokens(const pocr_seq *s);
/* token choice of the sequence's step-level generation (GenerateOptions
 * Temperature/TopK/Seed, internal/model/model.go:420-470): temperature <= 0
 * or top_k == 1 is greedy (generationUsesArgmaxSampling, 1858-1860);
 * otherwise every token, the prefill's first included, is drawn on the
 * device: from the top_k LM-head candidates for 1 < top_k < vocab
 * (model.go:3632-3638, 1950-1990), from every score for top_k 0 or >= vocab
 * (sampleFullLogitsScratch, 2215-2307).  The generator restarts at `seed`
 * here and at every pocr_generate (samplingRNGInto, 1846-1852);
 * pocr_decode_greedy, pocr_decode_batch and pocr_batch_step continue it. */
int pocr_seq_set_sampling(pocr_seq *s, double temperature, int top_k, uint64_t seed);
/* copy layer's first len rows of K/V (len*kv_heads*head_dim floats each) */
int pocr_seq_read_kv(pocr_seq *s, int layer, float *k, float *v);
/* drop cache rows beyond len (0 <= len <= current length); the rows kept are
 * untouched, like a kvCache whose len is reset (internal/model/model.go:3318) */
int pocr_seq_truncate(pocr_seq *s, int len);
int pocr_seq_write_kv(pocr_seq *s, int layer, const float *k, const float *v, int len);

/* one token step (forwardEmbeddingForSampling, internal/model/model.go:3475-3643).
 * need_logits=0 is a non-final prompt token.  logits (vocab floats) and token
 * are optional outputs. */
int pocr_step(pocr_seq *s, const float *emb, const int32_t pos3[3], int need_logits, float *logits,
              int32_t *token);
/* prompt prefill of n embeddings at positions pos3[n][3]: the same results
 * as n sequential pocr_step calls (token-by-token prefill,
 * internal/model/model.go:1514-1536), run on the device without host round
 * trips between tokens.  logits/token of the last row. */
int pocr_prefill(pocr_seq *s, int n, const float *emb, const int32_t *pos3, float *logits,
                 int32_t *token);
/* greedy decode loop kept on the device (decode loop, model.go:1538-1568):
 * feeds first_token at position first_pos, first_pos+1, ...; writes up to
 * max_new tokens (first_token first) and stops after an EOS id.  Returns the
 * number of tokens written (>=0) or an error status (<0).
 * EOS lists, here and in every generate/decode entry point: at most 1,024 ids
 * and none negative, else POCR_ERR_ARG (maxEOSTokenIDs and
 * ValidateGenerateOptions, model.go:432, 461-467).  The device loop stops on
 * every listed id (up to 16 in the step state, longer lists as a bitmap over
 * the vocabulary). */
int pocr_decode_greedy(pocr_seq *s, int32_t first_token, int32_t first_pos, int max_new,
                       const int32_t *eos, int n_eos, int32_t *out_tokens);
/* decode of n_seq (1..16) sequences of one model together: the
 * server's concurrent requests (cmd/paddleocrvl-server/main.go:1106, one
 * decode loop each, model.go:1538-1568) batched into one device step — each
 * layer's weights stream once for all of them (M = n_seq batched GEMV), each
 * sequence keeps its own KV cache.  Sequence i starts from first_tokens[i] at
 * first_positions[i]; its tokens go to out_tokens[i*max_new ...] (first token
 * first), out_counts[i] of them, stopping after an EOS id.  Greedy sequences
 * take the argmax, sampling ones (pocr_seq_set_sampling) draw from their own
 * generator.  Per-sequence results equal pocr_decode_greedy's up to f32
 * summation order.  Up to 4
 * sequences share GEMV passes; 5..16 need layer matrices with rows a
 * multiple of 16 and inputs a multiple of 256 (POCR_ERR_UNSUPPORTED
 * otherwise). */
int pocr_decode_batch(pocr_seq *const *seqs, int n_seq, const int32_t *first_tokens,
                      const int32_t *first_positions, int max_new, const int32_t *eos, int n_eos,
                      int32_t *out_tokens, int32_t *out_counts);
/* continuous batching: a decode batch that requests join and leave between
 * token steps, in place of the server's per-request slots, each running its
 * own decode loop (cmd/paddleocrvl-server/main.go:1106-1124, acquire/release;
 * model.go:1538-1568).  As many members decode at once as pocr_decode_batch
 * takes sequences (16, or 4 for models outside the wide step's shapes), one
 * batched device step per token; each member's tokens equal its
 * pocr_decode_greedy stream.  A batch is driven by one thread; a member
 * sequence accepts no other generation or cache call until it leaves
 * (POCR_ERR_ARG), and destroying it removes it from the batch. */
int pocr_batch_create(pocr_model *m, pocr_batch **out);
void pocr_batch_destroy(pocr_batch *b);
/* a prefilled sequence joins with the token its prefill chose, at position
 * first_pos, for at most max_new tokens (first_token counted) and the EOS
 * ids given; a sampling sequence keeps drawing from its generator.
 * POCR_ERR_ARG if the batch's limit of members is decoding or the capacity
 * is short. */
int pocr_batch_join(pocr_batch *b, pocr_seq *s, int32_t first_token, int32_t first_pos, int max_new,
                    const int32_t *eos, int n_eos);
/* up to max_steps token steps for every decoding member (fewer when a
 * member's budget ends first); members reaching an EOS id or max_new tokens
 * finish.  Returns the number of members still decoding. */
int pocr_batch_step(pocr_batch *b, int max_steps);
/* tokens a member has produced so far (>= 0), *finished set when it is done */
int pocr_batch_poll(pocr_batch *b, const pocr_seq *s, int *finished);
/* the member leaves, finished or not: copies up to cap of its tokens (first
 * token first) and returns how many it produced */
int pocr_batch_leave(pocr_batch *b, pocr_seq *s, int32_t *out_tokens, int cap);
/* whole greedy generation: GenerateWithOptions / generateWithImageEmbeds
 * (internal/model/model.go:1492-1572, 1618-1711) incl. multimodal positions
 * (1717-1783).  image rows replace ids equal to image_token_id in order.
 * use_prefill=1 runs pocr_prefill, 0 one pocr_step per prompt token. */
int pocr_generate(pocr_seq *s, const int32_t *ids, int n_ids, const float *image_embeds, int n_image,
                  int32_t image_token_id, const int32_t grid[3], int32_t merge, int max_new,
                  const int32_t *eos, int n_eos, int use_prefill, int32_t *out_tokens);

/* ---------------- checkpoints ---------------- */
/* gguf.Open (internal/gguf/gguf.go:111-251) with its validation (counts,
 * string sizes, keys and names, shapes, types, offsets within the file:
 * 253-296, 586-667).  Tensor types F32 (0), Q8_ROW/Q4_ROW/Q6_ROW
 * (1000/1001/1002, = POCR_Q8/Q4/Q6); metadata u32 (4), u64 (10), string (8).
 * Host only; no device needed. */
int pocr_gguf_open(const char *path, pocr_gguf **out);
void pocr_gguf_close(pocr_gguf *g);
int pocr_gguf_tensor_count(const pocr_gguf *g);
/* index of a tensor by name (File.Tensors), or POCR_ERR_ARG when missing */
int pocr_gguf_find(const pocr_gguf *g, const char *name);
/* name, type, dims (up to 8) and payload bytes (TensorBytes) of tensor i */
int pocr_gguf_tensor_info(const pocr_gguf *g, int i, const char **name, uint32_t *type, int *ndim, int64_t *dims,
                          int64_t *bytes);
/* the payload of tensor i (F32 values; Q*_ROW: f32 scales[rows] then the
 * packed rows), exactly `bytes` of it */
int pocr_gguf_read(const pocr_gguf *g, int i, void *dst, int64_t bytes);
int pocr_gguf_meta_count(const pocr_gguf *g);
/* metadata entry i: key, type, numeric value (u32/u64) or string */
int pocr_gguf_meta(const pocr_gguf *g, int i, const char **key, uint32_t *type, uint64_t *value, const char **str);
/* a decoder model from a checkpoint: the tensors preloadTextWeights reads
 * (internal/model/model.go:2861-2885) — model.embed_tokens / model.norm /
 * lm_head and model.layers.N.{input_layernorm, post_attention_layernorm,
 * self_attn.{q,k,v,o}_proj, mlp.{gate,up,down}_proj}.weight — with cfg from
 * config.json (internal/config/config.go:51).  Matrices Q*_ROW, the rest F32. */
int pocr_model_load_gguf(pocr_ctx *ctx, const pocr_config *cfg, const char *path, pocr_model **out);

/* ---------------- vision projector ---------------- */
/* mlp_AR of the vision tower (internal/model/vision.go:224-302): pre_norm
 * LayerNorm over vision_dim, linear_1 w1 [4·vd][4·vd] + b1, GELU(tanh),
 * linear_2 w2 [text_dim][4·vd] + b2, f32 row-major.  Both matrices are
 * quantized to Q8 rows here, as cacheVisionWeights does (vision.go:286-302).
 * 4·vision_dim a multiple of 128 and <= 8192, text_dim a multiple of 64;
 * POCR_ERR_UNSUPPORTED otherwise. */
int pocr_projector_create(pocr_ctx *ctx, int vision_dim, int text_dim, const float *norm_w, const float *norm_b,
                          const float *w1, const float *b1, const float *w2, const float *b2, float eps,
                          pocr_projector **out);
void pocr_projector_destroy(pocr_projector *p);
/* projectImage (vision.go:1029-1108; the op behind VulkanProjectImageF32,
 * internal/backend/vulkan_exec_stub.go:122, with the runtime's Q8 weights):
 * vision-encoder rows [T·H·W][vision_dim] (frame-major, then row, column) →
 * one row [text_dim] per 2×2 block, T·(H/2)·(W/2) of them, frame-major.
 * Returns the row count. */
int pocr_project_image(pocr_projector *p, const float *vision_rows, int grid_t, int grid_h, int grid_w,
                       float *out);
/* image generation from vision-encoder rows (EncodeImageWithGrid's
 * projection, vision.go:146, feeding generateWithImageEmbeds, model.go:
 * 1618-1711): the rows are projected on the device straight into the
 * prompt's image rows (placeholders = T·(H/2)·(W/2), merge 2), then as
 * pocr_generate with use_prefill=1.  grid = (T, H, W) of vision patches;
 * the projector belongs to the sequence's context. */
int pocr_generate_vision(pocr_seq *s, pocr_projector *proj, const int32_t *ids, int n_ids,
                         const float *vision_rows, int32_t image_token_id, const int32_t grid[3], int max_new,
                         const int32_t *eos, int n_eos, int32_t *out_tokens);
/* device time of one projection of a T·H·W grid (rows resident, HIP events
 * over `iters` back-to-back runs): the bench's measurement hook */
int pocr_time_project(pocr_projector *p, int grid_t, int grid_h, int grid_w, int iters, float *avg_us);

/* multimodal RoPE positions (internal/model/model.go:1717-1783), host only.
 * Returns the number of positions written, rope_delta via pointer. */
int pocr_mm_positions(const int32_t *ids, int n, int32_t image_token_id, const int32_t grid[3],
                      int32_t merge, int32_t *pos3, int32_t *rope_delta);

#ifdef __cplusplus
}
#endif
#endif /* POCR_HIP_H */
