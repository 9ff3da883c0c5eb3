/*
 * pocr_oracle.h — CPU restatement of RapidOCRvl's pure-Go ERNIE text-decoder
 * path, used ONLY as test infrastructure: the parity checker for the HIP
 * library and the CPU baseline timed beside it.  Nothing in the product
 * (rapidocrvl_amd/, include/) includes, links or loads this code.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the RapidOCRvl repository root).  Pinning of each function (golden vectors,
 * closed forms, brute force) lives in tests/test_oracle_*.py; functions whose
 * exact float rounding only the Go binary could fix are tolerance-pinned and
 * say so below ("parity unpinned" for bit-level rounding order).
 */
#ifndef POCR_ORACLE_H
#define POCR_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* quant type tags, same numbers as the GGUF tensor types
 * (internal/gguf/gguf.go:19-22) */
#define ORC_F32 0
#define ORC_Q8 1000
#define ORC_Q4 1001
#define ORC_Q6 1002

/* row-encoder tie modes */
#define ORC_TIE_HALF_AWAY 0 /* roundToInt, quant.go:436-441 (scalar Go, Q8 converter) */
#define ORC_TIE_AMD64 1     /* VRNDSCALEPS RNE (dot_amd64.s:5837-6005) where the
                               amd64 converter uses AVX2: Q4 all cols (cols>=8),
                               Q6 floor(cols/8)*8 prefix; Q8 bytes stay half-away */

/* ---- formats: encoders / unpack (a2, a3) ---- */
size_t orc_row_bytes(int qtype, int cols);
float orc_quantize_row(int qtype, int tie_mode, const float *w, int cols, uint8_t *out);
void orc_unpack_row(int qtype, const uint8_t *row, int cols, int8_t *out);
int orc_round_to_int(float x);

/* ---- matvec (a4, a5) ---- */
typedef struct {
    int qtype;           /* ORC_Q8 / ORC_Q4 / ORC_Q6 */
    int rows, cols;
    const float *scale;  /* [rows] */
    const uint8_t *data; /* rows * orc_row_bytes(qtype, cols) */
} orc_qmat;

/* plain fp32-activation semantics: out[r] = dot(int q[r], x) * scale[r] */
void orc_matvec(const orc_qmat *m, const float *x, float *out);
/* VNNI-emulation semantics (dot_amd64.go:140-167, dot_vnni_amd64.s:434-500,1043-1080) */
float orc_quantize_x_vnni(const float *x, int n, uint8_t *xq);
void orc_matvec_vnni(const orc_qmat *m, const float *x, float *out);
/* dotQ8VNNICore: Σ a·xq in int32 */
int32_t orc_vnni_core(const int8_t *a, const uint8_t *xq, int n);
/* finalizeDotQ8VNNI over one row range: 16-row blocks subtract in f32, the
 * tail in int32; then ·scaleX, then ·scale[i] */
void orc_finalize_vnni(const int32_t *dots, const int32_t *rowsum, const float *scale, float *out, int n,
                       float scale_x);
/* the same plain matvec on a matrix unpacked once (as the model keeps its
 * weights), for timing the CPU path without the per-call unpack; the handle
 * borrows m's scale array */
typedef struct orc_prepared orc_prepared;
orc_prepared *orc_prepare(const orc_qmat *m);
void orc_prepared_matvec(const orc_prepared *p, const float *x, float *out);
void orc_prepared_free(orc_prepared *p);

/* ---- small vector ops (a6-a13 pieces) ---- */
float orc_fast_exp(float x);
float orc_fast_rsqrt(float x);
float orc_silu(float x);
void orc_softmax(float *x, int n);
void orc_rmsnorm(float *out, const float *x, const float *w, int n, float eps);
void orc_add_rmsnorm(float *out, float *dst, const float *add, const float *w, int n, float eps);
void orc_add_rmsnorm_out_only(float *out, const float *dst, const float *add, const float *w, int n, float eps);
int orc_argmax(const float *x, int n);

/* ---- RoPE (a7) ---- */
void orc_rope_init(double theta, int head_dim, const int *sections, int n_sections,
                   double *freq, uint8_t *axis);
void orc_rope_table(const double *freq, const uint8_t *axis, int half, int t, int h, int w,
                    float *cos_t, float *sin_t);
void orc_apply_rope(float *x, const float *cos_t, const float *sin_t, int heads, int dim);

/* ---- attention over an fp32 cache (a9) ---- */
void orc_cache_attention(float *out, const float *q, const float *kcache, const float *vcache,
                         int len, int heads, int kv_heads, int dim);

/* ---- multimodal positions (a15) ---- */
int orc_mm_positions(const int32_t *ids, int n, int image_token_id, const int32_t grid[3],
                     int merge, int32_t *pos3 /* [n][3] */, int *rope_delta);

/* ---- the model (a14, a15) ---- */
typedef struct orc_model orc_model;
typedef struct orc_seq orc_seq;

orc_model *orc_model_create(int hidden, int inter, int layers, int heads, int kv_heads,
                            int head_dim, int vocab, float eps, double rope_theta);
void orc_model_free(orc_model *m);
/* which: 0=q 1=k 2=v 3=o 4=gate 5=up 6=down; layer -1 & which 7 = lm_head */
int orc_model_set_matrix(orc_model *m, int layer, int which, int qtype, int rows, int cols,
                         const float *scale, const uint8_t *data);
/* which: 0=ln1 1=ln2 ; layer -1 = final norm */
int orc_model_set_norm(orc_model *m, int layer, int which, const float *w);
int orc_model_set_embed(orc_model *m, const float *embed);
/* residual quirk for Q4/Q6 (model.go:3895-3902, 4051-4057): 1 = reproduce (default) */
void orc_model_set_quirk(orc_model *m, int on);
/* activation mode: 0 plain (default), 1 VNNI emulation for Q4/Q6 */
void orc_model_set_vnni(orc_model *m, int on);

orc_seq *orc_seq_create(orc_model *m, int capacity);
void orc_seq_free(orc_seq *s);
void orc_seq_reset(orc_seq *s);
int orc_seq_len(const orc_seq *s);
const float *orc_seq_k(const orc_seq *s, int layer);
const float *orc_seq_v(const orc_seq *s, int layer);
/* copy an externally prepared cache prefix (used for isolated attention tests) */
int orc_seq_load(orc_seq *s, int layer, const float *k, const float *v, int len);

/* one token step (forwardEmbeddingForSampling, model.go:3475-3643).
 * need_logits=0 → non-final prompt token (last layer K/V only).
 * Writes logits (if logits!=NULL) and greedy token (if token!=NULL). */
int orc_step(orc_model *m, orc_seq *s, const float *emb, const int32_t pos3[3], int need_logits,
             float *logits, int32_t *token, float *final_norm_out);

/* whole generation (GenerateWithOptions model.go:1492-1572 and
 * generateWithImageEmbeds 1618-1711, greedy).  image rows replace ids equal to
 * image_token_id in order; grid used for positions.  Returns tokens appended
 * (prompt not included) in out_tokens, count via return value, <0 on error. */
int orc_generate(orc_model *m, const int32_t *ids, int n_ids, const float *image_embeds,
                 int n_image, int image_token_id, const int32_t grid[3], int merge,
                 int max_new, const int32_t *eos, int n_eos, int32_t *out_tokens);

/* ---- vision projector ---- */
/* LayerNorm (ops.go:1060-1097), the scalar path: 8-lane partial sums
 * (sumF32Scalar 1448-1466, sumSquaresCenteredScalar 1468-1490), scale =
 * fastRsqrt(var/n + eps), out = (x − mean)·scale·w + b */
void orc_layernorm(float *out, const float *x, const float *w, const float *b, int n, float eps);
/* GELUTanh (ops.go:1140-1164), fastExpF32T's exponent wrap included */
float orc_gelu_tanh(float x);
/* projectImageRows (vision.go:1066-1108) with Q8 matrices
 * (matVecQ8BiasSerial, quant.go:1443-1473): x [T·H·W][vd] →
 * out [T·(H/2)·(W/2)][td]; q1 [4vd][4vd], q2 [td][4vd].  Returns the rows. */
int orc_project_image(const float *x, int grid_t, int grid_h, int grid_w, int vd, const float *norm_w,
                      const float *norm_b, const orc_qmat *q1, const float *b1, const orc_qmat *q2, const float *b2,
                      float eps, float *out);

/* ---- sampling LM head ---- */
/* fastRNG.Float64 (model.go:1829-1840): one SplitMix64 step of *state, the
 * top 53 bits of the mixed word as a double in [0, 1) */
double orc_rng_float64(uint64_t *state);
/* topKSelectWithWork (topk.go:322-345): the min(k, n) best of scores[0..n),
 * score descending, equal scores by lower index.  Returns the count. */
int orc_topk(const float *scores, int n, int k, int32_t *ids, float *out_scores);
/* sampleCandidateScoresScratch (model.go:1950-1990) over candidates sorted
 * as orc_topk returns them, with the branches it takes: temperature 1 →
 * sampleCandidateScoresTemp1Small (n <= 4, model.go:2139-2200) or
 * sampleCandidateScoresTemp1Scratch (model.go:2040-2063, f32 weights and
 * sums, pickWeightedRawFloat32 2418-2456); otherwise
 * sampleCandidateScoresSmall (n <= 4, model.go:1992-2038) or f64 sums with
 * f32-stored weights (pickWeightedFloat32 2342-2416).  Draws one value from
 * *state unless n <= 1.  Returns the chosen id. */
int32_t orc_sample_candidates(const int32_t *ids, const float *scores, int n, double temperature, uint64_t *state);
/* CumulativeSum (cumsum.go:9-58): one running sum below 4096 entries, else
 * four zero-based block sums shifted by the running block totals.  out may
 * be x.  Returns the running total of the block sums. */
float orc_cumsum(float *out, const float *x, int n);
/* pickCumulativeFloat32 (model.go:2326-2340): first i with pick <= cdf[i] by
 * binary search, -1 past the end */
int orc_pick_cumulative(const float *cdf, int n, float pick);
/* sampleFullLogitsScratch (model.go:2215-2307) with the generation scratch's
 * weight buffer and the portable ExpScaledVec (FastExpF32 per entry, f32
 * running sum); draws one value from *state.  Returns the chosen index. */
int32_t orc_sample_full(const float *logits, int n, double temperature, uint64_t *state);
/* orc_generate with GenerateOptions sampling (model.go:1538-1568, 1846-1879,
 * 3632-3638): temperature > 0 and top_k != 1 samples every token with a
 * generator seeded by seed — from the top_k candidates of the LM-head scores
 * when 1 < top_k < vocab, from all of them (orc_sample_full) when top_k is 0
 * or >= vocab; otherwise greedy.  Returns as orc_generate. */
int orc_generate_sampled(orc_model *m, const int32_t *ids, int n_ids, const float *image_embeds, int n_image,
                         int image_token_id, const int32_t grid[3], int merge, int max_new, const int32_t *eos,
                         int n_eos, double temperature, int top_k, uint64_t seed, int32_t *out_tokens);

/* thread pool for the CPU baseline (parallelForMax, ops.go:570-614) */
void orc_set_threads(int n);
int orc_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
