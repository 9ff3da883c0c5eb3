/*
 * pocr_oracle.c — CPU restatement of RapidOCRvl's pure-Go text-decoder path.
 *
 * TEST INFRASTRUCTURE ONLY: this is the parity oracle and the CPU baseline.
 * The HIP library never links or calls it.
 *
 * Build with -ffp-contract=off: Go evaluates a*b+c as two rounded operations
 * on the scalar paths restated here, so contraction into FMA must not happen.
 *
 * Reference files (paths relative to the RapidOCRvl repository root):
 *   internal/tensor/quant.go, ops.go, fused_matvec2.go, weighted_sum.go,
 *   argmax_quant.go, dot_amd64.go, dot_other.go, dot_vnni_amd64.s
 *   internal/model/model.go
 *
 * Pinning (see tests/test_oracle_*.py):
 *   encoders/unpack           bit-exact: golden vectors + exhaustive byte tables
 *   matvec plain              brute force in f64 on exact-arithmetic inputs;
 *                             tolerance otherwise (the Go FMA asm accumulation
 *                             order is parity unpinned at the ulp level)
 *   FastExp/fastRsqrt/SiLU    closed forms from ops.go:1092-1112,1374-1381
 *   softmax / attention       f64 brute force + reference KATs
 *   RoPE table/apply          f64 recomputation + model/rope_test.go KATs
 *   positions                 model/position_test.go vectors (exact)
 *   step quirk                2-layer toy model where the quirk changes h
 */
#define _GNU_SOURCE
#include "pocr_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* thread pool — parallelForMax (ops.go:596-614): worker w gets rows   */
/* [w*n/workers, (w+1)*n/workers)                                      */
/*                                                                     */
/* Goroutines cannot lose a job; this pool keeps that property:        */
/*  - each worker is created knowing the job generation current at its */
/*    creation, so a job posted before it first runs is still seen;    */
/*  - an idle worker spins briefly, then parks on job_cv; the poster   */
/*    bumps gen and broadcasts under mu, and a parking worker re-checks */
/*    gen under mu, so no wake-up falls between check and wait;        */
/*  - the caller waits for every worker to report the job (done_cv,    */
/*    same discipline), so a worker never skips a generation;          */
/*  - concurrent callers (ctypes releases the GIL) serialize on api,   */
/*    and a call made from inside a job runs inline.                   */
/* ------------------------------------------------------------------ */
typedef void (*range_fn)(void *ctx, int start, int end);

#define ORC_MAX_THREADS 256
#define ORC_SPIN 4000
static struct {
    int nthreads;
    pthread_t th[ORC_MAX_THREADS];
    atomic_uint gen;
    atomic_int done;
    atomic_int stop;
    range_fn fn;
    void *ctx;
    int n, workers;
    pthread_mutex_t api; /* one job (or one resize) at a time */
    pthread_mutex_t mu;  /* guards the parks on job_cv / done_cv */
    pthread_cond_t job_cv, done_cv;
} P = {.nthreads = 1,
       .api = PTHREAD_MUTEX_INITIALIZER,
       .mu = PTHREAD_MUTEX_INITIALIZER,
       .job_cv = PTHREAD_COND_INITIALIZER,
       .done_cv = PTHREAD_COND_INITIALIZER};

static _Thread_local int tl_in_job;

typedef struct {
    int id;
    unsigned start_gen;
} worker_arg;
static worker_arg P_args[ORC_MAX_THREADS];

static unsigned wait_gen_change(unsigned seen) {
    unsigned g;
    for (int spins = 0; spins < ORC_SPIN; spins++) {
        g = atomic_load_explicit(&P.gen, memory_order_acquire);
        if (g != seen) return g;
    }
    pthread_mutex_lock(&P.mu);
    while ((g = atomic_load_explicit(&P.gen, memory_order_acquire)) == seen) pthread_cond_wait(&P.job_cv, &P.mu);
    pthread_mutex_unlock(&P.mu);
    return g;
}

static void *pool_worker(void *arg) {
    const worker_arg *a = (const worker_arg *)arg;
    const int id = a->id;
    unsigned seen = a->start_gen;
    tl_in_job = 1;
    for (;;) {
        seen = wait_gen_change(seen);
        if (atomic_load(&P.stop)) return NULL;
        if (id < P.workers) {
            int s = (int)((long)id * P.n / P.workers);
            int e = (int)((long)(id + 1) * P.n / P.workers);
            P.fn(P.ctx, s, e);
        }
        if (atomic_fetch_add_explicit(&P.done, 1, memory_order_acq_rel) + 1 == P.nthreads - 1) {
            pthread_mutex_lock(&P.mu);
            pthread_cond_broadcast(&P.done_cv);
            pthread_mutex_unlock(&P.mu);
        }
    }
}

static void post_gen(void) {
    pthread_mutex_lock(&P.mu);
    atomic_fetch_add_explicit(&P.gen, 1, memory_order_acq_rel);
    pthread_cond_broadcast(&P.job_cv);
    pthread_mutex_unlock(&P.mu);
}

/* caller holds P.api */
static void pool_stop(void) {
    if (P.nthreads <= 1) return;
    atomic_store(&P.stop, 1);
    post_gen();
    for (int i = 1; i < P.nthreads; i++) pthread_join(P.th[i], NULL);
    atomic_store(&P.stop, 0);
    P.nthreads = 1;
}

void orc_set_threads(int n) {
    pthread_mutex_lock(&P.api);
    if (n < 1) n = 1;
    if (n > ORC_MAX_THREADS) n = ORC_MAX_THREADS;
    pool_stop();
    const unsigned g = atomic_load(&P.gen);
    int made = 1;
    for (int i = 1; i < n; i++) {
        P_args[i].id = i;
        P_args[i].start_gen = g;
        if (pthread_create(&P.th[i], NULL, pool_worker, &P_args[i]) != 0) break;
        made++;
    }
    P.nthreads = made;
    pthread_mutex_unlock(&P.api);
}

int orc_get_threads(void) { return P.nthreads; }

static void parallel_for_max(int n, int max_workers, range_fn fn, void *ctx) {
    int workers = max_workers < n ? max_workers : n;
    if (workers > P.nthreads) workers = P.nthreads;
    if (workers <= 1 || tl_in_job) {
        fn(ctx, 0, n);
        return;
    }
    pthread_mutex_lock(&P.api);
    if (workers > P.nthreads) workers = P.nthreads; /* resized while we waited */
    if (workers <= 1) {
        pthread_mutex_unlock(&P.api);
        fn(ctx, 0, n);
        return;
    }
    P.fn = fn;
    P.ctx = ctx;
    P.n = n;
    P.workers = workers;
    atomic_store(&P.done, 0);
    post_gen();
    tl_in_job = 1;
    fn(ctx, 0, n / workers);
    tl_in_job = 0;
    const int need = P.nthreads - 1;
    int spins = 0;
    while (atomic_load_explicit(&P.done, memory_order_acquire) < need && ++spins < ORC_SPIN) {
    }
    if (atomic_load_explicit(&P.done, memory_order_acquire) < need) {
        pthread_mutex_lock(&P.mu);
        while (atomic_load_explicit(&P.done, memory_order_acquire) < need) pthread_cond_wait(&P.done_cv, &P.mu);
        pthread_mutex_unlock(&P.mu);
    }
    pthread_mutex_unlock(&P.api);
}

/* ------------------------------------------------------------------ */
/* formats (a2, a3)                                                    */
/* ------------------------------------------------------------------ */

/* roundToInt: quant.go:436-441 — f32 add of ±0.5 then truncation */
int orc_round_to_int(float x) {
    if (x >= 0) return (int)(x + 0.5f);
    return (int)(x - 0.5f);
}

static int round_rne(float x) { return (int)rintf(x); }

size_t orc_row_bytes(int qtype, int cols) {
    switch (qtype) {
    case ORC_Q8: return (size_t)cols;
    case ORC_Q4: return (size_t)(cols + 1) / 2;
    case ORC_Q6: return (size_t)(cols * 6 + 7) / 8; /* PackedQ6Cols quant.go:2882 */
    }
    return 0;
}

/* maxAbsFloat32 (quant.go:397-434): max is order independent */
static float max_abs(const float *x, int n) {
    float m = 0;
    for (int i = 0; i < n; i++) {
        float a = x[i] < 0 ? -x[i] : x[i];
        if (a > m) m = a;
    }
    return m;
}

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* putQ6 (quant.go:2886-2895): OR the 6-bit code at bit 6*col, little endian */
static void put_q6(uint8_t *row, size_t row_len, int col, uint8_t v) {
    int bit = col * 6;
    int idx = bit / 8;
    int shift = bit % 8;
    uint16_t x = (uint16_t)((v & 0x3F) << shift);
    row[idx] |= (uint8_t)x;
    if ((size_t)idx + 1 < row_len) row[idx + 1] |= (uint8_t)(x >> 8);
}

/* getQ6 (quant.go:2897-2906) */
static uint8_t get_q6(const uint8_t *row, size_t row_len, int col) {
    int bit = col * 6;
    int idx = bit / 8;
    int shift = bit % 8;
    uint16_t x = row[idx];
    if ((size_t)idx + 1 < row_len) x |= (uint16_t)row[idx + 1] << 8;
    return (uint8_t)((x >> shift) & 0x3F);
}

/*
 * Row encoders.
 *   Q8: QuantizeQ8RowBytesInto quant.go:96-137 (+quantInt8 139-147)
 *   Q4: QuantizeQ4RowInto quant.go:291-354 (+q4Nib 357-365)
 *   Q6: QuantizeQ6RowInto quant.go:201-270 (+quantByte6 272-280)
 * scale = maxAbs/{127,7,31}; inv = 1/scale; code = clamp(round(w*inv));
 * all-zero row → zero bytes, scale 1.
 */
float orc_quantize_row(int qtype, int tie_mode, const float *w, int cols, uint8_t *out) {
    size_t nb = orc_row_bytes(qtype, cols);
    float maxv = max_abs(w, cols);
    if (maxv == 0) {
        memset(out, 0, nb);
        return 1.0f;
    }
    float qmax = qtype == ORC_Q8 ? 127.0f : (qtype == ORC_Q4 ? 7.0f : 31.0f);
    float scale = maxv / qmax;
    float inv = 1.0f / scale;
    int lim = (int)qmax;
    if (qtype == ORC_Q8) {
        for (int i = 0; i < cols; i++) out[i] = (uint8_t)(int8_t)clampi(orc_round_to_int(w[i] * inv), -127, 127);
        return scale;
    }
    memset(out, 0, nb);
    if (qtype == ORC_Q4) {
        int rne = tie_mode == ORC_TIE_AMD64 && cols >= 8;
        for (int i = 0; i < cols; i++) {
            float v = w[i] * inv;
            int r = rne ? round_rne(v) : orc_round_to_int(v);
            uint8_t nib = (uint8_t)(clampi(r, -lim, lim) + 8);
            if (i & 1) out[i / 2] |= (uint8_t)(nib << 4);
            else out[i / 2] |= nib;
        }
        return scale;
    }
    /* Q6 */
    int prefix = (tie_mode == ORC_TIE_AMD64 && cols >= 8) ? (cols / 8) * 8 : 0;
    for (int i = 0; i < cols; i++) {
        float v = w[i] * inv;
        int r = i < prefix ? round_rne(v) : orc_round_to_int(v);
        put_q6(out, nb, i, (uint8_t)(clampi(r, -lim, lim) + 32));
    }
    return scale;
}

/* unpack: q8ValueTable quant.go:2314-2320, unpackQ4RowFast 2358-2368
 * (q4Int8Table 2356: nibble-8), unpackQ6RowFast 2634-2656 (q6Int8Table 2592: code-32) */
void orc_unpack_row(int qtype, const uint8_t *row, int cols, int8_t *out) {
    size_t nb = orc_row_bytes(qtype, cols);
    switch (qtype) {
    case ORC_Q8:
        for (int c = 0; c < cols; c++) out[c] = (int8_t)row[c];
        break;
    case ORC_Q4:
        for (int c = 0; c < cols; c++) {
            uint8_t b = row[c / 2];
            out[c] = (int8_t)(((c & 1) ? (b >> 4) : (b & 0x0F)) - 8);
        }
        break;
    case ORC_Q6:
        for (int c = 0; c < cols; c++) out[c] = (int8_t)(get_q6(row, nb, c) - 32);
        break;
    }
}

/* ------------------------------------------------------------------ */
/* dots                                                                */
/* ------------------------------------------------------------------ */

/* dotQ8Scalar (quant.go:2179-2198): 8 f32 lanes, lane j accumulates
 * (a[i+j]*b[i+j] + a[i+8+j]*b[i+8+j]) per 16-block, then pairwise, then tail */
static float dot_i8(const int8_t *a, const float *b, int n) {
    float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 15 < n; i += 16)
        for (int j = 0; j < 8; j++) s[j] += (float)a[i + j] * b[i + j] + (float)a[i + 8 + j] * b[i + 8 + j];
    float sum = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
    for (; i < n; i++) sum += (float)a[i] * b[i];
    return sum;
}

/* dotF32Scalar-style 8-lane f32 dot (ops.go:626-645) */
static float dot_f32(const float *a, const float *b, int n) {
    float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 7 < n; i += 8)
        for (int j = 0; j < 8; j++) s[j] += a[i + j] * b[i + j];
    float sum = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
    for (; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* sumSquaresScalar (ops.go:1039-1058) */
static float sum_squares(const float *x, int n) {
    float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 7 < n; i += 8)
        for (int j = 0; j < 8; j++) s[j] += x[i + j] * x[i + j];
    float ss = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
    for (; i < n; i++) ss += x[i] * x[i];
    return ss;
}

/* ------------------------------------------------------------------ */
/* matvec                                                              */
/* ------------------------------------------------------------------ */

/* An unpacked view: int8 codes + row sums, as UnpackQ4Matrix/UnpackQ6Matrix
 * build at load (quant.go:2325-2354, 2605-2632). */
typedef struct {
    orc_qmat q;
    int8_t *codes;   /* rows*cols */
    int32_t *rowsum; /* rows */
} umat;

static void umat_build(umat *u, const orc_qmat *q) {
    u->q = *q;
    size_t nb = orc_row_bytes(q->qtype, q->cols);
    u->codes = (int8_t *)malloc((size_t)q->rows * q->cols);
    u->rowsum = (int32_t *)malloc(sizeof(int32_t) * (size_t)q->rows);
    for (int r = 0; r < q->rows; r++) {
        int8_t *dst = u->codes + (size_t)r * q->cols;
        orc_unpack_row(q->qtype, q->data + (size_t)r * nb, q->cols, dst);
        int32_t s = 0;
        for (int c = 0; c < q->cols; c++) s += dst[c];
        u->rowsum[r] = s;
    }
}

static void umat_free(umat *u) {
    free(u->codes);
    free(u->rowsum);
    u->codes = NULL;
    u->rowsum = NULL;
}

typedef struct {
    const umat *u;
    const float *x;
    float *out;
    const uint8_t *xq;
    float scale_x;
} mv_ctx;

/* matVecQ8Serial / matVecQ4Serial / matVecQ6Serial plain branch
 * (quant.go:1356-1384, 1853-1888, 1816-1851): out[r] = dot(q_r, x) * scale[r] */
static void mv_plain_range(void *vctx, int s, int e) {
    mv_ctx *c = (mv_ctx *)vctx;
    const umat *u = c->u;
    for (int r = s; r < e; r++)
        c->out[r] = dot_i8(u->codes + (size_t)r * u->q.cols, c->x, u->q.cols) * u->q.scale[r];
}

/* dotQ8VNNICore (dot_amd64.go:150-167 with useVNNI; VPDPBUSD in
 * dot_vnni_amd64.s): Σ a[i]·xq[i], s8 × u8 products summed in int32 */
int32_t orc_vnni_core(const int8_t *a, const uint8_t *xq, int n) {
    int32_t dot = 0;
    for (int i = 0; i < n; i++) dot += (int32_t)a[i] * (int32_t)xq[i];
    return dot;
}

/* finalizeDotQ8VNNI (dot_vnni_amd64.s:1043-1095) over one worker's row range:
 * blocks of 16 rows convert dot and rowSum to f32 and subtract in f32
 * (VCVTDQ2PS, VMULPS 128, VSUBPS); the n mod 16 tail rows subtract in int32
 * (IMULL 128, SUBL, wrapping) and convert the difference. Both then multiply
 * by scaleX, then by scale[i]. The forms agree while |dot| and |128·rowSum|
 * stay below 2^24. */
void orc_finalize_vnni(const int32_t *dots, const int32_t *rowsum, const float *scale, float *out, int n,
                       float scale_x) {
    int i = 0;
    for (; i + 16 <= n; i += 16)
        for (int j = i; j < i + 16; j++) {
            float v = (float)dots[j] - (float)rowsum[j] * 128.0f;
            v = v * scale_x;
            out[j] = v * scale[j];
        }
    for (; i < n; i++) {
        int32_t d = (int32_t)((uint32_t)dots[i] - (uint32_t)rowsum[i] * 128u);
        float v = (float)d * scale_x;
        out[i] = v * scale[i];
    }
}

/* matVecQ8Serial's VNNI branch (quant.go:1356-1373; the Q4/Q6 serial
 * functions 1816-1851, 1853-1888 have the same shape): the integer core for
 * the worker's rows into scratch, then one finalize over the range */
static void mv_vnni_range(void *vctx, int s, int e) {
    mv_ctx *c = (mv_ctx *)vctx;
    const umat *u = c->u;
    int cols = u->q.cols;
    if (e <= s) return;
    int32_t *dots = (int32_t *)malloc(sizeof(int32_t) * (size_t)(e - s));
    for (int r = s; r < e; r++) dots[r - s] = orc_vnni_core(u->codes + (size_t)r * cols, c->xq, cols);
    orc_finalize_vnni(dots, u->rowsum + s, u->q.scale + s, c->out + s, e - s, c->scale_x);
    free(dots);
}

/* shouldParallelQuantMatVec / parallelForQuantMatVec (quant.go:563-599):
 * parallel when rows*cols >= parallelWork/2 and rows >= 512; otherwise
 * shouldParallel (ops.go:574-579) with at most 8 workers for <=512 rows. */
static void run_rows(int rows, int cols, range_fn fn, void *ctx) {
    long work = (long)rows * cols;
    int par = (work >= (1L << 17) && rows >= 512) || (work >= (1L << 18) && rows >= 4);
    if (!par || P.nthreads <= 1) {
        fn(ctx, 0, rows);
        return;
    }
    parallel_for_max(rows, rows <= 512 ? 8 : P.nthreads, fn, ctx);
}

/* quantizeXForVNNIAVX2 (dot_amd64.go:228-252) + quantizeXForVNNIAsm
 * (dot_vnni_amd64.s:434-500): xq = clamp(RNE(x*inv)+128, 0, 255); x==0 → 128 */
float orc_quantize_x_vnni(const float *x, int n, uint8_t *xq) {
    float m = max_abs(x, n);
    if (m == 0) {
        memset(xq, 128, (size_t)n);
        return 1.0f;
    }
    float scale = m / 127.0f;
    float inv = 1.0f / scale;
    for (int i = 0; i < n; i++) {
        float v = rintf(x[i] * inv) + 128.0f;
        if (v < 0) v = 0;
        if (v > 255) v = 255;
        xq[i] = (uint8_t)(int)v;
    }
    return scale;
}

static void umat_matvec(const umat *u, const float *x, float *out, int vnni) {
    mv_ctx c = {u, x, out, NULL, 0};
    if (vnni && u->q.qtype != ORC_Q8 && u->q.cols >= 32) {
        uint8_t *xq = (uint8_t *)malloc((size_t)u->q.cols);
        c.scale_x = orc_quantize_x_vnni(x, u->q.cols, xq);
        c.xq = xq;
        run_rows(u->q.rows, u->q.cols, mv_vnni_range, &c);
        free(xq);
        return;
    }
    run_rows(u->q.rows, u->q.cols, mv_plain_range, &c);
}

void orc_matvec(const orc_qmat *m, const float *x, float *out) {
    umat u;
    umat_build(&u, m);
    umat_matvec(&u, x, out, 0);
    umat_free(&u);
}

struct orc_prepared {
    umat u;
};

orc_prepared *orc_prepare(const orc_qmat *m) {
    orc_prepared *p = (orc_prepared *)malloc(sizeof(orc_prepared));
    if (p) umat_build(&p->u, m);
    return p;
}

void orc_prepared_matvec(const orc_prepared *p, const float *x, float *out) { umat_matvec(&p->u, x, out, 0); }

void orc_prepared_free(orc_prepared *p) {
    if (!p) return;
    umat_free(&p->u);
    free(p);
}

void orc_matvec_vnni(const orc_qmat *m, const float *x, float *out) {
    umat u;
    umat_build(&u, m);
    umat_matvec(&u, x, out, 1);
    umat_free(&u);
}

/* ------------------------------------------------------------------ */
/* vector ops                                                          */
/* ------------------------------------------------------------------ */

static float bits_to_f32(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}
static uint32_t f32_to_bits(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    return b;
}

/* FastExpF32 (ops.go:1099-1112): t=x*log2e; n=RNE(t) via magic; 5th-degree
 * 2^f polynomial; result bits = bits(poly) + n<<23 */
float orc_fast_exp(float x) {
    const float log2e = 1.4426950408889634f;
    const float magic = 12582912.0f;
    float t = x * log2e;
    int32_t n = (int32_t)((t + magic) - magic);
    float f = t - (float)n;
    float f2 = f * f;
    float poly = (1.0f + 0.6931471824645996f * f) +
                 f2 * (0.24022650718688965f + 0.05550410971045494f * f +
                       f2 * (0.009618128649890423f + 0.0013352063251659274f * f));
    uint32_t bits = f32_to_bits(poly) + ((uint32_t)n << 23);
    return bits_to_f32(bits);
}

/* fastRsqrtF32 (ops.go:1374-1381) */
float orc_fast_rsqrt(float x) {
    float half = x * 0.5f;
    uint32_t i = 0x5f3759dfu - (f32_to_bits(x) >> 1);
    float y = bits_to_f32(i);
    y = y * (1.5f - half * y * y);
    return y * (1.5f - half * y * y);
}

/* SiLU (ops.go:1092-1094) */
float orc_silu(float x) { return x / (1.0f + orc_fast_exp(-x)); }

static float max32(float a, float b) { return b > a ? b : a; }

/* SoftmaxInPlace (ops.go:1199-1363): hand-specialised n=1..8, else max,
 * ExpVec (weighted_sum.go:213-227) sequential sum, multiply by 1/sum */
void orc_softmax(float *x, int n) {
    if (n <= 0) return;
    if (n == 1) {
        x[0] = 1;
        return;
    }
    if (n == 2) {
        float a = x[0], b = x[1];
        if (a >= b) {
            float e = orc_fast_exp(b - a);
            float inv = 1 / (1 + e);
            x[0] = inv;
            x[1] = e * inv;
        } else {
            float e = orc_fast_exp(a - b);
            float inv = 1 / (1 + e);
            x[0] = e * inv;
            x[1] = inv;
        }
        return;
    }
    if (n <= 8) {
        float m;
        switch (n) {
        case 3: m = max32(max32(x[0], x[1]), x[2]); break;
        case 4: m = max32(max32(x[0], x[1]), max32(x[2], x[3])); break;
        case 5: m = max32(max32(max32(x[0], x[1]), max32(x[2], x[3])), x[4]); break;
        case 6: m = max32(max32(max32(x[0], x[1]), max32(x[2], x[3])), max32(x[4], x[5])); break;
        case 7: m = max32(max32(max32(x[0], x[1]), max32(x[2], x[3])), max32(max32(x[4], x[5]), x[6])); break;
        default:
            m = max32(max32(max32(x[0], x[1]), max32(x[2], x[3])), max32(max32(x[4], x[5]), max32(x[6], x[7])));
        }
        float e[8];
        for (int i = 0; i < n; i++) e[i] = orc_fast_exp(x[i] - m);
        float sum;
        switch (n) {
        case 3: sum = e[0] + e[1] + e[2]; break;
        case 4: sum = (e[0] + e[1]) + (e[2] + e[3]); break;
        case 5: sum = (e[0] + e[1]) + (e[2] + e[3]) + e[4]; break;
        case 6: sum = (e[0] + e[1]) + (e[2] + e[3]) + (e[4] + e[5]); break;
        case 7: sum = (e[0] + e[1]) + (e[2] + e[3]) + (e[4] + e[5]) + e[6]; break;
        default: sum = (e[0] + e[1]) + (e[2] + e[3]) + (e[4] + e[5]) + (e[6] + e[7]);
        }
        float inv = 1 / sum;
        for (int i = 0; i < n; i++) x[i] = e[i] * inv;
        return;
    }
    float m = -INFINITY;
    for (int i = 0; i < n; i++) m = max32(m, x[i]);
    float sum = 0;
    for (int i = 0; i < n; i++) {
        float e = orc_fast_exp(x[i] - m);
        x[i] = e;
        sum += e;
    }
    float inv = 1 / sum;
    for (int i = 0; i < n; i++) x[i] *= inv;
}

/* RMSNorm (ops.go:1015-1037): out = x * fastRsqrt(ss/n+eps) * w */
void orc_rmsnorm(float *out, const float *x, const float *w, int n, float eps) {
    float ss = sum_squares(x, n);
    float scale = orc_fast_rsqrt(ss / (float)n + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

/* AddRMSNorm (ops.go:913-935): dst += add (in place), out = RMSNorm(dst) */
void orc_add_rmsnorm(float *out, float *dst, const float *add, const float *w, int n, float eps) {
    for (int i = 0; i < n; i++) dst[i] = dst[i] + add[i];
    float ss = sum_squares(dst, n);
    float scale = orc_fast_rsqrt(ss / (float)n + eps);
    for (int i = 0; i < n; i++) out[i] = dst[i] * scale * w[i];
}

/* AddRMSNormOutOnly (fused_matvec2.go:11-33): out = RMSNorm(dst + add), dst kept */
void orc_add_rmsnorm_out_only(float *out, const float *dst, const float *add, const float *w, int n,
                              float eps) {
    for (int i = 0; i < n; i++) out[i] = dst[i] + add[i];
    float ss = sum_squares(out, n);
    float scale = orc_fast_rsqrt(ss / (float)n + eps);
    for (int i = 0; i < n; i++) out[i] = out[i] * scale * w[i];
}

/* Argmax with ties → lowest index (argmax_quant.go:255-262: score > best) */
int orc_argmax(const float *x, int n) {
    if (n <= 0) return 0;
    int best = 0;
    float bv = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > bv) {
            bv = x[i];
            best = i;
        }
    return best;
}

/* ------------------------------------------------------------------ */
/* RoPE                                                                */
/* ------------------------------------------------------------------ */

/* initTextRoPE (model.go:877-902): freq_i = theta^(-2i/d) in f64; axis from
 * the mrope sections (default [16,24,24]) clamped to 2 */
void orc_rope_init(double theta, int head_dim, const int *sections, int n_sections, double *freq,
                   uint8_t *axis) {
    static const int def[3] = {16, 24, 24};
    if (!sections || n_sections <= 0) {
        sections = def;
        n_sections = 3;
    }
    int half = head_dim / 2;
    int section_end = sections[0];
    int ax = 0;
    for (int i = 0; i < half; i++) {
        while (ax + 1 < n_sections && i >= section_end) {
            ax++;
            section_end += sections[ax];
        }
        axis[i] = (uint8_t)(ax > 2 ? 2 : ax);
        freq[i] = pow(theta, -(double)(2 * i) / (double)head_dim);
    }
}

/* buildMRoPETable (model.go:7318-7357): pos (0,0,0) → cos 1, sin 0;
 * ang = f64(p_axis) * freq_i; cos/sin in f64 rounded to f32 (7397-7398) */
void orc_rope_table(const double *freq, const uint8_t *axis, int half, int t, int h, int w,
                    float *cos_t, float *sin_t) {
    if (t == 0 && h == 0 && w == 0) {
        for (int i = 0; i < half; i++) {
            cos_t[i] = 1;
            sin_t[i] = 0;
        }
        return;
    }
    for (int i = 0; i < half; i++) {
        int p = t;
        if (axis[i] == 1) p = h;
        else if (axis[i] == 2) p = w;
        double ang = (double)p * freq[i];
        cos_t[i] = (float)cos(ang);
        sin_t[i] = (float)sin(ang);
    }
}

/* ApplyMRoPETable (weighted_sum.go:231-250): rotate-half pairs (i, i+half) */
void orc_apply_rope(float *x, const float *cos_t, const float *sin_t, int heads, int dim) {
    int half = dim / 2;
    for (int h = 0; h < heads; h++) {
        float *b = x + (size_t)h * dim;
        for (int i = 0; i < half; i++) {
            float cs = cos_t[i], sn = sin_t[i];
            float a = b[i], c = b[half + i];
            b[i] = a * cs - c * sn;
            b[half + i] = c * cs + a * sn;
        }
    }
}

/* ------------------------------------------------------------------ */
/* attention over the fp32 cache                                       */
/* ------------------------------------------------------------------ */

/* one head: cacheAttentionScores (model.go:4623-4795) → SoftmaxInPlace →
 * weightedCacheValueSum (5201-5590); len==1 → copy V (copyCacheValue 4603).
 * Cache row t of kv head g starts at t*kvDim + g*dim (kvCache.key 5626). */
static void attend_head(float *dst, const float *q, const float *kc, const float *vc, int len,
                        int kvh, int kv_dim, int dim, float scale, float *scores) {
    int hb = kvh * dim;
    if (len == 1) {
        memcpy(dst, vc + hb, sizeof(float) * dim);
        return;
    }
    for (int t = 0; t < len; t++) scores[t] = dot_f32(q, kc + (size_t)t * kv_dim + hb, dim) * scale;
    orc_softmax(scores, len);
    /* ScaleCopy then ScaleAdd in token order (weightedCacheValueSum128 5479-5515) */
    for (int d = 0; d < dim; d++) dst[d] = scores[0] * vc[hb + d];
    for (int t = 1; t < len; t++) {
        const float *v = vc + (size_t)t * kv_dim + hb;
        float a = scores[t];
        for (int d = 0; d < dim; d++) dst[d] += a * v[d];
    }
}

typedef struct {
    float *out;
    const float *q, *kc, *vc;
    int len, heads, kv_heads, dim;
    float scale;
    float *scores; /* heads*len */
} attn_ctx;

static void attn_range(void *vctx, int s, int e) {
    attn_ctx *c = (attn_ctx *)vctx;
    int group = c->heads / c->kv_heads;
    for (int h = s; h < e; h++)
        attend_head(c->out + (size_t)h * c->dim, c->q + (size_t)h * c->dim, c->kc, c->vc, c->len, h / group,
                    c->kv_heads * c->dim, c->dim, c->scale, c->scores + (size_t)h * c->len);
}

/* invSqrt (model.go:7391): f32(1/sqrt(f64(dim))) */
static float inv_sqrt_dim(int dim) { return (float)(1.0 / sqrt((double)dim)); }

static void cache_attention_scratch(float *out, const float *q, const float *kc, const float *vc, int len,
                                    int heads, int kv_heads, int dim, float *scores) {
    attn_ctx c = {out, q, kc, vc, len, heads, kv_heads, dim, inv_sqrt_dim(dim), scores};
    /* head-parallel goroutines when heads>=8 && len>=64 (model.go:4001-4031) */
    if (heads >= 8 && len >= 64 && P.nthreads > 1) {
        int workers = heads < P.nthreads ? heads : P.nthreads;
        parallel_for_max(heads, workers, attn_range, &c);
    } else {
        attn_range(&c, 0, heads);
    }
}

void orc_cache_attention(float *out, const float *q, const float *kc, const float *vc, int len, int heads,
                         int kv_heads, int dim) {
    float *scores = (float *)malloc(sizeof(float) * (size_t)heads * (len > 0 ? len : 1));
    cache_attention_scratch(out, q, kc, vc, len, heads, kv_heads, dim, scores);
    free(scores);
}

/* ------------------------------------------------------------------ */
/* multimodal positions (model.go:1717-1783)                          */
/* ------------------------------------------------------------------ */
int orc_mm_positions(const int32_t *ids, int n, int image_token_id, const int32_t grid[3], int merge,
                     int32_t *pos3, int *rope_delta) {
    int pi = 0, st = 0, next_pos = 0;
    for (;;) {
        int ed = -1;
        for (int i = st; i < n; i++)
            if (ids[i] == image_token_id) {
                ed = i;
                break;
            }
        if (ed < 0) break;
        int st_idx = next_pos;
        for (int i = 0; i < ed - st; i++) {
            int p = st_idx + i;
            pos3[3 * pi] = p;
            pos3[3 * pi + 1] = p;
            pos3[3 * pi + 2] = p;
            pi++;
        }
        int text_len = ed - st;
        int max_pos = st_idx + text_len - 1;
        int gt = grid[0], gh = grid[1] / merge, gw = grid[2] / merge;
        for (int t = 0; t < gt; t++)
            for (int h = 0; h < gh; h++)
                for (int w = 0; w < gw; w++) {
                    if (pi >= n) return -1;
                    int pt = text_len + st_idx + t, ph = text_len + st_idx + h, pw = text_len + st_idx + w;
                    pos3[3 * pi] = pt;
                    pos3[3 * pi + 1] = ph;
                    pos3[3 * pi + 2] = pw;
                    pi++;
                    if (pt > max_pos) max_pos = pt;
                    if (ph > max_pos) max_pos = ph;
                    if (pw > max_pos) max_pos = pw;
                }
        next_pos = max_pos + 1;
        st = ed + gt * gh * gw;
    }
    if (st < n) {
        int st_idx = next_pos;
        for (int i = 0; i < n - st; i++) {
            int p = st_idx + i;
            pos3[3 * pi] = p;
            pos3[3 * pi + 1] = p;
            pos3[3 * pi + 2] = p;
            pi++;
        }
        next_pos = st_idx + n - st;
    }
    *rope_delta = pi == 0 ? 0 : next_pos - n;
    return pi;
}

/* ------------------------------------------------------------------ */
/* model                                                               */
/* ------------------------------------------------------------------ */
enum { W_Q, W_K, W_V, W_O, W_GATE, W_UP, W_DOWN, W_COUNT };

typedef struct {
    umat w[W_COUNT];
    int have[W_COUNT];
    const float *ln1, *ln2;
} orc_layer;

struct orc_model {
    int hidden, inter, layers, heads, kvh, hd, vocab;
    float eps;
    double theta;
    int quirk, vnni;
    orc_layer *L;
    umat lm;
    int have_lm;
    const float *embed, *final_norm;
    double *freq;
    uint8_t *axis;
    /* scratch (generationScratch / layerScratch, model.go:381-405) */
    float *h, *norm, *q, *k, *v, *head_out, *att, *g, *u, *mlp, *logits, *fnorm;
    float *cos_t, *sin_t, *scores;
    int scores_cap;
};

struct orc_seq {
    orc_model *m;
    int cap, len;
    float **k, **v; /* per layer [cap][kvDim] */
};

orc_model *orc_model_create(int hidden, int inter, int layers, int heads, int kv_heads, int head_dim,
                            int vocab, float eps, double rope_theta) {
    if (hidden <= 0 || layers <= 0 || heads <= 0 || kv_heads <= 0 || head_dim <= 0 || heads % kv_heads)
        return NULL;
    orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
    m->hidden = hidden;
    m->inter = inter;
    m->layers = layers;
    m->heads = heads;
    m->kvh = kv_heads;
    m->hd = head_dim;
    m->vocab = vocab;
    m->eps = eps;
    m->theta = rope_theta;
    m->quirk = 1;
    m->L = (orc_layer *)calloc((size_t)layers, sizeof(orc_layer));
    int q_rows = heads * head_dim, kv_rows = kv_heads * head_dim;
    int wide = q_rows > hidden ? q_rows : hidden;
    m->h = (float *)calloc((size_t)hidden, 4);
    m->norm = (float *)calloc((size_t)wide, 4);
    m->q = (float *)calloc((size_t)q_rows, 4);
    m->k = (float *)calloc((size_t)kv_rows, 4);
    m->v = (float *)calloc((size_t)kv_rows, 4);
    m->head_out = (float *)calloc((size_t)q_rows, 4);
    m->att = (float *)calloc((size_t)hidden, 4);
    m->g = (float *)calloc((size_t)inter, 4);
    m->u = (float *)calloc((size_t)inter, 4);
    m->mlp = (float *)calloc((size_t)hidden, 4);
    m->logits = (float *)calloc((size_t)vocab, 4);
    m->fnorm = (float *)calloc((size_t)hidden, 4);
    m->cos_t = (float *)calloc((size_t)head_dim / 2, 4);
    m->sin_t = (float *)calloc((size_t)head_dim / 2, 4);
    m->freq = (double *)calloc((size_t)head_dim / 2, 8);
    m->axis = (uint8_t *)calloc((size_t)head_dim / 2, 1);
    orc_rope_init(rope_theta, head_dim, NULL, 0, m->freq, m->axis);
    return m;
}

void orc_model_free(orc_model *m) {
    if (!m) return;
    for (int l = 0; l < m->layers; l++)
        for (int w = 0; w < W_COUNT; w++)
            if (m->L[l].have[w]) umat_free(&m->L[l].w[w]);
    if (m->have_lm) umat_free(&m->lm);
    free(m->L);
    free(m->h); free(m->norm); free(m->q); free(m->k); free(m->v); free(m->head_out); free(m->att);
    free(m->g); free(m->u); free(m->mlp); free(m->logits); free(m->fnorm); free(m->cos_t);
    free(m->sin_t); free(m->freq); free(m->axis); free(m->scores);
    free(m);
}

int orc_model_set_matrix(orc_model *m, int layer, int which, int qtype, int rows, int cols,
                         const float *scale, const uint8_t *data) {
    if (qtype != ORC_Q8 && qtype != ORC_Q4 && qtype != ORC_Q6) return -1;
    orc_qmat q = {qtype, rows, cols, scale, data};
    if (layer < 0) {
        if (which != 7) return -1;
        if (m->have_lm) umat_free(&m->lm);
        umat_build(&m->lm, &q);
        m->have_lm = 1;
        return 0;
    }
    if (layer >= m->layers || which < 0 || which >= W_COUNT) return -1;
    if (m->L[layer].have[which]) umat_free(&m->L[layer].w[which]);
    umat_build(&m->L[layer].w[which], &q);
    m->L[layer].have[which] = 1;
    return 0;
}

int orc_model_set_norm(orc_model *m, int layer, int which, const float *w) {
    if (layer < 0) {
        m->final_norm = w;
        return 0;
    }
    if (layer >= m->layers) return -1;
    if (which == 0) m->L[layer].ln1 = w;
    else m->L[layer].ln2 = w;
    return 0;
}

int orc_model_set_embed(orc_model *m, const float *embed) {
    m->embed = embed;
    return 0;
}

void orc_model_set_quirk(orc_model *m, int on) { m->quirk = on; }
void orc_model_set_vnni(orc_model *m, int on) { m->vnni = on; }

orc_seq *orc_seq_create(orc_model *m, int capacity) {
    orc_seq *s = (orc_seq *)calloc(1, sizeof(orc_seq));
    s->m = m;
    s->cap = capacity;
    s->k = (float **)calloc((size_t)m->layers, sizeof(float *));
    s->v = (float **)calloc((size_t)m->layers, sizeof(float *));
    size_t n = (size_t)capacity * m->kvh * m->hd;
    for (int l = 0; l < m->layers; l++) {
        s->k[l] = (float *)calloc(n ? n : 1, 4);
        s->v[l] = (float *)calloc(n ? n : 1, 4);
    }
    return s;
}

void orc_seq_free(orc_seq *s) {
    if (!s) return;
    for (int l = 0; l < s->m->layers; l++) {
        free(s->k[l]);
        free(s->v[l]);
    }
    free(s->k);
    free(s->v);
    free(s);
}

void orc_seq_reset(orc_seq *s) { s->len = 0; }
int orc_seq_len(const orc_seq *s) { return s->len; }
const float *orc_seq_k(const orc_seq *s, int layer) { return s->k[layer]; }
const float *orc_seq_v(const orc_seq *s, int layer) { return s->v[layer]; }

int orc_seq_load(orc_seq *s, int layer, const float *k, const float *v, int len) {
    if (len > s->cap || layer < 0 || layer >= s->m->layers) return -1;
    size_t n = (size_t)len * s->m->kvh * s->m->hd;
    memcpy(s->k[layer], k, n * 4);
    memcpy(s->v[layer], v, n * 4);
    s->len = len;
    return 0;
}

static void ensure_scores(orc_model *m, int len) {
    int need = m->heads * len;
    if (need > m->scores_cap) {
        free(m->scores);
        m->scores = (float *)malloc(sizeof(float) * (size_t)need);
        m->scores_cap = need;
    }
}

/* kvCache.append (model.go:5593-5612): row t = current length */
static void kv_append(orc_seq *s, int layer, int slot, const float *k, const float *v) {
    size_t kvd = (size_t)s->m->kvh * s->m->hd;
    memcpy(s->k[layer] + (size_t)slot * kvd, k, kvd * 4);
    memcpy(s->v[layer] + (size_t)slot * kvd, v, kvd * 4);
}

/* MatVecQ*AddRMSNorm (fused_matvec2.go:339,681,1154; in place) and
 * ...OutOnly (514,926,1399): v = residual + W·x; out = RMSNorm(v)·w */
static void matvec_add_rmsnorm(orc_model *m, const umat *W, const float *x, float *residual, float *out,
                               const float *nw, int in_place) {
    umat_matvec(W, x, m->mlp, m->vnni);
    if (in_place) orc_add_rmsnorm(out, residual, m->mlp, nw, W->q.rows, m->eps);
    else orc_add_rmsnorm_out_only(out, residual, m->mlp, nw, W->q.rows, m->eps);
}

/* SwiGLUGateUpQ*Scratch (quant.go:757-772 → matVecQ*SwiGLUScratch 794-1160):
 * g = dot_g·s_g, u = dot_u·s_u, out = SiLU(g)·u (SiLUMulInPlace ops.go:1125) */
static void swiglu(orc_model *m, const orc_layer *L, const float *x) {
    umat_matvec(&L->w[W_GATE], x, m->g, m->vnni);
    umat_matvec(&L->w[W_UP], x, m->u, m->vnni);
    for (int i = 0; i < m->inter; i++) m->g[i] = orc_silu(m->g[i]) * m->u[i];
}

int orc_step(orc_model *m, orc_seq *s, const float *emb, const int32_t pos3[3], int need_logits,
             float *logits, int32_t *token, float *final_norm_out) {
    int H = m->hidden, hd = m->hd, half = hd / 2;
    int q_rows = m->heads * hd;
    if (s->len >= s->cap) return -2;
    memcpy(m->h, emb, sizeof(float) * H);
    int has_rope = pos3[0] != 0 || pos3[1] != 0 || pos3[2] != 0; /* model.go:3485 */
    if (has_rope) orc_rope_table(m->freq, m->axis, half, pos3[0], pos3[1], pos3[2], m->cos_t, m->sin_t);
    int clen = s->len; /* cache length before this token's append */
    for (int li = 0; li < m->layers; li++) {
        orc_layer *L = &m->L[li];
        int last = li + 1 == m->layers;
        /* x = RMSNorm(h)·ln1 (model.go:3574) */
        orc_rmsnorm(m->norm, m->h, L->ln1, H, m->eps);
        if (last && !need_logits) {
            /* attentionCacheOnly (model.go:3650-3668) */
            umat_matvec(&L->w[W_K], m->norm, m->k, m->vnni);
            umat_matvec(&L->w[W_V], m->norm, m->v, m->vnni);
            if (has_rope) orc_apply_rope(m->k, m->cos_t, m->sin_t, m->kvh, hd);
            kv_append(s, li, clen, m->k, m->v);
            s->len = clen + 1;
            return 0;
        }
        int quant_o = L->w[W_O].q.qtype;
        int outonly_quirk = m->quirk && (quant_o == ORC_Q4 || quant_o == ORC_Q6);
        if (clen == 0) {
            /* first-token branch (model.go:3859-3911): no Q projection; head
             * outputs are V expanded over the group (expandValueHeads 4608) */
            umat_matvec(&L->w[W_K], m->norm, m->k, m->vnni);
            umat_matvec(&L->w[W_V], m->norm, m->v, m->vnni);
            if (has_rope) orc_apply_rope(m->k, m->cos_t, m->sin_t, m->kvh, hd);
            kv_append(s, li, 0, m->k, m->v);
            int group = m->heads / m->kvh;
            for (int h = 0; h < m->heads; h++) memcpy(m->head_out + (size_t)h * hd, m->v + (size_t)(h / group) * hd, hd * 4);
            matvec_add_rmsnorm(m, &L->w[W_O], m->head_out, m->h, m->norm, L->ln2, !outonly_quirk);
        } else {
            umat_matvec(&L->w[W_Q], m->norm, m->q, m->vnni);
            umat_matvec(&L->w[W_K], m->norm, m->k, m->vnni);
            umat_matvec(&L->w[W_V], m->norm, m->v, m->vnni);
            if (has_rope) {
                orc_apply_rope(m->q, m->cos_t, m->sin_t, m->heads, hd);
                orc_apply_rope(m->k, m->cos_t, m->sin_t, m->kvh, hd);
            }
            kv_append(s, li, clen, m->k, m->v);
            int len = clen + 1;
            ensure_scores(m, len);
            cache_attention_scratch(m->head_out, m->q, s->k[li], s->v[li], len, m->heads, m->kvh, hd, m->scores);
            /* len<=6 → matVecOutAddRMSNormCPU, in place for every format
             * (model.go:3980-3994 → 3706-3727); otherwise Q8 in place and
             * Q4/Q6 out-only (4043-4058) */
            int in_place = len <= 6 ? 1 : !outonly_quirk;
            matvec_add_rmsnorm(m, &L->w[W_O], m->head_out, m->h, m->norm, L->ln2, in_place);
        }
        (void)q_rows;
        /* MLP: gate/up SwiGLU, then down + residual (in place) + RMSNorm of the
         * next ln1, or final norm out-only on the last layer (model.go:5714-5800) */
        swiglu(m, L, m->norm);
        if (!last) {
            umat_matvec(&L->w[W_DOWN], m->g, m->mlp, m->vnni);
            for (int i = 0; i < H; i++) m->h[i] = m->h[i] + m->mlp[i];
            /* the next layer recomputes RMSNorm(h)·ln1 (model.go:3574) */
        } else {
            matvec_add_rmsnorm(m, &L->w[W_DOWN], m->g, m->h, m->fnorm, m->final_norm, 0);
        }
    }
    s->len = clen + 1;
    if (!need_logits) return 0;
    if (final_norm_out) memcpy(final_norm_out, m->fnorm, sizeof(float) * H);
    /* LM head: logits (matVecMaybeQuant) or greedy argmax (MatVecArgmaxQ*) */
    umat_matvec(&m->lm, m->fnorm, m->logits, m->vnni);
    if (logits) memcpy(logits, m->logits, sizeof(float) * m->vocab);
    if (token) *token = orc_argmax(m->logits, m->vocab);
    return 0;
}

static int is_eos(int id, const int32_t *eos, int n) {
    for (int i = 0; i < n; i++)
        if (eos[i] == id) return 1;
    return 0;
}

/* ---- vision projector ---- */

/* sumF32Scalar (ops.go:1448-1466) */
static float sum8(const float *x, int n) {
    float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 7 < n; i += 8)
        for (int k = 0; k < 8; k++) s[k] += x[i + k];
    float sum = (s[0] + s[1]) + (s[2] + s[3]) + (s[4] + s[5]) + (s[6] + s[7]);
    for (; i < n; i++) sum += x[i];
    return sum;
}

/* sumSquaresCenteredScalar (ops.go:1468-1490) */
static float sum_sq_centered8(const float *x, int n, float mean) {
    float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 7 < n; i += 8)
        for (int k = 0; k < 8; k++) {
            const float d = x[i + k] - mean;
            s[k] += d * d;
        }
    float v = (s[0] + s[1]) + (s[2] + s[3]) + (s[4] + s[5]) + (s[6] + s[7]);
    for (; i < n; i++) {
        const float d = x[i] - mean;
        v += d * d;
    }
    return v;
}

void orc_layernorm(float *out, const float *x, const float *w, const float *b, int n, float eps) {
    const float mean = sum8(x, n) / (float)n;
    const float var = sum_sq_centered8(x, n, mean);
    const float scale = orc_fast_rsqrt(var / (float)n + eps);
    for (int i = 0; i < n; i++) out[i] = (x[i] - mean) * scale * w[i] + b[i];
}

/* fastExpF32T (ops.go:1152-1164) */
static float fast_exp2_t(float x) {
    const float magic = 12582912.0f;
    int32_t n = (int32_t)((x + magic) - magic);
    float f = x - (float)n;
    float f2 = f * f;
    float poly = (1.0f + 0.6931471824645996f * f) +
                 f2 * (0.24022650718688965f + 0.05550410971045494f * f +
                       f2 * (0.009618128649890423f + 0.0013352063251659274f * f));
    return bits_to_f32(f32_to_bits(poly) + ((uint32_t)n << 23));
}

float orc_gelu_tanh(float x) {
    /* ops.go:1140-1150; the constants are the exact products rounded once */
    const float c1 = 0x1.26aec2p+1f;
    const float c3 = 0x1.a5a7dp-4f;
    const float x3 = x * (x * x);
    const float e = fast_exp2_t(c1 * x + c3 * x3);
    const float th = (e - 1.0f) / (e + 1.0f);
    return 0.5f * x * (1.0f + th);
}

int orc_project_image(const float *x, int grid_t, int grid_h, int grid_w, int vd, const float *norm_w,
                      const float *norm_b, const orc_qmat *q1, const float *b1, const orc_qmat *q2, const float *b2,
                      float eps, float *out) {
    const int bw = grid_w / 2, bh = grid_h / 2, rows = grid_t * bh * bw, K = 4 * vd, td = q2->rows;
    float *merged = (float *)malloc(sizeof(float) * (size_t)K);
    float *hid = (float *)malloc(sizeof(float) * (size_t)K);
    for (int row = 0; row < rows; row++) {
        const int t = row / (bh * bw), local = row - t * bh * bw, by = local / bw, bx = local - by * bw;
        const int base = t * grid_h * grid_w + by * 2 * grid_w + bx * 2;
        const int src[4] = {base, base + 1, base + grid_w, base + grid_w + 1};
        for (int q = 0; q < 4; q++) orc_layernorm(merged + q * vd, x + (size_t)src[q] * vd, norm_w, norm_b, vd, eps);
        orc_matvec(q1, merged, hid); /* dotQ8·scale */
        for (int i = 0; i < K; i++) hid[i] = orc_gelu_tanh(hid[i] + b1[i]);
        float *o = out + (size_t)row * td;
        orc_matvec(q2, hid, o);
        for (int i = 0; i < td; i++) o[i] = o[i] + b2[i];
    }
    free(merged);
    free(hid);
    return rows;
}

/* ---- sampling LM head ---- */

double orc_rng_float64(uint64_t *state) {
    /* model.go:1833-1840 */
    *state += 0x9e3779b97f4a7c15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

/* total order of topKSelectWithWork's comparison: score descending, equal
 * scores by lower index (no NaN scores). Each candidate becomes one u64 key
 * whose ascending order is that order: the high word is the complement of the
 * score's order-preserving bits (-0 folded onto +0, which compare equal), the
 * low word the index. The keys carry everything, so the sort needs no shared
 * state and concurrent calls cannot interfere. */
static uint64_t score_key(float s, int32_t i) {
    uint32_t u;
    if (s == 0.0f) s = 0.0f;
    memcpy(&u, &s, 4);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)(~u) << 32) | (uint32_t)i;
}
static int cmp_u64(const void *a, const void *b) {
    const uint64_t x = *(const uint64_t *)a, y = *(const uint64_t *)b;
    return x < y ? -1 : (x > y);
}

int orc_topk(const float *scores, int n, int k, int32_t *ids, float *out_scores) {
    /* topk.go:322-345: partial selection sort; score desc, ties lower id.
     * For k > 64 the same order comes from a full sort under the same total
     * order (the selection sort's k·n comparisons take minutes at k near the
     * vocabulary); the two agree for every input without NaN scores. */
    if (k <= 0 || n <= 0) return 0;
    if (k > n) k = n;
    int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * (size_t)n);
    for (int i = 0; i < n; i++) idx[i] = i;
    if (k > 64) {
        uint64_t *keys = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)n);
        for (int i = 0; i < n; i++) keys[i] = score_key(scores[i], i);
        qsort(keys, (size_t)n, sizeof(uint64_t), cmp_u64);
        for (int i = 0; i < n; i++) idx[i] = (int32_t)(uint32_t)keys[i];
        free(keys);
    } else {
        for (int i = 0; i < k; i++) {
            int best = i;
            for (int j = i + 1; j < n; j++) {
                const float sj = scores[idx[j]], sb = scores[idx[best]];
                if (sj > sb || (sj == sb && idx[j] < idx[best])) best = j;
            }
            const int32_t t = idx[i];
            idx[i] = idx[best];
            idx[best] = t;
        }
    }
    for (int i = 0; i < k; i++) {
        ids[i] = idx[i];
        out_scores[i] = scores[idx[i]];
    }
    free(idx);
    return k;
}

/* pickWeightedRawFloat32, model.go:2418-2456 (f32 running sum) */
static int pick_raw_f32(const float *w, int n, float pick) {
    float acc = 0.0f;
    for (int i = 0; i < n; i++) {
        acc += w[i];
        if (pick <= acc) return i;
    }
    return -1;
}

/* pickWeightedFloat32, model.go:2342-2416 (f64 running sum of f32 weights) */
static int pick_f64(const float *w, int n, double pick) {
    double acc = 0.0;
    for (int i = 0; i < n; i++) {
        acc += (double)w[i];
        if (pick <= acc) return i;
    }
    return -1;
}

static int32_t sample_candidates_w(const int32_t *ids, const float *sc, int n, double temperature, uint64_t *state,
                                   float *w, float *wv);

int32_t orc_sample_candidates(const int32_t *ids, const float *sc, int n, double temperature, uint64_t *state) {
    if (n <= 0) return 0;
    if (n == 1) return ids[0];
    float wv[4];
    float *w = n > 4 ? (float *)malloc(sizeof(float) * (size_t)n) : NULL;
    int32_t r = sample_candidates_w(ids, sc, n, temperature, state, w, wv);
    free(w);
    return r;
}

static int32_t sample_candidates_w(const int32_t *ids, const float *sc, int n, double temperature, uint64_t *state,
                                   float *w, float *wv) {
    if (temperature == 1.0) {
        /* model.go:1954-1963 */
        float mx = sc[0];
        for (int i = 1; i < n; i++) mx = sc[i] > mx ? sc[i] : mx;
        if (n == 2) { /* model.go:2145-2158 */
            const float s0 = sc[0], s1 = sc[1];
            if (s0 >= s1) {
                const double w1 = (double)orc_fast_exp(s1 - s0);
                return orc_rng_float64(state) * (1 + w1) <= 1 ? ids[0] : ids[1];
            }
            const double w0 = (double)orc_fast_exp(s0 - s1);
            return orc_rng_float64(state) * (w0 + 1) <= w0 ? ids[0] : ids[1];
        }
        if (n <= 4) { /* model.go:2159-2199 */
            for (int i = 0; i < n; i++) wv[i] = orc_fast_exp(sc[i] - mx);
            if (n == 3) {
                const float pick = (float)orc_rng_float64(state) * ((wv[0] + wv[1]) + wv[2]);
                if (pick <= wv[0]) return ids[0];
                if (pick <= wv[0] + wv[1]) return ids[1];
                return ids[2];
            }
            const float pick = (float)orc_rng_float64(state) * ((wv[0] + wv[1]) + (wv[2] + wv[3]));
            float acc = wv[0];
            if (pick <= acc) return ids[0];
            acc += wv[1];
            if (pick <= acc) return ids[1];
            acc += wv[2];
            if (pick <= acc) return ids[2];
            return ids[3];
        }
        /* sampleCandidateScoresTemp1Scratch, model.go:2040-2063 */
        float sum = 0.0f;
        for (int i = 0; i < n; i++) {
            w[i] = orc_fast_exp(sc[i] - mx);
            sum += w[i];
        }
        const float pick = (float)orc_rng_float64(state) * sum;
        const int idx = pick_raw_f32(w, n, pick);
        return idx >= 0 ? ids[idx] : ids[n - 1];
    }
    /* model.go:1965-1990 */
    const float inv = (float)(1.0 / temperature);
    float mxr = sc[0];
    for (int i = 1; i < n; i++) mxr = sc[i] > mxr ? sc[i] : mxr;
    const float mx = mxr * inv;
    if (n == 2) { /* sampleCandidateScoresSmall, model.go:1997-2011 */
        const float s0 = sc[0] * inv, s1 = sc[1] * inv;
        if (s0 >= s1) {
            const double w1 = (double)orc_fast_exp(s1 - s0);
            return orc_rng_float64(state) * (1 + w1) <= 1 ? ids[0] : ids[1];
        }
        const double w0 = (double)orc_fast_exp(s0 - s1);
        return orc_rng_float64(state) * (w0 + 1) <= w0 ? ids[0] : ids[1];
    }
    if (n <= 4) { /* model.go:2012-2037 */
        double d[4];
        for (int i = 0; i < n; i++) d[i] = (double)orc_fast_exp(sc[i] * inv - mx);
        if (n == 3) {
            const double pick = orc_rng_float64(state) * ((d[0] + d[1]) + d[2]);
            double acc = d[0];
            if (pick <= acc) return ids[0];
            acc += d[1];
            if (pick <= acc) return ids[1];
            return ids[2];
        }
        const double pick = orc_rng_float64(state) * ((d[0] + d[1]) + (d[2] + d[3]));
        double acc = d[0];
        if (pick <= acc) return ids[0];
        acc += d[1];
        if (pick <= acc) return ids[1];
        acc += d[2];
        if (pick <= acc) return ids[2];
        return ids[3];
    }
    double sum = 0.0;
    for (int i = 0; i < n; i++) {
        const double wi = (double)orc_fast_exp(sc[i] * inv - mx);
        w[i] = (float)wi;
        sum += wi;
    }
    const double pick = orc_rng_float64(state) * sum;
    const int idx = pick_f64(w, n, pick);
    return idx >= 0 ? ids[idx] : ids[n - 1];
}

/* ---- full-vocabulary draw ---- */

/* CumulativeSum (internal/tensor/cumsum.go:9-58): below 4096 entries one
 * running f32 sum; otherwise four blocks of (n+3)/4 entries, each summed from
 * zero, then every block after the first shifted by the running total of the
 * block sums before it (offset += blockSums[b] after block b is shifted).
 * out may be x.  Returns that running total. */
float orc_cumsum(float *out, const float *x, int n) {
    if (n <= 0) return 0.0f;
    if (n < 4096) {
        float cs = 0.0f;
        for (int i = 0; i < n; i++) {
            cs += x[i];
            out[i] = cs;
        }
        return cs;
    }
    const int bs = (n + 3) / 4;
    float bsum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int b = 0; b < 4; b++) {
        const int start = b * bs, end = start + bs < n ? start + bs : n;
        float cs = 0.0f;
        for (int i = start; i < end; i++) {
            cs += x[i];
            out[i] = cs;
        }
        bsum[b] = cs;
    }
    float offset = bsum[0];
    for (int b = 1; b < 4; b++) {
        const int start = b * bs, end = start + bs < n ? start + bs : n;
        for (int i = start; i < end; i++) out[i] += offset;
        offset += bsum[b];
    }
    return offset;
}

/* pickCumulativeFloat32 (model.go:2326-2340): binary search for the first
 * entry with pick <= cdf[i]; -1 when the search runs off the end */
int orc_pick_cumulative(const float *cdf, int n, float pick) {
    int lo = 0, hi = n;
    while (lo < hi) {
        const int mid = (int)((unsigned)(lo + hi) >> 1);
        if (pick <= cdf[mid]) hi = mid;
        else lo = mid + 1;
    }
    return lo < n ? lo : -1;
}

/* sampleTwoLogits (model.go:2309-2324) */
static int sample_two(const float *x, float inv, uint64_t *state) {
    const float s0 = x[0], s1 = x[1];
    if (s0 >= s1) {
        const double w1 = (double)orc_fast_exp((s1 - s0) * inv);
        return orc_rng_float64(state) * (1 + w1) <= 1 ? 0 : 1;
    }
    const double w0 = (double)orc_fast_exp((s0 - s1) * inv);
    return orc_rng_float64(state) * (w0 + 1) <= w0 ? 0 : 1;
}

/* sampleFullLogitsScratch (model.go:2215-2260) and, at temperature 1,
 * sampleFullLogitsTemp1Scratch (2264-2307), with the weight buffer the
 * generation scratch provides (makeSampleWeights, 2799-2807):
 *   T = float32(temperature); two logits → sampleTwoLogits(x, 1/T);
 *   m = max (tensor.Max); at T == 1 v_i = x_i·1 + (−m), otherwise
 *   v_i = x_i·(1/T) + (−m·(1/T)), all f32;
 *   w_i = FastExpF32(v_i), sum = Σ w_i in order from zero (ExpScaledVec,
 *   weighted_sum.go:314-329, with the portable expScaledVecFMA of
 *   dot_other.go:398-411);
 *   cdf = CumulativeSum(w); pick = float32(Float64()) · sum;
 *   the first i with pick <= cdf[i] by binary search, else n − 1.
 * Draws one value from *state.  Returns the chosen index. */
int32_t orc_sample_full(const float *x, int n, double temperature, uint64_t *state) {
    if (n <= 0) return 0;
    const float T = (float)temperature;
    if (n == 2) return sample_two(x, 1.0f / T, state);
    float m = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > m) m = x[i];
    float scale = 1.0f, bias = -m;
    if (T != 1.0f) {
        scale = 1.0f / T;
        bias = -(m * scale);
    }
    float *w = (float *)malloc(sizeof(float) * (size_t)n);
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        const float v = x[i] * scale + bias;
        w[i] = orc_fast_exp(v);
        sum += w[i];
    }
    orc_cumsum(w, w, n);
    const float pick = (float)orc_rng_float64(state) * sum;
    const int idx = orc_pick_cumulative(w, n, pick);
    free(w);
    return idx >= 0 ? idx : n - 1;
}

static int generate_impl(orc_model *m, const int32_t *ids, int n_ids, const float *image_embeds, int n_image,
                         int image_token_id, const int32_t grid[3], int merge, int max_new, const int32_t *eos,
                         int n_eos, double temperature, int top_k, uint64_t seed, int32_t *out_tokens);

int orc_generate(orc_model *m, const int32_t *ids, int n_ids, const float *image_embeds, int n_image,
                 int image_token_id, const int32_t grid[3], int merge, int max_new, const int32_t *eos,
                 int n_eos, int32_t *out_tokens) {
    return generate_impl(m, ids, n_ids, image_embeds, n_image, image_token_id, grid, merge, max_new, eos, n_eos,
                         0.0, 0, 0, out_tokens);
}

int orc_generate_sampled(orc_model *m, const int32_t *ids, int n_ids, const float *image_embeds, int n_image,
                         int image_token_id, const int32_t grid[3], int merge, int max_new, const int32_t *eos,
                         int n_eos, double temperature, int top_k, uint64_t seed, int32_t *out_tokens) {
    return generate_impl(m, ids, n_ids, image_embeds, n_image, image_token_id, grid, merge, max_new, eos, n_eos,
                         temperature, top_k, seed, out_tokens);
}

/* one token from the step's logits: greedy when not sampling; 1 < top_k <
 * vocab takes the candidates path of forwardEmbeddingForSampling (model.go:
 * 3632-3638, matVecTopKMaybeCPU 7202-7235) and sampleCandidateScoresScratch;
 * top_k 0 or >= vocab the full logits through sampleTokenScratch (1870-1879)
 * into sampleFullLogitsScratch */
static int32_t pick_token(const float *logits, int vocab, int sampling, int top_k, double temperature,
                          uint64_t *state, int32_t greedy) {
    if (!sampling) return greedy;
    if (top_k <= 0 || top_k >= vocab) return orc_sample_full(logits, vocab, temperature, state);
    int32_t *cid = (int32_t *)malloc(sizeof(int32_t) * (size_t)top_k);
    float *csc = (float *)malloc(sizeof(float) * (size_t)top_k);
    const int n = orc_topk(logits, vocab, top_k, cid, csc);
    const int32_t tok = orc_sample_candidates(cid, csc, n, temperature, state);
    free(cid);
    free(csc);
    return tok;
}

static int generate_impl(orc_model *m, const int32_t *ids, int n_ids, const float *image_embeds, int n_image,
                         int image_token_id, const int32_t grid[3], int merge, int max_new, const int32_t *eos,
                         int n_eos, double temperature, int top_k, uint64_t seed, int32_t *out_tokens) {
    if (n_ids <= 0 || max_new <= 0) return 0;
    /* generationUsesArgmaxSampling (model.go:1858-1860): greedy at
     * temperature <= 0 or top_k == 1, sampled otherwise */
    const int sampling = temperature > 0 && top_k != 1;
    uint64_t state = seed; /* samplingRNGInto, model.go:1846-1852 */
    float *logits = sampling ? (float *)malloc(sizeof(float) * (size_t)m->vocab) : NULL;
    int32_t *pos = (int32_t *)malloc(sizeof(int32_t) * 3 * (size_t)n_ids);
    int rope_delta = 0;
    if (n_image > 0) {
        int np = orc_mm_positions(ids, n_ids, image_token_id, grid, merge, pos, &rope_delta);
        if (np != n_ids) {
            free(pos);
            return -1;
        }
    } else {
        for (int i = 0; i < n_ids; i++) pos[3 * i] = pos[3 * i + 1] = pos[3 * i + 2] = i;
    }
    orc_seq *s = orc_seq_create(m, n_ids + max_new);
    int img = 0;
    int32_t next = 0;
    int rc = 0;
    for (int p = 0; p < n_ids; p++) {
        const float *emb;
        if (n_image > 0 && ids[p] == image_token_id) {
            if (img >= n_image) { rc = -3; goto done; }
            emb = image_embeds + (size_t)img * m->hidden;
            img++;
        } else {
            if (ids[p] < 0 || ids[p] >= m->vocab) { rc = -4; goto done; }
            emb = m->embed + (size_t)ids[p] * m->hidden;
        }
        orc_step(m, s, emb, pos + 3 * p, p == n_ids - 1, p == n_ids - 1 ? logits : NULL, &next, NULL);
    }
    if (img != n_image) { rc = -3; goto done; }
    next = pick_token(logits, m->vocab, sampling, top_k, temperature, &state, next);
    int n_out = 0;
    for (int i = 0; i < max_new; i++) {
        out_tokens[n_out++] = next;
        if (is_eos(next, eos, n_eos)) break;
        if (i + 1 >= max_new) break;
        int32_t p = n_ids + n_out - 1 + rope_delta; /* len(out)-1+ropeDelta (model.go:1695) */
        int32_t p3[3] = {p, p, p};
        orc_step(m, s, m->embed + (size_t)next * m->hidden, p3, 1, logits, &next, NULL);
        next = pick_token(logits, m->vocab, sampling, top_k, temperature, &state, next);
    }
    rc = n_out;
done:
    orc_seq_free(s);
    free(pos);
    free(logits);
    return rc;
}
