/*
 * srq_oracle.c -- CPU restatement of sr_go_tranformer's quantized-weight
 * inference path.  TEST INFRASTRUCTURE ONLY: the parity checker and the
 * timed CPU baseline.  No product code links, loads or calls it.
 *
 * M: = cmd/monolith/monolith.go of the reference.  Build with
 * -ffp-contract=off and without -ffast-math (see oracle/build.py): the
 * reduction orders below are the reference's and must not be re-associated.
 */
#include "srq_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define Q8_BLOCK 64
#define PAGE_TOKENS 32

/* ------------------------------------------------------------------ */
/* RNG: SplitMix64 (M:1411-1439)                                       */
/* ------------------------------------------------------------------ */
uint64_t or_rng_uint64(uint64_t *state) {
    *state += 0x9e3779b97f4a7c15ULL;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

double or_rng_float64(uint64_t *state) {
    return (double)(or_rng_uint64(state) >> 11) * (1.0 / 9007199254740992.0);
}

/* Go evaluates the two Float64 calls left to right (M:1437-1439). */
double or_rng_normal(uint64_t *state) {
    double u1 = or_rng_float64(state);
    double u2 = or_rng_float64(state);
    return sqrt(-2 * log(1 - u1)) * cos(2 * M_PI * u2);
}

int64_t or_rng_intn(uint64_t *state, int64_t n) {
    if (n <= 0) return -1;
    uint64_t bound = (uint64_t)n;
    uint64_t threshold = (0 - bound) % bound;
    for (;;) {
        uint64_t x = or_rng_uint64(state);
        if (x >= threshold) return (int64_t)(x % bound);
    }
}

void or_fill_normal(uint64_t *state, double scale, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = (float)(or_rng_normal(state) * scale);
}

void or_fill_uniform(uint64_t *state, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = (float)(or_rng_float64(state) * 2 - 1);
}

/* ------------------------------------------------------------------ */
/* Packing (M:3793-3898, readParam M:857-880)                          */
/* ------------------------------------------------------------------ */
float or_low_bit_scale(float amax, double levels) {
    if (amax == 0) return 0;
    float scale = (float)((double)amax / levels);
    if (scale == 0) return FLT_TRUE_MIN;
    /* Round downward so reconstruction stays finite near MaxFloat32. */
    if (scale > FLT_TRUE_MIN && (double)scale * levels > (double)amax) scale = nextafterf(scale, 0);
    return scale;
}

/* math.Round: half away from zero == C round(). */
static double clamp_round(float v, float scale, double lim) {
    double q = round((double)v / (double)scale);
    if (q > lim) q = lim;
    if (q < -lim) q = -lim;
    return q;
}

int8_t or_q8_value(float v, float scale) {
    if (scale == 0) return 0;
    return (int8_t)clamp_round(v, scale, 127);
}

int8_t or_q4_value(float v, float scale) {
    if (scale == 0) return 0;
    return (int8_t)clamp_round(v, scale, 7);
}

/* (*q4Weights).put (M:3819-3822): low nibble = even column, stale bits
 * cleared. */
static void q4_put(uint8_t *values, int64_t cols, int64_t row, int64_t col, int8_t v) {
    int64_t i = row * ((cols + 1) / 2) + col / 2;
    unsigned shift = (unsigned)(col % 2) * 4;
    values[i] = (uint8_t)((values[i] & ~(15u << shift)) | (((uint8_t)v & 15u) << shift));
}

/* readParam's block walk: values stream in row-major order; whenever a
 * 64-column block (or the row tail) completes, its amax -> scale -> codes
 * are written.  amax starts at +0 and takes f32(|x|). */
static void pack_generic(const float *src, int64_t rows, int64_t cols, int q4, void *values, float *scales) {
    int64_t groups = (cols + Q8_BLOCK - 1) / Q8_BLOCK;
    float block[Q8_BLOCK];
    if (q4) memset(values, 0, (size_t)(rows * ((cols + 1) / 2)));
    for (int64_t i = 0; i < rows * cols; i++) {
        int64_t row = i / cols, col = i % cols;
        block[col % Q8_BLOCK] = src[i];
        if (col % Q8_BLOCK == Q8_BLOCK - 1 || col == cols - 1) {
            int count = (int)(col % Q8_BLOCK) + 1;
            float amax = 0;
            for (int j = 0; j < count; j++) {
                float a = (float)fabs((double)block[j]);
                amax = a > amax ? a : amax;
            }
            float scale = q4 ? or_low_bit_scale(amax, 7) : or_low_bit_scale(amax, 127);
            scales[row * groups + col / Q8_BLOCK] = scale;
            for (int j = 0; j < count; j++) {
                int64_t c = col - count + 1 + j;
                if (q4)
                    q4_put((uint8_t *)values, cols, row, c, or_q4_value(block[j], scale));
                else
                    ((int8_t *)values)[row * cols + c] = or_q8_value(block[j], scale);
            }
        }
    }
}

void or_pack_q8(const float *src, int64_t rows, int64_t cols, int8_t *values, float *scales) {
    pack_generic(src, rows, cols, 0, values, scales);
}

void or_pack_q4(const float *src, int64_t rows, int64_t cols, uint8_t *values, float *scales) {
    pack_generic(src, rows, cols, 1, values, scales);
}

/* q4Pairs (M:3811-3817): [b][0] = sext(low nibble), [b][1] = sext(high). */
static float Q4P[256][2];
static int q4p_ready;
static void q4p_init(void) {
    if (q4p_ready) return;
    for (int i = 0; i < 256; i++) {
        Q4P[i][0] = (float)((int8_t)((uint8_t)(i << 4)) >> 4);
        Q4P[i][1] = (float)((int8_t)(uint8_t)i >> 4);
    }
    q4p_ready = 1;
}

void or_q4_pairs(float *table) {
    q4p_init();
    memcpy(table, Q4P, sizeof Q4P);
}

void or_copy_row(int fmt, int64_t rows, int64_t cols, const void *values, const float *scales, int64_t row,
                 float *dst) {
    (void)rows;
    int64_t groups = (cols + Q8_BLOCK - 1) / Q8_BLOCK;
    if (fmt == OR_Q4) {
        q4p_init();
        int64_t stride = (cols + 1) / 2;
        const uint8_t *wr = (const uint8_t *)values + row * stride;
        for (int64_t j = 0; j < cols; j++) dst[j] = Q4P[wr[j / 2]][j % 2] * scales[row * groups + j / Q8_BLOCK];
        return;
    }
    if (fmt == OR_F32) {
        memcpy(dst, (const float *)values + row * cols, (size_t)cols * sizeof(float));
        return;
    }
    const int8_t *q = (const int8_t *)values;
    for (int64_t g = 0; g < groups; g++) {
        float scale = scales[row * groups + g];
        int64_t end = (g + 1) * Q8_BLOCK < cols ? (g + 1) * Q8_BLOCK : cols;
        for (int64_t j = g * Q8_BLOCK; j < end; j++) dst[j] = (float)q[row * cols + j] * scale;
    }
}

/* ------------------------------------------------------------------ */
/* Persistent worker pool: kernelExecutor.parallel (M:3689-3782).      */
/* Tasks [n*w/W, n*(w+1)/W) per worker; inline if W<2 or work<131072.  */
/* ------------------------------------------------------------------ */
typedef void (*range_fn)(void *ctx, int64_t lo, int64_t hi);

typedef struct {
    pthread_t th[256];
    int nthreads;
    pthread_mutex_t mu;
    pthread_cond_t go, done;
    uint64_t generation;
    int pending;
    range_fn fn;
    void *ctx;
    int64_t n;
    int workers;
    int quit;
} pool_t;

static pool_t POOL;
static int pool_ready;
static pthread_mutex_t pool_init_mu = PTHREAD_MUTEX_INITIALIZER;

typedef struct {
    int id;
    uint64_t start_gen; /* generation current when the thread was made */
} worker_arg;
static worker_arg WARGS[256];

static void *pool_main(void *arg) {
    int id = ((worker_arg *)arg)->id;
    uint64_t seen = ((worker_arg *)arg)->start_gen;
    for (;;) {
        pthread_mutex_lock(&POOL.mu);
        while (POOL.generation == seen && !POOL.quit) pthread_cond_wait(&POOL.go, &POOL.mu);
        if (POOL.quit) {
            pthread_mutex_unlock(&POOL.mu);
            return NULL;
        }
        seen = POOL.generation;
        range_fn fn = POOL.fn;
        void *ctx = POOL.ctx;
        int64_t n = POOL.n;
        int W = POOL.workers;
        pthread_mutex_unlock(&POOL.mu);
        if (id < W) fn(ctx, n * id / W, n * (id + 1) / W);
        pthread_mutex_lock(&POOL.mu);
        if (--POOL.pending == 0) pthread_cond_signal(&POOL.done);
        pthread_mutex_unlock(&POOL.mu);
    }
}

static void pool_grow(int want) {
    pthread_mutex_lock(&pool_init_mu);
    if (!pool_ready) {
        pthread_mutex_init(&POOL.mu, NULL);
        pthread_cond_init(&POOL.go, NULL);
        pthread_cond_init(&POOL.done, NULL);
        pool_ready = 1;
    }
    while (POOL.nthreads < want && POOL.nthreads < 256) {
        /* Lock so a new thread's first view of generation is consistent. */
        pthread_mutex_lock(&POOL.mu);
        int id = POOL.nthreads;
        WARGS[id].id = id;
        WARGS[id].start_gen = POOL.generation;
        pthread_create(&POOL.th[id], NULL, pool_main, &WARGS[id]);
        POOL.nthreads++;
        pthread_mutex_unlock(&POOL.mu);
    }
    pthread_mutex_unlock(&pool_init_mu);
}

static void parallel(int workers, int64_t n, int64_t work, range_fn fn, void *ctx) {
    int W = workers < n ? workers : (int)n;
    if (W < 2 || work < 131072) {
        fn(ctx, 0, n);
        return;
    }
    pool_grow(W);
    pthread_mutex_lock(&POOL.mu);
    POOL.fn = fn;
    POOL.ctx = ctx;
    POOL.n = n;
    POOL.workers = W;
    POOL.pending = POOL.nthreads;
    POOL.generation++;
    pthread_cond_broadcast(&POOL.go);
    while (POOL.pending > 0) pthread_cond_wait(&POOL.done, &POOL.mu);
    pthread_mutex_unlock(&POOL.mu);
}

/* ------------------------------------------------------------------ */
/* Linear kernels (M:3942-4780)                                        */
/* ------------------------------------------------------------------ */
typedef struct {
    const or_param *w;
    float *y;
    const float *x;
    int n;
} lin_job;

/* The per-element order shared by every tile shape of linearQ8Into /
 * linearQ4Into: per block four interleaved f32 accumulators over
 * j = 0,1,2,3 mod 4, (a+b)+(c+d), the len%4 tail, then s += p*scale.
 * R rows share each weight conversion (the 4-row tile, M:4091-4125; the
 * pair and single-row helpers keep the same order, M:4126-4184). */
static inline float q_weight(int fmt, const void *wr, int64_t j) {
    if (fmt == OR_Q8) return (float)((const int8_t *)wr)[j];
    return Q4P[((const uint8_t *)wr)[j / 2]][j % 2];
}

static void quant_rows(const or_param *w, float *y, const float *x, int n, int r, int R, int64_t o) {
    int64_t in = w->cols, out = w->rows, groups = (in + Q8_BLOCK - 1) / Q8_BLOCK;
    const void *wr = w->fmt == OR_Q8 ? (const void *)((const int8_t *)w->values + o * in)
                                     : (const void *)((const uint8_t *)w->values + o * ((in + 1) / 2));
    const float *scales = w->scales + o * groups;
    float s[4] = {0, 0, 0, 0};
    for (int64_t g = 0; g < groups; g++) {
        float a[4] = {0, 0, 0, 0}, b[4] = {0, 0, 0, 0}, c[4] = {0, 0, 0, 0}, d[4] = {0, 0, 0, 0};
        int64_t j = g * Q8_BLOCK, end = (g + 1) * Q8_BLOCK < in ? (g + 1) * Q8_BLOCK : in;
        for (; j + 4 <= end; j += 4) {
            float v0 = q_weight(w->fmt, wr, j), v1 = q_weight(w->fmt, wr, j + 1);
            float v2 = q_weight(w->fmt, wr, j + 2), v3 = q_weight(w->fmt, wr, j + 3);
            for (int i = 0; i < R; i++) {
                const float *xi = x + (int64_t)(r + i) * in;
                a[i] += xi[j] * v0;
                b[i] += xi[j + 1] * v1;
                c[i] += xi[j + 2] * v2;
                d[i] += xi[j + 3] * v3;
            }
        }
        float p[4];
        for (int i = 0; i < R; i++) p[i] = (a[i] + b[i]) + (c[i] + d[i]);
        for (; j < end; j++) {
            float v = q_weight(w->fmt, wr, j);
            for (int i = 0; i < R; i++) p[i] += x[(int64_t)(r + i) * in + j] * v;
        }
        for (int i = 0; i < R; i++) s[i] += p[i] * scales[g];
    }
    for (int i = 0; i < R; i++) y[(int64_t)(r + i) * out + o] = s[i];
}

static void quant_range(void *ctx, int64_t lo, int64_t hi) {
    lin_job *job = (lin_job *)ctx;
    const or_param *w = job->w;
    int64_t out = w->rows, tiles = (out + 31) / 32;
    for (int64_t task = lo; task < hi; task++) {
        int r = (int)(task / tiles) * 4;
        int64_t o0 = (task % tiles) * 32, o1 = o0 + 32 < out ? o0 + 32 : out;
        for (int64_t o = o0; o < o1; o++) {
            if (r + 4 <= job->n) {
                quant_rows(w, job->y, job->x, job->n, r, 4, o);
            } else {
                int row = r;
                if (row + 2 <= job->n) {
                    quant_rows(w, job->y, job->x, job->n, row, 2, o);
                    row += 2;
                }
                for (; row < job->n && row < r + 4; row++) quant_rows(w, job->y, job->x, job->n, row, 1, o);
            }
        }
    }
}

/* q8NeedsWideSum (M:4346-4354). */
static const float WIDE_LIMIT = (float)(FLT_MAX / (2.0 * Q8_BLOCK * 127));
static int needs_wide(const float *x, int64_t count) {
    for (int64_t i = 0; i < count; i++)
        if (x[i] > WIDE_LIMIT || x[i] < -WIDE_LIMIT) return 1;
    return 0;
}

typedef struct {
    const or_param *w;
    float *y;
    const float *x;
} wide_job;

/* linearQ8WideInto / linearQ4WideInto (M:4356-4382, M:4754-4780). */
static void wide_range(void *ctx, int64_t lo, int64_t hi) {
    wide_job *job = (wide_job *)ctx;
    const or_param *w = job->w;
    int64_t in = w->cols, groups = (in + Q8_BLOCK - 1) / Q8_BLOCK;
    for (int64_t o = lo; o < hi; o++) {
        const void *wr = w->fmt == OR_Q8 ? (const void *)((const int8_t *)w->values + o * in)
                                         : (const void *)((const uint8_t *)w->values + o * ((in + 1) / 2));
        double sum = 0;
        for (int64_t g = 0; g < groups; g++) {
            double part = 0;
            int64_t end = (g + 1) * Q8_BLOCK < in ? (g + 1) * Q8_BLOCK : in;
            for (int64_t j = g * Q8_BLOCK; j < end; j++) part += (double)job->x[j] * (double)q_weight(w->fmt, wr, j);
            sum += part * (double)w->scales[o * groups + g];
        }
        job->y[o] = (float)sum;
    }
}

static void quant_linear(const or_param *w, float *y, const float *x, int n, int workers) {
    int64_t in = w->cols, out = w->rows;
    q4p_init();
    if (needs_wide(x, (int64_t)n * in)) {
        /* Per-row selection keeps ordinary rows on the ordinary order. */
        for (int row = 0; row < n; row++) {
            const float *xr = x + (int64_t)row * in;
            float *yr = y + (int64_t)row * out;
            if (!needs_wide(xr, in)) {
                quant_linear(w, yr, xr, 1, workers);
                continue;
            }
            wide_job job = {w, yr, xr};
            parallel(workers, out, in * out, wide_range, &job);
        }
        return;
    }
    lin_job job = {w, y, x, n};
    int64_t tasks = (int64_t)((n + 3) / 4) * ((out + 31) / 32);
    parallel(workers, tasks, (int64_t)n * in * out, quant_range, &job);
}

/* linearFP32Range (M:3970-4070): one sequential f32 accumulator per output
 * in every tile shape. */
static void f32_range(void *ctx, int64_t lo, int64_t hi) {
    lin_job *job = (lin_job *)ctx;
    const or_param *w = job->w;
    int64_t in = w->cols, out = w->rows, tiles = (out + 31) / 32;
    const float *W = (const float *)w->values;
    for (int64_t task = lo; task < hi; task++) {
        int r = (int)(task / tiles) * 4;
        int64_t o0 = (task % tiles) * 32, o1 = o0 + 32 < out ? o0 + 32 : out;
        int rend = r + 4 < job->n ? r + 4 : job->n;
        for (int row = r; row < rend; row++) {
            const float *xr = job->x + (int64_t)row * in;
            for (int64_t o = o0; o < o1; o++) {
                const float *wr = W + o * in;
                float sum = 0;
                for (int64_t j = 0; j < in; j++) sum += xr[j] * wr[j];
                job->y[(int64_t)row * out + o] = sum;
            }
        }
    }
}

void or_linear(const or_param *w, float *y, const float *x, int n, int workers) {
    if (w->fmt == OR_F32) {
        lin_job job = {w, y, x, n};
        int64_t tasks = (int64_t)((n + 3) / 4) * ((w->rows + 31) / 32);
        parallel(workers, tasks, (int64_t)n * w->cols * w->rows, f32_range, &job);
        return;
    }
    quant_linear(w, y, x, n, workers);
}

void or_linear_closed_f64(const or_param *w, double *y, const float *x, int n) {
    int64_t in = w->cols, out = w->rows, groups = (in + Q8_BLOCK - 1) / Q8_BLOCK;
    q4p_init();
    for (int row = 0; row < n; row++) {
        for (int64_t o = 0; o < out; o++) {
            double sum = 0;
            for (int64_t j = 0; j < in; j++) {
                double xv = x[(int64_t)row * in + j], wv;
                if (w->fmt == OR_F32) {
                    wv = ((const float *)w->values)[o * in + j];
                } else if (w->fmt == OR_Q8) {
                    wv = (double)((const int8_t *)w->values)[o * in + j] * (double)w->scales[o * groups + j / Q8_BLOCK];
                } else {
                    const uint8_t *wr = (const uint8_t *)w->values + o * ((in + 1) / 2);
                    wv = (double)Q4P[wr[j / 2]][j % 2] * (double)w->scales[o * groups + j / Q8_BLOCK];
                }
                sum += xv * wv;
            }
            y[(int64_t)row * out + o] = sum;
        }
    }
}

/* ------------------------------------------------------------------ */
/* Model, RoPE tables, KV pages, step                                   */
/* ------------------------------------------------------------------ */
struct or_model {
    or_config c;
    or_param emb, final_norm, output;
    int has_output;
    or_param *layer; /* [layers][OR_LAYER_PARAMS] */
    uint8_t *layer_set;
    float *cos_t, *sin_t; /* [context][hd/2] */
};

struct or_cache {
    or_model *m;
    int pos;
    int npages, cap;
    float **pages;
};

/* hfInverseFrequency (M:4961-4977), all Transformers-style f32 steps. */
float or_inverse_frequency(double theta, int head_dim, int index, const or_config *c) {
    float e = (float)(2 * index) / (float)head_dim;
    float inv = 1.0f / (float)pow(theta, (double)e);
    if (!c || !c->rope_llama3) return inv;
    float wave = (float)(2 * M_PI) / inv;
    float low_wave = (float)((double)c->rope_original / c->rope_low);
    float high_wave = (float)((double)c->rope_original / c->rope_high);
    float factor = (float)c->rope_factor;
    if (wave > low_wave) return inv / factor;
    if (wave >= high_wave) {
        float smooth = ((float)c->rope_original / wave - (float)c->rope_low) / (float)(c->rope_high - c->rope_low);
        return (1 - smooth) * inv / factor + smooth * inv;
    }
    return inv;
}

or_model *or_model_create(const or_config *c) {
    if (!c || c->dim <= 0 || c->heads <= 0 || c->kv_heads <= 0 || c->heads % c->kv_heads || c->dim % c->heads ||
        (c->dim / c->heads) % 2 || c->layers <= 0 || c->vocab <= 0 || c->hidden <= 0 || c->context <= 0)
        return NULL;
    or_model *m = (or_model *)calloc(1, sizeof *m);
    m->c = *c;
    m->layer = (or_param *)calloc((size_t)c->layers * OR_LAYER_PARAMS, sizeof(or_param));
    m->layer_set = (uint8_t *)calloc((size_t)c->layers * OR_LAYER_PARAMS, 1);
    int hd = c->dim / c->heads;
    m->cos_t = (float *)malloc(sizeof(float) * (size_t)c->context * (hd / 2));
    m->sin_t = (float *)malloc(sizeof(float) * (size_t)c->context * (hd / 2));
    /* Table fill (M:5034-5043). */
    for (int pos = 0; pos < c->context; pos++) {
        for (int j = 0; j < hd / 2; j++) {
            float inv = or_inverse_frequency(c->rope_theta, hd, j, c);
            double angle = (double)((float)pos * inv);
            m->cos_t[(size_t)pos * (hd / 2) + j] = (float)cos(angle);
            m->sin_t[(size_t)pos * (hd / 2) + j] = (float)sin(angle);
        }
    }
    return m;
}

void or_model_destroy(or_model *m) {
    if (!m) return;
    free(m->layer);
    free(m->layer_set);
    free(m->cos_t);
    free(m->sin_t);
    free(m);
}

const float *or_model_cos(const or_model *m) { return m->cos_t; }
const float *or_model_sin(const or_model *m) { return m->sin_t; }

int or_model_set(or_model *m, int layer, int kind, const or_param *p) {
    if (!m || !p) return OR_EINVAL;
    if (layer < 0) {
        if (kind == 0)
            m->emb = *p;
        else if (kind == 1)
            m->final_norm = *p;
        else if (kind == 2) {
            m->output = *p;
            m->has_output = 1;
        } else
            return OR_EINVAL;
        return OR_OK;
    }
    if (layer >= m->c.layers || kind < 0 || kind >= OR_LAYER_PARAMS) return OR_EINVAL;
    m->layer[(size_t)layer * OR_LAYER_PARAMS + kind] = *p;
    m->layer_set[(size_t)layer * OR_LAYER_PARAMS + kind] = 1;
    return OR_OK;
}

or_cache *or_cache_create(or_model *m) {
    or_cache *c = (or_cache *)calloc(1, sizeof *c);
    c->m = m;
    return c;
}

void or_cache_destroy(or_cache *c) {
    if (!c) return;
    for (int i = 0; i < c->npages; i++) free(c->pages[i]);
    free(c->pages);
    free(c);
}

int or_cache_pos(const or_cache *c) { return c->pos; }

static size_t page_elements(const or_model *m) {
    return (size_t)2 * PAGE_TOKENS * (m->c.dim / m->c.heads) * m->c.kv_heads * m->c.layers;
}

/* ensurePages (M:6023-6037). */
static void ensure_pages(or_cache *c, int end) {
    int needed = (end + PAGE_TOKENS - 1) / PAGE_TOKENS;
    if (needed > c->cap) {
        c->cap = needed * 2;
        c->pages = (float **)realloc(c->pages, sizeof(float *) * (size_t)c->cap);
    }
    while (c->npages < needed) c->pages[c->npages++] = (float *)calloc(page_elements(c->m), sizeof(float));
}

/* KVCache.row (M:6038-6043): page = [layer][K 32 x kvDim | V 32 x kvDim]. */
static float *cache_row(const or_cache *c, int layer, int pos, int which) {
    int kd = (c->m->c.dim / c->m->c.heads) * c->m->c.kv_heads;
    float *p = c->pages[pos / PAGE_TOKENS];
    size_t base = (size_t)layer * 2 * PAGE_TOKENS * kd + (size_t)(pos % PAGE_TOKENS) * kd;
    return p + base + (which ? (size_t)PAGE_TOKENS * kd : 0);
}

const float *or_cache_row(const or_cache *c, int layer, int pos, int which) {
    if (pos < 0 || pos / PAGE_TOKENS >= c->npages || layer < 0 || layer >= c->m->c.layers) return NULL;
    return cache_row(c, layer, pos, which);
}

int or_cache_set_rows(or_cache *c, int layer, int pos0, int count, const float *k, const float *v) {
    int kd = (c->m->c.dim / c->m->c.heads) * c->m->c.kv_heads;
    if (layer < 0 || layer >= c->m->c.layers || pos0 < 0 || pos0 + count > c->m->c.context) return OR_EINVAL;
    ensure_pages(c, pos0 + count);
    for (int i = 0; i < count; i++) {
        memcpy(cache_row(c, layer, pos0 + i, 0), k + (size_t)i * kd, sizeof(float) * kd);
        memcpy(cache_row(c, layer, pos0 + i, 1), v + (size_t)i * kd, sizeof(float) * kd);
    }
    return OR_OK;
}

int or_cache_set_pos(or_cache *c, int pos) {
    if (pos < 0 || pos > c->m->c.context) return OR_EINVAL;
    ensure_pages(c, pos);
    c->pos = pos;
    return OR_OK;
}

/* rmsInto (M:6182-6194). */
void or_rms(float *y, const float *x, const float *w, int n, int d, double eps) {
    for (int r = 0; r < n; r++) {
        double ss = 0;
        for (int j = 0; j < d; j++) ss += (double)x[(size_t)r * d + j] * (double)x[(size_t)r * d + j];
        float a = (float)(1 / sqrt(ss / (double)d + eps));
        for (int j = 0; j < d; j++) y[(size_t)r * d + j] = x[(size_t)r * d + j] * a * w[j];
    }
}

/* (*Model).rope, HF half-split branch (M:5264-5289). */
void or_rope(const or_model *m, float *x, int heads, int pos) {
    int hd = m->c.dim / m->c.heads;
    for (int h = 0; h < heads; h++) {
        for (int j = 0; j < hd / 2; j++) {
            int i = h * hd + j, zi = i + hd / 2;
            size_t ri = (size_t)pos * (hd / 2) + j;
            float c = m->cos_t[ri], s = m->sin_t[ri];
            float a = x[i], z = x[zi];
            x[i] = a * c - z * s;
            x[zi] = a * s + z * c;
        }
    }
}

/* attend (M:5293-5352). */
double or_attend(const float *q, float *out, float *scores, int hd, int length, const float *const *keys,
                 const float *const *vals) {
    float scale = (float)(1 / sqrt((double)hd));
    float max_score = -FLT_MAX;
    memset(out, 0, sizeof(float) * (size_t)hd);
    for (int s = 0; s < length; s++) {
        float dot = 0;
        for (int j = 0; j < hd; j++) dot += q[j] * keys[s][j];
        scores[s] = dot * scale;
        if (scores[s] > max_score) max_score = scores[s];
    }
    double sum = 0;
    for (int s = 0; s < length; s++) sum += exp((double)scores[s] - (double)max_score);
    double lse = (double)max_score + log(sum);
    for (int s = 0; s < length; s++) {
        float p = (float)exp((double)scores[s] - lse);
        for (int j = 0; j < hd; j++) out[j] += p * vals[s][j];
    }
    return lse;
}

typedef struct {
    or_model *m;
    or_cache **row_cache;
    const int *positions;
    const float *Q;
    float *A;
    int layer, rows;
} attn_job;

static void attn_range(void *ctx, int64_t lo, int64_t hi) {
    attn_job *job = (attn_job *)ctx;
    const or_config *c = &job->m->c;
    int hd = c->dim / c->heads, group = c->heads / c->kv_heads;
    int maxlen = c->context;
    float *scores = (float *)malloc(sizeof(float) * (size_t)maxlen);
    const float **keys = (const float **)malloc(sizeof(float *) * (size_t)maxlen);
    const float **vals = (const float **)malloc(sizeof(float *) * (size_t)maxlen);
    for (int64_t task = lo; task < hi; task++) {
        int i = (int)(task / c->heads), h = (int)(task % c->heads);
        int kh = h / group, len = job->positions[i] + 1;
        for (int s = 0; s < len; s++) {
            keys[s] = cache_row(job->row_cache[i], job->layer, s, 0) + (size_t)kh * hd;
            vals[s] = cache_row(job->row_cache[i], job->layer, s, 1) + (size_t)kh * hd;
        }
        size_t qi = (size_t)i * c->dim + (size_t)h * hd;
        or_attend(job->Q + qi, job->A + qi, scores, hd, len, keys, vals);
    }
    free(scores);
    free(keys);
    free(vals);
}

static void add_bias(float *x, const or_param *b, int64_t count) {
    if (!b || !b->values) return;
    const float *d = (const float *)b->values;
    int64_t len = b->rows * b->cols;
    for (int64_t i = 0; i < count; i++) x[i] += d[i % len];
}

int or_step(or_model *m, int sessions, or_cache **caches, const int *chunk_lens, const int *tokens,
            const uint8_t *want, float *logits, int workers) {
    const or_config *c = &m->c;
    if (sessions < 1 || sessions > 256) return OR_EINVAL;
    int n = 0;
    for (int i = 0; i < sessions; i++) {
        if (!caches[i] || caches[i]->m != m) return OR_EINVAL;
        for (int j = 0; j < i; j++)
            if (caches[j] == caches[i]) return OR_EINVAL;
        int len = chunk_lens[i];
        if (len < 1 || len > 1024 - n) return OR_EINVAL;
        if (caches[i]->pos < 0 || caches[i]->pos > c->context || len > c->context - caches[i]->pos) return OR_ERANGE;
        for (int j = 0; j < len; j++)
            if (tokens[n + j] < 0 || tokens[n + j] >= c->vocab) return OR_EINVAL;
        n += len;
    }
    int d = c->dim, hd = d / c->heads, kd = hd * c->kv_heads, H = c->hidden;
    float *X = (float *)calloc((size_t)n * d, 4), *N = (float *)calloc((size_t)n * d, 4);
    float *Q = (float *)calloc((size_t)n * d, 4), *K = (float *)calloc((size_t)n * kd, 4);
    float *V = (float *)calloc((size_t)n * kd, 4), *A = (float *)calloc((size_t)n * d, 4);
    float *T = (float *)calloc((size_t)n * d, 4), *G = (float *)calloc((size_t)n * H, 4);
    float *U = (float *)calloc((size_t)n * H, 4), *Hh = (float *)calloc((size_t)n * H, 4);
    or_cache **row_cache = (or_cache **)malloc(sizeof(void *) * (size_t)n);
    int *positions = (int *)malloc(sizeof(int) * (size_t)n);
    int *last_rows = (int *)malloc(sizeof(int) * (size_t)sessions);
    int r = 0;
    for (int i = 0; i < sessions; i++) {
        ensure_pages(caches[i], caches[i]->pos + chunk_lens[i]);
        for (int j = 0; j < chunk_lens[i]; j++) {
            row_cache[r] = caches[i];
            positions[r] = caches[i]->pos + j;
            or_copy_row(m->emb.fmt, m->emb.rows, m->emb.cols, m->emb.values, m->emb.scales, tokens[r],
                        X + (size_t)r * d);
            r++;
        }
        last_rows[i] = r - 1;
    }
    for (int l = 0; l < c->layers; l++) {
        const or_param *P = m->layer + (size_t)l * OR_LAYER_PARAMS;
        const uint8_t *set = m->layer_set + (size_t)l * OR_LAYER_PARAMS;
        or_rms(N, X, (const float *)P[OR_N1].values, n, d, c->norm_eps);
        or_linear(&P[OR_Q], Q, N, n, workers);
        or_linear(&P[OR_K], K, N, n, workers);
        or_linear(&P[OR_V], V, N, n, workers);
        if (set[OR_QB]) add_bias(Q, &P[OR_QB], (int64_t)n * d);
        if (set[OR_KB]) add_bias(K, &P[OR_KB], (int64_t)n * kd);
        if (set[OR_VB]) add_bias(V, &P[OR_VB], (int64_t)n * kd);
        for (int i = 0; i < n; i++) {
            or_rope(m, Q + (size_t)i * d, c->heads, positions[i]);
            or_rope(m, K + (size_t)i * kd, c->kv_heads, positions[i]);
            memcpy(cache_row(row_cache[i], l, positions[i], 0), K + (size_t)i * kd, sizeof(float) * kd);
            memcpy(cache_row(row_cache[i], l, positions[i], 1), V + (size_t)i * kd, sizeof(float) * kd);
        }
        attn_job aj = {m, row_cache, positions, Q, A, l, n};
        int maxpos = 0;
        for (int i = 0; i < n; i++) maxpos = positions[i] + 1 > maxpos ? positions[i] + 1 : maxpos;
        parallel(workers, (int64_t)n * c->heads, (int64_t)n * d * maxpos, attn_range, &aj);
        or_linear(&P[OR_O], T, A, n, workers);
        for (size_t i = 0; i < (size_t)n * d; i++) X[i] += T[i];
        or_rms(N, X, (const float *)P[OR_N2].values, n, d, c->norm_eps);
        or_linear(&P[OR_GATE], G, N, n, workers);
        or_linear(&P[OR_UP], U, N, n, workers);
        /* SwiGLU exactly as the step writes it (M:6411-6413). */
        for (size_t i = 0; i < (size_t)n * H; i++) Hh[i] = (float)((double)G[i] / (1 + exp(-(double)G[i]))) * U[i];
        or_linear(&P[OR_DOWN], T, Hh, n, workers);
        for (size_t i = 0; i < (size_t)n * d; i++) X[i] += T[i];
    }
    /* Compact selected rows, final norm, head, expand (M:6420-6448). */
    int heads = 0;
    for (int i = 0; i < sessions; i++) {
        if (!want || want[i]) {
            memcpy(T + (size_t)heads * d, X + (size_t)last_rows[i] * d, sizeof(float) * d);
            heads++;
        }
    }
    if (heads > 0) {
        or_rms(N, T, (const float *)m->final_norm.values, heads, d, c->norm_eps);
        const or_param *head = m->has_output ? &m->output : &m->emb;
        or_linear(head, logits, N, heads, workers);
    }
    if (want) {
        for (int i = sessions - 1; i >= 0; i--) {
            float *dst = logits + (size_t)i * c->vocab;
            if (want[i]) {
                heads--;
                memmove(dst, logits + (size_t)heads * c->vocab, sizeof(float) * c->vocab);
            } else {
                memset(dst, 0, sizeof(float) * c->vocab);
            }
        }
    }
    for (int i = 0; i < sessions; i++) caches[i]->pos += chunk_lens[i];
    free(X), free(N), free(Q), free(K), free(V), free(A), free(T), free(G), free(U), free(Hh);
    free(row_cache), free(positions), free(last_rows);
    return OR_OK;
}

/* inferHFIDs greedy rule (M:1215-1223): strict '>' keeps the lowest ID. */
int or_argmax(const float *logits, int vocab) {
    int best = 0;
    for (int j = 0; j < vocab; j++) {
        if (!isfinite(logits[j])) return -1;
        if (logits[j] > logits[best]) best = j;
    }
    return best;
}

/* ---- sampleWithBlocked (M:7320-7426) ---- */
typedef struct {
    int id;
    double logit, prob;
} cand;

/* candidateBefore (M:7284-7289). */
static int cand_cmp(const void *pa, const void *pb) {
    const cand *a = (const cand *)pa, *b = (const cand *)pb;
    if (a->logit == b->logit) return a->id < b->id ? -1 : (a->id > b->id);
    return a->logit > b->logit ? -1 : 1;
}

int or_sample(const float *logits, int vocab, const int *history, int nhistory, double temperature, int top_k,
              double top_p, double repeat_penalty, uint64_t *rng_state, int blocked) {
    if (vocab <= 0) return OR_EINVAL;
    uint8_t *seen = (uint8_t *)calloc((size_t)vocab, 1);
    if (temperature != 0 || repeat_penalty != 1)
        for (int i = 0; i < nhistory; i++)
            if (history[i] >= 0 && history[i] < vocab) seen[history[i]] = 1;
    if (temperature == 0) {
        int best = -1;
        double best_logit = 0;
        for (int id = 0; id < vocab; id++) {
            if (!isfinite(logits[id])) {
                free(seen);
                return OR_ENONFINITE;
            }
            if (id == blocked) continue;
            double x = logits[id];
            if (seen[id]) x = x > 0 ? x / repeat_penalty : x * repeat_penalty;
            if (best < 0 || x > best_logit) best = id, best_logit = x;
        }
        free(seen);
        return best < 0 ? OR_EINVAL : best;
    }
    cand *cs = (cand *)malloc(sizeof(cand) * (size_t)vocab);
    int count = 0;
    for (int id = 0; id < vocab; id++) {
        if (!isfinite(logits[id])) {
            free(cs), free(seen);
            return OR_ENONFINITE;
        }
        if (id == blocked) continue;
        double x = logits[id];
        if (seen[id]) x = x > 0 ? x / repeat_penalty : x * repeat_penalty;
        cs[count].id = id;
        cs[count].logit = x;
        count++;
    }
    free(seen);
    if (count == 0) {
        free(cs);
        return OR_EINVAL;
    }
    /* A bounded heap of the top k and a full sort truncated to k retain the
     * same candidates in the same order: candidateBefore is a total order. */
    qsort(cs, (size_t)count, sizeof(cand), cand_cmp);
    if (top_k > 0 && top_k < count) count = top_k;
    double total = 0, max_logit = cs[0].logit;
    for (int i = 0; i < count; i++) {
        cs[i].prob = exp((cs[i].logit - max_logit) / temperature);
        total += cs[i].prob;
    }
    if (top_p < 1) {
        double mass = 0;
        for (int i = 0; i < count; i++) {
            mass += cs[i].prob;
            if (mass >= top_p * total) {
                count = i + 1;
                total = mass;
                break;
            }
        }
    }
    double draw = or_rng_float64(rng_state) * total;
    int id = cs[count - 1].id;
    for (int i = 0; i < count; i++) {
        draw -= cs[i].prob;
        if (draw < 0) {
            id = cs[i].id;
            break;
        }
    }
    free(cs);
    return id;
}
