/*
 * srq_oracle.h -- CPU restatement of sr_go_tranformer's quantized-weight
 * inference path (cmd/monolith/monolith.go), used ONLY as test
 * infrastructure: the parity checker for the HIP kernels and the timed CPU
 * baseline.  Nothing in the product links or calls this code.
 *
 * Every function names the reference lines it restates (M: = cmd/monolith/
 * monolith.go).  The reduction orders are the reference's; compile with
 * -ffp-contract=off so no multiply-add is fused (the reference's own bits are
 * toolchain-specific: Go may fuse on arm64 and does not on amd64).
 *
 * Pinning (how each function is checked, see tests/test_oracle_*.py):
 *   rng / normal            closed form: SplitMix64 published constants, brute
 *                           force against an independent Python integer model
 *   pack q8/q4, scales      independent numpy-float64 restatement (bit-exact),
 *                           exhaustive edge sets, reference property tests
 *                           (q8_test.go:39-53, q4_test.go:95-143)
 *   q4 pair table, copyRow  all 256 byte codes enumerated (q4_test.go:95-126)
 *   linear q8/q4/f32        FP64 closed form, tol 2e-5*max(1,|want|)
 *                           (q8_test.go:55-96, q4_test.go:145-191), batch and
 *                           worker invariance bit-exact
 *   step (rms, rope, attn,  Transformers FP32 logits + every K/V row of the
 *   swiglu, kv pages)       reference's testdata/hf-* fixtures, tol 2e-5
 *                           (hf_inference_test.go:32-124); quantized forward
 *                           == FP32 forward on copyRow-reconstructed weights,
 *                           tol 3e-5 (q8_test.go:241-274)
 *   rope frequencies        testdata/hf-llama3/frequencies.json (exact f32)
 *   greedy / sampling       closed form (first max), brute force on tiny
 *                           distributions
 */
#ifndef SRQ_ORACLE_H
#define SRQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_F32 = 0, OR_Q8 = 1, OR_Q4 = 2 };
enum { OR_OK = 0, OR_EINVAL = -22, OR_ERANGE = -34, OR_ENOSPC = -28, OR_ENONFINITE = -33 };

/* ---- RNG (M:1411-1439) ---------------------------------------------- */
uint64_t or_rng_uint64(uint64_t *state);
double or_rng_float64(uint64_t *state);
double or_rng_normal(uint64_t *state);
int64_t or_rng_intn(uint64_t *state, int64_t n);
/* dst[i] = f32(Normal()*scale), sequential from *state (M:5218). */
void or_fill_normal(uint64_t *state, double scale, float *dst, int64_t n);
/* dst[i] = f32(Float64()*2-1) (linear_backward_test.go:35-45). */
void or_fill_uniform(uint64_t *state, float *dst, int64_t n);

/* ---- packing (M:3793-3898, M:857-880) -------------------------------- */
float or_low_bit_scale(float amax, double levels);
int8_t or_q8_value(float v, float scale);
int8_t or_q4_value(float v, float scale);
/* Stream rows*cols values through 64-column blocks exactly as readParam. */
void or_pack_q8(const float *src, int64_t rows, int64_t cols, int8_t *values, float *scales);
void or_pack_q4(const float *src, int64_t rows, int64_t cols, uint8_t *values, float *scales);
void or_q4_pairs(float *table /* [256][2] */);
/* copyRow (M:3900-3921). */
void or_copy_row(int fmt, int64_t rows, int64_t cols, const void *values, const float *scales,
                 int64_t row, float *dst);

/* ---- linear (M:3942-4780) ------------------------------------------- */
typedef struct {
    int fmt;           /* OR_F32 / OR_Q8 / OR_Q4 */
    int64_t rows, cols;
    const void *values; /* f32 data, int8 codes or packed nibbles */
    const float *scales;
} or_param;

/* y[n x rows] = x[n x cols] . W^T with the reference's tile order, wide-sum
 * fallback and worker partition (workers <= 1 runs inline). */
void or_linear(const or_param *w, float *y, const float *x, int n, int workers);
/* Sum_g f64(scale_g) * Sum_j f64(x_j) f64(code_j): the closed form the
 * reference's tests compare against (q8_test.go:113-117). */
void or_linear_closed_f64(const or_param *w, double *y, const float *x, int n);

/* ---- model step (M:4961-5352, M:5846-6456) --------------------------- */
typedef struct {
    int vocab, dim, layers, heads, kv_heads, hidden, context;
    double rope_theta, norm_eps;
    int tied;
    /* Llama 3 RoPE scaling (M:126-132, M:4961-4977); rope_llama3 = 0 off */
    int rope_llama3;
    double rope_factor, rope_low, rope_high;
    int rope_original;
} or_config;

enum { OR_N1 = 0, OR_Q, OR_K, OR_V, OR_O, OR_N2, OR_GATE, OR_UP, OR_DOWN, OR_QB, OR_KB, OR_VB, OR_LAYER_PARAMS };

typedef struct or_model or_model;
typedef struct or_cache or_cache;

or_model *or_model_create(const or_config *c);
void or_model_destroy(or_model *m);
/* Set a parameter; the model keeps the pointers (caller owns the memory).
 * layer = -1 addresses the embedding (kind 0), final norm (kind 1) and the
 * untied output head (kind 2). */
int or_model_set(or_model *m, int layer, int kind, const or_param *p);
/* hfInverseFrequency (M:4961-4977) */
float or_inverse_frequency(double theta, int head_dim, int index, const or_config *c);
const float *or_model_cos(const or_model *m);
const float *or_model_sin(const or_model *m);

or_cache *or_cache_create(or_model *m);
void or_cache_destroy(or_cache *c);
int or_cache_pos(const or_cache *c);
/* Row of the K (which=0) or V (which=1) plane at (layer, pos) (M:6038-6043). */
const float *or_cache_row(const or_cache *c, int layer, int pos, int which);
/* Overwrite a K/V row (used to seed the CPU baseline from device pages). */
int or_cache_set_rows(or_cache *c, int layer, int pos0, int count, const float *k, const float *v);
int or_cache_set_pos(or_cache *c, int pos);

/* prefillSelected (M:6245-6456): chunks are concatenated in tokens[];
 * want may be NULL (all sessions).  logits: [sessions x vocab]. */
int or_step(or_model *m, int sessions, or_cache **caches, const int *chunk_lens, const int *tokens,
            const uint8_t *want, float *logits, int workers);

/* Greedy argmax with the lowest-ID tie rule (M:1215-1223). -1 on non-finite. */
int or_argmax(const float *logits, int vocab);
/* sampleWithBlocked (M:7320-7426). Returns id, or <0 on error. */
int or_sample(const float *logits, int vocab, const int *history, int nhistory, double temperature,
              int top_k, double top_p, double repeat_penalty, uint64_t *rng_state, int blocked);

/* Single pieces of the step, exported for unit tests of the glue. */
void or_rms(float *y, const float *x, const float *w, int n, int d, double eps);
void or_rope(const or_model *m, float *x, int heads, int pos);
double or_attend(const float *q, float *out, float *scores, int hd, int length,
                 const float *const *keys, const float *const *vals);

#ifdef __cplusplus
}
#endif
#endif
