/*
 * srq.h -- C ABI of the MI355X (gfx950) quantized-weight inference path.
 *
 * Drop-in for the kernel seam of sr_go_tranformer's Go engine
 * (cmd/monolith/monolith.go, cited as M:line).  The Go engine (tokenizer,
 * scheduler, sampling policy, HTTP/SSE) stays as it is and calls these
 * entry points through cgo; see INTEGRATION.md for the binding.
 *
 * Conventions
 *  - Every function returns int: SRQ_OK (0) or a negative SRQ_E* code.  No
 *    function aborts or throws across the boundary; srq_last_error() gives
 *    a message for the calling thread's last failure.
 *  - Pointers documented as "device" address GPU memory (srq_alloc, or any
 *    HIP allocation on the executor's device).  All other pointers are host.
 *  - An srq_exec owns one HIP stream plus scratch.  Like kernelExecutor it
 *    has a single caller: calls on one executor must not overlap.  Every
 *    call joins its own GPU work before it returns (M:3704-3708), except
 *    where a function says otherwise.
 *  - Weights are device-resident and immutable after creation, so one
 *    srq_weight / srq_model can be shared read-only by many executors
 *    (M:4931-4932).
 */
#ifndef SRQ_H
#define SRQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SRQ_ABI_VERSION 1

#define SRQ_OK 0
#define SRQ_EDEVICE (-5)     /* HIP runtime / device failure                 */
#define SRQ_ENOMEM (-12)     /* device or host allocation failed             */
#define SRQ_EINVAL (-22)     /* precondition violated (shape, pointer, token) */
#define SRQ_ENOSPC (-28)     /* KV budget or page reservation exceeded        */
#define SRQ_ENONFINITE (-33) /* non-finite weight or logit                    */
#define SRQ_ERANGE (-34)     /* KV cache context exhausted                    */
#define SRQ_ECANCELED (-125) /* caller's cancel flag was set                  */
#define SRQ_EFILE (-2)       /* archive file missing, unreadable or short     */
#define SRQ_EFORMAT (-74)    /* archive metadata rejected (index, header,
                              * names, shapes, dtypes, extents)              */

/* Both enums are int-sized.  Compiled as C++ they have int as a fixed
 * underlying type, so a caller's out-of-range value (e.g. 7 from cgo) is a
 * valid value of the type that the entry points then reject with
 * SRQ_EINVAL, not undefined behaviour. */
#ifdef __cplusplus
typedef enum : int { SRQ_F32 = 0, SRQ_Q8 = 1, SRQ_Q4 = 2 } srq_format;
typedef enum : int { SRQ_SRC_F32 = 0, SRQ_SRC_BF16 = 1, SRQ_SRC_F16 = 2 } srq_src_dtype;
#else
typedef enum { SRQ_F32 = 0, SRQ_Q8 = 1, SRQ_Q4 = 2 } srq_format;
typedef enum { SRQ_SRC_F32 = 0, SRQ_SRC_BF16 = 1, SRQ_SRC_F16 = 2 } srq_src_dtype;
#endif

typedef struct srq_exec srq_exec;
typedef struct srq_weight srq_weight;
typedef struct srq_model srq_model;
typedef struct srq_pool srq_pool;
typedef struct srq_cache srq_cache;

/* ---- diagnostics ------------------------------------------------------ */
int srq_abi_version(void);
/* Message of the calling thread's last failed call ("" if none). */
const char *srq_last_error(void);

/* ---- device memory (for callers without a GPU allocator, e.g. cgo) ---- */
int srq_device_count(int *count);
int srq_alloc(int device, size_t bytes, void **dptr);
int srq_free(void *dptr);
int srq_copy_h2d(srq_exec *e, void *dst_device, const void *src_host, size_t bytes);
int srq_copy_d2h(srq_exec *e, void *dst_host, const void *src_device, size_t bytes);
int srq_copy_d2d(srq_exec *e, void *dst_device, const void *src_device, size_t bytes);

/* ---- executor: newKernelExecutor / close (M:3730-3782) ----------------- */
int srq_exec_create(int device, srq_exec **out);
/* Joins all outstanding work, then releases the stream and scratch. */
int srq_exec_destroy(srq_exec *e);
int srq_exec_synchronize(srq_exec *e);
/* The executor's hipStream_t, for callers that order their own work or
 * time kernels with HIP events.  Valid until srq_exec_destroy. */
void *srq_exec_stream(srq_exec *e);

/* ---- packing: readParam + lowBitScale + putQuantized (M:857-880,
 *      M:3819-3898) ----------------------------------------------------- */
/* Byte sizes of packed storage: Q8 values rows*cols int8; Q4 values
 * rows*ceil(cols/2) bytes (low nibble = even column, odd width => zero high
 * pad nibble); scales rows*ceil(cols/64) floats, index row*groups+g.
 * F32: values rows*cols*4, scales 0. */
int srq_packed_bytes(srq_format fmt, int64_t rows, int64_t cols, int64_t *values_bytes, int64_t *scales_bytes);
/* Pack a [rows x cols] row-major source (device; f32, bf16 or f16 words,
 * decoded exactly as M:884-920) into Q8 or Q4 storage (device), bit-exact
 * with the reference.  Non-finite source values => SRQ_ENONFINITE
 * ("non-finite HF weight", M:910-912). */
int srq_pack(srq_exec *e, srq_format fmt, int64_t rows, int64_t cols, const void *src, srq_src_dtype dtype,
             void *values, float *scales);
/* srq_pack from a host source, as readParam streams host values
 * (M:857-880): the bytes pass through pinned 16 MiB chunks into device
 * staging, then pack on the device with identical results.  cancel (host,
 * nullable) is polled between chunks (the reference's per-chunk context
 * check, M:894): SRQ_ECANCELED, nothing written. */
int srq_pack_host(srq_exec *e, srq_format fmt, int64_t rows, int64_t cols, const void *src_host,
                  srq_src_dtype dtype, void *values, float *scales, const volatile int32_t *cancel);

/* Synthetic initialisation: dst[i] = f32(Normal()*scale) of the reference's
 * RNG seeded with `seed` (RNG{seed}.Normal, M:1411-1439, as NewModel draws
 * weights, M:5218): element i uses the SplitMix64 draws 2i+1 and 2i+2, so
 * the device fills in parallel the sequence a serial RNG would produce
 * (FP64 log/cos may differ from Go's in the last ulp before the f32
 * rounding).  dst is device memory. */
int srq_fill_normal(srq_exec *e, float *dst, int64_t count, uint64_t seed, double scale);

/* ---- weights: Param{Rows, Cols, Q8, Q4, Data} (M:3784-3791) ------------ */
/* Allocate device storage and pack (Q8/Q4) or convert (F32) from src. */
int srq_weight_create(srq_exec *e, srq_format fmt, int64_t rows, int64_t cols, const void *src,
                      srq_src_dtype dtype, srq_weight **out);
/* srq_weight_create from a host source (staged as srq_pack_host). */
int srq_weight_create_host(srq_exec *e, srq_format fmt, int64_t rows, int64_t cols, const void *src_host,
                           srq_src_dtype dtype, const volatile int32_t *cancel, srq_weight **out);
/* Wrap caller-owned packed device storage (not freed by destroy). */
int srq_weight_wrap(srq_format fmt, int64_t rows, int64_t cols, void *values, float *scales, srq_weight **out);
int srq_weight_destroy(srq_weight *w);
int srq_weight_info(const srq_weight *w, int *fmt, int64_t *rows, int64_t *cols, void **values, float **scales);

/* copyRow (M:3900-3921) for count rows: dst[i] = row rows[i] dequantized.
 * rows and dst are device pointers; dst is [count x cols] f32. */
int srq_dequant_rows(srq_exec *e, const srq_weight *w, const int32_t *rows, int32_t count, float *dst);

/* ---- linear: linearIntoWithExecutor (M:3942-4780) ---------------------- */
/* y[n x w.rows] = x[n x w.cols] . W^T; x, y device, disjoint; n 1..1024.
 * Q8 / Q4 / F32 dispatch as the reference.  Rows holding any |x| above
 * MaxFloat32/(2*64*127) take an FP64 path (M:4346-4382), chosen per row.
 * Results are deterministic, and a row's bits depend on neither its
 * position in the batch nor on n within each of the two paths: n <= 16
 * takes the GEMV (bit-identical to the row computed alone), n > 16 the MFMA
 * GEMM (bit-identical for every n > 16; its split-K plan depends on the
 * matrix shape only).  The two paths differ in rounding (both within 1e-4
 * of the reference). */
int srq_linear(srq_exec *e, float *y, const float *x, const srq_weight *w, int32_t n);
/* Same computation, stream-ordered on the executor without joining: for
 * callers that chain work on the executor's stream (or time it with HIP
 * events).  Inputs must stay valid until the stream reaches the call. */
int srq_linear_enqueue(srq_exec *e, float *y, const float *x, const srq_weight *w, int32_t n);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid
 * hipMalloc): srq_linear_enqueue -- the same kernels and bit-identical
 * results, stream-ordered on the executor without joining -- that allocates
 * nothing.  The GEMM path's split-K partial sums and wide-row flags go to a
 * fixed device array of SRQ_NOALLOC_SCRATCH_BYTES owned by the library (one
 * per GPU, held until the process ends) instead of the executor's
 * workspace.  A call whose plan needs more runs its rows in GEMM
 * sub-batches that fit the array, with the same bits (a row's GEMM result
 * does not depend on the rows beside it); with 64 MiB every n up to 1024
 * fits, and a plan that could not fit 17 rows would be rejected with
 * SRQ_EINVAL before anything is enqueued.  Every call on one GPU shares that array and
 * leaves its contents behind: calls that overlap on one GPU (executors or
 * streams not ordered against each other) race, so the caller orders them. */
#define SRQ_NOALLOC_SCRATCH_BYTES (64u << 20)
int srq_linear_noalloc(srq_exec *e, float *y, const float *x, const srq_weight *w, int32_t n);

/* ---- model: HF Llama/Mistral/Qwen2 profile (M:4985-5050) --------------- */
typedef struct {
    int32_t vocab, dim, layers, heads, kv_heads, hidden, context;
    double rope_theta, norm_eps;
    int32_t tied;          /* 1: head = token embedding                      */
    int32_t qkv_bias;      /* 1: q/k/v biases present (Qwen2)                */
    int32_t rope_llama3;   /* 1: Llama 3 RoPE scaling (M:4966-4976)          */
    double rope_factor, rope_low, rope_high;
    int32_t rope_original;
} srq_model_config;

/* Tensor kinds for srq_model_load (names follow hfTensorSpecs M:406-421). */
enum {
    SRQ_T_EMBED = 0,      /* model.embed_tokens.weight   [vocab x dim]   */
    SRQ_T_FINAL_NORM = 1, /* model.norm.weight           [dim]           */
    SRQ_T_OUTPUT = 2,     /* lm_head.weight (untied)     [vocab x dim]   */
    SRQ_T_ATTN_NORM = 10, /* input_layernorm             [dim]           */
    SRQ_T_Q = 11,         /* self_attn.q_proj            [dim x dim]     */
    SRQ_T_K = 12,         /* self_attn.k_proj            [kvdim x dim]   */
    SRQ_T_V = 13,         /* self_attn.v_proj            [kvdim x dim]   */
    SRQ_T_O = 14,         /* self_attn.o_proj            [dim x dim]     */
    SRQ_T_FFN_NORM = 15,  /* post_attention_layernorm    [dim]           */
    SRQ_T_GATE = 16,      /* mlp.gate_proj               [hidden x dim]  */
    SRQ_T_UP = 17,        /* mlp.up_proj                 [hidden x dim]  */
    SRQ_T_DOWN = 18,      /* mlp.down_proj               [dim x hidden]  */
    SRQ_T_Q_BIAS = 19,    /* self_attn.q_proj.bias       [dim]           */
    SRQ_T_K_BIAS = 20,    /* self_attn.k_proj.bias       [kvdim]         */
    SRQ_T_V_BIAS = 21,    /* self_attn.v_proj.bias       [kvdim]         */
    /* srq_model_weight only (no counterpart in the reference's specs): the
     * fused matrices a step streams. */
    SRQ_T_QKV = 22,       /* q, k, v rows stacked       [dim+2*kvdim x dim] */
    SRQ_T_GATE_UP = 23    /* gate rows, then up rows    [2*hidden x dim] */
};

/* weight_format: "f32", "q8", "q4" or "q4-mixed" (M:566-582: q4-mixed keeps
 * embeddings and the head Q8).  Allocates all device storage up front. */
int srq_model_create(srq_exec *e, const srq_model_config *c, const char *weight_format, srq_model **out);
/* Load one tensor from device memory (f32/bf16/f16), packing on device. */
int srq_model_load(srq_model *m, int kind, int layer, const void *src, srq_src_dtype dtype);
/* readParam (M:857-880): load one tensor from host memory (staged as
 * srq_pack_host; cancel polled between 16 MiB chunks, SRQ_ECANCELED leaves
 * the tensor unwritten). */
int srq_model_load_host(srq_model *m, int kind, int layer, const void *src_host, srq_src_dtype dtype,
                        const volatile int32_t *cancel);
int srq_model_destroy(srq_model *m);
/* hfWeightLayoutFor byte accounting (M:591-619) of the resident weights. */
int srq_model_resident_bytes(const srq_model *m, int64_t *bytes);
/* Borrow a view of one matrix (valid while the model lives); SRQ_T_QKV and
 * SRQ_T_GATE_UP give the fused storage. */
int srq_model_weight(srq_model *m, int kind, int layer, srq_weight **out);
/* The FP32 RoPE tables (M:5034-5043), [context x head_dim/2] each, host. */
int srq_model_rope_tables(const srq_model *m, float *cos_out, float *sin_out);
/* openHFArchiveFormat (M:648-850) + readParam / readTensorValues
 * (M:855-920): load every tensor of m's profile from the Transformers
 * archive in directory dir -- model.safetensors, or the shards that
 * model.safetensors.index.json names -- converting F32 / F16 / BF16 values
 * and packing them to m's format on the device.  The archive is checked as
 * the reference checks it (index names and paths, at most 128 shards, file
 * and header size limits, duplicate-free UTF-8 JSON headers, the profile's
 * exact names and shapes from hfProfileSpecs M:426-440, dtype widths,
 * exact extents, no gaps, overlaps or trailing bytes, nothing missing):
 * failures are SRQ_EFORMAT (or SRQ_EFILE for I/O) and are found before any
 * weight is written.  A non-finite value fails with SRQ_ENONFINITE and the
 * tensor's name.  cancel (host, nullable) is polled between 16 MiB chunks
 * (the reference's context check, M:894): SRQ_ECANCELED.  After any failure
 * m holds partly loaded weights and should be destroyed.  source_bytes
 * (nullable) receives the archive's total file size.  Files are read with
 * pread through pinned staging; copies and packing overlap the reads. */
int srq_model_load_safetensors(srq_model *m, const char *dir, const volatile int32_t *cancel,
                               int64_t *source_bytes);
/* The archive checks of srq_model_load_safetensors alone, on the host, for
 * configuration c (no device, nothing allocated on a GPU): the reference
 * inspects the metadata before any parameter storage exists (M:121-122). */
int srq_archive_check(const srq_model_config *c, const char *dir, int64_t *source_bytes);

/* ---- paged KV: pagePool / KVCache (M:5846-6062) ------------------------ */
/* A pool owns max_pages device pages of 2*32*kvdim*layers floats, laid out
 * [layer][K 32 x kvdim | V 32 x kvdim] as the reference's pages. */
int srq_pool_create(srq_model *m, int32_t max_pages, srq_pool **out);
int srq_pool_destroy(srq_pool *p);
/* A cache reserves up to reserve_pages pages of its pool (pagePool
 * reservation); pages are taken as positions grow. */
int srq_cache_create(srq_pool *p, int32_t reserve_pages, srq_cache **out);
int srq_cache_destroy(srq_cache *c);
int srq_cache_pos(const srq_cache *c, int32_t *pos);
/* Copy K and V rows [pos0, pos0+count) of one layer to host [count x kvdim]. */
int srq_cache_read(srq_exec *e, const srq_cache *c, int32_t layer, int32_t pos0, int32_t count, float *k,
                   float *v);

/* ---- step: prefillSelected (M:6245-6456) ------------------------------- */
/* Appends chunk_lens[i] tokens (host, concatenated in tokens) to caches[i]
 * for 1..256 sessions, at most 1024 rows in total, and returns last-row
 * logits per session in *logits (device, [sessions x vocab], borrowed until
 * the executor's next step).  A cache owned by a live srq_decoder is
 * rejected (SRQ_EINVAL).  want (host, nullable) selects sessions whose
 * logits are computed; unselected rows are zeroed (M:6438-6448).  Every
 * argument is validated before anything is mutated; positions are committed
 * only on success.  cancel (host, nullable) is polled as layers complete
 * (M:6213, M:6377): the host then stays at most eight layers ahead of the
 * device (a progress event every four), so a flag raised while the step
 * runs stops it within about 8 to 12 layers;
 * nonzero => SRQ_ECANCELED once the layers already queued have drained, no
 * positions committed.  Without a flag the step is queued whole.
 * logits_host (nullable) receives a host copy.  With neither logits_host
 * nor a cancel flag the call returns once the step is queued (positions
 * committed): the executor's later calls run after it on its stream, and a
 * device fault surfaces at the next call that waits for the stream. */
int srq_step(srq_exec *e, srq_model *m, int32_t sessions, srq_cache *const *caches, const int32_t *chunk_lens,
             const int32_t *tokens, const uint8_t *want, float **logits, float *logits_host,
             const volatile int32_t *cancel);

/* Greedy argmax over rows of device logits with the lowest-ID tie rule
 * (M:1215-1223, M:7331-7358); ids (host) [rows].  SRQ_ENONFINITE if any
 * logit of a row is not finite. */
int srq_argmax(srq_exec *e, const float *logits, int32_t rows, int32_t vocab, int32_t *ids);

/* sampleWithBlocked (M:7320-7426) for rows of device logits [* x vocab].
 * Per row: value = f64(logit), repeat penalty for ids in the row's history
 * (divide if > 0, else multiply), the blocked id excluded; temperature 0 is
 * the first maximum (lowest id on ties) with no draw; otherwise candidates
 * ordered by value descending then id ascending, cut to top_k (0: off), then
 * to the shortest prefix holding top_p of the mass (>= 1: off), and one
 * SplitMix64 Float64 draw picks the candidate (M:7360-7425).  Host arrays:
 * row_ids [rows] (nullable: row k is logits row k) names the logits row each
 * of the rows samples, so a caller samples only the sessions of a step that
 * want a token; history [rows x history_stride] with history_len[rows] valid ids (both
 * nullable), blocked [rows] (-1 none; nullable), rng_state [rows] (in/out:
 * advanced by one draw per row sampled at temperature != 0), ids [rows] out.
 * SRQ_ENONFINITE if a row holds a non-finite logit; SRQ_EINVAL if a row has
 * no candidate.  Masses are summed exactly in fixed point (2^-44 of the top
 * probability), so a draw can differ from the reference's f64 running sums
 * only when it falls within ~1e-12 of a candidate boundary.  Device scratch:
 * at most 64 MiB per executor (about 1 MiB per row of a 128256-id
 * vocabulary); calls with more rows sample them in groups that fit, with
 * the same ids and states. */
typedef struct {
    double temperature;
    int32_t top_k;
    double top_p;
    double repeat_penalty;
} srq_sampling;
int srq_sample(srq_exec *e, const float *logits, int32_t rows, const int32_t *row_ids, int32_t vocab,
               const srq_sampling *params,
               const int32_t *history, const int32_t *history_len, int32_t history_stride, const int32_t *blocked,
               uint64_t *rng_state, int32_t *ids);

/* Graph-replayed greedy decoding for one session (the decode loop of
 * inferHFIDs, M:1212-1238).  create: reserves pages for max_steps positions
 * and captures one decode step (embed first_token -> layers -> final norm +
 * head -> device argmax -> next token) as a HIP graph.  run: enqueues
 * `steps` replays without joining (each replay commits one position).
 * tokens: joins, copies the tokens produced so far (host, [steps run]) and
 * commits the cache position.  If a step's logits were not finite it
 * returns SRQ_ENONFINITE with *count = the tokens before that step, and the
 * position committed through that step (inferHFIDs, M:1212-1238); replays
 * after it are discarded.  The decoder owns its workspace and, while it
 * lives, its cache: srq_step and a second srq_decoder_create on that cache
 * fail with SRQ_EINVAL until srq_decoder_destroy. */
typedef struct srq_decoder srq_decoder;
/* flags: SRQ_DECODER_EAGER launches every kernel of each step directly
 * instead of replaying a captured graph (for tracers that cannot follow
 * graph launches); results are identical. */
#define SRQ_DECODER_EAGER 1
int srq_decoder_create(srq_exec *e, srq_model *m, srq_cache *c, int32_t first_token, int32_t max_steps,
                       int32_t flags, srq_decoder **out);
int srq_decoder_run(srq_decoder *d, int32_t steps);
int srq_decoder_tokens(srq_decoder *d, int32_t *out, int32_t *count);
int srq_decoder_destroy(srq_decoder *d);

/* inferHFIDs (M:1185-1240): prefill ids in chunk-token steps, then count
 * greedy tokens (decode steps replayed as one HIP graph, argmax on device).
 * eos < 0 disables the EOS stop.  out_tokens (host) [count]; *produced
 * receives the number of tokens written, also when a step's logits are not
 * finite (SRQ_ENONFINITE: the tokens before that step). */
int srq_generate_greedy(srq_exec *e, srq_model *m, srq_cache *c, const int32_t *ids, int32_t n_ids,
                        int32_t chunk, int32_t count, int32_t eos, int32_t *out_tokens, int32_t *produced);

#ifdef __cplusplus
}
#endif
#endif
