/*
 * flux_amd.h -- C ABI of the MI355X-native (gfx950) SmolLM2 FP32 token loop.
 *
 * Drop-in boundary for Flux's native path.  The reference binds the same
 * functionality as PyTorch custom classes and CUDA launchers; every entry point
 * below names the reference interface it replaces (paths are relative to the
 * reference repository).  Plain pointers and sizes only: device pointers are
 * hipMalloc'd (or torch-allocated) device memory, streams are hipStream_t, and
 * nothing here depends on PyTorch.
 *
 * Conventions
 *  - Every function returns FLUX_OK (0) or an error code; flux_last_error()
 *    returns the calling thread's message for the last failure.  Invalid
 *    arguments are rejected before any launch (reference launchers return
 *    cudaErrorInvalidValue, e.g. csrc/packed_gate_up_gemv/packed_gate_up_gemv_cuda.cu:57-59).
 *  - Launches are asynchronous on the given stream and never allocate, except
 *    the runtime constructors, which own their buffers (as the reference's
 *    at::empty allocations in native_decode_runtime_cuda.cu:1162-1224).
 *  - Weights are borrowed: the caller keeps them alive for the runtime's life
 *    (the reference holds refcounted tensors, native_decode_runtime_cuda.cu:796-805).
 *  - Geometry is fixed to SmolLM2-135M: 30 layers, hidden 576, intermediate
 *    1536, 9 query heads, 3 KV heads, head_dim 64.  Vocabulary and capacity are
 *    runtime values; capacity may be up to FLUX_MAX_CAPACITY (the reference caps
 *    at 8192, native_decode_runtime_cuda.cu:36).
 */
#ifndef FLUX_AMD_H_
#define FLUX_AMD_H_

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FLUX_LAYERS 30
#define FLUX_HIDDEN 576
#define FLUX_INTERMEDIATE 1536
#define FLUX_QUERY_HEADS 9
#define FLUX_KV_HEADS 3
#define FLUX_HEAD_DIM 64
#define FLUX_PACKED_QKV_WIDTH 960
#define FLUX_PACKED_GATE_UP_WIDTH 3072
#define FLUX_MAX_CAPACITY 16384
/* Largest accepted bound of the fused decode kernel's cross-workgroup waits:
 * 1e9 ticks of the 100 MHz wall clock = 10 s. */
#define FLUX_MAX_WAIT_TICKS 1000000000ull

enum flux_status {
    FLUX_OK = 0,
    FLUX_ERROR_INVALID_VALUE = 1, /* bad pointer / size / shape */
    FLUX_ERROR_HIP = 2,           /* a HIP runtime call failed */
    FLUX_ERROR_STATE = 3,         /* capacity exhausted, reuse without prefill/reset */
    FLUX_ERROR_DEVICE = 4         /* a kernel reported a device-side error */
};

/* Borrowed model weights (row-major float32, device memory).
 * Mirrors the tensor arguments of NativeSmolLM2Decode / NativeSmolLM2Prefill
 * (csrc/native_decode_runtime/native_decode_runtime.h:59-77,
 *  csrc/native_prefill_runtime/native_prefill_runtime.h:16-31). */
typedef struct flux_weights {
    const float* embedding;                   /* [vocab, 576] */
    const float* lm_head;                     /* [vocab, 576] (tied: may equal embedding) */
    const float* final_norm;                  /* [576] */
    const float* input_norm[FLUX_LAYERS];     /* [576] */
    const float* packed_qkv[FLUX_LAYERS];     /* [960, 576] = cat(q, k, v) */
    const float* o_proj[FLUX_LAYERS];         /* [576, 576] */
    const float* post_norm[FLUX_LAYERS];      /* [576] */
    const float* gate_up[FLUX_LAYERS];        /* [3072, 576] = cat(gate, up) */
    const float* down[FLUX_LAYERS];           /* [576, 1536] */
    int64_t vocab_size;
} flux_weights;

typedef struct flux_decode flux_decode;
typedef struct flux_prefill flux_prefill;

/* Stable runtime-owned device buffers (NativeSmolLM2Decode::addresses(),
 * native_decode_runtime_cuda.cu:1490-1505, and the tensor accessors :1470-1488). */
typedef struct flux_decode_buffers {
    int64_t* input_token;      /* [1] */
    float* logits;             /* [vocab] */
    int64_t* generated_tokens; /* [capacity] */
    int64_t* generation_step;  /* [1] */
    float* key_cache;          /* [30, 1, 3, capacity, 64] */
    float* value_cache;        /* [30, 1, 3, capacity, 64] */
    int64_t* position;         /* [1] */
    int64_t* cache_length;     /* [1] */
    void* workspace;           /* exchange arena of the fused decode kernel */
    void* hidden_a;            /* layer-output exchange words, even layers */
    void* hidden_b;            /* layer-output exchange words, odd layers */
    void* final_norm_output;   /* argmax exchange words */
    void* attention_workspace; /* attention partial exchange words */
    int64_t capacity;
    int64_t vocab_size;
    int64_t workspace_bytes;
    int64_t cache_bytes;
    int64_t stable_buffer_bytes;
} flux_decode_buffers;

typedef struct flux_prefill_buffers {
    float* prefill_logits;          /* [vocab] */
    void* prefill_workspace;        /* activation slab */
    float* attention_output;        /* [S, 576] attention rows */
    float* final_hidden;            /* [576] final-norm output of the last row */
    int64_t* initial_token;         /* [1] prefill argmax */
    int64_t sequence_length;
    int64_t capacity;
    int64_t workspace_bytes;
} flux_prefill_buffers;

/* Thread-local message for the last failing call ("" if none). */
const char* flux_last_error(void);

/* Version string of this library. */
const char* flux_version(void);

/* ------------------------------------------------------------------------ */
/* Decode runtime: replaces torch.classes.flux.NativeSmolLM2Decode
 * (csrc/native_decode_runtime/native_decode_runtime.h:57-119,
 *  native_decode_runtime_cuda.cu:742-865; registered in
 *  native_decode_runtime_torch.cpp:38-79).
 * key_sources/value_sources: per layer [1, 3, source_lengths[i], 64] contiguous
 * float32 with source_lengths[i] >= position; may be NULL when position == 0.
 * Builds the stable buffers, imports the cache and runs one warm-up step (the
 * reference warms its step before capturing it).  `stream` orders the setup (the
 * reference's current stream). */
int flux_decode_create(const flux_weights* weights, const float* rope_cos, const float* rope_sin, int64_t capacity,
                       int64_t position, const int64_t* initial_token, const float* const* key_sources,
                       const float* const* value_sources, const int64_t* source_lengths, const double* epsilons,
                       const double* attention_scales, hipStream_t stream, flux_decode** out);

/* One decode step; returns the logits buffer.  (native_decode_runtime_cuda.cu:907-931,
 * which copies the token and replays a CUDA graph of ~300 launches.)  Here the whole
 * step is one kernel, launched directly: `token` (device [1,1] int64, or NULL for the
 * fed-back argmax) is read by the step itself in stream order, so there is no copy.
 * Like flux_decode_generate_greedy, it first returns FLUX_ERROR_DEVICE when an
 * earlier launch that has finished reported a device-side error (non-blocking
 * check of a host-visible error word); prefill or reset re-arms the runtime.
 * The fused kernel needs every workgroup resident at once (one per CU):
 * flux_decode_generate_greedy launches cooperatively (a grid that cannot be
 * co-resident fails at launch); a replay launches plainly (a cooperative launch
 * costs ~20 us per token), and a step that starts while other work holds CUs
 * reports device error 1 through its bounded waits instead of hanging.  `stream`
 * must stay valid until the runtime's next call on another stream, synchronising
 * call or destruction (the completion event is recorded then). */
int flux_decode_replay(flux_decode* runtime, const int64_t* token, hipStream_t stream, float** logits);

/* `decode_steps` greedy steps in one launch of the fused decode kernel; returns
 * the generated-token buffer.  (native_decode_runtime_cuda.cu:933-960)
 * A step computed after a device-side error holds token -1. */
int flux_decode_generate_greedy(flux_decode* runtime, int64_t decode_steps, hipStream_t stream,
                                int64_t** generated_tokens);

/* Synchronously restore token, cache and position.  (native_decode_runtime_cuda.cu:962-981) */
int flux_decode_reset(flux_decode* runtime, const int64_t* token, const float* const* key_sources,
                      const float* const* value_sources, const int64_t* source_lengths, int64_t position,
                      hipStream_t stream);

/* Synchronising scalar reads (read_scalar, native_decode_runtime_cuda.cu:1029-1040).
 * They also surface device-side errors as FLUX_ERROR_DEVICE. */
int flux_decode_position(flux_decode* runtime, int64_t* out);
int flux_decode_cache_length(flux_decode* runtime, int64_t* out);
int flux_decode_generation_step(flux_decode* runtime, int64_t* out);
int flux_decode_replay_count(const flux_decode* runtime, int64_t* out);
int flux_decode_capacity(const flux_decode* runtime, int64_t* out);
int flux_decode_get_buffers(const flux_decode* runtime, flux_decode_buffers* out);
/* Wait for outstanding work and return the device error word (0 = none). */
int flux_decode_device_error(flux_decode* runtime, int32_t* out);

/* Bound, in 100 MHz wall-clock ticks, of every cross-workgroup wait of later
 * flux_decode_generate_greedy launches (default 200 ms; replays keep the default).  A wait that exceeds it records device error 1; the steps it
 * affects report token -1, and the next runtime call raises FLUX_ERROR_DEVICE.
 * Bounds above FLUX_MAX_WAIT_TICKS (10 s) are rejected with
 * FLUX_ERROR_INVALID_VALUE and leave the current bound unchanged, so every wait
 * stays bounded.
 * No counterpart in the reference: the failure-handling test sets a tiny bound to
 * drive that path with every kernel still exiting normally. */
int flux_decode_set_wait_limit(flux_decode* runtime, uint64_t ticks);

/* Time the next `decode_steps` steps with events on `stream` (benchmark aid). */
/* Kernel launches and all device commands (launches, cross-stream event waits)
 * issued by flux_decode_replay since creation; the audit divides their growth by the
 * replays.  Counterpart of the launch count the reference's runtime audit takes with
 * torch.profiler (benchmarks/benchmark_flux.py:818-859). */
int flux_decode_replay_launches(const flux_decode* runtime, int64_t* kernel_launches, int64_t* device_commands);
/* Process-wide totals since load of the runtimes' host-blocking calls (stream/event
 * synchronisation, synchronous copies), device allocations and frees; the audit
 * compares them around replays (benchmarks/benchmark_flux.py:838-858). */
int flux_host_counters(int64_t* synchronizations, int64_t* allocations, int64_t* frees);
int flux_decode_generate_greedy_timed(flux_decode* runtime, int64_t decode_steps, hipStream_t stream,
                                      float* milliseconds);
void flux_decode_destroy(flux_decode* runtime);

/* ------------------------------------------------------------------------ */
/* Prefill runtime: replaces torch.classes.flux.NativeSmolLM2Prefill
 * (csrc/native_prefill_runtime/native_prefill_runtime.h:14-60,
 *  native_prefill_runtime_cuda.cu:355-445; registered in
 *  native_prefill_runtime_torch.cpp:5-45).  Creates its own decode runtime with
 * an empty cache, runs the prompt (input_ids: device [1, S] int64) and hands the
 * compact cache to the decode runtime without a copy. */
int flux_prefill_create(const flux_weights* weights, const float* rope_cos, const float* rope_sin, int64_t capacity,
                        const int64_t* input_ids, int64_t sequence_length, const double* epsilons,
                        const double* attention_scales, hipStream_t stream, flux_prefill** out);

/* Re-run the fixed-shape prompt and re-install the decode state
 * (native_prefill_runtime_cuda.cu:540-551). */
int flux_prefill_run(flux_prefill* runtime, const int64_t* input_ids, hipStream_t stream, float** logits);

/* max_new_tokens tokens: the prefill argmax plus max_new_tokens-1 decode steps
 * (native_prefill_runtime_cuda.cu:738-746). */
int flux_prefill_generate_greedy(flux_prefill* runtime, int64_t max_new_tokens, hipStream_t stream,
                                 int64_t** generated_tokens);

/* The attached decode runtime (owned by the prefill runtime). */
flux_decode* flux_prefill_decode(flux_prefill* runtime);
int flux_prefill_get_buffers(const flux_prefill* runtime, flux_prefill_buffers* out);
void flux_prefill_destroy(flux_prefill* runtime);

/* ------------------------------------------------------------------------ */
/* Single-layer decode runtime: replaces torch.classes.flux.NativeSmolLM2LayerDecode
 * (csrc/native_decode_runtime/native_decode_runtime.h:13-54,
 *  native_decode_runtime_cuda.cu:314-738,1340-1400; registered in
 *  native_decode_runtime_torch.cpp:5-36).
 * One decoder layer's token step (input hidden [1,1,576] -> output [1,1,576]) with
 * its own K/V cache [1,3,capacity,64] and device position.  A step is one launch of the
 * fused decode kernel in its single-layer mode (the reference replays a CUDA graph of the
 * step's kernels; the phases here exchange through an uncached arena, as the token
 * loop's do).  key_source/value_source: [1,3,source_length,64] contiguous,
 * source_length >= position (may be NULL when position == 0).  Each replay writes K/V
 * row *position, attends [0, *position] and advances the position.  Needs the same
 * device as flux_decode_create (every workgroup of a launch resident at once). */
typedef struct flux_layer_weights {
    const float* input_norm; /* [576] */
    const float* packed_qkv; /* [960, 576] */
    const float* o_proj;     /* [576, 576] */
    const float* post_norm;  /* [576] */
    const float* gate_up;    /* [3072, 576] */
    const float* down;       /* [576, 1536] */
} flux_layer_weights;

typedef struct flux_layer_decode flux_layer_decode;

/* NativeSmolLM2LayerDecode::addresses() counterparts (native_decode_runtime_cuda.cu:1388-1406).
 * The step's intermediates (query, attention, residual, SwiGLU, attention partials) are
 * exchanged through the workspace arena and not kept as arrays: those fields are NULL. */
typedef struct flux_layer_decode_buffers {
    float* input_hidden;       /* [576]: the last replay's (or the initial) input */
    float* output;             /* [576] */
    float* key_cache;          /* [1, 3, capacity, 64] */
    float* value_cache;        /* [1, 3, capacity, 64] */
    int64_t* position;         /* [1] */
    void* workspace;           /* exchange arena (uncached device memory) */
    float* query;              /* NULL */
    float* attention;          /* NULL */
    float* residual;           /* NULL */
    float* swiglu;             /* NULL */
    float* attention_partials; /* NULL */
    int64_t capacity;
    int64_t workspace_bytes;
} flux_layer_decode_buffers;

int flux_layer_decode_create(const flux_layer_weights* weights, const float* rope_cos, const float* rope_sin,
                             int64_t capacity, int64_t position, const float* initial_hidden, const float* key_source,
                             const float* value_source, int64_t source_length, double epsilon,
                             double attention_scale, hipStream_t stream, flux_layer_decode** out);
/* One step; returns the output buffer.  hidden (or NULL: the last input again) is read by
 * the step itself, in stream order, and kept as input_hidden; it must hold its value until
 * the step has run.  (native_decode_runtime_cuda.cu:456-481) */
int flux_layer_decode_replay(flux_layer_decode* runtime, const float* hidden, hipStream_t stream, float** output);
/* Synchronously restore hidden, cache and position.  (native_decode_runtime_cuda.cu:483-501) */
int flux_layer_decode_reset(flux_layer_decode* runtime, const float* hidden, const float* key_source,
                            const float* value_source, int64_t source_length, int64_t position, hipStream_t stream);
int flux_layer_decode_position(flux_layer_decode* runtime, int64_t* out);
int flux_layer_decode_replay_count(const flux_layer_decode* runtime, int64_t* out);
int flux_layer_decode_capacity(const flux_layer_decode* runtime, int64_t* out);
int flux_layer_decode_get_buffers(const flux_layer_decode* runtime, flux_layer_decode_buffers* out);
/* Kernel launches and all device commands (launches, cross-stream event waits) that replay()
 * has issued since creation: one launch per step.  Replaces the graph-node audit of the
 * reference's captured step (native_decode_runtime_cuda.cu:456-481). */
int flux_layer_decode_replay_launches(const flux_layer_decode* runtime, int64_t* kernel_launches,
                                     int64_t* device_commands);
void flux_layer_decode_destroy(flux_layer_decode* runtime);

/* ------------------------------------------------------------------------ */
/* Per-kernel launchers (isolated kernels of the token loop). */

/* rows x cols RMSNorm: out = w * (x * rsqrt(mean(x^2) + eps)), eps > 0 and finite, cols <= 65536.
 * Replaces rmsnorm_cuda_fp32 (csrc/rmsnorm/rmsnorm_cuda.h:9-19). */
int flux_rmsnorm_f32(const float* x, const float* weight, float* out, int64_t rows, int64_t cols, float eps,
                     hipStream_t stream);

/* residual_out = hidden + residual; norm_out = rmsnorm(residual_out); eps >= 0 and finite.
 * Replaces residual_rmsnorm_cuda_fp32 (csrc/residual_rmsnorm/residual_rmsnorm_cuda.cu:108-150). */
int flux_residual_rmsnorm_f32(const float* hidden, const float* residual, const float* weight, float* norm_out,
                              float* residual_out, int64_t rows, int64_t cols, float eps, hipStream_t stream);

/* Decode QKV step fused: rmsnorm(hidden) -> packed QKV GEMV [960,576] -> RoPE at
 * *position -> q_out [9,64]; K/V written to key/value cache [3, capacity, 64] row
 * *position.  Replaces the cuBLASLt QKV GEMV (native_decode_runtime_cuda.cu:213-218)
 * plus packed_qkv_rope_cache_at_position_cuda_fp32 (packed_qkv_rope_cache_cuda.cu:153-179). */
int flux_qkv_rope_cache_f32(const float* hidden, const float* norm_weight, float eps, const float* packed_qkv,
                            const float* rope_cos, const float* rope_sin, const int64_t* position, int64_t capacity,
                            float* key_cache, float* value_cache, float* q_out, hipStream_t stream);

/* One-token GQA attention over compact K/V [3, capacity, 64] for positions
 * [0, *position] with split-K partials in `workspace`.
 * Replaces gqa_decode_attention_cuda_fp32 (csrc/gqa_decode_attention/gqa_decode_attention_cuda.cu:551-633). */
int flux_gqa_decode_workspace_bytes(int64_t capacity, int64_t* bytes);
int flux_gqa_decode_attention_f32(const float* q, const float* key_cache, const float* value_cache,
                                  const int64_t* position, int64_t capacity, float scale, void* workspace,
                                  int64_t workspace_bytes, float* out, hipStream_t stream);

/* flux_gqa_decode_attention_f32 without a workspace argument: the split-K partials
 * go to a fixed scratch array inside the library (201,960 bytes per GPU, held until
 * the process ends), so the call allocates nothing -- for callers that cannot
 * allocate (code under hipGraph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  capacity must be in [1, FLUX_MAX_CAPACITY]; larger capacities are
 * rejected with FLUX_ERROR_INVALID_VALUE.  Every call on one GPU shares that GPU's
 * scratch: calls that overlap on one GPU (e.g. on two streams) race.  Results are
 * bit-identical to flux_gqa_decode_attention_f32 (same kernels).
 * No counterpart in the reference; added for callers that cannot allocate. */
int flux_gqa_decode_attention_noalloc_f32(const float* q, const float* key_cache, const float* value_cache,
                                          const int64_t* position, int64_t capacity, float scale, float* out,
                                          hipStream_t stream);

/* out[rows] = W[rows, 576] x[576] (+ residual[rows] if non-NULL).
 * Replaces the cuBLASLt o_proj GEMV (native_decode_runtime_cuda.cu:271-276) and
 * residual add. */
int flux_linear576_f32(const float* x, const float* weight, const float* residual, float* out, int64_t rows,
                       hipStream_t stream);

/* out[1536] = silu(Wg x) * (Wu x), x = rmsnorm(hidden) when norm_weight != NULL.
 * Replaces packed_gate_up_swiglu_cuda_fp32 (csrc/packed_gate_up_gemv/packed_gate_up_gemv_cuda.cu:25-63). */
int flux_gate_up_swiglu_f32(const float* hidden, const float* norm_weight, float eps, const float* packed_gate_up,
                            float* out, hipStream_t stream);

/* out[576] = residual + W_down[576,1536] s.  Replaces cublasSgemm + cublasSgeam
 * (native_decode_runtime_cuda.cu:290-309). */
int flux_down_residual_f32(const float* s, const float* down, const float* residual, float* out, hipStream_t stream);

/* logits = lm_head x (x = rmsnorm(hidden) when norm_weight != NULL) and the
 * exact lowest-index argmax into *token.  Replaces the lm_head cublasSgemm
 * (native_decode_runtime_cuda.cu:1078-1087) + greedy_argmax_cuda_fp32. */
int flux_lm_head_workspace_bytes(int64_t* bytes);
int flux_lm_head_argmax_f32(const float* hidden, const float* norm_weight, float eps, const float* lm_head,
                            int64_t vocab, float* logits, int64_t* token, void* workspace, int64_t workspace_bytes,
                            hipStream_t stream);

/* Greedy argmax (greedy_generation_cuda.cu:99-132): lowest index of the
 * maximum, NaN counts as maximum.  The _update form also writes
 * generated[*step] = token, *step += 1, *position = *attention_length. */
int flux_greedy_argmax_f32(const float* logits, int64_t vocab, int64_t* token, hipStream_t stream);
int flux_greedy_argmax_update_f32(const float* logits, int64_t vocab, int64_t* input_token, int64_t* generated_tokens,
                                  int64_t* generation_step, int64_t generated_capacity, int64_t* position,
                                  const int64_t* attention_length, hipStream_t stream);

/* Prefill linear on FP32 MFMA: C[m,n] = A[m,k] W[n,k]^T (+ residual[m,n]).
 * Replaces linear_fp32 / cublasSgemm (native_prefill_runtime_cuda.cu:285-302).
 * n % 64 == 0, k % 16 == 0. */
int flux_linear_f32(const float* a, const float* weight, const float* residual, float* c, int64_t m, int64_t n,
                    int64_t k, hipStream_t stream);

/* Prefill gate/up GEMM with SwiGLU epilogue: out[m,1536] = silu(x Wg^T) * (x Wu^T).
 * Replaces linear_fp32 + packed_swiglu_cuda_fp32 (csrc/packed_swiglu/packed_swiglu_cuda.cu:35-56). */
int flux_gate_up_swiglu_rows_f32(const float* x, const float* packed_gate_up, float* out, int64_t rows,
                                 hipStream_t stream);

/* Prefill QKV GEMM with RoPE epilogue for positions 0..rows-1: q_out [9,rows,64],
 * K/V cache rows [3, capacity, 64].  Replaces linear_fp32 +
 * packed_qkv_rope_cache_prefill_fp32_kernel (native_prefill_runtime_cuda.cu:124-163). */
int flux_qkv_rope_cache_rows_f32(const float* x, const float* packed_qkv, const float* rope_cos, const float* rope_sin,
                                 int64_t rows, float* q_out, float* key_cache, float* value_cache, int64_t capacity,
                                 hipStream_t stream);

/* Workspace (bytes) flux_prefill_attention_f32 needs for a prompt of `seq` tokens: the
 * split-key partials of the 128-query tiles that see more than one key chunk (chunks of
 * 128 to 1024 keys, longer for longer prompts); 0 for seq <= 128.  Counterpart of the
 * reference's partition workspace size (test_streaming_prefill_gqa.cu:503-512). */
int flux_prefill_attention_workspace_bytes(int64_t seq, int64_t* bytes);

/* Causal GQA prefill attention (FP32 MFMA, online softmax, keys split in chunks of
 * 128 to 1024 and merged): q [9,seq,64], K/V [3,capacity,64] -> out_rows [seq, 576].
 * `workspace` may be NULL when flux_prefill_attention_workspace_bytes reports 0.
 * Every pointer must be 16-byte aligned.
 * Replaces streaming_prefill_gqa_cuda_fp32 (csrc/streaming_prefill_gqa/
 * streaming_prefill_gqa_cuda.cu:423-460) + K15. */
int flux_prefill_attention_f32(const float* q, const float* key_cache, const float* value_cache, int64_t seq,
                               int64_t capacity, float scale, float* workspace, float* out_rows, hipStream_t stream);

/* hidden[s] = embedding[ids[s]] (zero row when out of vocabulary).
 * Replaces embedding_gather_fp32_kernel (native_prefill_runtime_cuda.cu:85-103). */
int flux_embedding_gather_f32(const int64_t* ids, const float* embedding, int64_t vocab, int64_t seq, float* hidden,
                              hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* Eager operator kernels behind torch.ops.flux.* (general shapes; element
 * strides are int64 arrays in tensor dimension order, all non-negative). */

/* HF RoPE of query [B,Hq,S,D] and key [B,Hk,S,D] (strided) with cos/sin
 * [rope_batch,S,D] (rope_batch 1 or B) into contiguous outputs; the two products
 * are rounded separately before the add.  Replaces rope_cuda_fp32
 * (csrc/rope/rope_cuda.cu:89-130; op schema csrc/rope/rope_torch.cpp:133-136). */
int flux_rope_f32(const float* query, const float* key, const float* cos, const float* sin, float* query_out,
                  float* key_out, int64_t batch, int64_t query_heads, int64_t key_heads, int64_t seq,
                  int64_t head_dim, int64_t rope_batch, const int64_t* query_strides, const int64_t* key_strides,
                  const int64_t* cos_strides, const int64_t* sin_strides, hipStream_t stream);

/* Softmax over each contiguous row of `width` values.
 * Replaces softmax_cuda_fp32 (csrc/softmax/softmax_cuda.cu:353-365). */
int flux_softmax_f32(const float* input, float* output, int64_t rows, int64_t width, hipStream_t stream);

/* softmax(fl(scores * scale) + mask) over contiguous scores [B,H,Q,K]; the mask
 * has sizes 1 or the scores' size per dimension and any non-negative strides.
 * Replaces attention_score_softmax_cuda_fp32 (csrc/softmax/softmax_cuda.cu:367-412). */
int flux_attention_score_softmax_f32(const float* scores, const float* mask, float* output, float scale,
                                     int64_t batch, int64_t heads, int64_t query_length, int64_t key_length,
                                     const int64_t* mask_sizes, const int64_t* mask_strides, hipStream_t stream);

/* out[r, i] = silu(packed[r, i]) * packed[r, I + i] for contiguous packed [rows, 2I].
 * Replaces packed_swiglu_cuda_fp32 (csrc/packed_swiglu/packed_swiglu_cuda.cu:35-56). */
int flux_packed_swiglu_f32(const float* packed, float* output, int64_t rows, int64_t intermediate,
                           hipStream_t stream);

/* One-token packed QKV [960] -> RoPE(q) into query_out [9,64]; RoPE(k) and v
 * written to row *position of key/value caches [1,3,capacity,64]; nothing is
 * written when *position is outside [0, capacity).  When cache_length is
 * non-NULL it receives *position + 1 (it may alias position).
 * Replaces packed_qkv_rope_cache_cuda_fp32 and
 * packed_qkv_rope_cache_at_position_cuda_fp32
 * (csrc/packed_qkv_rope_cache/packed_qkv_rope_cache_cuda.cu:125-179). */
int flux_packed_qkv_rope_cache_f32(const float* packed_qkv, const float* cos, const float* sin, float* key_cache,
                                   float* value_cache, const int64_t* position, int64_t* cache_length,
                                   float* query_out, int64_t capacity, int64_t packed_stride, int64_t cos_stride,
                                   int64_t sin_stride, const int64_t* key_strides, const int64_t* value_strides,
                                   hipStream_t stream);

/* One-token GQA attention of query [1,Hq,1,D] over strided caches [1,Hkv,capacity,D]
 * for the first clamp(*cache_length, 1, capacity) positions (all when
 * cache_length is NULL), with an optional additive mask broadcast from
 * [1|1, 1|Hq, 1, 1|capacity]; output [1,Hq,1,D] contiguous.  Split-key partials
 * go to `workspace` (size from the _workspace_bytes query; 0 when one chunk covers the capacity: 128 keys
 * for head_dim 64, 256 otherwise).
 * Replaces gqa_decode_attention_cuda_fp32
 * (csrc/gqa_decode_attention/gqa_decode_attention_cuda.cu:551-633). */
int flux_gqa_decode_attention_strided_workspace_bytes(int64_t query_heads, int64_t capacity, int64_t head_dim,
                                                      int64_t* bytes);
int flux_gqa_decode_attention_strided_f32(const float* query, const float* key_cache, const float* value_cache,
                                          const float* mask, const int64_t* cache_length, float* output,
                                          void* workspace, int64_t workspace_bytes, float scale, int64_t query_heads,
                                          int64_t kv_heads, int64_t capacity, int64_t head_dim,
                                          const int64_t* query_strides, const int64_t* key_strides,
                                          const int64_t* value_strides, const int64_t* mask_sizes,
                                          const int64_t* mask_strides, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FLUX_AMD_H_ */
