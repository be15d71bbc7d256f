// Internal launcher interface between the C++ runtime and the gfx950 kernels.
#pragma once

#include "flux_common.h"

#include <cstddef>
#include <cstdint>

namespace flux {

// Upper bound on attention chunks per KV head in the fused kernel (grid <= 384).
constexpr int kMaxAttnChunks = 128;

struct DecodeArgs {
    const LayerWeights* layers;  // device array [kLayers]
    const float* embedding;      // [vocab, 576]
    const float* lm_head;        // [vocab, 576]
    const float* final_norm;     // [576]
    float final_eps;
    const float* rope_cos;       // [capacity, 64]
    const float* rope_sin;
    float* key_cache;            // [30, 3, capacity, 64]
    float* value_cache;
    float* logits;               // [vocab]
    int64_t* input_token;
    int64_t* generated;          // [generated_capacity]
    int64_t* generation_step;
    int64_t* position;
    int64_t* cache_length;
    uint64_t* ll;                // LL arena (ll_arena_words())
    uint32_t* token_counter;
    int32_t* error;              // device error word (0 = none)
    int32_t* host_error;         // host-visible copy of the error word (mapped pinned memory)
    uint64_t wait_ticks;         // bound of every cross-workgroup wait (100 MHz wall clock)
    int64_t capacity;
    int64_t vocab;
    int64_t generated_capacity;
    int steps;
    // When set, the launch's first step reads its input token here instead of from
    // input_token (replay(token): the caller's token, read in stream order, no copy).
    const int64_t* token_in;
    // Layers per step: kLayers, or 1 for the single-layer step of NativeSmolLM2LayerDecode
    // (layers then holds that layer only, and the caches are its [3, capacity, 64]).
    int layer_count;
    // Single-layer step (hidden_out set): the step starts from hidden_in instead of the
    // token's embedding row (workgroup 0 copies it to hidden_save when that is set), writes
    // the last layer's output to hidden_out and advances *position and *cache_length by
    // one; no LM head, no argmax, no generation bookkeeping.
    const float* hidden_in;
    float* hidden_save;
    float* hidden_out;
};

// ---- fused decode ----
size_t ll_arena_words();
int fused_decode_threads();
size_t fused_decode_dynamic_lds();
int max_attention_positions(int grid);
hipError_t fused_decode_occupancy(int* blocks_per_cu);
// cooperative = false launches it plainly (profiling: rocprofv3 7.2 crashes at exit after
// cooperative launches); the occupancy check and the bounded waits remain the guard.
hipError_t launch_fused_decode(const DecodeArgs& args, int grid, hipStream_t stream, bool cooperative = true);
void* fused_decode_function();

// ---- isolated decode phases ----
hipError_t launch_qkv_rope_cache(const float* hidden, const float* norm_w, float eps, const float* qkv_w,
                                 const float* cos_table, const float* sin_table, const int64_t* position,
                                 int64_t capacity, float* key_cache, float* value_cache, float* q_out, int grid,
                                 hipStream_t stream);
hipError_t launch_gqa_decode(const float* q, const float* key_cache, const float* value_cache, const int64_t* position,
                             int64_t capacity, float scale, int chunks, float* partials, float* out,
                             hipStream_t stream);
int gqa_decode_max_positions(int chunks);
// launch_gqa_decode with the partials in the library's per-device scratch array
// (chunks <= gqa_decode_noalloc_max_chunks()); allocates nothing.
hipError_t launch_gqa_decode_noalloc(const float* q, const float* key_cache, const float* value_cache,
                                     const int64_t* position, int64_t capacity, float scale, int chunks, float* out,
                                     hipStream_t stream);
int gqa_decode_noalloc_max_chunks();
hipError_t launch_linear576_residual(const float* x, const float* w, const float* residual, float* out, int rows,
                                     int grid, hipStream_t stream);
hipError_t launch_gate_up_swiglu(const float* hidden, const float* norm_w, float eps, const float* gate_up, float* out,
                                 int grid, hipStream_t stream);
hipError_t launch_down_residual(const float* s, const float* w, const float* residual, float* out, int grid,
                                hipStream_t stream);
hipError_t launch_lm_head_argmax(const float* hidden, const float* norm_w, float eps, const float* lm_head,
                                 int64_t vocab, float* logits, float* part_v, int64_t* part_i, int grid,
                                 int64_t* token, hipStream_t stream);
hipError_t launch_argmax(const float* logits, int64_t n, int64_t* token, int64_t* generated, int64_t* step,
                         int64_t generated_capacity, int64_t* position, const int64_t* attention_length,
                         hipStream_t stream);
hipError_t launch_install_state(const int64_t* token_src, int64_t position_value, int64_t step_value,
                                bool write_generated0, int64_t* input_token, int64_t* position, int64_t* cache_length,
                                int64_t* step, int64_t* generated, int32_t* error, int32_t* host_error,
                                hipStream_t stream);
hipError_t launch_rmsnorm_rows(const float* x, const float* w, float* out, int64_t rows, int cols, float eps,
                               hipStream_t stream);
hipError_t launch_residual_rmsnorm_rows(const float* hidden, const float* residual, const float* w, float* norm_out,
                                        float* residual_out, int64_t rows, int cols, float eps, hipStream_t stream);

// ---- prefill ----
enum class GemmEpilogue : int {
    kStore = 0,         // C = A B^T
    kResidual = 1,      // C = R + A B^T
    kSwiglu = 2,        // gate/up interleaved tiles -> silu(g) * u into [M, N/2]
    kQkvRope = 3,       // RoPE + head-major q + compact K/V cache rows
};

struct GemmArgs {
    const float* a;     // [M, K] row-major
    const float* b;     // [N, K] row-major (weights)
    float* c;           // output (layout by epilogue)
    const float* residual;
    int64_t m;
    int n;
    int k;
    // kQkvRope
    const float* rope_cos;  // [capacity, 64] (row = position)
    const float* rope_sin;
    float* q_out;           // [9, M, 64]
    float* key_cache;       // [3, capacity, 64]
    float* value_cache;
    int64_t capacity;
    // Optional RMSNorm folded into the GEMM (only gemm_split_kernel takes it): A holds the
    // raw rows, each K value is scaled by norm_weight[k] and each output row by the inverse
    // RMS of its A row.  launch_gemm rejects a norm it cannot fold; launch_norm_gemm folds it
    // where it can and otherwise runs the RMSNorm kernel first.
    const float* norm_weight;
    float norm_eps;
    // Optional workspace (split_partials_floats(M, N) floats) that lets launch_gemm split K
    // over kSplitBlocksK (or, for the 576-column kernel, two) blocks when the grid leaves CUs
    // idle: one partial plane [M, N] per K part, then kSplitBlocksK partial row sums of
    // squares [M] (folded norm), summed in order by a second kernel that applies the
    // epilogue.  Null: every block covers all of K.
    float* split_partials;
    int64_t split_floats;  // floats available at split_partials: no split whose planes exceed it
    // Optional A given unreduced (QKV with the folded norm on gemm_reg_kernel only, see
    // gemm_sums_planes): A = a_residual + (plane 0 + plane 1 + plane 2) of the kSplitBlocksK
    // planes [M, K] at a_planes that launch_gemm_planes left, summed in the order of the reduce
    // kernel, so A is bitwise the rows that reduce would have written.  The blocks of the first
    // column tile also write those rows to a_rows_out.  args.a is then not read.
    const float* a_planes;
    const float* a_residual;
    float* a_rows_out;
};

// Blocks that share one output tile's K range when GemmArgs::split_partials is given.
constexpr int kSplitBlocksK = 3;
// Prompt lengths up to which the prefill runtime provides the partial planes (longer
// prompts fill the device without splitting K): for the widest GEMM (gate/up) up to
// kSplitKMaxRows rows, for the 576-column GEMMs up to kNarrowSplitMaxRows.
constexpr int64_t kSplitKMaxRows = 1024;
constexpr int64_t kNarrowSplitMaxRows = 16384;
// Floats of GemmArgs::split_partials for an [M, N] GEMM.
__host__ __device__ constexpr int64_t split_partials_floats(int64_t m, int64_t n) {
    return kSplitBlocksK * m * n + kSplitBlocksK * m;
}

hipError_t launch_gemm(const GemmArgs& args, GemmEpilogue epilogue, hipStream_t stream);
// epilogue(rmsnorm(A) * W^T): args.a holds the raw rows; `scratch` ([M, K]) receives the
// normalized rows when the norm cannot be folded into the GEMM.
hipError_t launch_norm_gemm(const GemmArgs& args, const float* norm_weight, float eps, float* scratch,
                            GemmEpilogue epilogue, hipStream_t stream);
// True when launch_norm_gemm folds the RMSNorm into this GEMM (no separate norm launch).
bool gemm_folds_norm(const GemmArgs& args, GemmEpilogue epilogue);
// True when launch_gemm splits K over kSplitBlocksK blocks for these args (partial planes in
// args.split_partials, then a reduce kernel).
bool gemm_writes_planes(const GemmArgs& args, GemmEpilogue epilogue);
// The split kernel alone for args where gemm_writes_planes holds: the kSplitBlocksK partial
// planes are left in args.split_partials unreduced (args.c and args.residual are not touched)
// for a GEMM that sums them into its A rows.
hipError_t launch_gemm_planes(const GemmArgs& args, GemmEpilogue epilogue, hipStream_t stream);
// True when launch_gemm takes GemmArgs::a_planes for this GEMM (shape and epilogue; the folded
// norm must be given too).
bool gemm_sums_planes(const GemmArgs& args, GemmEpilogue epilogue);
// c = residual + A·Wᵀ (args with the residual epilogue) and norm_out = rmsnorm(c) with the
// given weights: the norm that the next GEMM needs when it does not fold it.  A K-split
// 576-column GEMM reduces its partial planes inside the norm kernel.
hipError_t launch_gemm_residual_norm(const GemmArgs& args, const float* norm_weight, float eps, float* norm_out,
                                     hipStream_t stream);

// Workspace (floats) of launch_prefill_attention for a prompt of `seq` tokens (0 when
// every query tile fits in one key chunk).
size_t prefill_attention_workspace_floats(int64_t seq);
hipError_t launch_prefill_attention(const float* q, const float* key_cache, const float* value_cache, int64_t seq,
                                    int64_t capacity, float scale, float* workspace, float* out_rows,
                                    hipStream_t stream);

hipError_t launch_embedding_gather(const int64_t* ids, const float* embedding, int64_t vocab, int64_t seq,
                                   float* hidden, hipStream_t stream);

// ---- eager operators (torch.ops.flux.*) ----
struct RopeShape {
    int64_t batch;
    int64_t query_heads;
    int64_t key_heads;
    int64_t seq;
    int64_t head_dim;
    int64_t rope_batch;         // 1 (broadcast) or batch
    int64_t query_strides[4];   // [B, H, S, D] element strides
    int64_t key_strides[4];
    int64_t cos_strides[3];     // [B, S, D]
    int64_t sin_strides[3];
};
hipError_t launch_rope(const float* query, const float* key, const float* cos_table, const float* sin_table,
                       float* query_out, float* key_out, const RopeShape& shape, hipStream_t stream);

hipError_t launch_softmax(const float* input, float* output, int64_t rows, int64_t width, hipStream_t stream);
// mask_strides: element strides of the mask over [B, H, Q, K], 0 on broadcast dimensions.
hipError_t launch_attention_score_softmax(const float* scores, const float* mask, float* output, float scale,
                                          int64_t batch, int64_t heads, int64_t query_length, int64_t key_length,
                                          const int64_t mask_strides[4], hipStream_t stream);
hipError_t launch_packed_swiglu(const float* packed, float* out, int64_t rows, int64_t inter, hipStream_t stream);

struct PackedQkvArgs {
    const float* packed;      // [960], element stride packed_stride
    const float* cos;         // [64], element stride cos_stride
    const float* sin;
    float* key_cache;         // [1, 3, capacity, 64] with key_strides
    float* value_cache;
    const int64_t* position;  // cache row to write
    int64_t* cache_length;    // NULL or receives position + 1
    float* query_out;         // [9, 64] contiguous
    int64_t capacity;
    int64_t packed_stride;
    int64_t cos_stride;
    int64_t sin_stride;
    int64_t key_strides[4];
    int64_t value_strides[4];
};
hipError_t launch_packed_qkv_rope_cache(const PackedQkvArgs& args, hipStream_t stream);

struct GqaStridedArgs {
    const float* q;                // [1, Hq, 1, D] with q_strides
    const float* k;                // [1, Hkv, capacity, D] with k_strides
    const float* v;
    const float* mask;             // NULL or broadcast [1|1, 1|Hq, 1, 1|capacity]
    const int64_t* cache_length;   // NULL (= capacity) or device scalar, clamped to [1, capacity]
    float* out;                    // [Hq, D] contiguous
    float* workspace;              // gqa_strided_workspace_floats() floats (unused for one chunk)
    float scale;
    int query_heads;
    int groups;                    // Hq / Hkv
    int dim;
    int chunks;                    // gqa_strided_chunks(capacity, dim)
    int vec;                       // K and V rows contiguous, 16-byte aligned, dim % 4 == 0
    int64_t capacity;
    int64_t q_strides[4];
    int64_t k_strides[4];
    int64_t v_strides[4];
    int64_t mask_strides[4];       // 0 on broadcast dimensions
};
int gqa_strided_chunks(int64_t capacity, int64_t head_dim);  // 128-key chunks for head_dim 64, else 256
size_t gqa_strided_workspace_floats(int64_t query_heads, int64_t capacity, int64_t head_dim);
hipError_t launch_gqa_strided(const GqaStridedArgs& args, hipStream_t stream);

}  // namespace flux
