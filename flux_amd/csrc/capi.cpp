// extern "C" boundary of libflux_amd.so.  Declarations and the reference
// interface each entry point replaces: include/flux_amd.h.
#include "../../include/flux_amd.h"

#include "flux_kernels.h"
#include "runtime.h"

#include <cmath>
#include <cstdint>
#include <new>
#include <string>

struct flux_decode {
    flux::DecodeRuntime* impl;
    bool owned;
};

struct flux_prefill {
    flux::PrefillRuntime* impl;
    flux_decode decode_handle;
};

struct flux_layer_decode {
    flux::LayerDecodeRuntime* impl;
};

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& message) {
    g_last_error = message;
    return code;
}

template <class F>
int guarded(F&& body) {
    try {
        body();
        g_last_error.clear();
        return FLUX_OK;
    } catch (const flux::FluxError& e) {
        return fail(e.code, e.what());
    } catch (const std::bad_alloc&) {
        return fail(FLUX_ERROR_HIP, "flux: host allocation failed");
    } catch (const std::exception& e) {
        return fail(FLUX_ERROR_HIP, e.what());
    }
}

int from_hip(hipError_t status, const char* what) {
    if (status == hipSuccess) return FLUX_OK;
    return fail(status == hipErrorInvalidValue ? FLUX_ERROR_INVALID_VALUE : FLUX_ERROR_HIP,
                std::string(what) + ": " + hipGetErrorString(status));
}

int invalid(const char* message) { return fail(FLUX_ERROR_INVALID_VALUE, message); }
int invalid(const std::string& message) { return fail(FLUX_ERROR_INVALID_VALUE, message); }

int isolated_grid() {
    int cus = 0;
    try {
        cus = flux::device_cu_count();
    } catch (...) {
        cus = 256;
    }
    return cus > 0 ? cus : 256;
}

// Attention split of the isolated decode-attention launcher (independent of the
// fused kernel): enough chunks to cover `capacity` positions.
int isolated_chunks(int64_t capacity) { return flux::isolated_attention_chunks(capacity); }

}  // namespace

extern "C" {

const char* flux_last_error(void) { return g_last_error.c_str(); }

const char* flux_version(void) { return "flux_amd 0.1 gfx950"; }

// ---------------------------------------------------------------------------
int flux_decode_create(const flux_weights* weights, const float* rope_cos, const float* rope_sin, int64_t capacity,
                       int64_t position, const int64_t* initial_token, const float* const* key_sources,
                       const float* const* value_sources, const int64_t* source_lengths, const double* epsilons,
                       const double* attention_scales, hipStream_t stream, flux_decode** out) {
    if (weights == nullptr || out == nullptr) return invalid("flux_decode_create: null argument");
    *out = nullptr;
    return guarded([&] {
        flux::CacheSources sources{key_sources, value_sources, source_lengths};
        auto* impl = new flux::DecodeRuntime(*weights, rope_cos, rope_sin, capacity, position, initial_token, sources,
                                             epsilons, attention_scales, stream);
        *out = new flux_decode{impl, true};
    });
}

int flux_decode_replay(flux_decode* runtime, const int64_t* token, hipStream_t stream, float** logits) {
    if (runtime == nullptr) return invalid("flux_decode_replay: null runtime");
    return guarded([&] {
        float* result = runtime->impl->replay(token, stream);
        if (logits) *logits = result;
    });
}

int flux_decode_generate_greedy(flux_decode* runtime, int64_t decode_steps, hipStream_t stream,
                                int64_t** generated_tokens) {
    if (runtime == nullptr) return invalid("flux_decode_generate_greedy: null runtime");
    return guarded([&] {
        int64_t* result = runtime->impl->generate_greedy(decode_steps, stream);
        if (generated_tokens) *generated_tokens = result;
    });
}

int flux_decode_generate_greedy_timed(flux_decode* runtime, int64_t decode_steps, hipStream_t stream,
                                      float* milliseconds) {
    if (runtime == nullptr || milliseconds == nullptr) return invalid("flux_decode_generate_greedy_timed: null argument");
    return guarded([&] { runtime->impl->generate_greedy(decode_steps, stream, milliseconds); });
}

int flux_decode_reset(flux_decode* runtime, const int64_t* token, const float* const* key_sources,
                      const float* const* value_sources, const int64_t* source_lengths, int64_t position,
                      hipStream_t stream) {
    if (runtime == nullptr) return invalid("flux_decode_reset: null runtime");
    return guarded([&] {
        runtime->impl->reset(token, flux::CacheSources{key_sources, value_sources, source_lengths}, position, stream);
    });
}

int flux_decode_position(flux_decode* runtime, int64_t* out) {
    if (runtime == nullptr || out == nullptr) return invalid("flux_decode_position: null argument");
    return guarded([&] { *out = runtime->impl->position(); });
}

int flux_decode_cache_length(flux_decode* runtime, int64_t* out) {
    if (runtime == nullptr || out == nullptr) return invalid("flux_decode_cache_length: null argument");
    return guarded([&] { *out = runtime->impl->cache_length(); });
}

int flux_decode_generation_step(flux_decode* runtime, int64_t* out) {
    if (runtime == nullptr || out == nullptr) return invalid("flux_decode_generation_step: null argument");
    return guarded([&] { *out = runtime->impl->generation_step(); });
}

int flux_decode_replay_count(const flux_decode* runtime, int64_t* out) {
    if (runtime == nullptr || out == nullptr) return invalid("flux_decode_replay_count: null argument");
    *out = runtime->impl->replay_count();
    return FLUX_OK;
}

int flux_decode_capacity(const flux_decode* runtime, int64_t* out) {
    if (runtime == nullptr || out == nullptr) return invalid("flux_decode_capacity: null argument");
    *out = runtime->impl->capacity();
    return FLUX_OK;
}

int flux_decode_get_buffers(const flux_decode* runtime, flux_decode_buffers* out) {
    if (runtime == nullptr || out == nullptr) return invalid("flux_decode_get_buffers: null argument");
    runtime->impl->buffers(out);
    return FLUX_OK;
}

int flux_decode_device_error(flux_decode* runtime, int32_t* out) {
    if (runtime == nullptr || out == nullptr) return invalid("flux_decode_device_error: null argument");
    return guarded([&] { *out = runtime->impl->device_error(); });
}

int flux_decode_set_wait_limit(flux_decode* runtime, uint64_t ticks) {
    if (runtime == nullptr) return invalid("flux_decode_set_wait_limit: null argument");
    if (ticks > FLUX_MAX_WAIT_TICKS)
        return invalid("flux_decode_set_wait_limit: bound exceeds FLUX_MAX_WAIT_TICKS (1e9 ticks = 10 s)");
    runtime->impl->set_wait_limit(ticks);
    return FLUX_OK;
}


void flux_decode_destroy(flux_decode* runtime) {
    if (runtime == nullptr || !runtime->owned) return;
    delete runtime->impl;
    delete runtime;
}

// ---------------------------------------------------------------------------
int flux_prefill_create(const flux_weights* weights, const float* rope_cos, const float* rope_sin, int64_t capacity,
                        const int64_t* input_ids, int64_t sequence_length, const double* epsilons,
                        const double* attention_scales, hipStream_t stream, flux_prefill** out) {
    if (weights == nullptr || out == nullptr) return invalid("flux_prefill_create: null argument");
    *out = nullptr;
    return guarded([&] {
        auto* impl = new flux::PrefillRuntime(*weights, rope_cos, rope_sin, capacity, input_ids, sequence_length,
                                              epsilons, attention_scales, stream);
        *out = new flux_prefill{impl, flux_decode{impl->decode(), false}};
    });
}

int flux_prefill_run(flux_prefill* runtime, const int64_t* input_ids, hipStream_t stream, float** logits) {
    if (runtime == nullptr) return invalid("flux_prefill_run: null runtime");
    return guarded([&] {
        float* result = runtime->impl->prefill(input_ids, stream);
        if (logits) *logits = result;
    });
}

int flux_prefill_generate_greedy(flux_prefill* runtime, int64_t max_new_tokens, hipStream_t stream,
                                 int64_t** generated_tokens) {
    if (runtime == nullptr) return invalid("flux_prefill_generate_greedy: null runtime");
    return guarded([&] {
        int64_t* result = runtime->impl->generate_greedy(max_new_tokens, stream);
        if (generated_tokens) *generated_tokens = result;
    });
}

flux_decode* flux_prefill_decode(flux_prefill* runtime) { return runtime ? &runtime->decode_handle : nullptr; }

int flux_prefill_get_buffers(const flux_prefill* runtime, flux_prefill_buffers* out) {
    if (runtime == nullptr || out == nullptr) return invalid("flux_prefill_get_buffers: null argument");
    runtime->impl->buffers(out);
    return FLUX_OK;
}

void flux_prefill_destroy(flux_prefill* runtime) {
    if (runtime == nullptr) return;
    delete runtime->impl;
    delete runtime;
}

// ---------------------------------------------------------------------------
int flux_rmsnorm_f32(const float* x, const float* weight, float* out, int64_t rows, int64_t cols, float eps,
                     hipStream_t stream) {
    if (!x || !weight || !out || rows <= 0 || cols <= 0 || cols > 65536 || !(eps > 0.0f) || !std::isfinite(eps))
        return invalid("flux_rmsnorm_f32: invalid argument");
    return from_hip(flux::launch_rmsnorm_rows(x, weight, out, rows, static_cast<int>(cols), eps, stream),
                    "flux_rmsnorm_f32");
}

int flux_residual_rmsnorm_f32(const float* hidden, const float* residual, const float* weight, float* norm_out,
                              float* residual_out, int64_t rows, int64_t cols, float eps, hipStream_t stream) {
    if (!hidden || !residual || !weight || !norm_out || !residual_out || rows <= 0 || cols <= 0 || cols > 65536 ||
        !(eps >= 0.0f) || !std::isfinite(eps))
        return invalid("flux_residual_rmsnorm_f32: invalid argument");
    return from_hip(flux::launch_residual_rmsnorm_rows(hidden, residual, weight, norm_out, residual_out, rows,
                                                       static_cast<int>(cols), eps, stream),
                    "flux_residual_rmsnorm_f32");
}

int flux_qkv_rope_cache_f32(const float* hidden, const float* norm_weight, float eps, const float* packed_qkv,
                            const float* rope_cos, const float* rope_sin, const int64_t* position, int64_t capacity,
                            float* key_cache, float* value_cache, float* q_out, hipStream_t stream) {
    if (!hidden || !norm_weight || !packed_qkv || !rope_cos || !rope_sin || !position || !key_cache || !value_cache ||
        !q_out || capacity <= 0 || capacity > FLUX_MAX_CAPACITY || !(eps > 0.0f))
        return invalid("flux_qkv_rope_cache_f32: invalid argument");
    return from_hip(flux::launch_qkv_rope_cache(hidden, norm_weight, eps, packed_qkv, rope_cos, rope_sin, position,
                                                capacity, key_cache, value_cache, q_out, isolated_grid(), stream),
                    "flux_qkv_rope_cache_f32");
}

int flux_gqa_decode_workspace_bytes(int64_t capacity, int64_t* bytes) {
    if (bytes == nullptr || capacity <= 0 || capacity > FLUX_MAX_CAPACITY)
        return invalid("flux_gqa_decode_workspace_bytes: invalid argument");
    *bytes = static_cast<int64_t>(isolated_chunks(capacity)) * FLUX_KV_HEADS * 3 * (FLUX_HEAD_DIM + 2) * 4;
    return FLUX_OK;
}

int flux_gqa_decode_attention_f32(const float* q, const float* key_cache, const float* value_cache,
                                  const int64_t* position, int64_t capacity, float scale, void* workspace,
                                  int64_t workspace_bytes, float* out, hipStream_t stream) {
    int64_t needed = 0;
    if (!q || !key_cache || !value_cache || !position || !workspace || !out ||
        flux_gqa_decode_workspace_bytes(capacity, &needed) != FLUX_OK || workspace_bytes < needed)
        return invalid("flux_gqa_decode_attention_f32: invalid argument or workspace too small");
    return from_hip(flux::launch_gqa_decode(q, key_cache, value_cache, position, capacity, scale,
                                            isolated_chunks(capacity), static_cast<float*>(workspace), out, stream),
                    "flux_gqa_decode_attention_f32");
}

int flux_gqa_decode_attention_noalloc_f32(const float* q, const float* key_cache, const float* value_cache,
                                          const int64_t* position, int64_t capacity, float scale, float* out,
                                          hipStream_t stream) {
    if (!q || !key_cache || !value_cache || !position || !out)
        return invalid("flux_gqa_decode_attention_noalloc_f32: null argument");
    if (capacity <= 0 || capacity > FLUX_MAX_CAPACITY)
        return invalid("flux_gqa_decode_attention_noalloc_f32: capacity " + std::to_string(capacity) +
                       " is outside [1, " + std::to_string(FLUX_MAX_CAPACITY) +
                       "], the most positions its fixed scratch array holds partials for");
    const int chunks = isolated_chunks(capacity);
    if (chunks > flux::gqa_decode_noalloc_max_chunks())
        return invalid("flux_gqa_decode_attention_noalloc_f32: capacity needs more partials than the scratch holds");
    return from_hip(flux::launch_gqa_decode_noalloc(q, key_cache, value_cache, position, capacity, scale, chunks, out,
                                                    stream),
                    "flux_gqa_decode_attention_noalloc_f32");
}

int flux_linear576_f32(const float* x, const float* weight, const float* residual, float* out, int64_t rows,
                       hipStream_t stream) {
    if (!x || !weight || !out || rows <= 0 || rows > (int64_t{1} << 30))
        return invalid("flux_linear576_f32: invalid argument");
    return from_hip(flux::launch_linear576_residual(x, weight, residual, out, static_cast<int>(rows), isolated_grid(),
                                                    stream),
                    "flux_linear576_f32");
}

int flux_gate_up_swiglu_f32(const float* hidden, const float* norm_weight, float eps, const float* packed_gate_up,
                            float* out, hipStream_t stream) {
    if (!hidden || !packed_gate_up || !out || (norm_weight && !(eps > 0.0f)))
        return invalid("flux_gate_up_swiglu_f32: invalid argument");
    return from_hip(flux::launch_gate_up_swiglu(hidden, norm_weight, eps, packed_gate_up, out, isolated_grid(), stream),
                    "flux_gate_up_swiglu_f32");
}

int flux_down_residual_f32(const float* s, const float* down, const float* residual, float* out, hipStream_t stream) {
    if (!s || !down || !out) return invalid("flux_down_residual_f32: invalid argument");
    return from_hip(flux::launch_down_residual(s, down, residual, out, isolated_grid(), stream),
                    "flux_down_residual_f32");
}

int flux_lm_head_workspace_bytes(int64_t* bytes) {
    if (bytes == nullptr) return invalid("flux_lm_head_workspace_bytes: null argument");
    *bytes = static_cast<int64_t>(isolated_grid()) * 16;
    return FLUX_OK;
}

int flux_lm_head_argmax_f32(const float* hidden, const float* norm_weight, float eps, const float* lm_head,
                            int64_t vocab, float* logits, int64_t* token, void* workspace, int64_t workspace_bytes,
                            hipStream_t stream) {
    const int grid = isolated_grid();
    if (!hidden || !lm_head || !logits || !token || !workspace || vocab <= 0 || workspace_bytes < grid * 16 ||
        (norm_weight && !(eps > 0.0f)))
        return invalid("flux_lm_head_argmax_f32: invalid argument or workspace too small");
    auto* part_i = static_cast<int64_t*>(workspace);
    auto* part_v = reinterpret_cast<float*>(part_i + grid);
    return from_hip(flux::launch_lm_head_argmax(hidden, norm_weight, eps, lm_head, vocab, logits, part_v, part_i, grid,
                                                token, stream),
                    "flux_lm_head_argmax_f32");
}

int flux_greedy_argmax_f32(const float* logits, int64_t vocab, int64_t* token, hipStream_t stream) {
    if (!logits || !token || vocab <= 0) return invalid("flux_greedy_argmax_f32: invalid argument");
    return from_hip(flux::launch_argmax(logits, vocab, token, nullptr, nullptr, 0, nullptr, nullptr, stream),
                    "flux_greedy_argmax_f32");
}

int flux_greedy_argmax_update_f32(const float* logits, int64_t vocab, int64_t* input_token, int64_t* generated_tokens,
                                  int64_t* generation_step, int64_t generated_capacity, int64_t* position,
                                  const int64_t* attention_length, hipStream_t stream) {
    if (!logits || !input_token || !generated_tokens || !generation_step || generated_capacity <= 0 || !position ||
        !attention_length || vocab <= 0)
        return invalid("flux_greedy_argmax_update_f32: invalid argument");
    return from_hip(flux::launch_argmax(logits, vocab, input_token, generated_tokens, generation_step,
                                        generated_capacity, position, attention_length, stream),
                    "flux_greedy_argmax_update_f32");
}

int flux_linear_f32(const float* a, const float* weight, const float* residual, float* c, int64_t m, int64_t n,
                    int64_t k, hipStream_t stream) {
    if (!a || !weight || !c || m <= 0 || n <= 0 || k <= 0 || n % 64 != 0 || k % 16 != 0 || n > (1 << 30) ||
        k > (1 << 30))
        return invalid("flux_linear_f32: invalid argument (n % 64 == 0 and k % 16 == 0 required)");
    flux::GemmArgs args{};
    args.a = a;
    args.b = weight;
    args.c = c;
    args.residual = residual;
    args.m = m;
    args.n = static_cast<int>(n);
    args.k = static_cast<int>(k);
    return from_hip(flux::launch_gemm(args, residual ? flux::GemmEpilogue::kResidual : flux::GemmEpilogue::kStore,
                                      stream),
                    "flux_linear_f32");
}

int flux_gate_up_swiglu_rows_f32(const float* x, const float* packed_gate_up, float* out, int64_t rows,
                                 hipStream_t stream) {
    if (!x || !packed_gate_up || !out || rows <= 0) return invalid("flux_gate_up_swiglu_rows_f32: invalid argument");
    flux::GemmArgs args{};
    args.a = x;
    args.b = packed_gate_up;
    args.c = out;
    args.m = rows;
    args.n = FLUX_PACKED_GATE_UP_WIDTH;
    args.k = FLUX_HIDDEN;
    return from_hip(flux::launch_gemm(args, flux::GemmEpilogue::kSwiglu, stream), "flux_gate_up_swiglu_rows_f32");
}

int flux_qkv_rope_cache_rows_f32(const float* x, const float* packed_qkv, const float* rope_cos, const float* rope_sin,
                                 int64_t rows, float* q_out, float* key_cache, float* value_cache, int64_t capacity,
                                 hipStream_t stream) {
    if (!x || !packed_qkv || !rope_cos || !rope_sin || !q_out || !key_cache || !value_cache || rows <= 0 ||
        rows > capacity || capacity > FLUX_MAX_CAPACITY)
        return invalid("flux_qkv_rope_cache_rows_f32: invalid argument");
    flux::GemmArgs args{};
    args.a = x;
    args.b = packed_qkv;
    args.m = rows;
    args.n = FLUX_PACKED_QKV_WIDTH;
    args.k = FLUX_HIDDEN;
    args.rope_cos = rope_cos;
    args.rope_sin = rope_sin;
    args.q_out = q_out;
    args.key_cache = key_cache;
    args.value_cache = value_cache;
    args.capacity = capacity;
    return from_hip(flux::launch_gemm(args, flux::GemmEpilogue::kQkvRope, stream), "flux_qkv_rope_cache_rows_f32");
}

int flux_prefill_attention_workspace_bytes(int64_t seq, int64_t* bytes) {
    if (!bytes || seq <= 0 || seq > FLUX_MAX_CAPACITY)
        return invalid("flux_prefill_attention_workspace_bytes: invalid argument");
    *bytes = static_cast<int64_t>(flux::prefill_attention_workspace_floats(seq) * sizeof(float));
    return FLUX_OK;
}

int flux_prefill_attention_f32(const float* q, const float* key_cache, const float* value_cache, int64_t seq,
                               int64_t capacity, float scale, float* workspace, float* out_rows, hipStream_t stream) {
    if (!q || !key_cache || !value_cache || !out_rows || seq <= 0 || seq > capacity || capacity > FLUX_MAX_CAPACITY)
        return invalid("flux_prefill_attention_f32: invalid argument");
    if (flux::prefill_attention_workspace_floats(seq) > 0 && !workspace)
        return invalid("flux_prefill_attention_f32: this prompt length needs a workspace "
                       "(flux_prefill_attention_workspace_bytes)");
    for (const void* p : {static_cast<const void*>(q), static_cast<const void*>(key_cache),
                          static_cast<const void*>(value_cache), static_cast<const void*>(out_rows),
                          static_cast<const void*>(workspace)})
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
            return invalid("flux_prefill_attention_f32: pointers must be 16-byte aligned");
    return from_hip(
        flux::launch_prefill_attention(q, key_cache, value_cache, seq, capacity, scale, workspace, out_rows, stream),
        "flux_prefill_attention_f32");
}

int flux_embedding_gather_f32(const int64_t* ids, const float* embedding, int64_t vocab, int64_t seq, float* hidden,
                              hipStream_t stream) {
    if (!ids || !embedding || !hidden || vocab <= 0 || seq <= 0)
        return invalid("flux_embedding_gather_f32: invalid argument");
    return from_hip(flux::launch_embedding_gather(ids, embedding, vocab, seq, hidden, stream),
                    "flux_embedding_gather_f32");
}

int flux_decode_replay_launches(const flux_decode* runtime, int64_t* kernel_launches, int64_t* device_commands) {
    if (runtime == nullptr || kernel_launches == nullptr || device_commands == nullptr)
        return invalid("flux_decode_replay_launches: null argument");
    return guarded([&] { runtime->impl->replay_launches(kernel_launches, device_commands); });
}

int flux_host_counters(int64_t* synchronizations, int64_t* allocations, int64_t* frees) {
    if (synchronizations == nullptr || allocations == nullptr || frees == nullptr)
        return invalid("flux_host_counters: null argument");
    flux::host_counters(synchronizations, allocations, frees);
    return FLUX_OK;
}

// ---------------------------------------------------------------------------
// Single-layer decode runtime.

int flux_layer_decode_create(const flux_layer_weights* weights, const float* rope_cos, const float* rope_sin,
                             int64_t capacity, int64_t position, const float* initial_hidden, const float* key_source,
                             const float* value_source, int64_t source_length, double epsilon,
                             double attention_scale, hipStream_t stream, flux_layer_decode** out) {
    if (weights == nullptr || out == nullptr) return invalid("flux_layer_decode_create: null argument");
    *out = nullptr;
    return guarded([&] {
        const flux::LayerWeights layer{weights->input_norm, weights->packed_qkv, weights->o_proj, weights->post_norm,
                                       weights->gate_up,    weights->down,       static_cast<float>(epsilon),
                                       static_cast<float>(attention_scale)};
        auto* impl = new flux::LayerDecodeRuntime(layer, rope_cos, rope_sin, capacity, position, initial_hidden,
                                                  key_source, value_source, source_length, stream);
        *out = new flux_layer_decode{impl};
    });
}

int flux_layer_decode_replay(flux_layer_decode* runtime, const float* hidden, hipStream_t stream, float** output) {
    if (runtime == nullptr) return invalid("flux_layer_decode_replay: null runtime");
    return guarded([&] {
        float* result = runtime->impl->replay(hidden, stream);
        if (output) *output = result;
    });
}

int flux_layer_decode_reset(flux_layer_decode* runtime, const float* hidden, const float* key_source,
                            const float* value_source, int64_t source_length, int64_t position, hipStream_t stream) {
    if (runtime == nullptr) return invalid("flux_layer_decode_reset: null runtime");
    return guarded([&] { runtime->impl->reset(hidden, key_source, value_source, source_length, position, stream); });
}

int flux_layer_decode_position(flux_layer_decode* runtime, int64_t* out) {
    if (runtime == nullptr || out == nullptr) return invalid("flux_layer_decode_position: null argument");
    return guarded([&] { *out = runtime->impl->position(); });
}

int flux_layer_decode_replay_count(const flux_layer_decode* runtime, int64_t* out) {
    if (runtime == nullptr || out == nullptr) return invalid("flux_layer_decode_replay_count: null argument");
    *out = runtime->impl->replay_count();
    return FLUX_OK;
}

int flux_layer_decode_capacity(const flux_layer_decode* runtime, int64_t* out) {
    if (runtime == nullptr || out == nullptr) return invalid("flux_layer_decode_capacity: null argument");
    *out = runtime->impl->capacity();
    return FLUX_OK;
}

int flux_layer_decode_get_buffers(const flux_layer_decode* runtime, flux_layer_decode_buffers* out) {
    if (runtime == nullptr || out == nullptr) return invalid("flux_layer_decode_get_buffers: null argument");
    runtime->impl->buffers(out);
    return FLUX_OK;
}

int flux_layer_decode_replay_launches(const flux_layer_decode* runtime, int64_t* kernel_launches,
                                     int64_t* device_commands) {
    if (runtime == nullptr || kernel_launches == nullptr || device_commands == nullptr)
        return invalid("flux_layer_decode_replay_launches: null argument");
    runtime->impl->replay_launches(kernel_launches, device_commands);
    return FLUX_OK;
}

void flux_layer_decode_destroy(flux_layer_decode* runtime) {
    if (runtime == nullptr) return;
    delete runtime->impl;
    delete runtime;
}

// ---------------------------------------------------------------------------
// Eager operators.

namespace {
bool nonnegative(const int64_t* values, int count) {
    for (int i = 0; i < count; ++i)
        if (values[i] < 0) return false;
    return true;
}
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
}  // namespace

int flux_rope_f32(const float* query, const float* key, const float* cos, const float* sin, float* query_out,
                  float* key_out, int64_t batch, int64_t query_heads, int64_t key_heads, int64_t seq,
                  int64_t head_dim, int64_t rope_batch, const int64_t* query_strides, const int64_t* key_strides,
                  const int64_t* cos_strides, const int64_t* sin_strides, hipStream_t stream) {
    if (!query || !key || !cos || !sin || !query_out || !key_out || !query_strides || !key_strides || !cos_strides ||
        !sin_strides)
        return invalid("flux_rope_f32: null argument");
    if (batch <= 0 || query_heads <= 0 || key_heads <= 0 || seq <= 0 || head_dim <= 0 || (head_dim & 1) ||
        (rope_batch != 1 && rope_batch != batch))
        return invalid("flux_rope_f32: invalid shape (head_dim must be even, rope batch 1 or batch)");
    if (!nonnegative(query_strides, 4) || !nonnegative(key_strides, 4) || !nonnegative(cos_strides, 3) ||
        !nonnegative(sin_strides, 3))
        return invalid("flux_rope_f32: negative strides are unsupported");
    flux::RopeShape shape{batch, query_heads, key_heads, seq, head_dim, rope_batch, {}, {}, {}, {}};
    for (int i = 0; i < 4; ++i) {
        shape.query_strides[i] = query_strides[i];
        shape.key_strides[i] = key_strides[i];
    }
    for (int i = 0; i < 3; ++i) {
        shape.cos_strides[i] = cos_strides[i];
        shape.sin_strides[i] = sin_strides[i];
    }
    return from_hip(flux::launch_rope(query, key, cos, sin, query_out, key_out, shape, stream), "flux_rope_f32");
}

int flux_softmax_f32(const float* input, float* output, int64_t rows, int64_t width, hipStream_t stream) {
    if (!input || !output || rows <= 0 || width <= 0) return invalid("flux_softmax_f32: invalid argument");
    return from_hip(flux::launch_softmax(input, output, rows, width, stream), "flux_softmax_f32");
}

int flux_attention_score_softmax_f32(const float* scores, const float* mask, float* output, float scale,
                                     int64_t batch, int64_t heads, int64_t query_length, int64_t key_length,
                                     const int64_t* mask_sizes, const int64_t* mask_strides, hipStream_t stream) {
    if (!scores || !mask || !output || !mask_sizes || !mask_strides || batch <= 0 || heads <= 0 ||
        query_length <= 0 || key_length <= 0 || !std::isfinite(scale))
        return invalid("flux_attention_score_softmax_f32: invalid argument");
    const int64_t target[4] = {batch, heads, query_length, key_length};
    int64_t strides[4];
    for (int i = 0; i < 4; ++i) {
        if (mask_sizes[i] != 1 && mask_sizes[i] != target[i])
            return invalid("flux_attention_score_softmax_f32: mask is not broadcastable to scores");
        if (mask_strides[i] < 0) return invalid("flux_attention_score_softmax_f32: negative mask strides");
        strides[i] = mask_sizes[i] == 1 ? 0 : mask_strides[i];
    }
    return from_hip(flux::launch_attention_score_softmax(scores, mask, output, scale, batch, heads, query_length,
                                                         key_length, strides, stream),
                    "flux_attention_score_softmax_f32");
}

int flux_packed_swiglu_f32(const float* packed, float* output, int64_t rows, int64_t intermediate,
                           hipStream_t stream) {
    if (!packed || !output || rows <= 0 || intermediate <= 0)
        return invalid("flux_packed_swiglu_f32: invalid argument");
    return from_hip(flux::launch_packed_swiglu(packed, output, rows, intermediate, stream), "flux_packed_swiglu_f32");
}

int flux_packed_qkv_rope_cache_f32(const float* packed_qkv, const float* cos, const float* sin, float* key_cache,
                                   float* value_cache, const int64_t* position, int64_t* cache_length,
                                   float* query_out, int64_t capacity, int64_t packed_stride, int64_t cos_stride,
                                   int64_t sin_stride, const int64_t* key_strides, const int64_t* value_strides,
                                   hipStream_t stream) {
    if (!packed_qkv || !cos || !sin || !key_cache || !value_cache || !position || !query_out || !key_strides ||
        !value_strides || capacity <= 0)
        return invalid("flux_packed_qkv_rope_cache_f32: invalid argument");
    if (packed_stride <= 0 || cos_stride <= 0 || sin_stride <= 0 || !nonnegative(key_strides, 4) ||
        !nonnegative(value_strides, 4))
        return invalid("flux_packed_qkv_rope_cache_f32: strides must be positive");
    flux::PackedQkvArgs args{packed_qkv, cos, sin, key_cache, value_cache, position, cache_length, query_out,
                             capacity, packed_stride, cos_stride, sin_stride, {}, {}};
    for (int i = 0; i < 4; ++i) {
        args.key_strides[i] = key_strides[i];
        args.value_strides[i] = value_strides[i];
    }
    return from_hip(flux::launch_packed_qkv_rope_cache(args, stream), "flux_packed_qkv_rope_cache_f32");
}

int flux_gqa_decode_attention_strided_workspace_bytes(int64_t query_heads, int64_t capacity, int64_t head_dim,
                                                      int64_t* bytes) {
    if (!bytes || query_heads <= 0 || capacity <= 0 || capacity > FLUX_MAX_CAPACITY || head_dim <= 0 ||
        head_dim > 4096)
        return invalid("flux_gqa_decode_attention_strided_workspace_bytes: invalid argument");
    *bytes = static_cast<int64_t>(flux::gqa_strided_workspace_floats(query_heads, capacity, head_dim) * sizeof(float));
    return FLUX_OK;
}

int flux_gqa_decode_attention_strided_f32(const float* query, const float* key_cache, const float* value_cache,
                                          const float* mask, const int64_t* cache_length, float* output,
                                          void* workspace, int64_t workspace_bytes, float scale, int64_t query_heads,
                                          int64_t kv_heads, int64_t capacity, int64_t head_dim,
                                          const int64_t* query_strides, const int64_t* key_strides,
                                          const int64_t* value_strides, const int64_t* mask_sizes,
                                          const int64_t* mask_strides, hipStream_t stream) {
    if (!query || !key_cache || !value_cache || !output || !query_strides || !key_strides || !value_strides)
        return invalid("flux_gqa_decode_attention_strided_f32: null argument");
    if (query_heads <= 0 || kv_heads <= 0 || query_heads % kv_heads || query_heads > 65536 || capacity <= 0 ||
        capacity > FLUX_MAX_CAPACITY || head_dim <= 0 || head_dim > 4096 || !std::isfinite(scale))
        return invalid("flux_gqa_decode_attention_strided_f32: invalid shape or scale");
    if (!nonnegative(query_strides, 4) || !nonnegative(key_strides, 4) || !nonnegative(value_strides, 4))
        return invalid("flux_gqa_decode_attention_strided_f32: negative strides are unsupported");
    int64_t needed = 0;
    flux_gqa_decode_attention_strided_workspace_bytes(query_heads, capacity, head_dim, &needed);
    if (needed > 0 && (!workspace || workspace_bytes < needed))
        return invalid("flux_gqa_decode_attention_strided_f32: workspace missing or too small "
                       "(flux_gqa_decode_attention_strided_workspace_bytes)");
    flux::GqaStridedArgs args{};
    args.q = query;
    args.k = key_cache;
    args.v = value_cache;
    args.mask = mask;
    args.cache_length = cache_length;
    args.out = output;
    args.workspace = static_cast<float*>(workspace);
    args.scale = scale;
    args.query_heads = static_cast<int>(query_heads);
    args.groups = static_cast<int>(query_heads / kv_heads);
    args.dim = static_cast<int>(head_dim);
    args.chunks = flux::gqa_strided_chunks(capacity, head_dim);
    args.capacity = capacity;
    for (int i = 0; i < 4; ++i) {
        args.q_strides[i] = query_strides[i];
        args.k_strides[i] = key_strides[i];
        args.v_strides[i] = value_strides[i];
    }
    if (mask) {
        if (!mask_sizes || !mask_strides)
            return invalid("flux_gqa_decode_attention_strided_f32: mask needs sizes and strides");
        const int64_t target[4] = {1, query_heads, 1, capacity};
        for (int i = 0; i < 4; ++i) {
            if (mask_sizes[i] != 1 && mask_sizes[i] != target[i])
                return invalid("flux_gqa_decode_attention_strided_f32: mask is not broadcastable");
            if (mask_strides[i] < 0) return invalid("flux_gqa_decode_attention_strided_f32: negative mask strides");
            args.mask_strides[i] = mask_sizes[i] == 1 ? 0 : mask_strides[i];
        }
    }
    args.vec = key_strides[3] == 1 && value_strides[3] == 1 && (head_dim & 3) == 0 && (key_strides[1] & 3) == 0 &&
               (key_strides[2] & 3) == 0 && (value_strides[1] & 3) == 0 && (value_strides[2] & 3) == 0 &&
               aligned16(key_cache) && aligned16(value_cache);
    return from_hip(flux::launch_gqa_strided(args, stream), "flux_gqa_decode_attention_strided_f32");
}

}  // extern "C"
