// C++ host runtime of the MI355X SmolLM2 token loop (HIP runtime API only).
//
// DecodeRuntime      <-> flux::NativeSmolLM2Decode::Impl (csrc/native_decode_runtime/native_decode_runtime_cuda.cu:740-1338)
// LayerDecodeRuntime <-> flux::NativeSmolLM2LayerDecode::Impl (native_decode_runtime_cuda.cu:314-738)
// PrefillRuntime <-> flux::NativeSmolLM2Prefill::Impl (csrc/native_prefill_runtime/native_prefill_runtime_cuda.cu:353-700)
#pragma once

#include "../../include/flux_amd.h"
#include "flux_kernels.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace flux {

// Error carrying a flux_status code; the C ABI turns it into a return value.
struct FluxError : std::runtime_error {
    int code;
    FluxError(int c, const std::string& message) : std::runtime_error(message), code(c) {}
};

void check_hip(hipError_t status, const char* what);

// Borrowed K/V sources for cache import (per layer [1, 3, length, 64]).
struct CacheSources {
    const float* const* keys = nullptr;
    const float* const* values = nullptr;
    const int64_t* lengths = nullptr;
};

class DecodeRuntime {
public:
    DecodeRuntime(const flux_weights& weights, const float* rope_cos, const float* rope_sin, int64_t capacity,
                  int64_t position, const int64_t* initial_token, const CacheSources& sources,
                  const double* epsilons, const double* scales, hipStream_t stream);
    ~DecodeRuntime();
    DecodeRuntime(const DecodeRuntime&) = delete;
    DecodeRuntime& operator=(const DecodeRuntime&) = delete;

    float* replay(const int64_t* token, hipStream_t stream);
    int64_t* generate_greedy(int64_t decode_steps, hipStream_t stream, float* elapsed_ms = nullptr);
    void reset(const int64_t* token, const CacheSources& sources, int64_t position, hipStream_t stream);
    void wait_for_prefill(hipStream_t stream);
    void install_prefilled_state(const int64_t* token, int64_t position, hipStream_t stream);
    int64_t read_scalar(const int64_t* device_value);
    int32_t device_error();

    int64_t position() { return read_scalar(position_); }
    int64_t cache_length() { return read_scalar(cache_length_); }
    int64_t generation_step() { return read_scalar(generation_step_); }
    int64_t replay_count() const { return replay_count_; }
    int64_t capacity() const { return capacity_; }
    void buffers(flux_decode_buffers* out) const;
    // Kernel launches and all device commands (launches, event waits) issued by replay()
    // since creation.
    void replay_launches(int64_t* kernels, int64_t* commands) const;
    int device() const { return device_; }
    // Bound of every cross-workgroup wait of later generate_greedy launches, in 100 MHz
    // wall-clock ticks (replays keep the default bound).
    void set_wait_limit(uint64_t ticks) { args_.wait_ticks = ticks; }

private:
    void allocate();
    // Raises FluxError(FLUX_ERROR_DEVICE) when a finished launch reported a device-side
    // error (non-blocking: reads the host-visible error word).
    void check_host_error() const;
    void initialize_state(const int64_t* token, const CacheSources& sources, int64_t position, hipStream_t stream,
                          bool clear_outputs);
    void launch_steps(int64_t steps, hipStream_t stream, hipStream_t launch_stream);
    void release() noexcept;
    // completion_, recorded on last_stream_ first when replays were queued after it.
    hipEvent_t completion();

    int device_ = 0;
    int grid_ = 0;
    int64_t capacity_ = 0;
    int64_t vocab_ = 0;
    int64_t start_position_ = 0;
    int64_t replay_count_ = 0;
    bool pending_ = false;
    bool generation_started_ = false;

    const float* rope_cos_ = nullptr;
    const float* rope_sin_ = nullptr;
    float final_eps_ = 0.0f;

    // Owned device memory.
    void* cache_block_ = nullptr;
    void* state_block_ = nullptr;
    float* key_cache_ = nullptr;
    float* value_cache_ = nullptr;
    float* logits_ = nullptr;
    int64_t* input_token_ = nullptr;
    int64_t* generated_ = nullptr;
    int64_t* generation_step_ = nullptr;
    int64_t* position_ = nullptr;
    int64_t* cache_length_ = nullptr;
    uint64_t* ll_ = nullptr;
    uint32_t* token_counter_ = nullptr;
    int32_t* error_ = nullptr;
    int32_t* host_error_ = nullptr;         // mapped pinned host memory
    int32_t* host_error_device_ = nullptr;  // its device address
    // Cooperative launches unless FLUX_DECODE_PLAIN_LAUNCH is set to a value other than 0
    // (profiling runs: rocprofv3 7.2 crashes at exit after cooperative launches).
    bool cooperative_ = true;
    LayerWeights* layers_ = nullptr;
    size_t state_bytes_ = 0;
    size_t ll_bytes_ = 0;

    hipEvent_t completion_ = nullptr;
    hipStream_t last_stream_ = nullptr;  // stream of the last queued work
    bool completion_stale_ = false;      // work was queued on last_stream_ after completion_'s record
    int64_t replay_kernels_ = 0;
    int64_t replay_commands_ = 0;
    DecodeArgs args_{};
};

class PrefillRuntime {
public:
    PrefillRuntime(const flux_weights& weights, const float* rope_cos, const float* rope_sin, int64_t capacity,
                   const int64_t* input_ids, int64_t sequence_length, const double* epsilons, const double* scales,
                   hipStream_t stream);
    ~PrefillRuntime();
    PrefillRuntime(const PrefillRuntime&) = delete;
    PrefillRuntime& operator=(const PrefillRuntime&) = delete;

    float* prefill(const int64_t* input_ids, hipStream_t stream);
    int64_t* generate_greedy(int64_t max_new_tokens, hipStream_t stream);
    DecodeRuntime* decode() { return decode_.get(); }
    void buffers(flux_prefill_buffers* out) const;

private:
    void run(const int64_t* input_ids, hipStream_t stream);

    int device_ = 0;
    int64_t seq_ = 0;
    int64_t capacity_ = 0;
    int64_t vocab_ = 0;
    flux_weights weights_{};
    const float* rope_cos_ = nullptr;
    const float* rope_sin_ = nullptr;
    std::vector<float> eps_;
    std::vector<float> scales_;
    std::unique_ptr<DecodeRuntime> decode_;

    void* block_ = nullptr;
    size_t block_bytes_ = 0;
    float* hidden_a_ = nullptr;   // [S, 576] layer input/output
    float* hidden_b_ = nullptr;   // [S, 576] post-attention residual
    float* norm_ = nullptr;       // [S, 576]
    float* query_ = nullptr;      // [9, S, 64]
    float* attn_rows_ = nullptr;  // [S, 576]
    float* attn_workspace_ = nullptr;  // split-key attention partials
    float* split_partials_ = nullptr;  // K-split GEMM partial planes (short prompts), or null
    int64_t split_floats_ = 0;         // floats at split_partials_
    float* swiglu_ = nullptr;     // [S, 1536]
    float* final_hidden_ = nullptr;  // [576]
    float* logits_ = nullptr;     // [vocab]
    int64_t* initial_token_ = nullptr;
    float* part_v_ = nullptr;
    int64_t* part_i_ = nullptr;
    int lm_grid_ = 0;
};

// One decoder layer's token step: input hidden [576] -> output hidden [576], with the
// layer's own compact cache [1, 3, capacity, 64] and device position (advanced by every
// replay).  A replay is one launch of the fused decode kernel in its single-layer mode
// (the layer's phases exchange through an uncached arena, as the token loop's do).
class LayerDecodeRuntime {
public:
    LayerDecodeRuntime(const LayerWeights& layer, const float* rope_cos, const float* rope_sin, int64_t capacity,
                       int64_t position, const float* initial_hidden, const float* key_source,
                       const float* value_source, int64_t source_length, hipStream_t stream);
    ~LayerDecodeRuntime();
    LayerDecodeRuntime(const LayerDecodeRuntime&) = delete;
    LayerDecodeRuntime& operator=(const LayerDecodeRuntime&) = delete;

    float* replay(const float* hidden, hipStream_t stream);
    void reset(const float* hidden, const float* key_source, const float* value_source, int64_t source_length,
               int64_t position, hipStream_t stream);
    int64_t position();
    int64_t replay_count() const { return replay_count_; }
    int64_t capacity() const { return capacity_; }
    void buffers(flux_layer_decode_buffers* out) const;
    // Kernel launches and all device commands (launches, event waits) issued by replay()
    // since creation.
    void replay_launches(int64_t* kernels, int64_t* commands) const;

private:
    void validate_state(const float* hidden, const float* key_source, const float* value_source,
                        int64_t source_length, int64_t position) const;
    void initialize_state(const float* hidden, const float* key_source, const float* value_source,
                          int64_t source_length, int64_t position, hipStream_t stream, bool clear_output);
    // Raises FluxError(FLUX_ERROR_DEVICE) when a finished launch reported a device-side error.
    void check_host_error() const;
    void release() noexcept;

    int device_ = 0;
    int grid_ = 0;
    int64_t capacity_ = 0;
    int64_t start_position_ = 0;
    int64_t replay_count_ = 0;
    int64_t staged_position_ = 0;
    int64_t replay_kernels_ = 0;
    int64_t replay_commands_ = 0;
    bool pending_ = false;
    hipStream_t last_stream_ = nullptr;
    LayerWeights layer_{};
    const float* rope_cos_ = nullptr;
    const float* rope_sin_ = nullptr;

    void* block_ = nullptr;
    size_t block_bytes_ = 0;
    float* input_hidden_ = nullptr;   // [576]
    float* output_ = nullptr;         // [576]
    float* key_cache_ = nullptr;      // [3, capacity, 64]
    float* value_cache_ = nullptr;
    int64_t* position_ = nullptr;
    int64_t* cache_length_ = nullptr;
    int64_t* token_word_ = nullptr;   // the kernel's token and step words (unused by the layer step)
    int64_t* step_word_ = nullptr;
    uint32_t* token_counter_ = nullptr;
    int32_t* error_ = nullptr;
    LayerWeights* layers_ = nullptr;  // device copy of layer_
    void* ll_ = nullptr;              // exchange arena (uncached pool)
    size_t ll_bytes_ = 0;
    int32_t* host_error_ = nullptr;         // mapped pinned host memory
    int32_t* host_error_device_ = nullptr;  // its device address
    hipEvent_t completion_ = nullptr;
    DecodeArgs args_{};
};

int device_cu_count();
// Totals since load: host-blocking runtime calls, device allocations, device frees.
void host_counters(int64_t* synchronizations, int64_t* allocations, int64_t* frees);
// Key chunks of the isolated decode attention for `capacity` positions.
int isolated_attention_chunks(int64_t capacity);

}  // namespace flux
