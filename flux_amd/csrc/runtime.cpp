// C++ host runtime of the MI355X SmolLM2 token loop.  See runtime.h.
#include "runtime.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <utility>
#include <vector>

namespace flux {

void check_hip(hipError_t status, const char* what) {
    if (status != hipSuccess) {
        throw FluxError(FLUX_ERROR_HIP, std::string("flux native runtime: ") + what + " failed: " +
                                            hipGetErrorString(status));
    }
}

namespace {

// Host-visible effects of the runtimes, counted for the runtime audit: every
// device allocation and free, and every call that blocks the host on the GPU.
std::atomic<int64_t> g_host_syncs{0};
std::atomic<int64_t> g_device_allocs{0};
std::atomic<int64_t> g_device_frees{0};

hipError_t counted_malloc(void** ptr, size_t bytes) {
    g_device_allocs.fetch_add(1, std::memory_order_relaxed);
    return hipMalloc(ptr, bytes);
}
hipError_t counted_free(void* ptr) {
    g_device_frees.fetch_add(1, std::memory_order_relaxed);
    return hipFree(ptr);
}
// Exchange arenas of the fused decode kernel live in uncached device memory
// (hipDeviceMallocUncached): every access to them is a cross-CU publish or poll, and the
// polls of an uncached arena return sooner (ctx 8192: 0.4368 against 0.4436 ms/token with
// the arena in ordinary device memory).  Uncached memory that a kernel has read must not
// be freed while the process runs (later allocations have then held wrong values on
// MI355X), so arenas are never freed: a runtime takes one from this per-device pool and
// gives it back when it is destroyed.  The runtime counts the take and the return as its
// allocation and free; the pool holds at most as many arenas as runtimes were ever alive
// at once on a device.
class UncachedArenaPool {
public:
    hipError_t acquire(int device, size_t bytes, void** out) {
        {
            std::lock_guard<std::mutex> lock(mutex_);
            for (size_t i = 0; i < free_.size(); ++i) {
                if (free_[i].device == device && free_[i].bytes == bytes) {
                    *out = free_[i].ptr;
                    free_[i] = free_.back();
                    free_.pop_back();
                    g_device_allocs.fetch_add(1, std::memory_order_relaxed);
                    return hipSuccess;
                }
            }
        }
        const hipError_t status = hipExtMallocWithFlags(out, bytes, hipDeviceMallocUncached);
        if (status == hipSuccess) g_device_allocs.fetch_add(1, std::memory_order_relaxed);
        return status;
    }
    void release(int device, size_t bytes, void* ptr) {
        std::lock_guard<std::mutex> lock(mutex_);
        free_.push_back(Arena{device, bytes, ptr});
        g_device_frees.fetch_add(1, std::memory_order_relaxed);
    }

private:
    struct Arena {
        int device;
        size_t bytes;
        void* ptr;
    };
    std::mutex mutex_;
    std::vector<Arena> free_;
};

UncachedArenaPool& arena_pool() {
    static UncachedArenaPool* pool = new UncachedArenaPool();  // never destroyed: the arenas outlive main
    return *pool;
}

hipError_t counted_stream_sync(hipStream_t stream) {
    g_host_syncs.fetch_add(1, std::memory_order_relaxed);
    return hipStreamSynchronize(stream);
}
hipError_t counted_event_sync(hipEvent_t event) {
    g_host_syncs.fetch_add(1, std::memory_order_relaxed);
    return hipEventSynchronize(event);
}
hipError_t counted_memcpy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
    g_host_syncs.fetch_add(1, std::memory_order_relaxed);
    return hipMemcpy(dst, src, bytes, kind);
}

[[noreturn]] void invalid(const std::string& message) { throw FluxError(FLUX_ERROR_INVALID_VALUE, message); }
[[noreturn]] void bad_state(const std::string& message) { throw FluxError(FLUX_ERROR_STATE, message); }

size_t align_up(size_t value, size_t alignment) { return (value + alignment - 1) / alignment * alignment; }

void validate_weights(const flux_weights& w, const char* who) {
    if (w.vocab_size <= 0) invalid(std::string(who) + ": vocabulary must be non-empty");
    if (w.embedding == nullptr || w.lm_head == nullptr || w.final_norm == nullptr)
        invalid(std::string(who) + ": embedding, LM-head and final norm weights are required");
    for (int i = 0; i < kLayers; ++i) {
        if (!w.input_norm[i] || !w.packed_qkv[i] || !w.o_proj[i] || !w.post_norm[i] || !w.gate_up[i] || !w.down[i])
            invalid(std::string(who) + ": exactly 30 complete layer descriptors are required");
    }
}

void validate_scalars(const double* epsilons, const double* scales, const char* who) {
    if (epsilons == nullptr || scales == nullptr) invalid(std::string(who) + ": epsilons and scales are required");
    for (int i = 0; i < kLayers; ++i) {
        if (!std::isfinite(epsilons[i]) || epsilons[i] <= 0.0)
            invalid(std::string(who) + ": every RMSNorm epsilon must be positive");
        if (!std::isfinite(scales[i])) invalid(std::string(who) + ": every attention scale must be finite");
    }
}

std::string device_error_message(int32_t err) {
    return "flux native full decode: device-side error " + std::to_string(err) +
           (err == 1 ? " (cross-workgroup wait timed out; the steps it affected report token -1)"
                     : " (position outside capacity)");
}

// Default bound of every cross-workgroup wait of the fused decode kernel: 200 ms.
constexpr uint64_t kDefaultWaitTicks = 20ull * 1000 * 1000;

int decode_grid() {
    const int cus = device_cu_count();
    int blocks = 0;
    check_hip(fused_decode_occupancy(&blocks), "querying fused decode occupancy");
    if (blocks < 1) throw FluxError(FLUX_ERROR_HIP, "flux native decode: fused decode kernel cannot be resident");
    // One workgroup per CU; every workgroup must be co-resident (they exchange data),
    // and the fused kernel maps one work unit per wave, which needs 8 * grid >= 1536.
    const int grid = std::min(cus, 3 * kMaxAttnChunks);
    if (grid < 192)
        throw FluxError(FLUX_ERROR_HIP, "flux native decode: the fused decode kernel needs at least 192 CUs, found " +
                                            std::to_string(cus));
    return grid;
}

}  // namespace

int device_cu_count() {
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    int cus = 0;
    check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device), "querying CU count");
    return cus;
}

void host_counters(int64_t* synchronizations, int64_t* allocations, int64_t* frees) {
    *synchronizations = g_host_syncs.load(std::memory_order_relaxed);
    *allocations = g_device_allocs.load(std::memory_order_relaxed);
    *frees = g_device_frees.load(std::memory_order_relaxed);
}

void DecodeRuntime::replay_launches(int64_t* kernels, int64_t* commands) const {
    *kernels = replay_kernels_;
    *commands = replay_commands_;
}

int isolated_attention_chunks(int64_t capacity) {
    int chunks = 85;
    while (gqa_decode_max_positions(chunks) < capacity) chunks *= 2;
    return chunks;
}

// ---------------------------------------------------------------------------
// DecodeRuntime

DecodeRuntime::DecodeRuntime(const flux_weights& weights, const float* rope_cos, const float* rope_sin,
                             int64_t capacity, int64_t position, const int64_t* initial_token,
                             const CacheSources& sources, const double* epsilons, const double* scales,
                             hipStream_t stream)
    : capacity_(capacity), start_position_(position), rope_cos_(rope_cos), rope_sin_(rope_sin) {
    const char* plain = std::getenv("FLUX_DECODE_PLAIN_LAUNCH");
    cooperative_ = plain == nullptr || plain[0] == '\0' || std::strcmp(plain, "0") == 0;
    validate_weights(weights, "flux native full decode");
    validate_scalars(epsilons, scales, "flux native full decode");
    if (capacity < 1 || capacity > kMaxCapacity)
        invalid("flux native full decode: cache capacity must be in [1, " + std::to_string(kMaxCapacity) + "]");
    if (position < 0 || position >= capacity)
        invalid("flux native full decode: initial position must be inside capacity");
    if (rope_cos == nullptr || rope_sin == nullptr) invalid("flux native full decode: RoPE tables are required");
    if (initial_token == nullptr) invalid("flux native full decode: initial token is required");
    if (position > 0 && (sources.keys == nullptr || sources.values == nullptr || sources.lengths == nullptr))
        invalid("flux native full decode: reset requires one K/V tensor per layer");
    vocab_ = weights.vocab_size;
    final_eps_ = static_cast<float>(epsilons[0]);
    check_hip(hipGetDevice(&device_), "hipGetDevice");
    grid_ = decode_grid();
    if (capacity_ > max_attention_positions(grid_))
        invalid("flux native full decode: capacity exceeds what the fused attention split can hold on this device");

    try {
        allocate();
        std::vector<LayerWeights> host_layers(kLayers);
        for (int i = 0; i < kLayers; ++i) {
            host_layers[i] = LayerWeights{weights.input_norm[i], weights.packed_qkv[i], weights.o_proj[i],
                                          weights.post_norm[i], weights.gate_up[i], weights.down[i],
                                          static_cast<float>(epsilons[i]), static_cast<float>(scales[i])};
        }
        check_hip(hipMemcpyAsync(layers_, host_layers.data(), sizeof(LayerWeights) * kLayers, hipMemcpyHostToDevice,
                                 stream),
                  "uploading layer descriptors");
        check_hip(hipMemsetAsync(ll_, 0, ll_bytes_, stream), "clearing exchange arena");
        check_hip(hipMemsetAsync(token_counter_, 0, sizeof(uint32_t), stream), "clearing token counter");
        check_hip(hipMemsetAsync(error_, 0, sizeof(int32_t), stream), "clearing error word");

        args_ = DecodeArgs{layers_, weights.embedding, weights.lm_head, weights.final_norm, final_eps_,
                           rope_cos_, rope_sin_, key_cache_, value_cache_, logits_, input_token_, generated_,
                           generation_step_, position_, cache_length_, ll_, token_counter_, error_,
                           host_error_device_, kDefaultWaitTicks, capacity_, vocab_, capacity_, 1, nullptr,
                           kLayers, nullptr, nullptr, nullptr};

        check_hip(hipEventCreateWithFlags(&completion_, hipEventDisableTiming), "creating completion event");

        // Warm the step once (as the reference does before capturing its graph), then
        // restore the state.  A replay is one launch of the same kernel (see replay()).
        initialize_state(initial_token, sources, position, stream, false);
        check_hip(launch_fused_decode(args_, grid_, stream, cooperative_), "warming fused decode");
        check_hip(counted_stream_sync(stream), "warming fused decode");
        if (device_error() != 0) throw FluxError(FLUX_ERROR_DEVICE, "flux native full decode: warm-up step failed");
        initialize_state(initial_token, sources, position, stream, true);
        check_hip(counted_stream_sync(stream), "initialising decode state");
    } catch (...) {
        release();
        throw;
    }
}

DecodeRuntime::~DecodeRuntime() { release(); }

void DecodeRuntime::release() noexcept {
    int previous = -1;
    (void)hipGetDevice(&previous);
    (void)hipSetDevice(device_);
    if (pending_ && completion_ != nullptr) (void)counted_event_sync(completion());
    if (completion_) (void)hipEventDestroy(completion_);
    if (cache_block_) (void)counted_free(cache_block_);
    if (state_block_) (void)counted_free(state_block_);
    if (ll_) arena_pool().release(device_, ll_bytes_, ll_);
    if (host_error_) (void)hipHostFree(host_error_);
    completion_ = nullptr;
    cache_block_ = state_block_ = nullptr;
    ll_ = nullptr;
    host_error_ = host_error_device_ = nullptr;
    if (previous >= 0 && previous != device_) (void)hipSetDevice(previous);
}

void DecodeRuntime::allocate() {
    const size_t cache_elems = static_cast<size_t>(kLayers) * kKVHeads * capacity_ * kHeadDim;
    check_hip(counted_malloc(&cache_block_, 2 * cache_elems * sizeof(float)), "allocating K/V cache");
    key_cache_ = static_cast<float*>(cache_block_);
    value_cache_ = key_cache_ + cache_elems;

    ll_bytes_ = ll_arena_words() * sizeof(uint64_t);
    size_t offset = 0;
    auto take = [&](size_t bytes) {
        const size_t at = offset;
        offset = align_up(offset + bytes, 256);
        return at;
    };
    const size_t o_logits = take(sizeof(float) * vocab_);
    const size_t o_token = take(sizeof(int64_t));
    const size_t o_generated = take(sizeof(int64_t) * capacity_);
    const size_t o_step = take(sizeof(int64_t));
    const size_t o_position = take(sizeof(int64_t));
    const size_t o_length = take(sizeof(int64_t));
    const size_t o_counter = take(sizeof(uint32_t));
    const size_t o_error = take(sizeof(int32_t));
    const size_t o_layers = take(sizeof(LayerWeights) * kLayers);
    state_bytes_ = offset;
    check_hip(counted_malloc(&state_block_, state_bytes_), "allocating decode state");
    char* base = static_cast<char*>(state_block_);
    logits_ = reinterpret_cast<float*>(base + o_logits);
    input_token_ = reinterpret_cast<int64_t*>(base + o_token);
    generated_ = reinterpret_cast<int64_t*>(base + o_generated);
    generation_step_ = reinterpret_cast<int64_t*>(base + o_step);
    position_ = reinterpret_cast<int64_t*>(base + o_position);
    cache_length_ = reinterpret_cast<int64_t*>(base + o_length);
    token_counter_ = reinterpret_cast<uint32_t*>(base + o_counter);
    error_ = reinterpret_cast<int32_t*>(base + o_error);
    layers_ = reinterpret_cast<LayerWeights*>(base + o_layers);
    void* arena = nullptr;
    check_hip(arena_pool().acquire(device_, ll_bytes_, &arena), "allocating the uncached exchange arena");
    ll_ = static_cast<uint64_t*>(arena);
    // The kernel's error word also lands in mapped pinned host memory, so every runtime call
    // can see a finished launch's device error without synchronising.
    check_hip(hipHostMalloc(reinterpret_cast<void**>(&host_error_), sizeof(int32_t),
                            hipHostMallocMapped | hipHostMallocCoherent),
              "allocating the host-visible error word");
    *host_error_ = 0;
    check_hip(hipHostGetDevicePointer(reinterpret_cast<void**>(&host_error_device_), host_error_, 0),
              "mapping the host-visible error word");
}

void DecodeRuntime::check_host_error() const {
    const int32_t err = __atomic_load_n(host_error_, __ATOMIC_ACQUIRE);
    if (err != 0) throw FluxError(FLUX_ERROR_DEVICE, device_error_message(err));
}

void DecodeRuntime::initialize_state(const int64_t* token, const CacheSources& sources, int64_t position,
                                     hipStream_t stream, bool clear_outputs) {
    const size_t cache_bytes = static_cast<size_t>(kLayers) * kKVHeads * capacity_ * kHeadDim * sizeof(float);
    check_hip(hipMemsetAsync(key_cache_, 0, cache_bytes, stream), "clearing K cache");
    check_hip(hipMemsetAsync(value_cache_, 0, cache_bytes, stream), "clearing V cache");
    if (position > 0) {
        const size_t row_bytes = static_cast<size_t>(position) * kHeadDim * sizeof(float);
        const size_t dst_pitch = static_cast<size_t>(capacity_) * kHeadDim * sizeof(float);
        for (int i = 0; i < kLayers; ++i) {
            const size_t src_pitch = static_cast<size_t>(sources.lengths[i]) * kHeadDim * sizeof(float);
            const size_t layer_offset = static_cast<size_t>(i) * kKVHeads * capacity_ * kHeadDim;
            check_hip(hipMemcpy2DAsync(key_cache_ + layer_offset, dst_pitch, sources.keys[i], src_pitch, row_bytes,
                                       kKVHeads, hipMemcpyDeviceToDevice, stream),
                      "importing K cache");
            check_hip(hipMemcpy2DAsync(value_cache_ + layer_offset, dst_pitch, sources.values[i], src_pitch, row_bytes,
                                       kKVHeads, hipMemcpyDeviceToDevice, stream),
                      "importing V cache");
        }
    }
    check_hip(launch_install_state(token, position, 0, false, input_token_, position_, cache_length_, generation_step_,
                                   generated_, error_, host_error_device_, stream),
              "initialising device state");
    if (clear_outputs) {
        check_hip(hipMemsetAsync(logits_, 0, sizeof(float) * vocab_, stream), "clearing logits");
        check_hip(hipMemsetAsync(generated_, 0, sizeof(int64_t) * capacity_, stream), "clearing generated tokens");
    }
}

hipEvent_t DecodeRuntime::completion() {
    if (completion_stale_) {
        check_hip(hipEventRecord(completion_, last_stream_), "recording decode completion");
        completion_stale_ = false;
    }
    return completion_;
}

float* DecodeRuntime::replay(const int64_t* token, hipStream_t stream) {
    check_host_error();
    if (replay_count_ >= capacity_ - start_position_)
        bad_state("flux native full decode: fixed-capacity state is exhausted");
    check_hip(hipSetDevice(device_), "hipSetDevice");
    // Work already queued on the same stream is ordered by the stream itself; an event
    // wait there would only add a dependency packet between consecutive steps.
    if (pending_ && stream != last_stream_) {
        check_hip(hipStreamWaitEvent(stream, completion(), 0), "ordering consecutive replays");
        ++replay_commands_;
    }
    // The whole token step is one kernel, so a replay is one direct launch of it with the
    // caller's token pointer as an argument (DecodeArgs::token_in, read by the step in
    // stream order: no copy).  Measured per token at ctx 8192 against the same kernel
    // inside one 64-step launch (437.9 us): a one-node hipGraph replay (cooperative node,
    // token copy, event wait and record) 453.1 us and 27 us of host time; this launch
    // 439.7 us and 3 us.  The launch is plain, like the reference's replay (a cooperative
    // launch cost 21 us per token): every workgroup fits the device at once (occupancy is
    // checked at creation) and every cross-workgroup wait is bounded, so a step that
    // starts while other work holds CUs reports device error 1 instead of hanging.
    // The completion event is recorded only when another stream or a synchronising call
    // needs it; the caller's stream must stay valid until then.
    DecodeArgs args = args_;
    args.wait_ticks = kDefaultWaitTicks;
    args.token_in = token;
    check_hip(launch_fused_decode(args, grid_, stream, false), "launching decode step");
    ++replay_kernels_;
    ++replay_commands_;
    last_stream_ = stream;
    completion_stale_ = true;
    pending_ = true;
    ++replay_count_;
    return logits_;
}

void DecodeRuntime::launch_steps(int64_t steps, hipStream_t stream, hipStream_t) {
    DecodeArgs args = args_;
    // One launch runs many tokens; keep launches bounded so a single kernel stays short.
    constexpr int64_t kMaxStepsPerLaunch = 1024;
    for (int64_t done = 0; done < steps; done += kMaxStepsPerLaunch) {
        args.steps = static_cast<int>(std::min(kMaxStepsPerLaunch, steps - done));
        check_hip(launch_fused_decode(args, grid_, stream, cooperative_), "launching fused decode");
    }
}

int64_t* DecodeRuntime::generate_greedy(int64_t decode_steps, hipStream_t stream, float* elapsed_ms) {
    if (decode_steps < 0)
        invalid("flux native full decode: generation step count must be non-negative");
    if (decode_steps > capacity_ - start_position_ - replay_count_)
        bad_state("flux native full decode: fixed-capacity generation is exhausted");
    if (generation_started_) bad_state("flux native full decode: prefill or reset is required before reuse");
    check_host_error();
    check_hip(hipSetDevice(device_), "hipSetDevice");
    if (pending_ && stream != last_stream_)
        check_hip(hipStreamWaitEvent(stream, completion(), 0), "ordering greedy generation");
    if (decode_steps > 0) {
        hipEvent_t start = nullptr, stop = nullptr;
        if (elapsed_ms != nullptr) {
            check_hip(hipEventCreate(&start), "creating timing event");
            check_hip(hipEventCreate(&stop), "creating timing event");
            check_hip(hipEventRecord(start, stream), "recording timing event");
        }
        launch_steps(decode_steps, stream, stream);
        if (elapsed_ms != nullptr) {
            check_hip(hipEventRecord(stop, stream), "recording timing event");
            check_hip(counted_event_sync(stop), "waiting for timing event");
            check_hip(hipEventElapsedTime(elapsed_ms, start, stop), "reading timing events");
            (void)hipEventDestroy(start);
            (void)hipEventDestroy(stop);
        }
        check_hip(hipEventRecord(completion_, stream), "recording generation completion");
        last_stream_ = stream;
        completion_stale_ = false;
        pending_ = true;
        replay_count_ += decode_steps;
    }
    generation_started_ = true;
    return generated_;
}

void DecodeRuntime::reset(const int64_t* token, const CacheSources& sources, int64_t position, hipStream_t stream) {
    if (token == nullptr) invalid("flux native full decode: token is required");
    if (position < 0 || position >= capacity_)
        invalid("flux native full decode: reset position must be inside capacity");
    if (position > 0 && (sources.keys == nullptr || sources.values == nullptr || sources.lengths == nullptr))
        invalid("flux native full decode: reset requires one K/V tensor per layer");
    if (position > 0) {
        for (int i = 0; i < kLayers; ++i) {
            if (sources.keys[i] == nullptr || sources.values[i] == nullptr || sources.lengths[i] < position)
                invalid("flux native full decode: every K/V source must be contiguous float32 "
                        "[1, 3, sequence>=position, 64]");
        }
    }
    check_hip(hipSetDevice(device_), "hipSetDevice");
    if (pending_) {
        check_hip(counted_event_sync(completion()), "waiting to reset full runtime");
        pending_ = false;
    }
    initialize_state(token, sources, position, stream, true);
    check_hip(counted_stream_sync(stream), "resetting full runtime state");
    *host_error_ = 0;
    start_position_ = position;
    replay_count_ = 0;
    generation_started_ = false;
}

void DecodeRuntime::wait_for_prefill(hipStream_t stream) {
    if (pending_) {
        if (stream != last_stream_)
            check_hip(hipStreamWaitEvent(stream, completion(), 0), "ordering prefill after decode work");
        pending_ = false;
    }
}

void DecodeRuntime::install_prefilled_state(const int64_t* token, int64_t position, hipStream_t stream) {
    if (position < 1 || position > capacity_)
        invalid("flux native full decode: prefill position must be in [1, capacity]");
    // A prefill re-arms a runtime whose earlier launch reported a device error: the
    // install kernel clears both error words in stream order; the host copy is also
    // cleared here, once the failed launch has finished, so the next call does not
    // see the stale word before the install kernel has run.
    if (__atomic_load_n(host_error_, __ATOMIC_ACQUIRE) != 0) {
        check_hip(counted_stream_sync(stream), "waiting for the failed decode launch");
        *host_error_ = 0;
    }
    check_hip(launch_install_state(token, position, 1, true, input_token_, position_, cache_length_, generation_step_,
                                   generated_, error_, host_error_device_, stream),
              "installing prefilled state");
    check_hip(hipEventRecord(completion_, stream), "recording prefill completion");
    last_stream_ = stream;
    completion_stale_ = false;
    start_position_ = position;
    replay_count_ = 0;
    generation_started_ = false;
    pending_ = true;
}

int64_t DecodeRuntime::read_scalar(const int64_t* device_value) {
    check_hip(hipSetDevice(device_), "hipSetDevice");
    if (pending_) check_hip(counted_event_sync(completion()), "waiting to inspect runtime state");
    int64_t result = -1;
    check_hip(counted_memcpy(&result, device_value, sizeof(result), hipMemcpyDeviceToHost), "reading device state");
    int32_t err = 0;
    check_hip(counted_memcpy(&err, error_, sizeof(err), hipMemcpyDeviceToHost), "reading device error word");
    if (err != 0) throw FluxError(FLUX_ERROR_DEVICE, device_error_message(err));
    return result;
}

int32_t DecodeRuntime::device_error() {
    check_hip(hipSetDevice(device_), "hipSetDevice");
    if (pending_) check_hip(counted_event_sync(completion()), "waiting for runtime");
    int32_t err = 0;
    check_hip(counted_memcpy(&err, error_, sizeof(err), hipMemcpyDeviceToHost), "reading device error word");
    return err;
}

void DecodeRuntime::buffers(flux_decode_buffers* out) const {
    std::memset(out, 0, sizeof(*out));
    out->input_token = input_token_;
    out->logits = logits_;
    out->generated_tokens = generated_;
    out->generation_step = generation_step_;
    out->key_cache = key_cache_;
    out->value_cache = value_cache_;
    out->position = position_;
    out->cache_length = cache_length_;
    out->workspace = ll_;
    const size_t parity_words = ll_arena_words() / 2;
    out->hidden_a = ll_;
    out->hidden_b = ll_ + parity_words;
    out->final_norm_output = ll_ + parity_words / 2;
    out->attention_workspace = ll_ + parity_words / 4;
    out->capacity = capacity_;
    out->vocab_size = vocab_;
    out->workspace_bytes = static_cast<int64_t>(ll_bytes_);
    out->cache_bytes = static_cast<int64_t>(2) * kLayers * kKVHeads * capacity_ * kHeadDim * sizeof(float);
    out->stable_buffer_bytes = static_cast<int64_t>(sizeof(int64_t) * (5 + capacity_) + sizeof(float) * vocab_);
}

// ---------------------------------------------------------------------------
// PrefillRuntime

PrefillRuntime::PrefillRuntime(const flux_weights& weights, const float* rope_cos, const float* rope_sin,
                               int64_t capacity, const int64_t* input_ids, int64_t sequence_length,
                               const double* epsilons, const double* scales, hipStream_t stream)
    : seq_(sequence_length), capacity_(capacity), weights_(weights), rope_cos_(rope_cos), rope_sin_(rope_sin) {
    validate_weights(weights, "flux native prefill");
    validate_scalars(epsilons, scales, "flux native prefill");
    if (capacity < 1 || capacity > kMaxCapacity)
        invalid("flux native prefill: cache capacity must be in [1, " + std::to_string(kMaxCapacity) + "]");
    if (sequence_length < 1 || sequence_length > capacity)
        invalid("flux native prefill: prompt length must be in [1, capacity]");
    if (input_ids == nullptr || rope_cos == nullptr || rope_sin == nullptr)
        invalid("flux native prefill: input_ids and RoPE tables are required");
    vocab_ = weights.vocab_size;
    for (int i = 0; i < kLayers; ++i) {
        eps_.push_back(static_cast<float>(epsilons[i]));
        scales_.push_back(static_cast<float>(scales[i]));
    }
    check_hip(hipGetDevice(&device_), "hipGetDevice");
    lm_grid_ = std::max(1, device_cu_count());

    const int64_t s = seq_;
    size_t offset = 0;
    auto take = [&](size_t bytes) {
        const size_t at = offset;
        offset = align_up(offset + bytes, 256);
        return at;
    };
    const size_t o_a = take(sizeof(float) * s * kHidden);
    const size_t o_b = take(sizeof(float) * s * kHidden);
    const size_t o_norm = take(sizeof(float) * s * kHidden);
    const size_t o_q = take(sizeof(float) * s * kQHeads * kHeadDim);
    const size_t o_attn = take(sizeof(float) * s * kHidden);
    const size_t o_swiglu = take(sizeof(float) * s * kInter);
    const size_t o_attn_ws = take(sizeof(float) * prefill_attention_workspace_floats(s));
    // Partial planes of the K-split GEMMs, whose grids are small only for short and mid-length
    // prompts: sized for gate/up up to kSplitKMaxRows rows, for the 576-column GEMMs beyond.
    const bool split_k = s <= kNarrowSplitMaxRows;
    const int64_t split_n = s <= kSplitKMaxRows ? kGateUp : kHidden;
    const size_t o_split = take(split_k ? sizeof(float) * split_partials_floats(s, split_n) : 0);
    const size_t o_final = take(sizeof(float) * kHidden);
    const size_t o_logits = take(sizeof(float) * vocab_);
    const size_t o_token = take(sizeof(int64_t));
    const size_t o_pv = take(sizeof(float) * lm_grid_);
    const size_t o_pi = take(sizeof(int64_t) * lm_grid_);
    block_bytes_ = offset;

    // An empty-cache decode runtime at position 0 with a zero token.
    int64_t* zero_token = nullptr;
    check_hip(counted_malloc(&block_, block_bytes_), "allocating prefill workspace");
    char* base = static_cast<char*>(block_);
    hidden_a_ = reinterpret_cast<float*>(base + o_a);
    hidden_b_ = reinterpret_cast<float*>(base + o_b);
    norm_ = reinterpret_cast<float*>(base + o_norm);
    query_ = reinterpret_cast<float*>(base + o_q);
    attn_rows_ = reinterpret_cast<float*>(base + o_attn);
    swiglu_ = reinterpret_cast<float*>(base + o_swiglu);
    attn_workspace_ = reinterpret_cast<float*>(base + o_attn_ws);
    split_partials_ = split_k ? reinterpret_cast<float*>(base + o_split) : nullptr;
    split_floats_ = split_k ? split_partials_floats(s, split_n) : 0;
    final_hidden_ = reinterpret_cast<float*>(base + o_final);
    logits_ = reinterpret_cast<float*>(base + o_logits);
    initial_token_ = reinterpret_cast<int64_t*>(base + o_token);
    part_v_ = reinterpret_cast<float*>(base + o_pv);
    part_i_ = reinterpret_cast<int64_t*>(base + o_pi);
    try {
        zero_token = initial_token_;
        check_hip(hipMemsetAsync(zero_token, 0, sizeof(int64_t), stream), "initialising decode token");
        decode_ = std::make_unique<DecodeRuntime>(weights, rope_cos, rope_sin, capacity, 0, zero_token,
                                                  CacheSources{}, epsilons, scales, stream);
        prefill(input_ids, stream);
    } catch (...) {
        decode_.reset();
        (void)counted_free(block_);
        block_ = nullptr;
        throw;
    }
}

PrefillRuntime::~PrefillRuntime() {
    if (decode_) {
        try {
            (void)decode_->device_error();
        } catch (...) {
        }
    }
    decode_.reset();
    if (block_) (void)counted_free(block_);
}

float* PrefillRuntime::prefill(const int64_t* input_ids, hipStream_t stream) {
    if (input_ids == nullptr) invalid("flux native prefill: input_ids are required");
    check_hip(hipSetDevice(device_), "hipSetDevice");
    decode_->wait_for_prefill(stream);
    run(input_ids, stream);
    decode_->install_prefilled_state(initial_token_, seq_, stream);
    return logits_;
}

// Prompts up to which the down GEMM's partial planes are summed by the next QKV kernel: every
// one of the QKV kernel's 15 column blocks loads the residual and three planes of its rows, which
// beyond a few rows costs more than the reduce kernel it replaces (16 tokens: 1.24 against
// 1.19 ms; 1 token 1.10 → 1.04, 8 tokens 1.16 → 1.13).
constexpr int64_t kDownPlanesMaxRows = 8;

void PrefillRuntime::run(const int64_t* input_ids, hipStream_t stream) {
    flux_decode_buffers db;
    decode_->buffers(&db);
    check_hip(launch_embedding_gather(input_ids, weights_.embedding, vocab_, seq_, hidden_a_, stream),
              "launching embedding gather");
    const int64_t layer_elems = static_cast<int64_t>(kKVHeads) * capacity_ * kHeadDim;
    // The QKV and gate/up GEMMs fold their RMSNorm for short prompts; otherwise the norm runs
    // with the o_proj / down GEMM before it (launch_gemm_residual_norm), which lets a K-split
    // GEMM reduce its partial planes inside the norm kernel.
    GemmArgs qkv_shape{};
    qkv_shape.m = seq_;
    qkv_shape.n = kQKV;
    qkv_shape.k = kHidden;
    GemmArgs gu_shape{};
    gu_shape.m = seq_;
    gu_shape.n = kGateUp;
    gu_shape.k = kHidden;
    GemmArgs down_shape{};
    down_shape.m = seq_;
    down_shape.n = kHidden;
    down_shape.k = kInter;
    down_shape.split_partials = split_partials_;
    down_shape.split_floats = split_floats_;
    const bool qkv_folds = gemm_folds_norm(qkv_shape, GemmEpilogue::kQkvRope);
    const bool gu_folds = gemm_folds_norm(gu_shape, GemmEpilogue::kSwiglu);
    // Prompts of a few tokens: the down GEMM leaves its K-split partial planes unreduced and
    // the next layer's QKV kernel sums them with the residual into its A rows (writing the
    // hidden rows on the way), which takes the reduce kernel out of 29 of the 30 layers.
    const bool down_planes = seq_ <= kDownPlanesMaxRows && qkv_folds &&
                             gemm_sums_planes(qkv_shape, GemmEpilogue::kQkvRope) &&
                             gemm_writes_planes(down_shape, GemmEpilogue::kResidual);
    for (int layer = 0; layer < kLayers; ++layer) {
        float* keys = db.key_cache + layer * layer_elems;
        float* values = db.value_cache + layer * layer_elems;
        GemmArgs qkv{};
        qkv.split_partials = split_partials_;
        qkv.split_floats = split_floats_;
        qkv.b = weights_.packed_qkv[layer];
        qkv.m = seq_;
        qkv.n = kQKV;
        qkv.k = kHidden;
        qkv.rope_cos = rope_cos_;
        qkv.rope_sin = rope_sin_;
        qkv.q_out = query_;
        qkv.key_cache = keys;
        qkv.value_cache = values;
        qkv.capacity = capacity_;
        if (layer == 0 || qkv_folds) {
            qkv.a = hidden_a_;
            if (layer > 0 && down_planes) {
                qkv.a_planes = split_partials_;  // the previous layer's down GEMM, unreduced
                qkv.a_residual = hidden_b_;
                qkv.a_rows_out = hidden_a_;
            }
            check_hip(launch_norm_gemm(qkv, weights_.input_norm[layer], eps_[layer], norm_, GemmEpilogue::kQkvRope,
                                       stream),
                      "launching input RMSNorm + QKV GEMM");
        } else {
            qkv.a = norm_;  // normalized by the previous layer's down GEMM + norm
            check_hip(launch_gemm(qkv, GemmEpilogue::kQkvRope, stream), "launching QKV GEMM");
        }
        check_hip(launch_prefill_attention(query_, keys, values, seq_, capacity_, scales_[layer], attn_workspace_,
                                           attn_rows_, stream),
                  "launching prefill attention");
        GemmArgs o{};
        o.split_partials = split_partials_;
        o.split_floats = split_floats_;
        o.a = attn_rows_;
        o.b = weights_.o_proj[layer];
        o.c = hidden_b_;
        o.residual = hidden_a_;
        o.m = seq_;
        o.n = kHidden;
        o.k = kHidden;
        GemmArgs gu{};
        gu.split_partials = split_partials_;
        gu.split_floats = split_floats_;
        gu.b = weights_.gate_up[layer];
        gu.c = swiglu_;
        gu.m = seq_;
        gu.n = kGateUp;
        gu.k = kHidden;
        if (gu_folds) {
            check_hip(launch_gemm(o, GemmEpilogue::kResidual, stream), "launching o_proj GEMM");
            gu.a = hidden_b_;
            check_hip(launch_norm_gemm(gu, weights_.post_norm[layer], eps_[layer], norm_, GemmEpilogue::kSwiglu, stream),
                      "launching post-attention RMSNorm + gate/up GEMM");
        } else {
            check_hip(launch_gemm_residual_norm(o, weights_.post_norm[layer], eps_[layer], norm_, stream),
                      "launching o_proj GEMM + post-attention RMSNorm");
            gu.a = norm_;
            check_hip(launch_gemm(gu, GemmEpilogue::kSwiglu, stream), "launching gate/up GEMM");
        }
        GemmArgs dn{};
        dn.split_partials = split_partials_;
        dn.split_floats = split_floats_;
        dn.a = swiglu_;
        dn.b = weights_.down[layer];
        dn.c = hidden_a_;
        dn.residual = hidden_b_;
        dn.m = seq_;
        dn.n = kHidden;
        dn.k = kInter;
        if (layer + 1 < kLayers && !qkv_folds) {
            check_hip(launch_gemm_residual_norm(dn, weights_.input_norm[layer + 1], eps_[layer + 1], norm_, stream),
                      "launching down GEMM + next input RMSNorm");
        } else if (layer + 1 < kLayers && down_planes) {
            check_hip(launch_gemm_planes(dn, GemmEpilogue::kResidual, stream), "launching down GEMM (partial planes)");
        } else {
            check_hip(launch_gemm(dn, GemmEpilogue::kResidual, stream), "launching down GEMM");
        }
    }
    const float* last_row = hidden_a_ + (seq_ - 1) * kHidden;
    check_hip(launch_rmsnorm_rows(last_row, weights_.final_norm, final_hidden_, 1, kHidden, eps_[0], stream),
              "launching final RMSNorm");
    check_hip(launch_lm_head_argmax(final_hidden_, nullptr, 0.0f, weights_.lm_head, vocab_, logits_, part_v_, part_i_,
                                    lm_grid_, initial_token_, stream),
              "launching LM head + argmax");
}

int64_t* PrefillRuntime::generate_greedy(int64_t max_new_tokens, hipStream_t stream) {
    if (max_new_tokens < 1) invalid("flux native prefill: max_new_tokens must be positive");
    if (max_new_tokens > capacity_ - seq_ + 1)
        bad_state("flux native prefill: generation exceeds fixed cache capacity");
    return decode_->generate_greedy(max_new_tokens - 1, stream);
}

void PrefillRuntime::buffers(flux_prefill_buffers* out) const {
    std::memset(out, 0, sizeof(*out));
    out->prefill_logits = logits_;
    out->prefill_workspace = block_;
    out->attention_output = attn_rows_;
    out->final_hidden = final_hidden_;
    out->initial_token = initial_token_;
    out->sequence_length = seq_;
    out->capacity = capacity_;
    out->workspace_bytes = static_cast<int64_t>(block_bytes_);
}

// ---------------------------------------------------------------------------
// LayerDecodeRuntime

LayerDecodeRuntime::LayerDecodeRuntime(const LayerWeights& layer, const float* rope_cos, const float* rope_sin,
                                       int64_t capacity, int64_t position, const float* initial_hidden,
                                       const float* key_source, const float* value_source, int64_t source_length,
                                       hipStream_t stream)
    : capacity_(capacity), start_position_(position), layer_(layer), rope_cos_(rope_cos), rope_sin_(rope_sin) {
    if (capacity < 1 || capacity > kMaxCapacity)
        invalid("flux native decode: cache capacity must be in [1, " + std::to_string(kMaxCapacity) + "]");
    if (position < 0 || position >= capacity)
        invalid("flux native decode: initial position must be inside cache capacity");
    if (!std::isfinite(layer.eps) || !(layer.eps > 0.0f))
        invalid("flux native decode: epsilon must be positive and finite");
    if (!std::isfinite(layer.scale)) invalid("flux native decode: attention scale must be finite FP32");
    if (!layer.input_norm || !layer.qkv || !layer.o_proj || !layer.post_norm || !layer.gate_up || !layer.down)
        invalid("flux native decode: every layer weight is required");
    if (rope_cos == nullptr || rope_sin == nullptr) invalid("flux native decode: RoPE tables are required");
    validate_state(initial_hidden, key_source, value_source, source_length, position);
    check_hip(hipGetDevice(&device_), "hipGetDevice");
    grid_ = decode_grid();
    if (capacity_ > max_attention_positions(grid_))
        invalid("flux native decode: capacity exceeds what the fused attention split can hold on this device");

    try {
        const size_t cache_elems = static_cast<size_t>(kKVHeads) * capacity_ * kHeadDim;
        size_t offset = 0;
        auto take = [&](size_t bytes) {
            const size_t at = offset;
            offset = align_up(offset + bytes, 256);
            return at;
        };
        const size_t o_hidden = take(kHidden * sizeof(float));
        const size_t o_output = take(kHidden * sizeof(float));
        const size_t o_key = take(cache_elems * sizeof(float));
        const size_t o_value = take(cache_elems * sizeof(float));
        const size_t o_position = take(sizeof(int64_t));
        const size_t o_length = take(sizeof(int64_t));
        const size_t o_token = take(sizeof(int64_t));
        const size_t o_step = take(sizeof(int64_t));
        const size_t o_counter = take(sizeof(uint32_t));
        const size_t o_error = take(sizeof(int32_t));
        const size_t o_layers = take(sizeof(LayerWeights));
        block_bytes_ = offset;
        check_hip(counted_malloc(&block_, block_bytes_), "allocating layer decode buffers");
        char* base = static_cast<char*>(block_);
        input_hidden_ = reinterpret_cast<float*>(base + o_hidden);
        output_ = reinterpret_cast<float*>(base + o_output);
        key_cache_ = reinterpret_cast<float*>(base + o_key);
        value_cache_ = reinterpret_cast<float*>(base + o_value);
        position_ = reinterpret_cast<int64_t*>(base + o_position);
        cache_length_ = reinterpret_cast<int64_t*>(base + o_length);
        token_word_ = reinterpret_cast<int64_t*>(base + o_token);
        step_word_ = reinterpret_cast<int64_t*>(base + o_step);
        token_counter_ = reinterpret_cast<uint32_t*>(base + o_counter);
        error_ = reinterpret_cast<int32_t*>(base + o_error);
        layers_ = reinterpret_cast<LayerWeights*>(base + o_layers);
        ll_bytes_ = ll_arena_words() * sizeof(uint64_t);
        check_hip(arena_pool().acquire(device_, ll_bytes_, &ll_), "allocating the uncached exchange arena");
        check_hip(hipHostMalloc(reinterpret_cast<void**>(&host_error_), sizeof(int32_t),
                                hipHostMallocMapped | hipHostMallocCoherent),
                  "allocating the host-visible error word");
        *host_error_ = 0;
        check_hip(hipHostGetDevicePointer(reinterpret_cast<void**>(&host_error_device_), host_error_, 0),
                  "mapping the host-visible error word");
        check_hip(hipEventCreateWithFlags(&completion_, hipEventDisableTiming), "creating completion event");

        check_hip(hipMemcpyAsync(layers_, &layer_, sizeof(LayerWeights), hipMemcpyHostToDevice, stream),
                  "uploading layer descriptor");
        check_hip(hipMemsetAsync(ll_, 0, ll_bytes_, stream), "clearing exchange arena");
        check_hip(hipMemsetAsync(token_counter_, 0, sizeof(uint32_t), stream), "clearing token counter");
        check_hip(hipMemsetAsync(token_word_, 0, sizeof(int64_t), stream), "clearing token word");
        check_hip(hipMemsetAsync(step_word_, 0, sizeof(int64_t), stream), "clearing step word");
        check_hip(hipMemsetAsync(error_, 0, sizeof(int32_t), stream), "clearing error word");
        // The fused decode kernel in its single-layer mode: one layer, no token, no LM head.
        args_ = DecodeArgs{layers_, nullptr, nullptr, nullptr, 0.0f, rope_cos_, rope_sin_, key_cache_, value_cache_,
                           nullptr, token_word_, nullptr, step_word_, position_, cache_length_,
                           static_cast<uint64_t*>(ll_), token_counter_, error_, host_error_device_, kDefaultWaitTicks,
                           capacity_, 1, 0, 1, nullptr, 1, input_hidden_, nullptr, output_};

        // Warm one step, then restore the state (the reference warms the step before capture).
        initialize_state(initial_hidden, key_source, value_source, source_length, position, stream, false);
        check_hip(launch_fused_decode(args_, grid_, stream, false), "warming layer decode");
        check_hip(counted_stream_sync(stream), "warming layer decode");
        check_host_error();
        initialize_state(initial_hidden, key_source, value_source, source_length, position, stream, true);
        check_hip(counted_stream_sync(stream), "initialising layer decode state");
    } catch (...) {
        release();
        throw;
    }
}

LayerDecodeRuntime::~LayerDecodeRuntime() { release(); }

void LayerDecodeRuntime::release() noexcept {
    int previous = -1;
    (void)hipGetDevice(&previous);
    (void)hipSetDevice(device_);
    if (pending_ && completion_ != nullptr) (void)counted_event_sync(completion_);
    if (completion_) (void)hipEventDestroy(completion_);
    if (block_) (void)counted_free(block_);
    if (ll_) arena_pool().release(device_, ll_bytes_, ll_);
    if (host_error_) (void)hipHostFree(host_error_);
    completion_ = nullptr;
    block_ = nullptr;
    ll_ = nullptr;
    host_error_ = host_error_device_ = nullptr;
    if (previous >= 0 && previous != device_) (void)hipSetDevice(previous);
}

void LayerDecodeRuntime::check_host_error() const {
    const int32_t err = __atomic_load_n(host_error_, __ATOMIC_ACQUIRE);
    if (err != 0) throw FluxError(FLUX_ERROR_DEVICE, device_error_message(err));
}

void LayerDecodeRuntime::validate_state(const float* hidden, const float* key_source, const float* value_source,
                                        int64_t source_length, int64_t position) const {
    if (hidden == nullptr) invalid("flux native decode: hidden state is undefined");
    if (position < 0 || position >= capacity_)
        invalid("flux native decode: reset position must be inside cache capacity");
    if (position > 0 && (key_source == nullptr || value_source == nullptr || source_length < position))
        invalid("flux native decode: initial/reset K/V must be matching contiguous float32 CUDA tensors shaped "
                "[1, 3, sequence>=position, 64]");
}

void LayerDecodeRuntime::initialize_state(const float* hidden, const float* key_source, const float* value_source,
                                          int64_t source_length, int64_t position, hipStream_t stream,
                                          bool clear_output) {
    const size_t cache_bytes = static_cast<size_t>(kKVHeads) * capacity_ * kHeadDim * sizeof(float);
    check_hip(hipMemcpyAsync(input_hidden_, hidden, kHidden * sizeof(float), hipMemcpyDeviceToDevice, stream),
              "initialising hidden state");
    check_hip(hipMemsetAsync(key_cache_, 0, cache_bytes, stream), "clearing K cache");
    check_hip(hipMemsetAsync(value_cache_, 0, cache_bytes, stream), "clearing V cache");
    if (position > 0) {
        const size_t row_bytes = static_cast<size_t>(position) * kHeadDim * sizeof(float);
        const size_t src_pitch = static_cast<size_t>(source_length) * kHeadDim * sizeof(float);
        const size_t dst_pitch = static_cast<size_t>(capacity_) * kHeadDim * sizeof(float);
        check_hip(hipMemcpy2DAsync(key_cache_, dst_pitch, key_source, src_pitch, row_bytes, kKVHeads,
                                   hipMemcpyDeviceToDevice, stream),
                  "importing K cache");
        check_hip(hipMemcpy2DAsync(value_cache_, dst_pitch, value_source, src_pitch, row_bytes, kKVHeads,
                                   hipMemcpyDeviceToDevice, stream),
                  "importing V cache");
    }
    staged_position_ = position;
    check_hip(hipMemcpyAsync(position_, &staged_position_, sizeof(int64_t), hipMemcpyHostToDevice, stream),
              "initialising device position");
    check_hip(hipMemcpyAsync(cache_length_, &staged_position_, sizeof(int64_t), hipMemcpyHostToDevice, stream),
              "initialising device cache length");
    if (clear_output) check_hip(hipMemsetAsync(output_, 0, kHidden * sizeof(float), stream), "clearing layer output");
}

// The step, as native_decode_runtime_cuda.cu:192-310 orders it: RMSNorm + packed QKV GEMV + RoPE
// + cache row at *position; GQA over [0, *position]; o_proj + residual; RMSNorm + gate/up GEMV +
// SwiGLU; down + residual; then *position += 1.  One plain launch of the fused decode kernel in
// its single-layer mode: it reads the caller's hidden state directly (workgroup 0 keeps a copy
// as the input of a later replay that passes none), so there is no copy; the caller's buffer
// must hold its value until the step has run (stream order).  Every workgroup fits the device
// at once (occupancy is checked at creation) and every cross-workgroup wait is bounded.
float* LayerDecodeRuntime::replay(const float* hidden, hipStream_t stream) {
    if (replay_count_ >= capacity_ - start_position_) bad_state("flux native decode: fixed-capacity state is exhausted");
    check_hip(hipSetDevice(device_), "hipSetDevice");
    check_host_error();
    if (pending_ && stream != last_stream_) {
        check_hip(hipStreamWaitEvent(stream, completion_, 0), "ordering consecutive replays");
        ++replay_commands_;
    }
    DecodeArgs args = args_;
    if (hidden != nullptr) {
        args.hidden_in = hidden;
        args.hidden_save = input_hidden_;
    }
    check_hip(launch_fused_decode(args, grid_, stream, false), "launching layer step");
    ++replay_kernels_;
    ++replay_commands_;
    check_hip(hipEventRecord(completion_, stream), "recording replay completion");
    last_stream_ = stream;
    pending_ = true;
    ++replay_count_;
    return output_;
}

void LayerDecodeRuntime::reset(const float* hidden, const float* key_source, const float* value_source,
                               int64_t source_length, int64_t position, hipStream_t stream) {
    validate_state(hidden, key_source, value_source, source_length, position);
    check_hip(hipSetDevice(device_), "hipSetDevice");
    if (pending_) {
        check_hip(counted_event_sync(completion_), "waiting to reset runtime");
        pending_ = false;
    }
    initialize_state(hidden, key_source, value_source, source_length, position, stream, true);
    check_hip(hipMemsetAsync(error_, 0, sizeof(int32_t), stream), "clearing error word");
    check_hip(counted_stream_sync(stream), "resetting runtime state");
    *host_error_ = 0;
    start_position_ = position;
    replay_count_ = 0;
}

int64_t LayerDecodeRuntime::position() {
    check_hip(hipSetDevice(device_), "hipSetDevice");
    if (pending_) check_hip(counted_event_sync(completion_), "waiting to inspect device position");
    check_host_error();
    int64_t result = -1;
    check_hip(counted_memcpy(&result, position_, sizeof(result), hipMemcpyDeviceToHost), "reading device position");
    return result;
}

void LayerDecodeRuntime::replay_launches(int64_t* kernels, int64_t* commands) const {
    *kernels = replay_kernels_;
    *commands = replay_commands_;
}

void LayerDecodeRuntime::buffers(flux_layer_decode_buffers* out) const {
    std::memset(out, 0, sizeof(*out));
    out->input_hidden = input_hidden_;
    out->output = output_;
    out->key_cache = key_cache_;
    out->value_cache = value_cache_;
    out->position = position_;
    out->workspace = ll_;
    out->capacity = capacity_;
    out->workspace_bytes = static_cast<int64_t>(ll_bytes_);
}

}  // namespace flux
