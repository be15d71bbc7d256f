// gfx950 decode kernels for the SmolLM2 FP32 batch-1 token loop.
//
// One decode token is the reference's run_body (csrc/native_decode_runtime/
// native_decode_runtime_cuda.cu:1042-1098): embedding, 30 x decoder layer
// (:192-310), final RMSNorm, tied LM head, greedy argmax with device-side state
// update (csrc/greedy_generation/greedy_generation_cuda.cu:39-95).
//
// MI355X design.  Instead of ~10 launches per layer, the whole token runs in one
// persistent kernel: one 512-thread workgroup per CU, every workgroup owning
// fixed slices of every phase.  Phases exchange their (small) vectors through
// "LL" words: 64-bit stores holding {float value, 32-bit epoch}, written and
// polled with agent-scope relaxed atomics, so a consumer's poll *is* the data
// read and no separate flag/fence round trip is needed.  Weight slices and K/V
// chunks of a phase are loaded into registers before the phase polls its input,
// so HBM streaming overlaps the cross-CU dependency wait.
//
// Per layer the phases are
//   A  norm(h) -> packed QKV GEMV -> RoPE(q,k) -> K/V cache write   (480 waves)
//   B  split-K GQA attention partials, one (KV head, position chunk) per WG
//   B2 merge partials per query head                                 (9 WGs)
//   C  o_proj GEMV + residual                                        (576 waves)
//   D  norm(r) -> packed gate/up GEMV -> SwiGLU                      (1536 waves)
//   E  down GEMV + residual                                          (576 waves)
// and per token a final norm -> LM head -> exact lowest-index argmax.
//
// The same phase bodies are instantiated with plain-memory inputs/outputs for the
// isolated per-kernel launchers used by tests and the per-kernel benchmark.

#include "flux_common.h"
#include "flux_kernels.h"

#include <cfloat>
#include <cmath>

namespace flux {
namespace {

constexpr int kThreads = 512;
constexpr int kWavesPerWG = kThreads / kWave;
constexpr int kPosSlots = kThreads / 16;  // attention: 16 lanes (4 dims each) per position
constexpr int kAttnMaxIter = 8;           // positions per WG <= kPosSlots * kAttnMaxIter = 256
constexpr int kLmBatch = 8;
constexpr uint64_t kTimeoutTicks = 20ull * 1000 * 1000;  // 200 ms of the 100 MHz wall clock

// ---------------------------------------------------------------------------
// LL word helpers.
__device__ __forceinline__ uint64_t ll_pack(float v, uint32_t epoch) {
    return (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(v);
}

__device__ __forceinline__ void ll_store(uint64_t* p, float v, uint32_t epoch) {
    __hip_atomic_store(p, ll_pack(v, epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t ll_load(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Bounded waiting.  A workgroup whose wait exceeds the timeout records an error
// and stops waiting for the rest of the launch, so a bug can never hang the GPU.
struct WaitCtx {
    int* abort;        // LDS flag shared by the workgroup
    int32_t* error;    // global error word
};

__device__ __noinline__ void ll_timeout(int* abort, int32_t* error) {
    *abort = 1;
    __hip_atomic_store(error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int N>
__device__ __forceinline__ void ll_fetch(const uint64_t* __restrict__ base, const int (&idx)[N], uint32_t epoch,
                                         const WaitCtx& w, float (&out)[N]) {
    uint64_t word[N];
#pragma unroll
    for (int j = 0; j < N; ++j) word[j] = ll_load(base + idx[j]);
    bool ready = true;
#pragma unroll
    for (int j = 0; j < N; ++j) ready &= static_cast<uint32_t>(word[j] >> 32) == epoch;
    if (!ready) {
        const uint64_t start = wall_clock64();
        while (true) {
            if (*w.abort) break;
            __builtin_amdgcn_s_sleep(1);
            ready = true;
#pragma unroll
            for (int j = 0; j < N; ++j) {
                if (static_cast<uint32_t>(word[j] >> 32) != epoch) word[j] = ll_load(base + idx[j]);
                ready &= static_cast<uint32_t>(word[j] >> 32) == epoch;
            }
            if (ready) break;
            if (wall_clock64() - start > kTimeoutTicks) {
                ll_timeout(w.abort, w.error);
                break;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < N; ++j) out[j] = __uint_as_float(static_cast<uint32_t>(word[j]));
}

// ---------------------------------------------------------------------------
// Input/output policies: plain memory (isolated launches) or LL words (fused).
struct PlainIn {
    const float* p;
    template <int N>
    __device__ __forceinline__ void fetch(const int (&idx)[N], float (&out)[N]) const {
#pragma unroll
        for (int j = 0; j < N; ++j) out[j] = p[idx[j]];
    }
};

struct LLIn {
    const uint64_t* p;
    uint32_t epoch;
    WaitCtx w;
    template <int N>
    __device__ __forceinline__ void fetch(const int (&idx)[N], float (&out)[N]) const {
        ll_fetch<N>(p, idx, epoch, w, out);
    }
};

struct PlainOut {
    float* p;
    __device__ __forceinline__ void put(int i, float v) const { p[i] = v; }
};

struct LLOut {
    uint64_t* p;
    uint32_t epoch;
    __device__ __forceinline__ void put(int i, float v) const { ll_store(p + i, v, epoch); }
};

template <class In>
__device__ __forceinline__ void fetch_slice576(const In& in, int lane, float (&v)[9]) {
    int idx[9];
#pragma unroll
    for (int j = 0; j < 9; ++j) idx[j] = slice576_index(lane, j);
    in.fetch(idx, v);
}

template <class In>
__device__ __forceinline__ float fetch_one(const In& in, int i) {
    int idx[1] = {i};
    float v[1];
    in.fetch(idx, v);
    return v[0];
}

// Normalised 576-slice x = w * (h * inv_rms) with the sum of squares over the
// whole vector (wave reduction, identical in every lane).
__device__ __forceinline__ void norm_slice(const float (&h)[9], const float* __restrict__ weight, float eps,
                                           int lane, float (&x)[9]) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 9; ++j) ss = fmaf(h[j], h[j], ss);
    ss = wave_sum(ss);
    const float inv = rms_inverse(ss, kHidden, eps);
#pragma unroll
    for (int j = 0; j < 9; ++j) x[j] = weight[slice576_index(lane, j)] * (h[j] * inv);
}

// RoPE with HF rounding: each product rounded, then one add (no contraction),
// as packed_qkv_rope_cache_cuda.cu:40-48 (__fmul_rn/__fadd_rn) requires.
#pragma clang fp contract(off)
__device__ __forceinline__ float rope_first(float x, float paired, float c, float s) {
    const float a = x * c;
    const float b = (-paired) * s;
    return a + b;
}
__device__ __forceinline__ float rope_second(float x, float paired, float c, float s) {
    const float a = x * c;
    const float b = paired * s;
    return a + b;
}
#pragma clang fp contract(fast)

// ---------------------------------------------------------------------------
// Phase A: norm -> QKV GEMV (+RoPE) -> outputs.  Unit u pairs rows (d, d+32) of
// one 64-row head so RoPE stays inside the wave.  Units: 15 heads x 32 = 480.
struct QkvUnitWeights {
    float w0[9];
    float w1[9];
};

__device__ __forceinline__ void qkv_unit_rows(int unit, int& head, int& d, int& r0, int& r1) {
    head = unit >> 5;
    d = unit & 31;
    r0 = head * kHeadDim + d;
    r1 = r0 + 32;
}

__device__ __forceinline__ void qkv_load(const float* __restrict__ qkv_w, int unit, int lane, QkvUnitWeights& w) {
    int head, d, r0, r1;
    qkv_unit_rows(unit, head, d, r0, r1);
    load_row576(qkv_w + static_cast<int64_t>(r0) * kHidden, lane, w.w0);
    load_row576(qkv_w + static_cast<int64_t>(r1) * kHidden, lane, w.w1);
}

// Computes the unit's two rows and routes them: q -> q_out[h*64+d], k -> cache
// (and kv_out), v -> cache (and kv_out).  Lane 0 writes.
template <class QOut>
__device__ __forceinline__ void qkv_finish(const QkvUnitWeights& w, const float (&x)[9], int unit, int lane,
                                           const float* __restrict__ cos_row, const float* __restrict__ sin_row,
                                           float* __restrict__ key_row_base, float* __restrict__ value_row_base,
                                           int64_t head_stride, const QOut& out) {
    int head, d, r0, r1;
    qkv_unit_rows(unit, head, d, r0, r1);
    const float a = wave_sum(dot_lane<9>(x, w.w0));
    const float b = wave_sum(dot_lane<9>(x, w.w1));
    if (lane != 0) return;
    float lo, hi;
    if (head < kQHeads + kKVHeads) {
        lo = rope_first(a, b, cos_row[d], sin_row[d]);
        hi = rope_second(b, a, cos_row[d + 32], sin_row[d + 32]);
    } else {
        lo = a;
        hi = b;
    }
    if (head >= kQHeads) {
        const bool is_key = head < kQHeads + kKVHeads;
        const int g = is_key ? head - kQHeads : head - kQHeads - kKVHeads;
        float* row = (is_key ? key_row_base : value_row_base) + g * head_stride;
        // Write-through (agent scope) so later tokens on other XCDs read it from memory.
        __hip_atomic_store(row + d, lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(row + d + 32, hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    out.put(r0, lo);
    out.put(r1, hi);
}

// ---------------------------------------------------------------------------
// Phase B: attention partial for (KV group g, chunk c) over positions
// [begin, end).  Positions < `current` come from the cache (prefetched before the
// query is available); position `current` (if inside) comes from the new K/V.
// Thread t: position slot t/16, dims 4*(t%16)..+3.  Output per query head:
// o[64] (unnormalised), m, l.
struct AttnChunk {
    float4 k[kAttnMaxIter];
    float4 v[kAttnMaxIter];
};

__device__ __forceinline__ void attn_prefetch(const float* __restrict__ key_cache_g, const float* __restrict__ value_cache_g,
                                              int64_t begin, int64_t end, int64_t current, AttnChunk& ch) {
    const int slot = threadIdx.x >> 4;
    const int quad = threadIdx.x & 15;
#pragma unroll
    for (int i = 0; i < kAttnMaxIter; ++i) {
        const int64_t pos = begin + slot + static_cast<int64_t>(kPosSlots) * i;
        if (pos < end && pos < current) {
            ch.k[i] = *reinterpret_cast<const float4*>(key_cache_g + pos * kHeadDim + 4 * quad);
            ch.v[i] = *reinterpret_cast<const float4*>(value_cache_g + pos * kHeadDim + 4 * quad);
        } else {
            ch.k[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            ch.v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
}

// q4[h] = query dims of this thread for the 3 heads; knew/vnew = dims of the new row.
// red: LDS scratch of kWavesPerWG * kGroup * 66 floats.
template <class POut>
__device__ __forceinline__ void attn_compute(AttnChunk& ch, const float4 (&q4)[kGroup], float4 knew, float4 vnew,
                                             int64_t begin, int64_t end, int64_t current, float scale,
                                             float* red, const POut& out) {
    const int slot = threadIdx.x >> 4;
    const int quad = threadIdx.x & 15;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    float s[kGroup][kAttnMaxIter];
    float m[kGroup];
#pragma unroll
    for (int h = 0; h < kGroup; ++h) m[h] = -INFINITY;
#pragma unroll
    for (int i = 0; i < kAttnMaxIter; ++i) {
        const int64_t pos = begin + slot + static_cast<int64_t>(kPosSlots) * i;
        const bool valid = pos < end;
        if (pos == current) {
            ch.k[i] = knew;
            ch.v[i] = vnew;
        }
#pragma unroll
        for (int h = 0; h < kGroup; ++h) {
            float part = q4[h].x * ch.k[i].x;
            part = fmaf(q4[h].y, ch.k[i].y, part);
            part = fmaf(q4[h].z, ch.k[i].z, part);
            part = fmaf(q4[h].w, ch.k[i].w, part);
            const float dot = group_sum<16>(part);
            s[h][i] = valid ? dot * scale : -INFINITY;
            m[h] = fmaxf(m[h], s[h][i]);
        }
    }
    // Max over the 4 slots of this wave, then over waves.
#pragma unroll
    for (int h = 0; h < kGroup; ++h) {
        m[h] = fmaxf(m[h], __shfl_xor(m[h], 16, kWave));
        m[h] = fmaxf(m[h], __shfl_xor(m[h], 32, kWave));
    }
    float* red_m = red;                                // [waves][kGroup]
    float* red_l = red + kWavesPerWG * kGroup;         // [waves][kGroup]
    float* red_o = red + 2 * kWavesPerWG * kGroup;     // [waves][kGroup][64]
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < kGroup; ++h) red_m[wave * kGroup + h] = m[h];
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < kGroup; ++h) {
        float mm = red_m[h];
        for (int w = 1; w < kWavesPerWG; ++w) mm = fmaxf(mm, red_m[w * kGroup + h]);
        m[h] = mm;
    }
    float l[kGroup];
    float4 o[kGroup];
#pragma unroll
    for (int h = 0; h < kGroup; ++h) {
        l[h] = 0.0f;
        o[h] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (m[h] == -INFINITY) continue;
#pragma unroll
        for (int i = 0; i < kAttnMaxIter; ++i) {
            const float p = s[h][i] == -INFINITY ? 0.0f : expf(s[h][i] - m[h]);
            l[h] += p;
            o[h].x = fmaf(p, ch.v[i].x, o[h].x);
            o[h].y = fmaf(p, ch.v[i].y, o[h].y);
            o[h].z = fmaf(p, ch.v[i].z, o[h].z);
            o[h].w = fmaf(p, ch.v[i].w, o[h].w);
        }
    }
#pragma unroll
    for (int h = 0; h < kGroup; ++h) {
#pragma unroll
        for (int off = 16; off <= 32; off <<= 1) {
            l[h] += __shfl_xor(l[h], off, kWave);
            o[h].x += __shfl_xor(o[h].x, off, kWave);
            o[h].y += __shfl_xor(o[h].y, off, kWave);
            o[h].z += __shfl_xor(o[h].z, off, kWave);
            o[h].w += __shfl_xor(o[h].w, off, kWave);
        }
    }
    if (lane < 16) {
#pragma unroll
        for (int h = 0; h < kGroup; ++h) {
            float* dst = red_o + (wave * kGroup + h) * kHeadDim + 4 * quad;
            dst[0] = o[h].x; dst[1] = o[h].y; dst[2] = o[h].z; dst[3] = o[h].w;
            if (lane == 0) red_l[wave * kGroup + h] = l[h];
        }
    }
    __syncthreads();
    // Threads 0..191 finish (head h = t/64, dim d = t%64); thread t%64==0 also m,l.
    if (threadIdx.x < kGroup * kHeadDim) {
        const int h = threadIdx.x >> 6;
        const int dim = threadIdx.x & 63;
        float acc = 0.0f;
        float lsum = 0.0f;
        for (int w = 0; w < kWavesPerWG; ++w) {
            acc += red_o[(w * kGroup + h) * kHeadDim + dim];
            lsum += red_l[w * kGroup + h];
        }
        out.put(h, dim, acc);
        if (dim == 0) {
            out.put(h, kHeadDim, m[h]);
            out.put(h, kHeadDim + 1, lsum);
        }
    }
    __syncthreads();
}

// Partial output addressing: partial (g, c) has kGroup * 66 slots.
struct PartialPlainOut {
    float* p;
    __device__ __forceinline__ void put(int h, int j, float v) const { p[h * (kHeadDim + 2) + j] = v; }
};
struct PartialLLOut {
    uint64_t* p;
    uint32_t epoch;
    __device__ __forceinline__ void put(int h, int j, float v) const { ll_store(p + h * (kHeadDim + 2) + j, v, epoch); }
};

// Phase B2: merge `chunks` partials of one query head.  Wave w handles partials
// c = w, w+8, ...; lane = dim.  Returns (in lane-dim of thread < 64) the
// normalised output via `out.put(dim, value)`.
template <class In, class Out>
__device__ __forceinline__ void merge_head(const In& in, int chunks, int64_t partial_stride, float* red,
                                           const Out& out) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    float M = -INFINITY, L = 0.0f, O = 0.0f;
    for (int c = wave; c < chunks; c += kWavesPerWG) {
        const int base = static_cast<int>(c * partial_stride);
        const int idx[3] = {base + lane, base + kHeadDim, base + kHeadDim + 1};
        float v[3];
        in.fetch(idx, v);
        const float mc = v[1];
        if (mc == -INFINITY) continue;
        const float nm = fmaxf(M, mc);
        const float a = M == -INFINITY ? 0.0f : expf(M - nm);
        const float b = expf(mc - nm);
        O = O * a + v[0] * b;
        L = L * a + v[2] * b;
        M = nm;
    }
    float* red_m = red;
    float* red_l = red + kWavesPerWG;
    float* red_o = red + 2 * kWavesPerWG;
    red_o[wave * kHeadDim + lane] = O;
    if (lane == 0) {
        red_m[wave] = M;
        red_l[wave] = L;
    }
    __syncthreads();
    if (threadIdx.x < kHeadDim) {
        float mm = -INFINITY;
        for (int w = 0; w < kWavesPerWG; ++w) mm = fmaxf(mm, red_m[w]);
        float acc = 0.0f, lsum = 0.0f;
        for (int w = 0; w < kWavesPerWG; ++w) {
            if (red_m[w] == -INFINITY) continue;
            const float f = expf(red_m[w] - mm);
            acc += red_o[w * kHeadDim + threadIdx.x] * f;
            lsum += red_l[w] * f;
        }
        out.put(threadIdx.x, acc / lsum);
    }
    __syncthreads();
}

// Chunking of the attended positions [0, L) across `chunks` workgroups.
__device__ __forceinline__ void chunk_range(int64_t attended, int chunks, int c, int64_t& begin, int64_t& end) {
    const int64_t per = (attended + chunks - 1) / chunks;
    begin = per * c;
    end = begin + per < attended ? begin + per : attended;
    if (begin > end) begin = end;
}

// ---------------------------------------------------------------------------
// LM head + argmax: rows [row0, row1) for one wave, batches of kLmBatch rows.
template <class LogitsOut>
__device__ __forceinline__ void lm_rows(const float* __restrict__ lm_head, const float (&x)[9], int64_t row0, int64_t row1,
                                        int lane, const LogitsOut& logits, float& best_v, int64_t& best_i) {
    for (int64_t base = row0; base < row1; base += kLmBatch) {
        float w[kLmBatch][9];
#pragma unroll
        for (int r = 0; r < kLmBatch; ++r) {
            const int64_t row = base + r < row1 ? base + r : row1 - 1;
            load_row576(lm_head + row * kHidden, lane, w[r]);
        }
#pragma unroll
        for (int r = 0; r < kLmBatch; ++r) {
            const float v = wave_sum(dot_lane<9>(x, w[r]));
            const int64_t row = base + r;
            if (row < row1) {
                if (lane == 0) logits.put(row, v);
                if (argmax_precedes(v, row, best_v, best_i)) {
                    best_v = v;
                    best_i = row;
                }
            }
        }
    }
}

struct LogitsPlainOut {
    float* p;
    __device__ __forceinline__ void put(int64_t i, float v) const { p[i] = v; }
};

// Workgroup argmax reduction of per-wave (value, index); result valid in thread 0.
__device__ __forceinline__ void wg_argmax(float& v, int64_t& i, float* red_v, int64_t* red_i) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    if (lane == 0) {
        red_v[wave] = v;
        red_i[wave] = i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kWavesPerWG; ++w) {
            if (argmax_precedes(red_v[w], red_i[w], v, i)) {
                v = red_v[w];
                i = red_i[w];
            }
        }
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// LL arena layout (uint64 words), two parities (layer parity / token parity).
struct LLLayout {
    static constexpr int kQkv = 0;                                        // 960
    static constexpr int kAttnMerged = 1024;                              // 576
    static constexpr int kResid = 1024 + 640;                             // 576 (r)
    static constexpr int kSwiglu = 1024 + 1280;                           // 1536
    static constexpr int kHidden = 1024 + 1280 + 1536;                    // 576 (h)
    static constexpr int kArgmax = kHidden + 640;                         // 2 * 1024
    static constexpr int kPartials = kArgmax + 2048;                      // 3 * chunks * 3 * 66
    static constexpr int kPartialWords = kKVHeads * kMaxAttnChunks * kGroup * (kHeadDim + 2);
    static constexpr int kParity = kPartials + kPartialWords + 64;
    static constexpr int kTotal = 2 * kParity;
};

__device__ __forceinline__ uint32_t epoch_of(uint32_t token_counter, int stage) {
    // stage 0..29 = layers, 30 = argmax.  Never 0 for any token (memory starts zeroed).
    return token_counter * 32u + static_cast<uint32_t>(stage) + 1u;
}

// ---------------------------------------------------------------------------
// The fused persistent decode kernel: `args.steps` greedy tokens per launch.
__global__ void __launch_bounds__(kThreads, 1) fused_decode_kernel(DecodeArgs args) {
    __shared__ int abort_flag;
    __shared__ float red[kWavesPerWG * kGroup * (kHeadDim + 2)];
    __shared__ int64_t red_i[kWavesPerWG];
    __shared__ float red_v[kWavesPerWG];
    __shared__ int64_t token_shared;
    extern __shared__ float occupancy_pad[];  // dynamic LDS only to keep one WG per CU
    (void)occupancy_pad;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int G = gridDim.x;
    const int wg = blockIdx.x;
    const int gw = wave * G + wg;        // global wave id, interleaved across CUs
    const int TW = G * kWavesPerWG;      // total waves
    const int chunks = G / kKVHeads < kMaxAttnChunks ? G / kKVHeads : kMaxAttnChunks;
    const int64_t cap = args.capacity;
    const int64_t head_stride = cap * kHeadDim;
    const int64_t layer_stride = kKVHeads * head_stride;
    const int64_t partial_stride = kGroup * (kHeadDim + 2);

    if (threadIdx.x == 0) abort_flag = 0;
    const uint32_t counter0 = *args.token_counter;
    int64_t token = *args.input_token;
    int64_t position = *args.position;
    int64_t step = *args.generation_step;
    __syncthreads();
    const WaitCtx wctx{&abort_flag, args.error};

    for (int t = 0; t < args.steps; ++t) {
        __syncthreads();
        const bool stop = abort_flag != 0;
        __syncthreads();
        if (stop) break;
        if (position < 0 || position >= cap) {
            if (wg == 0 && threadIdx.x == 0)
                __hip_atomic_store(args.error, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        const uint32_t counter = counter0 + static_cast<uint32_t>(t);
        const int64_t attended = position + 1;
        const float* cos_row = args.rope_cos + position * kHeadDim;
        const float* sin_row = args.rope_sin + position * kHeadDim;
        const bool token_ok = token >= 0 && token < args.vocab;
        const float* emb_row = args.embedding + (token_ok ? token : 0) * kHidden;

        for (int layer = 0; layer < kLayers; ++layer) {
            const LayerWeights Lw = args.layers[layer];
            const uint32_t ep = epoch_of(counter, layer);
            const uint32_t ep_prev = epoch_of(counter, layer - 1);  // only used for layer > 0
            uint64_t* ll = args.ll + (layer & 1) * LLLayout::kParity;
            const uint64_t* ll_prev = args.ll + ((layer + 1) & 1) * LLLayout::kParity;
            float* key_layer = args.key_cache + layer * layer_stride;
            float* value_layer = args.value_cache + layer * layer_stride;

            // ---- A: QKV ----
            for (int unit = gw; unit < kQKV / 2; unit += TW) {
                QkvUnitWeights w;
                qkv_load(Lw.qkv, unit, lane, w);
                float h[9], x[9];
                if (layer == 0) {
#pragma unroll
                    for (int j = 0; j < 9; ++j) h[j] = token_ok ? emb_row[slice576_index(lane, j)] : 0.0f;
                } else {
                    fetch_slice576(LLIn{ll_prev + LLLayout::kHidden, ep_prev, wctx}, lane, h);
                }
                norm_slice(h, Lw.input_norm, Lw.eps, lane, x);
                qkv_finish(w, x, unit, lane, cos_row, sin_row, key_layer + position * kHeadDim,
                           value_layer + position * kHeadDim, head_stride, LLOut{ll + LLLayout::kQkv, ep});
            }

            // ---- B: attention partials ----
            if (wg < kKVHeads * chunks) {
                const int g = wg % kKVHeads;
                const int c = wg / kKVHeads;
                int64_t begin, end;
                chunk_range(attended, chunks, c, begin, end);
                AttnChunk ch;
                attn_prefetch(key_layer + g * head_stride, value_layer + g * head_stride, begin, end, position, ch);
                const int quad = threadIdx.x & 15;
                const LLIn qin{ll + LLLayout::kQkv, ep, wctx};
                float4 q4[kGroup];
#pragma unroll
                for (int h = 0; h < kGroup; ++h) {
                    const int base = (g * kGroup + h) * kHeadDim + 4 * quad;
                    const int idx[4] = {base, base + 1, base + 2, base + 3};
                    float v[4];
                    qin.fetch(idx, v);
                    q4[h] = make_float4(v[0], v[1], v[2], v[3]);
                }
                float4 knew = make_float4(0.f, 0.f, 0.f, 0.f), vnew = knew;
                if (position >= begin && position < end) {
                    const int kb = kQHeads * kHeadDim + g * kHeadDim + 4 * quad;
                    const int vb = (kQHeads + kKVHeads) * kHeadDim + g * kHeadDim + 4 * quad;
                    const int idx[8] = {kb, kb + 1, kb + 2, kb + 3, vb, vb + 1, vb + 2, vb + 3};
                    float v[8];
                    qin.fetch(idx, v);
                    knew = make_float4(v[0], v[1], v[2], v[3]);
                    vnew = make_float4(v[4], v[5], v[6], v[7]);
                }
                attn_compute(ch, q4, knew, vnew, begin, end, position, Lw.scale, red,
                             PartialLLOut{ll + LLLayout::kPartials + (g * chunks + c) * partial_stride, ep});
            }

            // ---- B2: merge per query head ----
            if (wg < kQHeads) {
                const int h = wg;
                const int g = h / kGroup;
                const int hh = h % kGroup;
                const LLIn pin{ll + LLLayout::kPartials + g * chunks * partial_stride + hh * (kHeadDim + 2), ep, wctx};
                merge_head(pin, chunks, partial_stride, red, LLOut{ll + LLLayout::kAttnMerged + h * kHeadDim, ep});
            }

            // ---- C: o_proj + residual ----
            for (int row = gw; row < kHidden; row += TW) {
                float w[9], a[9];
                load_row576(Lw.o_proj + static_cast<int64_t>(row) * kHidden, lane, w);
                fetch_slice576(LLIn{ll + LLLayout::kAttnMerged, ep, wctx}, lane, a);
                const float dot = wave_sum(dot_lane<9>(a, w));
                if (lane == 0) {
                    const float resid = layer == 0 ? (token_ok ? emb_row[row] : 0.0f)
                                                   : fetch_one(LLIn{ll_prev + LLLayout::kHidden, ep_prev, wctx}, row);
                    ll_store(ll + LLLayout::kResid + row, resid + dot, ep);
                }
            }

            // ---- D: norm -> gate/up -> SwiGLU ----
            for (int j = gw; j < kInter; j += TW) {
                float wg_[9], wu[9], r[9], x[9];
                load_row576(Lw.gate_up + static_cast<int64_t>(j) * kHidden, lane, wg_);
                load_row576(Lw.gate_up + static_cast<int64_t>(kInter + j) * kHidden, lane, wu);
                fetch_slice576(LLIn{ll + LLLayout::kResid, ep, wctx}, lane, r);
                norm_slice(r, Lw.post_norm, Lw.eps, lane, x);
                const float gsum = wave_sum(dot_lane<9>(x, wg_));
                const float usum = wave_sum(dot_lane<9>(x, wu));
                if (lane == 0) ll_store(ll + LLLayout::kSwiglu + j, silu(gsum) * usum, ep);
            }

            // ---- E: down + residual ----
            for (int row = gw; row < kHidden; row += TW) {
                float w[24], s[24];
                load_row1536(Lw.down + static_cast<int64_t>(row) * kInter, lane, w);
                int idx[24];
#pragma unroll
                for (int j = 0; j < 24; ++j) idx[j] = slice1536_index(lane, j);
                LLIn{ll + LLLayout::kSwiglu, ep, wctx}.fetch(idx, s);
                const float dot = wave_sum(dot_lane<24>(s, w));
                if (lane == 0) {
                    const float resid = fetch_one(LLIn{ll + LLLayout::kResid, ep, wctx}, row);
                    ll_store(ll + LLLayout::kHidden + row, resid + dot, ep);
                }
            }
        }

        // ---- final norm -> LM head -> argmax ----
        {
            const uint32_t ep_last = epoch_of(counter, kLayers - 1);
            const uint32_t ep_arg = epoch_of(counter, kLayers);
            const uint64_t* ll_last = args.ll + ((kLayers - 1) & 1) * LLLayout::kParity;
            uint64_t* ll_arg = args.ll + (t & 1) * LLLayout::kParity + LLLayout::kArgmax;
            const int64_t per = (args.vocab + TW - 1) / TW;
            const int64_t row0 = per * gw < args.vocab ? per * gw : args.vocab;
            const int64_t row1 = row0 + per < args.vocab ? row0 + per : args.vocab;
            float h[9], x[9];
            fetch_slice576(LLIn{ll_last + LLLayout::kHidden, ep_last, wctx}, lane, h);
            norm_slice(h, args.final_norm, args.final_eps, lane, x);
            float best_v = -INFINITY;
            int64_t best_i = INT64_MAX;
            lm_rows(args.lm_head, x, row0, row1, lane, LogitsPlainOut{args.logits}, best_v, best_i);
            wg_argmax(best_v, best_i, red_v, red_i);
            // Release this token's K/V cache rows (every wave) before signalling the argmax.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            __syncthreads();
            if (threadIdx.x == 0) {
                ll_store(ll_arg + 2 * wg, best_v, ep_arg);
                ll_store(ll_arg + 2 * wg + 1, __int_as_float(static_cast<int>(best_i)), ep_arg);
            }
            // Every workgroup reduces all G partials (thread t < G reads partial t).
            float v = -INFINITY;
            int64_t i = INT64_MAX;
            if (threadIdx.x < G) {
                const int idx[2] = {2 * static_cast<int>(threadIdx.x), 2 * static_cast<int>(threadIdx.x) + 1};
                float pv[2];
                LLIn{ll_arg, ep_arg, wctx}.fetch(idx, pv);
                v = pv[0];
                i = static_cast<int64_t>(__float_as_int(pv[1]));
            }
            // wave-level then workgroup-level argmax
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                const float ov = __shfl_xor(v, off, kWave);
                const int64_t oi = __shfl_xor(i, off, kWave);
                if (argmax_precedes(ov, oi, v, i)) {
                    v = ov;
                    i = oi;
                }
            }
            wg_argmax(v, i, red_v, red_i);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            if (threadIdx.x == 0) token_shared = (i >= 0 && i < args.vocab) ? i : 0;
            __syncthreads();
            const int64_t next = token_shared;
            if (wg == 0 && threadIdx.x == 0) {
                *args.input_token = next;
                if (step >= 0 && step < args.generated_capacity) args.generated[step] = next;
                *args.generation_step = step + 1;
                *args.position = attended;
                *args.cache_length = attended;
            }
            token = next;
            position = attended;
            step += 1;
        }
    }
    __syncthreads();
    if (wg == 0 && threadIdx.x == 0) *args.token_counter = counter0 + static_cast<uint32_t>(args.steps);
}

// ---------------------------------------------------------------------------
// Isolated launchers (tests, per-kernel benchmark): same phase bodies, plain I/O.

__global__ void __launch_bounds__(kThreads) qkv_rope_cache_kernel(const float* hidden, const float* norm_w, float eps,
                                                                  const float* qkv_w, const float* cos_table,
                                                                  const float* sin_table, const int64_t* position_ptr,
                                                                  int64_t capacity, float* key_cache, float* value_cache,
                                                                  float* q_out) {
    const int lane = threadIdx.x & 63;
    const int gw = (threadIdx.x >> 6) * gridDim.x + blockIdx.x;
    const int TW = gridDim.x * kWavesPerWG;
    const int64_t position = *position_ptr;
    if (position < 0 || position >= capacity) return;
    for (int unit = gw; unit < kQKV / 2; unit += TW) {
        QkvUnitWeights w;
        qkv_load(qkv_w, unit, lane, w);
        float h[9], x[9];
        fetch_slice576(PlainIn{hidden}, lane, h);
        norm_slice(h, norm_w, eps, lane, x);
        qkv_finish(w, x, unit, lane, cos_table + position * kHeadDim, sin_table + position * kHeadDim,
                   key_cache + position * kHeadDim, value_cache + position * kHeadDim, capacity * kHeadDim,
                   PlainOut{q_out});
    }
}

__global__ void __launch_bounds__(kThreads) attn_partial_kernel(const float* q_packed, const float* key_cache,
                                                                const float* value_cache, const int64_t* position_ptr,
                                                                int64_t capacity, float scale, int chunks,
                                                                float* partials) {
    __shared__ float red[kWavesPerWG * kGroup * (kHeadDim + 2)];
    const int g = blockIdx.x % kKVHeads;
    const int c = blockIdx.x / kKVHeads;
    const int64_t position = *position_ptr;
    if (position < 0 || position >= capacity) return;
    const int64_t attended = position + 1;
    int64_t begin, end;
    chunk_range(attended, chunks, c, begin, end);
    // Every position including the current one is read from the cache here.
    AttnChunk ch;
    attn_prefetch(key_cache + g * capacity * kHeadDim, value_cache + g * capacity * kHeadDim, begin, end, attended, ch);
    const int quad = threadIdx.x & 15;
    float4 q4[kGroup];
#pragma unroll
    for (int h = 0; h < kGroup; ++h)
        q4[h] = *reinterpret_cast<const float4*>(q_packed + (g * kGroup + h) * kHeadDim + 4 * quad);
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    attn_compute(ch, q4, zero, zero, begin, end, /*current=*/-1, scale, red,
                 PartialPlainOut{partials + (g * chunks + c) * kGroup * (kHeadDim + 2)});
}

__global__ void __launch_bounds__(kThreads) attn_merge_kernel(const float* partials, int chunks, float* out) {
    __shared__ float red[2 * kWavesPerWG + kWavesPerWG * kHeadDim];
    const int h = blockIdx.x;
    const int g = h / kGroup;
    const int hh = h % kGroup;
    const int64_t stride = kGroup * (kHeadDim + 2);
    merge_head(PlainIn{partials + g * chunks * stride + hh * (kHeadDim + 2)}, chunks, stride, red,
               PlainOut{out + h * kHeadDim});
}

__global__ void __launch_bounds__(kThreads) linear576_residual_kernel(const float* x, const float* w, const float* residual,
                                                                      float* out, int rows) {
    const int lane = threadIdx.x & 63;
    const int gw = (threadIdx.x >> 6) * gridDim.x + blockIdx.x;
    const int TW = gridDim.x * kWavesPerWG;
    for (int row = gw; row < rows; row += TW) {
        float wr[9], a[9];
        load_row576(w + static_cast<int64_t>(row) * kHidden, lane, wr);
        fetch_slice576(PlainIn{x}, lane, a);
        const float dot = wave_sum(dot_lane<9>(a, wr));
        if (lane == 0) out[row] = residual ? residual[row] + dot : dot;
    }
}

__global__ void __launch_bounds__(kThreads) gate_up_swiglu_kernel(const float* hidden, const float* norm_w, float eps,
                                                                  const float* gate_up, float* out) {
    const int lane = threadIdx.x & 63;
    const int gw = (threadIdx.x >> 6) * gridDim.x + blockIdx.x;
    const int TW = gridDim.x * kWavesPerWG;
    for (int j = gw; j < kInter; j += TW) {
        float wg_[9], wu[9], r[9], x[9];
        load_row576(gate_up + static_cast<int64_t>(j) * kHidden, lane, wg_);
        load_row576(gate_up + static_cast<int64_t>(kInter + j) * kHidden, lane, wu);
        fetch_slice576(PlainIn{hidden}, lane, r);
        if (norm_w != nullptr) {
            norm_slice(r, norm_w, eps, lane, x);
        } else {
#pragma unroll
            for (int q = 0; q < 9; ++q) x[q] = r[q];
        }
        const float gsum = wave_sum(dot_lane<9>(x, wg_));
        const float usum = wave_sum(dot_lane<9>(x, wu));
        if (lane == 0) out[j] = silu(gsum) * usum;
    }
}

__global__ void __launch_bounds__(kThreads) down_residual_kernel(const float* s, const float* w, const float* residual,
                                                                 float* out) {
    const int lane = threadIdx.x & 63;
    const int gw = (threadIdx.x >> 6) * gridDim.x + blockIdx.x;
    const int TW = gridDim.x * kWavesPerWG;
    for (int row = gw; row < kHidden; row += TW) {
        float wr[24], sv[24];
        load_row1536(w + static_cast<int64_t>(row) * kInter, lane, wr);
        int idx[24];
#pragma unroll
        for (int j = 0; j < 24; ++j) idx[j] = slice1536_index(lane, j);
        PlainIn{s}.fetch(idx, sv);
        const float dot = wave_sum(dot_lane<24>(sv, wr));
        if (lane == 0) out[row] = residual ? residual[row] + dot : dot;
    }
}

// LM head over rows with optional final norm; per-WG (value, index) partials.
__global__ void __launch_bounds__(kThreads) lm_head_partial_kernel(const float* hidden, const float* norm_w, float eps,
                                                                   const float* lm_head, int64_t vocab, float* logits,
                                                                   float* part_v, int64_t* part_i) {
    __shared__ float red_v[kWavesPerWG];
    __shared__ int64_t red_i[kWavesPerWG];
    const int lane = threadIdx.x & 63;
    const int gw = (threadIdx.x >> 6) * gridDim.x + blockIdx.x;
    const int TW = gridDim.x * kWavesPerWG;
    const int64_t per = (vocab + TW - 1) / TW;
    const int64_t row0 = per * gw < vocab ? per * gw : vocab;
    const int64_t row1 = row0 + per < vocab ? row0 + per : vocab;
    float h[9], x[9];
    fetch_slice576(PlainIn{hidden}, lane, h);
    if (norm_w != nullptr) {
        norm_slice(h, norm_w, eps, lane, x);
    } else {
#pragma unroll
        for (int q = 0; q < 9; ++q) x[q] = h[q];
    }
    float best_v = -INFINITY;
    int64_t best_i = INT64_MAX;
    lm_rows(lm_head, x, row0, row1, lane, LogitsPlainOut{logits}, best_v, best_i);
    wg_argmax(best_v, best_i, red_v, red_i);
    if (threadIdx.x == 0) {
        part_v[blockIdx.x] = best_v;
        part_i[blockIdx.x] = best_i;
    }
}

// Argmax over n (value, index) candidates (or over raw logits when part_i is
// null), optional greedy state update as greedy_argmax_update_cuda_fp32.
__global__ void __launch_bounds__(kThreads) argmax_finish_kernel(const float* part_v, const int64_t* part_i, int64_t n,
                                                                 int64_t* token, int64_t* generated, int64_t* step,
                                                                 int64_t generated_capacity, int64_t* position,
                                                                 const int64_t* attention_length) {
    __shared__ float red_v[kWavesPerWG];
    __shared__ int64_t red_i[kWavesPerWG];
    float v = -INFINITY;
    int64_t i = INT64_MAX;
    for (int64_t k = threadIdx.x; k < n; k += kThreads) {
        const float cv = part_v[k];
        const int64_t ci = part_i ? part_i[k] : k;
        if (argmax_precedes(cv, ci, v, i)) {
            v = cv;
            i = ci;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off, kWave);
        const int64_t oi = __shfl_xor(i, off, kWave);
        if (argmax_precedes(ov, oi, v, i)) {
            v = ov;
            i = oi;
        }
    }
    wg_argmax(v, i, red_v, red_i);
    if (threadIdx.x == 0) {
        const int64_t selected = i == INT64_MAX ? 0 : i;
        *token = selected;
        if (step != nullptr) {
            const int64_t s = *step;
            if (generated != nullptr && s >= 0 && s < generated_capacity) generated[s] = selected;
            *step = s + 1;
        }
        if (position != nullptr && attention_length != nullptr) *position = *attention_length;
    }
}

// Scalar state installation (no host-pageable async copies, graph-safe):
// input_token = *token_src, position = cache_length = position_value,
// generation_step = step_value, and generated[0] = token when requested.
__global__ void install_state_kernel(const int64_t* token_src, int64_t position_value, int64_t step_value,
                                     int write_generated0, int64_t* input_token, int64_t* position,
                                     int64_t* cache_length, int64_t* step, int64_t* generated) {
    if (threadIdx.x != 0) return;
    const int64_t token = *token_src;
    *input_token = token;
    *position = position_value;
    *cache_length = position_value;
    *step = step_value;
    if (write_generated0) generated[0] = token;
}

__global__ void rmsnorm_rows_kernel(const float* x, const float* w, float* out, int64_t rows, int cols, float eps) {
    __shared__ float red[kWavesPerWG];
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const float* xr = x + row * cols;
        float ss = 0.0f;
        for (int c = threadIdx.x; c < cols; c += blockDim.x) ss = fmaf(xr[c], xr[c], ss);
        ss = wave_sum(ss);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        float total = 0.0f;
        for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) total += red[w];
        const float inv = rms_inverse(total, cols, eps);
        for (int c = threadIdx.x; c < cols; c += blockDim.x) out[row * cols + c] = w[c] * (xr[c] * inv);
        __syncthreads();
    }
}

__global__ void residual_rmsnorm_rows_kernel(const float* hidden, const float* residual, const float* w, float* norm_out,
                                             float* residual_out, int64_t rows, int cols, float eps) {
    __shared__ float red[kWavesPerWG];
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        float ss = 0.0f;
        for (int c = threadIdx.x; c < cols; c += blockDim.x) {
            const float r = hidden[row * cols + c] + residual[row * cols + c];
            residual_out[row * cols + c] = r;
            ss = fmaf(r, r, ss);
        }
        ss = wave_sum(ss);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        float total = 0.0f;
        for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) total += red[w];
        const float inv = rms_inverse(total, cols, eps);
        for (int c = threadIdx.x; c < cols; c += blockDim.x) {
            const float r = hidden[row * cols + c] + residual[row * cols + c];
            norm_out[row * cols + c] = w[c] * (r * inv);
        }
        __syncthreads();
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// Host launchers.

size_t ll_arena_words() { return LLLayout::kTotal; }
int fused_decode_threads() { return kThreads; }
size_t fused_decode_dynamic_lds() { return 96 * 1024; }

int max_attention_positions(int grid) {
    const int chunks = grid / kKVHeads < kMaxAttnChunks ? grid / kKVHeads : kMaxAttnChunks;
    return chunks * kPosSlots * kAttnMaxIter;
}

hipError_t launch_fused_decode(const DecodeArgs& args, int grid, hipStream_t stream) {
    hipLaunchKernelGGL(fused_decode_kernel, dim3(grid), dim3(kThreads), fused_decode_dynamic_lds(), stream, args);
    return hipGetLastError();
}

hipError_t fused_decode_occupancy(int* blocks_per_cu) {
    hipError_t st = hipFuncSetAttribute(reinterpret_cast<const void*>(fused_decode_kernel),
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(fused_decode_dynamic_lds()));
    if (st != hipSuccess) return st;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, reinterpret_cast<const void*>(fused_decode_kernel),
                                                        kThreads, fused_decode_dynamic_lds());
}

hipError_t launch_qkv_rope_cache(const float* hidden, const float* norm_w, float eps, const float* qkv_w,
                                 const float* cos_table, const float* sin_table, const int64_t* position,
                                 int64_t capacity, float* key_cache, float* value_cache, float* q_out, int grid,
                                 hipStream_t stream) {
    hipLaunchKernelGGL(qkv_rope_cache_kernel, dim3(grid), dim3(kThreads), 0, stream, hidden, norm_w, eps, qkv_w,
                       cos_table, sin_table, position, capacity, key_cache, value_cache, q_out);
    return hipGetLastError();
}

hipError_t launch_gqa_decode(const float* q, const float* key_cache, const float* value_cache, const int64_t* position,
                             int64_t capacity, float scale, int chunks, float* partials, float* out,
                             hipStream_t stream) {
    hipLaunchKernelGGL(attn_partial_kernel, dim3(kKVHeads * chunks), dim3(kThreads), 0, stream, q, key_cache,
                       value_cache, position, capacity, scale, chunks, partials);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    hipLaunchKernelGGL(attn_merge_kernel, dim3(kQHeads), dim3(kThreads), 0, stream, partials, chunks, out);
    return hipGetLastError();
}

int gqa_decode_max_positions(int chunks) { return chunks * kPosSlots * kAttnMaxIter; }

hipError_t launch_linear576_residual(const float* x, const float* w, const float* residual, float* out, int rows,
                                     int grid, hipStream_t stream) {
    hipLaunchKernelGGL(linear576_residual_kernel, dim3(grid), dim3(kThreads), 0, stream, x, w, residual, out, rows);
    return hipGetLastError();
}

hipError_t launch_gate_up_swiglu(const float* hidden, const float* norm_w, float eps, const float* gate_up, float* out,
                                 int grid, hipStream_t stream) {
    hipLaunchKernelGGL(gate_up_swiglu_kernel, dim3(grid), dim3(kThreads), 0, stream, hidden, norm_w, eps, gate_up, out);
    return hipGetLastError();
}

hipError_t launch_down_residual(const float* s, const float* w, const float* residual, float* out, int grid,
                                hipStream_t stream) {
    hipLaunchKernelGGL(down_residual_kernel, dim3(grid), dim3(kThreads), 0, stream, s, w, residual, out);
    return hipGetLastError();
}

hipError_t launch_lm_head_argmax(const float* hidden, const float* norm_w, float eps, const float* lm_head,
                                 int64_t vocab, float* logits, float* part_v, int64_t* part_i, int grid,
                                 int64_t* token, hipStream_t stream) {
    hipLaunchKernelGGL(lm_head_partial_kernel, dim3(grid), dim3(kThreads), 0, stream, hidden, norm_w, eps, lm_head,
                       vocab, logits, part_v, part_i);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(kThreads), 0, stream, part_v, part_i,
                       static_cast<int64_t>(grid), token, nullptr, nullptr, int64_t{0}, nullptr, nullptr);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, int64_t n, int64_t* token, int64_t* generated, int64_t* step,
                         int64_t generated_capacity, int64_t* position, const int64_t* attention_length,
                         hipStream_t stream) {
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(kThreads), 0, stream, logits, nullptr, n, token, generated,
                       step, generated_capacity, position, attention_length);
    return hipGetLastError();
}

hipError_t launch_install_state(const int64_t* token_src, int64_t position_value, int64_t step_value,
                                bool write_generated0, int64_t* input_token, int64_t* position, int64_t* cache_length,
                                int64_t* step, int64_t* generated, hipStream_t stream) {
    hipLaunchKernelGGL(install_state_kernel, dim3(1), dim3(64), 0, stream, token_src, position_value, step_value,
                       write_generated0 ? 1 : 0, input_token, position, cache_length, step, generated);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_rows(const float* x, const float* w, float* out, int64_t rows, int cols, float eps,
                               hipStream_t stream) {
    const int grid = static_cast<int>(rows < 4096 ? rows : 4096);
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(grid), dim3(256), 0, stream, x, w, out, rows, cols, eps);
    return hipGetLastError();
}

hipError_t launch_residual_rmsnorm_rows(const float* hidden, const float* residual, const float* w, float* norm_out,
                                        float* residual_out, int64_t rows, int cols, float eps, hipStream_t stream) {
    const int grid = static_cast<int>(rows < 4096 ? rows : 4096);
    hipLaunchKernelGGL(residual_rmsnorm_rows_kernel, dim3(grid), dim3(256), 0, stream, hidden, residual, w, norm_out,
                       residual_out, rows, cols, eps);
    return hipGetLastError();
}

}  // namespace flux
