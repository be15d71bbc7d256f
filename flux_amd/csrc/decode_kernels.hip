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
//      (one chunk per 64 attended positions, at most 85 per KV head)
//   B2 merge partials per query head (36 WGs: query head x 16 dims)
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
#include <mutex>

namespace flux {
namespace {

// threadIdx.x read through an empty asm so that per-lane address arithmetic is
// recomputed where it is used instead of being hoisted out of the token/layer
// loops by LICM; hoisted lane-dependent values otherwise exhaust the VGPR budget
// of the persistent kernel and spill to scratch.
__device__ __forceinline__ unsigned tid_opaque() {
    unsigned t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

constexpr int kThreads = 512;
constexpr int kWavesPerWG = kThreads / kWave;
constexpr int kAttnRows = 224;            // attention rows per workgroup (LDS-resident K/V)
constexpr int kLmBatch = 4;
// A wait that has lasted this long (or its bound, if shorter) starts watching the
// device error word (so one workgroup's timeout ends every other workgroup's wait at
// once instead of each of them timing out in turn) and its own bound: 20 us of the
// 100 MHz wall clock.  Normal exchanges complete in 1-10 us and never reach it, so
// the poll loop of a normal wait does nothing but poll.
constexpr uint64_t kWatchErrorTicks = 2000;

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

// ---------------------------------------------------------------------------
// LL arena layout (uint64 words), two parities (layer parity / token parity).
//
// The vectors every workgroup reads (q/k/v, merged attention, r, SwiGLU output, h,
// argmax candidates) are written in kReplicas copies: the workgroups of XCD x poll
// copy x % kReplicas, so each cache line is polled by the 64 CUs of two XCDs instead
// of all 256.  Sixteen producers share each 128-byte line of a copy; with one copy, a
// 256-reader exchange of such lines took 2.0 us per round on MI355X, with one copy per
// XCD 1.4 us.  Measured per token at ctx 8192: 2 copies 0.461 ms, 4 copies 0.459,
// 8 copies 0.464, 16 copies 0.499 (the stores of more copies cost more than the
// spread polls gain).  The attention partials are read by a few merge workgroups only
// and have one copy.
struct LLLayout {
    static constexpr int kQkv = 0;                                        // 960
    static constexpr int kAttnMerged = 1024;                              // 576
    static constexpr int kResid = 1024 + 640;                             // 576 (r)
    static constexpr int kSwiglu = 1024 + 1280;                           // 1536
    static constexpr int kHidden = 1024 + 1280 + 1536;                    // 576 (h)
    static constexpr int kArgmax = kHidden + 640;                         // 2 * 1024
    static constexpr int kVectorWords = kArgmax + 2048;
    static constexpr int kReplicas = 4;
    // Copies start 32 words (256 bytes) apart beyond the vector block, so that equal
    // offsets of different copies do not fall on the same memory channel.
    static constexpr int kReplicaStride = kVectorWords + 32;
    static constexpr int kPartials = kReplicas * kReplicaStride;          // 3 * chunks * 3 * 66
    static constexpr int kPartialWords = kKVHeads * kMaxAttnChunks * kGroup * (kHeadDim + 2);
    static constexpr int kParity = kPartials + kPartialWords + 64;
    static constexpr int kTotal = 2 * kParity;
};

// Stores v into word i of every copy of a replicated vector (lane r writes copy r);
// v must be the same in lanes 0 .. kReplicas-1.
__device__ __forceinline__ void ll_store_replicas(uint64_t* copy0, int i, float v, uint32_t epoch, int lane) {
    if (lane < LLLayout::kReplicas) ll_store(copy0 + lane * LLLayout::kReplicaStride + i, v, epoch);
}

__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(x));
    return x;
}

// Bounded waiting.  A workgroup whose wait exceeds the limit records an error
// (device word and its host-visible copy) and stops waiting for the rest of the
// launch, so a bug can never hang the GPU; a wait that sees the device error word
// set stops too.  Outputs of such a launch are invalid: the greedy token of every
// step it finishes is written as -1.  The rarely used parts (host word, limit) sit
// in LDS so that the waits keep no extra registers live.
struct WaitShared {
    int32_t* host_error;  // host-visible error word (mapped pinned memory)
    uint64_t limit;       // wait bound in wall-clock ticks
};

struct WaitCtx {
    int* abort;                // LDS flag shared by the workgroup
    int32_t* error;            // device error word
    const WaitShared* shared;  // LDS
    uint64_t watch;            // min(kWatchErrorTicks, bound): when a wait starts checking
};

__device__ __noinline__ void record_error(int32_t* error, int32_t* host_error, int32_t code) {
    __hip_atomic_store(error, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(host_error, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __noinline__ void ll_timeout(int* abort, int32_t* error, const WaitShared* shared) {
    *abort = 1;
    record_error(error, shared->host_error, 1);
}

// true when a wait that has lasted w.watch ticks must stop: the device error word is
// set, or the wait exceeded its bound.
__device__ __forceinline__ bool wait_expired(const WaitCtx& w, uint64_t start) {
    const uint64_t waited = wall_clock64() - start;
    if (waited > w.watch) {
        if (__hip_atomic_load(w.error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
            *w.abort = 1;
            return true;
        }
        if (waited > w.shared->limit) {
            ll_timeout(w.abort, w.error, w.shared);
            return true;
        }
    }
    return false;
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
        // One poll per word in flight, re-issued as soon as it returns stale: polls compete
        // with the producers' stores and with each other at the memory side, so keeping
        // more of them in flight, or sleeping between them, makes the exchange slower.
        const uint64_t start = wall_clock64();
        while (true) {
#pragma unroll
            for (int j = 0; j < N; ++j)
                if (static_cast<uint32_t>(word[j] >> 32) != epoch) word[j] = ll_load(base + idx[j]);
            // The abort and time checks run while the re-polls are in flight.
            if (*w.abort) break;
            if (wait_expired(w, start)) break;
            ready = true;
#pragma unroll
            for (int j = 0; j < N; ++j) ready &= static_cast<uint32_t>(word[j] >> 32) == epoch;
            if (ready) break;
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

// QKV outputs: `v` is the same in every lane; the LL form writes every copy of the
// replicated q/k/v vector (p = copy 0), the plain form writes once from lane 0.
struct QkvPlainOut {
    float* p;
    __device__ __forceinline__ void put(int lane, int i, float v) const {
        if (lane == 0) p[i] = v;
    }
};
struct QkvLLOut {
    uint64_t* p;
    uint32_t epoch;
    __device__ __forceinline__ void put(int lane, int i, float v) const { ll_store_replicas(p, i, v, epoch, lane); }
};

template <class In>
__device__ __forceinline__ void fetch_slice576(const In& in, int lane, float (&v)[9]) {
    int idx[9];
#pragma unroll
    for (int j = 0; j < 9; ++j) idx[j] = slice576_index(lane, j);
    in.fetch(idx, v);
}


// Normalised 576-slice with the norm weights already in registers.
__device__ __forceinline__ void norm_slice_w(const float (&h)[9], const float (&wn)[9], float eps, float (&x)[9]) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 9; ++j) ss = fmaf(h[j], h[j], ss);
    ss = wave_sum_uniform(ss);
    const float inv = rms_inverse(ss, kHidden, eps);
#pragma unroll
    for (int j = 0; j < 9; ++j) x[j] = wn[j] * (h[j] * inv);
}

__device__ __forceinline__ void load_slice576(const float* __restrict__ v, int lane, float (&out)[9]) {
#pragma unroll
    for (int j = 0; j < 9; ++j) out[j] = v[slice576_index(lane, j)];
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

template <bool kStream = false>
__device__ __forceinline__ void qkv_load(const float* __restrict__ qkv_w, int unit, int lane, QkvUnitWeights& w) {
    int head, d, r0, r1;
    qkv_unit_rows(unit, head, d, r0, r1);
    load_row576<kStream>(qkv_w + static_cast<int64_t>(r0) * kHidden, lane, w.w0);
    load_row576<kStream>(qkv_w + static_cast<int64_t>(r1) * kHidden, lane, w.w1);
}

// Computes the unit's two rows and routes them: q -> q_out[h*64+d], k -> cache
// (and kv_out), v -> cache (and kv_out).  Lane 0 writes.
struct RopePair {
    float c_lo, s_lo, c_hi, s_hi;
};

__device__ __forceinline__ RopePair rope_pair(const float* __restrict__ cos_row, const float* __restrict__ sin_row,
                                              int unit) {
    const int d = unit & 31;
    return RopePair{cos_row[d], sin_row[d], cos_row[d + 32], sin_row[d + 32]};
}

// Normalised QKV row pair of one unit.  The RMS scale multiplies the finished dot
// products, q = inv_rms * sum_j (h_j * wn_j) * w_j, so the sum of squares and both
// dot products reduce at the same time (one reduction latency instead of two);
// the reductions end in wave-uniform values, so every lane holds the outputs.
// RoPE (products rounded separately, packed_qkv_rope_cache_cuda.cu:40-48) and
// routing as the reference: q -> out[r], k/v -> the cache row at the current
// position (lane 0 writes it) and out[r] (the output policy picks the lanes).
template <class QOut>
__device__ __forceinline__ void qkv_unit_compute(const QkvUnitWeights& w, const float (&h)[9], const float (&wn)[9],
                                                 float eps, int unit, int lane, const RopePair& rp,
                                                 float* __restrict__ key_row_base, float* __restrict__ value_row_base,
                                                 int64_t head_stride, const QOut& out) {
    int head, d, r0, r1;
    qkv_unit_rows(unit, head, d, r0, r1);
    float ss = 0.0f, pa = 0.0f, pb = 0.0f;
#pragma unroll
    for (int j = 0; j < 9; ++j) {
        ss = fmaf(h[j], h[j], ss);
        const float hw = h[j] * wn[j];
        pa = fmaf(hw, w.w0[j], pa);
        pb = fmaf(hw, w.w1[j], pb);
    }
    ss = wave_sum_uniform(ss);
    pa = wave_sum_uniform(pa);
    pb = wave_sum_uniform(pb);
    const float inv = rms_inverse(ss, kHidden, eps);
    const float a = pa * inv;
    const float b = pb * inv;
    float lo, hi;
    if (head < kQHeads + kKVHeads) {
        lo = rope_first(a, b, rp.c_lo, rp.s_lo);
        hi = rope_second(b, a, rp.c_hi, rp.s_hi);
    } else {
        lo = a;
        hi = b;
    }
    if (head >= kQHeads && lane == 0) {
        const bool is_key = head < kQHeads + kKVHeads;
        const int g = is_key ? head - kQHeads : head - kQHeads - kKVHeads;
        float* row = (is_key ? key_row_base : value_row_base) + g * head_stride;
        // Write-through (agent scope) so later tokens on other XCDs read it from memory.
        __hip_atomic_store(row + d, lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(row + d + 32, hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    out.put(lane, r0, lo);
    out.put(lane, r1, hi);
}

// ---------------------------------------------------------------------------
// Phase B: attention partial for (KV group g, chunk c) over the chunk's rows
// [begin, end), all resident in LDS when the compute starts.
//
// LDS layout of a chunk (row r = position - begin, kAttnRows rows at most):
//   K: the 16-byte piece c (dims 4c..4c+3) of row r sits at r*64 + 4*(c ^ (r & 15)).
//      QK reads one piece of 64 different rows per instruction; the xor spreads
//      those reads over all banks.
//   V: natural order, r*64 + d; PV reads one row per instruction, lane = dim.
// Cached rows are copied HBM -> LDS with global_load_lds_dwordx4 (no register
// staging); the current row comes from the QKV phase.
//
// Compute (3 query heads share the chunk):
//   QK  thread (position p = t & 127 [+128], part = t >> 7): dims 16*part..+15
//       of all 3 heads -> partial scores in LDS `sp`.
//   max waves 0..5 = (head, half of the positions): sum the 4 parts, scale, max
//       over the half (one wave reduction), p = 2^(s - m_half) -> LDS `pl`,
//       l_half.
//   PV  wave w (positions 16w..16w+15 [+128], all in half w >> 2), lane = dim.
//   combine  threads (head, dim): rescale the two halves to the chunk maximum.
// Output per query head: o[64] (unnormalised), m, l.
constexpr int kAttnScoreStride = 256;                // sp/pl row stride (positions)

// Optional timestamps inside the attention and merge bodies and per wave around phase B's
// K/V copy (compiled only with -DFLUX_TRACE; layer 15 of the third token of a launch).
#ifdef FLUX_TRACE
__device__ uint64_t g_flux_attn_trace[512][8];
__device__ uint64_t g_flux_copy_trace[256][8][4];
#define FLUX_ATTN_TRACE_PARAM , bool trace_on = false
#define FLUX_ATTN_TRACE(k)                                                                            \
    do {                                                                                              \
        if (trace_on && tid_opaque() == 0) g_flux_attn_trace[blockIdx.x][k] = wall_clock64();        \
    } while (0)
#else
#define FLUX_ATTN_TRACE_PARAM
#define FLUX_ATTN_TRACE(k) \
    do {                   \
    } while (0)
#endif

__device__ __forceinline__ int wave_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ int attn_k_index(int r, int d) { return r * kHeadDim + 4 * ((d >> 2) ^ (r & 15)) + (d & 3); }

__device__ __forceinline__ uint32_t lds_address(const float* p) {
    return static_cast<uint32_t>(reinterpret_cast<size_t>((__attribute__((address_space(3))) const float*)p));
}

// LDS-direct copies written as inline assembly, so that the compiler does not add a wait
// for them (vmcnt(0)) before unrelated LDS reads; the wave that issues them reads the data
// only after a later wait of its own (a poll's) has covered them.
__device__ __forceinline__ void copy16_to_lds_nt(const float* src, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, off nt" ::"v"(src), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void copy4_to_lds_nt(const float* src, uint32_t lds) {
    asm volatile("global_load_lds_dword %0, off nt" ::"v"(src), "{m0}"(lds) : "memory");
}

// Copy rows [begin, begin + rows) of one KV head into the chunk's LDS layout.
// One instruction moves 4 rows (1 KB): lane l -> row 4b + l/16, slot l%16.
// Waves [first_wave, kWavesPerWG) issue the copies.
__device__ __forceinline__ void attn_stage_lds(const float* __restrict__ key_g, const float* __restrict__ value_g,
                                               int64_t begin, int rows, float* k_lds, float* v_lds,
                                               int first_wave) {
    const int lane = tid_opaque() & 63;
    const int wave = wave_uniform(static_cast<int>(tid_opaque() >> 6));
    const int blocks = (rows + 3) >> 2;
    const int nwaves = kWavesPerWG - first_wave;
    const int r_in = lane >> 4;
    const int slot = lane & 15;
    for (int b = wave - first_wave; b < blocks && b >= 0; b += nwaves) {
        const int r = 4 * b + r_in;
        if (r < rows) {
            const int64_t row = (begin + r) * kHeadDim;
            // Non-temporal (aux 2): each cached row is read once per token and layer.
            __builtin_amdgcn_global_load_lds(key_g + row + 4 * (slot ^ (r & 15)), k_lds + b * 256, 16, 0, 2);
            __builtin_amdgcn_global_load_lds(value_g + row + 4 * slot, v_lds + b * 256, 16, 0, 2);
        }
    }
}

// Scratch LDS of attn_compute: sp [4][kGroup][256] partial scores, pl [256][4]
// probabilities, red [8][kGroup][64] per-wave outputs + 12 (m, l) words.
struct AttnScratch {
    float* sp;
    float* pl;
    float* red;
};
constexpr int kAttnSpFloats = 4 * kGroup * kAttnScoreStride;
constexpr int kAttnPlFloats = 4 * kAttnScoreStride;
constexpr int kAttnRedFloats = kWavesPerWG * kGroup * kHeadDim + 4 * kGroup;

// qv: the 3 query rows (LDS, 192 floats).  rows <= kAttnRows.  scale2 = scale*log2(e).
template <class POut>
__device__ __forceinline__ void attn_compute(const float* k_lds, const float* v_lds, const float* qv, int rows,
                                             float scale2, const AttnScratch& ws,
                                             const POut& out FLUX_ATTN_TRACE_PARAM) {
    const int t = tid_opaque();
    const int lane = t & 63;
    const int wave = wave_uniform(t >> 6);
    const int passes = rows > 128 ? 2 : 1;
    // ---- QK: partial dot products over 16 dims ----
    {
        const int part = wave >> 1;
        float q[kGroup][16];
#pragma unroll
        for (int h = 0; h < kGroup; ++h)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 a = *reinterpret_cast<const float4*>(qv + h * kHeadDim + 16 * part + 4 * k);
                q[h][4 * k] = a.x;
                q[h][4 * k + 1] = a.y;
                q[h][4 * k + 2] = a.z;
                q[h][4 * k + 3] = a.w;
            }
        for (int ps = 0; ps < passes; ++ps) {
            const int p = ps * 128 + (wave & 1) * 64 + lane;
            const int pr = p < rows ? p : 0;
            const int sw = pr & 15;
            const float* krow = k_lds + pr * kHeadDim;
            float4 kk[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) kk[k] = *reinterpret_cast<const float4*>(krow + 4 * ((4 * part + k) ^ sw));
            float acc[kGroup] = {0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
#pragma unroll
                for (int h = 0; h < kGroup; ++h) {
                    acc[h] = fmaf(q[h][4 * k], kk[k].x, acc[h]);
                    acc[h] = fmaf(q[h][4 * k + 1], kk[k].y, acc[h]);
                    acc[h] = fmaf(q[h][4 * k + 2], kk[k].z, acc[h]);
                    acc[h] = fmaf(q[h][4 * k + 3], kk[k].w, acc[h]);
                }
            }
            float* dst = ws.sp + part * (kGroup * kAttnScoreStride) + p;
#pragma unroll
            for (int h = 0; h < kGroup; ++h) dst[h * kAttnScoreStride] = acc[h];
        }
    }
    __syncthreads();
    FLUX_ATTN_TRACE(0);
    // ---- scores, per-half maximum, probabilities ----
    float* red_ml = ws.red + kWavesPerWG * kGroup * kHeadDim;  // m[kGroup][2], l[kGroup][2]
    if (wave < 2 * kGroup) {
        const int h = wave >> 1;
        const int half = wave & 1;
        float s[2];
        float m = -INFINITY;
#pragma unroll
        for (int ps = 0; ps < 2; ++ps) {
            s[ps] = -INFINITY;
            if (ps < passes) {
                const int p = ps * 128 + half * 64 + lane;
                const float* src = ws.sp + h * kAttnScoreStride + p;
                const float v = (src[0] + src[kGroup * kAttnScoreStride]) +
                                (src[2 * kGroup * kAttnScoreStride] + src[3 * kGroup * kAttnScoreStride]);
                s[ps] = p < rows ? v * scale2 : -INFINITY;
                m = fmaxf(m, s[ps]);
            }
        }
        m = wave_max_uniform(m);
        float l = 0.0f;
#pragma unroll
        for (int ps = 0; ps < 2; ++ps) {
            if (ps < passes) {
                const int p = ps * 128 + half * 64 + lane;
                const float e = s[ps] == -INFINITY ? 0.0f : fast_exp2(s[ps] - m);
                ws.pl[p * 4 + h] = e;
                l += e;
            }
        }
        l = wave_sum_uniform(l);
        if (lane == 0) {
            red_ml[h * 2 + half] = m;
            red_ml[2 * kGroup + h * 2 + half] = l;
        }
    }
    __syncthreads();
    FLUX_ATTN_TRACE(1);
    // ---- PV: lane = dim over this wave's 16 positions ----
    {
        float o0 = 0.f, o1 = 0.f, o2 = 0.f;
        for (int ps = 0; ps < passes; ++ps) {
            const int base = ps * 128 + wave * 16;
            if (base >= rows) break;
            const float* vsrc = v_lds + base * kHeadDim + lane;
            const float4* psrc = reinterpret_cast<const float4*>(ws.pl + base * 4);
            if (base + 16 <= rows) {
                float vv[16];
                float4 pp[16];
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    vv[j] = vsrc[j * kHeadDim];
                    pp[j] = psrc[j];
                }
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    o0 = fmaf(pp[j].x, vv[j], o0);
                    o1 = fmaf(pp[j].y, vv[j], o1);
                    o2 = fmaf(pp[j].z, vv[j], o2);
                }
            } else {
                const int n = rows - base;
                for (int j = 0; j < n; ++j) {
                    const float v = vsrc[j * kHeadDim];
                    const float4 pj = psrc[j];
                    o0 = fmaf(pj.x, v, o0);
                    o1 = fmaf(pj.y, v, o1);
                    o2 = fmaf(pj.z, v, o2);
                }
            }
        }
        float* dst = ws.red + wave * (kGroup * kHeadDim) + lane;
        dst[0] = o0;
        dst[kHeadDim] = o1;
        dst[2 * kHeadDim] = o2;
    }
    __syncthreads();
    FLUX_ATTN_TRACE(2);
    // ---- combine the 8 waves: halves rescaled to the chunk maximum ----
    if (wave < kGroup) {
        const int h = wave;
        const float m0 = red_ml[h * 2], m1 = red_ml[h * 2 + 1];
        const float M = fmaxf(m0, m1);
        const float f0 = m0 == -INFINITY ? 0.0f : fast_exp2(m0 - M);
        const float f1 = m1 == -INFINITY ? 0.0f : fast_exp2(m1 - M);
        const float* src = ws.red + h * kHeadDim + lane;
        constexpr int kS = kGroup * kHeadDim;
        const float a0 = (src[0] + src[kS]) + (src[2 * kS] + src[3 * kS]);
        const float a1 = (src[4 * kS] + src[5 * kS]) + (src[6 * kS] + src[7 * kS]);
        out.put(h, lane, a0 * f0 + a1 * f1);
        if (lane == 0) {
            out.put(h, kHeadDim, M);
            out.put(h, kHeadDim + 1, red_ml[2 * kGroup + h * 2] * f0 + red_ml[2 * kGroup + h * 2 + 1] * f1);
        }
    }
    __syncthreads();
    FLUX_ATTN_TRACE(3);
}

// ---------------------------------------------------------------------------
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

// Chunking of the attended positions [0, L) across `chunks` workgroups.
__device__ __forceinline__ void chunk_range(int64_t attended, int chunks, int c, int64_t& begin, int64_t& end) {
    const int64_t per = (attended + chunks - 1) / chunks;
    begin = per * c;
    end = begin + per < attended ? begin + per : attended;
    if (begin > end) begin = end;
}

// The same in 32-bit arithmetic (attended <= the 16384-position capacity), for the
// fused kernel, which recomputes it every layer.
__device__ __forceinline__ void chunk_range32(int attended, int chunks, int c, int& begin, int& end) {
    const int per = static_cast<int>((static_cast<unsigned>(attended) + chunks - 1) / static_cast<unsigned>(chunks));
    begin = per * c;
    end = begin + per < attended ? begin + per : attended;
    if (begin > end) begin = end;
}

// ---------------------------------------------------------------------------
// LM head + argmax: rows [row0, row1) for one wave, batches of kLmBatch rows.
// Rows [row0, row1) of the LM head, kLmBatch rows per stage, two stages in
// flight: the next stage's rows are requested before the current stage's dot
// products, so HBM keeps streaming while a wave computes.  `w` holds the first
// stage on entry (rows row0..row0+kLmBatch-1, clamped like below).
template <class LogitsOut>
__device__ __forceinline__ void lm_stage(const float (&x)[9], const float (&w)[kLmBatch][9], int64_t base, int64_t row1,
                                         const LogitsOut& logits, float& best_v, int64_t& best_i) {
    const int lane = tid_opaque() & 63;
#pragma unroll
    for (int r = 0; r < kLmBatch; ++r) {
        const float v = wave_sum_uniform(dot_lane<9>(x, w[r]));
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

// LM-head rows with the default cache policy (measured 0.15% faster per token than
// non-temporal loads here; the tied rows double as the next token's embedding row).
__device__ __forceinline__ void lm_load(const float* __restrict__ lm_head, int64_t base, int64_t row1, int lane,
                                        float (&w)[kLmBatch][9]) {
#pragma unroll
    for (int r = 0; r < kLmBatch; ++r) {
        const int64_t row = base + r < row1 ? base + r : (row1 > 0 ? row1 - 1 : 0);
        const float* p = lm_head + row * kHidden;
        const float4 a = *reinterpret_cast<const float4*>(p + 4 * lane);
        const float4 b = *reinterpret_cast<const float4*>(p + 256 + 4 * lane);
        w[r][0] = a.x; w[r][1] = a.y; w[r][2] = a.z; w[r][3] = a.w;
        w[r][4] = b.x; w[r][5] = b.y; w[r][6] = b.z; w[r][7] = b.w;
        w[r][8] = p[512 + lane];
    }
}

template <class LogitsOut>
__device__ __forceinline__ void lm_rows_pipelined(const float* __restrict__ lm_head, const float (&x)[9],
                                                  float (&wa)[kLmBatch][9], int64_t row0, int64_t row1, int lane,
                                                  const LogitsOut& logits, float& best_v, int64_t& best_i) {
    float wb[kLmBatch][9];
    for (int64_t base = row0; base < row1; base += 2 * kLmBatch) {
        const bool next_b = base + kLmBatch < row1;
        if (next_b) lm_load(lm_head, base + kLmBatch, row1, lane, wb);
        lm_stage(x, wa, base, row1, logits, best_v, best_i);
        if (!next_b) break;
        const bool next_a = base + 2 * kLmBatch < row1;
        if (next_a) lm_load(lm_head, base + 2 * kLmBatch, row1, lane, wa);
        lm_stage(x, wb, base + kLmBatch, row1, logits, best_v, best_i);
    }
}

struct LogitsPlainOut {
    float* p;
    __device__ __forceinline__ void put(int64_t i, float v) const { p[i] = v; }
};

// Workgroup argmax reduction of per-wave (value, index); result valid in thread 0.
__device__ __forceinline__ void wg_argmax(float& v, int64_t& i, float* red_v, int64_t* red_i) {
    const int lane = tid_opaque() & 63;
    const int wave = tid_opaque() >> 6;
    if (lane == 0) {
        red_v[wave] = v;
        red_i[wave] = i;
    }
    __syncthreads();
    if (tid_opaque() == 0) {
        for (int w = 1; w < kWavesPerWG; ++w) {
            if (argmax_precedes(red_v[w], red_i[w], v, i)) {
                v = red_v[w];
                i = red_i[w];
            }
        }
    }
    __syncthreads();
}

// One argmax step against the candidate a DPP move brings in (partner lanes outside
// the move's row mask see the identity -inf / INT_MAX, which never wins).
template <int kCtrl, int kRowMask>
__device__ __forceinline__ void argmax_dpp_step(float& v, int& i) {
    const float ov = __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), kCtrl, kRowMask, 0xF, false));
    const int oi = __builtin_amdgcn_update_dpp(INT32_MAX, i, kCtrl, kRowMask, 0xF, false);
    if (argmax_precedes(ov, oi, v, i)) {
        v = ov;
        i = oi;
    }
}

// Wave argmax (NaN first, then larger value, then lower index) with DPP row moves and
// row broadcasts, ending in a wave-uniform result read from lane 63: no LDS crossbar
// (a 64-bit __shfl_xor butterfly costs 18 dependent ds_bpermute round trips).
__device__ __forceinline__ void wave_argmax_uniform(float& v, int& i) {
    argmax_dpp_step<kDppRowRor8, 0xF>(v, i);
    argmax_dpp_step<kDppRowRor4, 0xF>(v, i);
    argmax_dpp_step<kDppQuadXor2, 0xF>(v, i);
    argmax_dpp_step<kDppQuadXor1, 0xF>(v, i);
    argmax_dpp_step<kDppRowBcast15, 0xA>(v, i);
    argmax_dpp_step<kDppRowBcast31, 0xC>(v, i);
    v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    i = __builtin_amdgcn_readlane(i, 63);
}

__device__ __forceinline__ uint32_t epoch_of(uint32_t token_counter, int stage) {
    // stage 0..29 = layers, 30 = argmax.  Never 0 for any token (memory starts zeroed).
    return token_counter * 32u + static_cast<uint32_t>(stage) + 1u;
}

// Optional phase timestamps for latency analysis (compiled only with -DFLUX_TRACE).
#ifdef FLUX_TRACE
__device__ uint64_t g_flux_trace[4][kLayers + 1][16];
__device__ uint64_t g_flux_trace_all[512][16];
#define FLUX_TRACE_POINT(slot)                                                                         \
    do {                                                                                               \
        if (t == 2 && tid_opaque() == 0 && (wg % 85) == 0 && wg / 85 < 4)                              \
            g_flux_trace[wg / 85][layer][slot] = wall_clock64();                                       \
        if (t == 2 && layer == 15 && tid_opaque() == 0) g_flux_trace_all[wg][slot] = wall_clock64();   \
    } while (0)
#define FLUX_COPY_TRACE(k)                                                                            \
    do {                                                                                              \
        if (t == 2 && layer == 15 && (tid_opaque() & 63) == 0)                                        \
            g_flux_copy_trace[wg][tid_opaque() >> 6][k] = wall_clock64();                              \
    } while (0)
#define FLUX_MERGE_TRACE(k)                                                                           \
    do {                                                                                              \
        if (t == 2 && layer == 15 && tid_opaque() == 0) g_flux_attn_trace[blockIdx.x][k] = wall_clock64(); \
    } while (0)
#define FLUX_TRACE_ARG , t == 2 && layer == 15
#else
#define FLUX_TRACE_POINT(slot) \
    do {                       \
    } while (0)
#define FLUX_COPY_TRACE(k) \
    do {                   \
    } while (0)
#define FLUX_MERGE_TRACE(k) \
    do {                    \
    } while (0)
#define FLUX_TRACE_ARG
#endif

// ---------------------------------------------------------------------------
// Workgroup-cooperative LL fetch into LDS.  Word k (0 <= k < count) is read from
// base + index(k) and stored to *dest(k); threads [first_thread, kThreads) poll,
// each at most kMax words in one batch.  Threads with fewer words poll nothing
// extra (their slots re-read word index(0) but are not stored).
template <int kMax, class IndexFn, class DestFn>
__device__ __forceinline__ void wg_ll_fetch_to(const uint64_t* __restrict__ base, int count, IndexFn index,
                                               DestFn dest, int first_thread, uint32_t epoch, const WaitCtx& w) {
    const int me = static_cast<int>(tid_opaque()) - first_thread;
    const int nthreads = kThreads - first_thread;
    if (me < 0) return;
    int idx[kMax];
    float v[kMax];
#pragma unroll
    for (int j = 0; j < kMax; ++j) {
        const int k = me + j * nthreads;
        idx[j] = index(k < count ? k : 0);
    }
    if (me < count) ll_fetch<kMax>(base, idx, epoch, w, v);
#pragma unroll
    for (int j = 0; j < kMax; ++j) {
        const int k = me + j * nthreads;
        if (k < count) *dest(k) = v[j];
    }
}

template <int kMax, class IndexFn>
__device__ __forceinline__ void wg_ll_fetch(const uint64_t* __restrict__ base, int count, IndexFn index,
                                            uint32_t epoch, const WaitCtx& w, float* lds) {
    wg_ll_fetch_to<kMax>(base, count, index, [=](int k) { return lds + k; }, 0, epoch, w);
}

struct Contiguous {
    __device__ __forceinline__ int operator()(int k) const { return k; }
};

// Lane slice of a 576-vector held in LDS.
__device__ __forceinline__ void lds_slice576(const float* vec, int lane, float (&v)[9]) {
#pragma unroll
    for (int j = 0; j < 9; ++j) v[j] = vec[slice576_index(lane, j)];
}

// Layer descriptors are copied into LDS once per launch; a layer's descriptor is
// read from there and moved into scalar registers (its pointers are wave-uniform),
// so the weight loads of a phase need no memory round trip before they issue.
__device__ __forceinline__ const float* uniform_ptr(const float* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = static_cast<uint32_t>(wave_uniform(static_cast<int>(static_cast<uint32_t>(v))));
    const uint32_t hi = static_cast<uint32_t>(wave_uniform(static_cast<int>(static_cast<uint32_t>(v >> 32))));
    return reinterpret_cast<const float*>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ LayerWeights uniform_desc(const LayerWeights& d) {
    LayerWeights u;
    u.input_norm = uniform_ptr(d.input_norm);
    u.qkv = uniform_ptr(d.qkv);
    u.o_proj = uniform_ptr(d.o_proj);
    u.post_norm = uniform_ptr(d.post_norm);
    u.gate_up = uniform_ptr(d.gate_up);
    u.down = uniform_ptr(d.down);
    u.eps = __int_as_float(wave_uniform(__float_as_int(d.eps)));
    u.scale = __int_as_float(wave_uniform(__float_as_int(d.scale)));
    return u;
}

// ---------------------------------------------------------------------------
// The fused persistent decode kernel: `args.steps` greedy tokens per launch.
// Requires gridDim.x * 8 >= 1536 (one unit per wave in every phase).
__global__ void __launch_bounds__(kThreads, 1) fused_decode_kernel(DecodeArgs args) {
    __shared__ int abort_flag;
    __shared__ WaitShared wait_shared;
    __shared__ int32_t step_error;
    __shared__ LayerWeights layer_desc[kLayers];
    __shared__ float red[kAttnRedFloats];
    __shared__ __align__(16) float attn_sp[kAttnSpFloats];
    __shared__ __align__(16) float attn_pl[kAttnPlFloats];
    __shared__ int64_t red_i[kWavesPerWG];
    __shared__ float red_v[kWavesPerWG];
    __shared__ float hvec[kHidden];   // layer input h (residual of C)
    __shared__ float rvec[kHidden];   // post-attention residual r (residual of E)
    __shared__ __align__(16) float vec[kInter];  // attention output / SwiGLU output / q of the group
    __shared__ __align__(16) float oproj_rows[3][kHidden];  // this layer's o_proj rows of waves 0-2
    extern __shared__ __align__(16) float part[];  // K/V rows of the attention chunk; merge staging

    const int lane = tid_opaque() & 63;
    const int wave = tid_opaque() >> 6;
    const int G = gridDim.x;
    const int wg = blockIdx.x;
    // This workgroup polls the copy of the replicated vectors that its XCD shares with one other.
    const int replica = static_cast<int>(xcc_id() % LLLayout::kReplicas) * LLLayout::kReplicaStride;
    const int gw = wave * G + wg;        // global wave id, interleaved across CUs
    const int chunks = G / kKVHeads < kMaxAttnChunks ? G / kKVHeads : kMaxAttnChunks;
    const int64_t cap = args.capacity;
    const int64_t head_stride = cap * kHeadDim;
    const int64_t layer_stride = kKVHeads * head_stride;
    const int partial_stride = kGroup * (kHeadDim + 2);

    if (tid_opaque() == 0) {
        abort_flag = 0;
        wait_shared = WaitShared{args.host_error, args.wait_ticks};
    }
    // Layers per step: kLayers for the token loop, 1 for the single-layer step
    // (NativeSmolLM2LayerDecode), whose descriptor array holds that layer only.
    const int n_layers = wave_uniform(args.layer_count);
    if (static_cast<int>(tid_opaque()) < n_layers) layer_desc[tid_opaque()] = args.layers[tid_opaque()];
    const uint32_t counter0 = *args.token_counter;
    // The token state is the same for every lane: kept in scalar registers.
    auto uniform64 = [](int64_t v) {
        const uint64_t u = static_cast<uint64_t>(v);
        const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
        const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
        return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
    };
    int64_t token = uniform64(args.token_in != nullptr ? *args.token_in : *args.input_token);
    int64_t position = uniform64(*args.position);
    int64_t step = uniform64(*args.generation_step);
    __syncthreads();
    const WaitCtx wctx{&abort_flag, args.error, &wait_shared,
                       args.wait_ticks < kWatchErrorTicks ? args.wait_ticks : kWatchErrorTicks};

    int t = 0;
    for (; t < args.steps; ++t) {
        __syncthreads();
        const bool stop = abort_flag != 0;
        __syncthreads();
        if (stop) break;
        if (position < 0 || position >= cap) {
            if (wg == 0 && tid_opaque() == 0) record_error(args.error, wait_shared.host_error, 2);
            break;
        }
        const uint32_t counter = counter0 + static_cast<uint32_t>(t);
        const int64_t attended = position + 1;
        const float* cos_row = args.rope_cos + position * kHeadDim;
        const float* sin_row = args.rope_sin + position * kHeadDim;
        const bool token_ok = token >= 0 && token < args.vocab;
        // Position chunks of this token's attention: one per 64 attended positions, at most
        // `chunks` (85 on 256 CUs, reached from 5377 positions on).  Short contexts then
        // merge a few partials instead of 85 mostly one-row ones (ctx 128: 0.457 -> 0.427 ms
        // per token, 1024: 0.472 -> 0.436; 64-row chunks measured faster than 32, 96 or 128).
        const int want_chunks = static_cast<int>((attended + 63) >> 6);
        const int tchunks_token = __builtin_amdgcn_readfirstlane(want_chunks < chunks ? want_chunks : chunks);
        const float* emb_row = args.embedding + (token_ok ? token : 0) * kHidden;

        for (int layer = 0; layer < n_layers; ++layer) {
            int tchunks = tchunks_token;
            asm volatile("" : "+s"(tchunks));
            const LayerWeights Lw = uniform_desc(layer_desc[layer]);
            const uint32_t ep = epoch_of(counter, layer);
            uint64_t* ll = args.ll + (layer & 1) * LLLayout::kParity;
            const uint64_t* ll_prev = args.ll + ((layer + 1) & 1) * LLLayout::kParity;
            float* key_layer = args.key_cache + layer * layer_stride;
            float* value_layer = args.value_cache + layer * layer_stride;

            // ---- A: norm(h) -> QKV GEMV -> RoPE -> cache (unit = row pair, one per wave) ----
            {
                FLUX_TRACE_POINT(0);
                const bool active = gw < kQKV / 2;
                QkvUnitWeights w;
                float wn[9];
                RopePair rp{};
                if (active) {
                    qkv_load<true>(Lw.qkv, gw, lane, w);
                    load_slice576(Lw.input_norm, lane, wn);
                    rp = rope_pair(cos_row, sin_row, gw);
                }
                if (layer == 0 && args.hidden_in != nullptr) {
                    // Single-layer step: the caller's hidden state (workgroup 0 also keeps a copy
                    // in hidden_save, the input of a later step that passes none).
                    for (int k = tid_opaque(); k < kHidden; k += kThreads) {
                        const float v = args.hidden_in[k];
                        hvec[k] = v;
                        if (wg == 0 && args.hidden_save != nullptr) args.hidden_save[k] = v;
                    }
                } else if (layer == 0) {
                    for (int k = tid_opaque(); k < kHidden; k += kThreads) hvec[k] = token_ok ? emb_row[k] : 0.0f;
                } else {
                    wg_ll_fetch<2>(ll_prev + replica + LLLayout::kHidden, kHidden, Contiguous{}, epoch_of(counter, layer - 1),
                                   wctx, hvec);
                }
                __syncthreads();
                FLUX_TRACE_POINT(1);
                if (active) {
                    float h[9];
                    lds_slice576(hvec, lane, h);
                    qkv_unit_compute(w, h, wn, Lw.eps, gw, lane, rp, key_layer + position * kHeadDim,
                                     value_layer + position * kHeadDim, head_stride, QkvLLOut{ll + LLLayout::kQkv, ep});
                }
            }

            // The o_proj rows of phase C (waves 0-2) are copied into LDS now, during the
            // attention, instead of after its merge.
            if (wave_uniform(static_cast<int>(tid_opaque() >> 6)) < 3 && gw < kHidden) {
                const int w3 = wave_uniform(static_cast<int>(tid_opaque() >> 6));
                const float* row = Lw.o_proj + static_cast<int64_t>(gw) * kHidden;
                const uint32_t dst = lds_address(oproj_rows[w3]);
                copy16_to_lds_nt(row + 4 * lane, dst);
                copy16_to_lds_nt(row + 256 + 4 * lane, dst + 1024);
                copy4_to_lds_nt(row + 512 + lane, dst + 2048);
            }

            // ---- B: attention partial of (KV group g, position chunk c) ----
            FLUX_TRACE_POINT(2);
            if (wg < kKVHeads * tchunks) {
                const int g = wg % kKVHeads;
                const int c = wg / kKVHeads;
                int begin32, end32;
                chunk_range32(static_cast<int>(attended), tchunks, c, begin32, end32);
                const int64_t begin = begin32, end = end32;
                const int64_t cached_end = end < position ? end : position;
                const int cached_rows = cached_end > begin ? static_cast<int>(cached_end - begin) : 0;
                float* k_lds = part;
                float* v_lds = part + kAttnRows * kHeadDim;
                // Waves 0-1 may still be finishing the QKV phase: waves 2-7 stage the cached
                // rows and poll the query (and the current row) for the whole workgroup.
                FLUX_COPY_TRACE(3);
                attn_stage_lds(key_layer + g * head_stride, value_layer + g * head_stride, begin, cached_rows, k_lds,
                               v_lds, 2);
                FLUX_COPY_TRACE(0);
                const bool has_current = position >= begin && position < end;
                const int cur = static_cast<int>(position - begin);
                // Words 0..191: q of heads 3g..3g+2 -> vec; 192..255: new k row; 256..319: new v row.
                const int qbase = g * kGroup * kHeadDim;
                const int kbase = kQHeads * kHeadDim + g * kHeadDim;
                wg_ll_fetch_to<1>(
                    ll + replica + LLLayout::kQkv, has_current ? kGroup * kHeadDim + 2 * kHeadDim : kGroup * kHeadDim,
                    [=](int k) {
                        return k < kGroup * kHeadDim
                                   ? qbase + k
                                   : kbase + ((k - kGroup * kHeadDim) >> 6) * (kKVHeads * kHeadDim) +
                                         ((k - kGroup * kHeadDim) & 63);
                    },
                    [=](int k) {
                        if (k < kGroup * kHeadDim) return vec + k;
                        const int d = (k - kGroup * kHeadDim) & 63;
                        return k < kGroup * kHeadDim + kHeadDim ? k_lds + attn_k_index(cur, d)
                                                                : v_lds + cur * kHeadDim + d;
                    },
                    2 * kWave, ep, wctx);
                FLUX_COPY_TRACE(1);
                __builtin_amdgcn_s_waitcnt(0);  // LDS-direct K/V loads have landed
                FLUX_COPY_TRACE(2);
                __syncthreads();
                FLUX_TRACE_POINT(3);
                attn_compute(k_lds, v_lds, vec, static_cast<int>(end - begin), Lw.scale * kLog2e,
                             AttnScratch{attn_sp, attn_pl, red},
                             PartialLLOut{ll + LLLayout::kPartials + (g * tchunks + c) * partial_stride, ep}
                                 FLUX_TRACE_ARG);
            }

            FLUX_TRACE_POINT(4);
            // ---- B2: merge chunk partials; WG (h, quarter) handles 16 dims of query head h ----
            if (wg < kQHeads * 4) {
                const int h = wg >> 2;
                const int quarter = wg & 3;
                const int g = h / kGroup;
                const int hh = h % kGroup;
                constexpr int kRun = 18;  // 16 dims + m + l per chunk
                const uint64_t* pbase = ll + LLLayout::kPartials + g * tchunks * partial_stride + hh * (kHeadDim + 2);
                wg_ll_fetch<(kMaxAttnChunks * kRun + kThreads - 1) / kThreads>(
                    pbase, tchunks * kRun,
                    [=](int k) {
                        const int cc = k / kRun;
                        const int j = k - cc * kRun;
                        return cc * partial_stride + (j < 16 ? 16 * quarter + j : kHeadDim + (j - 16));
                    },
                    ep, wctx, part);
                __syncthreads();
                FLUX_TRACE_POINT(5);
                // Global max of the chunk maxima: lane-strided, then a DPP reduction into a
                // scalar (every wave computes the same value).
                float M = -INFINITY;
                for (int cc = lane; cc < tchunks; cc += kWave) M = fmaxf(M, part[cc * kRun + 16]);
                M = wave_max_uniform(M);
                FLUX_MERGE_TRACE(4);
                // Wave w merges dims 2w (lanes 0-31) and 2w + 1 (lanes 32-63); lane slot
                // s = lane % 32 sums chunks s, s + 32, ...
                const int slot = lane & 31;
                const int d = 2 * wave + (lane >> 5);
                float O = 0.0f, L = 0.0f;
                for (int cc = slot; cc < tchunks; cc += 32) {
                    const float* pc = part + cc * kRun;
                    const float mc = pc[16];
                    if (mc == -INFINITY) continue;
                    const float f = fast_exp2(mc - M);
                    O = fmaf(pc[d], f, O);
                    L = fmaf(pc[17], f, L);
                }
                // Sum over each half: rows of 16 lanes, then row_bcast15 adds row 0 into
                // row 1 and row 2 into row 3, so lanes 31 and 63 hold the two halves' sums.
                O = row16_sum(O);
                L = row16_sum(L);
                O += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(O), kDppRowBcast15, 0xA, 0xF, false));
                L += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(L), kDppRowBcast15, 0xA, 0xF, false));
                if ((lane & 31) == 31) red[d] = O / L;
                __syncthreads();
                FLUX_MERGE_TRACE(5);
                // Thread (copy r = t / 16, dim d = t % 16) writes dim d of copy r: each copy's
                // 16 dims are one 128-byte line written by one instruction.
                if (tid_opaque() < 16 * LLLayout::kReplicas) {
                    const int dd = tid_opaque() & 15;
                    const int r = tid_opaque() >> 4;
                    ll_store(ll + r * LLLayout::kReplicaStride + LLLayout::kAttnMerged + h * kHeadDim + 16 * quarter + dd,
                             red[dd], ep);
                }
                __syncthreads();
            }

            // ---- C: o_proj + residual (row = gw) ----
            {
                FLUX_TRACE_POINT(6);
                const bool active = gw < kHidden;
                wg_ll_fetch<2>(ll + replica + LLLayout::kAttnMerged, kHidden, Contiguous{}, ep, wctx, vec);
                __syncthreads();  // the poll's wait also covered this wave's o_proj row copy
                FLUX_TRACE_POINT(7);
                if (active) {
                    // This wave's o_proj row was copied into LDS by inline-asm LDS-direct loads
                    // (phase B), which the compiler does not track.  The poll above already
                    // waited for loads issued after them (every thread of waves 0-2 polls a
                    // word while the vector is at least 3 waves wide); the explicit wait keeps
                    // the dependency if the fetch changes, and costs nothing once it has.
                    static_assert(kHidden >= 3 * kWave, "waves 0-2 must each poll a word of phase C's input");
                    __builtin_amdgcn_s_waitcnt(0);
                    float w[9], a[9];
                    lds_slice576(oproj_rows[wave_uniform(static_cast<int>(tid_opaque() >> 6)) % 3], lane, w);
                    lds_slice576(vec, lane, a);
                    const float dot = wave_sum_uniform(dot_lane<9>(a, w));
                    ll_store_replicas(ll + LLLayout::kResid, gw, hvec[gw] + dot, ep, lane);
                }
                __syncthreads();
            }

            // ---- D: norm(r) -> gate/up GEMV -> SwiGLU (unit j = gw) ----
            {
                const bool active = gw < kInter;
                float wg_[9], wu[9], wn[9];
                if (active) {
                    load_row576<true>(Lw.gate_up + static_cast<int64_t>(gw) * kHidden, lane, wg_);
                    load_row576<true>(Lw.gate_up + static_cast<int64_t>(kInter + gw) * kHidden, lane, wu);
                    load_slice576(Lw.post_norm, lane, wn);
                }
                FLUX_TRACE_POINT(8);
                wg_ll_fetch<2>(ll + replica + LLLayout::kResid, kHidden, Contiguous{}, ep, wctx, rvec);
                __syncthreads();
                FLUX_TRACE_POINT(9);
                if (active) {
                    // RMS scale applied after the dot products (see qkv_unit_compute).
                    float r[9];
                    lds_slice576(rvec, lane, r);
                    float ss = 0.0f, pg = 0.0f, pu = 0.0f;
#pragma unroll
                    for (int j = 0; j < 9; ++j) {
                        ss = fmaf(r[j], r[j], ss);
                        const float rw = r[j] * wn[j];
                        pg = fmaf(rw, wg_[j], pg);
                        pu = fmaf(rw, wu[j], pu);
                    }
                    ss = wave_sum_uniform(ss);
                    pg = wave_sum_uniform(pg);
                    pu = wave_sum_uniform(pu);
                    const float inv = rms_inverse(ss, kHidden, Lw.eps);
                    ll_store_replicas(ll + LLLayout::kSwiglu, gw, silu(pg * inv) * (pu * inv), ep, lane);
                }
                __syncthreads();
                FLUX_TRACE_POINT(12);
            }

            // ---- E: down GEMV + residual (row = gw) ----
            {
                const bool active = gw < kHidden;
                float w[24];
                if (active) load_row1536<true>(Lw.down + static_cast<int64_t>(gw) * kInter, lane, w);
                FLUX_TRACE_POINT(10);
                wg_ll_fetch<3>(ll + replica + LLLayout::kSwiglu, kInter, Contiguous{}, ep, wctx, vec);
                __syncthreads();
                FLUX_TRACE_POINT(11);
                if (active) {
                    float sv[24];
#pragma unroll
                    for (int j = 0; j < 24; ++j) sv[j] = vec[slice1536_index(lane, j)];
                    const float dot = wave_sum_uniform(dot_lane<24>(sv, w));
                    ll_store_replicas(ll + LLLayout::kHidden, gw, rvec[gw] + dot, ep, lane);
                }
                __syncthreads();
            }
        }

        if (args.hidden_out != nullptr) {
            // Single-layer step: workgroup 0 gathers the layer's output h into hidden_out and
            // advances the position; there is no LM head.  The step's K/V rows were written
            // through (agent-scope stores), so the next launch reads them from memory.
            if (wg == 0) {
                wg_ll_fetch<2>(args.ll + ((n_layers - 1) & 1) * LLLayout::kParity + replica + LLLayout::kHidden,
                               kHidden, Contiguous{}, epoch_of(counter, n_layers - 1), wctx, hvec);
                __syncthreads();
                for (int k = tid_opaque(); k < kHidden; k += kThreads) args.hidden_out[k] = hvec[k];
                if (tid_opaque() == 0) {
                    *args.position = attended;
                    *args.cache_length = attended;
                }
            }
            position = attended;
            continue;
        }

        // ---- final norm -> LM head -> argmax ----
        {
            const uint32_t ep_last = epoch_of(counter, kLayers - 1);
            const uint32_t ep_arg = epoch_of(counter, kLayers);
            const uint64_t* ll_last = args.ll + ((kLayers - 1) & 1) * LLLayout::kParity;
            uint64_t* ll_arg = args.ll + (t & 1) * LLLayout::kParity + LLLayout::kArgmax;  // copy 0
            const int TW = G * kWavesPerWG;
            const int64_t per = (args.vocab + TW - 1) / TW;
            const int64_t row0 = per * gw < args.vocab ? per * gw : args.vocab;
            const int64_t row1 = row0 + per < args.vocab ? row0 + per : args.vocab;
            [[maybe_unused]] const int layer = kLayers;  // read by the trace points
            FLUX_TRACE_POINT(0);
            float wl[kLmBatch][9];
            float wn[9];
            load_slice576(args.final_norm, lane, wn);
            wg_ll_fetch<2>(ll_last + replica + LLLayout::kHidden, kHidden, Contiguous{}, ep_last, wctx, hvec);
            // This token's K/V cache rows were written through (agent-scope stores, the last of
            // them in layer 29's QKV phase); every wave waits until its stores are acknowledged
            // before the workgroup signals its argmax candidate, so the next token's attention
            // reads them from memory.  Here nothing but those stores and the h poll are
            // outstanding; the logits stores issued below are not waited for.
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            lm_load(args.lm_head, row0, row1, lane, wl);
            FLUX_TRACE_POINT(1);
            float h[9], x[9];
            lds_slice576(hvec, lane, h);
            norm_slice_w(h, wn, args.final_eps, x);
            float best_v = -INFINITY;
            int64_t best_i = INT64_MAX;
            lm_rows_pipelined(args.lm_head, x, wl, row0, row1, lane, LogitsPlainOut{args.logits}, best_v, best_i);
            wg_argmax(best_v, best_i, red_v, red_i);
            // WG 0 reads the device error word before the argmax exchange; it decides below
            // whether this step's token is valid, by which time the load has returned.
            if (wg == 0 && tid_opaque() == 0)
                step_error = __hip_atomic_load(args.error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            FLUX_TRACE_POINT(2);
            if (wave == 0) {
                // The workgroup's candidate (valid in thread 0) goes to every copy.
                const float cand_v = __shfl(best_v, 0, kWave);
                const int cand_i = __shfl(static_cast<int>(best_i), 0, kWave);
                ll_store_replicas(ll_arg, 2 * wg, cand_v, ep_arg, lane);
                ll_store_replicas(ll_arg, 2 * wg + 1, __int_as_float(cand_i), ep_arg, lane);
            }
            // Every workgroup reduces all G partials: thread t < G reads partial t, each of
            // the polling waves reduces its 64 with DPP, and every thread then reduces the
            // waves' results from LDS in the same order (so all hold the same token).
            const int poll_waves = (G + kWave - 1) / kWave;
            if (wave < poll_waves) {
                float v = -INFINITY;
                int i = INT32_MAX;
                if (static_cast<int>(tid_opaque()) < G) {
                    const int idx[2] = {2 * static_cast<int>(tid_opaque()), 2 * static_cast<int>(tid_opaque()) + 1};
                    float pv[2];
                    LLIn{ll_arg + replica, ep_arg, wctx}.fetch(idx, pv);
                    v = pv[0];
                    i = __float_as_int(pv[1]);
                }
                wave_argmax_uniform(v, i);
                if (lane == 0) {
                    red_v[wave] = v;
                    red_i[wave] = i;
                }
            }
            __syncthreads();
            float v = red_v[0];
            int64_t i = red_i[0];
            for (int w = 1; w < poll_waves; ++w) {
                if (argmax_precedes(red_v[w], red_i[w], v, i)) {
                    v = red_v[w];
                    i = red_i[w];
                }
            }
            FLUX_TRACE_POINT(3);
            const int64_t next = (i >= 0 && i < args.vocab) ? i : 0;
            if (wg == 0 && tid_opaque() == 0) {
                // A step that ran after any workgroup's wait gave up computed from stale
                // inputs: its token is reported as -1, never as a plausible id.
                const bool failed = step_error != 0 || abort_flag != 0;
                const int64_t reported = failed ? int64_t{-1} : next;
                *args.input_token = reported;
                if (step >= 0 && step < args.generated_capacity) args.generated[step] = reported;
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
    if (wg == 0 && tid_opaque() == 0) {
        // A launch that ended early reports token -1 for the steps it did not compute, so
        // no earlier generation's tokens stay in those slots looking valid.
        if (t < args.steps) {
            for (int r = t; r < args.steps; ++r) {
                const int64_t slot = step + (r - t);
                if (slot >= 0 && slot < args.generated_capacity) args.generated[slot] = -1;
            }
            *args.input_token = -1;
        }
        *args.token_counter = counter0 + static_cast<uint32_t>(args.steps);
    }
}

// ---------------------------------------------------------------------------
// Isolated launchers (tests, per-kernel benchmark): same phase bodies, plain I/O.

__global__ void __launch_bounds__(kThreads) qkv_rope_cache_kernel(const float* hidden, const float* norm_w, float eps,
                                                                  const float* qkv_w, const float* cos_table,
                                                                  const float* sin_table, const int64_t* position_ptr,
                                                                  int64_t capacity, float* key_cache, float* value_cache,
                                                                  float* q_out) {
    const int lane = tid_opaque() & 63;
    const int gw = (tid_opaque() >> 6) * gridDim.x + blockIdx.x;
    const int TW = gridDim.x * kWavesPerWG;
    const int64_t position = *position_ptr;
    if (position < 0 || position >= capacity) return;
    for (int unit = gw; unit < kQKV / 2; unit += TW) {
        QkvUnitWeights w;
        qkv_load(qkv_w, unit, lane, w);
        float h[9], wn[9];
        fetch_slice576(PlainIn{hidden}, lane, h);
        load_slice576(norm_w, lane, wn);
        qkv_unit_compute(w, h, wn, eps, unit, lane,
                         rope_pair(cos_table + position * kHeadDim, sin_table + position * kHeadDim, unit),
                         key_cache + position * kHeadDim, value_cache + position * kHeadDim, capacity * kHeadDim,
                         QkvPlainOut{q_out});
    }
}

__global__ void __launch_bounds__(kThreads) attn_partial_kernel(const float* q_packed, const float* key_cache,
                                                                const float* value_cache, const int64_t* position_ptr,
                                                                int64_t capacity, float scale, int chunks,
                                                                float* partials) {
    __shared__ float red[kAttnRedFloats];
    __shared__ __align__(16) float attn_sp[kAttnSpFloats];
    __shared__ __align__(16) float attn_pl[kAttnPlFloats];
    __shared__ __align__(16) float qv[kGroup * kHeadDim];
    extern __shared__ __align__(16) float part[];
    const int g = blockIdx.x % kKVHeads;
    const int c = blockIdx.x / kKVHeads;
    const int64_t position = *position_ptr;
    if (position < 0 || position >= capacity) return;
    const int64_t attended = position + 1;
    int64_t begin, end;
    chunk_range(attended, chunks, c, begin, end);
    const int rows = static_cast<int>(end - begin);
    if (rows > kAttnRows) return;  // the launcher sizes chunks so this cannot happen
    // Every row including the current one is read from the cache here.
    float* k_lds = part;
    float* v_lds = part + kAttnRows * kHeadDim;
    attn_stage_lds(key_cache + g * capacity * kHeadDim, value_cache + g * capacity * kHeadDim, begin, rows, k_lds,
                   v_lds, 0);
    for (int k = tid_opaque(); k < kGroup * kHeadDim; k += kThreads) qv[k] = q_packed[g * kGroup * kHeadDim + k];
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    attn_compute(k_lds, v_lds, qv, rows, scale * kLog2e, AttnScratch{attn_sp, attn_pl, red},
                 PartialPlainOut{partials + (g * chunks + c) * kGroup * (kHeadDim + 2)});
}

// Merge of one query head's chunk partials.  Every partial word of the head is requested
// at once into LDS (one memory round trip; a loop that loads chunk after chunk waits for
// one round trip per iteration), then thread (dim d = t % 64, slot s = t / 64) sums the
// chunks s, s + 8, ... with weights 2^(m_c - M), and the 8 slots are added in order.
__global__ void __launch_bounds__(kThreads) attn_merge_kernel(const float* partials, int chunks, float* out) {
    __shared__ float red_o[kWavesPerWG][kHeadDim];
    __shared__ float red_l[kWavesPerWG];
    extern __shared__ float staged[];  // chunks * 66: o[64], m, l per chunk
    const int h = blockIdx.x;
    const int g = h / kGroup;
    const int hh = h % kGroup;
    const int lane = tid_opaque() & 63;
    const int wave = tid_opaque() >> 6;
    constexpr int kRow = kHeadDim + 2;
    const float* src = partials + static_cast<int64_t>(g) * chunks * kGroup * kRow + hh * kRow;
    for (int k = tid_opaque(); k < chunks * kRow; k += kThreads) {
        const int c = k / kRow;
        staged[k] = src[static_cast<int64_t>(c) * kGroup * kRow + (k - c * kRow)];
    }
    __syncthreads();
    float M = -INFINITY;
    for (int c = lane; c < chunks; c += kWave) M = fmaxf(M, staged[c * kRow + kHeadDim]);
    M = wave_max_uniform(M);
    float O = 0.0f, L = 0.0f;
    for (int c = wave; c < chunks; c += kWavesPerWG) {
        const float mc = staged[c * kRow + kHeadDim];
        if (mc == -INFINITY) continue;
        const float f = fast_exp2(mc - M);
        O = fmaf(staged[c * kRow + lane], f, O);
        L = fmaf(staged[c * kRow + kHeadDim + 1], f, L);
    }
    red_o[wave][lane] = O;
    if (lane == 0) red_l[wave] = L;
    __syncthreads();
    if (wave == 0) {
        float o = 0.0f, l = 0.0f;
#pragma unroll
        for (int w = 0; w < kWavesPerWG; ++w) {
            o += red_o[w][lane];
            l += red_l[w];
        }
        out[h * kHeadDim + lane] = o / l;
    }
}

__global__ void __launch_bounds__(kThreads) linear576_residual_kernel(const float* x, const float* w, const float* residual,
                                                                      float* out, int rows) {
    const int lane = tid_opaque() & 63;
    const int gw = (tid_opaque() >> 6) * gridDim.x + blockIdx.x;
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
    const int lane = tid_opaque() & 63;
    const int gw = (tid_opaque() >> 6) * gridDim.x + blockIdx.x;
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
    const int lane = tid_opaque() & 63;
    const int gw = (tid_opaque() >> 6) * gridDim.x + blockIdx.x;
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
    const int lane = tid_opaque() & 63;
    const int gw = (tid_opaque() >> 6) * gridDim.x + blockIdx.x;
    const int TW = gridDim.x * kWavesPerWG;
    const int64_t per = (vocab + TW - 1) / TW;
    const int64_t row0 = per * gw < vocab ? per * gw : vocab;
    const int64_t row1 = row0 + per < vocab ? row0 + per : vocab;
    // The first rows are requested before the hidden vector, and each stage's successor
    // before its dot products (lm_rows_pipelined), so the rows stream while a wave computes.
    float wl[kLmBatch][9];
    lm_load(lm_head, row0, row1, lane, wl);
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
    lm_rows_pipelined(lm_head, x, wl, row0, row1, lane, LogitsPlainOut{logits}, best_v, best_i);
    wg_argmax(best_v, best_i, red_v, red_i);
    if (tid_opaque() == 0) {
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
    for (int64_t k = tid_opaque(); k < n; k += kThreads) {
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
    if (tid_opaque() == 0) {
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
// generation_step = step_value, and generated[0] = token when requested; the
// device and host-visible error words (when given) are cleared.
__global__ void install_state_kernel(const int64_t* token_src, int64_t position_value, int64_t step_value,
                                     int write_generated0, int64_t* input_token, int64_t* position,
                                     int64_t* cache_length, int64_t* step, int64_t* generated, int32_t* error,
                                     int32_t* host_error) {
    if (tid_opaque() != 0) return;
    const int64_t token = *token_src;
    *input_token = token;
    *position = position_value;
    *cache_length = position_value;
    *step = step_value;
    if (write_generated0) generated[0] = token;
    if (error != nullptr) __hip_atomic_store(error, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (host_error != nullptr) __hip_atomic_store(host_error, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

}  // namespace

// ---------------------------------------------------------------------------
// Scratch of the allocation-free GQA decode entry point: the split-K partials of one
// call, (chunks x 3 KV heads x 3 query heads x 66) floats for the 85 chunks that cover
// every capacity up to FLUX_MAX_CAPACITY (85 x 224 = 19040 positions): 201,960 bytes.
// Each GPU the library runs on holds its own copy until the process ends.  Every call
// on one GPU shares it: calls that overlap on one GPU race.  Each call writes every
// partial it later merges, so nothing needs clearing between calls.
constexpr int kNoAllocChunks = 85;
constexpr size_t kNoAllocScratchFloats = static_cast<size_t>(kNoAllocChunks) * kKVHeads * kGroup * (kHeadDim + 2);
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

// Host code must not pass `scratch` itself to a kernel (on the host it names a stand-in,
// not the device copy): its device address is looked up once per device, with that
// device current, and kept here.
constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mutex;
static float* g_scratch_address[kMaxScratchDevices] = {};

static hipError_t scratch_address(float** out) {
    int device = -1;
    hipError_t st = hipGetDevice(&device);
    if (st != hipSuccess) return st;
    if (device < 0 || device >= kMaxScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_address[device] == nullptr) {
        void* address = nullptr;
        st = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
        if (st != hipSuccess) return st;
        g_scratch_address[device] = static_cast<float*>(address);
    }
    *out = g_scratch_address[device];
    return hipSuccess;
}

int gqa_decode_noalloc_max_chunks() { return kNoAllocChunks; }

// ---------------------------------------------------------------------------
// Host launchers.

size_t ll_arena_words() { return LLLayout::kTotal; }

#ifdef FLUX_TRACE
extern "C" int flux_debug_trace(uint64_t* host_out) {
    return static_cast<int>(hipMemcpyFromSymbol(host_out, HIP_SYMBOL(g_flux_trace), sizeof(g_flux_trace)));
}
extern "C" int flux_debug_attn_trace(uint64_t* host_out) {
    return static_cast<int>(hipMemcpyFromSymbol(host_out, HIP_SYMBOL(g_flux_attn_trace), sizeof(g_flux_attn_trace)));
}
extern "C" int flux_debug_copy_trace(uint64_t* host_out) {
    return static_cast<int>(hipMemcpyFromSymbol(host_out, HIP_SYMBOL(g_flux_copy_trace), sizeof(g_flux_copy_trace)));
}
extern "C" int flux_debug_trace_all(uint64_t* host_out) {
    return static_cast<int>(hipMemcpyFromSymbol(host_out, HIP_SYMBOL(g_flux_trace_all), sizeof(g_flux_trace_all)));
}
#endif
int fused_decode_threads() { return kThreads; }
size_t fused_decode_dynamic_lds() {
    // K/V staging of one attention chunk (also keeps one workgroup per CU).
    return 2 * kAttnRows * kHeadDim * sizeof(float);
}

int max_attention_positions(int grid) {
    const int chunks = grid / kKVHeads < kMaxAttnChunks ? grid / kKVHeads : kMaxAttnChunks;
    return chunks * kAttnRows;
}

// Cooperative launch: the runtime refuses to start a grid whose workgroups cannot all be
// resident at once (hipErrorCooperativeLaunchTooLarge), instead of letting the resident
// ones wait for the rest until their bounded waits expire.
hipError_t launch_fused_decode(const DecodeArgs& args, int grid, hipStream_t stream, bool cooperative) {
    DecodeArgs copy = args;
    void* params[] = {&copy};
    if (!cooperative)
        return hipLaunchKernel(reinterpret_cast<const void*>(fused_decode_kernel), dim3(grid), dim3(kThreads), params,
                               fused_decode_dynamic_lds(), stream);
    return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(fused_decode_kernel), dim3(grid), dim3(kThreads),
                                      params, static_cast<unsigned int>(fused_decode_dynamic_lds()), stream);
}

void* fused_decode_function() { return reinterpret_cast<void*>(fused_decode_kernel); }

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
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(attn_partial_kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       static_cast<int>(fused_decode_dynamic_lds()));
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(attn_partial_kernel, dim3(kKVHeads * chunks), dim3(kThreads), fused_decode_dynamic_lds(), stream,
                       q, key_cache, value_cache, position, capacity, scale, chunks, partials);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    hipLaunchKernelGGL(attn_merge_kernel, dim3(kQHeads), dim3(kThreads),
                       static_cast<size_t>(chunks) * (kHeadDim + 2) * sizeof(float), stream, partials, chunks, out);
    return hipGetLastError();
}

int gqa_decode_max_positions(int chunks) { return chunks * kAttnRows; }

// The split-K partials go to this GPU's `scratch` copy; no allocation of any kind.
hipError_t launch_gqa_decode_noalloc(const float* q, const float* key_cache, const float* value_cache,
                                     const int64_t* position, int64_t capacity, float scale, int chunks, float* out,
                                     hipStream_t stream) {
    if (chunks < 1 || chunks > kNoAllocChunks) return hipErrorInvalidValue;
    float* partials = nullptr;
    hipError_t st = scratch_address(&partials);
    if (st != hipSuccess) return st;
    return launch_gqa_decode(q, key_cache, value_cache, position, capacity, scale, chunks, partials, out, stream);
}

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
                                int64_t* step, int64_t* generated, int32_t* error, int32_t* host_error,
                                hipStream_t stream) {
    hipLaunchKernelGGL(install_state_kernel, dim3(1), dim3(64), 0, stream, token_src, position_value, step_value,
                       write_generated0 ? 1 : 0, input_token, position, cache_length, step, generated, error,
                       host_error);
    return hipGetLastError();
}

}  // namespace flux
