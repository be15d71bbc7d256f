// gfx950 prefill kernels: FP32-MFMA GEMMs with fused epilogues and a tiled
// online-softmax causal GQA attention on FP32 MFMA.
//
// Reference path: csrc/native_prefill_runtime/native_prefill_runtime_cuda.cu:553-665
// (cuBLAS SGEMM linear_fp32 :285-302, QKV RoPE/cache fill kernel :124-163, SwiGLU
// csrc/packed_swiglu/packed_swiglu_cuda.cu:14-31, residual add :267-278, heads->rows
// :249-265) and csrc/streaming_prefill_gqa/streaming_prefill_gqa_cuda.cu:43-460
// (online softmax with K/V tiles in shared memory, no score materialisation).
//
// MI355X design:
//  * GEMM: 128x128 (or 64x128) block tile, 4 waves in 2x2, each wave 64x64 (32x64)
//    on v_mfma_f32_32x32x2f32; tiles stream HBM -> LDS with global_load_lds.  The
//    epilogue consumes the accumulator layout directly: the two column tiles of a
//    wave hold columns j and j+32 of the same rows, which is exactly the RoPE pair
//    (a 64-column group = one head) and the gate/up pair (gate/up rows are
//    interleaved 32+32 per group).
//  * Attention: one block per (64-query tile, query head); 4 waves x 16 queries.
//    S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_16x16x4f32, so the S^T
//    accumulators are already the B operand of the PV product (no transpose).

#include "flux_common.h"
#include "flux_kernels.h"

#include <cfloat>
#include <cmath>

namespace flux {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBN = 128;        // block tile columns: 2 waves x 64 (one epilogue column group each)
constexpr int kBK = 16;
constexpr int kGemmThreads = 256;

// MFMA 32x32x2 accumulator element r of lane l -> (row, col) inside the 32x32 tile.
__device__ __forceinline__ int mfma32_row(int lane, int r) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

#pragma clang fp contract(off)
__device__ __forceinline__ float rope_lo(float x, float paired, float c, float s) {
    const float a = x * c;
    const float b = (-paired) * s;
    return a + b;
}
__device__ __forceinline__ float rope_hi(float x, float paired, float c, float s) {
    const float a = x * c;
    const float b = paired * s;
    return a + b;
}
#pragma clang fp contract(fast)

// Weight row used for virtual column `col` of the B operand.
template <GemmEpilogue E>
__device__ __forceinline__ int b_row(int col, int n) {
    if constexpr (E == GemmEpilogue::kSwiglu) {
        // Column group t (64 columns) = gate rows [32t, 32t+32) then up rows [half + 32t, ...).
        const int half = n / 2;
        const int t = col >> 6;
        const int v = col & 63;
        return v < 32 ? 32 * t + v : half + 32 * t + (v - 32);
    } else {
        return col;
    }
}

// LDS tile layout (A: BM rows, B: 128 rows; 16 floats of K per row, 64 B): the
// 16-byte piece c of row r sits at piece position c ^ ((r >> 2) & 3), so the 16
// lanes of one ds_read_b128 pass (16 consecutive rows, same piece) cover all banks.
__device__ __forceinline__ int tile_offset(int r, int c) { return r * kBK + 4 * (c ^ ((r >> 2) & 3)); }

// One global_load_lds_dwordx4: each lane copies 16 B from `src` to lds + 16 * lane.
__device__ __forceinline__ void lds_copy16(const float* src, float* lds) {
    __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
}

// C = epilogue(A[M,K] * W[N,K]^T) on v_mfma_f32_32x32x2f32.  Block tile (64*MI) x 128,
// 4 waves in 2 x 2, wave tile (32*MI) x 64.  K is consumed 16 at a time; MFMA
// instruction s (0..7) of a stage pairs K index s (lanes 0-31) with s + 8 (lanes
// 32-63), so each lane reads its 8 K values of a row with two ds_read_b128.
// Tiles stream HBM -> LDS with global_load_lds (no register staging), double buffered.
template <GemmEpilogue E, int MI>
__global__ void __launch_bounds__(kGemmThreads) gemm_kernel(GemmArgs args) {
    constexpr int kBMt = 64 * MI;
    __shared__ __align__(16) float a_s[2][kBMt * kBK];
    __shared__ __align__(16) float b_s[2][kBN * kBK];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 1;  // wave row
    const int wn = wave & 1;   // wave column group (64 columns)
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kBMt;
    const int n0 = blockIdx.x * kBN;
    const int K = args.k;
    const bool group_valid = n0 + wn * 64 < args.n;

    // Rows this wave streams: A blocks i = wave + 4j (16 rows each), B blocks likewise.
    constexpr int kABlocks = kBMt / 16;            // 4 or 8
    constexpr int kAPerWave = kABlocks / 4;        // 1 or 2
    const float* a_src[kAPerWave];
    const float* b_src[2];
#pragma unroll
    for (int j = 0; j < kAPerWave; ++j) {
        const int row = 16 * (wave + 4 * j) + (lane >> 2);
        const int64_t gr = m0 + row < args.m ? m0 + row : args.m - 1;
        a_src[j] = args.a + gr * K + 4 * ((lane & 3) ^ ((row >> 2) & 3));
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int row = 16 * (wave + 4 * j) + (lane >> 2);
        const int col = n0 + row < args.n ? n0 + row : args.n - 1;
        b_src[j] = args.b + static_cast<int64_t>(b_row<E>(col, args.n)) * K + 4 * ((lane & 3) ^ ((row >> 2) & 3));
    }
    auto issue_stage = [&](int k0, int buf) {
#pragma unroll
        for (int j = 0; j < kAPerWave; ++j)
            lds_copy16(a_src[j] + k0, &a_s[buf][(wave + 4 * j) * 16 * kBK]);
#pragma unroll
        for (int j = 0; j < 2; ++j)
            lds_copy16(b_src[j] + k0, &b_s[buf][(wave + 4 * j) * 16 * kBK]);
    };

    f32x16 acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Operand read offsets (floats) inside a tile for this lane: row, pieces 2h and 2h+1.
    const int h = lane >> 5;
    int a_off[MI][2], b_off[2][2];
#pragma unroll
    for (int i = 0; i < MI; ++i) {
        const int r = wm * 32 * MI + 32 * i + (lane & 31);
        a_off[i][0] = tile_offset(r, 2 * h);
        a_off[i][1] = tile_offset(r, 2 * h + 1);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int r = wn * 64 + 32 * j + (lane & 31);
        b_off[j][0] = tile_offset(r, 2 * h);
        b_off[j][1] = tile_offset(r, 2 * h + 1);
    }

    const int stages = K / kBK;
    issue_stage(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int s = 0; s < stages; ++s) {
        const int buf = s & 1;
        if (s + 1 < stages) issue_stage((s + 1) * kBK, buf ^ 1);
        f32x4 av[MI][2], bv[2][2];
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int q = 0; q < 2; ++q) av[i][q] = *reinterpret_cast<const f32x4*>(&a_s[buf][a_off[i][q]]);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 2; ++q) bv[j][q] = *reinterpret_cast<const f32x4*>(&b_s[buf][b_off[j][q]]);
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][kk >> 2][kk & 3], bv[j][kk >> 2][kk & 3],
                                                                   acc[i][j], 0, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(0);  // next stage's tiles have landed in LDS
        __syncthreads();
    }
    if (!group_valid) return;

    // Epilogue: for 32-row subtile i, lane holds columns c (acc[i][0]) and c + 32
    // (acc[i][1]) of the wave's 64-column group for 16 rows.
    const int j = lane & 31;
    const int g0 = n0 + wn * 64;  // first column of the group
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t row = m0 + wm * 32 * MI + 32 * i + mfma32_row(lane, r);
            if (row >= args.m) continue;
            const float lo = acc[i][0][r];
            const float hi = acc[i][1][r];
            if constexpr (E == GemmEpilogue::kStore) {
                args.c[row * args.n + g0 + j] = lo;
                args.c[row * args.n + g0 + 32 + j] = hi;
            } else if constexpr (E == GemmEpilogue::kResidual) {
                const int64_t i0 = row * args.n + g0 + j;
                args.c[i0] = args.residual[i0] + lo;
                args.c[i0 + 32] = args.residual[i0 + 32] + hi;
            } else if constexpr (E == GemmEpilogue::kSwiglu) {
                const int half = args.n / 2;
                args.c[row * half + (g0 >> 1) + j] = silu(lo) * hi;
            } else {  // kQkvRope: the column group is one head; columns j / j+32 are the RoPE pair.
                const int head = g0 / kHeadDim;
                if (head < kQHeads + kKVHeads) {
                    const float* cr = args.rope_cos + row * kHeadDim;
                    const float* sr = args.rope_sin + row * kHeadDim;
                    const float qlo = rope_lo(lo, hi, cr[j], sr[j]);
                    const float qhi = rope_hi(hi, lo, cr[j + 32], sr[j + 32]);
                    float* dst = head < kQHeads
                                     ? args.q_out + (static_cast<int64_t>(head) * args.m + row) * kHeadDim
                                     : args.key_cache +
                                           (static_cast<int64_t>(head - kQHeads) * args.capacity + row) * kHeadDim;
                    dst[j] = qlo;
                    dst[j + 32] = qhi;
                } else {
                    float* dst = args.value_cache +
                                 (static_cast<int64_t>(head - kQHeads - kKVHeads) * args.capacity + row) * kHeadDim;
                    dst[j] = lo;
                    dst[j + 32] = hi;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Causal GQA prefill attention.  The keys of a query tile are split into chunks of
// at most kChunkTiles key tiles; every (query tile, head, chunk) is one block, so
// no block streams more than 2048 keys (the causal tail would otherwise be one
// block per head walking all S keys).  A query tile with one chunk writes its rows
// directly; longer ones write (o, m, l) partials that prefill_attention_merge_kernel
// combines (csrc/streaming_prefill_gqa/streaming_prefill_gqa_cuda.cu splits the keys
// into partitions and merges them the same way).
constexpr int kQTile = 64;
constexpr int kKTile = 64;
constexpr int kAttnThreads = 256;
constexpr int kKVPad = 4;
constexpr int kChunkTiles = 32;
constexpr int kPartialRow = kHeadDim + 2;  // o[64], m, l

__host__ __device__ __forceinline__ int64_t attn_q_tiles(int64_t seq) { return (seq + kQTile - 1) / kQTile; }
__host__ __device__ __forceinline__ int64_t attn_max_chunks(int64_t seq) {
    return (attn_q_tiles(seq) + kChunkTiles - 1) / kChunkTiles;
}
// Blocks of chunk c: query tiles qt >= c * kChunkTiles, times the query heads.
__host__ __device__ __forceinline__ int64_t attn_chunk_blocks(int64_t seq, int64_t c) {
    return (attn_q_tiles(seq) - c * kChunkTiles) * kQHeads;
}
// Partial slot of (qt, h, c) for query tiles with more than one chunk.
__host__ __device__ __forceinline__ int64_t attn_partial_slot(int64_t seq, int64_t qt, int h, int64_t c) {
    return ((qt - kChunkTiles) * kQHeads + h) * attn_max_chunks(seq) + c;
}

__global__ void __launch_bounds__(kAttnThreads) prefill_attention_kernel(const float* __restrict__ q,
                                                                         const float* __restrict__ key_cache,
                                                                         const float* __restrict__ value_cache,
                                                                         int64_t seq, int64_t capacity, float scale,
                                                                         float* __restrict__ workspace,
                                                                         float* __restrict__ out_rows) {
    __shared__ __align__(16) float k_s[kKTile][kHeadDim + kKVPad];
    __shared__ __align__(16) float v_s[kKTile][kHeadDim + kKVPad];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t q_tiles = attn_q_tiles(seq);
    // Block b -> chunk c (chunk-major), then q tile (longest first) and head.
    int64_t idx = blockIdx.x;
    int64_t chunk = 0;
    while (idx >= attn_chunk_blocks(seq, chunk)) {
        idx -= attn_chunk_blocks(seq, chunk);
        ++chunk;
    }
    const int64_t qt = q_tiles - 1 - idx / kQHeads;
    const int h = static_cast<int>(idx % kQHeads);
    const int g = h / kGroup;
    const int64_t q0 = qt * kQTile;
    const int64_t row_base = q0 + wave * 16;
    const int64_t my_row = row_base + (lane & 15);  // query row of this lane in S^T / O^T layouts

    // B operand of S^T = K Q^T.  MFMA instruction s pairs k-slot jg = lane/16 with
    // dim 16 jg + s, so qreg[s] = Q[row = lane%16][16 jg + s] and a lane reads its 16
    // K values of a key row with four ds_read_b128.
    const int jg = lane >> 4;
    float qreg[16];
    {
        const int64_t r = my_row < seq ? my_row : seq - 1;
        const float* qp = q + (static_cast<int64_t>(h) * seq + r) * kHeadDim + 16 * jg;
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
            const float4 v = *reinterpret_cast<const float4*>(qp + 4 * s4);
            qreg[4 * s4] = v.x;
            qreg[4 * s4 + 1] = v.y;
            qreg[4 * s4 + 2] = v.z;
            qreg[4 * s4 + 3] = v.w;
        }
    }

    const float* kg = key_cache + static_cast<int64_t>(g) * capacity * kHeadDim;
    const float* vg = value_cache + static_cast<int64_t>(g) * capacity * kHeadDim;

    f32x4 o_acc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) o_acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;
    float l_run = 0.0f;

    const float scale2 = scale * kLog2e;  // scores in log2 units
    const int64_t last_key = q0 + kQTile - 1 < seq - 1 ? q0 + kQTile - 1 : seq - 1;
    const int64_t k_tiles = last_key / kKTile + 1;
    const int64_t kt_begin = chunk * kChunkTiles;
    const int64_t kt_end = kt_begin + kChunkTiles < k_tiles ? kt_begin + kChunkTiles : k_tiles;
    for (int64_t kt = kt_begin; kt < kt_end; ++kt) {
        const int64_t k0 = kt * kKTile;
        __syncthreads();
        // Stage K and V tiles (64 x 64 each): 1024 float4 per tile, 4 per thread.
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int idx = threadIdx.x + it * kAttnThreads;
            const int row = idx >> 4;
            const int col = (idx & 15) * 4;
            const int64_t key = k0 + row;
            float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
            if (key < seq) {
                kv = *reinterpret_cast<const float4*>(kg + key * kHeadDim + col);
                vv = *reinterpret_cast<const float4*>(vg + key * kHeadDim + col);
            }
            *reinterpret_cast<float4*>(&k_s[row][col]) = kv;
            *reinterpret_cast<float4*>(&v_s[row][col]) = vv;
        }
        __syncthreads();

        // S^T tile: 4 key blocks of 16 x (16 rows), K-dim 64 = 16 MFMA steps.
        f32x4 s_acc[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const float* krow = &k_s[kb * 16 + (lane & 15)][16 * jg];
            f32x4 kr[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) kr[t] = *reinterpret_cast<const f32x4*>(krow + 4 * t);
            s_acc[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 16; ++s)
                s_acc[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[s >> 2][s & 3], qreg[s], s_acc[kb], 0, 0, 0);
        }
        // Scale + causal mask; lane holds keys k0 + 16kb + 4(lane/16) + r for row my_row.
        float tile_max = -INFINITY;
        if (k0 + kKTile - 1 <= row_base) {  // every key of the tile precedes every query of the wave
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    s_acc[kb][r] *= scale2;
                    tile_max = fmaxf(tile_max, s_acc[kb][r]);
                }
        } else {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t key = k0 + 16 * kb + 4 * (lane >> 4) + r;
                    const float v = (key <= my_row && key < seq) ? s_acc[kb][r] * scale2 : -INFINITY;
                    s_acc[kb][r] = v;
                    tile_max = fmaxf(tile_max, v);
                }
            }
        }
        tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 16, kWave));
        tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32, kWave));
        const float m_new = fmaxf(m_run, tile_max);
        const float alpha = m_new == -INFINITY ? 1.0f : (m_run == -INFINITY ? 0.0f : fast_exp2(m_run - m_new));
        float psum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = s_acc[kb][r] == -INFINITY ? 0.0f : fast_exp2(s_acc[kb][r] - m_new);
                s_acc[kb][r] = p;
                psum += p;
            }
        }
        psum += __shfl_xor(psum, 16, kWave);
        psum += __shfl_xor(psum, 32, kWave);
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int db = 0; db < 4; ++db) o_acc[db] *= alpha;
        // O^T += V^T P^T: k-step (kb, r) uses keys 16kb + 4(lane/16) + r.
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int krow = 16 * kb + 4 * (lane >> 4) + r;
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const float a = v_s[krow][16 * db + (lane & 15)];
                    o_acc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, s_acc[kb][r], o_acc[db], 0, 0, 0);
                }
            }
        }
    }
    // O^T accumulator: lane holds d = 16db + 4(lane/16) + r for row my_row.
    if (my_row >= seq) return;
    if (k_tiles <= kChunkTiles) {
        const float inv = 1.0f / l_run;
        float* dst = out_rows + my_row * kHidden + h * kHeadDim;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[16 * db + 4 * (lane >> 4) + r] = o_acc[db][r] * inv;
        }
    } else {
        float* dst = workspace + (attn_partial_slot(seq, qt, h, chunk) * kQTile + (my_row - q0)) * kPartialRow;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[16 * db + 4 * (lane >> 4) + r] = o_acc[db][r];
        }
        if (lane < 16) {
            dst[kHeadDim] = m_run;  // log2 units
            dst[kHeadDim + 1] = l_run;
        }
    }
}

// Combines the chunk partials of query tiles with more than one chunk.  Block
// ((qt - kChunkTiles) * 9 + h) * 16 + row group; thread t -> row 4 * group + t / 64,
// dim t % 64.  All chunk loads of a thread are issued before the combine.
constexpr int kMergeMaxChunks = 8;  // kMaxCapacity / (kChunkTiles * kKTile)

__global__ void __launch_bounds__(kAttnThreads) prefill_attention_merge_kernel(const float* __restrict__ workspace,
                                                                               int64_t seq,
                                                                               float* __restrict__ out_rows) {
    const int64_t tile_head = blockIdx.x / (kQTile / 4);
    const int64_t qt = kChunkTiles + tile_head / kQHeads;
    const int h = static_cast<int>(tile_head % kQHeads);
    const int row = static_cast<int>(blockIdx.x % (kQTile / 4)) * 4 + static_cast<int>(threadIdx.x >> 6);
    const int d = threadIdx.x & 63;
    const int64_t q0 = qt * kQTile;
    if (q0 + row >= seq) return;
    const int64_t last_key = q0 + kQTile - 1 < seq - 1 ? q0 + kQTile - 1 : seq - 1;
    const int chunks = static_cast<int>((last_key / kKTile + kChunkTiles) / kChunkTiles);
    float o[kMergeMaxChunks], m[kMergeMaxChunks], l[kMergeMaxChunks];
#pragma unroll
    for (int c = 0; c < kMergeMaxChunks; ++c) {
        if (c < chunks) {
            const float* p = workspace + (attn_partial_slot(seq, qt, h, c) * kQTile + row) * kPartialRow;
            o[c] = p[d];
            m[c] = p[kHeadDim];
            l[c] = p[kHeadDim + 1];
        } else {
            o[c] = 0.0f;
            m[c] = -INFINITY;
            l[c] = 0.0f;
        }
    }
    float M = -INFINITY;
#pragma unroll
    for (int c = 0; c < kMergeMaxChunks; ++c) M = fmaxf(M, m[c]);
    float O = 0.0f, L = 0.0f;
#pragma unroll
    for (int c = 0; c < kMergeMaxChunks; ++c) {
        const float f = m[c] == -INFINITY ? 0.0f : fast_exp2(m[c] - M);
        O = fmaf(o[c], f, O);
        L = fmaf(l[c], f, L);
    }
    out_rows[(q0 + row) * kHidden + h * kHeadDim + d] = O / L;
}

__global__ void embedding_gather_kernel(const int64_t* ids, const float* embedding, int64_t vocab, int64_t seq,
                                        float* hidden) {
    const int64_t total = seq * (kHidden / 4);
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t row = i / (kHidden / 4);
        const int64_t col = (i % (kHidden / 4)) * 4;
        const int64_t token = ids[row];
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (token >= 0 && token < vocab) v = *reinterpret_cast<const float4*>(embedding + token * kHidden + col);
        *reinterpret_cast<float4*>(hidden + row * kHidden + col) = v;
    }
}

}  // namespace

hipError_t launch_gemm(const GemmArgs& args, GemmEpilogue epilogue, hipStream_t stream) {
    if (args.k % kBK != 0 || args.n % 64 != 0 || args.m <= 0) return hipErrorInvalidValue;
    if (epilogue == GemmEpilogue::kSwiglu && args.n % kBN != 0) return hipErrorInvalidValue;
    if (epilogue == GemmEpilogue::kQkvRope && args.n != kQKV) return hipErrorInvalidValue;
    // 128-row tiles when they already give the device two blocks per CU, else 64-row tiles.
    const unsigned gx = static_cast<unsigned>((args.n + kBN - 1) / kBN);
    const bool big = static_cast<int64_t>(gx) * ((args.m + 127) / 128) >= 512;
    const dim3 grid(gx, static_cast<unsigned>(big ? (args.m + 127) / 128 : (args.m + 63) / 64));
    const dim3 block(kGemmThreads);
#define FLUX_LAUNCH_GEMM(E)                                                                    \
    do {                                                                                       \
        if (big)                                                                               \
            hipLaunchKernelGGL(HIP_KERNEL_NAME(gemm_kernel<E, 2>), grid, block, 0, stream, args);             \
        else                                                                                   \
            hipLaunchKernelGGL(HIP_KERNEL_NAME(gemm_kernel<E, 1>), grid, block, 0, stream, args);             \
    } while (0)
    switch (epilogue) {
        case GemmEpilogue::kStore:
            FLUX_LAUNCH_GEMM(GemmEpilogue::kStore);
            break;
        case GemmEpilogue::kResidual:
            FLUX_LAUNCH_GEMM(GemmEpilogue::kResidual);
            break;
        case GemmEpilogue::kSwiglu:
            FLUX_LAUNCH_GEMM(GemmEpilogue::kSwiglu);
            break;
        case GemmEpilogue::kQkvRope:
            FLUX_LAUNCH_GEMM(GemmEpilogue::kQkvRope);
            break;
    }
#undef FLUX_LAUNCH_GEMM
    return hipGetLastError();
}

size_t prefill_attention_workspace_floats(int64_t seq) {
    const int64_t long_tiles = attn_q_tiles(seq) - kChunkTiles;
    if (long_tiles <= 0) return 0;
    return static_cast<size_t>(long_tiles * kQHeads * attn_max_chunks(seq) * kQTile * kPartialRow);
}

hipError_t launch_prefill_attention(const float* q, const float* key_cache, const float* value_cache, int64_t seq,
                                    int64_t capacity, float scale, float* workspace, float* out_rows,
                                    hipStream_t stream) {
    if (seq <= 0 || seq > capacity) return hipErrorInvalidValue;
    if (prefill_attention_workspace_floats(seq) > 0 && workspace == nullptr) return hipErrorInvalidValue;
    if (attn_max_chunks(seq) > kMergeMaxChunks) return hipErrorInvalidValue;
    int64_t blocks = 0;
    for (int64_t c = 0; c < attn_max_chunks(seq); ++c) blocks += attn_chunk_blocks(seq, c);
    hipLaunchKernelGGL(prefill_attention_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kAttnThreads), 0, stream, q,
                       key_cache, value_cache, seq, capacity, scale, workspace, out_rows);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    const int64_t long_tiles = attn_q_tiles(seq) - kChunkTiles;
    if (long_tiles > 0) {
        hipLaunchKernelGGL(prefill_attention_merge_kernel,
                           dim3(static_cast<unsigned>(long_tiles * kQHeads * (kQTile / 4))), dim3(kAttnThreads), 0,
                           stream, workspace, seq, out_rows);
        st = hipGetLastError();
    }
    return st;
}

hipError_t launch_embedding_gather(const int64_t* ids, const float* embedding, int64_t vocab, int64_t seq,
                                   float* hidden, hipStream_t stream) {
    const int64_t total = seq * (kHidden / 4);
    const int grid = static_cast<int>((total + 255) / 256 < 16384 ? (total + 255) / 256 : 16384);
    hipLaunchKernelGGL(embedding_gather_kernel, dim3(grid), dim3(256), 0, stream, ids, embedding, vocab, seq, hidden);
    return hipGetLastError();
}

}  // namespace flux
