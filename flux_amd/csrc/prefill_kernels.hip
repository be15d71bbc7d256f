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
//    interleaved 32+32 per group).  N = 576 outputs (o_proj, down) use 64x64 tiles.
//    Grids smaller than the device (short prompts) use copy-ring variants, or, for
//    K = 576 / 1536, a split-K kernel whose waves stream private LDS rings and which
//    folds the preceding RMSNorm into the QKV and gate/up GEMMs.  Grids that leave CUs
//    idle split K over blocks into partial planes, summed in order by a reduce kernel,
//    or by the RMSNorm kernel that the next GEMM needs (split_reduce_residual_norm_kernel).
//  * Attention: one block per (128-query tile, query head, key chunk); 4 waves x 32
//    queries (prompts up to 512 tokens: one block per 32-query tile and head, its
//    32-key chunks spread over 8 waves and combined in LDS).  S^T = K Q^T and
//    O^T += V^T P^T on v_mfma_f32_32x32x2f32, so the S^T
//    accumulators are already the B operand of the PV product (no transpose).  The
//    chunk length follows the prompt length; chunk partials are merged by a second
//    kernel.

#include "flux_common.h"
#include "flux_kernels.h"

#include <cfloat>
#include <cmath>
#include <type_traits>

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

// Epilogue of one wave's (32*MI) x 64 tile whose first row is row0 and whose column
// group (one head for RoPE, one gate/up pair for SwiGLU) starts at column g0.
// One output row of a wave's 64-column group: lo is column g0 + j, hi is column g0 + 32 + j.
template <GemmEpilogue E>
__device__ __forceinline__ void gemm_store_pair(const GemmArgs& args, int64_t row, int g0, int j, float lo, float hi) {
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
                             : args.key_cache + (static_cast<int64_t>(head - kQHeads) * args.capacity + row) * kHeadDim;
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

// One output value of the plain or residual epilogue.
template <GemmEpilogue E>
__device__ __forceinline__ void gemm_store_one(const GemmArgs& args, int64_t row, int col, float v) {
    static_assert(E == GemmEpilogue::kStore || E == GemmEpilogue::kResidual, "plain epilogues only");
    const int64_t i0 = row * args.n + col;
    if constexpr (E == GemmEpilogue::kResidual) {
        args.c[i0] = args.residual[i0] + v;
    } else {
        args.c[i0] = v;
    }
}

template <GemmEpilogue E, int MI>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& args, const f32x16 (&acc)[MI][2], int64_t row0, int g0,
                                              int lane) {
    // Epilogue: for 32-row subtile i, lane holds columns c (acc[i][0]) and c + 32
    // (acc[i][1]) of the wave's 64-column group for 16 rows.
    const int j = lane & 31;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t row = row0 + 32 * i + mfma32_row(lane, r);
            if (row >= args.m) continue;
            gemm_store_pair<E>(args, row, g0, j, acc[i][0][r], acc[i][1][r]);
        }
    }
}

// C = epilogue(A[M,K] * W[N,K]^T) on v_mfma_f32_32x32x2f32.  Block tile (32*MI*kWaves/2) x 128,
// kWaves waves in kWaves/2 x 2, wave tile (32*MI) x 64.  The 128-row tile of QKV runs as 8 waves
// of 32 x 64 (MI = 1) rather than 4 of 64 x 64: its 512 blocks fill the device in one round at
// two per CU, and four waves per SIMD hide the operand reads and epilogue better than two
// (8192 tokens: 34.89 -> 34.75 ms; gate/up, three rounds deep, was slower that way).
// K is consumed 16 at a time; MFMA instruction s (0..7) of a stage pairs K index s (lanes
// 0-31) with s + 8 (lanes 32-63), so each lane reads its 8 K values of a row with two
// ds_read_b128.
// Tiles stream HBM -> LDS with global_load_lds (no register staging), double buffered.
template <GemmEpilogue E, int MI, int kWaves = 4>
__global__ void __launch_bounds__(64 * kWaves) gemm_kernel(GemmArgs args) {
    static_assert(kWaves == 4 || kWaves == 8, "waves in kWaves / 2 rows x 2 column groups");
    constexpr int kBMt = 32 * MI * (kWaves / 2);
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

    // Rows this wave streams: A blocks i = wave + kWaves j (16 rows each), B blocks likewise.
    constexpr int kAPerWave = kBMt / 16 / kWaves;  // 1 or 2
    constexpr int kBPerWave = kBN / 16 / kWaves;   // 2 or 1
    const float* a_src[kAPerWave];
    const float* b_src[kBPerWave];
#pragma unroll
    for (int j = 0; j < kAPerWave; ++j) {
        const int row = 16 * (wave + kWaves * j) + (lane >> 2);
        const int64_t gr = m0 + row < args.m ? m0 + row : args.m - 1;
        a_src[j] = args.a + gr * K + 4 * ((lane & 3) ^ ((row >> 2) & 3));
    }
#pragma unroll
    for (int j = 0; j < kBPerWave; ++j) {
        const int row = 16 * (wave + kWaves * j) + (lane >> 2);
        const int col = n0 + row < args.n ? n0 + row : args.n - 1;
        b_src[j] = args.b + static_cast<int64_t>(b_row<E>(col, args.n)) * K + 4 * ((lane & 3) ^ ((row >> 2) & 3));
    }
    auto issue_stage = [&](int k0, int buf) {
#pragma unroll
        for (int j = 0; j < kAPerWave; ++j)
            lds_copy16(a_src[j] + k0, &a_s[buf][(wave + kWaves * j) * 16 * kBK]);
#pragma unroll
        for (int j = 0; j < kBPerWave; ++j)
            lds_copy16(b_src[j] + k0, &b_s[buf][(wave + kWaves * j) * 16 * kBK]);
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
        if constexpr (E == GemmEpilogue::kSwiglu) {
            // Written accumulator by accumulator: the compiler then schedules the stage's
            // operand reads and barrier ahead of its MFMAs, which measured 4% faster for
            // this shape (and slower for the others).
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int kk = 0; kk < 8; ++kk)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][kk >> 2][kk & 3],
                                                                       bv[j][kk >> 2][kk & 3], acc[i][j], 0, 0, 0);
        } else {
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][kk >> 2][kk & 3],
                                                                       bv[j][kk >> 2][kk & 3], acc[i][j], 0, 0, 0);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // next stage's tiles have landed in LDS
        __syncthreads();
    }
    if (!group_valid) return;
    gemm_epilogue<E, MI>(args, acc, m0 + wm * 32 * MI, n0 + wn * 64, lane);
}

// Waits until at most N vector-memory operations of this wave are outstanding
// (vmcnt only; the LDS and export counters are left alone).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit field");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Barrier for LDS hand-offs: this wave's LDS reads are complete and no memory access
// moves across it; global-memory copies still in flight are not waited for (each
// wave waits for its own with vmcnt where needed).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// gemm_kernel for grids smaller than the device (short prompts): with one block per
// CU or fewer nothing hides a block's copy latency, so stages stream through a ring
// of four buffers, three copies in flight (each buffer its own LDS variable so reads
// of one never wait on copies into another).  Step s reads stage s, starts the copy
// of stage s + 3 into the buffer stage s - 1 used, multiplies, then waits for stage
// s + 1.  The step count is rounded up to a multiple of 4 and copies past the last
// stage repeat it, so every step issues and waits alike; surplus steps skip the MFMAs.
template <GemmEpilogue E, int MI>
__global__ void __launch_bounds__(kGemmThreads) gemm_ring_kernel(GemmArgs args) {
    constexpr int kNS = 4;
    constexpr int kBMt = 64 * MI;
    __shared__ __align__(16) float a_s0[kBMt * kBK];
    __shared__ __align__(16) float a_s1[kBMt * kBK];
    __shared__ __align__(16) float a_s2[kBMt * kBK];
    __shared__ __align__(16) float a_s3[kBMt * kBK];
    __shared__ __align__(16) float b_s0[kBN * kBK];
    __shared__ __align__(16) float b_s1[kBN * kBK];
    __shared__ __align__(16) float b_s2[kBN * kBK];
    __shared__ __align__(16) float b_s3[kBN * kBK];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 1;
    const int wn = wave & 1;
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kBMt;
    const int n0 = blockIdx.x * kBN;
    const int K = args.k;
    const bool group_valid = n0 + wn * 64 < args.n;

    constexpr int kAPerWave = kBMt / 64;
    constexpr int kLoads = kAPerWave + 2;  // global_load_lds per wave per stage
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
    auto abuf = [&](auto bi) -> float* {
        constexpr int b = decltype(bi)::value;
        if constexpr (b == 0) return a_s0;
        else if constexpr (b == 1) return a_s1;
        else if constexpr (b == 2) return a_s2;
        else return a_s3;
    };
    auto bbuf = [&](auto bi) -> float* {
        constexpr int b = decltype(bi)::value;
        if constexpr (b == 0) return b_s0;
        else if constexpr (b == 1) return b_s1;
        else if constexpr (b == 2) return b_s2;
        else return b_s3;
    };
    const int stages = K / kBK;
    auto issue = [&](auto bi, int st) {
        const int k0 = (st < stages ? st : stages - 1) * kBK;
        float* as = abuf(bi);
        float* bs = bbuf(bi);
#pragma unroll
        for (int j = 0; j < kAPerWave; ++j) lds_copy16(a_src[j] + k0, as + (wave + 4 * j) * 16 * kBK);
#pragma unroll
        for (int j = 0; j < 2; ++j) lds_copy16(b_src[j] + k0, bs + (wave + 4 * j) * 16 * kBK);
    };

    f32x16 acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
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

    auto step = [&](auto bi, int s) {
        constexpr int b = decltype(bi)::value;
        const float* as = abuf(bi);
        const float* bs = bbuf(bi);
        f32x4 av[MI][2], bv[2][2];
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int q = 0; q < 2; ++q) av[i][q] = *reinterpret_cast<const f32x4*>(as + a_off[i][q]);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 2; ++q) bv[j][q] = *reinterpret_cast<const f32x4*>(bs + b_off[j][q]);
        issue(std::integral_constant<int, (b + kNS - 1) % kNS>{}, s + kNS - 1);
        if (s < stages) {
#pragma unroll
            for (int kk = 0; kk < 8; ++kk)
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][kk >> 2][kk & 3],
                                                                       bv[j][kk >> 2][kk & 3], acc[i][j], 0, 0, 0);
        }
        wait_vmcnt<(kNS - 2) * kLoads>();
        lds_barrier();
    };
    issue(std::integral_constant<int, 0>{}, 0);
    issue(std::integral_constant<int, 1>{}, 1);
    issue(std::integral_constant<int, 2>{}, 2);
    wait_vmcnt<(kNS - 2) * kLoads>();
    lds_barrier();
    for (int s = 0; s < stages; s += kNS) {
        step(std::integral_constant<int, 0>{}, s);
        step(std::integral_constant<int, 1>{}, s + 1);
        step(std::integral_constant<int, 2>{}, s + 2);
        step(std::integral_constant<int, 3>{}, s + 3);
    }
    wait_vmcnt<0>();  // no copy may still be landing in LDS when the block retires
    if (!group_valid) return;
    gemm_epilogue<E, MI>(args, acc, m0 + wm * 32 * MI, n0 + wn * 64, lane);
}

// Grids smaller than the device (short and mid-length prompts): one block per
// (32 * RT) x 64 output tile, RT = 1, 2 or 4.  Its kSplitWaves waves are RT row tiles
// of 32 times kSplitWaves / RT contiguous K ranges.  A wave streams its 32 A rows and the
// tile's 64 B rows over its K range, 16 K values (64 bytes per row) at a time, laid out
// and swizzled as in gemm_kernel, through a private ring of kSplitStages LDS buffers;
// while a stage's MFMAs run, the next stage's operands are already in registers and the
// kSplitStages - 2 after it are being copied.  No wave waits for another until the
// partial tiles of one row tile meet in LDS (RT < 4).  They are summed in K order (the
// result does not depend on timing), and the row tile's waves share its epilogue.
constexpr int kSplitWaves = 4;
constexpr int kSplitStages = 5;

template <int S, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (S < N) {
        f(std::integral_constant<int, S>{});
        static_for<S + 1, N>(f);
    }
}

// kStages = K / (kSplitWaves / RT * 16), fixed at compile time so the stage loop is
// straight-line code and every wait names exactly the copies it needs.
// kKB > 1: blockIdx.x = column tile * kKB + kb, and block kb covers the kb-th third of K;
// instead of the epilogue it writes its summed tile (and its rows' partial sums of squares)
// to partial plane kb of args.split_partials for gemm_split_reduce_kernel.
template <GemmEpilogue E, int kStages, int RT, bool kNorm, int kCols, int kKB>
__global__ void __launch_bounds__(64 * kSplitWaves) gemm_split_kernel(GemmArgs args) {
    static_assert(kSplitStages == 5, "the buffers below are spelled out");
    static_assert(RT == 1 || RT == 2 || RT == 4, "row tiles per block");
    // kCols = 64 (two 32-column MFMA tiles: the RoPE / SwiGLU pair layout) or 32 (plain and
    // residual epilogues only: twice the blocks, half the MFMAs per wave).
    static_assert(kCols == 64 || (kCols == 32 && !kNorm &&
                                  (E == GemmEpilogue::kStore || E == GemmEpilogue::kResidual)),
                  "32-column tiles carry no column pairs");
    constexpr int kTiles = kCols / 32;
    constexpr int kRows = 32 + kCols;  // A rows + B rows per stage
    constexpr int kCopies = kRows / 16;
    constexpr int kParts = kSplitWaves / RT;  // K ranges per row tile
    // One variable per ring slot: a read of one slot then never waits for copies into another.
    __shared__ __align__(16) float r0[kSplitWaves][kRows * kBK];
    __shared__ __align__(16) float r1[kSplitWaves][kRows * kBK];
    __shared__ __align__(16) float r2[kSplitWaves][kRows * kBK];
    __shared__ __align__(16) float r3[kSplitWaves][kRows * kBK];
    __shared__ __align__(16) float r4[kSplitWaves][kRows * kBK];
    __shared__ float partial[kParts > 1 ? kSplitWaves : 1][kTiles][16][64];
    __shared__ __align__(16) float norm_g[kNorm ? kHidden : 4];  // folded RMSNorm: weights of the K values
    __shared__ float norm_ss[kNorm ? kSplitWaves : 1][32];       // folded RMSNorm: sums of squares per row

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row_tile = wave % RT;
    const int part = wave / RT;
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * 32 * RT + 32 * row_tile;
    const int kb = kKB > 1 ? static_cast<int>(blockIdx.x % kKB) : 0;
    const int n0 = static_cast<int>(blockIdx.x / kKB) * kCols;
    const int K = args.k;
    constexpr int kSpan = kStages * kBK;  // this wave's K values start at (kb * kParts + part) * kSpan
    const int k_first = (kb * kParts + part) * kSpan;
    static_assert(!kNorm || kStages * kBK * kParts * kKB == kHidden, "the folded norm spans the hidden width");
    // Folded RMSNorm: the norm weights are requested before the first copies and stored to LDS
    // after them, so their latency overlaps the copies'.
    constexpr int kNormLoads = (kHidden + 64 * kSplitWaves - 1) / (64 * kSplitWaves);
    float norm_load[kNormLoads];
    if constexpr (kNorm) {
#pragma unroll
        for (int i = 0; i < kNormLoads; ++i) {
            const int k = threadIdx.x + 64 * kSplitWaves * i;
            norm_load[i] = k < kHidden ? args.norm_weight[k] : 0.0f;
        }
    }
    float ss = 0.0f;

    const float* src[kCopies];
#pragma unroll
    for (int i = 0; i < kCopies; ++i) {
        const int row = 16 * i + (lane >> 2);
        const int piece = (lane & 3) ^ ((row >> 2) & 3);
        const float* base;
        if (row < 32) {
            const int64_t ga = m0 + row < args.m ? m0 + row : args.m - 1;
            base = args.a + ga * K;
        } else {
            base = args.b + static_cast<int64_t>(b_row<E>(n0 + row - 32, args.n)) * K;
        }
        src[i] = base + k_first + 4 * piece;
    }
    auto slot = [&](auto bi) -> float* {
        constexpr int b = decltype(bi)::value % kSplitStages;
        if constexpr (b == 0) return r0[wave];
        else if constexpr (b == 1) return r1[wave];
        else if constexpr (b == 2) return r2[wave];
        else if constexpr (b == 3) return r3[wave];
        else return r4[wave];
    };
    auto issue = [&](auto st) {
        float* dst = slot(st);
#pragma unroll
        for (int i = 0; i < kCopies; ++i) lds_copy16(src[i] + decltype(st)::value * kBK, dst + i * 16 * kBK);
    };

    const int h = lane >> 5;
    const int ra = lane & 31;
    const int a_off0 = tile_offset(ra, 2 * h), a_off1 = tile_offset(ra, 2 * h + 1);
    int b_off[kTiles][2];
    f32x16 acc[kTiles];
#pragma unroll
    for (int j = 0; j < kTiles; ++j) {
        b_off[j][0] = tile_offset(32 + 32 * j + ra, 2 * h);
        b_off[j][1] = tile_offset(32 + 32 * j + ra, 2 * h + 1);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
    }
    struct Operands {
        f32x4 a[2];
        f32x4 b[kTiles][2];
        f32x4 g[2];  // folded RMSNorm: the weights of the a values
    };
    auto read = [&](auto st, Operands& o) {
        const float* t = slot(st);
        o.a[0] = *reinterpret_cast<const f32x4*>(t + a_off0);
        o.a[1] = *reinterpret_cast<const f32x4*>(t + a_off1);
        if constexpr (kNorm) {
            // This lane's K values: pieces 2h and 2h + 1 of the stage.
            const float* g = norm_g + k_first + decltype(st)::value * kBK + 8 * h;
            o.g[0] = *reinterpret_cast<const f32x4*>(g);
            o.g[1] = *reinterpret_cast<const f32x4*>(g + 4);
        }
#pragma unroll
        for (int j = 0; j < kTiles; ++j)
#pragma unroll
            for (int q = 0; q < 2; ++q) o.b[j][q] = *reinterpret_cast<const f32x4*>(t + b_off[j][q]);
    };
    // Folded RMSNorm: accumulate the squares of a stage's raw A values, then scale them by the
    // norm weights of their K indices.
    auto fold_norm = [&](Operands& o) {
        if constexpr (kNorm) {
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    ss = fmaf(o.a[q][e], o.a[q][e], ss);
                    o.a[q][e] *= o.g[q][e];
                }
        }
    };
    constexpr int kAhead = kSplitStages - 1;  // stages issued before the loop
    static_for<0, (kStages < kAhead ? kStages : kAhead)>([&](auto st) { issue(st); });
    if constexpr (kNorm) {
#pragma unroll
        for (int i = 0; i < kNormLoads; ++i) {
            const int k = threadIdx.x + 64 * kSplitWaves * i;
            if (k < kHidden) norm_g[k] = norm_load[i];
        }
        lds_barrier();  // waits for LDS traffic only, not for the copies in flight
    }
    Operands cur, nxt;
    wait_vmcnt<((kStages < kAhead ? kStages : kAhead) - 1) * kCopies>();
    read(std::integral_constant<int, 0>{}, cur);
    fold_norm(cur);
    static_for<0, kStages>([&](auto st) {
        constexpr int s = decltype(st)::value;
        // Slot (s + kAhead) % kSplitStages last held stage s - 1, whose operands were read in
        // step s - 2 and consumed in step s - 1.
        if constexpr (s + 1 < kStages) {
            constexpr int newest = s + kAhead - 1 < kStages ? s + kAhead - 1 : kStages - 1;
            wait_vmcnt<(newest - s - 1) * kCopies>();
            read(std::integral_constant<int, s + 1>{}, nxt);
        }
        if constexpr (s + kAhead < kStages) issue(std::integral_constant<int, s + kAhead>{});
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
#pragma unroll
            for (int j = 0; j < kTiles; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.a[kk >> 2][kk & 3], cur.b[j][kk >> 2][kk & 3], acc[j],
                                                              0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        // The folded norm scales the next stage's operands once this stage's MFMAs have issued:
        // its reads have landed by then, and no MFMA in flight reads those registers.
        if constexpr (s + 1 < kStages) fold_norm(nxt);
        cur = nxt;
    });
    wait_vmcnt<0>();  // no copy may still be landing in LDS when the block retires
    if constexpr (kNorm) {
        ss += __shfl_xor(ss, 32, 64);  // the two K halves of the lane's row
        if (lane < 32) norm_ss[wave][lane] = ss;
    }
    // Inverse RMS of output row `row` (0..31) of this wave's row tile, summed over the K parts
    // in order; read after the block barrier below (kParts > 1) or this wave's own writes.
    auto row_scale = [&](int row) {
        float total = norm_ss[kNorm ? row_tile : 0][row];
#pragma unroll
        for (int p = 1; p < kParts; ++p) total += norm_ss[kNorm ? row_tile + RT * p : 0][row];
        return rms_inverse(total, kHidden, args.norm_eps);
    };
    if constexpr (kKB > 1) {
        // Partial plane kb: this block's sums over its K range, unscaled; the norm's partial
        // sums of squares per row go after the planes.
        float* plane = args.split_partials + static_cast<int64_t>(kb) * args.m * args.n;
        float* plane_ss = args.split_partials + static_cast<int64_t>(kKB) * args.m * args.n +
                          static_cast<int64_t>(kb) * args.m;
        if constexpr (kParts == 1) {
#pragma unroll
            for (int j = 0; j < kTiles; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t out_row = m0 + mfma32_row(lane, r);
                    if (out_row < args.m) plane[out_row * args.n + n0 + 32 * j + (lane & 31)] = acc[j][r];
                }
            if constexpr (kNorm) {
                if (lane < 32 && m0 + lane < args.m) plane_ss[m0 + lane] = norm_ss[row_tile][lane];
            }
        } else {
#pragma unroll
            for (int j = 0; j < kTiles; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) partial[wave][j][r][lane] = acc[j][r];
            __syncthreads();
            const int j = lane & 31;
#pragma unroll
            for (int u = 0; u < 16 / kParts; ++u) {
                const int r = (16 / kParts) * part + u;
                float lo = partial[row_tile][0][r][lane], hi = partial[row_tile][kTiles - 1][r][lane];
#pragma unroll
                for (int p = 1; p < kParts; ++p) {
                    lo += partial[row_tile + RT * p][0][r][lane];
                    hi += partial[row_tile + RT * p][kTiles - 1][r][lane];
                }
                const int64_t out_row = m0 + mfma32_row(lane, r);
                if (out_row >= args.m) continue;
                plane[out_row * args.n + n0 + j] = lo;
                if constexpr (kCols == 64) plane[out_row * args.n + n0 + 32 + j] = hi;
            }
            if constexpr (kNorm) {
                if (part == 0 && lane < 32 && m0 + lane < args.m) {
                    float total = norm_ss[row_tile][lane];
#pragma unroll
                    for (int p = 1; p < kParts; ++p) total += norm_ss[row_tile + RT * p][lane];
                    plane_ss[m0 + lane] = total;
                }
            }
        }
    } else if constexpr (kParts == 1 && kCols == 32) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t out_row = m0 + mfma32_row(lane, r);
            if (out_row < args.m) gemm_store_one<E>(args, out_row, n0 + (lane & 31), acc[0][r]);
        }
    } else if constexpr (kParts == 1) {
        if constexpr (kNorm) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float inv = row_scale(mfma32_row(lane, r));
                acc[0][r] *= inv;
                acc[1][r] *= inv;
            }
        }
        const f32x16(&whole)[1][2] = reinterpret_cast<const f32x16(&)[1][kTiles]>(acc);
        gemm_epilogue<E, 1>(args, whole, m0, n0, lane);
    } else {
#pragma unroll
        for (int j = 0; j < kTiles; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) partial[wave][j][r][lane] = acc[j][r];
        __syncthreads();
        const int j = lane & 31;
#pragma unroll
        for (int u = 0; u < 16 / kParts; ++u) {
            const int r = (16 / kParts) * part + u;
            float lo = partial[row_tile][0][r][lane], hi = partial[row_tile][kTiles - 1][r][lane];
#pragma unroll
            for (int p = 1; p < kParts; ++p) {
                lo += partial[row_tile + RT * p][0][r][lane];
                hi += partial[row_tile + RT * p][kTiles - 1][r][lane];
            }
            if constexpr (kNorm) {
                const float inv = row_scale(mfma32_row(lane, r));
                lo *= inv;
                hi *= inv;
            }
            const int64_t out_row = m0 + mfma32_row(lane, r);
            if (out_row >= args.m) continue;
            if constexpr (kCols == 64) gemm_store_pair<E>(args, out_row, n0, j, lo, hi);
            else gemm_store_one<E>(args, out_row, n0 + j, lo);
        }
    }
}

// Small-M GEMM on v_mfma_f32_16x16x4f32 with the operands loaded straight into registers.
// Block = kRegWaves waves (three per SIMD), output tile (16 RT) rows x kCols columns; wave w
// sums the w-th of kRegWaves contiguous K slices (48 values at K = 576).  Lane l loads float4s
// of four consecutive K values from memory (L2): A rows l % 16 (+ 16 rt), B columns l % 16
// (+ 16 jb), K values 4 (l / 16) .. + 3 of each 16-value stage, so k-step s of the stage pairs
// component s of every operand (the MFMA's K index l / 16 stands for K value 4 (l / 16) + s).
// A ring of kDepth stages is in flight; at K = 576 it holds the whole slice, so each wave
// issues all of its loads at once and pays one memory round trip.  The LDS ring of
// gemm_split_kernel is shallower than a round trip at one wave per SIMD, and its K split
// needs a reduce kernel.  The waves' partial tiles are summed in LDS in K order and the block
// shares the epilogue.
constexpr int kRegWaves = 12;

// Scheduling barriers keep every load where it is issued: left free, the compiler sinks the
// loads to their uses (fewer live registers) and the ring is gone.
template <int kStages, int kDepth, typename Issue, typename Compute>
__device__ __forceinline__ void reg_pipeline(Issue&& issue, Compute&& compute) {
    static_for<0, (kStages < kDepth ? kStages : kDepth)>([&](auto st) { issue(st); });
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, kStages>([&](auto st) {
        compute(st);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (decltype(st)::value + kDepth < kStages) {
            issue(std::integral_constant<int, decltype(st)::value + kDepth>{});
            __builtin_amdgcn_sched_barrier(0);
        }
    });
}

template <GemmEpilogue E, int RT, int kCols, bool kNorm, int kK, bool kSumA = false>
__global__ void __launch_bounds__(64 * kRegWaves) gemm_reg_kernel(GemmArgs args) {
    static_assert(kK % (kRegWaves * 16) == 0, "whole 16-value stages per wave");
    static_assert(kCols == 32 || kCols == 64, "16-column blocks of a 32- or 64-column tile");
    static_assert(kCols == 64 || (E == GemmEpilogue::kStore || E == GemmEpilogue::kResidual),
                  "column pairs (RoPE, SwiGLU) need 64-column tiles");
    static_assert(!kNorm || kK == kHidden, "the folded norm spans the hidden width");
    static_assert(!kSumA || kSplitBlocksK == 3, "A summed from three planes");
    constexpr int kAParts = kSumA ? 4 : 1;  // residual + three planes, or the A rows
    constexpr int kJB = kCols / 16;
    constexpr int kRows = 16 * RT;
    constexpr int kStages = kK / (kRegWaves * 16);
    constexpr int kPerStage = RT * kAParts + kJB + (kNorm ? 1 : 0);  // float4 loads per lane per stage
    // Ring stages: as many as 72 registers hold (three waves share a SIMD's 512 per lane), 108
    // when A comes as four parts, so the whole slice is still in flight at once.
    constexpr int kRingRegs = kSumA ? 108 : 72;
    constexpr int kDepthFit = kRingRegs / (4 * kPerStage) < 2 ? 2 : kRingRegs / (4 * kPerStage);
    constexpr int kDepth = kDepthFit < 9 ? kDepthFit : 9;
    __shared__ float partial[kRegWaves][kRows][kCols + 1];
    __shared__ float norm_ss[kNorm ? kRegWaves : 1][kRows];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kRows;
    const int n0 = static_cast<int>(blockIdx.x) * kCols;
    const int kq = lane >> 4;
    const int r16 = lane & 15;
    const int k_first = wave * (kK / kRegWaves) + 4 * kq;  // this lane's first K value

    // Part 0 is the A rows (or the residual when A is summed); parts 1-3 the planes.
    const float* a_src[RT][kAParts];
    int64_t a_row[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        a_row[rt] = m0 + 16 * rt + r16;
        const int64_t row = a_row[rt] < args.m ? a_row[rt] : args.m - 1;
        if constexpr (kSumA) {
            a_src[rt][0] = args.a_residual + row * kK + k_first;
#pragma unroll
            for (int b = 0; b < 3; ++b) a_src[rt][1 + b] = args.a_planes + (b * args.m + row) * kK + k_first;
        } else {
            a_src[rt][0] = args.a + row * kK + k_first;
        }
    }
    const float* b_src[kJB];
#pragma unroll
    for (int jb = 0; jb < kJB; ++jb)
        b_src[jb] = args.b + static_cast<int64_t>(b_row<E>(n0 + 16 * jb + r16, args.n)) * kK + k_first;
    const float* g_src = kNorm ? args.norm_weight + k_first : nullptr;

    f32x4 ring_a[kDepth][RT][kAParts];
    f32x4 ring_b[kDepth][kJB];
    f32x4 ring_g[kNorm ? kDepth : 1];
    auto issue = [&](auto st) {
        constexpr int s = decltype(st)::value;
        constexpr int slot = s % kDepth;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int part = 0; part < kAParts; ++part)
                ring_a[slot][rt][part] = *reinterpret_cast<const f32x4*>(a_src[rt][part] + 16 * s);
#pragma unroll
        for (int jb = 0; jb < kJB; ++jb) ring_b[slot][jb] = *reinterpret_cast<const f32x4*>(b_src[jb] + 16 * s);
        if constexpr (kNorm) ring_g[slot] = *reinterpret_cast<const f32x4*>(g_src + 16 * s);
    };
    f32x4 acc[RT][kJB];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int jb = 0; jb < kJB; ++jb) acc[rt][jb] = f32x4{0.f, 0.f, 0.f, 0.f};
    float ss[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) ss[rt] = 0.0f;
    auto compute = [&](auto st) {
        constexpr int slot = decltype(st)::value % kDepth;
        f32x4 a[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            if constexpr (kSumA) {
                const f32x4* part = ring_a[slot][rt];
#pragma unroll
                for (int e = 0; e < 4; ++e) a[rt][e] = part[0][e] + ((part[1][e] + part[2][e]) + part[3][e]);
                if (blockIdx.x == 0 && a_row[rt] < args.m)
                    *reinterpret_cast<f32x4*>(args.a_rows_out + a_row[rt] * kK + k_first + 16 * decltype(st)::value) =
                        a[rt];
            } else {
                a[rt] = ring_a[slot][rt][0];
            }
            if constexpr (kNorm) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    ss[rt] = fmaf(a[rt][e], a[rt][e], ss[rt]);
                    a[rt][e] *= ring_g[slot][e];
                }
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int jb = 0; jb < kJB; ++jb)
                    acc[rt][jb] =
                        __builtin_amdgcn_mfma_f32_16x16x4f32(a[rt][s], ring_b[slot][jb][s], acc[rt][jb], 0, 0, 0);
    };
    reg_pipeline<kStages, kDepth>(issue, compute);

    // D[row 4 (l / 16) + r][column l % 16] of each 16 x 16 block.
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int jb = 0; jb < kJB; ++jb)
#pragma unroll
            for (int r = 0; r < 4; ++r) partial[wave][16 * rt + 4 * kq + r][16 * jb + r16] = acc[rt][jb][r];
    if constexpr (kNorm) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            float v = ss[rt];
            v += __shfl_xor(v, 16, kWave);
            v += __shfl_xor(v, 32, kWave);
            if (lane < 16) norm_ss[wave][16 * rt + lane] = v;
        }
    }
    __syncthreads();
    auto total = [&](int row, int col) {
        float t = partial[0][row][col];
#pragma unroll
        for (int w = 1; w < kRegWaves; ++w) t += partial[w][row][col];
        return t;
    };
    auto inv_rms = [&](int row) {
        if constexpr (kNorm) {
            float t = norm_ss[0][row];
#pragma unroll
            for (int w = 1; w < kRegWaves; ++w) t += norm_ss[w][row];
            return rms_inverse(t, kHidden, args.norm_eps);
        } else {
            return 1.0f;
        }
    };
    if constexpr (E == GemmEpilogue::kStore || E == GemmEpilogue::kResidual) {
        for (int i = static_cast<int>(threadIdx.x); i < kRows * kCols; i += 64 * kRegWaves) {
            const int row = i / kCols, col = i % kCols;
            const int64_t out_row = m0 + row;
            if (out_row < args.m) gemm_store_one<E>(args, out_row, n0 + col, total(row, col) * inv_rms(row));
        }
    } else {
        // Column pairs j / j + 32 of the 64-column group (the RoPE pair, or gate and up).
        for (int i = static_cast<int>(threadIdx.x); i < kRows * 32; i += 64 * kRegWaves) {
            const int row = i / 32, j = i % 32;
            const int64_t out_row = m0 + row;
            if (out_row >= args.m) continue;
            const float inv = inv_rms(row);
            gemm_store_pair<E>(args, out_row, n0, j, total(row, j) * inv, total(row, j + 32) * inv);
        }
    }
}

// Sums the kPlanes partial planes of a K-split gemm_split_kernel or gemm_narrow_kernel in plane order and
// applies the epilogue: thread -> (row, column pair j / j + 32 of a 64-column group) for
// kCols = 64, (row, column) for kCols = 32.  The folded norm's row scale comes from the
// summed partial sums of squares.
template <GemmEpilogue E, bool kNorm, int kCols, int kPlanes = kSplitBlocksK>
__global__ void __launch_bounds__(256) gemm_split_reduce_kernel(GemmArgs args) {
    constexpr bool kPair = kCols == 64;
    const int units = kPair ? args.n / 2 : args.n;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= args.m * units) return;
    const int64_t row = idx / units;
    const int u = static_cast<int>(idx - row * units);
    const int64_t plane = args.m * args.n;
    const float* p = args.split_partials + row * args.n;
    float inv = 1.0f;
    if constexpr (kNorm) {
        const float* ss = args.split_partials + kPlanes * plane + row;
        float total = ss[0];
#pragma unroll
        for (int b = 1; b < kPlanes; ++b) total += ss[b * args.m];
        inv = rms_inverse(total, kHidden, args.norm_eps);
    }
    if constexpr (kPair) {
        const int g0 = (u >> 5) * 64;
        const int j = u & 31;
        float lo = p[g0 + j], hi = p[g0 + 32 + j];
#pragma unroll
        for (int b = 1; b < kPlanes; ++b) {
            lo += p[b * plane + g0 + j];
            hi += p[b * plane + g0 + 32 + j];
        }
        if constexpr (kNorm) {
            lo *= inv;
            hi *= inv;
        }
        gemm_store_pair<E>(args, row, g0, j, lo, hi);
    } else {
        float v = p[u];
#pragma unroll
        for (int b = 1; b < kPlanes; ++b) v += p[b * plane + u];
        gemm_store_one<E>(args, row, u, v);
    }
}

// The reduce of a K-split 576-column GEMM with the residual epilogue, folded into the RMSNorm
// of its output: c = residual + (plane 0 + plane 1 + ...) and norm_out = w * (c * inv_rms(c)).
// Wave per row, the row in registers as float4 quads; the sums run in the order of
// gemm_split_reduce_kernel and the norm in that of rmsnorm_wave4_kernel, so both outputs are
// bitwise those of the reduce kernel followed by launch_rmsnorm_rows.
template <int kPlanes>
__global__ void __launch_bounds__(256) split_reduce_residual_norm_kernel(GemmArgs args, const float* __restrict__ w,
                                                                         float eps, float* __restrict__ norm_out) {
    constexpr int kQuads = 3;  // 144 quads of a 576-wide row over 64 lanes
    const int lane = threadIdx.x & 63;
    const int64_t plane = args.m * kHidden;
    for (int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); row < args.m;
         row += static_cast<int64_t>(gridDim.x) * 4) {
        float4 v[kQuads];
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < kQuads; ++j) {
            const int c = 4 * (lane + 64 * j);
            if (c < kHidden) {
                const float* p = args.split_partials + row * kHidden + c;
                float4 a = *reinterpret_cast<const float4*>(p);
#pragma unroll
                for (int b = 1; b < kPlanes; ++b) {
                    const float4 q = *reinterpret_cast<const float4*>(p + b * plane);
                    a = make_float4(a.x + q.x, a.y + q.y, a.z + q.z, a.w + q.w);
                }
                const float4 r = *reinterpret_cast<const float4*>(args.residual + row * kHidden + c);
                v[j] = make_float4(r.x + a.x, r.y + a.y, r.z + a.z, r.w + a.w);
                *reinterpret_cast<float4*>(args.c + row * kHidden + c) = v[j];
                ss = fmaf(v[j].x, v[j].x, ss);
                ss = fmaf(v[j].y, v[j].y, ss);
                ss = fmaf(v[j].z, v[j].z, ss);
                ss = fmaf(v[j].w, v[j].w, ss);
            }
        }
        const float inv = rms_inverse(wave_sum(ss), kHidden, eps);
#pragma unroll
        for (int j = 0; j < kQuads; ++j) {
            const int c = 4 * (lane + 64 * j);
            if (c < kHidden) {
                const float4 g = *reinterpret_cast<const float4*>(w + c);
                *reinterpret_cast<float4*>(norm_out + row * kHidden + c) =
                    make_float4(g.x * (v[j].x * inv), g.y * (v[j].y * inv), g.z * (v[j].z * inv),
                                g.w * (v[j].w * inv));
            }
        }
    }
}

// Narrow-column GEMM for the residual / plain epilogues of N = 576 outputs (o_proj,
// down): block tile 64 x 64, 4 waves in 2 x 2, wave tile 32 x 32 (one accumulator
// chain).  576 columns are 9 such tiles, so no wave computes a padded column group,
// and the 9 x (M / 64) blocks are small enough to spread evenly over the CUs.  A
// stage is 32 K values, one 128-byte line per row (16-byte pieces XOR-swizzled so a
// 16-lane read pass covers all 64 banks), streamed through a ring of four LDS buffers
// with three copies in flight, stepped as in gemm_ring_kernel.  For every grid size:
// at 8192 rows the ring measured 0.3 ms per prefill faster than two buffers (which
// fit more blocks per CU but wait on each stage's copy).
// kKB > 1: blockIdx.x = column tile * kKB + kb; block kb covers the kb-th part of K and
// writes its tile to partial plane kb of args.split_partials (gemm_split_reduce_kernel sums
// the planes and applies the epilogue).
template <GemmEpilogue E, int kKB>
__global__ void __launch_bounds__(kGemmThreads) gemm_narrow_kernel(GemmArgs args) {
    static_assert(E == GemmEpilogue::kStore || E == GemmEpilogue::kResidual, "plain epilogues only");
    constexpr int kNS = 4;
    constexpr int kRows = 64;
    constexpr int kDepth = 32;
    constexpr int kLoads = 4;  // global_load_lds per wave per stage
    __shared__ __align__(16) float a_s0[kRows * kDepth];
    __shared__ __align__(16) float a_s1[kRows * kDepth];
    __shared__ __align__(16) float a_s2[kRows * kDepth];
    __shared__ __align__(16) float a_s3[kRows * kDepth];
    __shared__ __align__(16) float b_s0[kRows * kDepth];
    __shared__ __align__(16) float b_s1[kRows * kDepth];
    __shared__ __align__(16) float b_s2[kRows * kDepth];
    __shared__ __align__(16) float b_s3[kRows * kDepth];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 1;
    const int wn = wave & 1;
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kRows;
    const int kb = kKB > 1 ? static_cast<int>(blockIdx.x % kKB) : 0;
    const int n0 = static_cast<int>(blockIdx.x / kKB) * kRows;
    const int K = args.k;
    const int k_first = kb * (K / kKB);

    const float* a_src[2];
    const float* b_src[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int row = 8 * (wave + 4 * j) + (lane >> 3);
        const int piece = (lane & 7) ^ ((row >> 1) & 7);
        const int64_t ga = m0 + row < args.m ? m0 + row : args.m - 1;
        a_src[j] = args.a + ga * K + k_first + 4 * piece;
        b_src[j] = args.b + static_cast<int64_t>(n0 + row) * K + k_first + 4 * piece;
    }
    auto abuf = [&](auto bi) -> float* {
        constexpr int b = decltype(bi)::value;
        if constexpr (b == 0) return a_s0;
        else if constexpr (b == 1) return a_s1;
        else if constexpr (b == 2) return a_s2;
        else return a_s3;
    };
    auto bbuf = [&](auto bi) -> float* {
        constexpr int b = decltype(bi)::value;
        if constexpr (b == 0) return b_s0;
        else if constexpr (b == 1) return b_s1;
        else if constexpr (b == 2) return b_s2;
        else return b_s3;
    };
    const int stages = K / kKB / kDepth;
    auto issue = [&](auto bi, int st) {
        const int k0 = (st < stages ? st : stages - 1) * kDepth;
        float* as = abuf(bi);
        float* bs = bbuf(bi);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            lds_copy16(a_src[j] + k0, as + (wave + 4 * j) * 8 * kDepth);
            lds_copy16(b_src[j] + k0, bs + (wave + 4 * j) * 8 * kDepth);
        }
    };

    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    const int h = lane >> 5;
    const int ra = wm * 32 + (lane & 31);
    const int rb = wn * 32 + (lane & 31);
    int a_off[4], b_off[4];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            a_off[2 * u + q] = ra * kDepth + 4 * ((4 * u + 2 * h + q) ^ ((ra >> 1) & 7));
            b_off[2 * u + q] = rb * kDepth + 4 * ((4 * u + 2 * h + q) ^ ((rb >> 1) & 7));
        }
    auto step = [&](auto bi, int s) {
        constexpr int b = decltype(bi)::value;
        const float* as = abuf(bi);
        const float* bs = bbuf(bi);
        f32x4 av[4], bv[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            av[p] = *reinterpret_cast<const f32x4*>(as + a_off[p]);
            bv[p] = *reinterpret_cast<const f32x4*>(bs + b_off[p]);
        }
        issue(std::integral_constant<int, (b + kNS - 1) % kNS>{}, s + kNS - 1);
        if (s < stages) {
#pragma unroll
            for (int p = 0; p < 4; ++p)
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[p][kk], bv[p][kk], acc, 0, 0, 0);
        }
        wait_vmcnt<(kNS - 2) * kLoads>();
        lds_barrier();
    };
    issue(std::integral_constant<int, 0>{}, 0);
    issue(std::integral_constant<int, 1>{}, 1);
    issue(std::integral_constant<int, 2>{}, 2);
    wait_vmcnt<(kNS - 2) * kLoads>();
    lds_barrier();
    for (int s = 0; s < stages; s += kNS) {
        step(std::integral_constant<int, 0>{}, s);
        step(std::integral_constant<int, 1>{}, s + 1);
        step(std::integral_constant<int, 2>{}, s + 2);
        step(std::integral_constant<int, 3>{}, s + 3);
    }
    wait_vmcnt<0>();  // no copy may still be landing in LDS when the block retires

    const int col = n0 + wn * 32 + (lane & 31);
    float* plane = args.split_partials + static_cast<int64_t>(kb) * args.m * args.n;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * 32 + mfma32_row(lane, r);
        if (row >= args.m) continue;
        const int64_t i0 = row * args.n + col;
        if constexpr (kKB > 1) {
            plane[i0] = acc[r];
        } else if constexpr (E == GemmEpilogue::kResidual) {
            args.c[i0] = args.residual[i0] + acc[r];
        } else {
            args.c[i0] = acc[r];
        }
    }
}

// ---------------------------------------------------------------------------
// Causal GQA prefill attention on v_mfma_f32_32x32x2f32.
//
// Block = (128-query tile, query head, chunk of at most attn_chunk_tiles(seq) 64-key tiles);
// 4 waves x 32 queries.  Per 64-key tile a wave computes S^T = K Q^T as two 32x32
// tiles (32 MFMAs each: instruction s pairs dims s and s + 32), then
// O^T += V^T P^T (16 MFMAs per 32 keys and 32-dim half): the S^T accumulator of a
// lane is exactly the B operand of the PV product, so P never leaves registers.
// O^T rows are dims 2i + db (db = 0, 1), so a lane's two V operands of one key are
// adjacent floats.  Q is pre-scaled by scale * log2(e) so scores are already in
// exp2 units.
//
// K/V tiles stream HBM -> LDS with global_load_lds: one K buffer, refilled with the
// next tile as soon as every wave has finished its S^T, and two V buffers, the
// next tile's copied while this tile's is read.  Each buffer is its own LDS
// variable, so reads of one never wait on copies into another.  Three blocks fit a
// CU (49 KB of LDS, at most 168 VGPRs), i.e. three waves per SIMD.
//
// A query tile's keys are split into chunks of attn_chunk_tiles(seq) tiles: about one
// block slot's even share of the causal work, so short prompts still spread over the device,
// and at most kMaxChunkTiles (1024 keys) for long ones.  A tile with one
// chunk writes its rows directly, longer ones write (o, m, l) partials that
// prefill_attention_merge_kernel combines
// (csrc/streaming_prefill_gqa/streaming_prefill_gqa_cuda.cu splits the keys into
// partitions and merges them the same way).  Items (query tile, chunk) are
// launched longest first so the tail of the grid is short chunks.
//
// A wave raises its issue priority (s_setprio 1) for its QK and PV MFMA blocks and drops it
// for the softmax: the other two waves of the SIMD then run their softmax and LDS work in
// the gaps of its MFMA stream rather than delaying it (8192 tokens 35.21 → 35.08 ms; the
// same around the GEMM kernels' MFMAs was slower).  Priority orders issue only; every wave
// still reaches every barrier.
constexpr int kQTile = 128;
constexpr int kKTile = 64;
constexpr int kAttnThreads = 256;
constexpr int kMaxChunkTiles = 16;  // 1024 keys: 24 (1536) measured 1.5% slower at 8192 tokens, 12 / 14 0.1%
constexpr int kPartialRow = kHeadDim + 4;  // o[64], m, l, 2 words of padding (16-byte rows)
constexpr int kMergeMaxChunks = 16;        // >= the chunks of any query tile up to kMaxCapacity
constexpr int kKVTileFloats = kKTile * kHeadDim;

__host__ __device__ __forceinline__ int64_t attn_q_tiles(int64_t seq) { return (seq + kQTile - 1) / kQTile; }
__host__ __device__ __forceinline__ int64_t attn_key_tiles(int64_t seq, int64_t qt) {
    const int64_t last = (qt + 1) * kQTile - 1 < seq - 1 ? (qt + 1) * kQTile - 1 : seq - 1;
    return last / kKTile + 1;
}
// Key tiles per chunk: the 9 heads' causal tile steps (query tile qt walks 2 (qt + 1)
// key tiles) divided over the device's 768 block slots (256 CUs x 3 resident blocks),
// rounded up to an even count in [2, kMaxChunkTiles].  Even, because each query tile adds
// two key tiles.  (Dividing over 256, 512, 1024 or 1536 instead measured slower at 2048 to
// 4096 tokens.)
__host__ __device__ __forceinline__ int64_t attn_chunk_tiles(int64_t seq) {
    const int64_t q = attn_q_tiles(seq);
    const int64_t share = (kQHeads * q * (q + 1) + 767) / 768;
    const int64_t even = (share + 1) / 2 * 2;
    return even < 2 ? 2 : (even > kMaxChunkTiles ? kMaxChunkTiles : even);
}
__host__ __device__ __forceinline__ int64_t attn_chunks(int64_t seq, int64_t qt) {
    const int64_t ct = attn_chunk_tiles(seq);
    return (attn_key_tiles(seq, qt) + ct - 1) / ct;
}
// Query tiles below attn_long_tile(seq) have a single chunk.
__host__ __device__ __forceinline__ int64_t attn_long_tile(int64_t seq) { return attn_chunk_tiles(seq) * kKTile / kQTile; }
__host__ __device__ __forceinline__ int64_t attn_max_chunks(int64_t seq) { return attn_chunks(seq, attn_q_tiles(seq) - 1); }
__host__ __device__ __forceinline__ int64_t attn_partial_slot(int64_t seq, int64_t qt, int h, int64_t c) {
    return ((qt - attn_long_tile(seq)) * kQHeads + h) * attn_max_chunks(seq) + c;
}
// Items of one head, longest first: every chunk of the last query tile, then the
// full chunks of the others (chunk-major), then their partial last chunks by
// decreasing length.  Inner query tiles have 2 (qt + 1) key tiles.
__host__ __device__ __forceinline__ int64_t attn_items(int64_t seq) {
    const int64_t q_tiles = attn_q_tiles(seq);
    int64_t n = attn_chunks(seq, q_tiles - 1);
    for (int64_t qt = 0; qt + 1 < q_tiles; ++qt) n += attn_chunks(seq, qt);
    return n;
}
__device__ __forceinline__ void attn_item(int64_t seq, int64_t i, int64_t& qt, int64_t& chunk) {
    const int64_t q_tiles = attn_q_tiles(seq);
    const int64_t ct = attn_chunk_tiles(seq);
    const int64_t last_chunks = attn_chunks(seq, q_tiles - 1);
    if (i < last_chunks) {
        qt = q_tiles - 1;
        chunk = i;
        return;
    }
    i -= last_chunks;
    // Full chunk c of inner tile qt needs 2 (qt + 1) >= ct (c + 1).
    for (int64_t c = 0;; ++c) {
        const int64_t first = ct / 2 * (c + 1) - 1;
        const int64_t count = q_tiles - 1 - first > 0 ? q_tiles - 1 - first : 0;
        if (count == 0) break;
        if (i < count) {
            qt = first + i;
            chunk = c;
            return;
        }
        i -= count;
    }
    // Partial chunks: length 2 (qt + 1) mod ct = len, longest first.
    for (int64_t len = ct - 2; len >= 2; len -= 2) {
        const int64_t r0 = len / 2 - 1;
        const int64_t count = q_tiles - 2 - r0 >= 0 ? (q_tiles - 2 - r0) / (ct / 2) + 1 : 0;
        if (i < count) {
            qt = r0 + (ct / 2) * i;
            chunk = 2 * (qt + 1) / ct;
            return;
        }
        i -= count;
    }
    qt = 0;  // not reached for i < attn_items(seq)
    chunk = 0;
}

// LDS tiles: K rows are padded to 17 16-byte pieces (68 words), so the 32 lanes that
// read one piece of 32 consecutive rows hit distinct banks; V rows are plain (the 32
// lanes of a V read cover one whole row).  Every read is a per-lane base plus an
// immediate offset.
constexpr int kKRow = kHeadDim + 4;                    // words per padded K row
constexpr int kKTileWords = kKTile * kKRow;           // 4352
constexpr int kKCopies = kKTileWords / 256;           // 17 global_load_lds of 1 KB
constexpr int kVCopies = kKVTileFloats / 256;         // 16

// max / sum of the values of lanes l and l ^ 32 (v_permlane32_swap: r[0] holds the
// low half's values in both halves, r[1] the high half's).
__device__ __forceinline__ float halves_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}


__global__ void __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(3)))
prefill_attention_kernel(const float* __restrict__ q, const float* __restrict__ key_cache,
                         const float* __restrict__ value_cache, int64_t seq, int64_t capacity, float scale,
                         float* __restrict__ workspace, float* __restrict__ out_rows) {
    __shared__ __align__(16) float ks[kKTileWords];
    __shared__ __align__(16) float v0s[kKVTileFloats];
    __shared__ __align__(16) float v1s[kKVTileFloats];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = static_cast<int>(blockIdx.x % kQHeads);
    int64_t qt, chunk;
    attn_item(seq, blockIdx.x / kQHeads, qt, chunk);
    const int g = h / kGroup;
    const int64_t qw0 = qt * kQTile + 32 * wave;  // first query of this wave
    const int col = lane & 31;
    const int half = lane >> 5;
    const int64_t my_q = qw0 + col;

    // B operand of S^T = K Q^T: qreg[s] = Q[my_q][s + 32 half] * scale * log2(e).
    float qreg[32];
    {
        const int64_t r = my_q < seq ? my_q : seq - 1;
        const float* qp = q + (static_cast<int64_t>(h) * seq + r) * kHeadDim + 32 * half;
        const float s2 = scale * kLog2e;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float4 v = *reinterpret_cast<const float4*>(qp + 4 * t);
            qreg[4 * t] = v.x * s2;
            qreg[4 * t + 1] = v.y * s2;
            qreg[4 * t + 2] = v.z * s2;
            qreg[4 * t + 3] = v.w * s2;
        }
    }

    const float* kg = key_cache + static_cast<int64_t>(g) * capacity * kHeadDim;
    const float* vg = value_cache + static_cast<int64_t>(g) * capacity * kHeadDim;
    const int64_t k_tiles = attn_key_tiles(seq, qt);
    const int64_t chunk_tiles = attn_chunk_tiles(seq);
    const int64_t kt_begin = chunk * chunk_tiles;
    const int64_t kt_end = kt_begin + chunk_tiles < k_tiles ? kt_begin + chunk_tiles : k_tiles;

    // Copies of key tile kt: K slot s (16 bytes) of the padded tile holds piece s % 17
    // of row s / 17 (piece 16 is padding and repeats piece 0); V slot s holds piece
    // s % 16 of row s / 16.  Copy i covers slots 64 i .. 64 i + 63; wave w issues
    // copies w, w + 4, ...  Rows past the prompt repeat its last row (they are masked).
    auto issue_k = [&](int64_t kt) {
        const int k0 = static_cast<int>(kt) * kKTile;
        const int last = static_cast<int>(seq) - 1 - k0;  // last valid row of the tile
#pragma unroll
        for (int j = 0; j < (kKCopies + 3) / 4; ++j) {
            const int i = wave + 4 * j;
            if (i < kKCopies) {
                const int slot = 64 * i + lane;
                int row = slot / 17;
                int piece = slot - 17 * row;
                piece = piece == 16 ? 0 : piece;
                row = row < last ? row : last;
                __builtin_amdgcn_global_load_lds(kg + static_cast<int64_t>(k0 + row) * kHeadDim + 4 * piece,
                                                 ks + 256 * i, 16, 0, 0);
            }
        }
    };
    auto issue_v = [&](float* vbuf, int64_t kt) {
        const int k0 = static_cast<int>(kt) * kKTile;
        const int last = static_cast<int>(seq) - 1 - k0;
#pragma unroll
        for (int j = 0; j < kVCopies / 4; ++j) {
            const int i = wave + 4 * j;
            int row = 4 * i + (lane >> 4);
            row = row < last ? row : last;
            __builtin_amdgcn_global_load_lds(vg + static_cast<int64_t>(k0 + row) * kHeadDim + 4 * (lane & 15),
                                             vbuf + 256 * i, 16, 0, 0);
        }
    };

    f32x16 o_acc[2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o_acc[db][r] = 0.0f;
    float m_run = -INFINITY;
    float l_run = 0.0f;

    const int seq32 = static_cast<int>(seq);
    const int qw = static_cast<int>(qw0);
    const int q_me = static_cast<int>(my_q);
    // QK of one tile: both 32-key halves when the second is visible to the wave (the
    // two accumulator chains alternate), the K operands of step t + 1 read from LDS
    // before the MFMAs of step t.
    auto qk = [&](const float* ks, f32x16* s_acc, auto both_c) {
        constexpr bool both = decltype(both_c)::value;
        const float* k0p = ks + col * kKRow + 32 * half;  // row col, dims 32 half ..
        const float* k1p = k0p + 32 * kKRow;                // row 32 + col
        f32x4 ka = *reinterpret_cast<const f32x4*>(k0p);
        f32x4 kb;
        if constexpr (both) kb = *reinterpret_cast<const f32x4*>(k1p);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            f32x4 na, nb;
            if (t < 7) {
                na = *reinterpret_cast<const f32x4*>(k0p + 4 * (t + 1));
                if constexpr (both) nb = *reinterpret_cast<const f32x4*>(k1p + 4 * (t + 1));
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s_acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka[e], qreg[4 * t + e], s_acc[0], 0, 0, 0);
                if constexpr (both)
                    s_acc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(kb[e], qreg[4 * t + e], s_acc[1], 0, 0, 0);
            }
            if (t < 7) {
                ka = na;
                if constexpr (both) kb = nb;
            }
        }
    };
    // One key tile: S^T from the K tile, an LDS barrier after which the K buffer is
    // refilled with the next tile, then softmax and O^T += V^T P^T from this tile's
    // V buffer.  Waves whose queries all precede the tile skip the math but not the
    // barriers.
    auto tile = [&](const float* vs, int64_t kt, int64_t kt_next) {
        const int k0 = static_cast<int>(kt) * kKTile;
        const bool active = k0 <= qw + 31;
        const bool need_mask = k0 + kKTile - 1 > qw || k0 + kKTile > seq32;
        const bool live1 = k0 + 32 <= qw + 31;  // second 32-key half visible to some query
        f32x16 s_acc[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) s_acc[kb][r] = 0.0f;
        __builtin_amdgcn_s_setprio(1);  // the MFMA block (see above the kernel)
        if (live1)
            qk(ks, s_acc, std::true_type{});
        else if (active)
            qk(ks, s_acc, std::false_type{});
        __builtin_amdgcn_s_setprio(0);
        lds_barrier();  // every wave is done with the K tile
        issue_k(kt_next);
        if (!active) return;
        // Lane holds keys k0 + 32 kb + 8 (r / 4) + 4 half + r % 4 of query my_q.
        if (!live1) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s_acc[1][r] = -INFINITY;
        }
        if (need_mask) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = k0 + 32 * kb + 8 * (r >> 2) + 4 * half + (r & 3);
                    s_acc[kb][r] = (key <= q_me && key < seq32) ? s_acc[kb][r] : -INFINITY;
                }
            }
        }
        float tile_max = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) tile_max = fmaxf(tile_max, s_acc[kb][r]);
        tile_max = halves_max(tile_max);
        const float m_new = fmaxf(m_run, tile_max);  // finite: the first key of a chunk precedes every query
        const float alpha = fast_exp2(m_run - m_new);
        float psum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = fast_exp2(s_acc[kb][r] - m_new);
                s_acc[kb][r] = p;
                psum += p;
            }
        }
        psum = halves_sum(psum);
        l_run = l_run * alpha + psum;
        m_run = m_new;
        // alpha is exactly 1 where the running max did not move: skip the rescale
        // when that holds for every lane (multiplying by 1 would not change a bit).
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int db = 0; db < 2; ++db) o_acc[db] *= alpha;
        }
        __builtin_amdgcn_s_setprio(1);  // the MFMA block (see above the kernel)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            if (kb == 1 && !live1) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float2 v = *reinterpret_cast<const float2*>(vs + (4 * half) * kHeadDim + 2 * col +
                                                                  (32 * kb + 8 * (r >> 2) + (r & 3)) * kHeadDim);
                o_acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(v.x, s_acc[kb][r], o_acc[0], 0, 0, 0);
                o_acc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(v.y, s_acc[kb][r], o_acc[1], 0, 0, 0);
            }
        }
        __builtin_amdgcn_s_setprio(0);
    };

    issue_k(kt_begin);
    issue_v(v0s, kt_begin);
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    for (int64_t kt = kt_begin; kt < kt_end; kt += 2) {
        const int64_t n1 = kt + 1 < kt_end ? kt + 1 : kt_end - 1;
        issue_v(v1s, n1);
        tile(v0s, kt, n1);
        __builtin_amdgcn_s_waitcnt(0);  // this wave's copies of tile kt + 1 have landed
        lds_barrier();
        if (kt + 1 < kt_end) {
            const int64_t n2 = kt + 2 < kt_end ? kt + 2 : kt_end - 1;
            issue_v(v0s, n2);
            tile(v1s, kt + 1, n2);
            __builtin_amdgcn_s_waitcnt(0);
            lds_barrier();
        }
    }

    // O^T accumulator: lane holds dims 2 (8 (r / 4) + 4 half + r % 4) + db of query my_q.
    if (my_q >= seq) return;
    const bool single = attn_chunks(seq, qt) == 1;
    const float inv = single ? 1.0f / l_run : 1.0f;
    float* dst = single ? out_rows + my_q * kHidden + h * kHeadDim
                        : workspace + (attn_partial_slot(seq, qt, h, chunk) * kQTile + (my_q - qt * kQTile)) * kPartialRow;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int i = 8 * (r >> 2) + 4 * half + (r & 3);
        *reinterpret_cast<float2*>(dst + 2 * i) = make_float2(o_acc[0][r] * inv, o_acc[1][r] * inv);
    }
    if (!single && half == 0) *reinterpret_cast<float2*>(dst + kHeadDim) = make_float2(m_run, l_run);  // m in log2 units
}

// Combines the chunk partials of query tiles with more than one chunk.  Block
// ((qt - attn_long_tile(seq)) * 9 + h) * 8 + row group; thread t -> row 16 * group + t / 16,
// dims 4 (t % 16) .. + 3.  All chunk loads of a thread are issued before the combine.
template <int kMaxChunks>
__global__ void __launch_bounds__(kAttnThreads) prefill_attention_merge_kernel(const float* __restrict__ workspace,
                                                                               int64_t seq,
                                                                               float* __restrict__ out_rows) {
    constexpr int kRowsPerBlock = kAttnThreads / 16;
    const int64_t tile_head = blockIdx.x / (kQTile / kRowsPerBlock);
    const int64_t qt = attn_long_tile(seq) + tile_head / kQHeads;
    const int h = static_cast<int>(tile_head % kQHeads);
    const int row = static_cast<int>(blockIdx.x % (kQTile / kRowsPerBlock)) * kRowsPerBlock +
                    static_cast<int>(threadIdx.x >> 4);
    const int d = 4 * static_cast<int>(threadIdx.x & 15);
    const int64_t q0 = qt * kQTile;
    if (q0 + row >= seq) return;
    const int chunks = static_cast<int>(attn_chunks(seq, qt));
    float4 o[kMaxChunks];
    float m[kMaxChunks], l[kMaxChunks];
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
        if (c < chunks) {
            const float* p = workspace + (attn_partial_slot(seq, qt, h, c) * kQTile + row) * kPartialRow;
            o[c] = *reinterpret_cast<const float4*>(p + d);
            const float2 ml = *reinterpret_cast<const float2*>(p + kHeadDim);
            m[c] = ml.x;
            l[c] = ml.y;
        } else {
            o[c] = make_float4(0.f, 0.f, 0.f, 0.f);
            m[c] = -INFINITY;
            l[c] = 0.0f;
        }
    }
    float M = -INFINITY;
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) M = fmaxf(M, m[c]);
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    float L = 0.0f;
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
        const float f = fast_exp2(m[c] - M);
        O.x = fmaf(o[c].x, f, O.x);
        O.y = fmaf(o[c].y, f, O.y);
        O.z = fmaf(o[c].z, f, O.z);
        O.w = fmaf(o[c].w, f, O.w);
        L = fmaf(l[c], f, L);
    }
    *reinterpret_cast<float4*>(out_rows + (q0 + row) * kHidden + h * kHeadDim + d) =
        make_float4(O.x / L, O.y / L, O.z / L, O.w / L);
}

// Short prompts: block = (32-query tile t, query head h).  The tile's causal keys are
// the 32-key chunks c = 0..t; chunk c goes to wave c % 8, and each wave runs the online
// softmax over its chunks with K, V and Q read from global memory straight into MFMA
// operands (a chunk is 16 KB of K/V, served by L2).  S^T = K Q^T and O^T += V^T P^T use
// the same operand layouts as prefill_attention_kernel.  The waves' (o, m, l) meet in
// LDS, where 512 threads combine them, so no partials leave the block and no merge
// kernel runs.  A 128-token prompt is 36 blocks of at most one chunk per wave, against 9
// blocks whose last wave walks 128 keys in the 128-query-tile kernel.
constexpr int kSmallQ = 32;
constexpr int kSmallWaves = 8;
// Measured against the 128-query-tile kernel (whole prefill, ms): 128 tokens 1.58 vs 1.81,
// 256: 1.81 vs 2.04, 512: 2.62 vs 2.71, 1024: 4.38 vs 4.36 (16 waves per block: slower
// from 512 on).
constexpr int64_t kSmallAttnMaxSeq = 512;

__global__ void __launch_bounds__(64 * kSmallWaves)
prefill_attention_small_kernel(const float* __restrict__ q, const float* __restrict__ key_cache,
                               const float* __restrict__ value_cache, int64_t seq, int64_t capacity, float scale,
                               float* __restrict__ out_rows) {
    __shared__ float o_s[kSmallWaves][kSmallQ][kHeadDim + 1];
    __shared__ float m_s[kSmallWaves][kSmallQ];
    __shared__ float l_s[kSmallWaves][kSmallQ];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int h = static_cast<int>(blockIdx.x % kQHeads);
    const int t = static_cast<int>(blockIdx.x / kQHeads);
    const int g = h / kGroup;
    const int col = lane & 31;
    const int half = lane >> 5;
    const int seq32 = static_cast<int>(seq);
    const int q_me = kSmallQ * t + col;

    // B operand of S^T = K Q^T: qreg[s] = Q[q_me][s + 32 half] * scale * log2(e).
    float qreg[32];
    {
        const int64_t r = q_me < seq32 ? q_me : seq32 - 1;
        const float* qp = q + (static_cast<int64_t>(h) * seq + r) * kHeadDim + 32 * half;
        const float s2 = scale * kLog2e;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = *reinterpret_cast<const float4*>(qp + 4 * i);
            qreg[4 * i] = v.x * s2;
            qreg[4 * i + 1] = v.y * s2;
            qreg[4 * i + 2] = v.z * s2;
            qreg[4 * i + 3] = v.w * s2;
        }
    }
    const float* kg = key_cache + static_cast<int64_t>(g) * capacity * kHeadDim;
    const float* vg = value_cache + static_cast<int64_t>(g) * capacity * kHeadDim;

    f32x16 o_acc[2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o_acc[db][r] = 0.0f;
    float m_run = -INFINITY;
    float l_run = 0.0f;
    for (int c = wave; c <= t; c += kSmallWaves) {
        const int k0 = kSmallQ * c;
        // A operand of S^T: this lane's key k0 + col (rows past the prompt repeat its last
        // row; they are masked), dims 32 half ..; the V operands of the chunk are requested
        // with it, before the softmax needs them.
        const int krow = k0 + col < seq32 ? k0 + col : seq32 - 1;
        const float* kp = kg + static_cast<int64_t>(krow) * kHeadDim + 32 * half;
        f32x4 kv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) kv[i] = *reinterpret_cast<const f32x4*>(kp + 4 * i);
        float2 vv[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
            const int vrow = key < seq32 ? key : seq32 - 1;
            vv[r] = *reinterpret_cast<const float2*>(vg + static_cast<int64_t>(vrow) * kHeadDim + 2 * col);
        }
        f32x16 s_acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) s_acc[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                s_acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[i][e], qreg[4 * i + e], s_acc, 0, 0, 0);
        // Lane holds keys k0 + 8 (r / 4) + 4 half + r % 4 of query q_me.  Every chunk a wave
        // takes holds a key <= q_me below the prompt length (key 32 t on the diagonal), so the
        // running maximum is finite after the first chunk.
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
            s_acc[r] = (key <= q_me && key < seq32) ? s_acc[r] : -INFINITY;
        }
        float tile_max = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) tile_max = fmaxf(tile_max, s_acc[r]);
        tile_max = halves_max(tile_max);
        const float m_new = fmaxf(m_run, tile_max);
        const float alpha = fast_exp2(m_run - m_new);
        float psum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p = fast_exp2(s_acc[r] - m_new);
            s_acc[r] = p;
            psum += p;
        }
        psum = halves_sum(psum);
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int db = 0; db < 2; ++db) o_acc[db] *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            o_acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[r].x, s_acc[r], o_acc[0], 0, 0, 0);
            o_acc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[r].y, s_acc[r], o_acc[1], 0, 0, 0);
        }
    }

    // O^T accumulator: lane holds dims 2 (8 (r / 4) + 4 half + r % 4) + db of query q_me.
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int i = 8 * (r >> 2) + 4 * half + (r & 3);
        o_s[wave][col][2 * i] = o_acc[0][r];
        o_s[wave][col][2 * i + 1] = o_acc[1][r];
    }
    if (half == 0) {
        m_s[wave][col] = m_run;
        l_s[wave][col] = l_run;
    }
    __syncthreads();
    // Thread -> query 32 t + (thread / 16), dims 4 (thread % 16) .. + 3; waves in order.
    const int qq = static_cast<int>(threadIdx.x >> 4);
    const int d = 4 * static_cast<int>(threadIdx.x & 15);
    const int qrow = kSmallQ * t + qq;
    if (qrow >= seq32) return;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSmallWaves; ++w) M = fmaxf(M, m_s[w][qq]);
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < kSmallWaves; ++w) {
        const float mw = m_s[w][qq];
        const float f = mw == -INFINITY ? 0.0f : fast_exp2(mw - M);
        const float* ow = &o_s[w][qq][d];
        O.x = fmaf(ow[0], f, O.x);
        O.y = fmaf(ow[1], f, O.y);
        O.z = fmaf(ow[2], f, O.z);
        O.w = fmaf(ow[3], f, O.w);
        L = fmaf(l_s[w][qq], f, L);
    }
    *reinterpret_cast<float4*>(out_rows + static_cast<int64_t>(qrow) * kHidden + h * kHeadDim + d) =
        make_float4(O.x / L, O.y / L, O.z / L, O.w / L);
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

// Grids below this many blocks (fewer than the device's CUs) use the ring kernel.
constexpr int64_t kRingBlocks = 256;
constexpr int64_t kSplitBlocks = 256;  // gemm_split_kernel while its grid fits the device once
constexpr int64_t kSplitKBlocks = 256;  // ... and with K split over blocks while that grid fits it too
constexpr int64_t kNarrowSplitBlocks = 1024;  // gemm_narrow_kernel splits K while the split grid is at most 4 per CU

// Tiling of gemm_split_kernel for this GEMM (rt = 0 when it does not take it), for K = 576
// (hidden) or 1536 (intermediate), while the grid fits the device once.  Plain and residual
// epilogues first try 32-column tiles (one row tile per block).  Otherwise 64-column tiles
// with the smallest row tiling that fits; shapes the 64 x 64 tile kernel takes use one row
// tile only: with more, their 9 column tiles leave too many CUs idle (measured slower at
// 1024 to 2048 rows).
struct SplitShape {
    int rt;
    int cols;
};
static SplitShape split_shape(const GemmArgs& args, GemmEpilogue epilogue) {
    if (args.k != kHidden && args.k != kInter) return {0, 0};
    const bool plain = epilogue == GemmEpilogue::kStore || epilogue == GemmEpilogue::kResidual;
    if (plain && (args.n / 32) * ((args.m + 31) / 32) <= kSplitBlocks) return {1, 32};
    const bool narrow_shape = plain && args.n % kBN != 0 && args.k % 32 == 0;
    for (int rt = 1; rt <= (narrow_shape ? 1 : 4); rt *= 2)
        if ((args.n / 64) * ((args.m + 32 * rt - 1) / (32 * rt)) <= kSplitBlocks) return {rt, 64};
    return {0, 0};
}

// Tiling of gemm_reg_kernel (rt = 0 when it does not take the GEMM): 16-row blocks with the
// narrowest column tile whose grid fits the device once (one block per CU), for the GEMMs over
// the hidden width (QKV, o_proj, gate/up).  The down projection (K = intermediate) measured
// faster on gemm_split_kernel at every prompt length.
#ifndef FLUX_REG_GEMM
#define FLUX_REG_GEMM 1
#endif
struct RegShape {
    int rt;
    int cols;
};
static RegShape reg_shape(const GemmArgs& args, GemmEpilogue epilogue) {
    if (!FLUX_REG_GEMM || args.k != kHidden || args.n % 64 != 0) return {0, 0};
    const bool pair = epilogue == GemmEpilogue::kQkvRope || epilogue == GemmEpilogue::kSwiglu;
    const int64_t r16 = (args.m + 15) / 16;
    if (!pair && (args.n / 32) * r16 <= kSplitBlocks) return {1, 32};
    if ((args.n / 64) * r16 <= kSplitBlocks) return {1, 64};
    return {0, 0};
}

// gemm_reg_kernel and gemm_split_kernel fold an RMSNorm of the A rows into the QKV and gate/up
// GEMMs (K = hidden).
static bool split_folds_norm(const GemmArgs& args, GemmEpilogue epilogue) {
    return args.k == kHidden && (epilogue == GemmEpilogue::kQkvRope || epilogue == GemmEpilogue::kSwiglu) &&
           (reg_shape(args, epilogue).rt != 0 || split_shape(args, epilogue).rt != 0);
}

static hipError_t launch_reg(const GemmArgs& args, GemmEpilogue epilogue, RegShape shape, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(args.n / shape.cols), static_cast<unsigned>((args.m + 16 * shape.rt - 1) /
                                                                                   (16 * shape.rt)));
    const dim3 block(64 * kRegWaves);
    const bool norm = args.norm_weight != nullptr;
#define FLUX_REG(E, COLS, NORM) \
    hipLaunchKernelGGL(HIP_KERNEL_NAME(gemm_reg_kernel<E, 1, COLS, NORM, kHidden>), grid, block, 0, stream, args)
#define FLUX_REG_PLAIN(E)                       \
    do {                                        \
        if (shape.cols == 32) FLUX_REG(E, 32, false); \
        else FLUX_REG(E, 64, false);            \
    } while (0)
#define FLUX_REG_PAIR(E)                        \
    do {                                        \
        if (norm) FLUX_REG(E, 64, true);        \
        else FLUX_REG(E, 64, false);            \
    } while (0)
    if (args.a_planes != nullptr) {
        hipLaunchKernelGGL(HIP_KERNEL_NAME(gemm_reg_kernel<GemmEpilogue::kQkvRope, 1, 64, true, kHidden, true>), grid,
                           block, 0, stream, args);
        return hipGetLastError();
    }
    switch (epilogue) {
        case GemmEpilogue::kStore:
            FLUX_REG_PLAIN(GemmEpilogue::kStore);
            break;
        case GemmEpilogue::kResidual:
            FLUX_REG_PLAIN(GemmEpilogue::kResidual);
            break;
        case GemmEpilogue::kSwiglu:
            FLUX_REG_PAIR(GemmEpilogue::kSwiglu);
            break;
        case GemmEpilogue::kQkvRope:
            FLUX_REG_PAIR(GemmEpilogue::kQkvRope);
            break;
    }
#undef FLUX_REG_PAIR
#undef FLUX_REG_PLAIN
#undef FLUX_REG
    return hipGetLastError();
}

// K parts of the 576-column kernel: kSplitBlocksK while that grid is at most
// kNarrowSplitBlocks blocks; beyond that two halves when they cut the blocks the busiest CU
// runs (in units of a whole-K block: ceil(2B / 256) / 2 against ceil(B / 256), B blocks) by
// at least 15%, or by at least 5% when the reduce is folded into the RMSNorm that follows
// (launch_gemm_residual_norm).  1 without partial planes.
// True when `parts` partial planes of this GEMM (and as many rows of sums of squares) fit the
// caller's workspace.
static bool planes_fit(const GemmArgs& args, int parts) {
    return args.split_partials != nullptr && parts * args.m * (static_cast<int64_t>(args.n) + 1) <= args.split_floats;
}

static int narrow_parts(const GemmArgs& args, bool fused_reduce) {
    if (!planes_fit(args, 2)) return 1;
    const int64_t blocks = static_cast<int64_t>(args.n / 64) * ((args.m + 63) / 64);
    if (args.k % (32 * kSplitBlocksK) == 0 && blocks * kSplitBlocksK <= kNarrowSplitBlocks &&
        planes_fit(args, kSplitBlocksK))
        return kSplitBlocksK;
    const int64_t cus = 256;
    const int64_t whole = (blocks + cus - 1) / cus;
    const int64_t halves = (2 * blocks + cus - 1) / cus;
    const int64_t keep = fused_reduce ? 19 : 17;  // per 20: the half-block count must stay under keep/20
    return args.k % 64 == 0 && 20 * halves <= keep * 2 * whole ? 2 : 1;
}

static hipError_t launch_narrow(const GemmArgs& args, GemmEpilogue epilogue, int parts, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(args.n / 64 * parts), static_cast<unsigned>((args.m + 63) / 64));
    const dim3 block(kGemmThreads);
#define FLUX_NARROW(E)                                                                                             \
    do {                                                                                                           \
        if (parts == kSplitBlocksK)                                                                                \
            hipLaunchKernelGGL(HIP_KERNEL_NAME(gemm_narrow_kernel<E, kSplitBlocksK>), grid, block, 0, stream, args); \
        else if (parts == 2)                                                                                       \
            hipLaunchKernelGGL(HIP_KERNEL_NAME(gemm_narrow_kernel<E, 2>), grid, block, 0, stream, args);            \
        else                                                                                                       \
            hipLaunchKernelGGL(HIP_KERNEL_NAME(gemm_narrow_kernel<E, 1>), grid, block, 0, stream, args);            \
    } while (0)
    if (epilogue == GemmEpilogue::kResidual) FLUX_NARROW(GemmEpilogue::kResidual);
    else FLUX_NARROW(GemmEpilogue::kStore);
#undef FLUX_NARROW
    return hipGetLastError();
}

static bool narrow_shape(const GemmArgs& args, GemmEpilogue epilogue) {
    return (epilogue == GemmEpilogue::kStore || epilogue == GemmEpilogue::kResidual) && args.n % kBN != 0 &&
           args.k % 32 == 0;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Whether gemm_split_kernel takes these args with K split over kSplitBlocksK blocks: its grid
// fits the device once even when tripled, and the caller's planes hold the split.
static bool split_k_taken(const GemmArgs& args, GemmEpilogue epilogue) {
    const SplitShape shape = split_shape(args, epilogue);
    if (shape.rt == 0) return false;
    const int64_t blocks = (args.n / shape.cols) * ((args.m + 32 * shape.rt - 1) / (32 * shape.rt));
    return planes_fit(args, kSplitBlocksK) && blocks * kSplitBlocksK <= kSplitKBlocks;
}

bool gemm_writes_planes(const GemmArgs& args, GemmEpilogue epilogue) {
    return reg_shape(args, epilogue).rt == 0 && split_k_taken(args, epilogue);
}

bool gemm_sums_planes(const GemmArgs& args, GemmEpilogue epilogue) {
    return epilogue == GemmEpilogue::kQkvRope && reg_shape(args, epilogue).rt != 0;
}

static hipError_t gemm_args_valid(const GemmArgs& args, GemmEpilogue epilogue) {
    if (args.k % kBK != 0 || args.n % 64 != 0 || args.m <= 0) return hipErrorInvalidValue;
    if (epilogue == GemmEpilogue::kSwiglu && args.n % kBN != 0) return hipErrorInvalidValue;
    if (epilogue == GemmEpilogue::kQkvRope && args.n != kQKV) return hipErrorInvalidValue;
    const bool norm = args.norm_weight != nullptr;
    if (norm && !split_folds_norm(args, epilogue)) return hipErrorInvalidValue;
    if (args.a_planes != nullptr && (!gemm_sums_planes(args, epilogue) || !norm || args.a_residual == nullptr ||
                                     args.a_rows_out == nullptr || !aligned16(args.a_planes) ||
                                     !aligned16(args.a_residual) || !aligned16(args.a_rows_out)))
        return hipErrorInvalidValue;
    return hipSuccess;
}

static hipError_t launch_gemm_split(const GemmArgs& args, GemmEpilogue epilogue, bool reduce, hipStream_t stream);

hipError_t launch_gemm(const GemmArgs& args, GemmEpilogue epilogue, hipStream_t stream) {
    const hipError_t valid = gemm_args_valid(args, epilogue);
    if (valid != hipSuccess) return valid;
    const RegShape reg = reg_shape(args, epilogue);
    if (reg.rt != 0) return launch_reg(args, epilogue, reg, stream);
    return launch_gemm_split(args, epilogue, true, stream);
}

hipError_t launch_gemm_planes(const GemmArgs& args, GemmEpilogue epilogue, hipStream_t stream) {
    const hipError_t valid = gemm_args_valid(args, epilogue);
    if (valid != hipSuccess) return valid;
    if (args.a_planes != nullptr || !gemm_writes_planes(args, epilogue)) return hipErrorInvalidValue;
    return launch_gemm_split(args, epilogue, false, stream);
}

// gemm_split_kernel and the remaining kernels of launch_gemm; `reduce` false stops after the
// partial planes of a K split.
static hipError_t launch_gemm_split(const GemmArgs& args, GemmEpilogue epilogue, bool reduce, hipStream_t stream) {
    const bool norm = args.norm_weight != nullptr;
    const SplitShape shape = split_shape(args, epilogue);
    const int rt = shape.rt;
    if (rt != 0) {
        const bool hidden = args.k == kHidden;
        dim3 grid(static_cast<unsigned>(args.n / shape.cols), static_cast<unsigned>((args.m + 32 * rt - 1) / (32 * rt)));
        const dim3 split_block(64 * kSplitWaves);
        // Grids of at most a third of the device split K over kSplitBlocksK blocks when the
        // caller provides the partial planes.
        const bool split_k = split_k_taken(args, epilogue);
        if (split_k) grid.x *= kSplitBlocksK;
#define FLUX_SPLIT_RT(E, ST, RT, NORM, COLS)                                                                        \
    do {                                                                                                            \
        if (split_k)                                                                                                \
            hipLaunchKernelGGL(HIP_KERNEL_NAME(gemm_split_kernel<E, ST * RT / kSplitBlocksK, RT, NORM, COLS,        \
                                                                 kSplitBlocksK>),                                   \
                               grid, split_block, 0, stream, args);                                                 \
        else                                                                                                        \
            hipLaunchKernelGGL(HIP_KERNEL_NAME(gemm_split_kernel<E, ST * RT, RT, NORM, COLS, 1>), grid, split_block, \
                               0, stream, args);                                                                    \
    } while (0)
#define FLUX_LAUNCH_SPLIT(E)                                                                            \
    do {                                                                                                \
        if (rt == 1) {                                                                                  \
            if (hidden) FLUX_SPLIT_RT(E, 9, 1, false, 64); else FLUX_SPLIT_RT(E, 24, 1, false, 64);     \
        } else if (rt == 2) {                                                                           \
            if (hidden) FLUX_SPLIT_RT(E, 9, 2, false, 64); else FLUX_SPLIT_RT(E, 24, 2, false, 64);     \
        } else {                                                                                        \
            if (hidden) FLUX_SPLIT_RT(E, 9, 4, false, 64); else FLUX_SPLIT_RT(E, 24, 4, false, 64);     \
        }                                                                                               \
    } while (0)
#define FLUX_LAUNCH_SPLIT_PLAIN(E)                                                                      \
    do {                                                                                                \
        if (shape.cols == 32) {                                                                         \
            if (hidden) FLUX_SPLIT_RT(E, 9, 1, false, 32); else FLUX_SPLIT_RT(E, 24, 1, false, 32);     \
        } else {                                                                                        \
            FLUX_LAUNCH_SPLIT(E);                                                                       \
        }                                                                                               \
    } while (0)
#define FLUX_LAUNCH_SPLIT_NORM(E)                                                                       \
    do {                                                                                                \
        if (rt == 1) FLUX_SPLIT_RT(E, 9, 1, true, 64);                                                  \
        else if (rt == 2) FLUX_SPLIT_RT(E, 9, 2, true, 64);                                             \
        else FLUX_SPLIT_RT(E, 9, 4, true, 64);                                                          \
    } while (0)
        switch (epilogue) {
            case GemmEpilogue::kStore:
                FLUX_LAUNCH_SPLIT_PLAIN(GemmEpilogue::kStore);
                break;
            case GemmEpilogue::kResidual:
                FLUX_LAUNCH_SPLIT_PLAIN(GemmEpilogue::kResidual);
                break;
            case GemmEpilogue::kSwiglu:
                if (norm) FLUX_LAUNCH_SPLIT_NORM(GemmEpilogue::kSwiglu);
                else FLUX_LAUNCH_SPLIT(GemmEpilogue::kSwiglu);
                break;
            case GemmEpilogue::kQkvRope:
                if (norm) FLUX_LAUNCH_SPLIT_NORM(GemmEpilogue::kQkvRope);
                else FLUX_LAUNCH_SPLIT(GemmEpilogue::kQkvRope);
                break;
        }
#undef FLUX_LAUNCH_SPLIT_PLAIN
#undef FLUX_LAUNCH_SPLIT_NORM
#undef FLUX_LAUNCH_SPLIT
#undef FLUX_SPLIT_RT
        hipError_t st = hipGetLastError();
        if (st != hipSuccess || !split_k || !reduce) return st;
        const int64_t units = shape.cols == 64 ? args.n / 2 : args.n;
        const dim3 rgrid(static_cast<unsigned>((args.m * units + 255) / 256));
#define FLUX_REDUCE(E, NORM, COLS) \
    hipLaunchKernelGGL(HIP_KERNEL_NAME(gemm_split_reduce_kernel<E, NORM, COLS>), rgrid, dim3(256), 0, stream, args)
        switch (epilogue) {
            case GemmEpilogue::kStore:
                if (shape.cols == 32) FLUX_REDUCE(GemmEpilogue::kStore, false, 32);
                else FLUX_REDUCE(GemmEpilogue::kStore, false, 64);
                break;
            case GemmEpilogue::kResidual:
                if (shape.cols == 32) FLUX_REDUCE(GemmEpilogue::kResidual, false, 32);
                else FLUX_REDUCE(GemmEpilogue::kResidual, false, 64);
                break;
            case GemmEpilogue::kSwiglu:
                if (norm) FLUX_REDUCE(GemmEpilogue::kSwiglu, true, 64);
                else FLUX_REDUCE(GemmEpilogue::kSwiglu, false, 64);
                break;
            case GemmEpilogue::kQkvRope:
                if (norm) FLUX_REDUCE(GemmEpilogue::kQkvRope, true, 64);
                else FLUX_REDUCE(GemmEpilogue::kQkvRope, false, 64);
                break;
        }
#undef FLUX_REDUCE
        return hipGetLastError();
    }
    const dim3 block(kGemmThreads);
    if (narrow_shape(args, epilogue)) {
        // Column counts that are not a multiple of 128 (576): 64 x 64 tiles, K split over
        // blocks where the grid leaves CUs idle (narrow_parts).
        const int parts = narrow_parts(args, false);
        hipError_t st = launch_narrow(args, epilogue, parts, stream);
        if (st != hipSuccess || parts == 1) return st;
        const dim3 rgrid(static_cast<unsigned>((args.m * args.n + 255) / 256));
#define FLUX_REDUCE_PLAIN(P)                                                                                        \
    do {                                                                                                            \
        if (epilogue == GemmEpilogue::kResidual)                                                                    \
            hipLaunchKernelGGL(HIP_KERNEL_NAME(gemm_split_reduce_kernel<GemmEpilogue::kResidual, false, 32, P>),    \
                               rgrid, dim3(256), 0, stream, args);                                                  \
        else                                                                                                        \
            hipLaunchKernelGGL(HIP_KERNEL_NAME(gemm_split_reduce_kernel<GemmEpilogue::kStore, false, 32, P>), rgrid, \
                               dim3(256), 0, stream, args);                                                         \
    } while (0)
        if (parts == 2) FLUX_REDUCE_PLAIN(2);
        else FLUX_REDUCE_PLAIN(kSplitBlocksK);
#undef FLUX_REDUCE_PLAIN
        return hipGetLastError();
    }
    // 128-row tiles when they already give the device two blocks per CU, else 64-row tiles;
    // grids smaller than the device take the copy ring.
    const unsigned gx = static_cast<unsigned>((args.n + kBN - 1) / kBN);
    const bool big = static_cast<int64_t>(gx) * ((args.m + 127) / 128) >= 512;
    const dim3 grid(gx, static_cast<unsigned>(big ? (args.m + 127) / 128 : (args.m + 63) / 64));
    const bool small = static_cast<int64_t>(grid.x) * grid.y < kRingBlocks;
#define FLUX_LAUNCH_GEMM(E)                                                                    \
    do {                                                                                       \
        if (big && E == GemmEpilogue::kQkvRope)                                                \
            hipLaunchKernelGGL(HIP_KERNEL_NAME(gemm_kernel<E, 1, 8>), grid, dim3(512), 0, stream, args);      \
        else if (big)                                                                          \
            hipLaunchKernelGGL(HIP_KERNEL_NAME(gemm_kernel<E, 2>), grid, block, 0, stream, args);             \
        else if (small)                                                                        \
            hipLaunchKernelGGL(HIP_KERNEL_NAME(gemm_ring_kernel<E, 1>), grid, block, 0, stream, args);        \
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

hipError_t launch_norm_gemm(const GemmArgs& args, const float* norm_weight, float eps, float* scratch,
                            GemmEpilogue epilogue, hipStream_t stream) {
    if (split_folds_norm(args, epilogue)) {
        GemmArgs folded = args;
        folded.norm_weight = norm_weight;
        folded.norm_eps = eps;
        return launch_gemm(folded, epilogue, stream);
    }
    const hipError_t e = launch_rmsnorm_rows(args.a, norm_weight, scratch, args.m, args.k, eps, stream);
    if (e != hipSuccess) return e;
    GemmArgs plain = args;
    plain.a = scratch;
    plain.norm_weight = nullptr;
    return launch_gemm(plain, epilogue, stream);
}

bool gemm_folds_norm(const GemmArgs& args, GemmEpilogue epilogue) { return split_folds_norm(args, epilogue); }

hipError_t launch_gemm_residual_norm(const GemmArgs& args, const float* norm_weight, float eps, float* norm_out,
                                     hipStream_t stream) {
    // The fused kernel reads and writes rows as float4: every buffer must be 16-byte aligned
    // (a norm weight that is a view into a larger tensor may not be), else the plain path runs.
    const bool fusable = narrow_shape(args, GemmEpilogue::kResidual) && args.n == kHidden &&
                         split_shape(args, GemmEpilogue::kResidual).rt == 0 && aligned16(args.c) &&
                         aligned16(args.residual) && aligned16(args.split_partials) && aligned16(norm_weight) &&
                         aligned16(norm_out);
    const int parts = fusable ? narrow_parts(args, true) : 1;
    if (parts == 1) {
        const hipError_t e = launch_gemm(args, GemmEpilogue::kResidual, stream);
        if (e != hipSuccess) return e;
        return launch_rmsnorm_rows(args.c, norm_weight, norm_out, args.m, static_cast<int>(args.n), eps, stream);
    }
    const hipError_t e = launch_narrow(args, GemmEpilogue::kResidual, parts, stream);
    if (e != hipSuccess) return e;
    const int64_t grid = (args.m + 3) / 4 < 65535 ? (args.m + 3) / 4 : 65535;
    if (parts == 2)
        hipLaunchKernelGGL(HIP_KERNEL_NAME(split_reduce_residual_norm_kernel<2>), dim3(static_cast<unsigned>(grid)),
                           dim3(256), 0, stream, args, norm_weight, eps, norm_out);
    else
        hipLaunchKernelGGL(HIP_KERNEL_NAME(split_reduce_residual_norm_kernel<kSplitBlocksK>),
                           dim3(static_cast<unsigned>(grid)), dim3(256), 0, stream, args, norm_weight, eps, norm_out);
    return hipGetLastError();
}

size_t prefill_attention_workspace_floats(int64_t seq) {
    if (seq <= kSmallAttnMaxSeq) return 0;  // prefill_attention_small_kernel keeps its partials in LDS
    const int64_t long_tiles = attn_q_tiles(seq) - attn_long_tile(seq);
    if (long_tiles <= 0 || attn_max_chunks(seq) <= 1) return 0;
    return static_cast<size_t>(long_tiles * kQHeads * attn_max_chunks(seq) * kQTile * kPartialRow);
}

hipError_t launch_prefill_attention(const float* q, const float* key_cache, const float* value_cache, int64_t seq,
                                    int64_t capacity, float scale, float* workspace, float* out_rows,
                                    hipStream_t stream) {
    if (seq <= 0 || seq > capacity) return hipErrorInvalidValue;
    if (prefill_attention_workspace_floats(seq) > 0 && workspace == nullptr) return hipErrorInvalidValue;
    if (seq <= kSmallAttnMaxSeq) {
        const dim3 grid(static_cast<unsigned>((seq + kSmallQ - 1) / kSmallQ * kQHeads));
        hipLaunchKernelGGL(prefill_attention_small_kernel, grid, dim3(64 * kSmallWaves), 0, stream, q, key_cache,
                           value_cache, seq, capacity, scale, out_rows);
        return hipGetLastError();
    }
    if (attn_max_chunks(seq) > kMergeMaxChunks) return hipErrorInvalidValue;
    const int64_t blocks = attn_items(seq) * kQHeads;
    hipLaunchKernelGGL(prefill_attention_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kAttnThreads), 0, stream, q,
                       key_cache, value_cache, seq, capacity, scale, workspace, out_rows);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    const int64_t long_tiles = attn_q_tiles(seq) - attn_long_tile(seq);
    if (long_tiles > 0 && attn_max_chunks(seq) > 1) {
        // Registers for at most 4, 8 or 16 chunks: fewer registers, more waves in flight.
        const dim3 grid(static_cast<unsigned>(long_tiles * kQHeads * (kQTile / (kAttnThreads / 16))));
        const int64_t chunks = attn_max_chunks(seq);
        if (chunks <= 4)
            hipLaunchKernelGGL(prefill_attention_merge_kernel<4>, grid, dim3(kAttnThreads), 0, stream, workspace, seq,
                               out_rows);
        else if (chunks <= 8)
            hipLaunchKernelGGL(prefill_attention_merge_kernel<8>, grid, dim3(kAttnThreads), 0, stream, workspace, seq,
                               out_rows);
        else
            hipLaunchKernelGGL(prefill_attention_merge_kernel<kMergeMaxChunks>, grid, dim3(kAttnThreads), 0, stream,
                               workspace, seq, out_rows);
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
