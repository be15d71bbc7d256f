// Eager operator kernels behind torch.ops.flux.* (the op-at-a-time Flux model
// path): RoPE, row softmax, scaled+masked attention-score softmax, packed
// SwiGLU, the one-token packed-QKV/RoPE/cache-append step and strided one-token
// GQA decode attention.  Reference kernels they replace:
//   rope_cuda.cu:12-85, softmax_cuda.cu:34-341, packed_swiglu_cuda.cu:13-56,
//   packed_qkv_rope_cache_cuda.cu:50-121, gqa_decode_attention_cuda.cu:76-633
// (all under csrc/ of the reference).
//
// All of these are HBM-bound elementwise or row reductions; they use 64-lane
// coalesced rows, DPP wave reductions and grid-stride loops, no MFMA.
#include "flux_kernels.h"

#include <cfloat>

namespace flux {
namespace {

// RoPE of one element pair with Hugging Face rounding: the two products are
// rounded separately before the add (q*cos + rotate_half(q)*sin as two torch
// pointwise kernels).  Contraction into an FMA is disabled here.
__device__ __forceinline__ float rope_value(float x, float paired, bool first_half, float c, float s) {
#pragma clang fp contract(off)
    const float a = x * c;
    const float b = (first_half ? -paired : paired) * s;
    return a + b;
}

// ---------------------------------------------------------------------------
// RoPE: one wave per (batch, head, position) row, lanes over head_dim.
__global__ void __launch_bounds__(256) rope_rows_kernel(const float* __restrict__ query,
                                                        const float* __restrict__ key,
                                                        const float* __restrict__ cos_table,
                                                        const float* __restrict__ sin_table, float* query_out,
                                                        float* key_out, RopeShape shape) {
    const int lane = threadIdx.x & 63;
    const int64_t heads = shape.query_heads + shape.key_heads;
    const int64_t rows = shape.batch * heads * shape.seq;
    const int64_t half = shape.head_dim / 2;
    for (int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); row < rows;
         row += static_cast<int64_t>(gridDim.x) * 4) {
        const int64_t t = row % shape.seq;
        const int64_t bh = row / shape.seq;
        const int64_t head_all = bh % heads;
        const int64_t b = bh / heads;
        const bool is_query = head_all < shape.query_heads;
        const int64_t head = is_query ? head_all : head_all - shape.query_heads;
        const int64_t* st = is_query ? shape.query_strides : shape.key_strides;
        const float* in = (is_query ? query : key) + b * st[0] + head * st[1] + t * st[2];
        const int64_t out_heads = is_query ? shape.query_heads : shape.key_heads;
        float* out = (is_query ? query_out : key_out) + ((b * out_heads + head) * shape.seq + t) * shape.head_dim;
        const int64_t rb = shape.rope_batch == 1 ? 0 : b;
        const float* c = cos_table + rb * shape.cos_strides[0] + t * shape.cos_strides[1];
        const float* s = sin_table + rb * shape.sin_strides[0] + t * shape.sin_strides[1];
        for (int64_t d = lane; d < shape.head_dim; d += 64) {
            const bool first = d < half;
            const int64_t pd = first ? d + half : d - half;
            out[d] = rope_value(in[d * st[3]], in[pd * st[3]], first, c[d * shape.cos_strides[2]],
                                s[d * shape.sin_strides[2]]);
        }
    }
}

// RoPE on float4 quads: thread per (row, quad); needs unit dimension strides,
// head_dim % 8 == 0 and 16-byte aligned rows (checked by the launcher).
__global__ void __launch_bounds__(256) rope_quads_kernel(const float* __restrict__ query,
                                                         const float* __restrict__ key,
                                                         const float* __restrict__ cos_table,
                                                         const float* __restrict__ sin_table, float* query_out,
                                                         float* key_out, RopeShape shape) {
    const int64_t quads = shape.head_dim / 4;
    const int64_t heads = shape.query_heads + shape.key_heads;
    const int64_t items = shape.batch * heads * shape.seq * quads;
    const int64_t half = shape.head_dim / 2;
    for (int64_t item = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; item < items;
         item += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t d0 = 4 * (item % quads);
        const int64_t row = item / quads;
        const int64_t t = row % shape.seq;
        const int64_t bh = row / shape.seq;
        const int64_t head_all = bh % heads;
        const int64_t b = bh / heads;
        const bool is_query = head_all < shape.query_heads;
        const int64_t head = is_query ? head_all : head_all - shape.query_heads;
        const int64_t* st = is_query ? shape.query_strides : shape.key_strides;
        const float* in = (is_query ? query : key) + b * st[0] + head * st[1] + t * st[2];
        const int64_t out_heads = is_query ? shape.query_heads : shape.key_heads;
        float* out = (is_query ? query_out : key_out) + ((b * out_heads + head) * shape.seq + t) * shape.head_dim;
        const int64_t rb = shape.rope_batch == 1 ? 0 : b;
        const float4 c = *reinterpret_cast<const float4*>(cos_table + rb * shape.cos_strides[0] +
                                                          t * shape.cos_strides[1] + d0);
        const float4 sn = *reinterpret_cast<const float4*>(sin_table + rb * shape.sin_strides[0] +
                                                           t * shape.sin_strides[1] + d0);
        const bool first = d0 < half;
        const float4 x = *reinterpret_cast<const float4*>(in + d0);
        const float4 p = *reinterpret_cast<const float4*>(in + (first ? d0 + half : d0 - half));
        *reinterpret_cast<float4*>(out + d0) =
            make_float4(rope_value(x.x, p.x, first, c.x, sn.x), rope_value(x.y, p.y, first, c.y, sn.y),
                        rope_value(x.z, p.z, first, c.z, sn.z), rope_value(x.w, p.w, first, c.w, sn.w));
    }
}

// ---------------------------------------------------------------------------
// Row softmax.  A "source" yields the pre-softmax value of (row, column):
// the plain input, or fl(fl(score * scale) + mask) with a broadcast mask.
// load4 returns columns [col, col + 4) (width % 4 == 0, 16-byte aligned rows).
struct PlainSource {
    const float* input;
    int64_t width;
    __device__ __forceinline__ int64_t row_context(int64_t) const { return 0; }
    __device__ __forceinline__ float load(int64_t row, int64_t, int64_t col) const {
        return input[row * width + col];
    }
    __device__ __forceinline__ float4 load4(int64_t row, int64_t, int64_t col) const {
        return *reinterpret_cast<const float4*>(input + row * width + col);
    }
};

struct MaskedScoreSource {
    const float* scores;
    const float* mask;
    float scale;
    int64_t width;  // key length
    int64_t heads;
    int64_t query_length;
    int64_t mask_strides[4];  // 0 on broadcast dimensions
    __device__ __forceinline__ int64_t row_context(int64_t row) const {
        const int64_t q = row % query_length;
        const int64_t h = (row / query_length) % heads;
        const int64_t b = row / (query_length * heads);
        return b * mask_strides[0] + h * mask_strides[1] + q * mask_strides[2];
    }
    __device__ __forceinline__ float load(int64_t row, int64_t mask_row, int64_t col) const {
#pragma clang fp contract(off)
        const float scaled = scores[row * width + col] * scale;
        return scaled + mask[mask_row + col * mask_strides[3]];
    }
    // The mask quad is one float4 when its key stride is 1 and the row start is
    // 16-byte aligned, one broadcast value when the key dimension is broadcast,
    // else four strided loads (e.g. HF's causal mask sliced from a wider one).
    __device__ __forceinline__ float4 load4(int64_t row, int64_t mask_row, int64_t col) const {
#pragma clang fp contract(off)
        const float4 sv = *reinterpret_cast<const float4*>(scores + row * width + col);
        float4 mv;
        const int64_t ks = mask_strides[3];
        if (ks == 0) {
            const float m = mask[mask_row];
            mv = make_float4(m, m, m, m);
        } else if (ks == 1 && ((reinterpret_cast<uintptr_t>(mask + mask_row) & 15) == 0)) {
            mv = *reinterpret_cast<const float4*>(mask + mask_row + col);
        } else {
            const float* m = mask + mask_row + col * ks;
            mv = make_float4(m[0], m[ks], m[2 * ks], m[3 * ks]);
        }
        return make_float4(sv.x * scale + mv.x, sv.y * scale + mv.y, sv.z * scale + mv.z, sv.w * scale + mv.w);
    }
};

__device__ __forceinline__ float max4(float4 v) { return fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)); }

__device__ __forceinline__ float4 exp4_shift(float4 v, float m) {
    return make_float4(expf(v.x - m), expf(v.y - m), expf(v.z - m), expf(v.w - m));
}

__device__ __forceinline__ float4 div4(float4 v, float d) { return make_float4(v.x / d, v.y / d, v.z / d, v.w / d); }

// One wave per row; kItems values per lane stay in registers (width <= 64*kItems).
template <int kItems, class Source>
__global__ void __launch_bounds__(256) softmax_wave_kernel(Source src, float* out, int64_t rows) {
    const int lane = threadIdx.x & 63;
    const int64_t width = src.width;
    for (int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); row < rows;
         row += static_cast<int64_t>(gridDim.x) * 4) {
        const int64_t ctx = src.row_context(row);
        float v[kItems];
        float mx = -FLT_MAX;
#pragma unroll
        for (int j = 0; j < kItems; ++j) {
            const int64_t col = lane + 64 * j;
            v[j] = col < width ? src.load(row, ctx, col) : -FLT_MAX;
            mx = fmaxf(mx, v[j]);
        }
        mx = wave_max(mx);
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < kItems; ++j) {
            const int64_t col = lane + 64 * j;
            if (col < width) {
                v[j] = expf(v[j] - mx);
                sum += v[j];
            }
        }
        sum = wave_sum(sum);
#pragma unroll
        for (int j = 0; j < kItems; ++j) {
            const int64_t col = lane + 64 * j;
            if (col < width) out[row * width + col] = v[j] / sum;
        }
    }
}

constexpr int kRowThreads = 512;
constexpr int kRowWaves = kRowThreads / 64;

__device__ __forceinline__ float block_max512(float v, float* red) {
    v = wave_max(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < kRowWaves; ++w) r = fmaxf(r, red[w]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ float block_sum512(float v, float* red) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < kRowWaves; ++w) r += red[w];
    __syncthreads();
    return r;
}

// One 512-thread block per row; kItems values per thread in registers
// (width <= 512*kItems).  kItems == 0 selects the unbounded form that re-reads
// the row for each pass.
template <int kItems, class Source>
__global__ void __launch_bounds__(kRowThreads) softmax_block_kernel(Source src, float* out, int64_t rows) {
    __shared__ float red[kRowWaves];
    const int64_t width = src.width;
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const int64_t ctx = src.row_context(row);
        if constexpr (kItems > 0) {
            float v[kItems];
            float mx = -FLT_MAX;
#pragma unroll
            for (int j = 0; j < kItems; ++j) {
                const int64_t col = threadIdx.x + kRowThreads * j;
                v[j] = col < width ? src.load(row, ctx, col) : -FLT_MAX;
                mx = fmaxf(mx, v[j]);
            }
            mx = block_max512(mx, red);
            float sum = 0.0f;
#pragma unroll
            for (int j = 0; j < kItems; ++j) {
                const int64_t col = threadIdx.x + kRowThreads * j;
                if (col < width) {
                    v[j] = expf(v[j] - mx);
                    sum += v[j];
                }
            }
            sum = block_sum512(sum, red);
#pragma unroll
            for (int j = 0; j < kItems; ++j) {
                const int64_t col = threadIdx.x + kRowThreads * j;
                if (col < width) out[row * width + col] = v[j] / sum;
            }
        } else {
            float mx = -FLT_MAX;
            for (int64_t col = threadIdx.x; col < width; col += kRowThreads) mx = fmaxf(mx, src.load(row, ctx, col));
            mx = block_max512(mx, red);
            float sum = 0.0f;
            for (int64_t col = threadIdx.x; col < width; col += kRowThreads) sum += expf(src.load(row, ctx, col) - mx);
            sum = block_sum512(sum, red);
            for (int64_t col = threadIdx.x; col < width; col += kRowThreads)
                out[row * width + col] = expf(src.load(row, ctx, col) - mx) / sum;
        }
    }
}

int grid_for(int64_t units, int64_t per_block) {
    const int64_t blocks = (units + per_block - 1) / per_block;
    return static_cast<int>(blocks < (int64_t{1} << 20) ? blocks : (int64_t{1} << 20));
}

// float4 form: one wave per row, kQuads float4 per lane (width <= 256 kQuads);
// the row stays in registers up to width 8192.
template <int kQuads, class Source>
__global__ void __launch_bounds__(256) softmax_wave4_kernel(Source src, float* out, int64_t rows) {
    const int lane = threadIdx.x & 63;
    const int64_t width = src.width;
    for (int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); row < rows;
         row += static_cast<int64_t>(gridDim.x) * 4) {
        const int64_t ctx = src.row_context(row);
        float4 v[kQuads];
        float mx = -FLT_MAX;
#pragma unroll
        for (int j = 0; j < kQuads; ++j) {
            const int64_t col = 4 * (lane + 64 * j);
            if (col < width) {
                v[j] = src.load4(row, ctx, col);
                mx = fmaxf(mx, max4(v[j]));
            }
        }
        mx = wave_max(mx);
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < kQuads; ++j) {
            const int64_t col = 4 * (lane + 64 * j);
            if (col < width) {
                v[j] = exp4_shift(v[j], mx);
                sum += (v[j].x + v[j].y) + (v[j].z + v[j].w);
            }
        }
        sum = wave_sum(sum);
#pragma unroll
        for (int j = 0; j < kQuads; ++j) {
            const int64_t col = 4 * (lane + 64 * j);
            if (col < width) *reinterpret_cast<float4*>(out + row * width + col) = div4(v[j], sum);
        }
    }
}

template <class Source>
hipError_t launch_softmax_rows(const Source& src, float* out, int64_t rows, bool vec, hipStream_t stream) {
    const int64_t width = src.width;
    const int wave_grid = grid_for(rows, 4);
    const int row_grid = grid_for(rows, 1);
    if (vec && width <= 8192) {
        if (width <= 256) {
            hipLaunchKernelGGL(HIP_KERNEL_NAME(softmax_wave4_kernel<1, Source>), dim3(wave_grid), dim3(256), 0, stream,
                               src, out, rows);
        } else if (width <= 512) {
            hipLaunchKernelGGL(HIP_KERNEL_NAME(softmax_wave4_kernel<2, Source>), dim3(wave_grid), dim3(256), 0, stream,
                               src, out, rows);
        } else if (width <= 1024) {
            hipLaunchKernelGGL(HIP_KERNEL_NAME(softmax_wave4_kernel<4, Source>), dim3(wave_grid), dim3(256), 0, stream,
                               src, out, rows);
        } else if (width <= 2048) {
            hipLaunchKernelGGL(HIP_KERNEL_NAME(softmax_wave4_kernel<8, Source>), dim3(wave_grid), dim3(256), 0, stream,
                               src, out, rows);
        } else if (width <= 4096) {
            hipLaunchKernelGGL(HIP_KERNEL_NAME(softmax_wave4_kernel<16, Source>), dim3(wave_grid), dim3(256), 0,
                               stream, src, out, rows);
        } else {
            hipLaunchKernelGGL(HIP_KERNEL_NAME(softmax_wave4_kernel<32, Source>), dim3(wave_grid), dim3(256), 0,
                               stream, src, out, rows);
        }
        return hipGetLastError();
    }
    if (width <= 64) {
        hipLaunchKernelGGL(HIP_KERNEL_NAME(softmax_wave_kernel<1, Source>), dim3(wave_grid), dim3(256), 0, stream, src,
                           out, rows);
    } else if (width <= 128) {
        hipLaunchKernelGGL(HIP_KERNEL_NAME(softmax_wave_kernel<2, Source>), dim3(wave_grid), dim3(256), 0, stream, src,
                           out, rows);
    } else if (width <= 256) {
        hipLaunchKernelGGL(HIP_KERNEL_NAME(softmax_wave_kernel<4, Source>), dim3(wave_grid), dim3(256), 0, stream, src,
                           out, rows);
    } else if (width <= 512) {
        hipLaunchKernelGGL(HIP_KERNEL_NAME(softmax_wave_kernel<8, Source>), dim3(wave_grid), dim3(256), 0, stream, src,
                           out, rows);
    } else if (width <= 1024) {
        hipLaunchKernelGGL(HIP_KERNEL_NAME(softmax_wave_kernel<16, Source>), dim3(wave_grid), dim3(256), 0, stream,
                           src, out, rows);
    } else if (width <= 2048) {
        hipLaunchKernelGGL(HIP_KERNEL_NAME(softmax_block_kernel<4, Source>), dim3(row_grid), dim3(kRowThreads), 0,
                           stream, src, out, rows);
    } else if (width <= 4096) {
        hipLaunchKernelGGL(HIP_KERNEL_NAME(softmax_block_kernel<8, Source>), dim3(row_grid), dim3(kRowThreads), 0,
                           stream, src, out, rows);
    } else if (width <= 8192) {
        hipLaunchKernelGGL(HIP_KERNEL_NAME(softmax_block_kernel<16, Source>), dim3(row_grid), dim3(kRowThreads), 0,
                           stream, src, out, rows);
    } else {
        hipLaunchKernelGGL(HIP_KERNEL_NAME(softmax_block_kernel<0, Source>), dim3(row_grid), dim3(kRowThreads), 0,
                           stream, src, out, rows);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// RMSNorm rows (HF rounding: w * (x * (1 / sqrt(mean(x^2) + eps)))), and the
// residual form that also stores r = hidden + residual and normalizes r.
// Wave per row with the row in registers as float4 quads (cols % 4 == 0,
// aligned rows, cols <= 4096); otherwise a block per row with scalar loads.
template <int kQuads, bool kResidual>
__global__ void __launch_bounds__(256) rmsnorm_wave4_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ residual,
                                                            const float* __restrict__ w, float* norm_out,
                                                            float* residual_out, int64_t rows, int cols, float eps) {
    const int lane = threadIdx.x & 63;
    for (int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); row < rows;
         row += static_cast<int64_t>(gridDim.x) * 4) {
        float4 v[kQuads];
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < kQuads; ++j) {
            const int c = 4 * (lane + 64 * j);
            if (c < cols) {
                v[j] = *reinterpret_cast<const float4*>(x + row * cols + c);
                if constexpr (kResidual) {
                    const float4 r = *reinterpret_cast<const float4*>(residual + row * cols + c);
                    v[j] = make_float4(v[j].x + r.x, v[j].y + r.y, v[j].z + r.z, v[j].w + r.w);
                    *reinterpret_cast<float4*>(residual_out + row * cols + c) = v[j];
                }
                ss = fmaf(v[j].x, v[j].x, ss);
                ss = fmaf(v[j].y, v[j].y, ss);
                ss = fmaf(v[j].z, v[j].z, ss);
                ss = fmaf(v[j].w, v[j].w, ss);
            }
        }
        const float inv = rms_inverse(wave_sum(ss), cols, eps);
#pragma unroll
        for (int j = 0; j < kQuads; ++j) {
            const int c = 4 * (lane + 64 * j);
            if (c < cols) {
                const float4 g = *reinterpret_cast<const float4*>(w + c);
                *reinterpret_cast<float4*>(norm_out + row * cols + c) =
                    make_float4(g.x * (v[j].x * inv), g.y * (v[j].y * inv), g.z * (v[j].z * inv),
                                g.w * (v[j].w * inv));
            }
        }
    }
}

template <bool kResidual>
__global__ void __launch_bounds__(256) rmsnorm_block_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ residual,
                                                            const float* __restrict__ w, float* norm_out,
                                                            float* residual_out, int64_t rows, int cols, float eps) {
    __shared__ float red[4];
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        float ss = 0.0f;
        for (int c = threadIdx.x; c < cols; c += 256) {
            float r = x[row * cols + c];
            if constexpr (kResidual) r = r + residual[row * cols + c];
            ss = fmaf(r, r, ss);
        }
        ss = wave_sum(ss);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        const float inv = rms_inverse((red[0] + red[1]) + (red[2] + red[3]), cols, eps);
        // Every thread has read red[] before the next row's writes.
        __syncthreads();
        for (int c = threadIdx.x; c < cols; c += 256) {
            float r = x[row * cols + c];
            if constexpr (kResidual) {
                r = r + residual[row * cols + c];
                residual_out[row * cols + c] = r;
            }
            norm_out[row * cols + c] = w[c] * (r * inv);
        }
    }
}

template <bool kResidual>
hipError_t launch_rmsnorm_any(const float* x, const float* residual, const float* w, float* norm_out,
                              float* residual_out, int64_t rows, int cols, float eps, hipStream_t stream) {
    auto aligned = [](const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const bool quads = cols % 4 == 0 && cols <= 4096 && aligned(x) && aligned(residual) && aligned(w) &&
                       aligned(norm_out) && aligned(residual_out);
    if (!quads) {
        hipLaunchKernelGGL(HIP_KERNEL_NAME(rmsnorm_block_kernel<kResidual>), dim3(grid_for(rows, 1)), dim3(256), 0,
                           stream, x, residual, w, norm_out, residual_out, rows, cols, eps);
        return hipGetLastError();
    }
    const int needed = (cols / 4 + 63) / 64;
    const dim3 grid(grid_for(rows, 4));
#define FLUX_LAUNCH_RMSNORM4(Q)                                                                                   \
    hipLaunchKernelGGL(HIP_KERNEL_NAME(rmsnorm_wave4_kernel<Q, kResidual>), grid, dim3(256), 0, stream, x, residual, \
                       w, norm_out, residual_out, rows, cols, eps)
    if (needed <= 1) {
        FLUX_LAUNCH_RMSNORM4(1);
    } else if (needed <= 2) {
        FLUX_LAUNCH_RMSNORM4(2);
    } else if (needed <= 3) {
        FLUX_LAUNCH_RMSNORM4(3);
    } else if (needed <= 4) {
        FLUX_LAUNCH_RMSNORM4(4);
    } else if (needed <= 8) {
        FLUX_LAUNCH_RMSNORM4(8);
    } else {
        FLUX_LAUNCH_RMSNORM4(16);
    }
#undef FLUX_LAUNCH_RMSNORM4
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Packed SwiGLU: out[r, i] = silu(p[r, i]) * p[r, I + i]; one block per row.
// `vec`: inter % 4 == 0 and both base pointers 16-byte aligned (float4 path).
__global__ void __launch_bounds__(256) packed_swiglu_kernel(const float* __restrict__ packed, float* out,
                                                            int64_t rows, int64_t inter, int vec) {
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const float* gate = packed + row * 2 * inter;
        const float* up = gate + inter;
        float* o = out + row * inter;
        if (vec) {
            for (int64_t i = 4 * static_cast<int64_t>(threadIdx.x); i < inter; i += 1024) {
                const float4 g = *reinterpret_cast<const float4*>(gate + i);
                const float4 u = *reinterpret_cast<const float4*>(up + i);
                *reinterpret_cast<float4*>(o + i) =
                    make_float4(silu(g.x) * u.x, silu(g.y) * u.y, silu(g.z) * u.z, silu(g.w) * u.w);
            }
        } else {
            for (int64_t i = threadIdx.x; i < inter; i += 256) o[i] = silu(gate[i]) * up[i];
        }
    }
}

// ---------------------------------------------------------------------------
// One-token packed QKV [960] -> RoPE(q), RoPE(k) at *position; K/V stored at
// cache row *position; q -> query_out [9, 64].  An out-of-range position
// writes nothing.  When cache_length is non-NULL it becomes position + 1 after
// every thread has read the position (one block, so a barrier orders them).
__global__ void __launch_bounds__(256) packed_qkv_rope_cache_kernel(PackedQkvArgs a) {
    __shared__ int64_t position_s;
    if (threadIdx.x == 0) position_s = *a.position;
    __syncthreads();
    const int64_t position = position_s;
    if (position < 0 || position >= a.capacity) return;
    constexpr int kQ = kQHeads * kHeadDim;
    constexpr int kK = kKVHeads * kHeadDim;
    for (int i = threadIdx.x; i < kQKV; i += 256) {
        const float x = a.packed[i * a.packed_stride];
        if (i < kQ + kK) {
            const int d = i & (kHeadDim - 1);
            const bool first = d < kHeadDim / 2;
            const int pi = first ? i + kHeadDim / 2 : i - kHeadDim / 2;
            const float r = rope_value(x, a.packed[pi * a.packed_stride], first, a.cos[d * a.cos_stride],
                                       a.sin[d * a.sin_stride]);
            if (i < kQ) {
                a.query_out[i] = r;
            } else {
                const int head = (i - kQ) / kHeadDim;
                a.key_cache[head * a.key_strides[1] + position * a.key_strides[2] + d * a.key_strides[3]] = r;
            }
        } else {
            const int j = i - kQ - kK;
            const int head = j / kHeadDim;
            const int d = j & (kHeadDim - 1);
            a.value_cache[head * a.value_strides[1] + position * a.value_strides[2] + d * a.value_strides[3]] = x;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0 && a.cache_length != nullptr) *a.cache_length = position + 1;
}

// ---------------------------------------------------------------------------
// Strided one-token GQA decode attention, any head_dim (head_dim 64 has the
// faster gqa_strided_chunk64_kernel below).  Block (query head h, key chunk c)
// scores keys [256c, 256c+256) of KV head h / groups: 16 lanes per key (4 keys
// per wave per step), then the chunk softmax and P.V with lanes over head_dim.
// With one chunk the block writes the normalized output; otherwise it writes
// (o[dim], m, l) partials that gqa_strided_merge_kernel combines.
constexpr int kGqaChunk = 256;

__global__ void __launch_bounds__(256) gqa_strided_chunk_kernel(GqaStridedArgs a) {
    extern __shared__ float gqa_smem[];
    float* qs = gqa_smem;                  // [dim]
    float* p = gqa_smem + a.dim;           // [256] scores, then probabilities
    float* red = p + kGqaChunk;            // [4 * 64] cross-wave partials
    float* stat = red + 4 * 64;            // [8] block reduction slots
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int h = blockIdx.x / a.chunks;
    const int c = blockIdx.x % a.chunks;
    const int kh = h / a.groups;
    int64_t valid = a.cache_length != nullptr ? *a.cache_length : a.capacity;
    valid = valid < 1 ? 1 : (valid > a.capacity ? a.capacity : valid);
    const int64_t begin = static_cast<int64_t>(c) * kGqaChunk;
    const int64_t left = valid - begin;
    const int n = left <= 0 ? 0 : (left >= kGqaChunk ? kGqaChunk : static_cast<int>(left));

    for (int d = t; d < a.dim; d += 256) qs[d] = a.q[h * a.q_strides[1] + d * a.q_strides[3]];
    __syncthreads();

    const int l16 = lane & 15;
    const int slot = t >> 4;  // 16 keys per block step
    const float* kbase = a.k + kh * a.k_strides[1];
    for (int base = 0; base < n; base += 16) {
        const int j = base + slot;
        float dot = 0.0f;
        if (j < n) {
            const float* krow = kbase + (begin + j) * a.k_strides[2];
            if (a.vec) {
                for (int d0 = 4 * l16; d0 < a.dim; d0 += 64) {
                    const float4 kv = *reinterpret_cast<const float4*>(krow + d0);
                    dot = fmaf(qs[d0], kv.x, dot);
                    dot = fmaf(qs[d0 + 1], kv.y, dot);
                    dot = fmaf(qs[d0 + 2], kv.z, dot);
                    dot = fmaf(qs[d0 + 3], kv.w, dot);
                }
            } else {
                for (int d = l16; d < a.dim; d += 16) dot = fmaf(qs[d], krow[d * a.k_strides[3]], dot);
            }
        }
        dot = row16_sum(dot);
        if (l16 == 0 && j < n) {
#pragma clang fp contract(off)
            float s = dot * a.scale;
            if (a.mask != nullptr) s = s + a.mask[h * a.mask_strides[1] + (begin + j) * a.mask_strides[3]];
            p[j] = s;
        }
    }
    __syncthreads();

    // Chunk softmax statistics (max starts at -FLT_MAX so fully masked chunks give p = 0).
    const float s = t < n ? p[t] : -FLT_MAX;
    float m = wave_max(fmaxf(s, -FLT_MAX));
    if (lane == 0) stat[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(stat[0], stat[1]), fmaxf(stat[2], stat[3]));
    const float e = t < n ? expf(s - m) : 0.0f;
    if (t < n) p[t] = e;
    float l = wave_sum(e);
    __syncthreads();
    if (lane == 0) stat[4 + wave] = l;
    __syncthreads();
    l = (stat[4] + stat[5]) + (stat[6] + stat[7]);

    const float* vbase = a.v + kh * a.v_strides[1];
    float* part = a.workspace + (static_cast<int64_t>(h) * a.chunks + c) * (a.dim + 2);
    for (int d0 = 0; d0 < a.dim; d0 += 64) {
        const int d = d0 + lane;
        float acc = 0.0f;
        if (d < a.dim) {
#pragma unroll 4
            for (int j = wave; j < n; j += 4) acc = fmaf(p[j], vbase[(begin + j) * a.v_strides[2] + d * a.v_strides[3]], acc);
        }
        red[wave * 64 + lane] = acc;
        __syncthreads();
        if (wave == 0 && d < a.dim) {
            const float o = (red[lane] + red[64 + lane]) + (red[128 + lane] + red[192 + lane]);
            if (a.chunks == 1) {
                a.out[h * a.dim + d] = o / l;
            } else {
                part[d] = o;
            }
        }
        __syncthreads();
    }
    if (a.chunks > 1 && t == 0) {
        part[a.dim] = m;
        part[a.dim + 1] = l;
    }
}

// head_dim 64: block (query head h, 128-key chunk).  Thread (slot = t / 16,
// l16 = t % 16) owns keys slot + 16 i (i < 8) and dims [4 l16, 4 l16 + 4): all
// 8 K and 8 V float4s are issued before any arithmetic, so one block waits for
// one HBM round trip.  QK is a 16-lane row reduction per key; P.V accumulates
// per lane and is reduced over the 16 slots (xor-16/32 shuffles, then LDS).
constexpr int kGqa64Keys = 8;
constexpr int kGqa64Chunk = 16 * kGqa64Keys;  // 128

template <bool kVec>
__device__ __forceinline__ float4 load_row4(const float* row, int64_t dim_stride, int d0) {
    if constexpr (kVec) {
        return *reinterpret_cast<const float4*>(row + d0);
    } else {
        return make_float4(row[d0 * dim_stride], row[(d0 + 1) * dim_stride], row[(d0 + 2) * dim_stride],
                           row[(d0 + 3) * dim_stride]);
    }
}

template <bool kVec>
__global__ void __launch_bounds__(256) gqa_strided_chunk64_kernel(GqaStridedArgs a) {
    __shared__ float red[4 * 64];
    __shared__ float stat[8];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int slot = t >> 4;
    const int d0 = 4 * (t & 15);
    const int h = blockIdx.x / a.chunks;
    const int c = blockIdx.x % a.chunks;
    const int kh = h / a.groups;
    int64_t valid = a.cache_length != nullptr ? *a.cache_length : a.capacity;
    valid = valid < 1 ? 1 : (valid > a.capacity ? a.capacity : valid);
    const int64_t begin = static_cast<int64_t>(c) * kGqa64Chunk;
    const int64_t left = valid - begin;
    const int n = left <= 0 ? 0 : (left >= kGqa64Chunk ? kGqa64Chunk : static_cast<int>(left));

    const float* kbase = a.k + kh * a.k_strides[1] + begin * a.k_strides[2];
    const float* vbase = a.v + kh * a.v_strides[1] + begin * a.v_strides[2];
    // Every load the block needs (q, its K and V rows and their mask values) is issued before
    // any arithmetic, so the block waits for one memory round trip.
    const float* qrow = a.q + h * a.q_strides[1];
    const float4 q4 = make_float4(qrow[d0 * a.q_strides[3]], qrow[(d0 + 1) * a.q_strides[3]],
                                  qrow[(d0 + 2) * a.q_strides[3]], qrow[(d0 + 3) * a.q_strides[3]]);
    float4 kv[kGqa64Keys], vv[kGqa64Keys];
    float mk[kGqa64Keys];
#pragma unroll
    for (int i = 0; i < kGqa64Keys; ++i) {
        const int j = slot + 16 * i;
        mk[i] = 0.0f;
        if (j < n) {
            kv[i] = load_row4<kVec>(kbase + j * a.k_strides[2], a.k_strides[3], d0);
            vv[i] = load_row4<kVec>(vbase + j * a.v_strides[2], a.v_strides[3], d0);
            if (a.mask != nullptr) mk[i] = a.mask[h * a.mask_strides[1] + (begin + j) * a.mask_strides[3]];
        } else {
            kv[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            vv[i] = kv[i];
        }
    }

    float score[kGqa64Keys];
    float mx = -FLT_MAX;
#pragma unroll
    for (int i = 0; i < kGqa64Keys; ++i) {
        float dot = q4.x * kv[i].x;
        dot = fmaf(q4.y, kv[i].y, dot);
        dot = fmaf(q4.z, kv[i].z, dot);
        dot = fmaf(q4.w, kv[i].w, dot);
        dot = row16_sum(dot);
        const int j = slot + 16 * i;
        float sc = -FLT_MAX;
        if (j < n) {
#pragma clang fp contract(off)
            sc = dot * a.scale;
            if (a.mask != nullptr) sc = sc + mk[i];
        }
        score[i] = sc;
        mx = fmaxf(mx, sc);
    }
    mx = wave_max(mx);
    if (lane == 0) stat[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(stat[0], stat[1]), fmaxf(stat[2], stat[3]));

    float l = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int i = 0; i < kGqa64Keys; ++i) {
        const int j = slot + 16 * i;
        const float e = j < n ? expf(score[i] - mx) : 0.0f;
        l += e;
        acc.x = fmaf(e, vv[i].x, acc.x);
        acc.y = fmaf(e, vv[i].y, acc.y);
        acc.z = fmaf(e, vv[i].z, acc.z);
        acc.w = fmaf(e, vv[i].w, acc.w);
    }
    // Sum over the 4 slots of this wave (rows of 16 lanes), then over the 4 waves.
    l += __shfl_xor(l, 16, kWave);
    l += __shfl_xor(l, 32, kWave);
    acc.x += __shfl_xor(acc.x, 16, kWave);
    acc.y += __shfl_xor(acc.y, 16, kWave);
    acc.z += __shfl_xor(acc.z, 16, kWave);
    acc.w += __shfl_xor(acc.w, 16, kWave);
    acc.x += __shfl_xor(acc.x, 32, kWave);
    acc.y += __shfl_xor(acc.y, 32, kWave);
    acc.z += __shfl_xor(acc.z, 32, kWave);
    acc.w += __shfl_xor(acc.w, 32, kWave);
    if (lane < 16) *reinterpret_cast<float4*>(red + wave * 64 + d0) = acc;
    if (lane == 0) stat[4 + wave] = l;
    __syncthreads();
    if (t < 64) {
        const float o = (red[t] + red[64 + t]) + (red[128 + t] + red[192 + t]);
        const float total = (stat[4] + stat[5]) + (stat[6] + stat[7]);
        if (a.chunks == 1) {
            a.out[h * 64 + t] = o / total;
        } else {
            float* part = a.workspace + (static_cast<int64_t>(h) * a.chunks + c) * 66;
            part[t] = o;
            if (t == 0) {
                part[64] = mx;
                part[65] = total;
            }
        }
    }
}

// Merge of the (o, m, l) chunk partials of one query head: chunk weights
// exp(m_c - M) are computed once (threads over chunks) and kept in LDS; then
// wave w sums chunks c = w mod 4 for 64 dims at a time and LDS adds the 4 waves.
constexpr int kGqaMaxChunks = 256;

__global__ void __launch_bounds__(256) gqa_strided_merge_kernel(const float* __restrict__ workspace, float* out,
                                                                int chunks, int dim) {
    __shared__ float weight[kGqaMaxChunks];
    __shared__ float red[4 * 64];
    __shared__ float stat[8];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int h = blockIdx.x;
    const int64_t stride = dim + 2;
    const float* parts = workspace + static_cast<int64_t>(h) * chunks * stride;
    // head_dim 64 with at most 64 chunks (contexts up to 8192): the chunk values this thread
    // sums are requested together with the (m, l) words, so the block waits for one memory
    // round trip instead of two.
    constexpr int kPre = 16;
    const bool pre = dim == 64 && chunks <= 4 * kPre;
    float pv[kPre];
    if (pre) {
#pragma unroll
        for (int k = 0; k < kPre; ++k) {
            const int c = wave + 4 * k;
            pv[k] = c < chunks ? parts[c * stride + lane] : 0.0f;
        }
    }
    const float m = t < chunks ? parts[t * stride + dim] : -FLT_MAX;
    const float l = t < chunks ? parts[t * stride + dim + 1] : 0.0f;
    float mx = wave_max(m);
    if (lane == 0) stat[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(stat[0], stat[1]), fmaxf(stat[2], stat[3]));
    const float w = t < chunks ? expf(m - mx) : 0.0f;
    if (t < chunks) weight[t] = w;
    float total = wave_sum(l * w);
    if (lane == 0) stat[4 + wave] = total;
    __syncthreads();
    total = (stat[4] + stat[5]) + (stat[6] + stat[7]);
    if (pre) {
        float o = 0.0f;
#pragma unroll
        for (int k = 0; k < kPre; ++k) {
            const int c = wave + 4 * k;
            if (c < chunks) o = fmaf(pv[k], weight[c], o);
        }
        red[wave * 64 + lane] = o;
        __syncthreads();
        if (wave == 0) out[h * 64 + lane] = ((red[lane] + red[64 + lane]) + (red[128 + lane] + red[192 + lane])) / total;
        return;
    }
    for (int d0 = 0; d0 < dim; d0 += 64) {
        const int d = d0 + lane;
        float o = 0.0f;
        if (d < dim) {
#pragma unroll 4
            for (int c = wave; c < chunks; c += 4) o = fmaf(parts[c * stride + d], weight[c], o);
        }
        red[wave * 64 + lane] = o;
        __syncthreads();
        if (wave == 0 && d < dim) out[h * dim + d] = ((red[lane] + red[64 + lane]) + (red[128 + lane] + red[192 + lane])) / total;
        __syncthreads();
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// Host launchers.

hipError_t launch_rope(const float* query, const float* key, const float* cos_table, const float* sin_table,
                       float* query_out, float* key_out, const RopeShape& shape, hipStream_t stream) {
    const int64_t rows = shape.batch * (shape.query_heads + shape.key_heads) * shape.seq;
    auto aligned = [](const float* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    bool quads = shape.head_dim % 8 == 0 && shape.query_strides[3] == 1 && shape.key_strides[3] == 1 &&
                 shape.cos_strides[2] == 1 && shape.sin_strides[2] == 1 && aligned(query) && aligned(key) &&
                 aligned(cos_table) && aligned(sin_table) && aligned(query_out) && aligned(key_out);
    for (int i = 0; i < 3; ++i) {
        quads = quads && shape.query_strides[i] % 4 == 0 && shape.key_strides[i] % 4 == 0;
        if (i < 2) quads = quads && shape.cos_strides[i] % 4 == 0 && shape.sin_strides[i] % 4 == 0;
    }
    if (quads) {
        hipLaunchKernelGGL(rope_quads_kernel, dim3(grid_for(rows * (shape.head_dim / 4), 256)), dim3(256), 0, stream,
                           query, key, cos_table, sin_table, query_out, key_out, shape);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(rope_rows_kernel, dim3(grid_for(rows, 4)), dim3(256), 0, stream, query, key, cos_table,
                       sin_table, query_out, key_out, shape);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_rows(const float* x, const float* w, float* out, int64_t rows, int cols, float eps,
                               hipStream_t stream) {
    return launch_rmsnorm_any<false>(x, nullptr, w, out, nullptr, rows, cols, eps, stream);
}

hipError_t launch_residual_rmsnorm_rows(const float* hidden, const float* residual, const float* w, float* norm_out,
                                        float* residual_out, int64_t rows, int cols, float eps, hipStream_t stream) {
    return launch_rmsnorm_any<true>(hidden, residual, w, norm_out, residual_out, rows, cols, eps, stream);
}

static bool quad_rows(const void* a, const void* b, int64_t width) {
    return (width & 3) == 0 && (reinterpret_cast<uintptr_t>(a) & 15) == 0 && (reinterpret_cast<uintptr_t>(b) & 15) == 0;
}

hipError_t launch_softmax(const float* input, float* output, int64_t rows, int64_t width, hipStream_t stream) {
    return launch_softmax_rows(PlainSource{input, width}, output, rows, quad_rows(input, output, width), stream);
}

hipError_t launch_attention_score_softmax(const float* scores, const float* mask, float* output, float scale,
                                          int64_t batch, int64_t heads, int64_t query_length, int64_t key_length,
                                          const int64_t mask_strides[4], hipStream_t stream) {
    MaskedScoreSource src{scores, mask, scale, key_length, heads, query_length, {0, 0, 0, 0}};
    for (int i = 0; i < 4; ++i) src.mask_strides[i] = mask_strides[i];
    return launch_softmax_rows(src, output, batch * heads * query_length, quad_rows(scores, output, key_length),
                               stream);
}

hipError_t launch_packed_swiglu(const float* packed, float* out, int64_t rows, int64_t inter, hipStream_t stream) {
    const int vec = (inter & 3) == 0 && (reinterpret_cast<uintptr_t>(packed) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    hipLaunchKernelGGL(packed_swiglu_kernel, dim3(grid_for(rows, 1)), dim3(256), 0, stream, packed, out, rows, inter,
                       vec);
    return hipGetLastError();
}

hipError_t launch_packed_qkv_rope_cache(const PackedQkvArgs& args, hipStream_t stream) {
    hipLaunchKernelGGL(packed_qkv_rope_cache_kernel, dim3(1), dim3(256), 0, stream, args);
    return hipGetLastError();
}

int gqa_strided_chunks(int64_t capacity, int64_t head_dim) {
    const int64_t chunk = head_dim == 64 ? kGqa64Chunk : kGqaChunk;
    return static_cast<int>((capacity + chunk - 1) / chunk);
}

size_t gqa_strided_workspace_floats(int64_t query_heads, int64_t capacity, int64_t head_dim) {
    const int chunks = gqa_strided_chunks(capacity, head_dim);
    if (chunks <= 1) return 0;
    return static_cast<size_t>(query_heads) * chunks * (head_dim + 2);
}

hipError_t launch_gqa_strided(const GqaStridedArgs& args, hipStream_t stream) {
    if (args.chunks < 1 || args.chunks > kGqaMaxChunks) return hipErrorInvalidValue;
    const dim3 grid(args.query_heads * args.chunks);
    if (args.dim == 64 && args.vec) {
        hipLaunchKernelGGL(HIP_KERNEL_NAME(gqa_strided_chunk64_kernel<true>), grid, dim3(256), 0, stream, args);
    } else if (args.dim == 64) {
        hipLaunchKernelGGL(HIP_KERNEL_NAME(gqa_strided_chunk64_kernel<false>), grid, dim3(256), 0, stream, args);
    } else {
        const size_t lds = (static_cast<size_t>(args.dim) + kGqaChunk + 4 * 64 + 8) * sizeof(float);
        hipLaunchKernelGGL(gqa_strided_chunk_kernel, grid, dim3(256), lds, stream, args);
    }
    hipError_t st = hipGetLastError();
    if (st != hipSuccess || args.chunks == 1) return st;
    hipLaunchKernelGGL(gqa_strided_merge_kernel, dim3(args.query_heads), dim3(256), 0, stream, args.workspace, args.out,
                       args.chunks, args.dim);
    return hipGetLastError();
}

}  // namespace flux
