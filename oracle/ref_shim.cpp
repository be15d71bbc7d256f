// C bindings for the reference's own std-only C++ CPU implementations, so the
// CPU oracle can be checked against them.  TEST INFRASTRUCTURE ONLY.
//
// Compiled together with the reference sources in place (never copied):
//   /root/reference/csrc/rmsnorm/rmsnorm.cpp
//   /root/reference/csrc/residual_rmsnorm/residual_rmsnorm.cpp
//   /root/reference/csrc/packed_swiglu/packed_swiglu.cpp
//   /root/reference/csrc/rope/rope.cpp
//   /root/reference/csrc/softmax/softmax.cpp
//   /root/reference/csrc/attention_score_softmax/attention_score_softmax.cpp
// by oracle/Makefile into oracle/_ref/libfluxref.so.
#include "attention_score_softmax.h"
#include "packed_swiglu.h"
#include "residual_rmsnorm.h"
#include "rmsnorm.h"
#include "rope.h"
#include "softmax.h"

#include <exception>

extern "C" {

int ref_rmsnorm(const float* x, const float* w, float* out, long rows, long cols, float eps) {
    try {
        flux::rmsnorm_fp32(x, w, out, rows, cols, eps);
        return 0;
    } catch (const std::exception&) {
        return 1;
    }
}

int ref_residual_rmsnorm(const float* h, const float* r, const float* w, float* norm_out, float* residual_out,
                         long rows, long cols, float eps) {
    try {
        flux::residual_rmsnorm_fp32(h, r, w, norm_out, residual_out, rows, cols, eps);
        return 0;
    } catch (const std::exception&) {
        return 1;
    }
}

int ref_packed_swiglu(const float* packed, float* out, long rows, long inter) {
    try {
        flux::packed_swiglu_fp32(packed, out, rows, inter);
        return 0;
    } catch (const std::exception&) {
        return 1;
    }
}

// Contiguous [heads, seq, dim] query/key with [seq, dim] cos/sin (batch 1).
int ref_rope(const float* q, const float* k, const float* cos, const float* sin, float* q_out, float* k_out,
             long q_heads, long k_heads, long seq, long dim) {
    try {
        const flux::RopeStrides qs{q_heads * seq * dim, seq * dim, dim, 1};
        const flux::RopeStrides ks{k_heads * seq * dim, seq * dim, dim, 1};
        const flux::RopeEmbeddingStrides es{seq * dim, dim, 1};
        flux::rope_fp32(q, k, cos, sin, q_out, k_out, 1, q_heads, k_heads, seq, dim, 1, qs, ks, es, es);
        return 0;
    } catch (const std::exception&) {
        return 1;
    }
}

int ref_softmax(const float* input, float* output, long rows, long width) {
    try {
        flux::softmax_fp32(input, output, rows, width);
        return 0;
    } catch (const std::exception&) {
        return 1;
    }
}

// Contiguous scores [B, H, Q, K]; contiguous mask [mb, mh, mq, mk] (each 1 or full).
int ref_attention_score_softmax(const float* scores, const float* mask, float* output, float scale, long batch,
                                long heads, long query_length, long key_length, long mb, long mh, long mq, long mk) {
    try {
        flux::attention_score_softmax_fp32(scores, mask, output, scale, batch, heads, query_length, key_length, mb,
                                           mh, mq, mk);
        return 0;
    } catch (const std::exception&) {
        return 1;
    }
}

}  // extern "C"
