"""``torch.ops.flux.*``: the reference's eager operator set on gfx950 HIP kernels.

Same schemas as the reference's TORCH_LIBRARY fragments (cited per op) and the
same argument validation and messages, FakeTensor contracts and ``*_native`` /
``*_native_out`` / ``native_*_is_available`` / ``native_*_load_error`` entry
points (``flux/ops/native_*.py``).  Each CUDA (ROCm) kernel is a call through
the C ABI of ``libflux_amd.so`` on the tensor's current stream.

There is no CPU kernel: the CPU dispatch key validates the arguments exactly
like the GPU path (so argument errors read the same) and then raises, and a
missing native library raises on every call.  Nothing here computes on the
host.
"""

from __future__ import annotations

import ctypes
import math
from typing import Sequence

import torch

from flux_amd import _native

_FLT_MAX = torch.finfo(torch.float32).max
_MAX_CAPACITY = 16384
_RMSNORM_MAX_WIDTH = 65536
_GQA_OUT_CHUNK = 128  # key chunk of the reference's gqa_decode_attention_out workspace shape

_LIBRARY = torch.library.Library("flux", "FRAGMENT")

# Schemas: csrc/rmsnorm/rmsnorm_torch.cpp:152-158, residual_rmsnorm_torch.cpp
# (residual_rmsnorm(_out)), rope_torch.cpp:133-136, softmax_torch.cpp,
# attention_score_softmax_torch.cpp:119-123, packed_swiglu_torch.cpp,
# gqa_decode_attention_torch.cpp:337-345, packed_qkv_rope_cache_torch.cpp:173-182,
# packed_gate_up_gemv_torch.cpp (all under the reference's csrc/).
SCHEMAS = {
    "rmsnorm": "rmsnorm(Tensor input, Tensor weight, float epsilon) -> Tensor",
    "rmsnorm_out": "rmsnorm_out(Tensor input, Tensor weight, float epsilon, Tensor(a!) output) -> Tensor(a!)",
    "residual_rmsnorm": ("residual_rmsnorm(Tensor hidden, Tensor residual, Tensor weight, float epsilon) -> "
                         "(Tensor norm_out, Tensor residual_out)"),
    "residual_rmsnorm_out": ("residual_rmsnorm_out(Tensor hidden, Tensor residual, Tensor weight, float epsilon, "
                             "Tensor(a!) norm_out, Tensor(b!) residual_out) -> (Tensor(a!), Tensor(b!))"),
    "rope": "rope(Tensor query, Tensor key, Tensor cos, Tensor sin) -> (Tensor, Tensor)",
    "softmax": "softmax(Tensor input) -> Tensor",
    "attention_score_softmax": ("attention_score_softmax(Tensor scores, Tensor additive_attention_mask, "
                                "float scale) -> Tensor"),
    "packed_swiglu": "packed_swiglu(Tensor packed) -> Tensor",
    "packed_swiglu_out": "packed_swiglu_out(Tensor packed, Tensor(a!) output) -> Tensor(a!)",
    "gqa_decode_attention": ("gqa_decode_attention(Tensor query, Tensor key_cache, Tensor value_cache, "
                             "Tensor? additive_attention_mask, float scale, Tensor? cache_length=None) -> Tensor"),
    "gqa_decode_attention_out": ("gqa_decode_attention_out(Tensor query, Tensor key_cache, Tensor value_cache, "
                                 "Tensor? additive_attention_mask, float scale, Tensor? cache_length, "
                                 "Tensor(a!) output, Tensor(b!) workspace) -> Tensor(a!)"),
    "packed_qkv_rope_cache": ("packed_qkv_rope_cache(Tensor packed_qkv, Tensor cos, Tensor sin, "
                              "Tensor(a!) key_cache, Tensor(b!) value_cache, Tensor(c!) cache_length) -> Tensor"),
    "packed_qkv_rope_cache_out": ("packed_qkv_rope_cache_out(Tensor packed_qkv, Tensor cos, Tensor sin, "
                                  "Tensor(a!) key_cache, Tensor(b!) value_cache, Tensor(c!) cache_length, "
                                  "Tensor(d!) query_output) -> Tensor(d!)"),
    "packed_gate_up_swiglu_out": "packed_gate_up_swiglu_out(Tensor input, Tensor weight, Tensor(a!) output) -> Tensor(a!)",
}

for _schema in SCHEMAS.values():
    _LIBRARY.define(_schema)


# ---------------------------------------------------------------------------
# Helpers.

def _check(condition, message: str) -> None:
    torch._check(condition, lambda: message)


def _grad_free(op: str, *tensors: torch.Tensor | None) -> None:
    _check(not torch.is_grad_enabled() or not any(t is not None and t.requires_grad for t in tensors),
           f"{op} is inference-only; use torch.no_grad() or torch.inference_mode() for tensors that require "
           "gradients")


def _finite_fp32(value: float) -> bool:
    return math.isfinite(value) and abs(value) <= _FLT_MAX


def _aliases(a: torch.Tensor, b: torch.Tensor) -> bool:
    return a.device == b.device and a.untyped_storage().data_ptr() == b.untyped_storage().data_ptr()


def _strides(tensor: torch.Tensor, count: int):
    return _native.length_array([int(s) for s in tensor.stride()[:count]])


def _call(function: str, *args) -> None:
    library = _native.load()
    _native.check(getattr(library, function)(*args))


def _stream(tensor: torch.Tensor) -> int:
    return _native.current_stream(tensor.device)


def _cpu_unsupported(op: str):
    raise RuntimeError(f"{op}: this build has no CPU kernel; Flux operators run on ROCm (HIP) GPU tensors "
                       "(move the tensors to a cuda device)")


def _require_gpu(op: str, tensor: torch.Tensor) -> None:
    _check(tensor.is_cuda, f"{op}: CUDA dispatch requires CUDA tensors")


# ---------------------------------------------------------------------------
# rmsnorm / rmsnorm_out (csrc/rmsnorm/rmsnorm_torch.cpp:15-127).

def _validate_rmsnorm(input: torch.Tensor, weight: torch.Tensor, epsilon: float) -> None:
    op = "flux::rmsnorm"
    _check(input.dim() >= 1, f"{op}: input must have at least one dimension")
    _check(input.shape[-1] > 0, f"{op}: input must have a non-empty final dimension")
    _check(input.numel() > 0, f"{op}: input must contain at least one row")
    _check(input.dtype == torch.float32, f"{op}: input must have dtype torch.float32")
    _check(weight.dtype == torch.float32, f"{op}: weight must have dtype torch.float32")
    _check(weight.dim() == 1, f"{op}: weight must be one-dimensional")
    _check(weight.shape[0] == input.shape[-1], f"{op}: weight length must equal input.size(-1)")
    _check(input.device == weight.device, f"{op}: input and weight must be on the same device")
    _check(epsilon > 0.0 and _finite_fp32(epsilon), f"{op}: epsilon must be a positive finite FP32 value")
    _grad_free(op, input, weight)


def _validate_rmsnorm_out(input, weight, epsilon, output) -> None:
    _validate_rmsnorm(input, weight, epsilon)
    op = "flux::rmsnorm_out"
    _check(input.is_contiguous() and weight.is_contiguous(), f"{op}: input and weight must be contiguous")
    _check(output.shape == input.shape, f"{op}: output shape must match input")
    _check(output.dtype == torch.float32 and output.device == input.device,
           f"{op}: output must be float32 on the input device")
    _check(output.is_contiguous(), f"{op}: output must be contiguous")


def _launch_rmsnorm(input, weight, epsilon, output) -> None:
    cols = int(input.shape[-1])
    _check(cols <= _RMSNORM_MAX_WIDTH, f"flux::rmsnorm: final dimension above {_RMSNORM_MAX_WIDTH} is unsupported")
    with torch.cuda.device(input.device):
        _call("flux_rmsnorm_f32", input.data_ptr(), weight.data_ptr(), output.data_ptr(), input.numel() // cols, cols,
              float(epsilon), _stream(input))


def _rmsnorm_cuda(input, weight, epsilon):
    _validate_rmsnorm(input, weight, epsilon)
    _require_gpu("flux::rmsnorm", input)
    x, w = input.contiguous(), weight.contiguous()
    output = torch.empty_like(x)
    _launch_rmsnorm(x, w, epsilon, output)
    return output


def _rmsnorm_out_cuda(input, weight, epsilon, output):
    _validate_rmsnorm_out(input, weight, epsilon, output)
    _require_gpu("flux::rmsnorm_out", input)
    _check(not _aliases(output, input) and not _aliases(output, weight),
           "flux::rmsnorm_out: output must not alias an input")
    _launch_rmsnorm(input, weight, epsilon, output)
    return output


# ---------------------------------------------------------------------------
# residual_rmsnorm / _out (csrc/residual_rmsnorm/residual_rmsnorm_torch.cpp:16-170).

def _validate_residual_rmsnorm(hidden, residual, weight, epsilon) -> None:
    op = "flux::residual_rmsnorm"
    _check(hidden.dim() >= 1, f"{op}: hidden must have at least one dimension")
    _check(hidden.shape[-1] > 0, f"{op}: hidden must have a non-empty final dimension")
    _check(hidden.numel() > 0, f"{op}: hidden must contain at least one row")
    _check(hidden.shape == residual.shape, f"{op}: hidden and residual must have the same shape")
    _check(hidden.dtype == torch.float32, f"{op}: hidden must have dtype torch.float32")
    _check(residual.dtype == torch.float32, f"{op}: residual must have dtype torch.float32")
    _check(weight.dtype == torch.float32, f"{op}: weight must have dtype torch.float32")
    _check(weight.dim() == 1, f"{op}: weight must be one-dimensional")
    _check(weight.shape[0] == hidden.shape[-1], f"{op}: weight length must equal hidden.size(-1)")
    _check(hidden.device == residual.device and hidden.device == weight.device,
           f"{op}: hidden, residual, and weight must be on the same device")
    _check(epsilon >= 0.0 and _finite_fp32(epsilon), f"{op}: epsilon must be a non-negative finite FP32 value")
    _grad_free(op, hidden, residual, weight)


def _launch_residual_rmsnorm(hidden, residual, weight, epsilon, norm_out, residual_out) -> None:
    cols = int(hidden.shape[-1])
    _check(cols <= _RMSNORM_MAX_WIDTH,
           f"flux::residual_rmsnorm: final dimension above {_RMSNORM_MAX_WIDTH} is unsupported")
    with torch.cuda.device(hidden.device):
        _call("flux_residual_rmsnorm_f32", hidden.data_ptr(), residual.data_ptr(), weight.data_ptr(),
              norm_out.data_ptr(), residual_out.data_ptr(), hidden.numel() // cols, cols, float(epsilon),
              _stream(hidden))


def _residual_rmsnorm_cuda(hidden, residual, weight, epsilon):
    _validate_residual_rmsnorm(hidden, residual, weight, epsilon)
    _require_gpu("flux::residual_rmsnorm", hidden)
    h, r, w = hidden.contiguous(), residual.contiguous(), weight.contiguous()
    norm_out, residual_out = torch.empty_like(h), torch.empty_like(h)
    _launch_residual_rmsnorm(h, r, w, epsilon, norm_out, residual_out)
    return norm_out, residual_out


def _residual_rmsnorm_out_cuda(hidden, residual, weight, epsilon, norm_out, residual_out):
    _validate_residual_rmsnorm(hidden, residual, weight, epsilon)
    op = "flux::residual_rmsnorm_out"
    _require_gpu(op, hidden)
    _check(hidden.is_contiguous() and residual.is_contiguous() and weight.is_contiguous(),
           f"{op}: inputs must be contiguous")
    for output in (norm_out, residual_out):
        _check(output.shape == hidden.shape, f"{op}: output shapes must match hidden")
        _check(output.dtype == torch.float32 and output.device == hidden.device and output.is_contiguous(),
               f"{op}: outputs must be contiguous float32 on the input device")
        _check(not any(_aliases(output, t) for t in (hidden, residual, weight)), f"{op}: outputs must not alias inputs")
    _check(not _aliases(norm_out, residual_out), f"{op}: outputs must not alias each other")
    _launch_residual_rmsnorm(hidden, residual, weight, epsilon, norm_out, residual_out)
    return norm_out, residual_out


# ---------------------------------------------------------------------------
# rope (csrc/rope/rope_torch.cpp:16-131).

def _validate_rope(query, key, cos, sin) -> None:
    op = "flux::rope"
    _check(query.dim() == 4 and key.dim() == 4, f"{op}: query and key must be rank four")
    _check(cos.dim() == 3 and sin.dim() == 3, f"{op}: cos and sin must be rank three")
    _check(query.dtype == torch.float32 and key.dtype == torch.float32,
           f"{op}: query and key must have dtype torch.float32")
    _check(cos.dtype == torch.float32 and sin.dtype == torch.float32,
           f"{op}: cos and sin must have dtype torch.float32")
    _check(query.device == key.device and query.device == cos.device and query.device == sin.device,
           f"{op}: all tensors must be on the same device")
    _check(all(s > 0 for s in query.shape) and key.shape[1] > 0, f"{op}: tensor dimensions must be non-empty")
    _check(query.shape[3] % 2 == 0, f"{op}: head_dim must be even")
    _check(key.shape[0] == query.shape[0] and key.shape[2] == query.shape[2] and key.shape[3] == query.shape[3],
           f"{op}: query and key batch, sequence, and head dimensions must match")
    _check(cos.shape == sin.shape, f"{op}: cos and sin shapes must match")
    _check((cos.shape[0] == 1 or cos.shape[0] == query.shape[0]) and cos.shape[1] == query.shape[2]
           and cos.shape[2] == query.shape[3], f"{op}: cos and sin shapes are not broadcastable to query and key")
    _grad_free(op, query, key, cos, sin)


def _rope_cuda(query, key, cos, sin):
    _validate_rope(query, key, cos, sin)
    _require_gpu("flux::rope", query)
    _check(all(s >= 0 for t in (query, key, cos, sin) for s in t.stride()),
           "flux::rope: negative tensor strides are unsupported")
    query_out = torch.empty(query.shape, dtype=torch.float32, device=query.device)
    key_out = torch.empty(key.shape, dtype=torch.float32, device=key.device)
    batch, query_heads, seq, dim = (int(s) for s in query.shape)
    with torch.cuda.device(query.device):
        _call("flux_rope_f32", query.data_ptr(), key.data_ptr(), cos.data_ptr(), sin.data_ptr(), query_out.data_ptr(),
              key_out.data_ptr(), batch, query_heads, int(key.shape[1]), seq, dim, int(cos.shape[0]),
              _strides(query, 4), _strides(key, 4), _strides(cos, 3), _strides(sin, 3), _stream(query))
    return query_out, key_out


# ---------------------------------------------------------------------------
# softmax (csrc/softmax/softmax_torch.cpp:14-85).

def _validate_softmax(input) -> None:
    op = "flux::softmax"
    _check(input.dim() >= 1, f"{op}: input must have at least one dimension")
    _check(input.shape[-1] > 0, f"{op}: input must have a non-empty final dimension")
    _check(input.numel() > 0, f"{op}: input must contain at least one row")
    _check(input.dtype == torch.float32, f"{op}: input must have dtype torch.float32")
    _grad_free(op, input)


def _softmax_cuda(input):
    _validate_softmax(input)
    _require_gpu("flux::softmax", input)
    x = input.contiguous()
    output = torch.empty_like(x)
    width = int(x.shape[-1])
    with torch.cuda.device(x.device):
        _call("flux_softmax_f32", x.data_ptr(), output.data_ptr(), x.numel() // width, width, _stream(x))
    return output


# ---------------------------------------------------------------------------
# attention_score_softmax (csrc/attention_score_softmax/attention_score_softmax_torch.cpp:15-117).

def _validate_attention_score_softmax(scores, mask, scale) -> None:
    op = "flux::attention_score_softmax"
    _check(scores.dim() == 4, f"{op}: scores must be rank four")
    _check(mask.dim() == 4, f"{op}: additive_attention_mask must be rank four")
    _check(scores.numel() > 0, f"{op}: scores dimensions must be non-empty")
    _check(scores.dtype == torch.float32, f"{op}: scores must have dtype torch.float32")
    _check(mask.dtype == torch.float32, f"{op}: additive_attention_mask must have dtype torch.float32")
    _check(scores.device == mask.device, f"{op}: tensor devices must match")
    _check(all(m == 1 or m == s for m, s in zip(mask.shape, scores.shape)),
           f"{op}: additive_attention_mask is not broadcastable to scores")
    _check(_finite_fp32(scale), f"{op}: scale must be a finite FP32 value")
    _grad_free(op, scores, mask)


def _attention_score_softmax_cuda(scores, additive_attention_mask, scale):
    _validate_attention_score_softmax(scores, additive_attention_mask, scale)
    _require_gpu("flux::attention_score_softmax", scores)
    mask = additive_attention_mask
    _check(all(s >= 0 for s in mask.stride()), "flux::attention_score_softmax: negative mask strides are unsupported")
    s = scores.contiguous()
    output = torch.empty_like(s)
    with torch.cuda.device(s.device):
        _call("flux_attention_score_softmax_f32", s.data_ptr(), mask.data_ptr(), output.data_ptr(), float(scale),
              *(int(d) for d in s.shape), _native.length_array([int(d) for d in mask.shape]), _strides(mask, 4),
              _stream(s))
    return output


# ---------------------------------------------------------------------------
# packed_swiglu / _out (csrc/packed_swiglu/packed_swiglu_torch.cpp:15-128).

def _validate_packed_swiglu(packed) -> None:
    op = "flux::packed_swiglu"
    _check(packed.dim() >= 1, f"{op}: packed must have at least one dimension")
    _check(packed.shape[-1] > 0, f"{op}: packed final dimension must be non-empty")
    _check(packed.shape[-1] % 2 == 0, f"{op}: packed final dimension must be even")
    _check(packed.numel() > 0, f"{op}: packed must contain at least one row")
    _check(packed.dtype == torch.float32, f"{op}: packed must have dtype torch.float32")
    _check(packed.is_contiguous(), f"{op}: packed must be contiguous; no implicit copy is performed")
    _grad_free(op, packed)


def _packed_swiglu_shape(packed) -> list:
    return [*packed.shape[:-1], packed.shape[-1] // 2]


def _launch_packed_swiglu(packed, output) -> None:
    inter = int(packed.shape[-1]) // 2
    with torch.cuda.device(packed.device):
        _call("flux_packed_swiglu_f32", packed.data_ptr(), output.data_ptr(), packed.numel() // (2 * inter), inter,
              _stream(packed))


def _packed_swiglu_cuda(packed):
    _validate_packed_swiglu(packed)
    _require_gpu("flux::packed_swiglu", packed)
    output = torch.empty(_packed_swiglu_shape(packed), dtype=torch.float32, device=packed.device)
    _launch_packed_swiglu(packed, output)
    return output


def _packed_swiglu_out_cuda(packed, output):
    _validate_packed_swiglu(packed)
    op = "flux::packed_swiglu_out"
    _require_gpu(op, packed)
    _check(list(output.shape) == _packed_swiglu_shape(packed), f"{op}: output shape is incorrect")
    _check(output.dtype == torch.float32 and output.device == packed.device and output.is_contiguous(),
           f"{op}: output must be contiguous float32 on the input device")
    _check(not _aliases(output, packed), f"{op}: output must not alias packed")
    _launch_packed_swiglu(packed, output)
    return output


# ---------------------------------------------------------------------------
# gqa_decode_attention / _out (csrc/gqa_decode_attention/gqa_decode_attention_torch.cpp:22-334).

def _validate_gqa(query, key_cache, value_cache, mask, scale, cache_length) -> None:
    op = "flux::gqa_decode_attention"
    _check(query.dim() == 4 and key_cache.dim() == 4 and value_cache.dim() == 4,
           f"{op}: Q/K/V tensors must be rank four")
    _check(query.shape[2] == 1, f"{op}: query length must be one")
    _check(query.shape[0] == 1, f"{op}: batch size must be one")
    _check(all(t.dtype == torch.float32 for t in (query, key_cache, value_cache)),
           f"{op}: Q/K/V tensors must have dtype torch.float32")
    _check(query.device == key_cache.device and query.device == value_cache.device,
           f"{op}: Q/K/V tensor devices must match")
    _check(key_cache.shape == value_cache.shape, f"{op}: key/value cache shapes must match")
    _check(query.shape[1] > 0 and query.shape[3] > 0 and key_cache.shape[1] > 0 and key_cache.shape[2] > 0,
           f"{op}: tensor dimensions must be non-empty")
    _check(query.shape[0] == key_cache.shape[0], f"{op}: cache batch must match query")
    _check(query.shape[3] == key_cache.shape[3], f"{op}: cache head dimension must match query")
    _check(query.shape[1] % key_cache.shape[1] == 0, f"{op}: query heads must be divisible by KV heads")
    _check(_finite_fp32(scale), f"{op}: scale must be a finite FP32 value")
    if mask is not None:
        _check(mask.dim() == 4, f"{op}: additive_attention_mask must be rank four")
        _check(mask.dtype == torch.float32, f"{op}: additive_attention_mask must be float32")
        _check(mask.device == query.device, f"{op}: mask device must match query")
        target = (query.shape[0], query.shape[1], 1, key_cache.shape[2])
        _check(all(m == 1 or m == t for m, t in zip(mask.shape, target)), f"{op}: mask is not broadcastable")
    if cache_length is not None:
        _check(cache_length.numel() == 1 and cache_length.dtype == torch.int64,
               f"{op}: cache_length must be a scalar int64 tensor")
        _check(cache_length.device == query.device, f"{op}: cache_length device must match query")
        _check(not cache_length.requires_grad, f"{op}: cache_length must not require gradients")
    _grad_free(op, query, key_cache, value_cache, mask)


def _launch_gqa(op, query, key_cache, value_cache, mask, scale, cache_length, output, workspace, workspace_bytes):
    tensors = [query, key_cache, value_cache] + ([mask] if mask is not None else [])
    _check(all(s >= 0 for t in tensors for s in t.stride()), f"{op}: negative tensor strides are unsupported")
    _check(key_cache.shape[2] <= _MAX_CAPACITY, f"{op}: cache capacity exceeds {_MAX_CAPACITY} tokens")
    with torch.cuda.device(query.device):
        _call("flux_gqa_decode_attention_strided_f32", query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
              _native.ptr(mask), _native.ptr(cache_length), output.data_ptr(), _native.ptr(workspace),
              int(workspace_bytes), float(scale), int(query.shape[1]), int(key_cache.shape[1]),
              int(key_cache.shape[2]), int(query.shape[3]), _strides(query, 4), _strides(key_cache, 4),
              _strides(value_cache, 4),
              None if mask is None else _native.length_array([int(d) for d in mask.shape]),
              None if mask is None else _strides(mask, 4), _stream(query))


def gqa_decode_workspace_bytes(query_heads: int, capacity: int, head_dim: int) -> int:
    """Device workspace (bytes) flux::gqa_decode_attention needs for this shape (0 if none)."""
    value = ctypes.c_int64(0)
    _call("flux_gqa_decode_attention_strided_workspace_bytes", int(query_heads), int(capacity), int(head_dim),
          ctypes.byref(value))
    return int(value.value)


def _gqa_cuda(query, key_cache, value_cache, additive_attention_mask, scale, cache_length=None):
    _validate_gqa(query, key_cache, value_cache, additive_attention_mask, scale, cache_length)
    op = "flux::gqa_decode_attention"
    _require_gpu(op, query)
    _check(key_cache.shape[2] <= _MAX_CAPACITY, f"{op}: cache capacity exceeds {_MAX_CAPACITY} tokens")
    output = torch.empty(query.shape, dtype=torch.float32, device=query.device)
    needed = gqa_decode_workspace_bytes(query.shape[1], key_cache.shape[2], query.shape[3])
    workspace = torch.empty(needed // 4, dtype=torch.float32, device=query.device) if needed else None
    _launch_gqa(op, query, key_cache, value_cache, additive_attention_mask, scale, cache_length, output, workspace,
                needed)
    return output


def gqa_decode_out_workspace_shape(query: torch.Tensor, key_cache: torch.Tensor) -> tuple[int, int, int, int]:
    """Workspace shape gqa_decode_attention_out accepts: ``[B, Hq, ceil(capacity/128), D+2]``."""
    chunks = (int(key_cache.shape[2]) + _GQA_OUT_CHUNK - 1) // _GQA_OUT_CHUNK
    return int(query.shape[0]), int(query.shape[1]), chunks, int(query.shape[3]) + 2


def _gqa_out_cuda(query, key_cache, value_cache, additive_attention_mask, scale, cache_length, output, workspace):
    _validate_gqa(query, key_cache, value_cache, additive_attention_mask, scale, cache_length)
    op = "flux::gqa_decode_attention_out"
    _require_gpu(op, query)
    _check(key_cache.shape[2] <= _MAX_CAPACITY, f"{op}: cache capacity exceeds {_MAX_CAPACITY} tokens")
    _check(query.shape[3] == 64 and key_cache.shape[2] > 512,
           f"{op}: stable workspace path requires head_dim=64 and capacity > 512")
    _check(output.shape == query.shape, f"{op}: output shape must match query")
    _check(output.dtype == torch.float32 and output.device == query.device and output.is_contiguous(),
           f"{op}: output must be contiguous float32 on the query device")
    _check(tuple(workspace.shape) == gqa_decode_out_workspace_shape(query, key_cache),
           f"{op}: workspace shape is incorrect")
    _check(workspace.dtype == torch.float32 and workspace.device == query.device and workspace.is_contiguous(),
           f"{op}: workspace must be contiguous float32 on the query device")
    _check(not _aliases(output, workspace), f"{op}: output and workspace must not alias")
    for tensor in (query, key_cache, value_cache):
        _check(not _aliases(output, tensor) and not _aliases(workspace, tensor), f"{op}: outputs must not alias Q/K/V")
    if additive_attention_mask is not None:
        _check(not _aliases(output, additive_attention_mask) and not _aliases(workspace, additive_attention_mask),
               f"{op}: outputs must not alias the mask")
    if cache_length is not None:
        _check(not _aliases(output, cache_length) and not _aliases(workspace, cache_length),
               f"{op}: outputs must not alias cache_length")
    _launch_gqa(op, query, key_cache, value_cache, additive_attention_mask, scale, cache_length, output, workspace,
                workspace.numel() * 4)
    return output


# ---------------------------------------------------------------------------
# packed_qkv_rope_cache / _out (csrc/packed_qkv_rope_cache/packed_qkv_rope_cache_torch.cpp:20-170).

def _validate_packed_qkv(packed_qkv, cos, sin, key_cache, value_cache, cache_length) -> None:
    op = "flux::packed_qkv_rope_cache"
    _check(packed_qkv.dim() == 3 and tuple(packed_qkv.shape) == (1, 1, 960),
           f"{op}: packed_qkv must have shape [1, 1, 960]")
    _check(tuple(cos.shape) == (1, 1, 64) and sin.shape == cos.shape, f"{op}: cos and sin must have shape [1, 1, 64]")
    _check(key_cache.dim() == 4 and value_cache.dim() == 4 and key_cache.shape == value_cache.shape
           and key_cache.shape[0] == 1 and key_cache.shape[1] == 3 and key_cache.shape[2] > 0
           and key_cache.shape[3] == 64, f"{op}: K/V cache must have matching shape [1, 3, capacity, 64]")
    _check(cache_length.dim() == 0 and cache_length.numel() == 1 and cache_length.dtype == torch.int64,
           f"{op}: cache_length must be a scalar torch.int64 tensor")
    for tensor in (packed_qkv, cos, sin, key_cache, value_cache):
        _check(tensor.dtype == torch.float32, f"{op}: data tensors must have dtype torch.float32")
        _check(tensor.device == packed_qkv.device, f"{op}: all tensors must be on the same device")
    _check(cache_length.device == packed_qkv.device, f"{op}: all tensors must be on the same device")
    _check(all(s > 0 for s in packed_qkv.stride()), f"{op}: packed_qkv strides must be positive")
    _check(all(s > 0 for s in (*key_cache.stride(), *value_cache.stride())), f"{op}: cache strides must be positive")
    _check(not torch.is_grad_enabled() or not any(
        t.requires_grad for t in (packed_qkv, cos, sin, key_cache, value_cache, cache_length)),
        f"{op} is inference-only; use torch.no_grad() or torch.inference_mode()")


def _launch_packed_qkv(packed_qkv, cos, sin, key_cache, value_cache, cache_length, query_output) -> None:
    with torch.cuda.device(packed_qkv.device):
        _call("flux_packed_qkv_rope_cache_f32", packed_qkv.data_ptr(), cos.data_ptr(), sin.data_ptr(),
              key_cache.data_ptr(), value_cache.data_ptr(), cache_length.data_ptr(), cache_length.data_ptr(),
              query_output.data_ptr(), int(key_cache.shape[2]), int(packed_qkv.stride(2)), int(cos.stride(2)),
              int(sin.stride(2)), _strides(key_cache, 4), _strides(value_cache, 4), _stream(packed_qkv))


def _packed_qkv_cuda(packed_qkv, cos, sin, key_cache, value_cache, cache_length):
    _validate_packed_qkv(packed_qkv, cos, sin, key_cache, value_cache, cache_length)
    _require_gpu("flux::packed_qkv_rope_cache", packed_qkv)
    query_output = torch.empty((1, 9, 1, 64), dtype=torch.float32, device=packed_qkv.device)
    _launch_packed_qkv(packed_qkv, cos, sin, key_cache, value_cache, cache_length, query_output)
    return query_output


def _packed_qkv_out_cuda(packed_qkv, cos, sin, key_cache, value_cache, cache_length, query_output):
    _validate_packed_qkv(packed_qkv, cos, sin, key_cache, value_cache, cache_length)
    op = "flux::packed_qkv_rope_cache_out"
    _require_gpu(op, packed_qkv)
    _check(tuple(query_output.shape) == (1, 9, 1, 64), f"{op}: query_output must have shape [1, 9, 1, 64]")
    _check(query_output.dtype == torch.float32 and query_output.device == packed_qkv.device
           and query_output.is_contiguous(), f"{op}: query_output must be contiguous float32 on the input device")
    _check(not any(_aliases(query_output, t) for t in (packed_qkv, cos, sin, key_cache, value_cache, cache_length)),
           f"{op}: query_output must not alias an input")
    _launch_packed_qkv(packed_qkv, cos, sin, key_cache, value_cache, cache_length, query_output)
    return query_output


# ---------------------------------------------------------------------------
# packed_gate_up_swiglu_out (csrc/packed_gate_up_gemv/packed_gate_up_gemv_torch.cpp:12-72).

def _validate_gate_up(input, weight) -> None:
    op = "flux::packed_gate_up_gemv"
    _check(input.device == weight.device, f"{op}: input and weight must be CUDA tensors on the same device")
    _check(tuple(input.shape) == (1, 1, 576), f"{op}: input must have shape [1, 1, 576]")
    _check(tuple(weight.shape) == (3072, 576), f"{op}: weight must have shape [3072, 576]")
    _check(input.dtype == torch.float32 and weight.dtype == torch.float32,
           f"{op}: input and weight must have dtype torch.float32")
    _check(input.is_contiguous() and weight.is_contiguous(), f"{op}: input and weight must be contiguous")
    _check(not torch.is_grad_enabled() or (not input.requires_grad and not weight.requires_grad),
           f"{op} is inference-only; use torch.no_grad() or torch.inference_mode()")


def _validate_gate_up_output(input, output) -> None:
    op = "flux::packed_gate_up_gemv_out"
    _check(output.device == input.device, f"{op}: output must be CUDA on the input device")
    _check(tuple(output.shape) == (1, 1, 1536), f"{op}: output shape is incorrect")
    _check(output.dtype == torch.float32 and output.is_contiguous(), f"{op}: output must be contiguous float32")


def _gate_up_out_cuda(input, weight, output):
    _validate_gate_up(input, weight)
    _validate_gate_up_output(input, output)
    op = "flux::packed_gate_up_gemv_out"
    _require_gpu(op, input)
    _check(not _aliases(output, input) and not _aliases(output, weight), f"{op}: output must not alias an input")
    with torch.cuda.device(input.device):
        _call("flux_gate_up_swiglu_f32", input.data_ptr(), None, 0.0, weight.data_ptr(), output.data_ptr(),
              _stream(input))
    return output


# ---------------------------------------------------------------------------
# Dispatcher registration: CUDA (ROCm) kernels, CPU argument checks, fakes.

def _cpu_kernel(name: str, validate):
    op = f"flux::{name}"

    def kernel(*args):
        validate(*args)
        _cpu_unsupported(op)

    return kernel


def _gqa_cpu_validate(query, key_cache, value_cache, mask, scale, cache_length=None, *outputs):
    _validate_gqa(query, key_cache, value_cache, mask, scale, cache_length)
    if cache_length is not None and cache_length.device.type == "cpu":
        length = int(cache_length.reshape(()).item())
        _check(1 <= length <= int(key_cache.shape[2]),
               "flux::gqa_decode_attention: cache_length must be within cache capacity")


_CUDA_KERNELS = {
    "rmsnorm": _rmsnorm_cuda,
    "rmsnorm_out": _rmsnorm_out_cuda,
    "residual_rmsnorm": _residual_rmsnorm_cuda,
    "residual_rmsnorm_out": _residual_rmsnorm_out_cuda,
    "rope": _rope_cuda,
    "softmax": _softmax_cuda,
    "attention_score_softmax": _attention_score_softmax_cuda,
    "packed_swiglu": _packed_swiglu_cuda,
    "packed_swiglu_out": _packed_swiglu_out_cuda,
    "gqa_decode_attention": _gqa_cuda,
    "gqa_decode_attention_out": _gqa_out_cuda,
    "packed_qkv_rope_cache": _packed_qkv_cuda,
    "packed_qkv_rope_cache_out": _packed_qkv_out_cuda,
    "packed_gate_up_swiglu_out": _gate_up_out_cuda,
}

_CPU_VALIDATORS = {
    "rmsnorm": _validate_rmsnorm,
    "rmsnorm_out": _validate_rmsnorm_out,
    "residual_rmsnorm": _validate_residual_rmsnorm,
    "residual_rmsnorm_out": lambda h, r, w, e, *_: _validate_residual_rmsnorm(h, r, w, e),
    "rope": _validate_rope,
    "softmax": _validate_softmax,
    "attention_score_softmax": _validate_attention_score_softmax,
    "packed_swiglu": _validate_packed_swiglu,
    "packed_swiglu_out": lambda p, *_: _validate_packed_swiglu(p),
    "gqa_decode_attention": _gqa_cpu_validate,
    "gqa_decode_attention_out": _gqa_cpu_validate,
    "packed_qkv_rope_cache": _validate_packed_qkv,
    "packed_qkv_rope_cache_out": lambda *a: _validate_packed_qkv(*a[:6]),
    "packed_gate_up_swiglu_out": lambda i, w, o: (_validate_gate_up(i, w), _validate_gate_up_output(i, o)),
}

for _name, _kernel in _CUDA_KERNELS.items():
    _LIBRARY.impl(_name, _kernel, "CUDA")
    _LIBRARY.impl(_name, _cpu_kernel(_name, _CPU_VALIDATORS[_name]), "CPU")


def _empty_contiguous(t: torch.Tensor) -> torch.Tensor:
    return torch.empty_like(t, memory_format=torch.contiguous_format)


@torch.library.register_fake("flux::rmsnorm")
def _rmsnorm_fake(input, weight, epsilon):
    _validate_rmsnorm(input, weight, epsilon)
    return _empty_contiguous(input)


@torch.library.register_fake("flux::rmsnorm_out")
def _rmsnorm_out_fake(input, weight, epsilon, output):
    _validate_rmsnorm_out(input, weight, epsilon, output)
    return output


@torch.library.register_fake("flux::residual_rmsnorm")
def _residual_rmsnorm_fake(hidden, residual, weight, epsilon):
    _validate_residual_rmsnorm(hidden, residual, weight, epsilon)
    return _empty_contiguous(hidden), _empty_contiguous(hidden)


@torch.library.register_fake("flux::residual_rmsnorm_out")
def _residual_rmsnorm_out_fake(hidden, residual, weight, epsilon, norm_out, residual_out):
    _validate_residual_rmsnorm(hidden, residual, weight, epsilon)
    return norm_out, residual_out


@torch.library.register_fake("flux::rope")
def _rope_fake(query, key, cos, sin):
    _validate_rope(query, key, cos, sin)
    return _empty_contiguous(query), _empty_contiguous(key)


@torch.library.register_fake("flux::softmax")
def _softmax_fake(input):
    _validate_softmax(input)
    return _empty_contiguous(input)


@torch.library.register_fake("flux::attention_score_softmax")
def _attention_score_softmax_fake(scores, additive_attention_mask, scale):
    _validate_attention_score_softmax(scores, additive_attention_mask, scale)
    return _empty_contiguous(scores)


@torch.library.register_fake("flux::packed_swiglu")
def _packed_swiglu_fake(packed):
    _validate_packed_swiglu(packed)
    return packed.new_empty(_packed_swiglu_shape(packed))


@torch.library.register_fake("flux::packed_swiglu_out")
def _packed_swiglu_out_fake(packed, output):
    _validate_packed_swiglu(packed)
    return output


@torch.library.register_fake("flux::gqa_decode_attention")
def _gqa_fake(query, key_cache, value_cache, additive_attention_mask, scale, cache_length=None):
    _validate_gqa(query, key_cache, value_cache, additive_attention_mask, scale, cache_length)
    return _empty_contiguous(query)


@torch.library.register_fake("flux::gqa_decode_attention_out")
def _gqa_out_fake(query, key_cache, value_cache, additive_attention_mask, scale, cache_length, output, workspace):
    _validate_gqa(query, key_cache, value_cache, additive_attention_mask, scale, cache_length)
    return output


@torch.library.register_fake("flux::packed_qkv_rope_cache")
def _packed_qkv_fake(packed_qkv, cos, sin, key_cache, value_cache, cache_length):
    _validate_packed_qkv(packed_qkv, cos, sin, key_cache, value_cache, cache_length)
    return packed_qkv.new_empty((1, 9, 1, 64))


@torch.library.register_fake("flux::packed_qkv_rope_cache_out")
def _packed_qkv_out_fake(packed_qkv, cos, sin, key_cache, value_cache, cache_length, query_output):
    _validate_packed_qkv(packed_qkv, cos, sin, key_cache, value_cache, cache_length)
    return query_output


@torch.library.register_fake("flux::packed_gate_up_swiglu_out")
def _gate_up_out_fake(input, weight, output):
    _validate_gate_up(input, weight)
    _validate_gate_up_output(input, output)
    return output


# ---------------------------------------------------------------------------
# Python entry points (flux/ops/native_*.py).

def _load_error() -> OSError | None:
    try:
        _native.load()
    except (RuntimeError, OSError) as error:
        return error if isinstance(error, OSError) else OSError(str(error))
    return None


def _require_library(what: str) -> None:
    error = _load_error()
    if error is not None:
        raise RuntimeError(f"Flux native {what} is not built. Build it with `python -m flux_amd.build` "
                           "(hipcc, gfx950).") from error


def _availability(*names: str) -> bool:
    return _load_error() is None and all(hasattr(torch.ops.flux, n) for n in names)


def native_rmsnorm_is_available() -> bool:
    """Whether ``flux::rmsnorm`` has its HIP kernel (``libflux_amd.so`` loads)."""
    return _availability("rmsnorm", "rmsnorm_out")


def native_residual_rmsnorm_is_available() -> bool:
    return _availability("residual_rmsnorm", "residual_rmsnorm_out")


def native_rope_is_available() -> bool:
    return _availability("rope")


def native_softmax_is_available() -> bool:
    return _availability("softmax")


def native_attention_score_softmax_is_available() -> bool:
    return _availability("attention_score_softmax")


def native_packed_swiglu_is_available() -> bool:
    return _availability("packed_swiglu", "packed_swiglu_out")


def native_gqa_decode_attention_is_available() -> bool:
    return _availability("gqa_decode_attention", "gqa_decode_attention_out")


def native_packed_qkv_rope_cache_is_available() -> bool:
    return _availability("packed_qkv_rope_cache", "packed_qkv_rope_cache_out")


def native_packed_gate_up_gemv_is_available() -> bool:
    return _availability("packed_gate_up_swiglu_out")


def native_rmsnorm_load_error() -> OSError | None:
    """The error that kept the native library from loading, if any."""
    return _load_error()


native_rope_load_error = native_rmsnorm_load_error
native_softmax_load_error = native_rmsnorm_load_error
native_packed_qkv_rope_cache_load_error = native_rmsnorm_load_error


def rms_norm_native(input: torch.Tensor, weight: torch.Tensor, epsilon: float) -> torch.Tensor:
    """Inference-only FP32 RMSNorm; non-contiguous input/weight are copied contiguous first."""
    _require_library("RMSNorm")
    return torch.ops.flux.rmsnorm(input, weight, epsilon)


def rms_norm_native_out(input: torch.Tensor, weight: torch.Tensor, epsilon: float,
                        output: torch.Tensor) -> torch.Tensor:
    """RMSNorm into a validated contiguous output; returns ``output``."""
    _require_library("RMSNorm out variant")
    return torch.ops.flux.rmsnorm_out(input, weight, epsilon, output)


def residual_rmsnorm_native(hidden: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                            epsilon: float) -> tuple[torch.Tensor, torch.Tensor]:
    """``(rmsnorm(hidden + residual), hidden + residual)`` as two new contiguous tensors."""
    _require_library("residual RMSNorm")
    return torch.ops.flux.residual_rmsnorm(hidden, residual, weight, epsilon)


def residual_rmsnorm_native_out(hidden: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, epsilon: float,
                                norm_out: torch.Tensor, residual_out: torch.Tensor
                                ) -> tuple[torch.Tensor, torch.Tensor]:
    _require_library("residual RMSNorm out variant")
    return torch.ops.flux.residual_rmsnorm_out(hidden, residual, weight, epsilon, norm_out, residual_out)


def rope_native(query: torch.Tensor, key: torch.Tensor, cos: torch.Tensor,
                sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Hugging Face ``apply_rotary_pos_emb`` for [B, H, S, D] query/key, contiguous outputs."""
    _require_library("RoPE")
    return torch.ops.flux.rope(query, key, cos, sin)


def softmax_native(input: torch.Tensor) -> torch.Tensor:
    """FP32 softmax over the final dimension."""
    _require_library("softmax")
    return torch.ops.flux.softmax(input)


def attention_score_softmax_native(scores: torch.Tensor, additive_attention_mask: torch.Tensor,
                                   scale: float) -> torch.Tensor:
    """``softmax(scores * scale + additive_attention_mask)`` over [B, H, Q, K] with a broadcast mask."""
    _require_library("attention score softmax")
    return torch.ops.flux.attention_score_softmax(scores, additive_attention_mask, scale)


def packed_swiglu_native(packed: torch.Tensor) -> torch.Tensor:
    """``silu(packed[..., :I]) * packed[..., I:]`` for contiguous packed [..., 2I]."""
    _require_library("packed SwiGLU")
    return torch.ops.flux.packed_swiglu(packed)


def packed_swiglu_native_out(packed: torch.Tensor, output: torch.Tensor) -> torch.Tensor:
    _require_library("packed SwiGLU out variant")
    return torch.ops.flux.packed_swiglu_out(packed, output)


def gqa_decode_attention_native(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                                additive_attention_mask: torch.Tensor | None, scale: float,
                                cache_length: torch.Tensor | None = None) -> torch.Tensor:
    """One-token GQA attention directly over the unexpanded FP32 K/V cache."""
    _require_library("GQA decode attention")
    return torch.ops.flux.gqa_decode_attention(query, key_cache, value_cache, additive_attention_mask, scale,
                                               cache_length)


def gqa_decode_attention_native_out(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                                    additive_attention_mask: torch.Tensor | None, scale: float,
                                    cache_length: torch.Tensor | None, output: torch.Tensor,
                                    workspace: torch.Tensor) -> torch.Tensor:
    """One-token GQA attention into stable buffers (workspace ``[1, Hq, ceil(capacity/128), D+2]``)."""
    _require_library("GQA decode attention out variant")
    return torch.ops.flux.gqa_decode_attention_out(query, key_cache, value_cache, additive_attention_mask, scale,
                                                   cache_length, output, workspace)


def packed_qkv_rope_cache_native(packed_qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                                 key_cache: torch.Tensor, value_cache: torch.Tensor,
                                 cache_length: torch.Tensor) -> torch.Tensor:
    """Rotate Q/K of one packed token, append K/V at ``cache_length``, advance it; returns Q [1, 9, 1, 64]."""
    _require_library("packed QKV/RoPE/cache")
    return torch.ops.flux.packed_qkv_rope_cache(packed_qkv, cos, sin, key_cache, value_cache, cache_length)


def packed_qkv_rope_cache_native_out(packed_qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                                     key_cache: torch.Tensor, value_cache: torch.Tensor, cache_length: torch.Tensor,
                                     query_output: torch.Tensor) -> torch.Tensor:
    _require_library("packed QKV/RoPE/cache out variant")
    return torch.ops.flux.packed_qkv_rope_cache_out(packed_qkv, cos, sin, key_cache, value_cache, cache_length,
                                                    query_output)


def packed_gate_up_swiglu_native_out(input: torch.Tensor, weight: torch.Tensor, output: torch.Tensor) -> torch.Tensor:
    """Decode gate/up GEMV with the SwiGLU epilogue: ``silu(Wg x) * (Wu x)`` into output [1, 1, 1536]."""
    _require_library("fused packed gate/up SwiGLU")
    return torch.ops.flux.packed_gate_up_swiglu_out(input, weight, output)


def decode_projection_out(input: torch.Tensor, weight: torch.Tensor, output: torch.Tensor) -> torch.Tensor:
    """One-token projection ``output[1, 1, N] = weight[N, 576] @ input[1, 1, 576]`` on the decode GEMV kernel.

    The counterpart of the reference's exact-shape cuBLASLt decode projections
    (``flux/model/smollm2_flux.py:86-116``): used for the [960, 576] and
    [576, 576] weights when decode scratch buffers are installed.
    """
    _require_library("decode projection")
    op = "flux::decode_projection_out"
    _check(input.is_cuda and input.device == weight.device == output.device, f"{op}: tensors must share a GPU")
    _check(tuple(input.shape) == (1, 1, 576) and input.is_contiguous(), f"{op}: input must be contiguous [1, 1, 576]")
    _check(weight.dim() == 2 and weight.shape[1] == 576 and weight.is_contiguous(),
           f"{op}: weight must be contiguous [N, 576]")
    _check(tuple(output.shape) == (1, 1, weight.shape[0]) and output.is_contiguous(),
           f"{op}: output must be contiguous [1, 1, N]")
    _check(all(t.dtype == torch.float32 for t in (input, weight, output)), f"{op}: tensors must be float32")
    _grad_free(op, input, weight)
    with torch.cuda.device(input.device):
        _call("flux_linear576_f32", input.data_ptr(), weight.data_ptr(), None, output.data_ptr(),
              int(weight.shape[0]), _stream(input))
    return output


OPERATOR_NAMES: Sequence[str] = tuple(SCHEMAS)
