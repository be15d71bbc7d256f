"""ctypes binding of ``libflux_amd.so`` (C ABI: ``include/flux_amd.h``).

This is the Python side a maintainer binds the boundary with; it replaces the
reference's ``torch.ops.load_library(flux/_C*.so)`` loader
(``flux/ops/native_rmsnorm.py:149-163``) and its TORCH_LIBRARY custom classes.
PyTorch is used only for device memory and the current stream.  There is no
fallback: when the library is missing every native entry point raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Any, Sequence

import torch

LAYERS = 30
HIDDEN = 576
_PACKAGE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.environ.get("FLUX_AMD_LIBRARY", os.path.join(_PACKAGE, "lib", "libflux_amd.so"))

FLUX_OK = 0
FLUX_ERROR_INVALID_VALUE = 1
FLUX_ERROR_HIP = 2
FLUX_ERROR_STATE = 3
FLUX_ERROR_DEVICE = 4

_f = ctypes.POINTER(ctypes.c_float)
_i64 = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p
_stream = ctypes.c_void_p


class FluxWeights(ctypes.Structure):
    _fields_ = [
        ("embedding", _vp),
        ("lm_head", _vp),
        ("final_norm", _vp),
        ("input_norm", _vp * LAYERS),
        ("packed_qkv", _vp * LAYERS),
        ("o_proj", _vp * LAYERS),
        ("post_norm", _vp * LAYERS),
        ("gate_up", _vp * LAYERS),
        ("down", _vp * LAYERS),
        ("vocab_size", ctypes.c_int64),
    ]


class DecodeBuffers(ctypes.Structure):
    _fields_ = [
        ("input_token", _vp),
        ("logits", _vp),
        ("generated_tokens", _vp),
        ("generation_step", _vp),
        ("key_cache", _vp),
        ("value_cache", _vp),
        ("position", _vp),
        ("cache_length", _vp),
        ("workspace", _vp),
        ("hidden_a", _vp),
        ("hidden_b", _vp),
        ("final_norm_output", _vp),
        ("attention_workspace", _vp),
        ("capacity", ctypes.c_int64),
        ("vocab_size", ctypes.c_int64),
        ("workspace_bytes", ctypes.c_int64),
        ("cache_bytes", ctypes.c_int64),
        ("stable_buffer_bytes", ctypes.c_int64),
    ]


class PrefillBuffers(ctypes.Structure):
    _fields_ = [
        ("prefill_logits", _vp),
        ("prefill_workspace", _vp),
        ("attention_output", _vp),
        ("final_hidden", _vp),
        ("initial_token", _vp),
        ("sequence_length", ctypes.c_int64),
        ("capacity", ctypes.c_int64),
        ("workspace_bytes", ctypes.c_int64),
    ]


class LayerWeightsStruct(ctypes.Structure):
    _fields_ = [(name, _vp) for name in ("input_norm", "packed_qkv", "o_proj", "post_norm", "gate_up", "down")]


class LayerDecodeBuffers(ctypes.Structure):
    _fields_ = [
        ("input_hidden", _vp),
        ("output", _vp),
        ("key_cache", _vp),
        ("value_cache", _vp),
        ("position", _vp),
        ("workspace", _vp),
        ("query", _vp),
        ("attention", _vp),
        ("residual", _vp),
        ("swiglu", _vp),
        ("attention_partials", _vp),
        ("capacity", ctypes.c_int64),
        ("workspace_bytes", ctypes.c_int64),
    ]


# (name, restype, argtypes) for every exported symbol.
_PROTOTYPES: list[tuple[str, Any, list[Any]]] = [
    ("flux_last_error", ctypes.c_char_p, []),
    ("flux_version", ctypes.c_char_p, []),
    ("flux_decode_create", ctypes.c_int,
     [ctypes.POINTER(FluxWeights), _vp, _vp, ctypes.c_int64, ctypes.c_int64, _vp, ctypes.POINTER(_vp),
      ctypes.POINTER(_vp), _i64, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double), _stream,
      ctypes.POINTER(_vp)]),
    ("flux_decode_replay", ctypes.c_int, [_vp, _vp, _stream, ctypes.POINTER(_vp)]),
    ("flux_decode_generate_greedy", ctypes.c_int, [_vp, ctypes.c_int64, _stream, ctypes.POINTER(_vp)]),
    ("flux_decode_generate_greedy_timed", ctypes.c_int, [_vp, ctypes.c_int64, _stream, ctypes.POINTER(ctypes.c_float)]),
    ("flux_decode_reset", ctypes.c_int,
     [_vp, _vp, ctypes.POINTER(_vp), ctypes.POINTER(_vp), _i64, ctypes.c_int64, _stream]),
    ("flux_decode_position", ctypes.c_int, [_vp, _i64]),
    ("flux_decode_cache_length", ctypes.c_int, [_vp, _i64]),
    ("flux_decode_generation_step", ctypes.c_int, [_vp, _i64]),
    ("flux_decode_replay_count", ctypes.c_int, [_vp, _i64]),
    ("flux_decode_capacity", ctypes.c_int, [_vp, _i64]),
    ("flux_decode_get_buffers", ctypes.c_int, [_vp, ctypes.POINTER(DecodeBuffers)]),
    ("flux_decode_device_error", ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_int32)]),
    ("flux_decode_set_wait_limit", ctypes.c_int, [_vp, ctypes.c_uint64]),
    ("flux_decode_replay_launches", ctypes.c_int, [_vp, _i64, _i64]),
    ("flux_host_counters", ctypes.c_int, [_i64, _i64, _i64]),
    ("flux_decode_destroy", None, [_vp]),
    ("flux_prefill_create", ctypes.c_int,
     [ctypes.POINTER(FluxWeights), _vp, _vp, ctypes.c_int64, _vp, ctypes.c_int64, ctypes.POINTER(ctypes.c_double),
      ctypes.POINTER(ctypes.c_double), _stream, ctypes.POINTER(_vp)]),
    ("flux_prefill_run", ctypes.c_int, [_vp, _vp, _stream, ctypes.POINTER(_vp)]),
    ("flux_prefill_generate_greedy", ctypes.c_int, [_vp, ctypes.c_int64, _stream, ctypes.POINTER(_vp)]),
    ("flux_prefill_decode", _vp, [_vp]),
    ("flux_prefill_get_buffers", ctypes.c_int, [_vp, ctypes.POINTER(PrefillBuffers)]),
    ("flux_prefill_destroy", None, [_vp]),
    ("flux_layer_decode_create", ctypes.c_int,
     [ctypes.POINTER(LayerWeightsStruct), _vp, _vp, ctypes.c_int64, ctypes.c_int64, _vp, _vp, _vp, ctypes.c_int64,
      ctypes.c_double, ctypes.c_double, _stream, ctypes.POINTER(_vp)]),
    ("flux_layer_decode_replay", ctypes.c_int, [_vp, _vp, _stream, ctypes.POINTER(_vp)]),
    ("flux_layer_decode_reset", ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64, _stream]),
    ("flux_layer_decode_position", ctypes.c_int, [_vp, _i64]),
    ("flux_layer_decode_replay_count", ctypes.c_int, [_vp, _i64]),
    ("flux_layer_decode_capacity", ctypes.c_int, [_vp, _i64]),
    ("flux_layer_decode_get_buffers", ctypes.c_int, [_vp, ctypes.POINTER(LayerDecodeBuffers)]),
    ("flux_layer_decode_replay_launches", ctypes.c_int, [_vp, _i64, _i64]),
    ("flux_layer_decode_destroy", None, [_vp]),
    ("flux_rmsnorm_f32", ctypes.c_int, [_vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_float, _stream]),
    ("flux_residual_rmsnorm_f32", ctypes.c_int,
     [_vp, _vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_float, _stream]),
    ("flux_qkv_rope_cache_f32", ctypes.c_int,
     [_vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp, ctypes.c_int64, _vp, _vp, _vp, _stream]),
    ("flux_gqa_decode_workspace_bytes", ctypes.c_int, [ctypes.c_int64, _i64]),
    ("flux_gqa_decode_attention_f32", ctypes.c_int,
     [_vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_float, _vp, ctypes.c_int64, _vp, _stream]),
    ("flux_gqa_decode_attention_noalloc_f32", ctypes.c_int,
     [_vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_float, _vp, _stream]),
    ("flux_linear576_f32", ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.c_int64, _stream]),
    ("flux_gate_up_swiglu_f32", ctypes.c_int, [_vp, _vp, ctypes.c_float, _vp, _vp, _stream]),
    ("flux_down_residual_f32", ctypes.c_int, [_vp, _vp, _vp, _vp, _stream]),
    ("flux_lm_head_workspace_bytes", ctypes.c_int, [_i64]),
    ("flux_lm_head_argmax_f32", ctypes.c_int,
     [_vp, _vp, ctypes.c_float, _vp, ctypes.c_int64, _vp, _vp, _vp, ctypes.c_int64, _stream]),
    ("flux_greedy_argmax_f32", ctypes.c_int, [_vp, ctypes.c_int64, _vp, _stream]),
    ("flux_greedy_argmax_update_f32", ctypes.c_int,
     [_vp, ctypes.c_int64, _vp, _vp, _vp, ctypes.c_int64, _vp, _vp, _stream]),
    ("flux_linear_f32", ctypes.c_int,
     [_vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _stream]),
    ("flux_gate_up_swiglu_rows_f32", ctypes.c_int, [_vp, _vp, _vp, ctypes.c_int64, _stream]),
    ("flux_qkv_rope_cache_rows_f32", ctypes.c_int,
     [_vp, _vp, _vp, _vp, ctypes.c_int64, _vp, _vp, _vp, ctypes.c_int64, _stream]),
    ("flux_prefill_attention_workspace_bytes", ctypes.c_int, [ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]),
    ("flux_prefill_attention_f32", ctypes.c_int,
     [_vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_float, _vp, _vp, _stream]),
    ("flux_embedding_gather_f32", ctypes.c_int, [_vp, _vp, ctypes.c_int64, ctypes.c_int64, _vp, _stream]),
    ("flux_rope_f32", ctypes.c_int,
     [_vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
      ctypes.c_int64, _i64, _i64, _i64, _i64, _stream]),
    ("flux_softmax_f32", ctypes.c_int, [_vp, _vp, ctypes.c_int64, ctypes.c_int64, _stream]),
    ("flux_attention_score_softmax_f32", ctypes.c_int,
     [_vp, _vp, _vp, ctypes.c_float, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _i64, _i64,
      _stream]),
    ("flux_packed_swiglu_f32", ctypes.c_int, [_vp, _vp, ctypes.c_int64, ctypes.c_int64, _stream]),
    ("flux_packed_qkv_rope_cache_f32", ctypes.c_int,
     [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _i64,
      _i64, _stream]),
    ("flux_gqa_decode_attention_strided_workspace_bytes", ctypes.c_int,
     [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _i64]),
    ("flux_gqa_decode_attention_strided_f32", ctypes.c_int,
     [_vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_float, ctypes.c_int64, ctypes.c_int64,
      ctypes.c_int64, ctypes.c_int64, _i64, _i64, _i64, _i64, _i64, _stream]),
]

EXPORTED_SYMBOLS = tuple(name for name, _, _ in _PROTOTYPES)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_load_error: str | None = None


class NativeError(RuntimeError):
    """A C-ABI call failed; ``code`` is the flux_status value."""

    def __init__(self, code: int, message: str) -> None:
        super().__init__(message)
        self.code = code


def load(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and return the native library; raise if it is not built."""
    global _lib, _load_error
    with _lock:
        if _lib is not None:
            return _lib
        library = path or LIBRARY_PATH
        if not os.path.exists(library):
            _load_error = f"{library} does not exist"
            raise RuntimeError(
                "flux_amd native library is not built (" + _load_error + "). "
                "Run `python -m flux_amd.build` (hipcc, gfx950) first."
            )
        lib = ctypes.CDLL(library)
        for name, restype, argtypes in _PROTOTYPES:
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def is_available() -> bool:
    try:
        load()
        return True
    except (RuntimeError, OSError):
        return False


def last_error() -> str:
    message = load().flux_last_error()
    return message.decode() if message else ""


def check(status: int) -> None:
    if status != FLUX_OK:
        raise NativeError(status, last_error() or f"flux native call failed with status {status}")


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else int(tensor.data_ptr())


def current_stream(device: torch.device | None = None) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


class _DeviceArray:
    """Exposes runtime-owned device memory to torch without a copy; holds the owner."""

    _typestr = {torch.float32: "<f4", torch.int64: "<i8", torch.int32: "<i4", torch.uint64: "<u8"}

    def __init__(self, address: int, shape: Sequence[int], dtype: torch.dtype, owner: Any) -> None:
        self.owner = owner
        self.__cuda_array_interface__ = {
            "shape": tuple(int(s) for s in shape),
            "typestr": self._typestr[dtype],
            "data": (int(address), False),
            "version": 2,
            "strides": None,
        }


def device_tensor(address: int, shape: Sequence[int], dtype: torch.dtype, owner: Any,
                  device: torch.device) -> torch.Tensor:
    """A torch view of runtime-owned memory; the view keeps ``owner`` alive."""
    tensor = torch.as_tensor(_DeviceArray(address, shape, dtype, owner), device=device)
    if int(tensor.data_ptr()) != int(address):
        raise RuntimeError("flux_amd: torch copied runtime-owned memory instead of viewing it")
    return tensor


def weights_struct(embedding: torch.Tensor, lm_head: torch.Tensor, final_norm: torch.Tensor,
                   input_norms: Sequence[torch.Tensor], packed_qkv: Sequence[torch.Tensor],
                   o_proj: Sequence[torch.Tensor], post_norms: Sequence[torch.Tensor],
                   gate_up: Sequence[torch.Tensor], down: Sequence[torch.Tensor]) -> FluxWeights:
    w = FluxWeights()
    w.embedding = ptr(embedding)
    w.lm_head = ptr(lm_head)
    w.final_norm = ptr(final_norm)
    for i in range(LAYERS):
        w.input_norm[i] = ptr(input_norms[i])
        w.packed_qkv[i] = ptr(packed_qkv[i])
        w.o_proj[i] = ptr(o_proj[i])
        w.post_norm[i] = ptr(post_norms[i])
        w.gate_up[i] = ptr(gate_up[i])
        w.down[i] = ptr(down[i])
    w.vocab_size = int(embedding.shape[0])
    return w


def double_array(values: Sequence[float]):
    return (ctypes.c_double * len(values))(*[float(v) for v in values])


def pointer_array(tensors: Sequence[torch.Tensor] | None):
    if tensors is None:
        return None
    return (_vp * len(tensors))(*[ptr(t) for t in tensors])


def length_array(values: Sequence[int] | None):
    if values is None:
        return None
    return (ctypes.c_int64 * len(values))(*[int(v) for v in values])
