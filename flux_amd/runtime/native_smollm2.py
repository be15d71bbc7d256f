"""Native MI355X SmolLM2 runtimes: prompt prefill, fused decode, greedy generation.

Drop-in for ``flux.runtime.native_smollm2`` (``/root/reference/flux/runtime/native_smollm2.py``):
same class names, constructors (``capture`` / ``capture_from_state``), methods,
properties, validation messages and error types.  Underneath, the reference's
TORCH_LIBRARY custom classes are replaced by the C ABI of ``libflux_amd.so``
(``include/flux_amd.h``) bound through ctypes; the runtime owns its device
buffers and the Python properties are zero-copy torch views of them.

Differences kept deliberately (each is a capability widening, not a change of
meaning): the cache capacity limit is 16384 instead of 8192 (the benchmark
configurations need 8320 and 8704 positions), and the RoPE tables are computed
once on the host CPU with the model's own ``inv_freq`` and HF's formula rather
than on the device.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any, Sequence

import torch
from torch import nn

from flux_amd import _native

MAX_CAPACITY = 16384

_ADDRESS_NAMES = (
    "input_token",
    "logits",
    "generated_tokens",
    "device_generation_step",
    "key_cache",
    "value_cache",
    "device_position",
    "device_cache_length",
    "workspace",
    "hidden_a",
    "hidden_b",
    "final_norm_output",
    "attention_workspace",
)

_PREFILL_ADDRESS_NAMES = (
    "prefill_logits",
    "prefill_workspace",
    "streaming_attention_output",
    "final_hidden",
) + _ADDRESS_NAMES


@dataclass(frozen=True)
class NativeDecodeRuntimeMemory:
    """Persistent memory attributable to the full native runtime."""

    cache_bytes: int
    workspace_bytes: int
    stable_buffer_bytes: int
    referenced_weight_bytes: int
    graph_resource_bytes: int | None = None

    @property
    def owned_tensor_bytes(self) -> int:
        return self.cache_bytes + self.workspace_bytes + self.stable_buffer_bytes


@dataclass(frozen=True)
class NativePrefillRuntimeMemory:
    """Persistent native prefill and directly attached decode storage."""

    cache_bytes: int
    prefill_workspace_bytes: int
    decode_workspace_bytes: int
    stable_buffer_bytes: int
    referenced_weight_bytes: int

    @property
    def owned_tensor_bytes(self) -> int:
        return self.cache_bytes + self.prefill_workspace_bytes + self.decode_workspace_bytes + self.stable_buffer_bytes


def native_smollm2_runtime_is_available() -> bool:
    """Whether the native decode runtime library loads."""
    return _native.is_available()


def native_smollm2_prefill_is_available() -> bool:
    """Whether the native prefill runtime library loads."""
    return _native.is_available()


def _rope_tables(model: nn.Module, length: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``[length, head_dim]`` cos/sin with HF's formula on the host CPU.

    ``LlamaRotaryEmbedding.forward`` (transformers modeling_llama.py:120-137):
    ``freqs = inv_freq x position``, ``emb = cat(freqs, freqs)``, ``cos/sin(emb) * scaling``.
    """
    rotary = model.model.rotary_emb
    inv_freq = rotary.inv_freq.detach().to("cpu", torch.float32)
    scaling = float(getattr(rotary, "attention_scaling", 1.0))
    positions = torch.arange(length, dtype=torch.long).unsqueeze(0)
    with torch.inference_mode():
        freqs = (inv_freq[None, :, None].expand(1, -1, 1) @ positions[:, None, :].float()).transpose(1, 2)
        emb = torch.cat((freqs, freqs), dim=-1)
        cos = (emb.cos() * scaling).reshape(length, -1).contiguous()
        sin = (emb.sin() * scaling).reshape(length, -1).contiguous()
    return cos, sin


def _model_weight_tensors(model: nn.Module, device: torch.device) -> list[torch.Tensor]:
    """Every weight the native runtimes read, each checked before its pointer crosses the C ABI.

    The kernels read raw device pointers, so a tensor on another device, of another
    dtype or shape, or with strides (a transposed or sliced view) would be read as
    garbage or fault the GPU.  The reference checks each tensor the same way
    (native_decode_runtime_cuda.cu:1108-1123, native_prefill_runtime_cuda.cu:460-482).
    Returns, in order: embedding, lm_head, final norm, then per layer the input norm,
    packed QKV, o_proj, post-attention norm, packed gate/up and down weights.
    """
    vocab = int(model.config.vocab_size)
    layers = list(model.model.layers)
    named = [("embedding", model.model.embed_tokens.weight, (vocab, 576)),
             ("lm_head", model.lm_head.weight, (vocab, 576)),
             ("final norm", model.model.norm.weight, (576,))]
    for i, layer in enumerate(layers):
        named += [(f"layer {i} input norm", layer.input_layernorm.weight, (576,)),
                  (f"layer {i} packed QKV", layer.self_attn.packed_qkv.weight, (960, 576)),
                  (f"layer {i} o_proj", layer.self_attn.o_proj.weight, (576, 576)),
                  (f"layer {i} post-attention norm", layer.post_attention_layernorm.weight, (576,)),
                  (f"layer {i} packed gate/up", layer.mlp.gate_up_proj.weight, (3072, 576)),
                  (f"layer {i} down", layer.mlp.down_proj.weight, (576, 1536))]
    for name, tensor, shape in named:
        if not isinstance(tensor, torch.Tensor):
            raise ValueError(f"native SmolLM2 runtime: {name} weight is missing")
        if tensor.device != device:
            raise ValueError(f"native SmolLM2 runtime: {name} weight is on {tensor.device}, expected {device}")
        if tensor.dtype != torch.float32:
            raise ValueError(f"native SmolLM2 runtime: {name} weight has dtype {tensor.dtype}, expected float32")
        if tuple(tensor.shape) != shape:
            raise ValueError(f"native SmolLM2 runtime: {name} weight has shape {list(tensor.shape)}, "
                             f"expected {list(shape)}")
        if not tensor.is_contiguous():
            raise ValueError(f"native SmolLM2 runtime: {name} weight must be contiguous")
    return [tensor.detach() for _, tensor, _ in named]


def _model_weights(model: nn.Module, device: torch.device
                   ) -> tuple[_native.FluxWeights, list[float], list[float], tuple[torch.Tensor, ...]]:
    """The C ABI weight struct, epsilons and attention scales, plus the tensors it borrows."""
    tensors = _model_weight_tensors(model, device)
    layers = list(model.model.layers)
    per_layer = [tensors[3 + k::6] for k in range(6)]
    weights = _native.weights_struct(tensors[0], tensors[1], tensors[2], *per_layer)
    epsilons = [float(layer.input_layernorm.variance_epsilon) for layer in layers]
    scales = [float(layer.self_attn.scaling) for layer in layers]
    return weights, epsilons, scales, tuple(tensors)


class _NativeAllocation:
    """Owns one native runtime object and destroys it when the last holder goes.

    Zero-copy tensor views of runtime buffers hold this object (torch keeps the
    view's ``__cuda_array_interface__`` owner alive from C++, which the garbage
    collector cannot traverse), and this object holds nothing that holds the
    views, so no reference cycle keeps device memory alive.  ``keepalive`` holds
    what the native object borrows (model weights, RoPE tables).
    """

    def __init__(self, raw: int, destroy: str, keepalive: Any) -> None:
        self.raw = ctypes.c_void_p(raw)
        self._destroy = destroy
        self.keepalive = keepalive

    def __del__(self) -> None:
        try:
            if self.raw:
                getattr(_native.load(), self._destroy)(self.raw)
        except Exception:  # pragma: no cover - interpreter shutdown
            pass
        self.raw = ctypes.c_void_p(0)


class _DecodeHandle:
    """A ``flux_decode*`` (owned, or borrowed from a prefill runtime) and torch views of its buffers."""

    def __init__(self, raw: int, device: torch.device, owner: _NativeAllocation) -> None:
        self.raw = ctypes.c_void_p(raw)
        self.device = device
        self.owner = owner
        buffers = _native.DecodeBuffers()
        _native.check(_native.load().flux_decode_get_buffers(self.raw, ctypes.byref(buffers)))
        self.buffers = buffers
        cap, vocab = int(buffers.capacity), int(buffers.vocab_size)
        self.capacity = cap
        self.vocab_size = vocab
        view = lambda address, shape, dtype: _native.device_tensor(address, shape, dtype, owner, device)  # noqa: E731
        self.logits = view(buffers.logits, (1, 1, vocab), torch.float32)
        self.input_token = view(buffers.input_token, (1, 1), torch.int64)
        self.generated_tokens = view(buffers.generated_tokens, (cap,), torch.int64)
        self.generation_step = view(buffers.generation_step, (), torch.int64)
        self.key_cache = view(buffers.key_cache, (30, 1, 3, cap, 64), torch.float32)
        self.value_cache = view(buffers.value_cache, (30, 1, 3, cap, 64), torch.float32)
        self.position = view(buffers.position, (), torch.int64)
        self.cache_length = view(buffers.cache_length, (), torch.int64)

    def addresses(self) -> list[int]:
        b = self.buffers
        return [int(x or 0) for x in (b.input_token, b.logits, b.generated_tokens, b.generation_step, b.key_cache,
                                      b.value_cache, b.position, b.cache_length, b.workspace, b.hidden_a, b.hidden_b,
                                      b.final_norm_output, b.attention_workspace)]

    def scalar(self, fn_name: str) -> int:
        out = ctypes.c_int64()
        with torch.cuda.device(self.device):
            _native.check(getattr(_native.load(), fn_name)(self.raw, ctypes.byref(out)))
        return int(out.value)

    def replay_count(self) -> int:
        out = ctypes.c_int64()
        _native.check(_native.load().flux_decode_replay_count(self.raw, ctypes.byref(out)))
        return int(out.value)

    def replay_launches(self) -> tuple[int, int]:
        """(kernel launches, all device commands) issued by replay() since creation."""
        kernels, total = ctypes.c_int64(), ctypes.c_int64()
        _native.check(_native.load().flux_decode_replay_launches(self.raw, ctypes.byref(kernels),
                                                                 ctypes.byref(total)))
        return int(kernels.value), int(total.value)

    def replay(self, token: torch.Tensor | None) -> torch.Tensor:
        if token is not None:
            if token.shape != (1, 1) or token.dtype != torch.long or token.device != self.device \
                    or not token.is_contiguous():
                raise RuntimeError("flux native full decode: replay token has shape "
                                   f"{tuple(token.shape)}, expected [1, 1] contiguous long on {self.device}")
        address = None if token is None else token.data_ptr()
        lib = _native.load()
        if torch.cuda.current_device() == self.device.index:
            # Per-token path: the runtime's device is current, so no device switch is needed.
            status = lib.flux_decode_replay(self.raw, address, torch.cuda.current_stream().cuda_stream, None)
        else:
            with torch.cuda.device(self.device):
                status = lib.flux_decode_replay(self.raw, address, _native.current_stream(self.device), None)
        if status != _native.FLUX_OK:
            _native.check(status)
        return self.logits

    def generate_greedy(self, steps: int) -> torch.Tensor:
        with torch.cuda.device(self.device):
            _native.check(_native.load().flux_decode_generate_greedy(
                self.raw, int(steps), _native.current_stream(self.device), None))
        return self.generated_tokens

    def generate_greedy_timed(self, steps: int) -> float:
        ms = ctypes.c_float()
        with torch.cuda.device(self.device):
            _native.check(_native.load().flux_decode_generate_greedy_timed(
                self.raw, int(steps), _native.current_stream(self.device), ctypes.byref(ms)))
        return float(ms.value)

    def device_error(self) -> int:
        out = ctypes.c_int32()
        with torch.cuda.device(self.device):
            _native.check(_native.load().flux_decode_device_error(self.raw, ctypes.byref(out)))
        return int(out.value)

    def set_wait_limit(self, ticks: int) -> None:
        """Bound (100 MHz ticks) of the cross-workgroup waits of later generate_greedy launches."""
        _native.check(_native.load().flux_decode_set_wait_limit(self.raw, int(ticks)))



class _PrefillHandle:
    def __init__(self, raw: int, device: torch.device, keepalive: Any) -> None:
        self.owner = _NativeAllocation(raw, "flux_prefill_destroy", keepalive)
        self.raw = self.owner.raw
        self.device = device
        buffers = _native.PrefillBuffers()
        _native.check(_native.load().flux_prefill_get_buffers(self.raw, ctypes.byref(buffers)))
        self.buffers = buffers
        decode_raw = _native.load().flux_prefill_decode(self.raw)
        self.decode = _DecodeHandle(decode_raw, device, self.owner)
        vocab = self.decode.vocab_size
        self.logits = _native.device_tensor(buffers.prefill_logits, (1, 1, vocab), torch.float32, self.owner, device)
        self.final_hidden = _native.device_tensor(buffers.final_hidden, (1, 1, 576), torch.float32, self.owner,
                                                  device)


class NativeSmolLM2Prefill:
    """Native FP32 prompt prefill with direct native-decode continuation.

    The native object owns the compact cache used by its decode runtime; prefill
    writes that storage directly, so the handoff copies no cache.
    (Reference: ``flux/runtime/native_smollm2.py:94-261``.)
    """

    def __init__(self) -> None:
        raise TypeError("use NativeSmolLM2Prefill.capture(...) to create a runtime")

    @classmethod
    def capture(cls, model: nn.Module, input_ids: torch.Tensor, *, max_decode_steps: int = 0) -> "NativeSmolLM2Prefill":
        if max_decode_steps < 0:
            raise ValueError("max_decode_steps must be non-negative")
        requested = input_ids.shape[1] + max_decode_steps if input_ids.ndim == 2 else 0
        NativeSmolLM2Decode._validate_capture_model_input(model, input_ids, requested)
        if int(input_ids.min().item()) < 0 or int(input_ids.max().item()) >= int(model.config.vocab_size):
            raise ValueError("input_ids contain a token outside the vocabulary")
        if not native_smollm2_prefill_is_available():
            raise RuntimeError("Flux native prefill runtime is not built. Run `python -m flux_amd.build` "
                               "and import again.")
        cos_cpu, sin_cpu = _rope_tables(model, requested)
        device = input_ids.device
        self = object.__new__(cls)
        self.model = model
        self.input_ids = input_ids
        self._rope_cos = cos_cpu.to(device)
        self._rope_sin = sin_cpu.to(device)
        weights, epsilons, scales, borrowed = _model_weights(model, device)
        raw = ctypes.c_void_p()
        with torch.cuda.device(device):
            _native.check(_native.load().flux_prefill_create(
                ctypes.byref(weights), _native.ptr(self._rope_cos), _native.ptr(self._rope_sin), requested,
                _native.ptr(input_ids), input_ids.shape[1], _native.double_array(epsilons),
                _native.double_array(scales), _native.current_stream(device), ctypes.byref(raw)))
        # The runtime borrows the weight storage: keep the tensors themselves alive (moving the
        # model or reassigning a parameter's data afterwards does not free what it reads).
        self._handle = _PrefillHandle(raw.value, device, keepalive=(borrowed, self._rope_cos, self._rope_sin))
        self.prefill_logits = self._handle.logits
        return self

    def prefill(self, input_ids: torch.Tensor | None = None) -> torch.Tensor:
        """Re-run the fixed-shape prompt on the caller's current stream."""
        ids = self.input_ids if input_ids is None else input_ids
        if ids.shape != self.input_ids.shape:
            raise ValueError("reused native prefill requires the captured prompt shape")
        if ids.dtype != torch.long or ids.device != self.input_ids.device:
            raise ValueError("reused input_ids must preserve CUDA device and long dtype")
        if not ids.is_contiguous():
            raise ValueError("reused input_ids must be contiguous")
        self.input_ids = ids
        with torch.cuda.device(ids.device):
            _native.check(_native.load().flux_prefill_run(self._handle.raw, _native.ptr(ids),
                                                          _native.current_stream(ids.device), None))
        return self._handle.logits

    def replay(self, token: torch.Tensor | None = None) -> torch.Tensor:
        """Continue directly with one native decode step."""
        return self._handle.decode.replay(token)

    def generate_greedy(self, max_new_tokens: int) -> torch.Tensor:
        """Run the complete fixed-length greedy token loop in native code."""
        if max_new_tokens < 1:
            raise ValueError("max_new_tokens must be positive")
        with torch.cuda.device(self._handle.device):
            _native.check(_native.load().flux_prefill_generate_greedy(
                self._handle.raw, int(max_new_tokens), _native.current_stream(self._handle.device), None))
        return self._handle.decode.generated_tokens.narrow(0, 0, max_new_tokens).view(1, max_new_tokens)

    @property
    def logits(self) -> torch.Tensor:
        return self._handle.logits

    @property
    def final_hidden(self) -> torch.Tensor:
        return self._handle.final_hidden

    @property
    def key_cache(self) -> torch.Tensor:
        return self._handle.decode.key_cache

    @property
    def value_cache(self) -> torch.Tensor:
        return self._handle.decode.value_cache

    @property
    def device_position(self) -> torch.Tensor:
        return self._handle.decode.position

    @property
    def device_cache_length(self) -> torch.Tensor:
        return self._handle.decode.cache_length

    @property
    def current_token(self) -> torch.Tensor:
        return self._handle.decode.input_token

    @property
    def generated_tokens(self) -> torch.Tensor:
        return self._handle.decode.generated_tokens

    @property
    def device_generation_step(self) -> torch.Tensor:
        return self._handle.decode.generation_step

    @property
    def cache_position(self) -> int:
        return self._handle.decode.scalar("flux_decode_position")

    @property
    def cache_length(self) -> int:
        return self._handle.decode.scalar("flux_decode_cache_length")

    @property
    def prompt_length(self) -> int:
        return int(self._handle.buffers.sequence_length)

    @property
    def capacity(self) -> int:
        return int(self._handle.buffers.capacity)

    @property
    def replay_count(self) -> int:
        return self._handle.decode.replay_count()

    @property
    def generation_step(self) -> int:
        return self._handle.decode.scalar("flux_decode_generation_step")

    @property
    def memory(self) -> NativePrefillRuntimeMemory:
        referenced = sum(t.numel() * t.element_size() for t in self.model.parameters())
        db = self._handle.decode.buffers
        return NativePrefillRuntimeMemory(
            cache_bytes=int(db.cache_bytes),
            prefill_workspace_bytes=int(self._handle.buffers.workspace_bytes),
            decode_workspace_bytes=int(db.workspace_bytes),
            stable_buffer_bytes=int(db.stable_buffer_bytes) + 8 + 4 * self._handle.decode.vocab_size,
            referenced_weight_bytes=referenced,
        )

    def stable_addresses(self) -> dict[str, int]:
        b = self._handle.buffers
        prefill = [int(b.prefill_logits), int(b.prefill_workspace), int(b.attention_output), int(b.final_hidden)]
        return dict(zip(_PREFILL_ADDRESS_NAMES, prefill + self._handle.decode.addresses(), strict=True))

    def device_error(self) -> int:
        """Device-side error word of the fused decode kernel (0 = none)."""
        return self._handle.decode.device_error()

    def native_object(self) -> Any:
        return self._handle


class NativeSmolLM2Decode:
    """Python owner of the native token-to-logits decode runtime.

    (Reference: ``flux/runtime/native_smollm2.py:263-605``.)
    """

    def __init__(self) -> None:
        raise TypeError("use NativeSmolLM2Decode.capture(...) to create a runtime")

    @classmethod
    def capture(cls, model: nn.Module, input_ids: torch.Tensor, *, max_decode_steps: int,
                initial_token: torch.Tensor | None = None) -> "NativeSmolLM2Decode":
        """Prefill eagerly (Hugging Face forward), then capture native decode."""
        from transformers import DynamicCache

        cls._validate_capture(model, input_ids, max_decode_steps)
        with torch.inference_mode():
            prefill = model(input_ids=input_ids, use_cache=True, logits_to_keep=1)
        if not isinstance(prefill.past_key_values, DynamicCache):
            raise TypeError("native SmolLM2 prefill expected Transformers DynamicCache, got "
                            f"{type(prefill.past_key_values).__name__}")
        token = prefill.logits.argmax(dim=-1) if initial_token is None else initial_token
        key_caches = [layer.keys for layer in prefill.past_key_values.layers]
        value_caches = [layer.values for layer in prefill.past_key_values.layers]
        if any(t is None for t in key_caches + value_caches):
            raise ValueError("prefill produced an uninitialized decoder cache")
        self = cls.capture_from_state(model, token.contiguous(), key_caches, value_caches,
                                      cache_position=input_ids.shape[1],
                                      cache_capacity=input_ids.shape[1] + max_decode_steps)
        self.prefill_logits = prefill.logits.detach()
        self.prefill_input_ids = input_ids
        self._prefill_cache = prefill.past_key_values
        return self

    @classmethod
    def capture_from_state(cls, model: nn.Module, initial_token: torch.Tensor, key_caches: Sequence[torch.Tensor],
                           value_caches: Sequence[torch.Tensor], *, cache_position: int,
                           cache_capacity: int) -> "NativeSmolLM2Decode":
        """Capture from an already-prefilled compact cache."""
        cls._validate_model_and_state(model, initial_token, key_caches, value_caches, cache_position=cache_position,
                                      cache_capacity=cache_capacity)
        if not native_smollm2_runtime_is_available():
            raise RuntimeError("Flux native full-model decode runtime is not built. Run "
                               "`python -m flux_amd.build` and import again.")
        device = initial_token.device
        cos_cpu, sin_cpu = _rope_tables(model, cache_capacity)
        self = object.__new__(cls)
        self.model = model
        self._rope_cos = cos_cpu.to(device)
        self._rope_sin = sin_cpu.to(device)
        self._source_key_caches = tuple(key_caches)
        self._source_value_caches = tuple(value_caches)
        weights, epsilons, scales, borrowed = _model_weights(model, device)
        raw = ctypes.c_void_p()
        with torch.cuda.device(device):
            _native.check(_native.load().flux_decode_create(
                ctypes.byref(weights), _native.ptr(self._rope_cos), _native.ptr(self._rope_sin), cache_capacity,
                cache_position, _native.ptr(initial_token), _native.pointer_array(key_caches),
                _native.pointer_array(value_caches), _native.length_array([k.shape[2] for k in key_caches]),
                _native.double_array(epsilons), _native.double_array(scales), _native.current_stream(device),
                ctypes.byref(raw)))
        owner = _NativeAllocation(raw.value, "flux_decode_destroy", (borrowed, self._rope_cos, self._rope_sin))
        self._handle = _DecodeHandle(raw.value, device, owner)
        self.prefill_logits = None
        self.prefill_input_ids = None
        self._prefill_cache = None
        return self

    @staticmethod
    def _validate_capture(model: nn.Module, input_ids: torch.Tensor, max_decode_steps: int) -> None:
        if input_ids.dtype != torch.long or input_ids.ndim != 2:
            raise ValueError("input_ids must be a rank-2 torch.long tensor")
        if input_ids.shape[0] != 1 or input_ids.shape[1] < 1:
            raise ValueError("native full decode requires a non-empty batch of one")
        if input_ids.device != next(model.parameters()).device:
            raise ValueError("input_ids must be on the model device")
        if max_decode_steps < 1:
            raise ValueError("max_decode_steps must be positive")
        NativeSmolLM2Decode._validate_capture_model_input(model, input_ids, input_ids.shape[1] + max_decode_steps)

    @staticmethod
    def _validate_capture_model_input(model: nn.Module, input_ids: torch.Tensor, requested: int) -> None:
        if input_ids.dtype != torch.long or input_ids.ndim != 2:
            raise ValueError("input_ids must be a rank-2 torch.long tensor")
        if input_ids.shape[0] != 1 or input_ids.shape[1] < 1:
            raise ValueError("native SmolLM2 runtime requires a non-empty batch of one")
        if not input_ids.is_contiguous():
            raise ValueError("input_ids must be contiguous")
        if input_ids.device != next(model.parameters()).device:
            raise ValueError("input_ids must be on the model device")
        if requested < input_ids.shape[1]:
            raise ValueError("requested capacity must include the complete prompt")
        if requested > int(model.config.max_position_embeddings):
            raise ValueError("requested native cache exceeds the model position limit")
        empty = torch.empty((1, 3, 0, 64), dtype=torch.float32, device=input_ids.device)
        NativeSmolLM2Decode._validate_model_and_state(model, input_ids[:, :1], [empty] * 30, [empty] * 30,
                                                      cache_position=0, cache_capacity=max(requested, 1))

    @staticmethod
    def _decode_workspace_bytes(capacity: int) -> int:
        """Bytes of the fused decode kernel's exchange arena (independent of capacity)."""
        return 2 * (1024 + 1280 + 1536 + 640 + 2048 + 3 * 128 * 3 * 66 + 64) * 8

    @staticmethod
    def _validate_model_and_state(model: nn.Module, initial_token: torch.Tensor, key_caches: Sequence[torch.Tensor],
                                  value_caches: Sequence[torch.Tensor], *, cache_position: int,
                                  cache_capacity: int) -> None:
        from flux_amd.model.smollm2_flux import (
            FINAL_FLUX_OPERATOR_CATEGORIES,
            FluxLlamaDecoderLayer,
            FluxPackedLlamaMLP,
        )

        if not torch.cuda.is_available():
            raise RuntimeError("Flux native full decode requires a ROCm GPU")
        if model.training:
            raise ValueError("Flux native full decode requires model.eval()")
        if set(getattr(model, "_flux_operator_categories", ())) != set(FINAL_FLUX_OPERATOR_CATEGORIES):
            raise ValueError("native full decode requires the retained Flux configuration")
        config = model.config
        geometry = (int(config.num_hidden_layers), int(config.hidden_size), int(config.intermediate_size),
                    int(config.num_attention_heads), int(config.num_key_value_heads), int(config.head_dim))
        if geometry != (30, 576, 1536, 9, 3, 64):
            raise ValueError("native full decode requires SmolLM2-135M geometry (30, 576, 1536, 9, 3, 64)")
        if len(model.model.layers) != 30 or not all(
                isinstance(layer, FluxLlamaDecoderLayer) and isinstance(layer.mlp, FluxPackedLlamaMLP)
                for layer in model.model.layers):
            raise TypeError("model does not contain 30 fully enabled Flux layers")
        if next(model.parameters()).dtype != torch.float32:
            raise TypeError("native full decode currently requires FP32 weights")
        epsilons = {float(model.model.norm.variance_epsilon)}
        for layer in model.model.layers:
            epsilons.add(float(layer.input_layernorm.variance_epsilon))
            epsilons.add(float(layer.post_attention_layernorm.variance_epsilon))
        if len(epsilons) != 1:
            raise ValueError("native full decode requires one shared RMSNorm epsilon")
        if cache_capacity < 1 or cache_capacity > MAX_CAPACITY:
            raise ValueError(f"cache_capacity must be in [1, {MAX_CAPACITY}]")
        if cache_capacity > int(config.max_position_embeddings):
            raise ValueError("cache_capacity exceeds the model position limit")
        if cache_position < 0 or cache_position >= cache_capacity:
            raise ValueError("cache_position must be inside cache_capacity")
        device = next(model.parameters()).device
        if (initial_token.shape != (1, 1) or initial_token.dtype != torch.long or initial_token.device != device
                or not initial_token.is_contiguous()):
            raise ValueError("initial_token must be contiguous CUDA long [1, 1]")
        if len(key_caches) != 30 or len(value_caches) != 30:
            raise ValueError("one K/V source is required for each of 30 layers")
        for name, tensors in (("key", key_caches), ("value", value_caches)):
            for index, tensor in enumerate(tensors):
                if (tensor.shape[:2] != (1, 3) or tensor.ndim != 4 or tensor.shape[2] < cache_position
                        or tensor.shape[3] != 64 or tensor.dtype != torch.float32 or tensor.device != device
                        or not tensor.is_contiguous()):
                    raise ValueError(f"{name} cache layer {index} is unsupported")
        if any(k.shape != v.shape for k, v in zip(key_caches, value_caches)):
            raise ValueError("each layer's K and V source shapes must match")

    def replay(self, token: torch.Tensor | None = None) -> torch.Tensor:
        """Asynchronously enqueue one launch of the fused step kernel (it reads ``token`` itself)."""
        return self._handle.replay(token)

    def generate_greedy(self, decode_steps: int) -> torch.Tensor:
        """``decode_steps`` greedy steps in one native call; returns the token buffer."""
        return self._handle.generate_greedy(decode_steps)

    def reset(self, token: torch.Tensor, key_caches: Sequence[torch.Tensor], value_caches: Sequence[torch.Tensor], *,
              cache_position: int) -> None:
        """Synchronously restore prefilled state outside steady replay."""
        if len(key_caches) != 30 or len(value_caches) != 30:
            raise RuntimeError("flux native full decode: reset requires one K/V tensor per layer")
        with torch.cuda.device(self._handle.device):
            _native.check(_native.load().flux_decode_reset(
                self._handle.raw, _native.ptr(token), _native.pointer_array(key_caches),
                _native.pointer_array(value_caches), _native.length_array([k.shape[2] for k in key_caches]),
                int(cache_position), _native.current_stream(self._handle.device)))

    @property
    def logits(self) -> torch.Tensor:
        return self._handle.logits

    @property
    def key_cache(self) -> torch.Tensor:
        return self._handle.key_cache

    @property
    def value_cache(self) -> torch.Tensor:
        return self._handle.value_cache

    @property
    def device_position(self) -> torch.Tensor:
        return self._handle.position

    @property
    def device_cache_length(self) -> torch.Tensor:
        return self._handle.cache_length

    @property
    def generated_tokens(self) -> torch.Tensor:
        return self._handle.generated_tokens

    @property
    def cache_position(self) -> int:
        return self._handle.scalar("flux_decode_position")

    @property
    def cache_length(self) -> int:
        return self._handle.scalar("flux_decode_cache_length")

    @property
    def capacity(self) -> int:
        return self._handle.capacity

    @property
    def replay_count(self) -> int:
        return self._handle.replay_count()

    @property
    def memory(self) -> NativeDecodeRuntimeMemory:
        referenced = sum(t.numel() * t.element_size() for t in self.model.parameters())
        b = self._handle.buffers
        return NativeDecodeRuntimeMemory(cache_bytes=int(b.cache_bytes), workspace_bytes=int(b.workspace_bytes),
                                         stable_buffer_bytes=int(b.stable_buffer_bytes),
                                         referenced_weight_bytes=referenced)

    def stable_addresses(self) -> dict[str, int]:
        return dict(zip(_ADDRESS_NAMES, self._handle.addresses(), strict=True))

    def device_error(self) -> int:
        return self._handle.device_error()

    def native_object(self) -> Any:
        return self._handle


def _check_layer_tensor(tensor: torch.Tensor, device: torch.device, sizes: tuple[int, ...], name: str) -> None:
    """``check_tensor`` of native_decode_runtime_cuda.cu:53-68 (same messages)."""
    if tensor is None:
        raise RuntimeError(f"flux native decode: {name} is undefined")
    if tensor.device != device:
        raise RuntimeError(f"flux native decode: {name} must be on {device}")
    if tensor.dtype != torch.float32:
        raise RuntimeError(f"flux native decode: {name} has the wrong dtype")
    if tuple(tensor.shape) != tuple(sizes):
        raise RuntimeError(f"flux native decode: {name} has shape {list(tensor.shape)}, expected {list(sizes)}")
    if not tensor.is_contiguous():
        raise RuntimeError(f"flux native decode: {name} must be contiguous")


_LAYER_ADDRESS_NAMES = ("input_hidden", "output", "key_cache", "value_cache", "device_position", "workspace", "query",
                        "attention", "residual", "swiglu", "attention_workspace")


class NativeSmolLM2LayerDecode:
    """One SmolLM2 decoder layer's token step as a replayable native step.

    Mirror of ``torch.classes.flux.NativeSmolLM2LayerDecode``
    (``csrc/native_decode_runtime/native_decode_runtime.h:13-54``, registered in
    ``native_decode_runtime_torch.cpp:5-36``): the constructor arguments, methods
    and validation messages are the reference's.  A step (RMSNorm + packed QKV GEMV
    + RoPE + cache row, GQA decode, o_proj + residual, RMSNorm + gate/up SwiGLU,
    down + residual, position advance) is one launch of the fused decode kernel in
    its single-layer mode, where the reference replays a CUDA graph of the step's
    kernels.  ``replay`` returns the stable ``[1, 1, 576]`` output.  The step's
    intermediates are exchanged through the workspace arena, so their addresses
    (query, attention, residual, swiglu, attention partials) are 0.
    """

    def __init__(self, initial_hidden: torch.Tensor, input_norm_weight: torch.Tensor,
                 packed_qkv_weight: torch.Tensor, attention_output_weight: torch.Tensor,
                 post_attention_norm_weight: torch.Tensor, packed_gate_up_weight: torch.Tensor,
                 down_projection_weight: torch.Tensor, rope_cos: torch.Tensor, rope_sin: torch.Tensor,
                 initial_key_cache: torch.Tensor, initial_value_cache: torch.Tensor, cache_capacity: int,
                 initial_position: int, epsilon: float, attention_scale: float) -> None:
        import math

        device = initial_hidden.device
        if device.type != "cuda":
            raise RuntimeError("flux native decode: initial_hidden must be a CUDA tensor")
        capacity = int(cache_capacity)
        position = int(initial_position)
        if capacity < 1 or capacity > MAX_CAPACITY:
            raise RuntimeError(f"flux native decode: cache capacity must be in [1, {MAX_CAPACITY}]")
        if position < 0 or position >= capacity:
            raise RuntimeError("flux native decode: initial position must be inside cache capacity")
        if not (math.isfinite(epsilon) and epsilon > 0.0):
            raise RuntimeError("flux native decode: epsilon must be positive and finite")
        if not math.isfinite(attention_scale) or abs(attention_scale) > torch.finfo(torch.float32).max:
            raise RuntimeError("flux native decode: attention scale must be finite FP32")
        weights = (
            (input_norm_weight, (576,), "input_norm_weight"),
            (packed_qkv_weight, (960, 576), "packed_qkv_weight"),
            (attention_output_weight, (576, 576), "attention_output_weight"),
            (post_attention_norm_weight, (576,), "post_attention_norm_weight"),
            (packed_gate_up_weight, (3072, 576), "packed_gate_up_weight"),
            (down_projection_weight, (576, 1536), "down_projection_weight"),
            (rope_cos, (capacity, 64), "rope_cos"),
            (rope_sin, (capacity, 64), "rope_sin"),
        )
        for tensor, sizes, name in weights:
            _check_layer_tensor(tensor, device, sizes, name)
        self._device = device
        self._capacity = capacity
        self._validate_state(initial_hidden, initial_key_cache, initial_value_cache, position)
        if not _native.is_available():
            raise RuntimeError("Flux native layer decode runtime is not built. Run `python -m flux_amd.build`.")
        lw = _native.LayerWeightsStruct(*[_native.ptr(t) for t, _, _ in weights[:6]])
        raw = ctypes.c_void_p()
        with torch.cuda.device(device):
            _native.check(_native.load().flux_layer_decode_create(
                ctypes.byref(lw), _native.ptr(rope_cos), _native.ptr(rope_sin), capacity, position,
                _native.ptr(initial_hidden), _native.ptr(initial_key_cache), _native.ptr(initial_value_cache),
                int(initial_key_cache.shape[2]), float(epsilon), float(attention_scale),
                _native.current_stream(device), ctypes.byref(raw)))
        # The runtime borrows the weights and tables: its allocation keeps them alive.
        self._owner = _NativeAllocation(raw.value, "flux_layer_decode_destroy", tuple(t for t, _, _ in weights))
        self._raw = self._owner.raw
        buffers = _native.LayerDecodeBuffers()
        _native.check(_native.load().flux_layer_decode_get_buffers(self._raw, ctypes.byref(buffers)))
        self._buffers = buffers
        owner = self._owner
        view = lambda address, shape, dtype: _native.device_tensor(address, shape, dtype, owner, device)  # noqa: E731
        self._output = view(buffers.output, (1, 1, 576), torch.float32)
        self._input_hidden = view(buffers.input_hidden, (1, 1, 576), torch.float32)
        self._key_cache = view(buffers.key_cache, (1, 3, capacity, 64), torch.float32)
        self._value_cache = view(buffers.value_cache, (1, 3, capacity, 64), torch.float32)
        self._position = view(buffers.position, (), torch.int64)
        self._workspace = view(buffers.workspace, (int(buffers.workspace_bytes) // 4,), torch.float32)

    def _validate_state(self, hidden: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                        position: int) -> None:
        _check_layer_tensor(hidden, self._device, (1, 1, 576), "hidden state")
        if position < 0 or position >= self._capacity:
            raise RuntimeError("flux native decode: reset position must be inside cache capacity")
        ok = (key_cache is not None and value_cache is not None and key_cache.device == self._device
              and value_cache.device == self._device and key_cache.dtype == torch.float32
              and value_cache.dtype == torch.float32 and key_cache.is_contiguous() and value_cache.is_contiguous()
              and key_cache.dim() == 4 and value_cache.shape == key_cache.shape and key_cache.shape[0] == 1
              and key_cache.shape[1] == 3 and key_cache.shape[2] >= position and key_cache.shape[3] == 64)
        if not ok:
            raise RuntimeError("flux native decode: initial/reset K/V must be matching contiguous float32 CUDA "
                               "tensors shaped [1, 3, sequence>=position, 64]")

    def replay(self, hidden: torch.Tensor | None = None) -> torch.Tensor:
        """Enqueue one step launch (it reads ``hidden``, or the last input when None, in
        stream order and keeps it as the input); returns the output buffer."""
        if hidden is not None:
            _check_layer_tensor(hidden, self._device, (1, 1, 576), "replay hidden state")
        with torch.cuda.device(self._device):
            _native.check(_native.load().flux_layer_decode_replay(
                self._raw, _native.ptr(hidden), _native.current_stream(self._device), None))
        return self._output

    def reset(self, hidden: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor, position: int) -> None:
        """Synchronously restore hidden state, cache and position."""
        self._validate_state(hidden, key_cache, value_cache, int(position))
        with torch.cuda.device(self._device):
            _native.check(_native.load().flux_layer_decode_reset(
                self._raw, _native.ptr(hidden), _native.ptr(key_cache), _native.ptr(value_cache),
                int(key_cache.shape[2]), int(position), _native.current_stream(self._device)))

    def output(self) -> torch.Tensor:
        return self._output

    def key_cache(self) -> torch.Tensor:
        return self._key_cache

    def value_cache(self) -> torch.Tensor:
        return self._value_cache

    def device_position(self) -> torch.Tensor:
        return self._position

    def workspace(self) -> torch.Tensor:
        return self._workspace

    def addresses(self) -> list[int]:
        b = self._buffers
        return [int(x or 0) for x in (b.input_hidden, b.output, b.key_cache, b.value_cache, b.position, b.workspace,
                                      b.query, b.attention, b.residual, b.swiglu, b.attention_partials)]

    def stable_addresses(self) -> dict[str, int]:
        return dict(zip(_LAYER_ADDRESS_NAMES, self.addresses(), strict=True))

    def position(self) -> int:
        out = ctypes.c_int64()
        with torch.cuda.device(self._device):
            _native.check(_native.load().flux_layer_decode_position(self._raw, ctypes.byref(out)))
        return int(out.value)

    def cache_length(self) -> int:
        return self.position()

    def capacity(self) -> int:
        return self._capacity

    def replay_count(self) -> int:
        out = ctypes.c_int64()
        _native.check(_native.load().flux_layer_decode_replay_count(self._raw, ctypes.byref(out)))
        return int(out.value)

    def workspace_bytes(self) -> int:
        return int(self._buffers.workspace_bytes)

    def replay_launches(self) -> tuple[int, int]:
        """(kernel launches, all device commands) that replay() has issued since creation."""
        kernels, commands = ctypes.c_int64(), ctypes.c_int64()
        _native.check(_native.load().flux_layer_decode_replay_launches(self._raw, ctypes.byref(kernels),
                                                                       ctypes.byref(commands)))
        return int(kernels.value), int(commands.value)



def native_smollm2_greedy_generate(model: nn.Module, input_ids: torch.Tensor, *, max_new_tokens: int) -> torch.Tensor:
    """Generate greedily with native prefill and fused native decode."""
    if max_new_tokens < 1:
        raise ValueError("max_new_tokens must be positive")
    runtime = NativeSmolLM2Prefill.capture(model, input_ids, max_decode_steps=max_new_tokens - 1)
    generated = runtime.generate_greedy(max_new_tokens)
    return torch.cat((input_ids, generated), dim=-1)


__all__ = [
    "NativeDecodeRuntimeMemory",
    "NativePrefillRuntimeMemory",
    "NativeSmolLM2Decode",
    "NativeSmolLM2LayerDecode",
    "NativeSmolLM2Prefill",
    "native_smollm2_greedy_generate",
    "native_smollm2_prefill_is_available",
    "native_smollm2_runtime_is_available",
]
