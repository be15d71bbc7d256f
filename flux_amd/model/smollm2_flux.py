"""``enable_flux_ops``: install Flux's packed SmolLM2 representation on a HF Llama.

Drop-in for ``flux.model.smollm2_flux`` (``/root/reference/flux/model/smollm2_flux.py``):
same category names and dependency rules (:58-80, :900-935), same validation
(:790-810), same packed parameters that the native runtimes consume
(``self_attn.packed_qkv.weight`` = cat(q, k, v) ``[960, 576]`` (:325-338) and
``mlp.gate_up_proj.weight`` = cat(gate, up) ``[3072, 576]`` (:151-165)), the
same state-dict transparency hooks (:167-214, :339-391) and the same eager
forward (:216-262, :422-683, :740-787): RMSNorm, residual RMSNorm, RoPE,
attention-score softmax, packed SwiGLU, the StaticCache one-token
packed-QKV/RoPE/cache step and one-token GQA decode attention run as
``torch.ops.flux`` kernels (``flux_amd.ops``, HIP on gfx950).  Those operators
have no CPU kernel, so an enabled model computes on ROCm GPU tensors only.

The reference's cuBLASLt decode projections (category ``cublaslt_projection``)
map to this build's decode GEMV kernel (``flux_amd.ops.decode_projection_out``).
"""

from __future__ import annotations

from collections.abc import Collection
from typing import Any

import torch
from torch import nn
from torch.nn import functional as F
from transformers import StaticCache
from transformers.models.llama.modeling_llama import (
    LlamaAttention,
    LlamaDecoderLayer,
    LlamaForCausalLM,
    LlamaMLP,
    LlamaRMSNorm,
    apply_rotary_pos_emb,
    repeat_kv,
)

from flux_amd import _native
from flux_amd.ops import (
    attention_score_softmax_native,
    decode_projection_out,
    gqa_decode_attention_native,
    gqa_decode_attention_native_out,
    packed_gate_up_swiglu_native_out,
    packed_qkv_rope_cache_native,
    packed_qkv_rope_cache_native_out,
    packed_swiglu_native,
    packed_swiglu_native_out,
    residual_rmsnorm_native,
    residual_rmsnorm_native_out,
    rms_norm_native,
    rms_norm_native_out,
    rope_native,
    softmax_native,
)

FLUX_OPERATOR_CATEGORIES = frozenset({"rmsnorm", "residual_rmsnorm", "rope", "softmax"})
FLUX_PACKED_MLP_CATEGORY = "mlp"
FLUX_PACKED_SWIGLU_CATEGORY = "packed_swiglu"
FLUX_PACKED_QKV_CATEGORY = "qkv"
FLUX_GQA_DECODE_ATTENTION_CATEGORY = "gqa_decode_attention"
FLUX_PACKED_QKV_ROPE_CACHE_CATEGORY = "packed_qkv_rope_cache"
FLUX_CUBLASLT_PROJECTION_CATEGORY = "cublaslt_projection"
FLUX_FUSED_GATE_UP_SWIGLU_CATEGORY = "fused_gate_up_swiglu"
_SUPPORTED_OPERATOR_CATEGORIES = FLUX_OPERATOR_CATEGORIES | {
    FLUX_GQA_DECODE_ATTENTION_CATEGORY,
    FLUX_PACKED_MLP_CATEGORY,
    FLUX_PACKED_SWIGLU_CATEGORY,
    FLUX_PACKED_QKV_CATEGORY,
    FLUX_PACKED_QKV_ROPE_CACHE_CATEGORY,
    FLUX_CUBLASLT_PROJECTION_CATEGORY,
    FLUX_FUSED_GATE_UP_SWIGLU_CATEGORY,
}
# The complete retained configuration the native runtimes require.
FINAL_FLUX_OPERATOR_CATEGORIES = _SUPPORTED_OPERATOR_CATEGORIES
# One-token StaticCache paths need capacity above the single-chunk size
# (reference smollm2_flux.py:81).
_GQA_DECODE_GRAPH_MINIMUM_CAPACITY = 513
# Decode projections served by the GEMV kernel (reference :86-97 lists the same shapes).
_DECODE_PROJECTION_SHAPES = frozenset({(960, 576), (576, 576)})


def _decode_projection_out(input: torch.Tensor, weight: torch.Tensor, output: torch.Tensor) -> torch.Tensor:
    """Exact-shape decode projection dispatch (reference ``_cublaslt_decode_projection_out``, :100-116)."""
    if tuple(weight.shape) not in _DECODE_PROJECTION_SHAPES:
        return F.linear(input, weight)
    return decode_projection_out(input, weight, output)


def native_library_is_available() -> bool:
    """Whether ``libflux_amd.so`` (the HIP path behind every category) loads."""
    return _native.is_available()


class FluxPackedLlamaMLP(nn.Module):
    """MLP owning one packed ``[gate; up]`` Parameter; state dicts keep HF keys."""

    def __init__(self, source: LlamaMLP, *, use_packed_swiglu: bool = False,
                 fuse_gate_up_swiglu: bool = False) -> None:
        super().__init__()
        if source.gate_proj.bias is not None or source.up_proj.bias is not None:
            raise ValueError("Flux packed MLP requires bias-free gate/up projections")
        if source.gate_proj.weight.requires_grad != source.up_proj.weight.requires_grad:
            raise ValueError("gate/up projection weights must agree on requires_grad")
        self.config = source.config
        self.hidden_size = source.hidden_size
        self.intermediate_size = source.intermediate_size
        self.act_fn = source.act_fn
        self.down_proj = source.down_proj
        self.use_packed_swiglu = use_packed_swiglu
        self.fuse_gate_up_swiglu = fuse_gate_up_swiglu
        self.gate_up_proj = nn.Linear(self.hidden_size, 2 * self.intermediate_size, bias=False, device="meta",
                                      dtype=source.gate_proj.weight.dtype)
        self.gate_up_proj.weight = nn.Parameter(
            torch.cat((source.gate_proj.weight, source.up_proj.weight), dim=0),
            requires_grad=source.gate_proj.weight.requires_grad,
        )
        self.register_state_dict_post_hook(FluxPackedLlamaMLP._unpack_state_dict_hook)
        self.register_load_state_dict_pre_hook(FluxPackedLlamaMLP._pack_state_dict_hook)

    @staticmethod
    def _unpack_state_dict_hook(module: "FluxPackedLlamaMLP", state_dict: dict[str, torch.Tensor], prefix: str,
                                _local_metadata: dict[str, Any]) -> None:
        key = prefix + "gate_up_proj.weight"
        if key not in state_dict:
            return
        gate, up = state_dict.pop(key).split(module.intermediate_size, dim=0)
        state_dict[prefix + "gate_proj.weight"] = gate
        state_dict[prefix + "up_proj.weight"] = up

    @staticmethod
    def _pack_state_dict_hook(_module: "FluxPackedLlamaMLP", state_dict: dict[str, torch.Tensor], prefix: str,
                              *_args: Any) -> None:
        key = prefix + "gate_up_proj.weight"
        gate_key, up_key = prefix + "gate_proj.weight", prefix + "up_proj.weight"
        if key in state_dict or not (gate_key in state_dict and up_key in state_dict):
            return
        state_dict[key] = torch.cat((state_dict.pop(gate_key), state_dict.pop(up_key)), dim=0)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        scratch = getattr(self, "_flux_decode_scratch", None)
        if self.fuse_gate_up_swiglu and scratch is not None:
            return self.down_proj(packed_gate_up_swiglu_native_out(hidden_states, self.gate_up_proj.weight,
                                                                   scratch.swiglu_output))
        gate_up = self.gate_up_proj(hidden_states)
        if self.use_packed_swiglu:
            if scratch is not None:
                return self.down_proj(packed_swiglu_native_out(gate_up, scratch.swiglu_output))
            return self.down_proj(packed_swiglu_native(gate_up))
        gate, up = gate_up.chunk(2, dim=-1)
        return self.down_proj(self.act_fn(gate) * up)


class FluxRMSNorm(LlamaRMSNorm):
    """RMSNorm on ``flux::rmsnorm`` sharing the source Parameter (keeps names and weight tying)."""

    def __init__(self, source: LlamaRMSNorm) -> None:
        nn.Module.__init__(self)
        self.weight = source.weight
        self.variance_epsilon = source.variance_epsilon

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        scratch = getattr(self, "_flux_decode_scratch", None)
        if scratch is not None:
            return rms_norm_native_out(hidden_states, self.weight, self.variance_epsilon, scratch.norm_output)
        return rms_norm_native(hidden_states, self.weight, self.variance_epsilon)


class FluxLlamaAttention(LlamaAttention):
    """Llama attention owning a packed ``[q; k; v]`` Parameter when ``use_packed_qkv``."""

    def __init__(self, source: LlamaAttention, *, use_rope: bool = True, use_softmax: bool = True,
                 fuse_attention_scores: bool = True, use_gqa_decode_attention: bool = False,
                 use_packed_qkv: bool = False, use_packed_qkv_rope_cache: bool = False,
                 use_cublaslt_projection: bool = False) -> None:
        nn.Module.__init__(self)
        self.config = source.config
        self.layer_idx = source.layer_idx
        self.head_dim = source.head_dim
        self.num_key_value_groups = source.num_key_value_groups
        self.scaling = source.scaling
        self.attention_dropout = source.attention_dropout
        self.is_causal = source.is_causal
        self.use_rope = use_rope
        self.use_softmax = use_softmax
        self.fuse_attention_scores = fuse_attention_scores
        self.use_gqa_decode_attention = use_gqa_decode_attention
        self.use_packed_qkv = use_packed_qkv
        self.use_packed_qkv_rope_cache = use_packed_qkv_rope_cache
        self.use_cublaslt_projection = use_cublaslt_projection
        projections = (source.q_proj, source.k_proj, source.v_proj)
        if use_packed_qkv:
            if any(p.bias is not None for p in projections):
                raise ValueError("Flux packed QKV requires bias-free projections")
            if len({p.in_features for p in projections}) != 1:
                raise ValueError("Q/K/V projections must have the same input width")
            if len({p.weight.dtype for p in projections}) != 1:
                raise ValueError("Q/K/V projection weights must have the same dtype")
            if len({p.weight.device for p in projections}) != 1:
                raise ValueError("Q/K/V projection weights must be on the same device")
            if len({p.weight.requires_grad for p in projections}) != 1:
                raise ValueError("Q/K/V projection weights must agree on requires_grad")
            self.query_width = source.q_proj.out_features
            self.key_width = source.k_proj.out_features
            self.value_width = source.v_proj.out_features
            if self.query_width % self.head_dim or self.key_width % self.head_dim:
                raise ValueError("Q/K projection widths must be divisible by head_dim")
            if self.value_width != self.key_width:
                raise ValueError("K/V projection widths must match")
            self.query_heads = self.query_width // self.head_dim
            self.key_value_heads = self.key_width // self.head_dim
            width = self.query_width + self.key_width + self.value_width
            self.packed_qkv = nn.Linear(source.q_proj.in_features, width, bias=False, device="meta",
                                        dtype=source.q_proj.weight.dtype)
            self.packed_qkv.weight = nn.Parameter(torch.cat(tuple(p.weight for p in projections), dim=0),
                                                  requires_grad=source.q_proj.weight.requires_grad)
            self.register_state_dict_post_hook(FluxLlamaAttention._unpack_qkv_state_dict_hook)
            self.register_load_state_dict_pre_hook(FluxLlamaAttention._pack_qkv_state_dict_hook)
        else:
            self.q_proj, self.k_proj, self.v_proj = projections
        self.o_proj = source.o_proj

    @staticmethod
    def _unpack_qkv_state_dict_hook(module: "FluxLlamaAttention", state_dict: dict[str, torch.Tensor], prefix: str,
                                    _local_metadata: dict[str, Any]) -> None:
        key = prefix + "packed_qkv.weight"
        if key not in state_dict:
            return
        q, k, v = state_dict.pop(key).split((module.query_width, module.key_width, module.value_width), dim=0)
        state_dict[prefix + "q_proj.weight"] = q
        state_dict[prefix + "k_proj.weight"] = k
        state_dict[prefix + "v_proj.weight"] = v

    @staticmethod
    def _pack_qkv_state_dict_hook(_module: "FluxLlamaAttention", state_dict: dict[str, torch.Tensor], prefix: str,
                                  *_args: Any) -> None:
        key = prefix + "packed_qkv.weight"
        names = tuple(prefix + n for n in ("q_proj.weight", "k_proj.weight", "v_proj.weight"))
        if key in state_dict or not all(n in state_dict for n in names):
            return
        state_dict[key] = torch.cat(tuple(state_dict.pop(n) for n in names), dim=0)

    def project_qkv(self, hidden_states: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        shape = hidden_states.shape[:-1]
        if self.use_packed_qkv:
            q, k, v = F.linear(hidden_states, self.packed_qkv.weight).split(
                (self.query_width, self.key_width, self.value_width), dim=-1)
            return (q.view(*shape, self.query_heads, self.head_dim).transpose(1, 2),
                    k.view(*shape, self.key_value_heads, self.head_dim).transpose(1, 2),
                    v.view(*shape, self.key_value_heads, self.head_dim).transpose(1, 2))
        hidden_shape = (*shape, -1, self.head_dim)
        return (self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2),
                self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2),
                self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2))

    def _static_decode_cache(self, hidden_states: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                             attention_mask: torch.Tensor | None, cache_layer: Any, cache_length: Any,
                             kwargs: dict[str, Any]) -> bool:
        """Whether one token can take the fused packed-QKV/RoPE/cache step (reference :437-487)."""
        if not (self.use_packed_qkv_rope_cache and cache_layer is not None
                and getattr(cache_layer, "is_initialized", False)):
            return False
        keys, values = getattr(cache_layer, "keys", None), getattr(cache_layer, "values", None)
        if keys is None or values is None or cache_length is None:
            return False
        device = hidden_states.device
        return (tuple(hidden_states.shape) == (1, 1, 576) and hidden_states.dtype == torch.float32
                and device.type == "cuda" and tuple(cos.shape) == tuple(sin.shape) == (1, 1, 64)
                and cos.dtype == sin.dtype == torch.float32 and cos.device == sin.device == device
                and self.query_width == 576 and self.key_width == self.value_width == 192
                and self.query_heads == 9 and self.key_value_heads == 3 and self.head_dim == 64
                and keys.shape == values.shape and keys.shape[0] == 1 and keys.shape[1] == 3
                and _GQA_DECODE_GRAPH_MINIMUM_CAPACITY <= keys.shape[2] <= 16384 and keys.shape[3] == 64
                and keys.dtype == values.dtype == torch.float32 and keys.device == values.device == device
                and cache_length.shape == () and cache_length.dtype == torch.int64 and cache_length.device == device
                and (attention_mask is None or (
                    attention_mask.ndim == 4 and attention_mask.dtype == torch.float32
                    and attention_mask.device == device
                    and all(m in (1, t) for m, t in zip(attention_mask.shape, (1, 9, 1, keys.shape[2])))))
                and not kwargs.get("output_attentions", False))

    def _gqa_decode_applies(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                            attention_mask: torch.Tensor | None, cache_length: Any, past_key_values: Any,
                            kwargs: dict[str, Any]) -> bool:
        """Whether one query token takes flux::gqa_decode_attention (reference :540-579)."""
        return (self.use_gqa_decode_attention and past_key_values is not None
                and query.shape[0] == 1 and query.shape[-2] == 1
                and query.dtype == key.dtype == value.dtype == torch.float32
                and query.ndim == key.ndim == value.ndim == 4 and key.shape == value.shape
                and query.shape[0] == key.shape[0] and query.shape[-1] == key.shape[-1] and key.shape[1] > 0
                and query.shape[1] % key.shape[1] == 0 and key.shape[-2] <= 16384
                and (cache_length is None or key.shape[-2] >= _GQA_DECODE_GRAPH_MINIMUM_CAPACITY)
                and (attention_mask is None or (
                    attention_mask.ndim == 4 and attention_mask.dtype == torch.float32
                    and attention_mask.device == query.device
                    and all(m in (1, t) for m, t in zip(attention_mask.shape,
                                                        (query.shape[0], query.shape[1], 1, key.shape[-2])))))
                and not kwargs.get("output_attentions", False))

    def forward(self, hidden_states: torch.Tensor, position_embeddings: tuple[torch.Tensor, torch.Tensor] | None = None,
                attention_mask: torch.Tensor | None = None, past_key_values: Any | None = None,
                **kwargs: Any) -> tuple[torch.Tensor, torch.Tensor | None]:
        """Flux attention (reference ``FluxLlamaAttention.forward``, :422-683)."""
        if position_embeddings is None:
            raise ValueError("position_embeddings must be provided")
        cos, sin = position_embeddings
        input_shape = hidden_states.shape[:-1]
        cache_length = None
        cache_layer = None
        fused_post_qkv = False
        if isinstance(past_key_values, StaticCache):
            cache_layer = past_key_values.layers[self.layer_idx]
            cache_length = getattr(cache_layer, "cumulative_length", None)
        scratch = getattr(self, "_flux_decode_scratch", None)
        if self._static_decode_cache(hidden_states, cos, sin, attention_mask, cache_layer, cache_length, kwargs):
            if (self.use_cublaslt_projection and scratch is not None
                    and getattr(scratch, "qkv_projection_output", None) is not None):
                packed = _decode_projection_out(hidden_states, self.packed_qkv.weight, scratch.qkv_projection_output)
            else:
                packed = self.packed_qkv(hidden_states)
            if scratch is None:
                query = packed_qkv_rope_cache_native(packed, cos, sin, cache_layer.keys, cache_layer.values,
                                                     cache_length)
            else:
                query = packed_qkv_rope_cache_native_out(packed, cos, sin, cache_layer.keys, cache_layer.values,
                                                         cache_length, scratch.query_output)
            del packed
            key, value = cache_layer.keys, cache_layer.values
            fused_post_qkv = True
        else:
            query, key, value = self.project_qkv(hidden_states)
            if self.use_rope:
                query, key = rope_native(query, key, cos, sin)
            else:
                query, key = apply_rotary_pos_emb(query, key, cos, sin)
            if past_key_values is not None:
                key, value = past_key_values.update(key, value, self.layer_idx)
                cache_layer = past_key_values.layers[self.layer_idx]
                cache_length = getattr(cache_layer, "cumulative_length", None)

        if self._gqa_decode_applies(query, key, value, attention_mask, cache_length, past_key_values, kwargs):
            if scratch is None:
                out = gqa_decode_attention_native(query, key, value, attention_mask, self.scaling, cache_length)
            else:
                out = gqa_decode_attention_native_out(query, key, value, attention_mask, self.scaling, cache_length,
                                                      scratch.attention_output, scratch.attention_workspace)
            out = out.transpose(1, 2).contiguous().reshape(*input_shape, -1).contiguous()
            if (self.use_cublaslt_projection and scratch is not None
                    and getattr(scratch, "attention_projection_output", None) is not None):
                return _decode_projection_out(out, self.o_proj.weight, scratch.attention_projection_output), None
            return self.o_proj(out), None
        if fused_post_qkv:
            raise RuntimeError("fused packed-QKV cache update requires native GQA decode attention")

        # Llama eager attention around the Flux softmax: grouped-query expansion,
        # scaled QK, additive mask, softmax, then V.
        key = repeat_kv(key, self.num_key_value_groups)
        value = repeat_kv(value, self.num_key_value_groups)
        weights = torch.matmul(query, key.transpose(2, 3))
        if self.use_softmax and self.fuse_attention_scores and attention_mask is not None and query.shape[-2] > 1:
            weights = attention_score_softmax_native(weights, attention_mask, self.scaling)
        elif self.use_softmax:
            weights = weights * self.scaling
            if attention_mask is not None:
                weights = weights + attention_mask
            weights = softmax_native(weights)
        else:
            weights = weights * self.scaling
            if attention_mask is not None:
                weights = weights + attention_mask
            weights = F.softmax(weights, dim=-1, dtype=torch.float32).to(query.dtype)
        out = torch.matmul(weights, value)
        out = out.transpose(1, 2).contiguous().reshape(*input_shape, -1).contiguous()
        return self.o_proj(out), weights


class FluxLlamaDecoderLayer(LlamaDecoderLayer):
    """Decoder layer holding the Flux attention / packed MLP / norm modules."""

    def __init__(self, source: LlamaDecoderLayer, *, use_rmsnorm: bool = True, use_residual_rmsnorm: bool = True,
                 use_rope: bool = True, use_softmax: bool = True, fuse_attention_scores: bool = True,
                 use_gqa_decode_attention: bool = False, use_packed_qkv_rope_cache: bool = False,
                 use_cublaslt_projection: bool = False, use_packed_mlp: bool = False,
                 use_packed_swiglu: bool = False, fuse_gate_up_swiglu: bool = False,
                 use_packed_qkv: bool = False) -> None:
        nn.Module.__init__(self)
        self.hidden_size = source.hidden_size
        self.self_attn = (
            FluxLlamaAttention(source.self_attn, use_rope=use_rope, use_softmax=use_softmax,
                               fuse_attention_scores=fuse_attention_scores,
                               use_gqa_decode_attention=use_gqa_decode_attention,
                               use_packed_qkv_rope_cache=use_packed_qkv_rope_cache,
                               use_cublaslt_projection=use_cublaslt_projection, use_packed_qkv=use_packed_qkv)
            if use_softmax or use_rope or use_gqa_decode_attention or use_packed_qkv
            else source.self_attn
        )
        self.mlp = (FluxPackedLlamaMLP(source.mlp, use_packed_swiglu=use_packed_swiglu,
                                       fuse_gate_up_swiglu=fuse_gate_up_swiglu)
                    if use_packed_mlp else source.mlp)
        self.input_layernorm = FluxRMSNorm(source.input_layernorm) if use_rmsnorm else source.input_layernorm
        self.post_attention_layernorm = (FluxRMSNorm(source.post_attention_layernorm)
                                         if use_rmsnorm else source.post_attention_layernorm)
        self.use_residual_rmsnorm = use_residual_rmsnorm

    def forward(self, hidden_states: torch.Tensor, attention_mask: torch.Tensor | None = None,
                position_ids: torch.LongTensor | None = None, past_key_values: Any | None = None,
                use_cache: bool | None = False,
                position_embeddings: tuple[torch.Tensor, torch.Tensor] | None = None,
                **kwargs: Any) -> torch.Tensor:
        """Llama layer with the post-attention add fused into residual RMSNorm (reference :740-787)."""
        residual = hidden_states
        hidden_states = self.input_layernorm(hidden_states)
        attention_output, _ = self.self_attn(hidden_states=hidden_states, attention_mask=attention_mask,
                                             position_ids=position_ids, past_key_values=past_key_values,
                                             use_cache=use_cache, position_embeddings=position_embeddings, **kwargs)
        if self.use_residual_rmsnorm:
            scratch = getattr(self, "_flux_decode_scratch", None)
            weight = self.post_attention_layernorm.weight
            eps = self.post_attention_layernorm.variance_epsilon
            if scratch is None:
                hidden_states, residual = residual_rmsnorm_native(attention_output, residual, weight, eps)
            else:
                hidden_states, residual = residual_rmsnorm_native_out(attention_output, residual, weight, eps,
                                                                      scratch.norm_output, scratch.residual_output)
        else:
            residual = residual + attention_output
            hidden_states = self.post_attention_layernorm(residual)
        hidden_states = self.mlp(hidden_states)
        return residual + hidden_states


def _check_model(model: nn.Module) -> LlamaForCausalLM:
    if not isinstance(model, LlamaForCausalLM):
        raise TypeError("Flux SmolLM2 integration requires LlamaForCausalLM")
    if model.training:
        raise ValueError("Flux custom operators are inference-only; call model.eval() first")
    if getattr(model, "_flux_ops_enabled", False):
        raise ValueError("Flux custom operators are already enabled on this model")
    dtypes = {p.dtype for p in model.parameters() if p.is_floating_point()}
    if dtypes != {torch.float32}:
        raise TypeError("Flux SmolLM2 integration currently requires all floating-point parameters to be "
                        f"torch.float32, found {sorted(map(str, dtypes))}")
    if not all(isinstance(layer, LlamaDecoderLayer) for layer in model.model.layers):
        raise TypeError("model contains a decoder layer unsupported by Flux integration")
    if not isinstance(model.model.norm, LlamaRMSNorm):
        raise TypeError("model final norm is not LlamaRMSNorm")
    return model


def _check_native_ops(operators: frozenset[str], *, fuse_attention_scores: bool) -> None:
    if operators and not native_library_is_available():
        raise RuntimeError(
            "Flux native operators are not built: " + ", ".join(sorted(operators))
            + ". Build the extension before enabling the model path."
        )


def enable_flux_ops(model: nn.Module, *, operators: Collection[str] = FLUX_OPERATOR_CATEGORIES,
                    fuse_attention_scores: bool = True) -> LlamaForCausalLM:
    """Replace supported modules on an evaluated FP32 Llama causal LM in place.

    Category rules follow ``smollm2_flux.py:900-935`` of the reference.  Returns
    the same model instance.
    """
    selected = frozenset(operators)
    unknown = selected - _SUPPORTED_OPERATOR_CATEGORIES
    if unknown:
        raise ValueError(f"unknown Flux operator categories: {sorted(unknown)}")
    if not selected:
        raise ValueError("at least one Flux operator category must be selected")
    if FLUX_PACKED_SWIGLU_CATEGORY in selected and FLUX_PACKED_MLP_CATEGORY not in selected:
        raise ValueError('"packed_swiglu" requires the "mlp" operator category')
    if FLUX_PACKED_QKV_ROPE_CACHE_CATEGORY in selected and not {
            "rope", FLUX_PACKED_QKV_CATEGORY, FLUX_GQA_DECODE_ATTENTION_CATEGORY}.issubset(selected):
        raise ValueError('"packed_qkv_rope_cache" requires the "rope", "qkv", and "gqa_decode_attention" '
                         'operator categories')
    if FLUX_CUBLASLT_PROJECTION_CATEGORY in selected and FLUX_PACKED_QKV_ROPE_CACHE_CATEGORY not in selected:
        raise ValueError('"cublaslt_projection" requires the "packed_qkv_rope_cache" operator category')
    if FLUX_FUSED_GATE_UP_SWIGLU_CATEGORY in selected and not {
            FLUX_PACKED_MLP_CATEGORY, FLUX_PACKED_SWIGLU_CATEGORY}.issubset(selected):
        raise ValueError('"fused_gate_up_swiglu" requires the "mlp" and "packed_swiglu" operator categories')

    llama = _check_model(model)
    _check_native_ops(selected, fuse_attention_scores=fuse_attention_scores)

    flags = dict(
        use_rmsnorm="rmsnorm" in selected,
        use_rope="rope" in selected,
        use_softmax="softmax" in selected,
        fuse_attention_scores=fuse_attention_scores,
        use_gqa_decode_attention=FLUX_GQA_DECODE_ATTENTION_CATEGORY in selected,
        use_packed_qkv_rope_cache=FLUX_PACKED_QKV_ROPE_CACHE_CATEGORY in selected,
        use_cublaslt_projection=FLUX_CUBLASLT_PROJECTION_CATEGORY in selected,
        use_packed_mlp=FLUX_PACKED_MLP_CATEGORY in selected,
        use_packed_swiglu=FLUX_PACKED_SWIGLU_CATEGORY in selected,
        fuse_gate_up_swiglu=FLUX_FUSED_GATE_UP_SWIGLU_CATEGORY in selected,
        use_packed_qkv=FLUX_PACKED_QKV_CATEGORY in selected,
    )
    if "residual_rmsnorm" in selected:
        for index in range(len(llama.model.layers)):
            llama.model.layers[index] = FluxLlamaDecoderLayer(llama.model.layers[index], use_residual_rmsnorm=True,
                                                              **flags)
    else:
        for layer in llama.model.layers:
            if flags["use_softmax"] or flags["use_rope"] or flags["use_packed_qkv"] \
                    or flags["use_gqa_decode_attention"]:
                layer.self_attn = FluxLlamaAttention(
                    layer.self_attn, use_rope=flags["use_rope"], use_softmax=flags["use_softmax"],
                    fuse_attention_scores=fuse_attention_scores,
                    use_gqa_decode_attention=flags["use_gqa_decode_attention"],
                    use_packed_qkv_rope_cache=flags["use_packed_qkv_rope_cache"],
                    use_cublaslt_projection=flags["use_cublaslt_projection"], use_packed_qkv=flags["use_packed_qkv"])
            if flags["use_rmsnorm"]:
                layer.input_layernorm = FluxRMSNorm(layer.input_layernorm)
                layer.post_attention_layernorm = FluxRMSNorm(layer.post_attention_layernorm)
            if flags["use_packed_mlp"]:
                layer.mlp = FluxPackedLlamaMLP(layer.mlp, use_packed_swiglu=flags["use_packed_swiglu"],
                                               fuse_gate_up_swiglu=flags["fuse_gate_up_swiglu"])
    if "rmsnorm" in selected:
        llama.model.norm = FluxRMSNorm(llama.model.norm)
    for module in (llama, llama.model):
        if hasattr(module, "_output_capturing_hooks_installed"):
            module._output_capturing_hooks_installed = False
    llama._flux_ops_enabled = True
    llama._flux_operator_categories = tuple(sorted(selected))
    llama._flux_attention_score_fusion_enabled = "softmax" in selected and fuse_attention_scores
    llama._flux_gqa_decode_attention_enabled = flags["use_gqa_decode_attention"]
    llama._flux_packed_mlp_enabled = flags["use_packed_mlp"]
    llama._flux_packed_swiglu_enabled = flags["use_packed_swiglu"]
    llama._flux_packed_qkv_enabled = flags["use_packed_qkv"]
    llama._flux_packed_qkv_rope_cache_enabled = flags["use_packed_qkv_rope_cache"]
    llama._flux_cublaslt_projection_enabled = flags["use_cublaslt_projection"]
    llama._flux_fused_gate_up_swiglu_enabled = flags["fuse_gate_up_swiglu"]
    return llama


def flux_operator_counts(model: nn.Module) -> dict[str, int]:
    """Number of installed Flux modules (reference ``smollm2_flux.py:1037-1076``)."""
    modules = list(model.modules())
    attn = [m for m in modules if isinstance(m, FluxLlamaAttention)]
    mlps = [m for m in modules if isinstance(m, FluxPackedLlamaMLP)]
    return {
        "decoder_layers": sum(isinstance(m, FluxLlamaDecoderLayer) for m in modules),
        "rmsnorm_modules": sum(isinstance(m, FluxRMSNorm) for m in modules),
        "attention_modules": len(attn),
        "packed_mlp_modules": len(mlps),
        "packed_qkv_modules": sum(m.use_packed_qkv for m in attn),
        "gqa_decode_attention_modules": sum(m.use_gqa_decode_attention for m in attn),
        "packed_qkv_rope_cache_modules": sum(m.use_packed_qkv_rope_cache for m in attn),
        "cublaslt_projection_modules": sum(m.use_cublaslt_projection for m in attn),
        "fused_gate_up_swiglu_modules": sum(m.fuse_gate_up_swiglu for m in mlps),
    }


__all__ = [
    "FINAL_FLUX_OPERATOR_CATEGORIES",
    "FLUX_OPERATOR_CATEGORIES",
    "FLUX_CUBLASLT_PROJECTION_CATEGORY",
    "FLUX_GQA_DECODE_ATTENTION_CATEGORY",
    "FLUX_FUSED_GATE_UP_SWIGLU_CATEGORY",
    "FLUX_PACKED_MLP_CATEGORY",
    "FLUX_PACKED_QKV_CATEGORY",
    "FLUX_PACKED_QKV_ROPE_CACHE_CATEGORY",
    "FLUX_PACKED_SWIGLU_CATEGORY",
    "FluxLlamaAttention",
    "FluxLlamaDecoderLayer",
    "FluxPackedLlamaMLP",
    "FluxRMSNorm",
    "enable_flux_ops",
    "flux_operator_counts",
    "native_library_is_available",
]
