"""Torch-CPU FP32 restatement of Hugging Face Llama eager for the token loop.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Every operation follows transformers 5.15.0 ``models/llama/modeling_llama.py``
in the same order and with the same rounding points, so that on the CPU this
module reproduces ``LlamaForCausalLM(attn_implementation="eager")`` (checked
bit-for-bit against committed golden vectors):

* RMSNorm ``weight * (h * rsqrt(mean(h^2) + eps))``  -- modeling_llama.py:53-68
* RoPE tables ``inv_freq = 1/theta^(arange(0,d,2)/d)``, ``cos/sin(cat(f, f))``
  -- modeling_llama.py:93-125; ``q*cos + rotate_half(q)*sin`` -- :130-160
* MLP ``down(silu(gate(x)) * up(x))`` -- :163-176
* eager attention ``softmax(QK^T * scaling + mask, fp32) V`` with repeat_kv
  -- :179-214; decoder layer residual order -- :283-318
* tied LM head on the last position.

The reference's native runtime implements the same step
(``csrc/native_decode_runtime/native_decode_runtime_cuda.cu:192-310,1042-1098``
decode, ``csrc/native_prefill_runtime/native_prefill_runtime_cuda.cu:553-665``
prefill), and Flux's system tests compare it against exactly this HF path
(``tests/test_system.py:356-415,455-497``).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
import torch.nn.functional as F


@dataclass
class OracleConfig:
    layers: int = 30
    hidden: int = 576
    intermediate: int = 1536
    q_heads: int = 9
    kv_heads: int = 3
    head_dim: int = 64
    rope_theta: float = 1.0e5
    eps: float = 1.0e-5


@dataclass
class OracleCache:
    """Per-layer compact K/V, each ``[1, kv_heads, length, head_dim]``."""

    keys: list[torch.Tensor] = field(default_factory=list)
    values: list[torch.Tensor] = field(default_factory=list)

    @property
    def length(self) -> int:
        return 0 if not self.keys else int(self.keys[0].shape[2])


def rope_inv_freq(config: OracleConfig) -> torch.Tensor:
    """``LlamaRotaryEmbedding.compute_default_rope_parameters`` (modeling_llama.py:96-118)."""
    dim = config.head_dim
    return 1.0 / (config.rope_theta ** (torch.arange(0, dim, 2, dtype=torch.float) / dim))


def rope_cos_sin(config: OracleConfig, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin ``[1, S, head_dim]`` for ``positions`` ``[1, S]`` (modeling_llama.py:120-137)."""
    inv_freq = rope_inv_freq(config)
    inv_freq_expanded = inv_freq[None, :, None].float().expand(positions.shape[0], -1, 1)
    position_ids_expanded = positions[:, None, :].float()
    freqs = (inv_freq_expanded @ position_ids_expanded).transpose(1, 2)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos() * 1.0, emb.sin() * 1.0


def rope_table(config: OracleConfig, length: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``[length, head_dim]`` tables, as the reference builds them for its runtime
    (``flux/runtime/native_smollm2.py:130-138``) but on the CPU."""
    positions = torch.arange(length, dtype=torch.long).unsqueeze(0)
    cos, sin = rope_cos_sin(config, positions)
    return cos.reshape(length, config.head_dim).contiguous(), sin.reshape(length, config.head_dim).contiguous()


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def rmsnorm(hidden: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    variance = hidden.pow(2).mean(-1, keepdim=True)
    return weight * (hidden * torch.rsqrt(variance + eps))


class OracleLlama:
    """CPU FP32 Llama eager forward over a HF-named state dict."""

    def __init__(self, state: dict[str, torch.Tensor], config: OracleConfig | None = None) -> None:
        self.config = config or OracleConfig()
        self.state = {k: v.detach().to("cpu", torch.float32) for k, v in state.items()}
        self.vocab = int(self.state["model.embed_tokens.weight"].shape[0])
        self.scaling = self.config.head_dim ** -0.5

    def _w(self, key: str) -> torch.Tensor:
        return self.state[key]

    def _attention(self, layer: int, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                   cache: OracleCache, mask: torch.Tensor | None) -> torch.Tensor:
        c = self.config
        p = f"model.layers.{layer}.self_attn."
        bsz, seq = x.shape[:2]
        shape = (bsz, seq, -1, c.head_dim)
        q = F.linear(x, self._w(p + "q_proj.weight")).view(shape).transpose(1, 2)
        k = F.linear(x, self._w(p + "k_proj.weight")).view(shape).transpose(1, 2)
        v = F.linear(x, self._w(p + "v_proj.weight")).view(shape).transpose(1, 2)
        cos_u, sin_u = cos.unsqueeze(1), sin.unsqueeze(1)
        q = (q * cos_u) + (rotate_half(q) * sin_u)
        k = (k * cos_u) + (rotate_half(k) * sin_u)
        if len(cache.keys) <= layer:
            cache.keys.append(k)
            cache.values.append(v)
        else:
            cache.keys[layer] = torch.cat((cache.keys[layer], k), dim=-2)
            cache.values[layer] = torch.cat((cache.values[layer], v), dim=-2)
        keys, values = cache.keys[layer], cache.values[layer]
        groups = c.q_heads // c.kv_heads
        keys_r = keys[:, :, None].expand(bsz, c.kv_heads, groups, keys.shape[2], c.head_dim).reshape(
            bsz, c.q_heads, keys.shape[2], c.head_dim)
        values_r = values[:, :, None].expand(bsz, c.kv_heads, groups, values.shape[2], c.head_dim).reshape(
            bsz, c.q_heads, values.shape[2], c.head_dim)
        scores = torch.matmul(q, keys_r.transpose(2, 3)) * self.scaling
        if mask is not None:
            scores = scores + mask
        probs = F.softmax(scores, dim=-1, dtype=torch.float32).to(q.dtype)
        out = torch.matmul(probs, values_r).transpose(1, 2).contiguous()
        out = out.reshape(bsz, seq, -1).contiguous()
        return F.linear(out, self._w(p + "o_proj.weight"))

    def decoder_layer(self, layer: int, hidden: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                      cache: OracleCache, mask: torch.Tensor | None) -> torch.Tensor:
        """One LlamaDecoderLayer (transformers modeling_llama.py LlamaDecoderLayer.forward)."""
        c = self.config
        p = f"model.layers.{layer}."
        residual = hidden
        x = rmsnorm(hidden, self._w(p + "input_layernorm.weight"), c.eps)
        hidden = residual + self._attention(layer, x, cos, sin, cache, mask)
        residual = hidden
        x = rmsnorm(hidden, self._w(p + "post_attention_layernorm.weight"), c.eps)
        gate = F.linear(x, self._w(p + "mlp.gate_proj.weight"))
        up = F.linear(x, self._w(p + "mlp.up_proj.weight"))
        return residual + F.linear(F.silu(gate) * up, self._w(p + "mlp.down_proj.weight"))

    def forward(self, ids: torch.Tensor, cache: OracleCache, *, all_logits: bool = False) -> torch.Tensor:
        """Run ``ids`` ``[1, S]`` after ``cache``; returns logits of the last (or all) rows."""
        c = self.config
        start = cache.length
        seq = ids.shape[1]
        positions = torch.arange(start, start + seq, dtype=torch.long).unsqueeze(0)
        cos, sin = rope_cos_sin(c, positions)
        emb = self._w("model.embed_tokens.weight")
        hidden = F.embedding(ids, emb)
        mask = None
        if seq > 1:
            total = start + seq
            key_pos = torch.arange(total)
            allowed = key_pos[None, :] <= positions[0][:, None]
            mask = torch.zeros(seq, total, dtype=torch.float32)
            mask.masked_fill_(~allowed, torch.finfo(torch.float32).min)
            mask = mask[None, None]
        for layer in range(c.layers):
            hidden = self.decoder_layer(layer, hidden, cos, sin, cache, mask)
        hidden = rmsnorm(hidden, self._w("model.norm.weight"), c.eps)
        if not all_logits:
            hidden = hidden[:, -1:, :]
        return F.linear(hidden, self._w("lm_head.weight"))

    def greedy(self, prompt: torch.Tensor, new_tokens: int, *, keep_logits: bool = False):
        """Greedy generation as ``LlamaForCausalLM.generate(do_sample=False)``.

        Returns (tokens ``[new_tokens]``, list of per-step logits ``[vocab]`` or None, cache).
        """
        cache = OracleCache()
        tokens: list[int] = []
        logits_list = [] if keep_logits else None
        with torch.inference_mode():
            logits = self.forward(prompt, cache)[0, -1]
            for step in range(new_tokens):
                if keep_logits:
                    logits_list.append(logits.clone())
                token = int(torch.argmax(logits))
                tokens.append(token)
                if step + 1 == new_tokens:
                    break
                logits = self.forward(torch.tensor([[token]], dtype=torch.long), cache)[0, -1]
        return tokens, logits_list, cache


def top2_margin(logits: torch.Tensor) -> float:
    top = torch.topk(logits.float(), 2).values
    return float(top[0] - top[1])
