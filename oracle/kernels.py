"""Per-kernel CPU references (float64 unless stated) -- TEST INFRASTRUCTURE ONLY.

Each function restates the closed form the reference's own kernel tests check
against (double-precision host references in ``csrc/tests/*.cu``):

* ``rmsnorm``            -- ``csrc/rmsnorm/rmsnorm_cuda.cu:23-64`` / ``flux/ops/rmsnorm.py:6-24``
* ``residual_rmsnorm``   -- ``csrc/residual_rmsnorm/residual_rmsnorm_cuda.cu:23-104``
* ``rope_rows``          -- ``csrc/packed_qkv_rope_cache/packed_qkv_rope_cache_cuda.cu:21-48``
                             (float32, products rounded separately; HF apply_rotary_pos_emb)
* ``qkv_rope_cache``     -- ``packed_qkv_rope_cache_cuda.cu:51-121`` composed with the QKV GEMV
* ``gqa_decode_attention`` -- ``flux/ops/gqa_decode_attention.py:10-83``,
                             ``csrc/tests/test_decode_ops.cu:158-195``
* ``gate_up_swiglu``     -- ``csrc/packed_gate_up_gemv/packed_gate_up_gemv_cuda.cu:25-48``
* ``greedy_argmax``      -- ``csrc/greedy_generation/greedy_generation_cuda.cu:20-95``
* ``causal_attention``   -- ``csrc/tests/test_streaming_prefill_gqa.cu:192-260``
* ``softmax_rows``       -- ``csrc/softmax/softmax.cpp:9-52`` (max-shifted exp, normalised)
* ``attention_score_softmax`` -- ``csrc/attention_score_softmax/attention_score_softmax.cpp:11-80``
* ``packed_swiglu``      -- ``csrc/packed_swiglu/packed_swiglu.cpp`` / ``flux/ops/packed_swiglu.py``
"""

from __future__ import annotations

import math

import numpy as np
import torch


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    x64 = x.double()
    inv = torch.rsqrt(x64.pow(2).mean(-1, keepdim=True) + eps)
    return weight.double() * (x64 * inv)


def residual_rmsnorm(hidden: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                     eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns (normalized float64, residual_out float32 exact sum)."""
    res = hidden.float() + residual.float()
    return rmsnorm(res, weight, eps), res


def rope_rows(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """float32 RoPE over the last dim with HF rounding: ``x*cos + rotate_half(x)*sin``."""
    half = x.shape[-1] // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    first = x.float() * cos.float()
    second = rot.float() * sin.float()
    return first + second


def qkv_rope_cache(hidden: torch.Tensor, norm_weight: torch.Tensor, eps: float, packed_qkv: torch.Tensor,
                   cos_row: torch.Tensor, sin_row: torch.Tensor, q_heads: int = 9, kv_heads: int = 3,
                   head_dim: int = 64):
    """Fused decode QKV step: norm -> GEMV [960,576] -> RoPE(q,k) -> (q [9,64], k [3,64], v [3,64])."""
    x = rmsnorm(hidden, norm_weight, eps)
    qkv = packed_qkv.double() @ x
    q = qkv[: q_heads * head_dim].view(q_heads, head_dim)
    k = qkv[q_heads * head_dim: (q_heads + kv_heads) * head_dim].view(kv_heads, head_dim)
    v = qkv[(q_heads + kv_heads) * head_dim:].view(kv_heads, head_dim)
    half = head_dim // 2

    def rope(t: torch.Tensor) -> torch.Tensor:
        rot = torch.cat((-t[:, half:], t[:, :half]), dim=-1)
        return t * cos_row.double() + rot * sin_row.double()

    return rope(q), rope(k), v


def gqa_decode_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, length: int,
                         scale: float, mask: torch.Tensor | None = None) -> torch.Tensor:
    """One-token GQA. q [Hq, D]; keys/values [Hkv, >=length, D]; returns [Hq, D] float64.

    ``mask`` (optional) is the additive mask already broadcast to [Hq, >=length];
    it is added after the scale, as in ``flux/ops/gqa_decode_attention.py:74-79``.
    Written as the per-head loop of the reference's host reference
    (``csrc/tests/test_decode_ops.cu:158-195``).
    """
    hq, d = q.shape
    hkv = keys.shape[0]
    groups = hq // hkv
    out = torch.empty(hq, d, dtype=torch.float64)
    for h in range(hq):
        g = h // groups
        k = keys[g, :length].double()
        v = values[g, :length].double()
        s = (k @ q[h].double()) * scale
        if mask is not None:
            s = s + mask[h, :length].double()
        s = s - s.max()
        p = torch.exp(s)
        out[h] = (p @ v) / p.sum()
    return out


def softmax_rows(x: torch.Tensor) -> torch.Tensor:
    """Softmax over the last dimension in float64: exp(x - max) / sum."""
    x64 = x.double()
    e = torch.exp(x64 - x64.max(dim=-1, keepdim=True).values)
    return e / e.sum(dim=-1, keepdim=True)


def attention_score_softmax(scores: torch.Tensor, mask: torch.Tensor, scale: float) -> torch.Tensor:
    """softmax(scores * scale + mask) over [B, H, Q, K] with the mask broadcast, float64."""
    return softmax_rows(scores.double() * scale + mask.double())


def packed_swiglu(packed: torch.Tensor) -> torch.Tensor:
    """``silu(packed[..., :I]) * packed[..., I:]`` in float64."""
    p = packed.double()
    inter = p.shape[-1] // 2
    gate, up = p[..., :inter], p[..., inter:]
    return gate * torch.sigmoid(gate) * up


def gate_up_swiglu(x: torch.Tensor, packed_gate_up: torch.Tensor) -> torch.Tensor:
    """``silu(W[:I] x) * (W[I:] x)`` in float64; ``packed_gate_up`` is ``[2I, H]``."""
    inter = packed_gate_up.shape[0] // 2
    gu = packed_gate_up.double() @ x.double()
    g, u = gu[:inter], gu[inter:]
    return g / (1.0 + torch.exp(-g)) * u


def greedy_argmax(logits: np.ndarray | torch.Tensor) -> int:
    """Lowest index of the maximum; any NaN counts as the maximum (first NaN wins).

    Mirrors ``pair_precedes`` (``greedy_generation_cuda.cu:20-37``), which follows
    torch's argmax NaN propagation. All ``-inf`` -> 0.
    """
    values = np.asarray(logits.cpu().numpy() if isinstance(logits, torch.Tensor) else logits,
                        dtype=np.float32).ravel()
    best_index = -1
    best = None
    for index, value in enumerate(values.tolist()):
        if best_index < 0:
            best_index, best = index, value
            continue
        if math.isnan(best):
            break
        if math.isnan(value) or value > best:
            best_index, best = index, value
    return max(best_index, 0)


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """Causal GQA prefill. q [Hq, S, D]; k/v [Hkv, >=S, D] -> [Hq, S, D] float64."""
    hq, seq, d = q.shape
    hkv = k.shape[0]
    groups = hq // hkv
    out = torch.empty(hq, seq, d, dtype=torch.float64)
    mask = torch.ones(seq, seq, dtype=torch.bool).tril()
    for h in range(hq):
        g = h // groups
        s = (q[h].double() @ k[g, :seq].double().T) * scale
        s = s.masked_fill(~mask, float("-inf"))
        p = torch.softmax(s, dim=-1)
        out[h] = p @ v[g, :seq].double()
    return out


def decode_bytes_per_token(attended: int, vocab: int = 49152, layers: int = 30) -> int:
    """Algorithmic HBM bytes of one decode token with ``attended`` K/V positions.

    Weights (tied LM head counted once) + embedding row + new K/V row write +
    K/V reads: B(L) = 538,060,032 + 2,304 + 46,080 + 46,080 * L at SmolLM2 shapes.
    """
    hidden, inter, qkv = 576, 1536, 960
    per_layer = 4 * (qkv * hidden + hidden * hidden + 2 * inter * hidden + hidden * inter + 2 * hidden)
    weights = layers * per_layer + 4 * hidden + 4 * vocab * hidden
    kv_row = layers * 2 * 3 * 64 * 4
    return weights + 4 * hidden + kv_row + kv_row * attended


def prefill_flops(seq: int, vocab: int = 49152, layers: int = 30) -> int:
    """Algorithmic FLOPs of one prefill: linear + causal attention + last-row LM head."""
    hidden, inter, qkv = 576, 1536, 960
    linear = 2 * layers * seq * (qkv * hidden + hidden * hidden + 2 * inter * hidden + hidden * inter)
    attention = layers * 9 * 2 * 2 * 64 * seq * (seq + 1) // 2
    return linear + attention + 2 * vocab * hidden
