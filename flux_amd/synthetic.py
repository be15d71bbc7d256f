"""Seeded synthetic SmolLM2-135M-geometry model and prompts.

The benchmark configurations are quoted on the SmolLM2-135M architecture with
seeded random weights (there is no network to fetch a checkpoint):

* Linear and Embedding weights ~ N(0, 0.02), RMSNorm weights = 1, which is the
  Hugging Face ``LlamaForCausalLM`` initialisation rule
  (transformers ``modeling_llama.py`` ``LlamaPreTrainedModel`` / ``LlamaRMSNorm``).
* The embedding is tied to the LM head (``SyntheticSpec`` can untie it for the
  token-feedback tests).
* RoPE theta 1e5, RMSNorm eps 1e-5, 9 query heads, 3 KV heads, head_dim 64.

Random numbers come from numpy's PCG64 ``standard_normal`` in float32, which is
bit-reproducible across x86 hosts for a given numpy version (unlike torch's CPU
``normal_``, whose vectorised path depends on the host's SIMD level). Tensors
are drawn in a fixed order so the same seed always yields the same bytes on the
build container and on the GPU box; ``weights_sha256`` fingerprints them.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np
import torch

LAYERS = 30
HIDDEN = 576
INTERMEDIATE = 1536
Q_HEADS = 9
KV_HEADS = 3
HEAD_DIM = 64
VOCAB = 49152
ROPE_THETA = 1.0e5
RMS_EPS = 1.0e-5
INIT_STD = 0.02
QKV_WIDTH = (Q_HEADS + 2 * KV_HEADS) * HEAD_DIM  # 960
GATE_UP_WIDTH = 2 * INTERMEDIATE  # 3072
# Longest context the benchmark configurations need is 8192 + 512 = 8704.
MAX_POSITIONS = 16384


@dataclass(frozen=True)
class SyntheticSpec:
    """Seed and shape of a synthetic model.

    ``permuted_head_seed`` (optional) unties the LM head: it becomes a seeded row
    permutation of the N(0, 0.02) embedding draw, and the input embedding is that
    draw times ``embedding_scale``.  With a large scale the embedded token
    dominates the final hidden state, so the greedy successor of token t is
    ``argsort(perm)[t]`` (the LM-head row holding t's embedding) and the greedy
    stream changes at every step -- a stream that exercises the on-device token
    feedback, which the tied synthetic model (whose greedy stream settles on one
    token) cannot.
    """

    seed: int = 0
    vocab: int = VOCAB
    layers: int = LAYERS
    max_positions: int = MAX_POSITIONS
    permuted_head_seed: int | None = None
    embedding_scale: float = 1.0

    @property
    def tied(self) -> bool:
        return self.permuted_head_seed is None


# The untied model of the token-feedback tests.
PERMUTED_HEAD_SPEC = SyntheticSpec(seed=0, permuted_head_seed=4242, embedding_scale=50.0)


def _layer_keys(index: int) -> list[tuple[str, tuple[int, ...]]]:
    p = f"model.layers.{index}."
    return [
        (p + "self_attn.q_proj.weight", (Q_HEADS * HEAD_DIM, HIDDEN)),
        (p + "self_attn.k_proj.weight", (KV_HEADS * HEAD_DIM, HIDDEN)),
        (p + "self_attn.v_proj.weight", (KV_HEADS * HEAD_DIM, HIDDEN)),
        (p + "self_attn.o_proj.weight", (HIDDEN, Q_HEADS * HEAD_DIM)),
        (p + "mlp.gate_proj.weight", (INTERMEDIATE, HIDDEN)),
        (p + "mlp.up_proj.weight", (INTERMEDIATE, HIDDEN)),
        (p + "mlp.down_proj.weight", (HIDDEN, INTERMEDIATE)),
    ]


def synthetic_state_dict(spec: SyntheticSpec = SyntheticSpec()) -> dict[str, torch.Tensor]:
    """Hugging Face Llama state dict (CPU float32) for the synthetic model.

    ``lm_head.weight`` is the same tensor object as the embedding when the spec
    is tied; otherwise it is the seeded row permutation described on
    ``SyntheticSpec``.
    """
    rng = np.random.Generator(np.random.PCG64(spec.seed))
    std = np.float32(INIT_STD)

    def draw(shape: tuple[int, ...]) -> torch.Tensor:
        values = rng.standard_normal(int(np.prod(shape)), dtype=np.float32)
        values *= std
        return torch.from_numpy(values.reshape(shape))

    state: dict[str, torch.Tensor] = {}
    state["model.embed_tokens.weight"] = draw((spec.vocab, HIDDEN))
    for index in range(spec.layers):
        for key, shape in _layer_keys(index):
            state[key] = draw(shape)
        p = f"model.layers.{index}."
        state[p + "input_layernorm.weight"] = torch.ones(HIDDEN)
        state[p + "post_attention_layernorm.weight"] = torch.ones(HIDDEN)
    state["model.norm.weight"] = torch.ones(HIDDEN)
    if spec.tied:
        state["lm_head.weight"] = state["model.embed_tokens.weight"]
    else:
        table = state["model.embed_tokens.weight"]
        perm = np.random.Generator(np.random.PCG64(spec.permuted_head_seed)).permutation(spec.vocab)
        state["lm_head.weight"] = table[torch.from_numpy(perm)].contiguous()
        state["model.embed_tokens.weight"] = table * np.float32(spec.embedding_scale)
    return state


def weights_sha256(state: dict[str, torch.Tensor]) -> str:
    """SHA-256 over every tensor's bytes in sorted-key order (tied tensors once)."""
    digest = hashlib.sha256()
    for key in sorted(state):
        if key == "lm_head.weight" and state[key] is state["model.embed_tokens.weight"]:
            continue
        digest.update(key.encode())
        digest.update(state[key].contiguous().numpy().tobytes())
    return digest.hexdigest()


def synthetic_prompt(seed: int, length: int, vocab: int = VOCAB) -> torch.Tensor:
    """Prompt of ``length`` token ids drawn uniformly from [0, vocab), shape [1, length]."""
    rng = np.random.Generator(np.random.PCG64(1_000_003 + seed))
    ids = rng.integers(0, vocab, size=length, dtype=np.int64)
    return torch.from_numpy(ids).reshape(1, length)


def llama_config(spec: SyntheticSpec = SyntheticSpec()):
    """``transformers.LlamaConfig`` for the synthetic geometry (eager attention)."""
    from transformers import LlamaConfig

    config = LlamaConfig(
        vocab_size=spec.vocab,
        hidden_size=HIDDEN,
        intermediate_size=INTERMEDIATE,
        num_hidden_layers=spec.layers,
        num_attention_heads=Q_HEADS,
        num_key_value_heads=KV_HEADS,
        head_dim=HEAD_DIM,
        max_position_embeddings=spec.max_positions,
        rms_norm_eps=RMS_EPS,
        rope_parameters={"rope_type": "default", "rope_theta": ROPE_THETA},
        tie_word_embeddings=spec.tied,
        attention_bias=False,
        attention_dropout=0.0,
        mlp_bias=False,
        pad_token_id=0,
        bos_token_id=None,
        eos_token_id=None,
    )
    config._attn_implementation = "eager"
    return config


def build_hf_model(spec: SyntheticSpec = SyntheticSpec(), device: str | torch.device = "cpu"):
    """Hugging Face ``LlamaForCausalLM`` (FP32, eval) holding the synthetic weights."""
    from transformers import LlamaForCausalLM

    config = llama_config(spec)
    with torch.device("meta"):
        model = LlamaForCausalLM(config)
    state = synthetic_state_dict(spec)
    model.load_state_dict(state, assign=True, strict=True)
    if spec.tied:
        model.tie_weights()
    # Non-persistent buffers (RoPE inv_freq) are not in the state dict: rebuild them.
    rotary = type(model.model.rotary_emb)(config)
    model.model.rotary_emb = rotary
    model = model.float().eval().to(device)
    return model
