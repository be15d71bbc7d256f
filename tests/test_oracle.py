"""Pin the CPU oracle before trusting it (CPU only).

* OracleLlama vs the golden vectors written from transformers' LlamaForCausalLM.
* Per-kernel closed forms vs known answers, brute force, HF fixtures and the
  reference's own C++ CPU implementations (oracle/_ref, built from
  /root/reference/csrc by oracle/Makefile when the reference is present).
* Planted mistakes (in the oracle, on the CPU) must fail these checks.
"""

from __future__ import annotations

import ctypes
import hashlib
import json
import math
import os

import numpy as np
import pytest
import torch

from flux_amd import synthetic
from oracle import kernels as ref
from oracle import llama_fp32
from oracle.llama_fp32 import OracleCache, OracleConfig, OracleLlama, rope_table
from tests.conftest import GOLDEN, ROOT, golden

REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libfluxref.so")


@pytest.fixture(scope="module")
def small_oracle() -> OracleLlama:
    return OracleLlama(synthetic.synthetic_state_dict(synthetic.SyntheticSpec(seed=2701, vocab=128)))


@pytest.fixture(scope="module")
def smol_oracle() -> OracleLlama:
    return OracleLlama(synthetic.synthetic_state_dict(synthetic.SyntheticSpec(seed=0)))


def test_synthetic_weights_are_reproducible():
    with open(os.path.join(GOLDEN, "weights.json")) as handle:
        meta = json.load(handle)
    small = synthetic.synthetic_state_dict(synthetic.SyntheticSpec(seed=2701, vocab=128))
    assert synthetic.weights_sha256(small) == meta["weights_seed2701_vocab128"]
    full = synthetic.synthetic_state_dict(synthetic.SyntheticSpec(seed=0))
    assert synthetic.weights_sha256(full) == meta["weights_seed0_vocab49152"]
    assert full["lm_head.weight"] is full["model.embed_tokens.weight"]
    emb = full["model.embed_tokens.weight"]
    assert emb.shape == (49152, 576) and abs(float(emb.std()) - 0.02) < 2e-4


def test_prompts_are_reproducible():
    record = golden("config1.npz")
    assert synthetic.synthetic_prompt(1, 128)[0].numpy().tolist() == record["prompt"].tolist()
    ids = synthetic.synthetic_prompt(2, 512)
    assert int(ids.min()) >= 0 and int(ids.max()) < 49152


def _probe_check(logits: torch.Tensor, record: dict, step: int, atol: float = 1e-5) -> None:
    top_idx = torch.from_numpy(record["top_indices"][step])
    torch.testing.assert_close(logits[top_idx], torch.from_numpy(record["top_values"][step]), atol=atol, rtol=1e-5)
    probe_idx = torch.from_numpy(record["probe_indices"])
    probe_idx = probe_idx[probe_idx < logits.numel()]
    torch.testing.assert_close(logits[probe_idx], torch.from_numpy(record["probe"][step]), atol=atol, rtol=1e-5)


def test_oracle_matches_hf_small_vocab(small_oracle):
    record = golden("small128.npz")
    prompt = torch.from_numpy(record["prompt"]).unsqueeze(0)
    tokens, logits, cache = small_oracle.greedy(prompt, len(record["tokens"]), keep_logits=True)
    assert tokens == record["tokens"].tolist()
    for step, row in enumerate(logits):
        _probe_check(row, record, step)


def test_oracle_matches_hf_config1(smol_oracle):
    record = golden("config1.npz")
    prompt = torch.from_numpy(record["prompt"]).unsqueeze(0)
    tokens, logits, cache = smol_oracle.greedy(prompt, 8, keep_logits=True)
    assert tokens == record["tokens"][:8].tolist()
    for step, row in enumerate(logits):
        _probe_check(row, record, step)
    # K/V after the prompt (positions recorded by the golden script).
    positions = torch.from_numpy(record["kv_positions"])
    for layer in (0, 15, 29):
        k = cache.keys[layer][0][:, positions]
        torch.testing.assert_close(k, torch.from_numpy(record[f"k{layer}"]), rtol=1e-5, atol=1e-6)


def _full_check(logits: torch.Tensor, record: dict, step: int, atol: float = 1e-5) -> None:
    """Top-8 at every step, top-64 + probe at the probe steps, every logit at the full-logit steps."""
    torch.testing.assert_close(logits[torch.from_numpy(record["top8_indices"][step])],
                               torch.from_numpy(record["top8_values"][step]), atol=atol, rtol=1e-5)
    steps = record["probe_steps"].tolist()
    if step in steps:
        _probe_check(logits, record, steps.index(step), atol)
    if "full_logit_steps" in record and step in record["full_logit_steps"].tolist():
        i = record["full_logit_steps"].tolist().index(step)
        torch.testing.assert_close(logits, torch.from_numpy(record["full_logits"][i]), atol=atol, rtol=1e-5)


def test_oracle_matches_hf_teacher_forced_stream(smol_oracle):
    """A token sequence that changes at every step, fed after the config-1 prompt: all 49 steps
    agree with HF (every logit at steps 0, 1, 24, 48) and so do the K/V rows the fed tokens write."""
    record = golden("teacher_config1.npz")
    teacher = record["teacher"].tolist()
    assert len(teacher) == 48 and all(a != b for a, b in zip(teacher, teacher[1:]))
    cache = OracleCache()
    prompt_len = len(record["prompt"])
    kv_steps = record["kv_steps"].tolist()
    with torch.inference_mode():
        logits = smol_oracle.forward(torch.from_numpy(record["prompt"]).unsqueeze(0), cache)[0, -1]
        _full_check(logits, record, 0)
        for step in range(1, len(teacher) + 1):
            logits = smol_oracle.forward(torch.tensor([[teacher[step - 1]]]), cache)[0, -1]
            _full_check(logits, record, step)
            assert int(torch.argmax(logits)) == int(record["tokens"][step])
            if step in kv_steps:
                pos = prompt_len + step - 1
                k = torch.stack([cache.keys[layer][0, :, pos] for layer in range(30)])
                torch.testing.assert_close(k, torch.from_numpy(record["kv_step_k"][kv_steps.index(step)]),
                                           rtol=1e-5, atol=1e-6)


def test_oracle_matches_hf_permuted_head_stream():
    """The untied permuted-head model's greedy stream changes at every step (its successor rule is
    argsort(perm)[token] when the scaled embedding dominates); the oracle reproduces HF's 64 tokens."""
    spec = synthetic.PERMUTED_HEAD_SPEC
    state = synthetic.synthetic_state_dict(spec)
    with open(os.path.join(GOLDEN, "weights.json")) as handle:
        assert synthetic.weights_sha256(state) == json.load(handle)["weights_permuted_head"]
    assert state["lm_head.weight"] is not state["model.embed_tokens.weight"]
    record = golden("permuted.npz")
    tokens, logits, _ = OracleLlama(state).greedy(torch.from_numpy(record["prompt"]).unsqueeze(0),
                                                  len(record["tokens"]), keep_logits=True)
    assert tokens == record["tokens"].tolist()
    for step, row in enumerate(logits):
        _full_check(row, record, step, atol=2e-5)
    perm = np.random.Generator(np.random.PCG64(spec.permuted_head_seed)).permutation(spec.vocab)
    successor = np.argsort(perm)
    assert sum(int(successor[a]) == b for a, b in zip(tokens, tokens[1:])) >= 48


def test_oracle_matches_hf_context_streams(smol_oracle):
    """Config-2 prompts of 128 and 512 tokens: the first 16 greedy steps agree with HF."""
    for length in (128, 512):
        record = golden(f"ctx{length}.npz")
        assert len(record["tokens"]) == 128
        prompt = torch.from_numpy(record["prompt"]).unsqueeze(0)
        assert torch.equal(prompt, synthetic.synthetic_prompt(2, length))
        tokens, logits, cache = smol_oracle.greedy(prompt, 16, keep_logits=True)
        assert tokens == record["tokens"][:16].tolist()
        for step, row in enumerate(logits):
            _full_check(row, record, step)
        last = torch.stack([cache.keys[layer][0, :, length - 1] for layer in range(30)])
        torch.testing.assert_close(last, torch.from_numpy(record["k_all_last"]), rtol=1e-5, atol=1e-6)


def test_qkv_rope_cache_pinned_to_hf_layer0():
    """oracle.kernels.qkv_rope_cache against HF: layer 0 of the config-1 prompt (embedding rows,
    unit norm, packed q/k/v rows, the position's RoPE row) gives HF's cached K and V rows; and its
    q/k agree with rope_rows (HF apply_rotary_pos_emb rounding) applied to the GEMV output."""
    record = golden("config1.npz")
    state = synthetic.synthetic_state_dict(synthetic.SyntheticSpec(seed=0))
    emb = state["model.embed_tokens.weight"]
    p = "model.layers.0."
    packed = torch.cat([state[p + "self_attn.q_proj.weight"], state[p + "self_attn.k_proj.weight"],
                        state[p + "self_attn.v_proj.weight"]])
    norm_w = state[p + "input_layernorm.weight"]
    positions = record["kv_positions"].tolist()
    cos, sin = rope_table(OracleConfig(), max(positions) + 1)
    for i, pos in enumerate(positions):
        hidden = emb[int(record["prompt"][pos])]
        q, k, v = ref.qkv_rope_cache(hidden, norm_w, 1e-5, packed, cos[pos], sin[pos])
        torch.testing.assert_close(k.float(), torch.from_numpy(record["k0"][:, i]), rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(v.float(), torch.from_numpy(record["v0"][:, i]), rtol=1e-5, atol=1e-6)
        qkv = packed.double() @ ref.rmsnorm(hidden, norm_w, 1e-5)
        torch.testing.assert_close(q.float(), ref.rope_rows(qkv[:576].float().view(9, 64), cos[pos], sin[pos]),
                                   rtol=1e-5, atol=1e-6)
    # A RoPE with the rotation sign flipped, or q/k routed from the wrong rows, misses HF's K row.
    pos = positions[-1]
    hidden = emb[int(record["prompt"][pos])]
    _, k, _ = ref.qkv_rope_cache(hidden, norm_w, 1e-5, packed, cos[pos], -sin[pos])
    assert not torch.allclose(k.float(), torch.from_numpy(record["k0"][:, -1]), rtol=1e-5, atol=1e-6)
    _, k2, _ = ref.qkv_rope_cache(hidden, norm_w, 1e-5, packed[[*range(576, 768), *range(576), *range(768, 960)]],
                                  cos[pos], sin[pos])
    assert not torch.allclose(k2.float(), torch.from_numpy(record["k0"][:, -1]), rtol=1e-5, atol=1e-6)


def test_product_rope_tables_match_hf():
    """The runtime's host RoPE tables (native_smollm2._rope_tables, built from the model's own
    inv_freq) are bit-identical to transformers' rotary_emb output at 8704 positions."""
    from types import SimpleNamespace

    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    from flux_amd.runtime.native_smollm2 import _rope_tables

    record = golden("rope.npz")
    rotary = LlamaRotaryEmbedding(synthetic.llama_config())
    cos, sin = _rope_tables(SimpleNamespace(model=SimpleNamespace(rotary_emb=rotary)), 8704)
    assert cos.shape == sin.shape == (8704, 64) and cos.dtype == torch.float32
    assert hashlib.sha256(cos.numpy().tobytes()).digest() == record["cos_sha256"].tobytes()
    assert hashlib.sha256(sin.numpy().tobytes()).digest() == record["sin_sha256"].tobytes()


def test_rope_table_matches_hf_rotary_embedding():
    record = golden("rope.npz")
    cos, sin = rope_table(OracleConfig(), 8704)
    assert hashlib.sha256(cos.numpy().tobytes()).digest() == record["cos_sha256"].tobytes()
    assert hashlib.sha256(sin.numpy().tobytes()).digest() == record["sin_sha256"].tobytes()
    rows = torch.from_numpy(record["rows"])
    assert torch.equal(cos[rows], torch.from_numpy(record["cos"]))


def test_rope_rows_bit_exact_vs_hf_apply_rotary():
    record = golden("ops.npz")
    cos = torch.from_numpy(record["rope_cos"])[:, None]  # [1,1,5,64]
    sin = torch.from_numpy(record["rope_sin"])[:, None]
    q_embed = ref.rope_rows(torch.from_numpy(record["rope_q"]), cos, sin)
    k_embed = ref.rope_rows(torch.from_numpy(record["rope_k"]), cos, sin)
    assert torch.equal(q_embed, torch.from_numpy(record["rope_q_embed"]))  # rtol=atol=0, test_references.py:321-331
    assert torch.equal(k_embed, torch.from_numpy(record["rope_k_embed"]))


def test_rope_identity_kat():
    x = torch.randn(3, 64, generator=torch.Generator().manual_seed(5))
    assert torch.equal(ref.rope_rows(x, torch.ones(64), torch.zeros(64)), x)


def test_rmsnorm_known_answer_and_hf():
    out = ref.rmsnorm(torch.tensor([[3.0, 4.0]]), torch.tensor([2.0, 0.5]), 0.0)
    torch.testing.assert_close(out, torch.tensor([[6 / 12.5 ** 0.5, 2 / 12.5 ** 0.5]], dtype=torch.float64))
    record = golden("ops.npz")
    out = ref.rmsnorm(torch.from_numpy(record["norm_x"]), torch.from_numpy(record["norm_w"]), 1e-5)
    torch.testing.assert_close(out.float(), torch.from_numpy(record["norm_y"]), rtol=1e-5, atol=1e-6)


def test_greedy_argmax_kats():
    v = np.zeros(1000, dtype=np.float32)
    v[177] = v[321] = 5.0
    assert ref.greedy_argmax(v) == 177
    v = np.full(64, -1.0, dtype=np.float32)
    v[19] = v[27] = 2.0
    assert ref.greedy_argmax(v) == 19
    assert ref.greedy_argmax(np.full(10, -np.inf, dtype=np.float32)) == 0
    assert ref.greedy_argmax(np.asarray([1.0, np.nan, 3.0, np.nan], dtype=np.float32)) == 1
    x = np.random.default_rng(0).standard_normal(4096).astype(np.float32)
    assert ref.greedy_argmax(x) == int(torch.argmax(torch.from_numpy(x)))


def test_gqa_decode_closed_forms():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(9, 64, generator=g)
    k = torch.randn(3, 40, 64, generator=g)
    v = torch.randn(3, 40, 64, generator=g)
    # Single attended position -> that V row, for every head of the group.
    out = ref.gqa_decode_attention(q, k, v, 1, 0.125)
    torch.testing.assert_close(out, v[:, 0].double().repeat_interleave(3, dim=0))
    # Zero query -> mean of V rows.
    out = ref.gqa_decode_attention(torch.zeros(9, 64), k, v, 33, 0.125)
    torch.testing.assert_close(out, v[:, :33].double().mean(1).repeat_interleave(3, dim=0))
    # Agreement with torch's softmax attention with repeat_kv.
    out = ref.gqa_decode_attention(q, k, v, 40, 0.125)
    kk = k.repeat_interleave(3, dim=0).double()
    vv = v.repeat_interleave(3, dim=0).double()
    p = torch.softmax((kk @ q.double()[:, :, None])[..., 0] * 0.125, dim=-1)
    torch.testing.assert_close(out, (p[:, None, :] @ vv)[:, 0])
    # Additive mask: a constant shift changes nothing; -inf everywhere but one
    # position selects that position's V row; a per-head mask indexes heads.
    torch.testing.assert_close(ref.gqa_decode_attention(q, k, v, 40, 0.125, torch.full((9, 40), 7.5)), out)
    only = torch.full((9, 40), float("-inf"))
    only[:, 17] = 0.0
    torch.testing.assert_close(ref.gqa_decode_attention(q, k, v, 40, 0.125, only),
                               v[:, 17].double().repeat_interleave(3, dim=0))
    per_head = torch.full((9, 40), float("-inf"))
    per_head[torch.arange(9), torch.arange(9) * 4] = 0.0
    torch.testing.assert_close(ref.gqa_decode_attention(q, k, v, 40, 0.125, per_head),
                               torch.stack([v[h // 3, 4 * h].double() for h in range(9)]))


def test_softmax_and_swiglu_closed_forms():
    torch.testing.assert_close(ref.softmax_rows(torch.zeros(3, 8)), torch.full((3, 8), 0.125, dtype=torch.float64))
    x = torch.randn(4, 33, generator=torch.Generator().manual_seed(5))
    torch.testing.assert_close(ref.softmax_rows(x.double() + 100.0), ref.softmax_rows(x))
    torch.testing.assert_close(ref.softmax_rows(x).sum(-1), torch.ones(4, dtype=torch.float64))
    one_hot = torch.tensor([[0.0, float("-inf"), float("-inf")]])
    assert torch.equal(ref.softmax_rows(one_hot), torch.tensor([[1.0, 0.0, 0.0]], dtype=torch.float64))
    scores = torch.randn(1, 2, 3, 4, generator=torch.Generator().manual_seed(6))
    mask = torch.tensor([0.0, 0.0, float("-inf"), float("-inf")]).view(1, 1, 1, 4)
    out = ref.attention_score_softmax(scores, mask, 0.5)
    assert torch.all(out[..., 2:] == 0)
    torch.testing.assert_close(out[..., :2], ref.softmax_rows(scores[..., :2] * 0.5))
    torch.testing.assert_close(ref.packed_swiglu(torch.tensor([[0.0, 2.0, 5.0, 7.0]])),
                               torch.tensor([[0.0, 2.0 / (1.0 + math.exp(-2.0)) * 7.0]], dtype=torch.float64))


def test_causal_attention_closed_forms():
    g = torch.Generator().manual_seed(4)
    k = torch.randn(3, 20, 64, generator=g)
    v = torch.randn(3, 20, 64, generator=g)
    out = ref.causal_attention(torch.zeros(9, 20, 64), k, v, 0.125)
    prefix = v.double().cumsum(1) / torch.arange(1, 21).double()[None, :, None]
    torch.testing.assert_close(out, prefix.repeat_interleave(3, dim=0))
    q = torch.randn(9, 20, 64, generator=g)
    out = ref.causal_attention(q, k, v, 0.125)
    for h in range(9):  # row 0 attends only to key 0
        torch.testing.assert_close(out[h, 0], v[h // 3, 0].double())
    # Every row t equals the one-token GQA over the prefix [0, t] (gqa_decode_attention is
    # pinned to torch.softmax with repeat_kv above): this fixes the scale, the causal
    # mask and the head grouping of every row, the last row included.
    for t in (1, 7, 19):
        torch.testing.assert_close(out[:, t], ref.gqa_decode_attention(q[:, t], k, v, t + 1, 0.125))
    # A planted scale mistake (scores scaled by 1/4 instead of 1/8) misses that check.
    wrong = ref.causal_attention(q, k, v, 0.25)
    assert not torch.allclose(wrong[:, 19], ref.gqa_decode_attention(q[:, 19], k, v, 20, 0.125))


def test_gate_up_swiglu_closed_form():
    x = torch.tensor([1.0, -2.0])
    w = torch.tensor([[1.0, 0.0], [0.0, 1.0], [2.0, 0.0], [0.0, 3.0]])  # gate rows then up rows
    out = ref.gate_up_swiglu(x, w)
    g = torch.tensor([1.0, -2.0], dtype=torch.float64)
    u = torch.tensor([2.0, -6.0], dtype=torch.float64)
    torch.testing.assert_close(out, g * torch.sigmoid(g) * u)


def test_algorithmic_byte_and_flop_models():
    # B(L) and F(S) of the measurement model (weights 538,060,032 B; per-position 46,080 B).
    assert ref.decode_bytes_per_token(0) == 538_060_032 + 2_304 + 46_080
    assert ref.decode_bytes_per_token(8192) == 538_060_032 + 2_304 + 46_080 * 8193
    assert ref.prefill_flops(1) == 212_336_640 + 34_560 * 2 + 56_623_104
    assert abs(ref.prefill_flops(8192) - 4.059e12) < 1e9


@pytest.mark.skipif(not os.path.exists(REF_LIB), reason="oracle/_ref not built (needs /root/reference)")
def test_oracle_against_reference_cpu_sources():
    lib = ctypes.CDLL(REF_LIB)
    fp = ctypes.POINTER(ctypes.c_float)
    L, F = ctypes.c_long, ctypes.c_float
    lib.ref_rmsnorm.argtypes = [fp, fp, fp, L, L, F]
    lib.ref_residual_rmsnorm.argtypes = [fp, fp, fp, fp, fp, L, L, F]
    lib.ref_packed_swiglu.argtypes = [fp, fp, L, L]
    lib.ref_rope.argtypes = [fp, fp, fp, fp, fp, fp, L, L, L, L]

    def p(t):
        return t.numpy().ctypes.data_as(fp)

    g = torch.Generator().manual_seed(9)
    x = torch.randn(4, 576, generator=g)
    w = torch.randn(576, generator=g)
    out = torch.empty(4, 576)
    assert lib.ref_rmsnorm(p(x), p(w), p(out), 4, 576, ctypes.c_float(1e-5)) == 0
    torch.testing.assert_close(out.double(), ref.rmsnorm(x, w, 1e-5), rtol=1e-5, atol=1e-6)
    r = torch.randn(4, 576, generator=g)
    norm, res = torch.empty(4, 576), torch.empty(4, 576)
    assert lib.ref_residual_rmsnorm(p(x), p(r), p(w), p(norm), p(res), 4, 576, ctypes.c_float(1e-5)) == 0
    en, er = ref.residual_rmsnorm(x, r, w, 1e-5)
    assert torch.equal(res, er)
    torch.testing.assert_close(norm.double(), en, rtol=1e-5, atol=1e-6)
    packed = torch.randn(3, 2 * 1536, generator=g)
    sw = torch.empty(3, 1536)
    assert lib.ref_packed_swiglu(p(packed), p(sw), 3, 1536) == 0
    torch.testing.assert_close(sw.double(), ref.packed_swiglu(packed), rtol=1e-5, atol=1e-6)
    # Softmax and the scaled + broadcast-masked attention-score softmax.
    lib.ref_softmax.argtypes = [fp, fp, L, L]
    lib.ref_attention_score_softmax.argtypes = [fp, fp, fp, F, L, L, L, L, L, L, L, L]
    for width in (1, 17, 129, 1000):
        x = 3.0 * torch.randn(5, width, generator=g)
        sm = torch.empty_like(x)
        assert lib.ref_softmax(p(x), p(sm), 5, width) == 0
        torch.testing.assert_close(sm.double(), ref.softmax_rows(x), rtol=1e-5, atol=1e-7)
    scores = 3.0 * torch.randn(2, 3, 5, 17, generator=g)
    for mshape in ((2, 1, 5, 17), (1, 3, 1, 17), (1, 1, 1, 1), (2, 3, 5, 17)):
        mask = torch.randn(mshape, generator=g)
        out = torch.empty_like(scores)
        assert lib.ref_attention_score_softmax(p(scores), p(mask.contiguous()), p(out), ctypes.c_float(0.25), 2, 3,
                                               5, 17, *mshape) == 0
        torch.testing.assert_close(out.double(), ref.attention_score_softmax(scores, mask, 0.25), rtol=1e-5,
                                   atol=1e-7)
    # RoPE: the reference's un-fused rounding equals ours bit for bit.
    q = torch.randn(9, 5, 64, generator=g)
    k = torch.randn(3, 5, 64, generator=g)
    cos, sin = rope_table(OracleConfig(), 5)
    qo, ko = torch.empty_like(q), torch.empty_like(k)
    assert lib.ref_rope(p(q), p(k), p(cos), p(sin), p(qo), p(ko), 9, 3, 5, 64) == 0
    assert torch.equal(qo, ref.rope_rows(q, cos, sin))
    assert torch.equal(ko, ref.rope_rows(k, cos, sin))


def test_planted_mistakes_are_caught(monkeypatch):
    """Mutations of the oracle (wrong RoPE sign, transposed attention operand) fail the pins."""
    record = golden("ops.npz")
    cos = torch.from_numpy(record["rope_cos"])[:, None]
    sin = torch.from_numpy(record["rope_sin"])[:, None]
    q = torch.from_numpy(record["rope_q"])
    half = 32
    wrong = q * cos + torch.cat((q[..., half:], -q[..., :half]), dim=-1) * sin
    assert not torch.equal(wrong, torch.from_numpy(record["rope_q_embed"]))
    monkeypatch.setattr(llama_fp32, "rotate_half", lambda x: torch.cat((x[..., x.shape[-1] // 2:],
                                                                          -x[..., :x.shape[-1] // 2]), dim=-1))
    small = OracleLlama(synthetic.synthetic_state_dict(synthetic.SyntheticSpec(seed=2701, vocab=128)))
    rec = golden("small128.npz")
    logits = small.forward(torch.from_numpy(rec["prompt"]).unsqueeze(0), OracleCache())[0, -1]
    with pytest.raises(AssertionError):
        _probe_check(logits, rec, 0)
