"""Native prefill + fused decode runtime vs the golden vectors (HF eager FP32, CPU).

Mirrors the reference system tests (tests/test_system.py:356-497): logits and
K/V caches against the HF path, exact greedy token equality, position/length/
step invariants, capacity exhaustion, prefill reuse and reset.  Golden vectors
were written by tests/golden/make_golden.py from transformers on the CPU.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from flux_amd import synthetic
from flux_amd.runtime import NativeSmolLM2Decode, NativeSmolLM2Prefill, native_smollm2_greedy_generate
from oracle.llama_fp32 import OracleCache, OracleLlama, top2_margin
from tests.conftest import golden

pytestmark = pytest.mark.gpu

# logits within max-abs 1e-3 / rel 1e-4 of the reference FP32 path.
LOGIT_ATOL = 1e-3
LOGIT_RTOL = 1e-4
# Reference system-test tolerance for K/V caches (tests/test_system.py:31-32).
KV_RTOL = 2e-4
KV_ATOL = 2e-5


def _check_probes(logits: torch.Tensor, record: dict, step: int) -> None:
    """Compare a [vocab] logit vector with the golden top-64 and probe slices of `step`."""
    values = logits.detach().float().cpu()
    top_idx = torch.from_numpy(record["top_indices"][step])
    torch.testing.assert_close(values[top_idx], torch.from_numpy(record["top_values"][step]),
                               atol=LOGIT_ATOL, rtol=LOGIT_RTOL)
    probe_idx = torch.from_numpy(record["probe_indices"])
    probe_idx = probe_idx[probe_idx < values.numel()]
    torch.testing.assert_close(values[probe_idx], torch.from_numpy(record["probe"][step]),
                               atol=LOGIT_ATOL, rtol=LOGIT_RTOL)


def _check_kv(runtime, record: dict) -> None:
    positions = torch.from_numpy(record["kv_positions"])
    for layer in (0, 15, 29):
        if f"k{layer}" not in record:
            continue
        k = runtime.key_cache[layer, 0][:, positions].float().cpu()
        v = runtime.value_cache[layer, 0][:, positions].float().cpu()
        torch.testing.assert_close(k, torch.from_numpy(record[f"k{layer}"]), rtol=KV_RTOL, atol=KV_ATOL)
        torch.testing.assert_close(v, torch.from_numpy(record[f"v{layer}"]), rtol=KV_RTOL, atol=KV_ATOL)


def _teacher_forced(runtime, record: dict) -> None:
    """Step 0 from prefill logits, then replay the golden tokens one by one."""
    tokens = record["tokens"]
    _check_probes(runtime.logits[0, 0], record, 0)
    for step in range(1, len(tokens)):
        token = torch.tensor([[int(tokens[step - 1])]], dtype=torch.long, device=runtime.logits.device)
        logits = runtime.replay(token)
        torch.cuda.synchronize()
        _check_probes(logits[0, 0], record, step)


def test_small_vocab_prefill_decode_matches_hf(small_model):
    record = golden("small128.npz")
    prompt = torch.from_numpy(record["prompt"]).unsqueeze(0).cuda()
    tokens = record["tokens"]
    runtime = NativeSmolLM2Prefill.capture(small_model, prompt, max_decode_steps=len(tokens) - 1)
    torch.cuda.synchronize()
    assert runtime.prompt_length == runtime.cache_position == runtime.cache_length == prompt.shape[1]
    assert runtime.key_cache.shape == (30, 1, 3, prompt.shape[1] + len(tokens) - 1, 64)
    _check_kv(runtime, record)
    _teacher_forced(runtime, record)
    assert runtime.cache_position == runtime.cache_length == prompt.shape[1] + len(tokens) - 1
    with pytest.raises(RuntimeError, match="exhausted"):
        runtime.replay(torch.tensor([[int(tokens[-1])]], device="cuda"))
    assert runtime.device_error() == 0


def test_small_vocab_greedy_generation_exact(small_model):
    record = golden("small128.npz")
    prompt = torch.from_numpy(record["prompt"]).unsqueeze(0).cuda()
    expected = torch.from_numpy(record["tokens"])
    n = len(expected)
    runtime = NativeSmolLM2Prefill.capture(small_model, prompt, max_decode_steps=n - 1)
    addresses = runtime.stable_addresses()
    generated = runtime.generate_greedy(n).clone()
    torch.cuda.synchronize()
    assert generated.shape == (1, n)
    assert generated[0].cpu().equal(expected)
    assert generated[:, :1].equal(runtime.prefill_logits.argmax(dim=-1))
    assert runtime.cache_position == runtime.cache_length == prompt.shape[1] + n - 1
    assert runtime.generation_step == n
    assert runtime.stable_addresses() == addresses
    assert runtime.device_error() == 0
    with pytest.raises(RuntimeError, match="prefill or reset"):
        runtime.generate_greedy(1)
    # Prefill reuse re-arms generation with identical results and addresses.
    runtime.prefill(prompt)
    repeated = runtime.generate_greedy(n).clone()
    torch.cuda.synchronize()
    assert repeated[0].cpu().equal(expected)
    assert runtime.stable_addresses() == addresses
    # The end-to-end helper.
    full = native_smollm2_greedy_generate(small_model, prompt, max_new_tokens=n)
    assert full[0, prompt.shape[1]:].cpu().equal(expected)


def test_config1_tokens_and_logits(smol_model):
    """Config 1: 128-token prompt, 32 greedy tokens (golden from HF eager FP32)."""
    record = golden("config1.npz")
    prompt = torch.from_numpy(record["prompt"]).unsqueeze(0).cuda()
    n = len(record["tokens"])
    runtime = NativeSmolLM2Prefill.capture(smol_model, prompt, max_decode_steps=n - 1)
    torch.cuda.synchronize()
    _check_kv(runtime, record)
    _teacher_forced(runtime, record)
    runtime.prefill(prompt)
    generated = runtime.generate_greedy(n).clone()
    torch.cuda.synchronize()
    assert generated[0].cpu().numpy().tolist() == record["tokens"].tolist()
    assert runtime.device_error() == 0


@pytest.mark.parametrize("length", [512, 1024, 2048, 8192])
def test_context_prefill_decode_matches_hf(smol_model, length):
    """Config 2/3 prompts: prefill caches + logits and greedy tokens vs golden."""
    record = golden(f"ctx{length}.npz")
    prompt = torch.from_numpy(record["prompt"]).unsqueeze(0).cuda()
    n = len(record["tokens"])
    runtime = NativeSmolLM2Prefill.capture(smol_model, prompt, max_decode_steps=n - 1)
    torch.cuda.synchronize()
    _check_kv(runtime, record)
    _teacher_forced(runtime, record)
    runtime.prefill(prompt)
    generated = runtime.generate_greedy(n).clone()
    torch.cuda.synchronize()
    assert generated[0].cpu().numpy().tolist() == record["tokens"].tolist()
    assert runtime.device_error() == 0


def test_decode_capture_from_hf_prefill(small_model):
    """NativeSmolLM2Decode.capture: eager HF prefill on the GPU, then native decode."""
    record = golden("small128.npz")
    prompt = torch.from_numpy(record["prompt"]).unsqueeze(0).cuda()
    n = len(record["tokens"])
    decode = NativeSmolLM2Decode.capture(small_model, prompt, max_decode_steps=n - 1)
    assert decode.cache_position == decode.cache_length == prompt.shape[1]
    generated = decode.generate_greedy(n - 1)
    torch.cuda.synchronize()
    assert generated[:n - 1].cpu().numpy().tolist() == record["tokens"][1:].tolist()
    token = decode.prefill_logits.argmax(dim=-1)
    decode.reset(token, decode._source_key_caches, decode._source_value_caches, cache_position=prompt.shape[1])
    assert decode.cache_position == decode.cache_length == prompt.shape[1]
    with pytest.raises(RuntimeError, match="one K/V tensor per layer"):
        decode.reset(token, decode._source_key_caches[:-1], decode._source_value_caches,
                     cache_position=prompt.shape[1])


def test_prefill_input_errors(small_model):
    ids = ((torch.arange(5).unsqueeze(0) * 11 + 3) % 128).cuda()
    with pytest.raises(ValueError, match="non-negative"):
        NativeSmolLM2Prefill.capture(small_model, ids, max_decode_steps=-1)
    with pytest.raises(ValueError, match="batch of one"):
        NativeSmolLM2Prefill.capture(small_model, ids.expand(2, -1))
    with pytest.raises(ValueError, match="vocabulary"):
        NativeSmolLM2Prefill.capture(small_model, torch.full_like(ids, 128))
    native = NativeSmolLM2Prefill.capture(small_model, ids)
    with pytest.raises(ValueError, match="prompt shape"):
        native.prefill(ids[:, :-1])


def test_end_to_end_8192_plus_512_is_deterministic(smol_model):
    """Config 5 shape: 8192-token prefill handed to 512 greedy steps in one call.

    Golden tokens exist for the first 4 steps; the full run must be bitwise
    repeatable and keep the position/step invariants."""
    record = golden("ctx8192.npz")
    prompt = torch.from_numpy(record["prompt"]).unsqueeze(0).cuda()
    runtime = NativeSmolLM2Prefill.capture(smol_model, prompt, max_decode_steps=511)
    first = runtime.generate_greedy(512).clone()
    logits_first = runtime.logits.clone()
    torch.cuda.synchronize()
    assert first[0, :4].cpu().numpy().tolist() == record["tokens"].tolist()
    assert runtime.cache_position == 8192 + 511
    assert runtime.generation_step == 512
    runtime.prefill(prompt)
    second = runtime.generate_greedy(512).clone()
    torch.cuda.synchronize()
    assert torch.equal(first, second)
    assert torch.equal(logits_first, runtime.logits)
    assert runtime.device_error() == 0


@pytest.mark.parametrize("length", [1, 45, 333, 1537, 3001])
def test_odd_length_prefill_matches_oracle(small_model, length):
    """Prompt lengths that end inside a 128-query attention tile and split the keys of the
    later tiles into chunks (333: 2-tile, 1537: 4-tile, 3001: 8-tile chunks), through the whole
    native prefill, against the CPU oracle: last-row logits, greedy token, K/V cache rows.
    1 to 1537 rows also take the GEMMs that fold the RMSNorm (QKV at all four, gate/up up to 333;
    1 and 45 rows end inside the first 32-row tile)."""
    g = torch.Generator().manual_seed(length)
    prompt = torch.randint(0, 128, (1, length), generator=g)
    runtime = NativeSmolLM2Prefill.capture(small_model, prompt.cuda(), max_decode_steps=1)
    torch.cuda.synchronize()
    oracle = OracleLlama(synthetic.synthetic_state_dict(synthetic.SyntheticSpec(seed=2701, vocab=128)))
    cache = OracleCache()
    with torch.inference_mode():
        expected = oracle.forward(prompt, cache)[0, -1]
    logits = runtime.logits[0, 0].float().cpu()
    torch.testing.assert_close(logits, expected, atol=LOGIT_ATOL, rtol=LOGIT_RTOL)
    if top2_margin(expected) > 1e-3:
        assert int(runtime.current_token.item()) == int(torch.argmax(expected))
    positions = torch.tensor(sorted({p for p in (0, 1535, 1536, length - 2, length - 1) if 0 <= p < length}))
    for layer in (0, 29):
        k = runtime.key_cache[layer, 0][:, positions].float().cpu()
        v = runtime.value_cache[layer, 0][:, positions].float().cpu()
        torch.testing.assert_close(k, cache.keys[layer][0][:, positions], rtol=KV_RTOL, atol=KV_ATOL)
        torch.testing.assert_close(v, cache.values[layer][0][:, positions], rtol=KV_RTOL, atol=KV_ATOL)
