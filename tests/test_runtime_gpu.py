"""Native prefill + fused decode runtime vs the golden vectors (HF eager FP32, CPU).

Mirrors the reference system tests (tests/test_system.py:356-497): logits and
K/V caches against the HF path, exact greedy token equality, position/length/
step invariants, capacity exhaustion, prefill reuse and reset.  Golden vectors
were written by tests/golden/make_golden.py from transformers on the CPU.

The token loop is pinned with streams whose token changes at every step:
teacher forcing through ``replay(token)`` with a seeded token sequence
(``teacher_*.npz``), and the free-running greedy stream of the untied
permuted-head model (``permuted.npz``), whose successor token differs at every
step, so the on-device argmax feedback is what decides each step's input.
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


def _assert_logits(values: torch.Tensor, expected: np.ndarray | torch.Tensor) -> None:
    expected = torch.as_tensor(expected, dtype=torch.float32)
    torch.testing.assert_close(values, expected, atol=LOGIT_ATOL, rtol=LOGIT_RTOL)


def _check_step(logits: torch.Tensor, record: dict, step: int) -> None:
    """Compare a [vocab] logit row with the golden vectors of `step`.

    Every step: the top-8 logits.  Probe steps: the top-64 and the 256-index probe.
    Full-logit steps: all logits."""
    values = logits.detach().float().cpu()
    if "top8_indices" in record:
        _assert_logits(values[torch.from_numpy(record["top8_indices"][step])], record["top8_values"][step])
    steps = record["probe_steps"].tolist() if "probe_steps" in record else list(range(len(record["top_values"])))
    if step in steps:
        i = steps.index(step)
        _assert_logits(values[torch.from_numpy(record["top_indices"][i])], record["top_values"][i])
        probe_idx = torch.from_numpy(record["probe_indices"])
        probe_idx = probe_idx[probe_idx < values.numel()]
        _assert_logits(values[probe_idx], record["probe"][i])
    if "full_logit_steps" in record and step in record["full_logit_steps"].tolist():
        i = record["full_logit_steps"].tolist().index(step)
        _assert_logits(values, record["full_logits"][i])


def _check_kv(runtime, record: dict) -> None:
    """K/V slices after the prompt: layers 0/15/29 at four positions, every layer at the last."""
    positions = torch.from_numpy(record["kv_positions"])
    for layer in (0, 15, 29):
        if f"k{layer}" not in record:
            continue
        k = runtime.key_cache[layer, 0][:, positions].float().cpu()
        v = runtime.value_cache[layer, 0][:, positions].float().cpu()
        torch.testing.assert_close(k, torch.from_numpy(record[f"k{layer}"]), rtol=KV_RTOL, atol=KV_ATOL)
        torch.testing.assert_close(v, torch.from_numpy(record[f"v{layer}"]), rtol=KV_RTOL, atol=KV_ATOL)
    if "k_all_last" in record:
        last = len(record["prompt"]) - 1
        torch.testing.assert_close(runtime.key_cache[:, 0, :, last].float().cpu(),
                                   torch.from_numpy(record["k_all_last"]), rtol=KV_RTOL, atol=KV_ATOL)
        torch.testing.assert_close(runtime.value_cache[:, 0, :, last].float().cpu(),
                                   torch.from_numpy(record["v_all_last"]), rtol=KV_RTOL, atol=KV_ATOL)


def _replay_stream(runtime, record: dict, fed: list[int], steps: int) -> None:
    """Step 0 from the prefill logits, then replay fed[s-1] for s = 1 .. steps-1, checking each step.

    Where the record keeps every layer's K/V row of a step (``kv_steps``), the row
    written at that step's position is checked too."""
    device = runtime.logits.device
    prompt_len = len(record["prompt"])
    kv_steps = record["kv_steps"].tolist() if "kv_steps" in record else []
    _check_step(runtime.logits[0, 0], record, 0)
    for step in range(1, steps):
        token = torch.tensor([[int(fed[step - 1])]], dtype=torch.long, device=device)
        logits = runtime.replay(token)
        torch.cuda.synchronize()
        _check_step(logits[0, 0], record, step)
        if step in kv_steps:
            i = kv_steps.index(step)
            pos = prompt_len + step - 1
            torch.testing.assert_close(runtime.key_cache[:, 0, :, pos].float().cpu(),
                                       torch.from_numpy(record["kv_step_k"][i]), rtol=KV_RTOL, atol=KV_ATOL)
            torch.testing.assert_close(runtime.value_cache[:, 0, :, pos].float().cpu(),
                                       torch.from_numpy(record["kv_step_v"][i]), rtol=KV_RTOL, atol=KV_ATOL)
    assert runtime.cache_position == prompt_len + steps - 1


def _decode_logits(runtime: NativeSmolLM2Prefill) -> torch.Tensor:
    """The decode runtime's logits row (the last decode step's; ``runtime.logits`` is the
    prefill's, as in the reference, native_prefill_runtime_cuda.cu:748)."""
    return runtime.native_object().decode.logits[0, 0]


def _capture(model, record: dict, decode_steps: int) -> NativeSmolLM2Prefill:
    prompt = torch.from_numpy(record["prompt"]).unsqueeze(0).cuda()
    runtime = NativeSmolLM2Prefill.capture(model, prompt, max_decode_steps=decode_steps)
    torch.cuda.synchronize()
    return runtime


@pytest.fixture(scope="module")
def permuted_model(gpu_device):
    from flux_amd.model import FINAL_FLUX_OPERATOR_CATEGORIES, enable_flux_ops

    model = synthetic.build_hf_model(synthetic.PERMUTED_HEAD_SPEC, device=gpu_device)
    enable_flux_ops(model, operators=FINAL_FLUX_OPERATOR_CATEGORIES)
    return model


def test_small_vocab_prefill_decode_matches_hf(small_model):
    """Vocab-128 model: every step's full logits against HF, every layer's whole K/V cache against the oracle."""
    record = golden("small128.npz")
    prompt = torch.from_numpy(record["prompt"]).unsqueeze(0).cuda()
    tokens = record["tokens"]
    runtime = _capture(small_model, record, len(tokens) - 1)
    assert runtime.prompt_length == runtime.cache_position == runtime.cache_length == prompt.shape[1]
    assert runtime.key_cache.shape == (30, 1, 3, prompt.shape[1] + len(tokens) - 1, 64)
    _check_kv(runtime, record)
    _replay_stream(runtime, record, tokens.tolist(), len(tokens))
    assert runtime.cache_position == runtime.cache_length == prompt.shape[1] + len(tokens) - 1
    # Every layer, every position: the oracle's cache after the same token stream.
    oracle = OracleLlama(synthetic.synthetic_state_dict(synthetic.SyntheticSpec(seed=2701, vocab=128)))
    _, _, cache = oracle.greedy(prompt.cpu(), len(tokens))
    for layer in range(30):
        torch.testing.assert_close(runtime.key_cache[layer].float().cpu(), cache.keys[layer], rtol=KV_RTOL,
                                   atol=KV_ATOL)
        torch.testing.assert_close(runtime.value_cache[layer].float().cpu(), cache.values[layer], rtol=KV_RTOL,
                                   atol=KV_ATOL)
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
    _assert_logits(_decode_logits(runtime).cpu(), record["full_logits"][n - 1])
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
    n = len(record["tokens"])
    runtime = _capture(smol_model, record, n - 1)
    _check_kv(runtime, record)
    _replay_stream(runtime, record, record["tokens"].tolist(), n)
    runtime.prefill(torch.from_numpy(record["prompt"]).unsqueeze(0).cuda())
    generated = runtime.generate_greedy(n).clone()
    torch.cuda.synchronize()
    assert generated[0].cpu().numpy().tolist() == record["tokens"].tolist()
    assert runtime.device_error() == 0


def test_config1_whole_cache_against_oracle(smol_model):
    """The SmolLM2-vocab model's whole K/V cache, not slices: after the config-1 prompt and
    one generate_greedy(32) call, every layer's K and V at all 159 written positions equal
    the CPU oracle's cache after the same greedy stream (the oracle is pinned to HF's
    tokens, logits and K/V slices by the committed goldens)."""
    record = golden("config1.npz")
    n = len(record["tokens"])
    prompt = torch.from_numpy(record["prompt"]).unsqueeze(0)
    runtime = _capture(smol_model, record, n - 1)
    generated = runtime.generate_greedy(n).clone()
    torch.cuda.synchronize()
    assert generated[0].cpu().numpy().tolist() == record["tokens"].tolist()
    oracle = OracleLlama(synthetic.synthetic_state_dict(synthetic.SyntheticSpec(seed=0)))
    tokens, _, cache = oracle.greedy(prompt, n)
    assert tokens == record["tokens"].tolist()
    written = prompt.shape[1] + n - 1
    for layer in range(30):
        torch.testing.assert_close(runtime.key_cache[layer, :, :, :written].float().cpu(),
                                   cache.keys[layer][:, :, :written], rtol=KV_RTOL, atol=KV_ATOL)
        torch.testing.assert_close(runtime.value_cache[layer, :, :, :written].float().cpu(),
                                   cache.values[layer][:, :, :written], rtol=KV_RTOL, atol=KV_ATOL)
    assert runtime.device_error() == 0


@pytest.mark.parametrize("name", ["teacher_config1", "teacher_ctx8192"])
def test_teacher_forced_changing_tokens(smol_model, name):
    """replay(token) with a seeded token sequence that changes at every step (48 steps after the
    config-1 prompt, 32 after the 8192-token prompt): per-step probes, all 49152 logits at the first,
    middle and last steps, and every layer's K/V row written at the fed positions."""
    record = golden(f"{name}.npz")
    teacher = record["teacher"].tolist()
    assert all(a != b for a, b in zip(teacher, teacher[1:]))
    runtime = _capture(smol_model, record, len(teacher))
    _check_kv(runtime, record)
    _replay_stream(runtime, record, teacher, len(teacher) + 1)
    assert runtime.device_error() == 0


def test_replays_queued_without_synchronising_keep_their_tokens(smol_model):
    """replay(token) passes the caller's token pointer to the step itself (no copy): the 48
    teacher tokens, each in its own tensor, are queued back to back with no synchronisation,
    so the step arguments change while earlier steps are still queued.  Every layer's K/V row
    at the fed positions and the last step's logits must still equal the teacher-forced golden
    (a step that read a later step's token would write a different K/V row)."""
    record = golden("teacher_config1.npz")
    teacher = record["teacher"].tolist()
    runtime = _capture(smol_model, record, len(teacher))
    prompt_len = len(record["prompt"])
    tokens = [torch.tensor([[t]], dtype=torch.long, device="cuda") for t in teacher]
    for token in tokens:
        runtime.replay(token)
    torch.cuda.synchronize()
    _check_step(runtime.native_object().decode.logits[0, 0], record, len(teacher))
    for i, step in enumerate(record["kv_steps"].tolist()):
        pos = prompt_len + step - 1
        torch.testing.assert_close(runtime.key_cache[:, 0, :, pos].float().cpu(),
                                   torch.from_numpy(record["kv_step_k"][i]), rtol=KV_RTOL, atol=KV_ATOL)
        torch.testing.assert_close(runtime.value_cache[:, 0, :, pos].float().cpu(),
                                   torch.from_numpy(record["kv_step_v"][i]), rtol=KV_RTOL, atol=KV_ATOL)
    # Mixing replay(None) (the fed-back argmax) with the same token tensor reused.
    runtime.prefill(torch.from_numpy(record["prompt"]).unsqueeze(0).cuda())
    runtime.replay(tokens[0])
    runtime.replay(tokens[1])
    runtime.replay(tokens[1])
    torch.cuda.synchronize()
    assert runtime.cache_position == prompt_len + 3
    assert runtime.device_error() == 0


def test_permuted_head_free_running_stream(permuted_model):
    """Untied permuted-head model: the HF greedy stream changes at every step, so each decode
    step's input is the previous step's on-device argmax.  64 tokens from one generate_greedy
    call must equal HF's exactly; the step-by-step replay of the same stream checks the
    logits of every step and all logits at steps 0, 1 and 63."""
    record = golden("permuted.npz")
    tokens = record["tokens"]
    n = len(tokens)
    assert all(a != b for a, b in zip(tokens.tolist(), tokens[1:].tolist()))
    runtime = _capture(permuted_model, record, n - 1)
    generated = runtime.generate_greedy(n).clone()
    torch.cuda.synchronize()
    assert generated[0].cpu().numpy().tolist() == tokens.tolist()
    _assert_logits(_decode_logits(runtime).cpu(), record["full_logits"][-1])
    assert runtime.device_error() == 0
    runtime.prefill(torch.from_numpy(record["prompt"]).unsqueeze(0).cuda())
    torch.cuda.synchronize()
    _replay_stream(runtime, record, tokens.tolist(), n)


@pytest.mark.parametrize("length", [128, 512, 1024, 2048, 4096, 8192])
def test_config2_context_decode_matches_hf(smol_model, length):
    """Config 2 (and config 3 prompts): prefill K/V and logits, then 128 decode steps both
    teacher-forced through replay() (top-8 every step, top-64 + probe at steps 0-3/31/63/127)
    and free-running in one generate_greedy call (tokens exact)."""
    record = golden(f"ctx{length}.npz")
    steps = 128
    runtime = _capture(smol_model, record, steps - 1)
    _check_kv(runtime, record)
    _replay_stream(runtime, record, record["tokens"].tolist(), steps)
    runtime.prefill(torch.from_numpy(record["prompt"]).unsqueeze(0).cuda())
    generated = runtime.generate_greedy(steps).clone()
    torch.cuda.synchronize()
    assert generated[0].cpu().numpy().tolist() == record["tokens"][:steps].tolist()
    _check_step(_decode_logits(runtime), record, steps - 1)
    assert runtime.device_error() == 0


def test_config5_8192_plus_512_steps(smol_model):
    """Config 5: 8192-token prefill handed to 512 decode steps in one generate_greedy(513) call;
    the last step writes position 8703 and the cache holds 8704 positions.  All 513 tokens match
    HF, the final logits match HF's step-512 probes, and a second run is bitwise identical."""
    record = golden("ctx8192.npz")
    assert len(record["tokens"]) == 513
    prompt = torch.from_numpy(record["prompt"]).unsqueeze(0).cuda()
    runtime = NativeSmolLM2Prefill.capture(smol_model, prompt, max_decode_steps=512)
    assert runtime.capacity == 8704
    first = runtime.generate_greedy(513).clone()
    logits_first = _decode_logits(runtime).clone()
    torch.cuda.synchronize()
    assert first[0].cpu().numpy().tolist() == record["tokens"].tolist()
    _check_step(logits_first, record, 512)
    assert runtime.cache_position == runtime.cache_length == 8704
    assert runtime.generation_step == 513
    runtime.prefill(prompt)
    second = runtime.generate_greedy(513).clone()
    torch.cuda.synchronize()
    assert torch.equal(first, second)
    assert torch.equal(logits_first, _decode_logits(runtime))
    assert runtime.device_error() == 0


def test_config5_every_step_logits(smol_model):
    """Config 5 replayed step by step: after the 8192-token prefill, replay(token) feeds HF's
    greedy stream for 512 steps (positions 8192..8703); every step's top-8 logits match HF's,
    and the probe steps their top-64 and 256-index probe."""
    record = golden("ctx8192.npz")
    runtime = _capture(smol_model, record, 512)
    _replay_stream(runtime, record, record["tokens"].tolist(), 513)
    assert runtime.cache_length == 8704
    assert runtime.device_error() == 0


def test_config5_tail_with_changing_tokens(smol_model):
    """Config 5's last 32 positions with changing tokens: after the 8192-token prefill, one
    generate_greedy(481) call runs 480 decode steps free (positions 8192..8671, tokens equal
    HF's), then replay(token) feeds 32 seeded tokens that change at every step at positions
    8672..8703 (the cache ends at 8704).  Every step's top-8 logits, the window's probes, all
    49152 logits at its first and last steps and every layer's K/V rows at its first, middle
    and last fed positions match HF."""
    record = golden("tail_ctx8192.npz")
    free = int(record["free_steps"])
    teacher = record["teacher"].tolist()
    assert all(a != b for a, b in zip(teacher, teacher[1:]))
    runtime = _capture(smol_model, record, free + len(teacher))
    prompt_len = len(record["prompt"])
    generated = runtime.generate_greedy(free + 1).clone()
    torch.cuda.synchronize()
    assert generated[0].cpu().numpy().tolist() == record["tokens"][:free + 1].tolist()
    _check_step(_decode_logits(runtime), record, free)
    kv_steps = record["kv_steps"].tolist()
    for i, token in enumerate(teacher):
        step = free + 1 + i
        logits = runtime.replay(torch.tensor([[token]], dtype=torch.long, device="cuda"))
        torch.cuda.synchronize()
        _check_step(logits[0, 0], record, step)
        if step in kv_steps:
            j = kv_steps.index(step)
            pos = prompt_len + step - 1
            torch.testing.assert_close(runtime.key_cache[:, 0, :, pos].float().cpu(),
                                       torch.from_numpy(record["kv_step_k"][j]), rtol=KV_RTOL, atol=KV_ATOL)
            torch.testing.assert_close(runtime.value_cache[:, 0, :, pos].float().cpu(),
                                       torch.from_numpy(record["kv_step_v"][j]), rtol=KV_RTOL, atol=KV_ATOL)
    assert runtime.cache_length == prompt_len + free + len(teacher) == 8704
    assert runtime.device_error() == 0


def test_zero_weight_runtime_closed_form(gpu_device):
    """Reference closed form (csrc/tests/test_native_runtimes.cu:32-78): with every linear and
    embedding weight zero and unit norms, every logit is exactly 0 and every greedy token is 0
    (lowest index of the maximum), through prefill, replay and generate_greedy."""
    from flux_amd.model import FINAL_FLUX_OPERATOR_CATEGORIES, enable_flux_ops

    model = synthetic.build_hf_model(synthetic.SyntheticSpec(seed=7, vocab=32), device=gpu_device)
    with torch.no_grad():
        for name, param in model.named_parameters():
            if "norm" not in name:
                param.zero_()
    enable_flux_ops(model, operators=FINAL_FLUX_OPERATOR_CATEGORIES)
    prompt = torch.tensor([[3, 1, 4, 1, 5, 9, 2, 6, 5, 3]], device=gpu_device)
    runtime = NativeSmolLM2Prefill.capture(model, prompt, max_decode_steps=12)
    torch.cuda.synchronize()
    assert torch.count_nonzero(runtime.prefill_logits).item() == 0
    assert int(runtime.current_token.item()) == 0
    logits = runtime.replay(torch.tensor([[17]], device=gpu_device))
    torch.cuda.synchronize()
    assert torch.count_nonzero(logits).item() == 0
    runtime.prefill(prompt)
    generated = runtime.generate_greedy(13).clone()
    torch.cuda.synchronize()
    assert generated.cpu().tolist() == [[0] * 13]
    assert torch.count_nonzero(_decode_logits(runtime)).item() == 0
    assert torch.count_nonzero(runtime.key_cache).item() == 0
    assert runtime.cache_position == 22
    assert runtime.device_error() == 0


def test_fused_argmax_ties_pick_the_lowest_index(gpu_device):
    """Argmax order of greedy_generation_cuda.cu:20-37 (ties -> lowest index, as torch.argmax):
    the LM-head rows of the untied vocab-128 model repeat with period 8, so every step's
    maximum is attained by 16 rows held by workgroups 8 apart.  In the fused kernel's argmax
    exchange those candidates meet in DPP row moves (8 lanes apart), row broadcasts (16, 32)
    and across polling waves (64), and the winner must be the class's lowest row (< 8).  The
    stream is checked token for token against the oracle on the same weights."""
    from flux_amd.model import FINAL_FLUX_OPERATOR_CATEGORIES, enable_flux_ops

    spec = synthetic.SyntheticSpec(seed=2701, vocab=128, permuted_head_seed=31, embedding_scale=50.0)
    state = synthetic.synthetic_state_dict(spec)
    state["lm_head.weight"] = state["lm_head.weight"][torch.arange(128) % 8].contiguous()
    model = synthetic.build_hf_model(spec, device=gpu_device)
    with torch.no_grad():
        model.lm_head.weight.copy_(state["lm_head.weight"])
    enable_flux_ops(model, operators=FINAL_FLUX_OPERATOR_CATEGORIES)
    prompt = (torch.arange(7).unsqueeze(0) * 11 + 3) % 128
    runtime = NativeSmolLM2Prefill.capture(model, prompt.to(gpu_device), max_decode_steps=15)
    generated = runtime.generate_greedy(16)[0].cpu().tolist()
    logits = _decode_logits(runtime).cpu()
    torch.cuda.synchronize()
    assert runtime.device_error() == 0
    expected, _, _ = OracleLlama(state).greedy(prompt, 16)
    assert generated == expected
    assert all(0 <= t < 8 for t in generated)
    assert len(set(generated)) > 1, f"stream {generated} does not change; it would not test the feedback"
    # Tied rows give bitwise-equal logits (each row's dot product is reduced in the same order).
    assert torch.equal(logits.reshape(16, 8), logits[:8].repeat(16, 1))


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


@pytest.mark.parametrize("length", [1, 7, 9, 45, 333, 512, 513, 1024, 1025, 1537, 3001])
def test_odd_length_prefill_matches_oracle(small_model, length):
    """Prompt lengths that end inside a 128-query attention tile and split the keys of the
    later tiles into chunks (333: 2-tile, 1537: 4-tile, 3001: 8-tile chunks), through the whole
    native prefill, against the CPU oracle: last-row logits, greedy token, K/V cache rows.
    Short prompts also take the GEMMs that fold the RMSNorm (1, 7, 9 and 45 rows end inside
    the first 16-row tile of the register kernel or 32-row tile of the split kernel).  1 | 7 | 9:
    up to 8 rows the next layer's QKV kernel sums the down GEMM's partial planes and residual
    (no reduce kernel), 9 rows take the reduce.  512 | 513 straddle the one-kernel
    attention's limit (512 tokens), and 1024 | 1025 the limit up to which the K-split planes
    are sized for gate/up (1024 rows), so both sides of each switch run."""
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


def test_decode_across_empty_position_chunks(small_model):
    """Decode steps whose attended lengths (5439 .. 5462) straddle 5441 .. 5460, where 85 position
    chunks of ceil(L / 85) rows leave the last chunk empty: its partial (m = -inf, l = 0) must drop
    out of the merge.  Teacher-forced changing tokens through replay(), logits against the CPU
    oracle at every step, and the last step's K/V rows of every layer."""
    prompt_len, steps = 5438, 24
    g = torch.Generator().manual_seed(5441)
    prompt = torch.randint(0, 128, (1, prompt_len), generator=g)
    fed = torch.randint(0, 128, (steps,), generator=g)
    runtime = NativeSmolLM2Prefill.capture(small_model, prompt.cuda(), max_decode_steps=steps)
    torch.cuda.synchronize()
    oracle = OracleLlama(synthetic.synthetic_state_dict(synthetic.SyntheticSpec(seed=2701, vocab=128)))
    cache = OracleCache()
    with torch.inference_mode():
        expected = oracle.forward(prompt, cache)[0, -1]
    torch.testing.assert_close(runtime.logits[0, 0].float().cpu(), expected, atol=LOGIT_ATOL, rtol=LOGIT_RTOL)
    for step in range(steps):
        token = int(fed[step])
        logits = runtime.replay(torch.tensor([[token]], dtype=torch.long, device="cuda"))
        torch.cuda.synchronize()
        with torch.inference_mode():
            expected = oracle.forward(torch.tensor([[token]]), cache)[0, -1]
        torch.testing.assert_close(logits[0, 0].float().cpu(), expected, atol=LOGIT_ATOL, rtol=LOGIT_RTOL,
                                   msg=lambda m: f"step {step} (attended {prompt_len + step + 1}): {m}")
    pos = prompt_len + steps - 1
    assert runtime.cache_position == pos + 1
    for layer in range(30):
        torch.testing.assert_close(runtime.key_cache[layer, 0][:, pos].float().cpu(), cache.keys[layer][0][:, pos],
                                   rtol=KV_RTOL, atol=KV_ATOL)
        torch.testing.assert_close(runtime.value_cache[layer, 0][:, pos].float().cpu(),
                                   cache.values[layer][0][:, pos], rtol=KV_RTOL, atol=KV_ATOL)
    assert runtime.device_error() == 0


@pytest.mark.parametrize("n_prompt,steps", [(5436, 8), (16380, 4)])
def test_decode_matches_prefill_at_chunk_cap_and_capacity(small_model, n_prompt, steps):
    """Teacher-forced decode steps through replay(): the first and the last step's logits equal
    those of the native prefill of the prompt extended by the fed tokens (the MFMA prefill path,
    independent of the decode GEMVs and of the decode attention), and the K/V rows the last step
    wrote equal the prefill's rows in every layer.
    - 5436 + 8: the attention splits the positions into one chunk per 64 up to its cap of 85
      chunks, which it reaches at 5441 attended positions, inside this run (5437 to 5444).
    - 16380 + 4: the largest capacity (16384 positions), where the chunks hold up to 193 rows
      and the attention takes its second 128-row pass (no other decode test attends past 8704)."""
    g = torch.Generator().manual_seed(n_prompt + steps)
    tokens = torch.randint(0, 128, (1, n_prompt + steps), generator=g).cuda()
    runtime = NativeSmolLM2Prefill.capture(small_model, tokens[:, :n_prompt], max_decode_steps=steps)
    decoded = []
    for step in range(steps):
        logits = runtime.replay(tokens[:, n_prompt + step:n_prompt + step + 1])
        decoded.append(logits[0, 0].float().cpu().clone())
    torch.cuda.synchronize()
    assert runtime.cache_position == n_prompt + steps
    assert runtime.device_error() == 0
    # Decode step s fed token n_prompt + s, so its logits are the prefill logits of n_prompt + s + 1 tokens.
    for step in (0, steps - 1):
        length = n_prompt + step + 1
        reference = NativeSmolLM2Prefill.capture(small_model, tokens[:, :length], max_decode_steps=0)
        torch.cuda.synchronize()
        torch.testing.assert_close(decoded[step], reference.logits[0, 0].float().cpu(), atol=LOGIT_ATOL,
                                   rtol=LOGIT_RTOL, msg=lambda m: f"decode step {step} (attended {length}): {m}")
        if step == steps - 1:
            pos = length - 1
            for layer in range(30):
                torch.testing.assert_close(runtime.key_cache[layer, 0][:, pos].float().cpu(),
                                           reference.key_cache[layer, 0][:, pos].float().cpu(),
                                           rtol=KV_RTOL, atol=KV_ATOL)
                torch.testing.assert_close(runtime.value_cache[layer, 0][:, pos].float().cpu(),
                                           reference.value_cache[layer, 0][:, pos].float().cpu(),
                                           rtol=KV_RTOL, atol=KV_ATOL)
        del reference
        torch.cuda.empty_cache()


def test_wait_timeout_reports_error_and_invalid_tokens(small_model):
    """Failure handling, forced from the host: a zero bound on the fused kernel's
    cross-workgroup waits makes them give up at once (every kernel still exits normally).
    The launch reports token -1 for every step, the next runtime call raises a device error
    instead of returning plausible results, and prefill re-arms the runtime."""
    record = golden("small128.npz")
    prompt = torch.from_numpy(record["prompt"]).unsqueeze(0).cuda()
    n = len(record["tokens"])
    runtime = NativeSmolLM2Prefill.capture(small_model, prompt, max_decode_steps=n - 1)
    handle = runtime.native_object().decode
    first = runtime.generate_greedy(n).clone()
    torch.cuda.synchronize()
    assert first[0].cpu().numpy().tolist() == record["tokens"].tolist()
    runtime.prefill(prompt)
    handle.set_wait_limit(0)
    failed = runtime.generate_greedy(n).clone()
    torch.cuda.synchronize()
    assert failed[0, 1:].cpu().tolist() == [-1] * (n - 1)  # slot 0 is the prefill's token
    assert runtime.device_error() == 1
    with pytest.raises(RuntimeError, match="device-side error 1"):
        runtime.replay(torch.tensor([[int(record["tokens"][0])]], device="cuda"))
    # An unbounded wait is refused before it reaches the runtime (no launch), so every
    # cross-workgroup wait stays bounded.
    with pytest.raises(RuntimeError, match="FLUX_MAX_WAIT_TICKS"):
        handle.set_wait_limit(2**64 - 1)
    with pytest.raises(RuntimeError, match="FLUX_MAX_WAIT_TICKS"):
        handle.set_wait_limit(1_000_000_001)
    handle.set_wait_limit(20_000_000)
    runtime.prefill(prompt)
    again = runtime.generate_greedy(n).clone()
    torch.cuda.synchronize()
    assert again[0].cpu().numpy().tolist() == record["tokens"].tolist()
    assert runtime.device_error() == 0
