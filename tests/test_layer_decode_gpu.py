"""NativeSmolLM2LayerDecode (single decoder layer, replayable native step) against
the CPU oracle's LlamaDecoderLayer, through the C ABI.

Mirrors the contract of the reference's torch.classes.flux.NativeSmolLM2LayerDecode
(csrc/native_decode_runtime/native_decode_runtime_cuda.cu:314-738): imported K/V
prefix, one cache row and one position per replay, optional hidden per replay,
synchronous reset, stable buffers and the fixed-capacity limit.  Hidden-state
tolerance: rtol/atol 1e-4; cache rows: the reference's rtol 2e-4 / atol 2e-5.
"""

from __future__ import annotations

import pytest
import torch

from flux_amd import synthetic
from flux_amd.runtime import NativeSmolLM2LayerDecode
from oracle.llama_fp32 import OracleCache, OracleConfig, OracleLlama, rope_cos_sin, rope_table

pytestmark = pytest.mark.gpu

LAYER = 3


@pytest.fixture(scope="module")
def layer_setup(gpu_device):
    state = synthetic.synthetic_state_dict(synthetic.SyntheticSpec(seed=41, vocab=128))
    g = torch.Generator().manual_seed(17)
    p = f"model.layers.{LAYER}."
    for name in ("input_layernorm.weight", "post_attention_layernorm.weight"):
        state[p + name] = 1.0 + 0.1 * torch.randn(576, generator=g)
    oracle = OracleLlama(state)
    w = {
        "input_norm": state[p + "input_layernorm.weight"],
        "qkv": torch.cat([state[p + f"self_attn.{n}_proj.weight"] for n in "qkv"], dim=0),
        "o_proj": state[p + "self_attn.o_proj.weight"],
        "post_norm": state[p + "post_attention_layernorm.weight"],
        "gate_up": torch.cat([state[p + "mlp.gate_proj.weight"], state[p + "mlp.up_proj.weight"]], dim=0),
        "down": state[p + "mlp.down_proj.weight"],
    }
    w = {k: v.contiguous().to(gpu_device) for k, v in w.items()}
    return oracle, w


def _runtime(layer_setup, device, capacity, position, hidden, keys, values):
    _, w = layer_setup
    cos, sin = rope_table(OracleConfig(), capacity)
    return NativeSmolLM2LayerDecode(hidden, w["input_norm"], w["qkv"], w["o_proj"], w["post_norm"], w["gate_up"],
                                    w["down"], cos.contiguous().to(device), sin.contiguous().to(device), keys, values,
                                    capacity, position, 1e-5, 64 ** -0.5)


def _oracle_step(oracle, cache, hidden, position):
    cos, sin = rope_cos_sin(oracle.config, torch.tensor([[position]]))
    return oracle.decoder_layer(LAYER, hidden.cpu(), cos, sin, cache, None)


@pytest.mark.parametrize("position,capacity", [(37, 64), (0, 40), (700, 1024)])
def test_layer_steps_match_oracle(layer_setup, gpu_device, position, capacity):
    oracle, _ = layer_setup
    g = torch.Generator().manual_seed(position)
    keys = torch.randn(1, 3, position + 5, 64, generator=g)
    values = torch.randn(1, 3, position + 5, 64, generator=g)
    hiddens = [torch.randn(1, 1, 576, generator=g) for _ in range(6)]
    runtime = _runtime(layer_setup, gpu_device, capacity, position, hiddens[0].to(gpu_device), keys.to(gpu_device),
                       values.to(gpu_device))
    assert runtime.position() == runtime.cache_length() == position
    addresses = runtime.stable_addresses()
    cache = OracleCache()
    cache.keys = [None] * LAYER + [keys[:, :, :position]]
    cache.values = [None] * LAYER + [values[:, :, :position]]
    first = None
    for step, hidden in enumerate(hiddens):
        out = runtime.replay(hidden.to(gpu_device) if step else None)
        torch.cuda.synchronize()
        expected = _oracle_step(oracle, cache, hidden, position + step)
        torch.testing.assert_close(out.cpu(), expected, rtol=1e-4, atol=1e-4)
        row = position + step
        torch.testing.assert_close(runtime.key_cache()[:, :, row].cpu(), cache.keys[LAYER][:, :, row], rtol=2e-4,
                                   atol=2e-5)
        torch.testing.assert_close(runtime.value_cache()[:, :, row].cpu(), cache.values[LAYER][:, :, row],
                                   rtol=2e-4, atol=2e-5)
        if step == 0:
            first = out.clone()
    # The imported prefix is untouched and the rows past the written ones are zero.
    assert torch.equal(runtime.key_cache()[:, :, :position].cpu(), keys[:, :, :position])
    assert torch.count_nonzero(runtime.key_cache()[:, :, position + len(hiddens):]) == 0
    assert runtime.position() == position + len(hiddens)
    assert runtime.replay_count() == len(hiddens)
    assert runtime.stable_addresses() == addresses
    # replay() without a hidden reuses the last installed input.
    again = runtime.replay().clone()
    torch.cuda.synchronize()
    expected = _oracle_step(oracle, cache, hiddens[-1], position + len(hiddens))
    torch.testing.assert_close(again.cpu(), expected, rtol=1e-4, atol=1e-4)
    # reset restores hidden, cache and position; the first step repeats bit for bit.
    runtime.reset(hiddens[0].to(gpu_device), keys.to(gpu_device), values.to(gpu_device), position)
    assert runtime.position() == position and runtime.replay_count() == 0
    assert torch.count_nonzero(runtime.output()) == 0
    assert torch.equal(runtime.replay(), first)


def test_layer_capacity_and_validation(layer_setup, gpu_device):
    g = torch.Generator().manual_seed(3)
    hidden = torch.randn(1, 1, 576, generator=g).to(gpu_device)
    keys = torch.randn(1, 3, 10, 64, generator=g).to(gpu_device)
    runtime = _runtime(layer_setup, gpu_device, 12, 10, hidden, keys, keys.clone())
    runtime.replay()
    runtime.replay()
    with pytest.raises(RuntimeError, match="fixed-capacity state is exhausted"):
        runtime.replay()
    assert runtime.position() == 12
    with pytest.raises(RuntimeError, match="reset position must be inside cache capacity"):
        runtime.reset(hidden, keys, keys.clone(), 12)
    with pytest.raises(RuntimeError, match=r"\[1, 3, sequence>=position, 64\]"):
        runtime.reset(hidden, keys[:, :, :5], keys[:, :, :5].clone(), 8)
    with pytest.raises(RuntimeError, match="replay hidden state has shape"):
        runtime.replay(hidden[..., :-1])
    with pytest.raises(RuntimeError, match="initial position must be inside cache capacity"):
        _runtime(layer_setup, gpu_device, 12, 12, hidden, keys, keys.clone())
    with pytest.raises(RuntimeError, match="rope_cos has shape"):
        _, w = layer_setup
        cos, sin = rope_table(OracleConfig(), 12)
        NativeSmolLM2LayerDecode(hidden, w["input_norm"], w["qkv"], w["o_proj"], w["post_norm"], w["gate_up"],
                                 w["down"], cos[:11].contiguous().to(gpu_device), sin.contiguous().to(gpu_device),
                                 keys, keys.clone(), 12, 0, 1e-5, 0.125)
    runtime.reset(hidden, keys, keys.clone(), 3)
    assert runtime.position() == 3
    assert runtime.workspace_bytes() > 0 and runtime.workspace().numel() * 4 == runtime.workspace_bytes()
    # Every replay above was one launch of the fused kernel's single-layer step on one stream.
    assert runtime.replay_launches() == (2, 2)


def test_layer_step_reads_hidden_in_stream_order(layer_setup, gpu_device):
    """A step reads the caller's hidden state itself (no copy): its output feeds the next
    step directly (the output buffer is read and rewritten by the same step), and a caller
    buffer rewritten on the same stream after replay() does not change the step that
    reads it.  Every output equals the oracle's chained decoder-layer steps."""
    oracle, _ = layer_setup
    g = torch.Generator().manual_seed(5)
    position = 21
    keys = torch.randn(1, 3, position, 64, generator=g)
    values = torch.randn(1, 3, position, 64, generator=g)
    first = torch.randn(1, 1, 576, generator=g)
    runtime = _runtime(layer_setup, gpu_device, 64, position, first.to(gpu_device), keys.to(gpu_device),
                       values.to(gpu_device))
    cache = OracleCache()
    cache.keys = [None] * LAYER + [keys]
    cache.values = [None] * LAYER + [values]
    hidden = first
    scratch = first.to(gpu_device).clone()
    for step in range(6):
        if step % 2 == 0:
            out = runtime.replay(scratch)
            scratch.fill_(float("nan"))  # stream-ordered after the step that reads it
        else:
            out = runtime.replay(runtime.output())
        expected = _oracle_step(oracle, cache, hidden, position + step)
        torch.cuda.synchronize()
        torch.testing.assert_close(out.cpu(), expected, rtol=1e-4, atol=1e-4)
        hidden = expected
        if step % 2 == 1:
            scratch.copy_(out)
    assert runtime.position() == position + 6
    assert runtime.replay_launches() == (6, 6)
