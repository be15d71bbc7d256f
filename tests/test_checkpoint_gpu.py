"""The native token loop on a model restored from a local checkpoint.

Mirrors the reference's checkpoint round trip (tests/test_system.py:191-207; the
unpack/pack state-dict hooks are flux/model/smollm2_flux.py:167-214,339-391): a
Flux-enabled model is written with ``save_pretrained`` and read back with
``LlamaForCausalLM.from_pretrained(path, local_files_only=True)``.  Here the restored
model then drives the native prefill and the fused decode runtime on the GPU, which
must reproduce the config-1 golden stream (HF eager FP32 on the CPU) exactly, with
the golden logits at every step.
"""

from __future__ import annotations

import pytest
import torch
from transformers import LlamaForCausalLM

from flux_amd.model import FINAL_FLUX_OPERATOR_CATEGORIES, enable_flux_ops
from flux_amd.runtime import NativeSmolLM2Prefill
from tests.conftest import golden
from tests.test_runtime_gpu import _check_kv, _replay_stream

pytestmark = pytest.mark.gpu


def test_native_path_on_a_locally_restored_checkpoint(smol_model, tmp_path):
    record = golden("config1.npz")
    expected_state = {k: v.detach().cpu().clone() for k, v in smol_model.state_dict().items()}
    assert not any("packed_qkv" in k or "gate_up_proj" in k for k in expected_state)
    smol_model.save_pretrained(tmp_path, safe_serialization=True)

    restored = LlamaForCausalLM.from_pretrained(tmp_path, local_files_only=True, attn_implementation="eager",
                                                dtype=torch.float32)
    assert set(restored.state_dict()) == set(expected_state)
    for name, value in restored.state_dict().items():
        assert torch.equal(value, expected_state[name]), name
    restored = restored.to("cuda:0").eval()
    enable_flux_ops(restored, operators=FINAL_FLUX_OPERATOR_CATEGORIES)
    layer = restored.model.layers[0]
    assert torch.equal(layer.self_attn.packed_qkv.weight, smol_model.model.layers[0].self_attn.packed_qkv.weight)
    assert torch.equal(layer.mlp.gate_up_proj.weight, smol_model.model.layers[0].mlp.gate_up_proj.weight)

    prompt = torch.from_numpy(record["prompt"]).unsqueeze(0).cuda()
    n = len(record["tokens"])
    runtime = NativeSmolLM2Prefill.capture(restored, prompt, max_decode_steps=n - 1)
    torch.cuda.synchronize()
    _check_kv(runtime, record)
    _replay_stream(runtime, record, record["tokens"].tolist(), n)
    runtime.prefill(prompt)
    generated = runtime.generate_greedy(n).clone()
    torch.cuda.synchronize()
    assert generated[0].cpu().numpy().tolist() == record["tokens"].tolist()
    assert runtime.device_error() == 0
