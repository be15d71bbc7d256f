"""CPU oracle for the SmolLM2 FP32 batch-1 token loop -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of the reference FP32 path
(Hugging Face ``LlamaForCausalLM`` eager, which Flux validates against:
``/root/reference/tests/test_system.py:356-415,455-497``) and the per-kernel
closed forms the reference's own kernel tests use.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import it, and only as the checker (or, for the baseline, the thing timed on
the CPU).  The HIP product path never imports, links or calls anything here.

Pinning (what checks each function; see ``tests/test_oracle.py``):

* ``llama_fp32.OracleLlama`` -- committed golden vectors written by
  ``tests/golden/make_golden.py`` from transformers 5.15.0 ``LlamaForCausalLM``
  eager FP32 (token streams, logit slices, K/V slices, RoPE table hashes).
* ``kernels.rmsnorm`` / ``residual_rmsnorm`` -- hand-verifiable known answer
  (``[3,4]``, ``w=[2,.5]``, ``eps=0`` -> ``[6/sqrt(12.5), 2/sqrt(12.5)]``, the
  case of ``csrc/rmsnorm/test_rmsnorm.cpp:33-44``), HF ``LlamaRMSNorm`` fixtures,
  and the reference's own C++ CPU implementation built into ``oracle/_ref``.
* ``kernels.rope_rows`` -- bit-exact against HF ``apply_rotary_pos_emb``
  fixtures; cos=1/sin=0 identity.
* ``kernels.gqa_decode_attention`` -- brute-force per-head loop, zero-query ->
  mean-of-V closed form, single-position -> V row.
* ``kernels.greedy_argmax`` -- ties to lowest index, NaN-is-max, all -inf -> 0
  (cases of ``csrc/tests/test_greedy_generation.cu:46-103``).
* ``kernels.causal_attention`` -- zero query -> prefix mean of V; row 0 -> the
  V row of key 0; every checked row t equals ``gqa_decode_attention`` over the
  prefix [0, t] (itself checked against ``torch.softmax`` with repeat_kv), which
  fixes the scale, the mask and the head grouping; a planted scale mistake fails.
"""
