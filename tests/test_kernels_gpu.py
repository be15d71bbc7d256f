"""Isolated gfx950 kernels vs the CPU oracle (float64 closed forms) through the C ABI.

Mirrors the reference's kernel tests: csrc/tests/test_decode_ops.cu (QKV/RoPE/cache,
GQA decode, gate/up), test_greedy_generation.cu (argmax KATs),
test_streaming_prefill_gqa.cu (prefill attention), csrc/rmsnorm|residual_rmsnorm tests.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from flux_amd import _native
from oracle import kernels as ref
from oracle.llama_fp32 import OracleConfig, rope_table

pytestmark = pytest.mark.gpu

H, I, D = 576, 1536, 64


def _lib():
    return _native.load()


def _s(dev):
    return _native.current_stream(dev)


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _randn(*shape, seed, std=1.0):
    return (torch.randn(*shape, generator=_gen(seed)) * std).float()


def _close(actual: torch.Tensor, expected: torch.Tensor, rtol: float, atol: float):
    torch.testing.assert_close(actual.detach().cpu().double(), expected.detach().cpu().double(), rtol=rtol, atol=atol)


def test_rmsnorm_kat_and_rows(gpu_device):
    # Hand KAT of csrc/rmsnorm/test_rmsnorm.cpp:33-44 (eps tiny): [3,4], w=[2,.5].
    x = torch.tensor([[3.0, 4.0]], device=gpu_device)
    w = torch.tensor([2.0, 0.5], device=gpu_device)
    out = torch.empty_like(x)
    _native.check(_lib().flux_rmsnorm_f32(x.data_ptr(), w.data_ptr(), out.data_ptr(), 1, 2, 1e-30, _s(gpu_device)))
    torch.cuda.synchronize()
    expected = torch.tensor([[6.0 / 12.5 ** 0.5, 2.0 / 12.5 ** 0.5]])
    _close(out, expected, rtol=1e-6, atol=1e-7)
    for rows in (1, 7, 300):
        x = _randn(rows, H, seed=rows).to(gpu_device)
        w = _randn(H, seed=rows + 1).to(gpu_device)
        out = torch.empty_like(x)
        _native.check(_lib().flux_rmsnorm_f32(x.data_ptr(), w.data_ptr(), out.data_ptr(), rows, H, 1e-5,
                                              _s(gpu_device)))
        torch.cuda.synchronize()
        _close(out, ref.rmsnorm(x.cpu(), w.cpu(), 1e-5), rtol=1e-5, atol=2e-6)


def test_residual_rmsnorm_exact_residual(gpu_device):
    rows = 5
    h = _randn(rows, H, seed=3).to(gpu_device)
    r = _randn(rows, H, seed=4).to(gpu_device)
    w = _randn(H, seed=5).to(gpu_device)
    norm = torch.empty_like(h)
    res = torch.empty_like(h)
    _native.check(_lib().flux_residual_rmsnorm_f32(h.data_ptr(), r.data_ptr(), w.data_ptr(), norm.data_ptr(),
                                                   res.data_ptr(), rows, H, 1e-5, _s(gpu_device)))
    torch.cuda.synchronize()
    expected_norm, expected_res = ref.residual_rmsnorm(h.cpu(), r.cpu(), w.cpu(), 1e-5)
    assert torch.equal(res.cpu(), expected_res)  # exact FP32 sum
    _close(norm, expected_norm, rtol=1e-5, atol=2e-6)


def _qkv_case(gpu_device, capacity, position, cos_one=False):
    hidden = _randn(H, seed=11).to(gpu_device)
    norm_w = (1.0 + 0.1 * _randn(H, seed=12)).to(gpu_device)
    qkv_w = _randn(960, H, seed=13, std=0.02).to(gpu_device)
    cos, sin = rope_table(OracleConfig(), capacity)
    if cos_one:
        cos, sin = torch.ones_like(cos), torch.zeros_like(sin)
    cos_d, sin_d = cos.to(gpu_device), sin.to(gpu_device)
    pos = torch.tensor([position], dtype=torch.long, device=gpu_device)
    kc = torch.full((3, capacity, D), 7.0, device=gpu_device)
    vc = torch.full((3, capacity, D), 7.0, device=gpu_device)
    q = torch.empty(9, D, device=gpu_device)
    _native.check(_lib().flux_qkv_rope_cache_f32(hidden.data_ptr(), norm_w.data_ptr(), 1e-5, qkv_w.data_ptr(),
                                                 cos_d.data_ptr(), sin_d.data_ptr(), pos.data_ptr(), capacity,
                                                 kc.data_ptr(), vc.data_ptr(), q.data_ptr(), _s(gpu_device)))
    torch.cuda.synchronize()
    eq, ek, ev = ref.qkv_rope_cache(hidden.cpu(), norm_w.cpu(), 1e-5, qkv_w.cpu(), cos[position], sin[position])
    return q.cpu(), kc.cpu(), vc.cpu(), eq, ek, ev


@pytest.mark.parametrize("capacity,position", [(257, 0), (257, 192), (8704, 8703)])
def test_qkv_rope_cache_matches_oracle(gpu_device, capacity, position):
    q, kc, vc, eq, ek, ev = _qkv_case(gpu_device, capacity, position)
    _close(q, eq, rtol=1e-4, atol=1e-5)
    _close(kc[:, position], ek, rtol=1e-4, atol=1e-5)
    _close(vc[:, position], ev, rtol=1e-4, atol=1e-5)
    # Only row `position` is written.
    untouched = torch.ones(capacity, dtype=torch.bool)
    untouched[position] = False
    assert torch.all(kc[:, untouched] == 7.0) and torch.all(vc[:, untouched] == 7.0)


def test_qkv_rope_identity_kat(gpu_device):
    # cos=1, sin=0 -> q is the plain projection (csrc/benchmarks/cuda_microbenchmarks.cu:315-360).
    q, kc, vc, eq, ek, ev = _qkv_case(gpu_device, 64, 5, cos_one=True)
    _close(q, eq, rtol=1e-4, atol=1e-5)
    # V is never rotated: same projection with or without RoPE.
    _close(vc[:, 5], ev, rtol=1e-4, atol=1e-5)


def _gqa(gpu_device, q, kc, vc, capacity, position, scale=0.125):
    ws_bytes = ctypes.c_int64()
    _native.check(_lib().flux_gqa_decode_workspace_bytes(capacity, ctypes.byref(ws_bytes)))
    ws = torch.empty(ws_bytes.value // 4, device=gpu_device)
    out = torch.empty(9, D, device=gpu_device)
    pos = torch.tensor([position], dtype=torch.long, device=gpu_device)
    _native.check(_lib().flux_gqa_decode_attention_f32(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(),
                                                       capacity, scale, ws.data_ptr(), ws_bytes.value,
                                                       out.data_ptr(), _s(gpu_device)))
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("capacity,length", [(257, 193), (257, 1), (8192, 8192), (16384, 16384), (8704, 4097)])
def test_gqa_decode_matches_bruteforce(gpu_device, capacity, length):
    q = _randn(9, D, seed=21).to(gpu_device)
    kc = _randn(3, capacity, D, seed=22).to(gpu_device)
    vc = _randn(3, capacity, D, seed=23).to(gpu_device)
    out = _gqa(gpu_device, q, kc, vc, capacity, length - 1)
    expected = ref.gqa_decode_attention(q.cpu(), kc.cpu(), vc.cpu(), length, 0.125)
    _close(out, expected, rtol=3e-4, atol=3e-5)  # tolerance of test_decode_ops.cu:158-250


def test_gqa_decode_zero_query_is_mean_of_values(gpu_device):
    capacity, length = 1000, 777
    q = torch.zeros(9, D, device=gpu_device)
    kc = _randn(3, capacity, D, seed=31).to(gpu_device)
    vc = _randn(3, capacity, D, seed=32).to(gpu_device)
    out = _gqa(gpu_device, q, kc, vc, capacity, length - 1)
    mean = vc[:, :length].double().mean(dim=1).cpu()
    expected = mean.repeat_interleave(3, dim=0)
    _close(out, expected, rtol=1e-5, atol=1e-6)


def test_gate_up_swiglu_and_down(gpu_device):
    x = _randn(H, seed=41).to(gpu_device)
    gu = _randn(2 * I, H, seed=42, std=0.02).to(gpu_device)
    out = torch.empty(I, device=gpu_device)
    _native.check(_lib().flux_gate_up_swiglu_f32(x.data_ptr(), None, 0.0, gu.data_ptr(), out.data_ptr(),
                                                 _s(gpu_device)))
    torch.cuda.synchronize()
    _close(out, ref.gate_up_swiglu(x.cpu(), gu.cpu()), rtol=5e-4, atol=2e-5)  # test_decode_ops.cu:252-287
    # With the fused post-attention norm.
    w = (1.0 + 0.1 * _randn(H, seed=43)).to(gpu_device)
    _native.check(_lib().flux_gate_up_swiglu_f32(x.data_ptr(), w.data_ptr(), 1e-5, gu.data_ptr(), out.data_ptr(),
                                                 _s(gpu_device)))
    torch.cuda.synchronize()
    xn = ref.rmsnorm(x.cpu(), w.cpu(), 1e-5)
    _close(out, ref.gate_up_swiglu(xn, gu.cpu()), rtol=5e-4, atol=2e-5)
    s = _randn(I, seed=44).to(gpu_device)
    dw = _randn(H, I, seed=45, std=0.02).to(gpu_device)
    resid = _randn(H, seed=46).to(gpu_device)
    o = torch.empty(H, device=gpu_device)
    _native.check(_lib().flux_down_residual_f32(s.data_ptr(), dw.data_ptr(), resid.data_ptr(), o.data_ptr(),
                                                _s(gpu_device)))
    torch.cuda.synchronize()
    _close(o, resid.cpu().double() + dw.cpu().double() @ s.cpu().double(), rtol=1e-5, atol=1e-5)
    # o_proj GEMV with residual.
    ow = _randn(H, H, seed=47, std=0.02).to(gpu_device)
    _native.check(_lib().flux_linear576_f32(x.data_ptr(), ow.data_ptr(), resid.data_ptr(), o.data_ptr(), H,
                                            _s(gpu_device)))
    torch.cuda.synchronize()
    _close(o, resid.cpu().double() + ow.cpu().double() @ x.cpu().double(), rtol=1e-5, atol=1e-5)


def _argmax(gpu_device, values):
    logits = torch.tensor(values, dtype=torch.float32, device=gpu_device)
    token = torch.full((1,), -5, dtype=torch.long, device=gpu_device)
    _native.check(_lib().flux_greedy_argmax_f32(logits.data_ptr(), logits.numel(), token.data_ptr(), _s(gpu_device)))
    torch.cuda.synchronize()
    return int(token.item())


def test_greedy_argmax_kats(gpu_device):
    # Cases of csrc/tests/test_greedy_generation.cu:46-103.
    v = [0.0] * 1000
    v[177] = v[321] = 5.0
    assert _argmax(gpu_device, v) == 177 == ref.greedy_argmax(np.asarray(v))
    v = [-1.0] * 64
    v[19] = v[27] = 2.0
    assert _argmax(gpu_device, v) == 19
    v = [0.0] * 49152
    v[0] = 1.0
    assert _argmax(gpu_device, v) == 0
    v[0] = 0.0
    v[49151] = 1.0
    assert _argmax(gpu_device, v) == 49151
    assert _argmax(gpu_device, [float("-inf")] * 300) == 0
    v = [1.0, float("nan"), 3.0, float("nan")]
    assert _argmax(gpu_device, v) == 1 == ref.greedy_argmax(np.asarray(v))


def test_greedy_argmax_update_state(gpu_device):
    logits = torch.zeros(32, device=gpu_device)
    logits[19] = 4.0
    token = torch.zeros(1, dtype=torch.long, device=gpu_device)
    generated = torch.full((8,), -1, dtype=torch.long, device=gpu_device)
    step = torch.tensor([2], dtype=torch.long, device=gpu_device)
    position = torch.tensor([3], dtype=torch.long, device=gpu_device)
    length = torch.tensor([9], dtype=torch.long, device=gpu_device)
    _native.check(_lib().flux_greedy_argmax_update_f32(logits.data_ptr(), 32, token.data_ptr(), generated.data_ptr(),
                                                       step.data_ptr(), 8, position.data_ptr(), length.data_ptr(),
                                                       _s(gpu_device)))
    torch.cuda.synchronize()
    assert token.item() == 19 and generated[2].item() == 19 and step.item() == 3 and position.item() == 9


@pytest.mark.parametrize("vocab", [128, 49152])
def test_lm_head_argmax(gpu_device, vocab):
    h = _randn(H, seed=51).to(gpu_device)
    w = (1.0 + 0.1 * _randn(H, seed=52)).to(gpu_device)
    lm = _randn(vocab, H, seed=53, std=0.02).to(gpu_device)
    logits = torch.empty(vocab, device=gpu_device)
    token = torch.empty(1, dtype=torch.long, device=gpu_device)
    ws_bytes = ctypes.c_int64()
    _native.check(_lib().flux_lm_head_workspace_bytes(ctypes.byref(ws_bytes)))
    ws = torch.empty(ws_bytes.value, dtype=torch.uint8, device=gpu_device)
    _native.check(_lib().flux_lm_head_argmax_f32(h.data_ptr(), w.data_ptr(), 1e-5, lm.data_ptr(), vocab,
                                                 logits.data_ptr(), token.data_ptr(), ws.data_ptr(), ws_bytes.value,
                                                 _s(gpu_device)))
    torch.cuda.synchronize()
    expected = lm.cpu().double() @ ref.rmsnorm(h.cpu(), w.cpu(), 1e-5)
    _close(logits, expected, rtol=1e-4, atol=1e-5)
    assert int(token.item()) == ref.greedy_argmax(logits.cpu().numpy())


@pytest.mark.parametrize("m,n,k", [(1, 64, 16), (70, 576, 48), (64, 192, 32), (16, 576, 576), (200, 576, 576),
                                   (130, 960, 576), (257, 576, 1536), (512, 576, 1536), (600, 1024, 576),
                                   (1200, 1024, 576), (1000, 576, 1536), (2048, 576, 1536), (300, 1024, 64),
                                   (300, 576, 64), (1024, 3072, 576)])
def test_mfma_linear(gpu_device, m, n, k):
    # k = 576 with at most 256 16-row tiles: the register kernel, 32 columns wide (16, 200 rows)
    # or 64 (130 rows).  Otherwise k = 576 or 1536 with at most 256 tiles: the split kernel, on
    # 32 x 32 tiles (257 rows), else on (32 RT) x 64 tiles with RT = 1 (512 rows), 2 (600 rows)
    # or 4 (1200 rows); widths that are not a multiple of 128 only with RT = 1. Otherwise those
    # widths take the 64 x 64 tile kernel when k % 32 == 0 (1000, 2048 rows), else the
    # 128-column kernel; grids under 256 blocks take their four-buffer ring variants (300 rows
    # with k = 64, 1000 rows, and the first three cases).
    a = _randn(m, k, seed=61).to(gpu_device)
    w = _randn(n, k, seed=62, std=0.05).to(gpu_device)
    r = _randn(m, n, seed=63).to(gpu_device)
    c = torch.empty(m, n, device=gpu_device)
    _native.check(_lib().flux_linear_f32(a.data_ptr(), w.data_ptr(), None, c.data_ptr(), m, n, k, _s(gpu_device)))
    torch.cuda.synchronize()
    expected = a.cpu().double() @ w.cpu().double().T
    _close(c, expected, rtol=1e-4, atol=1e-4)
    _native.check(_lib().flux_linear_f32(a.data_ptr(), w.data_ptr(), r.data_ptr(), c.data_ptr(), m, n, k,
                                         _s(gpu_device)))
    torch.cuda.synchronize()
    _close(c, expected + r.cpu().double(), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("rows", [1, 77, 300, 600])
def test_gate_up_swiglu_rows(gpu_device, rows):
    # 1 / 77: register kernel (16-row tiles), 300: split kernel with two 32-row tiles per block,
    # 600: four.
    x = _randn(rows, H, seed=71).to(gpu_device)
    gu = _randn(2 * I, H, seed=72, std=0.02).to(gpu_device)
    out = torch.empty(rows, I, device=gpu_device)
    _native.check(_lib().flux_gate_up_swiglu_rows_f32(x.data_ptr(), gu.data_ptr(), out.data_ptr(), rows,
                                                      _s(gpu_device)))
    torch.cuda.synchronize()
    g = x.cpu().double() @ gu.cpu().double()[:I].T
    u = x.cpu().double() @ gu.cpu().double()[I:].T
    _close(out, g / (1 + torch.exp(-g)) * u, rtol=5e-4, atol=2e-5)


@pytest.mark.parametrize("rows,capacity", [(1, 8), (129, 200), (512, 8704), (1900, 2048)])
def test_qkv_rope_cache_rows(gpu_device, rows, capacity):
    # 1 / 129 rows: register kernel (16-row tiles); 512: split kernel with one 32-row tile per
    # block; 1900: four per block.
    x = _randn(rows, H, seed=81).to(gpu_device)
    qkv = _randn(960, H, seed=82, std=0.02).to(gpu_device)
    cos, sin = rope_table(OracleConfig(), capacity)
    q = torch.empty(9, rows, D, device=gpu_device)
    kc = torch.zeros(3, capacity, D, device=gpu_device)
    vc = torch.zeros(3, capacity, D, device=gpu_device)
    cos_d, sin_d = cos.to(gpu_device), sin.to(gpu_device)  # keep alive across the async launch
    _native.check(_lib().flux_qkv_rope_cache_rows_f32(x.data_ptr(), qkv.data_ptr(), cos_d.data_ptr(),
                                                      sin_d.data_ptr(), rows, q.data_ptr(),
                                                      kc.data_ptr(), vc.data_ptr(), capacity, _s(gpu_device)))
    torch.cuda.synchronize()
    proj = x.cpu().double() @ qkv.cpu().double().T  # [rows, 960]
    half = 32

    def rope(t):  # t [rows, 64]
        rot = torch.cat((-t[:, half:], t[:, :half]), dim=-1)
        return t * cos[:rows].double() + rot * sin[:rows].double()

    for h in range(9):
        _close(q[h], rope(proj[:, 64 * h:64 * h + 64]), rtol=1e-4, atol=1e-4)
    for g in range(3):
        _close(kc[g, :rows], rope(proj[:, 576 + 64 * g:576 + 64 * g + 64]), rtol=1e-4, atol=1e-4)
        _close(vc[g, :rows], proj[:, 768 + 64 * g:768 + 64 * g + 64], rtol=1e-4, atol=1e-4)
    assert torch.all(kc[:, rows:] == 0) and torch.all(vc[:, rows:] == 0)


def _attention_workspace(seq, device):
    size = ctypes.c_int64()
    _native.check(_lib().flux_prefill_attention_workspace_bytes(seq, ctypes.byref(size)))
    return torch.empty(max(size.value // 4, 1), device=device)


@pytest.mark.parametrize("seq,capacity", [(1, 4), (63, 64), (64, 64), (65, 100), (200, 257), (300, 320),
                                          (512, 600), (513, 513), (1024, 1024), (1537, 1600), (2049, 2100),
                                          (3201, 3300), (4160, 4160)])
def test_prefill_attention_matches_oracle(gpu_device, seq, capacity):
    # Up to 512 tokens one block per 32-query tile and head spreads the tile's 32-key chunks
    # over 8 waves and combines them in LDS (300: some waves take two chunks, 512: every wave
    # of the last tiles).  From 513 on, keys are split into chunks of 2 (up to 1024 tokens)
    # to 16 (from about 4500 tokens on) 64-key tiles, and query tiles that see several
    # chunks take the split-key path and its merge (1024: 2-tile chunks, eight of them,
    # 3201: 10-tile chunks, six of them, and a one-query last tile).
    q = _randn(9, seq, D, seed=91).to(gpu_device)
    kc = _randn(3, capacity, D, seed=92).to(gpu_device)
    vc = _randn(3, capacity, D, seed=93).to(gpu_device)
    out = torch.empty(seq, H, device=gpu_device)
    ws = _attention_workspace(seq, gpu_device)
    _native.check(_lib().flux_prefill_attention_f32(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), seq, capacity, 0.125,
                                                    ws.data_ptr(), out.data_ptr(), _s(gpu_device)))
    torch.cuda.synchronize()
    expected = ref.causal_attention(q.cpu(), kc.cpu(), vc.cpu(), 0.125)  # [9, seq, 64]
    _close(out.view(seq, 9, D).transpose(0, 1), expected, rtol=2e-4, atol=2e-5)


@pytest.mark.parametrize("seq", [130, 16384])
def test_prefill_attention_zero_query_prefix_mean(gpu_device, seq):
    # Zero queries make every visible key equally likely, so row s is the mean of V[0..s]:
    # a closed form that pins the short-prompt kernel's in-block combine (130) and the
    # split-key merge at the largest capacity (16384).
    capacity = seq
    q = torch.zeros(9, seq, D, device=gpu_device)
    kc = _randn(3, capacity, D, seed=94).to(gpu_device)
    vc = _randn(3, capacity, D, seed=95).to(gpu_device)
    out = torch.empty(seq, H, device=gpu_device)
    ws = _attention_workspace(seq, gpu_device)
    _native.check(_lib().flux_prefill_attention_f32(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), seq, capacity, 0.125,
                                                    ws.data_ptr(), out.data_ptr(), _s(gpu_device)))
    torch.cuda.synchronize()
    prefix = vc.cpu().double().cumsum(dim=1) / torch.arange(1, capacity + 1).double()[None, :, None]
    expected = prefix[:, :seq].repeat_interleave(3, dim=0)
    _close(out.view(seq, 9, D).transpose(0, 1), expected, rtol=1e-5, atol=1e-6)


def test_embedding_gather(gpu_device):
    vocab = 100
    emb = _randn(vocab, H, seed=96).to(gpu_device)
    ids = torch.tensor([0, 5, 99, 100, -1, 7], dtype=torch.long, device=gpu_device)
    out = torch.empty(6, H, device=gpu_device)
    _native.check(_lib().flux_embedding_gather_f32(ids.data_ptr(), emb.data_ptr(), vocab, 6, out.data_ptr(),
                                                   _s(gpu_device)))
    torch.cuda.synchronize()
    expected = torch.zeros(6, H)
    for i, t in enumerate([0, 5, 99, 100, -1, 7]):
        if 0 <= t < vocab:
            expected[i] = emb.cpu()[t]
    assert torch.equal(out.cpu(), expected)
