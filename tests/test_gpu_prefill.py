"""The prefill attention kernel (starkv_prefill_attention) against the float64 causal
attention oracle, on the same inputs (fp16 K and V, q in bf16 / fp16 / fp32).

Cases: prompts of 1 token, lengths around the 64-key tile and 128-row block edges,
several prompts in one call (each attends to itself only), an empty prompt between
others, GQA groups 1 / 2 / 4 / 8, a long prompt, strided q and output. Tolerance: the
decode tolerance (max-abs <= 2e-2, mean |out - round(truth)| / mean |truth| <= 1e-3):
the kernel takes q in fp16 and rounds P to fp16 before P @ V, with fp32 accumulation.
"""
import numpy as np
import pytest
import torch

from oracle import ref
from starkv_serve.kernels.prefill import prefill_attention
from test_gpu_decode import assert_close

pytestmark = pytest.mark.gpu

D = 128


def _case(lengths, Hq, Hkv, seed, q_dtype=torch.bfloat16, peaked=1.0):
    g = torch.Generator().manual_seed(seed)
    T = sum(lengths)
    q = (torch.randn(T, Hq, D, generator=g) * peaked).to(q_dtype)
    k = torch.randn(T, Hkv, D, generator=g).to(torch.float16)
    v = torch.randn(T, Hkv, D, generator=g).to(torch.float16)
    return q, k, v


def _truth(q, k, v, lengths, scale):
    qsl = np.concatenate([[0], np.cumsum(lengths)])
    return ref.causal_attention(q.double().numpy(), k.double().numpy(), v.double().numpy(), qsl, scale)


CASES = {
    # name: (lengths, Hq, Hkv, q dtype)
    "one_token": ([1], 32, 32, torch.bfloat16),
    "tile_edges": ([63, 64, 65], 8, 8, torch.bfloat16),
    "block_edges": ([127, 128, 129, 255, 256, 257], 4, 2, torch.bfloat16),
    "ragged_gqa4": ([300, 17, 1000, 5], 32, 8, torch.bfloat16),
    "gqa8_fp16": ([200, 333], 16, 2, torch.float16),
    "fp32_query": ([150, 40], 8, 4, torch.float32),
    "empty_prompt": ([5, 0, 77, 0], 4, 4, torch.bfloat16),
    "long": ([2500], 4, 1, torch.bfloat16),
    "gqa3": ([90, 200], 6, 2, torch.bfloat16),
}


@pytest.mark.parametrize("name", list(CASES))
def test_prefill_vs_oracle(cuda, name):
    lengths, Hq, Hkv, qdt = CASES[name]
    scale = D ** -0.5
    q, k, v = _case(lengths, Hq, Hkv, seed=sum(map(ord, name)), q_dtype=qdt)
    out = prefill_attention(q.to(cuda), k.to(cuda), v.to(cuda), lengths, scale)
    torch.cuda.synchronize()
    assert out.dtype == qdt
    assert_close(out, _truth(q, k, v, lengths, scale), f"prefill {name}")


def test_prefill_peaked_softmax(cuda):
    """Large logits (q x 8): the running max moves often and far."""
    lengths = [400, 90]
    scale = D ** -0.5
    q, k, v = _case(lengths, 8, 4, seed=5, peaked=8.0)
    out = prefill_attention(q.to(cuda), k.to(cuda), v.to(cuda), lengths, scale)
    torch.cuda.synchronize()
    assert_close(out, _truth(q, k, v, lengths, scale), "prefill peaked")


def test_prefill_strided_query_and_output(cuda):
    """q and out as head slices of wider rows (element strides, 16-byte aligned)."""
    lengths, Hq, Hkv = [130, 7], 4, 2
    T = sum(lengths)
    scale = 0.1
    q, k, v = _case(lengths, Hq, Hkv, seed=9)
    wide_q = torch.zeros(T, Hq + 2, D, dtype=q.dtype)
    wide_q[:, 1:1 + Hq] = q
    wide_o = torch.full((T, Hq + 3, D), float("nan"), dtype=q.dtype, device=cuda)
    out = prefill_attention(wide_q.to(cuda)[:, 1:1 + Hq], k.to(cuda), v.to(cuda), lengths, scale,
                            out=wide_o[:, 2:2 + Hq])
    torch.cuda.synchronize()
    assert_close(out, _truth(q, k, v, lengths, scale), "prefill strided")
    assert torch.isnan(wide_o[:, :2]).all() and torch.isnan(wide_o[:, 2 + Hq:]).all()  # nothing else written


def test_prefill_bf16_kv_converted(cuda):
    """K and V handed over in bf16 are converted to fp16 once (exact for these values)."""
    lengths = [70]
    q, k, v = _case(lengths, 4, 4, seed=3)
    kb, vb = k.to(torch.bfloat16), v.to(torch.bfloat16)
    out = prefill_attention(q.to(cuda), kb.to(cuda), vb.to(cuda), lengths, 0.08)
    torch.cuda.synchronize()
    assert_close(out, _truth(q, kb.half(), vb.half(), lengths, 0.08), "prefill bf16 kv")
