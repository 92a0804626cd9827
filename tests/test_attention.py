"""The backend's per-layer implementation, host side (no GPU): the constructor's
checks and errors (attention.py:106-119), the operands ``to_device`` builds
(attention.py:134-166), the profiling-run and prefill paths of ``forward``."""
import types

import pytest
import torch

from starkv_serve import checkpoint as ck
from starkv_serve.attention import StarKVAttentionImpl, StarKVMetadata

RANKS = [16, 32, 48, 64]


@pytest.fixture(scope="module")
def layers(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("ck") / "fused_weights.pt")
    ck.write_fused_checkpoint(path, 2, len(RANKS), 128, 256, {0: (RANKS, 40), 1: (RANKS, 32)}, seed=1)
    bf = ck.load_fused_checkpoint(path, 2, len(RANKS), 128, dtype=torch.bfloat16, kv_quant=False).layers[0]
    q4 = ck.load_fused_checkpoint(path, 2, len(RANKS), 128, dtype=torch.bfloat16, kv_quant=True).layers[1]
    return bf, q4


def _impl(w, num_heads=8, num_kv_heads=4, **kw):
    rope = types.SimpleNamespace(cos_sin_cache=torch.zeros(64, 128))
    kw.setdefault("max_model_len", 1024)
    return StarKVAttentionImpl(num_heads, 128, 128 ** -0.5, num_kv_heads, starkv_layer=w, rotary_emb=rope, **kw)


@pytest.mark.parametrize("kw,msg", [
    (dict(alibi_slopes=[1.0]), "alibi"), (dict(sliding_window=128), "sliding window"),
    (dict(logits_soft_cap=30.0), "softcap"), (dict(attn_type="encoder"), "decoder self-attention"),
    (dict(kv_sharing_target_layer_name="x"), "decoder self-attention"), (dict(kv_cache_dtype="fp8"), "kv_cache_dtype"),
])
def test_unsupported_configurations_raise(layers, kw, msg):
    with pytest.raises(NotImplementedError, match=msg):
        _impl(layers[0], **kw)


def test_quant_cache_needs_mha_head_dim_128(layers):
    _impl(layers[1], num_heads=4, num_kv_heads=4)
    with pytest.raises(NotImplementedError, match="MHA"):
        _impl(layers[1], num_heads=8, num_kv_heads=4)


def test_max_model_len_required_without_vllm(layers):
    with pytest.raises(ValueError, match="max_model_len"):
        _impl(layers[0], max_model_len=None)


@pytest.mark.parametrize("quant", [False, True])
def test_to_device_operands(layers, quant):
    w = layers[1] if quant else layers[0]
    H = 4 if quant else 8
    impl = _impl(w, num_heads=H, num_kv_heads=4)
    impl.to_device(torch.device("cpu"), torch.bfloat16)
    assert impl.k_width == w.k_width
    assert impl.k_up.shape == (w.k_width, 128) and impl.k_up.dtype == torch.bfloat16
    assert impl.v_up_by_q.shape == (H, w.v_rank, 128)
    assert impl.kv_down.shape == (w.k_width + w.v_rank, 256)
    # query head h reads KV head h // (H / Hkv): its V basis, transposed
    g = H // 4
    for h in range(H):
        kv = h // g
        want = w.v_up[kv * 128:(kv + 1) * 128].to(torch.bfloat16).T
        assert torch.equal(impl.v_up_by_q[h], want)
    assert (impl.row is not None) == quant
    if quant:
        assert impl.row.nbytes % 16 == 0 and impl.k_nouts.numel() == 4


def _md(n_dec, n_pre, prompt=1, cached=0):
    """n_dec decodes, then n_pre prompts of `prompt` tokens each with `cached` tokens of
    context already in the cache."""
    T = n_dec + n_pre * prompt
    lens = [1] * n_dec + [prompt + cached] * n_pre
    return StarKVMetadata(num_actual_tokens=T, num_decodes=n_dec, num_decode_tokens=n_dec, num_prefills=n_pre,
                          max_seq_len=10, seq_lens=torch.tensor(lens, dtype=torch.int32),
                          block_table=torch.zeros(n_dec + n_pre, 1, dtype=torch.int32),
                          slot_mapping=torch.zeros(T, dtype=torch.int64),
                          prefill_seq_lens_cpu=[prompt + cached] * n_pre,
                          prefill_query_start_loc_cpu=[prompt * i for i in range(n_pre + 1)])


def test_forward_profiling_run_and_rejections(layers):
    impl = _impl(layers[0])
    out = torch.full((3, 8 * 128), 5.0)
    assert impl.forward(None, out, out, out, out, None, out) is out
    assert not out.any()
    # Chunked prompts / cached context: raised before any work is enqueued (CPU tensors here).
    with pytest.raises(NotImplementedError, match="every prompt in one step"):
        impl.forward(None, out, out, out, out, _md(1, 1, prompt=2, cached=3), out)
    with pytest.raises(NotImplementedError, match="output quantization"):
        impl.forward(None, out, out, out, out, _md(3, 0), out, output_scale=1.0)


def test_decode_lens_formed_once_per_step():
    """Padding rows (length 0) get one position; the clamped lengths are formed once per
    step and shared by every layer's decode."""
    md = StarKVMetadata(num_actual_tokens=3, num_decodes=3, num_decode_tokens=3, num_prefills=0, max_seq_len=9,
                        seq_lens=torch.tensor([5, 0, 9, 7], dtype=torch.int32),
                        block_table=torch.zeros(4, 1, dtype=torch.int32),
                        slot_mapping=torch.zeros(3, dtype=torch.int64))
    a = md.decode_lens(3)
    assert a.tolist() == [5, 1, 9] and a.dtype == torch.int32
    assert md.decode_lens(3) is a
    assert md.decode_lens(2).tolist() == [5, 1]


def test_decode_output_argument_checked():
    """`out=` of the decode wrappers: shape, dtype and layout are checked before any launch."""
    from starkv_serve import _hip
    fresh = _hip.output_for(None, (2, 4, 128), torch.bfloat16, "cpu")
    assert fresh.shape == (2, 4, 128) and fresh.dtype == torch.bfloat16
    ok = torch.empty(2, 4, 128, dtype=torch.float32)
    assert _hip.output_for(ok, (2, 4, 128), torch.bfloat16, "cpu") is ok
    with pytest.raises(ValueError, match="shape"):
        _hip.output_for(torch.empty(2, 5, 128), (2, 4, 128), torch.bfloat16, "cpu")
    with pytest.raises(ValueError, match="dtype"):
        _hip.output_for(torch.empty(2, 4, 128, dtype=torch.int32), (2, 4, 128), torch.bfloat16, "cpu")
    with pytest.raises(ValueError, match="contiguous"):
        _hip.output_for(torch.empty(2, 128, 4).transpose(1, 2), (2, 4, 128), torch.bfloat16, "cpu")
