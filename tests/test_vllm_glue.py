"""The serving glue around the attention backend, on the CPU: the metadata builder's
split of a step into decodes and prefills (attention.py:80-103 / vLLM's
split_decodes_and_prefills), the engine defaults and the --additional-config parse
(config.py:26-83), the cached checkpoint lookup, the KV-cache row bytes the backend
declares (attention.py:289-299), and the plugin's need for vLLM."""
from types import SimpleNamespace

import pytest
import torch

from starkv_serve import attention as A
from starkv_serve import checkpoint as ck
from starkv_serve import config as C
from starkv_serve import plugin
from starkv_serve.kernels.paged_quant import QuantRow


@pytest.mark.parametrize("qsl,tokens,want", [
    ([0, 1, 2, 3], 3, (3, 0, 3, 0)),                 # pure decode
    ([0, 1, 2, 9, 12], 12, (2, 2, 2, 10)),           # decodes first, then two prompts
    ([0, 5, 9], 9, (0, 2, 0, 9)),                    # prefill only
    ([0, 1, 1, 2, 30], 30, (3, 1, 2, 28)),           # a padding request (0 tokens) counts as a decode
    ([0], 0, (0, 0, 0, 0)),                          # empty step
])
def test_split_decodes_and_prefills(qsl, tokens, want):
    assert A.split_decodes_and_prefills(torch.tensor(qsl), tokens) == want


def test_split_rejects_decode_after_prefill():
    with pytest.raises(ValueError):
        A.split_decodes_and_prefills([0, 1, 8, 9], 9)


def test_build_metadata():
    qsl = torch.tensor([0, 1, 2, 9, 12], dtype=torch.int32)
    seq_lens = torch.tensor([40, 17, 7, 3], dtype=torch.int32)
    bt = torch.arange(16, dtype=torch.int32).view(4, 4)
    slots = torch.arange(12)
    md = A.build_metadata(12, qsl, 40, seq_lens, bt, slots, seq_lens_cpu_upper_bound=torch.tensor([40, 17, 7, 3]))
    assert (md.num_actual_tokens, md.num_decodes, md.num_decode_tokens, md.num_prefills, md.max_seq_len) == \
        (12, 2, 2, 2, 40)
    assert md.prefill_query_start_loc_cpu == [0, 7, 10]   # the prompts' offsets, rebased
    assert md.prefill_seq_lens_cpu == [7, 3]
    assert md.seq_lens is seq_lens and md.block_table is bt and md.slot_mapping is slots
    # a pure decode step carries no prefill lists
    md = A.build_metadata(2, [0, 1, 2], 17, seq_lens[:2], bt[:2], slots[:2])
    assert md.num_prefills == 0 and md.prefill_query_start_loc_cpu is None and md.prefill_seq_lens_cpu is None


def _vllm_config(max_len=4096, budget=2048, additional=None, hf=None):
    calls = []
    sched = SimpleNamespace(enable_chunked_prefill=True, max_num_batched_tokens=budget,
                            max_num_encoder_input_tokens=budget, encoder_cache_size=budget,
                            verify_max_model_len=lambda n: calls.append(n))
    cfg = SimpleNamespace(cache_config=SimpleNamespace(enable_prefix_caching=True, block_size=16),
                          scheduler_config=sched,
                          model_config=SimpleNamespace(max_model_len=max_len, hf_config=hf, dtype=torch.bfloat16),
                          additional_config=additional)
    return cfg, calls


def test_engine_defaults():
    cfg, calls = _vllm_config(max_len=4096, budget=2048)
    C.engine_defaults(cfg)
    s = cfg.scheduler_config
    assert not cfg.cache_config.enable_prefix_caching and not s.enable_chunked_prefill
    assert s.max_num_batched_tokens == s.max_num_encoder_input_tokens == s.encoder_cache_size == 4096
    assert calls == [4096]
    cfg, _ = _vllm_config(max_len=4096, budget=8192)  # a larger budget stays
    C.engine_defaults(cfg)
    assert cfg.scheduler_config.max_num_batched_tokens == 8192 and cfg.scheduler_config.encoder_cache_size == 8192


def test_starkv_config_and_checkpoint_lookup(tmp_path):
    for add in (None, {}, {"starkv": {}}, {"starkv": {"kv_quant": True}}):
        with pytest.raises(ValueError, match="fused checkpoint"):
            C.get_starkv_config(_vllm_config(additional=add)[0])
    path = str(tmp_path / "fused_weights.pt")
    ck.write_fused_checkpoint(path, 3, 4, 128, 256, {1: ([16, 32, 16, 48], 64)}, seed=5)
    hf = SimpleNamespace(hidden_size=512, num_attention_heads=4, num_key_value_heads=4, num_hidden_layers=3)
    for quant in (False, True):
        cfg = _vllm_config(additional={"starkv": {"weights": path, "kv_quant": quant}}, hf=hf)[0]
        assert C.get_starkv_config(cfg) == C.StarKVServeConfig(path, quant)
        a, b = C.starkv_checkpoint_for(cfg), C.starkv_checkpoint_for(cfg)
        assert a is b  # read once
        assert a.is_compressed(1) and not a.is_compressed(0) and a.layers[1].kv_quant == quant
        lw = a.layers[1]
        want = QuantRow(lw.k_width, 4, lw.v_rank).nbytes if quant else (lw.k_width + lw.v_rank) * 2
        assert A.cache_bytes_per_token(lw, 2) == want


def test_plugin_needs_vllm():
    try:
        import vllm  # noqa: F401
    except ImportError:
        with pytest.raises(ImportError, match="vLLM"):
            plugin.register()
    else:  # pragma: no cover
        pytest.skip("vLLM is installed")
