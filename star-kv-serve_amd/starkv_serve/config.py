"""Serving-time configuration, as the reference's plugin reads it (starkv_serve/config.py).

The model is served with the fused checkpoint named in vLLM's ``--additional-config``:

  --hf-overrides '{"architectures": ["StarKVLlamaForCausalLM"]}'
  --additional-config '{"starkv": {"weights": "/path/to/fused_weights.pt", "kv_quant": true}}'

``engine_defaults`` is what the reference's ``StarKVEngineDefaults.verify_and_update_config``
does to the engine config (config.py:26-51): the dense prefill lifts a step's own codes and
never reads the cache, so every prompt must arrive whole in one step with nothing cached
before it (prefix caching and chunked prefill off, a step budget of at least
``max_model_len`` tokens). None of this module needs vLLM: it works on any object with the
attributes vLLM's config has.
"""
from dataclasses import dataclass
from functools import lru_cache

import torch

from starkv_serve.checkpoint import StarKVCheckpoint, load_fused_checkpoint


def engine_defaults(vllm_config) -> None:
    """Turn prefix caching and chunked prefill off and raise the step's token budget to
    max_model_len (config.py:35-51), in place."""
    cache, sched = vllm_config.cache_config, vllm_config.scheduler_config
    max_len = vllm_config.model_config.max_model_len
    cache.enable_prefix_caching = False
    sched.enable_chunked_prefill = False
    if sched.max_num_batched_tokens < max_len:
        sched.max_num_batched_tokens = max_len
        # vLLM derives these from the step budget when the scheduler config is built.
        sched.max_num_encoder_input_tokens = sched.encoder_cache_size = max_len
    verify = getattr(sched, "verify_max_model_len", None)
    if verify is not None:
        verify(max_len)


@dataclass(frozen=True)
class StarKVServeConfig:
    weights: str
    kv_quant: bool = False


def get_starkv_config(vllm_config) -> StarKVServeConfig:
    """The ``starkv`` entry of ``additional_config`` (config.py:60-67): the fused
    checkpoint path is required."""
    raw = (getattr(vllm_config, "additional_config", None) or {}).get("starkv") or {}
    if not raw.get("weights"):
        raise ValueError(
            "StarKVLlamaForCausalLM needs the fused checkpoint written by train.py: "
            '--additional-config \'{"starkv": {"weights": "/path/to/fused_weights.pt"}}\''
        )
    return StarKVServeConfig(weights=raw["weights"], kv_quant=bool(raw.get("kv_quant", False)))


@lru_cache(maxsize=4)
def _cached_checkpoint(path: str, num_layers: int, num_kv_heads: int, head_dim: int, dtype: torch.dtype,
                       kv_quant: bool) -> StarKVCheckpoint:
    return load_fused_checkpoint(path, num_layers, num_kv_heads, head_dim, dtype=dtype, kv_quant=kv_quant)


def starkv_checkpoint_for(vllm_config) -> StarKVCheckpoint:
    """The checkpoint for the model in ``vllm_config`` (config.py:76-83): every decoder
    layer asks for it, the file is read once per (path, shape, dtype, kv_quant)."""
    cfg = get_starkv_config(vllm_config)
    hf = vllm_config.model_config.hf_config
    head_dim = getattr(hf, "head_dim", None) or hf.hidden_size // hf.num_attention_heads
    num_kv_heads = getattr(hf, "num_key_value_heads", None) or hf.num_attention_heads
    return _cached_checkpoint(cfg.weights, hf.num_hidden_layers, num_kv_heads, head_dim,
                              vllm_config.model_config.dtype, cfg.kv_quant)
