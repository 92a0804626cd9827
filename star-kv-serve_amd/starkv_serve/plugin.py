"""vLLM general-plugin entry point (the reference's starkv_serve/plugin.py:4-17).

``register`` makes vLLM serve ``StarKVLlamaForCausalLM`` with this package's attention
backend: it registers the architecture, attaches the engine defaults that the dense
prefill needs (``config.engine_defaults``) and registers the backend as vLLM's CUSTOM
attention backend. vLLM may call it more than once per process. It needs vLLM; without
it, it raises ImportError (this package's own decode model, ``starkv_serve.model``,
runs without vLLM).
"""


def register() -> None:
    try:
        from vllm import ModelRegistry
        from vllm.model_executor.models.config import MODELS_CONFIG_MAP, VerifyAndUpdateConfig
        from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend
    except ImportError as e:  # pragma: no cover - vLLM is not installed here
        raise ImportError("starkv_serve.plugin.register needs vLLM") from e

    from starkv_serve.config import engine_defaults

    class StarKVEngineDefaults(VerifyAndUpdateConfig):
        @staticmethod
        def verify_and_update_config(vllm_config) -> None:
            engine_defaults(vllm_config)

    if "StarKVLlamaForCausalLM" not in ModelRegistry.get_supported_archs():
        ModelRegistry.register_model("StarKVLlamaForCausalLM", "starkv_serve.vllm_model:StarKVLlamaForCausalLM")
    MODELS_CONFIG_MAP["StarKVLlamaForCausalLM"] = StarKVEngineDefaults
    register_backend(AttentionBackendEnum.CUSTOM, "starkv_serve.attention.StarKVAttentionBackend")
