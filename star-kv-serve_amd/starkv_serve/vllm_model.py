"""vLLM's model class for STAR-KV serving, over this package's attention layer.

vLLM builds its stock Llama decoder. In the layers the fused checkpoint compressed (those
with K/V factors, checkpoint.py:74-93), the decoder's self-attention module is
``CompressedSelfAttention`` instead of vLLM's LlamaAttention:

- ``q_proj`` only: a compressed layer has no K/V projection (its cache row is the codes
  ``hidden @ [k_down; v_down]^T``), and RoPE is applied to q alone, from the rotary
  table's ``cos_sin_cache``;
- the layer's input goes to the attention op unchanged: ``StarKVAttention`` with
  ``fused_write`` hands it to ``StarKVAttentionImpl.forward_from_hidden``, whose write
  kernel forms the codes itself (``starkv_write_kv``: the split-K GEMM and the scatter or
  3.2-bit pack), so no codes tensor is formed between the layers (the reference runs the
  codes' GEMM in torch and passes K/V codes, starkv_serve/model.py:68-74 there);
- ``o_proj`` as usual.

Weights: the fused checkpoint holds every weight of the model (checkpoint.py:3-9). The
compressed layers' ``q_proj`` and ``o_proj`` are copied by this class's loader, their K/V
factors are read by ``checkpoint.py`` when the layers are built, and every other weight
goes through vLLM's Llama loader.

It needs vLLM and is imported only by vLLM (``plugin.register`` names it); this image has
no vLLM, so it is not exercised here. ``starkv_serve.model`` is the same model without
vLLM, which the tests and the benchmark run.
"""
import functools

import torch
import torch.nn as nn
from vllm.config import get_current_vllm_config
from vllm.distributed import get_tensor_model_parallel_world_size
from vllm.model_executor.layers.linear import ReplicatedLinear
from vllm.model_executor.layers.rotary_embedding import get_rope
from vllm.model_executor.models.llama import LlamaDecoderLayer, LlamaForCausalLM
from vllm.model_executor.models.utils import extract_layer_index

from starkv_serve.attention import StarKVAttention
from starkv_serve.config import get_starkv_config, starkv_checkpoint_for


def _rope_q(cos_sin_cache: torch.Tensor, positions: torch.Tensor, q: torch.Tensor, head_dim: int) -> torch.Tensor:
    """NeoX rotate-half of q [T, H * head_dim] at `positions`, in fp32."""
    cos, sin = cos_sin_cache[positions].float().chunk(2, dim=-1)
    x = q.view(q.shape[0], -1, head_dim).float()
    x1, x2 = x.chunk(2, dim=-1)
    cos, sin = cos[:, None, :], sin[:, None, :]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1).to(q.dtype).view_as(q)


class CompressedSelfAttention(nn.Module):
    """Self-attention of a compressed layer. The constructor takes the arguments vLLM's
    LlamaDecoderLayer passes to its attention module; `starkv_layer` is bound by
    StarKVLlamaForCausalLM."""

    def __init__(self, config, hidden_size: int, num_heads: int, num_kv_heads: int,
                 max_position_embeddings: int = 8192, quant_config=None, bias: bool = False,
                 bias_o_proj: bool = False, cache_config=None, prefix: str = "", attn_type: str = "decoder",
                 *, starkv_layer=None):
        super().__init__()
        # Serving contract of the STAR-KV layers (the reference refuses the same).
        if get_tensor_model_parallel_world_size() != 1:
            raise NotImplementedError("STAR-KV serving supports tensor_parallel_size=1")
        if quant_config is not None:
            raise NotImplementedError("STAR-KV serving does not support weight quantization")
        if str(getattr(attn_type, "value", attn_type)).lower() != "decoder":
            raise NotImplementedError("STAR-KV serving supports decoder attention only")
        self.head_dim = getattr(config, "head_dim", None) or hidden_size // num_heads
        self.q_proj = ReplicatedLinear(hidden_size, num_heads * self.head_dim, bias=bias, prefix=f"{prefix}.q_proj")
        self.o_proj = ReplicatedLinear(num_heads * self.head_dim, hidden_size, bias=bias_o_proj,
                                       prefix=f"{prefix}.o_proj")
        self.rotary_emb = get_rope(self.head_dim, rotary_dim=self.head_dim, max_position=max_position_embeddings,
                                   base=getattr(config, "rope_theta", 10000.0),
                                   rope_scaling=getattr(config, "rope_scaling", None), is_neox_style=True)
        self.attn = StarKVAttention(num_heads, self.head_dim, self.head_dim ** -0.5, num_kv_heads,
                                    starkv_layer=starkv_layer, rotary_emb=self.rotary_emb, qkv_proj=None,
                                    cache_config=cache_config, prefix=f"{prefix}.attn", fused_write=True)

    def forward(self, positions: torch.Tensor, hidden_states: torch.Tensor) -> torch.Tensor:
        q, _ = self.q_proj(hidden_states)
        q = _rope_q(self.rotary_emb.cos_sin_cache, positions, q, self.head_dim)
        out, _ = self.o_proj(self.attn(q, hidden_states, None))
        return out


def _decoder_layer(vllm_config, prefix: str = "", config=None):
    """vLLM's Llama decoder layer; compressed layers get CompressedSelfAttention."""
    ckpt = starkv_checkpoint_for(vllm_config)
    li = extract_layer_index(prefix)
    if not ckpt.is_compressed(li):
        return LlamaDecoderLayer(vllm_config=vllm_config, prefix=prefix, config=config)
    attn = functools.partial(CompressedSelfAttention, starkv_layer=ckpt.layers[li])
    return LlamaDecoderLayer(vllm_config=vllm_config, prefix=prefix, config=config, attn_layer_type=attn)


# K/V factors of the compressed layers: read by checkpoint.py, never by a loader.
_FACTORS = (".k_proj.VS.weight", ".k_proj.U.weight", ".k_proj.head_ranks", ".v_proj.VS.weight",
            ".v_proj.U.weight")


class StarKVLlamaForCausalLM(LlamaForCausalLM):
    def __init__(self, *, vllm_config, prefix: str = ""):
        self.starkv = get_starkv_config(vllm_config)  # fails before any layer is built
        super().__init__(vllm_config=vllm_config, prefix=prefix, layer_type=_decoder_layer)

    def load_weights(self, weights):
        """Every weight from the fused checkpoint; the HF files supply only the config and
        tokenizer. Returns the names loaded."""
        del weights
        sd = torch.load(self.starkv.weights, map_location="cpu", mmap=True, weights_only=True)
        ckpt = starkv_checkpoint_for(get_current_vllm_config())
        params = dict(self.named_parameters())
        own, rest = set(), []
        for name, t in sd.items():
            if name.endswith(_FACTORS):
                continue
            if ".self_attn." in name and ckpt.is_compressed(extract_layer_index(name)):
                p = params[name]  # q_proj / o_proj of a compressed layer: plain replicated weights
                getattr(p, "weight_loader", lambda dst, src: dst.data.copy_(src))(p, t)
                own.add(name)
            else:
                rest.append((name, t))
        return own | set(super().load_weights(iter(rest)))
