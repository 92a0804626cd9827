"""The attention backend's per-layer implementation, over the MI355X library.

This restates ``StarKVAttentionImpl`` of the reference's vLLM backend
(starkv_serve/attention.py:105-217) with the same constructor arguments, checks and
errors, the same ``to_device`` attributes and the same ``forward`` contract:

- ``forward`` writes this step's K/V codes into the paged cache, then decodes every
  single-token request against the cache (attention.py:168-213).
- The bf16/fp16 write is ``write_codes``; the 3.2-bit write is ``pack_kv``.
- The decode is ``paged_starkv_decode`` / ``paged_quant_decode``.
- ``write_from_hidden`` is the fused route for the codes' own GEMM (model.py:71 + the
  write): one ``write_kv`` call from the layer's hidden states.
- Prefill is dense, as in the reference (attention.py:219-251): this step's codes are
  lifted back to K (RoPE applied) and V in float32 (torch GEMMs), rounded once to fp16,
  and every prompt attends causally to itself on this library's prefill kernel
  (``prefill_attention``, MFMA flash attention; the reference hands bf16 K / V to
  FlashAttention).

vLLM is not needed to import or run this module. The two values the reference reads
from vLLM are taken from it when it is importable, else from arguments:

- the model's ``max_model_len`` (``get_current_vllm_config``);
- whether the step runs inside a full CUDA/HIP graph (``get_forward_context``).

Differences from the reference, by design:

- The prefill lift and RoPE run in float32 and round K and V once to the model dtype;
  the reference lifts and rotates in the model dtype. Prefill metadata that the dense
  prefill cannot serve (chunked prompts, cached context) raises before any work is
  enqueued, where the reference raises after the cache write.
- The reference splits large decode batches so that its logits buffer stays under
  2^26 floats (attention.py:52, 198-199). The one-pass kernels keep logits on chip; the
  decode wrappers split batches above 1024 requests, and two-pass layers (wide V) so that
  a call's logits buffer stays under the same 2^26 floats.

The rest of the reference's backend module is here too: ``build_metadata`` is its
metadata builder's ``build`` (attention.py:80-103) on plain values, and where vLLM is
importable, ``StarKVMetadataBuilder``, ``StarKVAttentionBackend`` and ``StarKVAttention``
(attention.py:71-79, 254-316) wrap this implementation for vLLM.
"""
from dataclasses import dataclass
from typing import List, Optional

import torch
import torch.nn.functional as F

from starkv_serve.checkpoint import StarKVLayerWeights, layer_operands
from starkv_serve.kernels.kv_write import flush_write, write_codes, write_kv
from starkv_serve.kernels.paged_decode import paged_starkv_decode
from starkv_serve.kernels.paged_quant import HEAD_DIM, pack_kv, paged_quant_decode
from starkv_serve.kernels.prefill import prefill_attention

DECODER = "decoder"  # AttentionType.DECODER


@dataclass
class StarKVMetadata:
    """One step's batch, decodes first (attention.py:55-67)."""
    num_actual_tokens: int
    num_decodes: int
    num_decode_tokens: int
    num_prefills: int
    max_seq_len: int
    seq_lens: torch.Tensor       # [>= num_decodes] int32, length including this step's token
    block_table: torch.Tensor    # [>= num_decodes, max_blocks] int32
    slot_mapping: torch.Tensor   # [>= num_actual_tokens] int64 (-1: padding token)
    prefill_seq_lens_cpu: Optional[List[int]] = None
    prefill_query_start_loc_cpu: Optional[List[int]] = None

    def decode_lens(self, nd: int) -> torch.Tensor:
        """seq_lens[:nd] with padding rows (length 0) given one (null-block) position to
        attend to: formed once per step and shared by every layer."""
        c = self.__dict__.get("_decode_lens")
        if c is None or c[0] != nd:
            c = (nd, self.seq_lens[:nd].clamp(min=1))
            self.__dict__["_decode_lens"] = c
        return c[1]


try:  # looked up once: forward runs every layer of every step
    from vllm.config import CUDAGraphMode, get_current_vllm_config
    from vllm.forward_context import get_forward_context
    _HAVE_VLLM = True
except ImportError:
    _HAVE_VLLM = False


def _vllm_max_model_len() -> Optional[int]:
    return get_current_vllm_config().model_config.max_model_len if _HAVE_VLLM else None


def _vllm_in_full_graph() -> bool:
    return _HAVE_VLLM and get_forward_context().cudagraph_runtime_mode == CUDAGraphMode.FULL


def split_decodes_and_prefills(query_start_loc_cpu, num_tokens: int, decode_threshold: int = 1):
    """(num_decodes, num_prefills, num_decode_tokens, num_prefill_tokens) of a batch whose
    requests are ordered decodes first: the leading requests with at most
    `decode_threshold` query tokens are decodes. The restatement of vLLM's
    ``split_decodes_and_prefills`` (vllm/v1/attention/backends/utils.py), which the
    reference's builder calls (attention.py:83-84); raises ValueError if a decode follows
    a prefill (the builder asks vLLM to reorder the batch so that none does)."""
    qsl = [int(x) for x in query_start_loc_cpu]
    num_reqs = len(qsl) - 1
    lens = [qsl[i + 1] - qsl[i] for i in range(num_reqs)]
    nd = 0
    while nd < num_reqs and lens[nd] <= decode_threshold:
        nd += 1
    if any(q <= decode_threshold for q in lens[nd:]):
        raise ValueError("decode requests must come before prefills")
    return nd, num_reqs - nd, qsl[nd], num_tokens - qsl[nd]


def build_metadata(num_actual_tokens: int, query_start_loc_cpu, max_seq_len: int, seq_lens: torch.Tensor,
                   block_table: torch.Tensor, slot_mapping: torch.Tensor,
                   seq_lens_cpu_upper_bound=None) -> StarKVMetadata:
    """One step's StarKVMetadata from vLLM's common attention metadata (the reference's
    ``StarKVMetadataBuilder.build``, attention.py:80-103): decodes and prefills split as
    above; for the prefills, their query offsets rebased to 0 and their lengths (host lists,
    as the dense prefill needs them)."""
    nd, npf, ndt, _ = split_decodes_and_prefills(query_start_loc_cpu, num_actual_tokens, 1)
    prefill_lens = prefill_qsl = None
    if npf:
        qsl = [int(x) for x in query_start_loc_cpu[nd:nd + npf + 1]]
        prefill_qsl = [x - qsl[0] for x in qsl]
        if seq_lens_cpu_upper_bound is not None:
            prefill_lens = [int(x) for x in seq_lens_cpu_upper_bound[nd:nd + npf]]
    return StarKVMetadata(num_actual_tokens=num_actual_tokens, num_decodes=nd, num_decode_tokens=ndt,
                          num_prefills=npf, max_seq_len=int(max_seq_len), seq_lens=seq_lens,
                          block_table=block_table, slot_mapping=slot_mapping,
                          prefill_seq_lens_cpu=prefill_lens, prefill_query_start_loc_cpu=prefill_qsl)


def cache_bytes_per_token(layer: StarKVLayerWeights, elem_size: int) -> int:
    """The bytes per token a compressed layer's cache row takes: what the reference's
    ``StarKVAttention.get_kv_cache_spec`` declares as the row of its one head slot
    (attention.py:289-299, checkpoint.py:58-62)."""
    return layer.cache_bytes(elem_size)


def _attn_type_name(attn_type) -> str:
    return str(getattr(attn_type, "value", attn_type)).lower()


class StarKVAttentionImpl:
    """Per-layer attention over the compressed cache (attention.py:105-217)."""

    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: Optional[int] = None,
                 alibi_slopes=None, sliding_window=None, kv_cache_dtype: str = "auto", logits_soft_cap=None,
                 attn_type=DECODER, kv_sharing_target_layer_name=None, *, starkv_layer: StarKVLayerWeights,
                 rotary_emb, max_model_len: Optional[int] = None, fused_write: bool = False):
        if alibi_slopes is not None or sliding_window is not None or logits_soft_cap:
            raise NotImplementedError("STAR-KV attention: no alibi, sliding window or softcap")
        if _attn_type_name(attn_type) != DECODER or kv_sharing_target_layer_name is not None:
            raise NotImplementedError("STAR-KV attention: decoder self-attention only")
        if kv_cache_dtype not in ("auto", "float16", "bfloat16"):
            raise NotImplementedError(f"STAR-KV attention: kv_cache_dtype {kv_cache_dtype!r}")
        if starkv_layer.kv_quant and ((num_kv_heads or num_heads) != num_heads or head_size != HEAD_DIM):
            raise NotImplementedError("STAR-KV 4-bit cache: MHA with head_dim 128 only")
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.num_kv_heads = num_kv_heads or num_heads
        self.kv_cache_dtype = kv_cache_dtype
        self.w = starkv_layer
        self.rotary_emb = rotary_emb
        # fused_write: `forward` receives the layer's input as `key` (value unused) and
        # writes the cache row from it (forward_from_hidden).
        self.fused_write = fused_write
        vllm_len = _vllm_max_model_len()
        self.max_model_len = vllm_len if vllm_len is not None else max_model_len
        if self.max_model_len is None:
            raise ValueError("max_model_len is needed when vLLM is not present")

    def to_device(self, device: torch.device, dtype: torch.dtype) -> None:
        """The kernel operands on `device` (attention.py:134-166), before any graph capture."""
        ops = layer_operands(self.w, self.num_heads, device, dtype)
        self.k_ranks = ops.k_ranks
        self.k_head_offsets = ops.k_head_offsets
        self.k_width = ops.k_width
        self.k_up = ops.k_up
        self.v_up_by_q = ops.v_up_by_q
        self.kv_down = ops.kv_down
        self.row = ops.row
        self.kv_groups = ops.kv_groups
        if self.row is not None:
            self.k_nouts, self.head_of_lane, self.k_tiles = ops.k_nouts, ops.head_of_lane, ops.k_tiles
        # Prefill lifts every KV head in one batched product, which needs one width: the
        # codes are gathered into a padded [T, H, R] view. Lanes past a head's width point
        # at its first code; the rows of U they meet are zero (attention.py:144-160).
        w, H, Hd = self.w, self.num_kv_heads, self.head_size
        R = w.k_max_rank
        idx = torch.empty(H * R, dtype=torch.long)
        k_up_pad = torch.zeros(H, R, Hd, dtype=w.k_up.dtype)
        for h, (off, width) in enumerate(zip(w.k_head_offsets.tolist(), w.k_head_widths.tolist())):
            idx[h * R:h * R + width] = torch.arange(off, off + width)
            idx[h * R + width:(h + 1) * R] = off
            k_up_pad[h, :width] = w.k_up[off:off + width]
        self.k_prefill_gather = idx.to(device)
        # The decode kernels read an fp16 cos/sin table: converted once here, not per step.
        self.cos_sin16 = self.rotary_emb.cos_sin_cache.to(device=device, dtype=torch.float16).contiguous()
        self.k_up_T = k_up_pad.to(device=device, dtype=torch.float32).contiguous()
        # V's lift runs as an fp16 GEMM (fp32 accumulation, the result rounded once to fp16).
        self.v_up_f16 = w.v_up.to(device=device, dtype=torch.float16).contiguous()  # [H * Hd, v_rank]

    def _cache(self, kv_cache: torch.Tensor) -> torch.Tensor:
        cache = kv_cache.squeeze(1) if kv_cache.dim() == 4 else kv_cache  # [num_blocks, block_size, width]
        return cache if self.row is None else cache.view(torch.uint8)

    def forward(self, layer, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
                attn_metadata: Optional[StarKVMetadata], output: torch.Tensor, output_scale=None,
                output_block_scale=None, in_full_graph: Optional[bool] = None) -> torch.Tensor:
        """Writes the step's codes (`key` [T, k_width], `value` [T, v_rank]) and decodes
        `query` [T, H*128] into `output` [T, H*128] (attention.py:168-217). `in_full_graph`
        defaults to vLLM's forward context (False without vLLM)."""
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("STAR-KV attention: fused output quantization")
        if self.fused_write:
            return self.forward_from_hidden(query, key, kv_cache, attn_metadata, output, in_full_graph)
        if attn_metadata is None:  # profiling run
            return output.fill_(0)
        md = attn_metadata
        query_lens = self._prefill_lens(md) if md.num_prefills else None
        n = md.num_actual_tokens
        Hq, Hd = self.num_heads, self.head_size
        cache = self._cache(kv_cache)
        if self.row is None:
            # Padding tokens carry slot -1: the write sends them to the reserved null block 0.
            write_codes(key[:n], value[:n], cache, md.slot_mapping[:n])
        else:
            pack_kv(key[:n], value[:n], cache, md.slot_mapping[:n], self.row, self.k_ranks, self.k_head_offsets,
                    self.k_nouts)
        nd = md.num_decode_tokens
        if nd:
            self._decode(query[:nd].view(nd, Hq, Hd), cache, md, output[:nd].view(nd, Hq, Hd), in_full_graph)
        if md.num_prefills:
            self._dense_prefill(query_lens, query[nd:n].view(n - nd, Hq, Hd), key[nd:n], value[nd:n],
                                output[nd:n].view(n - nd, Hq, Hd))
        return output

    @staticmethod
    def _prefill_lens(md: StarKVMetadata) -> List[int]:
        """The prompts' lengths; each prompt must arrive whole, with no cached context
        (attention.py:221-230)."""
        p0, p1 = md.num_decodes, md.num_decodes + md.num_prefills
        qsl = md.prefill_query_start_loc_cpu
        if qsl is None:
            raise NotImplementedError("STAR-KV prefill needs prefill_query_start_loc_cpu")
        seq_lens = md.prefill_seq_lens_cpu or md.seq_lens[p0:p1].tolist()
        query_lens = [qsl[i + 1] - qsl[i] for i in range(len(seq_lens))]
        if list(seq_lens) != query_lens:
            raise NotImplementedError(
                "STAR-KV prefill needs every prompt in one step with no cached context "
                "(no prefix caching, no chunked prefill)")
        return query_lens

    def _dense_prefill(self, query_lens: List[int], q: torch.Tensor, k_codes: torch.Tensor, v_codes: torch.Tensor,
                       out: torch.Tensor) -> None:
        """STAR-KV's prefill (attention.py:219-251): K = RoPE(codes @ U) and V = codes @
        v_up for this step's tokens (positions from 0 in every prompt), each rounded once
        to fp16 (K lifted and rotated in fp32; V as an fp16 GEMM of the codes and v_up in
        fp16, accumulated in fp32), then causal attention of every prompt to itself on this
        library's prefill kernel. q and out [T, H_q, 128]."""
        T = q.shape[0]
        H, R, Hd = self.num_kv_heads, self.w.k_max_rank, self.head_size
        pos = torch.cat([torch.arange(L) for L in query_lens]).to(q.device)
        kp = k_codes[:, self.k_prefill_gather].float().view(T, H, R).transpose(0, 1).contiguous()
        k = torch.bmm(kp, self.k_up_T).transpose(0, 1)                                     # [T, H, Hd] fp32
        cos, sin = self.rotary_emb.cos_sin_cache[pos].float().chunk(2, dim=-1)
        cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
        k1, k2 = k.chunk(2, dim=-1)
        k = torch.cat([k1 * cos - k2 * sin, k2 * cos + k1 * sin], dim=-1).to(torch.float16)
        v = F.linear(v_codes.to(torch.float16), self.v_up_f16).view(T, H, Hd)
        prefill_attention(q, k, v, query_lens, self.scale, out=out)

    def write_from_hidden(self, hidden: torch.Tensor, kv_cache: torch.Tensor, slot_mapping: torch.Tensor,
                          return_codes: bool = False, deferred: bool = False) -> Optional[torch.Tensor]:
        """The step's write straight from the layer input: codes = hidden @ kv_down^T,
        rounded to the model dtype (model.py:71), written or packed into their slots.
        ``deferred``: launched by the decode call that follows (``write_kv``)."""
        cache = self._cache(kv_cache)
        if self.row is None:
            return write_kv(hidden, self.kv_down, cache, slot_mapping, self.k_width, return_codes=return_codes,
                            deferred=deferred)
        return write_kv(hidden, self.kv_down, cache, slot_mapping, self.k_width, row=self.row, k_ranks=self.k_ranks,
                        k_offsets=self.k_head_offsets, k_nouts=self.k_nouts, return_codes=return_codes,
                        deferred=deferred)

    def forward_from_hidden(self, query: torch.Tensor, hidden: torch.Tensor, kv_cache: torch.Tensor,
                            attn_metadata: Optional[StarKVMetadata], output: torch.Tensor,
                            in_full_graph: Optional[bool] = None) -> torch.Tensor:
        """``forward`` with the codes' GEMM fused into the write: the layer's input
        `hidden` [T, hidden_size] instead of `key` / `value` codes (model.py:71 + the
        write of attention.py:179-188), then the same decode and prefill."""
        if attn_metadata is None:  # profiling run
            return output.fill_(0)
        md = attn_metadata
        n = md.num_actual_tokens
        if md.num_prefills:
            codes = self.write_from_hidden(hidden[:n], kv_cache, md.slot_mapping[:n], return_codes=True)
            key, value = codes[:, :self.k_width], codes[:, self.k_width:]
            query_lens = self._prefill_lens(md)
        Hq, Hd = self.num_heads, self.head_size
        nd = md.num_decode_tokens
        # A decode-only step defers its write into the decode's first launch.
        deferred = not md.num_prefills and nd > 0
        if not md.num_prefills:
            self.write_from_hidden(hidden[:n], kv_cache, md.slot_mapping[:n], deferred=deferred)
        if nd:
            try:
                self._decode(query[:nd].view(nd, Hq, Hd), self._cache(kv_cache), md, output[:nd].view(nd, Hq, Hd),
                             in_full_graph)
            except BaseException:
                if deferred:
                    flush_write()
                raise
        if md.num_prefills:
            self._dense_prefill(query_lens, query[nd:n].view(n - nd, Hq, Hd), key[nd:n], value[nd:n],
                                output[nd:n].view(n - nd, Hq, Hd))
        return output

    def _decode(self, q: torch.Tensor, cache: torch.Tensor, md: StarKVMetadata, out: torch.Tensor,
                in_full_graph: Optional[bool]) -> None:
        nd = q.shape[0]
        full = _vllm_in_full_graph() if in_full_graph is None else in_full_graph
        # Inside a full graph nothing may depend on the step's lengths: the span is fixed.
        span = self.max_model_len if full else max(md.max_seq_len, 1)
        seq_lens = md.decode_lens(nd)
        cs = getattr(self, "cos_sin16", None)
        if cs is None:
            cs = self.rotary_emb.cos_sin_cache
        # The kernels write `out` in its own dtype and strides (no copy of the result).
        if self.row is None:
            paged_starkv_decode(q, cache, md.block_table[:nd], seq_lens, span, self.k_up, self.k_ranks,
                                self.k_head_offsets, self.k_width, self.v_up_by_q, cs, self.scale, out=out,
                                kv_groups=self.kv_groups)
        else:
            paged_quant_decode(q, cache, md.block_table[:nd], seq_lens, span, self.row, self.k_up,
                               self.head_of_lane, self.k_tiles, self.v_up_by_q, cs, self.scale, out=out,
                               kv_groups=self.kv_groups)


if _HAVE_VLLM:  # pragma: no cover - vLLM is not installed in this image
    from typing import ClassVar

    from vllm.model_executor.layers.attention.attention import (Attention, _encode_layer_name,
                                                                unified_attention_with_output)
    from vllm.v1.attention.backend import (AttentionBackend, AttentionCGSupport, AttentionMetadataBuilder,
                                           CommonAttentionMetadata)
    from vllm.v1.kv_cache_interface import FullAttentionSpec

    class StarKVMetadataBuilder(AttentionMetadataBuilder[StarKVMetadata]):
        """attention.py:71-103: decodes first; pure single-token decode batches are
        captured whole in HIP graphs."""
        _cudagraph_support: ClassVar[AttentionCGSupport] = AttentionCGSupport.UNIFORM_SINGLE_TOKEN_DECODE

        def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
            super().__init__(kv_cache_spec, layer_names, vllm_config, device)
            self._init_reorder_batch_threshold(1)

        def build(self, common_prefix_len: int, common_attn_metadata: CommonAttentionMetadata,
                  fast_build: bool = False) -> StarKVMetadata:
            m = common_attn_metadata
            return build_metadata(m.num_actual_tokens, m.query_start_loc_cpu, m.max_seq_len, m.seq_lens,
                                  m.block_table_tensor, m.slot_mapping, m.seq_lens_cpu_upper_bound)

    class StarKVAttentionBackend(AttentionBackend):
        """attention.py:254-268."""
        forward_includes_kv_cache_update: bool = True
        supported_dtypes: ClassVar[List[torch.dtype]] = [torch.float16, torch.bfloat16]

        @staticmethod
        def get_name() -> str:
            return "CUSTOM"  # registered as AttentionBackendEnum.CUSTOM by the plugin

        @staticmethod
        def get_impl_cls():
            return StarKVAttentionImpl

        @staticmethod
        def get_builder_cls():
            return StarKVMetadataBuilder

    class StarKVAttention(Attention):
        """An ``Attention`` whose K and V inputs are STAR-KV codes (attention.py:271-316)."""

        def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: int,
                     starkv_layer: StarKVLayerWeights, rotary_emb, qkv_proj=None, cache_config=None, prefix: str = "",
                     fused_write: bool = False):
            """`qkv_proj`: a stacked QKV projection whose K/V rows are dropped after loading
            (the codes replace them), or None for a Q-only layer. `fused_write`: `key` is the
            layer's input and the write forms the codes (forward_from_hidden)."""
            super().__init__(num_heads, head_size, scale, num_kv_heads=num_kv_heads, cache_config=cache_config,
                             prefix=prefix, attn_backend=StarKVAttentionBackend, starkv_layer=starkv_layer,
                             rotary_emb=rotary_emb, fused_write=fused_write)
            self.starkv_layer = starkv_layer
            self.fused_write = fused_write
            self._qkv_proj = (qkv_proj,)  # not registered a second time as a child module

        def get_kv_cache_spec(self, vllm_config) -> FullAttentionSpec:
            dtype = self.kv_cache_torch_dtype
            elem = torch.empty((), dtype=dtype).element_size()
            return FullAttentionSpec(block_size=vllm_config.cache_config.block_size, num_kv_heads=self.num_kv_heads,
                                     head_size=self.head_size, dtype=dtype, num_head_slots=1,
                                     state_content_bytes=cache_bytes_per_token(self.starkv_layer, elem))

        def forward(self, query, key, value, output_shape=None, output_dtype=None):
            output = torch.empty((query.shape[0], self.num_heads * self.head_size), dtype=output_dtype or query.dtype,
                                 device=query.device)
            if value is None:  # fused write: key is the layer's input, value is not read
                value = key.new_empty(0)
            if self.use_direct_call:
                unified_attention_with_output(query, key, value, output, self.layer_name)
            else:
                torch.ops.vllm.unified_attention_with_output(query, key, value, output,
                                                             _encode_layer_name(self.layer_name))
            return output

        def process_weights_after_loading(self, act_dtype: torch.dtype):
            super().process_weights_after_loading(act_dtype)
            qkv = self._qkv_proj[0]
            q_size = self.num_heads * self.head_size
            if qkv is not None and qkv.weight.shape[0] != q_size:  # the K/V rows are dead: the codes come from kv_down
                qkv.weight = torch.nn.Parameter(qkv.weight.data[:q_size].contiguous(), requires_grad=False)
            self.impl.to_device(qkv.weight.device, act_dtype)
