"""STAR-KV Llama for decode steps, without vLLM.

Restates the serving model of the reference (starkv_serve/model.py:18-106 there) over
this library: a stock Llama whose compressed layers (those the fused checkpoint holds
factors for, checkpoint.py:74-93) attend over the STAR-KV cache and whose other layers
keep full K/V.

- A compressed layer's ``qkv_proj`` keeps only its Q rows (model.py:68-74 there; the
  checkpoint has no K/V projection for it). Its cache row is written straight from the
  layer input (``StarKVAttentionImpl.forward_from_hidden``: the codes' GEMM
  ``hidden @ [k_down; v_down]^T`` fused with the scatter or 3.2-bit pack), then the
  decode runs over the paged cache.
- An uncompressed layer is vLLM's LlamaAttention (model.py:77-81 there): QKV, RoPE on q
  and k, k and v into paged key / value caches [num_blocks, block_size, H_kv, 128]
  (``write_kv_full``, one launch, as vLLM's reshape_and_cache), and paged decode
  attention over them (``paged_decode_full``).
- Everything else is the stock Llama decoder: RMSNorm, SiLU-gated MLP, residuals, the
  final norm and the LM head.

The weights of everything but the attention factors are random-init here (the harness
measures decode steps; there is no network for real checkpoints). The factors come from
a fused checkpoint through ``load_fused_checkpoint``, as the reference loads them.

Two kinds of step: ``decode_step`` (every request contributes its one next token) and
``prefill_step`` (whole prompts, each from position 0, as the reference serves them: a
compressed layer writes the prompt's codes and runs its dense prefill,
attention.py:219-251; a full layer writes K/V and runs causal attention over the prompt,
here on this library's prefill kernel where vLLM would run FlashAttention).
"""
import math
from dataclasses import dataclass
from typing import List, Optional

import torch
import torch.nn.functional as F

from starkv_serve.attention import StarKVAttentionImpl, StarKVMetadata
from starkv_serve.checkpoint import StarKVCheckpoint
from starkv_serve.kernels.prefill import prefill_attention
from starkv_serve.kernels.stock_decode import paged_decode_full, write_kv_full
from starkv_serve.workloads import cos_sin_table


@dataclass(frozen=True)
class LlamaShape:
    hidden_size: int = 4096
    num_layers: int = 32
    num_heads: int = 32
    num_kv_heads: int = 32
    head_dim: int = 128
    intermediate_size: int = 11008
    vocab_size: int = 32000
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0


LLAMA2_7B = LlamaShape()


class Rotary:
    """What StarKVAttentionImpl reads of vLLM's RotaryEmbedding (``cos_sin_cache``
    [max_pos, head_dim] = cat(cos, sin)), plus NeoX rotate-half on q and k."""

    def __init__(self, max_pos: int, dtype: torch.dtype, device, base: float):
        self.cos_sin_cache = cos_sin_table(max_pos, dtype, device, base)

    def apply(self, positions: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        """x [T, H, D] rotated at `positions` [T] (fp32 arithmetic, x's dtype out)."""
        cos, sin = self.cos_sin_cache[positions].float().chunk(2, dim=-1)
        cos, sin = cos[:, None, :], sin[:, None, :]
        x1, x2 = x.float().chunk(2, dim=-1)
        return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1).to(x.dtype)


@dataclass
class Layer:
    ln1: torch.Tensor
    ln2: torch.Tensor
    o_proj: torch.Tensor          # [hidden, H * D]
    gate_up: torch.Tensor         # [2 * intermediate, hidden]
    down: torch.Tensor            # [hidden, intermediate]
    q_proj: Optional[torch.Tensor] = None    # compressed: [H * D, hidden]
    impl: Optional[StarKVAttentionImpl] = None
    qkv_proj: Optional[torch.Tensor] = None  # uncompressed: [(H + 2 H_kv) * D, hidden]

    @property
    def compressed(self) -> bool:
        return self.impl is not None


class StarKVLlamaForCausalLM:
    """Decode steps of a Llama with STAR-KV attention in its compressed layers."""

    def __init__(self, shape: LlamaShape, starkv: Optional[StarKVCheckpoint], max_model_len: int, device,
                 dtype: torch.dtype = torch.bfloat16, seed: int = 0, stock: bool = False):
        """`starkv` = None or `stock` = True: every layer uncompressed (the stock model)."""
        self.shape, self.device, self.dtype = shape, torch.device(device), dtype
        self.max_model_len = max_model_len
        H, Hkv, D, hid = shape.num_heads, shape.num_kv_heads, shape.head_dim, shape.hidden_size
        self.scale = D ** -0.5
        self.rotary = Rotary(max_model_len + 1, dtype, self.device, shape.rope_theta)
        g = torch.Generator(device=self.device).manual_seed(seed)

        def w(*size, fan_in):
            t = torch.empty(*size, device=self.device, dtype=dtype)
            t.normal_(0.0, fan_in ** -0.5, generator=g)
            return t

        self.embed = w(shape.vocab_size, hid, fan_in=1)
        self.norm = torch.ones(hid, device=self.device, dtype=dtype)
        self.lm_head = w(shape.vocab_size, hid, fan_in=hid)
        self.layers: List[Layer] = []
        for li in range(shape.num_layers):
            lw = None if (starkv is None or stock or not starkv.is_compressed(li)) else starkv.layers[li]
            layer = Layer(ln1=torch.ones(hid, device=self.device, dtype=dtype),
                          ln2=torch.ones(hid, device=self.device, dtype=dtype),
                          o_proj=w(hid, H * D, fan_in=H * D),
                          gate_up=w(2 * shape.intermediate_size, hid, fan_in=hid),
                          down=w(hid, shape.intermediate_size, fan_in=shape.intermediate_size))
            if lw is not None:
                layer.q_proj = w(H * D, hid, fan_in=hid)
                layer.impl = StarKVAttentionImpl(H, D, self.scale, Hkv, starkv_layer=lw, rotary_emb=self.rotary,
                                                 max_model_len=max_model_len)
                layer.impl.to_device(self.device, dtype)
            else:
                layer.qkv_proj = w((H + 2 * Hkv) * D, hid, fan_in=hid)
            self.layers.append(layer)
        self.kv_caches: List = []

    # -- caches ---------------------------------------------------------------------------
    def cache_bytes_per_token(self) -> int:
        """KV-cache bytes per token over all layers."""
        s = self.shape
        total = 0
        for layer in self.layers:
            if layer.compressed:
                imp = layer.impl
                total += imp.row.nbytes if imp.row is not None else (imp.k_width + imp.w.v_rank) * 2
            else:
                total += 2 * s.num_kv_heads * s.head_dim * 2
        return total

    def allocate_kv_cache(self, num_blocks: int, block_size: int = 16) -> None:
        s = self.shape
        self.block_size = block_size
        self.kv_caches = []
        for layer in self.layers:
            if layer.compressed:
                imp = layer.impl
                if imp.row is not None:
                    c = torch.zeros(num_blocks, block_size, imp.row.nbytes, dtype=torch.uint8, device=self.device)
                else:
                    c = torch.zeros(num_blocks, block_size, imp.k_width + imp.w.v_rank, dtype=self.dtype,
                                    device=self.device)
                self.kv_caches.append(c)
            else:
                kc = torch.zeros(num_blocks, block_size, s.num_kv_heads, s.head_dim, dtype=self.dtype,
                                 device=self.device)
                self.kv_caches.append((kc, torch.zeros_like(kc)))

    # -- the step ---------------------------------------------------------------------------
    def _attention(self, li: int, h: torch.Tensor, positions: torch.Tensor, md: StarKVMetadata,
                   capture: Optional[list], in_graph: bool = False) -> torch.Tensor:
        """Inside a graph (`in_graph`) no launch depends on the step's lengths: every layer
        decodes over the span max_model_len, the lengths are read on the device."""
        s, layer = self.shape, self.layers[li]
        T = h.shape[0]
        H, Hkv, D = s.num_heads, s.num_kv_heads, s.head_dim
        k = v = None
        if layer.compressed:
            q = self.rotary.apply(positions, F.linear(h, layer.q_proj).view(T, H, D))
            out = torch.empty(T, H * D, dtype=self.dtype, device=self.device)
            layer.impl.forward_from_hidden(q.view(T, H * D), h, self.kv_caches[li], md, out, in_full_graph=in_graph)
        else:
            qkv = F.linear(h, layer.qkv_proj)
            q, k, v = qkv.split([H * D, Hkv * D, Hkv * D], dim=-1)
            q = self.rotary.apply(positions, q.reshape(T, H, D))
            k = self.rotary.apply(positions, k.reshape(T, Hkv, D))
            v = v.reshape(T, Hkv, D)
            kc, vc = self.kv_caches[li]
            write_kv_full(k, v, kc, vc, md.slot_mapping[:T])
            if md.num_prefills:  # whole prompts only (prefill_step): causal attention over each prompt
                out = prefill_attention(q, k, v, md.prefill_seq_lens_cpu, self.scale).view(T, H * D)
            else:
                span = self.max_model_len if in_graph else max(md.max_seq_len, 1)
                out = paged_decode_full(q, kc, vc, md.block_table[:T], md.seq_lens[:T], span,
                                        self.scale).view(T, H * D)
        if capture is not None:
            capture.append(dict(layer=li, q=q.view(T, H, D), out=out.view(T, H, D), h=h, k=k, v=v))
        return F.linear(out, layer.o_proj)

    @torch.no_grad()
    def attention_inputs(self, hidden: torch.Tensor, positions: torch.Tensor) -> List[tuple]:
        """Per layer, what its attention op takes for one step with input `hidden`: the
        rotated queries, and for an uncompressed layer the rotated keys and the values (a
        compressed layer takes `hidden` itself: its write computes the codes)."""
        s = self.shape
        T = hidden.shape[0]
        H, Hkv, D = s.num_heads, s.num_kv_heads, s.head_dim
        res = []
        for layer in self.layers:
            if layer.compressed:
                q = self.rotary.apply(positions, F.linear(hidden, layer.q_proj).view(T, H, D))
                res.append((q.reshape(T, H * D), None, None))
            else:
                q, k, v = F.linear(hidden, layer.qkv_proj).split([H * D, Hkv * D, Hkv * D], dim=-1)
                res.append((self.rotary.apply(positions, q.reshape(T, H, D)),
                            self.rotary.apply(positions, k.reshape(T, Hkv, D)), v.reshape(T, Hkv, D).contiguous()))
        return res

    @torch.no_grad()
    def attention_only(self, hidden: torch.Tensor, inputs: List[tuple], md: StarKVMetadata,
                       in_graph: bool = False) -> None:
        """The attention ops of every layer for one step (the "attention per step" figure:
        the cache write and the attention, summed over the layers, as the reference's
        benchmark sums its two attention ops, bench_serving.py:62-115; the projections and
        RoPE are outside, as there). `inputs` from attention_inputs. A compressed layer's
        write includes its codes' GEMM (hidden @ kv_down^T), which the reference runs
        outside the attention op (model.py:71)."""
        T = hidden.shape[0]
        for li, layer in enumerate(self.layers):
            q, k, v = inputs[li]
            if layer.compressed:
                out = torch.empty(T, q.shape[1], dtype=self.dtype, device=self.device)
                layer.impl.forward_from_hidden(q, hidden, self.kv_caches[li], md, out, in_full_graph=in_graph)
            else:
                kc, vc = self.kv_caches[li]
                write_kv_full(k, v, kc, vc, md.slot_mapping[:T])
                span = self.max_model_len if in_graph else max(md.max_seq_len, 1)
                paged_decode_full(q, kc, vc, md.block_table[:T], md.seq_lens[:T], span, self.scale)

    @torch.no_grad()
    def _layers(self, x: torch.Tensor, positions: torch.Tensor, md: StarKVMetadata, capture: Optional[list],
                in_graph: bool) -> torch.Tensor:
        s = self.shape
        for li, layer in enumerate(self.layers):
            h = F.rms_norm(x, (s.hidden_size,), layer.ln1, s.rms_norm_eps)
            x = x + self._attention(li, h, positions, md, capture, in_graph)
            h = F.rms_norm(x, (s.hidden_size,), layer.ln2, s.rms_norm_eps)
            gate, up = F.linear(h, layer.gate_up).chunk(2, dim=-1)
            x = x + F.linear(F.silu(gate) * up, layer.down)
        return x

    def _logits(self, x: torch.Tensor) -> torch.Tensor:
        s = self.shape
        return F.linear(F.rms_norm(x, (s.hidden_size,), self.norm, s.rms_norm_eps), self.lm_head)

    def decode_step(self, tokens: torch.Tensor, positions: torch.Tensor, md: StarKVMetadata,
                    capture: Optional[list] = None, in_graph: bool = False) -> torch.Tensor:
        """Logits [n, vocab] for one new token per request: tokens [n] at `positions` [n];
        `md` has every row as a decode (seq_lens = positions + 1, slot_mapping the new
        tokens' slots)."""
        return self._logits(self._layers(self.embed[tokens], positions, md, capture, in_graph))

    @torch.no_grad()
    def prefill_step(self, tokens: torch.Tensor, positions: torch.Tensor, md: StarKVMetadata,
                     capture: Optional[list] = None) -> torch.Tensor:
        """Logits [P, vocab] at the last token of each of P whole prompts: tokens [T] and
        positions [T] (0 .. L - 1 per prompt) laid end to end, `md` from
        ``prefill_metadata``. Every layer writes the prompts' cache rows (compressed: the
        codes through the fused write; full: K and V), so decode steps can follow."""
        if md.num_decodes or not md.num_prefills:
            raise ValueError("prefill_step: a prompts-only batch (prefill_metadata)")
        x = self._layers(self.embed[tokens], positions, md, capture, False)
        last = torch.tensor(md.prefill_query_start_loc_cpu[1:], device=x.device) - 1
        return self._logits(x[last])


class DecodeGraph:
    """Greedy decode steps of `n` sessions captured once in a HIP graph: each replay runs
    one whole step (metadata from the positions, the 32 layers, the LM head, argmax) and
    advances the static tokens and positions in place, so consecutive replays decode
    consecutive tokens with no host work between them; `logits` holds the last replay's
    logits. The block table is static: its rows must cover every position the replays
    reach (up to max_model_len - 1)."""

    def __init__(self, model: StarKVLlamaForCausalLM, block_table: torch.Tensor, tokens: torch.Tensor,
                 positions: torch.Tensor):
        if model.max_model_len > block_table.shape[1] * model.block_size:
            raise ValueError("the block table's rows must cover max_model_len positions")
        self.model, self.block_table = model, block_table
        self.tokens = tokens.clone()
        self.positions = positions.clone().long()
        self.graph = torch.cuda.CUDAGraph()
        self._body()  # eager first: every lazy initialisation outside the capture
        self.tokens.copy_(tokens)
        self.positions.copy_(positions)
        torch.cuda.synchronize()
        with torch.cuda.graph(self.graph):
            self._body()

    @torch.no_grad()
    def _body(self) -> None:
        m = self.model
        md = decode_metadata(self.block_table, self.positions, m.block_size, m.max_model_len)
        self.logits = m.decode_step(self.tokens, self.positions, md, in_graph=True)
        self.tokens.copy_(self.logits.argmax(-1))
        self.positions.add_(1)

    def reset(self, tokens: torch.Tensor, positions: torch.Tensor) -> None:
        self.tokens.copy_(tokens)
        self.positions.copy_(positions)

    def replay(self) -> None:
        self.graph.replay()


def decode_metadata(block_table: torch.Tensor, positions: torch.Tensor, block_size: int,
                    max_seq_len: int) -> StarKVMetadata:
    """A decode-only batch's metadata: request b's new token at positions[b] (slot from its
    block-table row), seq_lens = positions + 1."""
    n = positions.shape[0]
    if max_seq_len > block_table.shape[1] * block_size:
        raise ValueError(f"positions up to {max_seq_len - 1} need more than the block table's "
                         f"{block_table.shape[1]} blocks of {block_size}")
    rows = torch.arange(n, device=positions.device)
    slots = block_table[rows, positions // block_size].long() * block_size + positions % block_size
    return StarKVMetadata(num_actual_tokens=n, num_decodes=n, num_decode_tokens=n, num_prefills=0,
                          max_seq_len=int(max_seq_len), seq_lens=(positions + 1).to(torch.int32),
                          block_table=block_table, slot_mapping=slots)


def prefill_metadata(block_table: torch.Tensor, prompt_lens: List[int], block_size: int):
    """A prompts-only batch's metadata and positions: prompt b's tokens at positions
    0 .. L_b - 1, their slots from block-table row b, laid end to end. Returns (md,
    positions [T])."""
    lens = [int(L) for L in prompt_lens]
    if not lens or min(lens) < 1:
        raise ValueError("prefill_metadata: every prompt needs at least one token")
    if max(lens) > block_table.shape[1] * block_size:
        raise ValueError(f"a prompt of {max(lens)} tokens needs more than the block table's "
                         f"{block_table.shape[1]} blocks of {block_size}")
    dev = block_table.device
    rows = torch.cat([torch.full((L,), b, dtype=torch.long) for b, L in enumerate(lens)]).to(dev)
    positions = torch.cat([torch.arange(L) for L in lens]).to(dev)
    slots = block_table[rows, positions // block_size].long() * block_size + positions % block_size
    qsl = [0]
    for L in lens:
        qsl.append(qsl[-1] + L)
    md = StarKVMetadata(num_actual_tokens=qsl[-1], num_decodes=0, num_decode_tokens=0, num_prefills=len(lens),
                        max_seq_len=max(lens), seq_lens=torch.tensor(lens, dtype=torch.int32, device=dev),
                        block_table=block_table, slot_mapping=slots, prefill_seq_lens_cpu=lens,
                        prefill_query_start_loc_cpu=qsl)
    return md, positions


def ranks_for_ratio(num_kv_heads: int, head_dim: int, keep: float, multiple: int, generator: torch.Generator):
    """Per-head K ranks (multiples of `multiple`) keeping about `keep` of the K dimensions
    in all, drawn around the mean (the reference's 0.75-ratio checkpoint keeps ~21.5 % of K
    and ~31.5 % of V, train.py:356-389 / README.md:87-88)."""
    total = int(round(keep * num_kv_heads * head_dim / multiple)) * multiple
    lo = max(multiple, (total // num_kv_heads) // multiple * multiple)
    ranks = [lo] * num_kv_heads
    left = (total - lo * num_kv_heads) // multiple
    for i in torch.randperm(num_kv_heads, generator=generator).tolist()[:left]:
        ranks[i] += multiple
    return ranks


def v_rank_for_ratio(num_kv_heads: int, head_dim: int, keep: float, multiple: int) -> int:
    return max(multiple, int(math.floor(keep * num_kv_heads * head_dim / multiple)) * multiple)
