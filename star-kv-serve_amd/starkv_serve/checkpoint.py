"""Fused STAR-KV checkpoint (``fused_weights.pt``): loader, kernel operands and a
synthetic writer.

Drop-in for the reference's ``starkv_serve/checkpoint.py`` (same names, fields,
arguments and errors; checkpoint.py:26-169) and for the operand assembly of
``StarKVAttentionImpl.to_device`` (attention.py:134-166), which turns one loaded
layer into the tensors the decode and write kernels take.

Per compressed layer ``li`` the state dict holds, under
``model.layers.{li}.self_attn.`` (checkpoint.py:3-9):

    k_proj.VS.weight   [sum(ranks), hidden]  the heads' down factors, back to back
    k_proj.U.weight    [H*Hd, sum(ranks)]    block diagonal: head h's [Hd, rank_h] block
    k_proj.head_ranks  [H] int32
    v_proj.VS.weight   [r_v, hidden]         one V latent shared by the heads
    v_proj.U.weight    [H*Hd, r_v]

Layers without ``k_proj.head_ranks`` are uncompressed (skipped); a layer still in
the training-time U/Sigma/V form is rejected. The loader stores every K head at
its rank rounded up to ``K_ALIGN`` (zero rows past the rank), heads side by side
(``k_head_offsets``), U transposed to rank-major rows so a head's rows are one run;
V is padded to ``V_ALIGN`` for the bf16/fp16 cache. For the 3.2-bit cache the
K and V factors are first rotated by the block Hadamard of ``paged_quant``, in
float64, with a fresh generator per projection seeded ``HADAMARD_SEED`` and
consumed head by head: VS <- T^T VS, U <- U T, so U VS is unchanged while the
codes the cache stores are the rotated ones; V is then not padded.

``write_fused_checkpoint`` writes a random-init checkpoint in this format (the
reference's only writer is its training script, train.py:492-527), so a full
model configuration can be served and tested without trained weights.
"""
from dataclasses import dataclass
from typing import Optional

import torch

from starkv_serve import _hip

from starkv_serve.kernels.paged_decode import kv_head_groups
from starkv_serve.kernels.paged_quant import HADAMARD_SEED, QuantRow, block_hadamard, k_tables, n_outlier

K_ALIGN = 16  # stored K width per head: rank rounded up to this (one MFMA rank tile)
V_ALIGN = 16  # bf16/fp16 V width: rounded up to this


def _round_up(n: int, m: int) -> int:
    return (int(n) + m - 1) // m * m


def _prefix(layer_idx: int) -> str:
    return f"model.layers.{layer_idx}.self_attn."


@dataclass
class StarKVLayerWeights:
    """One compressed layer, repacked for the kernels (checkpoint.py:37-62)."""

    layer_idx: int
    k_head_ranks: torch.Tensor    # [H] int32, rank per KV head
    k_head_widths: torch.Tensor   # [H] int32, rank rounded up to K_ALIGN
    k_head_offsets: torch.Tensor  # [H] int32, first K code of each head
    k_width: int                  # K codes per token (sum of the widths)
    k_max_rank: int               # widest head
    k_down: torch.Tensor          # [k_width, hidden]: hidden -> K codes
    k_up: torch.Tensor            # [k_width, Hd]: K codes -> K before RoPE
    v_rank: int                   # stored V width (padded unless kv_quant)
    v_rank_real: int              # V rank in the checkpoint
    v_down: torch.Tensor          # [v_rank, hidden]
    v_up: torch.Tensor            # [H*Hd, v_rank]
    kv_quant: bool = False        # the cache holds 3.2-bit rows (QuantRow)

    @property
    def cache_width(self) -> int:
        """Codes per token: K, then V."""
        return self.k_width + self.v_rank

    def cache_bytes(self, elem_size: int) -> int:
        """Cache bytes per token for this layer."""
        if self.kv_quant:
            return QuantRow(self.k_width, self.k_head_ranks.numel(), self.v_rank).nbytes
        return self.cache_width * elem_size


@dataclass
class StarKVCheckpoint:
    layers: dict
    skip_layers: tuple

    def is_compressed(self, layer_idx: int) -> bool:
        return layer_idx in self.layers


def load_fused_checkpoint(path: str, num_layers: int, num_kv_heads: int, head_dim: int,
                          dtype: torch.dtype = torch.float16, kv_quant: bool = False) -> StarKVCheckpoint:
    """Every compressed layer of `path`, repacked (checkpoint.py:66-92). Raises
    ValueError for a layer in the legacy U/Sigma/V form and for a checkpoint with no
    compressed layer."""
    sd = torch.load(path, map_location="cpu", mmap=True, weights_only=True)
    layers = {}
    for li in range(num_layers):
        pre = _prefix(li)
        if f"{pre}k_proj.head_ranks" in sd:
            layers[li] = _repack_layer(sd, pre, li, num_kv_heads, head_dim, dtype, kv_quant)
        elif f"{pre}k_proj.Sigma_blocks.0.diag" in sd:
            raise ValueError(f"{path}: layer {li} is in the legacy U/Sigma/V format; serving needs the "
                             "fused format (Sigma folded into V, dead ranks pruned)")
    if not layers:
        raise ValueError(f"{path}: no fused STAR-KV layers found")
    return StarKVCheckpoint(layers=layers, skip_layers=tuple(li for li in range(num_layers) if li not in layers))


def _hadamard_fold(vs: torch.Tensor, u: torch.Tensor, ranks, gen: torch.Generator):
    """Per block of `ranks` rows (in order): VS_b <- T_b^T VS_b, U_b <- U_b T_b in
    float64, T_b = block_hadamard(rank, n_outlier(rank)) (checkpoint.py:96-103)."""
    vs, u = vs.double().clone(), u.double().clone()
    c = 0
    for r in ranks:
        t = block_hadamard(r, n_outlier(r), gen)
        vs[c:c + r] = t.T @ vs[c:c + r]
        u[:, c:c + r] = u[:, c:c + r] @ t
        c += r
    return vs.float(), u.float()


def _repack_layer(sd, pre, li, H, Hd, dtype, kv_quant) -> StarKVLayerWeights:
    """checkpoint.py:106-169."""
    ranks = [int(r) for r in sd[f"{pre}k_proj.head_ranks"].tolist()]
    if len(ranks) != H:
        raise ValueError(f"layer {li}: {len(ranks)} head ranks for {H} KV heads")
    k_vs = sd[f"{pre}k_proj.VS.weight"].float()
    k_u = sd[f"{pre}k_proj.U.weight"].float()
    R = sum(ranks)
    if k_vs.shape[0] != R or tuple(k_u.shape) != (H * Hd, R):
        raise ValueError(f"layer {li}: k_proj VS{tuple(k_vs.shape)} U{tuple(k_u.shape)} do not fit "
                         f"head ranks summing to {R} with H={H}, Hd={Hd}")
    if kv_quant:
        k_vs, k_u = _hadamard_fold(k_vs, k_u, ranks, torch.Generator().manual_seed(HADAMARD_SEED))

    hidden = k_vs.shape[1]
    widths = [_round_up(r, K_ALIGN) for r in ranks]
    offsets = [0] * H
    for h in range(1, H):
        offsets[h] = offsets[h - 1] + widths[h - 1]
    k_width = sum(widths)
    k_down = torch.zeros(k_width, hidden)
    k_up = torch.zeros(k_width, Hd)
    c = 0
    for h, r in enumerate(ranks):
        o = offsets[h]
        k_down[o:o + r] = k_vs[c:c + r]
        k_up[o:o + r] = k_u[h * Hd:(h + 1) * Hd, c:c + r].T  # head h's diagonal block, rank-major
        c += r

    v_vs = sd[f"{pre}v_proj.VS.weight"].float()
    v_u = sd[f"{pre}v_proj.U.weight"].float()
    rv = v_vs.shape[0]
    if tuple(v_u.shape) != (H * Hd, rv):
        raise ValueError(f"layer {li}: v_proj VS{tuple(v_vs.shape)} U{tuple(v_u.shape)}")
    if kv_quant:
        v_vs, v_u = _hadamard_fold(v_vs, v_u, [rv], torch.Generator().manual_seed(HADAMARD_SEED))
    rv_st = rv if kv_quant else _round_up(rv, V_ALIGN)
    v_down = torch.zeros(rv_st, hidden)
    v_down[:rv] = v_vs
    v_up = torch.zeros(H * Hd, rv_st)
    v_up[:, :rv] = v_u

    def i32(v):
        return torch.tensor(v, dtype=torch.int32)

    return StarKVLayerWeights(layer_idx=li, k_head_ranks=i32(ranks), k_head_widths=i32(widths),
                              k_head_offsets=i32(offsets), k_width=k_width, k_max_rank=max(widths),
                              k_down=k_down.to(dtype), k_up=k_up.to(dtype), v_rank=rv_st, v_rank_real=rv,
                              v_down=v_down.to(dtype), v_up=v_up.to(dtype), kv_quant=kv_quant)


@dataclass
class LayerOperands:
    """One layer's kernel operands on the device (attention.py:134-166)."""

    k_ranks: torch.Tensor         # [H_kv] int32
    k_head_offsets: torch.Tensor  # [H_kv] int32
    k_width: int
    k_up: torch.Tensor            # [k_width, Hd], rank-major
    v_up_by_q: torch.Tensor       # [H_q, v_rank, Hd]: query head h reads its KV head's V basis
    kv_down: torch.Tensor         # [k_width + v_rank, hidden]: hidden -> the cache row's codes
    v_rank: int
    row: Optional[QuantRow] = None         # 3.2-bit cache: the row layout
    k_nouts: Optional[torch.Tensor] = None
    head_of_lane: Optional[torch.Tensor] = None
    k_tiles: Optional[tuple] = None
    kv_groups: Optional[list] = None  # KV-head ranges, one decode call each (kv_head_groups)


def layer_operands(w: StarKVLayerWeights, num_heads: int, device, dtype: torch.dtype) -> LayerOperands:
    """The tensors ``paged_starkv_decode`` / ``paged_quant_decode`` and the write path
    take for layer `w`, with `num_heads` query heads (a multiple of the KV heads)."""
    H = w.k_head_ranks.numel()
    if num_heads % H:
        raise ValueError(f"{num_heads} query heads for {H} KV heads")
    # How the decode runs the layer, decided once here with the library's own rule
    # (starkv_decode_layer_groups): one call, or one call per range of consecutive KV heads
    # when the layer exceeds one call's heads, rank tiles or wave plan. A layer where a
    # single KV head does not fit one call is refused here (NotImplementedError), not at
    # serving time. The library must be built: these operands exist to be handed to it.
    # A 3.2-bit GQA layer is refused by StarKVAttentionImpl itself, as the reference does
    # (attention.py:116-117).
    ranks = w.k_head_ranks.tolist()
    groups = None
    if not w.kv_quant:
        groups = kv_head_groups(_hip.BF16, num_heads, ranks, w.v_rank)
    elif num_heads == H:
        groups = kv_head_groups(_hip.CACHE_Q3_2, num_heads, ranks, w.v_rank)
    Hd = w.k_up.shape[1]
    v_up = w.v_up.to(device=device, dtype=dtype)
    v_up_by_q = (v_up.view(H, Hd, w.v_rank).repeat_interleave(num_heads // H, dim=0)
                 .transpose(1, 2).contiguous())
    ops = LayerOperands(k_ranks=w.k_head_ranks.to(device), k_head_offsets=w.k_head_offsets.to(device),
                        k_width=w.k_width, k_up=w.k_up.to(device=device, dtype=dtype).contiguous(),
                        v_up_by_q=v_up_by_q,
                        kv_down=torch.cat([w.k_down, w.v_down]).to(device=device, dtype=dtype).contiguous(),
                        v_rank=w.v_rank, kv_groups=groups)
    if w.kv_quant:
        ops.row = QuantRow(w.k_width, H, w.v_rank)
        ops.k_nouts, ops.head_of_lane, ops.k_tiles = k_tables(w.k_head_ranks.tolist(), device)
    return ops


def write_fused_checkpoint(path: str, num_layers: int, num_kv_heads: int, head_dim: int, hidden: int,
                           compressed: dict, seed: int = 0, dtype: torch.dtype = torch.bfloat16) -> dict:
    """Writes a random-init checkpoint in the fused format and returns its state dict.

    `compressed` maps a layer index to ``(k_ranks, v_rank)``: per-KV-head K ranks and
    the shared V rank. Its factors are drawn so that codes of a unit-variance hidden
    state and the K/V they lift to have unit variance: VS ~ N(0, 1/hidden),
    U ~ N(0, 1/rank). Every other layer gets plain ``k_proj.weight`` /
    ``v_proj.weight`` [H*Hd, hidden], which the loader skips."""
    g = torch.Generator().manual_seed(seed)
    H, Hd = num_kv_heads, head_dim
    sd = {}

    def randn(*shape, std):
        return (torch.randn(*shape, generator=g) * std).to(dtype)

    for li in range(num_layers):
        pre = _prefix(li)
        if li not in compressed:
            sd[f"{pre}k_proj.weight"] = randn(H * Hd, hidden, std=hidden ** -0.5)
            sd[f"{pre}v_proj.weight"] = randn(H * Hd, hidden, std=hidden ** -0.5)
            continue
        ranks, rv = compressed[li]
        ranks = [int(r) for r in ranks]
        if len(ranks) != H or min(ranks) < 1 or rv < 1:
            raise ValueError(f"layer {li}: need {H} positive K ranks and a positive V rank")
        R = sum(ranks)
        k_u = torch.zeros(H * Hd, R)
        c = 0
        for h, r in enumerate(ranks):
            k_u[h * Hd:(h + 1) * Hd, c:c + r] = torch.randn(Hd, r, generator=g) * r ** -0.5
            c += r
        sd[f"{pre}k_proj.VS.weight"] = randn(R, hidden, std=hidden ** -0.5)
        sd[f"{pre}k_proj.U.weight"] = k_u.to(dtype)
        sd[f"{pre}k_proj.head_ranks"] = torch.tensor(ranks, dtype=torch.int32)
        sd[f"{pre}v_proj.VS.weight"] = randn(rv, hidden, std=hidden ** -0.5)
        sd[f"{pre}v_proj.U.weight"] = randn(H * Hd, rv, std=rv ** -0.5)
    torch.save(sd, path)
    return sd
