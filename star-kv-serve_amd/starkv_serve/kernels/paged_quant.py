"""Paged decode over the 3.2-bit STAR-KV cache, and its write path, on MI355X.

Drop-in for the reference's ``starkv_serve/kernels/paged_quant.py``: the same
format constants, ``QuantRow`` byte layout, ``k_tables``, ``block_hadamard``,
``pack_kv``, ``fold_q`` and ``paged_quant_decode`` with the same arguments and
results. The format (kv_quant.py, paged_quant.py:1-30): per token and KV head the
leading ``int(0.2 * rank)`` channels are quantized at 4 bits and the rest at 3
bits, each block with one symmetric bfloat16 scale, after a block-Hadamard
rotation that the checkpoint loader folds into the bases. Codes are 4-bit nibbles
either way.

GPU work happens in ``libstarkv_hip.so``: ``pack_kv`` quantizes and scatters one row
per token (bit for bit ``kv_quant._q``: IEEE division, round-half-even); decode
unpacks nibbles in registers straight out of LDS (no dequantized copy), with the
K logits on MFMA and split-K partials merged and lifted at the end.
"""
import math
from dataclasses import dataclass
from typing import Optional

import torch

from starkv_serve import _hip
from starkv_serve.kernels.paged_decode import _as_i32, _groups_for, _host_ints, _rows_for, cos_sin_for_kernel

OUTLIER_RATIO = 0.2
HADAMARD_SEED = 1234
EPS = 1e-5                       # amax floor: an all-zero block still gets a scale
HEAD_DIM = 128


def n_outlier(rank: int) -> int:
    """Outlier channels of a block of `rank` channels (paged_quant.py:46-47)."""
    return int(OUTLIER_RATIO * rank)


def _sylvester(m: int) -> torch.Tensor:
    """m x m Sylvester-Hadamard matrix (m a power of two), float64, unnormalised."""
    h = torch.ones(1, 1, dtype=torch.float64)
    base = torch.tensor([[1.0, 1.0], [1.0, -1.0]], dtype=torch.float64)
    while h.shape[0] < m:
        h = torch.kron(base, h)
    return h


def block_hadamard(rank: int, n_out: int, generator: torch.Generator) -> torch.Tensor:
    """rank x rank orthonormal T = diag(H_outlier, H_inlier) in float64 on the CPU
    (paged_quant.py:50-68). Each block applies a Hadamard to its largest power-of-two
    leading part (identity on the rest) with random row signs drawn from `generator`;
    blocks of size <= 1 draw nothing, so the stream is consumed exactly as the
    reference consumes it."""
    T = torch.eye(rank, dtype=torch.float64)
    for start, size in ((0, n_out), (n_out, rank - n_out)):
        if size <= 1:
            continue
        m = 1 << (size.bit_length() - 1)
        flips = torch.rand(m, generator=generator, device="cpu") < 0.5
        signs = 1.0 - 2.0 * flips.to(torch.float64)
        T[start:start + m, start:start + m] = signs[:, None] * _sylvester(m) / math.sqrt(m)
    return T


@dataclass(frozen=True)
class QuantRow:
    """Byte layout of one token's row in a 3.2-bit layer's cache page (paged_quant.py:71-111):

      [0, ks_off)        K nibbles: lane 2k in the low nibble of byte k, 2k+1 in the high
      [ks_off, vs_off)   K scales: (outlier, inlier) bfloat16 per KV head
      [vs_off, vq_off)   V scales: (outlier, inlier) bfloat16
      [vq_off, +v_bytes) V nibbles, outlier channels first then inliers (byte-aligned)
      padded to a multiple of 16 bytes.
    """
    k_width: int
    num_kv_heads: int
    v_rank: int

    @property
    def v_nout(self) -> int:
        return n_outlier(self.v_rank)

    @property
    def ks_off(self) -> int:
        return self.k_width // 2

    @property
    def vs_off(self) -> int:
        return self.ks_off + 4 * self.num_kv_heads

    @property
    def vq_off(self) -> int:
        return self.vs_off + 4

    @property
    def v_nbo(self) -> int:
        return (self.v_nout + 1) // 2

    @property
    def v_bytes(self) -> int:
        return self.v_nbo + (self.v_rank - self.v_nout + 1) // 2

    @property
    def nbytes(self) -> int:
        return (self.vq_off + self.v_bytes + 15) // 16 * 16


def k_tables(ranks: list, device) -> tuple:
    """(outlier lanes per head, head of every K lane, per-16-lane-tile (head, outlier
    lanes, is its head's last)) as int32 tensors (paged_quant.py:114-131). A head's
    stored width is its rank rounded up to 16, so no tile spans two heads."""
    nouts = [n_outlier(r) for r in ranks]
    lane_head, tile_head, tile_nout, tile_last = [], [], [], []
    for h, (r, no) in enumerate(zip(ranks, nouts)):
        tiles = (r + 15) // 16
        lane_head.extend([h] * (16 * tiles))
        for j in range(tiles):
            tile_head.append(h)
            tile_nout.append(min(16, max(0, no - 16 * j)))
            tile_last.append(1 if j == tiles - 1 else 0)

    def as_t(v):
        return torch.tensor(v, dtype=torch.int32, device=device)

    return as_t(nouts), as_t(lane_head), (as_t(tile_head), as_t(tile_nout), as_t(tile_last))


def _slot_bits(slot_mapping: torch.Tensor) -> int:
    if slot_mapping.dtype == torch.int64:
        return 64
    if slot_mapping.dtype == torch.int32:
        return 32
    raise TypeError(f"slot_mapping dtype {slot_mapping.dtype}")


def pack_kv(k_codes, v_codes, cache, slot_mapping, row: QuantRow, k_ranks, k_offsets, k_nouts):
    """Quantize the step's codes into their slots of ``cache`` [num_blocks, block_size, row bytes]
    (paged_quant.py:205-216). Slot -1 (graph padding) goes to the null block 0."""
    n = k_codes.shape[0]
    assert k_codes.stride(-1) == 1 and v_codes.stride(-1) == 1
    assert cache.dtype == torch.uint8 and cache.shape[-1] == row.nbytes and cache.stride(-1) == 1
    assert k_codes.dtype == v_codes.dtype
    if n == 0:
        return
    _hip.require_cuda(k_codes, v_codes, cache, slot_mapping, k_ranks, k_offsets, k_nouts)
    k_ranks, k_offsets, k_nouts = (_as_i32(t) for t in (k_ranks, k_offsets, k_nouts))
    slot_mapping = slot_mapping.contiguous()
    _slot_bits(slot_mapping)
    _hip.ops().pack_kv(k_codes, v_codes, cache, slot_mapping, row.num_kv_heads, k_ranks, k_offsets, k_nouts,
                       row.k_width, row.v_rank, row.nbytes)


def fold_q(q, k_up, head_of_lane, scale):
    """q [n, H, 128] (RoPE applied), U^T [W, 128] -> A|B [n, W, 128] fp16 (paged_quant.py:241-255):

      A[r,i] = (q_i U[r,i] + q_{i+64} U[r,i+64]) * scale
      B[r,i] = (q_{i+64} U[r,i] - q_i U[r,i+64]) * scale

    with q of head head_of_lane[r], so q . RoPE_l(U^T x) = sum_r x[r] ([cos_l | sin_l] . AB[r]).
    """
    n, W = q.shape[0], k_up.shape[0]
    assert q.stride(-1) == 1 and k_up.stride(-1) == 1
    ab = torch.empty(n, W, HEAD_DIM, device=q.device, dtype=torch.float16)
    if n == 0 or W == 0:
        return ab
    _hip.require_cuda(q, k_up, head_of_lane)
    _hip.ops().fold_q(q, k_up, _as_i32(head_of_lane), float(scale), ab)
    return ab


def paged_quant_decode(
    query: torch.Tensor,
    kv_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    max_seq_len: int,
    row: QuantRow,
    k_up: torch.Tensor,
    head_of_lane: torch.Tensor,
    k_tiles: tuple,
    v_up_by_q: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    scale: float,
    target_v_programs: int = 2048,
    *,
    out: Optional[torch.Tensor] = None,
    kv_groups: Optional[list] = None,
) -> torch.Tensor:
    """Attention output per query head, ``[n, H, 128]`` (paged_quant.py:357-411). MHA only.

    ``head_of_lane`` and ``target_v_programs`` are accepted for API compatibility; the
    per-tile table ``k_tiles`` is what the kernel reads. Keyword-only extensions, not in the
    reference's signature: ``out``, a tensor of that shape, bf16 / fp16 / fp32, written in
    place and returned; ``kv_groups``, the layer's head ranges (``kv_head_groups`` over the
    heads' K widths), computed once at load time; else they are computed here from a host
    copy of the tile table, read once per tensor. A layer beyond one library call (more
    than 32 heads or 96 rank tiles) runs as one call per head range, each reading its
    heads' K nibbles and scales and the whole V block.
    """
    del head_of_lane, target_v_programs
    n, H, D = query.shape
    assert D == HEAD_DIM and H == row.num_kv_heads, "4-bit decode: MHA, head_dim 128"
    assert kv_cache.dtype == torch.uint8 and kv_cache.shape[-1] == row.nbytes
    assert cos_sin_cache.shape[-1] == D and cos_sin_cache.shape[0] >= max_seq_len
    th, tn, tl = k_tiles
    _hip.require_cuda(query, kv_cache, block_table, seq_lens, k_up, th, tn, tl, v_up_by_q, cos_sin_cache)
    if kv_cache.stride(-1) != 1 or query.stride(-1) != 1 or k_up.stride(-1) != 1 or v_up_by_q.stride(-1) != 1:
        raise ValueError("STAR-KV HIP decode: the last dimension of every operand must be contiguous")
    out = _hip.output_for(out, (n, H, D), v_up_by_q.dtype, query.device)
    if n == 0:
        return out
    ops = _hip.ops()
    cs = cos_sin_for_kernel(cos_sin_cache)
    block_table = _as_i32(block_table)
    seq_lens = _as_i32(seq_lens)
    th, tn, tl = (_as_i32(t) for t in (th, tn, tl))
    k_tiles_n = row.k_width // 16
    assert th.numel() == k_tiles_n, "k_tiles must cover k_width / 16 tiles"
    max_seq_len, scale = int(max_seq_len), float(scale)
    if kv_groups is None:
        kv_groups = _groups_for(_hip.CACHE_Q3_2, H, head_widths(_host_ints(th), H), row.v_rank)
    if len(kv_groups) == 1 and tuple(kv_groups[0]) == (0, H):
        parts = [(0, H, 0, row.k_width)]
    else:
        widths = head_widths(_host_ints(th), H)
        parts = [(h0, h1, sum(widths[:h0]), sum(widths[h0:h1])) for h0, h1 in kv_groups]
    for h0, h1, lane0, kw in parts:
        t0, t1 = lane0 // 16, (lane0 + kw) // 16
        qg, og, kug, vug = query[:, h0:h1], out[:, h0:h1], k_up[lane0:lane0 + kw], v_up_by_q[h0:h1]
        thg, tng, tlg = th[t0:t1], tn[t0:t1], tl[t0:t1]
        step = _rows_for(bool(_quant_two_pass(row, h0, h1, lane0, kw)), h1 - h0, max_seq_len)
        for s in range(0, n, step):
            e = min(n, s + step)
            ops.quant_decode(qg[s:e], kv_cache, block_table[s:e], seq_lens[s:e], max_seq_len, kw, row.v_rank,
                             row.nbytes, kug, thg, tng, tlg, vug, cs, scale, og[s:e], row.k_width, H, h0, lane0)
    return out


def head_widths(tile_head, num_heads: int) -> list:
    """Per-head K widths (16 lanes per tile) from the per-tile head table."""
    w = [0] * num_heads
    for h in tile_head:
        w[int(h)] += 16
    return w


_qtwo = {}  # (row, group, path epoch) -> whether the group's decode takes two passes


def _quant_two_pass(row: QuantRow, h0: int, h1: int, lane0: int, kw: int) -> bool:
    key = (row.k_width, row.num_kv_heads, row.v_rank, h0, h1, lane0, kw, _hip.decode_path_epoch)
    two = _qtwo.get(key)
    if two is None:
        two = _qtwo[key] = bool(_hip.lib().starkv_quant_group_two_pass(row.k_width, row.num_kv_heads, row.v_rank, h0,
                                                                       h1 - h0, lane0, kw))
    return two
