"""Cache write of one layer step, on MI355X.

The reference computes a step's codes with the model's ``kv_down`` GEMM
(``starkv_serve/model.py:71``: ``kv = F.linear(hidden, kv_down)``) and writes them in
``StarKVAttentionImpl.forward`` (``attention.py:179-188``): ``cat`` + ``index_put``
into the bf16/fp16 cache, or ``pack_kv`` into the 3.2-bit cache. ``write_kv`` does
both in one call of the HIP library (``starkv_write_kv``: a split-K MFMA GEMM, then a
per-token store that rounds the codes to the model dtype exactly as ``F.linear``
returns them and scatters or quantizes them). ``write_codes`` is the unfused bf16/fp16
scatter of codes the caller already has (``starkv_write_codes``).

The fused kernel is built for a decode step's few tokens (its GEMM splits K to fill the
chip). A prompt's thousands of tokens take the codes' GEMM from the platform GEMM library
(``F.linear``: hipBLASLt, rounded once to the model dtype as the reference's own GEMM)
and then the same store kernels (``starkv_write_codes`` / ``starkv_pack_kv``): at 16,384
tokens, hidden 4096, 2160 codes, the fused kernel's GEMM takes 2.5 ms.
"""
from typing import Optional

import torch
import torch.nn.functional as F

from starkv_serve import _hip
from starkv_serve.kernels.paged_decode import _as_i32
from starkv_serve.kernels.paged_quant import QuantRow, pack_kv

# Tokens above which write_kv computes the codes with F.linear and then stores them.
FUSED_MAX_TOKENS = 256


def _slot_bits(slot_mapping: torch.Tensor) -> int:
    if slot_mapping.dtype == torch.int64:
        return 64
    if slot_mapping.dtype == torch.int32:
        return 32
    raise TypeError(f"slot_mapping dtype {slot_mapping.dtype}")


def write_kv(hidden: torch.Tensor, kv_down: torch.Tensor, kv_cache: torch.Tensor, slot_mapping: torch.Tensor,
             k_width: int, row: Optional[QuantRow] = None, k_ranks: Optional[torch.Tensor] = None,
             k_offsets: Optional[torch.Tensor] = None, k_nouts: Optional[torch.Tensor] = None,
             return_codes: bool = False, deferred: bool = False) -> Optional[torch.Tensor]:
    """Writes the codes of ``hidden`` [n, hidden_size] (bf16/fp16) under ``kv_down``
    [k_width + v_rank, hidden_size] into their slots of ``kv_cache``.

    Without ``row``: ``kv_cache`` [num_blocks, block_size, >= k_width + v_rank] of the
    model dtype gets the codes. With ``row`` (``QuantRow``): ``kv_cache`` uint8
    [num_blocks, block_size, row.nbytes] gets the packed 3.2-bit rows, with the K heads
    given by ``k_ranks`` / ``k_offsets`` / ``k_nouts`` (as ``pack_kv``). Slot -1 goes to
    the null block 0. Returns the rounded codes [n, k_width + v_rank] when
    ``return_codes`` (what ``F.linear(hidden, kv_down)`` returns), else None. Up to
    FUSED_MAX_TOKENS tokens run as one fused library call; more take F.linear, then the
    store. ``deferred`` (fused calls only): the write's launches wait for this thread's
    next decode call on the stream, which runs the code GEMM inside its own first launch
    (one launch fewer per decode step); the next write or ``flush_write()`` launches a
    write still pending."""
    n, hs = hidden.shape
    width = kv_down.shape[0]
    v_rank = width - k_width
    if kv_down.shape[1] != hs or v_rank <= 0:
        raise ValueError(f"kv_down {tuple(kv_down.shape)} does not fit hidden {tuple(hidden.shape)}, k_width {k_width}")
    if hidden.dtype != kv_down.dtype or hidden.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError("hidden and kv_down must share one dtype, bf16 or fp16")
    if hidden.stride(-1) != 1 or kv_down.stride(-1) != 1 or kv_cache.stride(-1) != 1:
        raise ValueError("the last dimension of hidden, kv_down and kv_cache must be contiguous")
    if row is not None:
        if kv_cache.dtype != torch.uint8 or kv_cache.shape[-1] != row.nbytes:
            raise ValueError("the 3.2-bit cache is uint8 [num_blocks, block_size, row.nbytes]")
        if (row.k_width, row.v_rank) != (k_width, v_rank):
            raise ValueError(f"row {row} does not match k_width {k_width}, v_rank {v_rank}")
    elif kv_cache.dtype != hidden.dtype:
        raise TypeError("the bf16/fp16 cache must have the model dtype")
    if n > FUSED_MAX_TOKENS:
        _hip.require_cuda(hidden, kv_down, kv_cache, slot_mapping)
        _slot_bits(slot_mapping)
        codes = F.linear(hidden, kv_down)
        if row is None:
            write_codes(codes[:, :k_width], codes[:, k_width:], kv_cache, slot_mapping)
        else:
            pack_kv(codes[:, :k_width], codes[:, k_width:], kv_cache, slot_mapping, row, k_ranks, k_offsets, k_nouts)
        return codes if return_codes else None
    codes = torch.empty(n, width, dtype=hidden.dtype, device=hidden.device) if return_codes else None
    if n == 0:
        return codes
    _hip.require_cuda(hidden, kv_down, kv_cache, slot_mapping)
    _slot_bits(slot_mapping)
    if row is not None:
        _hip.require_cuda(k_ranks, k_offsets, k_nouts)
        k_ranks, k_offsets, k_nouts = (_as_i32(t) for t in (k_ranks, k_offsets, k_nouts))
        heads, rb = row.num_kv_heads, row.nbytes
    else:
        heads, rb = 0, 0
    _hip.ops().write_kv(hidden, kv_down, int(k_width), kv_cache, slot_mapping.contiguous(), heads, k_ranks, k_offsets,
                        k_nouts, rb, codes, bool(deferred))
    return codes


def flush_write() -> None:
    """Launches this thread's deferred write (``write_kv(..., deferred=True)``), if any."""
    _hip.ops().flush_write()


def write_codes(key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """kv_cache[slot // block_size, slot % block_size] = cat(key, value) for every token
    (attention.py:179-184), cast to the cache dtype; slot -1 goes to the null block 0."""
    n = key.shape[0]
    if key.stride(-1) != 1 or value.stride(-1) != 1 or kv_cache.stride(-1) != 1:
        raise ValueError("the last dimension of key, value and kv_cache must be contiguous")
    if n == 0:
        return
    _hip.require_cuda(key, value, kv_cache, slot_mapping)
    _slot_bits(slot_mapping)
    _hip.ops().write_codes(key, value, kv_cache, slot_mapping.contiguous())
