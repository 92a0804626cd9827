"""Uncompressed paged decode attention on MI355X (libstarkv_hip.so).

The attention of the layers a STAR-KV checkpoint keeps uncompressed (the reference
serves them with vLLM's stock LlamaAttention, starkv_serve/model.py:77-81), and the
stock bf16 comparator of the benchmarks. Decode only: every request's single query
token attends to its first ``seq_lens[b]`` cached tokens.
"""
import torch

from starkv_serve import _hip
from starkv_serve.kernels.paged_decode import _as_i32


def paged_decode_full(query: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_table: torch.Tensor,
                      seq_lens: torch.Tensor, max_seq_len: int, scale: float) -> torch.Tensor:
    """``[n, H_q, 128]`` attention output in the query's dtype.

    query [n, H_q, 128]; k_cache / v_cache [num_blocks, block_size, H_kv, 128] (bf16 or
    fp16, last dimension contiguous); block_table [n, max_blocks]; seq_lens [n]."""
    n, Hq, D = query.shape
    Hkv = k_cache.shape[2]
    assert D == 128 and k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride()
    assert Hq % Hkv == 0 and k_cache.stride(-1) == 1 and query.stride(-1) == 1
    out = torch.empty((n, Hq, D), dtype=query.dtype, device=query.device)
    if n == 0:
        return out
    _hip.require_cuda(query, k_cache, v_cache, block_table, seq_lens)
    block_table, seq_lens = _as_i32(block_table), _as_i32(seq_lens)
    _hip.ops().stock_decode(query, k_cache, v_cache, block_table, seq_lens, int(max_seq_len), float(scale), out)
    return out


def write_kv_full(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor) -> None:
    """The step's ``key`` / ``value`` [n, H_kv, 128] into the paged caches
    [num_blocks, block_size, H_kv, 128] at ``slot_mapping`` [n] (slot -1: nothing), as
    vLLM's reshape_and_cache does for uncompressed layers; one launch."""
    n = key.shape[0]
    assert key.shape == value.shape and key.shape[1:] == k_cache.shape[2:] and k_cache.shape == v_cache.shape
    assert key.dtype == value.dtype == k_cache.dtype == v_cache.dtype and k_cache.stride() == v_cache.stride()
    assert key.stride(-1) == 1 and value.stride(-1) == 1 and k_cache.stride(-1) == 1
    if n == 0:
        return
    _hip.require_cuda(key, value, k_cache, v_cache, slot_mapping)
    slots = slot_mapping.contiguous()
    if slots.dtype != torch.int64:
        slots = _as_i32(slots)
    _hip.ops().stock_write(key, value, k_cache, v_cache, slots)
