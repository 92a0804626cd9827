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
    L = _hip.lib()
    block_table, seq_lens = _as_i32(block_table), _as_i32(seq_lens)
    ws = torch.empty(L.starkv_stock_decode_workspace_bytes(n, Hq, Hkv, int(max_seq_len)), dtype=torch.uint8,
                     device=query.device)
    rc = L.starkv_stock_decode(
        _hip.stream_of(query), query.data_ptr(), query.stride(0), query.stride(1), _hip.dtype_code(query),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        _hip.dtype_code(k_cache), k_cache.shape[1], block_table.data_ptr(), block_table.stride(0),
        block_table.stride(1), seq_lens.data_ptr(), n, Hq, Hkv, int(max_seq_len), float(scale), out.data_ptr(),
        out.stride(0), out.stride(1), _hip.dtype_code(out), ws.data_ptr(), ws.numel())
    _hip.check(rc, "paged_decode_full")
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
    bits = 64 if slots.dtype == torch.int64 else 32
    if bits == 32:
        slots = _as_i32(slots)
    rc = _hip.lib().starkv_stock_write(
        _hip.stream_of(key), key.data_ptr(), key.stride(0), key.stride(1), value.data_ptr(), value.stride(0),
        value.stride(1), _hip.dtype_code(key), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0),
        k_cache.stride(1), k_cache.stride(2), k_cache.shape[1], k_cache.shape[0], slots.data_ptr(), bits, n,
        key.shape[1])
    _hip.check(rc, "write_kv_full")
