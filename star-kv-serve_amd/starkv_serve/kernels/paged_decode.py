"""Paged STAR-KV decode over bf16/fp16 low-rank codes, on MI355X.

Drop-in for the reference's ``starkv_serve/kernels/paged_decode.py``: same function,
same arguments and meaning, same result (``[n, H_q, head_dim]`` in ``v_up_by_q``'s
dtype). The work runs in the HIP library (``libstarkv_hip.so``) on the current
stream: a prep launch (token prefix sums and wave plan in one workgroup, the query
folded into each head's basis in the others), one persistent decode kernel that
streams every cache page once through LDS with the K logits on MFMA and split-K
partials, and a merge that also lifts the low-rank output through ``v_up_by_q``. No host synchronisation; the grid
is a function of ``(n, max_seq_len)`` only, so the call can be graph-captured.

Layout contract (reference paged_decode.py:150-174, attention.py:158-160):
  query          [n, H_q, 128], RoPE applied
  kv_cache       [num_blocks, block_size, k_width + v_rank]; per token the K codes of
                 every KV head at its own width (rank rounded up to 16), then V codes
  block_table    [n, max_blocks] int32;  seq_lens [n] int32 (including the new token)
  k_up           [k_width, 128] = U^T rank-major; k_ranks / k_head_offsets [H_kv] int32
  v_up_by_q      [H_q, v_rank, 128]
  cos_sin_cache  [>= max_seq_len, 128] = cat(cos, sin)
"""
import weakref

import torch

from starkv_serve import _hip

# Reference tuning constants (paged_decode.py:22-28). The HIP path sizes its own
# split; these remain for API compatibility.
BLOCK_L = 64
BLOCK_R = 16
NUM_WARPS = 4
MAX_BLOCK_V = 512
TARGET_V_PROGRAMS = 256

HEAD_DIM = 128
MAX_REQUESTS_PER_LAUNCH = 1024
# Two-pass decodes keep fp32 logits [n, H, max_seq_len] in their workspace; batches are
# split so that a launch's logits stay within this many elements (the reference bounds
# its logits buffer the same way, attention.py:50-53).
MAX_LOGITS_PER_LAUNCH = 1 << 26

# fp16 copies of cos/sin tables given in another dtype, keyed by the table object and
# checked against its version counter, so an in-place update or a new table at a reused
# address is converted again. Nothing is cached while a graph is being captured: a copy
# made there holds no values until the graph is replayed.
_cs_cache = {}  # id(table) -> (weak reference to the table, its version, fp16 copy)


def _forget(key, r):
    entry = _cs_cache.get(key)
    if entry is not None and entry[0] is r:
        del _cs_cache[key]


def cos_sin_for_kernel(cos_sin_cache: torch.Tensor) -> torch.Tensor:
    """The kernels read an fp16 table (the MFMA B operand). A table in another dtype is
    converted; every cos and sin value lies in [-1, 1], where fp16 keeps 11 significant
    bits (bf16 keeps 8), so a bf16 table converts exactly apart from values below
    fp16's normal range (2^-14), which become fp16 subnormals (absolute error < 2^-25).
    StarKVAttentionImpl converts its table once at load time."""
    if cos_sin_cache.dtype == torch.float16 and cos_sin_cache.stride(-1) == 1:
        return cos_sin_cache
    if cos_sin_cache.is_cuda and torch.cuda.is_current_stream_capturing():
        return cos_sin_cache.to(torch.float16).contiguous()
    key = id(cos_sin_cache)
    hit = _cs_cache.get(key)
    if hit is not None and hit[0]() is cos_sin_cache and hit[1] == cos_sin_cache._version:
        return hit[2]
    t = cos_sin_cache.to(torch.float16).contiguous()
    _cs_cache[key] = (weakref.ref(cos_sin_cache, lambda r, k=key: _forget(k, r)), cos_sin_cache._version, t)
    return t


def _as_i32(t: torch.Tensor) -> torch.Tensor:
    """int32 and contiguous (the kernels read these side tensors as plain int32 arrays)."""
    return (t if t.dtype == torch.int32 else t.to(torch.int32)).contiguous()


def rows_per_launch(cache_kind: int, num_heads: int, k_width: int, v_rank: int, max_seq_len: int) -> int:
    """Requests per library call: at most 1024, and for two-pass decodes at most
    MAX_LOGITS_PER_LAUNCH logits."""
    rows = MAX_REQUESTS_PER_LAUNCH
    if _hip.lib().starkv_decode_two_pass(cache_kind, num_heads, k_width, v_rank):
        lcap = (int(max_seq_len) + 15) // 16 * 16
        rows = max(1, min(rows, MAX_LOGITS_PER_LAUNCH // (num_heads * lcap)))
    return rows


def paged_starkv_decode(
    query: torch.Tensor,
    kv_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    max_seq_len: int,
    k_up: torch.Tensor,
    k_ranks: torch.Tensor,
    k_head_offsets: torch.Tensor,
    k_width: int,
    v_up_by_q: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    scale: float,
    v_programs: int = TARGET_V_PROGRAMS,
) -> torch.Tensor:
    """Attention output per query head, ``[n, H_q, head_dim]`` (paged_decode.py:150-226).

    ``v_programs`` is accepted for API compatibility; the split-K layout is chosen
    by the library from the device and ``(n, max_seq_len)``.
    """
    del v_programs
    n, num_heads, head_dim = query.shape
    num_kv_heads = k_ranks.numel()
    v_rank = v_up_by_q.shape[1]
    # Same preconditions as the reference (paged_decode.py:172-174).
    assert head_dim % 2 == 0 and num_heads % num_kv_heads == 0
    assert kv_cache.shape[-1] == k_width + v_rank, "cache width != K codes + V codes"
    assert cos_sin_cache.shape[-1] == head_dim and cos_sin_cache.shape[0] >= max_seq_len
    if head_dim != HEAD_DIM:
        raise NotImplementedError(f"STAR-KV HIP decode: head_dim {head_dim} (128 only)")
    if kv_cache.dtype not in (torch.bfloat16, torch.float16):
        raise NotImplementedError(f"STAR-KV HIP decode: cache dtype {kv_cache.dtype}")
    _hip.require_cuda(query, kv_cache, block_table, seq_lens, k_up, k_ranks, k_head_offsets, v_up_by_q,
                      cos_sin_cache)
    if kv_cache.stride(-1) != 1 or query.stride(-1) != 1 or k_up.stride(-1) != 1 or v_up_by_q.stride(-1) != 1:
        raise ValueError("STAR-KV HIP decode: the last dimension of every operand must be contiguous")

    out = torch.empty((n, num_heads, head_dim), dtype=v_up_by_q.dtype, device=query.device)
    if n == 0:
        return out
    L = _hip.lib()
    cs = cos_sin_for_kernel(cos_sin_cache)
    block_table = _as_i32(block_table)
    seq_lens = _as_i32(seq_lens)
    k_ranks = _as_i32(k_ranks)
    k_head_offsets = _as_i32(k_head_offsets)
    kind = _hip.dtype_code(kv_cache)
    step = rows_per_launch(kind, num_heads, int(k_width), v_rank, int(max_seq_len))
    stream = _hip.stream_of(query)
    for s in range(0, n, step):
        e = min(n, s + step)
        m = e - s
        grid = L.starkv_decode_grid_for(kind, m, num_heads, num_kv_heads, int(k_width), v_rank, int(max_seq_len))
        ws = torch.empty(L.starkv_decode_workspace_bytes(kind, m, num_heads, num_kv_heads, int(k_width), v_rank,
                                                         int(max_seq_len), grid),
                         dtype=torch.uint8, device=query.device)
        q, bt, o = query[s:e], block_table[s:e], out[s:e]
        rc = L.starkv_lowrank_decode(
            stream, q.data_ptr(), q.stride(0), q.stride(1), _hip.dtype_code(q),
            kv_cache.data_ptr(), kv_cache.stride(0), kv_cache.stride(1), kind, kv_cache.shape[1],
            bt.data_ptr(), bt.stride(0), bt.stride(1), seq_lens[s:e].data_ptr(), m, num_heads, num_kv_heads,
            int(max_seq_len), k_up.data_ptr(), k_up.stride(0), _hip.dtype_code(k_up), k_ranks.data_ptr(),
            k_head_offsets.data_ptr(), int(k_width), v_up_by_q.data_ptr(), v_up_by_q.stride(0), v_up_by_q.stride(1),
            _hip.dtype_code(v_up_by_q), v_rank, cs.data_ptr(), cs.stride(0), _hip.dtype_code(cs), float(scale),
            o.data_ptr(), o.stride(0), o.stride(1), _hip.dtype_code(o), ws.data_ptr(), ws.numel(), grid)
        _hip.check(rc, "paged_starkv_decode")
    return out
