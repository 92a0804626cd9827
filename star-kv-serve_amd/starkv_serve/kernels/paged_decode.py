"""Paged STAR-KV decode over bf16/fp16 low-rank codes, on MI355X.

Drop-in for the reference's ``starkv_serve/kernels/paged_decode.py``: same function,
same arguments and meaning, same result (``[n, H_q, head_dim]`` in ``v_up_by_q``'s
dtype). The work runs in the HIP library (``libstarkv_hip.so``, launched through
``torch.ops.starkv.lowrank_decode``) on the current stream: a prep launch (page prefix
sums, wave plan, the query folded into each head's basis, and one 16-byte record per
cache page: its address, index and row count), one persistent decode kernel that streams
every cache page once through LDS, equal page ranges per workgroup, with the K logits on
MFMA and split-K partials, and a merge that also lifts the low-rank output through ``v_up_by_q``. No host
synchronisation; the grid is a function of ``(n, max_seq_len)`` only, so the call can be
graph-captured.

One library call takes at most 32 query heads and 96 rank tiles (a rank tile is 16 K lanes
seen by one query head). A larger layer (48- or 64-head MHA, wide GQA) is decoded as
groups of consecutive KV heads, one call per group: each call reads its group's K lanes
and the whole V code block, and writes its group's query heads (``kv_head_groups``).

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
from typing import Optional

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


def _forget_in(cache, key, r):
    entry = cache.get(key)
    if entry is not None and entry[0] is r:
        del cache[key]


def _forget(key, r):
    _forget_in(_cs_cache, key, r)


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


def _rows_for(two: bool, num_heads: int, max_seq_len: int) -> int:
    rows = MAX_REQUESTS_PER_LAUNCH
    if two:
        lcap = (int(max_seq_len) + 15) // 16 * 16
        rows = max(1, min(rows, MAX_LOGITS_PER_LAUNCH // (num_heads * lcap)))
    return rows


def rows_per_launch(cache_kind: int, num_heads: int, num_kv_heads: int, k_width: int, v_rank: int,
                    max_seq_len: int) -> int:
    """Requests per library call: at most 1024, and for two-pass decodes at most
    MAX_LOGITS_PER_LAUNCH logits."""
    key = (cache_kind, num_heads, num_kv_heads, k_width, v_rank, _hip.decode_path_epoch)
    two = _two_pass.get(key)
    if two is None:
        two = _two_pass[key] = bool(_hip.lib().starkv_decode_two_pass(cache_kind, num_heads, num_kv_heads, k_width,
                                                                      v_rank))
    return _rows_for(two, num_heads, max_seq_len)


_two_pass = {}  # (cache kind, H, H_kv, k_width, v_rank, path epoch) -> which decode form the library picks


def kv_head_groups(cache_kind: int, num_heads: int, k_ranks, v_rank: int) -> list:
    """KV-head ranges ``[(g0, g1), ...]`` decoded by one library call each: the whole layer
    when one call takes it, else greedy runs of consecutive KV heads, each as long as one
    call takes (``starkv_decode_layer_groups``, the library's own limits: 32 query heads,
    96 rank tiles and a wave plan of at most 16 tiles per wave per call). Raises
    NotImplementedError when a single KV head does not fit one call (more than 32 query
    heads per KV head, or more rank tiles over its query heads than those limits allow)."""
    ranks = [int(r) for r in k_ranks]
    groups = _hip.layer_groups(cache_kind, num_heads, len(ranks), ranks, v_rank)
    if not groups:
        raise NotImplementedError(f"STAR-KV HIP decode: a KV head of this layer ({num_heads} query heads over K ranks "
                                  f"{ranks}, v_rank {v_rank}) does not fit one decode call")
    return groups


# Host copies of device int tensors (a layer's KV-head ranks and offsets, the 3.2-bit tile
# table), keyed like the cos/sin copies: the head grouping needs them on the host, and
# reading them once per tensor keeps the decode free of host synchronisation afterwards.
# StarKVAttentionImpl computes its groups at load time and passes them in (kv_groups).
_host_cache = {}  # id(tensor) -> (weak reference, its version, list of ints)
_groups_cache = {}  # (kind, H, ranks, v_rank) -> kv_head_groups(...)


def _host_ints(t: torch.Tensor) -> list:
    if not t.is_cuda:
        return [int(x) for x in t.tolist()]
    key = id(t)
    hit = _host_cache.get(key)
    if hit is not None and hit[0]() is t and hit[1] == t._version:
        return hit[2]
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("STAR-KV HIP decode: the layer's head grouping is computed from its ranks on the host, "
                           "which cannot happen during graph capture: pass kv_groups, or run one decode of the "
                           "layer before capturing")
    vals = [int(x) for x in t.tolist()]
    _host_cache[key] = (weakref.ref(t, lambda r, k=key: _forget_in(_host_cache, k, r)), t._version, vals)
    return vals


def _groups_for(kind, num_heads, ranks, v_rank):
    key = (kind, num_heads, tuple(ranks), v_rank)
    g = _groups_cache.get(key)
    if g is None:
        g = _groups_cache[key] = kv_head_groups(kind, num_heads, ranks, v_rank)
    return g


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
    *,
    out: Optional[torch.Tensor] = None,
    kv_groups: Optional[list] = None,
) -> torch.Tensor:
    """Attention output per query head, ``[n, H_q, head_dim]`` (paged_decode.py:150-226).

    ``v_programs`` is accepted for API compatibility; the split-K layout is chosen
    by the library from the device and ``(n, max_seq_len)``. Keyword-only extensions, not
    in the reference's signature: ``out``, a tensor of that shape, bf16 / fp16 / fp32,
    written in place and returned (the attention layer hands over its output rows, saving
    a copy); ``kv_groups``, the layer's ``kv_head_groups`` computed once at load time (else
    they are computed here from a host copy of ``k_ranks``, read once per tensor).
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

    out = _hip.output_for(out, (n, num_heads, head_dim), v_up_by_q.dtype, query.device)
    if n == 0:
        return out
    ops = _hip.ops()
    cs = cos_sin_for_kernel(cos_sin_cache)
    block_table = _as_i32(block_table)
    seq_lens = _as_i32(seq_lens)
    kind = _hip.dtype_code(kv_cache)
    k_width, max_seq_len, scale = int(k_width), int(max_seq_len), float(scale)
    per = num_heads // num_kv_heads
    groups = kv_groups if kv_groups is not None else _groups_for(kind, num_heads, _host_ints(k_ranks), v_rank)
    if len(groups) == 1 and tuple(groups[0]) == (0, num_kv_heads):
        parts = [(query, out, kv_cache, k_up, _as_i32(k_ranks), _as_i32(k_head_offsets), v_up_by_q, num_heads,
                  num_kv_heads, k_width)]
    else:
        offs = _host_ints(k_head_offsets)
        ranks = _host_ints(k_ranks)
        parts = []
        for g0, g1 in groups:
            lo = offs[g0]
            kw = sum((r + 15) // 16 * 16 for r in ranks[g0:g1])
            parts.append((query[:, per * g0:per * g1], out[:, per * g0:per * g1], kv_cache[..., lo:],
                          k_up[lo:lo + kw], _as_i32(k_ranks[g0:g1]), _as_i32(k_head_offsets[g0:g1] - lo),
                          v_up_by_q[per * g0:per * g1], per * (g1 - g0), g1 - g0, kw))
    for qg, og, cg, kug, krg, kog, vug, hq, hkv, kw in parts:
        v_col = k_width - (cg.data_ptr() - kv_cache.data_ptr()) // kv_cache.element_size()
        step = rows_per_launch(kind, hq, hkv, kw, v_rank, max_seq_len)
        if step >= n:
            ops.lowrank_decode(qg, cg, block_table, seq_lens, max_seq_len, kug, krg, kog, kw, v_col, vug, cs, scale,
                               og)
            continue
        for s in range(0, n, step):
            e = min(n, s + step)
            ops.lowrank_decode(qg[s:e], cg, block_table[s:e], seq_lens[s:e], max_seq_len, kug, krg, kog, kw, v_col,
                               vug, cs, scale, og[s:e])
    return out
