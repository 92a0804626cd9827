"""Dense causal prefill attention on MI355X (libstarkv_hip.so, starkv_prefill_attention).

The attention half of the STAR-KV layer's prefill (starkv_serve/attention.py:219-251 in
the reference, which hands the lifted K and V to vLLM's flash_attn_varlen_func with
causal=True): every prompt attends to itself, no cached context.
"""
import ctypes
from typing import List, Optional

import torch

from starkv_serve import _hip


def block_list(query_lens: List[int]) -> List[int]:
    """The kernel's workgroup rows, (prompt, query block) pairs flattened, from the
    library's host helper starkv_prefill_block_list (the query block size is the
    kernel's): the blocks with the most keys first."""
    cu = [0]
    for L in query_lens:
        if L < 0:
            raise ValueError(f"negative prompt length {L}")
        cu.append(cu[-1] + int(L))
    lib = _hip.lib()
    cu_c = (ctypes.c_int32 * len(cu))(*cu)
    n = lib.starkv_prefill_block_list(cu_c, len(query_lens), None, 0)
    buf = (ctypes.c_int32 * (2 * max(n, 1)))()
    if n < 0 or lib.starkv_prefill_block_list(cu_c, len(query_lens), buf, n) != n:
        raise RuntimeError("starkv_prefill_block_list failed")
    return list(buf)[:2 * n]


def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, query_lens: List[int], scale: float,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal attention of each prompt to itself.

    q [T, H_q, 128] (bf16, fp16 or fp32); k, v [T, H_kv, 128] (converted to fp16 once
    here when they are not); query_lens: the prompts' token counts (host ints, summing to
    T). Returns ``out`` [T, H_q, 128] (new, in q's dtype, when not given)."""
    T, Hq, D = q.shape
    assert D == 128 and k.shape == v.shape and k.shape[0] == T and k.shape[2] == D and Hq % k.shape[1] == 0
    assert sum(query_lens) == T
    if out is None:
        out = torch.empty_like(q)
    if T == 0:
        return out
    _hip.require_cuda(q, k, v, out)
    if k.dtype != torch.float16:
        k = k.to(torch.float16)
    if v.dtype != torch.float16:
        v = v.to(torch.float16)
    q = q if q.stride(-1) == 1 else q.contiguous()
    k, v = k.contiguous(), v.contiguous()
    cu = [0]
    for L in query_lens:
        cu.append(cu[-1] + int(L))
    blocks = block_list(query_lens)
    meta = torch.tensor(cu + blocks, dtype=torch.int32).to(q.device, non_blocking=True)
    cu_d = meta[:len(cu)]
    blk_d = meta[len(cu):].view(-1, 2)
    _hip.ops().prefill(q, k, v, cu_d, blk_d, float(scale), out)
    return out
