"""starkv_lowrank_decode_noalloc (workspace in the library's fixed device array) against
starkv_lowrank_decode (workspace from the caller), through the C ABI: bit-identical
outputs on consecutive calls, the second smaller than the first, in the one-pass and
the two-pass form; a call whose workspace exceeds the array is refused."""
import pytest
import torch

from starkv_serve import _hip
from starkv_serve import workloads as W
from starkv_serve.kernels.paged_decode import cos_sin_for_kernel

pytestmark = pytest.mark.gpu


def decode(g, noalloc):
    L = _hip.lib()
    q, kv, bt, sl = g.query, g.kv_cache, g.block_table, g.seq_lens
    n, H, _ = q.shape
    Hkv = g.k_ranks.numel()
    grid = L.starkv_decode_grid(n, g.max_seq_len)
    out = torch.full((n, H, 128), float("nan"), dtype=g.v_up_by_q.dtype, device=q.device)
    cs, vq, U = cos_sin_for_kernel(g.cos_sin_cache), g.v_up_by_q, g.k_up
    args = [_hip.stream_of(q), q.data_ptr(), q.stride(0), q.stride(1), _hip.dtype_code(q), kv.data_ptr(),
            kv.stride(0), kv.stride(1), _hip.dtype_code(kv), kv.shape[1], bt.data_ptr(), bt.stride(0), bt.stride(1),
            sl.data_ptr(), n, H, Hkv, g.max_seq_len, U.data_ptr(), U.stride(0), _hip.dtype_code(U),
            g.k_ranks.data_ptr(), g.k_head_offsets.data_ptr(), g.k_width, g.k_width, vq.data_ptr(), vq.stride(0), vq.stride(1),
            _hip.dtype_code(vq), g.v_rank, cs.data_ptr(), cs.stride(0), _hip.dtype_code(cs), g.scale, out.data_ptr(),
            out.stride(0), out.stride(1), _hip.dtype_code(out)]
    if noalloc:
        rc = L.starkv_lowrank_decode_noalloc(*args, grid)
    else:
        ws = torch.empty(L.starkv_decode_workspace_bytes(_hip.dtype_code(kv), n, H, Hkv, g.k_width, g.v_rank,
                                                         g.max_seq_len, grid), dtype=torch.uint8, device=q.device)
        rc = L.starkv_lowrank_decode(*args, ws.data_ptr(), ws.numel(), grid)
    _hip.check(rc, "lowrank_decode_noalloc" if noalloc else "lowrank_decode")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("v_rank,ranks", [(64, None), (1280, [32] * 23 + [16] * 9)])
def test_noalloc_matches_workspace_entry(cuda, v_rank, ranks):
    cases = [[2000, 17, 700, 1024, 5, 333, 4096, 64], [300, 31, 9]]  # the second call is smaller
    for i, lengths in enumerate(cases):
        print(f"\n[noalloc] v_rank={v_rank} call {i}: {len(lengths)} requests", flush=True)
        g = W.make_lowrank(lengths, num_heads=32, ranks=ranks, v_rank=v_rank, seed=500 + i).to(cuda)
        want = decode(g, noalloc=False)
        got = decode(g, noalloc=True)
        assert torch.isfinite(got).all()
        assert torch.equal(got, want)


def test_noalloc_refuses_oversized_calls(cuda):
    L = _hip.lib()
    need = L.starkv_decode_workspace_bytes(_hip.BF16, 1024, 32, 32, 1280, 1280, 32768, 256)
    assert need > 64 << 20
    g = W.make_lowrank([100], num_heads=32, seed=7).to(cuda)
    q = g.query
    rc = L.starkv_lowrank_decode_noalloc(_hip.stream_of(q), q.data_ptr(), 0, 0, _hip.BF16, g.kv_cache.data_ptr(), 0,
                                         0, _hip.BF16, 16, g.block_table.data_ptr(), 0, 0, g.seq_lens.data_ptr(),
                                         1024, 32, 32, 32768, g.k_up.data_ptr(), 128, _hip.BF16, g.k_ranks.data_ptr(),
                                         g.k_head_offsets.data_ptr(), 1280, 1280, g.v_up_by_q.data_ptr(), 0, 0,
                                         _hip.BF16, 1280, 0, 128, _hip.F16, 1.0, 0, 0, 0, _hip.BF16, 256)
    assert rc != 0 and b"fixed scratch" in L.starkv_last_error()
