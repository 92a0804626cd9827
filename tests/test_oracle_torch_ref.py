"""Pin the fp32 PyTorch restatement (oracle/torch_ref.py, the CPU baseline's code)
against the float64 oracle and the C quantizer."""
import numpy as np
import torch

from oracle import cquant, ref, torch_ref
from starkv_serve import workloads as W


def test_lowrank_matches_float64_oracle():
    wl = W.make_lowrank([37, 5, 200, 16], num_heads=8, num_kv_heads=4, ranks=[16, 32, 20, 48], v_rank=32,
                        seed=21, poison=False)
    got = torch_ref.lowrank_decode(wl.query, wl.kv_cache, wl.block_table, wl.seq_lens, wl.max_seq_len, wl.k_up,
                                   wl.ranks, wl.k_head_offsets.tolist(), wl.k_width, wl.v_up_by_q,
                                   wl.cos_sin_cache, wl.scale).numpy()
    want = ref.lowrank_decode(wl.query.float().numpy(), wl.kv_cache.float().numpy(), wl.block_table.numpy(),
                              wl.seq_lens.numpy(), wl.max_seq_len, wl.k_up.float().numpy(), wl.ranks,
                              wl.k_head_offsets.tolist(), wl.k_width, wl.v_up_by_q.float().numpy(),
                              wl.cos_sin_cache.float().numpy(), wl.scale)
    assert np.abs(got - want).max() / np.abs(want).max() < 1e-5


def _quant_rows(wl, lay):
    """The C quantizer's packing of the workload's codes, as a cache."""
    widths, offsets, _ = ref.head_layout(wl.ranks)
    k, v = wl.k_codes.float().numpy(), wl.v_codes.float().numpy()
    rows = np.zeros((k.shape[0], 1, lay["nbytes"]), np.uint8)
    cquant.pack_kv(k, v, rows, np.arange(k.shape[0]), wl.ranks, offsets, [ref.n_outlier(r) for r in wl.ranks],
                   wl.v_rank, lay["ks_off"], lay["vs_off"], lay["vq_off"])
    return rows[:, 0]


def test_pack_rows_byte_exact_to_c_quantizer():
    for ranks, v_rank in (([16, 32, 48, 64], 64), ([20, 1, 33, 7], 37), ([64, 16], 1290)):
        wl = W.make_quant([40, 9], num_heads=len(ranks), ranks=ranks, v_rank=v_rank, seed=5, device="cpu")
        lay = ref.row_layout(wl.k_width, len(ranks), v_rank)
        want = _quant_rows(wl, lay)
        # exact .5 ties after the IEEE division, and all-zero blocks
        k = wl.k_codes.clone()
        k[0, :8] = torch.tensor([1.0, -1.0, 0.5, 3.5, -2.5, 7.0, 0.0, 0.25]).to(k.dtype)
        k[1, :] = 0
        wl.k_codes = k
        want = _quant_rows(wl, lay)
        got = torch_ref.pack_rows(wl.k_codes, wl.v_codes, lay, ranks).numpy()
        end = lay["vq_off"] + lay["v_bytes"]
        assert np.array_equal(got[:, :end], want[:, :end]), (ranks, v_rank)


def test_quant_matches_float64_oracle():
    wl = W.make_quant([37, 5, 200], num_heads=4, ranks=[16, 32, 20, 48], v_rank=40, seed=22, device="cpu")
    lay = ref.row_layout(wl.k_width, 4, wl.v_rank)
    rows = torch.from_numpy(_quant_rows(wl, lay))
    slots = wl.extra["slots"]
    cache = torch.zeros_like(wl.kv_cache)
    cache[slots // 16, slots % 16] = rows
    got = torch_ref.quant_decode(wl.query, cache, wl.block_table, wl.seq_lens, wl.max_seq_len, lay, wl.ranks,
                                 wl.k_up, wl.v_up_by_q, wl.cos_sin_cache, wl.scale).numpy()
    want = ref.quant_decode(wl.query.float().numpy(), cache.numpy(), wl.block_table.numpy(), wl.seq_lens.numpy(),
                            wl.max_seq_len, lay, wl.ranks, wl.k_up.float().numpy(), wl.v_up_by_q.float().numpy(),
                            wl.cos_sin_cache.float().numpy(), wl.scale)
    assert np.abs(got - want).max() / np.abs(want).max() < 1e-5
