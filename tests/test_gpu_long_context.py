"""Long-context decode over the 3.2-bit cache with the write path in the loop: 16
requests at context 32768, 32 heads, head_dim 128, block size 16, per-head K ranks
from {16, 32, 48, 64}, V rank 64. Each of 32 steps appends one token per request
through the fused write (the layer's Hadamard-folded kv_down GEMM, quantize, pack,
scatter: model.py:71 + attention.py:186-188) and then decodes with the lengths one
longer (attention.py:194-213).

Pins, per step:
- the 16 rows written are byte-exact the C oracle's packing (kv_quant._q) of the
  codes the write returns;
- every output is finite.
On the first and the last step, two requests' outputs against the float64 oracle
over the same cache (the oracle takes about 6 s per 32K request), within the decode
tolerance (max-abs 2e-2, mean-rel 1e-3). The split over workgroups is the one of
the full 16-request batch, so those two requests cross the same split boundaries as
in the batch.
"""
import numpy as np
import pytest
import torch

from oracle import cquant, ref
from starkv_serve import checkpoint as ck
from starkv_serve import workloads as W
from starkv_serve.kernels.kv_write import write_kv
from starkv_serve.kernels.paged_quant import paged_quant_decode
from test_gpu_decode import assert_close

pytestmark = pytest.mark.gpu

N_REQ, CONTEXT, STEPS, HIDDEN = 16, 32768, 32, 4096
CHECKED = (0, N_REQ - 1)  # requests compared to the oracle


def test_long_context_quant_write_and_decode(cuda, tmp_path):
    print(f"\n[long context] {N_REQ} x {CONTEXT}, 3.2-bit, {STEPS} write + decode steps", flush=True)
    # The cache holds CONTEXT tokens per request; the first CONTEXT - STEPS are the prompt.
    wl = W.make_quant([CONTEXT] * N_REQ, num_heads=32, v_rank=64, seed=3003, device=cuda, gen_device=cuda)
    path = str(tmp_path / "fused_weights.pt")
    ck.write_fused_checkpoint(path, 1, 32, 128, HIDDEN, {0: (wl.ranks, wl.v_rank)}, seed=3004)
    w = ck.load_fused_checkpoint(path, 1, 32, 128, dtype=torch.bfloat16, kv_quant=True).layers[0]
    ops = ck.layer_operands(w, 32, cuda, torch.bfloat16)
    assert ops.k_width == wl.k_width and ops.row.nbytes == wl.row.nbytes
    lay = ref.row_layout(ops.k_width, 32, ops.v_rank)
    widths, offsets, _ = ref.head_layout(wl.ranks)
    nouts = [ref.n_outlier(r) for r in wl.ranks]
    end = lay["vq_off"] + lay["v_bytes"]

    g = torch.Generator().manual_seed(3005)
    bt = wl.block_table
    bt_host = bt.cpu().numpy()
    rows = torch.arange(N_REQ, device=cuda)
    for step in range(STEPS):
        pos = CONTEXT - STEPS + step
        slots = bt[rows, pos // 16].long() * 16 + pos % 16
        hidden = torch.randn(N_REQ, HIDDEN, generator=g).to(torch.bfloat16).to(cuda)
        codes = write_kv(hidden, ops.kv_down, wl.kv_cache, slots, ops.k_width, row=ops.row, k_ranks=ops.k_ranks,
                         k_offsets=ops.k_head_offsets, k_nouts=ops.k_nouts, return_codes=True)
        seq_lens = torch.full((N_REQ,), pos + 1, dtype=torch.int32, device=cuda)
        q = torch.randn(N_REQ, 32, 128, generator=g).to(torch.bfloat16).to(cuda)
        out = paged_quant_decode(q, wl.kv_cache, bt, seq_lens, CONTEXT, ops.row, ops.k_up, ops.head_of_lane,
                                 ops.k_tiles, ops.v_up_by_q, wl.cos_sin_cache, wl.scale)
        torch.cuda.synchronize()

        c = codes.float().cpu().numpy()
        want = np.zeros((N_REQ, 1, ops.row.nbytes), np.uint8)
        cquant.pack_kv(c[:, :ops.k_width], c[:, ops.k_width:], want, np.arange(N_REQ), wl.ranks, offsets, nouts,
                       ops.v_rank, lay["ks_off"], lay["vs_off"], lay["vq_off"])
        flat = wl.kv_cache.view(-1, ops.row.nbytes)
        got = flat[slots].cpu().numpy()
        assert np.array_equal(got[:, :end], want[:, 0, :end]), step
        assert torch.isfinite(out).all(), step

        if step in (0, STEPS - 1):
            idx = list(CHECKED)
            truth = ref.quant_decode(q[idx].float().cpu().numpy(), wl.kv_cache.cpu().numpy(), bt_host[idx],
                                     np.full(len(idx), pos + 1), CONTEXT, lay, wl.ranks,
                                     ops.k_up.float().cpu().numpy(), ops.v_up_by_q.float().cpu().numpy(),
                                     wl.cos_sin_cache.float().cpu().numpy(), wl.scale)
            assert_close(out[idx], truth, f"long context step {step} requests {idx}")
