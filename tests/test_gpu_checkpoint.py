"""One layer end to end on the GPU: a synthetic fused_weights.pt -> the loader ->
kernel operands -> codes of random hidden states written into a paged cache (bf16:
torch index_put, as attention.py:179-184; 3.2-bit: pack_kv) -> decode, against the
float64 oracle on the same cache. Tolerance as in test_gpu_decode."""
import numpy as np
import pytest
import torch

from oracle import ref
from starkv_serve import checkpoint as ck
from starkv_serve import workloads as W
from starkv_serve.kernels.paged_decode import paged_starkv_decode
from starkv_serve.kernels.paged_quant import pack_kv, paged_quant_decode
from test_gpu_decode import assert_close

pytestmark = pytest.mark.gpu

HD, HIDDEN = 128, 512
RANKS = [16, 32, 48, 64, 24, 16, 40, 56]  # 8 KV heads, ranks not all multiples of 16
V_RANK = 40                               # padded to 48 for the bf16 cache


@pytest.mark.parametrize("kv_quant,num_heads", [(False, 8), (False, 16), (True, 8)])
def test_checkpoint_layer_to_decode(cuda, tmp_path, kv_quant, num_heads):
    print(f"\n[checkpoint] kv_quant={kv_quant} num_heads={num_heads}", flush=True)
    path = str(tmp_path / "fused_weights.pt")
    ck.write_fused_checkpoint(path, num_layers=3, num_kv_heads=len(RANKS), head_dim=HD, hidden=HIDDEN,
                              compressed={1: (RANKS, V_RANK)}, seed=11)
    c = ck.load_fused_checkpoint(path, 3, len(RANKS), HD, dtype=torch.bfloat16, kv_quant=kv_quant)
    assert c.skip_layers == (0, 2)
    w = c.layers[1]
    ops = ck.layer_operands(w, num_heads, cuda, torch.bfloat16)

    g = torch.Generator().manual_seed(5)
    lengths = [300, 77, 16, 1]
    bt, nblk = W._page_layout(lengths, g)
    blocks, slots = W._token_slots(lengths, bt)
    T = sum(lengths)
    x = torch.randn(T, HIDDEN, generator=g).to(torch.bfloat16).to(cuda)
    codes = x @ ops.kv_down.T  # [T, k_width + v_rank]: what the model's kv_down GEMM writes
    slot_mapping = (blocks * W.BLOCK_SIZE + slots).to(cuda)
    if kv_quant:
        cache = torch.zeros(nblk, W.BLOCK_SIZE, ops.row.nbytes, dtype=torch.uint8, device=cuda)
        pack_kv(codes[:, :w.k_width], codes[:, w.k_width:], cache, slot_mapping, ops.row, ops.k_ranks,
                ops.k_head_offsets, ops.k_nouts)
    else:
        cache = torch.full((nblk, W.BLOCK_SIZE, w.cache_width), float("nan"), dtype=torch.bfloat16, device=cuda)
        cache[blocks.to(cuda), slots.to(cuda)] = codes

    n = len(lengths)
    q = torch.randn(n, num_heads, HD, generator=g).to(torch.bfloat16).to(cuda)
    seq_lens = torch.tensor(lengths, dtype=torch.int32, device=cuda)
    max_len = max(lengths)
    cs = W.cos_sin_table(max_len + 1, torch.bfloat16, cuda)
    scale = HD ** -0.5
    bt_d = bt.to(cuda)
    if kv_quant:
        out = paged_quant_decode(q, cache, bt_d, seq_lens, max_len, ops.row, ops.k_up, ops.head_of_lane,
                                 ops.k_tiles, ops.v_up_by_q, cs, scale)
        lay = ref.row_layout(w.k_width, len(RANKS), w.v_rank)
        truth = ref.quant_decode(q.float().cpu().numpy(), cache.cpu().numpy(), bt.numpy(), np.array(lengths),
                                 max_len, lay, RANKS, ops.k_up.float().cpu().numpy(),
                                 ops.v_up_by_q.float().cpu().numpy(), cs.float().cpu().numpy(), scale)
    else:
        out = paged_starkv_decode(q, cache, bt_d, seq_lens, max_len, ops.k_up, ops.k_ranks, ops.k_head_offsets,
                                  ops.k_width, ops.v_up_by_q, cs, scale)
        truth = ref.lowrank_decode(q.float().cpu().numpy(), cache.float().cpu().numpy(), bt.numpy(),
                                   np.array(lengths), max_len, ops.k_up.float().cpu().numpy(), RANKS,
                                   w.k_head_offsets.tolist(), w.k_width, ops.v_up_by_q.float().cpu().numpy(),
                                   cs.float().cpu().numpy(), scale)
    torch.cuda.synchronize()
    assert out.shape == (n, num_heads, HD)
    assert_close(out, truth, f"checkpoint kv_quant={kv_quant} heads={num_heads}")
