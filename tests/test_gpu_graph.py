"""HIP-graph capture of the decode and write calls (the reference requires the decode
to be capturable with grids that depend on host ints only: paged_decode.py:201-202,
paged_quant.py:396-397; attention.py:196-197 captures it with max_seq_len =
max_model_len). Each graph is replayed several times with new inputs written in place,
with eager calls and synchronizations between the replays, and every replay must
equal the eager result bit for bit (the kernels are deterministic)."""
import pytest
import torch

from starkv_serve import checkpoint as ck
from starkv_serve import workloads as W
from starkv_serve.kernels.kv_write import write_kv
from starkv_serve.kernels.paged_decode import paged_starkv_decode
from starkv_serve.kernels.paged_quant import paged_quant_decode

pytestmark = pytest.mark.gpu

LENGTHS = [300, 77, 1000, 16, 513]
SPAN = 2048  # max_seq_len of the captured call (the graph's span), above every length


@pytest.mark.parametrize("quant", [False, True])
def test_decode_graph_replays(cuda, quant):
    print(f"\n[graph decode] quant={quant}", flush=True)
    if quant:
        wl = W.make_quant(LENGTHS, num_heads=8, ranks=[16, 32, 48, 64, 16, 32, 48, 64], seed=31, device=cuda,
                          max_seq_len=SPAN)
        fn = paged_quant_decode
    else:
        wl = W.make_lowrank(LENGTHS, num_heads=16, num_kv_heads=8, seed=31, max_seq_len=SPAN).to(cuda)
        fn = paged_starkv_decode
    args = wl.decode_args()
    fn(*args)  # warm-up (also converts and caches the cos/sin table)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out_g = fn(*args)
    gen = torch.Generator().manual_seed(7)
    for rep in range(4):
        wl.query.copy_(torch.randn(wl.query.shape, generator=gen).to(wl.query.dtype))
        lens = [max(1, L - int(torch.randint(0, L, (1,), generator=gen))) for L in LENGTHS]
        wl.seq_lens.copy_(torch.tensor(lens, dtype=wl.seq_lens.dtype))
        g.replay()
        torch.cuda.synchronize()
        eager = fn(*args)
        torch.cuda.synchronize()
        assert torch.isfinite(out_g).all(), rep
        assert torch.equal(out_g, eager), (rep, (out_g.float() - eager.float()).abs().max().item())


@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("n,hidden", [(24, 1024), (1, 1024), (2, 4096)])  # the split form; the direct form
def test_write_graph_replays(cuda, tmp_path, quant, n, hidden):
    print(f"\n[graph write] quant={quant} n={n} hidden={hidden}", flush=True)
    ranks = [16, 32, 48, 64]
    path = str(tmp_path / "w.pt")
    ck.write_fused_checkpoint(path, 1, len(ranks), 128, hidden, {0: (ranks, 64)}, seed=5)
    w = ck.load_fused_checkpoint(path, 1, len(ranks), 128, dtype=torch.bfloat16, kv_quant=quant).layers[0]
    ops = ck.layer_operands(w, len(ranks), cuda, torch.bfloat16)
    nb = 16
    if quant:
        cache = torch.zeros(nb, 16, ops.row.nbytes, dtype=torch.uint8, device=cuda)
        kw = dict(row=ops.row, k_ranks=ops.k_ranks, k_offsets=ops.k_head_offsets, k_nouts=ops.k_nouts)
    else:
        cache = torch.zeros(nb, 16, w.cache_width, dtype=torch.bfloat16, device=cuda)
        kw = {}
    x = torch.randn(n, hidden, device=cuda).to(torch.bfloat16)
    slots = torch.randperm(nb * 16, device=cuda)[:n]
    write_kv(x, ops.kv_down, cache, slots, w.k_width, **kw)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        write_kv(x, ops.kv_down, cache, slots, w.k_width, **kw)
    gen = torch.Generator().manual_seed(9)
    for rep in range(4):
        x.copy_(torch.randn(n, hidden, generator=gen).to(torch.bfloat16))
        slots.copy_(torch.randperm(nb * 16, generator=gen)[:n])
        cache.zero_()
        g.replay()
        torch.cuda.synchronize()
        got = cache.clone()
        cache.zero_()
        write_kv(x, ops.kv_down, cache, slots, w.k_width, **kw)
        torch.cuda.synchronize()
        assert torch.equal(got, cache), rep
        assert got.view(torch.uint8).any(), rep
