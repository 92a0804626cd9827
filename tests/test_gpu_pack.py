"""Cache write path on the GPU, bit for bit against the C oracle.

pack_kv (3.2-bit) must reproduce kv_quant._q exactly: every byte of
[0, vq_off + v_bytes) of every written row; the trailing pad bytes (never written by
the reference) are defined as 0 here. write_codes must equal torch's index_put.
"""
import numpy as np
import pytest
import torch

from oracle import cquant, ref
from starkv_serve.kernels import paged_quant as pq

pytestmark = pytest.mark.gpu


def _codes(n, W, R, ranks, offsets, widths, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(n, W, generator=g) * torch.exp(torch.randn(n, 1, generator=g) * 2)
    v = torch.randn(n, R, generator=g) * torch.exp(torch.randn(n, 1, generator=g) * 2)
    # exact rounding ties for some tokens: multiples of s/2 with s = 1
    k[0, offsets[0]:offsets[0] + 4] = torch.tensor([7.0, 3.5, 2.5, -0.5])
    k[1, :] = 0  # all-zero blocks
    v[2, :4] = torch.tensor([3.0, 1.5, -2.5, 0.5])
    for h, r in enumerate(ranks):
        k[:, offsets[h] + r:offsets[h] + widths[h]] = 0
    return k.to(dtype), v.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("ranks,R", [([16, 20, 48, 64, 33, 1, 128], 64), ([16, 32, 48, 64] * 8, 32),
                                     ([40, 24], 1290), ([5, 16], 7)])
def test_pack_kv_bit_exact(cuda, dtype, ranks, R):
    print(f"\n[pack_kv] dtype={dtype} ranks={len(ranks)} heads v_rank={R}", flush=True)
    widths, offsets, W = ref.head_layout(ranks)
    nouts = [ref.n_outlier(r) for r in ranks]
    row = pq.QuantRow(W, len(ranks), R)
    n, nb = 100, 12
    k, v = _codes(n, W, R, ranks, offsets, widths, dtype, seed=R)
    g = torch.Generator().manual_seed(1)
    init = torch.randint(0, 256, (nb, 16, row.nbytes + 32), generator=g, dtype=torch.uint8)
    slots = (torch.randperm((nb - 1) * 16, generator=g)[:n] + 16).to(torch.int64)
    slots[5] = -1  # padding token -> the null block's slot 0
    cache_ref = init.clone().numpy()
    cquant.pack_kv(k.float().numpy(), v.float().numpy(), cache_ref[:, :, :row.nbytes], slots.numpy(), ranks,
                   offsets, nouts, R, row.ks_off, row.vs_off, row.vq_off)
    buf = init.to(cuda)
    cache = buf[:, :, :row.nbytes]  # strided: slot stride nbytes + 32
    pq.pack_kv(k.to(cuda), v.to(cuda), cache, slots.to(cuda), row, torch.tensor(ranks, dtype=torch.int32, device=cuda),
               torch.tensor(offsets, dtype=torch.int32, device=cuda),
               torch.tensor(nouts, dtype=torch.int32, device=cuda))
    torch.cuda.synchronize()
    got = buf.cpu().numpy()
    end = row.vq_off + row.v_bytes
    written = np.zeros((nb, 16), bool)
    s = slots.clamp(min=0).numpy()
    written[s // 16, s % 16] = True
    assert np.array_equal(got[written][:, :end], cache_ref[written][:, :end])
    assert (got[written][:, end:row.nbytes] == 0).all()
    assert np.array_equal(got[~written], init.numpy()[~written])       # other rows untouched
    assert np.array_equal(got[:, :, row.nbytes:], init.numpy()[:, :, row.nbytes:])


def test_pack_kv_int32_slots(cuda):
    ranks, R = [16, 64], 32
    widths, offsets, W = ref.head_layout(ranks)
    row = pq.QuantRow(W, 2, R)
    k, v = _codes(8, W, R, ranks, offsets, widths, torch.bfloat16, seed=4)
    nouts, _, _ = pq.k_tables(ranks, cuda)
    c32 = torch.zeros(3, 16, row.nbytes, dtype=torch.uint8, device=cuda)
    c64 = torch.zeros_like(c32)
    sl = torch.arange(16, 24, device=cuda)
    args = (row, torch.tensor(ranks, dtype=torch.int32, device=cuda), torch.tensor(offsets, dtype=torch.int32,
                                                                                    device=cuda), nouts)
    pq.pack_kv(k.to(cuda), v.to(cuda), c32, sl.to(torch.int32), *args)
    pq.pack_kv(k.to(cuda), v.to(cuda), c64, sl, *args)
    assert torch.equal(c32, c64)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_write_codes_matches_index_put(cuda, dtype):
    from starkv_serve import _hip
    print(f"\n[write_codes] dtype={dtype}", flush=True)
    W, R, n, nb = 1280, 64, 37, 9
    g = torch.Generator().manual_seed(2)
    codes = torch.randn(n, W + R + 8, generator=g).to(dtype).to(cuda)  # key/value are views of one GEMM output
    key, value = codes[:, :W], codes[:, W:W + R]
    slots = (torch.randperm((nb - 1) * 16, generator=g)[:n] + 16).to(torch.int64).to(cuda)
    slots[3] = -1
    cache = torch.randn(nb, 16, W + R, generator=g).to(dtype).to(cuda)
    want = cache.clone()
    s = slots.clamp(min=0)
    want[s // 16, s % 16] = torch.cat([key, value], -1)
    rc = _hip.lib().starkv_write_codes(_hip.stream_of(cache), key.data_ptr(), key.stride(0), value.data_ptr(),
                                       value.stride(0), _hip.dtype_code(key), cache.data_ptr(), cache.stride(0),
                                       cache.stride(1), _hip.dtype_code(cache), 16, nb, slots.data_ptr(), 64, n, W, R)
    _hip.check(rc, "write_codes")
    torch.cuda.synchronize()
    assert torch.equal(cache, want)


@pytest.mark.parametrize("qdt,udt", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32)])
def test_fold_q_matches_oracle(cuda, qdt, udt):
    """starkv_fold_q: A|B of paged_quant.py:241-255 in fp16, against the float64 oracle
    (one fp16 rounding of an fp32 product: relative error <= 2^-11 of |A|B|, plus the
    fp32 rounding of two products)."""
    print(f"\n[fold_q] q {qdt}, k_up {udt}", flush=True)
    g = torch.Generator().manual_seed(12)
    ranks = [16, 48, 20, 64]
    nouts, lanes, _ = pq.k_tables(ranks, "cpu")
    W = lanes.numel()
    q = torch.randn(5, len(ranks), 128, generator=g).to(qdt)
    U = (torch.randn(W, 128, generator=g) * 0.3).to(udt)
    ab = pq.fold_q(q.to(cuda), U.to(cuda), lanes.to(cuda), 0.125)
    torch.cuda.synchronize()
    want = ref.fold_q(q.float().numpy(), U.float().numpy(), lanes.numpy(), 0.125)
    got = ab.float().cpu().numpy()
    assert got.shape == want.shape and ab.dtype == torch.float16
    err = np.abs(got - want)
    assert np.all(err <= np.abs(want) * 2.0 ** -10 + 1e-6), float(err.max())
