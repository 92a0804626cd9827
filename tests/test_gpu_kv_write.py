"""Fused cache write (starkv_write_kv: kv_down GEMM + scatter / 3.2-bit pack) on the GPU.

Pins:
- the codes it returns are the fp64 product hidden @ kv_down^T rounded once to the
  model dtype: within one unit in the last place of the truth, and equal to the
  correctly rounded value for all but the few codes whose fp32 sum lands across a
  rounding boundary (the GEMM's summation order differs from any other GEMM's);
- bf16/fp16 cache rows are those codes bit for bit; other slots are untouched;
- 3.2-bit rows equal the C oracle's packing (bit for bit kv_quant._q) of those codes
  on [0, vq_off + v_bytes), and the pad bytes are 0;
- slot -1 writes the null block 0; slots past the cache are skipped;
- the same for a prompt's many tokens (above FUSED_MAX_TOKENS: the codes from F.linear,
  then the store kernels);
- one token (hidden a multiple of 512) or two (hidden 4096) take the direct form (each
  workgroup owns whole codes): the same pins, K blocks wider than the form's LDS staging (144 codes)
  included, and 3.2-bit rows written without codes_out (no code-only jobs) equal those
  written with it.
"""
import math

import numpy as np
import pytest
import torch

from oracle import cquant, ref
from starkv_serve import checkpoint as ck
from starkv_serve.kernels.kv_write import write_codes, write_kv

pytestmark = pytest.mark.gpu

RANKS = [16, 32, 48, 64, 24, 16, 40, 56]
V_RANK = 40


def _layer(cuda, hidden, kv_quant, dtype, ranks=RANKS, v_rank=V_RANK):
    import tempfile
    import os
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "w.pt")
        ck.write_fused_checkpoint(path, 1, len(ranks), 128, hidden, {0: (ranks, v_rank)}, seed=hidden)
        w = ck.load_fused_checkpoint(path, 1, len(ranks), 128, dtype=dtype, kv_quant=kv_quant).layers[0]
    return w, ck.layer_operands(w, len(ranks), cuda, dtype)


def _ulp(x, dtype):
    """Spacing of `dtype` at |x| (float64 numpy)."""
    mant = 7 if dtype == torch.bfloat16 else 10
    e = np.floor(np.log2(np.maximum(np.abs(x), 1e-30)))
    return np.exp2(e - mant)


def _check_codes(codes, hidden, kv_down, dtype, label):
    truth = hidden.double().cpu().numpy() @ kv_down.double().cpu().numpy().T
    got = codes.double().cpu().numpy()
    err = np.abs(got - truth)
    assert np.all(err <= _ulp(truth, dtype) + 1e-6), (label, float(err.max()))
    exact = (codes.cpu() == torch.from_numpy(truth).to(dtype)).float().mean().item()
    print(f"{label}: codes correctly rounded {exact:.5f}, max |err| {err.max():.3g}", flush=True)
    assert exact > 0.99, label


def _slots(n, num_blocks, gen, past=None):
    """Distinct slots in [16, num_blocks * 16); the first token -1 (null block), the last
    one past the cache (by default when n > 2)."""
    s = torch.randperm(num_blocks * 16 - 16, generator=gen)[:n] + 16
    s[0] = -1
    if (n > 2) if past is None else past:
        s[-1] = num_blocks * 16 + 3
    return s


@pytest.mark.parametrize("n,hidden,dtype", [(1, 4096, torch.bfloat16), (2, 4096, torch.bfloat16),
                                            (2, 4096, torch.float16),
                                            (2, 3072, torch.float16), (1, 512, torch.float16),
                                            (1, 3072, torch.bfloat16), (37, 4096, torch.bfloat16),
                                            (64, 4096, torch.bfloat16), (130, 4096, torch.bfloat16),
                                            (9, 3072, torch.bfloat16), (21, 4096, torch.float16),
                                            (600, 4096, torch.bfloat16), (257, 4096, torch.float16)])
def test_write_kv_codes_and_cache(cuda, n, hidden, dtype):
    print(f"\n[write_kv] n={n} hidden={hidden} dtype={dtype}", flush=True)
    w, ops = _layer(cuda, hidden, False, dtype)
    g = torch.Generator().manual_seed(n)
    pad = 64 if n == 9 else 0  # strided hidden rows
    hid = (torch.randn(n, hidden + pad, generator=g)).to(dtype).to(cuda)[:, :hidden]
    nb = max(4, (n + 15) // 16 + 2)
    cache = torch.full((nb, 16, w.cache_width + 8), float("nan"), dtype=dtype, device=cuda)[:, :, :w.cache_width]
    slots = _slots(n, nb, g)
    before = cache.clone()
    codes = write_kv(hid, ops.kv_down, cache, slots.to(cuda), w.k_width, return_codes=True)
    torch.cuda.synchronize()
    _check_codes(codes, hid, ops.kv_down, dtype, f"n={n} hidden={hidden}")
    flat = cache.reshape(-1, w.cache_width)
    written = torch.zeros(nb * 16, dtype=torch.bool)
    for i, s in enumerate(slots.tolist()):
        s = max(s, 0)
        if s >= nb * 16:
            continue
        assert torch.equal(flat[s].view(torch.int16), codes[i].view(torch.int16)), (i, s)
        written[s] = True
    rest = ~written.to(cuda)
    assert torch.equal(flat[rest].view(torch.int16), before.reshape(-1, w.cache_width)[rest].view(torch.int16))


@pytest.mark.parametrize("n,ranks,v_rank,dtype", [(1, RANKS, V_RANK, torch.bfloat16),
                                                  (2, RANKS, V_RANK, torch.bfloat16),
                                                  (2, [144, 32, 16], 300, torch.bfloat16),
                                                  (1, [24] * 40, 1290, torch.float16),
                                                  (37, RANKS, V_RANK, torch.bfloat16),
                                                  (64, RANKS, V_RANK, torch.bfloat16),
                                                  (600, RANKS, V_RANK, torch.bfloat16)])
def test_write_kv_quant_rows(cuda, n, ranks, v_rank, dtype):
    print(f"\n[write_kv quant] n={n} heads={len(ranks)} v_rank={v_rank} dtype={dtype}", flush=True)
    w, ops = _layer(cuda, 4096, True, dtype, ranks, v_rank)
    row = ops.row
    g = torch.Generator().manual_seed(100 + n)
    hid = torch.randn(n, 4096, generator=g).to(dtype).to(cuda)
    nb = max(4, (n + 15) // 16 + 2)
    cache = torch.full((nb, 16, row.nbytes), 0xA5, dtype=torch.uint8, device=cuda)
    slots = _slots(n, nb, g)
    args = dict(row=row, k_ranks=ops.k_ranks, k_offsets=ops.k_head_offsets, k_nouts=ops.k_nouts)
    codes = write_kv(hid, ops.kv_down, cache, slots.to(cuda), w.k_width, return_codes=True, **args)
    cache2 = torch.full_like(cache, 0x5A)
    write_kv(hid, ops.kv_down, cache2, slots.to(cuda), w.k_width, **args)
    torch.cuda.synchronize()
    _check_codes(codes, hid, ops.kv_down, dtype, f"quant n={n}")
    lay = ref.row_layout(w.k_width, len(ranks), w.v_rank)
    assert lay["nbytes"] == row.nbytes
    c = codes.float().cpu().numpy()
    want = np.zeros((n, 1, row.nbytes), np.uint8)
    widths, offsets, _ = ref.head_layout(ranks)
    cquant.pack_kv(c[:, :w.k_width], c[:, w.k_width:], want, np.arange(n), ranks, offsets,
                   [ref.n_outlier(r) for r in ranks], w.v_rank, lay["ks_off"], lay["vs_off"], lay["vq_off"])
    flat2 = cache2.reshape(-1, row.nbytes).cpu().numpy()
    flat = cache.reshape(-1, row.nbytes).cpu().numpy()
    end = lay["vq_off"] + lay["v_bytes"]
    for i, s in enumerate(slots.tolist()):
        s = max(s, 0)
        if s >= nb * 16:
            continue
        assert np.array_equal(flat[s, :end], want[i, 0, :end]), (i, s)
        assert not flat[s, end:].any(), (i, s)
        assert np.array_equal(flat2[s], flat[s]), (i, s)  # written without codes_out


@pytest.mark.parametrize("quant", [False, True])
def test_write_kv_direct_skips_slots_past_the_cache(cuda, quant):
    """Two tokens (the direct form): token 0 to the null block, token 1 past the cache
    (skipped); every slot but slot 0 of block 0 keeps its bytes."""
    print(f"\n[write_kv direct past-cache] quant={quant}", flush=True)
    w, ops = _layer(cuda, 4096, quant, torch.bfloat16)
    g = torch.Generator().manual_seed(77)
    hid = torch.randn(2, 4096, generator=g).to(torch.bfloat16).to(cuda)
    nb = 4
    slots = _slots(2, nb, g, past=True)
    assert slots.tolist()[0] == -1 and slots.tolist()[1] >= nb * 16
    if quant:
        cache = torch.full((nb, 16, ops.row.nbytes), 0xA5, dtype=torch.uint8, device=cuda)
        args = dict(row=ops.row, k_ranks=ops.k_ranks, k_offsets=ops.k_head_offsets, k_nouts=ops.k_nouts)
    else:
        cache = torch.full((nb, 16, w.cache_width), 7.0, dtype=torch.bfloat16, device=cuda)
        args = {}
    before = cache.clone()
    codes = write_kv(hid, ops.kv_down, cache, slots.to(cuda), w.k_width, return_codes=True, **args)
    torch.cuda.synchronize()
    _check_codes(codes, hid, ops.kv_down, torch.bfloat16, f"direct past-cache quant={quant}")
    flat, flat0 = cache.reshape(nb * 16, -1), before.reshape(nb * 16, -1)
    assert torch.equal(flat[1:].view(torch.uint8), flat0[1:].view(torch.uint8)), "a slot other than the null slot changed"
    if quant:
        lay = ref.row_layout(w.k_width, len(RANKS), w.v_rank)
        c = codes.float().cpu().numpy()
        want = np.zeros((1, 1, ops.row.nbytes), np.uint8)
        widths, offsets, _ = ref.head_layout(RANKS)
        cquant.pack_kv(c[:1, :w.k_width], c[:1, w.k_width:], want, np.arange(1), RANKS, offsets,
                       [ref.n_outlier(r) for r in RANKS], w.v_rank, lay["ks_off"], lay["vs_off"], lay["vq_off"])
        end = lay["vq_off"] + lay["v_bytes"]
        got = flat[0].cpu().numpy()
        assert np.array_equal(got[:end], want[0, 0, :end]) and not got[end:].any()
    else:
        assert torch.equal(flat[0].view(torch.int16), codes[0].view(torch.int16))


def test_write_codes_matches_reference_scatter(cuda):
    """The unfused scatter: cache[slot // 16, slot % 16] = cat(key, value) (attention.py:179-184)."""
    g = torch.Generator().manual_seed(3)
    n, kw, rv = 50, 1280, 64
    key = torch.randn(n, kw, generator=g).to(torch.bfloat16).to(cuda)
    value = torch.randn(n, rv, generator=g).to(torch.bfloat16).to(cuda)
    cache = torch.zeros(8, 16, kw + rv, dtype=torch.bfloat16, device=cuda)
    slots = torch.randperm(8 * 16, generator=g)[:n].to(cuda)
    write_codes(key, value, cache, slots)
    want = torch.zeros_like(cache)
    want[slots // 16, slots % 16] = torch.cat([key, value], dim=1)
    torch.cuda.synchronize()
    assert torch.equal(cache, want)
