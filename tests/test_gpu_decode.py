"""Paged decode on the GPU (through the C ABI) against the float64 oracle.

Tolerance (bf16/fp16 outputs), per output tensor:
  max |out - truth| <= 2e-2
  mean |out - round(truth)| / mean |truth| <= 1e-3, round() = the output dtype
  all outputs finite (unused cache slots hold NaN: masking must keep them out)
The reference's own rounding error (logits stored in bf16, fp16 z accumulation) is
printed next to ours where it is emulated.
"""
import numpy as np
import pytest
import torch

from oracle import cquant, ref
from starkv_serve import _hip
from starkv_serve import workloads as W
from starkv_serve.kernels.paged_decode import cos_sin_for_kernel, paged_starkv_decode
from starkv_serve.kernels.paged_quant import paged_quant_decode

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_REL = 1e-3


def metrics(out, truth):
    o = out.float().cpu().numpy().astype(np.float64)
    tr = torch.from_numpy(truth).to(out.dtype).double().numpy()
    return dict(max_abs=float(np.abs(o - truth).max()),
                mean_rel=float(np.abs(o - tr).mean() / np.abs(truth).mean()),
                rel_l2=float(np.linalg.norm(o - truth) / np.linalg.norm(truth)),
                finite=bool(np.isfinite(o).all()))


def assert_close(out, truth, label):
    m = metrics(out, truth)
    print(f"{label}: {m}", flush=True)
    assert m["finite"], label
    assert m["max_abs"] <= MAX_ABS, (label, m)
    assert m["mean_rel"] <= MEAN_REL, (label, m)
    return m


def lowrank_truth(wl):
    """float64 oracle; the cache is handed over as float32 (exact for bf16/fp16 codes)."""
    cache = wl.kv_cache.cpu()
    if cache.dtype == torch.bfloat16:
        cache = (cache.view(torch.int16).numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    else:
        cache = cache.float().numpy()
    return ref.lowrank_decode(wl.query.float().cpu().numpy(), cache, wl.block_table.cpu().numpy(),
                              wl.seq_lens.cpu().numpy(), wl.max_seq_len, wl.k_up.float().cpu().numpy(), wl.ranks,
                              wl.k_head_offsets.tolist(), wl.k_width, wl.v_up_by_q.float().cpu().numpy(),
                              wl.cos_sin_cache.float().cpu().numpy(), wl.scale)


def run_lowrank(wl_gpu, grid=None):
    if grid is None:
        return paged_starkv_decode(*wl_gpu.decode_args())
    # Call the C ABI directly with an explicit split.
    q, kv, bt, sl = wl_gpu.query, wl_gpu.kv_cache, wl_gpu.block_table, wl_gpu.seq_lens
    n, H, _ = q.shape
    Hkv = wl_gpu.k_ranks.numel()
    tiles = (H // Hkv) * wl_gpu.k_width // 16
    out = torch.empty(n, H, 128, dtype=wl_gpu.v_up_by_q.dtype, device=q.device)
    L = _hip.lib()
    ws = torch.empty(L.starkv_decode_workspace_bytes(_hip.dtype_code(kv), n, H, Hkv, wl_gpu.k_width, wl_gpu.v_rank,
                                                     wl_gpu.max_seq_len, grid), dtype=torch.uint8, device=q.device)
    cs, vq, U = cos_sin_for_kernel(wl_gpu.cos_sin_cache), wl_gpu.v_up_by_q, wl_gpu.k_up  # the ABI takes fp16
    rc = L.starkv_lowrank_decode(_hip.stream_of(q), q.data_ptr(), q.stride(0), q.stride(1), _hip.dtype_code(q),
                                 kv.data_ptr(), kv.stride(0), kv.stride(1), _hip.dtype_code(kv), kv.shape[1],
                                 bt.data_ptr(), bt.stride(0), bt.stride(1), sl.data_ptr(), n, H, Hkv,
                                 wl_gpu.max_seq_len, U.data_ptr(), U.stride(0), _hip.dtype_code(U),
                                 wl_gpu.k_ranks.data_ptr(), wl_gpu.k_head_offsets.data_ptr(), wl_gpu.k_width,
                                 wl_gpu.k_width, vq.data_ptr(), vq.stride(0), vq.stride(1), _hip.dtype_code(vq), wl_gpu.v_rank,
                                 cs.data_ptr(), cs.stride(0), _hip.dtype_code(cs), wl_gpu.scale, out.data_ptr(),
                                 out.stride(0), out.stride(1), _hip.dtype_code(out), ws.data_ptr(), ws.numel(), grid)
    _hip.check(rc, "lowrank_decode")
    return out


LOWRANK_CASES = {
    # name: (lengths, kwargs)
    "b1_4096": ([4096], {}),
    "ragged_edges": ([1, 15, 16, 17, 100, 1000, 33, 2], {}),
    "gqa_h32_kv8": ([300, 17, 64], dict(num_kv_heads=8)),
    "fp16": ([513, 90, 2048], dict(dtype=torch.float16)),
    "strided_cache": ([200, 31], dict(col_pad=40)),
    "peaked_q": ([1500, 700], dict(peaked=4.0)),
    "v_rank_32": ([640, 129], dict(v_rank=32)),
    "v_rank_256_h16": ([333, 48], dict(v_rank=256, num_heads=16)),
    "graph_span": ([100, 37, 999], dict(max_seq_len=4096)),
    "ranks_not_16": ([77, 260], dict(ranks=[20, 1, 33, 64, 7, 48, 16, 50], num_heads=8)),
    "block_32": ([1000, 47, 64], dict(block_size=32)),
    "block_128": ([700, 129, 1], dict(block_size=128)),
    # pages too large for three LDS buffers: the two-buffer layout
    "wide_k1376": ([300, 17, 1024], dict(ranks=[48] * 22 + [32] * 10)),
    "wide_k1536_v256": ([150, 33], dict(ranks=[48] * 32, v_rank=256)),
    # beyond one call's 32 heads / 96 rank tiles: KV-head groups (v_col past the group's K)
    "groups_mha_rank64": ([250, 31, 1], dict(ranks=[64] * 32)),
    "groups_gqa_kv8_rank64": ([300, 17, 64], dict(num_kv_heads=8, ranks=[64] * 8)),
    "groups_mha_h48": ([200, 33, 5], dict(num_heads=48)),
    "groups_mha_h48_strided": ([120, 16], dict(num_heads=48, col_pad=40)),
    "groups_mha_h64_two_pass": ([150, 17], dict(num_heads=64, ranks=[32] * 40 + [16] * 24, v_rank=1280)),
    # 95 rank tiles, but nine heads of 8 tiles cannot share 8 waves of 16 tiles: the wave
    # plan splits the layer into groups (one call as a whole would return NaN rows)
    "groups_plan_w1520": ([250, 31], dict(ranks=[128] * 9 + [16] * 23)),
}


@pytest.mark.parametrize("name", list(LOWRANK_CASES))
def test_lowrank_decode_vs_oracle(cuda, name):
    lengths, kw = LOWRANK_CASES[name]
    kw = dict(kw)
    print(f"\n[lowrank] case={name} lengths={lengths[:8]} {kw}", flush=True)
    nh = kw.pop("num_heads", 32)
    wl = W.make_lowrank(lengths, num_heads=nh, seed=100 + len(name), **kw)
    out = paged_starkv_decode(*wl.to(cuda).decode_args())
    torch.cuda.synchronize()
    truth = lowrank_truth(wl)
    assert_close(out, truth, name)


def test_lowrank_reference_emulation_error_is_reported(cuda):
    wl = W.make_lowrank([700, 1100], num_heads=32, seed=5)
    out = paged_starkv_decode(*wl.to(cuda).decode_args())
    truth = lowrank_truth(wl)
    emu = ref.emulate_lowrank_reference(wl.query, wl.kv_cache, wl.block_table.numpy(), wl.seq_lens.numpy(),
                                        wl.max_seq_len, wl.k_up, wl.ranks, wl.k_head_offsets.tolist(), wl.k_width,
                                        wl.v_up_by_q, wl.cos_sin_cache, wl.scale)
    mo = assert_close(out, truth, "hip")
    me = metrics(torch.from_numpy(emu).to(out.dtype), truth)
    print(f"reference-rounding emulation: {me}", flush=True)
    assert mo["rel_l2"] <= me["rel_l2"] * 1.5 + 1e-4


def test_lowrank_bs64_ragged_full_size(cuda):
    lengths = W.ragged_lengths(1001)
    print(f"\n[lowrank] 64 requests, lengths U[1024, 8192]: {sum(lengths)} tokens", flush=True)
    wl = W.make_lowrank(lengths, num_heads=32, seed=1001, gen_device=cuda)
    g = wl.to(cuda)
    out = paged_starkv_decode(*g.decode_args())
    torch.cuda.synchronize()
    truth = lowrank_truth(wl)
    assert_close(out, truth, "bs64_ragged")
    # Size-independent property: permuting the physical pages changes nothing, bit for bit.
    nb = g.kv_cache.shape[0]
    perm = torch.cat([torch.zeros(1, dtype=torch.long), 1 + torch.randperm(nb - 1)]).to(cuda)
    inv = torch.argsort(perm).to(torch.int32)
    g2 = g.to(cuda)
    g2.kv_cache = g.kv_cache[perm]
    g2.block_table = inv[g.block_table.long()]
    out2 = paged_starkv_decode(*g2.decode_args())
    assert torch.equal(out, out2)
    # Different workgroup splits agree with the oracle too.
    for grid in (1, 7, 300):
        assert_close(run_lowrank(g, grid=grid), truth, f"bs64_ragged grid={grid}")


def test_lowrank_zero_length_and_truncation(cuda):
    wl = W.make_lowrank([50, 40, 30], num_heads=4, ranks=[16, 32, 48, 64], v_rank=32, seed=8)
    wl.seq_lens = torch.tensor([50, 0, 30], dtype=torch.int32)
    wl.max_seq_len = 40
    out = paged_starkv_decode(*wl.to(cuda).decode_args())
    truth = lowrank_truth(wl)
    assert torch.isnan(out[1]).all()       # softmax over an empty row, as the reference
    assert_close(out[[0, 2]], truth[[0, 2]], "truncated")


def test_decode_grid_rule(cuda):
    """Grid = min(CUs, max(n, ceil(n * max_seq_len / 256))): at least ~16 pages per
    workgroup, but a workgroup per request for short requests; never above the CUs."""
    L = _hip.lib()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    print(f"\n[grid] CUs={cus}", flush=True)
    for n, S in [(1, 4096), (1, 1), (64, 16), (64, 8192), (16, 32768), (300, 1), (1024, 48), (7, 700)]:
        want = min(cus, max(n, -(-n * S // 256)))
        assert L.starkv_decode_grid(n, S) == want, (n, S)
        # per layer: 64 tokens per workgroup (one-pass layers, and the logits pass of
        # two-pass ones; their P @ V pass takes ranges of several of those)
        for kind, kw, vr in ((_hip.BF16, 1280, 64), (_hip.BF16, 880, 1280), (_hip.CACHE_Q3_2, 1280, 64),
                             (_hip.CACHE_Q3_2, 880, 1290)):
            want = min(cus, max(n, -(-n * S // 64)))
            assert L.starkv_decode_grid_for(kind, n, 32, 32, kw, vr, S) == want, (kind, kw, vr, n, S)


def test_short_requests_one_workgroup_each(cuda):
    """64 requests of 16 tokens (one workgroup per request) against the oracle."""
    wl = W.make_lowrank([16] * 64, num_heads=32, seed=9)
    out = paged_starkv_decode(*wl.to(cuda).decode_args())
    torch.cuda.synchronize()
    assert_close(out, lowrank_truth(wl), "short requests")


def test_lowrank_block_size_not_power_of_two_is_rejected(cuda):
    # Pages are located with shifts, so block_size must be 16 * 2^s (16, 32, 64, ...).
    wl = W.make_lowrank([100, 20], num_heads=4, ranks=[16, 32, 48, 64], v_rank=32, seed=9, block_size=48)
    with pytest.raises(RuntimeError, match="power of two"):
        paged_starkv_decode(*wl.to(cuda).decode_args())


# ---------------------------------------------------------------------------
# 3.2-bit
# ---------------------------------------------------------------------------

def quant_truth(wl_gpu):
    cache = wl_gpu.kv_cache.cpu().numpy()
    lay = ref.row_layout(wl_gpu.k_width, len(wl_gpu.ranks), wl_gpu.v_rank)
    return ref.quant_decode(wl_gpu.query.float().cpu().numpy(), cache, wl_gpu.block_table.cpu().numpy(),
                            wl_gpu.seq_lens.cpu().numpy(), wl_gpu.max_seq_len, lay, wl_gpu.ranks,
                            wl_gpu.k_up.float().cpu().numpy(), wl_gpu.v_up_by_q.float().cpu().numpy(),
                            wl_gpu.cos_sin_cache.float().cpu().numpy(), wl_gpu.scale)


def check_packed_rows(wl_gpu, count=64):
    """The GPU-packed cache equals the C oracle's packing of the same codes (sampled rows)."""
    lay = ref.row_layout(wl_gpu.k_width, len(wl_gpu.ranks), wl_gpu.v_rank)
    slots = wl_gpu.extra["slots"].cpu().numpy()
    idx = np.linspace(0, len(slots) - 1, min(count, len(slots))).astype(int)
    k = wl_gpu.k_codes.float().cpu().numpy()[idx]
    v = wl_gpu.v_codes.float().cpu().numpy()[idx]
    want = np.zeros((len(idx), 1, lay["nbytes"]), np.uint8)
    widths, offsets, _ = ref.head_layout(wl_gpu.ranks)
    cquant.pack_kv(k, v, want, np.arange(len(idx)), wl_gpu.ranks, offsets,
                   [ref.n_outlier(r) for r in wl_gpu.ranks], wl_gpu.v_rank, lay["ks_off"], lay["vs_off"],
                   lay["vq_off"])
    c = wl_gpu.kv_cache.cpu().numpy()
    got = c[slots[idx] // c.shape[1], slots[idx] % c.shape[1]]
    end = lay["vq_off"] + lay["v_bytes"]
    assert np.array_equal(got[:, :end], want[:, 0, :end])


QUANT_CASES = {
    "b1_4096": ([4096], {}),
    "ragged_edges": ([1, 15, 16, 17, 100, 1000, 33, 2], {}),
    "v_rank_32": ([640, 129], dict(v_rank=32)),
    "peaked_q": ([1500, 700], dict(peaked=4.0)),
    "strided_cache": ([200, 31], dict(col_pad=48)),
    "graph_span": ([100, 37, 999], dict(max_seq_len=4096)),
    "fp16": ([513, 90], dict(dtype=torch.float16)),
    "block_64": ([900, 65, 3], dict(block_size=64)),
    # heads with more than 16 outlier ranks (several outlier tiles), a wave with more
    # tiles than it holds in registers, ranks that are not multiples of 16
    "big_heads": ([500, 77], dict(ranks=[256, 16, 100, 20], num_heads=4)),
    "ranks_not_16": ([77, 260], dict(ranks=[20, 1, 33, 64, 7, 48, 16, 50], num_heads=8)),
    # V lane maps over 3 and 5 blocks of 64 (outlier columns padded to 4)
    "v_rank_128": ([300, 45], dict(v_rank=128)),
    "v_rank_256_h8": ([200, 31], dict(v_rank=256, num_heads=8)),
    # beyond one call's 32 heads / 96 rank tiles / wave plan: head groups, each call
    # reading its heads' K nibbles and scales and the whole V block
    "groups_rank64_w2048": ([250, 31, 1], dict(ranks=[64] * 32)),
    "groups_w1792_v1290": ([150, 17], dict(ranks=[64] * 16 + [48] * 16, v_rank=1290)),
    "groups_h40": ([200, 33, 5], dict(num_heads=40)),
    # a group whose first K nibble sits 8 bytes into a 16-byte granule
    "groups_code_offset": ([120, 47], dict(ranks=[16] + [64] * 31)),
    "groups_plan_w1520": ([250, 31], dict(ranks=[128] * 9 + [16] * 23)),
}


@pytest.mark.parametrize("name", list(QUANT_CASES))
def test_quant_decode_vs_oracle(cuda, name):
    lengths, kw = QUANT_CASES[name]
    kw = dict(kw)
    print(f"\n[quant] case={name} lengths={lengths[:8]} {kw}", flush=True)
    nh = kw.pop("num_heads", 32)
    wl = W.make_quant(lengths, num_heads=nh, seed=200 + len(name), device=cuda, **kw)
    check_packed_rows(wl)
    out = paged_quant_decode(*wl.decode_args())
    torch.cuda.synchronize()
    assert_close(out, quant_truth(wl), name)


def test_quant_bs64_ragged_full_size(cuda):
    lengths = W.ragged_lengths(1002)
    print(f"\n[quant] 64 requests, lengths U[1024, 8192]: {sum(lengths)} tokens", flush=True)
    wl = W.make_quant(lengths, num_heads=32, seed=1002, device=cuda, gen_device=cuda)
    check_packed_rows(wl, count=256)
    out = paged_quant_decode(*wl.decode_args())
    torch.cuda.synchronize()
    assert_close(out, quant_truth(wl), "quant_bs64_ragged")


@pytest.mark.parametrize("quant", [False, True])
def test_more_requests_than_one_launch(cuda, quant):
    """1100 requests: the wrappers split the batch into library calls of at most 1024
    requests (attention.py:194-213 dispatches any batch); every request still matches."""
    g = torch.Generator().manual_seed(77)
    lengths = torch.randint(1, 48, (1100,), generator=g).tolist()
    print(f"\n[chunked] quant={quant} {len(lengths)} requests, {sum(lengths)} tokens", flush=True)
    if quant:
        wl = W.make_quant(lengths, num_heads=8, ranks=[16, 32, 48, 64, 16, 32, 48, 64], seed=78, device=cuda)
        out = paged_quant_decode(*wl.decode_args())
        torch.cuda.synchronize()
        assert_close(out, quant_truth(wl), "chunked quant")
    else:
        wl = W.make_lowrank(lengths, num_heads=8, seed=78).to(cuda)
        out = paged_starkv_decode(*wl.decode_args())
        torch.cuda.synchronize()
        assert_close(out, lowrank_truth(wl), "chunked bf16")


# ---------------------------------------------------------------------------
# Two-pass form: V ranks wider than the one-pass kernels take (the reference
# checkpoint's real shape, K width ~880 and V rank ~1290, train.py:360-362), and the
# two-pass form forced on the one-pass edge cases.
# ---------------------------------------------------------------------------

@pytest.fixture
def two_pass():
    prev = _hip.set_decode_path(2)
    yield
    _hip.set_decode_path(prev)


# K ranks of a 0.75-ratio layer: 880 lanes over 32 heads (widths multiples of 16).
RANKS_880 = [32] * 23 + [16] * 9


def subset_truth(wl, idx, quant):
    """The oracle on the requests idx only (requests are independent)."""
    sub = W.Workload(**{**wl.__dict__})
    sub.query = wl.query[idx]
    sub.block_table = wl.block_table[idx]
    sub.seq_lens = wl.seq_lens[idx]
    sub.lengths = [wl.lengths[i] for i in idx]
    return quant_truth(sub) if quant else lowrank_truth(sub)


@pytest.mark.parametrize("name", ["ragged_edges", "gqa_h32_kv8", "fp16", "strided_cache", "peaked_q",
                                  "graph_span", "ranks_not_16", "block_128", "wide_k1376", "v_rank_256_h16"])
def test_lowrank_two_pass_forced(cuda, two_pass, name):
    lengths, kw = LOWRANK_CASES[name]
    kw = dict(kw)
    print(f"\n[lowrank two-pass] case={name} lengths={lengths[:8]} {kw}", flush=True)
    nh = kw.pop("num_heads", 32)
    wl = W.make_lowrank(lengths, num_heads=nh, seed=100 + len(name), **kw)
    out = paged_starkv_decode(*wl.to(cuda).decode_args())
    torch.cuda.synchronize()
    assert_close(out, lowrank_truth(wl), name)


@pytest.mark.parametrize("name", ["ragged_edges", "v_rank_32", "strided_cache", "graph_span", "fp16",
                                  "block_64", "big_heads", "ranks_not_16", "v_rank_256_h8"])
def test_quant_two_pass_forced(cuda, two_pass, name):
    lengths, kw = QUANT_CASES[name]
    kw = dict(kw)
    print(f"\n[quant two-pass] case={name} lengths={lengths[:8]} {kw}", flush=True)
    nh = kw.pop("num_heads", 32)
    wl = W.make_quant(lengths, num_heads=nh, seed=200 + len(name), device=cuda, **kw)
    out = paged_quant_decode(*wl.decode_args())
    torch.cuda.synchronize()
    assert_close(out, quant_truth(wl), name)


def test_two_pass_grids_and_one_pass_agree(cuda, two_pass):
    """The two passes split the tokens identically for any grid; results agree with the
    one-pass form to within rounding."""
    wl = W.make_lowrank([700, 33, 1500, 16], num_heads=32, seed=31)
    g = wl.to(cuda)
    truth = lowrank_truth(wl)
    for grid in (1, 7, 300):
        assert_close(run_lowrank(g, grid=grid), truth, f"two-pass grid={grid}")
    two = paged_starkv_decode(*g.decode_args())
    _hip.set_decode_path(1)
    one = paged_starkv_decode(*g.decode_args())
    torch.cuda.synchronize()
    d = (two.float() - one.float()).abs().max().item()
    print(f"two-pass vs one-pass max |diff| = {d:.3e}", flush=True)
    assert d <= 2e-3


def test_two_pass_pv_ranges_over_logits_ranges(cuda, two_pass):
    """The P @ V pass over ranges of R = 1 .. 4 logits-pass ranges (the grid sets R: it is
    the grid over the split at 128 tokens per workgroup, here 47 for these lengths): every
    R against the oracle, with an empty request and requests that start and end inside
    the ranges."""
    wl = W.make_lowrank([700, 0, 1500, 16], num_heads=32, seed=33)
    g = wl.to(cuda)
    truth = lowrank_truth(wl)
    for grid in (47, 94, 141, 188, 200):
        print(f"\n[two-pass R] grid={grid}", flush=True)
        out = run_lowrank(g, grid=grid)
        torch.cuda.synchronize()
        o, t = out.float().cpu().numpy(), truth
        assert np.isnan(o[1]).all()  # the empty request: softmax over no tokens
        assert_close(out[[0, 2, 3]], t[[0, 2, 3]], f"two-pass grid={grid}")


def run_quant(wl_gpu, grid):
    """One 3.2-bit call through the C ABI with an explicit split."""
    q, kv, bt, sl = wl_gpu.query, wl_gpu.kv_cache, wl_gpu.block_table, wl_gpu.seq_lens
    n, H, _ = q.shape
    L = _hip.lib()
    out = torch.empty(n, H, 128, dtype=wl_gpu.v_up_by_q.dtype, device=q.device)
    ws = torch.empty(L.starkv_decode_workspace_bytes(_hip.CACHE_Q3_2, n, H, H, wl_gpu.k_width, wl_gpu.v_rank,
                                                     wl_gpu.max_seq_len, grid), dtype=torch.uint8, device=q.device)
    cs, vq, U = cos_sin_for_kernel(wl_gpu.cos_sin_cache), wl_gpu.v_up_by_q, wl_gpu.k_up
    th, tn, tl = wl_gpu.k_tiles
    rc = L.starkv_quant_decode(_hip.stream_of(q), q.data_ptr(), q.stride(0), q.stride(1), _hip.dtype_code(q),
                               kv.data_ptr(), kv.stride(0), kv.stride(1), kv.shape[1], bt.data_ptr(), bt.stride(0),
                               bt.stride(1), sl.data_ptr(), n, H, wl_gpu.max_seq_len, wl_gpu.k_width, wl_gpu.v_rank,
                               wl_gpu.row.nbytes, U.data_ptr(), U.stride(0), _hip.dtype_code(U), th.data_ptr(),
                               tn.data_ptr(), tl.data_ptr(), vq.data_ptr(), vq.stride(0), vq.stride(1),
                               _hip.dtype_code(vq), cs.data_ptr(), cs.stride(0), _hip.dtype_code(cs), wl_gpu.scale,
                               out.data_ptr(), out.stride(0), out.stride(1), _hip.dtype_code(out), ws.data_ptr(),
                               ws.numel(), grid)
    _hip.check(rc, "quant_decode")
    return out


def test_quant_two_pass_pv_ranges_and_windows(cuda):
    """3.2-bit P @ V over ranges of R = 1 .. 4 logits-pass ranges at V rank 1290 (W 880): the
    grids give R = 1 .. 4 and, short of the device's CUs, 2-4 column windows, each copying the
    V scales' bytes and its own chunks (the last window shorter); an empty request and
    requests that start and end inside the ranges."""
    wl = W.make_quant([700, 0, 1500, 16], num_heads=32, ranks=RANKS_880, v_rank=1290, seed=35, device=cuda)
    truth = quant_truth(wl)
    for grid in (47, 94, 141, 188, 200):
        print(f"\n[quant two-pass R] grid={grid}", flush=True)
        out = run_quant(wl, grid)
        torch.cuda.synchronize()
        o = out.float().cpu().numpy()
        assert np.isnan(o[1]).all()
        assert_close(out[[0, 2, 3]], truth[[0, 2, 3]], f"quant two-pass grid={grid}")


def test_two_pass_long_request_many_partials(cuda):
    """One request of 20,000 tokens at W 880, V rank 1280: the merge of its P @ V partials
    with every wave's batched loads in use (default grid: 157 partials, R = 2), and at grid
    1300 (16 tokens per logits range, R = 4: 313 partials) past the weights it keeps in
    registers (256), where it reads the ranges' maxima from memory."""
    wl = W.make_lowrank([20000], num_heads=32, seed=41, v_rank=1280, ranks=RANKS_880)
    g = wl.to(cuda)
    truth = lowrank_truth(wl)
    for grid in (None, 1300):
        print(f"\n[two-pass long] grid={grid}", flush=True)
        out = run_lowrank(g, grid=grid)
        torch.cuda.synchronize()
        assert_close(out, truth, f"two-pass long grid={grid}")


WIDE_CASES = {
    # name: (lengths, kwargs) -- V ranks the one-pass kernels do not take
    "bf16_v272": ([300, 17, 1024], dict(v_rank=272)),
    "bf16_v1024_w880": ([640, 129, 2000], dict(v_rank=1024, ranks=RANKS_880)),
    "bf16_v1296_w880": ([1, 15, 16, 17, 999, 4096], dict(v_rank=1296, ranks=RANKS_880)),
    "fp16_v1280_w880": ([513, 90, 2048], dict(v_rank=1280, ranks=RANKS_880, dtype=torch.float16)),
    "bf16_v2048_gqa": ([700, 64], dict(v_rank=2048, num_kv_heads=8, ranks=[32] * 8)),
    "bf16_v4096_h8": ([300, 31], dict(v_rank=4096, num_heads=8, ranks=[32] * 8)),  # two column windows
    "bf16_v1280_strided": ([200, 31], dict(v_rank=1280, ranks=RANKS_880, col_pad=48)),
    "bf16_v1280_graph_span": ([100, 37, 999], dict(v_rank=1280, ranks=RANKS_880, max_seq_len=4096)),
}


@pytest.mark.parametrize("name", list(WIDE_CASES))
def test_lowrank_wide_v_vs_oracle(cuda, name):
    lengths, kw = WIDE_CASES[name]
    kw = dict(kw)
    print(f"\n[lowrank wide] case={name} lengths={lengths[:8]} {kw}", flush=True)
    nh = kw.pop("num_heads", 32)
    wl = W.make_lowrank(lengths, num_heads=nh, seed=300 + len(name), **kw)
    two = _hip.lib().starkv_decode_two_pass(_hip.dtype_code(wl.kv_cache), nh, wl.k_ranks.numel(), wl.k_width,
                                            wl.v_rank)
    assert two == 1, (wl.k_width, wl.v_rank)
    out = paged_starkv_decode(*wl.to(cuda).decode_args())
    torch.cuda.synchronize()
    assert_close(out, lowrank_truth(wl), name)


QUANT_WIDE_CASES = {
    "v336": ([300, 17, 1024], dict(v_rank=336)),  # 67 outliers (padded to 68) + 269 inliers: 6 blocks
    "v1290_w880": ([1, 15, 16, 17, 999, 4096], dict(v_rank=1290, ranks=RANKS_880)),
    "v1024_w880_fp16": ([640, 129], dict(v_rank=1024, ranks=RANKS_880, dtype=torch.float16)),
    "v1291_odd": ([500, 77], dict(v_rank=1291, ranks=RANKS_880)),  # odd outlier count and inlier bytes
    "v4096_h8": ([300, 31], dict(v_rank=4096, num_heads=8, ranks=[32] * 8)),
    "v1290_graph_span": ([100, 37, 999], dict(v_rank=1290, ranks=RANKS_880, max_seq_len=4096)),
    "v1290_block64": ([900, 65, 3], dict(v_rank=1290, ranks=RANKS_880, block_size=64)),
    # one long request: 313 P @ V partials (3.2-bit: one per logits range), past the 256
    # merge weights held in registers
    "v1290_long": ([20000], dict(v_rank=1290, ranks=RANKS_880)),
}


@pytest.mark.parametrize("name", list(QUANT_WIDE_CASES))
def test_quant_wide_v_vs_oracle(cuda, name):
    lengths, kw = QUANT_WIDE_CASES[name]
    kw = dict(kw)
    print(f"\n[quant wide] case={name} lengths={lengths[:8]} {kw}", flush=True)
    nh = kw.pop("num_heads", 32)
    wl = W.make_quant(lengths, num_heads=nh, seed=400 + len(name), device=cuda, **kw)
    two = _hip.lib().starkv_decode_two_pass(_hip.CACHE_Q3_2, nh, nh, wl.k_width, wl.v_rank)
    assert two == 1, (wl.k_width, wl.v_rank)
    check_packed_rows(wl)
    out = paged_quant_decode(*wl.decode_args())
    torch.cuda.synchronize()
    assert_close(out, quant_truth(wl), name)


@pytest.mark.parametrize("quant", [False, True])
def test_wide_v_bs64_ragged_full_size(cuda, quant):
    """C1/C2-shaped batch (64 requests, lengths U[1024, 8192]) at the reference checkpoint's
    shape: K width 880, V rank 1280 (bf16, padded to 16) / 1290 (3.2-bit). The kernels run
    on all 64 requests; the oracle checks 8 of them (requests are independent), and a
    physical page permutation leaves every output bit-identical."""
    lengths = W.ragged_lengths(1006 + quant)
    print(f"\n[wide bs64] quant={quant} {sum(lengths)} tokens", flush=True)
    if quant:
        wl = W.make_quant(lengths, num_heads=32, ranks=RANKS_880, v_rank=1290, seed=1006, device=cuda,
                          gen_device=cuda)
        wl.k_codes = wl.v_codes = None
        out = paged_quant_decode(*wl.decode_args())
    else:
        wl = W.make_lowrank(lengths, num_heads=32, ranks=RANKS_880, v_rank=1280, seed=1006, gen_device=cuda).to(cuda)
        out = paged_starkv_decode(*wl.decode_args())
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    idx = [0, 9, 17, 26, 35, 44, 53, 63]
    assert_close(out[idx], subset_truth(wl, idx, quant), "wide bs64 subset")
    nb = wl.kv_cache.shape[0]
    perm = torch.cat([torch.zeros(1, dtype=torch.long), 1 + torch.randperm(nb - 1)]).to(cuda)
    inv = torch.argsort(perm).to(torch.int32)
    wl.kv_cache = wl.kv_cache[perm]
    wl.block_table = inv[wl.block_table.long()]
    out2 = paged_quant_decode(*wl.decode_args()) if quant else paged_starkv_decode(*wl.decode_args())
    assert torch.equal(out, out2)


def test_out_written_in_place(cuda):
    """`out=`: the kernels write the caller's rows (here fp32 columns of a wider, strided
    tensor) in place, bit-identical to a fresh output of the same dtype."""
    wl = W.make_lowrank([300, 17, 900], num_heads=32, seed=43).to(cuda)
    ref_out = paged_starkv_decode(*wl.decode_args()).float()
    wide = torch.full((3, 40, 128), float("nan"), dtype=torch.float32, device=cuda)
    got = paged_starkv_decode(*wl.decode_args(), out=wide[:, 4:36])
    assert got.data_ptr() == wide[:, 4:36].data_ptr()
    fresh = torch.empty(3, 32, 128, dtype=torch.float32, device=cuda)
    paged_starkv_decode(*wl.decode_args(), out=fresh)
    torch.cuda.synchronize()
    assert torch.equal(wide[:, 4:36], fresh)
    assert torch.isnan(wide[:, :4]).all() and torch.isnan(wide[:, 36:]).all()
    assert torch.equal(fresh.to(torch.bfloat16).float(), ref_out)  # same values, rounded once
    wq = W.make_quant([300, 17], num_heads=32, seed=44, device=cuda)
    oq = torch.empty(2, 32, 128, dtype=wq.v_up_by_q.dtype, device=cuda)
    assert paged_quant_decode(*wq.decode_args(), out=oq) is oq
    assert torch.equal(oq, paged_quant_decode(*wq.decode_args()))


def test_k_up_and_v_up_dtypes_independent(cuda):
    """k_up fp32 with v_up_by_q bf16 (and the reverse): each is read with its own dtype."""
    wl = W.make_lowrank([300, 17], num_heads=32, seed=41)
    truth = lowrank_truth(wl)
    g = wl.to(cuda)
    g.k_up = g.k_up.float()
    assert_close(paged_starkv_decode(*g.decode_args()), truth, "k_up fp32, v_up bf16")
    g = wl.to(cuda)
    g.v_up_by_q = g.v_up_by_q.float()
    out = paged_starkv_decode(*g.decode_args())
    assert out.dtype == torch.float32
    assert_close(out.to(torch.bfloat16), truth, "k_up bf16, v_up fp32")
