"""The fused-checkpoint loader, its kernel operands and the synthetic writer
(starkv_serve/checkpoint.py, after the reference's checkpoint.py:66-169 and
attention.py:134-166).

What pins the loader without the reference's own import:
- the product U VS of every K head and of V is what the checkpoint holds, exactly
  for the bf16/fp16 cache (a pure repack) and to fp32 rounding after the Hadamard
  fold of the 3.2-bit cache (T T^T = I);
- the rotated factors equal the oracle's block_hadamard (pinned by golden sign
  vectors) applied with a fresh generator per projection, head by head;
- widths, offsets, zero padding, skipped layers and the errors follow the format.
"""
import numpy as np
import pytest
import torch

from oracle import ref
from starkv_serve import checkpoint as ck
from starkv_serve.kernels.paged_quant import QuantRow

H, HD, HIDDEN = 4, 128, 96
LAYERS = {1: ([16, 24, 40, 64], 48), 3: ([32, 7, 16, 50], 32)}  # ranks not all multiples of 16


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("ckpt") / "fused_weights.pt")
    sd = ck.write_fused_checkpoint(path, num_layers=4, num_kv_heads=H, head_dim=HD, hidden=HIDDEN,
                                   compressed=LAYERS, seed=7, dtype=torch.float32)
    return path, sd


def _raw(sd, li):
    pre = f"model.layers.{li}.self_attn."
    return (sd[pre + "k_proj.VS.weight"].double(), sd[pre + "k_proj.U.weight"].double(),
            sd[pre + "v_proj.VS.weight"].double(), sd[pre + "v_proj.U.weight"].double())


@pytest.mark.parametrize("kv_quant", [False, True])
def test_layout(ckpt, kv_quant):
    path, _ = ckpt
    c = ck.load_fused_checkpoint(path, 4, H, HD, dtype=torch.float32, kv_quant=kv_quant)
    assert sorted(c.layers) == [1, 3] and c.skip_layers == (0, 2)
    assert c.is_compressed(1) and not c.is_compressed(0)
    for li, (ranks, rv) in LAYERS.items():
        w = c.layers[li]
        widths = [ref.align16(r) for r in ranks]
        assert w.k_head_ranks.tolist() == ranks and w.k_head_widths.tolist() == widths
        assert w.k_head_offsets.tolist() == [sum(widths[:h]) for h in range(H)]
        assert w.k_width == sum(widths) and w.k_max_rank == max(widths)
        assert w.v_rank_real == rv and w.v_rank == (rv if kv_quant else ref.align16(rv))
        assert w.k_down.shape == (w.k_width, HIDDEN) and w.k_up.shape == (w.k_width, HD)
        assert w.v_down.shape == (w.v_rank, HIDDEN) and w.v_up.shape == (H * HD, w.v_rank)
        for h, r in enumerate(ranks):  # rows between a head's rank and its width are zero
            o = w.k_head_offsets[h].item()
            assert not w.k_down[o + r:o + widths[h]].any() and not w.k_up[o + r:o + widths[h]].any()
        assert not w.v_down[rv:].any() and not w.v_up[:, rv:].any()
        if kv_quant:
            assert w.cache_bytes(2) == QuantRow(w.k_width, H, w.v_rank).nbytes
        else:
            assert w.cache_width == w.k_width + w.v_rank and w.cache_bytes(2) == 2 * w.cache_width


@pytest.mark.parametrize("kv_quant", [False, True])
def test_products_preserved(ckpt, kv_quant):
    """k_up[head rows]^T k_down[head rows] = U_h VS_h and v_up v_down = U_v VS_v."""
    path, sd = ckpt
    c = ck.load_fused_checkpoint(path, 4, H, HD, dtype=torch.float32, kv_quant=kv_quant)
    tol = 1e-5 if kv_quant else 0.0
    for li, (ranks, rv) in LAYERS.items():
        w = c.layers[li]
        kvs, ku, vvs, vu = _raw(sd, li)
        col = 0
        for h, r in enumerate(ranks):
            o = w.k_head_offsets[h].item()
            got = w.k_up[o:o + ref.align16(r)].double().T @ w.k_down[o:o + ref.align16(r)].double()
            want = ku[h * HD:(h + 1) * HD, col:col + r] @ kvs[col:col + r]
            assert (got - want).abs().max().item() <= tol * want.abs().max().item()
            col += r
        got = w.v_up.double() @ w.v_down.double()
        want = vu @ vvs
        assert (got - want).abs().max().item() <= tol * want.abs().max().item()


def test_rotation_matches_oracle_hadamard(ckpt):
    """3.2-bit cache: VS_h <- T_h^T VS_h, U_h <- U_h T_h with the oracle's T (golden-pinned),
    one generator per projection seeded 1234, consumed head by head."""
    path, sd = ckpt
    c = ck.load_fused_checkpoint(path, 4, H, HD, dtype=torch.float32, kv_quant=True)
    for li, (ranks, rv) in LAYERS.items():
        w = c.layers[li]
        kvs, ku, vvs, vu = (t.numpy() for t in _raw(sd, li))
        g = torch.Generator().manual_seed(1234)
        col = 0
        for h, r in enumerate(ranks):
            T = ref.block_hadamard(r, ref.n_outlier(r), g)
            o = w.k_head_offsets[h].item()
            np.testing.assert_allclose(w.k_down[o:o + r].numpy(), (T.T @ kvs[col:col + r]).astype(np.float32),
                                       rtol=0, atol=2e-6)
            np.testing.assert_allclose(w.k_up[o:o + r].numpy(),
                                       (ku[h * HD:(h + 1) * HD, col:col + r] @ T).T.astype(np.float32),
                                       rtol=0, atol=2e-6)
            col += r
        T = ref.block_hadamard(rv, ref.n_outlier(rv), torch.Generator().manual_seed(1234))
        np.testing.assert_allclose(w.v_down.numpy(), (T.T @ vvs).astype(np.float32), rtol=0, atol=2e-6)
        np.testing.assert_allclose(w.v_up.numpy(), (vu @ T).astype(np.float32), rtol=0, atol=2e-6)


def test_operands(ckpt):
    path, _ = ckpt
    for kv_quant in (False, True):
        c = ck.load_fused_checkpoint(path, 4, H, HD, dtype=torch.float32, kv_quant=kv_quant)
        w = c.layers[3]
        for nq in (H, 2 * H):
            ops = ck.layer_operands(w, nq, "cpu", torch.float32)
            grp = nq // H
            assert ops.v_up_by_q.shape == (nq, w.v_rank, HD) and ops.v_up_by_q.is_contiguous()
            for h in range(nq):
                kv = h // grp
                assert torch.equal(ops.v_up_by_q[h], w.v_up[kv * HD:(kv + 1) * HD].T)
            assert torch.equal(ops.kv_down, torch.cat([w.k_down, w.v_down]))
            assert ops.k_width == w.k_width and torch.equal(ops.k_up, w.k_up)
            if kv_quant:
                assert ops.row == QuantRow(w.k_width, H, w.v_rank)
                nouts, lanes, tiles = ref.k_tables(w.k_head_ranks.tolist())
                assert ops.k_nouts.tolist() == list(nouts) and ops.head_of_lane.tolist() == list(lanes)
                assert [t.tolist() for t in ops.k_tiles] == [list(x) for x in tiles]
            else:
                assert ops.row is None
        with pytest.raises(ValueError):
            ck.layer_operands(w, H + 1, "cpu", torch.float32)


def test_errors(tmp_path):
    base = ck.write_fused_checkpoint(str(tmp_path / "a.pt"), 2, H, HD, HIDDEN, {1: ([16] * H, 16)})
    # legacy U/Sigma/V layer
    legacy = dict(base)
    legacy["model.layers.0.self_attn.k_proj.Sigma_blocks.0.diag"] = torch.ones(4)
    torch.save(legacy, tmp_path / "legacy.pt")
    with pytest.raises(ValueError, match="legacy"):
        ck.load_fused_checkpoint(str(tmp_path / "legacy.pt"), 2, H, HD)
    # no compressed layer
    torch.save({"model.layers.0.self_attn.k_proj.weight": torch.zeros(4, 4)}, tmp_path / "none.pt")
    with pytest.raises(ValueError, match="no fused"):
        ck.load_fused_checkpoint(str(tmp_path / "none.pt"), 2, H, HD)
    # head-rank count and shape mismatches
    with pytest.raises(ValueError, match="head ranks"):
        ck.load_fused_checkpoint(str(tmp_path / "a.pt"), 2, H + 1, HD)
    bad = dict(base)
    bad["model.layers.1.self_attn.k_proj.U.weight"] = torch.zeros(H * HD, 5)
    torch.save(bad, tmp_path / "bad.pt")
    with pytest.raises(ValueError, match="k_proj"):
        ck.load_fused_checkpoint(str(tmp_path / "bad.pt"), 2, H, HD)
    bad = dict(base)
    bad["model.layers.1.self_attn.v_proj.U.weight"] = torch.zeros(H * HD, 3)
    torch.save(bad, tmp_path / "badv.pt")
    with pytest.raises(ValueError, match="v_proj"):
        ck.load_fused_checkpoint(str(tmp_path / "badv.pt"), 2, H, HD)
    with pytest.raises(ValueError):
        ck.write_fused_checkpoint(str(tmp_path / "c.pt"), 2, H, HD, HIDDEN, {1: ([16] * (H - 1), 16)})


def test_writer_statistics(tmp_path):
    """Codes of a unit-variance hidden state, and the K they lift to, have about unit variance."""
    sd = ck.write_fused_checkpoint(str(tmp_path / "s.pt"), 1, H, HD, 1024, {0: ([64] * H, 64)}, seed=3,
                                   dtype=torch.float32)
    w = ck.load_fused_checkpoint(str(tmp_path / "s.pt"), 1, H, HD, dtype=torch.float32).layers[0]
    x = torch.randn(2048, 1024, generator=torch.Generator().manual_seed(5))
    codes = x @ w.k_down.T
    assert 0.8 < codes.std().item() < 1.2
    k0 = codes[:, :64] @ w.k_up[:64]
    assert 0.8 < k0.std().item() < 1.2
    assert sd["model.layers.0.self_attn.k_proj.head_ranks"].dtype == torch.int32


def test_layer_the_decode_cannot_run_is_refused_at_load(tmp_path):
    """layer_operands replays the decode's wave plan on the host: a head of rank 272
    (17 rank tiles, above the 16 a decode wave holds) raises NotImplementedError at load
    time instead of decoding to NaN rows; 32 heads of rank 64 (128 rank tiles, above the
    96 one call takes) load, as KV-head groups."""
    path = str(tmp_path / "wide_k.pt")
    ck.write_fused_checkpoint(path, 2, 32, HD, 256, {0: ([272] + [16] * 31, 64), 1: ([64] * 32, 64)}, seed=9)
    layers = ck.load_fused_checkpoint(path, 2, 32, HD, dtype=torch.bfloat16).layers
    with pytest.raises(NotImplementedError):
        ck.layer_operands(layers[0], 32, torch.device("cpu"), torch.bfloat16)
    ck.layer_operands(layers[1], 32, torch.device("cpu"), torch.bfloat16)


@pytest.mark.parametrize("H,ranks,v_rank,want", [
    (32, [32] * 8, 64, None),                              # 64 tiles: fits one call
    (32, [64] * 32, 64, [(0, 24), (24, 32)]),              # MHA, 128 tiles: 96 + 32
    (32, [64] * 8, 64, [(0, 6), (6, 8)]),                  # GQA 4 heads per KV head, 128 tiles
    (48, [16] * 48, 64, [(0, 32), (32, 48)]),              # 48 heads: 32 + 16
    (64, [32] * 64, 1280, [(0, 32), (32, 64)]),            # two-pass layers split the same way
    (32, [128] * 8, 64, [(0, 3), (3, 6), (6, 8)]),         # GQA 4 heads per KV head of 8 tiles: 96 tiles a call
])
def test_kv_head_groups_partition(H, ranks, v_rank, want):
    """kv_head_groups: consecutive KV-head runs that cover the layer once, each a shape one
    library call takes (the host test the library applies), each as long as possible."""
    from starkv_serve import _hip
    from starkv_serve.kernels.paged_decode import kv_head_groups
    g = kv_head_groups(_hip.BF16, H, ranks, v_rank)
    hkv = len(ranks)
    per = H // hkv
    assert g == (want or [(0, hkv)])
    assert g[0][0] == 0 and g[-1][1] == hkv and all(a[1] == b[0] for a, b in zip(g, g[1:]))
    for g0, g1 in g:
        assert _hip.layer_fits(_hip.BF16, per * (g1 - g0), g1 - g0, ranks[g0:g1], v_rank)
        if g1 < hkv:  # one more KV head would not fit
            assert not _hip.layer_fits(_hip.BF16, per * (g1 + 1 - g0), g1 + 1 - g0, ranks[g0:g1 + 1], v_rank)


def test_kv_head_groups_refuses_a_kv_head_that_does_not_fit():
    from starkv_serve import _hip
    from starkv_serve.kernels.paged_decode import kv_head_groups
    with pytest.raises(NotImplementedError):
        kv_head_groups(_hip.BF16, 64, [16], 64)               # 64 query heads on one KV head
    with pytest.raises(NotImplementedError):
        kv_head_groups(_hip.BF16, 32, [208] * 4, 64)          # 8 heads x 13 tiles = 104 > 96


def test_side_tensors_normalised_to_contiguous_int32():
    """The decode wrappers pass side tensors (lengths, block tables, ranks, tile tables)
    as plain int32 arrays: strided or int64 inputs are converted, not misread."""
    from starkv_serve.kernels.paged_decode import _as_i32
    base = torch.arange(20, dtype=torch.int64)
    strided = base[::2]
    out = _as_i32(strided)
    assert out.dtype == torch.int32 and out.is_contiguous() and torch.equal(out, strided.to(torch.int32))
    same = torch.arange(5, dtype=torch.int32)
    assert _as_i32(same) is same


def _plan_fits_restated(tiles):
    """The decode's wave plan, restated: heads sorted by decreasing tiles (ties: lower
    head first) dealt to 8 waves in snake order, then, while the most loaded wave (ties:
    the higher index) is above ceil(total / 8), the head swap that lowers it the most
    (smallest resulting maximum, then lowest head indices); fits if no wave holds more
    than 16 tiles."""
    Hq, TT = len(tiles), sum(tiles)
    if not 1 <= Hq <= 32 or not 1 <= TT <= 96:
        return False
    order = sorted(range(Hq), key=lambda h: (-tiles[h], h))
    size = [tiles[h] for h in order]
    wave = [(p % 8) if (p // 8) % 2 == 0 else 7 - p % 8 for p in range(Hq)]
    load = [0] * 8
    for p in range(Hq):
        load[wave[p]] += size[p]
    target = (TT + 7) // 8
    for _ in range(64):
        A = max(range(8), key=lambda w: (load[w], w))
        if load[A] <= target:
            break
        best = None
        for a in range(Hq):
            if wave[a] != A:
                continue
            for b in range(Hq):
                if wave[b] == A:
                    continue
                d, lb = size[a] - size[b], load[wave[b]]
                if d > 0 and lb + d < load[A]:
                    cand = (max(load[A] - d, lb + d), a, b)
                    best = cand if best is None or cand < best else best
        if best is None:
            break
        _, a, b = best
        B, d = wave[b], size[a] - size[b]
        wave[a], wave[b] = B, A
        load[A] -= d
        load[B] += d
    return max(load) <= 16


def test_wave_plan_rule_matches_its_restatement():
    """starkv_decode_layer_fits (bf16, narrow V: only the plan and the caps decide) against
    an independent restatement of the wave plan, over random head-rank mixes around the
    limits, and the shape a too-simple tile count would accept (95 tiles, nine heads of 8)."""
    from starkv_serve import _hip
    g = torch.Generator().manual_seed(11)
    cases = [[128] * 9 + [16] * 23, [128] * 8 + [16] * 32, [256, 16, 100, 20], [192] * 8 + [16]]
    for _ in range(300):
        Hh = int(torch.randint(1, 33, (1,), generator=g))
        top = int(torch.randint(2, 17, (1,), generator=g))
        cases.append([16 * int(t) for t in torch.randint(1, top + 1, (Hh,), generator=g)])
    agree = 0
    for ranks in cases:
        want = _plan_fits_restated([(r + 15) // 16 for r in ranks])
        got = _hip.layer_fits(_hip.BF16, len(ranks), len(ranks), ranks, 64)
        assert got == want, ranks
        agree += got
    assert not _plan_fits_restated([8] * 9 + [1] * 23)
    assert 0 < agree < len(cases)  # both outcomes occur


@pytest.mark.parametrize("quant,H,ranks,v_rank,want", [
    (True, 32, [16, 32, 48, 64] * 8, 64, [(0, 32)]),
    (True, 32, [32] * 23 + [16] * 9, 1290, [(0, 32)]),             # the 0.75-ratio layer: one call
    (True, 32, [64] * 32, 64, [(0, 24), (24, 32)]),                # W 2048: 128 tiles
    (True, 32, [64] * 16 + [48] * 16, 1290, [(0, 26), (26, 32)]),  # W 1792, two-pass: 64 + 30 tiles
    (True, 40, [16, 32, 48, 64] * 10, 64, [(0, 32), (32, 40)]),    # 40 heads
    (True, 32, [128] * 9 + [16] * 23, 64, [(0, 23), (23, 32)]),    # 95 tiles, plan does not fit
    (False, 32, [128] * 9 + [16] * 23, 64, [(0, 23), (23, 32)]),
    (True, 64, [64] * 64, 1290, [(0, 24), (24, 48), (48, 64)]),
])
def test_head_groups_known_answers(quant, H, ranks, v_rank, want):
    """starkv_decode_layer_groups: greedy consecutive ranges, one call each; a layer that
    fits one call is one range, and the whole-layer check agrees."""
    from starkv_serve import _hip
    from starkv_serve.kernels.paged_decode import kv_head_groups
    kind = _hip.CACHE_Q3_2 if quant else _hip.BF16
    g = kv_head_groups(kind, H, ranks, v_rank)
    assert g == want
    assert g[0][0] == 0 and g[-1][1] == len(ranks) and all(a[1] == b[0] for a, b in zip(g, g[1:]))
    assert _hip.layer_fits(kind, H, len(ranks), ranks, v_rank) == (g == [(0, len(ranks))])


def test_quant_group_geometry_matches_whole_layer_queries():
    """The 3.2-bit group entry points, over the whole layer, size the workspace and pick the
    decode form exactly as the whole-layer queries do."""
    from starkv_serve import _hip
    L = _hip.lib()
    for H_, W, rv in [(32, 1232, 64), (32, 880, 1290), (8, 512, 256), (4, 400, 32)]:
        for n, span, grid in [(64, 8192, 256), (1, 16448, 256), (3, 100, 7)]:
            assert (L.starkv_quant_group_workspace_bytes(n, W, H_, rv, 0, H_, 0, W, span, grid) ==
                    L.starkv_decode_workspace_bytes(_hip.CACHE_Q3_2, n, H_, H_, W, rv, span, grid))
        assert (L.starkv_quant_group_two_pass(W, H_, rv, 0, H_, 0, W) ==
                L.starkv_decode_two_pass(_hip.CACHE_Q3_2, H_, H_, W, rv))
    # a group past the layer's heads or lanes, or a lane offset that is not a tile, is refused
    assert L.starkv_quant_group_workspace_bytes(1, 1232, 32, 64, 30, 4, 0, 64, 100, 1) == 0
    assert L.starkv_quant_group_workspace_bytes(1, 1232, 32, 64, 0, 4, 8, 64, 100, 1) == 0
    assert L.starkv_quant_group_workspace_bytes(1, 1232, 32, 64, 0, 4, 1200, 64, 100, 1) == 0


@pytest.mark.parametrize("quant", [False, True])
def test_decode_uses_the_load_time_groups(tmp_path, quant):
    """The groups the decode wrappers compute from host ranks equal the ones layer_operands
    stores at load time, for a layer whose 95 tiles pass the tile cap but not the wave plan
    (one call over it would return NaN rows); a 40-head 3.2-bit layer now loads as two
    groups."""
    from starkv_serve import _hip
    from starkv_serve.kernels import paged_decode as pd
    from starkv_serve.kernels import paged_quant as pq
    ranks = [128] * 9 + [16] * 23
    path = str(tmp_path / "plan.pt")
    ck.write_fused_checkpoint(path, 1, 32, HD, 64, {0: (ranks, 64)}, seed=3)
    layer = ck.load_fused_checkpoint(path, 1, 32, HD, dtype=torch.bfloat16, kv_quant=quant).layers[0]
    ops = ck.layer_operands(layer, 32, torch.device("cpu"), torch.bfloat16)
    kind = _hip.CACHE_Q3_2 if quant else _hip.BF16
    assert ops.kv_groups == [(0, 23), (23, 32)]
    assert pd._groups_for(kind, 32, pd._host_ints(ops.k_ranks), 64) == ops.kv_groups
    if quant:
        widths = pq.head_widths(pd._host_ints(ops.k_tiles[0]), 32)
        assert widths == [128] * 9 + [16] * 23
        assert pd._groups_for(kind, 32, widths, 64) == ops.kv_groups
        path40 = str(tmp_path / "h40.pt")
        ck.write_fused_checkpoint(path40, 1, 40, HD, 64, {0: ([16, 32, 48, 64] * 10, 64)}, seed=4)
        l40 = ck.load_fused_checkpoint(path40, 1, 40, HD, dtype=torch.bfloat16, kv_quant=True).layers[0]
        assert ck.layer_operands(l40, 40, torch.device("cpu"), torch.bfloat16).kv_groups == [(0, 32), (32, 40)]
