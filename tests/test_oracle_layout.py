"""Pin the oracle's row layout, outlier counts and tile tables (and the product's host
helpers) against hand-computed known answers and brute force."""
import pytest

from oracle import cquant, ref
from starkv_serve.kernels import paged_quant as pq


@pytest.mark.parametrize("W,H,R,expect", [
    # k_width, kv heads, v_rank -> (ks_off, vs_off, vq_off, v_nout, v_nbo, v_bytes, nbytes), by hand
    (1280, 32, 64, (640, 768, 772, 12, 6, 32, 816)),
    (1280, 32, 32, (640, 768, 772, 6, 3, 16, 800)),
    (880, 32, 1280, (440, 568, 572, 256, 128, 640, 1216)),
    (16, 1, 4, (8, 12, 16, 0, 0, 2, 32)),
    (32, 2, 7, (16, 24, 28, 1, 1, 4, 32)),
])
def test_quant_row_known_answers(W, H, R, expect):
    lay = ref.row_layout(W, H, R)
    got = tuple(lay[k] for k in ("ks_off", "vs_off", "vq_off", "v_nout", "v_nbo", "v_bytes", "nbytes"))
    assert got == expect
    row = pq.QuantRow(W, H, R)
    assert (row.ks_off, row.vs_off, row.vq_off, row.v_nout, row.v_nbo, row.v_bytes, row.nbytes) == expect


def test_n_outlier_is_floor_fifth():
    # int(0.2 * r) in double precision equals floor(r / 5) for every realistic rank.
    for r in range(0, 4097):
        assert ref.n_outlier(r) == r // 5
        assert pq.n_outlier(r) == r // 5
        if r < 600:
            assert cquant.n_outlier(r) == r // 5
    assert [ref.n_outlier(r) for r in (16, 32, 48, 64, 1280)] == [3, 6, 9, 12, 256]


def test_k_tables_known_answer():
    ranks = [16, 48, 20]
    nouts, hol, (th, tn, tl) = ref.k_tables(ranks)
    assert nouts.tolist() == [3, 9, 4]
    assert hol.tolist() == [0] * 16 + [1] * 48 + [2] * 32
    assert th.tolist() == [0, 1, 1, 1, 2, 2]
    assert tn.tolist() == [3, 9, 0, 0, 4, 0]
    assert tl.tolist() == [1, 0, 0, 1, 0, 1]
    n2, h2, (a, b, c) = pq.k_tables(ranks, "cpu")
    assert n2.tolist() == nouts.tolist() and h2.tolist() == hol.tolist()
    assert a.tolist() == th.tolist() and b.tolist() == tn.tolist() and c.tolist() == tl.tolist()


def test_k_tables_outliers_spanning_tiles():
    # rank 128 -> 25 outlier lanes: the first tile all outliers, the second 9.
    _, _, (th, tn, tl) = ref.k_tables([128])
    assert tn.tolist() == [16, 9, 0, 0, 0, 0, 0, 0]
    assert tl.tolist() == [0] * 7 + [1]


def test_head_layout_widths_and_offsets():
    widths, offsets, W = ref.head_layout([16, 20, 64, 1])
    assert widths == [16, 32, 64, 16] and offsets == [0, 16, 48, 112] and W == 128
