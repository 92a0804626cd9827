"""Pin the float64 decode oracle against an independent brute-force statement
(per-token loops, RoPE as a complex rotation), the z-form identity of the reference's
quant path, page-permutation invariance and closed forms."""
import numpy as np
import pytest
import torch

from oracle import cquant, ref
from starkv_serve import workloads as W


def _lowrank_np(wl):
    return dict(q=wl.query.float().numpy(), cache=wl.kv_cache.float().numpy(), bt=wl.block_table.numpy(),
                seq=wl.seq_lens.numpy(), U=wl.k_up.float().numpy(), vq=wl.v_up_by_q.float().numpy(),
                cs=wl.cos_sin_cache.float().numpy())


def _oracle(wl, a):
    return ref.lowrank_decode(a["q"], a["cache"], a["bt"], a["seq"], wl.max_seq_len, a["U"], wl.ranks,
                              wl.k_head_offsets.tolist(), wl.k_width, a["vq"], a["cs"], wl.scale)


def test_matches_bruteforce_gqa_ragged():
    wl = W.make_lowrank([5, 37, 16, 1], num_heads=4, num_kv_heads=2, ranks=[16, 20], v_rank=16, seed=11,
                        poison=False)
    a = _lowrank_np(wl)
    got = _oracle(wl, a)
    want = ref.lowrank_decode_bruteforce(a["q"], a["cache"], a["bt"], a["seq"], wl.max_seq_len, a["U"], wl.ranks,
                                         wl.k_head_offsets.tolist(), a["vq"], a["cs"], wl.scale)
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-12)


def test_nonzero_padding_lanes_are_ignored():
    # paged_decode.py:79-81 masks lanes >= rank: garbage there must not change the result.
    wl = W.make_lowrank([20, 9], num_heads=2, ranks=[20, 4], v_rank=16, seed=3, poison=False)
    a = _lowrank_np(wl)
    base = _oracle(wl, a)
    a2 = dict(a)
    c = a["cache"].copy()
    c[..., 20:32] = 1e3
    c[..., 36:48] = -7.0
    a2["cache"] = c
    np.testing.assert_allclose(_oracle(wl, a2), base, rtol=0, atol=0)


def test_z_form_identity():
    # q . RoPE_l(U^T x) == sum_r x[r] ([cos_l | sin_l] . AB[r])  (kv_quant.py:42-50)
    rng = np.random.default_rng(0)
    R, L = 24, 9
    q = rng.standard_normal((1, 1, 128))
    U = rng.standard_normal((R, 128))
    x = rng.standard_normal((L, R))
    cs = W.cos_sin_table(L, torch.float32).numpy().astype(np.float64)
    lift = ref._rope(x @ U, cs) @ q[0, 0]
    ab = ref.fold_q(q, U, np.zeros(R, int), 1.0)[0]
    z = cs @ ab.T
    np.testing.assert_allclose((x * z).sum(1), lift, rtol=1e-12, atol=1e-10)


def test_page_permutation_invariance():
    wl = W.make_lowrank([40, 70], num_heads=2, ranks=[16, 48], v_rank=32, seed=5, poison=False)
    a = _lowrank_np(wl)
    base = _oracle(wl, a)
    nb = a["cache"].shape[0]
    perm = np.concatenate([[0], 1 + np.random.default_rng(1).permutation(nb - 1)])
    inv = np.argsort(perm)
    a2 = dict(a)
    a2["cache"] = a["cache"][perm]
    a2["bt"] = inv[a["bt"]]
    np.testing.assert_allclose(_oracle(wl, a2), base, rtol=1e-13, atol=1e-14)


def test_one_token_closed_form():
    wl = W.make_lowrank([1], num_heads=3, ranks=[16, 32, 64], v_rank=16, seed=9, poison=False)
    a = _lowrank_np(wl)
    got = _oracle(wl, a)
    row = a["cache"][a["bt"][0, 0], 0]
    v = row[wl.k_width:wl.k_width + 16].astype(np.float64)
    for h in range(3):
        np.testing.assert_allclose(got[0, h], v @ a["vq"][h].astype(np.float64), rtol=1e-12)


def test_max_seq_len_truncates_and_zero_length_is_nan():
    wl = W.make_lowrank([30, 0 + 1], num_heads=1, ranks=[16], v_rank=16, seed=2, poison=False)
    a = _lowrank_np(wl)
    full = _oracle(wl, a)
    a2 = dict(a)
    a2["seq"] = np.array([30, 0], np.int32)
    got = ref.lowrank_decode(a2["q"], a2["cache"], a2["bt"], a2["seq"], 20, a2["U"], wl.ranks,
                             wl.k_head_offsets.tolist(), wl.k_width, a2["vq"], a2["cs"], wl.scale)
    assert np.isnan(got[1]).all()
    assert not np.allclose(got[0], full[0])  # only the first 20 tokens were attended


def test_quant_oracle_uses_all_stored_lanes():
    # The 3.2-bit path reads every lane of a head's 16-lane tiles (paged_quant.py:114-131):
    # with zero codes in the padding lanes it equals the low-rank oracle on the dequantized cache.
    rng = np.random.default_rng(4)
    ranks = [16, 20]
    widths, offsets, Wd = ref.head_layout(ranks)
    lay = ref.row_layout(Wd, 2, 16)
    L = 19
    k = rng.standard_normal((L, Wd)).astype(np.float32)
    for h, r in enumerate(ranks):
        k[:, offsets[h] + r:offsets[h] + widths[h]] = 0
    v = rng.standard_normal((L, 16)).astype(np.float32)
    cache = np.zeros((3, 16, lay["nbytes"]), np.uint8)
    cquant.pack_kv(k, v, cache, np.arange(16, 16 + L), ranks, offsets, [ref.n_outlier(r) for r in ranks], 16,
                   lay["ks_off"], lay["vs_off"], lay["vq_off"])
    bt = np.array([[1, 2]], np.int32)
    q = rng.standard_normal((1, 2, 128))
    U = rng.standard_normal((Wd, 128))
    vq = rng.standard_normal((2, 16, 128))
    cs = W.cos_sin_table(L, torch.float32).numpy()
    got = ref.quant_decode(q, cache, bt, [L], L, lay, ranks, U, vq, cs, 0.1)
    K, V = ref.unpack_rows(ref.gather_rows(cache, bt[0], L, 16), lay, ranks)
    flat = np.zeros((3, 16, Wd + 16))
    flat[1:].reshape(-1, Wd + 16)[:L] = np.concatenate([K, V], 1)
    want = ref.lowrank_decode(q, flat, bt, [L], L, U, [16, 32], offsets, Wd, vq, cs, 0.1)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_reference_emulation_pinned_in_wide_dtypes():
    """The reference-rounding emulation, run with float64 query and bases, equals the
    float64 oracle to fp32 accuracy (its K lift and P @ V stay fp32): a dropped term, a
    wrong head or offset, or a transposed operand in the emulation would not."""
    wl = W.make_lowrank([37, 5, 200], num_heads=8, num_kv_heads=4, ranks=[16, 32, 20, 48], v_rank=32, seed=21,
                        poison=False)
    a = _lowrank_np(wl)
    want = _oracle(wl, a)
    got = ref.emulate_lowrank_reference(torch.from_numpy(a["q"]).double(), a["cache"], a["bt"], a["seq"],
                                        wl.max_seq_len, a["U"], wl.ranks, wl.k_head_offsets.tolist(), wl.k_width,
                                        torch.from_numpy(a["vq"]).double(), a["cs"], wl.scale)
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < 2e-6, err
    # and with the model dtype it departs by the reference's own rounding (logits in bf16)
    emu = ref.emulate_lowrank_reference(wl.query, wl.kv_cache, a["bt"], a["seq"], wl.max_seq_len, wl.k_up,
                                        wl.ranks, wl.k_head_offsets.tolist(), wl.k_width, wl.v_up_by_q,
                                        wl.cos_sin_cache, wl.scale)
    assert 1e-4 < np.abs(emu - want).max() / np.abs(want).max() < 5e-2
