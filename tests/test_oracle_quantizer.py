"""Pin the C restatement of the 3.2-bit quantizer and packers (oracle/quant_oracle.c).

Checks: hand-computed codes at exact rounding ties (a round-half-away or
multiply-by-reciprocal mistake fails them), an independent numpy float32 restatement
on random and adversarial inputs, bfloat16 round-to-nearest-even against torch's
conversion, the byte layout of a tiny row by hand, and the pack -> unpack round trip
bound |x - deq(x)| <= s / 2 with clamping only at the block's amax.
"""
import numpy as np
import pytest
import torch

from oracle import cquant, ref


def np_quantize(x, bits):
    """kv_quant._q in numpy float32: IEEE division, round-half-even."""
    x = np.asarray(x, np.float32)
    qmax = np.float32(2 ** (bits - 1) - 1)
    amax = np.maximum(np.abs(x).max(initial=np.float32(0)), np.float32(1e-5)).astype(np.float32)
    s = np.float32(amax / qmax)
    q = np.rint((x / s).astype(np.float32))
    return (np.clip(q, -(2 ** (bits - 1)), qmax) + 8).astype(np.int32), s


def test_known_codes_at_ties():
    # 4-bit block with amax 7 -> s = 1 exactly; ties go to even.
    codes, s = cquant.quantize_block(np.array([7, 3.5, 2.5, -3.5, 1, -0.5, 0.5, -7]), 4)
    assert s == 1.0
    assert codes.tolist() == [15, 12, 10, 4, 9, 8, 8, 1]
    # 3-bit block with amax 3 -> s = 1.
    codes, s = cquant.quantize_block(np.array([3, 1.5, -2.5, 0.5, -3]), 3)
    assert s == 1.0
    assert codes.tolist() == [11, 10, 6, 8, 5]
    # all-zero block: amax floors at fp32(1e-5), every code is 8.
    codes, s = cquant.quantize_block(np.zeros(5), 3)
    assert codes.tolist() == [8] * 5
    assert s == np.float32(np.float32(1e-5) / np.float32(3))


def test_division_not_reciprocal_multiply():
    # Values a few ulps around (k + 1/2) * s, where x * (1/s) and x / s can round to
    # different codes; the oracle must follow the IEEE division (kv_quant.py:114-119).
    rng = np.random.default_rng(7)
    found = 0
    for _ in range(400):
        amax = np.float32(rng.uniform(0.1, 10))
        s = np.float32(amax / np.float32(3))
        inv = np.float32(np.float32(1) / s)
        for k in range(-3, 3):
            base = np.float32((k + 0.5) * float(s))
            for d in range(-3, 4):
                x = np.float32(np.nextafter(base, np.float32(np.inf) if d > 0 else np.float32(-np.inf))) if d else base
                for _ in range(abs(d) - 1):
                    x = np.nextafter(x, np.float32(np.inf) if d > 0 else np.float32(-np.inf)).astype(np.float32)
                div = np.rint(np.float32(x / s))
                recip = np.rint(np.float32(x * inv))
                if div != recip and abs(x) < amax:
                    codes, s2 = cquant.quantize_block(np.array([amax, x], np.float32), 3)
                    assert s2 == s
                    assert codes[1] == int(np.clip(div, -4, 3)) + 8
                    found += 1
    assert found > 0


@pytest.mark.parametrize("bits", [3, 4])
def test_matches_numpy_restatement(bits):
    rng = np.random.default_rng(bits)
    for trial in range(300):
        n = int(rng.integers(1, 70))
        scale = 10.0 ** rng.uniform(-6, 3)
        x = (rng.standard_normal(n) * scale).astype(np.float32)
        if trial % 5 == 0:  # exact ties: multiples of s/2
            k = rng.integers(-2 ** (bits - 1), 2 ** (bits - 1), n)
            x = (k.astype(np.float32) + np.float32(0.5) * rng.integers(0, 2, n)).astype(np.float32)
        c1, s1 = cquant.quantize_block(x, bits)
        c2, s2 = np_quantize(x, bits)
        assert s1 == s2
        assert c1.tolist() == c2.tolist()


def test_bf16_round_to_nearest_even():
    known = {1.0: 0x3F80, 1.00390625: 0x3F80, 1.01171875: 0x3F82, -2.0: 0xC000, 1.0078125: 0x3F81}
    for f, h in known.items():
        assert cquant.f32_to_bf16_bits(f) == h, f
    rng = np.random.default_rng(0)
    vals = (rng.standard_normal(5000) * 10.0 ** rng.uniform(-30, 30, 5000)).astype(np.float32)
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().astype(np.uint16)
    got = np.array([cquant.f32_to_bf16_bits(float(v)) for v in vals], dtype=np.uint16)
    assert (got == want).all()


def test_tiny_row_bytes_by_hand():
    # One KV head, rank 16 (nout 3, width 16), V rank 4 (nout 0).
    lay = ref.row_layout(16, 1, 4)
    k = np.zeros((1, 16), np.float32)
    k[0, :3] = [7, -7, 3.5]          # outliers: s_out = 1 -> codes 15, 1, 12
    k[0, 3:6] = [3, -1.5, 0.5]       # inliers: amax 3 -> s_in = 1 -> 11, 6, 8; zeros -> 8
    v = np.array([[3, -3, 1.5, 0]], np.float32)  # all inliers: s_in = 1 -> 11, 5, 10, 8
    cache = np.full((1, 16, lay["nbytes"]), 0xAB, np.uint8)
    cquant.pack_kv(k, v, cache, np.array([0]), [16], [0], [3], 4, lay["ks_off"], lay["vs_off"], lay["vq_off"])
    row = cache[0, 0]
    codes = [15, 1, 12, 11, 6, 8] + [8] * 10
    assert row[:8].tolist() == [codes[2 * i] | (codes[2 * i + 1] << 4) for i in range(8)]
    assert row[8:12].tolist() == [0x80, 0x3F, 0x80, 0x3F]          # (1.0, 1.0) bf16 little endian
    assert row[12:16].tolist() == [0x80, 0x3F, 0x80, 0x3F]         # V: no outliers -> 1.0, s_in 1.0
    assert row[16:18].tolist() == [11 | (5 << 4), 10 | (8 << 4)]
    assert (row[18:] == 0xAB).all()                                 # pad bytes are never written


def test_odd_v_blocks_pad_nibble():
    # v_rank 7: nout 1 (one outlier byte with a pad nibble 8), 6 inliers in 3 bytes.
    lay = ref.row_layout(16, 1, 7)
    v = np.array([[-7.0, 3, 2, 1, 0, -1, -2]], np.float32)
    cache = np.zeros((1, 16, lay["nbytes"]), np.uint8)
    cquant.pack_kv(np.zeros((1, 16), np.float32), v, cache, np.array([0]), [16], [0], [3], 7,
                   lay["ks_off"], lay["vs_off"], lay["vq_off"])
    row = cache[0, 0]
    vq = row[lay["vq_off"]:lay["vq_off"] + lay["v_bytes"]]
    assert vq.tolist() == [1 | (8 << 4), 11 | (10 << 4), 9 | (8 << 4), 7 | (6 << 4)]


def test_round_trip_bound_and_numpy_unpack():
    rng = np.random.default_rng(3)
    ranks = [16, 20, 48, 64, 33]
    widths, offsets, W = ref.head_layout(ranks)
    nouts = [ref.n_outlier(r) for r in ranks]
    R = 64
    lay = ref.row_layout(W, len(ranks), R)
    n = 40
    k = (rng.standard_normal((n, W)) * rng.uniform(0.01, 100, (n, 1))).astype(np.float32)
    for h, r in enumerate(ranks):
        k[:, offsets[h] + r:offsets[h] + widths[h]] = 0
    v = rng.standard_normal((n, R)).astype(np.float32)
    cache = np.zeros((3, 16, lay["nbytes"]), np.uint8)
    slots = rng.permutation(48)[:n]
    cquant.pack_kv(k, v, cache, slots, ranks, offsets, nouts, R, lay["ks_off"], lay["vs_off"], lay["vq_off"])
    rows = cache.reshape(-1, lay["nbytes"])[slots]
    K, V = ref.unpack_rows(rows, lay, ranks)
    for i in range(n):
        kc = cquant.unpack_k_row(rows[i], ranks, offsets, nouts, lay["ks_off"], W)
        vc = cquant.unpack_v_row(rows[i], R, lay["v_nout"], lay["vs_off"], lay["vq_off"])
        assert np.array_equal(kc.astype(np.float64), K[i]) and np.array_equal(vc.astype(np.float64), V[i])
    # |x - deq| <= s/2 (+ the bf16 scale's rounding); amax lanes hit the clamp exactly.
    for h, r in enumerate(ranks):
        o, no = offsets[h], nouts[h]
        for lo, hi, qmax in ((o, o + no, 7), (o + no, o + widths[h], 3)):
            if hi <= lo:
                continue
            blk = k[:, lo:hi]
            s = np.maximum(np.abs(blk).max(1, keepdims=True), 1e-5) / qmax
            err = np.abs(blk - K[:, lo:hi])
            assert (err <= s * (0.5 + qmax * 2 ** -8) + 1e-12).all()
