"""ORACLE -- test infrastructure only (the CPU baseline of bench.py and tests/).

The reference's decode math restated in float32 PyTorch on the CPU, the "PyTorch math"
the GPU kernels are compared with for speed. It follows the reference's readable
statement of the decode (model.py:1333-1386: lift the codes through U, RoPE, q.k,
softmax, P @ V codes, lift through v_up) over the paged gather of paged_decode.py:63-69
(rows of token l at block_table[b, l // block_size], slot l % block_size), the 3.2-bit
unpack of kv_quant.py:154-198 (unpack_k_ref / unpack_v_ref on the QuantRow layout of
paged_quant.py:71-111) and the quantizer of kv_quant.py:111-120 / paged_quant.py:146-202
(IEEE fp32 division by amax / 7 or amax / 3, round half to even, bfloat16 scales).

Pinned (tests/test_oracle_torch_ref.py): decode outputs against the float64 oracle
(oracle/ref.py) to fp32 accuracy, and packed rows byte-exact against the C quantizer
(oracle/quant_oracle.c).
"""
import torch

EPS = 1e-5


def _rope(k, cs):
    """NeoX rotate-half with cos = cs[:, :64], sin = cs[:, 64:] (paged_decode.py:89-95)."""
    h = k.shape[-1] // 2
    cos, sin = cs[:, :h], cs[:, h:]
    k0, k1 = k[:, :h], k[:, h:]
    return torch.cat([k0 * cos - k1 * sin, k1 * cos + k0 * sin], dim=1)


def _gather(cache, bt_row, L, bs):
    l = torch.arange(L)
    return cache[bt_row[l // bs].long(), l % bs]


def _attend_heads(q_b, keys_per_kv, V, v_up_by_q, scale, G):
    """q_b [Hq, D]; keys_per_kv: list of rotated K [L, D] per KV head -> out [Hq, D]."""
    logits = torch.stack([keys_per_kv[h // G] @ q_b[h] for h in range(q_b.shape[0])])  # [Hq, L]
    p = torch.softmax(logits * scale, dim=-1)
    acc = p @ V                                                                          # [Hq, r_v]
    return torch.bmm(acc[:, None, :], v_up_by_q)[:, 0, :]


def lowrank_decode(q, cache, block_table, seq_lens, max_seq_len, k_up, k_ranks, k_offsets, k_width, v_up_by_q,
                   cos_sin, scale):
    """paged_starkv_decode (paged_decode.py:150-226) in fp32 on the CPU: [n, Hq, D]."""
    q = q.float()
    n, Hq, D = q.shape
    Hkv = len(k_ranks)
    G = Hq // Hkv
    r_v = v_up_by_q.shape[1]
    bs = cache.shape[1]
    U = k_up.float()
    vq = v_up_by_q.float()
    cs_all = cos_sin.float()
    out = torch.full((n, Hq, D), float("nan"))
    for b in range(n):
        L = min(int(seq_lens[b]), int(max_seq_len))
        if L <= 0:
            continue
        rows = _gather(cache, block_table[b], L, bs).float()
        V = rows[:, k_width:k_width + r_v]
        cs = cs_all[:L]
        keys = []
        for kv in range(Hkv):
            R, off = int(k_ranks[kv]), int(k_offsets[kv])
            keys.append(_rope(rows[:, off:off + R] @ U[off:off + R], cs))
        out[b] = _attend_heads(q[b], keys, V, vq, scale, G)
    return out


def _bf16_pairs(u8, off, count):
    """count bfloat16 values from byte `off` of each row, as float32 [L, count]."""
    b = u8[:, off:off + 2 * count].to(torch.int32)
    return ((b[:, 0::2] | (b[:, 1::2] << 8)) << 16).view(torch.float32)


def unpack_rows(rows, lay, ranks):
    """uint8 rows [L, nbytes] -> (K [L, W], V [L, r_v]) fp32 (kv_quant.py:154-188)."""
    L = rows.shape[0]
    W, H, R = lay["k_width"], lay["num_kv_heads"], lay["v_rank"]
    kb = rows[:, :W // 2].to(torch.int32)
    nib = torch.stack([kb & 15, kb >> 4], -1).reshape(L, W).float() - 8
    sc = _bf16_pairs(rows, lay["ks_off"], 2 * H).reshape(L, H, 2)
    K = torch.empty(L, W)
    o = 0
    for h, r in enumerate(ranks):
        w, no = (r + 15) // 16 * 16, int(0.2 * r)
        K[:, o:o + no] = nib[:, o:o + no] * sc[:, h, 0:1]
        K[:, o + no:o + w] = nib[:, o + no:o + w] * sc[:, h, 1:2]
        o += w
    vs = _bf16_pairs(rows, lay["vs_off"], 2)
    nout, nbo = lay["v_nout"], lay["v_nbo"]
    vb = rows[:, lay["vq_off"]:lay["vq_off"] + lay["v_bytes"]].to(torch.int32)
    vn = torch.stack([vb & 15, vb >> 4], -1).reshape(L, -1).float() - 8
    V = torch.cat([vn[:, :nout] * vs[:, 0:1], vn[:, 2 * nbo:2 * nbo + R - nout] * vs[:, 1:2]], dim=1)
    return K, V


def quant_decode(q, cache_u8, block_table, seq_lens, max_seq_len, lay, ranks, k_up, v_up_by_q, cos_sin, scale):
    """paged_quant_decode (paged_quant.py:357-411) in fp32 on the CPU over the unpacked
    cache: [n, H, D]. Every stored lane of a head (its rank rounded to 16) is used."""
    q = q.float()
    n, H, D = q.shape
    bs = cache_u8.shape[1]
    U = k_up.float()
    vq = v_up_by_q.float()
    cs_all = cos_sin.float()
    widths = [(r + 15) // 16 * 16 for r in ranks]
    offsets = [sum(widths[:h]) for h in range(H)]
    out = torch.full((n, H, D), float("nan"))
    for b in range(n):
        L = min(int(seq_lens[b]), int(max_seq_len))
        if L <= 0:
            continue
        K, V = unpack_rows(_gather(cache_u8, block_table[b], L, bs), lay, ranks)
        cs = cs_all[:L]
        keys = [_rope(K[:, o:o + w] @ U[o:o + w], cs) for o, w in zip(offsets, widths)]
        out[b] = _attend_heads(q[b], keys, V, vq, scale, 1)
    return out


def _quantize(x, lo, hi, div):
    """kv_quant._q on a block [L, n] (kv_quant.py:111-120): per row scale amax / div in
    fp32 (IEEE division), codes round-half-even, clamped, +8; the scale as stored (bf16)."""
    a = x.abs().amax(dim=1, keepdim=True).clamp_min(EPS) if x.shape[1] else torch.full((x.shape[0], 1), EPS)
    s = a / div
    codes = torch.clamp(torch.round(x / s), lo, hi).to(torch.int32) + 8
    return codes, s.to(torch.bfloat16)


def _pack_nibbles(codes):
    """[L, 2m] codes -> [L, m] bytes, even lane low (paged_quant.py:166-170)."""
    return (codes[:, 0::2] | (codes[:, 1::2] << 4)).to(torch.uint8)


def pack_rows(k_codes, v_codes, lay, ranks):
    """pack_kv (paged_quant.py:139-216) of one step's codes into uint8 rows [L, nbytes]
    (bytes past vq_off + v_bytes are 0)."""
    L = k_codes.shape[0]
    W, H, R = lay["k_width"], lay["num_kv_heads"], lay["v_rank"]
    x = k_codes.float()
    rows = torch.zeros(L, lay["nbytes"], dtype=torch.uint8)
    kc = torch.empty(L, W, dtype=torch.int32)
    scales = torch.empty(L, H, 2, dtype=torch.bfloat16)
    o = 0
    for h, r in enumerate(ranks):
        w, no = (r + 15) // 16 * 16, int(0.2 * r)
        blk = x[:, o:o + w]
        if no:
            kc[:, o:o + no], scales[:, h, 0:1] = _quantize(blk[:, :no], -8, 7, 7.0)
        else:
            scales[:, h, 0] = 1.0
        kc[:, o + no:o + w], scales[:, h, 1:2] = _quantize(blk[:, no:], -4, 3, 3.0)
        o += w
    rows[:, :W // 2] = _pack_nibbles(kc)
    rows[:, lay["ks_off"]:lay["vs_off"]] = scales.reshape(L, 2 * H).view(torch.int16).view(torch.uint8).reshape(L, -1)
    v = v_codes.float()
    nout, nbo = lay["v_nout"], lay["v_nbo"]
    vsc = torch.empty(L, 2, dtype=torch.bfloat16)
    if nout:
        vo, vsc[:, 0:1] = _quantize(v[:, :nout], -8, 7, 7.0)
    else:
        vo = torch.zeros(L, 0, dtype=torch.int32)
        vsc[:, 0] = 1.0
    vi, vsc[:, 1:2] = _quantize(v[:, nout:], -4, 3, 3.0)
    pad8 = lambda c: torch.cat([c, torch.full((L, c.shape[1] % 2), 8, dtype=torch.int32)], 1)  # noqa: E731
    rows[:, lay["vs_off"]:lay["vq_off"]] = vsc.view(torch.int16).view(torch.uint8).reshape(L, -1)
    rows[:, lay["vq_off"]:lay["vq_off"] + nbo] = _pack_nibbles(pad8(vo))
    vib = _pack_nibbles(pad8(vi))
    rows[:, lay["vq_off"] + nbo:lay["vq_off"] + nbo + vib.shape[1]] = vib
    return rows


def write_step(hidden, kv_down, k_width, lay, ranks, cache_u8, slots):
    """One 3.2-bit cache-write step (model.py:71 + attention.py:185-188): codes = hidden @
    kv_down^T in fp32, rounded to kv_down's dtype (what F.linear returns), quantized, packed
    and scattered to their slots."""
    codes = (hidden.float() @ kv_down.float().T).to(kv_down.dtype)
    rows = pack_rows(codes[:, :k_width], codes[:, k_width:], lay, ranks)
    bs = cache_u8.shape[1]
    cache_u8[slots // bs, slots % bs] = rows
    return codes
