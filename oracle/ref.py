"""ORACLE -- test infrastructure only (tests/, smoke, bench.py CPU baseline).

CPU restatement of STAR-KV's paged decode path in float64 numpy. Each function
cites the reference lines it restates. How each one is pinned (checked against
something other than itself) -- see tests/test_oracle_*.py:

  row_layout / n_outlier / k_tables   hand-computed known answers; brute-force
                                      enumeration of r // 5; tile counts vs widths
  block_hadamard                      orthonormality, block structure, Sylvester
                                      pattern; sign vectors against golden vectors
                                      written from the reference (tests/golden/)
  unpack_rows (numpy)                 against the C restatement and against the
                                      round-trip bound |x - deq(x)| <= s/2
  lowrank_decode / quant_decode       against an independent brute-force float64
                                      loop (complex-number RoPE, per-token gathers),
                                      the z-form identity (kv_quant.py:42-50), page
                                      permutation invariance, one-token closed form
  emulate_lowrank_reference           reports the reference's own rounding error;
                                      not used as a pass/fail truth
  dense_prefill                       a prompt's last token equals lowrank_decode over
                                      the same codes; a first token returns its own V
                                      lifted; causality (a later token changes no
                                      earlier output)
  causal_attention                    torch's float64 CPU scaled_dot_product_attention
                                      (is_causal) per prompt and head; a first token
                                      returns its own V; dense_prefill equals it over
                                      the lifted K and V
"""
import math

import numpy as np

HEAD_DIM = 128
OUTLIER_RATIO = 0.2
HADAMARD_SEED = 1234
K_ALIGN = 16


def n_outlier(rank: int) -> int:
    """paged_quant.py:46-47 / kv_quant.py:76-77."""
    return int(OUTLIER_RATIO * rank)


def align16(n: int) -> int:
    return -(-int(n) // 16) * 16


def row_layout(k_width: int, num_kv_heads: int, v_rank: int) -> dict:
    """QuantRow, paged_quant.py:71-111."""
    v_nout = n_outlier(v_rank)
    ks_off = k_width // 2
    vs_off = ks_off + 4 * num_kv_heads
    vq_off = vs_off + 4
    v_nbo = (v_nout + 1) // 2
    v_bytes = v_nbo + (v_rank - v_nout + 1) // 2
    nbytes = -(-(vq_off + v_bytes) // 16) * 16
    return dict(k_width=k_width, num_kv_heads=num_kv_heads, v_rank=v_rank, v_nout=v_nout,
                ks_off=ks_off, vs_off=vs_off, vq_off=vq_off, v_nbo=v_nbo, v_bytes=v_bytes,
                nbytes=nbytes)


def head_layout(ranks):
    """Widths rounded to K_ALIGN, prefix-sum offsets (checkpoint.py:125-128)."""
    widths = [align16(r) for r in ranks]
    offsets = [sum(widths[:h]) for h in range(len(ranks))]
    return widths, offsets, sum(widths)


def k_tables(ranks):
    """paged_quant.py:114-131: (nouts [H], head_of_lane [W], (tile_head, tile_nout, tile_last))."""
    nouts = [n_outlier(r) for r in ranks]
    lanes, head, t_out, last = [], [], [], []
    for h, (r, no) in enumerate(zip(ranks, nouts)):
        tiles = -(-r // 16)
        lanes += [h] * (16 * tiles)
        for j in range(tiles):
            head.append(h)
            t_out.append(max(0, min(16, no - 16 * j)))
            last.append(int(j == tiles - 1))
    a = lambda v: np.asarray(v, dtype=np.int32)  # noqa: E731
    return a(nouts), a(lanes), (a(head), a(t_out), a(last))


def block_hadamard(rank: int, n_out: int, generator):
    """paged_quant.py:50-68 (= kv_quant.py:84-103). Signs come from torch's CPU generator."""
    import torch
    T = np.eye(rank, dtype=np.float64)
    for a, n in ((0, n_out), (n_out, rank - n_out)):
        if n <= 1:
            continue
        m = 1 << (n.bit_length() - 1)
        H = np.ones((1, 1))
        while H.shape[0] < m:
            H = np.block([[H, H], [H, -H]])
        u = torch.rand(m, generator=generator, device="cpu").numpy()
        signs = np.where(u < 0.5, -1.0, 1.0)
        T[a:a + m, a:a + m] = signs[:, None] * H / math.sqrt(m)
    return T


# ---------------------------------------------------------------------------
# Paged gathers
# ---------------------------------------------------------------------------

def gather_rows(cache: np.ndarray, block_table_row: np.ndarray, L: int, block_size: int) -> np.ndarray:
    """Rows of tokens 0..L-1: cache[bt[l // bs], l % bs] (paged_decode.py:63-69)."""
    l = np.arange(L)
    return cache[block_table_row[l // block_size], l % block_size]


def unpack_rows(rows: np.ndarray, lay: dict, ranks) -> tuple:
    """Dequantize uint8 rows [L, nbytes] -> (K [L, W] f64, V [L, R] f64). kv_quant.py:154-188."""
    rows = np.asarray(rows, dtype=np.uint8)
    W, H, R = lay["k_width"], lay["num_kv_heads"], lay["v_rank"]
    kb = rows[:, :W // 2].astype(np.int64)
    nib = np.stack([kb & 15, kb >> 4], -1).reshape(rows.shape[0], W) - 8
    sc = rows[:, lay["ks_off"]:lay["ks_off"] + 4 * H].copy().view(np.uint16).astype(np.uint32) << 16
    sc = sc.view(np.float32).astype(np.float64).reshape(-1, H, 2)
    widths, offsets, _ = head_layout(ranks)
    K = np.zeros((rows.shape[0], W))
    for h in range(H):
        o, w, no = offsets[h], widths[h], n_outlier(ranks[h])
        K[:, o:o + no] = nib[:, o:o + no] * sc[:, h, 0:1]
        K[:, o + no:o + w] = nib[:, o + no:o + w] * sc[:, h, 1:2]
    vs = rows[:, lay["vs_off"]:lay["vs_off"] + 4].copy().view(np.uint16).astype(np.uint32) << 16
    vs = vs.view(np.float32).astype(np.float64).reshape(-1, 2)
    nout, nbo = lay["v_nout"], lay["v_nbo"]
    vb = rows[:, lay["vq_off"]:lay["vq_off"] + lay["v_bytes"]].astype(np.int64)
    vn = np.stack([vb & 15, vb >> 4], -1).reshape(rows.shape[0], -1) - 8
    V = np.concatenate([vn[:, :nout] * vs[:, 0:1],
                        vn[:, 2 * nbo:2 * nbo + R - nout] * vs[:, 1:2]], axis=1)
    return K, V


# ---------------------------------------------------------------------------
# Decode math, float64
# ---------------------------------------------------------------------------

def _rope(k: np.ndarray, cs: np.ndarray) -> np.ndarray:
    """NeoX rotate-half with cos = cs[:, :64], sin = cs[:, 64:] (paged_decode.py:89-95)."""
    h = k.shape[-1] // 2
    cos, sin = cs[:, :h], cs[:, h:]
    k0, k1 = k[:, :h], k[:, h:]
    return np.concatenate([k0 * cos - k1 * sin, k1 * cos + k0 * sin], axis=1)


def _attend(q, keys_rot, V, scale, v_up_h):
    """softmax(q . k * scale) @ V, lifted by v_up_h [r_v, D]. Returns [D]."""
    logits = keys_rot @ q * scale
    m = logits.max()
    p = np.exp(logits - m)
    p /= p.sum()
    return (p @ V) @ v_up_h


def lowrank_decode(q, cache, block_table, seq_lens, max_seq_len, k_up, k_ranks, k_offsets, k_width,
                   v_up_by_q, cos_sin, scale):
    """float64 truth for paged_starkv_decode (paged_decode.py:150-226, model.py:1333-1386).

    cache [nb, bs, W + r_v] codes; only the first rank_h lanes of a head are read
    (paged_decode.py:79-81). Returns [n, H_q, D] float64.
    """
    q = np.asarray(q, np.float64)
    n, Hq, D = q.shape
    Hkv = len(k_ranks)
    G = Hq // Hkv
    r_v = v_up_by_q.shape[1]
    bs = cache.shape[1]
    k_up = np.asarray(k_up, np.float64)
    vq = np.asarray(v_up_by_q, np.float64)
    cs_all = np.asarray(cos_sin, np.float64)
    out = np.full((n, Hq, D), np.nan)
    for b in range(n):
        L = min(int(seq_lens[b]), int(max_seq_len))
        if L <= 0:
            continue
        rows = gather_rows(cache, np.asarray(block_table[b]), L, bs).astype(np.float64)
        V = rows[:, k_width:k_width + r_v]
        cs = cs_all[:L]
        for kv in range(Hkv):
            R, off = int(k_ranks[kv]), int(k_offsets[kv])
            keys = _rope(rows[:, off:off + R] @ k_up[off:off + R], cs)
            for g in range(G):
                h = kv * G + g
                out[b, h] = _attend(q[b, h], keys, V, scale, vq[h])
    return out


def quant_decode(q, cache_u8, block_table, seq_lens, max_seq_len, lay, ranks, k_up, v_up_by_q,
                 cos_sin, scale):
    """float64 truth for paged_quant_decode (paged_quant.py:357-411) on the dequantized
    cache. MHA; every stored lane of a head (its rank rounded to 16) is used, as the
    reference's 16-lane tiles do (paged_quant.py:114-131, 282-304)."""
    q = np.asarray(q, np.float64)
    n, H, D = q.shape
    bs = cache_u8.shape[1]
    widths, offsets, W = head_layout(ranks)
    k_up = np.asarray(k_up, np.float64)
    vq = np.asarray(v_up_by_q, np.float64)
    cs_all = np.asarray(cos_sin, np.float64)
    out = np.full((n, H, D), np.nan)
    for b in range(n):
        L = min(int(seq_lens[b]), int(max_seq_len))
        if L <= 0:
            continue
        rows = gather_rows(cache_u8, np.asarray(block_table[b]), L, bs)
        K, V = unpack_rows(rows, lay, ranks)
        cs = cs_all[:L]
        for h in range(H):
            o, w = offsets[h], widths[h]
            keys = _rope(K[:, o:o + w] @ k_up[o:o + w], cs)
            out[b, h] = _attend(q[b, h], keys, V, scale, vq[h])
    return out


def lowrank_decode_bruteforce(q, cache, block_table, seq_lens, max_seq_len, k_up, k_ranks, k_offsets,
                              v_up_by_q, cos_sin, scale):
    """An independent float64 statement for small inputs: per-token loops, RoPE as a
    complex rotation (z_i = k_i + j k_{i+64}; z *= e^{j theta}), explicit softmax."""
    n, Hq, D = q.shape
    Hkv = len(k_ranks)
    G = Hq // Hkv
    r_v = v_up_by_q.shape[1]
    bs = cache.shape[1]
    out = np.full((n, Hq, D), np.nan)
    h2 = D // 2
    for b in range(n):
        L = min(int(seq_lens[b]), int(max_seq_len))
        if L <= 0:
            continue
        for h in range(Hq):
            kv = h // G
            R, off = int(k_ranks[kv]), int(k_offsets[kv])
            width = cache.shape[2] - r_v
            logits = []
            vrows = []
            for l in range(L):
                row = np.asarray(cache[int(block_table[b][l // bs]), l % bs], np.float64)
                k = sum(row[off + r] * np.asarray(k_up[off + r], np.float64) for r in range(R))
                zc = (k[:h2] + 1j * k[h2:]) * (np.asarray(cos_sin[l, :h2], np.float64)
                                                 + 1j * np.asarray(cos_sin[l, h2:], np.float64))
                krot = np.concatenate([zc.real, zc.imag])
                logits.append(float(np.dot(np.asarray(q[b, h], np.float64), krot)) * scale)
                vrows.append(row[width:width + r_v])
            logits = np.array(logits)
            w = np.exp(logits - logits.max())
            w = w / w.sum()
            o = sum(w[l] * vrows[l] for l in range(L))
            out[b, h] = o @ np.asarray(v_up_by_q[h], np.float64)
    return out


def dense_prefill(q, k_codes, v_codes, query_start_loc, k_up, k_ranks, k_offsets, v_up, cos_sin, scale):
    """float64 truth for the backend's dense prefill (attention.py:219-251): per prompt
    (tokens query_start_loc[i] .. query_start_loc[i + 1], positions from 0, no cached
    context), K of KV head h = RoPE(codes[:, off_h : off_h + rank_h] @ k_up[off_h : ...]),
    V = v_codes @ v_up^T ([T, H_kv * D]), causal softmax(q . k * scale) @ V per query head
    (query head h reads KV head h // (H_q / H_kv)). q [T, H_q, D]. Returns [T, H_q, D]."""
    q = np.asarray(q, np.float64)
    T, Hq, D = q.shape
    Hkv = len(k_ranks)
    G = Hq // Hkv
    kc = np.asarray(k_codes, np.float64)
    U = np.asarray(k_up, np.float64)
    Vall = np.asarray(v_codes, np.float64) @ np.asarray(v_up, np.float64).T  # [T, Hkv * D]
    cs_all = np.asarray(cos_sin, np.float64)
    out = np.zeros((T, Hq, D))
    qsl = [int(x) for x in query_start_loc]
    for i in range(len(qsl) - 1):
        a, b = qsl[i], qsl[i + 1]
        L = b - a
        if L <= 0:
            continue
        cs = cs_all[:L]
        causal = np.tril(np.ones((L, L), bool))
        for kv in range(Hkv):
            R, off = int(k_ranks[kv]), int(k_offsets[kv])
            keys = _rope(kc[a:b, off:off + R] @ U[off:off + R], cs)        # [L, D]
            V = Vall[a:b, kv * D:(kv + 1) * D]
            for g in range(G):
                h = kv * G + g
                logits = (q[a:b, h] @ keys.T) * scale
                logits = np.where(causal, logits, -np.inf)
                p = np.exp(logits - logits.max(axis=1, keepdims=True))
                p /= p.sum(axis=1, keepdims=True)
                out[a:b, h] = p @ V
    return out


def causal_attention(q, k, v, query_start_loc, scale):
    """float64 truth for the prefill kernel's attention over given K and V (the
    flash_attn_varlen_func call of attention.py:243-249, causal=True): per prompt (tokens
    query_start_loc[i] .. query_start_loc[i + 1]), softmax(q . k * scale) @ v over the
    prompt's tokens up to the query's own; query head h reads KV head h // (H_q / H_kv).
    q [T, H_q, D], k and v [T, H_kv, D]. Returns [T, H_q, D]."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    T, Hq, D = q.shape
    G = Hq // k.shape[1]
    out = np.zeros((T, Hq, D))
    qsl = [int(x) for x in query_start_loc]
    for i in range(len(qsl) - 1):
        a, b = qsl[i], qsl[i + 1]
        if b <= a:
            continue
        causal = np.tril(np.ones((b - a, b - a), bool))
        for h in range(Hq):
            logits = np.where(causal, (q[a:b, h] @ k[a:b, h // G].T) * scale, -np.inf)
            p = np.exp(logits - logits.max(axis=1, keepdims=True))
            out[a:b, h] = (p / p.sum(axis=1, keepdims=True)) @ v[a:b, h // G]
    return out


def fold_q(q, k_up, head_of_lane, scale):
    """A|B of paged_quant.py:241-255 in float64: [n, W, 128]."""
    q = np.asarray(q, np.float64)
    U = np.asarray(k_up, np.float64)
    h2 = U.shape[1] // 2
    qh = q[:, np.asarray(head_of_lane), :]                           # [n, W, 128]
    A = qh[..., :h2] * U[None, :, :h2] + qh[..., h2:] * U[None, :, h2:]
    B = qh[..., h2:] * U[None, :, :h2] - qh[..., :h2] * U[None, :, h2:]
    return np.concatenate([A, B], -1) * scale


# ---------------------------------------------------------------------------
# The reference's own roundings (reporting only)
# ---------------------------------------------------------------------------

def emulate_lowrank_reference(q, cache, block_table, seq_lens, max_seq_len, k_up, k_ranks, k_offsets,
                              k_width, v_up_by_q, cos_sin, scale):
    """paged_starkv_decode's rounding points, emulated with torch CPU: fp32 lift+RoPE+dot,
    logits stored in the query dtype (paged_decode.py:179-180), mul_(scale) in that dtype
    and softmax to that dtype (199), fp32 P@V (144), sum, round to the weight dtype (225),
    bmm in the weight dtype (225)."""
    import torch
    qt = torch.as_tensor(q)
    dt = qt.dtype
    n, Hq, D = qt.shape
    Hkv = len(k_ranks)
    G = Hq // Hkv
    r_v = v_up_by_q.shape[1]
    bs = cache.shape[1]
    cache_t = torch.as_tensor(cache).float()
    U = torch.as_tensor(k_up).float()
    cs_t = torch.as_tensor(cos_sin).float()
    vq = torch.as_tensor(v_up_by_q)
    out = torch.full((n, Hq, D), float("nan"), dtype=vq.dtype)
    for b in range(n):
        L = min(int(seq_lens[b]), int(max_seq_len))
        if L <= 0:
            continue
        l = torch.arange(L)
        bt = torch.as_tensor(np.asarray(block_table[b])).long()
        rows = cache_t[bt[l // bs], l % bs]
        V = rows[:, k_width:k_width + r_v].to(dt)
        logits = torch.empty(Hq, L, dtype=dt)
        cs = cs_t[:L]
        h2 = D // 2
        for h in range(Hq):
            kv = h // G
            R, off = int(k_ranks[kv]), int(k_offsets[kv])
            k = rows[:, off:off + R] @ U[off:off + R]
            k0, k1 = k[:, :h2], k[:, h2:]
            kr = torch.cat([k0 * cs[:, :h2] - k1 * cs[:, h2:], k1 * cs[:, :h2] + k0 * cs[:, h2:]], 1)
            logits[h] = (kr @ qt[b, h].float()).to(dt)
        probs = torch.softmax(logits.mul_(scale), dim=-1)
        acc = (probs.float() @ V.float()).to(vq.dtype)              # [Hq, r_v]
        out[b] = torch.bmm(acc[:, None, :], vq)[:, 0, :]
    return out.float().numpy()
