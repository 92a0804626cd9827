"""Pin the float64 dense-prefill oracle (attention.py:219-251 restated) against the
decode oracle (itself pinned by a brute-force loop): the last token of a prompt attends
to exactly the prompt's tokens, as a decode over the same codes does. Also: a prompt's
first token returns its own lifted V, and outputs are causal."""
import numpy as np

from oracle import ref

D = 128


def _case(lengths, ranks, Hq, v_rank, seed):
    rng = np.random.default_rng(seed)
    Hkv = len(ranks)
    widths, offsets, W = ref.head_layout(ranks)
    T = sum(lengths)
    k_codes = rng.standard_normal((T, W))
    for h, (r, w) in enumerate(zip(ranks, widths)):
        k_codes[:, offsets[h] + r:offsets[h] + w] = 7.0  # padding lanes: must be ignored
    v_codes = rng.standard_normal((T, v_rank))
    k_up = np.zeros((W, D))
    for h, r in enumerate(ranks):
        k_up[offsets[h]:offsets[h] + r] = rng.standard_normal((r, D)) / np.sqrt(r)
    v_up = rng.standard_normal((Hkv * D, v_rank)) / np.sqrt(v_rank)
    q = rng.standard_normal((T, Hq, D))
    pos = np.arange(max(lengths) + 1)[:, None]
    theta = 10000.0 ** (-np.arange(D // 2) / (D // 2))
    cs = np.concatenate([np.cos(pos * theta), np.sin(pos * theta)], axis=1)
    qsl = np.concatenate([[0], np.cumsum(lengths)])
    return dict(q=q, k_codes=k_codes, v_codes=v_codes, qsl=qsl, k_up=k_up, ranks=ranks, offsets=offsets, W=W,
                v_up=v_up, cs=cs, scale=D ** -0.5, Hkv=Hkv, Hq=Hq, v_rank=v_rank)


def _prefill(c, **over):
    c = {**c, **over}
    return ref.dense_prefill(c["q"], c["k_codes"], c["v_codes"], c["qsl"], c["k_up"], c["ranks"], c["offsets"],
                             c["v_up"], c["cs"], c["scale"])


def test_last_token_matches_decode_oracle():
    lengths = [37, 1, 20, 16]
    c = _case(lengths, ranks=[16, 20, 48, 5], Hq=8, v_rank=32, seed=1)
    out = _prefill(c)
    G = c["Hq"] // c["Hkv"]
    # v_up_by_q[h] = v_up rows of KV head h // G, transposed: [r_v, D]
    vq = np.stack([c["v_up"][(h // G) * D:(h // G + 1) * D].T for h in range(c["Hq"])])
    bs = 16
    for i, L in enumerate(lengths):
        a = c["qsl"][i]
        rows = np.concatenate([c["k_codes"][a:a + L], c["v_codes"][a:a + L]], axis=1)
        pages = -(-L // bs)
        cache = np.zeros((pages, bs, rows.shape[1]))
        cache.reshape(-1, rows.shape[1])[:L] = rows
        bt = np.arange(pages, dtype=np.int32)[None, :]
        dec = ref.lowrank_decode(c["q"][a + L - 1][None], cache, bt, [L], L, c["k_up"], c["ranks"], c["offsets"],
                                 c["W"], vq, c["cs"], c["scale"])
        np.testing.assert_allclose(out[a + L - 1], dec[0], rtol=1e-10, atol=1e-12)


def test_first_token_returns_its_value():
    lengths = [5, 9]
    c = _case(lengths, ranks=[32, 16], Hq=4, v_rank=16, seed=2)
    out = _prefill(c)
    G = c["Hq"] // c["Hkv"]
    for a in c["qsl"][:-1]:
        vfull = c["v_codes"][a] @ c["v_up"].T
        for h in range(c["Hq"]):
            np.testing.assert_allclose(out[a, h], vfull[(h // G) * D:(h // G + 1) * D], rtol=1e-12, atol=1e-12)


def test_causal_and_prompts_independent():
    c = _case([12, 7], ranks=[16, 16], Hq=2, v_rank=16, seed=3)
    base = _prefill(c)
    # Changing the last token of prompt 0 changes only that token's own output.
    k2 = c["k_codes"].copy()
    k2[11] += 1.0
    v2 = c["v_codes"].copy()
    v2[11] -= 2.0
    out = _prefill(c, k_codes=k2, v_codes=v2)
    np.testing.assert_array_equal(out[:11], base[:11])
    np.testing.assert_array_equal(out[12:], base[12:])
    assert not np.allclose(out[11], base[11])


def test_causal_attention_matches_torch_sdpa():
    """causal_attention (the prefill kernel's truth) against torch's float64 CPU
    scaled_dot_product_attention, per prompt, with GQA."""
    import torch
    rng = np.random.default_rng(7)
    lengths, Hq, Hkv = [5, 1, 70], 8, 2
    T = sum(lengths)
    q, k, v = rng.standard_normal((T, Hq, D)), rng.standard_normal((T, Hkv, D)), rng.standard_normal((T, Hkv, D))
    qsl = np.concatenate([[0], np.cumsum(lengths)])
    out = ref.causal_attention(q, k, v, qsl, 0.09)
    G = Hq // Hkv
    for i in range(len(lengths)):
        a, b = qsl[i], qsl[i + 1]
        qt = torch.from_numpy(q[a:b]).transpose(0, 1)
        kt = torch.from_numpy(k[a:b]).repeat_interleave(G, dim=1).transpose(0, 1)
        vt = torch.from_numpy(v[a:b]).repeat_interleave(G, dim=1).transpose(0, 1)
        o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=True, scale=0.09)
        np.testing.assert_allclose(out[a:b], o.transpose(0, 1).numpy(), rtol=1e-12, atol=1e-12)
    # a prompt's first token attends to itself alone
    np.testing.assert_allclose(out[qsl[:-1].astype(int)], v[qsl[:-1].astype(int)].repeat(G, axis=1), atol=1e-14)


def test_dense_prefill_is_causal_attention_over_lifted_kv():
    """dense_prefill = causal_attention over RoPE(codes @ U) and codes @ v_up^T."""
    c = _case([9, 33], [16, 32], 4, 64, 11)
    T = c["q"].shape[0]
    k = np.zeros((T, c["Hkv"], D))
    for h, (r, off) in enumerate(zip(c["ranks"], c["offsets"])):
        lifted = c["k_codes"][:, off:off + r] @ c["k_up"][off:off + r]
        for i in range(len(c["qsl"]) - 1):
            a, b = int(c["qsl"][i]), int(c["qsl"][i + 1])
            k[a:b, h] = ref._rope(lifted[a:b], c["cs"][:b - a])
    v = (c["v_codes"] @ c["v_up"].T).reshape(T, c["Hkv"], D)
    np.testing.assert_allclose(ref.causal_attention(c["q"], k, v, c["qsl"], c["scale"]), _prefill(c), atol=1e-12)
