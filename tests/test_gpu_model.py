"""The vLLM-free STAR-KV Llama decode step (starkv_serve/model.py) on a shrunk shape:
4 layers (1 and 2 compressed from a fused checkpoint, 0 and 3 full), 4 heads x 128,
3 requests. The prompts' cache rows are written through the layers' own write paths
(the fused codes write for compressed layers, K/V scatter for full ones); then two
decode steps run, and each layer's attention output of each step is compared with the
float64 oracle over the cache as it stands after that step's write: compressed layers
with oracle/ref.py's decode (bf16 codes or the 3.2-bit rows), full layers with plain
softmax attention over the gathered K/V. Tolerance as the decode tests (max-abs 2e-2,
mean-rel 1e-3). Also the stock model (every layer full) and the uncompressed-attention
kernel alone against the oracle, with GQA, and the step captured in a HIP graph
(DecodeGraph) against the same steps run eagerly over the same span."""
import numpy as np
import pytest
import torch

from oracle import ref
from starkv_serve import checkpoint as ck
from starkv_serve import model as M
from starkv_serve.kernels.stock_decode import paged_decode_full, write_kv_full
from test_gpu_decode import assert_close

pytestmark = pytest.mark.gpu

SHAPE = M.LlamaShape(hidden_size=512, num_layers=4, num_heads=4, num_kv_heads=4, head_dim=128,
                     intermediate_size=1024, vocab_size=1000)
PROMPTS = [100, 37, 260]
STEPS = 2


def full_attention_truth(q, kc, vc, bt, seq_lens, scale):
    """float64 softmax attention of q [n, Hq, D] over the gathered caches."""
    q = q.float().cpu().numpy().astype(np.float64)
    kc, vc = kc.float().cpu().numpy(), vc.float().cpu().numpy()
    n, Hq, D = q.shape
    G = Hq // kc.shape[2]
    out = np.zeros((n, Hq, D))
    for b in range(n):
        L = int(seq_lens[b])
        l = np.arange(L)
        K = kc[bt[b, l // 16], l % 16].astype(np.float64)
        V = vc[bt[b, l // 16], l % 16].astype(np.float64)
        for h in range(Hq):
            s = K[:, h // G] @ q[b, h] * scale
            p = np.exp(s - s.max())
            out[b, h] = (p / p.sum()) @ V[:, h // G]
    return out


def decode_layer_truth(model, c, bt_host, seq):
    """float64 truth of one layer's decode output `c` (a decode_step capture entry) over
    the layer's cache as the step left it: oracle/ref.py's decode for a compressed layer
    (bf16 codes or 3.2-bit rows), softmax attention over the gathered K/V for a full one."""
    li, layer = c["layer"], model.layers[c["layer"]]
    if not layer.compressed:
        kc, vc = model.kv_caches[li]
        return full_attention_truth(c["q"], kc, vc, bt_host, seq, model.scale)
    imp = layer.impl
    q = c["q"].float().cpu().numpy()
    vq = imp.v_up_by_q.float().cpu().numpy()
    cs = imp.rotary_emb.cos_sin_cache.float().cpu().numpy()
    ranks = imp.w.k_head_ranks.tolist()
    if imp.row is None:
        cache = model.kv_caches[li].float().cpu().numpy()
        return ref.lowrank_decode(q, cache, bt_host, seq, int(seq.max()), imp.k_up.float().cpu().numpy(), ranks,
                                  imp.k_head_offsets.tolist(), imp.k_width, vq, cs, imp.scale)
    lay = ref.row_layout(imp.k_width, len(ranks), imp.w.v_rank)
    return ref.quant_decode(q, model.kv_caches[li].cpu().numpy(), bt_host, seq, int(seq.max()), lay, ranks,
                            imp.k_up.float().cpu().numpy(), vq, cs, imp.scale)


def build(cuda, tmp_path, kv_quant, stock=False):
    path = str(tmp_path / "fused_weights.pt")
    comp = {1: ([16, 32, 16, 48], 64), 2: ([32, 16, 16, 16], 96)}
    ck.write_fused_checkpoint(path, SHAPE.num_layers, SHAPE.num_kv_heads, SHAPE.head_dim, SHAPE.hidden_size, comp,
                              seed=11)
    c = ck.load_fused_checkpoint(path, SHAPE.num_layers, SHAPE.num_kv_heads, SHAPE.head_dim, dtype=torch.bfloat16,
                                 kv_quant=kv_quant)
    model = M.StarKVLlamaForCausalLM(SHAPE, c, max_model_len=512, device=cuda, seed=12, stock=stock)
    pages = [(L + STEPS + 15) // 16 for L in PROMPTS]
    g = torch.Generator().manual_seed(13)
    perm = (torch.randperm(sum(pages), generator=g) + 1).to(torch.int32)
    # Rows cover max_model_len (512) positions; columns past a request's pages hold the null block.
    bt = torch.zeros(len(PROMPTS), 512 // 16, dtype=torch.int32)
    o = 0
    for b, p in enumerate(pages):
        bt[b, :p] = perm[o:o + p]
        o += p
    model.allocate_kv_cache(sum(pages) + 1)
    bt = bt.to(cuda)
    # The prompts' rows, through each layer's write path.
    rows = torch.cat([torch.full((L,), b) for b, L in enumerate(PROMPTS)]).to(cuda)
    pos = torch.cat([torch.arange(L) for L in PROMPTS]).to(cuda)
    slots = bt[rows, pos // 16].long() * 16 + pos % 16
    for li, layer in enumerate(model.layers):
        hid = torch.randn(len(pos), SHAPE.hidden_size, generator=g).to(torch.bfloat16).to(cuda)
        if layer.compressed:
            layer.impl.write_from_hidden(hid, model.kv_caches[li], slots)
        else:
            kc, vc = model.kv_caches[li]
            kc[slots // 16, slots % 16] = torch.randn(len(pos), 4, 128, generator=g).to(torch.bfloat16).to(cuda)
            vc[slots // 16, slots % 16] = torch.randn(len(pos), 4, 128, generator=g).to(torch.bfloat16).to(cuda)
    return model, bt


@pytest.mark.parametrize("kv_quant", [False, True])
def test_model_decode_steps_against_oracle(cuda, tmp_path, kv_quant):
    print(f"\n[model] shrunk Llama, kv_quant={kv_quant}", flush=True)
    model, bt = build(cuda, tmp_path, kv_quant)
    bt_host = bt.cpu().numpy()
    tokens = torch.tensor([5, 17, 999], device=cuda)
    for step in range(STEPS):
        positions = torch.tensor(PROMPTS, device=cuda) + step
        md = M.decode_metadata(bt, positions, 16, int(positions.max()) + 1)
        cap = []
        logits = model.decode_step(tokens, positions, md, capture=cap)
        torch.cuda.synchronize()
        assert torch.isfinite(logits).all()
        seq = (positions + 1).cpu().numpy()
        assert [c["layer"] for c in cap] == [0, 1, 2, 3]
        for c in cap:
            assert_close(c["out"], decode_layer_truth(model, c, bt_host, seq), f"step {step} layer {c['layer']}")
        tokens = logits.argmax(-1)


def test_stock_model_and_gqa_kernel(cuda, tmp_path):
    model, bt = build(cuda, tmp_path, False, stock=True)
    assert not any(layer.compressed for layer in model.layers)
    positions = torch.tensor(PROMPTS, device=cuda)
    md = M.decode_metadata(bt, positions, 16, int(positions.max()) + 1)
    cap = []
    logits = model.decode_step(torch.tensor([1, 2, 3], device=cuda), positions, md, capture=cap)
    assert torch.isfinite(logits).all()
    seq = (positions + 1).cpu().numpy()
    for c in cap:
        kc, vc = model.kv_caches[c["layer"]]
        assert_close(c["out"], full_attention_truth(c["q"], kc, vc, bt.cpu().numpy(), seq, model.scale),
                     f"stock layer {c['layer']}")
    # the kernel alone: GQA groups of 2 and 4, many splits (one long request), block size 32
    g = torch.Generator().manual_seed(21)
    for Hq, Hkv, lens, bs in ((8, 4, [3000, 5], 16), (16, 4, [700], 32), (4, 4, [1, 16, 17], 16)):
        pages = [(L + bs - 1) // bs for L in lens]
        nb = sum(pages) + 1
        kc = torch.randn(nb, bs, Hkv, 128, generator=g).to(torch.bfloat16)
        vc = torch.randn(nb, bs, Hkv, 128, generator=g).to(torch.bfloat16)
        btk = torch.zeros(len(lens), max(pages), dtype=torch.int32)
        perm = torch.randperm(nb - 1, generator=g) + 1
        o = 0
        for b, p in enumerate(pages):
            btk[b, :p] = perm[o:o + p]
            o += p
        q = torch.randn(len(lens), Hq, 128, generator=g).to(torch.bfloat16)
        out = paged_decode_full(q.to(cuda), kc.to(cuda), vc.to(cuda), btk.to(cuda),
                                torch.tensor(lens, dtype=torch.int32, device=cuda), max(lens), 128 ** -0.5)
        # the truth gathers with block_size bs: fold the block into 16-token pages
        truth = np.zeros((len(lens), Hq, 128))
        qn, kn, vn = q.double().numpy(), kc.double().numpy(), vc.double().numpy()
        for b, L in enumerate(lens):
            l = np.arange(L)
            K = kn[btk[b, l // bs].numpy(), l % bs]
            V = vn[btk[b, l // bs].numpy(), l % bs]
            for h in range(Hq):
                s = K[:, h // (Hq // Hkv)] @ qn[b, h] * 128 ** -0.5
                p = np.exp(s - s.max())
                truth[b, h] = (p / p.sum()) @ V[:, h // (Hq // Hkv)]
        assert_close(out, truth, f"stock kernel Hq={Hq} Hkv={Hkv} lens={lens} bs={bs}")


@pytest.mark.parametrize("mode", ["bf16", "quant", "stock"])
def test_decode_graph_replays_match_eager(cuda, tmp_path, mode):
    """Three greedy steps replayed from one captured step equal three eager steps over the
    graph's span bit for bit (logits and tokens), with eager work and synchronizations
    between the replays; then a reset and a replay repeat the first step."""
    print(f"\n[model graph] {mode}", flush=True)
    model, bt = build(cuda, tmp_path, mode == "quant", stock=mode == "stock")
    tokens = torch.tensor([5, 17, 999], device=cuda)
    positions = torch.tensor(PROMPTS, device=cuda)
    dg = M.DecodeGraph(model, bt, tokens, positions)
    want, tok, pos = [], tokens.clone(), positions.clone()
    for _ in range(3):
        md = M.decode_metadata(bt, pos, 16, model.max_model_len)
        logits = model.decode_step(tok, pos, md, in_graph=True)
        tok = logits.argmax(-1)
        pos = pos + 1
        want.append((logits.clone(), tok.clone()))
    torch.cuda.synchronize()
    dg.reset(tokens, positions)
    for step, (lw, tw) in enumerate(want):
        dg.replay()
        torch.cuda.synchronize()
        assert torch.equal(dg.logits, lw), f"step {step}"
        assert torch.equal(dg.tokens, tw), f"step {step}"
        assert torch.equal(dg.positions, positions + step + 1)
        torch.randn(1000, device=cuda).sum().item()  # eager work between replays
    dg.reset(tokens, positions)
    dg.replay()
    torch.cuda.synchronize()
    assert torch.equal(dg.logits, want[0][0])


@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
def test_stock_write_matches_index_put(cuda, slot_dtype):
    """write_kv_full against torch's index_put on the same caches: bit-exact, slot -1
    writes nothing, strided key/value rows (views of one QKV output), block size 32."""
    print(f"\n[stock write] slots {slot_dtype}", flush=True)
    g = torch.Generator().manual_seed(31)
    nb, bs, Hkv, n = 9, 32, 4, 12
    qkv = torch.randn(n, (8 + 2 * Hkv) * 128, generator=g).to(torch.bfloat16).to(cuda)
    k = qkv[:, 8 * 128:(8 + Hkv) * 128].view(n, Hkv, 128)
    v = qkv[:, (8 + Hkv) * 128:].view(n, Hkv, 128)
    slots = torch.randperm(nb * bs, generator=g)[:n].to(slot_dtype)
    slots[3] = -1
    slots = slots.to(cuda)
    kc = torch.randn(nb, bs, Hkv, 128, generator=g).to(torch.bfloat16).to(cuda)
    vc = torch.randn(nb, bs, Hkv, 128, generator=g).to(torch.bfloat16).to(cuda)
    want_k, want_v = kc.clone(), vc.clone()
    ok = slots >= 0
    s = slots[ok].long()
    want_k[s // bs, s % bs] = k[ok]
    want_v[s // bs, s % bs] = v[ok]
    write_kv_full(k, v, kc, vc, slots)
    torch.cuda.synchronize()
    assert torch.equal(kc, want_k) and torch.equal(vc, want_v)
