"""The full decode step at its own shape: a random-init Llama-2-7B-shaped model (32 layers,
32 heads x 128, hidden 4096, MLP 11008, vocab 32000) with layers 0, 1, 2 and 31 keeping
full K/V and the others compressed at the 0.75 ratio (K ranks multiples of 16 keeping
~21.5 % of K: K width 880; V rank 1280), the factors written to a fused checkpoint and
read back by load_fused_checkpoint, one session of 16,384 context tokens, in the
bf16-code, 3.2-bit and stock modes.

Per mode, two eager decode steps:
- every layer's attention output and the logits are finite;
- step 1: compressed layer 3 and uncompressed layer 0, step 2: compressed layer 30 and
  uncompressed layer 31 (stock mode: all four uncompressed) against the float64 oracle
  over the cache as that step left it, at the decode tolerance (max-abs 2e-2, mean-rel
  1e-3);
- 3.2-bit: sampled context rows of layer 3 (written by the fused write) byte-exact to the
  C quantizer on the codes the write computed;
then the same two steps over the graph span, replayed from one captured step
(DecodeGraph), bit-identical to the eager steps over that span.
"""
import time

import numpy as np
import pytest
import torch

from oracle import cquant, ref
from starkv_serve import checkpoint as ck
from starkv_serve import model as M
from test_gpu_decode import assert_close
from test_gpu_model import full_attention_truth

pytestmark = pytest.mark.gpu

SHAPE = M.LLAMA2_7B
CONTEXT = 16384
STEPS = 2
FULL = (0, 1, 2, 31)
CHECKS = ((3, 0), (30, 31))  # per step: (a compressed layer, an uncompressed layer)
SEED = 4000


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory):
    t = time.time()
    g = torch.Generator().manual_seed(SEED)
    comp = {li: (M.ranks_for_ratio(32, 128, 0.215, 16, g), M.v_rank_for_ratio(32, 128, 0.315, 32))
            for li in range(SHAPE.num_layers) if li not in FULL}
    path = str(tmp_path_factory.mktemp("config4") / "fused_weights.pt")
    ck.write_fused_checkpoint(path, SHAPE.num_layers, SHAPE.num_kv_heads, SHAPE.head_dim, SHAPE.hidden_size, comp,
                              seed=SEED)
    print(f"\n[config 4] fused checkpoint written in {time.time() - t:.1f} s", flush=True)
    return path, comp


def _build(cuda, path, mode):
    c = None if mode == "stock" else ck.load_fused_checkpoint(
        path, SHAPE.num_layers, SHAPE.num_kv_heads, SHAPE.head_dim, dtype=torch.bfloat16, kv_quant=mode == "quant")
    pages = (CONTEXT + STEPS + 15) // 16
    model = M.StarKVLlamaForCausalLM(SHAPE, c, max_model_len=16 * pages, device=cuda, seed=SEED + 1,
                                     stock=mode == "stock")
    model.allocate_kv_cache(pages + 1)
    gg = torch.Generator(device=cuda).manual_seed(SEED + 2)
    bt = (torch.randperm(pages, device=cuda, generator=gg) + 1).to(torch.int32).view(1, pages)
    pos = torch.arange(CONTEXT, device=cuda)
    slots = bt[0, pos // 16].long() * 16 + pos % 16
    rows = None
    for li, layer in enumerate(model.layers):
        cache = model.kv_caches[li]
        if not layer.compressed:
            cache[0].normal_(generator=gg)
            cache[1].normal_(generator=gg)
        elif layer.impl.row is None:
            cache.normal_(generator=gg)
        else:  # 3.2-bit rows through the fused write (codes = hidden @ kv_down^T, packed)
            for a in range(0, CONTEXT, 4096):
                hid = torch.randn(4096, SHAPE.hidden_size, device=cuda, generator=gg).to(torch.bfloat16)
                codes = layer.impl.write_from_hidden(hid, cache, slots[a:a + 4096], return_codes=(li == 3))
                if li == 3:
                    rows = (codes, slots[a:a + 4096]) if rows is None else \
                        (torch.cat([rows[0], codes]), torch.cat([rows[1], slots[a:a + 4096]]))
    torch.cuda.synchronize()
    return model, bt, rows


def _check_rows(model, rows, count=256):
    """Sampled 3.2-bit rows of layer 3 against the C quantizer on the same codes."""
    imp = model.layers[3].impl
    codes, slots = rows
    idx = np.linspace(0, codes.shape[0] - 1, count).astype(int)
    k = codes[idx, :imp.k_width].float().cpu().numpy()
    v = codes[idx, imp.k_width:].float().cpu().numpy()
    ranks = imp.w.k_head_ranks.tolist()
    lay = ref.row_layout(imp.k_width, len(ranks), imp.w.v_rank)
    want = np.zeros((count, 1, lay["nbytes"]), np.uint8)
    _, offsets, _ = ref.head_layout(ranks)
    cquant.pack_kv(k, v, want, np.arange(count), ranks, offsets, [ref.n_outlier(r) for r in ranks], imp.w.v_rank,
                   lay["ks_off"], lay["vs_off"], lay["vq_off"])
    s = slots[idx].cpu().numpy()
    c = model.kv_caches[3].cpu().numpy()
    got = c[s // 16, s % 16]
    end = lay["vq_off"] + lay["v_bytes"]
    assert np.array_equal(got[:, :end], want[:, 0, :end])


def _truth(model, li, c, bt_host, seq):
    layer = model.layers[li]
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


@pytest.mark.timeout(600)
@pytest.mark.parametrize("mode", ["bf16", "quant", "stock"])
def test_config4_llama2_7b_one_16k_session(cuda, checkpoint, mode):
    path, comp = checkpoint
    t0 = time.time()
    print(f"\n[config 4] mode={mode}: 32 layers, 1 session x {CONTEXT} tokens", flush=True)
    model, bt, rows = _build(cuda, path, mode)
    if mode != "stock":
        compressed = [li for li, layer in enumerate(model.layers) if layer.compressed]
        assert compressed == [li for li in range(SHAPE.num_layers) if li not in FULL]
        imp = model.layers[3].impl
        assert imp.k_width == sum(comp[3][0]) == 880 and imp.w.v_rank == 1280
        assert imp.kv_groups == [(0, 32)]
    print(f"[config 4] {mode}: built and filled in {time.time() - t0:.1f} s", flush=True)
    if rows is not None:
        _check_rows(model, rows)
    bt_host = bt.cpu().numpy()
    tokens0 = torch.tensor([1234], device=cuda)
    pos0 = torch.tensor([CONTEXT], device=cuda)
    tok, pos = tokens0.clone(), pos0.clone()
    for step in range(STEPS):
        md = M.decode_metadata(bt, pos, 16, int(pos.max()) + 1)
        cap = []
        logits = model.decode_step(tok, pos, md, capture=cap)
        torch.cuda.synchronize()
        assert torch.isfinite(logits).all(), f"step {step}"
        assert [c["layer"] for c in cap] == list(range(SHAPE.num_layers))
        for c in cap:
            assert torch.isfinite(c["out"]).all(), f"step {step} layer {c['layer']}"
        seq = (pos + 1).cpu().numpy()
        for li in CHECKS[step]:
            assert_close(cap[li]["out"], _truth(model, li, cap[li], bt_host, seq), f"{mode} step {step} layer {li}")
        print(f"[config 4] {mode}: step {step} checked ({time.time() - t0:.1f} s)", flush=True)
        tok, pos = logits.argmax(-1), pos + 1

    # The same two steps over the graph span, eagerly, then replayed from one captured step.
    want, tok, pos = [], tokens0.clone(), pos0.clone()
    for _ in range(STEPS):
        md = M.decode_metadata(bt, pos, 16, model.max_model_len)
        logits = model.decode_step(tok, pos, md, in_graph=True)
        tok, pos = logits.argmax(-1), pos + 1
        want.append((logits.clone(), tok.clone()))
    torch.cuda.synchronize()
    dg = M.DecodeGraph(model, bt, tokens0, pos0)
    dg.reset(tokens0, pos0)
    for step, (lw, tw) in enumerate(want):
        dg.replay()
        torch.cuda.synchronize()
        assert torch.equal(dg.logits, lw), f"{mode} graph step {step}"
        assert torch.equal(dg.tokens, tw), f"{mode} graph step {step}"
        torch.randn(1000, device=cuda).sum().item()  # eager work between replays
    print(f"[config 4] {mode}: graph replays equal eager steps ({time.time() - t0:.1f} s)", flush=True)
    del dg, model
    torch.cuda.empty_cache()
