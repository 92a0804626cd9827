"""Prompts through the model, then decode (config 4's path from prompts, on the shrunk
4-layer shape of test_gpu_model: layers 1 and 2 compressed, 0 and 3 full): three whole
prompts of 100, 37 and 260 tokens in one prefill_step, then two decode steps from the
prompts' greedy next tokens.

Checks:
- the prefill's logits are finite, one row per prompt;
- each layer's prefill attention output against the float64 oracle: a compressed layer
  against ref.dense_prefill over the step's codes (hidden @ kv_down^T rounded to bf16,
  formed here in float64 from the captured layer input), a full layer against
  ref.causal_attention over its captured K and V; tolerance as the decode tests (max-abs
  2e-2, mean-rel 1e-3);
- the two decode steps' layer outputs against the decode oracle over the caches the
  prefill (and the steps) wrote: this checks every cache row the prefill wrote, in the bf16
  and 3.2-bit modes and the stock model.
"""
import numpy as np
import pytest
import torch

from oracle import ref
from starkv_serve import model as M
from test_gpu_decode import assert_close
from test_gpu_model import SHAPE, build, decode_layer_truth

pytestmark = pytest.mark.gpu

PROMPTS = [100, 37, 260]


def prefill_layer_truth(model, c, qsl):
    li, layer = c["layer"], model.layers[c["layer"]]
    q = c["q"].float().cpu().numpy()
    if not layer.compressed:
        return ref.causal_attention(q, c["k"].float().cpu().numpy(), c["v"].float().cpu().numpy(), qsl, model.scale)
    imp = layer.impl
    codes = (c["h"].double() @ imp.kv_down.double().T).to(torch.bfloat16).double().cpu().numpy()
    return ref.dense_prefill(q, codes[:, :imp.k_width], codes[:, imp.k_width:], qsl, imp.w.k_up.float().numpy(),
                             imp.w.k_head_ranks.tolist(), imp.w.k_head_offsets.tolist(), imp.w.v_up.float().numpy(),
                             imp.rotary_emb.cos_sin_cache.float().cpu().numpy(), imp.scale)


@pytest.mark.parametrize("mode", ["bf16", "quant", "stock"])
def test_prompts_then_decode_against_oracle(cuda, tmp_path, mode):
    print(f"\n[prompts] mode={mode} prompts={PROMPTS}", flush=True)
    model, bt = build(cuda, tmp_path, mode == "quant", stock=mode == "stock")
    # build() filled the prompts' rows with random ones; the prefill overwrites every one.
    g = torch.Generator().manual_seed(77)
    tokens = torch.randint(0, SHAPE.vocab_size, (sum(PROMPTS),), generator=g).to(cuda)
    md, positions = M.prefill_metadata(bt, PROMPTS, 16)
    cap = []
    logits = model.prefill_step(tokens, positions, md, capture=cap)
    torch.cuda.synchronize()
    assert logits.shape == (len(PROMPTS), SHAPE.vocab_size) and torch.isfinite(logits).all()
    assert [c["layer"] for c in cap] == list(range(SHAPE.num_layers))
    qsl = md.prefill_query_start_loc_cpu
    for c in cap:
        assert torch.isfinite(c["out"]).all()
        assert_close(c["out"], prefill_layer_truth(model, c, qsl), f"{mode} prefill layer {c['layer']}")
    print(f"[prompts] {mode}: prefill checked", flush=True)

    bt_host = bt.cpu().numpy()
    nxt = logits.argmax(-1)
    for step in range(2):
        pos = torch.tensor(PROMPTS, device=cuda) + step
        dmd = M.decode_metadata(bt, pos, 16, int(pos.max()) + 1)
        cap = []
        logits = model.decode_step(nxt, pos, dmd, capture=cap)
        torch.cuda.synchronize()
        assert torch.isfinite(logits).all()
        seq = (pos + 1).cpu().numpy()
        for c in cap:
            assert_close(c["out"], decode_layer_truth(model, c, bt_host, seq), f"{mode} step {step} layer {c['layer']}")
        nxt = logits.argmax(-1)
