"""The backend's per-layer forward on the GPU (attention.py:168-213): a decode step
with graph-padding rows, through ``StarKVAttentionImpl`` over a vLLM-shaped cache
[num_blocks, 1, block_size, width] (bf16 for both modes; the 3.2-bit rows are viewed
as bytes, as the reference does).

1. The prompt tokens go in through the fused write (``write_from_hidden``).
2. The step's own token: its codes are the model's GEMM (hidden @ kv_down^T,
   model.py:71), handed to ``forward`` as key / value.
3. ``forward`` writes them and decodes.

Checks:
- the real requests' outputs against the float64 oracle over the resulting cache,
  within the decode tolerance (max-abs 2e-2, mean-rel 1e-3), both eager (span =
  max_seq_len) and in-graph (span = max_model_len);
- padding rows (slot -1, length 0) write only the null block 0 and give finite
  outputs;
- output rows past the batch's tokens are untouched.

A mixed batch (decodes, then whole prompts) checks the dense prefill as well: the
prompts' outputs against the float64 dense-prefill oracle over the step's own codes.
"""
import types

import numpy as np
import pytest
import torch

from oracle import ref
from starkv_serve import checkpoint as ck
from starkv_serve import workloads as W
from starkv_serve.attention import StarKVAttentionImpl, StarKVMetadata
from test_gpu_decode import assert_close

pytestmark = pytest.mark.gpu

HIDDEN, MAX_MODEL_LEN = 512, 2048
RANKS = [16, 32, 48, 64, 24, 16, 40, 56]
V_RANK = 48
LENGTHS = [300, 77, 16, 1]  # after this step
PAD = 2                     # graph-padding rows


@pytest.mark.parametrize("quant,num_heads,in_graph,fused", [(False, 16, False, False), (False, 16, True, False),
                                                            (True, 8, False, False), (True, 8, True, False),
                                                            (False, 16, False, True), (True, 8, True, True)])
def test_forward_decode_step(cuda, tmp_path, quant, num_heads, in_graph, fused):
    """`fused`: the layer is built with fused_write (the vLLM model's compressed layers):
    forward receives the layer's input as key and the write kernel forms the codes."""
    print(f"\n[attention forward] quant={quant} heads={num_heads} in_graph={in_graph} fused={fused}", flush=True)
    path = str(tmp_path / "fused_weights.pt")
    ck.write_fused_checkpoint(path, 1, len(RANKS), 128, HIDDEN, {0: (RANKS, V_RANK)}, seed=21)
    w = ck.load_fused_checkpoint(path, 1, len(RANKS), 128, dtype=torch.bfloat16, kv_quant=quant).layers[0]
    g = torch.Generator().manual_seed(22)
    T = max(LENGTHS) + 1
    cs = W.cos_sin_table(MAX_MODEL_LEN, torch.bfloat16, cuda)
    rope = types.SimpleNamespace(cos_sin_cache=cs)
    impl = StarKVAttentionImpl(num_heads, 128, 128 ** -0.5, len(RANKS), starkv_layer=w, rotary_emb=rope,
                               max_model_len=MAX_MODEL_LEN, fused_write=fused)
    impl.to_device(cuda, torch.bfloat16)

    bt, nblk = W._page_layout(LENGTHS, g)
    n = len(LENGTHS)
    width = impl.row.nbytes // 2 if quant else w.cache_width
    kv_cache = torch.zeros(nblk, 1, W.BLOCK_SIZE, width, dtype=torch.bfloat16, device=cuda)
    if not quant:
        kv_cache.fill_(float("nan"))  # unused slots: masking must keep them out

    # 1. prompt tokens (positions 0 .. L-2) through the fused write
    prompt = [L - 1 for L in LENGTHS]
    blocks, slots = W._token_slots(prompt, bt)
    if blocks.numel():
        x = torch.randn(blocks.numel(), HIDDEN, generator=g).to(torch.bfloat16).to(cuda)
        impl.write_from_hidden(x, kv_cache, (blocks * W.BLOCK_SIZE + slots).to(cuda))

    # 2. this step: one token per request at position L - 1, plus padding rows
    pos = torch.tensor([L - 1 for L in LENGTHS])
    step_slots = bt[torch.arange(n), pos // W.BLOCK_SIZE].long() * W.BLOCK_SIZE + pos % W.BLOCK_SIZE
    slot_mapping = torch.cat([step_slots, torch.full((PAD,), -1, dtype=torch.long)]).to(cuda)
    hidden = torch.randn(n + PAD, HIDDEN, generator=g).to(torch.bfloat16).to(cuda)
    codes = hidden @ impl.kv_down.T
    key, value = codes[:, :impl.k_width], codes[:, impl.k_width:]
    query = torch.randn(n + PAD, num_heads * 128, generator=g).to(torch.bfloat16).to(cuda)
    seq_lens = torch.tensor(LENGTHS + [0] * PAD, dtype=torch.int32, device=cuda)
    block_table = torch.cat([bt, torch.zeros(PAD, bt.shape[1], dtype=torch.int32)]).to(cuda)
    md = StarKVMetadata(num_actual_tokens=n + PAD, num_decodes=n + PAD, num_decode_tokens=n + PAD, num_prefills=0,
                        max_seq_len=max(LENGTHS), seq_lens=seq_lens, block_table=block_table,
                        slot_mapping=slot_mapping)
    output = torch.full((n + PAD + 3, num_heads * 128), 7.0, dtype=torch.bfloat16, device=cuda)
    null_before = kv_cache[0].clone()
    if fused:
        impl.forward(None, query, hidden, hidden.new_empty(0), kv_cache, md, output, in_full_graph=in_graph)
    else:
        impl.forward(None, query, key, value, kv_cache, md, output, in_full_graph=in_graph)
    torch.cuda.synchronize()

    assert torch.all(output[n + PAD:] == 7.0)
    out = output[:n + PAD].view(n + PAD, num_heads, 128)
    assert torch.isfinite(out).all()
    # Padding rows wrote their codes into the null block only (block 0, slot 0).
    changed = (kv_cache[0].view(torch.int16) != null_before.view(torch.int16)).view(W.BLOCK_SIZE, -1).any(dim=1)
    assert not changed[1:].any()

    cache = kv_cache.squeeze(1)
    q = query[:n].view(n, num_heads, 128).float().cpu().numpy()
    if quant:
        lay = ref.row_layout(impl.k_width, len(RANKS), w.v_rank)
        truth = ref.quant_decode(q, cache.view(torch.uint8).cpu().numpy(), bt.numpy(), np.array(LENGTHS),
                                 max(LENGTHS), lay, RANKS, impl.k_up.float().cpu().numpy(),
                                 impl.v_up_by_q.float().cpu().numpy(), cs.float().cpu().numpy(), impl.scale)
    else:
        truth = ref.lowrank_decode(q, cache.float().cpu().numpy(), bt.numpy(), np.array(LENGTHS), max(LENGTHS),
                                   impl.k_up.float().cpu().numpy(), RANKS, w.k_head_offsets.tolist(), impl.k_width,
                                   impl.v_up_by_q.float().cpu().numpy(), cs.float().cpu().numpy(), impl.scale)
    assert_close(out[:n], truth, f"forward quant={quant} in_graph={in_graph} fused={fused}")


@pytest.mark.parametrize("quant,num_heads", [(False, 16), (True, 8)])
def test_forward_mixed_decode_and_prefill(cuda, tmp_path, quant, num_heads):
    """Decodes first, then whole prompts (attention.py:194-217): the decodes against the
    decode oracle over the cache the step wrote, the prompts against the dense-prefill
    oracle over the step's own codes."""
    print(f"\n[attention mixed] quant={quant} heads={num_heads}", flush=True)
    path = str(tmp_path / "fused_weights.pt")
    ck.write_fused_checkpoint(path, 1, len(RANKS), 128, HIDDEN, {0: (RANKS, V_RANK)}, seed=31)
    w = ck.load_fused_checkpoint(path, 1, len(RANKS), 128, dtype=torch.bfloat16, kv_quant=quant).layers[0]
    g = torch.Generator().manual_seed(32)
    cs = W.cos_sin_table(MAX_MODEL_LEN, torch.bfloat16, cuda)
    impl = StarKVAttentionImpl(num_heads, 128, 128 ** -0.5, len(RANKS), starkv_layer=w,
                               rotary_emb=types.SimpleNamespace(cos_sin_cache=cs), max_model_len=MAX_MODEL_LEN)
    impl.to_device(cuda, torch.bfloat16)
    dec_lens, prompts = [200, 17, 1], [37, 100, 1]
    lengths = dec_lens + prompts
    bt, nblk = W._page_layout(lengths, g)
    width = impl.row.nbytes // 2 if quant else w.cache_width
    kv_cache = torch.zeros(nblk, 1, W.BLOCK_SIZE, width, dtype=torch.bfloat16, device=cuda)
    nd, npf = len(dec_lens), len(prompts)
    # The decodes' earlier tokens, through the fused write.
    blocks, slots = W._token_slots([L - 1 for L in dec_lens], bt[:nd])
    x = torch.randn(blocks.numel(), HIDDEN, generator=g).to(torch.bfloat16).to(cuda)
    impl.write_from_hidden(x, kv_cache, (blocks * W.BLOCK_SIZE + slots).to(cuda))
    # This step: one token per decode (position L - 1), then every prompt token.
    pos = torch.tensor([L - 1 for L in dec_lens])
    dslots = bt[torch.arange(nd), pos // W.BLOCK_SIZE].long() * W.BLOCK_SIZE + pos % W.BLOCK_SIZE
    pb, ps = W._token_slots(prompts, bt[nd:])
    slot_mapping = torch.cat([dslots, pb * W.BLOCK_SIZE + ps]).to(cuda)
    T = nd + sum(prompts)
    hidden = torch.randn(T, HIDDEN, generator=g).to(torch.bfloat16).to(cuda)
    codes = hidden @ impl.kv_down.T
    key, value = codes[:, :impl.k_width], codes[:, impl.k_width:]
    query = torch.randn(T, num_heads * 128, generator=g).to(torch.bfloat16).to(cuda)
    qsl = [0]
    for L in prompts:
        qsl.append(qsl[-1] + L)
    md = StarKVMetadata(num_actual_tokens=T, num_decodes=nd, num_decode_tokens=nd, num_prefills=npf,
                        max_seq_len=max(lengths), seq_lens=torch.tensor(lengths, dtype=torch.int32, device=cuda),
                        block_table=bt.to(cuda), slot_mapping=slot_mapping, prefill_seq_lens_cpu=list(prompts),
                        prefill_query_start_loc_cpu=qsl)
    output = torch.full((T, num_heads * 128), 7.0, dtype=torch.bfloat16, device=cuda)
    impl.forward(None, query, key, value, kv_cache, md, output)
    torch.cuda.synchronize()
    out = output.view(T, num_heads, 128)
    assert torch.isfinite(out).all()

    cache = kv_cache.squeeze(1)
    q = query.view(T, num_heads, 128).float().cpu().numpy()
    if quant:
        lay = ref.row_layout(impl.k_width, len(RANKS), w.v_rank)
        dtruth = ref.quant_decode(q[:nd], cache.view(torch.uint8).cpu().numpy(), bt[:nd].numpy(),
                                  np.array(dec_lens), max(dec_lens), lay, RANKS, impl.k_up.float().cpu().numpy(),
                                  impl.v_up_by_q.float().cpu().numpy(), cs.float().cpu().numpy(), impl.scale)
    else:
        dtruth = ref.lowrank_decode(q[:nd], cache.float().cpu().numpy(), bt[:nd].numpy(), np.array(dec_lens),
                                    max(dec_lens), impl.k_up.float().cpu().numpy(), RANKS, w.k_head_offsets.tolist(),
                                    impl.k_width, impl.v_up_by_q.float().cpu().numpy(), cs.float().cpu().numpy(),
                                    impl.scale)
    assert_close(out[:nd], dtruth, f"mixed: decodes quant={quant}")
    c = codes.float().cpu().numpy()
    ptruth = ref.dense_prefill(q[nd:], c[nd:, :impl.k_width], c[nd:, impl.k_width:], qsl, w.k_up.float().numpy(),
                               RANKS, w.k_head_offsets.tolist(), w.v_up.float().numpy(), cs.float().cpu().numpy(),
                               impl.scale)
    # The prefill kernel takes K and V lifted in fp32 and rounded once to fp16, q in fp16
    # and P in fp16 with fp32 accumulation: the decode tolerance holds.
    assert_close(out[nd:], ptruth, f"mixed: prompts quant={quant}")
