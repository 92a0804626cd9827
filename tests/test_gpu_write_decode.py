"""A deferred cache write (``write_kv(..., deferred=True)``, C ABI starkv_write_kv_deferred)
launched inside the next decode call: its code GEMM rides in the decode's first launch
(prep), its store follows, then the decode kernels.

Pins, per layer kind (bf16 codes and 3.2-bit; one-pass and two-pass V ranks; a layer
decoded as two KV-head groups; five requests, and one or two, whose write takes the
direct form, its 3.2-bit V latent packed by the logits pass of a two-pass decode):
- deferred write + decode gives the same output and the same cache bytes, bit for bit,
  as the write launched on its own followed by the same decode;
- a deferred write launched by flush_write() leaves the cache of the immediate write;
- a second write launches a pending one first (both rows land, in order);
- the decode over the deferred write matches the float64 oracle (through the layer's
  decode tolerance), so the kernels read the new rows.
"""
import types

import numpy as np
import pytest
import torch

from oracle import ref
from starkv_serve import checkpoint as ck
from starkv_serve import workloads as W
from starkv_serve.attention import StarKVAttentionImpl, StarKVMetadata
from starkv_serve.kernels.kv_write import flush_write
from test_gpu_decode import assert_close

pytestmark = pytest.mark.gpu

HIDDEN, MAX_MODEL_LEN = 4096, 2048
LENGTHS = [300, 77, 16, 1, 520]  # after this step
R8 = [16, 32, 48, 64, 24, 16, 40, 56]

CASES = {
    # name: (ranks, v_rank, num_heads, quant, lengths)
    "bf16_one_pass": (R8, 48, 16, False, LENGTHS),
    "bf16_two_pass": (R8, 320, 16, False, LENGTHS),
    "quant_one_pass": (R8, 48, 8, True, LENGTHS),
    "quant_two_pass": (R8, 400, 8, True, LENGTHS),
    "bf16_kv_groups": ([64] * 32, 64, 32, False, LENGTHS),
    "bf16_one_pass_1req": (R8, 48, 16, False, [520]),
    "bf16_two_pass_2req": (R8, 320, 16, False, [300, 77]),
    "quant_one_pass_2req": (R8, 48, 8, True, [16, 300]),
    "quant_two_pass_1req": (R8, 400, 8, True, [1030]),
    "quant_two_pass_2req": (R8, 1290, 8, True, [77, 520]),
    "quant_two_pass_1req_f16": (R8, 1290, 8, True, [700]),
}
DTYPES = {"quant_two_pass_1req_f16": torch.float16}  # the model dtype, bf16 unless listed


def _layer(cuda, tmp_path, name):
    ranks, v_rank, num_heads, quant, _ = CASES[name]
    dt = DTYPES.get(name, torch.bfloat16)
    path = str(tmp_path / "fused_weights.pt")
    ck.write_fused_checkpoint(path, 1, len(ranks), 128, HIDDEN, {0: (ranks, v_rank)}, seed=31)
    w = ck.load_fused_checkpoint(path, 1, len(ranks), 128, dtype=dt, kv_quant=quant).layers[0]
    cs = W.cos_sin_table(MAX_MODEL_LEN, dt, cuda)
    impl = StarKVAttentionImpl(num_heads, 128, 128 ** -0.5, len(ranks), starkv_layer=w,
                               rotary_emb=types.SimpleNamespace(cos_sin_cache=cs), max_model_len=MAX_MODEL_LEN,
                               fused_write=True)
    impl.to_device(cuda, dt)
    return w, impl, cs


def _step(cuda, impl, w, quant, g, lengths=LENGTHS, dt=torch.bfloat16):
    """A cache with the prompts written, this step's slots, hidden rows and query."""
    bt, nblk = W._page_layout(lengths, g)
    n = len(lengths)
    width = impl.row.nbytes // 2 if quant else w.cache_width
    kv_cache = torch.zeros(nblk, 1, W.BLOCK_SIZE, width, dtype=torch.bfloat16, device=cuda)
    blocks, slots = W._token_slots([L - 1 for L in lengths], bt)
    x = torch.randn(blocks.numel(), HIDDEN, generator=g).to(dt).to(cuda)
    impl.write_from_hidden(x, kv_cache, (blocks * W.BLOCK_SIZE + slots).to(cuda))
    pos = torch.tensor([L - 1 for L in lengths])
    step_slots = (bt[torch.arange(n), pos // W.BLOCK_SIZE].long() * W.BLOCK_SIZE + pos % W.BLOCK_SIZE).to(cuda)
    hidden = torch.randn(n, HIDDEN, generator=g).to(dt).to(cuda)
    query = torch.randn(n, impl.num_heads * 128, generator=g).to(dt).to(cuda)
    md = StarKVMetadata(num_actual_tokens=n, num_decodes=n, num_decode_tokens=n, num_prefills=0,
                        max_seq_len=max(lengths), seq_lens=torch.tensor(lengths, dtype=torch.int32, device=cuda),
                        block_table=bt.to(cuda), slot_mapping=step_slots)
    return kv_cache, bt, step_slots, hidden, query, md


def _decode(impl, query, cache, md):
    n = query.shape[0]
    out = torch.full((n, impl.num_heads, 128), float("nan"), dtype=query.dtype, device=query.device)
    impl._decode(query.view(n, impl.num_heads, 128), impl._cache(cache), md, out, False)
    return out


@pytest.mark.parametrize("name", list(CASES))
def test_deferred_write_then_decode_is_bit_identical(cuda, tmp_path, name):
    ranks, v_rank, num_heads, quant, lengths = CASES[name]
    print(f"\n[deferred write] case={name}", flush=True)
    w, impl, cs = _layer(cuda, tmp_path, name)
    g = torch.Generator().manual_seed(32)
    cache0, bt, slots, hidden, query, md = _step(cuda, impl, w, quant, g, lengths, DTYPES.get(name, torch.bfloat16))

    # The write on its own, then the decode.
    ca = cache0.clone()
    impl.write_from_hidden(hidden, ca, slots)
    out_a = _decode(impl, query, ca, md)
    # The write deferred into the decode.
    cb = cache0.clone()
    impl.write_from_hidden(hidden, cb, slots, deferred=True)
    out_b = _decode(impl, query, cb, md)
    torch.cuda.synchronize()
    assert torch.equal(ca.view(torch.int16), cb.view(torch.int16)), "cache bytes differ"
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16)), "outputs differ"
    assert torch.isfinite(out_b.float()).all()

    # The decode read the new rows: the float64 oracle over the written cache.
    n = len(lengths)
    cache = cb.squeeze(1)
    q = query.view(n, num_heads, 128).float().cpu().numpy()
    if quant:
        lay = ref.row_layout(impl.k_width, len(ranks), v_rank)
        truth = ref.quant_decode(q, cache.view(torch.uint8).cpu().numpy(), bt.numpy(), np.array(lengths),
                                 max(lengths), lay, ranks, impl.k_up.float().cpu().numpy(),
                                 impl.v_up_by_q.float().cpu().numpy(), cs.float().cpu().numpy(), impl.scale)
    else:
        c32 = (cache.cpu().view(torch.int16).numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        truth = ref.lowrank_decode(q, c32, bt.numpy(), np.array(lengths), max(lengths),
                                   impl.k_up.float().cpu().numpy(), ranks, impl.k_head_offsets.tolist(),
                                   impl.k_width, impl.v_up_by_q.float().cpu().numpy(), cs.float().cpu().numpy(),
                                   impl.scale)
    assert_close(out_b, truth, name)


@pytest.mark.parametrize("name", ["quant_two_pass_2req", "bf16_two_pass_2req"])
def test_deferred_direct_write_skips_slots_past_the_cache(cuda, tmp_path, name):
    """A deferred direct write (two tokens) whose second slot lies past the cache: the decode
    that carries it (the 3.2-bit V latent packed by its logits pass) leaves the cache as the
    immediate write does, and gives the same output."""
    quant, lengths = CASES[name][3], CASES[name][4]
    print(f"\n[deferred direct write past-cache] case={name}", flush=True)
    w, impl, _ = _layer(cuda, tmp_path, name)
    g = torch.Generator().manual_seed(34)
    cache0, _, slots, hidden, query, md = _step(cuda, impl, w, quant, g, lengths)
    slots = slots.clone()
    slots[1] = cache0.shape[0] * W.BLOCK_SIZE + 5  # past the cache: skipped
    ca = cache0.clone()
    impl.write_from_hidden(hidden, ca, slots)
    out_a = _decode(impl, query, ca, md)
    cb = cache0.clone()
    impl.write_from_hidden(hidden, cb, slots, deferred=True)
    out_b = _decode(impl, query, cb, md)
    torch.cuda.synchronize()
    assert torch.equal(ca.view(torch.int16), cb.view(torch.int16)), "cache bytes differ"
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16)), "outputs differ"


@pytest.mark.parametrize("name", ["bf16_one_pass", "quant_one_pass", "bf16_two_pass_2req", "quant_two_pass_1req"])
def test_deferred_write_flushed_and_replaced(cuda, tmp_path, name):
    quant, lengths = CASES[name][3], CASES[name][4]
    print(f"\n[deferred write flush] case={name}", flush=True)
    w, impl, _ = _layer(cuda, tmp_path, name)
    g = torch.Generator().manual_seed(33)
    cache0, _, slots, hidden, query, md = _step(cuda, impl, w, quant, g, lengths)
    hidden2 = torch.randn(hidden.shape, generator=g).to(torch.bfloat16).to(cuda)
    slots2 = slots.flip(0)  # the same slots in the other order: the second write must land last

    ca = cache0.clone()
    impl.write_from_hidden(hidden, ca, slots)
    cb = cache0.clone()
    impl.write_from_hidden(hidden, cb, slots, deferred=True)
    flush_write()
    torch.cuda.synchronize()
    assert torch.equal(ca.view(torch.int16), cb.view(torch.int16)), "flushed write differs"

    # A pending write is launched by the next write, before it.
    impl.write_from_hidden(hidden2, ca, slots2)
    out_a = _decode(impl, query, ca, md)
    cc = cache0.clone()
    impl.write_from_hidden(hidden, cc, slots, deferred=True)
    impl.write_from_hidden(hidden2, cc, slots2, deferred=True)
    out_c = _decode(impl, query, cc, md)
    cd = cache0.clone()
    impl.write_from_hidden(hidden, cd, slots)
    impl.write_from_hidden(hidden2, cd, slots2)
    out_d = _decode(impl, query, cd, md)
    torch.cuda.synchronize()
    assert torch.equal(cc.view(torch.int16), cd.view(torch.int16)), "two writes differ"
    assert torch.equal(out_c.view(torch.int16), out_d.view(torch.int16))
    assert torch.equal(ca.view(torch.int16), cd.view(torch.int16))
    assert torch.equal(out_a.view(torch.int16), out_d.view(torch.int16))
