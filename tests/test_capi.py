"""The C-ABI library loads and exports every entry point include/starkv_hip.h declares;
argument validation fails loudly without touching the GPU."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "starkv_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(starkv_\w+)\s*\(", text)))


def test_header_declares_the_api():
    names = declared()
    for n in ("starkv_lowrank_decode", "starkv_quant_decode", "starkv_pack_kv", "starkv_write_codes",
              "starkv_fold_q", "starkv_decode_grid", "starkv_decode_workspace_bytes", "starkv_last_error",
              "starkv_abi_version", "starkv_write_kv", "starkv_write_kv_workspace_bytes",
              "starkv_decode_two_pass", "starkv_decode_set_path"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from starkv_serve import _hip
    assert os.path.exists(_hip.LIB_PATH), "build the library first (__graft_entry__.build())"
    raw = ctypes.CDLL(_hip.LIB_PATH)
    for n in declared():
        assert hasattr(raw, n), n
    assert set(declared()) == set(_hip.SIGNATURES)
    assert _hip.lib().starkv_abi_version() == _hip.ABI_VERSION


def test_bad_arguments_return_errors():
    from starkv_serve import _hip
    L = _hip.lib()
    rc = L.starkv_pack_kv(None, None, 0, None, 0, 2, None, 0, 0, 16, 1, None, 64, 1, 32, None, None, None, 1280, 64, 999)
    assert rc != 0 and b"row_bytes" in L.starkv_last_error()
    rc = L.starkv_write_codes(None, None, 0, None, 0, 2, None, 0, 0, 2, 16, 1, None, 48, 1, 16, 16)
    assert rc != 0 and b"int32 or int64" in L.starkv_last_error()
    with pytest.raises(RuntimeError, match="row_bytes"):
        _hip.check(L.starkv_pack_kv(None, None, 0, None, 0, 2, None, 0, 0, 16, 1, None, 64, 1, 32, None, None,
                                    None, 1280, 64, 999), "pack_kv")


def test_workspace_size_is_a_host_function():
    from starkv_serve import _hip
    L = _hip.lib()
    BF16, F16, Q = _hip.BF16, _hip.F16, _hip.CACHE_Q3_2
    a = L.starkv_decode_workspace_bytes(BF16, 64, 32, 32, 1280, 64, 8192, 256)
    b = L.starkv_decode_workspace_bytes(BF16, 64, 32, 32, 1280, 64, 8192, 128)
    assert a > b > 64 * 80 * 4096
    # the one-pass form needs no logits buffer: the context length only sizes the page
    # records, 16 bytes for every page a request of max_seq_len tokens can have
    c = L.starkv_decode_workspace_bytes(BF16, 64, 32, 32, 1280, 64, 100, 256)
    assert a - c == 64 * (8192 // 16 - (100 + 15) // 16) * 16
    assert L.starkv_decode_workspace_bytes(BF16, 0, 32, 32, 1280, 64, 100, 256) == 0


def test_two_pass_selection():
    """Which V ranks take the two-pass form (a host function of the layer shape)."""
    from starkv_serve import _hip
    L = _hip.lib()
    BF16, F16, Q = _hip.BF16, _hip.F16, _hip.CACHE_Q3_2
    assert L.starkv_decode_two_pass(BF16, 32, 32, 1280, 64) == 0
    # V rank 256 in one pass needs all of a wave's tiles in registers next to four V blocks:
    # spill-free up to 8 tiles per wave (K width 1024), two passes at 10 (K width 1280)
    assert L.starkv_decode_two_pass(BF16, 32, 32, 1024, 256) == 0
    assert L.starkv_decode_two_pass(BF16, 32, 32, 1280, 256) == 1
    assert L.starkv_decode_two_pass(BF16, 32, 32, 1120, 64) == 0      # 9 tiles per wave, one V block
    assert L.starkv_decode_two_pass(Q, 32, 32, 1232, 64) == 0         # 10 tiles: 9 in registers, 1 streamed
    assert L.starkv_decode_two_pass(BF16, 32, 32, 880, 272) == 1
    assert L.starkv_decode_two_pass(F16, 32, 32, 880, 1280) == 1
    assert L.starkv_decode_two_pass(Q, 32, 32, 1280, 64) == 0
    # V rank 256: 51 outliers (padded to 52) + 205 inliers, 5 blocks: one pass with 4 tiles
    # per wave (K width 512), two passes with 7 (K width 880: 8 tiles and 5 V blocks spill)
    assert L.starkv_decode_two_pass(Q, 32, 32, 512, 256) == 0
    assert L.starkv_decode_two_pass(Q, 32, 32, 880, 256) == 1
    assert L.starkv_decode_two_pass(Q, 32, 32, 880, 1290) == 1
    # two-pass workspaces add the fp32 logits [n, H, max_seq_len rounded up to 16] (and a
    # page record per request for the 17th page)
    one = L.starkv_decode_workspace_bytes(BF16, 64, 32, 32, 880, 1280, 8192, 256)
    two = L.starkv_decode_workspace_bytes(BF16, 64, 32, 32, 880, 1280, 8200, 256)
    assert two - one == 64 * 32 * 16 * 4 + 64 * 16
    assert one >= 64 * 32 * 8192 * 4 + 320 * 32 * 1280 * 4
    # forcing a form
    assert _hip.set_decode_path(2) == 0
    try:
        assert L.starkv_decode_two_pass(BF16, 32, 32, 1280, 64) == 1
        assert L.starkv_decode_set_path(1) == 2
        assert L.starkv_decode_two_pass(BF16, 32, 32, 880, 1280) == 0
        assert L.starkv_decode_set_path(7) == -1 and b"mode 7" in L.starkv_last_error()
    finally:
        _hip.set_decode_path(0)


def test_write_kv_validation():
    """Fused write, immediate and deferred: argument checks return errors before any
    launch (no GPU here)."""
    from starkv_serve import _hip
    L = _hip.lib()
    F32, F16, BF16 = 0, 1, 2

    def call(fn=L.starkv_write_kv, **kw):
        a = dict(stream=None, hidden=None, h_s0=4096, kv_down=None, w_s0=4096, w_dtype=BF16, n=0, hidden_size=4096,
                 k_width=1280, v_rank=64, cache=None, c_s0=0, c_s1=1344, cache_dtype=BF16, block_size=16,
                 num_blocks=1, slots=None, slot_bits=32, heads=32, ranks=None, offsets=None, nouts=None,
                 row_bytes=0, codes=None, co_s0=0, ws=None, ws_bytes=0)
        a.update(kw)
        return fn(*a.values())

    assert call() == 0  # n = 0: nothing to do
    assert call(w_dtype=F32) != 0 and b"bf16 or fp16" in L.starkv_last_error()
    assert call(hidden_size=4000, h_s0=4000, w_s0=4000) != 0 and b"multiple of 64" in L.starkv_last_error()
    assert call(k_width=1288) != 0 and b"multiple of 16" in L.starkv_last_error()
    assert call(slot_bits=16) != 0 and b"int32 or int64" in L.starkv_last_error()
    assert call(cache_dtype=F16) != 0 and b"model dtype" in L.starkv_last_error()
    assert call(row_bytes=800) != 0 and b"QuantRow.nbytes 816" in L.starkv_last_error()
    assert call(row_bytes=816, c_s1=800) != 0 and b"slot stride" in L.starkv_last_error()
    assert call(n=1) != 0 and b"null pointer" in L.starkv_last_error()
    # The deferred form runs the same checks and records nothing when it fails or has no
    # tokens: flushing then launches nothing (no GPU here).
    assert call(L.starkv_write_kv_deferred) == 0
    assert L.starkv_flush_write() == 0
    assert call(L.starkv_write_kv_deferred, k_width=1288) != 0 and b"multiple of 16" in L.starkv_last_error()
    assert call(L.starkv_write_kv_deferred, n=1) != 0 and b"null pointer" in L.starkv_last_error()
    assert L.starkv_flush_write() == 0
    # workspace: split-K partials, a pure function of (n, width, hidden)
    assert L.starkv_write_kv_workspace_bytes(64, 1344, 4096) == 16 * 64 * 1344 * 4
    assert L.starkv_write_kv_workspace_bytes(1024, 1344, 4096) == 1 * 1024 * 1344 * 4
    assert L.starkv_write_kv_workspace_bytes(0, 1344, 4096) == 0


def test_layer_fits_host_plan():
    """The host restatement of the wave plan accepts what the decode runs and refuses
    what it cannot (more than 32 heads, more than 96 tiles, a head of more than 16
    tiles, V rank above 4096, 3.2-bit GQA)."""
    from starkv_serve import _hip
    BF16, Q = _hip.BF16, _hip.CACHE_Q3_2
    fits = _hip.layer_fits
    assert fits(BF16, 32, 32, [16, 32, 48, 64] * 8, 64)
    assert fits(Q, 32, 32, [16, 32, 48, 64] * 8, 64)
    assert fits(BF16, 32, 32, [32] * 23 + [16] * 9, 1280)           # the 0.75-ratio shape, two-pass
    assert fits(Q, 32, 32, [32] * 23 + [16] * 9, 1290)
    assert fits(BF16, 32, 8, [32] * 8, 2048)                        # GQA 4: 64 tiles
    assert fits(BF16, 4, 4, [256, 16, 100, 20], 64)                 # one head of 16 tiles
    assert not fits(BF16, 4, 4, [272, 16, 16, 16], 64)              # a head of 17 tiles
    assert not fits(BF16, 64, 64, [16] * 64, 64)                    # 64 query heads
    assert not fits(BF16, 32, 8, [64] * 8, 64)                      # GQA 4 x 4 tiles x 8 = 128 tiles
    assert not fits(BF16, 32, 32, [16] * 32, 4097)                  # V rank
    assert not fits(Q, 32, 16, [16] * 16, 64)                       # 3.2-bit is MHA only
    # eight heads of 12 tiles (96 in all) take one wave each; a ninth head passes the
    # 96-tile cap
    assert fits(BF16, 8, 8, [192] * 8, 64)
    assert not fits(BF16, 9, 9, [192] * 8 + [16], 64)


OPS = {
    "lowrank_decode": "(Tensor query, Tensor kv_cache, Tensor block_table, Tensor seq_lens, SymInt max_seq_len",
    "quant_decode": "(Tensor query, Tensor kv_cache, Tensor block_table, Tensor seq_lens, SymInt max_seq_len",
    "pack_kv": "(Tensor k_codes, Tensor v_codes, Tensor(a!) cache, Tensor slot_mapping",
    "write_codes": "(Tensor key, Tensor value, Tensor(a!) kv_cache, Tensor slot_mapping)",
    "write_kv": "(Tensor hidden, Tensor kv_down, SymInt k_width, Tensor(a!) kv_cache",
    "fold_q": "(Tensor q, Tensor k_up, Tensor head_of_lane, float scale, Tensor(a!) ab)",
    "stock_decode": "(Tensor query, Tensor k_cache, Tensor v_cache, Tensor block_table",
    "stock_write": "(Tensor key, Tensor value, Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor slot_mapping)",
}


def test_operator_library_registers_every_op():
    """torch.ops.starkv (libstarkv_torch.so over the C ABI): every launch entry point is an
    operator with a schema that marks the tensors it writes."""
    import torch
    from starkv_serve import _hip
    ops = _hip.ops()
    for name, head in OPS.items():
        schema = str(getattr(ops, name).default._schema)
        assert schema.startswith(f"starkv::{name}"), schema
        assert head.replace("SymInt", "int") in schema.replace("SymInt", "int"), schema
    assert "Tensor(a!) out" in str(ops.lowrank_decode.default._schema)
    del torch


def test_operators_refuse_cpu_tensors():
    """The operators are registered for the GPU only: CPU tensors find no kernel and raise
    (no CPU fallback)."""
    import torch
    from starkv_serve import _hip
    t = torch.zeros(4, dtype=torch.bfloat16)
    s = torch.zeros(1, dtype=torch.int64)
    with pytest.raises(NotImplementedError, match="CPU"):
        _hip.ops().write_codes(t.view(1, 4), t.view(1, 4), t.view(1, 1, 4), s)


def _block_list_restated(lens, qb=128):
    """starkv_prefill_block_list restated: every (prompt, qb-row block), the blocks with
    the most keys (min(L, qb (b + 1))) first, ties in prompt then block order."""
    blocks = [(min(L, qb * (b + 1)), i, b) for i, L in enumerate(lens) for b in range((L + qb - 1) // qb)]
    blocks.sort(key=lambda t: (-t[0], t[1], t[2]))
    return [v for _, i, b in blocks for v in (i, b)]


def test_prefill_block_list_host():
    """starkv_prefill_block_list (C, host) against its restatement: one (prompt, 128-row
    query block) pair per query block, empty prompts skipped, the longest causal rows
    first; a bad prefix is refused; the prefill entry point checks its arguments before
    launching."""
    from starkv_serve import _hip
    from starkv_serve.kernels.prefill import block_list
    L = _hip.lib()
    lens = [1, 0, 128, 129, 300, 0, 5, 257]
    cu = (ctypes.c_int32 * (len(lens) + 1))(*np.concatenate([[0], np.cumsum(lens)]).astype(int).tolist())
    n = L.starkv_prefill_block_list(cu, len(lens), None, 0)
    buf = (ctypes.c_int32 * (2 * n))()
    assert L.starkv_prefill_block_list(cu, len(lens), buf, n) == n == 1 + 1 + 2 + 3 + 1 + 3
    assert list(buf) == _block_list_restated(lens) == block_list(lens)
    assert list(buf)[:2] == [4, 2]  # the 300-token prompt's third block: 300 keys
    bad = (ctypes.c_int32 * 3)(0, 5, 2)
    assert L.starkv_prefill_block_list(bad, 2, None, 0) == -1
    rc = L.starkv_prefill_attention(None, None, 0, 0, 2, None, None, 0, 0, 1, None, None, 1, 32, 32, 64, 0.1, None,
                                    0, 0, 2)
    assert rc != 0 and b"null pointer" in L.starkv_last_error()


def test_build_rejects_kernels_that_spill():
    """The build reads hipcc's kernel resource report and refuses scratch spills: the parse
    finds the kernels with a nonzero ScratchSize and only those."""
    import build
    report = "\n".join([
        "x.hip:1:1: remark: Function Name: _Z1av [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:1:1: remark:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:1:1: remark:     ScratchSize [bytes/lane]: 16 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark: Function Name: _Z1bv [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert build._spills(report) == [("_Z1av", 16)]
    assert build._spills("") == []
