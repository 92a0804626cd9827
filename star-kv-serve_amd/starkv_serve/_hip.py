"""Bindings of libstarkv_hip.so, the C ABI declared in include/starkv_hip.h.

Two routes, one library instance:
- ``ops()``: ``torch.ops.starkv``, the operator library libstarkv_torch.so
  (csrc/torch_ops.cpp). The kernel wrappers launch through it: tensors go in as
  tensors, the workspace comes from torch's caching allocator and the launch goes on
  the current HIP stream.
- ``lib()``: ctypes over the C ABI itself, for the host-only queries (grids,
  workspace sizes, layer checks, the decode-form switch, timing) and for tests that
  drive the C ABI directly. Tensors cross it as data pointers, strides and dtype codes.

There is no fallback: if either library is missing or fails to load, every entry
point raises.
"""
import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libstarkv_hip.so")
OPS_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libstarkv_torch.so")
ABI_VERSION = 6

F32, F16, BF16 = 0, 1, 2
CACHE_Q3_2 = 16  # cache kind of the 3.2-bit QuantRow cache
_DTYPES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES = {
    "starkv_abi_version": (_I, []),
    "starkv_last_error": (ctypes.c_char_p, []),
    "starkv_write_codes": (_I, [_P, _P, _I64, _P, _I64, _I, _P, _I64, _I64, _I, _I, _I64, _P, _I, _I, _I, _I]),
    "starkv_pack_kv": (_I, [_P, _P, _I64, _P, _I64, _I, _P, _I64, _I64, _I, _I64, _P, _I, _I, _I, _P, _P, _P,
                            _I, _I, _I]),
    "starkv_fold_q": (_I, [_P, _P, _I64, _I64, _I, _P, _I64, _I, _P, _I, _I, _F, _P]),
    "starkv_write_kv_workspace_bytes": (_SZ, [_I, _I, _I]),
    "starkv_write_kv": (_I, [_P, _P, _I64, _P, _I64, _I, _I, _I, _I, _I, _P, _I64, _I64, _I, _I, _I64, _P, _I,
                             _I, _P, _P, _P, _I, _P, _I64, _P, _SZ]),
    "starkv_write_kv_deferred": (_I, [_P, _P, _I64, _P, _I64, _I, _I, _I, _I, _I, _P, _I64, _I64, _I, _I, _I64, _P,
                                      _I, _I, _P, _P, _P, _I, _P, _I64, _P, _SZ]),
    "starkv_flush_write": (_I, []),
    "starkv_decode_grid": (_I, [_I, _I]),
    "starkv_decode_grid_for": (_I, [_I, _I, _I, _I, _I, _I, _I]),
    "starkv_stock_decode_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "starkv_stock_decode": (_I, [_P, _P, _I64, _I64, _I, _P, _P, _I64, _I64, _I64, _I, _I, _P, _I64, _I64, _P,
                                 _I, _I, _I, _I, _F, _P, _I64, _I64, _I, _P, _SZ]),
    "starkv_stock_write": (_I, [_P, _P, _I64, _I64, _P, _I64, _I64, _I, _P, _P, _I64, _I64, _I64, _I, _I64, _P, _I,
                                _I, _I]),
    "starkv_prefill_block_list": (_I, [ctypes.POINTER(ctypes.c_int32), _I, ctypes.POINTER(ctypes.c_int32), _I]),
    "starkv_prefill_attention": (_I, [_P, _P, _I64, _I64, _I, _P, _P, _I64, _I64, _I, _P, _P, _I, _I, _I, _I, _F,
                                      _P, _I64, _I64, _I]),
    "starkv_profile_begin": (_I, [_I, _I]),
    "starkv_profile_end": (_I, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I)]),
    "starkv_profile_times": (_I, [ctypes.POINTER(ctypes.c_double), _I]),
    "starkv_decode_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I, _I, _I, _I]),
    "starkv_decode_two_pass": (_I, [_I, _I, _I, _I, _I]),
    "starkv_decode_set_path": (_I, [_I]),
    "starkv_decode_layer_fits": (_I, [_I, _I, _I, ctypes.POINTER(ctypes.c_int32), _I]),
    "starkv_lowrank_decode": (_I, [_P, _P, _I64, _I64, _I, _P, _I64, _I64, _I, _I, _P, _I64, _I64, _P, _I,
                                   _I, _I, _I, _P, _I64, _I, _P, _P, _I, _I, _P, _I64, _I64, _I, _I, _P, _I64,
                                   _I, _F, _P, _I64, _I64, _I, _P, _SZ, _I]),
    "starkv_lowrank_decode_noalloc": (_I, [_P, _P, _I64, _I64, _I, _P, _I64, _I64, _I, _I, _P, _I64, _I64, _P,
                                           _I, _I, _I, _I, _P, _I64, _I, _P, _P, _I, _I, _P, _I64, _I64, _I, _I,
                                           _P, _I64, _I, _F, _P, _I64, _I64, _I, _I]),
    "starkv_quant_decode": (_I, [_P, _P, _I64, _I64, _I, _P, _I64, _I64, _I, _P, _I64, _I64, _P, _I, _I, _I,
                                 _I, _I, _I, _P, _I64, _I, _P, _P, _P, _P, _I64, _I64, _I, _P, _I64, _I, _F,
                                 _P, _I64, _I64, _I, _P, _SZ, _I]),
    "starkv_quant_decode_group": (_I, [_P, _P, _I64, _I64, _I, _P, _I64, _I64, _I, _P, _I64, _I64, _P, _I, _I,
                                       _I, _I, _I, _I, _P, _I64, _I, _P, _P, _P, _P, _I64, _I64, _I, _P, _I64, _I,
                                       _F, _P, _I64, _I64, _I, _P, _SZ, _I, _I, _I, _I, _I]),
    "starkv_quant_group_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I, _I, _I, _I, _I, _I]),
    "starkv_quant_group_two_pass": (_I, [_I, _I, _I, _I, _I, _I, _I]),
    "starkv_decode_layer_groups": (_I, [_I, _I, _I, ctypes.POINTER(ctypes.c_int32), _I,
                                        ctypes.POINTER(ctypes.c_int32), _I]),
}

_LIB = None


def lib():
    """The loaded library; raises RuntimeError if it is missing or stale."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"STAR-KV HIP library not built: {LIB_PATH} is missing "
                               "(run `python star-kv-serve_amd/build.py`)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        if L.starkv_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI {L.starkv_abi_version()} != {ABI_VERSION}; rebuild it")
        _LIB = L
    return _LIB


_OPS = None


def ops():
    """``torch.ops.starkv``; raises RuntimeError if the operator library is missing. The C
    library is loaded first, so both routes share its state (decode-form switch, timing):
    the operator library binds to the already-loaded libstarkv_hip.so by its soname."""
    global _OPS
    if _OPS is None:
        lib()
        if not os.path.exists(OPS_PATH):
            raise RuntimeError(f"STAR-KV operator library not built: {OPS_PATH} is missing "
                               "(run `python star-kv-serve_amd/build.py`)")
        torch.ops.load_library(OPS_PATH)
        _OPS = torch.ops.starkv
    return _OPS


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().starkv_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {msg} (code {rc})")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def stream_of(t: torch.Tensor) -> int:
    """Handle of the current stream on t's device (the launch stream)."""
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def layer_fits(cache_kind: int, num_heads: int, num_kv_heads: int, k_ranks, v_rank: int) -> bool:
    """Whether the decode takes a layer of this shape (host-side; k_ranks a list of ints)."""
    arr = (ctypes.c_int32 * len(k_ranks))(*[int(r) for r in k_ranks])
    return bool(lib().starkv_decode_layer_fits(int(cache_kind), int(num_heads), int(num_kv_heads), arr, int(v_rank)))


def layer_groups(cache_kind: int, num_heads: int, num_kv_heads: int, k_ranks, v_rank: int) -> list:
    """KV-head ranges ``[(g0, g1), ...]``, one decode call each (``starkv_decode_layer_groups``;
    host-side, k_ranks a list of ints); an empty list when some single KV head does not fit
    one call."""
    ranks = [int(r) for r in k_ranks]
    arr = (ctypes.c_int32 * max(len(ranks), 1))(*ranks)
    cap = max(len(ranks), 1)
    out = (ctypes.c_int32 * (2 * cap))()
    k = lib().starkv_decode_layer_groups(int(cache_kind), int(num_heads), int(num_kv_heads), arr, int(v_rank), out,
                                         cap)
    if k < 0:
        check(1, "decode_layer_groups")
    return [(out[2 * i], out[2 * i + 1]) for i in range(k)]


decode_path_epoch = 0  # bumped by set_decode_path: host caches of the decode form key on it


def set_decode_path(mode: int) -> int:
    """0 = automatic (default), 1 = one-pass only, 2 = two-pass always; returns the previous mode."""
    global decode_path_epoch
    prev = lib().starkv_decode_set_path(int(mode))
    if prev < 0:
        check(1, "decode_set_path")
    decode_path_epoch += 1
    return prev


def profile_begin(max_calls: int, whole_call: bool = False) -> None:
    """Arm event timing for the next `max_calls` decode calls: of their decode kernels, or
    of the whole call (prep to merge) with whole_call."""
    check(lib().starkv_profile_begin(int(max_calls), 1 if whole_call else 0), "profile_begin")


def profile_end() -> list:
    """Per-call milliseconds of the timed calls; disarms the timing."""
    ms = ctypes.c_double(0.0)
    calls = ctypes.c_int(0)
    check(lib().starkv_profile_end(ctypes.byref(ms), ctypes.byref(calls)), "profile_end")
    buf = (ctypes.c_double * max(calls.value, 1))()
    k = lib().starkv_profile_times(buf, calls.value)
    return [buf[i] for i in range(k)]


def output_for(out, shape, dtype, device) -> torch.Tensor:
    """The decode's output: a new tensor of `shape` and `dtype`, or the caller's `out`
    (any of bf16 / fp16 / fp32, last dimension contiguous), which the kernels write in
    place."""
    if out is None:
        return torch.empty(shape, dtype=dtype, device=device)
    if tuple(out.shape) != tuple(shape):
        raise ValueError(f"out has shape {tuple(out.shape)}, expected {tuple(shape)}")
    if out.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"out dtype {out.dtype} (bf16, fp16 or fp32)")
    if out.device != torch.device(device) or out.stride(-1) != 1:
        raise ValueError("out must be on the query's device with a contiguous last dimension")
    return out


def require_cuda(*ts: torch.Tensor) -> None:
    dev = ts[0].device
    for t in ts:
        if t.device.type != "cuda":
            raise RuntimeError("STAR-KV kernels run on the GPU only; got a tensor on "
                               f"{t.device}")
        if t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
