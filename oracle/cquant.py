"""ORACLE (test infrastructure only): ctypes binding of ``quant_oracle.c``.

The shared object is built by ``__graft_entry__.build()`` (or on first use here,
with gcc) into ``oracle/_build/liboracle.so``.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SRC = os.path.join(_HERE, "quant_oracle.c")
_SO = os.path.join(_HERE, "_build", "liboracle.so")
_LIB = None


def build(force: bool = False) -> str:
    """Compile the C restatement (gcc, IEEE float: no -ffast-math)."""
    if force or not os.path.exists(_SO) or os.path.getmtime(_SO) < os.path.getmtime(_SRC):
        os.makedirs(os.path.dirname(_SO), exist_ok=True)
        tmp = _SO + ".tmp%d" % os.getpid()
        subprocess.check_call(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-fno-fast-math",
                               "-ffp-contract=off", _SRC, "-o", tmp, "-lm"])
        os.replace(tmp, _SO)
    return _SO


def lib():
    global _LIB
    if _LIB is None:
        L = ctypes.CDLL(build())
        P, I, I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        L.oracle_n_outlier.argtypes = [I]
        L.oracle_n_outlier.restype = I
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_quantize_block.argtypes = [P, I, I, P, P]
        L.oracle_pack_k_row.argtypes = [P, I, P, P, P, I, P]
        L.oracle_pack_v_row.argtypes = [P, I, I, I, I, P]
        L.oracle_pack_kv.argtypes = [P, I64, P, I64, I, P, I64, I64, I, I64, P, I, P, P, P, I, I, I, I]
        L.oracle_pack_kv.restype = I
        L.oracle_unpack_k_row.argtypes = [P, I, P, P, P, I, P]
        L.oracle_unpack_v_row.argtypes = [P, I, I, I, I, P]
        _LIB = L
    return _LIB


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def n_outlier(rank: int) -> int:
    return lib().oracle_n_outlier(int(rank))


def f32_to_bf16_bits(x: float) -> int:
    return int(lib().oracle_f32_to_bf16(ctypes.c_float(x)))


def quantize_block(x: np.ndarray, bits: int):
    """kv_quant._q on one block -> (codes int32 [n] in 0..15, fp32 scale)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    codes = np.empty(x.shape[0], dtype=np.int32)
    s = np.empty(1, dtype=np.float32)
    lib().oracle_quantize_block(_p(x), x.shape[0], bits, _p(codes), _p(s))
    return codes, float(s[0])


def pack_kv(k: np.ndarray, v: np.ndarray, cache: np.ndarray, slots: np.ndarray, ranks, offsets,
            nouts, v_rank: int, ks_off: int, vs_off: int, vq_off: int) -> None:
    """In place: quantize k [n, W] / v [n, R] (float32 values) into cache [nb, bs, row] uint8."""
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    assert cache.dtype == np.uint8 and cache.ndim == 3 and cache.strides[2] == 1
    slots = np.ascontiguousarray(slots, dtype=np.int64)
    r = np.ascontiguousarray(ranks, dtype=np.int32)
    o = np.ascontiguousarray(offsets, dtype=np.int32)
    no = np.ascontiguousarray(nouts, dtype=np.int32)
    rc = lib().oracle_pack_kv(_p(k), k.shape[1], _p(v), v.shape[1], k.shape[0], _p(cache),
                              cache.strides[0], cache.strides[1], cache.shape[1], cache.shape[0], _p(slots),
                              r.shape[0], _p(r), _p(o), _p(no), int(v_rank), ks_off, vs_off, vq_off)
    if rc != 0:
        raise IndexError("oracle pack_kv: slot outside the cache")


def unpack_k_row(row: np.ndarray, ranks, offsets, nouts, ks_off: int, k_width: int) -> np.ndarray:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    r = np.ascontiguousarray(ranks, dtype=np.int32)
    o = np.ascontiguousarray(offsets, dtype=np.int32)
    no = np.ascontiguousarray(nouts, dtype=np.int32)
    out = np.zeros(k_width, dtype=np.float32)
    lib().oracle_unpack_k_row(_p(row), r.shape[0], _p(r), _p(o), _p(no), ks_off, _p(out))
    return out


def unpack_v_row(row: np.ndarray, R: int, nout: int, vs_off: int, vq_off: int) -> np.ndarray:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    out = np.zeros(R, dtype=np.float32)
    lib().oracle_unpack_v_row(_p(row), R, nout, vs_off, vq_off, _p(out))
    return out
