"""Integer/byte restatement (numpy) and the ctypes loader of the C restatement — TEST INFRASTRUCTURE ONLY.

Bit-level definitions used by the parity tests:
  bf16_rne       fp32 -> bf16 bits, round to nearest even (what torch's ``.to(torch.bfloat16)`` does)
  dequant_bits   RNE_bf16(q*s + z) with fp32 arithmetic, low nibble = even column (smel/quant.py:42, 51-67)
  dispatch       stable counting sort of flat expert ids -> (counts, offsets, order, inv) (smel/moe.py:216-223,
                 249-250)
  topk           descending value, lower index first among equal values (deterministic torch.topk, smel/moe.py:165)
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "c", "liboracle.so")


def build_c(force: bool = False) -> str:
    """Compile oracle/c/oracle.c with gcc (no GPU involved)."""
    import subprocess
    if force or not os.path.exists(LIB_PATH) or \
            os.path.getmtime(LIB_PATH) < os.path.getmtime(os.path.join(HERE, "c", "oracle.c")):
        subprocess.run(["make", "-s", "-C", HERE] + (["-B"] if force else []) + ["c/liboracle.so"], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build_c()
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
        L.oracle_bf16_rne.argtypes = [vp, vp, i64]
        L.oracle_dequant_int4.argtypes = [vp, vp, vp, vp, i64, i64, i64, i32]
        L.oracle_dispatch.argtypes = [vp, i64, i64, vp, vp, vp, vp]
        L.oracle_dispatch.restype = i32
        L.oracle_topk.argtypes = [vp, i64, i64, i64, vp, vp]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


# ------------------------------------------------------------------------------------------------ numpy restatement


def bf16_rne(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit pattern (uint16), round half to even; NaN stays NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def unpack_nibbles(q: np.ndarray) -> np.ndarray:
    q = np.asarray(q, dtype=np.uint8)
    return np.stack((q & 0xF, q >> 4), axis=-1).reshape(*q.shape[:-1], q.shape[-1] * 2)


def dequant_bits(q: np.ndarray, scale_bits: np.ndarray, zero_bits: np.ndarray) -> np.ndarray:
    """[..., K/2] bytes + [..., G] bf16 bits -> [..., K] bf16 bits."""
    nib = unpack_nibbles(q).astype(np.float32)
    K = nib.shape[-1]
    G = scale_bits.shape[-1]
    s = np.repeat(bf16_bits_to_f32(scale_bits), K // G, axis=-1)
    z = np.repeat(bf16_bits_to_f32(zero_bits), K // G, axis=-1)
    return bf16_rne((nib * s).astype(np.float32) + z)


def dispatch(topi: np.ndarray, E: int):
    """topi [T, K] -> (counts [E], offsets [E+1], order [TK], inv [TK]) int32 via numpy's stable argsort."""
    flat = np.asarray(topi, dtype=np.int64).reshape(-1)
    order = np.argsort(flat, kind="stable").astype(np.int32)
    counts = np.bincount(flat, minlength=E).astype(np.int32)
    offsets = np.zeros(E + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size, dtype=np.int32)
    return counts, offsets, order, inv


def topk(p: np.ndarray, k: int):
    """[rows, n] -> (values, indices int32): lexicographic (-value, index)."""
    order = np.argsort(-np.asarray(p, dtype=np.float32), axis=-1, kind="stable")[..., :k].astype(np.int32)
    return np.take_along_axis(p, order, axis=-1), order


# ----------------------------------------------------------------------------------------------- C restatement


def c_dequant_bits(q, scale_bits, zero_bits, out_f32=False):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    s = np.ascontiguousarray(scale_bits, dtype=np.uint16)
    z = np.ascontiguousarray(zero_bits, dtype=np.uint16)
    K = q.shape[-1] * 2
    rows = q.size // q.shape[-1]
    group = K // s.shape[-1]
    out = np.empty((*q.shape[:-1], K), dtype=np.float32 if out_f32 else np.uint16)
    lib().oracle_dequant_int4(_p(q), _p(s), _p(z), _p(out), rows, K, group, int(out_f32))
    return out


def c_dispatch(topi: np.ndarray, E: int):
    flat = np.ascontiguousarray(topi, dtype=np.int32).reshape(-1)
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    order = np.empty(flat.size, np.int32)
    inv = np.empty(flat.size, np.int32)
    rc = lib().oracle_dispatch(_p(flat), flat.size, E, _p(counts), _p(offsets), _p(order), _p(inv))
    if rc != 0:
        raise ValueError("expert id out of range")
    return counts, offsets, order, inv


def c_topk(p: np.ndarray, k: int):
    p = np.ascontiguousarray(p, dtype=np.float32)
    rows, n = p.shape
    v = np.empty((rows, k), np.float32)
    idx = np.empty((rows, k), np.int32)
    lib().oracle_topk(_p(p), rows, n, k, _p(v), _p(idx))
    return v, idx


def c_bf16_rne(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().oracle_bf16_rne(_p(x), _p(y), x.size)
    return y
