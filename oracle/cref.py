"""ctypes loader for the C restatement of the oracle (test infrastructure only)."""

import ctypes
import os
import subprocess

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(ORACLE_DIR, "liboracle_c.so")

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        lib = ctypes.CDLL(LIB)
        P = ctypes.c_void_p
        lib.oracle_quantize_group.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int64, P,
                                              ctypes.c_int64, P, P]
        lib.oracle_pack.argtypes = [P, ctypes.c_int64, ctypes.c_int, P]
        lib.oracle_paged_attention_f64.argtypes = [
            P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, ctypes.c_int, ctypes.c_int, P, P,
            ctypes.c_int, P, ctypes.c_int, P, ctypes.c_int, P]
        lib.oracle_fake_quantize.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_int, ctypes.c_int, P]
        lib.oracle_f32_to_bf16.argtypes = [P, ctypes.c_int64, P]
        _lib = lib
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def quantize_group(x):
    """One group over all rows of a 2-D float32 array -> (q, scale, zp)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, c = x.shape
    q = np.zeros((rows, c), np.uint8)
    s = np.zeros(c, np.float32)
    z = np.zeros(c, np.float32)
    load().oracle_quantize_group(_p(x), rows, c, c, _p(q), c, _p(s), _p(z))
    return q, s, z


def pack(q):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    rows = int(np.prod(q.shape[:-1]))
    c = q.shape[-1]
    out = np.zeros(q.shape[:-1] + ((c + 1) // 2,), np.uint8)
    load().oracle_pack(_p(q), rows, c, _p(out))
    return out


def paged_attention_f64(query, k_pages, v_pages, k_scale, k_zp, page_table, seq_lens,
                        page_rows=16, group_rows=128):
    query = np.ascontiguousarray(query, np.float32)
    k_pages = np.ascontiguousarray(k_pages, np.uint8)
    v_pages = np.ascontiguousarray(v_pages, np.float32)
    k_scale = np.ascontiguousarray(k_scale, np.float32)
    k_zp = np.ascontiguousarray(k_zp, np.float32)
    page_table = np.ascontiguousarray(page_table, np.int32)
    seq_lens = np.ascontiguousarray(seq_lens, np.int32)
    B, Hq, D = query.shape
    Hkv, R = k_pages.shape[1], k_pages.shape[2]
    out = np.zeros((B, Hq, D), np.float64)
    load().oracle_paged_attention_f64(
        _p(query), B, Hq, D, _p(k_pages), _p(v_pages), Hkv, R, _p(k_scale), _p(k_zp),
        k_scale.shape[2], _p(page_table), page_table.shape[1], _p(seq_lens),
        group_rows // page_rows, _p(out))
    return out


def fake_quantize(x, block, rounding, recip=0):
    """Quantize-dequantize of one stream x [rows, C] in blocks (rounding 0
    half-up, 1 half-even; recip 1 for the reciprocal scale)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, c = x.shape
    out = np.zeros_like(x)
    load().oracle_fake_quantize(_p(x), rows, c, int(block), int(rounding), int(recip), _p(out))
    return out


def f32_to_bf16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.shape, np.uint16)
    load().oracle_f32_to_bf16(_p(x), x.size, _p(out))
    return out
