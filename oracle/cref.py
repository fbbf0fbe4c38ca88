"""ctypes binding of the plain-C oracle (``oracle/c/quant_ref.c``), built by ``oracle/Makefile``.

Test infrastructure (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "liblemoq_oracle_c.so")

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE, "-B"], check=True, capture_output=True)
    return LIB


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        lib = ctypes.CDLL(LIB)
        P, I64 = ctypes.c_void_p, ctypes.c_int64
        lib.oracle_rtn_w8.argtypes = [P, I64, I64, I64, P, P, P]
        lib.oracle_rtn_w8.restype = None
        lib.oracle_kv_quant_rows.argtypes = [P, I64, I64, P, P]
        lib.oracle_kv_quant_rows.restype = None
        lib.oracle_rtn.argtypes = [P, I64, I64, I64, ctypes.c_int, ctypes.c_int, P, P, P]
        lib.oracle_rtn.restype = None
        lib.oracle_mxfp4.argtypes = [P, I64, I64, P, P]
        lib.oracle_mxfp4.restype = None
        lib.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        lib.oracle_f32_to_f16.restype = ctypes.c_uint16
        _lib = lib
    return _lib


def rtn_w8(w: np.ndarray, group: int):
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    ng = -(-cols // group)
    codes = np.zeros((rows, ng * group), dtype=np.int8)
    s32 = np.zeros((rows, ng), dtype=np.float32)
    s16 = np.zeros((rows, ng), dtype=np.uint16)
    load().oracle_rtn_w8(w.ctypes.data, rows, cols, group, codes.ctypes.data, s32.ctypes.data, s16.ctypes.data)
    return codes, s32, s16.view(np.float16)


def kv_quant_rows(x16: np.ndarray):
    xf = np.ascontiguousarray(np.asarray(x16, dtype=np.float16).astype(np.float32))
    d = xf.shape[-1]
    rows = xf.size // d if d else 0
    codes = np.zeros(xf.shape, dtype=np.int8)
    s16 = np.zeros(xf.shape[:-1], dtype=np.uint16)
    load().oracle_kv_quant_rows(xf.ctypes.data, rows, d, codes.ctypes.data, s16.ctypes.data)
    return codes, s16.view(np.float16)


def f32_to_f16(values: np.ndarray) -> np.ndarray:
    lib = load()
    v = np.asarray(values, dtype=np.float32).reshape(-1)
    out = np.array([lib.oracle_f32_to_f16(float(t)) for t in v], dtype=np.uint16)
    return out.view(np.float16).reshape(np.shape(values))


def rtn(w: np.ndarray, group: int, bits: int, symmetric: bool):
    """Codes (int32, rows x padded), scale and zero (float32) of ``oracle_rtn``."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    ng = -(-cols // group)
    codes = np.zeros((rows, ng * group), dtype=np.int32)
    s32 = np.zeros((rows, ng), dtype=np.float32)
    z32 = np.zeros((rows, ng), dtype=np.float32)
    load().oracle_rtn(w.ctypes.data, rows, cols, group, bits, 1 if symmetric else 0, codes.ctypes.data,
                      s32.ctypes.data, z32.ctypes.data)
    return codes, s32, z32


def mxfp4(w: np.ndarray):
    """Unpacked E2M1 codes (rows x nblk*32) and E8M0 scale bytes of ``oracle_mxfp4``."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    nblk = -(-cols // 32)
    codes = np.zeros((rows, nblk * 32), dtype=np.uint8)
    scales = np.zeros((rows, nblk), dtype=np.uint8)
    load().oracle_mxfp4(w.ctypes.data, rows, cols, codes.ctypes.data, scales.ctypes.data)
    return codes, scales
