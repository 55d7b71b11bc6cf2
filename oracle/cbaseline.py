"""ctypes binding of oracle/c/baseline.c: the C1 and C2 programs restated in C
over host threads (the numpy oracle's algorithm, oracle/ops.py c1_rowsum and
c2_reference), so bench.py's cpu_baseline leg can time them on every host core.

Test infrastructure, like the rest of oracle/: only tests/, smoke() and
bench.py's cpu_baseline leg load it; the plugin never does. Pinned by
tests/test_oracle_c.py (the f16 rounding over all 65,536 bf16 values against
numpy, and both programs against the numpy oracle).
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
SRC = HERE / "c" / "baseline.c"
SRC_C1 = HERE / "c" / "c1_row.c"
LIB = HERE / "liboracle_c.so"

_lib = None


def build() -> pathlib.Path:
    """Compiles the library in-tree with gcc (x86-64-v3: AVX2 and FMA, which
    every EPYC host of the GPU boxes has)."""
    tmp = LIB.with_suffix(".so.tmp")
    flags = ["-O3", "-march=x86-64-v3", "-fopenmp-simd", "-fPIC", "-Wall", "-Wextra"]
    c1o = LIB.with_suffix(".c1_row.o")
    subprocess.run(["gcc", *flags, "-c", "-o", str(c1o), str(SRC_C1)], check=True)
    subprocess.run(["gcc", *flags, "-shared", "-o", str(tmp), str(SRC), str(c1o), "-lm", "-lpthread"], check=True)
    c1o.unlink()
    os.replace(tmp, LIB)
    return LIB


def lib():
    """The loaded library; built first when it is missing or older than its
    source."""
    global _lib
    if _lib is None:
        if not LIB.exists() or LIB.stat().st_mtime < max(SRC.stat().st_mtime, SRC_C1.stat().st_mtime):
            build()
        L = ctypes.CDLL(str(LIB))
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.pjrtx_oracle_c2.argtypes = [p, i64, i64, p, p, p, p, p, ctypes.c_int]
        L.pjrtx_oracle_c2.restype = ctypes.c_int
        L.pjrtx_oracle_c1.argtypes = [p, p, i64, i64, p, ctypes.c_int]
        L.pjrtx_oracle_c1.restype = ctypes.c_int
        L.pjrtx_oracle_bf16_to_f16_table.argtypes = [p]
        L.pjrtx_oracle_bf16_to_f16_table.restype = None
        L.pjrtx_oracle_tanh.argtypes = [ctypes.c_double]
        L.pjrtx_oracle_tanh.restype = ctypes.c_double
        _lib = L
    return _lib


def host_threads() -> int:
    return len(os.sched_getaffinity(0))


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def c2(logits_bf16_bits: np.ndarray, threads: int | None = None):
    """Outputs of the C2 program (as oracle.ops.c2_reference): argmax values
    (bf16 bits), indices (int32), f16 sum / max / min (f16 bits)."""
    x = np.ascontiguousarray(logits_bf16_bits, dtype=np.uint16)
    rows, cols = x.shape
    mv = np.empty(rows, np.uint16)
    mi = np.empty(rows, np.int32)
    s, mx, mn = (np.empty(rows, np.uint16) for _ in range(3))
    lib().pjrtx_oracle_c2(_ptr(x), rows, cols, _ptr(mv), _ptr(mi), _ptr(s), _ptr(mx), _ptr(mn),
                          threads or host_threads())
    return mv, mi, s.view(np.float16), mx.view(np.float16), mn.view(np.float16)


def c1(x: np.ndarray, y: np.ndarray, threads: int | None = None) -> np.ndarray:
    """sum(tanh(x*y + 0.5)*x - max(y, 0), axis=1) in double, rounded to f32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.ascontiguousarray(y, dtype=np.float32)
    out = np.empty(x.shape[0], np.float32)
    lib().pjrtx_oracle_c1(_ptr(x), _ptr(y), x.shape[0], x.shape[1], _ptr(out), threads or host_threads())
    return out


def tanh(t: float) -> float:
    """The restatement's tanh (exp by range reduction and a Taylor series)."""
    return lib().pjrtx_oracle_tanh(float(t))


def bf16_to_f16_table() -> np.ndarray:
    """f16 bits of every bf16 bit pattern, by the library's rounding."""
    out = np.empty(65536, np.uint16)
    lib().pjrtx_oracle_bf16_to_f16_table(_ptr(out))
    return out
