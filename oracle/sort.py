"""Numpy restatement of stablehlo.sort and chlo.top_k — TEST INFRASTRUCTURE ONLY.

Only tests/ use this module, as the checker; the plugin never calls it.

Semantics restated (reference: src/backend/mlx_metal/lowering_indexing.zig:
290-356 for what is accepted; execution_node_indexing_order.zig:12-72 and
api.cc:3248-3347 for the MLX sort / argsort / take_along_axis chain):
  * every operand is permuted by the stable order of operand 0 along the
    sort dimension (the reference's key/value form, api_test.cc:2310-2360);
  * LT/LE comparators sort ascending, GT/GE descending; equal keys keep their
    positions' order in both directions (StableHLO is_stable). The reference
    reverses an ascending sort for GT, which lists equal keys last-first;
    JAX's CPU backend, the reference's declared oracle, keeps them in order,
    and so does this module;
  * TOTALORDER compares use IEEE totalOrder (-NaN < -inf < -0 < +0 < +inf <
    +NaN); FLOAT compares treat -0 and +0 as equal and put every NaN after
    +inf, as numpy.sort does;
  * top_k: the k largest along the last dim under totalOrder, largest first,
    equal values by position, with s32 positions (XLA's TopK).

Parity pins (tests/test_oracle_sort.py): the reference's KAT api_test.cc:
2310-2360 (sort, argsort, take_along_axis); the op-suite cases of
jax_op_suite.py:435-438 on their input (closed forms); a pure-Python
brute force (Python's stable sorted with keys built from float values, not
bit patterns) on small random inputs with planted ties, NaNs and signed
zeros, for every key class and both directions.
"""
from __future__ import annotations

import numpy as np

_UINT = {1: np.uint8, 2: np.uint16, 4: np.uint32}
_INF_BITS = {np.dtype(np.float32): 0x7F800000, np.dtype(np.float16): 0x7C00}


def key_image(x: np.ndarray, compare_type: str = "TOTALORDER", descending: bool = False,
              bf16: bool = False) -> np.ndarray:
    """Order-preserving unsigned image (uint64) of each key. `bf16` marks a
    uint16 array holding bfloat16 bits."""
    x = np.asarray(x)
    if bf16:
        bits, width, inf, is_float = x.astype(np.uint64), 16, 0x7F80, True
    elif x.dtype.kind == "f":
        width = x.dtype.itemsize * 8
        bits = x.view(_UINT[x.dtype.itemsize]).astype(np.uint64)
        inf, is_float = _INF_BITS[x.dtype], True
    else:
        width, is_float = x.dtype.itemsize * 8, False
        bits = x.view(_UINT[x.dtype.itemsize]).astype(np.uint64) if x.dtype.kind in "iu" else x.astype(np.uint64)
    mask = np.uint64((1 << width) - 1)
    sign = np.uint64(1 << (width - 1))
    if not is_float:
        img = bits ^ sign if (x.dtype.kind == "i" and compare_type != "UNSIGNED") else bits
    else:
        mag = bits & ~sign & mask
        nan = mag > np.uint64(inf)
        if compare_type != "TOTALORDER":
            bits = np.where(mag == 0, np.uint64(0), bits)
        img = np.where((bits & sign) != 0, ~bits & mask, bits | sign)
        if compare_type != "TOTALORDER":
            img = np.where(nan, mask, img)
    img = img.astype(np.uint64)
    return (~img & mask) if descending else img


def sort_order(keys: np.ndarray, dimension: int = -1, compare_type: str = "TOTALORDER", descending: bool = False,
               bf16: bool = False) -> np.ndarray:
    """Positions of the stable order along `dimension`."""
    return np.argsort(key_image(keys, compare_type, descending, bf16), axis=dimension, kind="stable")


def sort_stablehlo(operands: list[np.ndarray], dimension: int = -1, compare_type: str = "TOTALORDER",
                   descending: bool = False, bf16: bool = False) -> list[np.ndarray]:
    """stablehlo.sort: every operand permuted by operand 0's stable order."""
    order = sort_order(operands[0], dimension, compare_type, descending, bf16)
    return [np.take_along_axis(np.asarray(o), order, axis=dimension) for o in operands]


def top_k(x: np.ndarray, k: int, bf16: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """chlo.top_k: (values, s32 positions) of the k largest along the last dim."""
    order = sort_order(x, -1, "TOTALORDER", True, bf16)[..., :k]
    return np.take_along_axis(np.asarray(x), order, axis=-1), order.astype(np.int32)


# ------------------------------------------------- independent brute force

def _py_key(v: float, compare_type: str):
    """Sort key built from the value (math.isnan / copysign), not its bits."""
    import math
    if isinstance(v, (int, np.integer)):
        return (int(v),)
    v = float(v)
    if math.isnan(v):
        neg = math.copysign(1.0, v) < 0
        if compare_type == "TOTALORDER":
            return (0,) if neg else (4,)
        return (4,)
    if compare_type == "TOTALORDER":
        return (2, v, math.copysign(1.0, v))
    return (2, v, 0.0)


def sort_row_bruteforce(values: list, compare_type: str = "TOTALORDER", descending: bool = False) -> list[int]:
    """Positions of one row in stable order, by Python's sorted (TimSort is
    stable, and stays stable with reverse=True)."""
    return sorted(range(len(values)), key=lambda i: _py_key(values[i], compare_type), reverse=descending)
