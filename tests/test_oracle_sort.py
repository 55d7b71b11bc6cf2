"""The sort / top_k oracle (oracle/sort.py) pinned against the reference's
KAT (api_test.cc:2310-2360), the op-suite cases of jax_op_suite.py:435-438
(closed forms on their tie-free ascending input), and a pure-Python stable
brute force on small inputs with ties, NaNs and signed zeros."""
import json
import pathlib

import numpy as np
import pytest

from oracle import ops as O
from oracle import sort as S

KATS = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def test_reference_sort_kat():
    k = KATS["sort_kv"]
    x = np.array(k["input"], np.float32)
    vals = np.array(k["values"], np.int32)
    out_x, out_v = S.sort_stablehlo([x, vals], 1)
    np.testing.assert_array_equal(out_x, np.array(k["sorted"], np.float32))
    np.testing.assert_array_equal(S.sort_order(x, 1), np.array(k["order"]))
    np.testing.assert_array_equal(out_v, np.array(k["values_sorted"]))


def test_op_suite_cases():
    # jax_op_suite.py:122 input, ascending along axis 1 with no ties.
    f32_a = (np.arange(12, dtype=np.float32).reshape(3, 4) - np.float32(3.0)) / np.float32(7.0)
    np.testing.assert_array_equal(S.sort_stablehlo([f32_a], 1)[0], f32_a)                        # sort
    np.testing.assert_array_equal(S.sort_stablehlo([f32_a], 1, descending=True)[0], f32_a[:, ::-1])  # descending
    np.testing.assert_array_equal(S.sort_order(f32_a, 1), np.tile(np.arange(4), (3, 1)))          # argsort
    v, i = S.top_k(f32_a, 2)                                                                     # top_k(x, 2)
    np.testing.assert_array_equal(v, f32_a[:, [3, 2]])
    np.testing.assert_array_equal(i, np.tile(np.array([3, 2], np.int32), (3, 1)))


def _planted(rng, n, dtype):
    if dtype in ("f32", "f16", "bf16"):
        pool = np.array([0.0, -0.0, 1.5, -1.5, np.inf, -np.inf, np.nan, -np.nan, 2.0, 2.0, -3.25], np.float32)
        x = np.where(rng.random(n) < 0.5, rng.choice(pool, n), rng.integers(-4, 5, n).astype(np.float32))
        if dtype == "f16":
            return x.astype(np.float16), False
        if dtype == "bf16":
            return O.f32_to_bf16_bits(x.astype(np.float32)), True
        return x.astype(np.float32), False
    info = np.iinfo(dtype)
    pool = np.array([info.min, info.max, 0, 1], dtype=dtype)
    x = np.where(rng.random(n) < 0.3, rng.choice(pool, n), rng.integers(-3 if info.min < 0 else 0, 4, n).astype(dtype))
    return x.astype(dtype), False


def _values(x, bf16):
    if bf16:
        return [float(v) for v in O.bf16_bits_to_f32(x)]
    return [v.item() for v in x]


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16", np.int32, np.uint8, np.int8, np.int16, np.uint32])
@pytest.mark.parametrize("compare_type", ["TOTALORDER", "FLOAT"])
@pytest.mark.parametrize("descending", [False, True])
def test_matches_python_stable_sort(dtype, compare_type, descending):
    rng = np.random.default_rng(7)
    if not isinstance(dtype, str) and compare_type == "FLOAT":
        pytest.skip("integer keys have no FLOAT compare")
    for n in (1, 2, 5, 17, 64):
        x, bf16 = _planted(rng, n, dtype)
        want = S.sort_row_bruteforce(_values(x, bf16), compare_type, descending)
        got = S.sort_order(x, 0, compare_type, descending, bf16)
        np.testing.assert_array_equal(got, want, err_msg=f"{dtype} {compare_type} desc={descending} n={n} {x}")


def test_top_k_matches_bruteforce_and_properties():
    rng = np.random.default_rng(3)
    for dtype in ("f32", "bf16"):
        for n, k in ((8, 3), (33, 33), (40, 1)):
            x, bf16 = _planted(rng, n, dtype)
            v, i = S.top_k(x, k, bf16)
            want = S.sort_row_bruteforce(_values(x, bf16), "TOTALORDER", True)[:k]
            np.testing.assert_array_equal(i, want)
            np.testing.assert_array_equal(v.view(np.uint8), x[want].view(np.uint8))


def test_images_reduce_to_textbook_orders():
    # Finite, NaN-free floats: the image order is numpy's value order with
    # position as the tie break; signed ints: numpy's order.
    rng = np.random.default_rng(1)
    x = rng.standard_normal(1000).astype(np.float32)
    np.testing.assert_array_equal(S.sort_order(x, 0), np.argsort(x, kind="stable"))
    y = rng.integers(-50, 50, 1000).astype(np.int32)
    np.testing.assert_array_equal(S.sort_order(y, 0), np.argsort(y, kind="stable"))
    np.testing.assert_array_equal(S.sort_order(y, 0, descending=True), np.argsort(-y.astype(np.int64), kind="stable"))
