"""stablehlo.sort and chlo.top_k on the GPU against the oracle
(oracle/sort.py), bit-exact: keys, payloads and positions. Shapes cover the
three paths of kernels/sort.hip: rows that fit one LDS block, rows sorted by
a global bitonic network, and top_k reduced block by block (one and two
reduction rounds), plus sorts along a non-last dimension, several operands,
both comparator directions (and a swapped LT), FLOAT and TOTALORDER
compares with planted ties, NaNs and signed zeros."""
import json
import pathlib

import numpy as np
import pytest

from oracle import ops as O
from oracle import sort as S
from pjrtx_amd.hlo import Builder

pytestmark = pytest.mark.gpu

KATS = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_kats.json").read_text())
HDT = {"f32": np.float32, "f16": np.float16, "s32": np.int32, "u8": np.uint8, "s16": np.int16, "u32": np.uint32}


def _keys(rng, shape, dtype, planted=True):
    n = int(np.prod(shape))
    if dtype in ("f32", "f16", "bf16"):
        x = rng.standard_normal(n).astype(np.float32)
        if planted:
            pool = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, -np.nan], np.float32)
            m = rng.random(n) < 0.15
            x[m] = rng.choice(pool, int(m.sum()))
            t = rng.random(n) < 0.15
            x[t] = np.round(x[t])  # ties
        x = x.reshape(shape)
        if dtype == "bf16":
            return O.f32_to_bf16_bits(x)
        return x.astype(HDT[dtype])
    info = np.iinfo(HDT[dtype])
    lo, hi = max(info.min, -1000), min(info.max, 1000)
    x = rng.integers(lo, hi + 1, n).astype(HDT[dtype])
    if planted:
        m = rng.random(n) < 0.05
        x[m] = rng.choice(np.array([info.min, info.max], dtype=HDT[dtype]), int(m.sum()))
    return x.reshape(shape)


def _sort_program(shape, dtypes, dim, direction="LT", compare_type=None, swap=False):
    b = Builder("jit_sort")
    ops = [b.param(shape, dt) for dt in dtypes]
    outs = b.sort(ops, dim, direction, compare_type, swap)
    return b.build(outs)


def _run_sort(client, arrays, dtypes, dim, direction="LT", compare_type=None, swap=False):
    exe = client.compile(_sort_program(arrays[0].shape, dtypes, dim, direction, compare_type, swap))
    outs = exe(*arrays, dtypes=dtypes)
    return outs if isinstance(outs, (list, tuple)) else [outs]


def _check_sort(client, arrays, dtypes, dim, direction="LT", compare_type=None, swap=False):
    ct = compare_type or ("TOTALORDER" if dtypes[0] in ("f32", "f16", "bf16") else "SIGNED")
    desc = (direction in ("GT", "GE")) != swap
    want = S.sort_stablehlo(arrays, dim, ct, desc, bf16=dtypes[0] == "bf16")
    got = _run_sort(client, arrays, dtypes, dim, direction, compare_type, swap)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(np.asarray(g).view(np.uint8), np.ascontiguousarray(w).view(np.uint8))


def test_reference_kat(client):
    k = KATS["sort_kv"]
    x = np.array(k["input"], np.float32)
    v = np.array(k["values"], np.int32)
    i = np.broadcast_to(np.arange(3, dtype=np.int32), (2, 3)).copy()
    sx, sv, si = _run_sort(client, [x, v, i], ["f32", "s32", "s32"], 1)
    np.testing.assert_array_equal(sx, np.array(k["sorted"], np.float32))
    np.testing.assert_array_equal(sv, np.array(k["values_sorted"]))
    np.testing.assert_array_equal(si, np.array(k["order"]))


def test_op_suite_cases(client):
    f32_a = (np.arange(12, dtype=np.float32).reshape(3, 4) - np.float32(3.0)) / np.float32(7.0)
    (s,) = _run_sort(client, [f32_a], ["f32"], 1)
    np.testing.assert_array_equal(s, f32_a)
    (d,) = _run_sort(client, [f32_a], ["f32"], 1, "GT")
    np.testing.assert_array_equal(d, f32_a[:, ::-1])
    b = Builder("jit_topk")
    x = b.param((3, 4), "f32")
    v, i = b.top_k(x, 2)
    vals, idx = client.compile(b.build([v, i]))(f32_a)
    np.testing.assert_array_equal(vals, f32_a[:, [3, 2]])
    np.testing.assert_array_equal(idx, np.tile(np.array([3, 2], np.int32), (3, 1)))


@pytest.mark.parametrize("shape,dim", [((5, 1), 1), ((7, 3), 1), ((3, 1000), 1), ((2, 4096), 1), ((300, 37), 1),
                                       ((6, 50, 3), 1), ((64, 9), 0), ((2, 5000), 1), ((3, 20000), 1),
                                       ((40000,), 0)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_sort_with_positions(client, shape, dim, dtype):
    rng = np.random.default_rng(sum(shape) + dim)
    x = _keys(rng, shape, dtype)
    pos = np.broadcast_to(np.arange(shape[dim], dtype=np.int32).reshape([-1 if d == dim else 1 for d in range(len(shape))]),
                          shape).copy()
    _check_sort(client, [x, pos], [dtype, "s32"], dim)


@pytest.mark.parametrize("direction,swap,compare_type", [("GT", False, None), ("LT", True, None), ("GE", False, None),
                                                         ("LT", False, "FLOAT"), ("GT", False, "FLOAT")])
@pytest.mark.parametrize("n", [100, 6000])
def test_sort_directions_and_compare_types(client, direction, swap, compare_type, n):
    rng = np.random.default_rng(n)
    x = _keys(rng, (4, n), "f32")
    payload = _keys(rng, (4, n), "f16", planted=False)
    _check_sort(client, [x, payload], ["f32", "f16"], 1, direction, compare_type, swap)


@pytest.mark.parametrize("dtype", ["s32", "u8", "s16", "u32", "f16"])
def test_sort_key_types(client, dtype):
    rng = np.random.default_rng(5)
    x = _keys(rng, (9, 777), dtype)
    _check_sort(client, [x], [dtype], 1)
    _check_sort(client, [x], [dtype], 1, "GT")


@pytest.mark.parametrize("shape,k,dtype", [((3, 4), 4, "f32"), ((5, 100), 7, "f32"), ((64, 128256), 50, "bf16"),
                                           ((3, 300000), 100, "f32"), ((2, 10000), 3000, "f32"),
                                           ((4, 6000), 6000, "bf16"), ((8, 5000), 1, "bf16"),
                                           ((2, 3, 9000), 16, "f32")])
def test_top_k(client, shape, k, dtype):
    rng = np.random.default_rng(k + shape[-1])
    x = _keys(rng, shape, dtype)
    b = Builder("jit_topk")
    p = b.param(shape, dtype)
    v, i = b.top_k(p, k)
    vals, idx = client.compile(b.build([v, i]))(x, dtypes=[dtype])
    wv, wi = S.top_k(x, k, bf16=dtype == "bf16")
    np.testing.assert_array_equal(idx, wi)
    np.testing.assert_array_equal(np.asarray(vals).view(np.uint8), np.ascontiguousarray(wv).view(np.uint8))


def test_top_k_zero(client):
    b = Builder("jit_topk0")
    p = b.param((3, 10), "f32")
    v, i = b.top_k(p, 0)
    vals, idx = client.compile(b.build([v, i]))(np.ones((3, 10), np.float32))
    assert vals.shape == (3, 0) and idx.shape == (3, 0)
