"""Pins of the C restatement of C1 and C2 (oracle/c/baseline.c, the
multi-threaded CPU baseline bench.py times): the f16 rounding on every bf16
value against numpy's, and both programs against the numpy oracle, including
the argmax rule's special cases (reference: api.cc:4046-4170, KATs
api_test.cc:930-1055)."""
import json
import pathlib

import numpy as np
import pytest

from oracle import cbaseline, ops

KATS = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def test_bf16_to_f16_rounding_matches_numpy_on_every_bf16_value():
    got = cbaseline.bf16_to_f16_table()
    want = ops.bf16_bits_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16)).astype(np.float16)
    wbits = want.view(np.uint16)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got.view(np.float16)), nan)
    np.testing.assert_array_equal(got[~nan], wbits[~nan])  # includes subnormals, overflow to inf, ties


@pytest.mark.parametrize("threads", [1, 3, 16])
def test_c2_matches_numpy_oracle(threads):
    x = ops.c2_inputs(13, 5000, seed=4)
    # special cases: a NaN row (first NaN wins), ties (lowest index), -inf,
    # f16 overflow (|v| > 65504 rounds to inf) and f16 subnormals
    def b(v):
        return ops.f32_to_bf16_bits(np.array([v], np.float32))[0]
    x[1, [7, 100, 4000]] = b(np.nan)
    x[2, :] = b(0.5)
    x[3, :] = b(-np.inf)
    x[4, 10] = b(1e5)
    x[5, :] = b(3e-6)
    got = cbaseline.c2(x, threads=threads)
    want = ops.c2_reference(x)
    np.testing.assert_array_equal(got[0], want[0])
    np.testing.assert_array_equal(got[1], want[1])
    for g, w in zip(got[2:], want[2:]):
        np.testing.assert_array_equal(np.isnan(g), np.isnan(w))
        ok = ~np.isnan(w)
        np.testing.assert_array_equal(g[ok], w[ok])


def test_c2_kats():
    k = KATS["argmax"]
    mv, idx, *_ = cbaseline.c2(ops.f32_to_bf16_bits(np.array(k["input"], np.float32)))
    np.testing.assert_array_equal(idx, k["indices"])
    np.testing.assert_array_equal(ops.bf16_bits_to_f32(mv), k["values"])
    k = KATS["reduce_f16"]
    _, _, s, mx, mn = cbaseline.c2(ops.f32_to_bf16_bits(np.array(k["input"], np.float32)))
    for got, key in ((s, "sum"), (mx, "max"), (mn, "min")):
        np.testing.assert_array_equal(got.astype(np.float32), k[key])


def test_c1_matches_numpy_oracle():
    x, y = ops.c1_inputs(37, 3000, seed=5)
    np.testing.assert_allclose(cbaseline.c1(x, y, threads=5), ops.c1_rowsum(x, y), rtol=1e-6, atol=1e-6)


def test_tanh_against_numpy():
    # the restatement's own tanh (exp by range reduction + series): closed
    # forms at 0 and at large |t|, odd symmetry, and numpy's tanh over a grid
    assert cbaseline.tanh(0.0) == 0.0 and cbaseline.tanh(50.0) == 1.0 and cbaseline.tanh(-1e300) == -1.0
    t = np.concatenate([np.linspace(-20, 20, 20001), np.geomspace(1e-12, 1, 200), [-3.5, 0.5, 1.5]])
    got = np.array([cbaseline.tanh(v) for v in t])
    np.testing.assert_allclose(got, np.tanh(t), rtol=0, atol=1e-15)
    np.testing.assert_array_equal(np.array([cbaseline.tanh(-v) for v in t]), -got)
