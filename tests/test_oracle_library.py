"""Pins the gather / scatter / dot / attention oracle restatements against the
reference's known answers (tests/golden/reference_kats.json, transcribed from
src/backend/mlx_metal/api_test.cc) and against independent forms (brute-force
loops, vectorized special cases, closed forms)."""
import json
import pathlib

import numpy as np
import pytest

from oracle import ops

KATS = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def test_gather_kats():
    k = KATS["gather_axis0"]
    out = ops.gather_stablehlo(np.array(k["operand"], np.float32), np.array(k["indices"])[:, None], [1], [0], [0], 1,
                               [1, 2])
    np.testing.assert_array_equal(out, k["expected"])
    k = KATS["gather_axis1"]
    out = ops.gather_stablehlo(np.array(k["operand"], np.float32), np.array(k["indices"])[:, None], [0], [1], [1], 1,
                               [3, 1])
    np.testing.assert_array_equal(out, k["expected"])
    k = KATS["gather_point"]
    out = ops.gather_stablehlo(np.array(k["operand"], np.float32), np.array(k["indices"]), [], [0, 1], [0, 1], 1,
                               [1, 1])
    np.testing.assert_array_equal(out, k["expected"])


def test_gather_rows_matches_definition_and_clamps():
    rng = np.random.default_rng(0)
    table = rng.standard_normal((17, 5)).astype(np.float32)
    idx = rng.integers(-17, 17, size=(3, 4)).astype(np.int32)
    want = ops.gather_stablehlo(table, np.where(idx < 0, idx + 17, idx)[..., None], [2], [0], [0], 2, [1, 5])
    np.testing.assert_array_equal(ops.gather_rows(table, idx), want)
    # out of range after wrapping: clamped to the last / first row
    np.testing.assert_array_equal(ops.gather_rows(table, np.array([40, -40])), table[[16, 0]])


def test_batched_gather_definition():
    x = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    idx = np.array([[2, 0], [1, 2]], np.int32)[..., None]
    out = ops.gather_stablehlo(x, idx, [2], [1], [1], 2, [1, 1, 4], operand_batching_dims=[0],
                               start_indices_batching_dims=[0])
    want = np.stack([x[0, [2, 0]], x[1, [1, 2]]])
    np.testing.assert_array_equal(out, want)


@pytest.mark.parametrize("mode", ["set", "add"])
def test_scatter_kats(mode):
    combiner = "set" if mode == "set" else "add"
    k = KATS["scatter_1d"]
    out = ops.scatter_stablehlo(np.array(k["operand"], np.float32), np.array(k["indices"])[:, None],
                                np.array(k["updates"], np.float32), [], [0], [0], 1, combiner)
    np.testing.assert_array_equal(out, k[mode])
    k = KATS["scatter_point"]
    out = ops.scatter_stablehlo(np.array(k["operand"], np.float32), np.array(k["indices"]),
                                np.array(k["updates"], np.float32), [], [0, 1], [0, 1], 1, combiner)
    np.testing.assert_array_equal(out, k[mode])
    k = KATS["scatter_window"]
    out = ops.scatter_stablehlo(np.array(k["operand"], np.float32), np.array(k["indices"])[:, None],
                                np.array(k["updates"], np.float32), [1], [0], [0], 1, combiner)
    np.testing.assert_array_equal(out, k[mode])


def test_scatter_batched_kat():
    k = KATS["scatter_batched"]
    x = np.array(k["operand"], np.float32).reshape(2, 3, 4)
    u = np.array(k["updates"], np.float32).reshape(2, 2, 4)
    out = ops.scatter_stablehlo(x, np.array(k["indices"]), u, [2], [1], [1], 2, "set", input_batching_dims=[0],
                                scatter_indices_batching_dims=[0])
    np.testing.assert_array_equal(out.reshape(-1), k["set"])


def test_scatter_row_forms_match_definition():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((9, 3)).astype(np.float32)
    idx = np.array([3, 3, 0, 8, 3, 11, -1, 0], np.int32)  # duplicates and out-of-bounds
    u = rng.standard_normal((8, 3)).astype(np.float32)
    want = ops.scatter_stablehlo(x, idx[:, None], u, [1], [0], [0], 1, "add")
    np.testing.assert_array_equal(ops.scatter_rows_add(x, idx, u), want)  # same f32 op order: bit-exact
    xi = rng.integers(-5, 5, (9, 3)).astype(np.int32)
    ui = rng.integers(-1000, 1000, (8, 3)).astype(np.int32)
    want_i = ops.scatter_stablehlo(xi, idx[:, None], ui, [1], [0], [0], 1, "add")
    np.testing.assert_array_equal(ops.scatter_rows_add_int(xi, idx, ui), want_i)


def test_scatter_sequential_order_is_pinned():
    # Float addition is not associative: (1e8 + 1) - 1e8 == 0 in f32, while
    # 1e8 - 1e8 + 1 == 1. The oracle must apply updates in update order.
    x = np.zeros((1, 1), np.float32)
    u = np.array([[1e8], [1.0], [-1e8]], np.float32)
    out = ops.scatter_rows_add(x, np.zeros(3, np.int32), u)
    assert out[0, 0] == np.float32(0.0)
    out2 = ops.scatter_rows_add(x, np.zeros(3, np.int32), u[[0, 2, 1]])
    assert out2[0, 0] == np.float32(1.0)


def test_dot_kat_and_forms():
    k = KATS["dot_2x2"]
    np.testing.assert_array_equal(ops.dot_general_f64(np.array(k["lhs"]), np.array(k["rhs"]), (), (), (1,), (0,)),
                                  k["expected"])
    rng = np.random.default_rng(2)
    a = rng.standard_normal((2, 3, 4, 5))
    b = rng.standard_normal((2, 3, 6, 5))
    got = ops.dot_general_f64(a, b, (0, 1), (0, 1), (3,), (3,))
    brute = np.zeros((2, 3, 4, 6))
    for i in range(2):
        for j in range(3):
            brute[i, j] = a[i, j] @ b[i, j].T
    np.testing.assert_allclose(got, brute, rtol=1e-12)
    # rank-3 x rank-2 with batch dims only on the left (jax_op_suite attention_scores_rhs_contract_last)
    q = rng.standard_normal((2, 3, 4, 5))
    kc = rng.standard_normal((2, 6, 5))
    got = ops.dot_general_f64(q, kc, (0,), (0,), (3,), (2,))  # [2, 3, 4, 6]
    np.testing.assert_allclose(got, np.einsum("bhqd,bkd->bhqk", q, kc), rtol=1e-12)


def test_attention_oracle_closed_forms():
    # Identical keys -> uniform weights over the causal prefix -> context is
    # the running mean of V rows (exact in this small case up to bf16 rounding).
    L, D = 4, 8
    q = ops.f32_to_bf16_bits(np.ones((1, L, D), np.float32))
    k = ops.f32_to_bf16_bits(np.ones((1, L, D), np.float32))
    vv = np.arange(L * D, dtype=np.float32).reshape(1, L, D) / 8
    v = ops.f32_to_bf16_bits(vv)
    ctx = ops.bf16_bits_to_f32(ops.attention_bf16(q, k, v, causal=True))
    want = np.cumsum(vv, axis=1) / np.arange(1, L + 1)[None, :, None]
    np.testing.assert_allclose(ctx, want, rtol=1e-2)
    # Non-causal with one dominant key -> that key's value row.
    k2 = np.zeros((1, L, D), np.float32)
    k2[0, 2] = 100.0
    ctx2 = ops.bf16_bits_to_f32(ops.attention_bf16(q, ops.f32_to_bf16_bits(k2), v, causal=False))
    np.testing.assert_allclose(ctx2[0], np.broadcast_to(vv[0, 2], (L, D)), rtol=1e-2)


def test_scatter_f64_and_segment_lengths():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((5, 3)).astype(np.float32)
    idx = np.array([0, 4, 4, 9, -2, 4, 1], np.int32)
    u = rng.standard_normal((7, 3)).astype(np.float32)
    np.testing.assert_array_equal(ops.segment_lengths(idx, 5), [1, 1, 0, 0, 3])
    exact = ops.scatter_rows_add_f64(x, idx, u)
    want = x.astype(np.float64)
    for j, r in enumerate(idx):
        if 0 <= r < 5:
            want[r] += u[j]
    np.testing.assert_array_equal(exact, want)
    np.testing.assert_allclose(ops.scatter_rows_add(x, idx, u), exact, rtol=1e-6)


def _bf16_round_py(x: float) -> float:
    """Nearest-even bf16 rounding of an f32 value, by integer arithmetic on its
    bits (independent of the numpy helpers)."""
    import struct
    u = struct.unpack("<I", struct.pack("<f", x))[0]
    lsb = (u >> 16) & 1
    u = ((u + 0x7FFF + lsb) >> 16) << 16
    return struct.unpack("<f", struct.pack("<I", u & 0xFFFFFFFF))[0]


def test_scatter_bf16_sequential_matches_brute_force():
    # Pure-Python loop: f32 add of the two widened values, then bf16 rounding,
    # one update at a time in index order.
    import struct
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 4)).astype(np.float32)
    u = (0.3 * rng.standard_normal((40, 4))).astype(np.float32)
    idx = rng.integers(-1, 4, 40).astype(np.int32)  # -1 and 3 are out of bounds
    xb, ub = ops.f32_to_bf16_bits(x), ops.f32_to_bf16_bits(u)
    got = ops.bf16_bits_to_f32(ops.scatter_rows_add_bf16_bits(xb, idx, ub))
    want = ops.bf16_bits_to_f32(xb).astype(np.float64).tolist()
    uf = ops.bf16_bits_to_f32(ub).tolist()
    f32 = lambda v: struct.unpack("<f", struct.pack("<f", v))[0]
    for j, r in enumerate(idx):
        if 0 <= r < 3:
            want[r] = [_bf16_round_py(f32(a + b)) for a, b in zip(want[r], uf[j])]
    np.testing.assert_array_equal(got, np.array(want, np.float32))
    # Small integers are exact in bf16: the sum is the closed form.
    xi = ops.f32_to_bf16_bits(np.zeros((2, 3), np.float32))
    ui = ops.f32_to_bf16_bits(np.ones((10, 3), np.float32))
    out = ops.bf16_bits_to_f32(ops.scatter_rows_add_bf16_bits(xi, np.array([0] * 7 + [1] * 3), ui))
    np.testing.assert_array_equal(out, [[7, 7, 7], [3, 3, 3]])
    # Order matters once rounding bites: 256 + 1 + 1 rounds each +1 away.
    a = ops.f32_to_bf16_bits(np.array([[256.0]], np.float32))
    ones = ops.f32_to_bf16_bits(np.array([[1.0], [1.0], [256.0]], np.float32))
    o1 = ops.bf16_bits_to_f32(ops.scatter_rows_add_bf16_bits(a, np.array([0, 0, 0]), ones))
    assert o1[0, 0] == 512.0  # 256+1 -> 256, +1 -> 256, +256 -> 512
