"""Argmax / argmin edge cases on the GPU against the oracle's comparator
(oracle/ops.py argmax_rows_bruteforce: NaN first, then the larger value,
ties to the lower index, the winner's own value bits).

The shapes cover both ways the generated reduce kernel folds an argmax:
splits short enough for one unrolled pass per thread (the index is found
after the workgroup's maximum is known) and longer splits walked in several
passes (a per-sub-chunk maximum, then a scan). Signed zeros compare equal,
so the first zero wins and keeps its sign; the first NaN wins whatever its
sign or payload. Bit-exact throughout."""
import numpy as np
import pytest

from oracle import ops
from pjrtx_amd.hlo import Builder

pytestmark = pytest.mark.gpu

BF16_NEG_ZERO = 0x8000
BF16_NEG_NAN = 0xFFC1   # negative quiet NaN with a payload bit


def expected(bits, kind, reverse_index=False):
    vals = ops.bf16_bits_to_f32(bits)
    rows, n = vals.shape
    want_i = np.empty(rows, np.int64)
    want_bits = np.empty(rows, np.uint16)
    for r in range(rows):
        row = vals[r, ::-1] if reverse_index else vals[r]
        rowb = bits[r, ::-1] if reverse_index else bits[r]
        # Vectorised comparator: NaN first, else the extreme value; ties (==,
        # so -0 == +0) to the lowest index value.
        nan = np.isnan(row)
        if nan.any():
            i = int(np.argmax(nan))
        else:
            m = row.max() if kind == "max" else row.min()
            i = int(np.argmax(row == m))
        want_i[r] = i
        want_bits[r] = rowb[i]
    return want_i, want_bits


def program(rows, n, kind, reverse_index=False):
    b = Builder("jit_arg")
    x = b.param((rows, n), "bf16")
    idx = None
    if reverse_index:
        it = b.iota((rows, n), 1, "s32")
        idx = b.subtract(b.scalar_like(n - 1, it), it)
    v, i = b.argmax(x, 1, "s32", kind=kind, idx=idx)
    return b.build([v, i])


def check(client, bits, kind, reverse_index=False):
    rows, n = bits.shape
    exe = client.compile(program(rows, n, kind, reverse_index))
    vals, idx = exe(bits, dtypes=["bf16"])
    want_i, want_bits = expected(bits, kind, reverse_index)
    np.testing.assert_array_equal(idx, want_i)
    got = np.asarray(vals, np.uint16)
    nan = np.isnan(ops.bf16_bits_to_f32(want_bits))
    np.testing.assert_array_equal(np.isnan(ops.bf16_bits_to_f32(got)), nan)
    np.testing.assert_array_equal(got[~nan], want_bits[~nan])


def edge_rows(n, kind, seed):
    """Eight rows of bf16 bits: random, ties, signed zeros both ways round,
    NaNs of both signs, all -inf/+inf, the winner in the last column."""
    rng = np.random.default_rng(seed)
    sign = -1.0 if kind == "max" else 1.0        # values on the losing side of zero
    v = sign * np.abs(rng.standard_normal((8, n))).astype(np.float32) - sign * 0.0
    bits = ops.f32_to_bf16_bits(v)
    bits[1] = ops.f32_to_bf16_bits(rng.integers(-3, 4, n).astype(np.float32))   # heavy ties
    a, c = n // 3, (2 * n) // 3
    bits[2, a], bits[2, c] = BF16_NEG_ZERO, 0x0000      # -0 first: it wins, sign kept
    bits[3, a], bits[3, c] = 0x0000, BF16_NEG_ZERO      # +0 first
    bits[4, c], bits[4, n - 1] = BF16_NEG_NAN, 0x7FC0   # first NaN (negative) wins
    bits[4, a] = ops.f32_to_bf16_bits(np.float32(-sign * 1e30))
    bits[5, :] = ops.f32_to_bf16_bits(np.float32(sign * np.inf))
    bits[6, n - 1] = ops.f32_to_bf16_bits(np.float32(-sign * 50.0))
    bits[7, 0] = ops.f32_to_bf16_bits(np.float32(-sign * 50.0))
    bits[7, n - 1] = bits[7, 0]
    return bits


@pytest.mark.parametrize("kind", ["max", "min"])
@pytest.mark.parametrize("n", [
    64,          # one split, partial sub-chunks
    8016,        # one pass per thread, ragged last sub-chunk
    50000,       # several splits, one pass each
    50001,       # odd length: scalar loads, element-wise fold
    1 << 20,     # 16384-element splits: still one (8-deep) pass
    (3 << 20) + 8,   # long splits walked in several passes, short last split
])
def test_edge_rows(client, kind, n):
    check(client, edge_rows(n, kind, seed=n), kind)


@pytest.mark.parametrize("n", [4096, (3 << 20) + 8])
def test_index_operand_not_the_column(client, n):
    """Index values n-1-col: ties go to the higher column."""
    bits = edge_rows(n, "max", seed=7)
    check(client, bits, "max", reverse_index=True)


def test_c2_shape_winner_everywhere(client):
    """64 x 128256 (the benchmark's shape): the row's winner placed in every
    split and at each split's first and last element."""
    rows, n = 64, 128256
    rng = np.random.default_rng(5)
    bits = ops.f32_to_bf16_bits(rng.standard_normal((rows, n)).astype(np.float32))
    for r in range(rows):
        pos = (r * 8016 + (0 if r % 3 == 0 else 8015 if r % 3 == 1 else 4000)) % n
        bits[r, pos] = ops.f32_to_bf16_bits(np.float32(60.0))
        if r % 4 == 0:   # a tie later in the row
            bits[r, (pos + 30000) % n] = bits[r, pos]
    check(client, bits, "max")


@pytest.mark.parametrize("rows,n", [(64, 128256), (24, 50000), (5, 50000), (1, 128256), (13, 9000)])
def test_fused_combine_matches_combine_kernel(client, monkeypatch, rows, n):
    """Split rows folded by the last-arriving workgroup of each row (the
    default: every split of a row runs on one XCD; a row count that is not a
    multiple of 8 gets a padded grid whose extra workgroups leave at once)
    give the same bits as the separate combine kernel
    (PJRTX_REDUCE_FUSED_COMBINE=0), on every one of several back-to-back
    executions (the per-row arrival counters are put back to zero by each
    launch), for the argmax, f16 sum, max and min of the benchmark's program."""
    from pjrtx_amd import programs
    bits = ops.f32_to_bf16_bits(np.random.default_rng(21).standard_normal((rows, n)).astype(np.float32))
    text = programs.c2_argmax_f16_reductions(rows, n)
    monkeypatch.setenv("PJRTX_REDUCE_FUSED_COMBINE", "0")
    sep = client.compile(text)
    want = sep(bits, dtypes=["bf16"])
    monkeypatch.delenv("PJRTX_REDUCE_FUSED_COMBINE")
    fused = client.compile(text)
    assert "_combine" not in " ".join(fused.step_names())
    assert "_combine" in " ".join(sep.step_names())
    want_idx = ops.argmax_rows(ops.bf16_bits_to_f32(bits))[1]
    np.testing.assert_array_equal(want[1], want_idx)
    for _ in range(6):
        got = fused(bits, dtypes=["bf16"])
        assert len(got) == len(want)
        for g, w in zip(got, want):
            np.testing.assert_array_equal(np.asarray(g).view(np.uint8), np.asarray(w).view(np.uint8))


@pytest.mark.parametrize("rows,n", [(64, 128256), (5, 50000)])
def test_combine_fallback_without_xcd_placement(client, run_fresh, rows, n):
    """With the XCD placement probe disabled (PJRTX_XCD_LOCAL=0, read once per
    process) split reductions run the main kernel plus the `_combine`
    kernel; the C2 program's results are the same bits as the default
    one-launch fold."""
    from pjrtx_amd import programs
    bits = ops.f32_to_bf16_bits(np.random.default_rng(23).standard_normal((rows, n)).astype(np.float32))
    text = programs.c2_argmax_f16_reductions(rows, n)
    want = client.compile(text)(bits, dtypes=["bf16"])
    other = run_fresh(text, [bits], ["bf16"], {"PJRTX_XCD_LOCAL": "0"})
    assert len(other) == len(want)
    for g, w in zip(other, want):
        np.testing.assert_array_equal(np.asarray(g).view(np.uint8), np.asarray(w).view(np.uint8))
    np.testing.assert_array_equal(want[1], ops.argmax_rows(ops.bf16_bits_to_f32(bits))[1])
