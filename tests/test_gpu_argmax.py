"""GPU argmax (the decoder's greedy pick, rxw8_argmax) against the reference's
own vectors, bit for bit: crates/rxla-core/tests/argmax.rs:30-110 (ties take
the lowest index, the first NaN wins, +-inf and +-0), regenerated into
tests/golden/argmax.npz, plus a vocab-151936 batch with planted ties and NaNs
checked against the reference's scan (argmax.rs:25-38) restated in numpy."""
import numpy as np
import pytest

from conftest import golden_npz

pytestmark = pytest.mark.gpu


def rx():
    import rxla_amd
    return rxla_amd


def first_max(x, axis):
    """The reference test's scan (argmax.rs:25-38): best moves to i when the
    current best is not NaN and x[i] is NaN or greater."""
    x = np.moveaxis(np.asarray(x, np.float32), axis, -1)
    flat = x.reshape(-1, x.shape[-1])
    out = np.zeros(flat.shape[0], np.int32)
    for r, row in enumerate(flat):
        best = 0
        for i in range(1, row.size):
            if not np.isnan(row[best]) and (np.isnan(row[i]) or row[i] > row[best]):
                best = i
        out[r] = best
    return out.reshape(x.shape[:-1])


def gpu_argmax(rt, x, axis, keep_dims=False):
    r = rx()
    return r.argmax(rt, rt.buffer(np.ascontiguousarray(x, np.float32)), axis, keep_dims).to_numpy()


def test_reference_axes_vectors(rt):
    g = golden_npz("argmax.npz")
    x = g["x234"]
    for axis in range(3):
        want = g[f"axis{axis}"]
        got = gpu_argmax(rt, x, axis)
        np.testing.assert_array_equal(got.reshape(-1), want)
        np.testing.assert_array_equal(got.reshape(-1), first_max(x, axis).reshape(-1))
        kept = gpu_argmax(rt, x, axis, keep_dims=True)
        assert kept.shape == tuple(1 if i == axis else d for i, d in enumerate(x.shape))
        np.testing.assert_array_equal(kept.reshape(-1), want)


def test_reference_row_vectors(rt):
    g = golden_npz("argmax.npz")
    rows, want = g["rows6"], g["rows6_expected"]
    for row, w in zip(rows, want):  # each vector on its own, as the reference runs them
        np.testing.assert_array_equal(gpu_argmax(rt, row, 0), w)
    np.testing.assert_array_equal(gpu_argmax(rt, rows, 1), want)


def test_empty_other_axis_and_errors(rt):
    r = rx()
    assert gpu_argmax(rt, np.zeros((0, 3), np.float32), 1).shape == (0,)
    for shape, axis in (((3, 0), 1), ((2, 3), 2)):
        with pytest.raises(r.Error) as e:
            r.argmax(rt, rt.buffer(np.zeros(shape, np.float32)), axis)
        assert e.value.code == r.Status.INVALID_ARGUMENT


@pytest.mark.parametrize("cols", [151936, 6000, 2047])
def test_vocab_rows_with_planted_ties_and_nans(rt, cols):
    rng = np.random.default_rng(cols)
    x = rng.standard_normal((8, cols)).astype(np.float32)
    top = np.float32(10.0)
    x[0, [5, cols // 2, cols - 1]] = top             # tie: lowest index wins
    x[1, [cols - 1, 3]] = [np.nan, np.nan]           # first NaN wins
    x[2, :] = -np.inf                                # all -inf: index 0
    x[2, cols // 2] = -np.inf
    x[3, [7, cols - 2]] = [np.inf, np.inf]           # +inf tie
    x[4, :] = 0.0
    x[4, ::2] = -0.0                                  # +0 == -0: index 0
    x[5, cols - 1] = np.nan                           # NaN beats +inf at a lower index
    x[5, 1] = np.inf
    x[6, [cols // 3, 2 * cols // 3]] = top            # tie across argmax chunks
    got = gpu_argmax(rt, x, 1)
    want = first_max(x, 1)
    print(f"cols={cols} got={got.tolist()}")
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(got[:7], [5, 3, 0, 7, 0, cols - 1, cols // 3])
    # a column-wise reduction (inner stride > 1) over the same data
    np.testing.assert_array_equal(gpu_argmax(rt, x[:, :64], 0), first_max(x[:, :64], 0))
