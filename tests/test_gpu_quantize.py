"""GPU W8 encoder (rxw8_quantize_w8) bit for bit against the oracle's
restatement of benchmarks/quantize_qwen3_5_w8.py:27-44, which the CPU tests
pin by closed forms and the reference's rounding KATs."""
import numpy as np
import pytest

import oracle
from conftest import golden_npz

pytestmark = pytest.mark.gpu


def rx():
    import rxla_amd
    return rxla_amd


def gpu_quantize(rt, w, g, bf16=False):
    r = rx()
    buf = rt.buffer(oracle.bf16_bits(w), r.DType.BF16) if bf16 else rt.buffer(w)
    u, s = r.quantize_w8(rt, buf, g)
    assert u.dtype == r.DType.U8 and s.dtype == r.DType.F32
    return u.to_numpy(), s.to_numpy()


def test_closed_forms(rt):
    w = np.zeros((3, 8), np.float32)
    w[1] = [0.5, -1.0, 0.25, 1.0, -0.5, 0.0, 0.75, -0.25]
    w[2] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, -127.0]  # s == 1: exact ties go to even
    u8, s = gpu_quantize(rt, w, 8)
    assert s[0, 0] == np.float32(np.float32(1e-12) / np.float32(127.0))
    assert np.all(u8[0] == 128)                      # zero row
    assert u8[1, 3] == 255 and u8[1, 1] == 1         # +-amax -> +-127
    assert s[2, 0] == 1.0
    np.testing.assert_array_equal(u8[2], [255, 128, 130, 130, 128, 126, 126, 1])
    uo, so = oracle.quantize_w8(w, 8)
    np.testing.assert_array_equal(u8, uo)
    np.testing.assert_array_equal(s.view(np.uint32), so.view(np.uint32))


def test_reference_rounding_kats(rt):
    r = golden_npz("rounding.npz")
    x, expected = r["x"], r["expected"]
    finite = np.isfinite(x)
    row = np.concatenate([x[finite].clip(-127, 127), [127.0]]).astype(np.float32)
    u8, s = gpu_quantize(rt, row[None, :], row.size)
    assert s[0, 0] == 1.0
    want = np.clip(expected[finite], -127, 127).astype(np.int32)
    np.testing.assert_array_equal(u8[0, :-1].astype(np.int32) - 128, want)


@pytest.mark.parametrize("g", [4096, 128, 64, 96])
def test_random_matrix_bit_exact(rt, g):
    rng = np.random.default_rng(g)
    k = 4096 if g != 96 else 96 * 40
    w = (rng.standard_normal((4096, k)) * 0.02).astype(np.float32)
    w[7, :] = 0.0                          # zero row: s = 1e-12 / 127, codes 128
    w[9, 5] = 3.0                          # one large outlier per row
    u8, s = gpu_quantize(rt, w, g)
    uo, so = oracle.quantize_w8(w, g)
    np.testing.assert_array_equal(s.view(np.uint32), so.view(np.uint32))
    np.testing.assert_array_equal(u8, uo)


def test_bf16_input_widens_exactly(rt):
    rng = np.random.default_rng(5)
    w = oracle.round_bf16((rng.standard_normal((256, 1024)) * 0.02).astype(np.float32))
    u8, s = gpu_quantize(rt, w, 128, bf16=True)
    uo, so = oracle.quantize_w8(w, 128)
    np.testing.assert_array_equal(s.view(np.uint32), so.view(np.uint32))
    np.testing.assert_array_equal(u8, uo)


def test_encoder_errors(rt):
    r = rx()
    w = rt.buffer(np.zeros((4, 100), np.float32))
    for g in (0, -128, 64):  # non-positive, or 100 % 64 != 0
        with pytest.raises(r.Error) as e:
            r.quantize_w8(rt, w, g)
        assert e.value.code == r.Status.INVALID_ARGUMENT
    with pytest.raises(r.Error) as e:
        r.quantize_w8(rt, rt.buffer(np.zeros((4, 128), np.int32)), 128)
    assert e.value.code == r.Status.INVALID_ARGUMENT
