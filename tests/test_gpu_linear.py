"""GPU parity for the W8A16 linear (K1 GEMV, generic kernel) and dequantisation
against the CPU oracle, through the C ABI (rxla_amd -> librxw8.so).

Tolerance: max relative error <= 1e-2, measured
normwise as max|gpu - oracle| / max|oracle|. Dequantisation is bit-exact.
"""
import numpy as np
import pytest

import oracle
from conftest import elem_rel_err, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-2
# Per element (floor at 1% of the rms): within one bf16 ulp, whose relative
# spacing is at most 2^-7. The GEMV forms the reference's product, the f32 sum
# of bf16(x) * bf16(dequantised W), and rounds it to bf16; against the same
# cast points with exact (f64) accumulation only the summation order differs,
# so two independently rounded bf16 results can be one ulp apart.
ELEM_TOL = 2.0 ** -7


def exact(x, u8, s):
    """The reference's cast points (bf16 x, bf16 dequantised W, bf16 result)
    with exact accumulation."""
    return oracle.quantized_linear(x, u8, s, oracle.COMPUTE_BF16, oracle.ACCUM_F64, threads=16)


def rx():
    import rxla_amd
    return rxla_amd


def quantized(rng, n, k, g, std=0.02):
    w = (rng.standard_normal((n, k)) * std).astype(np.float32)
    return oracle.quantize_w8(w, g)


def run_linear(rt, x, u8, s, x_dtype=None, out_dtype=None, compute=None):
    r = rx()
    x_dtype = x_dtype or r.DType.F32
    out_dtype = out_dtype or r.DType.F32
    compute = compute or r.DType.BF16
    xb = rt.buffer(oracle.bf16_bits(x) if x_dtype == r.DType.BF16 else x, x_dtype)
    y = r.quantized_linear(rt, xb, rt.buffer(u8, r.DType.U8), rt.buffer(s, r.DType.F32),
                           compute, out_dtype).to_numpy()
    return r.bf16_to_f32(y) if out_dtype == r.DType.BF16 else y


def test_c1_single_linear_f32_boundary(rt):
    # x f32 [8,1024] ~N(0,1); W [1024,1024] ~N(0,0.02), per-channel, seed 0
    rng = np.random.default_rng(0)
    x = rng.standard_normal((8, 1024)).astype(np.float32)
    u8, s = quantized(rng, 1024, 1024, 1024)
    ref = oracle.quantized_linear(x, u8, s, oracle.COMPUTE_BF16)
    y = run_linear(rt, x, u8, s)
    e_elem = elem_rel_err(y, exact(oracle.round_bf16(x), u8, s))
    print(f"C1 rel_err={rel_err(y, ref):.3e} elem_rel_err(vs exact)={e_elem:.3e}")
    assert rel_err(y, ref) <= TOL
    assert e_elem <= ELEM_TOL
    np.testing.assert_array_equal(oracle.round_bf16(y), y)  # bf16-valued, like the reference


@pytest.mark.parametrize("n", [4096, 6144, 24576])
@pytest.mark.parametrize("b", [1, 4, 16])
def test_c2_decode_gemv_sweep(rt, b, n):
    rng = np.random.default_rng(1000 + 10 * b + n)
    x = oracle.round_bf16(rng.standard_normal((b, 4096)).astype(np.float32))
    u8, s = quantized(rng, n, 4096, 4096)
    ref = oracle.quantized_linear(x, u8, s, oracle.COMPUTE_BF16, threads=16)
    y = run_linear(rt, x, u8, s, x_dtype=rx().DType.BF16, out_dtype=rx().DType.BF16)
    err = rel_err(y, ref)
    e_elem = elem_rel_err(y, exact(x, u8, s))
    print(f"C2 B={b} N={n} rel_err={err:.3e} elem_rel_err(vs exact)={e_elem:.3e}")
    assert err <= TOL
    assert e_elem <= ELEM_TOL


@pytest.mark.parametrize("m,k,g", [(8, 2048, 64), (8, 2048, 128), (8, 2048, 512),
                                   # groups wider than a wave's K slice at 1 and 4 rows
                                   (1, 4096, 2048), (4, 4096, 1024), (16, 4096, 2048)])
def test_grouped_scales(rt, m, k, g):
    rng = np.random.default_rng(g + m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    u8, s = quantized(rng, 1024, k, g)
    ref = oracle.quantized_linear(x, u8, s, oracle.COMPUTE_BF16)
    err = rel_err(run_linear(rt, x, u8, s), ref)
    print(f"G={g} rel_err={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("m,n,k,g", [(2, 32, 64, 32), (3, 40, 96, 32), (5, 24, 64, 8),
                                     (70, 128, 256, 256), (200, 64, 128, 64)])
def test_other_shapes(rt, m, n, k, g):
    """Shapes outside the MFMA tiling (generic kernel) and M > 64 (chunked)."""
    rng = np.random.default_rng(m + n + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    u8, s = quantized(rng, n, k, g)
    ref = oracle.quantized_linear(x, u8, s, oracle.COMPUTE_BF16)
    assert rel_err(run_linear(rt, x, u8, s), ref) <= TOL


def test_f32_compute_path(rt):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((4, 256)).astype(np.float32)
    u8, s = quantized(rng, 64, 256, 128)
    ref = oracle.quantized_linear(x, u8, s, oracle.COMPUTE_F32)
    y = run_linear(rt, x, u8, s, compute=rx().DType.F32)
    assert rel_err(y, ref) < 1e-5


@pytest.mark.parametrize("m,n,k,g", [(1, 1000, 1024, 128), (16, 4096, 1024, 128),
                                     (33, 777, 512, 64), (100, 256, 2048, 2048),
                                     (5, 96, 4096, 4096),
                                     # K ranges of whole groups (the 0.8B down projection)
                                     (16, 1024, 3584, 128), (40, 512, 8192, 2048),
                                     # one group wider than LDS: equal parts of it
                                     (3, 256, 12288, 12288)])
def test_f32_compute_matrix_core_path(rt, m, n, k, g):
    """F32 compute on the matrix cores: x as bf16 hi + lo parts (16 significant
    bits), exact codes, f32 accumulation; channel and row tails included, and
    inputs too wide for one LDS staging (several launches over K ranges)."""
    rng = np.random.default_rng(m * 7 + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    u8, s = quantized(rng, n, k, g)
    ref = oracle.quantized_linear(x, u8, s, oracle.COMPUTE_F32, oracle.ACCUM_F64)
    y = run_linear(rt, x, u8, s, compute=rx().DType.F32)
    err = rel_err(y, ref)
    print(f"F32 compute m={m} n={n} k={k} g={g} rel_err={err:.3e}")
    assert err < 1e-5


@pytest.mark.parametrize("ksplit", ["1", "3"])
@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("m,n,k,g", [(1, 256, 64, 64), (130, 512, 256, 128), (300, 1024, 1024, 128),
                                     (257, 768, 3584, 128), (129, 256, 2048, 2048),
                                     (1024, 4096, 1024, 64), (200, 640, 512, 128), (64, 128, 1024, 128),
                                     (150, 1040, 1024, 128)])
def test_f32_compute_gemm_tiles(rt, monkeypatch, m, n, k, g, packed, ksplit):
    """F32 compute on the GEMM tiles for long inputs (rxw8_gemm_f32c,
    forced here at every size): x split into bf16 hi + lo, exact codes, group
    sums scaled in f32; ragged M, a half n tile (N % 256 == 128), N % 256 ==
    16, one k tile, 28 scale groups, per-channel scales; row-major and packed
    weights; whole K, or 3 K splits (scale groups, or k tiles of the one
    group) summed by rxw8_gemm_f32c_reduce. Within 1e-5 of the f64 oracle (on
    sampled rows at M = 1024) and of the row-tile kernel."""
    monkeypatch.setenv("RXW8_F32_GEMM_KSPLIT", ksplit)
    r = rx()
    rng = np.random.default_rng(m * 3 + n + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    u8, s = quantized(rng, n, k, g)
    rows = np.arange(m) if m <= 300 else np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, 40)]))
    ref = oracle.quantized_linear(x[rows], u8, s, oracle.COMPUTE_F32, oracle.ACCUM_F64, threads=16)
    run = run_linear_packed_f32 if packed else (lambda rt_, x_, u_, s_: run_linear(rt_, x_, u_, s_, compute=r.DType.F32))
    monkeypatch.setenv("RXW8_F32_GEMM", "1")
    y = run(rt, x, u8, s)
    monkeypatch.setenv("RXW8_F32_GEMM", "0")
    monkeypatch.delenv("RXW8_F32_GEMM_KSPLIT")
    try:
        y_rows = run(rt, x, u8, s)
    except r.Error as e:  # the packed GEMV has no tiling for K = 64
        assert e.code == r.Status.UNIMPLEMENTED and packed and k == 64
        y_rows = y
    err = rel_err(y[rows], ref)
    print(f"F32 GEMM m={m} n={n} k={k} g={g} packed={packed} ksplit={ksplit}: rel_err={err:.3e}, "
          f"vs row tiles {rel_err(y, y_rows):.3e}")
    assert err < 1e-5
    assert rel_err(y, y_rows) < 1e-5


def test_f32_compute_exact_on_integer_inputs(rt):
    """One-hot / small-integer x with unit scales: every product and sum is
    exact in f32, so the matrix-core F32 path must reproduce it bit for bit
    (every code 0..255 -> -128..127, and lo parts of integers are zero)."""
    k = np.arange(1024)
    codes = ((k[None, :] + 4 * np.arange(160)[:, None]) % 256).astype(np.uint8)  # [160, 1024]
    s = np.ones((160, 8), np.float32)
    x = np.zeros((20, 1024), np.float32)
    for r in range(4):
        x[r, r] = 1.0
    x[4:] = np.random.default_rng(3).integers(-3, 4, (16, 1024))
    x[5] = 0.0
    x[5, 7], x[5, 9] = 1.0 + 2.0 ** -12, 2.0  # 1 + 2^-12 is not a bf16: needs the lo part
    want = (x.astype(np.float64) @ (codes.astype(np.float64) - 128).T).astype(np.float32)
    y = run_linear(rt, x, codes, s, compute=rx().DType.F32)
    np.testing.assert_array_equal(y, want)


def run_linear_packed_f32(rt, x, u8, s):
    r = rx()
    packed = r.pack_weight(rt, rt.buffer(u8, r.DType.U8))
    return r.quantized_linear(rt, rt.buffer(x), packed, rt.buffer(s, r.DType.F32),
                              r.DType.F32, r.DType.F32).to_numpy()


@pytest.mark.parametrize("m,n,k,g", [(1, 1024, 1024, 128), (5, 4096, 1024, 128), (8, 256, 2048, 2048),
                                     (9, 7168, 1024, 128), (16, 1024, 2048, 128),
                                     # 32 staged rows of K do not fit: chunks of 8 rows
                                     (16, 1024, 3584, 128), (40, 1024, 3584, 128),
                                     # chunks of 16 rows
                                     (37, 512, 1024, 64)])
def test_f32_compute_packed_gemv(rt, monkeypatch, m, n, k, g):
    """F32 compute on packed weights: the GEMV stages each f32 row as bf16
    hi and lo rows (batch columns t and 8 / 16 + t), multiplies the exact
    codes u - 128 and adds the two parts in f32 (no bf16 rounding). Inputs
    longer than one workgroup's rows run as chunks of rows side by side in
    one launch (beyond 16 rows the GEMM tiles are switched off here)."""
    if m > 16:
        monkeypatch.setenv("RXW8_F32_GEMM", "0")
    rng = np.random.default_rng(m * 11 + n + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    u8, s = quantized(rng, n, k, g)
    ref = oracle.quantized_linear(x, u8, s, oracle.COMPUTE_F32, oracle.ACCUM_F64)
    y = run_linear_packed_f32(rt, x, u8, s)
    err = rel_err(y, ref)
    print(f"F32 compute packed m={m} n={n} k={k} g={g} rel_err={err:.3e}")
    assert err < 1e-5


@pytest.mark.parametrize("m", [1, 7, 16])
def test_f32_compute_packed_many_channels(rt, m):
    """F32 compute on packed weights with many 128-channel tiles (an LM head,
    N / 128 >= 4 x 256 CUs): the row kernel that stages x once per workgroup
    (rxw8_linear_f32_mfma_pk_*), reading the tile layout; a channel count
    that is not a multiple of 128 (a partial last tile)."""
    n, k, g = 131072 + 144, 1024, 128
    rng = np.random.default_rng(m * 7 + 3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    u8, s = quantized(rng, n, k, g)
    ref = oracle.quantized_linear(x, u8, s, oracle.COMPUTE_F32, oracle.ACCUM_F64)
    y = run_linear_packed_f32(rt, x, u8, s)
    err = rel_err(y, ref)
    print(f"F32 compute packed (row kernel) m={m} n={n} rel_err={err:.3e}")
    assert err < 1e-5


def test_f32_compute_packed_exact_on_integer_inputs(rt):
    """The packed F32 GEMV on the integer case of the row-major path above:
    bit for bit, including the row whose value needs the lo part."""
    k = np.arange(1024)
    codes = ((k[None, :] + 4 * np.arange(160)[:, None]) % 256).astype(np.uint8)
    s = np.ones((160, 8), np.float32)
    x = np.zeros((12, 1024), np.float32)
    for r in range(4):
        x[r, r] = 1.0
    x[4:] = np.random.default_rng(3).integers(-3, 4, (8, 1024))
    x[5] = 0.0
    x[5, 7], x[5, 9] = 1.0 + 2.0 ** -12, 2.0
    want = (x.astype(np.float64) @ (codes.astype(np.float64) - 128).T).astype(np.float32)
    np.testing.assert_array_equal(run_linear_packed_f32(rt, x, codes, s), want)


def test_rank3_input_and_empty_batch(rt):
    r = rx()
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 3, 512)).astype(np.float32)
    u8, s = quantized(rng, 256, 512, 512)
    y = run_linear(rt, x, u8, s)
    assert y.shape == (2, 3, 256)
    assert rel_err(y, oracle.quantized_linear(x, u8, s).reshape(2, 3, 256)) <= TOL
    empty = rt.buffer(np.zeros((0, 512), np.float32))
    out = r.quantized_linear(rt, empty, rt.buffer(u8), rt.buffer(s))
    assert out.shape == (0, 256)


def test_dequant_bit_exact_all_codes(rt):
    r = rx()
    codes = np.tile(np.arange(256, dtype=np.uint8), (64, 4))  # [64, 1024]
    rng = np.random.default_rng(5)
    for groups in (1, 8):
        s = (np.abs(rng.standard_normal((64, groups))) * 1e-3).astype(np.float32)
        s[0, 0] = np.float32(1e-12) / np.float32(127.0)
        want = oracle.dequantize_w8(codes, s)
        got = r.dequantize(rt, rt.buffer(codes), rt.buffer(s), r.DType.F32).to_numpy()
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        got16 = r.dequantize(rt, rt.buffer(codes), rt.buffer(s), r.DType.BF16).to_numpy()
        np.testing.assert_array_equal(got16, oracle.bf16_bits(want))


def test_gemv_codes_exact_on_integer_inputs(rt):
    """With s = 1 and one-hot x the W8A16 result is exact, so every code
    (0..255 -> -128..127) and the -128 fold are checked bit for bit."""
    k = np.arange(4096)
    codes = ((k[None, :] + 4 * np.arange(64)[:, None]) % 256).astype(np.uint8)  # [64, 4096]
    s = np.ones((64, 1), np.float32)
    x = np.zeros((5, 4096), np.float32)
    for r in range(4):
        x[r, r] = 1.0  # y[r, i] = code[i, r] - 128: r + 4 i covers all 256 codes
    x[4, :256] = 1.0   # one full cycle: sum(-128..127) = -128
    want = (x.astype(np.float64) @ (codes.astype(np.float64) - 128).T).astype(np.float32)
    assert sorted(set(want[:4].ravel().tolist())) == list(range(-128, 128))
    y = run_linear(rt, x, codes, s)
    np.testing.assert_array_equal(y, want)


def test_deterministic_split_k(rt):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((4, 4096)).astype(np.float32)
    u8, s = quantized(rng, 4096, 4096, 4096)
    a = run_linear(rt, x, u8, s)
    b = run_linear(rt, x, u8, s)
    np.testing.assert_array_equal(a, b)


def test_validation_rejects_before_launch(rt):
    r = rx()
    x = rt.buffer(np.zeros((2, 64), np.float32))
    w = rt.buffer(np.zeros((32, 64), np.uint8))
    bad_scale = rt.buffer(np.zeros((32, 3), np.float32))  # 64 % 3 != 0
    with pytest.raises(r.Error) as e:
        r.quantized_linear(rt, x, w, bad_scale)
    assert e.value.code == r.Status.INVALID_ARGUMENT
    with pytest.raises(r.Error):
        r.quantized_linear(rt, x, rt.buffer(np.zeros((32, 64), np.float32)),
                           rt.buffer(np.zeros((32, 1), np.float32)))
    y = rt.buffer(np.full((2, 16), 7.0, np.float32))  # wrong width: untouched
    with pytest.raises(r.Error):
        r.quantized_linear(rt, x, w, rt.buffer(np.ones((32, 1), np.float32)), out=y)
    np.testing.assert_array_equal(y.to_numpy(), 7.0)
    with pytest.raises(r.Error):
        r.QuantizedLinear(32, 48).apply(rt, x, w, rt.buffer(np.ones((32, 1), np.float32)))


def test_bf16_weight_linear_lm_head(rt):
    r = rx()
    rng = np.random.default_rng(7)
    x = rng.standard_normal((8, 2048)).astype(np.float32)
    e = oracle.bf16_bits(rng.standard_normal((4096, 2048)).astype(np.float32) * 0.02)
    ref = oracle.linear_bf16w(x, e)
    y = r.linear_bf16(rt, rt.buffer(x), rt.buffer(e, r.DType.BF16)).to_numpy()
    assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("b,n,k,g", [(1, 4096, 4096, 4096), (16, 6144, 4096, 4096),
                                     (8, 2048, 2048, 128), (4, 1024, 6144, 6144),
                                     (8, 2048, 6144, 2048),  # 3-way k split
                                     # the decoder's gate|up width and the bench's roofline
                                     # kernel (rxw8_gemv_w8_pk_mb1_rw3_u4_w12 at B=1)
                                     (1, 24576, 4096, 4096), (4, 24576, 4096, 4096),
                                     (16, 24576, 4096, 4096)])
def test_packed_weights_bit_identical(rt, b, n, k, g):
    """The tiled layout holds the same bytes: results equal the row-major path."""
    r = rx()
    rng = np.random.default_rng(b * 7 + n)
    x = oracle.round_bf16(rng.standard_normal((b, k)).astype(np.float32))
    u8, s = quantized(rng, n, k, g)
    wb = rt.buffer(u8)
    packed = r.pack_weight(rt, wb)
    assert packed.shape == (n // 16, k // 64, 1024)
    tiles = packed.to_numpy()
    # block (t, c), lane l = row 16t + l%16, columns 64c + 16(l/16) .. +16
    lane = 37
    np.testing.assert_array_equal(tiles[3, 5, lane * 16:(lane + 1) * 16],
                                  u8[16 * 3 + lane % 16, 64 * 5 + 16 * (lane // 16):][:16])
    xb, sb = rt.buffer(oracle.bf16_bits(x), r.DType.BF16), rt.buffer(s)
    y_row = r.quantized_linear(rt, xb, wb, sb, r.DType.BF16, r.DType.F32).to_numpy()
    y_pk = r.quantized_linear(rt, xb, packed, sb, r.DType.BF16, r.DType.F32).to_numpy()
    np.testing.assert_array_equal(y_pk, y_row)
    assert rel_err(y_pk, oracle.quantized_linear(x, u8, s)) <= TOL


def test_packed_bf16_lm_head(rt):
    r = rx()
    rng = np.random.default_rng(8)
    x = rng.standard_normal((8, 2048)).astype(np.float32)
    e = oracle.bf16_bits(rng.standard_normal((4096, 2048)).astype(np.float32) * 0.02)
    eb = rt.buffer(e, r.DType.BF16)
    pk = r.pack_weight(rt, eb)
    assert pk.shape == (256, 64, 512)
    y_row = r.linear_bf16(rt, rt.buffer(x), eb).to_numpy()
    y_pk = r.linear_bf16(rt, rt.buffer(x), pk).to_numpy()
    np.testing.assert_array_equal(y_pk, y_row)
    assert rel_err(y_pk, oracle.linear_bf16w(x, e)) <= TOL


@pytest.mark.parametrize("packed", [False, True])
def test_full_vocab_lm_head(rt, packed):
    """The C5 head: bf16 embedding [151936, 2048] reused as lm_head at batch 8
    (622 MB of weights; the decode step's largest GEMV), row-major and in the
    decoder's packed layout."""
    r = rx()
    rng = np.random.default_rng(151936 + packed)
    x = rng.standard_normal((8, 2048)).astype(np.float32)
    e = oracle.bf16_bits((rng.standard_normal((151936, 2048)) * 0.02).astype(np.float32))
    eb = rt.buffer(e, r.DType.BF16)
    w = r.pack_weight(rt, eb) if packed else eb
    y = r.linear_bf16(rt, rt.buffer(x), w).to_numpy()
    ref = oracle.linear_bf16w(x, e, threads=16)
    err = rel_err(y, ref)
    e_elem = elem_rel_err(y, ref)
    print(f"lm_head 8x2048x151936 packed={packed} rel_err={err:.3e} elem_rel_err={e_elem:.3e}")
    assert err <= TOL
    # both sides round the f32 sum of bf16(x) . W (exact products) to bf16
    assert e_elem <= ELEM_TOL


def test_pack_weight_validation(rt):
    r = rx()
    with pytest.raises(r.Error) as e:
        r.pack_weight(rt, rt.buffer(np.zeros((24, 64), np.uint8)))  # 24 % 16 != 0
    assert e.value.code == r.Status.INVALID_ARGUMENT


@pytest.mark.parametrize("m,n,k,g,packed", [
    (1, 4096, 4096, 4096, False), (4, 6144, 4096, 4096, True), (16, 24576, 4096, 4096, False),
    (8, 2048, 2048, 2048, True), (8, 12288, 2048, 2048, True),
    # grouped scales (the scale tile staged per workgroup), row-major and packed
    (8, 4096, 2048, 128, True), (8, 2048, 6144, 64, False), (1, 1024, 4096, 2048, False)])
def test_reference_cast_point_gemv(rt, monkeypatch, m, n, k, g, packed):
    """The GEMV casts every dequantised weight to bf16 before the product,
    bf16((u - 128) * s) (crates/rxla-nn/src/layers.rs:288-297), and applies no
    scale after the sum. Against the oracle with the same cast points and
    exact (f64) accumulation, only the f32 summation of the kernel and the
    final bf16 rounding differ: each output within one bf16 ulp (2^-7
    relative, floor at 1% of the rms), and closer to that oracle than the
    exact-code product with the scale after the sum (RXW8_GEMV_REF_CAST=0)."""
    r = rx()
    rng = np.random.default_rng(m * 7 + n + g)
    x = oracle.round_bf16(rng.standard_normal((m, k)).astype(np.float32))
    u8, s = quantized(rng, n, k, g)
    ref = oracle.quantized_linear(x, u8, s, oracle.COMPUTE_BF16, oracle.ACCUM_F64, threads=16)

    def run():
        w = rt.buffer(u8, r.DType.U8)
        if packed:
            w = r.pack_weight(rt, w)
        y = r.quantized_linear(rt, rt.buffer(oracle.bf16_bits(x), r.DType.BF16), w,
                               rt.buffer(s, r.DType.F32), r.DType.BF16, r.DType.F32)
        return y.to_numpy()

    monkeypatch.setenv("RXW8_GEMV_REF_CAST", "0")
    y_exact = run()
    monkeypatch.delenv("RXW8_GEMV_REF_CAST")
    y_rc = run()
    e_rc, e_exact = elem_rel_err(y_rc, ref), elem_rel_err(y_exact, ref)
    same = float(np.mean(y_rc == ref))
    print(f"ref-cast m={m} n={n} k={k} g={g} packed={packed}: elem_rel_err {e_rc:.3e} "
          f"(exact-code {e_exact:.3e}); bit-equal {same:.4f}; normwise {rel_err(y_rc, ref):.3e} "
          f"(exact-code {rel_err(y_exact, ref):.3e})")
    np.testing.assert_array_equal(oracle.round_bf16(y_rc), y_rc)
    assert e_rc <= ELEM_TOL
    assert rel_err(y_rc, ref) <= rel_err(y_exact, ref)


@pytest.mark.parametrize("packed", [True, False])
def test_quantized_linear_group_sweep(rt, packed):
    """The nine decode shapes of BASELINE configs[1] (B 1/4/16 x N 4096/6144/
    24576, K 4096) in one rxw8_quantized_linear_group call (two launches: up to
    4 rows, 16 rows), plus a grouped-scale product with f32 input and output:
    every output within one bf16 ulp of the reference-order oracle and of
    the single call (the grouped launch runs its own tilings, 96-row tiles up
    to 4 rows and 192-row tiles beyond, so summation order may differ)."""
    r = rx()
    rng = np.random.default_rng(4096 + packed)
    probs = [(b, n, 4096, 4096, r.DType.BF16) for n in (4096, 6144, 24576) for b in (1, 4, 16)]
    probs.append((8, 1024, 2048, 128, r.DType.F32))
    xs, ws, ss, ys, refs, singles = [], [], [], [], [], []
    for b, n, k, g, dt in probs:
        x = oracle.round_bf16(rng.standard_normal((b, k)).astype(np.float32))
        u8, s = quantized(rng, n, k, g)
        xb = rt.buffer(oracle.bf16_bits(x), r.DType.BF16) if dt == r.DType.BF16 else rt.buffer(x)
        wb = rt.buffer(u8, r.DType.U8)
        if packed:
            wb = r.pack_weight(rt, wb)
        sb = rt.buffer(s, r.DType.F32)
        xs.append(xb), ws.append(wb), ss.append(sb)
        ys.append(rt.buffer(np.full((b, n), np.nan, np.float32)))
        refs.append(exact(x, u8, s))
        singles.append(r.quantized_linear(rt, xb, wb, sb, r.DType.BF16, r.DType.F32).to_numpy())
    r.quantized_linear_group(rt, xs, ws, ss, ys)
    for (b, n, k, g, _), y, ref, single in zip(probs, ys, refs, singles):
        got = y.to_numpy()
        e = elem_rel_err(got, ref)
        print(f"group B={b} N={n} K={k} G={g} packed={packed}: elem_rel_err {e:.3e}, "
              f"equal to the single call {float(np.mean(got == single)):.4f}")
        assert e <= ELEM_TOL
        assert elem_rel_err(got, single) <= ELEM_TOL


def test_quantized_linear_group_validation(rt):
    r = rx()
    x = rt.buffer(np.zeros((4, 512), np.float32))
    w = rt.buffer(np.full((32, 512), 128, np.uint8))
    s = rt.buffer(np.ones((32, 1), np.float32))
    y = rt.buffer(np.full((4, 32), 7.0, np.float32))
    wp = r.pack_weight(rt, w)
    x17 = rt.buffer(np.zeros((17, 512), np.float32))
    y17 = rt.buffer(np.zeros((17, 32), np.float32))
    for args, code in ((([x, x], [w, wp], [s, s], [y, y]), r.Status.INVALID_ARGUMENT),
                       (([x17], [w], [s], [y17]), r.Status.UNIMPLEMENTED),
                       (([x], [w], [s], [y17]), r.Status.INVALID_ARGUMENT)):
        with pytest.raises(r.Error) as e:
            r.quantized_linear_group(rt, *args)
        assert e.value.code == code
    rt.synchronize()
    np.testing.assert_array_equal(y.to_numpy(), 7.0)
