"""Pins the CPU oracle (oracle/) before it is trusted as the GPU parity checker.

Each check is either a golden vector the reference's own tests hold (see
tests/golden/make_golden.py for the source lines), a closed form, or an
independent f64 numpy restatement written from the reference sources -- chosen
so that a plausible mistake in the oracle (wrong rounding, dropped offset,
wrong kv-head mapping, missing mask, wrong clamp) fails one of them.
"""
import math

import numpy as np
import pytest

import oracle
from conftest import golden_json, golden_npz, rel_err


# ---- independent numpy helpers (not the oracle's code) ----------------------------

def np_bf16_round(x):
    """RNE f32 -> bf16 -> f32 in numpy integer arithmetic."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def np_quantize(w, g):
    """benchmarks/quantize_qwen3_5_w8.py:31-40 restated in numpy float32."""
    w = np.asarray(w, np.float32)
    n, k = w.shape
    grouped = w.reshape(n, k // g, g)
    amax = np.abs(grouped).max(axis=2)
    scale = (np.maximum(amax, np.float32(1e-12)) / np.float32(127.0)).astype(np.float32)
    q = np.clip(np.rint(grouped / scale[:, :, None]), -127, 127)
    return (q + 128).astype(np.uint8).reshape(n, k), scale


def np_dequant(u8, s):
    n, k = u8.shape
    g = k // s.shape[1]
    return ((u8.astype(np.float32) - np.float32(128.0)) * np.repeat(s, g, axis=1)).astype(np.float32)


# ---- conversions ---------------------------------------------------------------------

def test_bf16_cast_kats():
    kat = golden_json("cast_kat.json")
    got = oracle.round_bf16(np.array(kat["input"], np.float32))
    np.testing.assert_array_equal(got, np.array(kat["bf16"], np.float32))


def test_bf16_all_bit_patterns_round_trip():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = oracle.bf16_to_f32(bits)
    back = oracle.bf16_bits(f)
    nan = np.isnan(f)
    np.testing.assert_array_equal(back[~nan], bits[~nan])
    assert np.all(np.isnan(oracle.bf16_to_f32(back[nan])))


def test_bf16_rne_ties_and_random_against_numpy():
    ties = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x3F80C000, 0x3F807FFF],
                    np.uint32).view(np.float32)
    np.testing.assert_array_equal(oracle.bf16_bits(ties),
                                  np.array([0x3F80, 0x3F82, 0xBF80, 0x3F81, 0x3F80], np.uint16))
    x = np.random.default_rng(1).standard_normal(100000).astype(np.float32) * 1e3
    np.testing.assert_array_equal(oracle.round_bf16(x), np_bf16_round(x))


# ---- a1 / a2 ---------------------------------------------------------------------------

def test_quantizer_matches_numpy_restatement():
    rng = np.random.default_rng(0)
    for g in (1024, 128, 64, 8):
        w = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
        u8, s = oracle.quantize_w8(w, g)
        u8n, sn = np_quantize(w, g)
        np.testing.assert_array_equal(s, sn)
        np.testing.assert_array_equal(u8, u8n)


def test_quantizer_closed_forms():
    w = np.zeros((3, 8), np.float32)
    w[1] = [0.5, -1.0, 0.25, 1.0, -0.5, 0.0, 0.75, -0.25]
    w[2] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, -127.0]  # s == 1: exact ties
    u8, s = oracle.quantize_w8(w, 8)
    assert s[0, 0] == np.float32(np.float32(1e-12) / np.float32(127.0))
    assert np.all(u8[0] == 128)  # zero row
    assert u8[1, 3] == 255 and u8[1, 1] == 1  # +-amax -> +-127
    assert s[2, 0] == 1.0
    np.testing.assert_array_equal(u8[2], [255, 128, 130, 130, 128, 126, 126, 1])


def test_quantizer_rounds_ties_even_like_reference_rounding_kats():
    r = golden_npz("rounding.npz")
    x, expected = r["x"], r["expected"]
    finite = np.isfinite(x)
    vals = x[finite]
    row = np.concatenate([vals.clip(-127, 127), [127.0]]).astype(np.float32)  # amax 127 -> s = 1
    u8, s = oracle.quantize_w8(row[None, :], row.size)
    assert s[0, 0] == 1.0
    want = np.clip(expected[finite], -127, 127)
    np.testing.assert_array_equal(u8[0, :-1].astype(np.int32) - 128, want.astype(np.int32))


def test_dequant_exhaustive_256_codes():
    codes = np.tile(np.arange(256, dtype=np.uint8), (16, 1))
    rng = np.random.default_rng(3)
    s = np.abs(rng.standard_normal((16, 1))).astype(np.float32) * np.float32(1e-3)
    s[0, 0] = np.float32(1.0 / 127.0)
    s[1, 0] = np.float32(1e-12) / np.float32(127.0)
    got = oracle.dequantize_w8(codes, s)
    np.testing.assert_array_equal(got.view(np.uint32), np_dequant(codes, s).view(np.uint32))


def test_quantized_linear_exact_small_ints():
    # crates/rxla-core/tests/matmul.rs:97-108: [[1,2,3],[4,5,6]] . [1,2,3] = [14, 32]
    u8 = (np.array([[1, 2, 3], [4, 5, 6]]) + 128).astype(np.uint8)
    s = np.ones((2, 1), np.float32)
    x = np.array([[1.0, 2.0, 3.0]], np.float32)
    for compute in (oracle.COMPUTE_F32, oracle.COMPUTE_BF16):
        np.testing.assert_array_equal(oracle.quantized_linear(x, u8, s, compute), [[14.0, 32.0]])


@pytest.mark.parametrize("m,n,k,g", [(8, 96, 256, 256), (3, 64, 512, 64), (1, 32, 64, 8)])
def test_quantized_linear_against_f64(m, n, k, g):
    rng = np.random.default_rng(m * 1000 + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    u8, s = np_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32), g)
    wdq = np_dequant(u8, s).astype(np.float64)
    y32 = oracle.quantized_linear(x, u8, s, oracle.COMPUTE_F32)
    assert rel_err(y32, x.astype(np.float64) @ wdq.T) < 1e-5
    # bf16 compute: bf16(x), bf16(W) (layers.rs:292-294), f64 sum, bf16 result
    ref = np_bf16_round((np_bf16_round(x).astype(np.float64) @
                         np_bf16_round(wdq.astype(np.float32)).astype(np.float64).T).astype(np.float32))
    y16 = oracle.quantized_linear(x, u8, s, oracle.COMPUTE_BF16)
    y64 = oracle.quantized_linear(x, u8, s, oracle.COMPUTE_BF16, oracle.ACCUM_F64)
    np.testing.assert_array_equal(oracle.round_bf16(y16), y16)  # bf16-valued result
    assert np.max(np.abs(y64 - ref) / np.maximum(np.abs(ref), 1e-30)) <= 2.0 ** -8
    assert rel_err(y16, ref) < 4e-3
    # dropping the -128 offset or the scale must be visible
    bad = x.astype(np.float64) @ (u8.astype(np.float64) * np.repeat(s, k // s.shape[1], 1)).T
    assert rel_err(bad, ref) > 0.5


# ---- attention ------------------------------------------------------------------------

@pytest.mark.parametrize("kv_heads", [1, 2, 4])
@pytest.mark.parametrize("precision", [0, 1])
def test_gqa_reference_head_masks(kv_heads, precision):
    g = golden_npz("gqa_head_masks.npz")
    out = oracle.gqa_attention(g["q"], g[f"k{kv_heads}"], g[f"v{kv_heads}"], g["mask"],
                               precision=precision)
    assert np.max(np.abs(out - g[f"expected{kv_heads}"])) < 2e-6  # tests/gqa.rs:95-99


def test_causal_masks_reference_vectors():
    """crates/rxla-core/tests/causal_attention.rs:59-69 (extreme I32 positions)
    and :168-174 (the static (2, 4, 1) mask as positions offset + i)."""
    g = golden_npz("causal_attention.npz")
    np.testing.assert_array_equal(oracle.causal_attention_mask(g["x_qpos"], g["x_kpos"]), g["x_mask"])
    np.testing.assert_array_equal(oracle.causal_attention_mask(np.arange(2) + 1, np.arange(4)),
                                  g["static_241"])
    # a subtraction-based mask would overflow on these positions
    assert oracle.causal_attention_mask([np.iinfo(np.int32).max], [np.iinfo(np.int32).min])[0, 0] == 0


def test_causal_sdpa_reference_vectors():
    """causal_attention.rs:35-56 (runtime positions; zero scores average the
    visible values) and :93-175 (full and chunked causal attention against
    the test's f64 loop), through the oracle's f64 GQA with one head."""
    g = golden_npz("causal_attention.npz")
    for qpos, want in zip(g["rt_qpos"], g["rt_expected"]):
        m = oracle.causal_attention_mask(qpos, g["rt_kpos"])
        out = oracle.gqa_attention(np.zeros((1, 1, 2, 1), np.float32), np.zeros((1, 1, 4, 1), np.float32),
                                   g["rt_v"][None, None], m, scale=1.0, precision=1)
        np.testing.assert_allclose(out[0, 0, :, 0], want, atol=2e-5)
    q, k, v = (g[n][None, None] for n in ("full_q", "full_k", "full_v"))
    full = oracle.gqa_attention(q, k, v, oracle.causal_attention_mask(np.arange(5), np.arange(7)),
                                scale=1.0, precision=1)[0, 0]
    np.testing.assert_allclose(full, g["full_expected"], atol=2e-5)
    for start, end in g["chunks"]:
        m = oracle.causal_attention_mask(np.arange(start, end), np.arange(7))
        part = oracle.gqa_attention(q[:, :, start:end], k, v, m, scale=1.0, precision=1)[0, 0]
        np.testing.assert_allclose(part, full[start:end], atol=2e-5)


def test_masked_decode_reference_steps():
    g = golden_npz("masked_decode.npz")
    kc = np.full((2, 4, 2), g["init_k"], np.float32)
    vc = np.full((2, 4, 2), g["init_v"], np.float32)
    for step in range(4):
        kc, vc, acc = oracle.kv_update_at(kc, vc, g["k"][step], g["v"][step], [0, step, 0])
        mask = np.where(np.arange(4) <= step, 0.0, -np.inf).astype(np.float32)
        out = oracle.gqa_attention(g["q"][step][None], kc[None], vc[None], mask[None, None, None])
        assert np.max(np.abs(out[0, :, 0, :] - g["expected"][step])) < 2e-6


def test_decode_form_matches_masked_general_form():
    rng = np.random.default_rng(5)
    b, hq, hkv, lmax, d = 3, 8, 2, 40, 16
    q = rng.standard_normal((b, hq, d)).astype(np.float32)
    kc = oracle.bf16_bits(rng.standard_normal((b, hkv, lmax, d)))
    vc = oracle.bf16_bits(rng.standard_normal((b, hkv, lmax, d)))
    lens = np.array([1, 17, 40], np.int32)
    dec = oracle.gqa_decode_bf16cache(q, kc, vc, lens)
    mask = np.where(np.arange(lmax)[None, :] < lens[:, None], 0.0, -np.inf).astype(np.float32)
    gen = oracle.gqa_attention(q[:, :, None, :], oracle.bf16_to_f32(kc), oracle.bf16_to_f32(vc),
                               mask[:, None, None, :])
    np.testing.assert_allclose(dec, gen[:, :, 0, :], rtol=0, atol=1e-6)
    # independent f64 numpy restatement: kv = h // (hq // hkv)
    kf, vf = oracle.bf16_to_f32(kc).astype(np.float64), oracle.bf16_to_f32(vc).astype(np.float64)
    for bi in range(b):
        for h in range(hq):
            kv = h // (hq // hkv)
            L = lens[bi]
            s = kf[bi, kv, :L] @ q[bi, h].astype(np.float64) / math.sqrt(d)
            p = np.exp(s - s.max())
            p /= p.sum()
            np.testing.assert_allclose(dec[bi, h], p @ vf[bi, kv, :L], rtol=0, atol=2e-6)


# ---- KV cache ---------------------------------------------------------------------------

def test_kv_update_clamps_like_reference():
    t = golden_json("kv_clamp.json")
    kc = np.zeros(t["shape"], np.float32)
    vc = np.zeros(t["shape"], np.float32)
    for pos, k, v in t["steps"]:
        kc, vc, _ = oracle.kv_update_at(kc, vc, np.full(t["update_shape"], k, np.float32),
                                        np.full(t["update_shape"], v, np.float32), [pos, 0])
    np.testing.assert_array_equal(kc.ravel(), t["expected_keys"])
    np.testing.assert_array_equal(vc.ravel(), t["expected_values"])


def test_kv_update_checked_table():
    t = golden_json("kv_checked.json")
    kc = np.zeros(t["shape"], np.float32)
    vc = np.zeros(t["shape"], np.float32)
    for st in t["steps"]:
        keys = np.array([np.nan if x is None else x for x in st["keys"]], np.float32)
        kc, vc, acc = oracle.kv_update_at(kc, vc, keys.reshape(2, 2),
                                          np.array(st["values"], np.float32).reshape(2, 2),
                                          [st["row"], st["col"]], checked=True)
        assert acc == st["accepted"]
        np.testing.assert_array_equal(kc.ravel(), st["expected_keys"])
        np.testing.assert_array_equal(vc.ravel(), st["expected_values"])


def test_dynamic_update_slice_rank4_against_numpy():
    rng = np.random.default_rng(7)
    op = rng.integers(0, 1000, (2, 3, 9, 4)).astype(np.uint16)
    up = rng.integers(0, 1000, (1, 3, 2, 4)).astype(np.uint16)
    for starts in ([1, 0, 7, 0], [5, -3, 20, 9], [0, 0, -1, 0]):
        got = oracle.dynamic_update_slice(op, up, starts)
        want = op.copy()
        st = [min(max(s, 0), D - u) for s, D, u in zip(starts, op.shape, up.shape)]
        want[st[0]:st[0] + 1, st[1]:st[1] + 3, st[2]:st[2] + 2, st[3]:st[3] + 4] = up
        np.testing.assert_array_equal(got, want)


# ---- elementwise / reductions -----------------------------------------------------------

def test_argmax_reference_cases():
    g = golden_npz("argmax.npz")
    x = g["x234"]
    np.testing.assert_array_equal(oracle.argmax_rows(np.moveaxis(x, 2, -1).reshape(-1, 4)),
                                  g["axis2"])
    np.testing.assert_array_equal(oracle.argmax_rows(np.moveaxis(x, 1, -1).reshape(-1, 3)),
                                  g["axis1"])
    np.testing.assert_array_equal(oracle.argmax_rows(x.reshape(2, 12).T.copy()), g["axis0"])
    np.testing.assert_array_equal(oracle.argmax_rows(g["rows6"]), g["rows6_expected"])


def test_rope_closed_forms():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((5, 3, 128)).astype(np.float32)
    pos = np.array([0, 1, 7, 1000, 8191], np.int32)
    y = oracle.rope_split_half(x, pos, 1e6)
    np.testing.assert_array_equal(y[0], x[0])  # position 0 is the identity
    freqs = oracle.rope_freqs(1e6, 128)
    assert freqs[0] == 1.0
    f64 = 1e6 ** (-2.0 * np.arange(64) / 128.0)
    np.testing.assert_allclose(freqs, f64, rtol=2e-6)
    # angles are formed in f32 as in the reference (positions.to_f32() * freqs)
    ang = (pos[:, None, None].astype(np.float32) * freqs[None, None, :]).astype(np.float64)
    a, b = x[..., :64].astype(np.float64), x[..., 64:].astype(np.float64)
    want = np.concatenate([a * np.cos(ang) - b * np.sin(ang), b * np.cos(ang) + a * np.sin(ang)], -1)
    np.testing.assert_allclose(y, want, rtol=0, atol=2e-5)
    # rotation keeps each (i, i + 64) pair's norm
    np.testing.assert_allclose(y[..., :64] ** 2 + y[..., 64:] ** 2, a ** 2 + b ** 2, rtol=1e-5)


def test_rms_norm_and_silu_against_f64():
    rng = np.random.default_rng(13)
    x = rng.standard_normal((4, 256)).astype(np.float32)
    w = rng.standard_normal(256).astype(np.float32)
    for zc in (False, True):
        y = oracle.rms_norm(x, w, 1e-6, zc)
        xd = x.astype(np.float64)
        want = xd / np.sqrt((xd ** 2).mean(-1, keepdims=True) + 1e-6) * ((1.0 + w) if zc else w)
        np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-6)
    c = np.full((1, 16), 3.0, np.float32)
    np.testing.assert_allclose(oracle.rms_norm(c, np.ones(16, np.float32), 1e-6),
                               3.0 / np.sqrt(9.0 + 1e-6), rtol=1e-6)
    g, u = x[:2].ravel(), x[2:].ravel()
    gd = g.astype(np.float64)
    np.testing.assert_allclose(oracle.silu_mul(g, u), gd / (1 + np.exp(-gd)) * u, rtol=1e-5,
                               atol=1e-7)


def test_take_rows_clamps():
    table = np.arange(20, dtype=np.uint16).reshape(5, 4)
    got = oracle.take_rows(table, np.array([-3, 0, 4, 5, 99], np.int32))
    np.testing.assert_array_equal(got, table[[0, 0, 4, 4, 4]])


# ---- decoder composition ------------------------------------------------------------------

from decoder_fixtures import numpy_decoder_step, tiny_config, tiny_params  # noqa: E402


def test_decoder_prefill_equals_stepwise_decode():
    cfg = tiny_config()
    params = tiny_params(cfg, seed=21)
    rng = np.random.default_rng(22)
    ids = rng.integers(0, cfg["vocab"], (2, 6)).astype(np.int32)
    a = oracle.Decoder(cfg, params, 2)
    la, na = a.forward(ids)
    b = oracle.Decoder(cfg, params, 2)
    for t in range(6):
        lb, nb = b.forward(ids[:, t:t + 1])
    np.testing.assert_array_equal(la, lb)
    np.testing.assert_array_equal(na, nb)
    np.testing.assert_array_equal(a.k_cache, b.k_cache)
    np.testing.assert_array_equal(a.lens, [6, 6])


def test_decoder_against_numpy_composition():
    cfg = tiny_config()
    params = tiny_params(cfg, seed=31, std=0.1)  # large enough that attention matters
    rng = np.random.default_rng(32)
    ids = rng.integers(0, cfg["vocab"], (2, 5)).astype(np.int32)
    dec = oracle.Decoder(cfg, params, 2)
    logits, nxt = dec.forward(ids)
    want = numpy_decoder_step(cfg, params, ids)
    assert rel_err(logits, want) < 2e-3
    # a decoder that skipped RoPE differs by far more
    assert rel_err(logits, numpy_decoder_step(cfg, params, ids, skip_rope=True)) > 5e-2
