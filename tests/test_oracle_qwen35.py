"""Pins for the Qwen3.5 hybrid-model oracle (oracle/qwen35.py) by facts the
mathematics fixes, so a dropped term, a wrong sign or a transposed operand
fails here rather than being restated in a GPU test."""
import numpy as np
import pytest

import oracle
from oracle import qwen35 as q35


def test_causal_conv_is_a_flipped_convolution():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 9, 5))
    w = rng.standard_normal((5, 4))
    out = q35.depthwise_causal_conv(x, w)
    for b in range(2):
        for c in range(5):
            # correlation with w == convolution with w reversed, first S outputs
            want = np.convolve(x[b, :, c], w[c, ::-1])[:9]
            np.testing.assert_allclose(out[b, :, c], want, rtol=1e-12, atol=1e-12)
    # causal: output t ignores inputs after t
    x2 = x.copy()
    x2[:, 5:] = 77.0
    np.testing.assert_array_equal(q35.depthwise_causal_conv(x2, w)[:, :5], out[:, :5])


def test_delta_rule_stores_value_under_unit_key():
    """With g = 1 and beta = 1 the delta rule sets S^T k = v for the key just
    written (k unit): reading with q = k returns v exactly."""
    rng = np.random.default_rng(1)
    b, s, h, d = 2, 7, 3, 8
    k = rng.standard_normal((b, s, h, d))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((b, s, h, d))
    out = q35.delta_rule(k, k, v, np.ones((b, s, h)), np.ones((b, s, h)))
    np.testing.assert_allclose(out, v, rtol=1e-10, atol=1e-10)


def test_delta_rule_decay_and_linear_attention_limit():
    """g scales the whole state; with beta = 0 nothing is ever written; with
    orthonormal keys (d >= s) and beta = 1, g = 1 the output is the plain
    linear-attention sum sum_{u<=t} (q . k_u) v_u."""
    rng = np.random.default_rng(2)
    b, s, h, d = 1, 5, 2, 8
    basis = np.linalg.qr(rng.standard_normal((d, d)))[0]
    k = np.broadcast_to(basis[:s][None, :, None, :], (b, s, h, d)).copy()
    q = rng.standard_normal((b, s, h, d))
    v = rng.standard_normal((b, s, h, d))
    ones = np.ones((b, s, h))
    out = q35.delta_rule(q, k, v, ones, ones)
    want = np.zeros_like(out)
    for t in range(s):
        for u in range(t + 1):
            want[:, t] += (q[:, t] * k[:, u]).sum(-1)[..., None] * v[:, u]
    np.testing.assert_allclose(out, want, rtol=1e-10, atol=1e-10)
    assert not q35.delta_rule(q, k, v, np.zeros((b, s, h)), ones).any()
    # one step of decay g: the state written at t=0 reads back scaled by g_1
    g = np.full((b, s, h), 0.5)
    out_g = q35.delta_rule(k, k, v, ones, g)
    np.testing.assert_allclose(out_g[:, 0], v[:, 0], rtol=1e-12)


def test_norms_and_activations_closed_forms():
    x = np.array([[3.0, 4.0, 0.0, 0.0]])
    np.testing.assert_allclose(q35.l2_norm(x), x / np.sqrt(25 + 1e-6))
    # zero-centred RMSNorm with w = 0 is the plain normalisation (rms 1)
    y = q35.rms_norm(x, np.zeros(4), 0.0, True)
    np.testing.assert_allclose((y * y).mean(), 1.0)
    np.testing.assert_allclose(q35.rms_norm(x, np.full(4, 2.0), 0.0, False), 2 * y)
    z = np.array([-30.0, -1.0, 0.0, 1e-3, 2.0, 50.0])
    np.testing.assert_allclose(q35.softplus(z), np.log1p(np.exp(z)), rtol=1e-12)
    assert q35.softplus(np.array([800.0]))[0] == 800.0  # no overflow
    np.testing.assert_allclose(q35.sigmoid(z), 1 / (1 + np.exp(-z)), rtol=1e-12)
    np.testing.assert_allclose(q35.silu(z), z / (1 + np.exp(-z)), rtol=1e-12)


def test_partial_rope_full_width_matches_the_decoder_rope():
    """rotary_dim = D reduces to the split-half RoPE the C oracle restates
    (rotary.rs:17-74); the channels past rotary_dim pass through."""
    rng = np.random.default_rng(3)
    s, d, theta = 6, 16, 1e4
    x = rng.standard_normal((s, d)).astype(np.float32)
    ang = q35.rope_angles(theta, d, s)
    got = q35.partial_rope(x.astype(np.float64), ang, d)
    want = oracle.rope_split_half(x[:, None, :], np.arange(s, dtype=np.int32), theta)[:, 0]
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5)
    part = q35.partial_rope(x.astype(np.float64), q35.rope_angles(theta, 8, s), 8)
    np.testing.assert_array_equal(part[:, 8:], x[:, 8:])


def test_projection_and_dequant_against_the_c_oracle():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 64)).astype(np.float32)
    u8, s = oracle.quantize_w8((rng.standard_normal((24, 64)) * 0.05).astype(np.float32), 16)
    np.testing.assert_array_equal(q35.dequant(u8, s), oracle.dequantize_w8(u8, s))
    want = oracle.quantized_linear(x, u8, s, oracle.COMPUTE_BF16, oracle.ACCUM_F64)
    np.testing.assert_array_equal(q35.projection(x, u8, s, "bf16"), oracle.round_bf16(want))
    # the default compute dtype is F32 (rxla-nn lib.rs:432): f32 x against the
    # f32 dequantised weights, accumulated in f64 on both sides
    want = oracle.quantized_linear(x, u8, s, oracle.COMPUTE_F32, oracle.ACCUM_F64)
    np.testing.assert_array_equal(q35.projection(x, u8, s), want)
    assert q35.config()["compute"] == "f32"


def test_f32_projection_closed_form():
    """Integer activations and codes with power-of-two scales: every product
    and sum is exact, so the F32 projection equals the integer matrix product
    (a dropped scale, a transposed operand or a bf16 cast of x fails this:
    x holds 257, which bf16 cannot represent)."""
    x = np.array([[257.0, -3.0, 1.0, 0.0], [2.0, 5.0, -7.0, 11.0]], np.float32)
    codes = np.array([[1, 2, 3, 4], [-5, 6, -7, 8], [127, -127, 0, 1]])
    s = np.array([[0.5], [0.25], [2.0]], np.float32)
    y = q35.projection(x, (codes + 128).astype(np.uint8), s)
    np.testing.assert_array_equal(y, (x.astype(np.float64) @ (codes * s).T).astype(np.float32))
    assert y[0, 0] == np.float32((257 * 1 - 3 * 2 + 3) * 0.5)


def test_forward_runs_and_the_first_row_ignores_the_future():
    cfg = q35.config(layers=[q35.LINEAR, q35.FULL, q35.LINEAR])
    p = q35.random_params(cfg, seed=5)
    ids = np.random.default_rng(6).integers(0, cfg["vocab"], (2, 6))
    lg = q35.forward(cfg, p, ids)
    assert lg.shape == (2, 6, cfg["vocab"]) and np.isfinite(lg).all()
    ids2 = ids.copy()
    ids2[:, 3:] = (ids2[:, 3:] + 1) % cfg["vocab"]
    lg2 = q35.forward(cfg, p, ids2)
    np.testing.assert_allclose(lg2[:, :3], lg[:, :3], rtol=1e-12, atol=1e-12)  # causal
    assert np.abs(lg2[:, 3:] - lg[:, 3:]).max() > 0


def test_lora_head_is_a_low_rank_update_scaled_by_alpha_over_rank():
    """The LoRA head adds (alpha / r) (n A^T) B^T: zero with B = 0, a matrix of
    rank <= r over the positions, linear in alpha."""
    cfg = q35.config(layers=[q35.LINEAR], lora_rank=2, lora_alpha=4.0, vocab=96, hidden=32)
    p = q35.random_params(cfg, seed=7)
    ids = np.random.default_rng(8).integers(0, cfg["vocab"], (1, 9))
    base = q35.forward(dict(cfg, lora_rank=0), p, ids)
    lg = q35.forward(cfg, p, ids)
    diff = (lg - base)[0]
    sv = np.linalg.svd(diff, compute_uv=False)
    assert sv[1] > 1e-3 * sv[0] and sv[2] < 1e-9 * sv[0]  # rank exactly 2
    lg2 = q35.forward(dict(cfg, lora_alpha=8.0), p, ids)
    np.testing.assert_allclose(lg2 - base, 2 * (lg - base), rtol=1e-9, atol=1e-12)
    zb = dict(p)
    zb["model.language_model.embed_tokens.lora_B.weight"] = np.zeros_like(
        p["model.language_model.embed_tokens.lora_B.weight"])
    np.testing.assert_array_equal(q35.forward(cfg, zb, ids), base)
