"""General attention masks on the GPU (rxw8_gqa_attention,
rxw8_causal_attention_mask): any query count with an additive mask that
broadcasts to [..., Hq, Sq, Sk], and causal masks from runtime I32 positions.
Pinned by the reference's own vectors (tests/gqa.rs:32-102 per-head masks at
kv_heads 1/2/4 within 2e-6; tests/causal_attention.rs:25-70 runtime and
extreme I32 positions, :93-175 full and chunked causal attention within 2e-5)
and by the oracle's f64 GQA on larger seeded cases."""
import numpy as np
import pytest

import oracle
from conftest import golden_npz, rel_err

pytestmark = pytest.mark.gpu


def rx():
    import rxla_amd
    return rxla_amd


def gqa(rt, q, k, v, mask=None, scale=None):
    r = rx()
    m = rt.buffer(np.ascontiguousarray(mask, np.float32)) if mask is not None else None
    return r.gqa_attention(rt, rt.buffer(q), rt.buffer(k), rt.buffer(v), m, scale).to_numpy()


@pytest.mark.parametrize("kv_heads", [1, 2, 4])
def test_reference_head_masks(rt, kv_heads):
    g = golden_npz("gqa_head_masks.npz")
    out = gqa(rt, g["q"], g[f"k{kv_heads}"], g[f"v{kv_heads}"], g["mask"])
    assert out.shape == (2, 4, 3, 3)
    assert np.max(np.abs(out - g[f"expected{kv_heads}"])) < 2e-6  # tests/gqa.rs:95-99


def test_runtime_position_masks(rt):
    r = rx()
    g = golden_npz("causal_attention.npz")
    m = r.causal_attention_mask(rt, rt.buffer(g["x_qpos"]), rt.buffer(g["x_kpos"])).to_numpy()
    np.testing.assert_array_equal(m, g["x_mask"])  # 16,777,216 / i32::MAX / i32::MIN exact
    for qpos, want in zip(g["rt_qpos"], g["rt_expected"]):
        mb = r.causal_attention_mask(rt, rt.buffer(qpos), rt.buffer(g["rt_kpos"]))
        out = r.scaled_dot_product_attention(rt, rt.buffer(np.zeros((2, 1), np.float32)),
                                             rt.buffer(np.zeros((4, 1), np.float32)),
                                             rt.buffer(g["rt_v"]), mb, scale=1.0).to_numpy()
        assert out.shape == (2, 1)
        assert np.max(np.abs(out[:, 0] - want)) < 2e-5  # causal_attention.rs:52-54
    empty = r.causal_attention_mask(rt, rt.buffer(np.zeros(2, np.int32)),
                                    rt.buffer(np.zeros(0, np.int32)))
    assert empty.shape == (2, 0)
    with pytest.raises(r.Error) as e:
        r.causal_attention_mask(rt, rt.buffer(np.zeros((2, 1), np.int32)), rt.buffer(g["x_kpos"]))
    assert e.value.code == r.Status.INVALID_ARGUMENT


def test_static_masks_and_their_checks(rt):
    r = rx()
    g = golden_npz("causal_attention.npz")
    np.testing.assert_array_equal(r.causal_attention_mask_static(rt, 2, 4, 1).to_numpy(),
                                  g["static_241"])
    for q, k, o in g["static_bad"]:
        with pytest.raises(r.Error) as e:
            r.causal_attention_mask_static(rt, int(q), int(k), int(o))
        assert e.value.code == r.Status.INVALID_ARGUMENT
    assert r.causal_attention_mask_static(rt, 0, 4, 0).shape == (0, 4)
    one = r.causal_attention_mask_static(rt, 1, 1, 2 ** 31 - 1)
    assert one.shape == (1, 1) and one.to_numpy()[0, 0] == 0.0


def test_full_and_chunked_causal_attention(rt):
    r = rx()
    g = golden_npz("causal_attention.npz")
    q, k, v = (rt.buffer(g[n]) for n in ("full_q", "full_k", "full_v"))
    full = r.scaled_dot_product_attention(rt, q, k, v, r.causal_attention_mask_static(rt, 5, 7, 0),
                                          scale=1.0).to_numpy()
    assert np.max(np.abs(full - g["full_expected"])) < 2e-5  # causal_attention.rs:152-167
    for start, end in g["chunks"]:
        qc = rt.buffer(np.ascontiguousarray(g["full_q"][start:end]))
        m = r.causal_attention_mask_static(rt, int(end - start), 7, int(start))
        part = r.scaled_dot_product_attention(rt, qc, k, v, m, scale=1.0).to_numpy()
        assert np.max(np.abs(part - full[start:end])) < 2e-5  # :138-150


@pytest.mark.parametrize("mask_kind", ["none", "2d", "per_head", "batch_key", "causal_pos"])
@pytest.mark.parametrize("g_heads", [(8, 2), (4, 4), (8, 1)])
def test_seeded_cases_against_the_oracle(rt, mask_kind, g_heads):
    hq, hkv = g_heads
    rng = np.random.default_rng(hq * 10 + hkv + len(mask_kind))
    b, sq, sk, d, dv = 2, 37, 300, 128, 64
    q = rng.standard_normal((b, hq, sq, d)).astype(np.float32)
    k = rng.standard_normal((b, hkv, sk, d)).astype(np.float32)
    v = rng.standard_normal((b, hkv, sk, dv)).astype(np.float32)
    mask = None
    if mask_kind == "2d":
        mask = rng.standard_normal((sq, sk)).astype(np.float32)
    elif mask_kind == "per_head":
        mask = np.where(rng.random((1, hq, sq, sk)) < 0.3, -np.inf,
                        rng.standard_normal((1, hq, sq, sk))).astype(np.float32)
        mask[..., 0] = 0.0
    elif mask_kind == "batch_key":
        mask = np.where(rng.random((b, 1, 1, sk)) < 0.5, -np.inf, 0.0).astype(np.float32)
        mask[..., 5] = 0.0
    elif mask_kind == "causal_pos":  # a chunk of 37 rows starting at position 250
        mask = oracle.causal_attention_mask(250 + np.arange(sq), np.arange(sk))
    got = gqa(rt, q, k, v, mask)
    want = oracle.gqa_attention(q, k, v, mask, precision=1)
    err = rel_err(got, want)
    print(f"GQA Hq={hq} Hkv={hkv} mask={mask_kind}: rel_err {err:.2e}")
    assert err <= 1e-5
    assert np.max(np.abs(got - want)) < 2e-5


def test_batch_dims_broadcast_and_all_masked_rows(rt):
    """A rank-5 batch prefix [2, 3] with a mask that broadcasts over the
    second batch dim only; a row whose keys are all masked is NaN, as the
    reference's max-subtract softmax gives."""
    rng = np.random.default_rng(9)
    q = rng.standard_normal((2, 3, 4, 5, 16)).astype(np.float32)
    k = rng.standard_normal((2, 3, 2, 9, 16)).astype(np.float32)
    v = rng.standard_normal((2, 3, 2, 9, 8)).astype(np.float32)
    mask = rng.standard_normal((2, 1, 4, 5, 9)).astype(np.float32)
    mask[1, 0, 2, 3, :] = -np.inf  # batch (1, *), head 2, row 3: nothing visible
    got = gqa(rt, q, k, v, mask, scale=0.3)
    want = np.stack([oracle.gqa_attention(q[:, j], k[:, j], v[:, j], mask[:, 0], scale=0.3,
                                          precision=1) for j in range(3)], axis=1)
    assert np.isnan(got[1, :, 2, 3]).all()
    ok = ~np.isnan(want)
    assert np.isnan(want[1, :, 2, 3]).all()
    assert np.max(np.abs(got[ok] - want[ok])) < 2e-5


def test_error_contract(rt):
    r = rx()
    f = lambda *s: rt.buffer(np.zeros(s, np.float32))  # noqa: E731
    q, k, v = f(2, 4, 3, 2), f(2, 2, 5, 2), f(2, 2, 5, 7)
    assert r.gqa_attention(rt, q, k, v).shape == (2, 4, 3, 7)
    assert r.gqa_attention(rt, q, k, v, f(3, 5)).shape == (2, 4, 3, 7)  # tests/gqa.rs:20-21

    def code(fn):
        with pytest.raises(r.Error) as e:
            fn()
        return e.value.code

    for bad_k in (f(2, 3, 5, 2), f(1, 2, 5, 2), f(2, 5, 2), f(2, 0, 5, 2)):  # tests/gqa.rs:15-19
        assert code(lambda: r.gqa_attention(rt, q, bad_k, v)) == r.Status.INVALID_ARGUMENT
    assert code(lambda: r.gqa_attention(rt, q, k, v, f(4, 5))) == r.Status.INVALID_ARGUMENT
    assert code(lambda: r.gqa_attention(rt, q, f(2, 2, 0, 2), f(2, 2, 0, 7))) == r.Status.INVALID_ARGUMENT
    assert code(lambda: r.gqa_attention(rt, q, k, v, scale=float("inf"))) == r.Status.INVALID_ARGUMENT
    qb = rt.buffer(np.zeros((2, 4, 3, 2), np.uint16), r.DType.BF16)
    assert code(lambda: r.gqa_attention(rt, qb, k, v)) == r.Status.INVALID_ARGUMENT
