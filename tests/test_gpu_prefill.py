"""GPU parity for the causal prefill attention (S new query rows per sequence,
flash-style blocks of 64 keys) against the CPU oracle's grouped attention with
the causal mask key_pos <= q_pos (attention.rs:14-32, 83-135), through the C
ABI.

The kernel scores with q at f32 accuracy (bf16 hi + lo parts on the MFMA) and
feeds the probabilities to P.V rounded to bf16, so outputs sit about 1e-3 from
the f32 oracle: the north-star bound (max relative error <= 1e-2) is asserted,
plus a tighter 4e-3 that a wrong mask, index or scale would break."""
import numpy as np
import pytest

import oracle
from conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-2
TIGHT = 4e-3


def rx():
    import rxla_amd
    return rxla_amd


def oracle_prefill(q, kc_bits, vc_bits, starts):
    """q [B,S,Hq,D] f32; caches [B,Hkv,Lmax,D] bf16 bits; row i of sequence b
    at position starts[b] + i (starts already in [0, Lmax - S])."""
    b, s, hq, d = q.shape
    lmax = kc_bits.shape[2]
    k = oracle.bf16_to_f32(kc_bits)
    v = oracle.bf16_to_f32(vc_bits)
    out = np.empty_like(q)
    for bi in range(b):
        pos = starts[bi] + np.arange(s)
        mask = np.where(np.arange(lmax)[None, :] <= pos[:, None], 0.0, -np.inf).astype(np.float32)
        o = oracle.gqa_attention(q[bi].transpose(1, 0, 2)[None], k[bi:bi + 1], v[bi:bi + 1],
                                 mask[None, None], threads=16)
        out[bi] = o[0].transpose(1, 0, 2)
    return out


def run_prefill(rt, q, kc_bits, vc_bits, starts, out_bf16=False, q_bf16=False):
    r = rx()
    qb = rt.buffer(oracle.bf16_bits(q), r.DType.BF16) if q_bf16 else rt.buffer(q)
    out = r.grouped_query_attention_prefill(
        rt, qb, rt.buffer(kc_bits, r.DType.BF16), rt.buffer(vc_bits, r.DType.BF16),
        rt.buffer(np.asarray(starts, np.int32)),
        out_dtype=r.DType.BF16 if out_bf16 else r.DType.F32).to_numpy()
    return r.bf16_to_f32(out) if out_bf16 else out


def make(rng, b, s, hq, hkv, lmax, d=128):
    q = rng.standard_normal((b, s, hq, d)).astype(np.float32)
    kc = oracle.bf16_bits(rng.standard_normal((b, hkv, lmax, d)).astype(np.float32))
    vc = oracle.bf16_bits(rng.standard_normal((b, hkv, lmax, d)).astype(np.float32))
    return q, kc, vc


@pytest.mark.parametrize("group", [1, 2, 4, 8])
@pytest.mark.parametrize("s,starts", [(1, [0, 5]), (15, [0, 40]), (64, [0, 0]), (100, [3, 150]),
                                      (130, [64, 1])])
def test_prefill_matches_oracle(rt, group, s, starts):
    """Ragged row blocks (S = 1, 15, 100, 130), whole blocks (64), rows that
    start at position 0 and mid-cache, block-aligned and unaligned starts."""
    rng = np.random.default_rng(1000 * group + s)
    hkv, lmax = 2, 320
    q, kc, vc = make(rng, len(starts), s, hkv * group, hkv, lmax)
    ref = oracle_prefill(q, kc, vc, np.array(starts))
    out = run_prefill(rt, q, kc, vc, starts)
    err = rel_err(out, ref)
    print(f"G={group} S={s} starts={starts} rel_err={err:.3e}")
    assert err <= TOL
    assert err <= TIGHT


def test_prefill_c5_shape(rt):
    """C5 prompt: 8 sequences x 1024 rows, 16 q / 8 kv heads, bf16 output;
    rows checked on a sample of sequences against the oracle."""
    rng = np.random.default_rng(2024)
    b, s, hq, hkv, lmax = 8, 1024, 16, 8, 1280
    q, kc, vc = make(rng, b, s, hq, hkv, lmax)
    starts = np.zeros(b, np.int32)
    out = run_prefill(rt, q, kc, vc, starts, out_bf16=True)
    assert np.isfinite(out).all()
    for bi in (0, 5):
        ref = oracle_prefill(q[bi:bi + 1], kc[bi:bi + 1], vc[bi:bi + 1], starts[bi:bi + 1])
        err = rel_err(out[bi:bi + 1], ref)
        print(f"C5 prefill seq {bi} rel_err={err:.3e}")
        assert err <= TOL
        assert err <= TIGHT


@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_prefill_bf16_q_and_first_row_is_value_row(rt, group):
    """Row 0 at position 0 sees key 0 alone: its output is exactly v[0]
    (softmax of one key: probability exactly 1), which pins the mask edge,
    the V^T indexing and each head's kv head for every group size."""
    rng = np.random.default_rng(7 + group)
    hq = 2 * group
    q, kc, vc = make(rng, 2, 70, hq, 2, 128)
    out = run_prefill(rt, q, kc, vc, [0, 0], q_bf16=True)
    v0 = oracle.bf16_to_f32(vc[:, :, 0, :])  # [B, Hkv, D]
    for h in range(hq):
        np.testing.assert_allclose(out[:, 0, h], v0[:, h // group], rtol=0, atol=0)
    ref = oracle_prefill(oracle.round_bf16(q), kc, vc, np.array([0, 0]))
    assert rel_err(out, ref) <= TIGHT


def test_prefill_starts_are_clamped(rt):
    """starts < 0 behave as 0; starts past Lmax - S behave as Lmax - S."""
    rng = np.random.default_rng(8)
    s, lmax = 40, 200
    q, kc, vc = make(rng, 2, s, 4, 2, lmax)
    out = run_prefill(rt, q, kc, vc, [-7, 500])
    ref = oracle_prefill(q, kc, vc, np.array([0, lmax - s]))
    assert rel_err(out, ref) <= TIGHT


@pytest.mark.parametrize("hq,hkv,d", [(8, 1, 64), (6, 3, 96), (4, 4, 256), (5, 1, 32), (12, 4, 128)])
def test_any_group_and_head_dim(rt, hq, hkv, d):
    """Group sizes and head dims outside the MFMA kernel (D = 128, Hq/Hkv in
    {1, 2, 4, 8}) run on the general GQA kernel with the same causal-from-starts
    rule: f32 scores and probabilities, so it matches the f32 oracle closely."""
    rng = np.random.default_rng(hq * 100 + d)
    s, lmax = 37, 150
    q, kc, vc = make(rng, 2, s, hq, hkv, lmax, d=d)
    starts = [0, 90]
    out = run_prefill(rt, q, kc, vc, starts)
    ref = oracle_prefill(q, kc, vc, np.array(starts))
    err = rel_err(out, ref)
    print(f"prefill Hq={hq} Hkv={hkv} D={d}: rel_err {err:.2e}")
    assert err <= 1e-5
    out16 = run_prefill(rt, q, kc, vc, [500, -3], out_bf16=True, q_bf16=True)  # clamped starts
    ref16 = oracle_prefill(oracle.round_bf16(q), kc, vc, np.array([lmax - s, 0]))
    assert rel_err(out16, ref16) <= TIGHT


def test_prefill_errors(rt):
    r = rx()
    rng = np.random.default_rng(9)
    q, kc, vc = make(rng, 2, 80, 4, 2, 64)  # S > Lmax
    with pytest.raises(r.Error) as e:
        run_prefill(rt, q, kc, vc, [0, 0])
    assert e.value.code == r.Status.INVALID_ARGUMENT
    q, kc, vc = make(rng, 2, 8, 6, 4, 64)  # 6 query heads over 4 kv heads
    with pytest.raises(r.Error) as e:
        run_prefill(rt, q, kc, vc, [0, 0])
    assert e.value.code == r.Status.INVALID_ARGUMENT
    q, kc, vc = make(rng, 1, 8, 2, 1, 64, d=640)  # head dim beyond the general kernel
    with pytest.raises(r.Error) as e:
        run_prefill(rt, q, kc, vc, [0])
    assert e.value.code == r.Status.UNIMPLEMENTED
