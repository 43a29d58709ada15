"""The decode attention entry point that allocates nothing
(rxw8_gqa_decode_noalloc) against rxw8_gqa_decode_into, bit for bit, through
the C ABI: two calls in a row on one GPU, the second smaller, so the second
reads a scratch array that still holds the first call's partials and
counters."""
import numpy as np
import pytest

import oracle
from conftest import rel_err

pytestmark = pytest.mark.gpu


def rx():
    import rxla_amd
    return rxla_amd


def make_case(seed, b, hq, hkv, lmax, lens, masked=False):
    rng = np.random.default_rng(seed)
    q = oracle.round_bf16(rng.standard_normal((b, hq, 128)).astype(np.float32))
    kc = oracle.bf16_bits(rng.standard_normal((b, hkv, lmax, 128)).astype(np.float32))
    vc = oracle.bf16_bits(rng.standard_normal((b, hkv, lmax, 128)).astype(np.float32))
    mask = None
    if masked:
        mask = np.where(rng.random((b, hq, lmax)) < 0.1, -np.inf, 0.0).astype(np.float32)
        mask[:, :, 0] = 0.0  # every row keeps a visible key
    return q, kc, vc, np.asarray(lens, np.int32), mask


def both(rt, case):
    r = rx()
    q, kc, vc, lens, mask = case
    bufs = (rt.buffer(q), rt.buffer(kc, r.DType.BF16), rt.buffer(vc, r.DType.BF16),
            rt.buffer(lens))
    m = rt.buffer(mask) if mask is not None else None
    want = rt.zeros(q.shape, r.DType.F32)
    r.grouped_query_attention(rt, *bufs, mask=m, out=want)
    got = rt.zeros(q.shape, r.DType.F32)
    r.grouped_query_attention_noalloc(rt, *bufs, got, mask=m)
    return got.to_numpy(), want.to_numpy()


def test_noalloc_equals_allocating_entry_point_on_two_calls(rt):
    c4 = make_case(80, 8, 32, 8, 8192, np.random.default_rng(81).integers(512, 8193, 8))
    small = make_case(82, 2, 8, 2, 700, [700, 300], masked=True)
    for name, case in (("C4", c4), ("small+mask", small)):
        got, want = both(rt, case)
        print(f"noalloc {name}: max|diff|={np.max(np.abs(got - want)):.3e}", flush=True)
        np.testing.assert_array_equal(got, want)
    q, kc, vc, lens, _ = c4
    assert rel_err(both(rt, c4)[0], oracle.gqa_decode_bf16cache(q, kc, vc, lens, threads=16)) <= 1e-4


@pytest.mark.parametrize("b,hq,hkv", [(64, 8, 2), (128, 8, 1)])
def test_noalloc_length_proportional_plans(rt, b, hq, hkv):
    """Ragged rows on the length-proportional split plan (units workgroups per
    kv head shared by the rows): one partial slot per workgroup, so these fit
    the scratch (B = 64, Hkv = 2 and B = 128, Hkv = 1 at Lmax 4096), bit for
    bit equal to the allocating entry point and within 1e-4 of the oracle."""
    lens = np.random.default_rng(b + hkv).integers(1, 4097, b)
    case = make_case(85 + b, b, hq, hkv, 4096, lens)
    got, want = both(rt, case)
    np.testing.assert_array_equal(got, want)
    q, kc, vc, lens, _ = case
    err = rel_err(got, oracle.gqa_decode_bf16cache(q, kc, vc, lens, threads=16))
    print(f"noalloc B={b} Hq={hq} Hkv={hkv}: rel_err vs oracle {err:.3e}", flush=True)
    assert err <= 1e-4


def test_noalloc_rejects_a_plan_beyond_its_scratch(rt, monkeypatch):
    r = rx()
    # 64 forced splits of 8 x 8 (row, kv head) pairs at G = 8 need 17.0 MB of
    # partials, more than the 16 MiB scratch: refused before any launch.
    monkeypatch.setenv("RXW8_ATTN_SPLITS", "64")
    q, kc, vc, lens, _ = make_case(83, 8, 64, 8, 4096, [4096] * 8)
    out = rt.buffer(np.full(q.shape, 7.0, np.float32))
    with pytest.raises(r.Error) as e:
        r.grouped_query_attention_noalloc(rt, rt.buffer(q), rt.buffer(kc, r.DType.BF16),
                                          rt.buffer(vc, r.DType.BF16), rt.buffer(lens), out)
    assert e.value.code == r.Status.RESOURCE_EXHAUSTED
    np.testing.assert_array_equal(out.to_numpy(), 7.0)
    monkeypatch.delenv("RXW8_ATTN_SPLITS")
    small = make_case(84, 3, 16, 2, 1500, [1500, 1, 777])
    got, want = both(rt, small)
    np.testing.assert_array_equal(got, want)
