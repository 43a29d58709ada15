"""The XLA GPU custom-call handlers (rxw8_xla_*): called exactly as XLA calls
an untyped status-returning custom call (stream, operand+result pointers,
backend_config text, status), they give the direct C ABI's results bit for
bit, on the stream they are handed; a malformed backend_config launches
nothing and reports through rxw8_last_error."""
import ctypes

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def rx():
    import rxla_amd
    return rxla_amd


def call(rt, name, bufs, opaque):
    r = rx()
    ptrs = (ctypes.c_void_p * len(bufs))(*[b.ptr for b in bufs])
    text = opaque.encode()
    getattr(r._lib, name)(ctypes.c_void_p(rt.stream()), ptrs, text, len(text), None)


@pytest.mark.parametrize("xd,yd,compute", [("f32", "f32", "bf16"), ("bf16", "bf16", "bf16"),
                                           ("f32", "f32", "f32")])
def test_quantized_linear_matches_the_c_abi(rt, xd, yd, compute):
    r = rx()
    dt = {"f32": r.DType.F32, "bf16": r.DType.BF16}
    rng = np.random.default_rng(1)
    m, n, k, g = 8, 640, 1024, 128
    x = rng.standard_normal((m, k)).astype(np.float32)
    u8, s = oracle.quantize_w8((rng.standard_normal((n, k)) * 0.02).astype(np.float32), g)
    xb = rt.buffer(oracle.bf16_bits(x), r.DType.BF16) if xd == "bf16" else rt.buffer(x)
    wb, sb = rt.buffer(u8), rt.buffer(s)
    want = r.quantized_linear(rt, xb, wb, sb, dt[compute], dt[yd]).to_numpy()
    y = rt.zeros((m, n), dt[yd])
    call(rt, "rxw8_xla_quantized_linear", [xb, wb, sb, y],
         f"m={m};n={n};k={k};g={g};x={xd};y={yd};compute={compute}")
    np.testing.assert_array_equal(y.to_numpy(), want)


def test_gqa_decode_and_prefill_match_the_c_abi(rt):
    r = rx()
    rng = np.random.default_rng(2)
    b, hq, hkv, lmax, d, s = 2, 8, 2, 96, 128, 20
    kc = rt.buffer(oracle.bf16_bits(rng.standard_normal((b, hkv, lmax, d)).astype(np.float32)),
                   r.DType.BF16)
    vc = rt.buffer(oracle.bf16_bits(rng.standard_normal((b, hkv, lmax, d)).astype(np.float32)),
                   r.DType.BF16)
    q = rt.buffer(oracle.bf16_bits(rng.standard_normal((b, hq, d)).astype(np.float32)), r.DType.BF16)
    lens = rt.buffer(np.array([37, 96], np.int32))
    want = r.grouped_query_attention(rt, q, kc, vc, lens, scale=0.1).to_numpy()
    out = rt.zeros((b, hq, d), r.DType.F32)
    call(rt, "rxw8_xla_gqa_decode", [q, kc, vc, lens, out],
         f"b={b};hq={hq};hkv={hkv};lmax={lmax};d={d};q=bf16;cache=bf16;out=f32;scale=0.1")
    np.testing.assert_array_equal(out.to_numpy(), want)
    qp = rt.buffer(rng.standard_normal((b, s, hq // 2, d)).astype(np.float32))
    starts = rt.buffer(np.array([0, 50], np.int32))
    wantp = r.grouped_query_attention_prefill(rt, qp, kc, vc, starts).to_numpy()
    outp = rt.zeros((b, s, hq // 2, d), r.DType.F32)
    call(rt, "rxw8_xla_gqa_prefill", [qp, kc, vc, starts, outp],
         f"b={b};s={s};hq={hq // 2};hkv={hkv};lmax={lmax};q=f32;out=f32")
    np.testing.assert_array_equal(outp.to_numpy(), wantp)


@pytest.mark.parametrize("opaque", ["m=8;n=640;k=1024;x=f32;y=f32",           # no g
                                    "m=8;n=640;k=1024;g=100;x=f32;y=f32",     # k % g
                                    "m=8;n=640;k=1024;g=128;x=f64;y=f32",     # dtype name
                                    "m=8x;n=640;k=1024;g=128;x=f32;y=f32"])   # number
def test_bad_backend_config_launches_nothing(rt, opaque):
    r = rx()
    rng = np.random.default_rng(3)
    u8, s = oracle.quantize_w8((rng.standard_normal((640, 1024)) * 0.02).astype(np.float32), 128)
    xb, wb, sb = rt.buffer(rng.standard_normal((8, 1024)).astype(np.float32)), rt.buffer(u8), rt.buffer(s)
    y = rt.buffer(np.full((8, 640), 7.0, np.float32))
    call(rt, "rxw8_xla_quantized_linear", [xb, wb, sb, y], opaque)
    assert (y.to_numpy() == 7.0).all()
    assert "backend_config" in r._lib.rxw8_last_error().decode()


# the refused call records nothing, so torch reports the captured graph as empty
@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_each_stream_has_its_own_workspaces_and_none_grows_in_a_capture(rt):
    """The handlers keep one runtime per stream XLA passes. A call whose split
    workspace would have to grow while its stream is being captured (an XLA
    command buffer) fails with FAILED_PRECONDITION and records nothing; the
    same call outside the capture sizes the workspace and matches the C ABI."""
    import torch

    r = rx()
    rng = np.random.default_rng(4)

    def decode_bufs(b, hkv, lmax, fill=None):
        hq, d = 4 * hkv, 128
        kc = rt.buffer(oracle.bf16_bits(rng.standard_normal((b, hkv, lmax, d)).astype(np.float32)),
                       r.DType.BF16)
        vc = rt.buffer(oracle.bf16_bits(rng.standard_normal((b, hkv, lmax, d)).astype(np.float32)),
                       r.DType.BF16)
        q = rt.buffer(rng.standard_normal((b, hq, d)).astype(np.float32))
        lens = rt.buffer(np.full(b, lmax, np.int32))
        out = rt.buffer(np.full((b, hq, d), 7.0, np.float32))
        cfg = f"b={b};hq={hq};hkv={hkv};lmax={lmax};d={d};q=f32;cache=bf16;out=f32"
        return [q, kc, vc, lens, out], cfg

    small, small_cfg = decode_bufs(2, 2, 64)      # one split: no workspace
    big, big_cfg = decode_bufs(2, 2, 4096)        # many splits: partials + counters
    rt.synchronize()
    s = torch.cuda.Stream()

    def call_on(bufs, opaque):
        ptrs = (ctypes.c_void_p * len(bufs))(*[b.ptr for b in bufs])
        text = opaque.encode()
        r._lib.rxw8_xla_gqa_decode(ctypes.c_void_p(s.cuda_stream), ptrs, text, len(text), None)

    call_on(small, small_cfg)  # creates the stream's runtime
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="thread_local"):
        call_on(big, big_cfg)
    assert "captured" in r._lib.rxw8_last_error().decode()
    g.replay()
    torch.cuda.synchronize()
    assert (big[4].to_numpy() == 7.0).all()
    call_on(big, big_cfg)
    s.synchronize()
    want = r.grouped_query_attention(rt, *big[:4]).to_numpy()
    np.testing.assert_array_equal(big[4].to_numpy(), want)


# ---- typed FFI (api_version 4): XLA's call frame, stream from the API table

def ffi_call(rt, name, operands, results, attrs=None):
    import xla_ffi_frames as xf
    api = xf.FakeApi(stream=rt.stream())
    fr = xf.Frame(api, operands, results, attrs)
    err = getattr(rx()._lib, name)(fr.ptr())
    return err, api


def fbuf(b):
    import xla_ffi_frames as xf
    r = rx()
    code = {r.DType.F32: xf.F32, r.DType.BF16: xf.BF16, r.DType.U8: xf.U8, r.DType.I32: xf.S32}
    return (code[b.dtype], list(b.shape), b.ptr)


@pytest.mark.parametrize("xd,compute", [("f32", "bf16"), ("bf16", "bf16"), ("f32", "f32")])
def test_typed_ffi_quantized_linear_matches_the_c_abi(rt, xd, compute):
    r = rx()
    dt = {"f32": r.DType.F32, "bf16": r.DType.BF16}
    rng = np.random.default_rng(11)
    m, n, k, g = 8, 640, 1024, 128
    x = rng.standard_normal((m, k)).astype(np.float32)
    u8, s = oracle.quantize_w8((rng.standard_normal((n, k)) * 0.02).astype(np.float32), g)
    xb = rt.buffer(oracle.bf16_bits(x), r.DType.BF16) if xd == "bf16" else rt.buffer(x)
    wb, sb = rt.buffer(u8), rt.buffer(s)
    want = r.quantized_linear(rt, xb, wb, sb, dt[compute], r.DType.F32).to_numpy()
    y = rt.zeros((m, n), r.DType.F32)
    err, api = ffi_call(rt, "rxw8_xla_ffi_quantized_linear", [fbuf(xb), fbuf(wb), fbuf(sb)],
                        [fbuf(y)], {"compute": compute})
    assert err is None and api.errors == [] and api.stream_calls == 1
    np.testing.assert_array_equal(y.to_numpy(), want)


def test_typed_ffi_attention_matches_the_c_abi(rt):
    r = rx()
    rng = np.random.default_rng(12)
    b, hq, hkv, lmax, d, s = 2, 8, 2, 96, 128, 20
    kc = rt.buffer(oracle.bf16_bits(rng.standard_normal((b, hkv, lmax, d)).astype(np.float32)),
                   r.DType.BF16)
    vc = rt.buffer(oracle.bf16_bits(rng.standard_normal((b, hkv, lmax, d)).astype(np.float32)),
                   r.DType.BF16)
    q = rt.buffer(oracle.bf16_bits(rng.standard_normal((b, hq, d)).astype(np.float32)), r.DType.BF16)
    lens = rt.buffer(np.array([37, 96], np.int32))
    want = r.grouped_query_attention(rt, q, kc, vc, lens, scale=0.1).to_numpy()
    out = rt.zeros((b, hq, d), r.DType.F32)
    err, api = ffi_call(rt, "rxw8_xla_ffi_gqa_decode", [fbuf(q), fbuf(kc), fbuf(vc), fbuf(lens)],
                        [fbuf(out)], {"scale": 0.1})
    assert err is None and api.errors == []
    np.testing.assert_array_equal(out.to_numpy(), want)
    qp = rt.buffer(oracle.bf16_bits(rng.standard_normal((b, s, hq, d)).astype(np.float32)),
                   r.DType.BF16)
    starts = rt.buffer(np.array([0, 40], np.int32))
    want = r.grouped_query_attention_prefill(rt, qp, kc, vc, starts).to_numpy()
    outp = rt.zeros((b, s, hq, d), r.DType.F32)
    err, api = ffi_call(rt, "rxw8_xla_ffi_gqa_prefill", [fbuf(qp), fbuf(kc), fbuf(vc), fbuf(starts)],
                        [fbuf(outp)])
    assert err is None and api.errors == []
    np.testing.assert_array_equal(outp.to_numpy(), want)


def test_typed_ffi_shape_error_leaves_the_result_untouched(rt):
    r = rx()
    x = rt.buffer(np.ones((4, 64), np.float32))
    w = rt.buffer(np.full((32, 64), 130, np.uint8))
    s = rt.buffer(np.ones((32, 1), np.float32))
    y = rt.buffer(np.full((4, 33), 7.0, np.float32))  # N mismatch
    err, api = ffi_call(rt, "rxw8_xla_ffi_quantized_linear", [fbuf(x), fbuf(w), fbuf(s)], [fbuf(y)])
    assert err is not None and api.errors and api.errors[0][0] == int(r.Status.INVALID_ARGUMENT)
    rt.synchronize()
    np.testing.assert_array_equal(y.to_numpy(), 7.0)
