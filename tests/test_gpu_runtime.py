"""Runtime behaviour on the GPU that the op tests do not see on their own:
sharing a process, device and stream with PyTorch."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def test_kernel_lookups_leave_no_hip_error_for_torch(rt):
    """Every code object's kernels are looked up (GEMV, misc, attention, GEMM),
    then torch allocates and launches: no HIP error may be left pending for it."""
    import torch
    import rxla_amd as rx

    torch.cuda.synchronize()
    rng = np.random.default_rng(1)
    x = rng.standard_normal((130, 256)).astype(np.float32)
    u8, s = oracle.quantize_w8((rng.standard_normal((128, 256)) * 0.02).astype(np.float32), 256)
    rx.quantized_linear(rt, rt.buffer(x[:4]), rt.buffer(u8), rt.buffer(s))   # GEMV
    rx.quantized_linear(rt, rt.buffer(x), rt.buffer(u8), rt.buffer(s))       # GEMM
    rx.dequantize(rt, rt.buffer(u8), rt.buffer(s))                           # misc module
    q = rng.standard_normal((1, 4, 128)).astype(np.float32)
    kc = oracle.bf16_bits(rng.standard_normal((1, 2, 16, 128)).astype(np.float32))
    rx.grouped_query_attention(rt, rt.buffer(q), rt.buffer(kc, rx.DType.BF16),
                               rt.buffer(kc, rx.DType.BF16), rt.buffer(np.array([5], np.int32)))
    rt.synchronize()
    t = torch.ones(1024, device="cuda") * 3  # raises if a HIP error is pending
    torch.cuda.synchronize()
    assert float(t.sum()) == 3072.0


def test_wrapped_torch_tensors_on_torch_stream(rt):
    """rxw8 writes into torch-owned memory on torch's stream; ordering follows
    that stream."""
    import torch
    import rxla_amd as rx

    stream = torch.cuda.Stream()
    rt.set_stream(stream.cuda_stream)
    try:
        rng = np.random.default_rng(2)
        x = rng.standard_normal((200, 512)).astype(np.float32)
        u8, s = oracle.quantize_w8((rng.standard_normal((256, 512)) * 0.02).astype(np.float32), 128)
        with torch.cuda.stream(stream):
            xt = torch.from_numpy(x).cuda()
            ut = torch.from_numpy(u8).cuda()
            st = torch.from_numpy(s).cuda()
            yt = torch.full((200, 256), float("nan"), device="cuda")
        rx.quantized_linear(rt, rt.wrap_tensor(xt), rt.wrap_tensor(ut), rt.wrap_tensor(st),
                            out=rt.wrap_tensor(yt))
        with torch.cuda.stream(stream):
            y = yt.cpu()
        ref = oracle.quantized_linear(x, u8, s)
        assert float(np.abs(y.numpy() - ref).max() / np.abs(ref).max()) <= 1e-2
    finally:
        rt.set_stream(0)
