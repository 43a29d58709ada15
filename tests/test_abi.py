"""CPU checks of the C ABI: the library loads, exports every symbol that
include/rxw8.h declares, and reports errors with the PJRT numbering -- all
without a GPU (no compute call is made)."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "rxw8.h")
LIB = os.path.join(ROOT, "rxla_amd", "librxw8.so")


def _ensure_built():
    if not os.path.exists(LIB):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "rxla_amd", "csrc")], check=True)


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rxw8_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_op_surface():
    syms = declared_symbols()
    for name in ("rxw8_quantized_linear", "rxw8_gqa_decode", "rxw8_kv_update_at",
                 "rxw8_decoder_bind_parameter", "rxw8_decoder_forward", "rxw8_dequantize"):
        assert name in syms


def test_library_exports_every_declared_symbol():
    _ensure_built()
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (rxw8_\w+)", out))
    missing = [s for s in declared_symbols() if s not in exported]
    assert not missing, missing
    import rxla_amd._ffi as ffi
    assert sorted(ffi.EXPORTS) == declared_symbols()


def test_library_has_no_cpu_compute_path():
    """The product library must not link the oracle or carry a CPU fallback."""
    _ensure_built()
    out = subprocess.run(["nm", "-D", LIB], capture_output=True, text=True, check=True).stdout
    assert "rxo_" not in out
    needed = subprocess.run(["readelf", "-d", LIB], capture_output=True, text=True).stdout
    assert "librxw8_oracle" not in needed and "libamdhip64" in needed


def test_status_codes_and_errors_without_gpu():
    _ensure_built()
    import rxla_amd as rx

    lib = rx._lib
    assert lib.rxw8_abi_version() == 1
    assert [int(s) for s in rx.Status][:4] == [0, 1, 2, 3]
    assert rx.Status.UNAUTHENTICATED == 16
    retry = {s for s in rx.Status if lib.rxw8_status_is_retryable(int(s))}
    assert retry == {rx.Status.CANCELLED, rx.Status.DEADLINE_EXCEEDED,
                     rx.Status.RESOURCE_EXHAUSTED, rx.Status.ABORTED, rx.Status.UNAVAILABLE}
    # NULL handles are rejected before anything touches a device
    assert lib.rxw8_runtime_create(0, None) == rx.Status.INVALID_ARGUMENT
    assert b"NULL" in lib.rxw8_last_error()
    assert lib.rxw8_buffer_release(None) == rx.Status.INVALID_ARGUMENT
    assert lib.rxw8_quantized_linear(None, None, None, None, 4, 5, None) == rx.Status.INVALID_ARGUMENT


def test_buffer_shapes_are_checked_before_anything_else():
    """Buffer shapes whose element count or byte size overflows int64 are
    rejected with INVALID_ARGUMENT before any handle or device is touched (the
    shape is checked first, so a NULL runtime still reports the shape)."""
    _ensure_built()
    import rxla_amd as rx

    lib = rx._lib
    I64 = ctypes.c_int64
    out = ctypes.c_void_p()
    cases = [((1 << 40, 1 << 30, 1 << 2), b"element count"),  # 2^72 elements
             ((1 << 61, 1), b"byte size"),                      # 2^61 elements x 4 bytes
             ((-1, 4), b"negative")]
    for dims, what in cases:
        d = (I64 * len(dims))(*dims)
        for call in (lambda: lib.rxw8_buffer_create(None, int(rx.DType.F32), d, len(dims), out),
                     lambda: lib.rxw8_buffer_from_host(None, int(rx.DType.F32), d, len(dims), None, out),
                     lambda: lib.rxw8_buffer_wrap(None, int(rx.DType.F32), d, len(dims), None, out)):
            assert call() == rx.Status.INVALID_ARGUMENT
            assert what in lib.rxw8_last_error(), (dims, lib.rxw8_last_error())
    # an empty shape never overflows: its other dims are not multiplied
    d = (I64 * 3)(0, 1 << 62, 1 << 62)
    assert lib.rxw8_buffer_create(None, int(rx.DType.F32), d, 3, out) == rx.Status.INVALID_ARGUMENT
    assert b"NULL" in lib.rxw8_last_error()


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_runtime_create_without_device_is_failed_precondition():
    _ensure_built()
    import rxla_amd as rx

    with pytest.raises(rx.Error) as e:
        rx.Runtime(0)
    assert e.value.code == rx.Status.FAILED_PRECONDITION
    assert not e.value.is_retryable


@pytest.mark.parametrize("order", ["rxla_amd,torch", "torch,rxla_amd"])
def test_one_hip_runtime_with_torch_in_either_import_order(order):
    """librxw8.so and PyTorch must share one HIP/HSA runtime whichever is
    imported first (two runtimes in one process do not see the GPU twice)."""
    _ensure_built()
    code = (f"import sys; sys.path.insert(0, {ROOT!r})\n"
            f"import {order.split(',')[0]}\nimport {order.split(',')[1]}\n"
            "maps = open('/proc/self/maps').read().splitlines()\n"
            "hip = {l.split()[-1] for l in maps if 'libamdhip64' in l}\n"
            "hsa = {l.split()[-1] for l in maps if 'libhsa-runtime64' in l}\n"
            "print(len(hip), len(hsa))\n")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                         timeout=300, check=True).stdout.split()
    assert out[-2:] == ["1", "1"], out


def test_every_kernel_routes_to_its_code_object():
    """runtime.cpp looks a kernel up only in the code object its name prefix
    selects; every kernel of every source must land in the object built from
    that source (a miss would surface only as a launch error on the GPU)."""
    csrc = os.path.join(ROOT, "rxla_amd", "csrc")
    make = open(os.path.join(csrc, "Makefile")).read()
    sources = dict(re.findall(r"^CO_(\w+)\s*:=\s*(\S+)", make, flags=re.M))
    rt_src = open(os.path.join(csrc, "runtime.cpp")).read()
    order = re.findall(r'\{"(\w+)", rxw8_co_\w+, rxw8_co_\w+_end\}', rt_src)
    routes = [(p, int(i)) for p, i in re.findall(r'\{"(rxw8_\w+)", (\d+)\}', rt_src)]
    assert sorted(order) == sorted(sources) and routes

    def module_of(name):
        for prefix, idx in routes:
            if name.startswith(prefix):
                return order[idx]
        return None

    seen = 0
    for co, src in sources.items():
        text = open(os.path.join(csrc, src)).read()
        # (macro-generated GEMV names are checked by prefix below)
        names = re.findall(r'extern "C" __global__ void\s+(?:__launch_bounds__\([^)]*\)\s+)?'
                           r'(rxw8_\w+)\(', text)
        for name in names:
            assert module_of(name) == co, (name, co, module_of(name))
            seen += 1
    launched = set()
    for f in ("ops.cpp", "decoder.cpp"):
        launched |= set(re.findall(r'"(rxw8_[a-z0-9_]+?)(?:%|")', open(os.path.join(csrc, f)).read()))
    for name in launched:
        if name.startswith(("rxw8_gemv_w8", "rxw8_gemv_bf16")):
            continue  # formatted names, checked by prefix below
        assert module_of(name) is not None, name
    assert module_of("rxw8_gemv_w8_pk_mb1_rw1_u4") == "gemv"
    assert module_of("rxw8_gemv_rc_w8_pk_mb1_rw1_u4_w16_xg_rn") == "gemv_rc"
    assert seen > 10
