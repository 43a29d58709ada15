"""The typed-FFI handlers (rxw8_xla_ffi_*, HLO api_version 4) on the CPU:
they answer XLA's metadata query with FFI API 0.1, do nothing outside the
execute stage, and reject malformed call frames through the frame's own
XLA_FFI_Error_Create before they ask for a stream or touch a device."""
import ctypes

import pytest

import xla_ffi_frames as xf

HANDLERS = ["rxw8_xla_ffi_quantized_linear", "rxw8_xla_ffi_gqa_decode", "rxw8_xla_ffi_gqa_prefill"]


def lib():
    import rxla_amd
    return rxla_amd._lib


def linear_frame(api, **kw):
    ops = kw.pop("ops", [(xf.F32, [8, 64], 0x1000), (xf.U8, [32, 64], 0x2000),
                         (xf.F32, [32, 1], 0x3000)])
    res = kw.pop("res", [(xf.F32, [8, 32], 0x4000)])
    return xf.Frame(api, ops, res, **kw)


@pytest.mark.parametrize("name", HANDLERS)
def test_metadata_query_reports_api_0_1(name):
    api = xf.FakeApi()
    meta = xf.Metadata(ctypes.sizeof(xf.Metadata), xf.ApiVersion(ctypes.sizeof(xf.ApiVersion), None, -1, -1), 77)
    ext = xf.MetadataExtension(xf.ExtensionBase(ctypes.sizeof(xf.MetadataExtension), 1, None),
                               ctypes.pointer(meta))
    fr = xf.Frame(api, [], [])
    fr.frame.extension_start = ctypes.addressof(ext)
    assert getattr(lib(), name)(fr.ptr()) is None
    assert (meta.api_version.major_version, meta.api_version.minor_version, meta.traits) == (0, 1, 0)
    assert api.errors == [] and api.stream_calls == 0


def test_stages_other_than_execute_do_nothing():
    api = xf.FakeApi()
    fr = linear_frame(api, stage=xf.INSTANTIATE)
    assert lib().rxw8_xla_ffi_quantized_linear(fr.ptr()) is None
    assert api.errors == [] and api.stream_calls == 0


@pytest.mark.parametrize("case", ["operand_count", "dtype", "attr_kind", "attr_value", "small_frame"])
def test_malformed_frames_fail_before_device_work(case):
    api = xf.FakeApi()
    if case == "operand_count":
        fr = linear_frame(api, ops=[(xf.F32, [8, 64], 0x1000), (xf.U8, [32, 64], 0x2000)])
    elif case == "dtype":
        fr = linear_frame(api, res=[(xf.F64, [8, 32], 0x4000)])
    elif case == "attr_kind":
        fr = linear_frame(api, attrs={"compute": 1.0})
    elif case == "attr_value":
        fr = linear_frame(api, attrs={"compute": "f64"})
    else:
        fr = linear_frame(api)
        fr.frame.struct_size = 64
    err = lib().rxw8_xla_ffi_quantized_linear(fr.ptr())
    assert err == xf.FakeApi.ERROR
    assert len(api.errors) == 1 and api.errors[0][0] == 3, api.errors  # INVALID_ARGUMENT
    assert api.errors[0][1].startswith("rxw8_quantized_linear: ")
    assert api.stream_calls == 0


def test_decode_scale_attribute_must_be_a_float_scalar():
    api = xf.FakeApi()
    ops = [(xf.BF16, [2, 8, 128], 1), (xf.BF16, [2, 2, 64, 128], 2), (xf.BF16, [2, 2, 64, 128], 3),
           (xf.S32, [2], 4)]
    fr = xf.Frame(api, ops, [(xf.F32, [2, 8, 128], 5)], attrs={"scale": "0.1"})
    assert lib().rxw8_xla_ffi_gqa_decode(fr.ptr()) == xf.FakeApi.ERROR
    assert api.errors[0][0] == 3 and "scale" in api.errors[0][1]
    assert api.stream_calls == 0
