"""Call frames of XLA's FFI C API (xla/ffi/api/c_api.h, FFI API 0.1) built
with ctypes, as XLA hands them to a typed (api_version 4) custom-call handler,
plus a stand-in for the API table whose XLA_FFI_Error_Create and
XLA_FFI_Stream_Get record their calls. Test infrastructure only."""
import ctypes
from ctypes import (CFUNCTYPE, POINTER, Structure, c_char_p, c_float, c_int, c_int64, c_size_t,
                    c_uint32, c_void_p)

# XLA_FFI_DataType (= xla::PrimitiveType)
S32, U8, F16, F32, F64, BF16, S64 = 4, 6, 10, 11, 12, 16, 5
EXECUTE, INSTANTIATE = 3, 0
ATTR_SCALAR, ATTR_STRING = 3, 4


class ExtensionBase(Structure):
    _fields_ = [("struct_size", c_size_t), ("type", c_int), ("next", c_void_p)]


class ApiVersion(Structure):
    _fields_ = [("struct_size", c_size_t), ("extension_start", c_void_p),
                ("major_version", c_int), ("minor_version", c_int)]


class ErrorCreateArgs(Structure):
    _fields_ = [("struct_size", c_size_t), ("extension_start", c_void_p), ("message", c_char_p),
                ("errc", c_int)]


class StreamGetArgs(Structure):
    _fields_ = [("struct_size", c_size_t), ("extension_start", c_void_p), ("ctx", c_void_p),
                ("stream", c_void_p)]


ERROR_CREATE = CFUNCTYPE(c_void_p, POINTER(ErrorCreateArgs))
STREAM_GET = CFUNCTYPE(c_void_p, POINTER(StreamGetArgs))


class Api(Structure):
    _fields_ = [("struct_size", c_size_t), ("extension_start", c_void_p),
                ("api_version", ApiVersion), ("internal_api", c_void_p),
                ("error_create", ERROR_CREATE), ("error_get_message", c_void_p),
                ("error_destroy", c_void_p), ("handler_register", c_void_p),
                ("stream_get", STREAM_GET)]


class Buffer(Structure):
    _fields_ = [("struct_size", c_size_t), ("extension_start", c_void_p), ("dtype", c_int),
                ("data", c_void_p), ("rank", c_int64), ("dims", POINTER(c_int64))]


class Args(Structure):
    _fields_ = [("struct_size", c_size_t), ("extension_start", c_void_p), ("size", c_int64),
                ("types", POINTER(c_int)), ("args", POINTER(c_void_p))]


class ByteSpan(Structure):
    _fields_ = [("ptr", c_char_p), ("len", c_size_t)]


class Scalar(Structure):
    _fields_ = [("dtype", c_int), ("value", c_void_p)]


class Attrs(Structure):
    _fields_ = [("struct_size", c_size_t), ("extension_start", c_void_p), ("size", c_int64),
                ("types", POINTER(c_int)), ("names", POINTER(POINTER(ByteSpan))),
                ("attrs", POINTER(c_void_p))]


class CallFrame(Structure):
    _fields_ = [("struct_size", c_size_t), ("extension_start", c_void_p), ("api", POINTER(Api)),
                ("ctx", c_void_p), ("stage", c_int), ("args", Args), ("rets", Args),
                ("attrs", Attrs), ("future", c_void_p)]


class Metadata(Structure):
    _fields_ = [("struct_size", c_size_t), ("api_version", ApiVersion), ("traits", c_uint32)]


class MetadataExtension(Structure):
    _fields_ = [("extension_base", ExtensionBase), ("metadata", POINTER(Metadata))]


class FakeApi:
    """An XLA_FFI_Api table whose Error_Create records (code, message) and
    returns a non-null handle, and whose Stream_Get returns `stream`."""

    ERROR = 0x5A5A0

    def __init__(self, stream=0):
        self.errors = []
        self.stream = stream
        self.stream_calls = 0

        def error_create(args):
            self.errors.append((args.contents.errc, args.contents.message.decode()))
            return self.ERROR

        def stream_get(args):
            self.stream_calls += 1
            args.contents.stream = self.stream
            return None

        self._cb = (ERROR_CREATE(error_create), STREAM_GET(stream_get))
        self.api = Api(ctypes.sizeof(Api), None, ApiVersion(ctypes.sizeof(ApiVersion), None, 0, 1),
                       None, self._cb[0], None, None, None, self._cb[1])


class Frame:
    """A call frame of buffers (dtype, dims, device pointer) for operands and
    results, and attributes: float -> F32 scalar, str -> string."""

    def __init__(self, api, operands, results, attrs=None, stage=EXECUTE):
        self._keep = []
        self.frame = CallFrame()
        self.frame.struct_size = ctypes.sizeof(CallFrame)
        self.frame.api = ctypes.pointer(api.api)
        self.frame.ctx = 0xC0FFEE
        self.frame.stage = stage
        self.frame.args = self._args(operands)
        self.frame.rets = self._args(results)
        self.frame.attrs = self._attrs(attrs or {})

    def _args(self, bufs):
        n = len(bufs)
        types = (c_int * n)(*([1] * n))
        ptrs = (c_void_p * n)()
        for i, (dtype, dims, ptr) in enumerate(bufs):
            d = (c_int64 * len(dims))(*dims)
            b = Buffer(ctypes.sizeof(Buffer), None, dtype, ptr, len(dims), d)
            self._keep += [d, b]
            ptrs[i] = ctypes.addressof(b)
        self._keep += [types, ptrs]
        return Args(ctypes.sizeof(Args), None, n, types, ptrs)

    def _attrs(self, attrs):
        n = len(attrs)
        types = (c_int * max(n, 1))()
        names = (POINTER(ByteSpan) * max(n, 1))()
        vals = (c_void_p * max(n, 1))()
        for i, (k, v) in enumerate(attrs.items()):
            key = k.encode()
            span = ByteSpan(key, len(key))
            names[i] = ctypes.pointer(span)
            if isinstance(v, str):
                raw = v.encode()
                val = ByteSpan(raw, len(raw))
                types[i] = ATTR_STRING
                self._keep += [raw]
            else:
                f = c_float(v)
                val = Scalar(F32, ctypes.addressof(f))
                types[i] = ATTR_SCALAR
                self._keep += [f]
            vals[i] = ctypes.addressof(val)
            self._keep += [key, span, val]
        self._keep += [types, names, vals]
        return Attrs(ctypes.sizeof(Attrs), None, n, types, names, vals)

    def ptr(self):
        return ctypes.addressof(self.frame)
