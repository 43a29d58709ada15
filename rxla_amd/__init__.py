"""rxla_amd: MI355X-native (gfx950) W8A16 decode/prefill hot path of RXLA.

Python host mirror of the C ABI in ``include/rxw8.h`` (``librxw8.so``). The
names follow the reference's operator surface:

* ``QuantizedLinear(out_features, group_size).apply(x, weight, scale)`` --
  ``rxla_nn::QuantizedLinear`` (crates/rxla-nn/src/layers.rs:231-298)
* ``grouped_query_attention(q, k_cache, v_cache, lens, mask, scale)`` --
  ``Tensor::grouped_query_attention`` (crates/rxla-core/src/attention.rs:83-135)
  in its decode form over a contiguous per-sequence cache
* ``KvCache.update_at / update_at_checked`` -- crates/rxla-core/src/kv_cache.rs:53-111
* ``DecoderModel.compile().bind_parameters(...).run(...)`` --
  ``AppliedModel::compile`` / ``CompiledModel::bind_parameters`` / ``BoundModel::run``
  (crates/rxla-nn/src/applied.rs:135-239,808-815)

Errors raise :class:`Error` carrying the PJRT-numbered status code
(vendor/xla/pjrt/c/pjrt_c_api.h:168-186). Everything runs on the gfx950
kernels; nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes
import enum
import os
from ctypes import POINTER, byref, c_float, c_int, c_int32, c_int64, c_void_p

import numpy as np

from . import _ffi

_lib = _ffi.load()


class Status(enum.IntEnum):
    OK = 0
    CANCELLED = 1
    UNKNOWN = 2
    INVALID_ARGUMENT = 3
    DEADLINE_EXCEEDED = 4
    NOT_FOUND = 5
    ALREADY_EXISTS = 6
    PERMISSION_DENIED = 7
    RESOURCE_EXHAUSTED = 8
    FAILED_PRECONDITION = 9
    ABORTED = 10
    OUT_OF_RANGE = 11
    UNIMPLEMENTED = 12
    INTERNAL = 13
    UNAVAILABLE = 14
    DATA_LOSS = 15
    UNAUTHENTICATED = 16


class DType(enum.IntEnum):
    U8 = 1
    I32 = 2
    F16 = 3
    BF16 = 4
    F32 = 5


_NP = {DType.U8: np.uint8, DType.I32: np.int32, DType.F16: np.float16,
       DType.BF16: np.uint16, DType.F32: np.float32}
_FROM_NP = {np.dtype(np.uint8): DType.U8, np.dtype(np.int32): DType.I32,
            np.dtype(np.float16): DType.F16, np.dtype(np.float32): DType.F32}


class Error(RuntimeError):
    """A failed rxw8 call (mirrors rxla_pjrt::Error::Pjrt{code, message})."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{Status(code).name if code in Status._value2member_map_ else code}: "
                         f"{message}")
        self.code = Status(code) if code in Status._value2member_map_ else code
        self.message = message

    @property
    def is_retryable(self) -> bool:
        return bool(_lib.rxw8_status_is_retryable(int(self.code)))


def _check(rc: int):
    if rc != 0:
        raise Error(rc, _lib.rxw8_last_error().decode("utf-8", "replace"))


def _dims(shape):
    arr = (c_int64 * max(1, len(shape)))(*[int(d) for d in shape])
    return arr, len(shape)


class Runtime:
    """One HIP device + stream with the gfx950 kernels loaded (Client::load)."""

    def __init__(self, device: int = 0):
        h = c_void_p()
        _check(_lib.rxw8_runtime_create(int(device), byref(h)))
        self._h = h

    @property
    def handle(self):
        return self._h

    def close(self):
        if self._h:
            _check(_lib.rxw8_runtime_destroy(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self):
        _check(_lib.rxw8_runtime_synchronize(self._h))

    def set_stream(self, stream_ptr):
        _check(_lib.rxw8_runtime_set_stream(self._h, c_void_p(stream_ptr or None)))

    def stream(self) -> int:
        s = c_void_p()
        _check(_lib.rxw8_runtime_stream(self._h, byref(s)))
        return s.value or 0

    def device_info(self):
        cus = c_int()
        name = ctypes.create_string_buffer(256)
        _check(_lib.rxw8_runtime_device_info(self._h, byref(cus), name, 256))
        return {"compute_units": cus.value, "name": name.value.decode()}

    # ---- buffers ----------------------------------------------------------------
    def buffer(self, array, dtype: DType | None = None) -> "Buffer":
        """Upload a numpy array (bf16 data is passed as uint16 bit patterns
        with dtype=DType.BF16)."""
        a = np.ascontiguousarray(array)
        if dtype is None:
            dtype = _FROM_NP.get(a.dtype)
            if dtype is None:
                raise TypeError(f"no rxw8 dtype for numpy {a.dtype}")
        a = np.ascontiguousarray(a, dtype=_NP[DType(dtype)])
        dims, rank = _dims(a.shape)
        h = c_void_p()
        _check(_lib.rxw8_buffer_from_host(self._h, int(dtype), dims, rank,
                                          a.ctypes.data_as(c_void_p), byref(h)))
        return Buffer(h)

    def zeros(self, shape, dtype: DType) -> "Buffer":
        dims, rank = _dims(shape)
        h = c_void_p()
        _check(_lib.rxw8_buffer_create(self._h, int(dtype), dims, rank, byref(h)))
        return Buffer(h)

    def wrap(self, ptr: int, shape, dtype: DType) -> "Buffer":
        """Non-owning view of device memory (e.g. ``tensor.data_ptr()``)."""
        dims, rank = _dims(shape)
        h = c_void_p()
        _check(_lib.rxw8_buffer_wrap(self._h, int(dtype), dims, rank, c_void_p(ptr), byref(h)))
        return Buffer(h)

    def wrap_tensor(self, t) -> "Buffer":
        import torch
        m = {torch.uint8: DType.U8, torch.int32: DType.I32, torch.float16: DType.F16,
             torch.bfloat16: DType.BF16, torch.float32: DType.F32}
        if not t.is_contiguous():
            raise ValueError("wrap_tensor needs a contiguous tensor")
        return self.wrap(t.data_ptr(), tuple(t.shape), m[t.dtype])


class Buffer:
    """Refcounted device buffer (rxla_pjrt::Buffer)."""

    def __init__(self, handle):
        self._h = handle

    @property
    def handle(self):
        return self._h

    def release(self):
        if self._h:
            _check(_lib.rxw8_buffer_release(self._h))
            self._h = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    @property
    def dtype(self) -> DType:
        d = c_int()
        _check(_lib.rxw8_buffer_dtype(self._h, byref(d)))
        return DType(d.value)

    @property
    def shape(self):
        dims = (c_int64 * 8)()
        r = c_int()
        _check(_lib.rxw8_buffer_dims(self._h, dims, byref(r)))
        return tuple(dims[i] for i in range(r.value))

    @property
    def ptr(self) -> int:
        p = c_void_p()
        _check(_lib.rxw8_buffer_device_ptr(self._h, byref(p)))
        return p.value or 0

    def _keep(self, *owners):
        """Keep `owners` (the buffers a view's memory belongs to) alive with it."""
        self._owners = owners
        return self

    def to_numpy(self) -> np.ndarray:
        """Blocking download (Buffer::to_vec). BF16 comes back as uint16 bits."""
        out = np.empty(self.shape, _NP[self.dtype])
        _check(_lib.rxw8_buffer_to_host(self._h, out.ctypes.data_as(c_void_p), out.nbytes))
        return out

    def copy_from(self, array):
        a = np.ascontiguousarray(array, dtype=_NP[self.dtype])
        _check(_lib.rxw8_buffer_copy_from_host(self._h, a.ctypes.data_as(c_void_p), a.nbytes))


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- ops ------------------------------------------------------------------------

def quantize_w8(rt: Runtime, w: Buffer, group_size: int) -> tuple[Buffer, Buffer]:
    """The W8 encoder (benchmarks/quantize_qwen3_5_w8.py:27-44) on the device:
    F32|BF16 [N, K] -> (U8 [N, K] codes = int8 + 128, F32 [N, K/group] scales)."""
    hw, hs = c_void_p(), c_void_p()
    _check(_lib.rxw8_quantize_w8(rt.handle, w.handle, int(group_size), byref(hw), byref(hs)))
    return Buffer(hw), Buffer(hs)


def dequantize(rt: Runtime, weight: Buffer, scale: Buffer, out_dtype=DType.F32) -> Buffer:
    h = c_void_p()
    _check(_lib.rxw8_dequantize(rt.handle, weight.handle, scale.handle, int(out_dtype), byref(h)))
    return Buffer(h)


def pack_weight(rt: Runtime, weight: Buffer) -> Buffer:
    """Tiled copy of a U8 [N,K] or BF16 [N,K] weight for the packed GEMV path."""
    h = c_void_p()
    _check(_lib.rxw8_pack_weight(rt.handle, weight.handle, byref(h)))
    return Buffer(h)


def quantized_linear(rt: Runtime, x: Buffer, weight: Buffer, scale: Buffer,
                     compute_dtype=DType.BF16, out_dtype=DType.F32, out: Buffer | None = None):
    if out is not None:
        _check(_lib.rxw8_quantized_linear_into(rt.handle, x.handle, weight.handle, scale.handle,
                                               int(compute_dtype), out.handle))
        return out
    h = c_void_p()
    _check(_lib.rxw8_quantized_linear(rt.handle, x.handle, weight.handle, scale.handle,
                                      int(compute_dtype), int(out_dtype), byref(h)))
    return Buffer(h)


def quantized_linear_group(rt: Runtime, xs, weights, scales, outs):
    """Independent W8A16 linears (BF16 compute) in one grouped launch per class
    of rows: outs[i] receives quantized_linear(xs[i], weights[i], scales[i])
    (rxw8_quantized_linear_group)."""
    n = len(xs)
    if not (len(weights) == len(scales) == len(outs) == n):
        raise ValueError("quantized_linear_group: xs, weights, scales and outs differ in length")
    arr = lambda bufs: (c_void_p * n)(*[b.handle for b in bufs])  # noqa: E731
    _check(_lib.rxw8_quantized_linear_group(rt.handle, n, arr(xs), arr(weights), arr(scales),
                                            arr(outs)))
    return outs


def linear_bf16(rt: Runtime, x: Buffer, weight: Buffer, out_dtype=DType.F32,
                out: Buffer | None = None):
    if out is not None:
        _check(_lib.rxw8_linear_bf16_into(rt.handle, x.handle, weight.handle, out.handle))
        return out
    h = c_void_p()
    _check(_lib.rxw8_linear_bf16(rt.handle, x.handle, weight.handle, int(out_dtype), byref(h)))
    return Buffer(h)


class QuantizedLinear:
    """``rxla_nn::QuantizedLinear::new(out_features, group_size)`` applied to
    explicit ``weight`` (U8 [out, in]) and ``scale`` (F32 [out, in/G])."""

    def __init__(self, out_features: int, group_size: int, compute_dtype=DType.BF16):
        self.out_features = int(out_features)
        self.group_size = int(group_size)
        self.compute_dtype = compute_dtype

    def apply(self, rt: Runtime, x: Buffer, weight: Buffer, scale: Buffer,
              out_dtype=DType.F32) -> Buffer:
        if self.out_features <= 0 or self.group_size <= 0:
            raise Error(Status.INVALID_ARGUMENT,
                        "QuantizedLinear requires positive widths and a group size dividing "
                        "the input width")
        ws, ss = weight.shape, scale.shape
        in_features = x.shape[-1] if x.shape else 0
        out = ws[0] * 16 if len(ws) == 3 else ws[0]  # packed [N/16, K/64, 1024]
        if (out != self.out_features or in_features % self.group_size
                or ss != (self.out_features, in_features // self.group_size)):
            raise Error(Status.INVALID_ARGUMENT,
                        f"QuantizedLinear({self.out_features}, {self.group_size}) does not "
                        f"match weight {ws} / scale {ss} for input width {in_features}")
        return quantized_linear(rt, x, weight, scale, self.compute_dtype, out_dtype)


def grouped_query_attention(rt: Runtime, q: Buffer, k_cache: Buffer, v_cache: Buffer,
                            lens: Buffer, mask: Buffer | None = None, scale: float | None = None,
                            out_dtype=DType.F32, out: Buffer | None = None) -> Buffer:
    s = 0.0 if scale is None else float(scale)
    m = mask.handle if mask is not None else None
    if out is not None:
        _check(_lib.rxw8_gqa_decode_into(rt.handle, q.handle, k_cache.handle, v_cache.handle,
                                         lens.handle, m, ctypes.c_float(s), out.handle))
        return out
    h = c_void_p()
    _check(_lib.rxw8_gqa_decode(rt.handle, q.handle, k_cache.handle, v_cache.handle,
                                lens.handle, m, ctypes.c_float(s), int(out_dtype), byref(h)))
    return Buffer(h)


def gqa_attention(rt: Runtime, q: Buffer, k: Buffer, v: Buffer, mask: Buffer | None = None,
                  scale: float | None = None, out: Buffer | None = None) -> Buffer:
    """``Tensor::grouped_query_attention(k, v, mask, scale)`` (attention.rs:83-135)
    for any query count: q [..., Hq, Sq, D], k/v [..., Hkv, Sk, D|Dv] F32, an
    additive F32 mask broadcastable to [..., Hq, Sq, Sk]; F32 [..., Hq, Sq, Dv]."""
    sp = byref(c_float(scale)) if scale is not None else None
    m = mask.handle if mask is not None else None
    if out is not None:
        _check(_lib.rxw8_gqa_attention_into(rt.handle, q.handle, k.handle, v.handle, m, sp,
                                            out.handle))
        return out
    h = c_void_p()
    _check(_lib.rxw8_gqa_attention(rt.handle, q.handle, k.handle, v.handle, m, sp, byref(h)))
    return Buffer(h)


def scaled_dot_product_attention(rt: Runtime, q: Buffer, k: Buffer, v: Buffer,
                                 mask: Buffer | None = None, scale: float | None = None) -> Buffer:
    """``Tensor::scaled_dot_product_attention`` (attention.rs:150-252) on equal
    batch prefixes: softmax(q k^T * scale + mask) v, as one-head GQA (q
    [..., Sq, D], k [..., Sk, D], v [..., Sk, Dv], rank >= 2)."""
    def with_head(b):
        s = b.shape
        return rt.wrap(b.ptr, s[:-2] + (1,) + s[-2:], b.dtype)
    qh, kh, vh = with_head(q), with_head(k), with_head(v)
    # a mask with batch dims gains the same head axis, so its batch dims stay aligned
    mh = with_head(mask) if mask is not None and len(mask.shape) >= 3 else mask
    o = gqa_attention(rt, qh, kh, vh, mh, scale)
    return rt.wrap(o.ptr, q.shape[:-1] + (v.shape[-1],), o.dtype)._keep(o)


def causal_attention_mask(rt: Runtime, query_positions: Buffer, key_positions: Buffer) -> Buffer:
    """``Tensor::causal_attention_mask`` (attention.rs:14-32): F32 [Q, K], 0 iff
    key_positions[j] <= query_positions[i] (signed I32), else -inf."""
    h = c_void_p()
    _check(_lib.rxw8_causal_attention_mask(rt.handle, query_positions.handle,
                                           key_positions.handle, byref(h)))
    return Buffer(h)


def causal_attention_mask_static(rt: Runtime, queries: int, keys: int, query_offset: int) -> Buffer:
    """``Graph::causal_attention_mask(queries, keys, query_offset)``
    (attention.rs:45-67): key j visible to row i iff j <= query_offset + i;
    counts and offset nonnegative and I32-representable, as the reference checks."""
    imax = 2 ** 31 - 1
    if (queries < 0 or keys < 0 or keys > imax + 1 or query_offset < 0 or query_offset > imax
            or queries > imax + 1 - query_offset):
        raise Error(Status.INVALID_ARGUMENT,
                    "causal mask requires nonnegative I32-representable positions")
    qpos = (np.arange(queries, dtype=np.int64) + query_offset).astype(np.int32)  # wraps like iota + offset
    kpos = np.arange(keys, dtype=np.int64).astype(np.int32)
    return causal_attention_mask(rt, rt.buffer(qpos), rt.buffer(kpos))


def argmax(rt: Runtime, x: Buffer, axis: int, keep_dims: bool = False) -> Buffer:
    """``Tensor::argmax`` (crates/rxla-core/src/indexing.rs:350-374): I32
    index of the first maximum along ``axis``; the first NaN wins."""
    h = c_void_p()
    _check(_lib.rxw8_argmax(rt.handle, x.handle, int(axis), int(bool(keep_dims)), byref(h)))
    return Buffer(h)


def grouped_query_attention_noalloc(rt: Runtime, q: Buffer, k_cache: Buffer, v_cache: Buffer,
                                    lens: Buffer, out: Buffer, mask: Buffer | None = None,
                                    scale: float | None = None) -> Buffer:
    """``grouped_query_attention`` into ``out`` without any device allocation:
    the split workspace is the library's fixed per-GPU scratch array
    (``rxw8_gqa_decode_noalloc``). Calls that overlap on one GPU race."""
    s = 0.0 if scale is None else float(scale)
    m = mask.handle if mask is not None else None
    _check(_lib.rxw8_gqa_decode_noalloc(rt.handle, q.handle, k_cache.handle, v_cache.handle,
                                        lens.handle, m, ctypes.c_float(s), out.handle))
    return out


def grouped_query_attention_prefill(rt: Runtime, q: Buffer, k_cache: Buffer, v_cache: Buffer,
                                    starts: Buffer, scale: float | None = None,
                                    out_dtype=DType.F32, out: Buffer | None = None) -> Buffer:
    """Causal attention of S new rows per sequence (q [B,S,Hq,D]) against
    caches that already hold their keys; row i of sequence b sits at position
    starts[b] + i (attention.rs:14-32, 83-135)."""
    s = 0.0 if scale is None else float(scale)
    if out is not None:
        _check(_lib.rxw8_gqa_prefill_into(rt.handle, q.handle, k_cache.handle, v_cache.handle,
                                          starts.handle, ctypes.c_float(s), out.handle))
        return out
    h = c_void_p()
    _check(_lib.rxw8_gqa_prefill(rt.handle, q.handle, k_cache.handle, v_cache.handle,
                                 starts.handle, ctypes.c_float(s), int(out_dtype), byref(h)))
    return Buffer(h)


class KvCache:
    """Paired fixed-capacity K/V state (crates/rxla-core/src/kv_cache.rs:7-111)."""

    def __init__(self, rt: Runtime, shape, dtype=DType.BF16, keys: Buffer | None = None,
                 values: Buffer | None = None):
        self.rt = rt
        self.keys = keys if keys is not None else rt.zeros(shape, dtype)
        self.values = values if values is not None else rt.zeros(shape, dtype)

    def _starts(self, starts):
        if isinstance(starts, Buffer):
            return starts
        return self.rt.buffer(np.asarray(starts, np.int32))

    def update_at(self, keys: Buffer, values: Buffer, starts):
        """Paired dynamic_update_slice; out-of-range starts are clamped."""
        st = self._starts(starts)
        _check(_lib.rxw8_kv_update_at(self.rt.handle, self.keys.handle, self.values.handle,
                                      keys.handle, values.handle, st.handle, 0, None))
        return self.keys, self.values

    def update_at_checked(self, keys: Buffer, values: Buffer, starts) -> Buffer:
        """Update only when every start fits; returns the F32 ``accepted`` scalar."""
        st = self._starts(starts)
        acc = self.rt.zeros((), DType.F32)
        _check(_lib.rxw8_kv_update_at(self.rt.handle, self.keys.handle, self.values.handle,
                                      keys.handle, values.handle, st.handle, 1, acc.handle))
        return acc


class SafeTensors:
    """A memory-mapped safetensors checkpoint (crates/rxla-safetensors/src/
    model.rs:340-440): headers are validated at open, payloads are read only by
    ``upload`` / ``to_buffer``, which convert like the reference loader (U8 and
    I32 verbatim; F32 / F16 / BF16 among themselves, narrowing with
    round-to-nearest-even)."""

    def __init__(self, path):
        h = c_void_p()
        _check(_lib.rxw8_safetensors_open(os.fsencode(os.fspath(path)), byref(h)))
        self._h = h
        self.path = os.fspath(path)
        n = c_int64()
        _check(_lib.rxw8_safetensors_num_tensors(h, byref(n)))
        self._info = {}
        for i in range(n.value):
            name = ctypes.c_char_p()
            dt = c_int()
            dims = (c_int64 * 8)()
            rank = c_int()
            _check(_lib.rxw8_safetensors_tensor_info(h, i, byref(name), byref(dt), dims, byref(rank)))
            self._info[name.value.decode()] = (i, DType(dt.value) if dt.value else None,
                                               tuple(dims[j] for j in range(rank.value)))

    def close(self):
        if self._h:
            _check(_lib.rxw8_safetensors_close(self._h))
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self):
        """{name: (dtype or None when not representable, shape)}"""
        return {k: (v[1], v[2]) for k, v in self._info.items()}

    def metadata(self, key: str, default=None):
        v = ctypes.c_char_p()
        rc = _lib.rxw8_safetensors_metadata(self._h, key.encode(), byref(v))
        if rc == Status.NOT_FOUND:
            return default
        _check(rc)
        return v.value.decode()

    def upload(self, name: str, dst: Buffer, offset: int = 0):
        if name not in self._info:
            raise Error(Status.NOT_FOUND, f"missing tensor {name!r}")
        _check(_lib.rxw8_safetensors_upload(self._h, self._info[name][0], dst.handle, int(offset)))

    def to_buffer(self, rt: Runtime, name: str, dtype: DType | None = None) -> Buffer:
        if name not in self._info:
            raise Error(Status.NOT_FOUND, f"missing tensor {name!r}")
        _, sdt, shape = self._info[name]
        dt = dtype if dtype is not None else sdt
        if dt is None:
            raise Error(Status.UNIMPLEMENTED, f"tensor {name!r} has no rxw8 dtype")
        buf = rt.zeros(shape, dt)
        self.upload(name, buf)
        return buf


from .model import DecoderConfig, DecoderModel, Qwen35Config, Qwen35Model  # noqa: E402

__all__ = ["Runtime", "Buffer", "DType", "Status", "Error", "quantize_w8", "dequantize",
           "pack_weight",
           "quantized_linear",
           "linear_bf16", "QuantizedLinear", "grouped_query_attention",
           "grouped_query_attention_prefill", "grouped_query_attention_noalloc", "gqa_attention",
           "scaled_dot_product_attention", "causal_attention_mask", "causal_attention_mask_static",
           "argmax", "KvCache",
           "SafeTensors",
           "DecoderConfig", "DecoderModel", "Qwen35Config", "Qwen35Model", "bf16_to_f32"]
