"""CPU oracle for the rxw8 hot path -- TEST INFRASTRUCTURE ONLY.

numpy-facing ctypes wrappers over ``oracle/_build/librxw8_oracle.so`` (built
from ``rxw8_oracle.c`` by ``oracle/Makefile``). Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import
this module; the product (``rxla_amd``) never does.

Each wrapper restates one reference function; the citation lives beside the
C definition (``rxw8_oracle.h``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_void_p

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "librxw8_oracle.so")
_lib = None

COMPUTE_F32, COMPUTE_BF16 = 0, 1
ACCUM_F32, ACCUM_F64 = 0, 1


def build() -> str:
    """Compile the oracle library (make -C oracle)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _p(a):
    return a.ctypes.data_as(c_void_p)


def _declare(L):
    L.rxo_bf16_from_f32.restype = ctypes.c_uint16
    L.rxo_bf16_from_f32.argtypes = [c_float]
    L.rxo_f32_from_bf16.restype = c_float
    L.rxo_f32_from_bf16.argtypes = [ctypes.c_uint16]
    L.rxo_f32_to_bf16.argtypes = [c_void_p, c_void_p, c_int64]
    L.rxo_bf16_to_f32.argtypes = [c_void_p, c_void_p, c_int64]
    L.rxo_quantize_w8.restype = c_int
    L.rxo_quantize_w8.argtypes = [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p]
    L.rxo_dequantize_w8.restype = c_int
    L.rxo_dequantize_w8.argtypes = [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p]
    L.rxo_quantized_linear.restype = c_int
    L.rxo_quantized_linear.argtypes = [c_void_p, c_int64, c_int64, c_void_p, c_void_p,
                                       c_int64, c_int64, c_int, c_int, c_void_p, c_int]
    L.rxo_linear_bf16w.restype = c_int
    L.rxo_linear_bf16w.argtypes = [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int,
                                   c_void_p, c_int]
    L.rxo_gqa_attention.restype = c_int
    L.rxo_gqa_attention.argtypes = [c_void_p, c_void_p, c_void_p] + [c_int64] * 7 + [
        c_void_p, c_int64, c_int64, c_int64, c_float, c_int, c_void_p, c_int]
    L.rxo_gqa_decode_bf16cache.restype = c_int
    L.rxo_gqa_decode_bf16cache.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p] + [
        c_int64] * 5 + [c_float, c_int, c_void_p, c_int]
    L.rxo_dynamic_update_slice.restype = c_int
    L.rxo_dynamic_update_slice.argtypes = [c_void_p, c_void_p, c_int, c_int64, c_void_p,
                                           c_void_p, c_void_p]
    L.rxo_kv_update_at.restype = c_int
    L.rxo_kv_update_at.argtypes = [c_void_p, c_void_p, c_void_p, c_int, c_int64, c_void_p,
                                   c_void_p, c_void_p, c_void_p, c_int, c_void_p]
    L.rxo_rope_freqs.argtypes = [c_float, c_int64, c_void_p]
    L.rxo_rope_split_half.argtypes = [c_void_p, c_int64, c_int64, c_int64, c_void_p,
                                      c_int64, c_float]
    L.rxo_rms_norm.argtypes = [c_void_p, c_int64, c_int64, c_void_p, c_float, c_int,
                               c_void_p]
    L.rxo_silu_mul.argtypes = [c_void_p, c_void_p, c_int64, c_void_p]
    L.rxo_take_rows.argtypes = [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p]
    L.rxo_argmax_rows.argtypes = [c_void_p, c_int64, c_int64, c_void_p]
    L.rxo_decoder_forward.restype = c_int
    L.rxo_decoder_forward.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_int]
    L.rxo_decoder_forward_trace.restype = c_int
    L.rxo_decoder_forward_trace.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                            c_int64, c_int64, c_void_p, c_void_p, c_void_p,
                                            c_int, c_void_p]


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- conversions -----------------------------------------------------------

def bf16_bits(x) -> np.ndarray:
    """f32 -> bf16 bit patterns (uint16), RNE."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().rxo_f32_to_bf16(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(bits) -> np.ndarray:
    bits = _c(bits, np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().rxo_bf16_to_f32(_p(bits), _p(out), bits.size)
    return out


def round_bf16(x) -> np.ndarray:
    return bf16_to_f32(bf16_bits(x))


# ---- a1/a2 -------------------------------------------------------------------

def quantize_w8(w, group: int):
    w = _c(w, np.float32)
    n, k = w.shape
    u8 = np.empty((n, k), np.uint8)
    s = np.empty((n, k // group), np.float32)
    if lib().rxo_quantize_w8(_p(w), n, k, group, _p(u8), _p(s)):
        raise ValueError("quantize_w8: bad shape")
    return u8, s


def dequantize_w8(u8, scale) -> np.ndarray:
    u8 = _c(u8, np.uint8)
    scale = _c(scale, np.float32)
    n, k = u8.shape
    g = k // scale.shape[1]
    out = np.empty((n, k), np.float32)
    if lib().rxo_dequantize_w8(_p(u8), _p(scale), n, k, g, _p(out)):
        raise ValueError("dequantize_w8: bad shape")
    return out


def quantized_linear(x, u8, scale, compute=COMPUTE_BF16, accum=ACCUM_F32, threads=0):
    x = _c(x, np.float32)
    u8 = _c(u8, np.uint8)
    scale = _c(scale, np.float32)
    k = x.shape[-1]
    m = int(np.prod(x.shape[:-1])) if x.ndim > 1 else 1
    n = u8.shape[0]
    g = k // scale.shape[1]
    y = np.empty(x.shape[:-1] + (n,), np.float32)
    if lib().rxo_quantized_linear(_p(x), m, k, _p(u8), _p(scale), n, g, compute, accum,
                                  _p(y), threads):
        raise ValueError("quantized_linear: bad shape")
    return y


def linear_bf16w(x, w_bits, accum=ACCUM_F32, threads=0):
    x = _c(x, np.float32)
    w_bits = _c(w_bits, np.uint16)
    k = x.shape[-1]
    m = int(np.prod(x.shape[:-1]))
    n = w_bits.shape[0]
    y = np.empty(x.shape[:-1] + (n,), np.float32)
    if lib().rxo_linear_bf16w(_p(x), m, k, _p(w_bits), n, accum, _p(y), threads):
        raise ValueError("linear_bf16w: bad shape")
    return y


# ---- attention ---------------------------------------------------------------

def gqa_attention(q, k, v, mask=None, scale=None, precision=0, threads=0):
    """q [B,Hq,Sq,D], k [B,Hkv,Sk,D], v [B,Hkv,Sk,Dv]; mask broadcastable to
    [B,Hq,Sq,Sk] (additive f32)."""
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    b, hq, sq, d = q.shape
    _, hkv, sk, _ = k.shape
    dv = v.shape[3]
    if scale is None:
        scale = 1.0 / float(np.sqrt(np.float32(d)))
    out = np.empty((b, hq, sq, dv), np.float32)
    mp, sb, sh, si = None, 0, 0, 0
    if mask is not None:
        m4 = np.asarray(mask, np.float32)
        while m4.ndim < 4:
            m4 = m4[None]
        np.broadcast_shapes(m4.shape, (b, hq, sq, sk))  # raises when incompatible
        if m4.shape[3] != sk:
            m4 = np.broadcast_to(m4, m4.shape[:3] + (sk,))
        m4 = np.ascontiguousarray(m4)
        sb, sh, si = [m4.strides[i] // 4 if m4.shape[i] > 1 else 0 for i in range(3)]
        mp = m4.ctypes.data_as(c_void_p)
    rc = lib().rxo_gqa_attention(_p(q), _p(k), _p(v), b, hq, hkv, sq, sk, d, dv, mp, sb,
                                 sh, si, float(scale), precision, _p(out), threads)
    if rc:
        raise ValueError("gqa_attention: bad shape")
    return out


def causal_attention_mask(query_positions, key_positions):
    """Tensor::causal_attention_mask (crates/rxla-core/src/attention.rs:14-32):
    [Q, K] f32, 0 where key_positions[j] <= query_positions[i] (signed I32
    compare), else -inf."""
    qp = np.asarray(query_positions, np.int32)
    kp = np.asarray(key_positions, np.int32)
    return np.where(kp[None, :] <= qp[:, None], np.float32(0.0), np.float32(-np.inf)).astype(np.float32)


def gqa_decode_bf16cache(q, kc_bits, vc_bits, lens, scale=None, precision=0, threads=0):
    """q [B,Hq,D] f32; caches [B,Hkv,Lmax,D] bf16 bits; lens [B] int32."""
    q = _c(q, np.float32)
    kc_bits = _c(kc_bits, np.uint16)
    vc_bits = _c(vc_bits, np.uint16)
    lens = _c(lens, np.int32)
    b, hq, d = q.shape
    _, hkv, lmax, _ = kc_bits.shape
    if scale is None:
        scale = 1.0 / float(np.sqrt(np.float32(d)))
    out = np.empty((b, hq, d), np.float32)
    if lib().rxo_gqa_decode_bf16cache(_p(q), _p(kc_bits), _p(vc_bits), _p(lens), b, hq, hkv,
                                      lmax, d, float(scale), precision, _p(out), threads):
        raise ValueError("gqa_decode_bf16cache: bad shape or lens")
    return out


# ---- KV ------------------------------------------------------------------------

def dynamic_update_slice(operand, update, starts):
    out = np.array(operand, copy=True, order="C")
    update = np.ascontiguousarray(update, dtype=out.dtype)
    dims = np.asarray(out.shape, np.int64)
    udims = np.asarray(update.shape, np.int64)
    st = np.asarray(starts, np.int32)
    if lib().rxo_dynamic_update_slice(_p(out), _p(dims), out.ndim, out.itemsize, _p(update),
                                      _p(udims), _p(st)):
        raise ValueError("dynamic_update_slice: bad shape")
    return out


def kv_update_at(kc, vc, ku, vu, starts, checked=False):
    kc = np.array(kc, copy=True, order="C")
    vc = np.array(vc, copy=True, order="C")
    ku = np.ascontiguousarray(ku, dtype=kc.dtype)
    vu = np.ascontiguousarray(vu, dtype=kc.dtype)
    dims = np.asarray(kc.shape, np.int64)
    udims = np.asarray(ku.shape, np.int64)
    st = np.asarray(starts, np.int32)
    acc = np.zeros(1, np.float32)
    if lib().rxo_kv_update_at(_p(kc), _p(vc), _p(dims), kc.ndim, kc.itemsize, _p(ku), _p(vu),
                              _p(udims), _p(st), int(checked), _p(acc)):
        raise ValueError("kv_update_at: bad shape")
    return kc, vc, float(acc[0])


# ---- elementwise -------------------------------------------------------------------

def rope_freqs(theta, rot_dim):
    out = np.empty(rot_dim // 2, np.float32)
    lib().rxo_rope_freqs(float(theta), rot_dim, _p(out))
    return out


def rope_split_half(x, pos, theta, rot_dim=None):
    """x [..., R, D] rows; pos has one entry per leading index (rows_per_pos =
    x.shape[-2])."""
    x = np.array(x, dtype=np.float32, copy=True, order="C")
    d = x.shape[-1]
    rot_dim = d if rot_dim is None else rot_dim
    pos = _c(pos, np.int32)
    rows = x.size // d
    rows_per_pos = rows // pos.size
    lib().rxo_rope_split_half(_p(x), rows, d, rot_dim, _p(pos), rows_per_pos, float(theta))
    return x


def rms_norm(x, w, eps, zero_centered=False):
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    h = x.shape[-1]
    y = np.empty_like(x)
    lib().rxo_rms_norm(_p(x), x.size // h, h, _p(w), float(eps), int(zero_centered), _p(y))
    return y


def silu_mul(gate, up):
    gate = _c(gate, np.float32)
    up = _c(up, np.float32)
    out = np.empty_like(gate)
    lib().rxo_silu_mul(_p(gate), _p(up), gate.size, _p(out))
    return out


def take_rows(table, ids):
    table = np.ascontiguousarray(table)
    ids = _c(ids, np.int32)
    v = table.shape[0]
    row_bytes = table.itemsize * (table.size // v)
    out = np.empty(ids.shape + table.shape[1:], table.dtype)
    lib().rxo_take_rows(_p(table), v, row_bytes, _p(ids), ids.size, _p(out))
    return out


def argmax_rows(x):
    x = _c(x, np.float32)
    cols = x.shape[-1]
    out = np.empty(x.shape[:-1], np.int32)
    lib().rxo_argmax_rows(_p(x), x.size // cols, cols, _p(out))
    return out


# ---- decoder ---------------------------------------------------------------------------

class _Cfg(ctypes.Structure):
    _fields_ = [("layers", c_int64), ("hidden", c_int64), ("q_heads", c_int64),
                ("kv_heads", c_int64), ("head_dim", c_int64), ("intermediate", c_int64),
                ("vocab", c_int64), ("max_seq", c_int64), ("group", c_int64),
                ("eps", c_float), ("theta", c_float), ("qk_norm", c_int32), ("accum", c_int32)]


class _Params(ctypes.Structure):
    _fields_ = [(name, POINTER(c_void_p)) for name in
                ("in_norm", "q_norm", "k_norm", "post_norm", "qkv_w", "o_w", "gu_w",
                 "down_w", "qkv_s", "o_s", "gu_s", "down_s")] + [
        ("embed", c_void_p), ("final_norm", c_void_p)]


class Decoder:
    """Oracle decoder state: parameters (numpy) + bf16 KV caches + lens."""

    def __init__(self, cfg: dict, params: dict, batch: int):
        self.cfg = dict(cfg)
        self.params = params
        self.batch = batch
        c = self.cfg
        self._c = _Cfg(c["layers"], c["hidden"], c["q_heads"], c["kv_heads"], c["head_dim"],
                       c["intermediate"], c["vocab"], c["max_seq"], c["group"], c["eps"],
                       c["theta"], int(c.get("qk_norm", True)), int(c.get("accum", ACCUM_F32)))
        nl = c["layers"]
        self._keep = []

        def arr(name, dtype):
            ptrs = (c_void_p * nl)()
            for i in range(nl):
                a = np.ascontiguousarray(params[f"layers.{i}.{name}"], dtype=dtype)
                self._keep.append(a)
                ptrs[i] = a.ctypes.data
            self._keep.append(ptrs)
            return ctypes.cast(ptrs, POINTER(c_void_p))

        p = _Params()
        p.in_norm = arr("input_layernorm.weight", np.float32)
        p.post_norm = arr("post_attention_layernorm.weight", np.float32)
        if c.get("qk_norm", True):
            p.q_norm = arr("self_attn.q_norm.weight", np.float32)
            p.k_norm = arr("self_attn.k_norm.weight", np.float32)
        p.qkv_w = arr("self_attn.qkv_proj.weight", np.uint8)
        p.qkv_s = arr("self_attn.qkv_proj.scale", np.float32)
        p.o_w = arr("self_attn.o_proj.weight", np.uint8)
        p.o_s = arr("self_attn.o_proj.scale", np.float32)
        p.gu_w = arr("mlp.gate_up_proj.weight", np.uint8)
        p.gu_s = arr("mlp.gate_up_proj.scale", np.float32)
        p.down_w = arr("mlp.down_proj.weight", np.uint8)
        p.down_s = arr("mlp.down_proj.scale", np.float32)
        emb = np.ascontiguousarray(params["embed_tokens.weight"], np.uint16)
        fn = np.ascontiguousarray(params["norm.weight"], np.float32)
        self._keep += [emb, fn]
        p.embed = emb.ctypes.data
        p.final_norm = fn.ctypes.data
        self._p = p
        shape = (nl, batch, c["kv_heads"], c["max_seq"], c["head_dim"])
        self.k_cache = np.zeros(shape, np.uint16)
        self.v_cache = np.zeros(shape, np.uint16)
        self.lens = np.zeros(batch, np.int32)

    def forward(self, ids, threads=0, trace=False):
        """Runs ids [b, s] from the current lengths; returns (logits [b, V],
        next ids [b]) and, with trace, also the residual stream [layers + 1,
        b, s, H]: entry l is the input of layer l, the last the output of the
        final layer (before the final norm)."""
        ids = _c(ids, np.int32)
        b, s = ids.shape
        assert b == self.batch
        logits = np.empty((b, self.cfg["vocab"]), np.float32)
        nxt = np.empty(b, np.int32)
        hs = np.empty((self.cfg["layers"] + 1, b, s, self.cfg["hidden"]), np.float32) if trace else None
        rc = lib().rxo_decoder_forward_trace(ctypes.byref(self._c), ctypes.byref(self._p),
                                             _p(self.k_cache), _p(self.v_cache), _p(self.lens),
                                             b, s, _p(ids), _p(logits), _p(nxt), threads,
                                             _p(hs) if trace else None)
        if rc:
            raise ValueError(f"decoder_forward failed ({rc})")
        return (logits, nxt, hs) if trace else (logits, nxt)
