"""Decoder plan: the compiled Qwen-style dense W8 decoder behind the C ABI.

Mirrors the reference's model ABI flow (crates/rxla-nn/src/applied.rs):
``AppliedModel::compile`` (:808-815) -> ``CompiledModel::bind_parameters``
(:156-172, path-addressed parameters validated by ``order_parameters``
:948-990 / ``validate_buffer`` :1274) -> ``BoundModel::run`` (:222-239).
The composition follows crates/rxla-models/src/qwen3_5/mod.rs:199-273 with
dense full-attention layers (layers.rs:28-101) and the SwiGLU MLP
(layers.rs:270-293).
"""
from __future__ import annotations

import ctypes
from ctypes import byref, c_char_p, c_int, c_int32, c_int64, c_void_p
from dataclasses import dataclass

import numpy as np

from . import Buffer, DType, Error, Runtime, Status, _check, _ffi, _lib


@dataclass
class DecoderConfig:
    layers: int = 28
    hidden: int = 2048
    q_heads: int = 16
    kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 6144
    vocab: int = 151936
    max_batch: int = 8
    max_seq: int = 1280
    group: int = 0  # 0: per-output-channel scales on every projection
    eps: float = 1e-6
    theta: float = 1e6
    qk_norm: bool = True

    def c(self):
        return _ffi.DecoderConfig(self.layers, self.hidden, self.q_heads, self.kv_heads,
                                  self.head_dim, self.intermediate, self.vocab, self.max_batch,
                                  self.max_seq, self.group, self.eps, self.theta,
                                  int(self.qk_norm))

    def as_dict(self):
        return dict(self.__dict__)


class DecoderModel:
    """``compile()`` validates the config and allocates the plan (KV cache,
    activations); ``bind_parameters`` attaches weights by schema path;
    ``forward`` / ``generate`` run it."""

    def __init__(self, rt: Runtime, cfg: DecoderConfig):
        self.rt = rt
        self.cfg = cfg
        self._h = None
        self._bound = []

    def compile(self) -> "DecoderModel":
        h = c_void_p()
        c = self.cfg.c()
        _check(_lib.rxw8_decoder_create(self.rt.handle, byref(c), byref(h)))
        self._h = h
        return self

    def close(self):
        if self._h:
            _check(_lib.rxw8_decoder_destroy(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def schema(self):
        """[(path, dtype, shape)] in declaration order."""
        n = c_int()
        _check(_lib.rxw8_decoder_num_parameters(self._h, byref(n)))
        out = []
        for i in range(n.value):
            path = c_char_p()
            dt = c_int()
            dims = (c_int64 * 8)()
            rank = c_int()
            _check(_lib.rxw8_decoder_parameter_info(self._h, i, byref(path), byref(dt), dims,
                                                    byref(rank)))
            out.append((path.value.decode(), DType(dt.value),
                        tuple(dims[j] for j in range(rank.value))))
        return out

    def bind_parameter(self, path: str, buf: Buffer):
        _check(_lib.rxw8_decoder_bind_parameter(self._h, path.encode(), buf.handle))
        self._bound.append(buf)

    def bind_parameters(self, params: dict) -> "DecoderModel":
        for path, buf in params.items():
            self.bind_parameter(path, buf)
        return self

    def reset(self):
        _check(_lib.rxw8_decoder_reset(self._h))

    def lens(self) -> np.ndarray:
        out = np.zeros(self.cfg.max_batch, np.int32)
        _check(_lib.rxw8_decoder_lens(self._h, out.ctypes.data_as(ctypes.POINTER(c_int32)),
                                      out.size))
        return out

    def forward(self, ids: Buffer, logits: Buffer | None = None, next_ids: Buffer | None = None):
        b, s = ids.shape
        nxt = next_ids if next_ids is not None else self.rt.zeros((b,), DType.I32)
        _check(_lib.rxw8_decoder_forward(self._h, ids.handle, b, s, nxt.handle,
                                         logits.handle if logits is not None else None))
        return nxt

    def generate(self, prompt: Buffer, steps: int, out_ids: Buffer | None = None,
                 use_graph: bool = True) -> Buffer:
        b, s = prompt.shape
        out = out_ids if out_ids is not None else self.rt.zeros((b, steps + 1), DType.I32)
        _check(_lib.rxw8_decoder_generate(self._h, prompt.handle, b, s, steps, out.handle,
                                          int(use_graph)))
        return out
