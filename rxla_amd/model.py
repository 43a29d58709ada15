"""Compiled model plans behind the C ABI: the Qwen-style dense W8 decoder
(DecoderModel) and the Qwen3.5 hybrid W8 text model (Qwen35Model).

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

import re

from . import Buffer, DType, Error, Runtime, SafeTensors, Status, _check, _ffi, _lib, dequantize


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


class _CompiledPlan:
    """Shared model ABI flow of the compiled plans: ``compile()`` validates the
    config and allocates the plan; ``schema()`` lists path-addressed
    parameters; ``bind_parameter(s)`` attaches weights (retained by the plan);
    ``load_safetensors`` validates a checkpoint against the schema, then
    uploads and binds. Subclasses name their C entry points by ``_PREFIX``."""

    _PREFIX = ""
    CHECKPOINT_PREFIXES = ("",)
    _FUSED = ()

    def __init__(self, rt: Runtime, cfg):
        self.rt = rt
        self.cfg = cfg
        self._h = None
        self._bound = []

    def _fn(self, name):
        return getattr(_lib, self._PREFIX + name)

    def compile(self):
        h = c_void_p()
        self._c = self.cfg.c()  # kept alive while the plan exists
        _check(self._fn("create")(self.rt.handle, byref(self._c), byref(h)))
        self._h = h
        return self

    def close(self):
        if self._h:
            _check(self._fn("destroy")(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def schema(self):
        """[(path, dtype, shape)] in declaration order."""
        n = c_int()
        _check(self._fn("num_parameters")(self._h, byref(n)))
        out = []
        for i in range(n.value):
            path = c_char_p()
            dt = c_int()
            dims = (c_int64 * 8)()
            rank = c_int()
            _check(self._fn("parameter_info")(self._h, i, byref(path), byref(dt), dims, byref(rank)))
            out.append((path.value.decode(), DType(dt.value),
                        tuple(dims[j] for j in range(rank.value))))
        return out

    def bind_parameter(self, path: str, buf: Buffer):
        _check(self._fn("bind_parameter")(self._h, path.encode(), buf.handle))
        self._bound.append(buf)

    def bind_parameters(self, params: dict):
        for path, buf in params.items():
            self.bind_parameter(path, buf)
        return self

    # ---- checkpoints ------------------------------------------------------------
    def checkpoint_plan(self, st: SafeTensors, mapping: dict | None = None) -> dict:
        """Schema path -> (checkpoint keys stacked along dim 0, dequantise), all
        validated before any payload is read (rxla-safetensors model.rs:384-440:
        exact path match or an explicit mapping, dtype compatibility, shapes).

        Keys are found under the prefixes "", "model." and
        "model.language_model." (the names quantize_qwen3_5_w8.py keeps). The
        fused projections take q_proj / k_proj / v_proj and gate_proj / up_proj
        rows in that order (projections.rs:21-69). A float schema parameter
        stored as U8 codes with a sibling ".scale" (the encoder quantizes every
        2-D tensor, e.g. embed_tokens) is dequantised exactly on the device:
        bf16((u - 128) * s) (layers.rs:277-294)."""
        info = st.tensors()

        def find(key):
            for p in self.CHECKPOINT_PREFIXES:
                if p + key in info:
                    return p + key
            return None

        floats = (DType.F32, DType.F16, DType.BF16)
        plan, errors = {}, []
        for path, dtype, shape in self.schema():
            if mapping and path in mapping:
                keys = [mapping[path]] if isinstance(mapping[path], str) else list(mapping[path])
                missing = [k for k in keys if k not in info]
            else:
                k = find(path)
                keys, missing = ([k], []) if k else ([], [path])
                if not k:
                    for pat, parts in self._FUSED:
                        m = pat.match(path)
                        if m:
                            found = [find(f"{m.group(1)}{part}.{m.group(2)}") for part in parts]
                            if all(found):
                                keys, missing = found, []
                            else:
                                missing = [f"{m.group(1)}{part}.{m.group(2)}"
                                           for part, f in zip(parts, found) if not f]
            if missing:
                errors.append(f"{path}: missing checkpoint tensor(s) {missing}")
                continue
            deq = False
            rows = 0
            for k in keys:
                sdt, sshape = info[k]
                if dtype in floats and sdt == DType.U8:
                    scale = k[:-len(".weight")] + ".scale" if k.endswith(".weight") else None
                    if len(keys) != 1 or scale not in info or len(sshape) != 2:
                        errors.append(f"{path}: {k} is U8 without a usable .scale for {dtype.name} storage")
                        break
                    deq = True
                elif not (sdt == dtype or (dtype in floats and sdt in floats)):
                    errors.append(f"{path}: incompatible checkpoint dtype {sdt} of {k} for "
                                  f"{dtype.name} storage")
                    break
                if len(sshape) != len(shape) or tuple(sshape[1:]) != tuple(shape[1:]):
                    errors.append(f"{path}: {k} has shape {sshape}, schema {shape}")
                    break
                rows += sshape[0] if sshape else 1
            else:
                if (shape and rows != shape[0]) or (not shape and rows != 1):
                    errors.append(f"{path}: checkpoint rows {rows} != schema {shape}")
                    continue
                plan[path] = (keys, deq)
        if errors:
            raise Error(Status.INVALID_ARGUMENT, "checkpoint does not match the decoder schema: "
                        + "; ".join(errors[:8]) + (" ..." if len(errors) > 8 else ""))
        return plan

    def load_safetensors(self, checkpoint, mapping: dict | None = None):
        """Validate every parameter against the checkpoint, then upload and bind
        (CompiledModel::bind_parameters over load_parameter_schema_with_mapping)."""
        st = checkpoint if isinstance(checkpoint, SafeTensors) else SafeTensors(checkpoint)
        try:
            g = st.metadata("group_size")
            if g is not None and self.cfg.group not in (0, int(g)):
                raise Error(Status.INVALID_ARGUMENT,
                            f"checkpoint group_size {g} != decoder group {self.cfg.group}")
            plan = self.checkpoint_plan(st, mapping)
            info = st.tensors()
            for path, dtype, shape in self.schema():
                keys, deq = plan[path]
                if deq:
                    w = st.to_buffer(self.rt, keys[0])
                    s_ = st.to_buffer(self.rt, keys[0][:-len(".weight")] + ".scale", DType.F32)
                    buf = dequantize(self.rt, w, s_, dtype)
                else:
                    buf = self.rt.zeros(shape, dtype)
                    off = 0
                    for k in keys:
                        st.upload(k, buf, off)
                        off += int(np.prod(info[k][1], dtype=np.int64))
                self.bind_parameter(path, buf)
        finally:
            if st is not checkpoint:
                st.close()
        return self


class DecoderModel(_CompiledPlan):
    """The dense decoder plan (KV cache, activations); ``forward`` /
    ``generate`` run it."""

    _PREFIX = "rxw8_decoder_"
    CHECKPOINT_PREFIXES = ("", "model.", "model.language_model.")
    _FUSED = ((re.compile(r"^(layers\.\d+\.self_attn\.)qkv_proj\.(weight|scale)$"),
               ("q_proj", "k_proj", "v_proj")),
              (re.compile(r"^(layers\.\d+\.mlp\.)gate_up_proj\.(weight|scale)$"),
               ("gate_proj", "up_proj")))

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

    def forward_layers(self, hidden_in: Buffer, first: int, last: int,
                       hidden_out: Buffer | None = None, logits: Buffer | None = None,
                       commit: bool = False) -> Buffer:
        """Teacher forcing: layers [first, last) of one step from the F32
        residual rows ``hidden_in`` [b, s, hidden] (rxw8_decoder_forward_layers).
        Returns the residual rows leaving layer last - 1."""
        b, s, _ = hidden_in.shape
        out = hidden_out if hidden_out is not None else self.rt.zeros(hidden_in.shape, DType.F32)
        _check(_lib.rxw8_decoder_forward_layers(
            self._h, hidden_in.handle, b, s, first, last, out.handle,
            logits.handle if logits is not None else None, int(commit)))
        return out

    def generate(self, prompt: Buffer, steps: int, out_ids: Buffer | None = None,
                 use_graph: bool = True) -> Buffer:
        b, s = prompt.shape
        out = out_ids if out_ids is not None else self.rt.zeros((b, steps + 1), DType.I32)
        _check(_lib.rxw8_decoder_generate(self._h, prompt.handle, b, s, steps, out.handle,
                                          int(use_graph)))
        return out


LINEAR, FULL = 0, 1


def _compute_dtype(name):
    if name in ("f32", DType.F32):
        return int(DType.F32)
    if name in ("bf16", DType.BF16):
        return int(DType.BF16)
    raise ValueError(f"compute dtype must be 'f32' or 'bf16', not {name!r}")


@dataclass
class Qwen35Config:
    """Qwen3_5Config (crates/rxla-models/src/qwen3_5/mod.rs:16-33); defaults
    are the official 0.8B text topology (qwen3_5_0_8b_w8, mod.rs:59-85), with
    ``layers`` either a count (every ``full_attention_interval``-th layer is
    full attention) or an explicit list of LINEAR / FULL kinds."""
    vocab: int = 248320
    hidden: int = 1024
    intermediate: int = 3584
    layers: object = 24
    heads: int = 8
    kv_heads: int = 2
    head_dim: int = 256
    linear_heads: int = 16
    linear_head_dim: int = 128
    conv_kernel: int = 4
    max_positions: int = 262144
    rotary_dim: int = 64
    group: int = 128
    full_attention_interval: int = 4
    theta: float = 1e7
    eps: float = 1e-6
    lora_rank: int = 0
    lora_alpha: float = 0.0
    max_batch: int = 1
    max_seq: int = 4096
    # projection compute dtype: "f32", the reference's default (rxla-nn
    # lib.rs:432), or the "bf16" opt-in (Cx::with_layer_compute_dtype)
    compute: str = "f32"

    @classmethod
    def tiny(cls, **kw):
        """Qwen3_5Config::tiny (mod.rs:36-57)."""
        c = dict(vocab=128, hidden=32, intermediate=64, layers=[LINEAR, FULL], heads=4, kv_heads=2,
                 head_dim=8, linear_heads=4, linear_head_dim=8, conv_kernel=4, max_positions=128,
                 rotary_dim=4, group=8, max_seq=128)
        c.update(kw)
        return cls(**c)

    def kinds(self):
        if isinstance(self.layers, int):
            return [FULL if (i + 1) % self.full_attention_interval == 0 else LINEAR
                    for i in range(self.layers)]
        return [FULL if k in (FULL, "full") else LINEAR for k in self.layers]

    def c(self):
        kinds = self.kinds()
        arr = (c_int32 * len(kinds))(*kinds)
        c = _ffi.Qwen35Config(self.vocab, self.hidden, self.intermediate, len(kinds), self.heads,
                              self.kv_heads, self.head_dim, self.linear_heads,
                              self.linear_head_dim, self.conv_kernel, self.max_positions,
                              self.rotary_dim, self.group, self.full_attention_interval,
                              ctypes.cast(arr, ctypes.POINTER(c_int32)), self.theta, self.eps,
                              self.lora_rank, self.lora_alpha, self.max_batch, self.max_seq,
                              _compute_dtype(self.compute))
        c._kinds = arr  # the array must outlive the create call
        return c


class Qwen35Model(_CompiledPlan):
    """The Qwen3.5 hybrid W8 plan: ``forward(ids [B, S] I32)`` returns logits
    [B, S, V] F32 for every position, as qwen3_5 (mod.rs:197-273) does.
    Checkpoints written by the reference encoder (quantize_qwen3_5_w8.py:
    "model.language_model." names, U8 codes + F32 scales) bind verbatim."""

    _PREFIX = "rxw8_qwen35_"
    CHECKPOINT_PREFIXES = ("",)

    def forward(self, ids: Buffer, logits: Buffer | None = None) -> Buffer:
        shape = tuple(ids.shape)
        if logits is None:  # a wrong rank reaches the C check (InvalidQwenTokenShape)
            logits = self.rt.zeros(shape + (self.cfg.vocab,) if len(shape) == 2 else (1,), DType.F32)
        _check(_lib.rxw8_qwen35_forward(self._h, ids.handle, logits.handle))
        return logits
