"""ctypes declarations for librxw8.so (the C ABI in include/rxw8.h).

The library is built in-tree by ``rxla_amd/csrc/Makefile``
(``__graft_entry__.build()``). There is no fallback: importing this module
without the built library raises ImportError.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import (POINTER, Structure, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t,
                    c_void_p)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "librxw8.so")

# Every symbol include/rxw8.h declares (checked by tests/test_abi.py).
EXPORTS = [
    "rxw8_last_error", "rxw8_status_is_retryable", "rxw8_abi_version",
    "rxw8_runtime_create", "rxw8_runtime_destroy", "rxw8_runtime_set_stream",
    "rxw8_runtime_stream", "rxw8_runtime_synchronize", "rxw8_runtime_device_info",
    "rxw8_buffer_create", "rxw8_buffer_from_host", "rxw8_buffer_wrap", "rxw8_buffer_to_host",
    "rxw8_buffer_copy_from_host", "rxw8_buffer_retain", "rxw8_buffer_release",
    "rxw8_buffer_dtype", "rxw8_buffer_dims", "rxw8_buffer_device_ptr",
    "rxw8_quantize_w8", "rxw8_dequantize", "rxw8_pack_weight", "rxw8_quantized_linear", "rxw8_quantized_linear_into",
    "rxw8_quantized_linear_group", "rxw8_linear_bf16", "rxw8_linear_bf16_into",
    "rxw8_gqa_decode", "rxw8_gqa_decode_into",
    "rxw8_gqa_decode_noalloc", "rxw8_gqa_attention", "rxw8_gqa_attention_into",
    "rxw8_causal_attention_mask",
    "rxw8_gqa_prefill", "rxw8_gqa_prefill_into", "rxw8_kv_update_at", "rxw8_argmax",
    "rxw8_safetensors_open", "rxw8_safetensors_close", "rxw8_safetensors_num_tensors",
    "rxw8_safetensors_tensor_info", "rxw8_safetensors_find", "rxw8_safetensors_metadata",
    "rxw8_safetensors_upload",
    "rxw8_decoder_create", "rxw8_decoder_destroy", "rxw8_decoder_num_parameters",
    "rxw8_decoder_parameter_info", "rxw8_decoder_bind_parameter", "rxw8_decoder_reset",
    "rxw8_decoder_forward", "rxw8_decoder_forward_layers", "rxw8_decoder_generate",
    "rxw8_decoder_lens",
    "rxw8_qwen35_create", "rxw8_qwen35_destroy", "rxw8_qwen35_num_parameters",
    "rxw8_qwen35_parameter_info", "rxw8_qwen35_bind_parameter", "rxw8_qwen35_forward",
    "rxw8_xla_quantized_linear", "rxw8_xla_gqa_decode", "rxw8_xla_gqa_prefill",
    "rxw8_xla_ffi_quantized_linear", "rxw8_xla_ffi_gqa_decode", "rxw8_xla_ffi_gqa_prefill",
]


class DecoderConfig(Structure):
    _fields_ = [("layers", c_int64), ("hidden", c_int64), ("q_heads", c_int64),
                ("kv_heads", c_int64), ("head_dim", c_int64), ("intermediate", c_int64),
                ("vocab", c_int64), ("max_batch", c_int64), ("max_seq", c_int64),
                ("group", c_int64), ("eps", c_float), ("theta", c_float),
                ("qk_norm", c_int32)]


class Qwen35Config(Structure):
    _fields_ = [("vocab", c_int64), ("hidden", c_int64), ("intermediate", c_int64),
                ("layers", c_int64), ("heads", c_int64), ("kv_heads", c_int64),
                ("head_dim", c_int64), ("linear_heads", c_int64), ("linear_head_dim", c_int64),
                ("conv_kernel", c_int64), ("max_positions", c_int64), ("rotary_dim", c_int64),
                ("group", c_int64), ("full_attention_interval", c_int64),
                ("layer_kinds", POINTER(c_int32)), ("theta", c_float), ("eps", c_float),
                ("lora_rank", c_int64), ("lora_alpha", c_float), ("max_batch", c_int64),
                ("max_seq", c_int64), ("compute_dtype", c_int32)]


def _declare(L):
    vp, i64p = c_void_p, POINTER(c_int64)
    sigs = {
        "rxw8_last_error": (c_char_p, []),
        "rxw8_status_is_retryable": (c_int, [c_int]),
        "rxw8_abi_version": (c_int, []),
        "rxw8_runtime_create": (c_int, [c_int, POINTER(vp)]),
        "rxw8_runtime_destroy": (c_int, [vp]),
        "rxw8_runtime_set_stream": (c_int, [vp, vp]),
        "rxw8_runtime_stream": (c_int, [vp, POINTER(vp)]),
        "rxw8_runtime_synchronize": (c_int, [vp]),
        "rxw8_runtime_device_info": (c_int, [vp, POINTER(c_int), ctypes.c_char_p, c_size_t]),
        "rxw8_buffer_create": (c_int, [vp, c_int, i64p, c_int, POINTER(vp)]),
        "rxw8_buffer_from_host": (c_int, [vp, c_int, i64p, c_int, vp, POINTER(vp)]),
        "rxw8_buffer_wrap": (c_int, [vp, c_int, i64p, c_int, vp, POINTER(vp)]),
        "rxw8_buffer_to_host": (c_int, [vp, vp, c_size_t]),
        "rxw8_buffer_copy_from_host": (c_int, [vp, vp, c_size_t]),
        "rxw8_buffer_retain": (c_int, [vp]),
        "rxw8_buffer_release": (c_int, [vp]),
        "rxw8_buffer_dtype": (c_int, [vp, POINTER(c_int)]),
        "rxw8_buffer_dims": (c_int, [vp, i64p, POINTER(c_int)]),
        "rxw8_buffer_device_ptr": (c_int, [vp, POINTER(vp)]),
        "rxw8_quantize_w8": (c_int, [vp, vp, c_int64, POINTER(vp), POINTER(vp)]),
        "rxw8_dequantize": (c_int, [vp, vp, vp, c_int, POINTER(vp)]),
        "rxw8_pack_weight": (c_int, [vp, vp, POINTER(vp)]),
        "rxw8_quantized_linear": (c_int, [vp, vp, vp, vp, c_int, c_int, POINTER(vp)]),
        "rxw8_quantized_linear_into": (c_int, [vp, vp, vp, vp, c_int, vp]),
        "rxw8_quantized_linear_group": (c_int, [vp, c_int, POINTER(vp), POINTER(vp), POINTER(vp),
                                                POINTER(vp)]),
        "rxw8_linear_bf16": (c_int, [vp, vp, vp, c_int, POINTER(vp)]),
        "rxw8_linear_bf16_into": (c_int, [vp, vp, vp, vp]),
        "rxw8_gqa_decode": (c_int, [vp, vp, vp, vp, vp, vp, c_float, c_int, POINTER(vp)]),
        "rxw8_gqa_decode_into": (c_int, [vp, vp, vp, vp, vp, vp, c_float, vp]),
        "rxw8_gqa_decode_noalloc": (c_int, [vp, vp, vp, vp, vp, vp, c_float, vp]),
        "rxw8_gqa_attention": (c_int, [vp, vp, vp, vp, vp, POINTER(c_float), POINTER(vp)]),
        "rxw8_gqa_attention_into": (c_int, [vp, vp, vp, vp, vp, POINTER(c_float), vp]),
        "rxw8_causal_attention_mask": (c_int, [vp, vp, vp, POINTER(vp)]),
        "rxw8_gqa_prefill": (c_int, [vp, vp, vp, vp, vp, c_float, c_int, POINTER(vp)]),
        "rxw8_gqa_prefill_into": (c_int, [vp, vp, vp, vp, vp, c_float, vp]),
        "rxw8_kv_update_at": (c_int, [vp, vp, vp, vp, vp, vp, c_int, vp]),
        "rxw8_argmax": (c_int, [vp, vp, c_int, c_int, POINTER(vp)]),
        "rxw8_safetensors_open": (c_int, [c_char_p, POINTER(vp)]),
        "rxw8_safetensors_close": (c_int, [vp]),
        "rxw8_safetensors_num_tensors": (c_int, [vp, i64p]),
        "rxw8_safetensors_tensor_info": (c_int, [vp, c_int64, POINTER(c_char_p), POINTER(c_int),
                                                 i64p, POINTER(c_int)]),
        "rxw8_safetensors_find": (c_int, [vp, c_char_p, i64p]),
        "rxw8_safetensors_metadata": (c_int, [vp, c_char_p, POINTER(c_char_p)]),
        "rxw8_safetensors_upload": (c_int, [vp, c_int64, vp, c_int64]),
        "rxw8_decoder_create": (c_int, [vp, POINTER(DecoderConfig), POINTER(vp)]),
        "rxw8_decoder_destroy": (c_int, [vp]),
        "rxw8_decoder_num_parameters": (c_int, [vp, POINTER(c_int)]),
        "rxw8_decoder_parameter_info": (c_int, [vp, c_int, POINTER(c_char_p), POINTER(c_int),
                                                i64p, POINTER(c_int)]),
        "rxw8_decoder_bind_parameter": (c_int, [vp, c_char_p, vp]),
        "rxw8_decoder_reset": (c_int, [vp]),
        "rxw8_decoder_forward": (c_int, [vp, vp, c_int64, c_int64, vp, vp]),
        "rxw8_decoder_forward_layers": (c_int, [vp, vp, c_int64, c_int64, c_int64, c_int64, vp,
                                                vp, c_int]),
        "rxw8_decoder_generate": (c_int, [vp, vp, c_int64, c_int64, c_int64, vp, c_int]),
        "rxw8_decoder_lens": (c_int, [vp, POINTER(c_int32), c_int64]),
        "rxw8_qwen35_create": (c_int, [vp, POINTER(Qwen35Config), POINTER(vp)]),
        "rxw8_qwen35_destroy": (c_int, [vp]),
        "rxw8_qwen35_num_parameters": (c_int, [vp, POINTER(c_int)]),
        "rxw8_qwen35_parameter_info": (c_int, [vp, c_int, POINTER(c_char_p), POINTER(c_int),
                                               i64p, POINTER(c_int)]),
        "rxw8_qwen35_bind_parameter": (c_int, [vp, c_char_p, vp]),
        "rxw8_qwen35_forward": (c_int, [vp, vp, vp]),
        "rxw8_xla_quantized_linear": (None, [vp, POINTER(vp), c_char_p, c_size_t, vp]),
        "rxw8_xla_gqa_decode": (None, [vp, POINTER(vp), c_char_p, c_size_t, vp]),
        "rxw8_xla_ffi_quantized_linear": (vp, [vp]),
        "rxw8_xla_ffi_gqa_decode": (vp, [vp]),
        "rxw8_xla_ffi_gqa_prefill": (vp, [vp]),
        "rxw8_xla_gqa_prefill": (None, [vp, POINTER(vp), c_char_p, c_size_t, vp]),
    }
    for name, (res, args) in sigs.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    return L


def _share_torch_hip_runtime():
    """Make librxw8.so bind to the HIP runtime PyTorch will use.

    PyTorch wheels for ROCm carry their own libamdhip64.so (soname
    libamdhip64.so.7, found through torch/lib). librxw8.so links
    libamdhip64.so.7 from /opt/rocm. Whichever is mapped first satisfies the
    soname; if /opt/rocm's is, a later `import torch` maps a second HIP and
    HSA runtime by path and finds no GPU. Preloading torch's copy by path
    (without importing torch) leaves one runtime in the process, so device
    pointers and streams can be shared both ways. RXW8_SYSTEM_HIP=1 keeps
    /opt/rocm's runtime (for processes that never use torch).
    """
    if os.environ.get("RXW8_SYSTEM_HIP") == "1":
        return
    import importlib.util
    try:
        spec = importlib.util.find_spec("torch")
    except (ImportError, ValueError):
        return
    if spec is None or not spec.submodule_search_locations:
        return
    for d in spec.submodule_search_locations:
        path = os.path.join(d, "lib", "libamdhip64.so")
        if os.path.exists(path):
            ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
            return


def load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
            "g.build()'` (there is no CPU fallback for the rxw8 kernels)")
    _share_torch_hip_runtime()
    return _declare(ctypes.CDLL(LIB_PATH))
