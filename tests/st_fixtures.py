"""Write safetensors files byte by byte (format: u64 LE header length, JSON
header, data section), including bf16 tensors (numpy uint16 bit patterns) and
deliberately malformed headers for the reader's error tests."""
import json
import struct

import numpy as np

NP_DTYPE = {"U8": np.uint8, "I32": np.int32, "F16": np.float16, "F32": np.float32,
            "BF16": np.uint16, "I64": np.int64, "F64": np.float64}


def header_bytes(header: dict) -> bytes:
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)  # the writers pad the header to 8 bytes
    return struct.pack("<Q", len(h)) + h


def write(path, tensors: dict, metadata: dict | None = None):
    """tensors: {name: (dtype string, array)}; arrays are stored C-contiguous."""
    header, blobs, off = {}, [], 0
    for name, (dt, arr) in tensors.items():
        a = np.array(arr, dtype=NP_DTYPE[dt], order="C")  # keeps 0-d shapes
        b = a.tobytes()
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    if metadata:
        header["__metadata__"] = metadata
    with open(path, "wb") as f:
        f.write(header_bytes(header))
        for b in blobs:
            f.write(b)


def write_raw(path, header_obj_or_bytes, data: bytes = b"", length_override=None):
    h = header_obj_or_bytes if isinstance(header_obj_or_bytes, bytes) else json.dumps(
        header_obj_or_bytes).encode()
    n = len(h) if length_override is None else length_override
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", n) + h + data)
