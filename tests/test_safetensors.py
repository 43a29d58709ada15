"""The safetensors reader's header handling (no GPU): what the reference's
checkpoint loader validates before reading payloads
(crates/rxla-safetensors/src/model.rs:340-440), against files written here and
by the safetensors package itself."""
import numpy as np
import pytest

import st_fixtures as stf


def rx():
    import rxla_amd
    return rxla_amd


def test_reads_names_dtypes_shapes_metadata(tmp_path):
    r = rx()
    p = tmp_path / "a.safetensors"
    stf.write(p, {"w": ("U8", np.arange(12, dtype=np.uint8).reshape(3, 4)),
                  "s": ("F32", np.ones((3, 1), np.float32)),
                  "e": ("BF16", np.zeros((2, 5), np.uint16)),
                  "h": ("F16", np.zeros(7, np.float16)),
                  "i": ("I32", np.zeros((1, 1, 2), np.int32)),
                  "big": ("I64", np.zeros(3, np.int64)),
                  "scalar": ("F32", np.float32(3.0))},
              {"format": "rxla-qwen3.5-w8-v1", "group_size": "128"})
    with r.SafeTensors(p) as st:
        t = st.tensors()
        assert t["w"] == (r.DType.U8, (3, 4))
        assert t["s"] == (r.DType.F32, (3, 1))
        assert t["e"] == (r.DType.BF16, (2, 5))
        assert t["h"] == (r.DType.F16, (7,))
        assert t["i"] == (r.DType.I32, (1, 1, 2))
        assert t["big"] == (None, (3,))  # listed, not representable
        assert t["scalar"] == (r.DType.F32, ())
        assert st.metadata("format") == "rxla-qwen3.5-w8-v1"
        assert st.metadata("group_size") == "128"
        assert st.metadata("absent") is None


def test_reads_files_of_the_safetensors_package(tmp_path):
    from safetensors.numpy import save_file
    r = rx()
    p = tmp_path / "pkg.safetensors"
    save_file({"model.layers.0.mlp.down_proj.weight": np.zeros((4, 8), np.uint8),
               "model.layers.0.mlp.down_proj.scale": np.zeros((4, 1), np.float32),
               "model.norm.weight": np.ones(8, np.float32)}, str(p),
              metadata={"format": "rxla-qwen3.5-w8-v1", "group_size": "8"})
    with r.SafeTensors(p) as st:
        t = st.tensors()
        assert t["model.layers.0.mlp.down_proj.weight"] == (r.DType.U8, (4, 8))
        assert t["model.norm.weight"] == (r.DType.F32, (8,))
        assert st.metadata("group_size") == "8"


def test_unicode_names_and_escapes(tmp_path):
    r = rx()
    p = tmp_path / "u.safetensors"
    # JSON text with a \u escape, an escaped quote and a surrogate pair
    hdr = (b'{"a\\u00e9\\"b": {"dtype": "U8", "shape": [2], "data_offsets": [0, 2]}, '
           b'"\\ud83d\\ude00": {"dtype": "U8", "shape": [1], "data_offsets": [2, 3]}}')
    stf.write_raw(p, hdr, b"\x01\x02\x03")
    with r.SafeTensors(p) as st:
        names = set(st.tensors())
        assert "aé\"b" in names
        assert "\U0001F600" in names


def expect_error(r, path, code):
    with pytest.raises(r.Error) as e:
        r.SafeTensors(path)
    assert e.value.code == code, e.value
    return str(e.value)


@pytest.mark.parametrize("case", ["short_file", "header_too_long", "bad_json", "trailing",
                                  "not_object", "size_mismatch", "past_end", "overlap",
                                  "unknown_dtype", "bad_shape", "negative_offset", "duplicate",
                                  "metadata_not_string", "missing_field", "numel_wraps",
                                  "bytes_overflow"])
def test_malformed_headers(tmp_path, case):
    r = rx()
    p = tmp_path / f"{case}.safetensors"
    ok = {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]}
    data = b"\0" * 8
    if case == "short_file":
        p.write_bytes(b"\x01\x02")
    elif case == "header_too_long":
        stf.write_raw(p, {"a": ok}, data, length_override=10_000)
    elif case == "bad_json":
        stf.write_raw(p, b'{"a": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]', data)
    elif case == "trailing":
        stf.write_raw(p, b'{"a": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]}} x', data)
    elif case == "not_object":
        stf.write_raw(p, b'[1, 2]', data)
    elif case == "size_mismatch":
        stf.write_raw(p, {"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 4]}}, data)
    elif case == "past_end":
        stf.write_raw(p, {"a": {"dtype": "U8", "shape": [16], "data_offsets": [0, 16]}}, data)
    elif case == "overlap":
        stf.write_raw(p, {"a": ok, "b": {"dtype": "U8", "shape": [4], "data_offsets": [2, 6]}}, data)
    elif case == "unknown_dtype":
        stf.write_raw(p, {"a": {"dtype": "Q4", "shape": [4], "data_offsets": [0, 4]}}, data)
    elif case == "bad_shape":
        stf.write_raw(p, {"a": {"dtype": "U8", "shape": [2.5], "data_offsets": [0, 4]}}, data)
    elif case == "negative_offset":
        stf.write_raw(p, {"a": {"dtype": "U8", "shape": [4], "data_offsets": [-1, 3]}}, data)
    elif case == "duplicate":
        stf.write_raw(p, b'{"a": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]}, '
                         b'"a": {"dtype": "U8", "shape": [4], "data_offsets": [4, 8]}}', data)
    elif case == "metadata_not_string":
        stf.write_raw(p, {"a": ok, "__metadata__": {"group_size": 128}}, data)
    elif case == "missing_field":
        stf.write_raw(p, {"a": {"dtype": "U8", "shape": [4]}}, data)
    elif case == "numel_wraps":  # 2^62 * 2^62 * 16 = 2^128 wraps a 128-bit count to 0
        stf.write_raw(p, {"a": {"dtype": "U8", "shape": [2 ** 62, 2 ** 62, 16],
                                "data_offsets": [0, 0]}}, data)
    elif case == "bytes_overflow":  # 2^62 F32 elements: 2^64 bytes
        stf.write_raw(p, {"a": {"dtype": "F32", "shape": [2 ** 62], "data_offsets": [0, 0]}}, data)
    msg = expect_error(r, p, r.Status.DATA_LOSS)
    assert str(p.name) in msg


def test_missing_file_and_zero_size_tensors(tmp_path):
    r = rx()
    expect_error(r, tmp_path / "nope.safetensors", r.Status.NOT_FOUND)
    p = tmp_path / "z.safetensors"
    stf.write_raw(p, {"empty": {"dtype": "F32", "shape": [0, 3], "data_offsets": [0, 0]},
                      "one": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}, b"\x07")
    with r.SafeTensors(p) as st:
        assert st.tensors()["empty"] == (r.DType.F32, (0, 3))
