"""Writes the golden fixtures in tests/golden/ from the reference's own tests.

Each fixture restates the inputs and the expected values that a reference test
holds (the reference computes its expectations with f64 loops or literal
tables inside the test). Nothing here imports or runs the reference; the
sources were read as text. Run: ``python tests/golden/make_golden.py``.

Fixtures (npz without pickles, or JSON):
* cast_kat.json          crates/rxla-core/tests/cast.rs:14-28
* gqa_head_masks.npz     crates/rxla-core/tests/gqa.rs:32-102
* masked_decode.npz      crates/rxla-core/tests/masked_decode.rs:54-142
* kv_clamp.json          crates/rxla-core/tests/kv_cache.rs:114-172
* kv_checked.json        crates/rxla-core/tests/kv_cache_checked.rs:3-101
* argmax.npz             crates/rxla-core/tests/argmax.rs:30-110
* rounding.npz           crates/rxla-core/tests/rounding.rs:23-102 (round_ties_even rows)
* causal_attention.npz   crates/rxla-core/tests/causal_attention.rs:25-70,93-175
"""
from __future__ import annotations

import hashlib
import json
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F32 = np.float32


def f32(x):
    return float(np.float32(x))


def cast_kat():
    # tests/cast.rs:25-27: [0, 1, -2.5, 0.3333, 1000.25] through F16 and BF16.
    return {"input": [0.0, 1.0, -2.5, 0.3333, 1000.25],
            "f16": [0.0, 1.0, -2.5, 0.33325195, 1000.0],
            "bf16": [0.0, 1.0, -2.5, 0.33398438, 1000.0]}


def gqa_head_masks():
    # tests/gqa.rs:36-47,57-62: q [2,4,3,2]; mask [1,4,3,4] broadcast over batch.
    qv = np.array([f32((i % 9.0 - 4.0) / 5.0) for i in range(48)], F32)
    mask = np.array([-np.inf if i % 4 == 3 else f32((i % 7.0) / 8.0) for i in range(48)], F32)
    out = {"q": qv.reshape(2, 4, 3, 2), "mask": mask.reshape(1, 4, 3, 4)}
    for kv_heads in (1, 2, 4):
        keys = np.array([f32((i % 11.0 - 5.0) / 7.0) for i in range(2 * kv_heads * 4 * 2)], F32)
        values = np.array([f32((i % 13.0 - 6.0) / 3.0) for i in range(2 * kv_heads * 4 * 3)], F32)
        expected = []
        # tests/gqa.rs:63-93: f64 loops, kv = head / (4 / kv_heads)
        for batch in range(2):
            for head in range(4):
                for row in range(3):
                    kv = head // (4 // kv_heads)
                    logits = []
                    for col in range(4):
                        dot = sum(float(qv[((batch * 4 + head) * 3 + row) * 2 + d]) *
                                  float(keys[((batch * kv_heads + kv) * 4 + col) * 2 + d])
                                  for d in range(2))
                        logits.append(dot / math.sqrt(2.0) +
                                      float(mask[(head * 3 + row) * 4 + col]))
                    mx = max(logits)
                    probs = [math.exp(v - mx) for v in logits]
                    s = sum(probs)
                    for d in range(3):
                        expected.append(sum(probs[c] / s *
                                            float(values[((batch * kv_heads + kv) * 4 + c) * 3 + d])
                                            for c in range(4)))
        out[f"k{kv_heads}"] = keys.reshape(2, kv_heads, 4, 2)
        out[f"v{kv_heads}"] = values.reshape(2, kv_heads, 4, 3)
        out[f"expected{kv_heads}"] = np.array(expected, np.float64).reshape(2, 4, 3, 3)
    return out


def masked_decode():
    # tests/masked_decode.rs:96-141: cache [2 heads, 4 positions, 2 dims] starts
    # at 100 (K) / 1000 (V); step s writes k/v at position s, q attends to
    # positions <= s. Expected outputs and probabilities from f64 loops.
    qs, ks, vs, outs, probs = [], [], [], [], []
    keys, values = [], []
    for step in range(4):
        s = float(step)
        q = [f32(0.5 + s / 4.0), -0.25, 0.75, f32(0.1 + s / 3.0)]
        k = [f32(s / 2.0), 0.5, f32(1.0 - s / 3.0), -0.25]
        v = [s + 1.0, -s, 2.0 * s, 0.25 + s]
        keys.append(k)
        values.append(v)
        out = np.zeros((2, 2), np.float64)
        p = np.zeros((2, 4), np.float64)
        for head in range(2):
            logits = [sum(float(q[head * 2 + d]) * float(key[head * 2 + d]) for d in range(2)) /
                      math.sqrt(2.0) for key in keys]
            mx = max(logits)
            ex = [math.exp(l - mx) for l in logits]
            den = sum(ex)
            for d in range(2):
                out[head, d] = sum(val[head * 2 + d] * e / den for val, e in zip(values, ex))
            for t in range(4):
                p[head, t] = ex[t] / den if t <= step else 0.0
        qs.append(q)
        ks.append(k)
        vs.append(v)
        outs.append(out)
        probs.append(p)
    return {"q": np.array(qs, F32).reshape(4, 2, 1, 2), "k": np.array(ks, F32).reshape(4, 2, 1, 2),
            "v": np.array(vs, F32).reshape(4, 2, 1, 2), "expected": np.array(outs),
            "probabilities": np.array(probs), "init_k": np.float32(100.0),
            "init_v": np.float32(1000.0)}


def kv_clamp():
    # tests/kv_cache.rs:125-159: cache [3,1]; updates (position, key, value)
    # clamp -5 -> 0 and 99 -> 2; a later start of 1 writes the middle row.
    return {"shape": [3, 1], "update_shape": [1, 1],
            "steps": [[-5, 1.0, 10.0], [99, 3.0, 30.0], [1, 2.0, 20.0]],
            "expected_keys": [1.0, 2.0, 3.0], "expected_values": [10.0, 20.0, 30.0]}


def kv_checked():
    # tests/kv_cache_checked.rs:44-101: cache [4,2], update [2,2] at (row, col).
    steps = [[0, 0, True], [-1, 0, False], [3, 0, False], [2, 0, True], [1, 1, False],
             [2147483647, 0, False], [1, 0, True]]
    ek, ev = [0.0] * 8, [0.0] * 8
    rows = []
    for step, (row, col, valid) in enumerate(steps):
        data = [float(step + 1)] * 4 if valid else [float("nan")] * 4
        vals = [-x for x in data] if valid else [float("inf")] * 4
        if valid:
            ek[row * 2:row * 2 + 4] = data
            ev[row * 2:row * 2 + 4] = vals
        rows.append({"row": row, "col": col, "valid": valid,
                     "keys": [None if math.isnan(x) else x for x in data],
                     "values": vals, "accepted": 1.0 if valid else 0.0,
                     "expected_keys": list(ek), "expected_values": list(ev)})
    return {"shape": [4, 2], "update_shape": [2, 2], "steps": rows}


def argmax():
    # tests/argmax.rs:30-40 reference(): first max wins, a NaN beats numbers
    # and the first NaN wins.
    def reference(values, outer, length, inner):
        out = []
        for o in range(outer):
            for j in range(inner):
                best = 0
                for i in range(1, length):
                    a = values[(o * length + i) * inner + j]
                    b = values[(o * length + best) * inner + j]
                    if not math.isnan(b) and (math.isnan(a) or a > b):
                        best = i
                out.append(best)
        return out

    values = [float((i % 7) - 3) for i in range(24)]
    values[1] = float("nan")
    values[17] = float("nan")
    values[3] = float("inf")
    values[7] = float("inf")
    values[10] = float("-inf")
    res = {"x234": np.array(values, F32).reshape(2, 3, 4)}
    for axis, (outer, length, inner) in enumerate([(1, 2, 12), (2, 3, 4), (6, 4, 1)]):
        res[f"axis{axis}"] = np.array(reference(values, outer, length, inner), np.int32)
    rows = [[-np.inf] * 6, [0.0, -0.0, 0.0, -0.0, 0.0, -0.0], [1.0, 4.0, 4.0, 2.0, 4.0, 3.0],
            [np.inf] * 6, [np.nan] * 6, [np.inf, 2.0, np.nan, np.nan, 5.0, 1.0]]
    res["rows6"] = np.array(rows, F32)
    res["rows6_expected"] = np.array([reference(r, 1, 6, 1)[0] for r in rows], np.int32)
    return res


def rounding():
    # tests/rounding.rs:26-45 data; expected = f32::round_ties_even.
    data = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 0.0, -0.0, np.inf, -np.inf, np.nan,
                     np.finfo(F32).max, -np.finfo(F32).max], F32)
    extra = np.array([0x3effffff, 0x3f000001], np.uint32).view(F32)
    tail = np.array([-0.1, 0.1, 16777216.0], F32)
    x = np.concatenate([data, extra, tail]).astype(F32)
    return {"x": x, "expected": np.rint(x).astype(F32)}


def causal_attention():
    imax, imin = 2 ** 31 - 1, -2 ** 31
    out = {}
    # causal_attention.rs:35-56: q, k zero vectors (every score 0), scale 1,
    # key positions [0, 1, 2, 3], values [10, 20, 30, 40]; with query positions
    # [0, 2] the rows average values 0..0 and 0..2, with [1, 3] 0..1 and 0..3
    out["rt_kpos"] = np.array([0, 1, 2, 3], np.int32)
    out["rt_v"] = np.array([[10.0], [20.0], [30.0], [40.0]], F32)
    out["rt_qpos"] = np.array([[0, 2], [1, 3]], np.int32)
    out["rt_expected"] = np.array([[10.0, 20.0], [15.0, 25.0]], F32)
    # causal_attention.rs:59-69: extreme I32 positions, mask [2, 4]
    out["x_qpos"] = np.array([16_777_216, imax], np.int32)
    out["x_kpos"] = np.array([16_777_216, 16_777_217, imax, imin], np.int32)
    out["x_mask"] = np.array([[0.0, -np.inf, -np.inf, 0.0], [0.0, 0.0, 0.0, 0.0]], F32)
    # causal_attention.rs:72-91: static masks; rows (queries, keys, offset)
    out["static_bad"] = np.array([[-1, 2, 0], [2, -1, 0], [2, 2, -1], [2, 2, imax],
                                  [1, 2 ** 63 - 1, 0]], np.int64)
    out["static_ok"] = np.array([[0, 4, 0], [1, 1, imax]], np.int64)
    out["static_241"] = np.array([[0.0, 0.0, -np.inf, -np.inf], [0.0, 0.0, 0.0, -np.inf]], F32)
    # causal_attention.rs:93-175: q [5, 2], k [7, 2], v [7, 2], causal mask
    # (5, 7, 0), scale 1; chunks (0, 2), (2, 5), (4, 5) with offset = start
    # equal the full rows; row i = softmax over keys 0..i, in f64
    qv = np.array([f32((i - 3.0) * 0.125) for i in range(10)], F32).reshape(5, 2)
    kv = np.array([f32((i - 6.0) * 0.125) for i in range(14)], F32).reshape(7, 2)
    vv = np.array([f32((i - 5.0) * 0.25) for i in range(14)], F32).reshape(7, 2)
    full = np.zeros((5, 2))
    for i in range(5):
        sc = [math.exp(sum(float(qv[i, d]) * float(kv[j, d]) for d in range(2)))
              for j in range(i + 1)]
        tot = sum(sc)
        for d in range(2):
            full[i, d] = sum(sc[j] / tot * float(vv[j, d]) for j in range(i + 1))
    out.update(full_q=qv, full_k=kv, full_v=vv, full_expected=full,
               chunks=np.array([[0, 2], [2, 5], [4, 5]], np.int64))
    return out


def main():
    manifest = {}

    def save_json(name, obj):
        path = os.path.join(HERE, name)
        with open(path, "w") as f:
            json.dump(obj, f, indent=1, allow_nan=True)
        manifest[name] = hashlib.sha256(open(path, "rb").read()).hexdigest()

    def save_npz(name, arrays):
        path = os.path.join(HERE, name)
        np.savez(path, **arrays)
        manifest[name] = hashlib.sha256(open(path, "rb").read()).hexdigest()

    save_json("cast_kat.json", cast_kat())
    save_npz("gqa_head_masks.npz", gqa_head_masks())
    save_npz("masked_decode.npz", masked_decode())
    save_json("kv_clamp.json", kv_clamp())
    save_json("kv_checked.json", kv_checked())
    save_npz("argmax.npz", argmax())
    save_npz("rounding.npz", rounding())
    save_npz("causal_attention.npz", causal_attention())
    with open(os.path.join(HERE, "MANIFEST.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print(json.dumps(manifest, indent=1))


if __name__ == "__main__":
    main()
