"""GPU side of the safetensors loader: payload uploads with the reference's
dtype rules (crates/rxla-safetensors/src/model.rs:340-440) and a whole decoder
bound from a checkpoint laid out like the output of
benchmarks/quantize_qwen3_5_w8.py (separate q/k/v and gate/up projections,
U8 codes + F32 ".scale", F32 norms, names under "model.language_model.")."""
import numpy as np
import pytest

import oracle
import st_fixtures as stf
from decoder_fixtures import tiny_config, tiny_params

pytestmark = pytest.mark.gpu


def rx():
    import rxla_amd
    return rxla_amd


SPECIAL = np.array([0.0, -0.0, 1.0, -1.5, 3.3333333, 65504.0, 65520.0, 1e5, -1e5, 6.1e-5,
                    5.96e-8, 2.98e-8, 1e-9, 1.0009765625, 1.00146484375, np.inf, -np.inf,
                    np.nan, 1e38, -3.4e38, 1.1754944e-38, 1e-40], np.float32)


def test_upload_conversions_are_bit_exact(rt, tmp_path):
    """F32 -> BF16 / F16 round to nearest even (oracle bf16, numpy f16);
    F16 / BF16 -> F32 exactly; U8 and I32 verbatim."""
    r = rx()
    rng = np.random.default_rng(5)
    f = np.concatenate([SPECIAL, (rng.standard_normal(4000) * 10.0 ** rng.integers(-8, 6, 4000))
                        .astype(np.float32)])
    with np.errstate(over="ignore"):  # values beyond f16's range round to +-inf, as intended
        h = f.astype(np.float16)
    b = oracle.bf16_bits(f)
    u = rng.integers(0, 256, 300).astype(np.uint8)
    i = rng.integers(-2**31, 2**31, 77).astype(np.int32)
    p = tmp_path / "c.safetensors"
    stf.write(p, {"f": ("F32", f), "h": ("F16", h), "b": ("BF16", b), "u": ("U8", u), "i": ("I32", i)})
    with r.SafeTensors(p) as st:
        def got(name, dt):
            return st.to_buffer(rt, name, dt).to_numpy()
        np.testing.assert_array_equal(got("f", r.DType.BF16), b)
        np.testing.assert_array_equal(got("f", r.DType.F16).view(np.uint16), h.view(np.uint16))
        np.testing.assert_array_equal(got("f", r.DType.F32).view(np.uint32), f.view(np.uint32))
        hf = got("h", r.DType.F32)
        np.testing.assert_array_equal(np.isnan(hf), np.isnan(h))
        ok = ~np.isnan(h)
        np.testing.assert_array_equal(hf[ok], h[ok].astype(np.float32))
        np.testing.assert_array_equal(got("h", r.DType.BF16)[ok], oracle.bf16_bits(h[ok].astype(np.float32)))
        bf = got("b", r.DType.F32)
        np.testing.assert_array_equal(bf.view(np.uint32)[~np.isnan(f)],
                                      (b.astype(np.uint32) << 16)[~np.isnan(f)])
        np.testing.assert_array_equal(got("u", None), u)
        np.testing.assert_array_equal(got("i", None), i)


def test_upload_offsets_and_errors(rt, tmp_path):
    r = rx()
    p = tmp_path / "o.safetensors"
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    c = -np.arange(9, dtype=np.float32).reshape(3, 3)
    stf.write(p, {"a": ("F32", a), "c": ("F32", c), "u": ("U8", np.ones((2, 3), np.uint8))})
    with r.SafeTensors(p) as st:
        buf = rt.zeros((5, 3), r.DType.F32)
        st.upload("a", buf, 0)
        st.upload("c", buf, 6)  # rows stacked one after another (fused projections)
        np.testing.assert_array_equal(buf.to_numpy(), np.concatenate([a, c]))
        with pytest.raises(r.Error) as e:
            st.upload("c", buf, 7)  # 9 elements at 7 exceed 15
        assert e.value.code == r.Status.OUT_OF_RANGE
        with pytest.raises(r.Error) as e:
            st.upload("a", rt.zeros((2, 3), r.DType.U8))  # float payload into U8 storage
        assert e.value.code == r.Status.INVALID_ARGUMENT
        with pytest.raises(r.Error) as e:
            st.upload("u", rt.zeros((2, 3), r.DType.F32))  # U8 payload into float storage
        assert e.value.code == r.Status.INVALID_ARGUMENT
        with pytest.raises(r.Error) as e:
            st.upload("nope", buf)
        assert e.value.code == r.Status.NOT_FOUND


def small_cfg():
    return tiny_config(layers=2, hidden=512, q_heads=4, kv_heads=2, head_dim=128,
                       intermediate=1024, vocab=1008, max_seq=40, group=128)


def reference_checkpoint(cfg, params, embed="bf16"):
    """The tiny decoder's parameters under the reference encoder's names,
    with the fused projections split back into their parts."""
    H, D, I = cfg["hidden"], cfg["head_dim"], cfg["intermediate"]
    HQ, HKV = cfg["q_heads"], cfg["kv_heads"]
    pre = "model.language_model."
    t = {}
    for path, v in params.items():
        if ".qkv_proj." in path:
            kind = path.rsplit(".", 1)[1]
            base = path.replace("qkv_proj." + kind, "")
            dt = "U8" if kind == "weight" else "F32"
            edges = [0, HQ * D, (HQ + HKV) * D, (HQ + 2 * HKV) * D]
            for name, lo, hi in zip(("q_proj", "k_proj", "v_proj"), edges, edges[1:]):
                t[pre + base + name + "." + kind] = (dt, v[lo:hi])
        elif ".gate_up_proj." in path:
            kind = path.rsplit(".", 1)[1]
            base = path.replace("gate_up_proj." + kind, "")
            dt = "U8" if kind == "weight" else "F32"
            t[pre + base + "gate_proj." + kind] = (dt, v[:I])
            t[pre + base + "up_proj." + kind] = (dt, v[I:])
        elif path == "embed_tokens.weight":
            f32 = oracle.bf16_to_f32(v)
            if embed == "bf16":
                t[pre + path] = ("BF16", v)
            elif embed == "f32":
                t[pre + path] = ("F32", f32)
            else:  # W8 embedding, as the encoder writes every 2-D tensor
                u8, s = oracle.quantize_w8(f32, 128)
                t[pre + path] = ("U8", u8)
                t[pre + "embed_tokens.scale"] = ("F32", s)
        elif v.dtype == np.uint8:
            t[pre + path] = ("U8", v)
        else:
            t[pre + path] = ("F32", v)
    return t


def build(rt, cfg, batch=2):
    r = rx()
    dc = r.DecoderConfig(layers=cfg["layers"], hidden=cfg["hidden"], q_heads=cfg["q_heads"],
                         kv_heads=cfg["kv_heads"], head_dim=cfg["head_dim"],
                         intermediate=cfg["intermediate"], vocab=cfg["vocab"], max_batch=batch,
                         max_seq=cfg["max_seq"], group=cfg["group"], eps=cfg["eps"],
                         theta=cfg["theta"], qk_norm=cfg["qk_norm"])
    return r.DecoderModel(rt, dc).compile()


def run(rt, model, ids_list, vocab):
    r = rx()
    outs = []
    for ids in ids_list:
        lg = rt.zeros((ids.shape[0], vocab), r.DType.F32)
        model.forward(rt.buffer(ids), logits=lg)
        outs.append(lg.to_numpy())
    return np.stack(outs)


@pytest.mark.parametrize("embed", ["bf16", "f32", "w8"])
def test_decoder_from_reference_checkpoint_matches_direct_binding(rt, tmp_path, embed):
    """Logits of a decoder loaded from the checkpoint equal, bit for bit, those
    of the same decoder bound directly with the values the loader must produce
    (an F32 embedding rounds to bf16; a W8 one dequantises to bf16((u-128)s))."""
    cfg = small_cfg()
    params = tiny_params(cfg, seed=123, std=0.05)
    ckpt = reference_checkpoint(cfg, params, embed)
    p = tmp_path / "w8.safetensors"
    stf.write(p, ckpt, {"format": "rxla-qwen3.5-w8-v1", "group_size": "128"})
    direct = dict(params)
    if embed == "w8":
        pre = "model.language_model."
        direct["embed_tokens.weight"] = oracle.bf16_bits(
            oracle.dequantize_w8(ckpt[pre + "embed_tokens.weight"][1], ckpt[pre + "embed_tokens.scale"][1]))
    a = build(rt, cfg)
    for path, dtype, shape in a.schema():
        a.bind_parameter(path, rt.buffer(direct[path], dtype))
    b = build(rt, cfg).load_safetensors(p)
    rng = np.random.default_rng(124)
    ids = [rng.integers(0, cfg["vocab"], (2, 20)).astype(np.int32),
           rng.integers(0, cfg["vocab"], (2, 1)).astype(np.int32)]
    np.testing.assert_array_equal(run(rt, a, ids, cfg["vocab"]), run(rt, b, ids, cfg["vocab"]))


def test_checkpoint_validation_happens_before_upload(rt, tmp_path):
    r = rx()
    cfg = small_cfg()
    params = tiny_params(cfg, seed=125)
    ckpt = reference_checkpoint(cfg, params)
    pre = "model.language_model."
    del ckpt[pre + "layers.1.self_attn.v_proj.weight"]
    k = pre + "layers.0.mlp.down_proj.weight"
    ckpt[k] = ("U8", ckpt[k][1][:, :-128])  # wrong shape
    p = tmp_path / "bad.safetensors"
    stf.write(p, ckpt)
    model = build(rt, cfg)
    with pytest.raises(r.Error) as e:
        model.load_safetensors(p)
    assert e.value.code == r.Status.INVALID_ARGUMENT
    msg = str(e.value)
    assert "v_proj" in msg and "down_proj" in msg
    assert model._bound == []  # nothing was uploaded or bound
    p2 = tmp_path / "g.safetensors"
    stf.write(p2, reference_checkpoint(cfg, params), {"group_size": "64"})
    with pytest.raises(r.Error) as e:
        build(rt, cfg).load_safetensors(p2)
    assert "group_size" in str(e.value)
