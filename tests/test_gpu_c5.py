"""The C5 decoder at its configured size: 28 layers,
hidden 2048, 16 q / 8 kv heads x 128, SwiGLU 6144, vocab 151936 (bf16
embedding reused as lm_head), per-output-channel W8 projections encoded on the
device by rxw8_quantize_w8 from N(0, 0.02) weights, batch 8.

* Against the CPU oracle decoder (crates/rxla-models/src/qwen3_5/mod.rs:199-273
  restated in oracle/rxw8_oracle.c): an 8 x 16 prompt and 4 greedy decode
  steps, every side fed the same ids. At 28 layers the network amplifies
  summation-order noise: the oracle with f32 accumulation and the oracle
  with f64 accumulation (same bf16 cast points) differ by about 1.5e-2,
  above the north-star 1e-2. The teacher-forced test below shows that every
  layer's own arithmetic stays within 1e-2 of the oracle's; so end to end
  the GPU logits must lie within max(1e-2, 2 x that floor) of the f64
  oracle, the floor measured in the test on the same inputs.
* Layer by layer (teacher forcing through rxw8_decoder_forward_layers): each
  of the 28 layers fed the oracle's own input, within 1e-2 normwise.
* At full size on the GPU alone (prompt 8 x 1024, 256 greedy steps): finite
  logits at every step, each id equal to the first maximum of its step's
  logits, graph replay (generate) equal to the eager step-by-step ids, and
  lengths 1280 at the end."""
import numpy as np
import pytest

import oracle
from conftest import elem_rel_err, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-2  # max relative error on logits, normwise


def rx():
    import rxla_amd
    return rxla_amd


@pytest.fixture(scope="module")
def c5(rt):
    """The full C5 model bound on the GPU plus host copies of every parameter."""
    import torch

    r = rx()
    from rxla_amd.model import DecoderConfig, DecoderModel
    cfg = DecoderConfig(max_batch=8, max_seq=1280)
    model = DecoderModel(rt, cfg).compile()
    gen = torch.Generator(device="cuda").manual_seed(2025)
    host = {}
    pending = {}
    for path, dtype, shape in model.schema():
        if path.endswith(".scale"):
            buf = pending.pop(path)
        elif dtype == r.DType.U8:
            w = torch.randn(shape, device="cuda", generator=gen) * 0.02
            torch.cuda.synchronize()
            buf, sc = r.quantize_w8(rt, rt.wrap_tensor(w), shape[1])  # per output channel
            rt.synchronize()
            del w
            pending[path[:-len(".weight")] + ".scale"] = sc
        elif dtype == r.DType.BF16:
            t = (torch.randn(shape, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
            host[path] = t.view(torch.int16).cpu().numpy().view(np.uint16)
            buf = rt.buffer(host[path], r.DType.BF16)
            del t
        else:
            t = 1.0 + 0.1 * torch.randn(shape, device="cuda", generator=gen)
            host[path] = t.cpu().numpy().astype(np.float32)
            buf = rt.buffer(host[path])
        if path not in host:
            host[path] = buf.to_numpy()
        model.bind_parameter(path, buf)
    rt.synchronize()
    c = cfg.as_dict()
    c["max_seq"] = 32
    return model, c, host


ORDERS = {
    # the product schedule: every weight bf16((u - 128) * s) before the
    # product (the reference's cast point, layers.rs:288-297); decode steps
    # apply each RMSNorm's row factor after the projection it feeds
    "default": {},
    # the reference's order throughout: every RMSNorm applied before the bf16
    # cast of the projection input
    "reference": {"RXW8_DEC_ROW_NORM": "0"},
    # exact codes u - 128 with the scale after the f32 sum (not the
    # reference's cast point; measured for comparison only)
    "exact_codes": {"RXW8_GEMV_REF_CAST": "0"},
}
# Per element of a layer's contribution, floored at its rms: the contribution
# is the sum of two bf16-rounded branch outputs (o_proj, down), so one-ulp
# flips (2^-8 relative) of elements near the rms and their propagation through
# the layer's norms and SwiGLU bound it; the measured maximum over the 28 layers
# and both steps is 3.2e-2.
ELEM_LAYER_TOL = 5e-2


@pytest.mark.parametrize("order", list(ORDERS))
def test_c5_short_prompt_matches_oracle(rt, c5, order, monkeypatch):
    for k, v in ORDERS[order].items():
        monkeypatch.setenv(k, v)
    r = rx()
    model, cfg, host = c5
    batch, s, steps = 8, 16, 4
    model.reset()
    dec64 = oracle.Decoder(dict(cfg, accum=oracle.ACCUM_F64), host, batch)
    dec32 = oracle.Decoder(cfg, host, batch)
    ids = np.random.default_rng(16).integers(0, cfg["vocab"], (batch, s)).astype(np.int32)
    for step in range(steps + 1):
        logits = rt.zeros((batch, cfg["vocab"]), r.DType.F32)
        nxt = model.forward(rt.buffer(ids), logits=logits).to_numpy()
        got = logits.to_numpy()
        want, want_next = dec64.forward(ids)
        other, _ = dec32.forward(ids)
        floor = rel_err(other, want)
        err = rel_err(got, want)
        print(f"C5 {order} step {step}: GPU vs f64 oracle rel_err={err:.3e} (vs f32 oracle "
              f"{rel_err(got, other):.3e}); f32 vs f64 oracle {floor:.3e}; "
              f"elem(floor rms) {elem_rel_err(got, want, floor=1.0):.3e}; argmax agreement "
              f"{float((nxt == want_next).mean()):.3f}", flush=True)
        assert np.isfinite(got).all()
        assert err <= max(TOL, 2.0 * floor)
        ids = want_next.reshape(batch, 1).astype(np.int32)  # every side takes the same ids
    np.testing.assert_array_equal(model.lens(), [s + steps] * batch)


@pytest.mark.parametrize("order", ["default", "reference"])
def test_c5_layerwise_teacher_forced(rt, c5, order, monkeypatch):
    """Each of the 28 layers, fed the f64 oracle's own input for that layer
    (teacher forcing through rxw8_decoder_forward_layers), against the oracle
    layer's output: an 8 x 16 prompt step, then one decode step whose keys
    are the teacher-forced prompt's. The layer's own contribution
    (output - input: attention and MLP branches) must be within 1e-2 normwise
    of the oracle's, so summation noise amplified through earlier layers is
    not charged to this one."""
    for k, v in ORDERS[order].items():
        monkeypatch.setenv(k, v)
    r = rx()
    model, cfg, host = c5
    batch, s = 8, 16
    L, V = cfg["layers"], cfg["vocab"]
    model.reset()
    dec = oracle.Decoder(dict(cfg, accum=oracle.ACCUM_F64), host, batch)
    ids = np.random.default_rng(16).integers(0, V, (batch, s)).astype(np.int32)
    worst = []
    for step in range(2):
        want, want_next, hs = dec.forward(ids, trace=True)
        for l in range(L):
            logits = rt.zeros((batch, V), r.DType.F32) if l == L - 1 else None
            out = model.forward_layers(rt.buffer(hs[l]), l, l + 1, logits=logits,
                                       commit=l == L - 1).to_numpy()
            d_gpu, d_ref = out - hs[l], hs[l + 1] - hs[l]
            e_delta, e_res = rel_err(d_gpu, d_ref), rel_err(out, hs[l + 1])
            e_elem = elem_rel_err(d_gpu, d_ref, floor=1.0)
            worst.append((e_delta, e_elem, step, l))
            print(f"C5 {order} step {step} layer {l:2d}: layer delta rel_err={e_delta:.3e} "
                  f"elem(floor rms)={e_elem:.3e}; residual rel_err={e_res:.3e}", flush=True)
        got = logits.to_numpy()
        print(f"C5 {order} step {step} logits (tail after teacher-forced layer {L - 1}): "
              f"rel_err={rel_err(got, want):.3e}", flush=True)
        ids = want_next.reshape(batch, 1).astype(np.int32)
    np.testing.assert_array_equal(model.lens(), [s + 1] * batch)
    worst.sort(reverse=True)
    print(f"C5 {order} worst layer deltas: {worst[:3]}", flush=True)
    assert worst[0][0] <= TOL, worst[:3]
    assert max(w[1] for w in worst) <= ELEM_LAYER_TOL, worst


def test_c5_full_size_generate_properties(rt, c5):
    r = rx()
    model, cfg, _ = c5
    batch, s, steps = 8, 1024, 256
    prompt = np.random.default_rng(5).integers(0, cfg["vocab"], (batch, s)).astype(np.int32)
    model.reset()
    eager = np.zeros((batch, steps + 1), np.int32)
    logits = rt.zeros((batch, cfg["vocab"]), r.DType.F32)
    ids = rt.buffer(prompt)
    for step in range(steps + 1):
        nxt = model.forward(ids, logits=logits).to_numpy()
        lg = logits.to_numpy()
        assert np.isfinite(lg).all(), f"non-finite logits at step {step}"
        np.testing.assert_array_equal(nxt, np.argmax(lg, axis=1))  # first maximum
        eager[:, step] = nxt
        ids = rt.buffer(nxt.reshape(batch, 1))
    # the prompt, then 256 single ids at positions 1024 .. 1279
    np.testing.assert_array_equal(model.lens(), [s + steps] * batch)
    model.reset()
    out = model.generate(rt.buffer(prompt), steps, use_graph=True).to_numpy()
    np.testing.assert_array_equal(model.lens(), [s + steps] * batch)
    print(f"C5 full size: {len(np.unique(out))} distinct ids over {out.size}; "
          f"graph == eager: {bool((out == eager).all())}", flush=True)
    np.testing.assert_array_equal(out, eager)
