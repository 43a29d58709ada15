"""Qwen3.5 hybrid W8 model on the GPU (rxw8_qwen35_*) against the numpy
oracle of crates/rxla-models/src/qwen3_5 (oracle/qwen35.py): logits of every
position within 1e-3 normwise at the reference's compute dtype F32 (every
projection f32 x against f32 dequantised weights, rxla-nn lib.rs:432), within
1e-2 for the BF16 opt-in; the schema equal to the reference encoder's layout
(quantize_qwen3_5_w8.py), checkpoint loading, and the error contract of
qwen3_5 / Qwen3_5Config::validate (mod.rs:100-131, 197-209)."""
import numpy as np
import pytest

import st_fixtures as stf
from conftest import rel_err
from oracle import qwen35 as q35

pytestmark = pytest.mark.gpu

TOL = 1e-3       # F32 compute (the default): logits normwise
TOL_BF16 = 1e-2  # the BF16 opt-in


def rx():
    import rxla_amd
    return rxla_amd


CONFIGS = {
    # Qwen3_5Config::tiny: every projection on the generic path (K = 32, G = 8)
    "tiny": dict(q35.config(), max_batch=2, max_seq=24),
    # widths on the MFMA GEMV / GEMM paths, D = 64 with partial RoPE, Dl = 32
    "small": dict(q35.config(vocab=512, hidden=256, intermediate=512,
                             layers=[q35.LINEAR, q35.FULL, q35.LINEAR, q35.FULL], heads=4,
                             kv_heads=2, head_dim=64, linear_heads=4, linear_head_dim=32,
                             rotary_dim=16, group=64), max_batch=2, max_seq=80),
    # the 0.8B layer widths (hidden 1024, D 256, rotary 64, Hl 16 x Dl 128,
    # intermediate 3584, G 128) on 4 layers and a 2048-entry vocabulary
    "wide": dict(q35.config(vocab=2048, hidden=1024, intermediate=3584,
                            layers=q35.layer_types(4), heads=8, kv_heads=2, head_dim=256,
                            linear_heads=16, linear_head_dim=128, rotary_dim=64, group=128),
                 max_batch=1, max_seq=32),
}
# Dl 64, D 128 with one KV head (G = 4), a vocabulary that is not a multiple
# of the head kernel's 128 channels
CONFIGS["mid"] = dict(q35.config(vocab=1000, hidden=512, intermediate=1024,
                                 layers=[q35.LINEAR, q35.LINEAR, q35.FULL], heads=4, kv_heads=1,
                                 head_dim=128, linear_heads=8, linear_head_dim=64, rotary_dim=32,
                                 group=128), max_batch=2, max_seq=64)
CONFIGS["wide_linear"] = dict(CONFIGS["wide"], layers=[q35.LINEAR], max_seq=256)
CONFIGS["small_mha"] = dict(CONFIGS["small"], kv_heads=4, layers=[q35.FULL, q35.LINEAR])  # G = 1
# sequences of >= 128 positions (Dl 64 and 128)
CONFIGS["mid_long"] = dict(CONFIGS["mid"], layers=[q35.LINEAR, q35.FULL], max_seq=200)
CONFIGS["wide_full"] = dict(CONFIGS["wide"], layers=[q35.FULL], max_seq=160)


def model_config(cfg):
    r = rx()
    return r.Qwen35Config(vocab=cfg["vocab"], hidden=cfg["hidden"], intermediate=cfg["intermediate"],
                          layers=[r.model.FULL if k == q35.FULL else r.model.LINEAR
                                  for k in cfg["layers"]],
                          heads=cfg["heads"], kv_heads=cfg["kv_heads"], head_dim=cfg["head_dim"],
                          linear_heads=cfg["linear_heads"], linear_head_dim=cfg["linear_head_dim"],
                          conv_kernel=cfg["conv_kernel"], max_positions=cfg.get("max_positions", 4096),
                          rotary_dim=cfg["rotary_dim"], group=cfg["group"], theta=cfg["theta"],
                          eps=cfg["eps"], lora_rank=cfg.get("lora_rank", 0),
                          lora_alpha=cfg.get("lora_alpha", 0.0), max_batch=cfg["max_batch"],
                          max_seq=cfg["max_seq"], compute=cfg.get("compute", "f32"))


def build(rt, cfg, params):
    m = rx().Qwen35Model(rt, model_config(cfg)).compile()
    for path, dtype, shape in m.schema():
        m.bind_parameter(path, rt.buffer(np.ascontiguousarray(params[path]), dtype))
    return m


def run(rt, m, ids):
    r = rx()
    return m.forward(rt.buffer(ids.astype(np.int32))).to_numpy()


@pytest.mark.parametrize("name,b,s", [("tiny", 2, 13), ("small", 2, 13), ("small", 2, 70),
                                      ("small", 1, 1), ("mid", 2, 37), ("mid", 1, 64),
                                      ("small_mha", 2, 45), ("wide_linear", 1, 16),
                                      ("wide_linear", 1, 203), ("wide_full", 1, 77),
                                      ("wide_full", 1, 160),
                                      ("mid_long", 2, 150), ("mid_long", 1, 200),
                                      ("wide_full", 1, 16), ("wide", 1, 16), ("wide", 1, 32)])
def test_logits_match_the_oracle(rt, name, b, s):
    cfg = CONFIGS[name]
    p = q35.random_params(cfg, seed=11, std=0.05)
    ids = np.random.default_rng(12).integers(0, cfg["vocab"], (b, s))
    got = run(rt, build(rt, cfg, p), ids)
    want = q35.forward(cfg, p, ids)
    assert got.shape == (b, s, cfg["vocab"])
    err = rel_err(got, want)
    print(f"qwen35 {name} b={b} s={s}: rel err {err:.2e}")
    assert err <= TOL
    # the greedy token of every position agrees wherever the oracle's margin is clear
    top2 = np.sort(want, axis=-1)[..., -2:]
    clear = (top2[..., 1] - top2[..., 0]) > 0.05 * np.abs(want).max()
    np.testing.assert_array_equal(got.argmax(-1)[clear], want.argmax(-1)[clear])


@pytest.mark.parametrize("name,b,s", [("mid", 2, 1), ("mid", 2, 9), ("mid", 1, 16), ("mid", 2, 37),
                                      ("wide_linear", 1, 1), ("wide_linear", 1, 7),
                                      ("wide_linear", 1, 16)])
def test_short_sequence_mixer(rt, monkeypatch, name, b, s):
    """The gated-delta mixer in one launch per (sequence, head)
    (rxw8_q35_linear_short_d64 / _d128: conv + SiLU, L2 norms, beta / g, the
    recurrence and the gated RMSNorm), forced on at every length here (the
    default takes it up to 4 positions), and the three-launch path forced
    on: both within TOL of the oracle, and within 1e-5 of each other (the
    same arithmetic; only the partition of the state's column sums differs)."""
    cfg = CONFIGS[name]
    p = q35.random_params(cfg, seed=21, std=0.05)
    ids = np.random.default_rng(22).integers(0, cfg["vocab"], (b, s))
    want = q35.forward(cfg, p, ids)
    monkeypatch.setenv("RXW8_Q35_SHORT", "1")
    fused = run(rt, build(rt, cfg, p), ids)
    monkeypatch.setenv("RXW8_Q35_SHORT", "0")
    split = run(rt, build(rt, cfg, p), ids)
    e_fused, e_split, e_pair = rel_err(fused, want), rel_err(split, want), rel_err(fused, split)
    print(f"qwen35 short mixer {name} b={b} s={s}: fused {e_fused:.2e}, three launches "
          f"{e_split:.2e}, between {e_pair:.2e}")
    assert e_fused <= TOL and e_split <= TOL
    assert e_pair <= 1e-5


@pytest.mark.parametrize("name,b,s", [("mid", 2, 1), ("mid", 2, 37), ("mid", 1, 64),
                                      ("mid_long", 2, 150), ("wide_linear", 1, 65),
                                      ("wide_linear", 1, 128), ("wide_linear", 1, 203)])
def test_chunked_delta_rule(rt, monkeypatch, name, b, s):
    """The delta rule in chunks of 64 positions (rxw8_q35_delta_chunk_d* /
    rxw8_q35_delta_scan_d*: per chunk (I + A) Delta = diag(beta) (V -
    diag(Gamma) K S0) solved in parallel, the state carried from chunk to
    chunk on the matrix cores), forced on at every length here (the default
    takes it from 256 positions), against the sequential recurrence forced on:
    one partial chunk, exactly one chunk, several with a partial last one, Dl
    64 and 128; both within TOL of the oracle and within 1e-4 of each other
    (the same terms, reassociated)."""
    cfg = CONFIGS[name]
    p = q35.random_params(cfg, seed=61, std=0.05)
    ids = np.random.default_rng(62).integers(0, cfg["vocab"], (b, s))
    want = q35.forward(cfg, p, ids)
    monkeypatch.setenv("RXW8_Q35_SHORT", "0")
    monkeypatch.setenv("RXW8_Q35_CHUNKED", "1")
    chunked = run(rt, build(rt, cfg, p), ids)
    monkeypatch.setenv("RXW8_Q35_CHUNKED", "0")
    seq = run(rt, build(rt, cfg, p), ids)
    e_c, e_s, e_pair = rel_err(chunked, want), rel_err(seq, want), rel_err(chunked, seq)
    print(f"qwen35 chunked delta rule {name} b={b} s={s}: chunked {e_c:.2e}, sequential {e_s:.2e}, "
          f"between {e_pair:.2e}")
    assert e_c <= TOL and e_s <= TOL
    assert e_pair <= 1e-4


@pytest.mark.parametrize("name,b,s", [("mid_long", 2, 150), ("wide_full", 1, 160)])
def test_f32_gemm_split_k_residuals(rt, monkeypatch, name, b, s):
    """Every F32 projection that fits the GEMM tiles forced onto them
    (rxw8_gemm_f32c) with 3 K splits, the residual projections included (the
    reduce launch adds the partials to the f32 residual stream): within TOL of
    the oracle and within 1e-5 of the default plan."""
    cfg = CONFIGS[name]
    p = q35.random_params(cfg, seed=51, std=0.05)
    ids = np.random.default_rng(52).integers(0, cfg["vocab"], (b, s))
    want = q35.forward(cfg, p, ids)
    base = run(rt, build(rt, cfg, p), ids)
    monkeypatch.setenv("RXW8_F32_GEMM", "1")
    monkeypatch.setenv("RXW8_F32_GEMM_KSPLIT", "3")
    got = run(rt, build(rt, cfg, p), ids)
    e_got, e_base, e_pair = rel_err(got, want), rel_err(base, want), rel_err(got, base)
    print(f"qwen35 split-K F32 GEMM {name} b={b} s={s}: forced {e_got:.2e}, default {e_base:.2e}, "
          f"between {e_pair:.2e}")
    assert e_got <= TOL and e_base <= TOL
    assert e_pair <= 1e-5


@pytest.mark.parametrize("name,b,s", [("mid_long", 2, 40), ("wide_linear", 1, 65)])
def test_norm_writes_the_gemm_operands(rt, monkeypatch, name, b, s):
    """From 17 rows under F32 compute, the RMSNorms ahead of the input
    projections and gate|up, and the gated norm ahead of out_proj, write the
    F32 GEMM's bf16 hi / lo operand parts themselves (no f32 rows, no split
    launch): the same arithmetic as norm + rxw8_gemm_split_x, so the logits
    equal the separate launches' bit for bit."""
    cfg = CONFIGS[name]
    p = q35.random_params(cfg, seed=71, std=0.05)
    ids = np.random.default_rng(72).integers(0, cfg["vocab"], (b, s))
    fused = run(rt, build(rt, cfg, p), ids)
    monkeypatch.setenv("RXW8_Q35_NORM_SPLIT", "0")
    apart = run(rt, build(rt, cfg, p), ids)
    np.testing.assert_array_equal(fused, apart)
    assert rel_err(fused, q35.forward(cfg, p, ids)) <= TOL


@pytest.mark.parametrize("name,b,s,std", [("tiny", 2, 13, 0.05), ("small", 2, 13, 0.05),
                                          ("small", 2, 70, 0.05), ("mid", 2, 37, 0.03),
                                          ("wide", 1, 16, 0.02), ("wide_full", 1, 77, 0.02)])
def test_bf16_compute_opt_in(rt, name, b, s, std):
    """compute "bf16" (Cx::with_layer_compute_dtype(BF16)): the packed W8A16
    GEMV / GEMM with bf16 activations against the oracle's BF16 cast points.
    The random network amplifies bf16 rounding flips at the wider widths (the
    oracle moves by 7e-3 at std 0.05 when only its accumulation order
    changes), hence the smaller weights there."""
    cfg = dict(CONFIGS[name], compute="bf16")
    p = q35.random_params(cfg, seed=41, std=std)
    ids = np.random.default_rng(42).integers(0, cfg["vocab"], (b, s))
    err = rel_err(run(rt, build(rt, cfg, p), ids), q35.forward(cfg, p, ids))
    print(f"qwen35 bf16 {name} b={b} s={s}: rel err {err:.2e}")
    assert err <= TOL_BF16


@pytest.mark.parametrize("s", [13, 70])
def test_row_major_weight_path(rt, monkeypatch, s):
    """BF16 compute with RXW8_Q35_UNPACKED=1 keeps the fused projections
    row-major (the path widths outside the tile layout take): same logits
    within tolerance."""
    monkeypatch.setenv("RXW8_Q35_UNPACKED", "1")
    cfg = dict(CONFIGS["small"], compute="bf16")
    p = q35.random_params(cfg, seed=31)
    ids = np.random.default_rng(32).integers(0, cfg["vocab"], (2, s))
    assert rel_err(run(rt, build(rt, cfg, p), ids), q35.forward(cfg, p, ids)) <= TOL_BF16


def test_sequences_are_independent_and_causal(rt):
    """Row b of the batch depends only on sequence b; position i only on
    tokens <= i (bit for bit: the same kernels see the same shapes)."""
    cfg = CONFIGS["small"]
    m = build(rt, cfg, q35.random_params(cfg, seed=13))
    rng = np.random.default_rng(14)
    ids = rng.integers(0, cfg["vocab"], (2, 40))
    a = run(rt, m, ids)
    ids2 = ids.copy()
    ids2[1] = rng.integers(0, cfg["vocab"], 40)  # other sequence changed
    ids2[0, 25:] = (ids2[0, 25:] + 7) % cfg["vocab"]  # future of sequence 0 changed
    b = run(rt, m, ids2)
    np.testing.assert_array_equal(a[0, :25], b[0, :25])
    assert np.abs(a[0, 25:] - b[0, 25:]).max() > 0
    np.testing.assert_array_equal(run(rt, m, ids), a)  # deterministic


def test_graph_replays_match_the_eager_forward(rt):
    """The second call with the same buffers is captured into a HIP graph and
    later calls replay it: every replay equals the eager result bit for bit,
    with other eager work (including a linear that grows the runtime's
    workspaces, which forces a re-capture) and synchronizations in between."""
    r = rx()
    cfg = CONFIGS["mid"]
    m = build(rt, cfg, q35.random_params(cfg, seed=21))
    ids = rt.buffer(np.random.default_rng(22).integers(0, cfg["vocab"], (2, 37)).astype(np.int32))
    logits = rt.zeros((2, 37, cfg["vocab"]), r.DType.F32)
    m.forward(ids, logits)
    eager = logits.to_numpy()
    rng = np.random.default_rng(23)
    for i in range(5):
        m.forward(ids, logits)
        rt.synchronize()
        np.testing.assert_array_equal(logits.to_numpy(), eager)
        x = rng.standard_normal((64 * (i + 1), 1024)).astype(np.float32)
        w = rng.integers(0, 256, (4096, 1024)).astype(np.uint8)
        sc = np.full((4096, 8), 1e-3, np.float32)
        r.quantized_linear(rt, rt.buffer(x), rt.buffer(w), rt.buffer(sc)).to_numpy()
    other = rt.zeros((2, 37, cfg["vocab"]), r.DType.F32)  # a new key: eager again
    m.forward(ids, other)
    np.testing.assert_array_equal(other.to_numpy(), eager)


def test_lora_head(rt):
    cfg = dict(CONFIGS["small"], lora_rank=4, lora_alpha=64.0)
    p = q35.random_params(cfg, seed=15)
    ids = np.random.default_rng(16).integers(0, cfg["vocab"], (2, 9))
    got = run(rt, build(rt, cfg, p), ids)
    want = q35.forward(cfg, p, ids)
    nolora = dict(cfg, lora_rank=0)
    base = q35.forward(nolora, p, ids)
    got_base = run(rt, build(rt, nolora, p), ids)
    print(f"lora: base {rel_err(got_base, base):.2e} update {rel_err(got - got_base, want - base):.2e} "
          f"total {rel_err(got, want):.2e} visible {rel_err(want, base):.2e}")
    assert rel_err(want, base) > 0.05  # the update is visible at this tolerance
    # the update alone (its input, the final norm, carries the base's bf16 deviations)
    assert rel_err(got - got_base, want - base) <= TOL
    assert rel_err(got, want) <= TOL


def test_schema_is_the_encoder_layout(rt):
    """Paths, dtypes and shapes equal the reference encoder's output for the
    same topology (random_params follows quantize_qwen3_5_w8.py:27-55)."""
    r = rx()
    for name in ("small", "wide"):
        cfg = CONFIGS[name]
        p = q35.random_params(cfg, seed=0)
        m = r.Qwen35Model(rt, model_config(cfg)).compile()
        sch = m.schema()
        assert sorted(path for path, _, _ in sch) == sorted(p)
        for path, dtype, shape in sch:
            assert tuple(p[path].shape) == shape, path
            assert dtype == (r.DType.U8 if p[path].dtype == np.uint8 else r.DType.F32), path


def test_checkpoint_loads_verbatim(rt, tmp_path):
    r = rx()
    cfg = CONFIGS["small"]
    p = q35.random_params(cfg, seed=17)
    ck = tmp_path / "q35.safetensors"
    stf.write(ck, {k: ("U8" if v.dtype == np.uint8 else "F32", v) for k, v in p.items()},
              {"format": "rxla-qwen3.5-w8-v1", "group_size": str(cfg["group"])})
    ids = np.random.default_rng(18).integers(0, cfg["vocab"], (2, 11))
    direct = run(rt, build(rt, cfg, p), ids)
    loaded = r.Qwen35Model(rt, model_config(cfg)).compile().load_safetensors(ck)
    np.testing.assert_array_equal(run(rt, loaded, ids), direct)
    bad = tmp_path / "g.safetensors"
    stf.write(bad, {k: ("U8" if v.dtype == np.uint8 else "F32", v) for k, v in p.items()},
              {"group_size": "32"})
    with pytest.raises(r.Error) as e:
        r.Qwen35Model(rt, model_config(cfg)).compile().load_safetensors(bad)
    assert "group_size" in str(e.value)


def test_checkpoint_validation_happens_before_upload(rt, tmp_path):
    r = rx()
    cfg = CONFIGS["small"]
    p = q35.random_params(cfg, seed=41)
    pre = "model.language_model.layers."
    ck = {k: ("U8" if v.dtype == np.uint8 else "F32", v) for k, v in p.items()}
    del ck[pre + "1.self_attn.k_norm.weight"]
    key = pre + "0.linear_attn.conv1d.weight"
    ck[key] = ("F32", ck[key][1][:-1])  # one channel short
    bad = tmp_path / "bad.safetensors"
    stf.write(bad, ck)
    m = r.Qwen35Model(rt, model_config(cfg)).compile()
    with pytest.raises(r.Error) as e:
        m.load_safetensors(bad)
    assert e.value.code == r.Status.INVALID_ARGUMENT
    assert "k_norm" in str(e.value) and "conv1d" in str(e.value)
    assert m._bound == []  # nothing was uploaded or bound


def test_error_contract(rt):
    r = rx()
    cfg = dict(CONFIGS["tiny"], max_positions=16)
    p = q35.random_params(cfg, seed=19)
    m = build(rt, cfg, p)

    def code(fn):
        with pytest.raises(r.Error) as e:
            fn()
        return e.value.code

    assert code(lambda: m.forward(rt.buffer(np.zeros((1, 17), np.int32)))) == r.Status.INVALID_ARGUMENT
    assert code(lambda: m.forward(rt.buffer(np.zeros((3, 4), np.int32)))) == r.Status.OUT_OF_RANGE
    assert code(lambda: m.forward(rt.buffer(np.zeros(4, np.int32)))) == r.Status.INVALID_ARGUMENT
    assert code(lambda: m.forward(rt.buffer(np.zeros((1, 4), np.int32)),
                                  rt.zeros((1, 4, 3), r.DType.F32))) == r.Status.INVALID_ARGUMENT
    unbound = r.Qwen35Model(rt, model_config(cfg)).compile()
    assert code(lambda: unbound.forward(rt.buffer(np.zeros((1, 4), np.int32)))) == \
        r.Status.FAILED_PRECONDITION
    path, dtype, shape = unbound.schema()[0]
    assert code(lambda: unbound.bind_parameter("nope", rt.zeros(shape, dtype))) == r.Status.NOT_FOUND
    assert code(lambda: unbound.bind_parameter(path, rt.zeros((1,), dtype))) == r.Status.INVALID_ARGUMENT
    unbound.bind_parameter(path, rt.zeros(shape, dtype))
    assert code(lambda: unbound.bind_parameter(path, rt.zeros(shape, dtype))) == r.Status.ALREADY_EXISTS
    for bad in (dict(rotary_dim=9), dict(rotary_dim=12), dict(heads=3), dict(group=5),
                dict(eps=0.0)):
        assert code(lambda: r.Qwen35Model(rt, model_config(dict(cfg, **bad))).compile()) == \
            r.Status.INVALID_ARGUMENT, bad
    assert code(lambda: r.Qwen35Model(rt, model_config(dict(cfg, linear_head_dim=12))).compile()) == \
        r.Status.UNIMPLEMENTED
