"""Oracle for the hybrid Qwen3.5 W8 text model (TEST INFRASTRUCTURE ONLY:
imported by tests/ as the checker, never by the product path).

A numpy restatement, in float64 with the reference's cast points, of
crates/rxla-models/src/qwen3_5/mod.rs:234-273 (model) and layers.rs (mixers):
  * W8 embedding gather: (f32(u8) - 128) * scale, rows clamped   mod.rs:158-179
  * zero-centred RMSNorm: x * rsqrt(mean(x^2) + eps) * (1 + w)    layers.rs(nn):459-491
  * projections (rxla-nn layers.rs:257-298) at the layer compute dtype, which
    qwen3_5() leaves at the Cx default F32 (rxla-nn lib.rs:432; qwen3_5/
    layers.rs:4-9 reads cx.layer_compute_dtype()):
      F32  (cfg compute "f32", the default): f32 x . ((u8 - 128) * s)^T in
           f64, returned as f32 (dot_general at HIGHEST precision, emitter.rs:58)
      BF16 (cfg compute "bf16", an opt-in): bf16(x) . bf16(W)^T rounded to bf16
  * full attention with output gate and partial RoPE              layers.rs:28-100
  * gated-delta linear attention (causal depthwise conv + SiLU,
    L2-normalised q/k, delta-rule recurrence, gated RMSNorm)      layers.rs:113-268
  * SwiGLU MLP                                                    layers.rs:270-293
  * tied W8 LM head: f32 logits against the dequantised table,
    plus the optional F32 LoRA update (lora_rank, lora_alpha)     mod.rs:158-195
It returns logits for every position ([B, S, V]), as the reference does.
"""
from __future__ import annotations

import numpy as np

from . import bf16_bits, bf16_to_f32, round_bf16

LINEAR, FULL = "linear", "full"


def config(**kw):
    """Defaults follow Qwen3_5Config::tiny (mod.rs:37-55) except group 8 and
    widths the callers override."""
    c = dict(vocab=128, hidden=32, intermediate=64, layers=[LINEAR, FULL], heads=4, kv_heads=2,
             head_dim=8, linear_heads=4, linear_head_dim=8, conv_kernel=4, theta=1e7,
             rotary_dim=4, eps=1e-6, group=8, compute="f32")
    c.update(kw)
    return c


def layer_types(n, interval=4):
    """Qwen3_5Config::qwen3_5_0_8b_w8 (mod.rs:61-71): every `interval`-th layer
    is full attention."""
    return [FULL if (i + 1) % interval == 0 else LINEAR for i in range(n)]


def dequant(u8, scale):
    """(f32(u8) - 128) * scale per group, as f32 (layers.rs:277-287)."""
    n, k = u8.shape
    g = k // scale.shape[1]
    w = (u8.astype(np.float32) - np.float32(128)).reshape(n, k // g, g)
    return (w * scale.astype(np.float32)[:, :, None]).reshape(n, k).astype(np.float32)


def projection(x, u8, scale, compute="f32"):
    """QuantizedLinear::apply (layers.rs:257-298) with f64 accumulation.
    compute "f32": f32(f32(x) . W^T), W = (f32(u8) - 128) * s in f32;
    compute "bf16": f32(bf16(bf16(x) . bf16(W)^T))."""
    if compute == "f32":
        xf = np.asarray(x, np.float32).astype(np.float64)
        return (xf @ dequant(u8, scale).astype(np.float64).T).astype(np.float32)
    if compute != "bf16":
        raise ValueError(f"compute dtype {compute!r}")
    xb = round_bf16(np.asarray(x, np.float32)).astype(np.float64)
    wb = round_bf16(dequant(u8, scale)).astype(np.float64)
    return round_bf16((xb @ wb.T).astype(np.float32))


def rms_norm(x, w, eps, zero_centered):
    x = np.asarray(x, np.float64)
    s = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    ww = np.asarray(w, np.float64) + (1.0 if zero_centered else 0.0)
    return x * s * ww


def sigmoid(x):
    x = np.asarray(x, np.float64)
    return np.where(x >= 0, 1.0 / (1.0 + np.exp(-np.abs(x))), np.exp(-np.abs(x)) / (1.0 + np.exp(-np.abs(x))))


def silu(x):
    return np.asarray(x, np.float64) * sigmoid(x)


def softplus(x):
    """max(x, 0) + log1p(exp(-|x|)) (rxla-core ops.rs:256-262)."""
    x = np.asarray(x, np.float64)
    return np.maximum(x, 0.0) + np.log1p(np.exp(-np.abs(x)))


def l2_norm(x):
    """x * rsqrt(sum(x^2) + 1e-6) over the last axis (layers.rs:102-111)."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).sum(axis=-1, keepdims=True) + 1e-6)


def rope_angles(theta, rotary_dim, seq):
    half = rotary_dim // 2
    freqs = np.array([np.float32(theta) ** np.float32(-2.0 * i / rotary_dim) for i in range(half)],
                     np.float32)
    return (np.arange(seq, dtype=np.float32)[:, None] * freqs[None, :]).astype(np.float32)


def partial_rope(x, angles, rotary_dim):
    """SplitHalf rotation of the first rotary_dim channels (layers.rs:11-26);
    x [..., S, D], angles [S, rotary_dim/2]."""
    half = rotary_dim // 2
    c, s_ = np.cos(angles.astype(np.float64)), np.sin(angles.astype(np.float64))
    a, b = x[..., :half], x[..., half:rotary_dim]
    return np.concatenate([a * c - b * s_, b * c + a * s_, x[..., rotary_dim:]], axis=-1)


def depthwise_causal_conv(x, w):
    """x [B, S, C], w [C, k]: out[t, c] = sum_j w[c, j] x[t - (k-1) + j, c]
    (conv2d_oihw with padding (k-1, 0), layers.rs:131-146; a correlation)."""
    k = w.shape[1]
    b, s, c = x.shape
    xp = np.concatenate([np.zeros((b, k - 1, c)), x], axis=1)
    out = np.zeros((b, s, c))
    for j in range(k):
        out += xp[:, j:j + s, :] * w[None, None, :, j]
    return out


def delta_rule(q, k, v, beta, g):
    """The recurrence of layers.rs:197-234 over positions t, per (batch, head):
    S <- g_t S;  predicted_j = sum_i S_ij k_i;  delta = (v - predicted) beta_t;
    S_ij += k_i delta_j;  out_j = sum_i S_ij q_i.  q, k, v [B, S, H, D];
    beta, g [B, S, H]; the state starts at zero."""
    b, s, hl, dl = q.shape
    state = np.zeros((b, hl, dl, dl))
    out = np.zeros((b, s, hl, dl))
    for t in range(s):
        state = state * g[:, t][:, :, None, None]
        predicted = np.einsum("bhij,bhi->bhj", state, k[:, t])
        delta = (v[:, t] - predicted) * beta[:, t][:, :, None]
        state = state + k[:, t][..., :, None] * delta[..., None, :]
        out[:, t] = np.einsum("bhij,bhi->bhj", state, q[:, t])
    return out


def gated_delta(x, p, pre, cfg):
    """layers.rs:113-268 for one linear-attention layer; x [B, S, H] f32."""
    b, s, _ = x.shape
    hl, dl = cfg["linear_heads"], cfg["linear_head_dim"]
    width = hl * dl
    cd = cfg.get("compute", "f32")
    mixed = projection(x, p[pre + "in_proj_qkv.weight"], p[pre + "in_proj_qkv.scale"], cd)
    conv_w = np.asarray(p[pre + "conv1d.weight"], np.float64).reshape(3 * width, -1)
    mixed = silu(depthwise_causal_conv(mixed.astype(np.float64), conv_w))
    q = l2_norm(mixed[..., :width].reshape(b, s, hl, dl)) * (1.0 / np.sqrt(np.float32(dl)))
    k = l2_norm(mixed[..., width:2 * width].reshape(b, s, hl, dl))
    v = mixed[..., 2 * width:].reshape(b, s, hl, dl)
    z = projection(x, p[pre + "in_proj_z.weight"], p[pre + "in_proj_z.scale"], cd).reshape(b, s, hl, dl)
    beta = sigmoid(projection(x, p[pre + "in_proj_b.weight"], p[pre + "in_proj_b.scale"], cd))
    a = projection(x, p[pre + "in_proj_a.weight"], p[pre + "in_proj_a.scale"], cd).astype(np.float64)
    decay = softplus(a + np.asarray(p[pre + "dt_bias"], np.float64)) * \
        (-np.exp(np.asarray(p[pre + "A_log"], np.float64)))
    out = delta_rule(q, k, v, beta, np.exp(decay))
    o = rms_norm(out, p[pre + "norm.weight"], cfg["eps"], False) * silu(z)
    return projection(o.reshape(b, s, width).astype(np.float32), p[pre + "out_proj.weight"],
                      p[pre + "out_proj.scale"], cd)


def full_attention(x, p, pre, cfg, angles):
    """layers.rs:28-100: gated output, zero-centred q/k norms, partial RoPE,
    causal GQA over the sequence."""
    b, s, _ = x.shape
    hq, hkv, d = cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    cd = cfg.get("compute", "f32")
    qg = projection(x, p[pre + "q_proj.weight"], p[pre + "q_proj.scale"], cd).reshape(b, s, hq, 2 * d)
    query, gate = qg[..., :d].astype(np.float64), sigmoid(qg[..., d:].reshape(b, s, hq * d))
    query = rms_norm(query, p[pre + "q_norm.weight"], cfg["eps"], True).transpose(0, 2, 1, 3)
    key = projection(x, p[pre + "k_proj.weight"], p[pre + "k_proj.scale"], cd).reshape(b, s, hkv, d)
    key = rms_norm(key, p[pre + "k_norm.weight"], cfg["eps"], True).transpose(0, 2, 1, 3)
    value = projection(x, p[pre + "v_proj.weight"], p[pre + "v_proj.scale"], cd).reshape(
        b, s, hkv, d).astype(np.float64).transpose(0, 2, 1, 3)
    query = partial_rope(query, angles, cfg["rotary_dim"])
    key = partial_rope(key, angles, cfg["rotary_dim"])
    g = hq // hkv
    out = np.zeros((b, hq, s, d))
    causal = np.where(np.arange(s)[None, :] <= np.arange(s)[:, None], 0.0, -np.inf)
    for h in range(hq):
        sc = np.einsum("bsd,btd->bst", query[:, h], key[:, h // g]) / np.sqrt(np.float32(d)) + causal
        sc = np.exp(sc - sc.max(axis=-1, keepdims=True))
        out[:, h] = np.einsum("bst,btd->bsd", sc / sc.sum(axis=-1, keepdims=True), value[:, h // g])
    att = out.transpose(0, 2, 1, 3).reshape(b, s, hq * d) * gate
    return projection(att.astype(np.float32), p[pre + "o_proj.weight"], p[pre + "o_proj.scale"], cd)


def mlp(x, p, pre, compute="f32"):
    g = projection(x, p[pre + "gate_proj.weight"], p[pre + "gate_proj.scale"], compute).astype(np.float64)
    u = projection(x, p[pre + "up_proj.weight"], p[pre + "up_proj.scale"], compute).astype(np.float64)
    return projection((silu(g) * u).astype(np.float32), p[pre + "down_proj.weight"],
                      p[pre + "down_proj.scale"], compute)


def forward(cfg, p, ids):
    """ids [B, S] int -> logits [B, S, V] (float64), mod.rs:197-273."""
    ids = np.asarray(ids)
    b, s = ids.shape
    root = "model.language_model."
    emb_u8, emb_s = p[root + "embed_tokens.weight"], p[root + "embed_tokens.scale"]
    table = dequant(emb_u8, emb_s)
    h = table[np.clip(ids, 0, cfg["vocab"] - 1)].astype(np.float64)
    angles = rope_angles(cfg["theta"], cfg["rotary_dim"], s)
    for i, kind in enumerate(cfg["layers"]):
        pre = f"{root}layers.{i}."
        n = rms_norm(h, p[pre + "input_layernorm.weight"], cfg["eps"], True).astype(np.float32)
        if kind == LINEAR:
            mixed = gated_delta(n, p, pre + "linear_attn.", cfg)
        else:
            mixed = full_attention(n, p, pre + "self_attn.", cfg, angles)
        h = h + mixed
        n = rms_norm(h, p[pre + "post_attention_layernorm.weight"], cfg["eps"], True).astype(np.float32)
        h = h + mlp(n, p, pre + "mlp.", cfg.get("compute", "f32"))
    n = rms_norm(h, p[root + "norm.weight"], cfg["eps"], True)
    logits = n @ table.astype(np.float64).T
    rank = cfg.get("lora_rank", 0)
    if rank:
        # tied-head LoRA (mod.rs:174-195): base + (n A^T) B^T * (alpha / rank)
        a = np.asarray(p[root + "embed_tokens.lora_A.weight"], np.float64)
        b_ = np.asarray(p[root + "embed_tokens.lora_B.weight"], np.float64)
        logits = logits + ((n @ a.T) @ b_.T) * (np.float32(cfg["lora_alpha"]) / np.float32(rank))
    return logits


def random_params(cfg, seed=0, std=0.05):
    """Random-init weights in the reference encoder's layout
    (quantize_qwen3_5_w8.py:27-55): 2-D weights as U8 codes + F32 scales, the
    rest F32."""
    from . import quantize_w8

    rng = np.random.default_rng(seed)
    G = cfg["group"]
    p = {}
    root = "model.language_model."

    def q8(name, n, k):
        w = (rng.standard_normal((n, k)) * std).astype(np.float32)
        u8, s = quantize_w8(w, G)
        p[name + ".weight"], p[name + ".scale"] = u8, s

    H, I = cfg["hidden"], cfg["intermediate"]
    emb = rng.standard_normal((cfg["vocab"], H)).astype(np.float32)
    p[root + "embed_tokens.weight"], p[root + "embed_tokens.scale"] = quantize_w8(emb, G)
    for i, kind in enumerate(cfg["layers"]):
        pre = f"{root}layers.{i}."
        p[pre + "input_layernorm.weight"] = (0.1 * rng.standard_normal(H)).astype(np.float32)
        p[pre + "post_attention_layernorm.weight"] = (0.1 * rng.standard_normal(H)).astype(np.float32)
        if kind == LINEAR:
            hl, dl = cfg["linear_heads"], cfg["linear_head_dim"]
            w = hl * dl
            a = pre + "linear_attn."
            q8(a + "in_proj_qkv", 3 * w, H)
            p[a + "conv1d.weight"] = (0.5 * rng.standard_normal((3 * w, 1, cfg["conv_kernel"]))).astype(np.float32)
            q8(a + "in_proj_z", w, H)
            q8(a + "in_proj_b", hl, H)
            q8(a + "in_proj_a", hl, H)
            p[a + "A_log"] = (0.5 * rng.standard_normal(hl)).astype(np.float32)
            p[a + "dt_bias"] = (0.5 * rng.standard_normal(hl)).astype(np.float32)
            p[a + "norm.weight"] = (1 + 0.1 * rng.standard_normal(dl)).astype(np.float32)
            q8(a + "out_proj", H, w)
        else:
            hq, hkv, d = cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
            a = pre + "self_attn."
            q8(a + "q_proj", hq * 2 * d, H)
            p[a + "q_norm.weight"] = (0.1 * rng.standard_normal(d)).astype(np.float32)
            q8(a + "k_proj", hkv * d, H)
            p[a + "k_norm.weight"] = (0.1 * rng.standard_normal(d)).astype(np.float32)
            q8(a + "v_proj", hkv * d, H)
            q8(a + "o_proj", H, hq * d)
        q8(pre + "mlp.gate_proj", I, H)
        q8(pre + "mlp.up_proj", I, H)
        q8(pre + "mlp.down_proj", H, I)
    p[root + "norm.weight"] = (0.1 * rng.standard_normal(H)).astype(np.float32)
    rank = cfg.get("lora_rank", 0)
    if rank:
        p[root + "embed_tokens.lora_A.weight"] = (0.1 * rng.standard_normal((rank, H))).astype(np.float32)
        p[root + "embed_tokens.lora_B.weight"] = (0.1 * rng.standard_normal((cfg["vocab"], rank))).astype(np.float32)
    return p


__all__ = ["config", "layer_types", "forward", "random_params", "dequant", "projection",
           "rms_norm", "l2_norm", "softplus", "sigmoid", "silu", "partial_rope",
           "depthwise_causal_conv", "delta_rule", "gated_delta", "full_attention", "rope_angles",
           "bf16_bits", "bf16_to_f32", "LINEAR", "FULL"]
