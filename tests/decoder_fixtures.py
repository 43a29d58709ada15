"""Synthetic decoder parameters and an independent numpy f64 composition.

The numpy composition restates crates/rxla-models/src/qwen3_5/mod.rs:199-273
and layers.rs:28-101,270-293 (dense full-attention layers without the output
gate), with the W8A16 cast points of crates/rxla-nn/src/layers.rs:289-297:
bf16(x), bf16(dequant(W)), bf16 result, everything else f32/f64.
"""
import numpy as np


def np_bf16(x):
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def np_bf16_bits(x):
    return (np_bf16(x).view(np.uint32) >> 16).astype(np.uint16)


def quantize(w, g):
    w = np.asarray(w, np.float32)
    n, k = w.shape
    grouped = w.reshape(n, k // g, g)
    scale = (np.maximum(np.abs(grouped).max(axis=2), np.float32(1e-12)) /
             np.float32(127.0)).astype(np.float32)
    q = np.clip(np.rint(grouped / scale[:, :, None]), -127, 127)
    return (q + 128).astype(np.uint8).reshape(n, k), scale


def dequant(u8, s):
    g = u8.shape[1] // s.shape[1]
    return (u8.astype(np.float32) - np.float32(128)) * np.repeat(s, g, axis=1)


def tiny_config(**kw):
    cfg = dict(layers=2, hidden=128, q_heads=4, kv_heads=2, head_dim=32, intermediate=192,
               vocab=300, max_seq=16, group=64, eps=1e-6, theta=1e6, qk_norm=True)
    cfg.update(kw)
    return cfg


def tiny_params(cfg, seed=0, std=0.02):
    """Random-init weights, W8-quantised per group; norms near 1; bf16 embedding."""
    rng = np.random.default_rng(seed)
    H, D, I = cfg["hidden"], cfg["head_dim"], cfg["intermediate"]
    HQ, HKV, G, V = cfg["q_heads"], cfg["kv_heads"], cfg["group"], cfg["vocab"]
    p = {}

    def q8(n, k, name):
        w = (rng.standard_normal((n, k)) * std).astype(np.float32)
        u8, s = quantize(w, G if G > 0 else k)  # group 0: per-output-channel
        p[name + ".weight"], p[name + ".scale"] = u8, s

    for l in range(cfg["layers"]):
        pre = f"layers.{l}."
        p[pre + "input_layernorm.weight"] = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        p[pre + "post_attention_layernorm.weight"] = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        if cfg.get("qk_norm", True):
            p[pre + "self_attn.q_norm.weight"] = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
            p[pre + "self_attn.k_norm.weight"] = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
        q8((HQ + 2 * HKV) * D, H, pre + "self_attn.qkv_proj")
        q8(H, HQ * D, pre + "self_attn.o_proj")
        q8(2 * I, H, pre + "mlp.gate_up_proj")
        q8(H, I, pre + "mlp.down_proj")
    p["embed_tokens.weight"] = np_bf16_bits(rng.standard_normal((V, H)).astype(np.float32))
    p["norm.weight"] = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    return p


def _rms(x, w, eps):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w


def _lin(x, u8, s):
    y = np_bf16(x).astype(np.float64) @ np_bf16(dequant(u8, s)).astype(np.float64).T
    return np_bf16(y.astype(np.float32)).astype(np.float64)


def numpy_decoder_step(cfg, p, ids, skip_rope=False):
    """Prefill `ids` [B, S] from empty caches; returns last-position logits."""
    B, S = ids.shape
    H, D, I = cfg["hidden"], cfg["head_dim"], cfg["intermediate"]
    HQ, HKV, V, eps = cfg["q_heads"], cfg["kv_heads"], cfg["vocab"], cfg["eps"]
    emb = (p["embed_tokens.weight"].astype(np.uint32) << 16).view(np.float32)
    h = emb[np.clip(ids, 0, V - 1)].astype(np.float64)  # [B, S, H]
    pos = np.arange(S)
    freqs = cfg["theta"] ** (-2.0 * np.arange(D // 2) / D)
    ang = pos[:, None] * freqs[None, :]
    cos, sin = np.cos(ang), np.sin(ang)

    def rope(x):  # x [B, S, heads, D]
        if skip_rope:
            return x
        a, b = x[..., :D // 2], x[..., D // 2:]
        c, s_ = cos[None, :, None, :], sin[None, :, None, :]
        return np.concatenate([a * c - b * s_, b * c + a * s_], -1)

    for l in range(cfg["layers"]):
        pre = f"layers.{l}."
        n = _rms(h, p[pre + "input_layernorm.weight"], eps)
        qkv = _lin(n, p[pre + "self_attn.qkv_proj.weight"], p[pre + "self_attn.qkv_proj.scale"])
        q = qkv[..., :HQ * D].reshape(B, S, HQ, D)
        k = qkv[..., HQ * D:(HQ + HKV) * D].reshape(B, S, HKV, D)
        v = qkv[..., (HQ + HKV) * D:].reshape(B, S, HKV, D)
        if cfg.get("qk_norm", True):
            q = _rms(q, p[pre + "self_attn.q_norm.weight"], eps)
            k = _rms(k, p[pre + "self_attn.k_norm.weight"], eps)
        q, k = rope(q), rope(k)
        k = np_bf16(k.astype(np.float32)).astype(np.float64)  # bf16 KV cache
        v = np_bf16(v.astype(np.float32)).astype(np.float64)
        att = np.zeros((B, S, HQ, D))
        causal = np.where(pos[None, :] <= pos[:, None], 0.0, -np.inf)
        for hh in range(HQ):
            kv = hh // (HQ // HKV)
            sc = np.einsum("bsd,btd->bst", q[:, :, hh], k[:, :, kv]) / np.sqrt(D) + causal
            pr = np.exp(sc - sc.max(-1, keepdims=True))
            pr /= pr.sum(-1, keepdims=True)
            att[:, :, hh] = np.einsum("bst,btd->bsd", pr, v[:, :, kv])
        h = h + _lin(att.reshape(B, S, HQ * D), p[pre + "self_attn.o_proj.weight"],
                     p[pre + "self_attn.o_proj.scale"])
        n = _rms(h, p[pre + "post_attention_layernorm.weight"], eps)
        gu = _lin(n, p[pre + "mlp.gate_up_proj.weight"], p[pre + "mlp.gate_up_proj.scale"])
        g, u = gu[..., :I], gu[..., I:]
        a = g / (1 + np.exp(-g)) * u
        h = h + _lin(a, p[pre + "mlp.down_proj.weight"], p[pre + "mlp.down_proj.scale"])
    n = _rms(h[:, -1], p["norm.weight"], eps)
    logits = np_bf16(n).astype(np.float64) @ emb.astype(np.float64).T
    return np_bf16(logits.astype(np.float32))
