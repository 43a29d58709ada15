#!/usr/bin/env python3
"""rxw8 benchmark: W8A16 decode GEMV HBM GB/s.

One step = one pass of the decode dequant-GEMV over the whole sweep
B in {1, 4, 16} x N in {4096, 6144, 24576}, K = 4096, per-output-channel
scales (9 launches). Weights are in the tiled layout of rxw8_pack_weight
(packed once, outside the timed region; same bytes as the row-major U8).
Every launch reads a copy of the int8 weights of its own: each N has a pool
of 48 / 36 / 12 copies and launch (b, n) of step t reads copy
(3 t + index of b) mod pool size, so a copy is read again only after at
least 790 MB of other weights of that N (3 x the 256 MB MALL): no weight byte
is served from the MALL and the figure is HBM bandwidth.

value        = sweep algorithmic bytes / wall time of the timed steps (GB/s);
               each step is the 9 products in one rxw8_quantized_linear_group
               call (two grouped launches: B 1 and 4 on 96-row tiles, then
               B 16 on 192-row tiles), replayed from HIP
               graphs: one of 48 consecutive steps (every pool turns over a
               whole number of times in it) replayed K // 48 times, then one
               of the first K % 48 steps (a graph boundary idles the GPU for
               ~8 us); single_launches times the same steps as 9
               rxw8_quantized_linear_into calls (the per-shape plans)
roofline     = the GEMV kernel of the largest sweep shape, B=1 N=24576
               (rxw8_gemv_rc_w8_pk_mb1_rw1_u4: 4 waves splitting K, 16-row
               tiles, 1536 workgroups): algorithmic bytes per launch /
               launch duration, from HIP events on the runtime's stream around
               runs of back-to-back launches of the shape; traffic = the HBM
               bytes per launch recorded in profiles/ by two rocprofv3 --pmc
               passes (FETCH_SIZE, WRITE_SIZE) over `bench.py --pmc-probe gemv`
cpu_baseline = the CPU oracle (reference-order restatement, OpenMP) timed on
               this host over a bounded sample of the same sweep; its
               "decoder" entry times 8 full-size C5 decode steps (batch 8,
               caches at 1024 positions) through the oracle decoder

Algorithmic bytes per launch: N*K (u8 weights) + 4*N (f32 scales)
+ 2*B*K (bf16 x) + 2*B*N (bf16 y).

Further legs (same JSON line, extra keys; --skip-* to leave one out):
prefill_gemm  BASELINE configs[2]: x bf16 [M,4096] for M in {512, 2048, 8192}
              against W [12288,4096] and the [4096,12288] down projection;
              2*M*N*K flops per launch over the mean launch time (HIP events
              around back-to-back launches), roofline against dense bf16 MFMA
decode_attention  BASELINE configs[3]: batch 8, 32/8 heads, D 128, lengths
              uniform in [512, 8192], bf16 cache; bytes = K and V rows read
              (lens * 8 heads * 128 * 2 B * 2) + q + out, three rotating cache copies
prefill_attention  the C5 prompt's causal attention (8 x 1024 rows, 16/8
              heads, D 128) on rxw8_gqa_prefill: flops over HIP-event time,
              roofline against dense bf16 MFMA
decoder       BASELINE configs[4]: 28-layer synthetic decoder (random-init
              weights, W8 per output channel), batch 8, prompt 1024, 256
              greedy steps through rxw8_decoder_generate (decode steps replay
              one HIP graph); decode tokens/s = 8*256 / (generate time -
              prefill time)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
K = 4096
BS = (1, 4, 16)
NS = (4096, 6144, 24576)


def gemv_bytes(b, n, k=K):
    return n * k + 4 * n + 2 * b * k + 2 * b * n


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def recorded_traffic(name="gemv_B1_N24576_traffic.txt"):
    """HBM bytes per launch (or per call) from a committed counter summary
    (two rocprofv3 --pmc passes, calibrated by a copy of known size); None
    when the summary is absent."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        for line in open(path):
            if line.startswith("TRAFFIC_BYTES_PER_LAUNCH="):
                return int(line.split("=", 1)[1])
    except OSError:
        pass
    return None


def cpu_baseline(budget_s=12.0):
    """Oracle (reference-order CPU restatement) over the same sweep shapes."""
    import oracle

    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or len(os.sched_getaffinity(0))
    rng = np.random.default_rng(0)
    ws = {n: oracle.quantize_w8((rng.standard_normal((n, K)) * 0.02).astype(np.float32), K)
          for n in NS}
    xs = {b: oracle.round_bf16(rng.standard_normal((b, K)).astype(np.float32)) for b in BS}
    total_bytes, total_t, passes = 0, 0.0, 0
    while total_t < budget_s and passes < 200:
        for n in NS:
            for b in BS:
                u8, s = ws[n]
                t0 = time.perf_counter()
                oracle.quantized_linear(xs[b], u8, s, oracle.COMPUTE_BF16, threads=threads)
                total_t += time.perf_counter() - t0
                total_bytes += gemv_bytes(b, n)
        passes += 1
    return {"value": round(total_bytes / total_t / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"{passes} pass(es) of the 9-shape sweep (B in {list(BS)}, N in {list(NS)}, "
                      f"K={K}) through oracle.quantized_linear (bf16 compute, f32 accumulation), "
                      f"{total_t:.1f} s"}


SPIN_CYCLES = 2_000_000  # torch.cuda._sleep spacer, about 1 ms of shader clocks
ROOF_CYCLES = 2          # passes over the weight copies per roofline event pair
MALL_BYTES = 256 << 20   # MI355X last-level (Infinity) cache
# Weight copies per N of the sweep: (copies - 1) x N x K >= 790 MB (3 x the
# MALL) of other weights of that N stream between two reads of one copy.
# Multiples of 3 (the three batch sizes of a step) whose turns all fit
# GRAPH_STEPS steps a whole number of times: 48 steps x 3 launches per N =
# 3 x 48 = 4 x 36 = 12 x 12.
POOL = {4096: 48, 6144: 36, 24576: 12}
GRAPH_STEPS = 48
ATTN_COPIES = 3          # rotating KV caches of the C4 leg


def cpu_decoder_baseline(steps=8, ctx=1024, batch=8, seed=11):
    """C5 on the CPU: the oracle decoder (reference-order C restatement, OpenMP)
    at full size, timing `steps` greedy decode steps (after one untimed step) of
    `batch` sequences whose caches already hold `ctx` positions (zero K/V: the prompt's 8 x 1024 prefill
    is 28 TFLOP, beyond a bounded CPU sample). Weights are random W8 codes and
    scales and a random bf16 embedding (values do not change the work)."""
    import oracle

    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or len(os.sched_getaffinity(0))
    cfg = dict(layers=28, hidden=2048, q_heads=16, kv_heads=8, head_dim=128, intermediate=6144,
               vocab=151936, max_seq=ctx + steps + 1, group=0, eps=1e-6, theta=1e6, qk_norm=True)
    rng = np.random.default_rng(seed)
    H, D, I, V = cfg["hidden"], cfg["head_dim"], cfg["intermediate"], cfg["vocab"]
    qkv = (cfg["q_heads"] + 2 * cfg["kv_heads"]) * D

    def codes(n, k):
        return rng.integers(0, 256, (n, k), dtype=np.uint8)

    def scales(n, k):
        return (rng.random((n, 1), np.float32) * 1e-3 + 1e-4).astype(np.float32)

    p = {"embed_tokens.weight": rng.integers(0x3C00, 0x4000, (V, H), dtype=np.uint16),
         "norm.weight": np.ones(H, np.float32)}
    for l in range(cfg["layers"]):
        pre = f"layers.{l}."
        p[pre + "input_layernorm.weight"] = np.ones(H, np.float32)
        p[pre + "post_attention_layernorm.weight"] = np.ones(H, np.float32)
        p[pre + "self_attn.q_norm.weight"] = np.ones(D, np.float32)
        p[pre + "self_attn.k_norm.weight"] = np.ones(D, np.float32)
        for name, n, k in (("self_attn.qkv_proj", qkv, H), ("self_attn.o_proj", H, H),
                           ("mlp.gate_up_proj", 2 * I, H), ("mlp.down_proj", H, I)):
            p[pre + name + ".weight"], p[pre + name + ".scale"] = codes(n, k), scales(n, k)
    dec = oracle.Decoder(cfg, p, batch)
    dec.lens[:] = ctx
    ids = rng.integers(0, V, (batch, 1)).astype(np.int32)
    _, nxt = dec.forward(ids, threads=threads)  # untimed: first touch of the caches
    ids = nxt.reshape(batch, 1)
    t0 = time.perf_counter()
    for _ in range(steps):
        _, nxt = dec.forward(ids, threads=threads)
        ids = nxt.reshape(batch, 1)
    dt = time.perf_counter() - t0
    return {"decode_tokens_per_s": round(batch * steps / dt, 2), "ms_per_step": round(dt / steps * 1e3, 1),
            "cores": threads, "kind": "port",
            "sample": f"{steps} greedy decode steps of the 28-layer C5 decoder at full size, batch "
                      f"{batch}, caches at {ctx} positions, through oracle.Decoder (C, OpenMP)"}


class SweepPools:
    """The sweep's operands: POOL[n] weight copies per N (row-major U8 as
    encoded, and the packed copies the timed legs read), bf16 x [B, K] and
    bf16 y [B, N]. Launch (b, n) of step t reads copy (3 t + index of b) mod
    POOL[n]; launch_next continues a per-N cursor for the per-shape timing."""

    def __init__(self, rt, rx, torch, stream, gen):
        self.rt, self.rx, self.torch = rt, rx, torch
        log(f"encoding {sum(POOL.values())} weight copies ({POOL}) from N(0, 0.02)")
        self.rowmajor = {n: [c5_quantized(rt, rx, torch, stream, gen, n, K) for _ in range(POOL[n])]
                         for n in NS}
        self.packed = {n: [(rx.pack_weight(rt, u), s) for u, s in self.rowmajor[n]] for n in NS}
        with torch.cuda.stream(stream):
            self.xs = {b: torch.randn((b, K), device="cuda", generator=gen).to(torch.bfloat16)
                       for b in BS}
            self.ys = {(b, n): torch.empty((b, n), dtype=torch.bfloat16, device="cuda")
                       for b in BS for n in NS}
        stream.synchronize()
        rt.synchronize()
        self.xb = {b: rt.wrap_tensor(self.xs[b]) for b in BS}
        self.yb = {k: rt.wrap_tensor(v) for k, v in self.ys.items()}
        self.plan = [(b, n) for n in NS for b in BS]
        self.cursor = {n: 0 for n in NS}

    def launch(self, b, n, copy, wts):
        u, s = wts[n][copy % POOL[n]]
        self.rx.quantized_linear(self.rt, self.xb[b], u, s, self.rx.DType.BF16,
                                 out=self.yb[(b, n)])

    def launch_step(self, step, wts):
        for b, n in self.plan:
            self.launch(b, n, 3 * step + BS.index(b), wts)

    def launch_step_grouped(self, step, wts):
        """The step's nine products in one rxw8_quantized_linear_group call
        (two launches: B 1 and 4, then B 16)."""
        xs, ws, ss, ys = [], [], [], []
        for b, n in self.plan:
            u, s = wts[n][(3 * step + BS.index(b)) % POOL[n]]
            xs.append(self.xb[b]), ws.append(u), ss.append(s), ys.append(self.yb[(b, n)])
        self.rx.quantized_linear_group(self.rt, xs, ws, ss, ys)

    def launch_next(self, b, n, wts):
        self.launch(b, n, self.cursor[n], wts)
        self.cursor[n] += 1

    def release(self):
        self.rowmajor = self.packed = None


def c5_quantized(rt, rx, torch, stream, gen, n, k, std=0.02, group=None):
    """BASELINE configs[1] weights: W ~ N(0, std) f32 [n, k] on the device,
    encoded by rxw8_quantize_w8 (the reference encoder's arithmetic) per output
    channel (group = k) or per group; returns (U8 [n, k], F32 scale) buffers."""
    with torch.cuda.stream(stream):
        w = torch.randn((n, k), device="cuda", generator=gen) * std
    stream.synchronize()
    u, s_ = rx.quantize_w8(rt, rt.wrap_tensor(w), group or k)
    rt.synchronize()
    del w
    return u, s_


def bench_gemm(rt, rx, torch, stream, reps=10):
    """C3 prefill dequant-GEMM shapes; returns per-shape TFLOP/s and the MFMA
    roofline of the largest one."""
    gen = torch.Generator(device="cuda").manual_seed(1)
    shapes = [(m, n, k) for m in (512, 2048, 8192) for n, k in ((12288, 4096), (4096, 12288))]
    ws = {(n, k): c5_quantized(rt, rx, torch, stream, gen, n, k) for n, k in ((12288, 4096), (4096, 12288))}
    with torch.cuda.stream(stream):
        xs = {(m, k): torch.randn((m, k), device="cuda", generator=gen).to(torch.bfloat16)
              for m in (512, 2048, 8192) for k in (4096, 12288)}
    stream.synchronize()
    wb = {key: (rx.pack_weight(rt, u), s_) for key, (u, s_) in ws.items()}
    rt.synchronize()
    out = {}
    for m, n, k in shapes:
        with torch.cuda.stream(stream):
            y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        yb, xb, (u, s_) = rt.wrap_tensor(y), rt.wrap_tensor(xs[(m, k)]), wb[(n, k)]
        # steady state: about 60 ms of back-to-back launches before timing, so
        # the clocks have settled at their sustained level under MFMA load
        warm = max(3, int(0.06 / (2 * m * n * k / 1.0e15)))
        for _ in range(warm):
            rx.quantized_linear(rt, xb, u, s_, rx.DType.BF16, out=yb)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            rx.quantized_linear(rt, xb, u, s_, rx.DType.BF16, out=yb)
        e1.record(stream)
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / reps
        out[f"M{m}_N{n}_K{k}"] = {"us": round(t * 1e6, 1), "TFLOPs": round(2 * m * n * k / t / 1e12, 1)}
    big = out["M8192_N12288_K4096"]
    return out, {"bound": "mfma", "achieved": big["TFLOPs"], "peak": MFMA_BF16_PEAK_TFLOPS,
                 "unit": "TFLOP/s", "frac": round(big["TFLOPs"] / MFMA_BF16_PEAK_TFLOPS, 4),
                 "traffic": recorded_traffic("gemm_M8192_N12288_K4096_traffic.txt"),
                 "traffic_source": "profiles/gemm_M8192_N12288_K4096_traffic.txt (FETCH_SIZE + "
                                   "WRITE_SIZE per call of both kernels, copy-calibrated, "
                                   "bench.py --pmc-probe gemm)",
                 "kernel": "rxw8_gemm_dequant_w + rxw8_w8a16_gemm_bf16w_t256 (M >= 4096 path)",
                 "shape": "M=8192 N=12288 K=4096", "mean_launch_us": big["us"],
                 "timing": f"HIP events around {reps} back-to-back launches after ~60 ms "
                           "of warmup launches of the shape"}


def bench_attention(rt, rx, torch, stream, reps=20):
    """C4 decode attention; bytes = the K/V rows each sequence reads + q + out."""
    gen = torch.Generator(device="cuda").manual_seed(2)
    B, HQ, HKV, D, LMAX = 8, 32, 8, 128, 8192
    lens = np.random.default_rng(4).integers(512, 8193, B).astype(np.int32)
    with torch.cuda.stream(stream):
        caches = [(torch.randn((B, HKV, LMAX, D), device="cuda", generator=gen).to(torch.bfloat16),
                   torch.randn((B, HKV, LMAX, D), device="cuda", generator=gen).to(torch.bfloat16))
                  for _ in range(ATTN_COPIES)]
        q = torch.randn((B, HQ, D), device="cuda", generator=gen).to(torch.bfloat16)
        o = torch.empty((B, HQ, D), dtype=torch.bfloat16, device="cuda")
        lt = torch.from_numpy(lens).to("cuda")
    stream.synchronize()
    cb = [(rt.wrap_tensor(k), rt.wrap_tensor(v)) for k, v in caches]
    qb, ob, lb = rt.wrap_tensor(q), rt.wrap_tensor(o), rt.wrap_tensor(lt)
    nbytes = int(lens.sum()) * HKV * D * 2 * 2 + 2 * B * HQ * D * 2 + 4 * B
    for c in range(100):
        rx.grouped_query_attention(rt, qb, cb[c % ATTN_COPIES][0], cb[c % ATTN_COPIES][1], lb, out=ob)
    with torch.cuda.stream(stream):
        torch.cuda._sleep(SPIN_CYCLES)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        rx.grouped_query_attention(rt, qb, cb[i % ATTN_COPIES][0], cb[i % ATTN_COPIES][1], lb, out=ob)
    e1.record(stream)
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / reps
    gbs = nbytes / t / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": recorded_traffic("attention_c4_traffic.txt"),
            "traffic_source": "profiles/attention_c4_traffic.txt (FETCH_SIZE + WRITE_SIZE per call, "
                              "copy-calibrated, bench.py --pmc-probe attention)",
            "kernels": "rxw8_gqa_decode_d128_g4 (splits merged in-kernel)",
            "us_per_call": round(t * 1e6, 2), "bytes_per_call": nbytes,
            "lens": lens.tolist(),
            "timing": f"HIP events around {reps} back-to-back calls after a spin kernel, "
                      f"{ATTN_COPIES} rotating cache copies (each call reads ~207 MB, so a "
                      "copy returns after 400+ MB: none is served from the 256 MB MALL)"}


def bench_prefill_attention(rt, rx, torch, stream, reps=10):
    """C5 prompt attention: 8 sequences x 1024 causal rows, 16 q / 8 kv heads,
    D 128, keys already in a bf16 cache [8, 8, 1280, 128]; f32 q, bf16 out.
    Flops = 4 * D * Hq * sum over rows of (visible keys) (QK^T and P.V)."""
    gen = torch.Generator(device="cuda").manual_seed(6)
    B, S, HQ, HKV, D, LMAX = 8, 1024, 16, 8, 128, 1280
    with torch.cuda.stream(stream):
        q = torch.randn((B, S, HQ, D), device="cuda", generator=gen)
        kc = torch.randn((B, HKV, LMAX, D), device="cuda", generator=gen).to(torch.bfloat16)
        vc = torch.randn((B, HKV, LMAX, D), device="cuda", generator=gen).to(torch.bfloat16)
        o = torch.empty((B, S, HQ, D), dtype=torch.bfloat16, device="cuda")
        starts = torch.zeros(B, dtype=torch.int32, device="cuda")
    stream.synchronize()
    qb, kb, vb, ob, sb = (rt.wrap_tensor(t) for t in (q, kc, vc, o, starts))
    for _ in range(400):  # ~60 ms of warmup: sustained clocks under MFMA load
        rx.grouped_query_attention_prefill(rt, qb, kb, vb, sb, out=ob)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        rx.grouped_query_attention_prefill(rt, qb, kb, vb, sb, out=ob)
    e1.record(stream)
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / reps
    flops = 4 * D * HQ * B * S * (S + 1) // 2
    tf = flops / t / 1e12
    return {"bound": "mfma", "achieved": round(tf, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
            "kernel": "rxw8_gqa_prefill_r2_d128_g2", "us_per_call": round(t * 1e6, 1),
            "flops_per_call": flops, "shape": "B=8 S=1024 Hq=16 Hkv=8 D=128, causal from 0",
            "note": "flops count the visible (causal) keys once; q enters as bf16 hi + lo, "
                    "so the MFMA work is 1.5x this count",
            "timing": f"HIP events around {reps} back-to-back calls after 400 warmup calls"}


def bench_decoder(rt, rx, torch, stream, prompt_len=1024, steps=256, batch=8):
    """C5: random-init W8 decoder; decode tokens/s from generate - prefill."""
    from rxla_amd.model import DecoderConfig, DecoderModel

    cfg = DecoderConfig(max_batch=batch, max_seq=prompt_len + steps)
    model = DecoderModel(rt, cfg).compile()
    gen = torch.Generator(device="cuda").manual_seed(3)
    keep = []
    pending_scale = {}
    with torch.cuda.stream(stream):
        for path, dtype, shape in model.schema():
            if path.endswith(".scale"):
                t = pending_scale.pop(path)
            elif dtype == rx.DType.U8:
                w = torch.randn(shape, device="cuda", generator=gen) * 0.02
                g = cfg.group if cfg.group > 0 else shape[1]
                wg = w.view(shape[0], shape[1] // g, g)
                sc = wg.abs().amax(dim=2).clamp_min(1e-12) / 127.0
                t = (torch.round(wg / sc[:, :, None]).clamp(-127, 127) + 128).to(torch.uint8)
                t = t.view(shape).contiguous()
                pending_scale[path[:-len(".weight")] + ".scale"] = sc.contiguous()
                del w, wg
            elif dtype == rx.DType.BF16:
                t = (torch.randn(shape, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
            else:
                t = torch.ones(shape, device="cuda", dtype=torch.float32)
            keep.append(t)
            stream.synchronize()
            model.bind_parameter(path, rt.wrap_tensor(t))
    rt.synchronize()
    ids = np.random.default_rng(5).integers(0, cfg.vocab, (batch, prompt_len)).astype(np.int32)
    prompt = rt.buffer(ids)
    out_ids = rt.zeros((batch, steps + 1), rx.DType.I32)

    def timed(fn):
        model.reset()
        rt.synchronize()
        t0 = time.perf_counter()
        fn()
        rt.synchronize()
        return time.perf_counter() - t0

    timed(lambda: model.generate(prompt, steps, out_ids=out_ids, use_graph=True))  # warm + capture
    t_prefill = min(timed(lambda: model.forward(prompt)) for _ in range(2))
    t_total = min(timed(lambda: model.generate(prompt, steps, out_ids=out_ids, use_graph=True))
                  for _ in range(2))
    t_decode = t_total - t_prefill
    toks = out_ids.to_numpy()
    weight_bytes = sum(int(np.prod(sh)) * (1 if dt == rx.DType.U8 else 4 if dt == rx.DType.F32 else 2)
                       for _, dt, sh in model.schema())
    kv_bytes = sum(cfg.layers * cfg.kv_heads * cfg.head_dim * 2 * 2 * batch * (prompt_len + i + 1)
                   for i in range(steps)) / steps
    step_bytes = weight_bytes + kv_bytes
    return {"decode_tokens_per_s": round(batch * steps / t_decode, 1),
            "ms_per_decode_step": round(t_decode / steps * 1e3, 4),
            "prefill_ms": round(t_prefill * 1e3, 2),
            "prefill_tokens_per_s": round(batch * prompt_len / t_prefill, 1),
            "decode_step_bytes": int(step_bytes),
            "decode_step_GBs": round(step_bytes / (t_decode / steps) / 1e9, 1),
            "decode_step_hbm_frac": round(step_bytes / (t_decode / steps) / 1e9 / HBM_PEAK_GBS, 4),
            "config": {"layers": cfg.layers, "hidden": cfg.hidden, "q_heads": cfg.q_heads,
                       "kv_heads": cfg.kv_heads, "head_dim": cfg.head_dim,
                       "intermediate": cfg.intermediate, "vocab": cfg.vocab, "batch": batch,
                       "prompt": prompt_len, "steps": steps, "scales": "per-output-channel"},
            "distinct_tokens": int(len(np.unique(toks))),
            "timing": "wall clock around rxw8_decoder_generate / rxw8_decoder_forward, "
                      "synchronized, best of 2"}


def qwen35_weights(rt, rx, torch, stream, model, group, seed=7):
    """Random-init W8 parameters for a Qwen35Model, generated on the device:
    2-D weights ~N(0, 0.02) quantised per group as the reference encoder does
    (quantize_qwen3_5_w8.py:27-44: s = max|w_g| / 127, u8 = rne(w / s) + 128);
    zero-centred norm weights 0, the gated norm's weight 1, conv ~N(0, 0.1),
    A_log and dt_bias 0."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    keep, pending = [], {}
    with torch.cuda.stream(stream):
        for path, dtype, shape in model.schema():
            if path.endswith(".scale"):
                t = pending.pop(path)
            elif dtype == rx.DType.U8:
                t = torch.empty(shape, dtype=torch.uint8, device="cuda")
                sc = torch.empty((shape[0], shape[1] // group), dtype=torch.float32, device="cuda")
                step = max(1, (1 << 26) // shape[1])  # quantise in row chunks (bounded scratch)
                for r0 in range(0, shape[0], step):
                    w = torch.randn((min(step, shape[0] - r0), shape[1]), device="cuda",
                                    generator=gen) * 0.02
                    wg = w.view(w.shape[0], shape[1] // group, group)
                    s_ = wg.abs().amax(dim=2).clamp_min(1e-12) / 127.0
                    t[r0:r0 + w.shape[0]] = (torch.round(wg / s_[:, :, None]).clamp(-127, 127)
                                             + 128).to(torch.uint8).view(w.shape)
                    sc[r0:r0 + w.shape[0]] = s_
                pending[path[:-len(".weight")] + ".scale"] = sc
            elif "conv1d" in path:
                t = torch.randn(shape, device="cuda", generator=gen) * 0.1
            elif path.endswith("linear_attn.norm.weight"):
                t = torch.ones(shape, device="cuda", dtype=torch.float32)
            else:
                t = torch.zeros(shape, device="cuda", dtype=torch.float32)
            keep.append(t)
            stream.synchronize()
            model.bind_parameter(path, rt.wrap_tensor(t))
    rt.synchronize()
    return keep


def bench_f32_linear(rt, rx, torch, stream, reps=10, n=248320, k=1024, g=128):
    """The F32-compute W8 linear (rxw8_linear_f32_mfma_*: f32 x split into bf16
    hi + lo, exact codes, f32 results), the Qwen3.5 default compute, at its
    largest product, the tied LM head W [248320, 1024] U8 with G = 128
    scales: S = 16 rows is bound by the weight stream (bytes N K + 4 N K / G
    + 4 S K + 4 S N), S = 1024 by the matrix cores (2 S N K flops; the hi / lo
    parts make the MFMA work twice that). Two weight copies (254 MB each)
    alternate so neither is read from the MALL; HIP events around `reps`
    back-to-back calls after a spin kernel."""
    gen = torch.Generator(device="cuda").manual_seed(3)
    ws = [c5_quantized(rt, rx, torch, stream, gen, n, k, group=g) for _ in range(2)]
    out = {}
    for S in (16, 1024):
        with torch.cuda.stream(stream):
            x = torch.randn((S, k), device="cuda", generator=gen)
            y = torch.empty((S, n), dtype=torch.float32, device="cuda")
        stream.synchronize()
        xb, yb = rt.wrap_tensor(x), rt.wrap_tensor(y)
        for i in range(4):
            rx.quantized_linear(rt, xb, ws[i % 2][0], ws[i % 2][1], rx.DType.F32, out=yb)
        with torch.cuda.stream(stream):
            torch.cuda._sleep(SPIN_CYCLES)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(reps):
            rx.quantized_linear(rt, xb, ws[i % 2][0], ws[i % 2][1], rx.DType.F32, out=yb)
        e1.record(stream)
        torch.cuda.synchronize()
        sec = e0.elapsed_time(e1) * 1e-3 / reps
        if S == 16:
            nbytes = n * k + 4 * n * (k // g) + 4 * S * k + 4 * S * n
            gbs = nbytes / sec / 1e9
            out[f"S{S}"] = {"bound": "hbm", "us": round(sec * 1e6, 2), "achieved": round(gbs, 1),
                            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                            "bytes": nbytes}
        else:
            tf = 2.0 * S * n * k / sec / 1e12
            out[f"S{S}"] = {"bound": "mfma", "us": round(sec * 1e6, 2), "achieved": round(tf, 1),
                            "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                            "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                            "mfma_frac": round(2 * tf / MFMA_BF16_PEAK_TFLOPS, 4),
                            "flops": 2 * S * n * k}
        del x, y
    # S = 16 on the tile-layout copies (the Qwen3.5 plan's head up to 16 rows:
    # rxw8_linear_f32_mfma_pk_r1_w8, contiguous 1 KiB wave loads)
    pk = [(rx.pack_weight(rt, w), s) for w, s in ws]
    with torch.cuda.stream(stream):
        x = torch.randn((16, k), device="cuda", generator=gen)
        y = torch.empty((16, n), dtype=torch.float32, device="cuda")
    stream.synchronize()
    xb, yb = rt.wrap_tensor(x), rt.wrap_tensor(y)
    for i in range(4):
        rx.quantized_linear(rt, xb, pk[i % 2][0], pk[i % 2][1], rx.DType.F32, out=yb)
    with torch.cuda.stream(stream):
        torch.cuda._sleep(SPIN_CYCLES)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        rx.quantized_linear(rt, xb, pk[i % 2][0], pk[i % 2][1], rx.DType.F32, out=yb)
    e1.record(stream)
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3 / reps
    nbytes = n * k + 4 * n * (k // g) + 4 * 16 * k + 4 * 16 * n
    gbs = nbytes / sec / 1e9
    out["S16_packed"] = {"bound": "hbm", "us": round(sec * 1e6, 2), "achieved": round(gbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "bytes": nbytes}
    del x, y, pk
    del ws
    return {"kernel": "rxw8_linear_f32_mfma_r1_w8 (S 16, row-major) / rxw8_linear_f32_mfma_pk_r1_w8 "
                      "(S16_packed, tile layout) / rxw8_gemm_split_x + rxw8_gemm_f32c (S 1024)",
            "shape": f"W [{n}, {k}] U8, G {g} (the Qwen3.5-0.8B tied LM head), x F32 [S, {k}]",
            "runs": out,
            "note": "mfma_frac counts the hi and lo MFMAs (twice the algorithmic flops)",
            "timing": f"HIP events around {reps} back-to-back calls over 2 alternating weight "
                      "copies after a spin kernel"}


# The reference's own published W8 runs of this workload (RTX 5080, JAX CUDA 13
# PJRT plugin; docs/QWEN3.5-BENCHMARK.md:68-80): mean ms per run by sequence.
QWEN35_REFERENCE_MS = {1: 2.393, 16: 10.535}


def bench_qwen35(rt, rx, torch, stream, sequences=(1, 16, 256, 1024), warmup=2, iterations=10,
                 compute="f32"):
    """The reference's qwen3_5_bench workload (crates/rxla-safetensors/examples/
    qwen3_5_bench.rs:44-99) on the official 0.8B text topology with random
    weights: batch 1, token ids 1000 + i, full logits [1, S, 248320] per run;
    tokens/s = S / mean run time. compute "f32" is the reference's precision
    (the example leaves the layer compute dtype at the Cx default F32);
    "bf16" is the opt-in."""
    cfg = rx.Qwen35Config(max_batch=1, max_seq=max(sequences), compute=compute)
    model = rx.Qwen35Model(rt, cfg).compile()
    keep = qwen35_weights(rt, rx, torch, stream, model, cfg.group)
    weight_bytes = sum(int(np.prod(sh)) * (1 if dt == rx.DType.U8 else 4)
                       for _, dt, sh in model.schema())
    res = {}
    for S in sequences:
        ids = rt.buffer(np.arange(1000, 1000 + S, dtype=np.int32).reshape(1, S))
        logits = rt.zeros((1, S, cfg.vocab), rx.DType.F32)
        for _ in range(warmup):
            model.forward(ids, logits)
        rt.synchronize()
        samples = []
        for _ in range(iterations):
            t0 = time.perf_counter()
            model.forward(ids, logits)
            rt.synchronize()
            samples.append(time.perf_counter() - t0)
        lg = logits.to_numpy()
        mean = float(np.mean(samples))
        res[f"S{S}"] = {"mean_ms": round(mean * 1e3, 3),
                        "p50_ms": round(float(np.median(samples)) * 1e3, 3),
                        "tokens_per_s": round(S / mean, 1),
                        "weight_GBs": round(weight_bytes / mean / 1e9, 1),
                        "finite": bool(np.isfinite(lg).all()),
                        "checksum": float(lg.astype(np.float64).sum())}
        if S in QWEN35_REFERENCE_MS:
            res[f"S{S}"]["reference_ms_rtx5080"] = QWEN35_REFERENCE_MS[S]
        del logits
    del keep, model
    return {"runs": res, "weight_bytes": weight_bytes, "compute_dtype": compute,
            "config": "Qwen3.5-0.8B text topology (24 layers, 18 gated-delta + 6 full attention, "
                      "hidden 1024, vocab 248320, G 128), batch 1, random W8 weights, "
                      f"projections computed in {compute}",
            "timing": f"wall clock around rxw8_qwen35_forward, synchronized; {warmup} warmup, "
                      f"mean of {iterations}"}


def pmc_probe(kind, rounds=3):
    """A short fixed program for rocprofv3 runs: one roofline leg launched as
    the bench times it (gemv / gemv16: `rounds` x [spin spacer, ROOF_CYCLES
    passes over the 12 weight copies of N = 24576 back to back] at B = 1 / 16;
    sweep: 2 x 48 whole steps of the sweep, eager, with the bench's copy
    rotation (counters summed over a step's 9 launches); attention:
    `rounds` x [spin spacer, 20 C4 calls over the rotating caches]; gemm: 30
    launches of the C3 roofline shape; gemm_all: 20 launches of each of the
    six C3 shapes; decoder: the C5 leg with 16 decode
    steps; prefill: the prefill-attention leg) plus 4 plain 256 MiB device
    copies (torch) that calibrate what FETCH_SIZE / WRITE_SIZE read for a
    known number of bytes."""
    import torch
    import rxla_amd as rx

    rt = rx.Runtime(0)
    stream = torch.cuda.Stream()
    rt.set_stream(stream.cuda_stream)
    gen = torch.Generator(device="cuda").manual_seed(0)
    with torch.cuda.stream(stream):
        src = torch.randn(1 << 26, device="cuda", generator=gen)  # 256 MiB
        dst = torch.empty_like(src)
    stream.synchronize()
    if kind in ("gemv", "gemv16"):  # B=1 (or 16), N=24576, K=4096, packed, its 12 rotating copies
        n, b = 24576, (16 if kind == "gemv16" else 1)
        ws = [c5_quantized(rt, rx, torch, stream, gen, n, K) for _ in range(POOL[n])]
        with torch.cuda.stream(stream):
            x = torch.randn((b, K), device="cuda", generator=gen).to(torch.bfloat16)
            y = torch.empty((b, n), dtype=torch.bfloat16, device="cuda")
        stream.synchronize()
        wb = [(rx.pack_weight(rt, u), s_) for u, s_ in ws]
        rt.synchronize()
        xb, yb = rt.wrap_tensor(x), rt.wrap_tensor(y)
        for _ in range(rounds):
            with torch.cuda.stream(stream):
                torch.cuda._sleep(SPIN_CYCLES)
            for i in range(ROOF_CYCLES * POOL[n]):
                u, s_ = wb[i % POOL[n]]
                rx.quantized_linear(rt, xb, u, s_, rx.DType.BF16, out=yb)
        reps = rounds * ROOF_CYCLES * POOL[n]
        log(f"pmc probe gemv B={b} N={n} K={K}: {reps} launches, {gemv_bytes(b, n)} algorithmic B each")
    elif kind == "sweep":  # whole sweep steps with the bench's rotation, eager
        pools = SweepPools(rt, rx, torch, stream, gen)
        for st in range(2 * GRAPH_STEPS):
            pools.launch_step(st, pools.packed)
        step_bytes = sum(gemv_bytes(b, n) for b, n in pools.plan)
        log(f"pmc probe sweep: {2 * GRAPH_STEPS} steps of {len(pools.plan)} launches, "
            f"{step_bytes} algorithmic B per step")
    elif kind == "gemm":  # C3 roofline shape M=8192 N=12288 K=4096, 10 launches after warm-up
        m, n = 8192, 12288
        u, sb = c5_quantized(rt, rx, torch, stream, gen, n, K)
        with torch.cuda.stream(stream):
            x = torch.randn((m, K), device="cuda", generator=gen).to(torch.bfloat16)
            y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        stream.synchronize()
        ub = rx.pack_weight(rt, u)
        xb, yb = rt.wrap_tensor(x), rt.wrap_tensor(y)
        for _ in range(30):
            rx.quantized_linear(rt, xb, ub, sb, rx.DType.BF16, out=yb)
        log(f"pmc probe gemm M={m} N={n} K={K}: 30 launches")
    elif kind == "gemm_all":  # every C3 shape, 20 launches each, in the order of bench_gemm
        ws = {}
        for n_, k_ in ((12288, 4096), (4096, 12288)):
            u, sb = c5_quantized(rt, rx, torch, stream, gen, n_, k_)
            ws[(n_, k_)] = (rx.pack_weight(rt, u), sb)
        rt.synchronize()
        for m in (512, 2048, 8192):
            for (n_, k_), (ub, sb) in ws.items():
                with torch.cuda.stream(stream):
                    x = torch.randn((m, k_), device="cuda", generator=gen).to(torch.bfloat16)
                    y = torch.empty((m, n_), dtype=torch.bfloat16, device="cuda")
                stream.synchronize()
                xb, yb = rt.wrap_tensor(x), rt.wrap_tensor(y)
                for _ in range(20):
                    rx.quantized_linear(rt, xb, ub, sb, rx.DType.BF16, out=yb)
                rt.synchronize()
                log(f"pmc probe gemm_all M={m} N={n_} K={k_}: 20 launches")
                del x, y
    elif kind == "attention":  # C4, as bench_attention times it
        B, HQ, HKV, D, LMAX = 8, 32, 8, 128, 8192
        lens = np.random.default_rng(4).integers(512, 8193, B).astype(np.int32)
        with torch.cuda.stream(stream):
            caches = [(torch.randn((B, HKV, LMAX, D), device="cuda", generator=gen).to(torch.bfloat16),
                       torch.randn((B, HKV, LMAX, D), device="cuda", generator=gen).to(torch.bfloat16))
                      for _ in range(ATTN_COPIES)]
            q = torch.randn((B, HQ, D), device="cuda", generator=gen).to(torch.bfloat16)
            o = torch.empty((B, HQ, D), dtype=torch.bfloat16, device="cuda")
            lt = torch.from_numpy(lens).to("cuda")
        stream.synchronize()
        cb = [(rt.wrap_tensor(k), rt.wrap_tensor(v)) for k, v in caches]
        qb, ob, lb = rt.wrap_tensor(q), rt.wrap_tensor(o), rt.wrap_tensor(lt)
        calls = 0
        for _ in range(rounds):
            with torch.cuda.stream(stream):
                torch.cuda._sleep(SPIN_CYCLES)
            for i in range(20):
                rx.grouped_query_attention(rt, qb, cb[i % ATTN_COPIES][0], cb[i % ATTN_COPIES][1], lb, out=ob)
                calls += 1
        log(f"pmc probe attention C4 lens={lens.tolist()}: {calls} calls")
    elif kind == "decoder":  # C5: prompt 1024, 16 greedy steps (generate run 3 times)
        r = bench_decoder(rt, rx, torch, stream, steps=16)
        log(f"pmc probe decoder C5: 16 decode steps per generate, {r['ms_per_decode_step']} ms/step")
    elif kind == "prefill":  # the C5 prompt's causal attention, as bench_prefill_attention times it
        r = bench_prefill_attention(rt, rx, torch, stream)
        log(f"pmc probe prefill attention: {r['us_per_call']} us/call")
    else:
        raise SystemExit(f"unknown --pmc-probe {kind}")
    rt.synchronize()
    with torch.cuda.stream(stream):
        for _ in range(4):
            dst.copy_(src)
    torch.cuda.synchronize()
    log("pmc probe: 4 copies of 268435456 B")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--skip-gemm", action="store_true")
    ap.add_argument("--skip-attention", action="store_true")
    ap.add_argument("--skip-decoder", action="store_true")
    ap.add_argument("--skip-qwen35", action="store_true")
    ap.add_argument("--pmc-probe", choices=["gemv", "gemv16", "sweep", "gemm", "gemm_all", "attention", "decoder",
                                            "prefill"],
                    help="counter-collection program only")
    ap.add_argument("--qwen35-only", action="store_true",
                    help="(profiling) run only the Qwen3.5 leg and print its JSON")
    ap.add_argument("--decoder-only", action="store_true",
                    help="(profiling) run only the C5 decoder leg and print its JSON")
    args = ap.parse_args()
    if args.pmc_probe:
        pmc_probe(args.pmc_probe)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); multi-GPU runs are "
              "not part of this build", file=sys.stderr)
        sys.exit(2)

    import torch
    import rxla_amd as rx

    rt = rx.Runtime(0)
    info = rt.device_info()
    stream = torch.cuda.Stream()  # default priority
    rt.set_stream(stream.cuda_stream)
    if args.qwen35_only:
        print(json.dumps({"qwen35": bench_qwen35(rt, rx, torch, stream)}), flush=True)
        return
    if args.decoder_only:
        print(json.dumps({"decoder": bench_decoder(rt, rx, torch, stream)}), flush=True)
        return
    gen = torch.Generator(device="cuda").manual_seed(0)
    pools = SweepPools(rt, rx, torch, stream, gen)
    xb, yb, ys = pools.xb, pools.yb, pools.ys
    wb, wb_row = pools.packed, pools.rowmajor
    plan = pools.plan
    step_bytes = sum(gemv_bytes(b, n) for b, n in plan)

    def launch_all(step, events=None, wts=None, grouped=True):
        if grouped:
            pools.launch_step_grouped(step, wts or wb)
        else:
            pools.launch_step(step, wts or wb)

    # Eager warmup (sizes workspaces, resolves kernels), then HIP graphs: one
    # holding GRAPH_STEPS consecutive steps (every pool turns over a whole
    # number of times in it, so replays follow each other seamlessly) and one
    # holding the first K % GRAPH_STEPS steps; the timed region replays the
    # first K // GRAPH_STEPS times, then the second once (a graph boundary
    # idles the GPU for ~8 us).
    for i in range(args.warmup):
        launch_all(GRAPH_STEPS - args.warmup + i)
    torch.cuda.synchronize()

    def step_graph(first, count, wts=None, grouped=True):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for st in range(first, first + count):
                launch_all(st, wts=wts, grouped=grouped)
        return g

    def timed_graphs(wts=None, grouped=True):
        full = (step_graph(0, GRAPH_STEPS, wts, grouped) if args.steps >= GRAPH_STEPS else None)
        rem = (step_graph(0, args.steps % GRAPH_STEPS, wts, grouped)
               if args.steps % GRAPH_STEPS else None)
        return full, rem

    def run_steps(full, rem, steps):
        for _ in range(steps // GRAPH_STEPS):
            full.replay()
        if rem is not None:
            rem.replay()

    graph_full, graph_rem = timed_graphs()
    # replays equal eager launches: after a graph of steps [0, n) every output
    # holds step n - 1's result
    for g, last in ((graph_full, GRAPH_STEPS - 1), (graph_rem, args.steps % GRAPH_STEPS - 1)):
        if g is None:
            continue
        launch_all(last)
        torch.cuda.synchronize()
        ref = {k: v.clone() for k, v in ys.items()}
        g.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(ys[k], ref[k]) for k in ys), "graph replay differs from eager launch"
    # warm the timed graphs; the last warm step is GRAPH_STEPS - 1, so the
    # timed step 0 reads copies last read a whole pool turn ago
    if graph_full is not None:
        graph_full.replay()
    else:
        for st in range(GRAPH_STEPS):
            launch_all(st)

    # Timed region: exactly K steps, synchronized on both sides.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run_steps(graph_full, graph_rem, args.steps)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    log(f"timed {args.steps} graph steps in {wall:.4f} s")

    # Kernel durations: per shape, one HIP event pair on the runtime stream
    # around one pass over that N's pool (one launch per copy, the pool's
    # cursor continuing across shapes), queued behind a ~1 ms spin kernel (no
    # memory traffic: a fill spacer would leave dirty cache lines whose
    # write-back lands inside the timed launches) so the host submits them all
    # before the GPU reaches the first event. Every copy is read again only
    # after at least 512 MB of other weights: none comes from the MALL.
    def spacer():
        with torch.cuda.stream(stream):
            torch.cuda._sleep(SPIN_CYCLES)

    events = []
    rounds = 3
    for _ in range(rounds):
        for b, n in plan:
            spacer()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _c in range(POOL[n]):
                pools.launch_next(b, n, wb)
            e1.record(stream)
            events.append((b, n, e0, e1))
    # The roofline shape (B=1, N=24576): ROOF_CYCLES passes over its pool of
    # 12 copies per event pair (1.2 GB between reuses of a copy).
    roof_events = []
    for _ in range(rounds):
        spacer()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _c in range(ROOF_CYCLES * POOL[24576]):
            pools.launch_next(1, 24576, wb)
        e1.record(stream)
        roof_events.append((e0, e1))
    torch.cuda.synchronize()

    def timed_variant(wts, grouped):
        full, rem = timed_graphs(wts, grouped)
        if full is not None:
            full.replay()
        else:
            for st in range(GRAPH_STEPS):
                launch_all(st, wts=wts, grouped=grouped)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        run_steps(full, rem, args.steps)
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    # The same sweep on the reference's row-major U8 weights (the layout the
    # XLA handlers and direct QuantizedLinear::apply calls receive), and as
    # nine single launches per step (one rxw8_quantized_linear_into each):
    # graphs of the same steps, same step count, timed the same way.
    wall_row = timed_variant(wb_row, True)
    log(f"timed {args.steps} row-major graph steps in {wall_row:.4f} s")
    wall_single = timed_variant(wb, False)
    log(f"timed {args.steps} single-launch graph steps in {wall_single:.4f} s")

    per_shape = {}
    for b, n, e0, e1 in events:
        per_shape.setdefault((b, n), []).append(e0.elapsed_time(e1) * 1e-3 / POOL[n])

    def kernel_stats(sel):
        ev = [(b, n, e0, e1) for b, n, e0, e1 in events if sel(b)]
        mb = float(np.mean([gemv_bytes(b, n) for b, n, _, _ in ev]))
        ms = float(np.mean([e0.elapsed_time(e1) * 1e-3 / POOL[n] for b, n, e0, e1 in ev]))
        return mb, ms

    mean_bytes, mean_s = kernel_stats(lambda b: b <= 4)
    b16_bytes, b16_s = kernel_stats(lambda b: b > 4)
    # roofline shape: B=1, N=24576 (the largest decode GEMV of the sweep)
    roof_s = float(np.median([e0.elapsed_time(e1) * 1e-3 / (ROOF_CYCLES * POOL[24576])
                              for e0, e1 in roof_events]))
    roof_bytes = gemv_bytes(1, 24576)
    achieved = roof_bytes / roof_s / 1e9
    sweep = {f"B{b}_N{n}": {"us": round(float(np.median(v)) * 1e6, 2),
                            "GBs": round(gemv_bytes(b, n) / float(np.median(v)) / 1e9, 1)}
             for (b, n), v in sorted(per_shape.items())}
    log(json.dumps(sweep))

    value = step_bytes * args.steps / wall / 1e9
    out = {
        "metric": "W8A16 GEMV HBM GB/s (% peak) + decode tokens/sec, synthetic Qwen-style 28L",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: W ~ N(0, 0.02) f32 encoded per output channel on the device by "
                "rxw8_quantize_w8 (the reference encoder's arithmetic), x ~ N(0, 1) rounded to "
                "bf16; torch generator seed 0",
        "config": {"workload": "decode dequant-GEMV sweep (BASELINE configs[1])",
                   "batch": list(BS), "out_features": list(NS), "in_features": K,
                   "scales": "per-output-channel f32",
                   "weight_copies": {str(n): POOL[n] for n in NS},
                   "weight_layout": "packed",
                   "products_per_step": len(plan),
                   "launches_per_step": "2 (rxw8_quantized_linear_group: B 1 and 4, then B 16)",
                   "bytes_per_step": step_bytes,
                   "steps_per_graph_replay": GRAPH_STEPS,
                   "copy_rotation": "launch (b, n) of step t reads copy (3 t + index of b) mod "
                                    "copies[n]: a copy is read again after >= 790 MB of other "
                                    "weights (>= 3 x the 256 MB MALL)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": recorded_traffic(),
                     "kernel": "rxw8_gemv_rc_w8_pk_mb1_rw1_u4",
                     "shape": "B=1 N=24576 K=4096", "launch_us": round(roof_s * 1e6, 3),
                     "launch_bytes": roof_bytes,
                     "timing": "median of HIP event pairs on the runtime stream around "
                               f"{ROOF_CYCLES * POOL[24576]} back-to-back launches of the shape "
                               f"({ROOF_CYCLES} passes over its {POOL[24576]} weight copies, "
                               "after a spin kernel), divided by the launch count (includes "
                               "the inter-kernel gaps)",
                     "traffic_source": "profiles/gemv_B1_N24576_traffic.txt (FETCH_SIZE + "
                                       "WRITE_SIZE per launch, copy-calibrated)",
                     "b_le_4_mean": {"achieved": round(mean_bytes / mean_s / 1e9, 2),
                                     "mean_launch_us": round(mean_s * 1e6, 3),
                                     "mean_launch_bytes": int(mean_bytes)}},
        "roofline_b16": {"bound": "hbm", "achieved": round(b16_bytes / b16_s / 1e9, 2),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(b16_bytes / b16_s / 1e9 / HBM_PEAK_GBS, 4),
                         "kernels": "N=24576: rxw8_gemv_rc_w8_pk_mb1_rw6_u4_w12 (96-row tiles, "
                                    "LDS-DMA staging); N=4096 / 6144: the per-shape plans (8-wave "
                                    "16-row tiles; 4-wave split-K + rxw8_gemv_splitk_reduce)",
                         "mean_launch_us": round(b16_s * 1e6, 3)},
        "sweep": sweep,
        "sweep_timing": "per shape, the median over HIP event pairs around one pass over that "
                        "N's weight copies (48 / 36 / 12 launches, each copy read again only after "
                        ">= 790 MB of other weights) after a spin kernel, divided by the launch count",
        "rowmajor": {"value": round(step_bytes * args.steps / wall_row / 1e9, 2), "unit": "GB/s",
                     "ms_per_step": round(wall_row / args.steps * 1e3, 4),
                     "weight_layout": "row-major U8 [N, K] (the reference's weight ABI)",
                     "timing": "same sweep, step count and graph replays as `value`"},
        "single_launches": {"value": round(step_bytes * args.steps / wall_single / 1e9, 2),
                            "unit": "GB/s", "ms_per_step": round(wall_single / args.steps * 1e3, 4),
                            "launches_per_step": len(plan) + 1,
                            "timing": "the same steps as nine rxw8_quantized_linear_into calls "
                                      "each (per-shape plans; one splits K and adds a reduce "
                                      "launch), same step count and graph replays as `value`"},
        "device": info,
    }
    del graph_full, graph_rem
    pools.release()
    torch.cuda.synchronize()
    if not args.skip_gemm:
        log("prefill GEMM shapes ...")
        out["prefill_gemm"], out["roofline_gemm"] = bench_gemm(rt, rx, torch, stream)
        log(json.dumps(out["prefill_gemm"]))
    if not args.skip_attention:
        log("decode attention ...")
        out["roofline_attention"] = bench_attention(rt, rx, torch, stream)
    if not args.skip_attention:
        log("prefill attention ...")
        out["roofline_prefill_attention"] = bench_prefill_attention(rt, rx, torch, stream)
    if not args.skip_decoder:
        log("synthetic 28-layer decoder: prefill 8x1024, 256 greedy steps ...")
        out["decoder"] = bench_decoder(rt, rx, torch, stream)
        log(json.dumps(out["decoder"]))
    if not args.skip_qwen35:
        log("F32-compute W8 linear at the Qwen3.5 LM head ...")
        out["roofline_f32_linear"] = bench_f32_linear(rt, rx, torch, stream)
        log(json.dumps(out["roofline_f32_linear"]))
        log("Qwen3.5-0.8B topology, full-sequence logits ...")
        out["qwen35"] = bench_qwen35(rt, rx, torch, stream)
        log(json.dumps(out["qwen35"]))
        out["qwen35_bf16_opt_in"] = bench_qwen35(rt, rx, torch, stream, sequences=(16,),
                                                 compute="bf16")
        log(json.dumps(out["qwen35_bf16_opt_in"]))
    if not args.no_cpu_baseline:
        log("timing the CPU baseline (oracle) ...")
        out["cpu_baseline"] = cpu_baseline()
        log("timing the CPU decoder baseline (oracle, C5 decode steps) ...")
        out["cpu_baseline"]["decoder"] = cpu_decoder_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
