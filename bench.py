#!/usr/bin/env python3
"""Benchmark of the Q4 decode hot path on one MI355X.

Workload (the metric's configuration): the Gemma-12B-class decode layer at
batch 1 -- hidden 3840, fused QKV GEMV 8192x3840 (q 16x256, k and v 8x256),
O GEMV 3840x4096, fused FFN 3840 <-> 15360 with GeGLU (tanh GELU) -- over 48
distinct seeded layers (6.72 GB of Q4 weights, far above the 256 MB Infinity
Cache). Weights are registered once per layer (the kernels' tiled layout), as
the reference's runtime registers resident weights. One step = one decode
token through the three matmuls of all 48 layers, replayed from a HIP graph;
weights and activations are resident in HBM before the timed region starts.

Prints ONE JSON line. `value` is achieved HBM GB/s of algorithmic bytes
(20 B per 32 weights plus activations in and out, once) over the whole step.
`roofline` is the dominant kernel -- the one-token FFN's first launch
(q4_ffn1_kernel: gate/up, GeGLU and the down projection in 64-row slices of
the intermediate, over half the time of a layer; a second launch sums the
slices' partial outputs) -- timed with HIP events on its stream over a graph of
its 48 launches (alv_ffn_partials); `traffic` is its HBM bytes per launch from
the committed FETCH_SIZE / WRITE_SIZE profile. `cpu_baseline` times the oracle's
restatement of the reference CPU path (per call: dequantize to fp32, fp32
matvec) on a bounded sample: one layer's QKV + O + FFN.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5]
    python bench.py --profile-pass   # short eager workload for rocprofv3 --pmc
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published
H, I_FF = 3840, 15360
VOC, KH = 262144, 4096  # Gemma-4 LM head: vocabulary x padded hidden
N_QKV, K_O = 8192, 4096
LAYERS = 48


def q4_bytes(N: int, K: int) -> int:
    return N * (K // 32) * 20


def layer_bytes() -> dict:
    """Algorithmic HBM bytes of one launch of each op: Q4 weights once, fp32
    activations in and out once (the gate/up launch writes its activation as
    bf16)."""
    w = {"qkv": q4_bytes(N_QKV, H), "o": q4_bytes(H, K_O), "ffn": 3 * q4_bytes(I_FF, H),
         "ffn_gate_up": 2 * q4_bytes(I_FF, H), "ffn_partials": 3 * q4_bytes(I_FF, H)}
    # ffn_partials (the one-token FFN's first launch) is credited with the FFN's
    # own bytes: its slices' partial outputs are traffic, not algorithmic bytes.
    act = {"qkv": 4 * (H + N_QKV), "o": 4 * (K_O + H), "ffn": 4 * (H + H), "ffn_gate_up": 4 * H + 2 * I_FF,
           "ffn_partials": 4 * (H + H)}
    return {k: w[k] + act[k] for k in w}


# The one-token FFN's first launch (gate/up, GeGLU and each 64-row slice's down
# partial; one fp32 token, registered weights): the layer's dominant kernel.
ROOFLINE_KERNEL = "q4_ffn1_kernel<16, 3, false, false>"
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "q4_ffn1_traffic_gemma12b_decode.txt")
CALIBRATION_BYTES = 256 << 20


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def synth_q4_dev(torch, N: int, K: int, gen, dev):
    nb = K // 32
    W = torch.randint(0, 256, (N, nb, 20), dtype=torch.uint8, device=dev, generator=gen)
    s = torch.empty((N, nb), device=dev).uniform_(0.001, 0.02, generator=gen)
    sb = s.to(torch.bfloat16).view(torch.int16).to(torch.int32)
    W[:, :, 16] = (sb & 0xFF).to(torch.uint8)
    W[:, :, 17] = ((sb >> 8) & 0xFF).to(torch.uint8)
    W[:, :, 18:] = 0
    return W.view(N, nb * 20)


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def cpu_baseline(threads: int, host: dict | None = None) -> dict:
    """The oracle (a C restatement of the reference's CPU path) timed on this
    host: one 12B-class layer per call as the reference computes it (per call
    dequantize each matrix to fp32, fp32 matvec, the FFN's bf16 rounding
    points) with `threads` OpenMP threads and with one; the pre-dequantized
    variant of small models (weights dequantized at load, matvecs per call);
    and the 2048 x 2048 gemv_q the reference publishes a CPU time for
    (47.91 ms, tests/bench/gemv_q_bench.txt:3). Median of 10 after 2
    warm-ups (median of 3 after 1 for the one-thread layer, to bound the
    sample to seconds). `host`: the GPU run's first layer and inputs
    (build_layers), timed in place of seeded synthetic ones."""
    import ctypes

    import numpy as np

    import oracle

    L = oracle.lib()
    u8, f32 = ctypes.POINTER(ctypes.c_uint8), ctypes.POINTER(ctypes.c_float)
    ptr = lambda a, t: a.ctypes.data_as(t)  # noqa: E731
    if host:
        Wq, Wo, Wg, Wu, Wd = (np.ascontiguousarray(host[k]) for k in ("Wq", "Wo", "Wg", "Wu", "Wd"))
        xq, xo, xf = (np.ascontiguousarray(host[k], dtype=np.float32) for k in ("x_qkv", "x_o", "x_ffn"))
    else:
        Wq = oracle.synth_q4(N_QKV, H, oracle.seed_for(3, 0))
        Wo = oracle.synth_q4(H, K_O, oracle.seed_for(3, 1))
        Wg = oracle.synth_q4(I_FF, H, oracle.seed_for(3, 2))
        Wu = oracle.synth_q4(I_FF, H, oracle.seed_for(3, 3))
        Wd = oracle.synth_q4(H, I_FF, oracle.seed_for(3, 4))
        xo = oracle.synth_normal(K_O, oracle.seed_for(3, 5))
        xq = xf = xo[:H].copy()
    yq, yo, yf = np.empty(N_QKV, np.float32), np.empty(H, np.float32), np.empty(H, np.float32)

    def layer(th: int, pre: bool = False) -> float:
        g = L.orc_time_gemv_predequant if pre else L.orc_time_gemv_faithful
        f = L.orc_time_ffn_predequant if pre else L.orc_time_ffn_faithful
        t = g(ptr(Wq, u8), ptr(xq, f32), ptr(yq, f32), N_QKV, H, 1, th)
        t += g(ptr(Wo, u8), ptr(xo, f32), ptr(yo, f32), H, K_O, 1, th)
        t += f(ptr(Wg, u8), ptr(Wu, u8), ptr(Wd, u8), ptr(xf, f32), ptr(yf, f32), H, I_FF, 1, th)
        return t

    def med(fn, warm: int, n: int) -> float:
        for _ in range(warm):
            fn()
        return statistics.median(fn() for _ in range(n))

    lb = sum(layer_bytes().values())
    t_all = med(lambda: layer(threads), 2, 10)
    t_one = med(lambda: layer(1), 1, 3)
    # The pre-dequantized variant holds 224 M fp32 weights (0.9 GB) per call.
    t_pre = med(lambda: layer(threads, True), 2, 10)
    W1 = oracle.synth_q4(2048, 2048, oracle.seed_for(1, 0))
    x1 = oracle.synth_normal(2048, oracle.seed_for(1, 1))
    y1 = np.empty(2048, np.float32)
    c1 = lambda th: L.orc_time_gemv_faithful(ptr(W1, u8), ptr(x1, f32), ptr(y1, f32), 2048, 2048, 1, th)  # noqa: E731
    c1_all, c1_one = med(lambda: c1(threads), 2, 10), med(lambda: c1(1), 2, 10)
    return {
        "value": round(lb / t_all / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "us_per_layer": round(t_all * 1e6, 1),
        "nproc": os.cpu_count(),
        "cpu_model": _cpu_model(),
        "rows": {
            "layer_faithful_all_threads": {"threads": threads, "ms": round(t_all * 1e3, 2), "GBps": round(lb / t_all / 1e9, 3)},
            "layer_faithful_1_thread": {"threads": 1, "ms": round(t_one * 1e3, 2), "GBps": round(lb / t_one / 1e9, 3)},
            "layer_predequantized_all_threads": {"threads": threads, "ms": round(t_pre * 1e3, 2),
                                                  "GBps_q4_equiv": round(lb / t_pre / 1e9, 3)},
            "c1_gemv_2048x2048": {"ms_all_threads": round(c1_all * 1e3, 3), "ms_1_thread": round(c1_one * 1e3, 3),
                                  "reference_numpy_ms": 47.91},
        },
        "inputs": "the GPU run's first layer and inputs" if host else "seeded synthetic (oracle.synth_q4)",
        "sample": (f"1 layer (QKV {N_QKV}x{H} + O {H}x{K_O} + FFN {H}x{I_FF}) through the oracle's "
                   f"restatement of the reference CPU path (per call: dequantize to an fp32 matrix, "
                   f"fp32 matvec; FFN bf16 rounding points), median of 10 after 2 warm-ups, {threads} "
                   f"OpenMP threads (the box's CPU share; nproc {os.cpu_count()}); rows: 1 thread "
                   f"(median of 3), pre-dequantized weights, C1 2048x2048"),
    }


def build_layers(torch, aa, nl, dev, host: dict | None = None):
    """nl layers of synthetic registered weights and the ops' inputs. With
    `host` (a dict), the first layer's combined-layout matrices and the
    inputs are also copied into it as NumPy arrays (the CPU baseline's
    inputs)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(0xA1E00300)
    layers = []
    for i in range(nl):
        mq = synth_q4_dev(torch, N_QKV, H, gen, dev)
        mo = synth_q4_dev(torch, H, K_O, gen, dev)
        wg = synth_q4_dev(torch, I_FF, H, gen, dev)
        wu = synth_q4_dev(torch, I_FF, H, gen, dev)
        wd = synth_q4_dev(torch, H, I_FF, gen, dev)
        if host is not None and i == 0:
            for k, t in (("Wq", mq), ("Wo", mo), ("Wg", wg), ("Wu", wu), ("Wd", wd)):
                host[k] = t.cpu().numpy().reshape(-1)
        wq, wo = aa.Q4Weight(mq, N_QKV, H), aa.Q4Weight(mo, H, K_O)
        ffn = aa.FfnWeights(wg, wu, wd, H, I_FF, "gelu")
        del mq, mo, wg, wu, wd
        layers.append((wq, wo, ffn))
    torch.cuda.empty_cache()
    xs = {k: torch.randn(n, device=dev, generator=gen) for k, n in (("qkv", H), ("o", K_O), ("ffn", H))}
    ys = {k: torch.empty(n, device=dev) for k, n in (("qkv", N_QKV), ("o", H), ("ffn", H))}
    if host is not None:
        for k in xs:
            host["x_" + k] = xs[k].cpu().numpy()
    return layers, xs, ys


def profile_pass(torch, aa, dev) -> int:
    """Eager launches for counter collection: a calibration copy of known size
    (torch.mul reading and writing CALIBRATION_BYTES), then 8 layers of each op,
    the two-launch FFN's gate/up launch alone and the one-launch FFN's first
    launch alone, 4 FFN calls of 16 tokens and 4 of 512."""
    src = torch.ones(CALIBRATION_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    del src, dst
    layers, xs, ys = build_layers(torch, aa, 8, dev)
    for wq, wo, ffn in layers:
        wq(xs["qkv"], ys["qkv"])
        wo(xs["o"], ys["o"])
        ffn.gate_up(xs["ffn"])
        ffn.partials(xs["ffn"])
        ffn(xs["ffn"], ys["ffn"])
    # 16-token decode and the M = 512 prefill (bf16-valued activations).
    x16, y16 = torch.randn(16 * H, device=dev), torch.empty(16 * H, device=dev)
    xp = torch.randn(512 * H, device=dev).bfloat16().float()
    yp = torch.empty(512 * H, device=dev)
    for _, _, ffn in layers[:4]:
        ffn(x16, y16, M=16)
        ffn(xp, yp, M=512)
    torch.cuda.synchronize()
    for _, _, ffn in layers:
        ffn.close()
    print("profile pass done", flush=True)
    return 0


def vendor_gemm_us(torch, dev, M: int, H: int, I: int, nl: int) -> dict:
    """µs per call of torch.matmul (the platform's hipBLASLt / rocBLAS bf16
    GEMM) at the M-token FFN's two products, gate and up together (M x 2I x H)
    and down (M x H x I), over nl distinct random bf16 weight sets: a yardstick
    for the Q4 prefill kernels, which also dequantize and apply the GeGLU."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(0xA1E00B1A)
    x = torch.randn(M, H, device=dev, dtype=torch.bfloat16, generator=gen)
    h = torch.randn(M, I, device=dev, dtype=torch.bfloat16, generator=gen)
    wgu = [torch.randn(2 * I, H, device=dev, dtype=torch.bfloat16, generator=gen) for _ in range(nl)]
    wd = [torch.randn(H, I, device=dev, dtype=torch.bfloat16, generator=gen) for _ in range(nl)]

    def timed(fn, reps: int = 3) -> float:
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / (reps * nl)

    gu = timed(lambda: [x @ w.t() for w in wgu])
    dn = timed(lambda: [h @ w.t() for w in wd])
    del wgu, wd
    torch.cuda.empty_cache()
    return {"gate_up_us": round(gu, 2), "down_us": round(dn, 2), "sum_us": round(gu + dn, 2),
            "TFLOPs": round(2.0 * M * 3 * I * H / (gu + dn) / 1e6, 1),
            "note": "torch.matmul bf16 on pre-dequantized weights, no GeGLU; scale reference only"}


_CAPTURE_STREAM = None


def decode_step(torch, aa, dev, nl: int = 48, pos: int = 1500, reps: int = 10) -> dict:
    """A whole Gemma-4-shaped decode step on the device (alveare_amd.layer):
    token embedding, nl layers -- every sixth global (q 8192 + k 512 rows,
    O 3840x8192, one 512-wide kv head), the rest sliding (QKV 8192x3840, O
    3840x4096, window 1024) -- each with its norms, RoPE, KV-cache insert and
    attention over `pos` positions of synthetic cache, the FFN 3840<->15360,
    then the final norm, the 262144x4096 LM head, softcap and greedy token.
    One HIP graph per token, replayed `reps` times (each replay advances the
    position)."""
    import numpy as np

    from alveare_amd import layer

    gen = torch.Generator(device=dev)
    gen.manual_seed(0xA1E00700)
    rng = np.random.default_rng(0xA1E00700)
    pos_dev = torch.zeros(1, dtype=torch.int32, device=dev)
    tables = {s: layer.cos_sin_table_gemma(1e4 if s else 1e6, 256 if s else 512, 2048) for s in (True, False)}
    layers, wbytes = [], 0
    for l in range(nl):
        sliding = (l + 1) % 6 != 0
        D = 256 if sliding else 512
        n_qkv = 8192 if sliding else 8192 + 512
        q_size = 16 * D
        norms = {k: rng.uniform(0.5, 1.5, D if k in ("q", "k") else H).astype(np.float32)
                 for k in ("attn", "q", "k", "post_attn", "ffn", "post_ffw")}
        L = layer.Gemma4DecodeLayer(qkv=synth_q4_dev(torch, n_qkv, H, gen, dev), o=synth_q4_dev(torch, H, q_size, gen, dev),
                                    gate=synth_q4_dev(torch, I_FF, H, gen, dev), up=synth_q4_dev(torch, I_FF, H, gen, dev),
                                    down=synth_q4_dev(torch, H, I_FF, gen, dev), norms=norms, scale=0.9, sliding=sliding,
                                    H=H, I=I_FF, max_seq=2048, device=dev, rope_table=tables[sliding], pos_dev=pos_dev)
        L.kcache.normal_(generator=gen)
        L.vcache.normal_(generator=gen)
        layers.append(L)
        wbytes += q4_bytes(n_qkv, H) + q4_bytes(H, q_size) + 3 * q4_bytes(I_FF, H)
        torch.cuda.empty_cache()
    head = aa.Q4Weight(synth_q4_dev(torch, VOC, KH, gen, dev), VOC, KH)
    wbytes += q4_bytes(VOC, KH)
    table = (torch.randn(VOC, H, device=dev, generator=gen) * 0.05).half()
    dec = layer.Gemma4Decoder(layers, table, np.ones(H, np.float32), head, VOC, softcap=30.0)
    torch.cuda.empty_cache()
    dec.step(token=1, pos=pos)  # eager step: sizes the decoder stream's scratch
    torch.cuda.synchronize()
    g = dec.capture()
    dec.token_dev.fill_(1)
    pos_dev.fill_(pos)
    with torch.cuda.stream(dec.stream):
        for _ in range(2):
            g.replay()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            g.replay()
        b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / reps
    end_pos = int(pos_dev.item())
    del g
    for L in layers:
        L.close()
    head.close()
    del layers, dec, table
    torch.cuda.empty_cache()
    return {"us_per_token": round(us, 1), "tokens_per_s": round(1e6 / us, 1), "layers": nl, "context_pos": pos,
            "end_pos": end_pos, "weight_GB_per_token": round(wbytes / 1e9, 3), "GBps_weights": round(wbytes / us / 1e3, 1),
            "note": "embedding, 48 layers with attention over the cache, final norm, LM head, softcap and argmax; "
                    "one HIP graph per token, device-resident token and position"}


READ_SHAPES = [(wg, depth) for wg in (2, 4, 8) for depth in (4, 8, 16)]


# The reference runtime's registered (zero-padded) Gemma-4 shapes and its
# published per-call times on the XDNA2 NPU (host-observed, 20-call average,
# benchmarks/reports/20260722-223400-7c67e12.md:11-17): name -> (padded N,
# padded K, real N, real K, NPU ms). The FFN and the batched GEMM follow.
PADDED_GEMV = {
    "qkv_sliding_8192x4096": (8192, 4096, 8192, 3840, 1.73),
    "o_sliding_8192x4096": (8192, 4096, 3840, 4096, 1.70),
    "qk_global_10240x4096": (10240, 4096, 8704, 3840, 2.19),
    "o_global_4096x8192": (4096, 8192, 3840, 8192, 1.73),
    "lm_head_chunk_16384x4096": (16384, 4096, 16384, 3840, 3.37),
}
PADDED_FFN = (4096, 16384, 3840, 15360, 9.65)       # ffn_fused H=4096, I=16384 (gelu)
PADDED_GEMM = (16, 16384, 4096, 15360, 3840, 205.23)  # gemm_q B=16, 16384x4096


def padded_shapes(torch, aa, dev) -> dict:
    """Per-call time at the shapes the reference's C++ runtime registers
    (runtime/cpp/src/weights.cpp:300-330, model.cpp:374-379; zero padding from
    tools/quantize_gemma4.py:145-187) beside the same ops at the real shapes.
    Registration trims the all-zero padding, so the padded call streams the
    real matrix: GB/s is reported against the executed bytes and against the
    padded bytes. Distinct weight sets rotate past the Infinity Cache."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(0xA1E00500)

    def padded(N, K, Np, Kp):
        W = synth_q4_dev(torch, N, K, gen, dev)
        P = torch.zeros((Np, Kp // 32 * 20), dtype=torch.uint8, device=dev)
        P[:N, :K // 32 * 20] = W
        return W, P

    out = {}
    for name, (Np, Kp, N, K, npu_ms) in PADDED_GEMV.items():
        n = max(4, min(32, (400 << 20) // q4_bytes(N, K)))
        reals, pads = [], []
        for _ in range(n):
            W, P = padded(N, K, Np, Kp)
            reals.append(aa.Q4Weight(W, N, K))
            pads.append(aa.Q4Weight(P, Np, Kp))
            del W, P
        x = torch.randn(Kp, device=dev, generator=gen)
        x[K:] = 0
        yp = torch.empty(Np, device=dev)
        yr = torch.empty(N, device=dev)
        xr = x[:K].contiguous()
        us_p = graph_us(torch, lambda: [w(x, yp) for w in pads], 5, n)
        us_r = graph_us(torch, lambda: [w(xr, yr) for w in reals], 5, n)
        eb = q4_bytes(N, K) + 4 * (K + Np)
        out[name] = {"us": round(us_p, 3), "us_unpadded": round(us_r, 3), "exec_shape": list(pads[0].exec_shape),
                     "GBps_executed": round(eb / us_p / 1e3, 1),
                     "GBps_padded_bytes": round((q4_bytes(Np, Kp) + 4 * (Kp + Np)) / us_p / 1e3, 1),
                     "reference_npu_ms": npu_ms, "speedup_vs_npu": round(npu_ms * 1e3 / us_p, 1)}
        for w in reals + pads:
            w.close()
        torch.cuda.empty_cache()
    Hp, Ip, H_, I_, npu_ms = PADDED_FFN
    fr, fp = [], []
    for _ in range(4):
        g, pg = padded(I_, H_, Ip, Hp)
        u, pu = padded(I_, H_, Ip, Hp)
        d, pd = padded(H_, I_, Hp, Ip)
        fr.append(aa.FfnWeights(g, u, d, H_, I_, "gelu"))
        fp.append(aa.FfnWeights(pg, pu, pd, Hp, Ip, "gelu"))
        del g, u, d, pg, pu, pd
    x = torch.randn(Hp, device=dev, generator=gen)
    x[H_:] = 0
    xr = x[:H_].contiguous()
    yp, yr = torch.empty(Hp, device=dev), torch.empty(H_, device=dev)
    us_p = graph_us(torch, lambda: [f(x, yp) for f in fp], 5, 4)
    us_r = graph_us(torch, lambda: [f(xr, yr) for f in fr], 5, 4)
    eb = 3 * q4_bytes(I_, H_) + 8 * H_
    out["ffn_fused_4096x16384"] = {"us": round(us_p, 3), "us_unpadded": round(us_r, 3),
                                   "exec_shape": list(fp[0].exec_shape),
                                   "GBps_executed": round(eb / us_p / 1e3, 1),
                                   "GBps_padded_bytes": round((3 * q4_bytes(Ip, Hp) + 8 * Hp) / us_p / 1e3, 1),
                                   "reference_npu_ms": npu_ms, "speedup_vs_npu": round(npu_ms * 1e3 / us_p, 1)}
    for f in fr + fp:
        f.close()
    del fr, fp
    torch.cuda.empty_cache()
    B, Np, Kp, N, K, npu_ms = PADDED_GEMM
    reals, pads = [], []
    for _ in range(8):
        W, P = padded(N, K, Np, Kp)
        reals.append(aa.Q4Weight(W, N, K))
        pads.append(aa.Q4Weight(P, Np, Kp))
        del W, P
    X = torch.randn(B, Kp, device=dev, generator=gen).bfloat16().float()
    X[:, K:] = 0
    Xr = X[:, :K].contiguous()
    Yp, Yr = torch.empty(B, Np, device=dev), torch.empty(B, N, device=dev)
    us_p = graph_us(torch, lambda: [w(X, Yp, M=B) for w in pads], 3, 8)
    us_r = graph_us(torch, lambda: [w(Xr, Yr, M=B) for w in reals], 3, 8)
    out["gemm_b16_16384x4096"] = {"us": round(us_p, 3), "us_unpadded": round(us_r, 3),
                                  "exec_shape": list(pads[0].exec_shape),
                                  "GBps_executed": round((q4_bytes(N, K) + 4 * B * (K + Np)) / us_p / 1e3, 1),
                                  "reference_npu_ms": npu_ms, "speedup_vs_npu": round(npu_ms * 1e3 / us_p, 1)}
    for w in reals + pads:
        w.close()
    torch.cuda.empty_cache()
    out["note"] = ("us per call at the reference runtime's registered padded shape and at the real shape; "
                   "registration trims the zero padding, so both stream the same bytes; reference_npu_ms is "
                   "its published XDNA2 per-call time (benchmarks/reports/20260722-223400-7c67e12.md:11-17)")
    return out


_PROBE = None


def probe_lib():
    """measure/libalveare_probe.so (the streaming-read probe), built by
    __graft_entry__.build() beside the product library."""
    global _PROBE
    if _PROBE is None:
        import ctypes
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "measure", "libalveare_probe.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built (run __graft_entry__.build())")
        lib = ctypes.CDLL(path)
        lib.alvprobe_stream_read.restype = ctypes.c_int
        lib.alvprobe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                                             ctypes.c_int, ctypes.c_void_p]
        lib.alvprobe_last_error.restype = ctypes.c_char_p
        _PROBE = lib
    return _PROBE


def read_floor(torch, aa, dev) -> dict:
    """The practical ceiling per launch: a plain streaming read of each op's
    weight bytes, from distinct regions of a 2 GiB buffer (far beyond the
    Infinity Cache), timed like the ops: the default shape (4 workgroups per
    CU, 4 loads in flight per thread) and the fastest of a sweep over queue
    depth (measure/libalveare_probe.so: 2-8 workgroups per CU,
    4-16 loads per thread, up to 512 KiB in flight per CU)."""
    L = probe_lib()
    big = torch.empty(2 << 30, dtype=torch.uint8, device=dev)
    sink = torch.zeros(2048, dtype=torch.int32, device=dev)
    sizes = {"qkv": q4_bytes(N_QKV, H), "o": q4_bytes(H, K_O), "ffn_gate_up": 2 * q4_bytes(I_FF, H),
             "ffn_down": q4_bytes(H, I_FF)}
    out = {}
    for k, nbytes in sizes.items():
        nb = nbytes // 256 * 256
        n = min(48, big.numel() // nb)

        def timed(wg, depth, nb=nb, n=n):
            def fn():
                st = torch.cuda.current_stream().cuda_stream
                for i in range(n):
                    rc = L.alvprobe_stream_read(big.data_ptr() + i * nb, nb, sink.data_ptr(), wg, depth, st)
                    if rc:
                        raise RuntimeError(f"alvprobe_stream_read failed: {L.alvprobe_last_error().decode()}")
            return graph_us(torch, fn, 3, n)

        us = timed(4, 4)
        sweep = {f"{wg}x{depth}": timed(wg, depth) for wg, depth in READ_SHAPES}
        best = min(sweep, key=sweep.get)
        out[k] = {"us": round(us, 3), "GBps": round(nb / us / 1e3, 1),
                  "best_shape": best, "best_us": round(sweep[best], 3),
                  "best_GBps": round(nb / sweep[best] / 1e3, 1),
                  "sweep_us": {s: round(v, 3) for s, v in sweep.items()}}
    layer = out["qkv"]["us"] + out["o"]["us"] + out["ffn_gate_up"]["us"] + out["ffn_down"]["us"]
    out["layer_us"] = round(layer, 3)
    out["layer_best_us"] = round(sum(out[k]["best_us"] for k in sizes), 3)
    del big
    torch.cuda.empty_cache()
    return out


def graph_us(torch, fn, reps: int, per: int) -> float:
    """Mean time of one of the `per` launches `fn` enqueues: a HIP graph of
    fn replayed `reps` times between HIP events on the replay stream."""
    s = torch.cuda.current_stream()
    # Warm up on the capture stream itself: per-stream scratch (prefill) is
    # sized by an ordinary call, never during capture.
    global _CAPTURE_STREAM
    if _CAPTURE_STREAM is None:
        _CAPTURE_STREAM = torch.cuda.Stream()
    cs = _CAPTURE_STREAM
    cs.wait_stream(s)
    with torch.cuda.stream(cs):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        fn()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(s)
    for _ in range(reps):
        g.replay()
    b.record(s)
    torch.cuda.synchronize()
    del g
    return a.elapsed_time(b) * 1e3 / (reps * per)


def eager_calls(torch, aa, dev, n: int = 200) -> dict:
    """Wall time per eager call from Python, the host cost the reference's
    per-call profile counts (tests/bench/gemma4_profile.txt: per-call host
    overhead plus host<->device copies): device tensors in and out (Python ->
    ctypes -> plan -> launch, n calls then one synchronize), and the drop-in
    dispatch with host NumPy bf16 in and out (upload, launch, download: each
    call synchronises), for the 8192x3840 QKV GEMV and the 3840<->15360 FFN."""
    import numpy as np

    from alveare_amd.runtime import Q4Dispatch, ResidentWeight

    gen = torch.Generator(device=dev)
    gen.manual_seed(0xEA6E)
    wq_t = synth_q4_dev(torch, N_QKV, H, gen, dev)
    wq = aa.Q4Weight(wq_t, N_QKV, H)
    ffn = aa.pack_ffn_fused_weights(synth_q4_dev(torch, I_FF, H, gen, dev), synth_q4_dev(torch, I_FF, H, gen, dev),
                                    synth_q4_dev(torch, H, I_FF, gen, dev), H, I_FF)
    x = torch.randn(H, device=dev)
    yq = torch.empty(N_QKV, device=dev)
    yf = torch.empty(H, device=dev)

    def per_call(fn, sync_each: bool) -> float:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
            if sync_each:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n * 1e6

    out = {"gemv_8192x3840_device_tensors": round(per_call(lambda: wq(x, yq), False), 2),
           "ffn_3840x15360_device_tensors": round(per_call(lambda: ffn(x, yf), False), 2)}
    d = Q4Dispatch(H, I_FF, "gemma4", dev, host_io=True)
    rw = ResidentWeight(wq_t.reshape(-1), (N_QKV, H // 32 * 20))
    l = d.register_ffn(*(synth_q4_dev(torch, r, c, gen, dev).view(r, c // 32 * 20) for r, c in
                         ((I_FF, H), (I_FF, H), (H, I_FF))))
    xh = np.asarray(x.cpu().numpy(), np.float32)
    out["gemv_8192x3840_host_numpy_bf16"] = round(per_call(lambda: d.run_gemv_npu(rw, xh), True), 2)
    out["ffn_3840x15360_host_numpy_bf16"] = round(per_call(lambda: d.run_ffn_fused_npu(l, xh), True), 2)
    out["note"] = ("per call, wall clock; device-tensor calls are launch-bound on the host when shorter than the "
                   "kernel; the reference's decode profile spends about 106 us of host overhead and 417 us of "
                   "host<->device copies per call")
    wq.close()
    ffn.close()
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--profile-pass", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="only the headline workload (no extra_configs): the run profiled for the roofline kernel")
    ap.add_argument("--decode-step", action="store_true",
                    help="only the whole-decode-step measurement (its own JSON line): the run profiled for the "
                         "decode step's kernel breakdown")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this path runs on a single MI355X and takes no collective; "
              "multi-GPU runs are not part of it (use --gpus 1).", file=sys.stderr)
        return 2

    import torch

    import alveare_amd as aa

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    aa.lib()
    if args.profile_pass:
        return profile_pass(torch, aa, dev)
    if args.decode_step:
        print(json.dumps(decode_step(torch, aa, dev, reps=max(1, args.steps))), flush=True)
        return 0
    nl = args.layers
    log(f"building {nl} synthetic layers on {torch.cuda.get_device_name(dev)}")
    t0 = time.time()
    host = {} if not args.no_cpu_baseline else None
    layers, xs, ys = build_layers(torch, aa, nl, dev, host)
    torch.cuda.synchronize()
    log(f"layers ready in {time.time() - t0:.1f}s; {torch.cuda.memory_allocated() / 1e9:.2f} GB held by torch")

    def step():
        for wq, wo, ffn in layers:
            wq(xs["qkv"], ys["qkv"])
            wo(xs["o"], ys["o"])
            ffn(xs["ffn"], ys["ffn"])

    # Per-op breakdown and the roofline kernel: a graph of the op's launches
    # over all layers (distinct weights), HIP events on the replay stream.
    lb = layer_bytes()
    ops = {
        "qkv": (lambda: [wq(xs["qkv"], ys["qkv"]) for wq, _, _ in layers], 1),
        "o": (lambda: [wo(xs["o"], ys["o"]) for _, wo, _ in layers], 1),
        "ffn": (lambda: [ffn(xs["ffn"], ys["ffn"]) for _, _, ffn in layers], 1),
        "ffn_gate_up": (lambda: [ffn.gate_up(xs["ffn"]) for _, _, ffn in layers], 1),
        "ffn_partials": (lambda: [ffn.partials(xs["ffn"]) for _, _, ffn in layers], 1),
    }
    breakdown = {}
    for k, (fn, per) in ops.items():
        us = graph_us(torch, fn, 10, nl * per)
        breakdown[k] = {"us": round(us, 3), "GBps": round(lb[k] / us / 1e3, 1)}

    floor = read_floor(torch, aa, dev)

    # Whole step from a HIP graph (the launch-bound loop of 3 x 48 ops).
    for _ in range(max(1, args.warmup)):
        step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(max(1, args.warmup)):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s = torch.cuda.current_stream()
    torch.cuda.synchronize()
    start.record(s)
    for _ in range(args.steps):
        g.replay()
    end.record(s)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    step_bytes = nl * (lb["qkv"] + lb["o"] + lb["ffn"])
    gbs = step_bytes / (ms * 1e-3) / 1e9
    gu_us = breakdown["ffn_partials"]["us"]
    gu_gbs = lb["ffn_partials"] / (gu_us * 1e-6) / 1e9

    extra = {}
    if not args.no_extra:
        # Small-M decode against the 12B-class FFN (M tokens share one weight
        # read) and prefill at M = 512 (MFMA tiled kernel, GeGLU fused): per call
        # over distinct layers.
        extra = {"small_m_ffn": {}, "prefill_ffn_m512": None}
        for M in (2, 4, 8, 16):
            xm = torch.randn(M * H, device=dev)
            ym = torch.empty(M * H, device=dev)
            us = graph_us(torch, lambda: [ffn(xm, ym, M=M) for _, _, ffn in layers], 2, nl)
            byts = 3 * q4_bytes(I_FF, H) + M * (4 * H + 4 * H)
            extra["small_m_ffn"][str(M)] = {"us": round(us, 3), "GBps": round(byts / us / 1e3, 1)}
        Mp = 512
        # bf16-valued activations, as the reference's prefill passes them (x_bf16):
        # one activation term per token tile.
        xp = torch.randn(Mp * H, device=dev).bfloat16().float()
        yp = torch.empty(Mp * H, device=dev)
        npf = min(nl, 8)
        us = graph_us(torch, lambda: [ffn(xp, yp, M=Mp) for _, _, ffn in layers[:npf]], 2, npf)
        flops = 2.0 * Mp * 3 * I_FF * H
        extra["prefill_ffn_m512"] = {"us": round(us, 2), "TFLOPs": round(flops / us / 1e6, 1),
                                     "mfma_frac_bf16_dense": round(flops / us / 1e6 / 2500.0, 4)}
        # For scale only (not the product path): the vendor bf16 GEMM
        # (torch.matmul -> hipBLASLt) on already-dequantized bf16 weights of the
        # same shapes, without the GeGLU between the two products.
        extra["prefill_ffn_m512"]["vendor_bf16_gemm_reference"] = vendor_gemm_us(torch, dev, Mp, H, I_FF, npf)

        # Where the streaming kernel should hand over to the MFMA tiled kernel
        # (small-M decode against the 12B-class FFN): both kernels at M = 8 ... 128
        # (finely between 16 and 48, where the crossovers lie),
        # selected with the library's ALV_TILED_MIN_M knob, for fp32 activations
        # (three bf16 terms on the tiled kernel) and bf16-valued ones (one term).
        cross = {}
        xm32 = torch.randn(128 * H, device=dev)
        xm16 = xm32.bfloat16().float()
        ym = torch.empty(128 * H, device=dev)
        ncross = min(nl, 16)
        prev = os.environ.get("ALV_TILED_MIN_M")
        try:
            for xname, xm in (("x_fp32", xm32), ("x_bf16_valued", xm16)):
                for kind, knob in (("streaming", "1000000"), ("tiled", "1")):
                    os.environ["ALV_TILED_MIN_M"] = knob
                    row = cross.setdefault(f"{kind}_{xname}", {})
                    for M in (8, 16, 17, 20, 24, 28, 32, 40, 48, 64, 96, 128):
                        us = graph_us(torch, lambda: [ffn(xm, ym, M=M) for _, _, ffn in layers[:ncross]], 2, ncross)
                        row[str(M)] = round(us, 2)
        finally:
            if prev is None:
                os.environ.pop("ALV_TILED_MIN_M", None)
            else:
                os.environ["ALV_TILED_MIN_M"] = prev
        extra["small_m_crossover_ffn_us"] = cross

        # C1 and C2 as HBM numbers: 128 distinct 2048 x 2048 weights (336 MB) and
        # 32 distinct Gemma-3-1B-like FFNs 1152 <-> 6912 (478 MB), rotated so the
        # working set exceeds the Infinity Cache.
        g1 = torch.Generator(device=dev)
        g1.manual_seed(0xA1E00100)
        c1w = [aa.Q4Weight(synth_q4_dev(torch, 2048, 2048, g1, dev), 2048, 2048) for _ in range(128)]
        x1 = torch.randn(2048, device=dev, generator=g1)
        y1 = torch.empty(2048, device=dev)
        us = graph_us(torch, lambda: [w(x1, y1) for w in c1w], 5, 128)
        b1 = q4_bytes(2048, 2048) + 4 * 2048 * 2
        extra["c1_gemv_2048x2048_x128"] = {"us": round(us, 3), "GBps": round(b1 / us / 1e3, 1)}
        for w in c1w:
            w.close()
        del c1w
        H2, I2 = 1152, 6912
        g2 = torch.Generator(device=dev)
        g2.manual_seed(0xA1E00200)
        c2f = []
        for _ in range(32):
            wg, wu, wd = (synth_q4_dev(torch, I2, H2, g2, dev), synth_q4_dev(torch, I2, H2, g2, dev),
                          synth_q4_dev(torch, H2, I2, g2, dev))
            c2f.append(aa.FfnWeights(wg, wu, wd, H2, I2, "gelu"))
            del wg, wu, wd
        x2 = torch.randn(H2, device=dev, generator=g2)
        y2 = torch.empty(H2, device=dev)
        us = graph_us(torch, lambda: [f(x2, y2) for f in c2f], 5, 32)
        b2 = 3 * q4_bytes(I2, H2) + 4 * H2 * 2
        extra["c2_ffn_1152x6912_x32"] = {"us": round(us, 3), "GBps": round(b2 / us / 1e3, 1)}
        for f in c2f:
            f.close()
        del c2f
        torch.cuda.empty_cache()

        # LM head: the reference's 262144 x 4096 Q4 head (671 MB, beyond the
        # Infinity Cache), GEMV + softcap 30 + greedy argmax per call.
        gen = torch.Generator(device=dev)
        gen.manual_seed(0xA1E00600)
        head = aa.Q4Weight(synth_q4_dev(torch, VOC, KH, gen, dev), VOC, KH)
        torch.cuda.empty_cache()
        xh = torch.zeros(KH, device=dev)
        xh[:H] = torch.randn(H, device=dev, generator=gen)
        lh = torch.empty(VOC, device=dev)
        us = graph_us(torch, lambda: [aa.lm_head(head, xh, VOC, 30.0, lh) for _ in range(8)], 5, 8)
        hb = q4_bytes(VOC, KH) + 4 * KH + 4 * VOC
        extra["lm_head_262144x4096"] = {"us": round(us, 2), "GBps": round(hb / us / 1e3, 1),
                                        "pct_of_peak": round(100 * hb / us / 1e3 / HBM_PEAK_GBS, 1)}
        head.close()
        del head

        # GPU quantizer on the LM head's float32 weights (262144 x 3840, 4.03 GB)
        # zero-padded to 4096 columns, as the reference's quantizer pads it
        # (tools/quantize_gemma4.py:130-133): bytes = fp32 read + Q4 written.
        wq = torch.randn(VOC, H, device=dev, generator=gen).mul_(0.02)
        qout = torch.empty((VOC, KH // 32 * 20), dtype=torch.uint8, device=dev)
        L = aa.lib()

        def quant():
            st = torch.cuda.current_stream().cuda_stream
            rc = L.alv_quantize_q4(wq.data_ptr(), VOC, H, H, qout.data_ptr(), VOC, KH, st)
            if rc:
                raise RuntimeError(f"alv_quantize_q4 failed ({rc})")

        us = graph_us(torch, quant, 5, 1)
        qb = 4 * VOC * H + q4_bytes(VOC, KH)
        extra["quantize_262144x3840_to_4096"] = {"us": round(us, 1), "GBps": round(qb / us / 1e3, 1)}
        del wq, qout
        torch.cuda.empty_cache()

        extra["padded_shapes"] = padded_shapes(torch, aa, dev)
        extra["decode_step_gemma4_48l"] = decode_step(torch, aa, dev)
        extra["eager_call_us"] = eager_calls(torch, aa, dev)

    from measure import profiling

    out = {
        "metric": "Q4 GEMV/fused-FFN achieved HBM GB/s (% of peak) + µs/layer at 3840×15360",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": (f"gemma-12b-class decode layer x{nl}: fused qkv gemv {N_QKV}x{H}, o gemv {H}x{K_O}, "
                         f"ffn_fused {H}<->{I_FF} gelu_tanh; q4 group 32 (20 B/32 w), scales ~U(0.001,0.02) "
                         f"bf16, batch 1, fp32 activations; registered (tiled) weights"),
            "layers": nl,
            "weight_bytes_per_layer": q4_bytes(N_QKV, H) + q4_bytes(H, K_O) + 3 * q4_bytes(I_FF, H),
            "hip_graph": True,
        },
        "us_per_layer": round(ms * 1e3 / nl, 3),
        "pct_of_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
        "breakdown": breakdown,
        "read_floor": floor,
        "roofline": {
            "bound": "hbm",
            "kernel": ROOFLINE_KERNEL + " (one-token ffn: gate/up 15360x3840 x2 + GeGLU + down 3840x15360 in "
                                        "64-row slices; its partials are summed by ffn1_sum_kernel)",
            "achieved": round(gu_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
            "traffic": profiling.read_traffic(TRAFFIC_FILE, ROOFLINE_KERNEL),
            "algorithmic_bytes_per_launch": lb["ffn_partials"],
            "avg_launch_us": gu_us,
        },
        "cpu_baseline": None,
        "extra_configs": extra,
    }
    if not args.no_cpu_baseline:
        threads = args.cpu_threads or int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, os.cpu_count() or 1)
        try:
            out["cpu_baseline"] = cpu_baseline(threads, host)
        except Exception as e:  # the baseline is reported, never required
            out["cpu_baseline"] = {"error": repr(e)}
    print(json.dumps(out), flush=True)
    for _, _, ffn in layers:
        ffn.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
