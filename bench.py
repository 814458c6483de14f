"""Speculative-verify hot path on one MI355X: weight/KV-stream GB/s and verify-step µs.

Headline (``value``): the 8B-shaped 8-bit decoder-layer projection set (q, k, v, o, gate, up,
down; hidden 4096, 32/8 heads x 128, intermediate 12288, group 64) at M = 16 verify rows. One
step = that set for one layer, launched the way a verify forward issues it (q/k/v in one
launch, o, gate/up in one launch, down), rotating over a pool of distinct layers (>= 1.5 GB,
far past the 256 MB Infinity Cache) so every byte comes from HBM. K steps are captured as one
HIP graph; ``ms_per_step`` is the median over >= 10 event-bracketed replays, divided by K.
``value`` = algorithmic bytes / that time.

``roofline`` is for the dominant kernel (the gate/up qmm launch): its algorithmic bytes over its
average duration (median of replays of a graph of K back-to-back launches, HIP events on the
launch stream). ``legs`` carries the same block for each part of the metric: that launch, the
single 4096x4096 qmm, verify attention at 32k keys (bf16, fp16, head dim 256, 8- and 4-bit KV),
the MoE block and the 64-layer verify step at 16k context, each with its fraction of the
8 TB/s peak, of a measured bandwidth (``bandwidth``: the best of a device copy, an fp16 matvec
over 512 MB as the reference measures it, calibrate.py:871-894, and the library's streaming
read probe over 1 GiB; the probe over one gate+up launch's 108 MB is reported beside it) and, where
MFMA does the work, the useful FLOP/s as a fraction of the 2.5 PFLOP/s dense bf16 peak.
``extra`` holds the sweeps (qmm M, attention L, verify width x depth) and the prefill wide path
(stock vs wide at M 256..2048, and its dequantize kernel, also a leg). ``cpu_baseline``: the C
restatement (oracle/dspark_oracle.c, OpenMP on every core of this process's affinity) on a
bounded sample of the layer set, with torch-CPU fp32 and C attention / MoE legs beside it.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--quick]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mlx-dspark_amd"))

METRIC = "verify-step µs + weight/KV-stream GB/s (% of HBM peak), M=16 qmm & attention"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0   # dense bf16 / fp16
MALL_BYTES = 256 << 20
REPEATS = 11                # timed replays per measurement (the median is reported)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ------------------------------------------------------------------ byte accounting

def qmm_bytes(n: int, k: int, bits: int, m: int) -> int:
    """Algorithmic bytes of one affine qmm: packed weights + bf16 scales/biases + x + y."""
    return n * k * bits // 8 + 2 * 2 * n * (k // 64) + 2 * m * k + 2 * m * n


def attn_bytes(hq: int, hk: int, d: int, mq: int, L: int, kv_bits: int = 16) -> int:
    """K/V stream (L keys incl. the verify rows) + q + out; quantized K/V add their per-64
    scales and biases (2 bytes each)."""
    kv_row = d * kv_bits // 8 + (0 if kv_bits == 16 else 2 * 2 * (d // 64))
    return 2 * hk * L * kv_row + 2 * 2 * hq * mq * d


def attn_flops(hq: int, mq: int, d: int, L: int) -> int:
    return 4 * hq * mq * d * L


def leg(name: str, nbytes: int, us: float, bw_measured: float | None, flops: int | None = None, **more) -> dict:
    """One leg of the metric: time, achieved GB/s and its fractions of the peak and of the
    measured bandwidth; MFMA utilisation when FLOPs are given."""
    gbs = nbytes / (us * 1e-6) / 1e9
    out = {"name": name, "bytes": int(nbytes), "us": round(us, 3), "GBs": round(gbs, 1),
           "bound": "hbm", "peak": HBM_PEAK_GBS, "frac": round(gbs / HBM_PEAK_GBS, 4),
           "frac_of_measured": round(gbs / bw_measured, 4) if bw_measured else None}
    if flops:
        tf = flops / (us * 1e-6) / 1e12
        out["TFLOPs"] = round(tf, 2)
        out["mfma_util"] = round(tf / MFMA_PEAK_TFLOPS, 5)
    out.update(more)
    return out


# ------------------------------------------------------------------ timing helpers

def _median_replay_ms(g, repeats: int = REPEATS) -> float:
    import torch

    g.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(repeats):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1))
    return statistics.median(times)


def gate_up_kernel_name(ls) -> str:
    """The kernel the layer set's gate+up launch runs (the library's plan query), with its grid."""
    from dspark_rocm import ops

    P = ls.packs[0]
    p = ops.packed_multi_plan([ls.x["gu"]], [P["gate"], P["up"]])
    k = P["gate"].k
    if p["kernel"] == "per CU":
        name = f"qmm_cu_kernel<{ls.bits},{p['tiles_per_workgroup']},{k // 64 // p['slices']}>"
    elif p["kernel"] == "whole-K tile":
        name = f"qmm_wk_kernel<{ls.bits},8,true,true>"
    else:
        name = f"qmm_sk_kernel<{ls.bits},4,{16 if k // 64 // p['slices'] > 8 else 8},true,true,false>"
    return (f"{name} gate+up launch, packed form (N=2x{P['gate'].n}, K={k}, M={ls.m}; "
            f"{p['workgroups']} workgroups, {p['kernel']})")


def time_graph(fn, repeats: int = REPEATS, warm: int = 2):
    """Capture ``fn`` (which enqueues work on the current stream) into a HIP graph on a warmed
    side stream; returns (median ms per replay over ``repeats`` event-bracketed replays, graph)."""
    import torch

    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # per-stream workspaces are allocated (and zeroed) here, outside the capture
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        fn()
    torch.cuda.synchronize()
    return _median_replay_ms(g, repeats), g


def time_eager(fn, repeats: int = REPEATS, warm: int = 2) -> float:
    """Median ms of ``fn`` called eagerly between two HIP events (for single large library ops,
    which stay out of graphs: some record memsets)."""
    import torch

    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(repeats):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1))
    return statistics.median(times)


# ------------------------------------------------------------------ bandwidth

def measure_bandwidth(dev) -> dict:
    """Achievable HBM bandwidth, median of REPEATS eager calls each: a 1 GiB device copy (read +
    write bytes), the library's streaming-read probe (``dspark_stream_read``, 16-byte
    non-temporal loads) over 1 GiB and over 108 MB (one gate+up launch's bytes), and an fp16
    matvec streaming a 512 MB matrix (the reference's probe, calibrate.py:871-894)."""
    import torch

    from dspark_rocm import ops

    out = {}
    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    ms = time_eager(lambda: b.copy_(a))
    out["copy_GBs"] = round(2 * n / (ms * 1e-3) / 1e9, 1)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    ms = time_eager(lambda: ops.stream_read(a, sink))
    out["read_GBs"] = round(n / (ms * 1e-3) / 1e9, 1)
    # 108 MB at a time, rotating over the 9 disjoint slices of the 1 GiB buffer (more than the
    # 256 MB MALL), so no call reads from the last one's cache
    m = 107872256
    slices = [a[i * m:(i + 1) * m] for i in range(n // m)]
    chain = 2 * len(slices)

    def reads():
        for i in range(chain):
            ops.stream_read(slices[i % len(slices)], sink)

    ms = time_eager(reads) / chain  # back to back, as the qmm legs are timed
    out["read_108MB_GBs"] = round(m / (ms * 1e-3) / 1e9, 1)
    del a, b, slices
    dim = int(((512 << 20) / 2) ** 0.5) // 64 * 64
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    w = torch.randn((dim, dim), generator=g, device=dev).to(torch.float16)
    v = torch.randn(dim, generator=g, device=dev).to(torch.float16)
    y = torch.empty(dim, dtype=torch.float16, device=dev)
    ms = time_eager(lambda: torch.mv(w, v, out=y))
    out["matvec_GBs"] = round(w.numel() * 2 / (ms * 1e-3) / 1e9, 1)
    del w
    torch.cuda.empty_cache()
    out["measured_GBs"] = max(out["copy_GBs"], out["read_GBs"], out["matvec_GBs"])
    return out


# ------------------------------------------------------------------ workloads

class LayerSet:
    """The projection set of an 8B-shaped layer: q/k/v/o/gate/up/down, 8- or 4-bit g64, M rows; a
    pool of layers. Each matrix is held in the reference layout and in the packed qmm form
    (``ops.qmm_pack``); ``packed`` selects which one the launches read (the products are
    bit-identical)."""

    H, HQ, HK, D, I = 4096, 32, 8, 128, 12288

    def __init__(self, dev, bits: int, m: int, layers: int, seed: int = 1):
        import torch

        from dspark_rocm import ops
        from dspark_rocm.quant import random_quantized

        self.bits, self.m = bits, m
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        H, I, D = self.H, self.I, self.D
        shapes = {"q": (self.HQ * D, H), "k": (self.HK * D, H), "v": (self.HK * D, H), "o": (H, self.HQ * D),
                  "gate": (I, H), "up": (I, H), "down": (H, I)}
        self.shapes = shapes
        self.layers = [{name: random_quantized(n, k, bits, generator=g, device=dev) for name, (n, k) in shapes.items()}
                       for _ in range(layers)]
        self.packs = [{name: ops.qmm_pack(*L[name], bits=bits) for name in shapes} for L in self.layers]
        self.packed = True
        self.x = {k: torch.randn((m, kk), generator=g, device=dev).to(torch.bfloat16)
                  for k, kk in (("qkv", H), ("o", self.HQ * D), ("gu", H), ("down", I))}
        self.y = {name: torch.empty((m, n), dtype=torch.bfloat16, device=dev) for name, (n, _) in shapes.items()}
        self.bytes_per_step = sum(qmm_bytes(n, k, bits, m) for n, k in shapes.values())
        self.flops_per_step = sum(2 * m * n * k for n, k in shapes.values())
        self.weight_bytes = sum(n * k * bits // 8 + 4 * n * (k // 64) for n, k in shapes.values())
        self.gu_bytes = sum(qmm_bytes(*shapes[n], bits, m) for n in ("gate", "up")) - 2 * m * H  # x once
        self.gu_flops = 2 * 2 * m * I * H

    def gate_up(self, i: int) -> None:
        """The step's dominant launch: gate and up projections as one two-problem qmm launch."""
        from dspark_rocm import ops

        x, y = self.x, self.y
        if self.packed:
            P = self.packs[i % len(self.packs)]
            ops.quantized_matmul_packed_multi([x["gu"]], [P["gate"], P["up"]], outs=[y["gate"], y["up"]])
            return
        L = self.layers[i % len(self.layers)]
        ops.quantized_matmul_multi([x["gu"]], [L["gate"][0], L["up"][0]], [L["gate"][1], L["up"][1]],
                                   [L["gate"][2], L["up"][2]], bits=self.bits, outs=[y["gate"], y["up"]])

    def step(self, i: int) -> None:
        from dspark_rocm import ops

        b, y, x = self.bits, self.y, self.x
        if self.packed:
            P = self.packs[i % len(self.packs)]
            ops.quantized_matmul_packed_multi([x["qkv"]], [P[n] for n in "qkv"], outs=[y["q"], y["k"], y["v"]])
            ops.quantized_matmul_packed(x["o"], P["o"], out=y["o"])
            self.gate_up(i)
            ops.quantized_matmul_packed(x["down"], P["down"], out=y["down"])
            return
        L = self.layers[i % len(self.layers)]
        ops.quantized_matmul_multi([x["qkv"]], [L[n][0] for n in "qkv"], [L[n][1] for n in "qkv"],
                                   [L[n][2] for n in "qkv"], bits=b, outs=[y["q"], y["k"], y["v"]])
        ops.quantized_matmul(x["o"], *L["o"], bits=b, out=y["o"])
        self.gate_up(i)
        ops.quantized_matmul(x["down"], *L["down"], bits=b, out=y["down"])


def bench_qmm_single(dev, bits: int, m: int, n: int = 4096, k: int = 4096):
    """One [n, k] qmm, chained over a >= 1 GB pool (graph, median of replays) and as single
    isolated launches (cold from HBM, median of 20)."""
    import torch

    from dspark_rocm import ops
    from dspark_rocm.quant import random_quantized

    g = torch.Generator(device=dev)
    g.manual_seed(bits * 100 + m)
    wbytes = n * k * bits // 8 + 4 * n * (k // 64)
    pool = max(8, (4 * MALL_BYTES) // wbytes + 1)
    mats = [random_quantized(n, k, bits, generator=g, device=dev) for _ in range(pool)]
    x = torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)

    def chain():
        for i in range(pool):
            ops.quantized_matmul(x, *mats[i], bits=bits, out=y)

    ms_chain, _ = time_graph(chain)
    us_chain = ms_chain * 1e3 / pool
    singles = []
    for i in range(20):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        ops.quantized_matmul(x, *mats[i % pool], bits=bits, out=y)
        e1.record()
        torch.cuda.synchronize()
        singles.append(e0.elapsed_time(e1) * 1e3)
    us_single = statistics.median(singles)
    # the same matrices in the packed qmm form (what a loaded model's projections use): same bits
    packs = [ops.qmm_pack(*mt, bits=bits) for mt in mats]

    def chain_packed():
        for i in range(pool):
            ops.quantized_matmul_packed(x, packs[i], out=y)

    ms_packed, _ = time_graph(chain_packed)
    us_packed = ms_packed * 1e3 / pool
    del packs
    by = qmm_bytes(n, k, bits, m)
    return {"shape": f"{n}x{k}", "bits": bits, "M": m, "bytes": by, "us_chained": round(us_chain, 3),
            "GBs_chained": round(by / us_chain / 1e3, 1), "us_single": round(us_single, 3),
            "GBs_single": round(by / us_single / 1e3, 1), "us_chained_packed": round(us_packed, 3),
            "GBs_chained_packed": round(by / us_packed / 1e3, 1)}


def bench_attention(dev, L: int, hq=32, hk=8, d=128, mq=16, dtype="bf16", kv_bits: int = 16):
    """Verify attention: ``mq`` rows over L cached keys (+ the mq new rows), causal, rotated KV
    sets >= 1 GB; bf16 / fp16 K/V or an 8- / 4-bit quantized cache."""
    import torch

    from dspark_rocm import ops
    from dspark_rocm.quant import quantize_rows

    tdt = {"bf16": torch.bfloat16, "f16": torch.float16}[dtype]
    g = torch.Generator(device=dev)
    g.manual_seed(L + d + kv_bits)
    Lt = L + mq
    per = attn_bytes(hq, hk, d, mq, Lt, kv_bits)
    pool = max(2, (4 * MALL_BYTES) // per + 1)
    cap = Lt + 64
    kv = []
    for _ in range(pool):
        if kv_bits == 16:
            kb = torch.randn((1, hk, cap, d), generator=g, device=dev).to(tdt)
            vb = torch.randn((1, hk, cap, d), generator=g, device=dev).to(tdt)
            kv.append((kb[:, :, :Lt], vb[:, :, :Lt]))
        else:
            trips = []
            for _ in range(2):
                t = quantize_rows(torch.randn((1, hk, cap, d), generator=g, device=dev), kv_bits, 64, tdt)
                trips.append(tuple(a[:, :, :Lt] for a in t))
            kv.append(tuple(trips))
    q = torch.randn((1, hq, mq, d), generator=g, device=dev).to(tdt)
    out = torch.empty_like(q)
    scale = d ** -0.5

    def chain():
        for kk, vv in kv:
            if kv_bits == 16:
                ops.verify_attention(q, kk, vv, scale=scale, causal=True, out=out)
            else:
                ops.verify_attention_quantized(q, kk, vv, scale=scale, causal=True, bits=kv_bits, out=out)

    ms, _ = time_graph(chain)
    us = ms * 1e3 / pool
    by = attn_bytes(hq, hk, d, mq, Lt, kv_bits)
    res = {"L": L, "rows": mq, "heads": f"{hq}/{hk}/{d}", "dtype": dtype, "kv_bits": kv_bits, "bytes": by,
           "blocks": ops.verify_attention_blocks(1, hq, hk, mq, d, Lt), "us_chained": round(us, 3),
           "GBs_chained": round(by / us / 1e3, 1), "flops": attn_flops(hq, mq, d, Lt)}
    del kv
    torch.cuda.empty_cache()
    return res


def bench_moe(dev, m=16, E=128, k=8, H=2048, I=768, bits=4):
    """The routed-expert block (route + gate/up + down + combine) over rotated expert pools."""
    import torch

    from dspark_rocm import ops
    from dspark_rocm.quant import random_quantized

    g = torch.Generator(device=dev)
    g.manual_seed(4)

    def stack(n, kk):
        ws = [random_quantized(n, kk, bits, generator=g, device=dev) for _ in range(E)]
        return tuple(torch.stack([w[i] for w in ws]) for i in range(3))

    per_layer = 3 * E * I * H * bits // 8
    pool = max(2, (4 * MALL_BYTES) // per_layer + 1)
    layers = [(stack(I, H), stack(I, H), stack(H, I)) for _ in range(pool)]
    # the packed expert form (what SwitchGLU.pack() holds for a loaded model), bit-identical
    packed = [tuple((ops.moe_pack(w, bits=bits), s, b) for (w, s, b) in L) for L in layers]
    x = torch.randn((m, H), generator=g, device=dev).to(torch.bfloat16)
    logits = torch.randn((m, E), generator=g, device=dev).to(torch.bfloat16)
    _, inds, _ = ops.moe_switch_glu(x, logits, *packed[0], k=k, bits=bits)
    distinct = int(torch.unique(inds).numel())

    def chain(ls):
        def f():
            for gu in ls:
                ops.moe_switch_glu(x, logits, *gu, k=k, bits=bits)
        return f

    ms, _ = time_graph(chain(packed))
    us = ms * 1e3 / pool
    ms_rm, _ = time_graph(chain(layers))
    us_rm = ms_rm * 1e3 / pool
    per_expert = 3 * (I * H * bits // 8 + 4 * I * (H // 64))
    by = distinct * per_expert + 2 * m * H * 2 + 2 * m * E
    del layers, packed
    torch.cuda.empty_cache()
    return {"experts": E, "top_k": k, "distinct_experts": distinct, "bytes": by, "us_chained": round(us, 3),
            "GBs_chained": round(by / us / 1e3, 1), "flops": 3 * 2 * m * k * I * H, "weights": "packed experts",
            "us_chained_row_major": round(us_rm, 3)}


VERIFY_ARGS = dict(hidden_size=5120, num_hidden_layers=64, intermediate_size=25600, num_attention_heads=64,
                   num_key_value_heads=8, head_dim=128, vocab_size=151936, rope_theta=1e6, bits=8, lm_head_bits=8)


def verify_step_bytes(context: int, rows: int) -> tuple[int, int]:
    from dspark_rocm import roofline

    H, I, hq, hk, d = 5120, 25600, 64, 8, 128
    per_layer = sum(roofline.qmm_param_bytes(n, k, 8) for n, k in
                    ((hq * d, H), (hk * d, H), (hk * d, H), (H, hq * d), (I, H), (I, H), (H, I)))
    weights = 64 * per_layer + roofline.qmm_param_bytes(VERIFY_ARGS["vocab_size"], H, 8)
    kv = 64 * roofline.attention_bytes(hq, hk, d, rows, context + rows)
    return weights, kv


def bench_prefill_wide(dev, n: int = 12288, k: int = 4096, bits: int = 8, widths=(256, 512, 1024, 2048)) -> dict:
    """The prefill wide path on the 8B-shaped gate projection ([12288, 4096] 8-bit): per width M,
    the stock path (torch dequantize + fp32 GEMM), the wide path (one dequantize launch + the same
    fp32 GEMM, bit-identical) and its bf16 variant (dequantize to bf16 + bf16 GEMM), each called
    eagerly back to back over 4 distinct matrices (as a prefill runs them); and the dequantize
    kernel alone, graph-replayed (bytes: the packed weight, scales and biases read, the fp32
    weight written)."""
    import torch

    from dspark_rocm import ops, wide_gemm
    from dspark_rocm.nn import QuantizedLinear

    g = torch.Generator(device=dev)
    g.manual_seed(7)
    mats = [QuantizedLinear.random(n, k, bits=bits, device=dev, generator=g) for _ in range(4)]
    out = {"shape": f"{n}x{k}", "bits": bits, "widths": []}
    for M in widths:
        x = torch.randn((M, k), generator=g, device=dev).to(torch.bfloat16)
        row = {"M": M}
        for name, fn in (("stock_us", lambda m: wide_gemm._orig_call(m, x)),
                         ("wide_us", lambda m: wide_gemm.wide_rows(m, x, exact=True)),
                         ("wide_bf16_us", lambda m: wide_gemm.wide_rows(m, x, exact=False))):
            ms = time_eager(lambda: [fn(m) for m in mats]) / len(mats)
            row[name] = round(ms * 1e3, 1)
        row["speedup"] = round(row["stock_us"] / row["wide_us"], 2)
        row["speedup_bf16"] = round(row["stock_us"] / row["wide_bf16_us"], 2)
        row["bf16_TFLOPs"] = round(2 * M * n * k / (row["wide_bf16_us"] * 1e-6) / 1e12, 1)
        out["widths"].append(row)
    nbytes = n * k * bits // 8 + 4 * n * (k // 64) + 4 * n * k
    outs = [torch.empty((n, k), dtype=torch.float32, device=dev) for _ in mats]
    ms, _ = time_graph(lambda: [ops.dequantize(m.weight, m.scales, m.biases, bits=bits, out=o)
                                for m, o in zip(mats, outs)])
    ms /= len(mats)
    out["dequantize_us"] = round(ms * 1e3, 2)
    out["dequantize_bytes"] = nbytes
    out["dequantize_GBs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
    return out


DSPARK_TAP = (5, 17, 29, 41, 46)


def bench_verify_forward(dev, context: int = 16384, rows: int = 16, widths=(1, 2, 4, 8, 16), shallow: int = 512):
    """Speculative verify steps of a random-init dense 8-bit 64-layer target (hidden 5120, heads
    64/8 x 128, intermediate 25600, vocab 151936, RoPE 1e6) over a synthetic bf16 KV cache:
    the forward, lm_head, device argmax and greedy accept, each captured as one hipGraph (the KV
    write lands at the same positions every replay; rollback is cache metadata on the host).

    The headline point is ``rows`` rows at ``context``. Its drafts are the step's own target
    tokens, found by feeding them back until they stop changing (row i's token depends only on
    rows 0..i, so each pass fixes at least one more), so all ``rows - 1`` drafts must be
    accepted: the reported count checks the step end to end. (Drafts from single-row steps do
    not serve here: verify widths split the keys differently, and over 64 random layers those
    last-bit differences reach ~0.6 in the logits, while a random 151936-entry vocabulary has
    top-2 margins of ~0.1.) The curve times every width at ``context`` and
    at ``shallow`` (the reference's verify curve and depth slope, calibrate.py:121-140,
    :247-277, with the KV inflated to depth as calibrate.py:214-244 does)."""
    import torch

    from dspark_rocm.model import DenseModel, ModelArgs, Target

    args = ModelArgs(**VERIFY_ARGS)
    t0 = time.perf_counter()
    model = DenseModel.random(args, device=dev, seed=5)
    tgt = Target(model, max_rows=rows)
    cache = tgt.make_cache(context + rows)
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    for c in cache:                       # synthetic KV at depth
        c.keys[:, :, :context].normal_(generator=g)
        c.values[:, :, :context].normal_(generator=g)
        c.offset = context
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    e = tgt.engine
    # the drafter's hidden-state tap, as a DSpark round verifies with it (generate.py:1547): the
    # reference's default target_layer_ids (config.py:233); the tapped residual streams are
    # written where the step forms them, no extra launch
    e.set_tap(DSPARK_TAP)
    # self-consistent drafts: the step's own target tokens fed back until they stop changing
    seq = torch.randint(0, args.vocab_size, (rows,), generator=g, device=dev).tolist()
    passes = 0
    for passes in range(1, rows + 1):
        e.ids[:rows].copy_(torch.tensor(seq, device=dev))
        e.step(rows, cache, context, accept=False)
        tt = torch.argmax(e.logits[:rows].float(), dim=-1).tolist()
        nxt = seq[:1] + tt[:rows - 1]
        if nxt == seq:
            break
        seq = nxt
    e.ids[:rows].copy_(torch.tensor(seq, device=dev))
    e.draft[:rows - 1].copy_(torch.tensor(seq[1:], dtype=torch.int32, device=dev))

    def step():
        e.step(rows, cache, context, accept=True)

    ms, _ = time_graph(step)
    accepted = int(e.n_acc.item())
    weights, kv = verify_step_bytes(context, rows)
    by = weights + kv
    curve = []
    for depth in (shallow, context):
        for w in widths:
            e.ids[:w].copy_(torch.tensor(seq[:w], device=dev))
            if w > 1:
                e.draft[:w - 1].copy_(torch.tensor(seq[1:w], dtype=torch.int32, device=dev))
            ms_w, _ = time_graph(lambda w=w, depth=depth: e.step(w, cache, depth, accept=True))
            wb, kb = verify_step_bytes(depth, w)
            curve.append({"depth": depth, "width": w, "ms": round(ms_w, 4),
                          "GBs": round((wb + kb) / (ms_w * 1e-3) / 1e9, 1)})
    slope = {str(w): round((next(c["ms"] for c in curve if c["depth"] == context and c["width"] == w) -
                            next(c["ms"] for c in curve if c["depth"] == shallow and c["width"] == w))
                           / (context - shallow) * 1e3, 5) for w in widths}
    res = {"layers": 64, "hidden": 5120, "context": context, "rows": rows, "weight_bytes": weights, "kv_bytes": kv,
           "bytes": by, "ms_graph": round(ms, 4), "GBs": round(by / (ms * 1e-3) / 1e9, 1),
           "frac_of_peak": round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "accepted": accepted,
           "accepted_expected": rows - 1, "draft_passes": passes, "launches": 64 * 9 + 4, "tap": list(e.tap),
           "build_s": round(build_s, 1),
           "curve": curve, "depth_slope_us_per_token": slope}
    del model, tgt, cache, e
    torch.cuda.empty_cache()
    return res


# ------------------------------------------------------------------ CPU baseline

def _cpu_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(bits: int, m: int, budget_s: float = 8.0) -> dict:
    """The C restatement (oracle/dspark_oracle.c, OpenMP on every core of this process's
    affinity) on the layer set of the same shapes, repeated until about ``budget_s`` seconds
    of CPU work have been timed; beside it torch-CPU fp32 (dequantize-and-matmul) on the same
    set, and the C restatement of verify attention (one 32/8/128 verify at 32k keys) and of
    the MoE block's expert work."""
    import numpy as np
    import torch

    from oracle import c_oracle, quant_ref

    cores = len(os.sched_getaffinity(0))
    c_oracle.set_threads(cores)
    torch.set_num_threads(cores)
    r = np.random.Generator(np.random.PCG64(1))
    shapes = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (12288, 4096), (12288, 4096), (4096, 12288)]
    mats = []
    for n, k in shapes:
        w, s, b = quant_ref.random_packed(r, n, k, bits)
        x = quant_ref.bf16_bits(r.standard_normal((m, k)).astype(np.float32))
        mats.append((n, k, x, w, quant_ref.bf16_bits(s), quant_ref.bf16_bits(b)))
        c_oracle.qmm(x, w[:8], mats[-1][4][:8], mats[-1][5][:8], bits)          # warm
    tot_bytes, tot_s, passes = 0, 0.0, 0
    while passes == 0 or tot_s < budget_s:
        for n, k, x, w, sb, bb in mats:
            t0 = time.perf_counter()
            c_oracle.qmm(x, w, sb, bb, bits)
            tot_s += time.perf_counter() - t0
            tot_bytes += qmm_bytes(n, k, bits, m)
        passes += 1
    gbs = tot_bytes / tot_s / 1e9
    cpu = _cpu_name()
    out = {"value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
           "sample": f"the 8B-shaped {bits}-bit layer set (7 projections, M={m}) {passes} times, "
                     f"oracle/dspark_oracle.c orc_qmm with {cores} OpenMP threads on {cpu}; {tot_s:.2f} s",
           "ms_per_step": round(tot_s * 1e3 / passes, 2), "legs": {}}
    # torch-CPU fp32: dequantize each matrix once (not timed), then the fp32 matmuls
    dq = [(torch.from_numpy(quant_ref.dequantize(w, quant_ref.bf16_from_bits(sb), quant_ref.bf16_from_bits(bb),
                                                 bits).astype(np.float32)),
           torch.from_numpy(quant_ref.bf16_from_bits(x))) for n, k, x, w, sb, bb in mats]
    t_torch, tp = 0.0, 0
    while tp == 0 or t_torch < budget_s / 2:
        t0 = time.perf_counter()
        for wf, xf in dq:
            xf @ wf.T
        t_torch += time.perf_counter() - t0
        tp += 1
    fp32_bytes = sum(n * k * 4 + 4 * m * (n + k) for n, k, *_ in mats)
    out["legs"]["layer_set_torch_fp32"] = {"ms_per_step": round(t_torch * 1e3 / tp, 2), "threads": cores,
                                           "GBs_of_fp32_weights": round(fp32_bytes * tp / t_torch / 1e9, 2),
                                           "GBs_algorithmic": round(sum(qmm_bytes(n, k, bits, m) for n, k, *_ in mats)
                                                                    * tp / t_torch / 1e9, 3)}
    del dq
    # C attention: 32/8/128, 16 rows over 32768 + 16 keys
    Lt = 32768 + 16
    q = quant_ref.bf16_bits(r.standard_normal((1, 32, 16, 128)).astype(np.float32))
    kk = quant_ref.bf16_bits(r.standard_normal((1, 8, Lt, 128)).astype(np.float32))
    vv = quant_ref.bf16_bits(r.standard_normal((1, 8, Lt, 128)).astype(np.float32))
    t0 = time.perf_counter()
    c_oracle.attention(q, kk, vv, 128 ** -0.5, True)
    ta = time.perf_counter() - t0
    out["legs"]["verify_attention_32k_c"] = {"ms": round(ta * 1e3, 2), "threads": cores,
                                             "GBs": round(attn_bytes(32, 8, 128, 16, Lt) / ta / 1e9, 3)}
    del kk, vv
    # C MoE expert work: 16 tokens x top-8 over 128 experts (2048 / 768, 4-bit): the routed
    # (token, expert) pairs' gate, up and down qmms through orc_qmm, grouped per expert
    lg = quant_ref.bf16_bits(r.standard_normal((16, 128)).astype(np.float32))
    inds, _ = c_oracle.route(lg, 8)
    experts = sorted(set(int(e) for e in inds.reshape(-1)))
    xm = quant_ref.bf16_bits(r.standard_normal((16, 2048)).astype(np.float32))
    eg = {e: (quant_ref.random_packed(r, 768, 2048, 4), quant_ref.random_packed(r, 768, 2048, 4),
              quant_ref.random_packed(r, 2048, 768, 4)) for e in experts}
    t0 = time.perf_counter()
    for e in experts:
        rows = [t for t in range(16) if e in inds[t]]
        xs = xm[rows]
        (gw, gs, gb), (uw, us, ub), (dw, ds, db) = eg[e]
        c_oracle.qmm(xs, gw, quant_ref.bf16_bits(gs), quant_ref.bf16_bits(gb), 4)
        c_oracle.qmm(xs, uw, quant_ref.bf16_bits(us), quant_ref.bf16_bits(ub), 4)
        hx = quant_ref.bf16_bits(r.standard_normal((len(rows), 768)).astype(np.float32))
        c_oracle.qmm(hx, dw, quant_ref.bf16_bits(ds), quant_ref.bf16_bits(db), 4)
    tm = time.perf_counter() - t0
    per_expert = 3 * (768 * 2048 * 4 // 8 + 4 * 768 * (2048 // 64))
    out["legs"]["moe_experts_c"] = {"ms": round(tm * 1e3, 2), "threads": cores, "distinct_experts": len(experts),
                                    "GBs": round(len(experts) * per_expert / tm / 1e9, 3)}
    return out


def load_traffic():
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(p) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


# ------------------------------------------------------------------ single workloads (profiling)

def _only_gate_up(dev):
    import torch

    ls = LayerSet(dev, 8, 16, 8)
    ms, _ = time_graph(lambda: [ls.gate_up(i) for i in range(50)])
    torch.cuda.synchronize()
    return leg("gate+up qmm launch", ls.gu_bytes, ms * 1e3 / 50, None, ls.gu_flops)


def _only_layer_set(dev):
    ls = LayerSet(dev, 8, 16, 8)
    ms, _ = time_graph(lambda: [ls.step(i) for i in range(50)])
    return leg("8-bit layer set step", ls.bytes_per_step, ms * 1e3 / 50, None, ls.flops_per_step)


ONLY = {
    "gate_up": _only_gate_up,
    "layer_set": _only_layer_set,
    "qmm4096_8bit": lambda dev: bench_qmm_single(dev, 8, 16),
    "qmm4096_4bit": lambda dev: bench_qmm_single(dev, 4, 16),
    "attn32k": lambda dev: bench_attention(dev, 32768),
    "attn16k_64x8": lambda dev: bench_attention(dev, 16384, hq=64, hk=8),
    "attn32k_d256": lambda dev: bench_attention(dev, 32768, hq=24, hk=4, d=256),
    "attn32k_kv8": lambda dev: bench_attention(dev, 32768, kv_bits=8),
    "attn32k_kv4": lambda dev: bench_attention(dev, 32768, kv_bits=4),
    "moe": lambda dev: bench_moe(dev),
    "verify_step": lambda dev: bench_verify_forward(dev, widths=(16,)),
    "prefill_wide": lambda dev: bench_prefill_wide(dev),
}


# ------------------------------------------------------------------ main

def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=8, help="distinct layers in the rotated pool")
    ap.add_argument("--quick", action="store_true", help="only the headline layer set and its gate/up launch")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-verify-step", action="store_true", help="skip the 64-layer verify-step legs")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 256 MiB device copy (for scaling rocprof byte counters)")
    ap.add_argument("--only", choices=sorted(ONLY), default=None,
                    help="run one workload alone (for profilers) and print its leg as JSON")
    a = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU; multi-GPU sharding is design-only "
                                   f"(requested --gpus {a.gpus}, WORLD_SIZE {world})"}), flush=True)
        sys.exit(2)

    import torch

    from dspark_rocm import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    M, bits = 16, 8

    if a.copy_calibration:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log("copy calibration: 268435456 bytes read + written by one copy kernel")
        del src, dst

    bw = None
    if a.only:
        res = ONLY[a.only](dev)
        print(json.dumps({"only": a.only, "result": res}), flush=True)
        return
    bw = measure_bandwidth(dev)
    mbw = bw["measured_GBs"]
    log(f"device {torch.cuda.get_device_name(dev)}; measured bandwidth {bw}")
    log(f"building the layer-set pool of {a.layers} layers")
    ls = LayerSet(dev, bits, M, a.layers)
    log(f"layer-set pool: {ls.weight_bytes * a.layers / 1e9:.2f} GB weights; step bytes {ls.bytes_per_step}")

    for i in range(a.warmup):
        ls.step(i)
    torch.cuda.synchronize()

    # timed region: K steps as one graph, median over REPEATS event-bracketed replays
    K = a.steps
    ms_total, _ = time_graph(lambda: [ls.step(i) for i in range(K)])
    ms_step = ms_total / K
    gbs = ls.bytes_per_step / (ms_step * 1e-3) / 1e9
    log(f"layer-set graph: {ms_step * 1e3:.2f} us/step, {gbs:.1f} GB/s (median of {REPEATS} replays)")

    log(f"gate/up kernel: {gate_up_kernel_name(ls)}")
    # dominant kernel: K gate/up launches back to back (rotating layers) as one graph, HIP events
    # on the launch stream around each replay; average launch = replay / K
    gu_total, _ = time_graph(lambda: [ls.gate_up(i) for i in range(K)])
    gu_us = gu_total * 1e3 / K
    traffic = load_traffic()
    legs = {"qmm_gate_up": leg("gate+up qmm launch, 2 x [12288, 4096] 8-bit packed, M=16", ls.gu_bytes, gu_us, mbw,
                               ls.gu_flops)}
    gu = legs["qmm_gate_up"]
    log(f"gate/up launch: {gu_us:.2f} us, {gu['GBs']} GB/s")
    roofline = {"kernel": gate_up_kernel_name(ls), "bound": "hbm", "achieved": gu["GBs"], "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": gu["frac"], "traffic": (traffic or {}).get("qmm_gate_up_bytes"),
                "bytes_per_launch": ls.gu_bytes, "avg_launch_us": gu["us"], "frac_of_measured": gu["frac_of_measured"],
                "mfma_util": gu["mfma_util"]}
    legs["layer_set_step"] = leg("8B-shaped 8-bit layer set step (4 launches)", ls.bytes_per_step, ms_step * 1e3,
                                 mbw, ls.flops_per_step)
    extra = {}
    if not a.quick:
        ls.packed = False
        ref_ms, _ = time_graph(lambda: [ls.step(i) for i in range(K)])
        ref_gu, _ = time_graph(lambda: [ls.gate_up(i) for i in range(K)])
        ls.packed = True
        extra["layer_set_reference_layout"] = {"step_us": round(ref_ms * 1e3 / K, 3),
                                               "GBs": round(ls.bytes_per_step / (ref_ms / K * 1e-3) / 1e9, 1),
                                               "gate_up_us": round(ref_gu * 1e3 / K, 3)}
        log(f"layer set, reference layout: {ref_ms * 1e3 / K:.2f} us/step, gate/up {ref_gu * 1e3 / K:.2f} us")
        ls4 = LayerSet(dev, 4, M, a.layers, seed=2)
        ms4, _ = time_graph(lambda: [ls4.step(i) for i in range(K)])
        gu4, _ = time_graph(lambda: [ls4.gate_up(i) for i in range(K)])
        legs["layer_set_step_4bit"] = leg("the same layer set in 4-bit", ls4.bytes_per_step, ms4 * 1e3 / K, mbw,
                                          ls4.flops_per_step, gate_up_us=round(gu4 * 1e3 / K, 3))
        log(f"layer set 4-bit: {ms4 * 1e3 / K:.2f} us/step, gate/up {gu4 * 1e3 / K:.2f} us")
        del ls4
        del ls
        torch.cuda.empty_cache()
        extra["qmm_4096x4096"] = []
        for b in (4, 8):
            for m in (1, 2, 4, 8, 16):
                r = bench_qmm_single(dev, b, m)
                extra["qmm_4096x4096"].append(r)
                log(f"qmm 4096x4096 {b}-bit M={m}: {r['us_chained']} us chained ({r['GBs_chained']} GB/s), "
                    f"{r['us_single']} us single, packed form {r['us_chained_packed']} us chained")
                if m == 16:
                    legs[f"qmm_4096x4096_{b}bit"] = leg(f"one 4096x4096 {b}-bit qmm, M=16, chained", r["bytes"],
                                                        r["us_chained"], mbw, 2 * 16 * 4096 * 4096,
                                                        us_single=r["us_single"],
                                                        us_chained_packed=r["us_chained_packed"])
        extra["verify_attention"] = []
        for L in (512, 4096, 16384, 32768):
            r = bench_attention(dev, L)
            extra["verify_attention"].append(r)
            log(f"verify attention L={L}: {r['us_chained']} us ({r['GBs_chained']} GB/s), NB={r['blocks']}")
        r = extra["verify_attention"][-1]
        legs["verify_attention_32k"] = leg("verify attention 32/8/128 bf16, 16 rows at 32768 (+16) keys", r["bytes"],
                                           r["us_chained"], mbw, r["flops"])
        for name, kw in (("verify_attention_32k_f16", dict(dtype="f16")),
                         ("verify_attention_32k_d256", dict(hq=24, hk=4, d=256)),
                         ("verify_attention_32k_kv8", dict(kv_bits=8)),
                         ("verify_attention_32k_kv4", dict(kv_bits=4))):
            r = bench_attention(dev, 32768, **kw)
            extra.setdefault("verify_attention_variants", []).append(r)
            kv_label = "" if r["kv_bits"] == 16 else f", {r['kv_bits']}-bit KV"
            legs[name] = leg(f"verify attention {r['heads']} {r['dtype']}{kv_label}, 16 rows at 32k",
                             r["bytes"], r["us_chained"], mbw, r["flops"])
            log(f"{name}: {r['us_chained']} us ({r['GBs_chained']} GB/s)")
        r = bench_moe(dev)
        extra["moe_block"] = r
        legs["moe_block"] = leg("MoE block, 128 experts top-8, 2048/768 4-bit, 16 tokens", r["bytes"], r["us_chained"],
                                mbw, r["flops"], distinct_experts=r["distinct_experts"])
        log(f"MoE block: {r['us_chained']} us ({r['GBs_chained']} GB/s, packed experts; row-major {r['us_chained_row_major']} us), {r['distinct_experts']} experts")
        r = bench_prefill_wide(dev)
        extra["prefill_wide"] = r
        legs["prefill_dequantize"] = leg("prefill wide path: dequantize [12288, 4096] 8-bit to fp32 once",
                                         r["dequantize_bytes"], r["dequantize_us"], mbw)
        log(f"prefill wide path: {[(w['M'], w['stock_us'], w['wide_us'], w['wide_bf16_us']) for w in r['widths']]}, "
            f"dequantize {r['dequantize_us']} us ({r['dequantize_GBs']} GB/s)")
        if not a.no_verify_step:
            r = bench_verify_forward(dev)
            extra["verify_step"] = r
            legs["verify_step_16k"] = leg("64-layer 8-bit verify step (hidden 5120, 64/8x128, I 25600, vocab 151936),"
                                          " 16 rows at 16k", r["bytes"], r["ms_graph"] * 1e3, mbw, None,
                                          ms=r["ms_graph"], accepted=r["accepted"],
                                          accepted_expected=r["accepted_expected"])
            log(f"verify step (64 layers, 16 rows @ 16k): {r['ms_graph']} ms ({r['GBs']} GB/s, "
                f"{r['frac_of_peak']:.1%} of peak), accepted {r['accepted']}/{r['accepted_expected']}; "
                f"curve {[(c['depth'], c['width'], c['ms']) for c in r['curve']]}")

    cpu = None
    if not a.quick and not a.no_cpu:
        cpu = cpu_baseline(bits, M)
        log(f"CPU baseline: {cpu['value']} GB/s on {cpu['cores']} threads; legs {cpu['legs']}")

    line = {"metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": K, "warmup": a.warmup,
            "ms_per_step": round(ms_step, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "8B-shaped 8-bit layer projection set (q,k,v,o,gate,up,down; hidden 4096, "
                                   "heads 32/8x128, intermediate 12288, group 64) at M=16 verify rows, "
                                   f"rotated over {a.layers} distinct layers, weights in the packed qmm form",
                       "M": M, "bits": bits, "bytes_per_step": legs["layer_set_step"]["bytes"],
                       "launches_per_step": 4, "timing": f"hipGraph of {K} steps, median of {REPEATS} replays"},
            "roofline": roofline, "bandwidth": bw, "legs": legs, "cpu_baseline": cpu, "extra": extra}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
