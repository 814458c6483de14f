"""Speculative-verify hot path on one MI355X: weight/KV-stream GB/s and verify-step µs.

Headline (``value``): the 8B-shaped 8-bit decoder-layer projection set (q, k, v, o, gate, up,
down; hidden 4096, 32/8 heads x 128, intermediate 12288, group 64) at M = 16 verify rows. One
step = that set for one layer, launched the way a verify forward issues it (q/k/v in one
launch, o, gate/up in one launch, down), rotating over a pool of distinct layers (>= 1.5 GB,
far past the 256 MB Infinity Cache) so every byte comes from HBM. The K timed steps are one
HIP-graph replay bracketed by events. ``value`` = algorithmic bytes / measured time.

Also reported under ``extra``: the same layer set in 4-bit and read from the reference layout,
the single 4096x4096 qmm (4- and 8-bit, M = 1..16), multi-row verify attention at 512..32k keys
(32/8/128, 16 rows), the 128-expert top-8 MoE block and the 64-layer verify step at 16k context
— each as µs per call and GB/s, chained over rotated pools.

``roofline`` is for the dominant kernel (the gate/up qmm launch): its algorithmic bytes over its
average duration, taken from HIP events around that launch in an event-bracketed replay of the
same steps on the same stream. ``cpu_baseline`` is the C/OpenMP restatement of the qmm
(oracle/dspark_oracle.c) timed on this host on a bounded sample (one full layer set).

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--quick]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mlx-dspark_amd"))

METRIC = "verify-step µs + weight/KV-stream GB/s (% of HBM peak), M=16 qmm & attention"
HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ------------------------------------------------------------------ byte accounting

def qmm_bytes(n: int, k: int, bits: int, m: int) -> int:
    """Algorithmic bytes of one affine qmm: packed weights + bf16 scales/biases + x + y."""
    return n * k * bits // 8 + 2 * 2 * n * (k // 64) + 2 * m * k + 2 * m * n


def attn_bytes(hq: int, hk: int, d: int, mq: int, L: int) -> int:
    """K/V stream (L keys incl. the verify rows) + q + out."""
    return 2 * 2 * hk * L * d + 2 * 2 * hq * mq * d


# ------------------------------------------------------------------ timing helpers

def time_graph(fn, reps: int, warm: int = 3):
    """Capture ``fn`` (which enqueues work on the current stream) into a HIP graph, replay it
    ``reps`` times between events; returns (ms per replay, graph)."""
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
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps, g


def time_eager(fn, reps: int, warm: int = 3) -> float:
    import torch

    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


# ------------------------------------------------------------------ workloads

class LayerSet:
    """The projection set of an 8B-shaped layer: q/k/v/o/gate/up/down, 8- or 4-bit g64, M rows; a
    pool of layers.
    Each matrix is held in the reference layout and in the packed qmm form (``ops.qmm_pack``);
    ``packed`` selects which one the launches read (the products are bit-identical)."""

    H, HQ, HK, D, I = 4096, 32, 8, 128, 12288

    def __init__(self, dev, bits: int, m: int, layers: int, seed: int = 1):
        import torch

        from dspark_rocm.quant import random_quantized

        self.bits, self.m = bits, m
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        H, I, D = self.H, self.I, self.D
        shapes = {"q": (self.HQ * D, H), "k": (self.HK * D, H), "v": (self.HK * D, H), "o": (H, self.HQ * D),
                  "gate": (I, H), "up": (I, H), "down": (H, I)}
        self.shapes = shapes
        self.layers = []
        for _ in range(layers):
            self.layers.append({name: random_quantized(n, k, bits, generator=g, device=dev)
                                for name, (n, k) in shapes.items()})
        from dspark_rocm import ops

        self.packs = [{name: ops.qmm_pack(*L[name], bits=bits) for name in shapes} for L in self.layers]
        self.packed = True
        self.x = {k: (torch.randn((m, kk), generator=g, device=dev) ).to(torch.bfloat16)
                  for k, kk in (("qkv", H), ("o", self.HQ * D), ("gu", H), ("down", I))}
        self.y = {name: torch.empty((m, n), dtype=torch.bfloat16, device=dev) for name, (n, _) in shapes.items()}
        self.bytes_per_step = sum(qmm_bytes(n, k, bits, m) for n, k in shapes.values())
        self.weight_bytes = sum(n * k * bits // 8 + 4 * n * (k // 64) for n, k in shapes.values())
        self.gu_bytes = sum(qmm_bytes(*shapes[n], bits, m) for n in ("gate", "up")) - 2 * m * H  # x once

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


def bench_qmm_single(dev, bits: int, m: int, n: int = 4096, k: int = 4096, reps: int = 200):
    """One [n, k] qmm, single launch (cold from HBM) and chained over a >= 1 GB pool."""
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
    ctr = [0]

    def one():
        w, s, b = mats[ctr[0] % pool]
        ctr[0] += 1
        ops.quantized_matmul(x, w, s, b, bits=bits, out=y)

    def chain():
        for i in range(pool):
            ops.quantized_matmul(x, *mats[i], bits=bits, out=y)

    ms_chain, _ = time_graph(chain, max(1, reps // pool))
    us_chain = ms_chain * 1e3 / pool
    # single isolated launches (each after a full sync), rotating so the weights are not cached
    singles = []
    for _ in range(20):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        one()
        e1.record()
        torch.cuda.synchronize()
        singles.append(e0.elapsed_time(e1) * 1e3)
    singles.sort()
    us_single = singles[len(singles) // 2]
    by = qmm_bytes(n, k, bits, m)
    return {"shape": f"{n}x{k}", "bits": bits, "M": m, "bytes": by, "us_chained": round(us_chain, 3),
            "GBs_chained": round(by / us_chain / 1e3, 1), "us_single": round(us_single, 3),
            "GBs_single": round(by / us_single / 1e3, 1)}


def bench_attention(dev, L: int, hq=32, hk=8, d=128, mq=16, reps: int = 50):
    """Verify attention: 16 rows over L cached keys (+ the 16 new rows), rotated KV sets >= 1 GB."""
    import torch

    from dspark_rocm import ops

    g = torch.Generator(device=dev)
    g.manual_seed(L)
    Lt = L + mq
    per = 2 * 2 * hk * Lt * d
    pool = max(2, (4 * MALL_BYTES) // per + 1)
    cap = Lt + 64
    kv = []
    for _ in range(pool):
        kb = torch.randn((1, hk, cap, d), generator=g, device=dev).to(torch.bfloat16)
        vb = torch.randn((1, hk, cap, d), generator=g, device=dev).to(torch.bfloat16)
        kv.append((kb[:, :, :Lt], vb[:, :, :Lt]))
    q = torch.randn((1, hq, mq, d), generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    scale = d ** -0.5

    def chain():
        for kk, vv in kv:
            ops.verify_attention(q, kk, vv, scale=scale, causal=True, out=out)

    ms, _ = time_graph(chain, max(1, reps // pool))
    us = ms * 1e3 / pool
    by = attn_bytes(hq, hk, d, mq, Lt)
    return {"L": L, "rows": mq, "heads": f"{hq}/{hk}/{d}", "bytes": by, "blocks": ops.verify_attention_blocks(1, hq, hk, mq, d, Lt),
            "us_chained": round(us, 3), "GBs_chained": round(by / us / 1e3, 1)}


def bench_moe(dev, m=16, E=128, k=8, H=2048, I=768, bits=4, reps: int = 30):
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
    x = torch.randn((m, H), generator=g, device=dev).to(torch.bfloat16)
    logits = torch.randn((m, E), generator=g, device=dev).to(torch.bfloat16)
    _, inds, _ = ops.moe_switch_glu(x, logits, *layers[0], k=k, bits=bits)
    distinct = int(torch.unique(inds).numel())

    def chain():
        for gu in layers:
            ops.moe_switch_glu(x, logits, *gu, k=k, bits=bits)

    ms, _ = time_graph(chain, max(1, reps // pool))
    us = ms * 1e3 / pool
    per_expert = 3 * (I * H * bits // 8 + 4 * I * (H // 64))
    by = distinct * per_expert + 2 * m * H * 2 + 2 * m * E
    return {"experts": E, "top_k": k, "distinct_experts": distinct, "bytes": by, "us_chained": round(us, 3),
            "GBs_chained": round(by / us / 1e3, 1)}


def bench_verify_forward(dev, context: int = 16384, rows: int = 16, reps: int = 10):
    """One speculative verify step of a random-init dense 8-bit 64-layer target (hidden
    5120, heads 64/8 x 128, intermediate 25600, vocab 151936, RoPE 1e6) with `rows` verify rows
    over a `context`-row synthetic bf16 KV cache: the forward, lm_head, device argmax and
    greedy accept, captured as one hipGraph (the KV write lands at the same positions each
    replay); rollback is cache metadata on the host."""
    import torch

    from dspark_rocm import roofline
    from dspark_rocm.model import DenseModel, ModelArgs, Target

    args = ModelArgs(hidden_size=5120, num_hidden_layers=64, intermediate_size=25600, num_attention_heads=64,
                     num_key_value_heads=8, head_dim=128, vocab_size=151936, rope_theta=1e6, bits=8, lm_head_bits=8)
    t0 = time.perf_counter()
    model = DenseModel.random(args, device=dev, seed=5)
    tgt = Target(model, max_rows=rows)
    cache = tgt.make_cache(context + rows)
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    for c in cache:                       # synthetic KV at depth (calibrate.py:214-244 does the same)
        c.keys[:, :, :context].normal_(generator=g)
        c.values[:, :, :context].normal_(generator=g)
        c.offset = context
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    e = tgt.engine
    e.ids[:rows].copy_(torch.randint(0, args.vocab_size, (rows,), generator=g, device=dev))
    e.draft[:rows - 1].copy_(e.ids[1:rows].to(torch.int32))

    def step():
        e.step(rows, cache, context, accept=True)

    ms, _ = time_graph(step, reps)
    H, I, hq, hk, d = 5120, 25600, 64, 8, 128
    per_layer = sum(roofline.qmm_param_bytes(n, k, 8) for n, k in
                    ((hq * d, H), (hk * d, H), (hk * d, H), (H, hq * d), (I, H), (I, H), (H, I)))
    weights = 64 * per_layer + roofline.qmm_param_bytes(args.vocab_size, H, 8)
    kv = 64 * roofline.attention_bytes(hq, hk, d, rows, context + rows)
    by = weights + kv
    n = int(e.n_acc.item())
    return {"layers": 64, "hidden": H, "context": context, "rows": rows, "weight_bytes": weights, "kv_bytes": kv,
            "bytes": by, "ms_graph": round(ms, 4), "GBs": round(by / (ms * 1e-3) / 1e9, 1),
            "frac_of_peak": round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "accepted": n,
            "launches": 64 * 10 + 5, "build_s": round(build_s, 1)}


def cpu_baseline(bits: int, m: int, budget_s: float = 10.0) -> dict:
    """The C restatement (oracle/dspark_oracle.c, OpenMP) on the layer set of the same shapes,
    repeated until about ``budget_s`` seconds of CPU work have been timed."""
    import numpy as np

    from oracle import c_oracle, quant_ref

    cores = len(os.sched_getaffinity(0))
    cores = min(cores, 16)
    c_oracle.set_threads(cores)
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
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"the 8B-shaped {bits}-bit layer set (7 projections, M={m}) {passes} times, "
                      f"oracle/dspark_oracle.c orc_qmm with {cores} OpenMP threads on {cpu}; {tot_s:.2f} s",
            "ms_per_step": round(tot_s * 1e3 / passes, 2)}


def load_traffic():
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(p) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=8, help="distinct layers in the rotated pool")
    ap.add_argument("--quick", action="store_true", help="skip the single-qmm, attention and MoE extras and the CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-verify-step", action="store_true", help="skip the full 64-layer verify-forward extra")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 256 MiB device copy (for scaling rocprof byte counters)")
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
    log(f"device {torch.cuda.get_device_name(dev)}; building the layer-set pool of {a.layers} layers")
    ls = LayerSet(dev, bits, M, a.layers)
    log(f"layer-set pool: {ls.weight_bytes * a.layers / 1e9:.2f} GB weights; step bytes {ls.bytes_per_step}")

    if a.copy_calibration:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log("copy calibration: 268435456 bytes read + written by one copy kernel")
        del src, dst

    for i in range(a.warmup):
        ls.step(i)
    torch.cuda.synchronize()

    # timed region: K steps as one graph replay
    K = a.steps
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ls.step(0)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        for i in range(K):
            ls.step(i)
    g.replay()  # warm replay
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    ms_total = e0.elapsed_time(e1)
    ms_step = ms_total / K
    gbs = ls.bytes_per_step / (ms_step * 1e-3) / 1e9
    log(f"layer-set graph: {ms_step * 1e3:.2f} us/step, {gbs:.1f} GB/s")

    # eager, for reference (host-issue bound at these sizes)
    t0 = time.perf_counter()
    eager_ms = time_eager(lambda: [ls.step(i) for i in range(a.layers)], 3) / a.layers
    # dominant kernel: K gate/up launches back to back (rotating layers) as one graph, HIP events
    # on the launch stream around the replay; average launch = total / K
    gu_total, _ = time_graph(lambda: [ls.gate_up(i) for i in range(K)], 1)
    gu_avg = gu_total / K
    gu_gbs = ls.gu_bytes / (gu_avg * 1e-3) / 1e9
    log(f"gate/up launch: avg {gu_avg * 1e3:.2f} us, {gu_gbs:.1f} GB/s; eager step {eager_ms * 1e3:.1f} us "
        f"({time.perf_counter() - t0:.1f} s)")

    traffic = load_traffic()
    roofline = {"kernel": "qmm_sk_kernel<8,4,16,true,true,false> gate+up launch, packed form (N=2x12288, K=4096, M=16; "
                          "grid 384x4)", "bound": "hbm",
                "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                "traffic": (traffic or {}).get("qmm_gate_up_bytes"),
                "bytes_per_launch": ls.gu_bytes, "avg_launch_us": round(gu_avg * 1e3, 3)}

    extra = {"layer_set_step_us": round(ms_step * 1e3, 3), "layer_set_eager_step_us": round(eager_ms * 1e3, 3),
             "layer_set_frac_of_peak": round(gbs / HBM_PEAK_GBS, 4)}
    if not a.quick:
        # the same set read from the reference layout (what a drop-in caller passes per call)
        ls.packed = False
        ref_ms, _ = time_graph(lambda: [ls.step(i) for i in range(K)], 1)
        ref_gu, _ = time_graph(lambda: [ls.gate_up(i) for i in range(K)], 1)
        ls.packed = True
        extra["layer_set_reference_layout"] = {"step_us": round(ref_ms * 1e3 / K, 3),
                                        "GBs": round(ls.bytes_per_step / (ref_ms / K * 1e-3) / 1e9, 1),
                                        "gate_up_us": round(ref_gu * 1e3 / K, 3)}
        log(f"layer set, reference layout: {ref_ms * 1e3 / K:.2f} us/step, gate/up {ref_gu * 1e3 / K:.2f} us")
        extra["qmm_4096x4096"] = []
        for b in (4, 8):
            for m in (1, 2, 4, 8, 16):
                r = bench_qmm_single(dev, b, m)
                extra["qmm_4096x4096"].append(r)
                log(f"qmm 4096x4096 {b}-bit M={m}: {r['us_chained']} us chained ({r['GBs_chained']} GB/s), "
                    f"{r['us_single']} us single")
        # the same 8B-shaped layer set quantized 4-bit (packed form): the 4-bit small-M qmm at a
        # layer's size, where the single 4096 x 4096 matrix is launch-bound
        ls4 = LayerSet(dev, 4, M, a.layers, seed=2)
        ms4, _ = time_graph(lambda: [ls4.step(i) for i in range(K)], 1)
        gu4, _ = time_graph(lambda: [ls4.gate_up(i) for i in range(K)], 1)
        s4 = ms4 / K
        extra["layer_set_4bit"] = {"step_us": round(s4 * 1e3, 3), "bytes_per_step": ls4.bytes_per_step,
                            "GBs": round(ls4.bytes_per_step / (s4 * 1e-3) / 1e9, 1),
                            "frac_of_peak": round(ls4.bytes_per_step / (s4 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                            "gate_up_us": round(gu4 * 1e3 / K, 3),
                            "gate_up_GBs": round(ls4.gu_bytes / (gu4 / K * 1e-3) / 1e9, 1)}
        log(f"layer set 4-bit: {s4 * 1e3:.2f} us/step ({extra['layer_set_4bit']['GBs']} GB/s), gate/up {gu4 * 1e3 / K:.2f} us "
            f"({extra['layer_set_4bit']['gate_up_GBs']} GB/s)")
        del ls4
        extra["verify_attention"] = []
        for L in (512, 4096, 16384, 32768):
            r = bench_attention(dev, L)
            extra["verify_attention"].append(r)
            log(f"verify attention L={L}: {r['us_chained']} us ({r['GBs_chained']} GB/s), NB={r['blocks']}")
        r = bench_moe(dev)
        extra["moe_block"] = r
        log(f"MoE block: {r['us_chained']} us ({r['GBs_chained']} GB/s), {r['distinct_experts']} experts")
        if not a.no_verify_step:
            r = bench_verify_forward(dev)
            extra["verify_step"] = r
            log(f"verify step (64 layers, 16 rows @ 16k): {r['ms_graph']} ms ({r['GBs']} GB/s, "
                f"{r['frac_of_peak']:.1%} of peak), {r['bytes'] / 1e9:.2f} GB/step; built in {r['build_s']} s")
            torch.cuda.empty_cache()

    cpu = None
    if not a.quick and not a.no_cpu:
        cpu = cpu_baseline(bits, M)
        log(f"CPU baseline: {cpu['value']} GB/s on {cpu['cores']} threads")

    line = {"metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": K, "warmup": a.warmup,
            "ms_per_step": round(ms_step, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "8B-shaped 8-bit layer projection set (q,k,v,o,gate,up,down; hidden 4096, "
                                   "heads 32/8x128, intermediate 12288, group 64) at M=16 verify rows, "
                                   f"rotated over {a.layers} distinct layers, weights in the packed qmm form",
                       "M": M, "bits": bits,
                       "bytes_per_step": ls.bytes_per_step, "launches_per_step": 4, "timing": "hipGraph replay"},
            "roofline": roofline, "cpu_baseline": cpu, "extra": extra}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
