"""Verify-step MoE layer benchmark on one MI355X.

Workload (default): a Mixtral-8x7B-shape MoE layer (hidden 4096, ffn 14336, 8 experts,
top-2, bf16) at 32 verify tokens (8 sequences x 4 draft tokens), router gate biased for a
Zipf s=1.2 expert load. One step = one FusedMoE forward (routing + experts + combine)
through the C ABI, with inputs resident in HBM. Expert weights are N(0, 0.02), hidden states
N(0, 1), synthetic; two copies of the expert pool are rotated so no step finds the previous
step's weights in a cache.

Other workloads (--workload): the MoE blocks with a shared expert, one call each through
smx_fused_moe_shared_forward -- qwen15 (Qwen1.5-MoE-A2.7B: hidden 2048, 60 experts of ffn
1408, top-4, gated shared expert of ffn 5632, 64 tokens) and dsv2lite (DeepSeek-V2-Lite:
hidden 2048, 64 experts of ffn 1408, top-6, shared ffn 2816); router logits 2*N(0,1), no
renormalisation. --layers N runs a stack of N layers with distinct weights per step
(DeepSeek-V2-Lite has 26), --sweep-tokens runs one line per token count, --graph replays
each step from a HIP graph.

c1 is the reference's CPU-runnable configuration: hidden 1024, ffn 2816, 8 experts, top-2, fp32,
32 tokens (4 sequences x 8 draft tokens), router logits x Wg^T with Wg ~ N(0, 0.02).

Prints one JSON line per token count: value = algorithmic HBM bytes / measured time (GB/s),
with us per step timed by HIP events around the K steps only; then the roofline of the
dominant kernel (gate/up), timed in a second pass of K steps with HIP events that the
library records on the launch stream around each kernel; the parity of the layer call against
the numpy oracle on the same inputs (ids, weight bits, both output error metrics); and the CPU
baseline: the same layer on the host cores through two restatements, C++ (oracle/cpu_moe.cpp,
cblas_sgemm on MKL under OpenMP) and torch (oracle/torch_cpu.py, GEMMs on MKL), weights
converted to fp32 once, outside the timing, median of >= 20 calls after 3 warm-up calls each;
the faster is the baseline, the other reported beside it. The
default Mixtral run also times 8, 16, 48 and 64 tokens (the rest of the metric's 8-64 range)
with the same event-timed loop and reports them under "sweep", and under "workloads" the other
configurations of the benchmark's definition: c1 (fp32, with its gate/up roofline and CPU
baseline), Mixtral at 1 and 4 tokens (unbiased gate), Qwen1.5-MoE at 64 tokens, and the
26-layer DeepSeek-V2-Lite stack at 1, 32 and 128 tokens (parity: its first layer).

    python bench.py [--steps K] [--warmup W] [--tokens T] [--no-cpu] [--no-parity]
    python bench.py --workload c1
    python bench.py --workload dsv2lite --layers 26 --sweep-tokens 1,2,4,8,16,32,64,128 --no-cpu
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import torch

METRIC = "MoE layer us/verify-step + achieved HBM GB/s (% peak), Mixtral shape, 8-64 tokens"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16 matrix-core peak of one MI355X
MFMA_FP32_PEAK_TFLOPS = 157.3   # dense fp32 matrix-core peak

WORKLOADS = {
    "mixtral": dict(title="Mixtral-8x7B-shape MoE layer verify step", tokens=32, hidden=4096,
                    ffn=14336, experts=8, topk=2, shared_ffn=0, gated=False, renormalize=True),
    "qwen15": dict(title="Qwen1.5-MoE-A2.7B-shape MoE block (gated shared expert) verify step",
                   tokens=64, hidden=2048, ffn=1408, experts=60, topk=4, shared_ffn=5632,
                   gated=True, renormalize=False),
    "dsv2lite": dict(title="DeepSeek-V2-Lite-shape MoE block (2 shared experts) verify step",
                     tokens=32, hidden=2048, ffn=1408, experts=64, topk=6, shared_ffn=2816,
                     gated=False, renormalize=False),
    "c1": dict(title="MoE layer H1024/I2816/E8/top-2 fp32 verify step (the reference's CPU-runnable "
                     "configuration)", tokens=32, hidden=1024, ffn=2816, experts=8, topk=2,
               shared_ffn=0, gated=False, renormalize=True, dtype="fp32"),
}
# The rest of the headline metric's 8-64 token range, timed beside the default Mixtral run.
HEADLINE_SWEEP = (8, 16, 48, 64)
# The other configurations of the benchmark's definition, timed beside the default run (the
# same event-timed loop and weight rotation) under "workloads": name -> (workload, tokens,
# layers, overrides of the workload's settings, CPU baseline).
EXTRA_WORKLOADS = {
    "c1_fp32_t32": ("c1", 32, 1, {}, True),
    "c2_mixtral_t1": ("mixtral", 1, 1, {"zipf": 0.0}, False),
    "c2_mixtral_t4": ("mixtral", 4, 1, {"zipf": 0.0}, False),
    "c4_qwen15_t64": ("qwen15", 64, 1, {}, False),
    "c5_dsv2lite_26layers_t1": ("dsv2lite", 1, 26, {}, False),
    "c5_dsv2lite_26layers_t32": ("dsv2lite", 32, 26, {}, False),
    "c5_dsv2lite_26layers_t128": ("dsv2lite", 128, 26, {}, False),
}
DTYPES = {"bf16": (torch.bfloat16, 2, 2), "fp32": (torch.float32, 4, 0)}  # torch dtype, bytes, SMX code


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="mixtral")
    ap.add_argument("--tokens", type=int, default=None)
    ap.add_argument("--sweep-tokens", type=str, default=None,
                    help="comma-separated token counts, one JSON line each")
    ap.add_argument("--hidden", type=int, default=None)
    ap.add_argument("--ffn", type=int, default=None)
    ap.add_argument("--experts", type=int, default=None)
    ap.add_argument("--topk", type=int, default=None)
    ap.add_argument("--layers", type=int, default=1, help="layers with distinct weights per step")
    ap.add_argument("--graph", action="store_true", help="replay each step from a HIP graph")
    ap.add_argument("--layer", action="store_true",
                    help="time the whole post-attention layer call (residual add + RMSNorm + "
                         "router gate + top-k + MoE, smx_moe_layer_forward) and, beside it, the "
                         "unfused sequence (norm kernel, torch gate GEMM, MoE call)")
    ap.add_argument("--zipf", type=float, default=1.2,
                    help="Mixtral gate bias exponent (0 = unbiased)")
    ap.add_argument("--rotate", type=int, default=None,
                    help="copies of the weights rotated per step (default: enough copies for "
                         ">= 1 GB of weights, at least 2)")
    ap.add_argument("--dtype", choices=sorted(DTYPES), default=None,
                    help="activation and weight dtype (default: the workload's, bf16 but c1 fp32)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-parity", action="store_true", help="skip the parity check against the oracle")
    ap.add_argument("--no-sweep", action="store_true",
                    help="skip the 8/16/48/64-token lines of the default Mixtral run")
    ap.add_argument("--no-workloads", action="store_true",
                    help="skip the other configurations (C1, C2 at 1 and 4 tokens, Qwen1.5-MoE, "
                         "the DeepSeek-V2-Lite stack) timed beside the default Mixtral run")
    ap.add_argument("--cpu-runs", type=int, default=20,
                    help="CPU baseline: timed layer calls (after 3 warm-up calls); the median is reported")
    ap.add_argument("--h2d", action="store_true",
                    help="measure host -> device streaming of expert pages through the transfer "
                         "engine (pinned host memory, chunked copies), alone and beside the MoE "
                         "kernels")
    ap.add_argument("--tiled-min-tokens", type=int, default=None,
                    help="expected tokens per active expert at which the tiled MFMA expert "
                         "kernels replace the streaming ones (0 = always, a huge value = never; "
                         "default: the library's)")
    ap.add_argument("--fused-down-max-tokens", type=int, default=None,
                    help="largest batch whose down projection and combine run as one kernel "
                         "(0 = never; default: the library's)")
    ap.add_argument("--gateup-waves", type=int, default=None, choices=[0, 1, 2, 4],
                    help="waves per workgroup of the weight-streaming gate/up kernel (0 = the "
                         "library's rule)")
    ap.add_argument("--routing-in-gateup", type=int, default=None, choices=[0, 1],
                    help="small batches routed inside the gate/up launch (1, the library's "
                         "default) or by the routing kernels (0)")
    ap.add_argument("--expert-items", type=int, default=None, choices=[0, 1],
                    help="gate/up items of the in-launch routing in expert order where the "
                         "library's rule takes them (1, the default) or by range (0)")
    ap.add_argument("--gateup-item-walk", type=int, default=None, choices=[0, 1],
                    help="gate/up grids beyond one residency as workgroups walking several items "
                         "(1, the library's default) or one workgroup per item (0)")
    ap.add_argument("--library-gemm", action="store_true",
                    help="only time torch.matmul (the ROCm library GEMM) on one expert's dense "
                         "gate/up and down shapes, the practical reference for the tiled kernels")
    ap.add_argument("--read-floor", action="store_true",
                    help="only time smx_stream_read (plain streaming reads, one launch each) at the "
                         "sizes of the small-batch expert launches: the practical floor of a read "
                         "of that size in one launch, and of the gate/up + down pair")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device copy 10 times (HBM counter calibration)")
    return ap.parse_args()


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "traffic_gateup_kernel_mixtral_t32.json")


def copy_calibration():
    """A plain copy of known size, profiled beside the MoE kernels to scale the HBM byte
    counters (FETCH_SIZE / WRITE_SIZE) to bytes."""
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": n, "copy_calibration_bytes_written": n,
                      "launches": 10}), flush=True)


def read_floor(steps):
    """Best time per launch of a plain streaming read (smx_stream_read) over workgroup sizes, at
    the byte counts of the DeepSeek-V2-Lite block's launches at one token (gate/up 92.3 MB, down
    46.1 MB, both 138.4 MB), 289 MB and 1 GiB; the source rotates over regions of a 4 GiB buffer
    so that no launch finds its bytes in a cache. Also the gate/up + down pair as two launches
    back to back."""
    from ae_amd import _lib
    L = _lib.lib()
    pool_bytes = 4 << 30
    buf = torch.empty(pool_bytes, dtype=torch.uint8, device="cuda").fill_(1)
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    base = buf.data_ptr()
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    unit = 16 << 10

    def timed(launches):  # launches: list of (offset, bytes, per_wg); returns us per pass
        # passes rotate over regions at least 300 MiB (and at least one pass) apart, as many as
        # fit in the buffer (at most 12): no pass finds its bytes in a cache
        span = max(off + nb for off, nb, _ in launches)
        stride = -(-max(span, 300 << 20) // (1 << 20)) * (1 << 20)
        regions = min(12, pool_bytes // stride)
        for _ in range(5):
            for off, nb, pw in launches:
                _lib.check("smx_stream_read", L.smx_stream_read(base + off, nb, pw, sink.data_ptr(), sp))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            for off, nb, pw in launches:
                _lib.check("smx_stream_read", L.smx_stream_read(base + off + (i % regions) * stride,
                                                                nb, pw, sink.data_ptr(), sp))
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / steps

    best = {}
    for mb in (23.0, 46.1, 92.3, 138.4, 289.0, 1073.7):
        rows = []
        for pw in (32 << 10, 64 << 10, 128 << 10, 256 << 10):
            nb = int(mb * 1e6) // pw * pw
            us = timed([(0, nb, pw)])
            rows.append({"per_workgroup_kib": pw >> 10, "workgroups": nb // pw, "us": round(us, 2),
                         "tbs": round(nb / us / 1e6, 3)})
        b = min(rows, key=lambda r: r["us"] / (r["workgroups"] * r["per_workgroup_kib"]))
        best[mb] = b
        print(json.dumps({"read_floor_mb": mb, "best": b, "all": rows}), flush=True)
    g, d = best[92.3], best[46.1]
    pg, pd = g["per_workgroup_kib"] << 10, d["per_workgroup_kib"] << 10
    ng, nd = int(92.3e6) // pg * pg, int(46.1e6) // pd * pd
    us = timed([(0, ng, pg), (ng + (1 << 20), nd, pd)])
    print(json.dumps({"read_floor_pair_mb": [92.3, 46.1], "us": round(us, 2),
                      "tbs": round((ng + nd) / us / 1e6, 3),
                      "hbm_frac": round((ng + nd) / us / 1e6 / (HBM_PEAK_GBS / 1000), 4)}), flush=True)


def library_gemm():
    """torch.matmul in bf16 (hipBLASLt on ROCm) on one Mixtral expert's dense shapes: gate/up
    [M, 4096] x [4096, 2 * 14336] and down [M, 14336] x [14336, 4096], weights row-major
    [N, K] as nn.Linear stores them, for M tokens per expert."""
    dev = "cuda"
    out = {}
    for M, K, N in [(512, 4096, 28672), (1024, 4096, 28672), (2048, 4096, 28672),
                    (1024, 14336, 4096)]:
        a = torch.randn((M, K), device=dev, dtype=torch.bfloat16)
        b = torch.randn((N, K), device=dev, dtype=torch.bfloat16)
        for _ in range(5):
            torch.matmul(a, b.t())
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = 20
        e0.record()
        for _ in range(n):
            torch.matmul(a, b.t())
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1000.0 / n
        out[f"{M}x{K}x{N}"] = {"us": round(us, 1),
                               "tflops": round(2.0 * M * K * N / (us * 1e-6) / 1e12, 1)}
    print(json.dumps({"library_gemm_bf16": out, "peak_tflops": MFMA_BF16_PEAK_TFLOPS}), flush=True)


def measured_traffic(T, H, I, E, k, workload):
    """HBM bytes per gateup_kernel launch measured with rocprofv3 counters for this workload
    (committed under profiles/), or None."""
    if workload != "mixtral":
        return None
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("workload") != {"tokens": T, "hidden": H, "ffn": I, "experts": E, "top_k": k}:
        return None
    return t.get("bytes_per_launch")


class Layer:
    """One MoE layer's weights in HBM: `copies` expert pools (and shared pages) to rotate."""

    def __init__(self, g, dev, H, I, E, Is, copies, dtype):
        self.pools, self.shared = [], []
        for _ in range(copies):
            pool = torch.empty((E, 3 * I * H), dtype=dtype, device=dev)
            for e in range(E):  # fill page by page to bound the fp32 temporary
                pool[e] = (torch.randn(3 * I * H, generator=g, device=dev) * 0.02).to(dtype)
            self.pools.append(pool)
            if Is:
                self.shared.append((torch.randn(3 * Is * H, generator=g, device=dev) * 0.02).to(dtype))


def run_tokens(args, wl, T, layers, L, dev, light=False):
    """Measure one token count. light: only the event-timed loop (the headline's sweep points);
    otherwise also the per-kernel stage pass, the roofline, the parity check and the CPU
    baseline. Returns the JSON object."""
    from ae_amd import _lib
    from ae_amd.layers._torch import ptr

    H, I, E, k, Is = args.hidden, args.ffn, args.experts, args.topk, wl["shared_ffn"]
    dtype, es, dcode = DTYPES[args.dtype]
    dname = "bf16" if args.dtype == "bf16" else "fp32"
    g = torch.Generator(device=dev).manual_seed(1000 + T)
    x = torch.randn((T, H), generator=g, device=dev).to(dtype)
    if args.workload in ("mixtral", "c1"):
        wg = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(dtype)
        if args.workload == "mixtral" and args.zipf > 0:
            p = torch.arange(1, E + 1, dtype=torch.float64) ** (-args.zipf)
            bias = torch.log(p / p.sum()).to(device=dev, dtype=dtype)
            routing = f"zipf s={args.zipf}"
        else:
            bias = torch.zeros(E, dtype=dtype, device=dev)
            routing = "gate N(0,0.02), unbiased"
        logits = torch.nn.functional.linear(x, wg) + bias
    else:
        logits = (torch.randn((T, E), generator=g, device=dev) * 2.0).to(dtype)
        routing = "logits 2*N(0,1)"
    sgate = torch.randn((T, 1), generator=g, device=dev).to(dtype) if wl["gated"] else None
    y = torch.empty_like(x)
    w_out = torch.empty((T, k), dtype=torch.float32, device=dev)
    ids_out = torch.empty((T, k), dtype=torch.int32, device=dev)
    if Is:
        nbytes = L.smx_moe_shared_workspace_size(T, H, I, E, k, Is, dcode)
    else:
        nbytes = L.smx_moe_workspace_size(T, H, I, E, k, dcode)
    if nbytes == 0:
        raise SystemExit(f"unsupported shape T={T} H={H} I={I} E={E} k={k} shared={Is}")
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    renorm = 1 if wl["renormalize"] else 0
    if args.layer:
        residual = torch.randn((T, H), generator=g, device=dev).to(dtype)
        norm_w = (1 + 0.1 * torch.randn(H, generator=g, device=dev)).to(dtype)
        gate_w = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(dtype)
        sgate_w = (torch.randn(H, generator=g, device=dev) * 0.02).to(dtype) if wl["gated"] else None
        lbytes = L.smx_moe_layer_workspace_size(T, H, I, E, k, Is, dcode)
        lws = torch.empty(lbytes, dtype=torch.uint8, device=dev)

    def call(layer, c, stream):
        if args.layer:
            sp = ctypes.c_void_p(stream.cuda_stream)
            rc = L.smx_moe_layer_forward(
                ptr(x), ptr(residual), dcode, T, H, ptr(norm_w), 1e-5, ptr(gate_w), E, k,
                renorm, ptr(layer.pools[c]), E, 3 * I * H, ptr(slots),
                ptr(layer.shared[c] if Is else None), Is, ptr(sgate_w), 1.0, None, ptr(w_out),
                ptr(ids_out), ptr(lws), lbytes, sp)
            _lib.check("smx_moe_layer_forward", rc)
            return
        call_moe(layer, c, stream)

    def call_moe(layer, c, stream, lg=None):
        sp = ctypes.c_void_p(stream.cuda_stream)
        pool = layer.pools[c]
        lg = logits if lg is None else lg
        if Is:
            rc = L.smx_fused_moe_shared_forward(
                ptr(x), ptr(y), dcode, T, H, ptr(lg), dcode, E, k, renorm,
                ptr(pool), E, 3 * I * H, ptr(slots), ptr(layer.shared[c]), Is, ptr(sgate), 1.0,
                ptr(w_out), ptr(ids_out), ptr(ws), nbytes, sp)
            _lib.check("smx_fused_moe_shared_forward", rc)
        else:
            rc = L.smx_fused_moe_forward(
                ptr(x), ptr(y), dcode, T, H, ptr(lg), dcode, E, k, renorm,
                ptr(pool), E, 3 * I * H, ptr(slots), ptr(w_out), ptr(ids_out), ptr(ws), nbytes, sp)
            _lib.check("smx_fused_moe_forward", rc)

    slots = torch.arange(E, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream(dev)
    copies = len(layers[0].pools)

    def step(i, s=None):
        for layer in layers:
            call(layer, i % copies, s or stream)

    # ---- routing facts for the algorithmic byte count (same logits for every layer); the
    # outputs of this first call are the ones the parity check compares with the oracle
    call(layers[0], 0, stream)
    torch.cuda.synchronize()
    y_first = (x if args.layer else y).clone()
    ids_np = ids_out.cpu().numpy()
    w_first = w_out.cpu().numpy().copy()
    active = sorted(set(int(v) for v in ids_np.reshape(-1)))
    counts = [int((ids_np == e).sum()) for e in range(E)]
    weight_bytes = len(active) * 3 * H * I * es + 3 * H * Is * es
    layer_bytes = (weight_bytes + 2 * T * H * es + T * E * es + T * k * 8
                   + (T * es if wl["gated"] else 0))
    if args.layer:  # residual read + write, the in-place normalized states, norm and gate weights
        layer_bytes += 3 * T * H * es + H * es + E * H * es + (H * es if wl["gated"] else 0)
    step_bytes = layer_bytes * len(layers)
    gateup_bytes = ((len(active) * 2 * H * I + 2 * H * Is) * es + T * H * es
                    + (T * k * I + T * Is) * es)
    gateup_flops = 2.0 * (T * k * 2 * H * I + T * 2 * H * Is)
    step_flops = 2.0 * (T * k * 3 * H * I + T * 3 * H * Is) * len(layers)
    # the library's choice of expert kernels: expected tokens per active expert vs its threshold
    n_assign = T * k
    exp_active = min(max(E * (1.0 - (1.0 - k / E) ** T), 1.0), min(E, n_assign))
    tiled = n_assign > 0 and n_assign / exp_active >= L.smx_tiled_min_tokens()
    # and of the fused down projection + combine (a few tokens, short weight rows per output)
    fd = L.smx_fused_down_max_tokens()
    units = T * (k * -(-I * es // 1024) + -(-Is * es // 1024))
    fused_down = not tiled and 1 <= T <= 8 and (T <= fd if fd >= 0 else units <= 48)
    # and whether the routing runs inside the gate/up launch (small batches, logits in the
    # activation dtype)
    plan = _lib.plan_info(T, H, I, E, k, dcode, Is)
    on = bool(L.smx_routing_in_gateup())
    in_launch = bool(plan["topk_in_gateup"])
    # larger top-k: its own launch, the sort inside the gate/up launch
    sort_in_launch = in_launch or (on and not tiled and E <= 64 and T * k <= 768)
    if args.layer:  # the layer call routes from the norm kernel's picks (one token: in the norm)
        in_launch = not tiled and E <= 64 and (T == 1 or (on and T * k <= 768))
    # one token in one launch (gate/up, then the fused down + combine workgroups in the same
    # grid): the library's plan, when the routing runs inside the launch and nothing captures
    single = bool(plan["single_launch"]) and in_launch and not args.layer and not args.graph

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    graphs = None
    if args.graph:
        side = torch.cuda.Stream(dev)
        side.wait_stream(stream)
        graphs = []
        with torch.cuda.stream(side):
            for c in range(copies):
                step(c, side)  # warm the capture stream
        torch.cuda.synchronize()
        for c in range(copies):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                step(c, torch.cuda.current_stream(dev))
            graphs.append(gr)
        for c in range(copies):
            graphs[c].replay()
        torch.cuda.synchronize()

    # ---- timed region: K steps, HIP events only before and after (no per-kernel events: each
    # event recorded between kernels costs the stream several microseconds)
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_start.record(stream)
    for i in range(args.steps):
        if graphs is not None:
            graphs[i % copies].replay()
        else:
            step(i)
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_step = t_start.elapsed_time(t_end) / args.steps
    us_step = 1000.0 * ms_step
    value = step_bytes / (us_step * 1e-6) / 1e9
    if light:
        return {"us_per_step": round(us_step, 2), "gbs": round(value, 1),
                "hbm_frac": round(value / HBM_PEAK_GBS, 4), "algorithmic_bytes": step_bytes,
                "active_experts": len(active), "steps": args.steps}

    # ---- stage pass (eager, 1 layer): the same steps again with HIP events recorded by the
    # library on the launch stream before routing and after each kernel
    per_kernel = graphs is None and len(layers) == 1
    ev = None
    if per_kernel:
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(args.steps)]
        for row in ev:  # materialise the event handles
            for e_ in row:
                e_.record(stream)
        handles = [(ctypes.c_void_p * 5)(*[e_.cuda_event for e_ in row]) for row in ev]
        torch.cuda.synchronize()
        for i in range(args.steps):
            _lib.check("smx_set_profile_events", L.smx_set_profile_events(handles[i], 5))
            step(i)
        torch.cuda.synchronize()
        _lib.check("smx_set_profile_events", L.smx_set_profile_events(None, 0))
    unfused_us = None
    if args.layer:
        from ae_amd.layers import add_rmsnorm_gate

        def unfused(i):
            add_rmsnorm_gate(x, residual, norm_w, 1e-5)
            lg = torch.nn.functional.linear(x, gate_w)
            call_moe(layers[0], i % copies, stream, lg)

        for i in range(args.warmup):
            unfused(i)
        u0 = torch.cuda.Event(enable_timing=True)
        u1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        u0.record(stream)
        for i in range(args.steps):
            unfused(i)
        u1.record(stream)
        torch.cuda.synchronize()
        unfused_us = 1000.0 * u0.elapsed_time(u1) / args.steps
    config = {
        "workload": f"{wl['title']}, {T} tokens" + (f", {len(layers)} layers" if len(layers) > 1 else ""),
        "tokens": T, "hidden": H, "ffn": I, "experts": E, "top_k": k,
        "routing": routing, "active_experts": len(active), "tokens_per_expert": counts,
        "pool_copies_rotated": copies,
        "expert_kernels": ("tiled" if tiled else
                           "streaming, one launch (gate/up and the fused down + combine)" if single
                           else "streaming"),
        "down_combine": "fused" if fused_down else "split",
        "routing_launch": ("inside the gate/up launch" if in_launch else
                           "top-k kernel, sort inside the gate/up launch" if sort_in_launch
                           else "routing kernels"),
    }
    if sort_in_launch and plan["expert_items"]:
        config["gateup_items"] = "expert order, first weights issued before the routing"
    if Is:
        config.update({"shared_ffn": Is, "shared_gate": wl["gated"]})
    if len(layers) > 1:
        config["layers"] = len(layers)
    if graphs is not None:
        config["hip_graph"] = True
    if args.layer:
        config["layer_call"] = "residual add + RMSNorm + router gate + top-k + MoE"
    headline = args.workload == "mixtral" and not args.layer and len(layers) == 1
    out = {
        "metric": METRIC if headline else
        f"{'post-attention layer call (add+RMSNorm+gate+top-k+MoE)' if args.layer else 'MoE'} "
        f"{'stack' if len(layers) > 1 else 'layer'} us/verify-step + achieved HBM GB/s, {args.workload}",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dname,
        "data": f"synthetic: N(0,0.02) expert weights, N(0,1) hidden states, "
                + ("gate N(0,0.02) + Zipf bias" if args.workload == "mixtral" and args.zipf > 0 else
                   "gate N(0,0.02)" if args.workload in ("mixtral", "c1") else "router logits 2*N(0,1)"),
        "config": config,
        "us_per_step": round(us_step, 2),
        "layer_hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "algorithmic_bytes": step_bytes,
        "tflops": round(step_flops / (us_step * 1e-6) / 1e12, 1),
        "wall_s_timed": round(wall, 4),
        "roofline": None,
        "cpu_baseline": None,
    }
    if args.layer:
        out["unfused_us_per_step"] = round(unfused_us, 2)
    if per_kernel:
        stage = [0.0] * 4
        for row in ev:
            for s in range(4):
                stage[s] += row[s].elapsed_time(row[s + 1])
        stage_us = [1000.0 * v / args.steps for v in stage]
        gateup_gbs = gateup_bytes / (stage_us[1] * 1e-6) / 1e9
        # with the fused down projection + combine no combine kernel runs: the last interval is
        # only the cost of recording an event, and is reported as 0
        # routing inside the gate/up launch: the first interval is only an event's cost
        out["stage_us"] = {"route": 0.0 if in_launch else round(stage_us[0], 2),
                           "gate_up": round(stage_us[1], 2),
                           "down": round(stage_us[2], 2),
                           "combine": 0.0 if fused_down else round(stage_us[3], 2)}
        if single:  # one launch streams every weight row of the layer
            layer_gbs = layer_bytes / (stage_us[1] * 1e-6) / 1e9
            out["stage_us"]["down"] = 0.0  # no down launch: the interval is only an event's cost
            out["roofline"] = {
                "kernel": "gateup_kernel with the fused down + combine workgroups (the whole layer "
                          "in one launch: W1/W3 and W2 streams, SiLU*up, combine)",
                "bound": "hbm",
                "achieved": round(layer_gbs, 1),
                "peak": HBM_PEAK_GBS,
                "unit": "GB/s",
                "frac": round(layer_gbs / HBM_PEAK_GBS, 4),
                "traffic": None,
                "algorithmic_bytes": layer_bytes,
                "us_per_launch": round(stage_us[1], 2),
            }
        elif tiled:  # many tokens per expert: the matrix cores bound the tiled kernels
            tflops = gateup_flops / (stage_us[1] * 1e-6) / 1e12
            peak = MFMA_BF16_PEAK_TFLOPS if dname == "bf16" else MFMA_FP32_PEAK_TFLOPS
            out["roofline"] = {
                "kernel": "tile_gateup_kernel (W1/W3 x 128-token MFMA tiles + SiLU*up epilogue)",
                "bound": "mfma",
                "achieved": round(tflops, 1),
                "peak": peak,
                "unit": "TFLOP/s",
                "frac": round(tflops / peak, 4),
                "traffic": None,
                "algorithmic_flops": gateup_flops,
                "hbm_gbs": round(gateup_bytes / (stage_us[1] * 1e-6) / 1e9, 1),
                "us_per_launch": round(stage_us[1], 2),
            }
        else:
            out["roofline"] = {
                "kernel": "gateup_kernel (W1/W3 stream + SiLU*up epilogue)",
                "bound": "hbm",
                "achieved": round(gateup_gbs, 1),
                "peak": HBM_PEAK_GBS,
                "unit": "GB/s",
                "frac": round(gateup_gbs / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic(T, H, I, E, k, args.workload),
                "algorithmic_bytes": gateup_bytes,
                "us_per_launch": round(stage_us[1], 2),
            }
    oracle_out = None
    # a stack's parity is its first layer's call (every layer runs the same kernels)
    parity = not args.no_parity and not args.layer
    cpu = not args.no_cpu and len(layers) == 1
    if parity or cpu:
        host = _host_inputs(args, wl, x, logits, sgate, layers[0], slots)
        if parity:
            out["parity"], oracle_out = parity_check(args, host, y_first, w_first, ids_np)
            if len(layers) > 1:
                out["parity"]["scope"] = "the first layer's call of the stack"
        if cpu:
            out["cpu_baseline"] = cpu_baseline(args, host, layer_bytes, T, oracle_out)
    return out


def run_workloads(args, dev, L, mixtral_layers):
    """The other configurations of the benchmark's definition, one compact entry each: us per
    step, algorithmic GB/s and HBM fraction from the same event-timed loop as the headline,
    the per-kernel stages and gate/up roofline of single layers, parity against the oracle
    (a stack: its first layer) and, for the reference's CPU-runnable configuration, the CPU
    baseline. Weights of each workload are freed before the next one is built."""
    keep = ("us_per_step", "layer_hbm_frac", "algorithmic_bytes", "stage_us", "roofline",
            "parity", "cpu_baseline")
    out = {}
    built = {}
    for name, (wname, T, nlayers, over, cpu) in EXTRA_WORKLOADS.items():
        wl = WORKLOADS[wname]
        a = argparse.Namespace(**vars(args))
        a.workload = wname
        for key in ("hidden", "ffn", "experts", "topk"):
            setattr(a, key, wl[key])
        a.dtype = wl.get("dtype", "bf16")
        a.layers = nlayers
        a.no_cpu = not cpu
        a.no_parity = False
        for key, v in over.items():
            setattr(a, key, v)
        if wname == "mixtral":
            layers = mixtral_layers
        else:
            key = (wname, nlayers)
            if key not in built:
                built.clear()  # free the previous workload's weights first
                torch.cuda.empty_cache()
                es = DTYPES[a.dtype][1]
                page_bytes = 3 * a.hidden * a.ffn * es
                pool_bytes = a.experts * page_bytes + 3 * a.hidden * wl["shared_ffn"] * es
                copies = max(2, -(-(1 << 30) // pool_bytes)) if nlayers == 1 else 1
                g = torch.Generator(device=dev).manual_seed(0)
                built[key] = [Layer(g, dev, a.hidden, a.ffn, a.experts, wl["shared_ffn"], copies,
                                    DTYPES[a.dtype][0]) for _ in range(nlayers)]
            layers = built[key]
        r = run_tokens(a, wl, T, layers, L, dev)
        entry = {"workload": r["config"]["workload"], "dtype": r["dtype"],
                 "gbs": r["value"], "ms_per_step": r["ms_per_step"],
                 "active_experts": r["config"]["active_experts"],
                 "expert_kernels": r["config"]["expert_kernels"],
                 "down_combine": r["config"]["down_combine"],
                 "routing": r["config"]["routing"]}
        entry.update({k: r[k] for k in keep if r.get(k) is not None})
        if entry.get("parity"):
            p = entry["parity"]
            entry["parity"] = {k: p[k] for k in ("ids_equal", "weight_bits_equal", "max_rel_err",
                                                 "elem_rel_err_p99", "tol_max_rel_err", "pass",
                                                 "scope") if k in p}
        out[name] = entry
    built.clear()
    torch.cuda.empty_cache()
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the multi-GPU sharding of this path is a design, not a measured run)",
              file=sys.stderr)
        sys.exit(2)
    if args.read_floor:
        read_floor(args.steps)
        return
    if args.copy_calibration:
        copy_calibration()
        return
    if args.library_gemm:
        library_gemm()
        return
    if args.h2d:
        h2d_bench(args)
        return

    from ae_amd import _lib

    wl = WORKLOADS[args.workload]
    for key in ("hidden", "ffn", "experts", "topk"):
        if getattr(args, key) is None:
            setattr(args, key, wl[key])
    if args.dtype is None:
        args.dtype = wl.get("dtype", "bf16")
    tokens = ([int(v) for v in args.sweep_tokens.split(",")] if args.sweep_tokens
              else [args.tokens if args.tokens is not None else wl["tokens"]])
    # the default run is the headline: Mixtral at 32 tokens, plus the rest of the 8-64 range
    headline_sweep = (args.workload == "mixtral" and not args.sweep_tokens and args.tokens is None
                      and args.layers == 1 and not args.layer and not args.graph and not args.no_sweep)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    L = _lib.lib()
    if args.tiled_min_tokens is not None:
        _lib.check("smx_set_tiled_min_tokens", L.smx_set_tiled_min_tokens(args.tiled_min_tokens))
    if args.fused_down_max_tokens is not None:
        _lib.check("smx_set_fused_down_max_tokens",
                   L.smx_set_fused_down_max_tokens(args.fused_down_max_tokens))
    if args.gateup_waves is not None:
        _lib.check("smx_set_gateup_waves", L.smx_set_gateup_waves(args.gateup_waves))
    if args.gateup_item_walk is not None:
        _lib.check("smx_set_gateup_item_walk", L.smx_set_gateup_item_walk(args.gateup_item_walk))
    if args.routing_in_gateup is not None:
        _lib.check("smx_set_routing_in_gateup", L.smx_set_routing_in_gateup(args.routing_in_gateup))
    if args.expert_items is not None:
        _lib.check("smx_set_gateup_expert_items", L.smx_set_gateup_expert_items(args.expert_items))
    g = torch.Generator(device=dev).manual_seed(0)
    es = DTYPES[args.dtype][1]
    page_bytes = 3 * args.hidden * args.ffn * es
    if args.rotate is None:  # enough copies that no step finds its weights in a cache
        pool_bytes = args.experts * page_bytes + 3 * args.hidden * wl["shared_ffn"] * es
        args.rotate = max(2, -(-(1 << 30) // pool_bytes))
    copies = args.rotate if args.layers == 1 else 1  # a stack of layers is its own rotation
    layers = [Layer(g, dev, args.hidden, args.ffn, args.experts, wl["shared_ffn"], copies,
                    DTYPES[args.dtype][0]) for _ in range(args.layers)]
    for T in tokens:
        out = run_tokens(args, wl, T, layers, L, dev)
        if headline_sweep:
            out["sweep"] = {str(t): run_tokens(args, wl, t, layers, L, dev, light=True)
                            for t in HEADLINE_SWEEP}
            if not args.no_workloads:
                out["workloads"] = run_workloads(args, dev, L, layers)
        print(json.dumps(out), flush=True)


PCIE_GEN5_X16_GBS = 64.0  # host link of one MI355X, per direction, before protocol overhead


def h2d_bench(args):
    """Expert pages (Mixtral shape: 3*14336*4096 bf16 = 352 MB each) streamed from pinned host
    memory into pool slots: the transfer engine at several chunk counts, torch's pinned copy and
    a pageable copy for comparison, and the engine while the MoE kernels run on another stream."""
    from ae_amd import _lib
    from ae_amd.backend import HtoDTransferEngine, free_pinned_tensor, make_pinned_tensor
    from ae_amd.layers._torch import ptr

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    torch.zeros(1, device=dev)
    H, I, E = 4096, 14336, 8
    page = 3 * I * H
    n_pages = 4
    page_bytes = page * 2
    host, hp = make_pinned_tensor(n_pages * page_bytes, torch.bfloat16)
    out = {}
    try:
        host = host.view(n_pages, page)
        host.copy_(torch.randint(-1000, 1000, (n_pages, page), dtype=torch.int16).view(torch.bfloat16))
        pool = torch.empty((2 * n_pages, page), dtype=torch.bfloat16, device=dev)
        stream = torch.cuda.Stream(dev)
        eng = HtoDTransferEngine()
        eng.start()
        for e in range(n_pages):  # warm-up: first touch of the destination pages
            eng.submit_weight_loading_task(host[e], pool[2 * e], stream, f"warm{e}", 1, 1)
        for e in range(n_pages):
            assert eng.wait_for_completion(f"warm{e}")[0]
        rates = {}
        for chunks in (1, 4, 16):
            t0 = time.perf_counter()
            for e in range(n_pages):
                eng.submit_weight_loading_task(host[e], pool[2 * e], stream, f"c{chunks}p{e}", chunks, 1)
            for e in range(n_pages):
                assert eng.wait_for_completion(f"c{chunks}p{e}")[0]
            dt = time.perf_counter() - t0
            rates[chunks] = n_pages * page_bytes / dt / 1e9
            eng.clear_condition([f"c{chunks}p{e}" for e in range(n_pages)])
        ok = all(torch.equal(pool[2 * e].cpu().view(torch.int16), host[e].view(torch.int16))
                 for e in range(n_pages))  # bit patterns (random ones include NaN encodings)
        # torch's copy from the same pinned memory
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for e in range(n_pages):
            pool[2 * e + 1].copy_(host[e], non_blocking=True)
        torch.cuda.synchronize()
        torch_rate = n_pages * page_bytes / (time.perf_counter() - t0) / 1e9
        # pageable source, one page
        pageable = host[0].clone()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        pool[1].copy_(pageable)
        torch.cuda.synchronize()
        pageable_rate = page_bytes / (time.perf_counter() - t0) / 1e9
        del pageable
        # engine beside the MoE kernels (Mixtral layer, 32 tokens, on the default stream)
        T, k = 32, 2
        g = torch.Generator(device=dev).manual_seed(0)
        epool = torch.empty((E, page), dtype=torch.bfloat16, device=dev)
        for e in range(E):
            epool[e] = (torch.randn(page, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
        logits = torch.randn((T, E), generator=g, device=dev).to(torch.bfloat16)
        y = torch.empty_like(x)
        slots = torch.arange(E, dtype=torch.int64, device=dev)
        L = _lib.lib()
        nb = L.smx_moe_workspace_size(T, H, I, E, k, _lib.SMX_BF16)
        ws = torch.empty(nb, dtype=torch.uint8, device=dev)
        cs = torch.cuda.current_stream(dev)
        sp = ctypes.c_void_p(cs.cuda_stream)

        def moe():
            _lib.check("smx_fused_moe_forward", L.smx_fused_moe_forward(
                ptr(x), ptr(y), _lib.SMX_BF16, T, H, ptr(logits), _lib.SMX_BF16, E, k, 1,
                ptr(epool), E, page, ptr(slots), None, None, ptr(ws), nb, sp))

        for _ in range(5):
            moe()
        torch.cuda.synchronize()
        steps = 40
        a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a0.record(cs)
        for _ in range(steps):
            moe()
        a1.record(cs)
        torch.cuda.synchronize()
        moe_alone_us = 1000.0 * a0.elapsed_time(a1) / steps
        t0 = time.perf_counter()
        for e in range(n_pages):
            eng.submit_weight_loading_task(host[e], pool[2 * e], stream, f"ov{e}", 4, 1)
        a0.record(cs)
        for _ in range(steps):
            moe()
        a1.record(cs)
        for e in range(n_pages):
            assert eng.wait_for_completion(f"ov{e}")[0]
        h2d_dt = time.perf_counter() - t0
        torch.cuda.synchronize()
        moe_beside_us = 1000.0 * a0.elapsed_time(a1) / steps
        eng.stop()
        value = rates[4]
        out = {
            "metric": "host -> device expert page streaming GB/s (pinned host memory, transfer engine)",
            "value": round(value, 2),
            "unit": "GB/s",
            "n_gpus": 1,
            "higher_is_better": True,
            "dtype": "bf16",
            "data": "synthetic bf16 expert pages",
            "config": {"workload": "Mixtral-8x7B expert pages (352 MB each) into pool slots",
                       "pages": n_pages, "page_bytes": page_bytes},
            "roofline": {"bound": "pcie", "achieved": round(value, 2), "peak": PCIE_GEN5_X16_GBS,
                         "unit": "GB/s", "frac": round(value / PCIE_GEN5_X16_GBS, 4)},
            "engine_gbs_by_chunks": {str(c): round(r, 2) for c, r in rates.items()},
            "torch_pinned_copy_gbs": round(torch_rate, 2),
            "pageable_copy_gbs": round(pageable_rate, 2),
            "bit_exact": ok,
            "overlap": {"moe_us_alone": round(moe_alone_us, 2),
                        "moe_us_beside_h2d": round(moe_beside_us, 2),
                        "h2d_gbs_beside_moe": round(n_pages * page_bytes / h2d_dt / 1e9, 2)},
        }
    finally:
        free_pinned_tensor(hp)
    print(json.dumps(out), flush=True)


def _host_inputs(args, wl, x, logits, sgate, layer, slots):
    """The layer's inputs on the host, as the oracle reads them (bf16 as bit patterns)."""
    import numpy as np

    def store(t):
        t = t.detach().cpu().contiguous()
        if t.dtype == torch.bfloat16:
            return t.view(torch.int16).numpy().view(np.uint16)
        return t.numpy()

    return dict(x=store(x), logits=logits.float().cpu().numpy(), pool=store(layer.pools[0]),
                slots=slots.cpu().numpy(), shared=store(layer.shared[0]) if layer.shared else None,
                sgate=sgate.float().cpu().numpy().reshape(-1) if sgate is not None else None,
                dtype="bf16" if args.dtype == "bf16" else "f32", k=args.topk,
                renorm=wl["renormalize"])


def parity_check(args, h, y_gpu, w_gpu, ids_gpu):
    """The first layer call's outputs against the numpy oracle on the same inputs (same logit
    bits): ids equal, weight bits equal, max |y - ref| / max |ref| and the elementwise
    |y - ref| / max(|ref|, 1e-3 max |ref|). Returns (parity object, oracle output)."""
    import numpy as np
    from oracle import moe_ref as ref

    t0 = time.perf_counter()
    if h["shared"] is None:
        y_ref, w_ref, ids_ref = ref.fused_moe_forward(h["x"], h["logits"], h["pool"], h["slots"],
                                                      h["k"], h["renorm"], h["dtype"])
    else:
        y_ref, w_ref, ids_ref = ref.fused_moe_shared_forward(
            h["x"], h["logits"], h["pool"], h["slots"], h["k"], h["renorm"], h["dtype"],
            shared_page=h["shared"], shared_gate_logits=h["sgate"])
    oracle_s = time.perf_counter() - t0
    y = y_gpu.float().cpu().numpy().astype(np.float64)
    want = y_ref.astype(np.float64)
    floor = 1e-3 * max(float(np.abs(want).max()), 1e-30)
    el = np.abs(y - want) / np.maximum(np.abs(want), floor)
    tol = 1e-2 if args.dtype == "bf16" else 1e-4
    max_rel = float(np.abs(y - want).max()) / max(float(np.abs(want).max()), 1e-30)
    return {
        "against": "numpy oracle (oracle/moe_ref.py) on the same inputs and logit bits",
        "ids_equal": bool(np.array_equal(ids_gpu, ids_ref)),
        "weight_bits_equal": bool(np.array_equal(np.ascontiguousarray(w_gpu, np.float32).view(np.uint32),
                                                 np.ascontiguousarray(w_ref, np.float32).view(np.uint32))),
        "max_rel_err": float(f"{max_rel:.3e}"),
        "elem_rel_err_median": float(f"{np.median(el):.3e}"),
        "elem_rel_err_p99": float(f"{np.quantile(el, 0.99):.3e}"),
        "elem_rel_err_max": float(f"{el.max():.3e}"),
        "tol_max_rel_err": tol,
        "pass": bool(np.array_equal(ids_gpu, ids_ref)) and max_rel <= tol,
        "oracle_s": round(oracle_s, 2),
    }, y_ref


def cpu_baseline(args, h, layer_bytes, T, oracle_y=None):
    """The layer on the host cores, inputs already in host memory, the pool's pages converted to
    fp32 once before timing; 3 warm-up calls, then the median of --cpu-runs calls. Two
    restatements: torch (oracle/torch_cpu.py, GEMMs on torch's MKL) and C++
    (oracle/cpu_moe.cpp, cblas_sgemm on the image's MKL under OpenMP); the faster is the
    baseline, the other is reported beside it ("torch_cpu" or "cpp_mkl")."""
    import numpy as np
    from oracle.torch_cpu import TorchCpuMoE

    affinity = len(os.sched_getaffinity(0))
    threads = min(affinity, int(os.environ.get("OMP_NUM_THREADS", affinity)))
    torch.set_num_threads(threads)
    moe = TorchCpuMoE(h["pool"], h["slots"], args.hidden, h["dtype"], shared_page=h["shared"])
    if h["dtype"] == "bf16":
        xf = torch.from_numpy(h["x"].view(np.int16)).view(torch.bfloat16).float()
    else:
        xf = torch.from_numpy(h["x"]).float()
    lf = torch.from_numpy(h["logits"])
    sg = torch.from_numpy(h["sgate"]) if h["sgate"] is not None else None

    def run():
        return moe.forward(xf, lf, h["k"], h["renorm"], shared_gate=sg)

    for _ in range(3):
        y_cpu, _, _ = run()
    times = []
    for _ in range(args.cpu_runs):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    dt = float(np.median(times))
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # the first processor's block
                key, _, val = line.partition(":")
                info[key.strip()] = val.strip()
    except OSError:
        pass
    flags = set(info.get("flags", "").split())
    cpu_model = (f"{info.get('model name', '?')} (family {info.get('cpu family', '?')}, model "
                 f"{info.get('model', '?')}, stepping {info.get('stepping', '?')}, "
                 f"{'AVX-512' if 'avx512f' in flags else 'AVX2' if 'avx2' in flags else 'no AVX2'})")
    out = {
        "value": round(layer_bytes / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "us_per_step": round(dt * 1e6, 1),
        "sample": f"median of {args.cpu_runs} calls (after 3 warm-up calls) of the same layer and "
                  f"{T} tokens through a torch-CPU restatement of the layer "
                  f"(oracle/torch_cpu.py: fp32 MKL GEMMs on "
                  f"{'bf16-rounded values' if h['dtype'] == 'bf16' else 'fp32 values'}, weights "
                  f"converted to fp32 before timing), {threads} threads",
        "cpu_model": cpu_model,
        "affinity_cpus": affinity,
        "torch_threads": torch.get_num_threads(),
        "blas": "MKL" if torch.backends.mkl.is_available() else "torch CPU BLAS",
        "us_min": round(min(times) * 1e6, 1),
        "us_max": round(max(times) * 1e6, 1),
    }
    if oracle_y is not None:
        want = oracle_y.astype(np.float64)
        out["max_rel_err_vs_oracle"] = float(
            f"{float(np.abs(y_cpu.numpy() - want).max()) / max(float(np.abs(want).max()), 1e-30):.3e}")
    cpp = cpp_mkl_baseline(args, h, moe, xf, lf, layer_bytes, threads, oracle_y)
    if cpp is None:
        return out
    if cpp["us_per_step"] >= out["us_per_step"]:
        out["cpp_mkl"] = cpp
        return out
    # the faster restatement is the baseline; the other is reported beside it
    torch_keys = ("value", "us_per_step", "us_min", "us_max", "sample", "torch_threads", "blas",
                  "max_rel_err_vs_oracle")
    torch_cpu = {k: out.pop(k) for k in torch_keys if k in out}
    out.update(cpp)
    out["blas"] = "MKL (libmkl_rt, sequential, one call per OpenMP thread)"
    out["torch_cpu"] = torch_cpu
    return out


def cpp_mkl_baseline(args, h, moe, xf, lf, layer_bytes, threads, oracle_y=None):
    """The C++ restatement (oracle/cpu_moe.cpp: cblas_sgemm per expert on the image's MKL,
    OpenMP threads) on the same fp32 weights as the torch one, timed the same way. None where it
    does not apply (shared-expert blocks, fp16) or MKL is missing."""
    import numpy as np
    from oracle import cpu_mkl

    if h["shared"] is not None or h["dtype"] not in ("bf16", "f32") or not cpu_mkl.available():
        return None
    I = next(iter(moe.w1.values())).shape[0]
    cm = cpu_mkl.MklCpuMoE(moe.w1, moe.w3, moe.w2, moe.E, args.hidden, I, h["dtype"], threads=threads)
    xn, ln = xf.numpy(), lf.numpy().astype(np.float32)

    def run():
        return cm.forward(xn, ln, h["k"], h["renorm"])

    for _ in range(3):
        y, _, _ = run()
    times = []
    for _ in range(args.cpu_runs):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    dt = float(np.median(times))
    out = {
        "value": round(layer_bytes / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "us_per_step": round(dt * 1e6, 1),
        "us_min": round(min(times) * 1e6, 1),
        "us_max": round(max(times) * 1e6, 1),
        "sample": f"median of {args.cpu_runs} calls (after 3 warm-up calls) of the same layer and "
                  f"inputs through oracle/cpu_moe.cpp (one sequential-MKL cblas_sgemm per OpenMP "
                  f"thread and column slice, per expert product), {threads} threads",
    }
    if oracle_y is not None:
        want = oracle_y.astype(np.float64)
        out["max_rel_err_vs_oracle"] = float(
            f"{float(np.abs(y - want).max()) / max(float(np.abs(want).max()), 1e-30):.3e}")
    return out


if __name__ == "__main__":
    main()
