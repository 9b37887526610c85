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

Prints one JSON line per token count: value = algorithmic HBM bytes / measured time (GB/s),
with us per step timed by HIP events around the K steps only; then the roofline of the
dominant kernel (gate/up), timed in a second pass of K steps with HIP events that the
library records on the launch stream around each kernel; and the CPU oracle timed on a
bounded sample of the same workload.

    python bench.py [--steps K] [--warmup W] [--tokens T] [--no-cpu]
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

WORKLOADS = {
    "mixtral": dict(title="Mixtral-8x7B-shape MoE layer verify step", tokens=32, hidden=4096,
                    ffn=14336, experts=8, topk=2, shared_ffn=0, gated=False, renormalize=True),
    "qwen15": dict(title="Qwen1.5-MoE-A2.7B-shape MoE block (gated shared expert) verify step",
                   tokens=64, hidden=2048, ffn=1408, experts=60, topk=4, shared_ffn=5632,
                   gated=True, renormalize=False),
    "dsv2lite": dict(title="DeepSeek-V2-Lite-shape MoE block (2 shared experts) verify step",
                     tokens=32, hidden=2048, ffn=1408, experts=64, topk=6, shared_ffn=2816,
                     gated=False, renormalize=False),
}


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
    ap.add_argument("--rotate", type=int, default=2, help="copies of the weights rotated per step")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-calls", type=int, default=12,
                    help="CPU baseline sample: layer calls (the default is ~10 s of host work "
                         "for the Mixtral layer at 32 tokens)")
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
    ap.add_argument("--library-gemm", action="store_true",
                    help="only time torch.matmul (the ROCm library GEMM) on one expert's dense "
                         "gate/up and down shapes, the practical reference for the tiled kernels")
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


def run_tokens(args, wl, T, layers, L, dev):
    from ae_amd import _lib
    from ae_amd.layers._torch import ptr

    H, I, E, k, Is = args.hidden, args.ffn, args.experts, args.topk, wl["shared_ffn"]
    dtype, es = torch.bfloat16, 2
    g = torch.Generator(device=dev).manual_seed(1000 + T)
    x = torch.randn((T, H), generator=g, device=dev).to(dtype)
    if args.workload == "mixtral":
        wg = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(dtype)
        if args.zipf > 0:
            p = torch.arange(1, E + 1, dtype=torch.float64) ** (-args.zipf)
            bias = torch.log(p / p.sum()).to(device=dev, dtype=dtype)
        else:
            bias = torch.zeros(E, dtype=dtype, device=dev)
        logits = torch.nn.functional.linear(x, wg) + bias
        routing = f"zipf s={args.zipf}" if args.zipf > 0 else "unbiased"
    else:
        logits = (torch.randn((T, E), generator=g, device=dev) * 2.0).to(dtype)
        routing = "logits 2*N(0,1)"
    sgate = torch.randn((T, 1), generator=g, device=dev).to(dtype) if wl["gated"] else None
    y = torch.empty_like(x)
    w_out = torch.empty((T, k), dtype=torch.float32, device=dev)
    ids_out = torch.empty((T, k), dtype=torch.int32, device=dev)
    if Is:
        nbytes = L.smx_moe_shared_workspace_size(T, H, I, E, k, Is, _lib.SMX_BF16)
    else:
        nbytes = L.smx_moe_workspace_size(T, H, I, E, k, _lib.SMX_BF16)
    if nbytes == 0:
        raise SystemExit(f"unsupported shape T={T} H={H} I={I} E={E} k={k} shared={Is}")
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    renorm = 1 if wl["renormalize"] else 0
    if args.layer:
        residual = torch.randn((T, H), generator=g, device=dev).to(dtype)
        norm_w = (1 + 0.1 * torch.randn(H, generator=g, device=dev)).to(dtype)
        gate_w = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(dtype)
        sgate_w = (torch.randn(H, generator=g, device=dev) * 0.02).to(dtype) if wl["gated"] else None
        lbytes = L.smx_moe_layer_workspace_size(T, H, I, E, k, Is, _lib.SMX_BF16)
        lws = torch.empty(lbytes, dtype=torch.uint8, device=dev)

    def call(layer, c, stream):
        if args.layer:
            sp = ctypes.c_void_p(stream.cuda_stream)
            rc = L.smx_moe_layer_forward(
                ptr(x), ptr(residual), _lib.SMX_BF16, T, H, ptr(norm_w), 1e-5, ptr(gate_w), E, k,
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
                ptr(x), ptr(y), _lib.SMX_BF16, T, H, ptr(lg), _lib.SMX_BF16, E, k, renorm,
                ptr(pool), E, 3 * I * H, ptr(slots), ptr(layer.shared[c]), Is, ptr(sgate), 1.0,
                ptr(w_out), ptr(ids_out), ptr(ws), nbytes, sp)
            _lib.check("smx_fused_moe_shared_forward", rc)
        else:
            rc = L.smx_fused_moe_forward(
                ptr(x), ptr(y), _lib.SMX_BF16, T, H, ptr(lg), _lib.SMX_BF16, E, k, renorm,
                ptr(pool), E, 3 * I * H, ptr(slots), ptr(w_out), ptr(ids_out), ptr(ws), nbytes, sp)
            _lib.check("smx_fused_moe_forward", rc)

    slots = torch.arange(E, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream(dev)
    copies = len(layers[0].pools)

    def step(i, s=None):
        for layer in layers:
            call(layer, i % copies, s or stream)

    # ---- routing facts for the algorithmic byte count (same logits for every layer)
    call(layers[0], 0, stream)
    torch.cuda.synchronize()
    ids_np = ids_out.cpu().numpy()
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
    # and whether the routing runs inside the gate/up launch (small batches, logits in bf16)
    group = 8 if E <= 8 else 16 if E <= 16 else 32 if E <= 32 else 64
    on = bool(L.smx_routing_in_gateup())
    in_launch = on and not tiled and E <= 64 and (
        (T * k <= 64 and T <= 32 and T * group <= 256) or
        (T * k <= 256 and T <= 64 and T * group <= 512))
    # larger top-k: its own launch, the sort inside the gate/up launch
    sort_in_launch = in_launch or (on and not tiled and E <= 64 and T * k <= 256 and T <= 64)
    if args.layer:  # the layer call routes from the norm kernel's picks (one token: in the norm)
        in_launch = not tiled and E <= 64 and (T == 1 or (on and T * k <= 256 and T <= 64))

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
    value = step_bytes / (us_step * 1e-6) / 1e9
    config = {
        "workload": f"{wl['title']}, {T} tokens" + (f", {len(layers)} layers" if len(layers) > 1 else ""),
        "tokens": T, "hidden": H, "ffn": I, "experts": E, "top_k": k,
        "routing": routing, "active_experts": len(active), "tokens_per_expert": counts,
        "pool_copies_rotated": copies,
        "expert_kernels": "tiled" if tiled else "streaming",
        "down_combine": "fused" if fused_down else "split",
        "routing_launch": ("inside the gate/up launch" if in_launch else
                           "top-k kernel, sort inside the gate/up launch" if sort_in_launch
                           else "routing kernels"),
    }
    if Is:
        config.update({"shared_ffn": Is, "shared_gate": wl["gated"]})
    if len(layers) > 1:
        config["layers"] = len(layers)
    if graphs is not None:
        config["hip_graph"] = True
    if args.layer:
        config["layer_call"] = "residual add + RMSNorm + router gate + top-k + MoE"
    out = {
        "metric": METRIC if args.workload == "mixtral" and not args.layer else
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
        "dtype": "bf16",
        "data": "synthetic: N(0,0.02) expert weights, N(0,1) hidden states, "
                + ("gate N(0,0.02) + Zipf bias" if args.workload == "mixtral" else "router logits 2*N(0,1)"),
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
        if tiled:  # many tokens per expert: the matrix cores bound the tiled kernels
            tflops = gateup_flops / (stage_us[1] * 1e-6) / 1e12
            out["roofline"] = {
                "kernel": "tile_gateup_kernel (W1/W3 x 128-token MFMA tiles + SiLU*up epilogue)",
                "bound": "mfma",
                "achieved": round(tflops, 1),
                "peak": MFMA_BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s",
                "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
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
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args, wl, x, logits, sgate, layers[0], slots,
                                           layer_bytes)
    print(json.dumps(out), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the multi-GPU sharding of this path is a design, not a measured run)",
              file=sys.stderr)
        sys.exit(2)
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
    tokens = ([int(v) for v in args.sweep_tokens.split(",")] if args.sweep_tokens
              else [args.tokens if args.tokens is not None else wl["tokens"]])
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    L = _lib.lib()
    if args.tiled_min_tokens is not None:
        _lib.check("smx_set_tiled_min_tokens", L.smx_set_tiled_min_tokens(args.tiled_min_tokens))
    if args.fused_down_max_tokens is not None:
        _lib.check("smx_set_fused_down_max_tokens",
                   L.smx_set_fused_down_max_tokens(args.fused_down_max_tokens))
    g = torch.Generator(device=dev).manual_seed(0)
    copies = args.rotate if args.layers == 1 else 1  # a stack of layers is its own rotation
    layers = [Layer(g, dev, args.hidden, args.ffn, args.experts, wl["shared_ffn"], copies,
                    torch.bfloat16) for _ in range(args.layers)]
    for T in tokens:
        run_tokens(args, wl, T, layers, L, dev)


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


def cpu_baseline(args, wl, x, logits, sgate, layer, slots, layer_bytes):
    """The numpy oracle on the host cores, on the same workload (one layer); a bounded sample
    of --cpu-calls layer calls (inputs copied to host memory before timing)."""
    import numpy as np
    from oracle import moe_ref as ref

    def bits(t):
        return t.cpu().view(torch.int16).numpy().view(np.uint16)

    xb = bits(x)
    lf = logits.float().cpu().numpy()
    pb = bits(layer.pools[0])
    sl = slots.cpu().numpy()
    shared = bits(layer.shared[0]) if layer.shared else None
    sg = sgate.float().cpu().numpy().reshape(-1) if sgate is not None else None
    renorm = wl["renormalize"]

    def run(n):
        if shared is None:
            return ref.fused_moe_forward(xb[:n], lf[:n], pb, sl, args.topk, renorm, ref.BF16)
        return ref.fused_moe_shared_forward(xb[:n], lf[:n], pb, sl, args.topk, renorm, ref.BF16,
                                            shared, None if sg is None else sg[:n])

    try:
        from threadpoolctl import threadpool_info
        cores = max(int(i["num_threads"]) for i in threadpool_info() if i.get("user_api") == "blas")
    except Exception:
        cores = len(os.sched_getaffinity(0))
    run(1)  # warm BLAS
    t0 = time.perf_counter()
    for _ in range(args.cpu_calls):
        run(xb.shape[0])
    dt = (time.perf_counter() - t0) / args.cpu_calls
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(layer_bytes / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "us_per_step": round(dt * 1e6, 1),
        "sample": f"{args.cpu_calls} layer calls of the same workload through the numpy oracle "
                  f"(fp32 OpenBLAS GEMMs on bf16-rounded values), {cores} threads, {cpu_model}",
    }


if __name__ == "__main__":
    main()
