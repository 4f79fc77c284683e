#!/usr/bin/env python3
"""Throughput of the MI355X GatedDeltaNet path on one GPU; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Workloads (synthetic, seeded; inputs resident in HBM before the timed region):
  prefill  config C1: GDN layer prefill from projection outputs (mixed_qkv, z, a, b)
           to the gated-norm output, B=4 T=4096 Hk=16 Hv=32 d=128 (headline).
           A "step" is one omx_gdn_prefill call over the whole batch.
  decode   config C2: one cached decode step (conv cache + fp32 state in place), B=64.
  core     one chunk_gated_delta_rule call at --batch/--seq-len/--k-heads/--v-heads
           (C1 by default; C4 is --batch 1 --seq-len 65536 --v-heads 64).
  bwd      one chunk_gated_delta_rule_bwd call (the VJP: forward recompute, reverse state-
           gradient scan, chunk-parallel gradients) at the core workload's shape.
  layer_bwd one gdn_prefill_bwd call at C1 (the layer's VJP: conv, gates, rule, gated norm).
  layer_module the whole GatedDeltaNet layer at C1 with D=2048 (projection GEMMs included):
           a forward, and a training step (forward + gradients of every parameter and the
           input); the line's value is the training step's tokens/s.
  copy     a plain 256 MiB device copy, the calibration of the HBM traffic counters.
The headline line reports prefill tokens/s with the MFMA roofline of the chunked
rule, timed at the core-function boundary (chunk_gated_delta_rule on the same
shapes: the chunk-parallel preparation kernel and the state scan), and carries the
decode step's HBM roofline as "decode", the rule's backward pass (VJP) at C1 as
"backward", the layer's backward as "layer_backward" and the whole layer with its
projections (forward and training step) as "layer_module".  Only one GPU is
used: --gpus above 1 exits with a message.

Kernel durations come from HIP events recorded on the stream the kernels run on
(torch's current stream, which the library launches on).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
C = 64


def prefill_flops_per_token_head(dk, dv, c=C):
    """Matmuls of deltanet.py:107,115,116,130,133,136,137,142: 2C(3dk+2dv) + 6 dk dv."""
    return 2 * c * (3 * dk + 2 * dv) + 6 * dk * dv


def bwd_flops_per_token_head(dk, dv, c=C):
    """Matmuls of the reverse pass, forward recompute included (the fp64 oracle's
    products, oracle/gdn_vjp.py): 8 of C x C x dk, 5 of C x C x dv, 8 of C x dk x dv and
    the two C^3 products of dL = X^T dX X^T, per chunk; the triangular inverse excluded."""
    return 16 * c * dk + 10 * c * dv + 16 * dk * dv + 4 * c * c


def decode_bytes_per_seq(Hk, Hv, dk, dv, K=4):
    conv_dim = 2 * Hk * dk + Hv * dv
    return (Hv * dk * dv * 4 * 2 + 2 * conv_dim * (K - 1) * 2 + conv_dim * 2 + 2 * Hv * 2
            + 2 * Hv * dv * 2)


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


def time_launches(fn, steps, warmup):
    """Run fn warmup+steps times back to back.

    Returns (wall seconds of the timed steps, ms per call from one pair of HIP
    events around all timed calls on the current stream -- the stream the
    library launches on).  The timed region is bracketed by a device
    synchronisation on both sides.
    """
    import torch
    for _ in range(warmup):
        fn()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, start.elapsed_time(end) / steps


def cpu_cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


# ----------------------------------------------------------------------------- decode (C2)

def bench_decode(B, steps, warmup, cpu_baseline):
    import torch
    from omegalax_amd import gdn_decode_step, workloads as W
    Hk, Hv, d = 16, 32, 128
    _say(f"decode: B={B} generating inputs")
    arrs = W.decode_inputs(B)
    t = W.to_device(arrs)
    dims = dict(num_k_heads=Hk, head_k_dim=d, num_v_heads=Hv, head_v_dim=d)

    def step():
        gdn_decode_step(t["mixed_qkv"], t["z"], t["a"], t["b"], t["conv_w"], t["A_log"],
                        t["dt_bias"], t["norm_w"], t["conv_state"], t["state"], **dims)

    _say(f"decode: B={B} timing {steps} steps")
    wall, ms = time_launches(step, steps, warmup)
    nbytes = decode_bytes_per_seq(Hk, Hv, d, d) * B
    gbs = nbytes / (ms * 1e-3) / 1e9
    res = {
        "batch": B, "ms_per_step": wall / steps * 1e3, "kernel_ms": ms,
        "tokens_per_s": B * steps / wall,
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": gbs / PEAK_HBM_GBS,
                     "traffic": MEASURED_TRAFFIC.get(("decode", B, Hk, Hv, d)),
                     "algorithmic_bytes": nbytes},
    }
    if cpu_baseline:
        res["cpu_baseline"] = cpu_decode_baseline()
    return res


def cpu_decode_baseline(B=8, budget_s=10.0):
    """Oracle decode step (numpy fp64, the 'port') on a bounded sample: B=8 sequences."""
    from oracle import gdn_oracle as O
    from omegalax_amd import workloads as W
    d = W.decode_inputs(B)
    S = d["state"].astype(np.float64)
    conv = d["conv_state"]
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s or n == 0:
        _, conv, S = O.gdn_decode_step(d["mixed_qkv"], d["z"], d["a"], d["b"], d["conv_w"],
                                       d["A_log"], d["dt_bias"], d["norm_w"], conv, S,
                                       Hk=16, dk=128, Hv=32, dv=128)
        n += 1
    el = time.perf_counter() - t0
    return {"value": B * n / el, "unit": "tokens/s", "cores": cpu_cores(), "kind": "port",
            "sample": f"{n} decode steps of the numpy fp64 oracle at B={B}, C2 head layout"}


# ----------------------------------------------------------------------------- core call

# HBM bytes per call from two rocprofv3 --pmc runs (FETCH_SIZE x 2.0 and WRITE_SIZE x 1.0,
# scaled by a plain copy kernel's counters), for the shapes they were taken on; summaries
# and commands in profiles/prefill_c1.md and profiles/decode_step_c2_b64.md.
MEASURED_TRAFFIC = {
    ("core", 4, 4096, 16, 32, 128): 1_154_719_808,  # prep 152.2 MiB + 284.7, scan 408.3 + 256.0
    ("decode", 64, 16, 32, 128): 277_401_702,       # state read + written once
}


def bench_core(B, T, Hk, Hv, d, steps, warmup, arrs=None):
    """One chunk_gated_delta_rule call (bf16 q/k/v, fp32 gates) over [B, T]: the
    chunk-parallel preparation kernel and the state scan, HIP-event timed."""
    import torch
    from omegalax_amd import chunk_gated_delta_rule, workloads as W
    rng = np.random.default_rng(7)

    def act(*shape):
        x = W.round_bf16(rng.standard_normal(shape, dtype=np.float32))
        return torch.from_numpy(x).cuda().bfloat16()

    q, k, v = act(B, T, Hk, d), act(B, T, Hk, d), act(B, T, Hv, d)
    if arrs is None:
        arrs = W.layer_inputs(B, T, Hk, Hv, d, d) if B * T <= 16384 else None
    if arrs is not None:
        g32, beta32 = W.gates_f32(arrs["a"], arrs["b"], arrs["A_log"], arrs["dt_bias"])
    else:
        g32 = -0.1 * rng.random((B, T, Hv), dtype=np.float32)
        beta32 = rng.random((B, T, Hv), dtype=np.float32)
    g = torch.from_numpy(g32).cuda()
    beta = torch.from_numpy(beta32).cuda()

    def core():
        chunk_gated_delta_rule(q, k, v, g, beta, C)

    _say(f"core: B={B} T={T} Hk={Hk} Hv={Hv} timing {steps} launches")
    wall, ms = time_launches(core, steps, warmup)
    flops = prefill_flops_per_token_head(d, d) * B * T * Hv
    tf = flops / (ms * 1e-3) / 1e12
    return {
        "ms_per_step": wall / steps * 1e3, "kernel_ms": ms,
        "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": tf / PEAK_BF16_TFLOPS,
                     "traffic": MEASURED_TRAFFIC.get(("core", B, T, Hk, Hv, d)),
                     "algorithmic_flops": flops,
                     "kernels": "prep_kernel + scan_kernel (the two launches of one call)"},
    }


def bench_bwd(B, T, Hk, Hv, d, steps, warmup):
    """One chunk_gated_delta_rule_bwd call (bf16 q/k/v, fp32 gates and cotangent), HIP-event
    timed: the backward variants of the prep and scan, the reverse scan, the chunk-parallel
    gradient kernel and the q/k finalisation."""
    import torch
    from omegalax_amd import chunk_gated_delta_rule_bwd, workloads as W
    rng = np.random.default_rng(8)

    def act(*shape):
        x = W.round_bf16(rng.standard_normal(shape, dtype=np.float32))
        return torch.from_numpy(x).cuda().bfloat16()

    q, k, v = act(B, T, Hk, d), act(B, T, Hk, d), act(B, T, Hv, d)
    a = rng.standard_normal((B, T, Hv), dtype=np.float32)
    A_log = rng.uniform(0, np.log(16), Hv).astype(np.float32)
    dt = rng.uniform(-2, 0, Hv).astype(np.float32)
    g = torch.from_numpy((-np.exp(A_log) * np.logaddexp(a + dt, 0)).astype(np.float32)).cuda()
    beta = torch.from_numpy(1 / (1 + np.exp(-rng.standard_normal((B, T, Hv), dtype=np.float32)))).cuda()
    do = torch.from_numpy(rng.standard_normal((B, T, Hv, d), dtype=np.float32)).cuda()

    def bwd():
        chunk_gated_delta_rule_bwd(q, k, v, g, beta, do, C)

    _say(f"bwd: B={B} T={T} Hk={Hk} Hv={Hv} timing {steps} launches")
    wall, ms = time_launches(bwd, steps, warmup)
    flops = bwd_flops_per_token_head(d, d) * B * T * Hv
    tf = flops / (ms * 1e-3) / 1e12
    return {
        "ms_per_step": wall / steps * 1e3, "kernel_ms": ms,
        "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": tf / PEAK_BF16_TFLOPS, "traffic": None,
                     "algorithmic_flops": flops,
                     "kernels": "prep (bwd) + scan (bwd) + rscan + cgrad + qk_final"},
    }


def bench_layer_bwd(steps, warmup, B=4, T=4096):
    """One gdn_prefill_bwd call at C1 (bf16 activations, bf16 output cotangent)."""
    import torch
    from omegalax_amd import gdn_prefill_bwd, workloads as W
    Hk, Hv, d = 16, 32, 128
    arrs = W.layer_inputs(B, T, Hk, Hv, d, d)
    t = W.to_device(arrs)
    rng = np.random.default_rng(9)
    dout = torch.from_numpy(rng.standard_normal((B, T, Hv * d), dtype=np.float32)).cuda().bfloat16()
    dims = dict(num_k_heads=Hk, head_k_dim=d, num_v_heads=Hv, head_v_dim=d)

    def step():
        gdn_prefill_bwd(t["mixed_qkv"], t["z"], t["a"], t["b"], t["conv_w"], t["A_log"],
                        t["dt_bias"], t["norm_w"], dout, **dims)

    _say(f"layer_bwd: B={B} T={T} timing {steps} calls")
    wall, ms = time_launches(step, steps, warmup)
    return {"ms_per_step": wall / steps * 1e3, "kernel_ms": ms,
            "tokens_per_s": B * T * steps / wall}


# ----------------------------------------------------------------------------- layer module (C1)

def bench_layer_module(steps, warmup, B=4, T=4096, D=2048):
    """GatedDeltaNet.__call__ (deltanet.py:226-306) at C1 with its projections, which run as
    hipBLASLt GEMMs through F.linear: the forward hidden -> out, and a training step (the
    forward plus the gradients of every parameter and of the input for a fixed output
    cotangent)."""
    import torch
    from omegalax_amd import GDNConfig, GDNParams, gated_deltanet_forward, workloads as W
    Hk, Hv, d = 16, 32, 128
    cfg = GDNConfig(hidden_size=D, num_k_heads=Hk, head_k_dim=d, num_v_heads=Hv, head_v_dim=d)
    _say(f"layer module: B={B} T={T} D={D} generating parameters and inputs")
    arrs = W.module_params(D, Hk, Hv, d, d)
    lin = {"in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj"}
    params = GDNParams(**{k_: torch.from_numpy(v_).cuda().to(torch.bfloat16 if k_ in lin else torch.float32)
                          for k_, v_ in arrs.items()})
    gen = torch.Generator(device="cuda").manual_seed(1001)
    h = torch.randn((B, T, D), generator=gen, device="cuda").bfloat16()
    R = torch.randn((B, T, D), generator=gen, device="cuda").bfloat16()

    def fwd():
        with torch.no_grad():
            gated_deltanet_forward(params, cfg, h)

    leaves = [getattr(params, f).requires_grad_() for f in params.__dataclass_fields__]
    hx = h.clone().requires_grad_()

    def train():
        out = gated_deltanet_forward(params, cfg, hx)
        torch.autograd.grad(out, leaves + [hx], R)

    _say(f"layer module: timing {steps} forwards and {max(steps // 2, 5)} training steps")
    wall_f, ms_f = time_launches(fwd, steps, warmup)
    n_t = max(steps // 2, 5)
    wall_t, ms_t = time_launches(train, n_t, warmup)
    for leaf in leaves:
        leaf.requires_grad_(False)
    return {"config": f"GatedDeltaNet forward / training step at C1 with projections (D={D})",
            "forward_ms": ms_f, "forward_tokens_per_s": B * T * steps / wall_f,
            "train_step_ms": ms_t, "train_tokens_per_s": B * T * n_t / wall_t}


# ----------------------------------------------------------------------------- prefill (C1)

def bench_prefill(steps, warmup, cpu_baseline, B=4, T=4096):
    import torch
    from omegalax_amd import gdn_prefill, workloads as W
    Hk, Hv, d = 16, 32, 128
    _say(f"prefill: B={B} T={T} generating inputs")
    arrs = W.layer_inputs(B, T, Hk, Hv, d, d)
    t = W.to_device(arrs)
    dims = dict(num_k_heads=Hk, head_k_dim=d, num_v_heads=Hv, head_v_dim=d)

    def step():
        gdn_prefill(t["mixed_qkv"], t["z"], t["a"], t["b"], t["conv_w"], t["A_log"],
                    t["dt_bias"], t["norm_w"], **dims)

    _say(f"prefill: timing {steps} layer steps")
    wall, ms_step = time_launches(step, steps, warmup)
    tokens = B * T

    # the dominant kernels, prep + scan, at the core-function boundary on the same shapes
    core = bench_core(B, T, Hk, Hv, d, steps, warmup, arrs)
    res = {
        "tokens_per_s": tokens * steps / wall, "ms_per_step": wall / steps * 1e3,
        "step_event_ms": ms_step, "core_kernel_ms": core["kernel_ms"],
        "roofline": core["roofline"],
    }
    if cpu_baseline:
        res["cpu_baseline"] = cpu_prefill_baseline()
    return res


def cpu_prefill_baseline(budget_s=15.0):
    """Oracle layer prefill (numpy restatement, fp32 core like the reference) on a bounded
    C1 sample: B=1, T=512, the C1 head layout; numpy's BLAS uses the visible cores."""
    from oracle import gdn_oracle as O
    from omegalax_amd import workloads as W
    B, T = 1, 512
    d = W.layer_inputs(B, T)
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s or n == 0:
        O.gdn_prefill_layer(d["mixed_qkv"], d["z"], d["a"], d["b"], d["conv_w"], d["A_log"],
                            d["dt_bias"], d["norm_w"], Hk=16, dk=128, Hv=32, dv=128,
                            dtype=np.float32)
        n += 1
    el = time.perf_counter() - t0
    return {"value": B * T * n / el, "unit": "tokens/s", "cores": cpu_cores(), "kind": "port",
            "sample": f"{n} runs of the numpy fp32 layer prefill restatement, B={B} T={T}, C1 head layout"}


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=["prefill", "decode", "core", "bwd", "layer_bwd",
                                           "layer_module", "copy"],
                    default="prefill")
    ap.add_argument("--decode-batch", type=int, default=64)
    ap.add_argument("--batch", type=int, default=4, help="core workload: sequences")
    ap.add_argument("--seq-len", type=int, default=4096, help="core workload: tokens each")
    ap.add_argument("--k-heads", type=int, default=16, help="core workload")
    ap.add_argument("--v-heads", type=int, default=32, help="core workload")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the GDN path shards by sequence and head with no exchange; see DESIGN.md)",
              file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    cpu = not args.no_cpu_baseline
    if args.workload == "copy":
        # calibration of the FETCH_SIZE / WRITE_SIZE counters: a plain 256 MiB device copy
        src = torch.empty(1 << 26, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        wall, ms = time_launches(lambda: dst.copy_(src), args.steps, args.warmup)
        gbs = 2 * src.numel() * 4 / (ms * 1e-3) / 1e9
        print(json.dumps({"metric": "device copy GB/s (counter calibration)", "value": gbs,
                          "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
                          "warmup": args.warmup, "ms_per_step": wall / args.steps * 1e3,
                          "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                          "dtype": "f32", "data": "synthetic",
                          "config": {"workload": "256 MiB read + 256 MiB written"}}), flush=True)
        return 0
    if args.workload == "layer_module":
        res = bench_layer_module(args.steps, args.warmup)
        line = {
            "metric": "GatedDeltaNet training-step tokens/s (projections included, config C1)",
            "value": res["train_tokens_per_s"], "unit": "tokens/s", "n_gpus": 1,
            "steps": max(args.steps // 2, 5), "warmup": args.warmup,
            "ms_per_step": res["train_step_ms"], "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded N(0,1) hidden states and output cotangent, random-init params)",
            "config": {"workload": res["config"]}, "layer_module": res,
        }
        print(json.dumps(line), flush=True)
        return 0
    if args.workload == "layer_bwd":
        res = bench_layer_bwd(args.steps, args.warmup)
        line = {
            "metric": "gdn_prefill_bwd tokens/s (GDN layer backward, config C1)",
            "value": res["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": res["ms_per_step"], "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded N(0,1) activations and cotangent, random-init params)",
            "config": {"workload": "C1 GDN layer backward B=4 T=4096 Hk=16 Hv=32 d=128"},
            "kernel_ms": res["kernel_ms"],
        }
        print(json.dumps(line), flush=True)
        return 0
    if args.workload == "bwd":
        B, T, Hk, Hv = args.batch, args.seq_len, args.k_heads, args.v_heads
        res = bench_bwd(B, T, Hk, Hv, 128, args.steps, args.warmup)
        line = {
            "metric": "chunk_gated_delta_rule_bwd TFLOP/s (bf16 MFMA roofline)",
            "value": res["roofline"]["achieved"], "unit": "TFLOP/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded N(0,1) activations and cotangents, random-init gates)",
            "config": {"workload": f"chunk_gated_delta_rule_bwd B={B} T={T} Hk={Hk} Hv={Hv} d=128",
                       "chunk": C},
            "roofline": res["roofline"], "kernel_ms": res["kernel_ms"],
        }
        print(json.dumps(line), flush=True)
        return 0
    if args.workload == "core":
        B, T, Hk, Hv = args.batch, args.seq_len, args.k_heads, args.v_heads
        core = bench_core(B, T, Hk, Hv, 128, args.steps, args.warmup)
        line = {
            "metric": "chunk_gated_delta_rule TFLOP/s (bf16 MFMA roofline)",
            "value": core["roofline"]["achieved"], "unit": "TFLOP/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": core["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded N(0,1) activations, random-init params)",
            "config": {"workload": f"chunk_gated_delta_rule B={B} T={T} Hk={Hk} Hv={Hv} d=128",
                       "chunk": C},
            "roofline": core["roofline"], "kernel_ms": core["kernel_ms"],
        }
        print(json.dumps(line), flush=True)
        return 0
    if args.workload == "decode":
        dec = bench_decode(args.decode_batch, args.steps, args.warmup, cpu)
        line = {
            "metric": "decode-step HBM GB/s (GDN decode, config C2)",
            "value": dec["roofline"]["achieved"], "unit": "GB/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": dec["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic (seeded N(0,1) activations, random-init params)",
            "config": {"workload": f"C2 decode step B={args.decode_batch} Hk=16 Hv=32 d=128"},
            "roofline": dec["roofline"], "decode": dec,
        }
        if cpu:
            line["cpu_baseline"] = dec.pop("cpu_baseline")
        print(json.dumps(line), flush=True)
        return 0
    pre = bench_prefill(args.steps, args.warmup, cpu)
    dec = bench_decode(args.decode_batch, max(args.steps, 20), args.warmup, False)
    bwd = bench_bwd(4, 4096, 16, 32, 128, max(args.steps // 2, 5), args.warmup)
    lbwd = bench_layer_bwd(max(args.steps // 2, 5), args.warmup)
    mod = bench_layer_module(args.steps, args.warmup)
    line = {
        "metric": "GDN prefill tokens/s + %MFMA peak; decode-step HBM GB/s + %of 8 TB/s",
        "value": pre["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": pre["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, random-init params)",
        "config": {"workload": "C1 GDN layer prefill (projection outputs -> gated-norm output)",
                   "batch": 4, "seq_len": 4096, "k_heads": 16, "v_heads": 32, "head_dim": 128,
                   "chunk": 64},
        "roofline": pre["roofline"],
        "decode": {"config": f"C2 B={args.decode_batch}", "roofline": dec["roofline"],
                   "kernel_ms": dec["kernel_ms"], "tokens_per_s": dec["tokens_per_s"]},
        "prefill_detail": {k_: pre[k_] for k_ in ("step_event_ms", "core_kernel_ms")},
        "backward": {"config": "chunk_gated_delta_rule_bwd at C1 (B=4 T=4096 Hk=16 Hv=32 d=128)",
                     "kernel_ms": bwd["kernel_ms"], "roofline": bwd["roofline"]},
        "layer_backward": {"config": "gdn_prefill_bwd at C1", "kernel_ms": lbwd["kernel_ms"],
                           "tokens_per_s": lbwd["tokens_per_s"]},
        "layer_module": mod,
    }
    if cpu:
        line["cpu_baseline"] = pre["cpu_baseline"]
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
