#!/usr/bin/env python3
"""Throughput of the MI355X GatedDeltaNet path on one GPU; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Workloads (synthetic, seeded; inputs resident in HBM before the timed region):
  prefill  (default, the headline) config C1: GDN layer prefill from the projection
           outputs (mixed_qkv, z, a, b) to the gated-norm output, B=4 T=4096 Hk=16 Hv=32
           d=128.  A "step" is one omx_gdn_prefill call over the whole batch.  The line
           also carries C3, C4, the C2 decode step at B=1, 8, 64 and 256 (with its CPU
           baseline), the backward passes,
           the whole layer with its projections and the gate projections, each under its
           own key.
  c1       the C1 leg of the headline alone (the layer step and the core call).
  decode   config C2: one cached decode step (conv cache + fp32 state in place) at
           --decode-batch, rotating through enough state sets that no step finds its state
           in the 256 MB last-level cache.
  c3       config C3: packed layer prefill, 8 sequences in T=32768 with initial states.
  core     one chunk_gated_delta_rule call at --batch/--seq-len/--k-heads/--v-heads
           (C1 by default; C4 is --batch 1 --seq-len 65536 --v-heads 64).
  bwd      one chunk_gated_delta_rule_bwd call (the VJP: forward recompute, reverse state-
           gradient scan, chunk-parallel gradients) at the core workload's shape.
  layer_bwd one gdn_prefill_bwd call at C1 (the layer's VJP: conv, gates, rule, gated norm).
  layer_module the whole GatedDeltaNet layer at C1 with D=2048 (projection GEMMs included):
           a forward, and a training step (forward + gradients of every parameter and the
           input); the line's value is the training step's tokens/s.
  ab_proj  the gate projections in_proj_a, in_proj_b at C1 (D=2048, Hv=32) in one pass
           over the hidden rows (omx_gdn_ab_proj), with the two library GEMMs it replaces
           timed beside it.
  copy     a plain 256 MiB device copy, the calibration of the HBM traffic counters.

Every "roofline" object divides the algorithmic work of one timed call by that call's
own HIP-event time: the headline's is the C1 layer step whose tokens/s is `value`; the
core call's (the chunked rule alone: deltanet.py:53-153) is under "core".  "traffic" is
the HBM bytes one call moves, read from rocprofv3 FETCH_SIZE/WRITE_SIZE counters in the
run named by "traffic_source" (a profile constant: counters cannot be read inside this
process); null where no such run exists.  Only one GPU is used: --gpus above 1 exits
with a message.

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


def cpu_model():
    """The host CPU's model string (what lscpu prints as "Model name")."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


# ----------------------------------------------------------------------------- decode (C2)

def bench_decode(B, steps, warmup, cpu_baseline, min_rotation_bytes=512 << 20):
    """One cached decode step per call, rotating through distinct (inputs, conv cache,
    state) sets: at least 4 and at least ``min_rotation_bytes`` of state in total, so a
    step never finds its state in the 256 MB Infinity Cache, as in a multi-layer decode
    where each layer's state is read once per token."""
    import torch
    from omegalax_amd import gdn_decode_step, workloads as W
    Hk, Hv, d = 16, 32, 128
    _say(f"decode: B={B} generating inputs")
    arrs = W.decode_inputs(B)
    base = W.to_device(arrs)
    state_bytes = base["state"].numel() * 4
    n_sets = max(4, -(-min_rotation_bytes // state_bytes))
    gen = torch.Generator(device="cuda").manual_seed(1002)
    sets = [base]
    for _ in range(n_sets - 1):
        t = dict(base)
        t["state"] = 0.02 * torch.randn(base["state"].shape, generator=gen, device="cuda")
        for key in ("mixed_qkv", "z", "a", "b", "conv_state"):
            t[key] = torch.randn(base[key].shape, generator=gen, device="cuda").bfloat16()
        sets.append(t)
    dims = dict(num_k_heads=Hk, head_k_dim=d, num_v_heads=Hv, head_v_dim=d)
    it = [0]

    def step():
        t = sets[it[0] % n_sets]
        it[0] += 1
        gdn_decode_step(t["mixed_qkv"], t["z"], t["a"], t["b"], t["conv_w"], t["A_log"],
                        t["dt_bias"], t["norm_w"], t["conv_state"], t["state"], **dims)

    _say(f"decode: B={B} timing {steps} steps over {n_sets} state sets "
         f"({n_sets * state_bytes / 2**20:.0f} MiB)")
    wall, ms = time_launches(step, steps, warmup)
    nbytes = decode_bytes_per_seq(Hk, Hv, d, d) * B
    gbs = nbytes / (ms * 1e-3) / 1e9
    traffic = MEASURED_TRAFFIC.get(("decode", B, Hk, Hv, d))
    res = {
        "batch": B, "ms_per_step": wall / steps * 1e3, "kernel_ms": ms,
        "tokens_per_s": B * steps / wall, "state_sets": n_sets,
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": gbs / PEAK_HBM_GBS, "traffic": traffic and traffic[0],
                     "traffic_source": traffic and traffic[1], "algorithmic_bytes": nbytes},
    }
    if cpu_baseline:
        res["cpu_baseline"] = cpu_decode_baseline()
    return res


def cpu_decode_baseline(batches=(1, 8, 64), budget_s=4.0):
    """Oracle decode step (numpy fp64 restatement, the 'port') at C2's head layout, timed
    per batch size on whole steps while they fit ``budget_s`` (at least one step each).
    B=256 is not timed: its fp64 state alone is 1 GiB, and the step scales with the state
    it streams, so it is reported as B=64's rate (tokens/s per sequence are flat in B on
    this path, as the three timed sizes show)."""
    from oracle import gdn_oracle as O
    from omegalax_amd import workloads as W
    per_b = {}
    for B in batches:
        d = W.decode_inputs(B)
        S = d["state"].astype(np.float64)
        conv = d["conv_state"]
        n = 0
        t0 = time.perf_counter()
        while True:
            _, conv, S = O.gdn_decode_step(d["mixed_qkv"], d["z"], d["a"], d["b"], d["conv_w"],
                                           d["A_log"], d["dt_bias"], d["norm_w"], conv, S,
                                           Hk=16, dk=128, Hv=32, dv=128)
            n += 1
            el = time.perf_counter() - t0
            if el * (n + 1) / n > budget_s:
                break
        per_b[f"B={B}"] = {"tokens_per_s": B * n / el, "ms_per_step": el / n * 1e3, "steps": n}
    top = per_b[f"B={batches[-1]}"]
    return {"value": top["tokens_per_s"], "unit": "tokens/s", "cores": cpu_cores(),
            "cpu_model": cpu_model(), "kind": "port", "per_batch": per_b,
            "sample": f"whole decode steps of the numpy fp64 oracle (conv update, recurrent "
                      f"step, gated norm) at C2's head layout (Hk=16 Hv=32 d=128) for "
                      f"B in {list(batches)}, about {budget_s:.0f} s each; value is "
                      f"B={batches[-1]}'s"}


# ----------------------------------------------------------------------------- core call

# HBM bytes per call from two rocprofv3 --pmc runs (FETCH_SIZE x 2.0 and WRITE_SIZE x 1.0,
# scaled by a plain copy kernel's counters), for the shapes they were taken on, with the
# profiles/ summary that gives the commands and per-kernel figures.
MEASURED_TRAFFIC = {
    ("core", 4, 4096, 16, 32, 128): (1_153_999_872, "profiles/prefill_c1.md (core call)"),
    ("core", 1, 65536, 16, 64, 128): (7_707_787_264, "profiles/prefill_c3_c4.md (C4 core call)"),
    ("decode", 64, 16, 32, 128): (277_346_304, "profiles/decode_step_c2.md (B=64)"),
    ("decode", 256, 16, 32, 128): (1_108_210_688, "profiles/decode_step_c2.md (B=256)"),
    # layer step: prep 155.3 + 283.3 MiB, scan (with the gated norm) 546.6 + 136.0
    ("prefill", 4, 4096, 16, 32, 128): (1_175_575_552, "profiles/prefill_c1.md (layer kernels)"),
    ("c3", 32768, 8): (2_954_456_781, "profiles/prefill_c3_c4.md (C3 layer call)"),
    ("bwd", 4, 4096, 16, 32, 128): (6_873_572_192, "profiles/bwd_c1.md (backward call)"),
}


def bench_core(B, T, Hk, Hv, d, steps, warmup, arrs=None, long_memory=False):
    """One chunk_gated_delta_rule call (bf16 q/k/v, fp32 gates) over [B, T]: the
    chunk-parallel preparation kernel and the state scan, HIP-event timed.  Inputs are
    drawn on the device (seeded); ``long_memory`` draws C4's gates, e^g ~ U(0.9, 0.9999)."""
    import torch
    from omegalax_amd import chunk_gated_delta_rule, workloads as W
    gen = torch.Generator(device="cuda").manual_seed(7)
    act = lambda *shape: torch.randn(shape, generator=gen, device="cuda").bfloat16()
    q, k, v = act(B, T, Hk, d), act(B, T, Hk, d), act(B, T, Hv, d)
    if arrs is not None:
        g32, beta32 = W.gates_f32(arrs["a"], arrs["b"], arrs["A_log"], arrs["dt_bias"])
        g = torch.from_numpy(g32).cuda()
        beta = torch.from_numpy(beta32).cuda()
    elif long_memory:
        g = torch.log(0.9 + 0.0999 * torch.rand((B, T, Hv), generator=gen, device="cuda"))
        beta = torch.sigmoid(torch.randn((B, T, Hv), generator=gen, device="cuda")).bfloat16().float()
    else:
        a = torch.randn((B, T, Hv), generator=gen, device="cuda")
        A_log = torch.log(1 + 15 * torch.rand(Hv, generator=gen, device="cuda"))
        dt = -2 * torch.rand(Hv, generator=gen, device="cuda")
        g = -torch.exp(A_log) * torch.nn.functional.softplus(a + dt)
        beta = torch.sigmoid(torch.randn((B, T, Hv), generator=gen, device="cuda")).bfloat16().float()

    def core():
        chunk_gated_delta_rule(q, k, v, g, beta, C)

    _say(f"core: B={B} T={T} Hk={Hk} Hv={Hv} timing {steps} launches")
    wall, ms = time_launches(core, steps, warmup)
    flops = prefill_flops_per_token_head(d, d) * B * T * Hv
    tf = flops / (ms * 1e-3) / 1e12
    traffic = MEASURED_TRAFFIC.get(("core", B, T, Hk, Hv, d))
    return {
        "config": f"chunk_gated_delta_rule B={B} T={T} Hk={Hk} Hv={Hv} d={d}",
        "ms_per_step": wall / steps * 1e3, "kernel_ms": ms,
        "tokens_per_s": B * T * steps / wall,
        "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": tf / PEAK_BF16_TFLOPS,
                     "traffic": traffic and traffic[0], "traffic_source": traffic and traffic[1],
                     "algorithmic_flops": flops,
                     "kernels": "the launches of one chunk_gated_delta_rule call"},
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
    traffic = MEASURED_TRAFFIC.get(("bwd", B, T, Hk, Hv, d))
    return {
        "ms_per_step": wall / steps * 1e3, "kernel_ms": ms,
        "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": tf / PEAK_BF16_TFLOPS,
                     "traffic": traffic and traffic[0], "traffic_source": traffic and traffic[1],
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
    """C1: one gdn_prefill call (projection outputs -> gated-norm output) per step; the
    roofline divides the step's algorithmic FLOPs (the chunked rule's matmuls, 94.49 GFLOP)
    by the step's own HIP-event time.  The core call on the same shapes is timed after it
    and reported under its own key."""
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
    flops = prefill_flops_per_token_head(d, d) * tokens * Hv
    tf = flops / (ms_step * 1e-3) / 1e12
    traffic = MEASURED_TRAFFIC.get(("prefill", B, T, Hk, Hv, d))
    res = {
        "tokens_per_s": tokens * steps / wall, "ms_per_step": wall / steps * 1e3,
        "step_event_ms": ms_step,
        "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": tf / PEAK_BF16_TFLOPS,
                     "traffic": traffic and traffic[0], "traffic_source": traffic and traffic[1],
                     "algorithmic_flops": flops,
                     "kernels": "the launches of one gdn_prefill call (the whole layer step)"},
        "core": bench_core(B, T, Hk, Hv, d, steps, warmup, arrs),
    }
    del t
    if cpu_baseline:
        res["cpu_baseline"] = cpu_prefill_baseline()
    return res


def bench_c3(steps, warmup, total=32768, n=8):
    """C3: packed layer prefill, ``n`` sequences (seeded Dirichlet lengths, minimum 256) in
    one row of ``total`` tokens, each from its own initial state, final states returned.
    Inputs are drawn on the device; cu_seqlens is a device tensor."""
    import torch
    from omegalax_amd import gdn_prefill, workloads as W
    Hk, Hv, d = 16, 32, 128
    lens = W.varlen_lengths(total, n)
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)).cuda()
    p = W.layer_params(np.random.default_rng(1010), Hk, Hv, d, d)
    p = {k_: torch.from_numpy(v_).cuda() for k_, v_ in p.items()}
    gen = torch.Generator(device="cuda").manual_seed(1003)
    conv_dim = 2 * Hk * d + Hv * d
    x = torch.randn((1, total, conv_dim), generator=gen, device="cuda").bfloat16()
    z = torch.randn((1, total, Hv, d), generator=gen, device="cuda").bfloat16()
    a = torch.randn((1, total, Hv), generator=gen, device="cuda").bfloat16()
    b = torch.randn((1, total, Hv), generator=gen, device="cuda").bfloat16()
    s0 = 0.02 * torch.randn((n, Hv, d, d), generator=gen, device="cuda")
    dims = dict(num_k_heads=Hk, head_k_dim=d, num_v_heads=Hv, head_v_dim=d)

    def step():
        gdn_prefill(x, z, a, b, p["conv_w"], p["A_log"], p["dt_bias"], p["norm_w"],
                    cu_seqlens=cu, initial_state=s0, output_final_state=True, **dims)

    _say(f"c3: T={total} in {n} packed sequences (longest {int(lens.max())}), timing {steps} steps")
    wall, ms = time_launches(step, steps, warmup)
    flops = prefill_flops_per_token_head(d, d) * total * Hv
    tf = flops / (ms * 1e-3) / 1e12
    traffic = MEASURED_TRAFFIC.get(("c3", total, n))
    return {"config": f"C3 packed layer prefill T={total}, {n} sequences "
                      f"(lengths {lens.tolist()}), initial states, Hk=16 Hv=32 d=128",
            "ms_per_step": wall / steps * 1e3, "kernel_ms": ms,
            "tokens_per_s": total * steps / wall,
            "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": tf / PEAK_BF16_TFLOPS,
                         "traffic": traffic and traffic[0], "traffic_source": traffic and traffic[1],
                         "algorithmic_flops": flops,
                         "kernels": "the launches of one gdn_prefill call"}}


def cpu_prefill_baseline(T=4096, budget_s=20.0):
    """Oracle layer prefill (numpy restatement, fp32 core like the reference; numpy's BLAS
    uses the visible cores) on a bounded C1 sample: one of C1's four sequences, B=1 T=4096
    in the C1 head layout.  C1's sequences are independent, so C1 takes four times the
    sample's time on this path: the tokens/s rate is the same."""
    from oracle import gdn_oracle as O
    from omegalax_amd import workloads as W
    B = 1
    d = W.layer_inputs(B, T)
    n = 0
    t0 = time.perf_counter()
    while True:  # whole runs only, while the next one still fits the budget
        O.gdn_prefill_layer(d["mixed_qkv"], d["z"], d["a"], d["b"], d["conv_w"], d["A_log"],
                            d["dt_bias"], d["norm_w"], Hk=16, dk=128, Hv=32, dv=128,
                            dtype=np.float32)
        n += 1
        el = time.perf_counter() - t0
        if el * (n + 1) / n > budget_s:
            break
    return {"value": B * T * n / el, "unit": "tokens/s", "cores": cpu_cores(),
            "cpu_model": cpu_model(), "kind": "port",
            "sample": f"{n} run(s) of the numpy fp32 layer prefill restatement on one C1 "
                      f"sequence (B=1 T={T}, Hk=16 Hv=32 d=128); C1 (4 such sequences) "
                      f"extrapolates to {4 * el / n:.1f} s at the same tokens/s"}


def bench_ab_proj(steps, warmup):
    """The gate projections a = in_proj_a(h), b = in_proj_b(h) at C1 (D=2048, Hv=32,
    deltanet.py:240-241): the one-pass kernel against the two library GEMMs it replaces."""
    import torch
    from omegalax_amd import gdn_ab_projections
    F = torch.nn.functional
    g = torch.Generator(device="cuda").manual_seed(1001)
    M, D, Hv = 4 * 4096, 2048, 32
    h = torch.randn(M, D, generator=g, device="cuda").bfloat16()
    wa, wb = ((0.02 * torch.randn(Hv, D, generator=g, device="cuda")).bfloat16()
              for _ in range(2))
    wall, ms = time_launches(lambda: gdn_ab_projections(h, wa, wb), steps, warmup)
    _, ms_lib = time_launches(lambda: (F.linear(h, wa), F.linear(h, wb)), steps, warmup)
    gbs = (M * D + 2 * Hv * D + 2 * M * Hv) * 2 / (ms * 1e-3) / 1e9
    return {"config": f"in_proj_a + in_proj_b, M={M} D={D} Hv={Hv}",
            "ms_per_step": wall / steps * 1e3, "kernel_ms": ms, "two_library_gemms_ms": ms_lib,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gbs / PEAK_HBM_GBS}}


def bench_qkv_conv(steps, warmup):
    """in_proj_qkv at C1 (M = 4 x 4096 tokens, D=2048, N = conv_dim = 8192,
    deltanet.py:234) three ways: the library GEMM (F.linear, hipBLASLt) the layer uses,
    the library's own GEMM kernel (omx_gdn_qkv_conv_proj, conv = 0), and that kernel with
    the causal conv + SiLU (deltanet.py:243) in its epilogue (conv = 1): the prototype of
    the projection-side fusion, measured against the GEMM it would replace."""
    import torch
    from omegalax_amd import qkv_conv_projection
    F = torch.nn.functional
    g = torch.Generator(device="cuda").manual_seed(1002)
    B, T, D, N = 4, 4096, 2048, 8192
    x = torch.randn(B, T, D, generator=g, device="cuda").bfloat16()
    w = (torch.randn(N, D, generator=g, device="cuda") / D ** 0.5).bfloat16()
    cw = (0.5 * torch.randn(N, 4, generator=g, device="cuda")).float()
    _, ms_lib = time_launches(lambda: F.linear(x, w), steps, warmup)
    _, ms_own = time_launches(lambda: qkv_conv_projection(x, w), steps, warmup)
    wall, ms_fused = time_launches(lambda: qkv_conv_projection(x, w, cw), steps, warmup)
    flops = 2.0 * B * T * D * N
    tf = lambda ms: flops / (ms * 1e-3) / 1e12
    return {"config": f"in_proj_qkv M={B * T} D={D} N={N}, conv K=4 over sequences of {T}",
            "library_gemm_ms": ms_lib, "own_gemm_ms": ms_own, "fused_gemm_conv_ms": ms_fused,
            "ms_per_step": wall / steps * 1e3,
            "tflops": {"library_gemm": tf(ms_lib), "own_gemm": tf(ms_own),
                       "fused_gemm_conv": tf(ms_fused)},
            "roofline": {"bound": "mfma", "achieved": tf(ms_fused), "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": tf(ms_fused) / PEAK_BF16_TFLOPS}}


def _line(metric, value, unit, steps, warmup, ms, dtype, config, **extra):
    line = {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": steps,
            "warmup": warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": dtype,
            "data": "synthetic (seeded N(0,1) activations, random-init params)",
            "config": config}
    line.update(extra)
    return json.dumps(line)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=["prefill", "c1", "decode", "c3", "core", "bwd",
                                           "layer_bwd", "layer_module", "copy", "ab_proj",
                                           "qkv_conv"],
                    default="prefill")
    ap.add_argument("--decode-batch", type=int, default=64)
    ap.add_argument("--batch", type=int, default=4, help="core workload: sequences")
    ap.add_argument("--seq-len", type=int, default=4096, help="core workload: tokens each")
    ap.add_argument("--k-heads", type=int, default=16, help="core workload")
    ap.add_argument("--v-heads", type=int, default=32, help="core workload")
    ap.add_argument("--long-memory", action="store_true",
                    help="core workload: C4's gates, e^g ~ U(0.9, 0.9999)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the GDN path shards by sequence and value-head group with no exchange, so one "
              "GPU's throughput is one shard's)",
              file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    cpu = not args.no_cpu_baseline
    K, W_ = args.steps, args.warmup
    if args.workload == "copy":
        # calibration of the FETCH_SIZE / WRITE_SIZE counters: a plain 256 MiB device copy
        src = torch.empty(1 << 26, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        wall, ms = time_launches(lambda: dst.copy_(src), K, W_)
        gbs = 2 * src.numel() * 4 / (ms * 1e-3) / 1e9
        print(_line("device copy GB/s (counter calibration)", gbs, "GB/s", K, W_,
                    wall / K * 1e3, "f32", {"workload": "256 MiB read + 256 MiB written"}),
              flush=True)
        return 0
    if args.workload == "ab_proj":
        res = bench_ab_proj(K, W_)
        print(_line("gate projections HBM GB/s (one pass over the hidden rows, config C1)",
                    res["roofline"]["achieved"], "GB/s", K, W_, res["ms_per_step"], "bf16",
                    {"workload": res["config"]}, kernel_ms=res["kernel_ms"],
                    two_library_gemms_ms=res["two_library_gemms_ms"], roofline=res["roofline"]),
              flush=True)
        return 0
    if args.workload == "qkv_conv":
        res = bench_qkv_conv(K, W_)
        print(_line("in_proj_qkv + conv TFLOP/s (prototype epilogue fusion, config C1)",
                    res["roofline"]["achieved"], "TFLOP/s", K, W_, res["ms_per_step"], "bf16",
                    {"workload": res["config"]}, qkv_conv=res, roofline=res["roofline"]),
              flush=True)
        return 0
    if args.workload == "layer_module":
        res = bench_layer_module(K, W_)
        n_t = max(K // 2, 5)
        print(_line("GatedDeltaNet training-step tokens/s (projections included, config C1)",
                    res["train_tokens_per_s"], "tokens/s", n_t, W_, res["train_step_ms"],
                    "bf16", {"workload": res["config"]}, layer_module=res), flush=True)
        return 0
    if args.workload == "layer_bwd":
        res = bench_layer_bwd(K, W_)
        print(_line("gdn_prefill_bwd tokens/s (GDN layer backward, config C1)",
                    res["tokens_per_s"], "tokens/s", K, W_, res["ms_per_step"], "bf16",
                    {"workload": "C1 GDN layer backward B=4 T=4096 Hk=16 Hv=32 d=128"},
                    kernel_ms=res["kernel_ms"]), flush=True)
        return 0
    if args.workload == "bwd":
        B, T, Hk, Hv = args.batch, args.seq_len, args.k_heads, args.v_heads
        res = bench_bwd(B, T, Hk, Hv, 128, K, W_)
        print(_line("chunk_gated_delta_rule_bwd TFLOP/s (bf16 MFMA roofline)",
                    res["roofline"]["achieved"], "TFLOP/s", K, W_, res["ms_per_step"], "bf16",
                    {"workload": f"chunk_gated_delta_rule_bwd B={B} T={T} Hk={Hk} Hv={Hv} d=128",
                     "chunk": C}, roofline=res["roofline"], kernel_ms=res["kernel_ms"]),
              flush=True)
        return 0
    if args.workload == "core":
        B, T, Hk, Hv = args.batch, args.seq_len, args.k_heads, args.v_heads
        core = bench_core(B, T, Hk, Hv, 128, K, W_, long_memory=args.long_memory)
        print(_line("chunk_gated_delta_rule TFLOP/s (bf16 MFMA roofline)",
                    core["roofline"]["achieved"], "TFLOP/s", K, W_, core["ms_per_step"], "bf16",
                    {"workload": core["config"], "chunk": C}, roofline=core["roofline"],
                    kernel_ms=core["kernel_ms"]), flush=True)
        return 0
    if args.workload == "c1":
        pre = bench_prefill(K, W_, cpu)
        extra = {"roofline": pre["roofline"], "step_event_ms": pre["step_event_ms"],
                 "core": {k_: pre["core"][k_] for k_ in ("config", "kernel_ms", "roofline")}}
        if cpu:
            extra["cpu_baseline"] = pre["cpu_baseline"]
        print(_line("C1 GDN layer prefill tokens/s", pre["tokens_per_s"], "tokens/s", K, W_,
                    pre["ms_per_step"], "bf16",
                    {"workload": "C1 GDN layer prefill B=4 T=4096 Hk=16 Hv=32 d=128"}, **extra),
              flush=True)
        return 0
    if args.workload == "c3":
        res = bench_c3(K, W_)
        print(_line("C3 packed GDN layer prefill tokens/s", res["tokens_per_s"], "tokens/s", K,
                    W_, res["ms_per_step"], "bf16", {"workload": res["config"]},
                    roofline=res["roofline"], kernel_ms=res["kernel_ms"]), flush=True)
        return 0
    if args.workload == "decode":
        dec = bench_decode(args.decode_batch, K, W_, cpu)
        extra = {"roofline": dec["roofline"], "decode": dec}
        if cpu:
            extra["cpu_baseline"] = dec.pop("cpu_baseline")
        print(_line("decode-step HBM GB/s (GDN decode, config C2)", dec["roofline"]["achieved"],
                    "GB/s", K, W_, dec["ms_per_step"], "f32",
                    {"workload": f"C2 decode step B={args.decode_batch} Hk=16 Hv=32 d=128"},
                    **extra), flush=True)
        return 0
    # the headline: C1 layer prefill, with every other config under its own key
    pre = bench_prefill(K, W_, cpu)
    c3 = bench_c3(max(K // 2, 5), W_)
    c4 = bench_core(1, 65536, 16, 64, 128, max(K // 4, 3), min(W_, 2), long_memory=True)
    dec1 = bench_decode(1, max(K, 20), W_, False)
    dec8 = bench_decode(8, max(K, 20), W_, False)
    dec64 = bench_decode(64, max(K, 20), W_, False)
    dec256 = bench_decode(256, max(K, 20), W_, False)
    bwd = bench_bwd(4, 4096, 16, 32, 128, max(K // 2, 5), W_)
    lbwd = bench_layer_bwd(max(K // 2, 5), W_)
    mod = bench_layer_module(K, W_)
    abp = bench_ab_proj(max(K, 20), W_)
    qkv = bench_qkv_conv(max(K // 2, 5), W_)
    dec = lambda r: {"config": f"C2 B={r['batch']} (state rotated over {r['state_sets']} sets)",
                     "roofline": r["roofline"], "kernel_ms": r["kernel_ms"],
                     "tokens_per_s": r["tokens_per_s"]}
    extra = {
        "roofline": pre["roofline"],
        "core": {k_: pre["core"][k_] for k_ in ("config", "kernel_ms", "roofline")},
        "prefill_detail": {"step_event_ms": pre["step_event_ms"]},
        "c3": c3,
        "c4": {"config": "C4 core call B=1 T=65536 Hk=16 Hv=64 d=128, e^g ~ U(0.9, 0.9999)",
               "kernel_ms": c4["kernel_ms"], "tokens_per_s": c4["tokens_per_s"],
               "roofline": c4["roofline"]},
        "decode": dec(dec64),
        "decode_b256": dec(dec256),
        "decode_b1": dec(dec1),
        "decode_b8": dec(dec8),
        "backward": {"config": "chunk_gated_delta_rule_bwd at C1 (B=4 T=4096 Hk=16 Hv=32 d=128)",
                     "kernel_ms": bwd["kernel_ms"], "roofline": bwd["roofline"]},
        "layer_backward": {"config": "gdn_prefill_bwd at C1", "kernel_ms": lbwd["kernel_ms"],
                           "tokens_per_s": lbwd["tokens_per_s"]},
        "layer_module": mod,
        "gate_projections": abp,
        "qkv_conv_fusion": qkv,
    }
    if cpu:
        extra["cpu_baseline"] = pre["cpu_baseline"]
        extra["decode_cpu_baseline"] = cpu_decode_baseline()
    print(_line("GDN prefill tokens/s + %MFMA peak; decode-step HBM GB/s + %of 8 TB/s",
                pre["tokens_per_s"], "tokens/s", K, W_, pre["ms_per_step"], "bf16",
                {"workload": "C1 GDN layer prefill (projection outputs -> gated-norm output)",
                 "batch": 4, "seq_len": 4096, "k_heads": 16, "v_heads": 32, "head_dim": 128,
                 "chunk": 64}, **extra), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
