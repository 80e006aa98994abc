"""Headline benchmark: Qwen3-8B-shape int4 (Q4_K) greedy decode at batch 1 on one MI355X.

Workload: 36 layers, hidden 4096, MLP 12288, 32 q / 8 kv heads,
head_dim 128, vocab 151936, seeded N(0, 0.02) weights quantized to Q4_K on the GPU, bf16 KV cache
prefilled to 4096 positions with N(0, 1) values, then K timed greedy decode steps (default 256).

A step is one full token: embed, 36 layers, final norm + LM head + argmax, token store, all in HIP
graphs (8 steps per graph).  value = tokens/s over the timed steps.

roofline: the dominant kernel (fused RMSNorm + gate|up GEMV + SwiGLU) timed live with HIP events on
the stream a HIP graph of its 36 launches (one per layer, 2 GB of weights, well above the 256 MB
MALL) is replayed on; achieved = algorithmic bytes per launch / average launch time; traffic = HBM
bytes per launch from the committed FETCH_SIZE/WRITE_SIZE counter summary under profiles/.

cpu_baseline: the CPU oracle's Qwen3 decoder (oracle.reference.Qwen3CpuModel, dense fp32 weights
dequantized by the oracle) on a bounded sample of the same workload, scaled to tokens/s.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

HBM_PEAK_GBS = 8000.0
HEADLINE_METRIC = "Qwen3-8B-shape int4 decode tok/s @bs1; q-matmul HBM GB/s vs ~8 TB/s peak"
PROFILES = Path(__file__).resolve().parent / "profiles"
# HBM traffic of the dominant kernel (two rocprofv3 --pmc passes), per decode path
TRAFFIC_PROFILES = {
    "decode_layers_persistent": PROFILES / "decode_layers_qwen3_8b_int4_kv4096_pmc.md",
    "gate_up_rmsnorm_swiglu_gemv": PROFILES / "gate_up_gemv_qwen3_8b_pmc.md",
}
PROMPT_POSITIONS = 4096


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=256)
    p.add_argument("--warmup", type=int, default=16)
    p.add_argument("--steps-per-graph", type=int, default=8)
    p.add_argument("--model", choices=("8b", "0.6b"), default="8b")
    p.add_argument("--policy", choices=("uniform", "q4_k_m"), default="uniform",
                   help="weight types: uniform Q4_K (the headline int4 config) or the Q4_K_M mix")
    p.add_argument("--positions", type=int, default=PROMPT_POSITIONS, help="KV positions prefilled before timing")
    p.add_argument("--kernel-reps", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-sample-steps", type=int, default=3)
    p.add_argument("--no-graph", action="store_true")
    p.add_argument("--per-op", action="store_true",
                   help="one launch per op instead of the persistent layers kernel (t2h_qwen3_decode_layers)")
    p.add_argument("--profile-kernel", action="store_true",
                   help="counter-collection target: run the dominant kernel (the persistent layers kernel, or "
                        "with --per-op the gate|up GEMV over all layers) plus a 256 MiB copy (the calibration for "
                        "FETCH_SIZE/WRITE_SIZE), no timing, no JSON line")
    return p.parse_args()


def profile_kernel_target(per_op: bool) -> int:
    """Launch sequence for `rocprofv3 --pmc FETCH_SIZE|WRITE_SIZE`: the dominant kernel twice over all
    layers (the persistent layers kernel at KV 4096, 2 dispatches; or, per op, the gate|up GEMV once per
    layer, 72 dispatches), then one plain 256 MiB device copy whose traffic is known (256 MiB read + 256 MiB
    written), so counter readings can be scaled to bytes."""
    import torch

    from torch2vk_amd import kernels
    from torch2vk_amd.qwen3.config import QWEN3_8B
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.qwen3.weights import synthetic_weights

    dev = torch.device("cuda:0")
    w = synthetic_weights(QWEN3_8B, device=dev, seed=0)
    if per_op:
        dec = Qwen3Decoder(w, max_positions=64, max_new_tokens=4, device=dev, persistent=False)
        dec.h.normal_()
        for _ in range(2):
            for i in range(QWEN3_8B.layers):
                kernels.q4k_rmsnorm_swiglu(dec.h, w.norms[f"layers.{i}.post_norm"], w.packed[f"layers.{i}.gate"],
                                           w.packed[f"layers.{i}.up"], dec.act)
    else:
        dec = Qwen3Decoder(w, max_positions=PROMPT_POSITIONS + 64, max_new_tokens=4, device=dev, persistent=True)
        gen = torch.Generator(device=dev)
        gen.manual_seed(1)
        dec.k_cache[:, :PROMPT_POSITIONS].normal_(generator=gen)
        dec.v_cache[:, :PROMPT_POSITIONS].normal_(generator=gen)
        dec.h.normal_()
        dec.position.fill_(PROMPT_POSITIONS)
        for _ in range(2):
            dec.run_decode_layers()
        dec.check_status()
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    print("[bench] profile-kernel target done", file=sys.stderr, flush=True)
    return 0


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build is single-GPU); got --gpus {args.gpus}", file=sys.stderr)
        return 2
    if args.profile_kernel:
        return profile_kernel_target(args.per_op)
    import torch

    from torch2vk_amd import kernels
    from torch2vk_amd.qwen3.config import QWEN3_0_6B, QWEN3_8B
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.qwen3.weights import synthetic_weights

    if not torch.cuda.is_available():
        print("no HIP device", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    cfg = QWEN3_8B if args.model == "8b" else QWEN3_0_6B
    t_setup = time.time()
    weights = synthetic_weights(cfg, device=dev, seed=0, policy=args.policy)
    total_steps = args.warmup + args.steps + args.steps_per_graph
    s_cap = args.positions + total_steps + 64
    dec = Qwen3Decoder(weights, max_positions=s_cap, max_new_tokens=total_steps + 8, device=dev,
                       persistent=False if args.per_op else None)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    for layer in range(cfg.layers):
        dec.k_cache[layer, :args.positions].normal_(generator=gen)
        dec.v_cache[layer, :args.positions].normal_(generator=gen)
    first_token = int(torch.randint(0, cfg.vocab, (1,), generator=gen, device=dev).item())
    dec.reset(position=args.positions, token=first_token)
    dec.stop_on_eos = False
    torch.cuda.synchronize()
    print(f"[bench] setup {time.time() - t_setup:.1f}s: {cfg.name} packed weights "
          f"{weights.packed_bytes() / 1e9:.3f} GB, KV capacity {s_cap}", file=sys.stderr, flush=True)

    use_graph = not args.no_graph
    spg = args.steps_per_graph
    if use_graph:
        dec.graph(spg)
    dec.run_steps(args.warmup, steps_per_graph=spg, use_graph=use_graph)
    torch.cuda.synchronize()
    print(f"[bench] warmup {args.warmup} steps done", file=sys.stderr, flush=True)

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dec.run_steps(args.steps, steps_per_graph=spg, use_graph=use_graph)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    elapsed = t1 - t0
    tok_s = args.steps / elapsed
    ms_per_step = elapsed * 1000.0 / args.steps
    n_generated = int(dec.length.item())
    print(f"[bench] timed {args.steps} steps: {ms_per_step:.3f} ms/token, {tok_s:.1f} tok/s "
          f"({n_generated} tokens stored)", file=sys.stderr, flush=True)

    kern = kernel_timing(dec, weights, args.kernel_reps)
    print(f"[bench] kernel timing: {json.dumps(kern['per_launch_us'])}", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(cfg, weights, args.positions, args.cpu_sample_steps)
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)

    dom = kern["dominant"]
    headline = args.model == "8b" and args.policy == "uniform"
    policy_text = "Q4_K uniform int4" if args.policy == "uniform" else "Q4_K_M (Q4_K + Q6_K)"
    line = {
        "metric": HEADLINE_METRIC if headline else f"Qwen3-{args.model.upper()}-shape {args.policy} decode tok/s @bs1",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": f"synthetic (seeded N(0,0.02) weights quantized on the GPU, {policy_text}; KV cache N(0,1))",
        "config": {
            "workload": f"{cfg.name}-shape {policy_text} greedy decode, batch 1, KV prefilled to "
                        f"{args.positions} positions, {args.steps} timed steps"
                        + (f", HIP graphs of {spg} steps" if use_graph else ", eager launches")
                        + (", persistent layers kernel" if dec.persistent else ", one launch per op"),
            "layers_launch": "persistent" if dec.persistent else "per-op",
            "weights": args.policy,
            "kv_positions": args.positions,
            "batch": 1,
            "graph_steps": spg if use_graph else 0,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dom["kernel"],
            "achieved": round(dom["gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4),
            "traffic": profiled_traffic(TRAFFIC_PROFILES[dom["kernel"]]) if headline else None,
            "traffic_source": TRAFFIC_PROFILES[dom["kernel"]].name if headline else None,
            "bytes_per_launch": dom["bytes"],
            "avg_launch_us": round(dom["us"], 3),
        },
        "qmatmul_gbs": round(kern["qmatmul_gbs"], 1),
        "kernel_us_per_token": round(kern["us_per_token"], 1),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def _graph_us_per_call(calls, reps: int) -> float:
    """Average duration of one call in `calls` when they run back to back inside a HIP graph, the way
    the decode step runs them.  Timed with HIP events on the stream the graph is replayed on."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):                      # warm outside capture
        for f in calls:
            f()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for f in calls:
            f()
    stream = torch.cuda.current_stream()
    graph.replay()
    stream.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        graph.replay()
    end.record(stream)
    end.synchronize()
    us = start.elapsed_time(end) * 1000.0 / (reps * len(calls))
    del graph
    return us


def kernel_timing(dec, weights, reps: int) -> dict:
    """Per-launch timing of each decode kernel class: each class's launches over all layers' weights
    captured in one HIP graph (as in the decode step, so launch gaps match it) and replayed `reps` times."""
    c = dec.config
    L = c.layers
    wb = lambda n: weights.packed[n].numel()  # noqa: E731
    pos = int(dec.position.item())
    kv_len = min(pos + 1, dec.max_positions)
    # algorithmic bytes per launch: packed weights + activations read + outputs written.  Each class
    # runs through the decoder's own sub-step, so the GEMV of each tensor's type is the one timed.
    classes = {
        "qkv_rmsnorm_gemv": (
            dec._qkv,
            lambda i: wb(f"layers.{i}.q") + wb(f"layers.{i}.k") + wb(f"layers.{i}.v") + c.hidden * 8
            + (c.q_dim + 2 * c.kv_dim) * 4),
        "attn_decode": (
            dec._attention,
            lambda i: 2 * kv_len * c.kv_dim * 2 + (c.q_dim + 2 * c.kv_dim) * 4 + c.q_dim * 2),
        "o_gemv_residual": (
            lambda i: dec._linear_residual(dec.attn, f"layers.{i}.o"),
            lambda i: wb(f"layers.{i}.o") + c.q_dim * 2 + c.hidden * 8),
        "gate_up_rmsnorm_swiglu_gemv": (
            dec._gate_up,
            lambda i: wb(f"layers.{i}.gate") + wb(f"layers.{i}.up") + c.hidden * 8 + c.mlp * 2),
        "down_gemv_residual": (
            lambda i: dec._linear_residual(dec.act, f"layers.{i}.down"),
            lambda i: wb(f"layers.{i}.down") + c.mlp * 2 + c.hidden * 8),
    }
    per_launch_us, gbs, bytes_per = {}, {}, {}
    total_us = q_bytes = q_us = 0.0
    for name, (fn, nbytes) in classes.items():
        us = _graph_us_per_call([lambda i=i: fn(i) for i in range(L)], reps)
        b = sum(nbytes(i) for i in range(L)) / L
        per_launch_us[name] = round(us, 3)
        bytes_per[name] = int(b)
        gbs[name] = b / (us * 1e-6) / 1e9
        total_us += us * L
        if name != "attn_decode":
            q_bytes += b * L
            q_us += us * L
    # LM head (fused final norm + GEMV + per-block argmax)
    name = "lm_head_rmsnorm_argmax_gemv"
    us = _graph_us_per_call([dec._lm_head] * 4, reps)
    b = wb("lm_head") + c.hidden * 8 + dec.partial_scores.numel() * 8
    per_launch_us[name] = round(us, 3)
    bytes_per[name] = int(b)
    gbs[name] = b / (us * 1e-6) / 1e9
    total_us += us
    q_bytes += b
    q_us += us
    dominant = "gate_up_rmsnorm_swiglu_gemv"
    if dec.persistent:
        # the launch that runs every layer of a token: each layer's weights and norms, the K/V rows read
        # and the new row written, the residual stream in and out
        name = "decode_layers_persistent"
        us = _graph_us_per_call([dec.run_decode_layers] * 2, reps)
        b = 0
        for i in range(L):
            b += sum(wb(f"layers.{i}.{n}") for n in ("q", "k", "v", "o", "gate", "up", "down"))
            b += sum(weights.norms[f"layers.{i}.{n}"].numel() * 4 for n in ("input_norm", "post_norm", "q_norm",
                                                                              "k_norm"))
        b += L * (2 * kv_len * c.kv_dim * 2 + 2 * c.kv_dim * 2) + 2 * c.hidden * 4
        per_launch_us[name] = round(us, 3)
        bytes_per[name] = int(b)
        gbs[name] = b / (us * 1e-6) / 1e9
        dominant = name
        # what a token runs: this launch and the LM head (the per-op classes above are for comparison)
        lm = "lm_head_rmsnorm_argmax_gemv"
        total_us = us + per_launch_us[lm]
        q_bytes = b + bytes_per[lm]
        q_us = total_us
    return {
        "per_launch_us": per_launch_us,
        "gbs": {k: round(v, 1) for k, v in gbs.items()},
        "bytes": bytes_per,
        "us_per_token": total_us,
        "qmatmul_gbs": q_bytes / (q_us * 1e-6) / 1e9,
        "dominant": {"kernel": dominant, "us": per_launch_us[dominant], "bytes": bytes_per[dominant],
                     "gbs": gbs[dominant]},
    }


def profiled_traffic(profile: Path) -> int | None:
    """HBM bytes per launch of the dominant kernel, from the committed counter summary (two
    rocprofv3 --pmc passes, FETCH_SIZE and WRITE_SIZE, scaled by a 256 MiB copy's readings)."""
    try:
        text = profile.read_text()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", text, re.M)
    return int(m.group(1)) if m else None


def cpu_baseline(cfg, weights, positions: int, steps: int) -> dict:
    """The CPU oracle's decoder on one layer + the LM head at full 8B shapes, scaled to a token."""
    import numpy as np
    import torch

    import oracle
    from oracle.reference import Qwen3CpuModel, Qwen3Shape

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    c = cfg
    dense = {}
    for name in ("q", "k", "v", "o", "gate", "up", "down"):
        packed = weights.packed[f"layers.0.{name}"].cpu().numpy()
        k = c.hidden if name != "o" and name != "down" else (c.q_dim if name == "o" else c.mlp)
        dense[f"layers.0.{name}"] = torch.from_numpy(getattr(oracle, f"dequant_{weights.types[f'layers.0.{name}']}")(
            packed, k))
    for name in ("input_norm", "post_norm", "q_norm", "k_norm"):
        dense[f"layers.0.{name}"] = weights.norms[f"layers.0.{name}"].cpu()
    dense["norm"] = weights.norms["norm"].cpu()
    dense["embed"] = torch.zeros(8, c.hidden)
    lm = torch.from_numpy(getattr(oracle, f"dequant_{weights.types['lm_head']}")(
        weights.packed["lm_head"].cpu().numpy(), c.hidden))
    dense["lm_head"] = lm
    shape = Qwen3Shape(hidden=c.hidden, layers=1, heads=c.heads, kv_heads=c.kv_heads, head_dim=c.head_dim,
                       mlp=c.mlp, vocab=c.vocab, rope_theta=c.rope_theta)
    model = Qwen3CpuModel(shape, dense, max_positions=positions + steps + 1)
    g = torch.Generator().manual_seed(1)
    model.k_cache[:, :positions].normal_(generator=g)
    model.v_cache[:, :positions].normal_(generator=g)
    layer_times = []
    for s in range(steps):
        t0 = time.perf_counter()
        hidden = model.forward(torch.tensor([s % 8]), start=positions + s)
        layer_times.append(time.perf_counter() - t0)
    lm_times = []
    for _ in range(2):
        t0 = time.perf_counter()
        logits = model.logits(hidden)
        int(torch.argmax(logits))
        lm_times.append(time.perf_counter() - t0)
    t_layer = statistics.median(layer_times)
    t_lm = statistics.median(lm_times)
    t_token = c.layers * t_layer + t_lm
    del np
    return {
        "value": round(1.0 / t_token, 4),
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "sample": f"CPU oracle decoder (torch {torch.__version__}, fp32 dense weights dequantized by the oracle): "
                  f"1 of {c.layers} layers at KV position {positions} timed over {steps} steps (median "
                  f"{t_layer * 1e3:.1f} ms) x {c.layers} + LM head+argmax (median {t_lm * 1e3:.1f} ms)",
    }


if __name__ == "__main__":
    sys.exit(main())
