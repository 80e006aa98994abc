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
    "prefill_gate_up_gemm": PROFILES / "gemm_swiglu_q8_0_m16384_pmc.md",
    "asr_decode_layers_0_6b": PROFILES / "decode_layers_qwen3_0_6b_x4_int4_kv1540_pmc.md",
}
PROMPT_POSITIONS = 4096


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--config", choices=("decode", "prefill", "asr", "linear"), default="decode",
                   help="decode: BASELINE configs[2], the headline (default; with --model 0.6b, configs[1]: a "
                        "128-token prompt through the chunked prefill, then 128 greedy tokens); prefill: configs[3], "
                        "8 x 2048 tokens through the 36-layer 8B shape with Q8_0 weights; asr: configs[4], the "
                        "24-layer encoder over 4 x 1500 frames then a 0.6B-shape int4 decoder for 64 tokens per "
                        "utterance; linear: configs[0], one Q4_K linear x[1,1024] . W[3072,1024]^T")
    p.add_argument("--steps", type=int, default=None, help="timed steps (default 256 decode tokens, 5 prefill or "
                                                           "asr passes)")
    p.add_argument("--warmup", type=int, default=None, help="untimed steps (default 16 decode, 1 prefill/asr)")
    p.add_argument("--steps-per-graph", type=int, default=8)
    p.add_argument("--model", choices=("8b", "0.6b", "1.7b"), default="8b")
    p.add_argument("--policy", choices=("uniform", "q4_k_m"), default="uniform",
                   help="weight types: uniform Q4_K (the headline int4 config) or the Q4_K_M mix")
    p.add_argument("--positions", type=int, default=PROMPT_POSITIONS, help="KV positions prefilled before timing")
    p.add_argument("--kernel-reps", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-sample-steps", type=int, default=5, help="CPU baseline runs (the median is reported)")
    p.add_argument("--no-graph", action="store_true")
    p.add_argument("--per-op", action="store_true",
                   help="one launch per op instead of the persistent layers kernel (t2h_qwen3_decode_layers)")
    p.add_argument("--phase-trace", action="store_true",
                   help="run the persistent decode kernel's traced instantiation at the configured KV position and "
                        "print its per-phase timeline (markdown), no JSON line")
    p.add_argument("--profile-kernel", action="store_true",
                   help="counter-collection target: run the dominant kernel (the persistent layers kernel, or "
                        "with --per-op the gate|up GEMV over all layers) plus a 256 MiB copy (the calibration for "
                        "FETCH_SIZE/WRITE_SIZE), no timing, no JSON line")
    return p.parse_args()


def profile_kernel_target(per_op: bool, config: str = "decode") -> int:
    """Launch sequence for `rocprofv3 --pmc FETCH_SIZE|WRITE_SIZE`: the dominant kernel of the config twice,
    then one plain 256 MiB device copy whose traffic is known (256 MiB read + 256 MiB written), so counter
    readings can be scaled to bytes.  decode: the persistent layers kernel at KV 4096 (2 dispatches), or per
    op the gate|up GEMV once per layer (72 dispatches); prefill: the gate|up + SwiGLU GEMM at M 16384 (5
    times its 2 weight dequantisations then the bf16-weight GEMM; then twice dequantising every tile in the
    loop) and causal flash attention over 8 x 2048 tokens (2 dispatches); asr: the 0.6B-shape persistent layers
    kernel for 4 sequences at KV 1540 each (2 dispatches)."""
    import torch

    from torch2vk_amd import kernels
    from torch2vk_amd.qwen3.config import QWEN3_0_6B, QWEN3_8B
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.qwen3.weights import synthetic_weights

    dev = torch.device("cuda:0")
    if config == "prefill":
        c = QWEN3_8B
        gen = torch.Generator(device=dev)
        gen.manual_seed(0)
        gate = kernels.quantize(torch.randn(c.mlp, c.hidden, generator=gen, device=dev) * 0.02, "q8_0")
        up = kernels.quantize(torch.randn(c.mlp, c.hidden, generator=gen, device=dev) * 0.02, "q8_0")
        x = torch.randn(8 * 2048, c.hidden, generator=gen, device=dev).to(torch.bfloat16)
        act = torch.empty(8 * 2048, c.mlp, dtype=torch.bfloat16, device=dev)
        # the step's form: each weight dequantised once to bf16, then the bf16 tile loop (2 + 1 dispatches;
        # five times, so that a kernel trace averages over warm launches) ...
        for _ in range(5):
            kernels.gemm_swiglu(x, gate, up, "q8_0", out=act)
        # ... and the same GEMM dequantising every tile in its loop
        saved = kernels.DEQUANT_FIRST_ROWS
        kernels.DEQUANT_FIRST_ROWS = 0
        try:
            for _ in range(2):
                kernels.gemm_swiglu(x, gate, up, "q8_0", out=act)
        finally:
            kernels.DEQUANT_FIRST_ROWS = saved
        # and causal flash attention over the same 8 x 2048 tokens (32 q heads over 8 kv heads, D 128)
        q = torch.randn(8, 2048, c.heads, c.head_dim, generator=gen, device=dev).to(torch.bfloat16)
        k = torch.randn(8, 2048, c.kv_heads, c.head_dim, generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn(8, 2048, c.kv_heads, c.head_dim, generator=gen, device=dev).to(torch.bfloat16)
        o = torch.empty_like(q)
        for _ in range(2):
            kernels.flash_attn_prefill(q, k, v, out=o, causal=True)
        _profile_copy(dev)
        return 0
    if config == "asr":
        from torch2vk_amd.qwen3.model import Qwen3DecoderGroup

        w = synthetic_weights(QWEN3_0_6B, device=dev, seed=2)
        decs = [Qwen3Decoder(w, max_positions=1600, max_new_tokens=4, device=dev, persistent=True) for _ in range(4)]
        gen = torch.Generator(device=dev)
        gen.manual_seed(1)
        for dec in decs:
            dec.k_cache[:, :1539].normal_(generator=gen)
            dec.v_cache[:, :1539].normal_(generator=gen)
            dec.h.normal_()
            dec.position.fill_(1539)
        group = Qwen3DecoderGroup(decs)
        for _ in range(2):
            group.run_decode_layers()
        for dec in decs:
            dec.check_status()
        _profile_copy(dev)
        return 0
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
    _profile_copy(dev)
    return 0


def phase_trace(args) -> int:
    """Per-phase timeline of the persistent decode kernel (its traced instantiation) at KV position
    args.positions: for each phase of the middle layers, when blocks enter it, have its input in hand and
    finish, relative to the previous phase's last block finishing; printed as a markdown table."""
    import numpy as np
    import torch

    from torch2vk_amd import kernels
    from torch2vk_amd.qwen3.config import QWEN3_0_6B, QWEN3_8B
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.qwen3.weights import synthetic_weights

    from torch2vk_amd.qwen3.model import Qwen3DecoderGroup

    dev = torch.device("cuda:0")
    # --config asr: the C5 decoder's launch, four 0.6B sequences side by side (64 blocks each); the table is
    # sequence 0's blocks
    n_seq = 4 if args.config == "asr" else 1
    cfg = QWEN3_8B if args.model == "8b" and n_seq == 1 else QWEN3_0_6B
    w = synthetic_weights(cfg, device=dev, seed=0)
    decs = [Qwen3Decoder(w, max_positions=args.positions + 64, max_new_tokens=4, device=dev, persistent=True)
            for _ in range(n_seq)]
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    for dec in decs:
        dec.k_cache[:, :args.positions].normal_(generator=gen)
        dec.v_cache[:, :args.positions].normal_(generator=gen)
        dec.position.fill_(args.positions)
    runner = decs[0] if n_seq == 1 else Qwen3DecoderGroup(decs)
    trace = kernels.decode_layers_trace(cfg.layers, dev)
    launches = []
    for _ in range(max(3, args.kernel_reps)):
        for dec in decs:
            dec.h.normal_(generator=gen)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        runner.run_decode_layers(trace=trace)
        end.record()
        end.synchronize()
        launches.append((start.elapsed_time(end) * 1e3, trace.cpu().numpy().copy()))
    for dec in decs:
        status = decode_status(dec)
        if status:
            print(f"[bench] persistent kernel status {status:#x}: trace invalid", file=sys.stderr)
            return 3
    us_launch = float(np.median([u for u, _ in launches]))
    names = kernels.DECODE_TRACE_PHASES
    # the blocks that ran each phase: those that stamped its input in hand (the buffer starts zeroed; the
    # merge runs on as many blocks as there are q heads and not at all up to 256 positions, where the
    # attention runs on one block per kv head)
    ran = launches[-1][1][:, :, :, 1] != 0                       # [layers, phases, blocks]
    ran[:, :, 256 // n_seq:] = False                             # sequence 0's blocks
    n_blocks = [int(ran[2, ph].sum()) for ph in range(6)]
    rows = []   # [layer, phase] -> begin, ready_med, ready_max, end_med, end_max, polls, first_med (us from prev end)
    periods = []
    for _, tr in launches[1:]:
        t = tr[..., :4].astype(np.float64) * 0.01     # 100 MHz -> us
        lo, hi = 2, cfg.layers - 1
        down = ran[2, 5]
        periods.append((t[hi - 1, 5, down, 3].max() - t[lo - 1, 5, down, 3].max()) / (hi - lo))
        for layer in range(lo, hi):
            prev = t[layer - 1, 5, down, 3].max()
            r = []
            for ph in range(6):
                sel = ran[layer, ph]
                if not sel.any():
                    r.append([np.nan] * 7)
                    continue
                e = t[layer, ph, sel]
                r.append([np.median(e[:, 0]) - prev, np.median(e[:, 1]) - prev, e[:, 1].max() - prev,
                          np.median(e[:, 3]) - prev, e[:, 3].max() - prev,
                          float(tr[layer, ph, sel, 4].mean()),
                          np.median(e[e[:, 2] > 0, 2]) - prev if (e[:, 2] > 0).any() else np.nan])
                prev = e[:, 3].max()
            rows.append(r)
    m = np.mean(np.array(rows), axis=0)
    period = float(np.mean(periods))
    print(f"| phase | blocks | start (median) | input in hand (median / last) | first unit or softmax (median) | "
          f"end (median / last) | polls per wait |\n|---|---|---|---|---|---|---|")
    for ph in range(6):
        b, rm, rx, em, ex, pl, fm = m[ph]
        print(f"| {names[ph]} | {n_blocks[ph]} | {b:.2f} | {rm:.2f} / {rx:.2f} | {fm:.2f} | {em:.2f} / {ex:.2f} | "
              f"{pl:.1f} |")
    crit = m[:, 4]
    print(f"\nlaunch {us_launch:.1f} us ({cfg.layers} layers, {n_seq} sequence(s), KV position {args.positions}); "
          f"layer period "
          f"{period:.2f} us; sum of phase critical-path steps {np.nansum(crit):.2f} us")
    att = []
    for _, tr in launches[1:]:
        t = tr.astype(np.float64) * 0.01
        for layer in range(2, cfg.layers - 1):
            e = t[layer, 1, ran[layer, 1]]
            att.append([np.median(e[:, k] - e[:, 1]) for k in (5, 2, 6, 7, 3)])
    a5 = np.mean(np.array(att), axis=0)
    print(f"\nattention, median block, from input in hand: scores {a5[0]:.2f}, softmax {a5[1]:.2f}, P.V {a5[2]:.2f}, "
          f"waves merged {a5[3]:.2f}, end {a5[4]:.2f} us")
    wait = m[:, 1] - m[:, 0]
    after = m[:, 3] - m[:, 1]
    print("\nper phase (median block): wait for input " + ", ".join(f"{names[i]} {wait[i]:.2f}" for i in range(6)) +
          " us; input in hand to end " + ", ".join(f"{names[i]} {after[i]:.2f}" for i in range(6)) + " us")
    return 0


def _profile_copy(dev) -> None:
    """The calibration launch of a counter run: one plain 256 MiB device-to-device copy."""
    import torch

    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    print("[bench] profile-kernel target done", file=sys.stderr, flush=True)


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build is single-GPU); got --gpus {args.gpus}", file=sys.stderr)
        return 2
    if args.steps is None:
        args.steps = 256 if args.config == "decode" else 5
    if args.warmup is None:
        args.warmup = 16 if args.config == "decode" else 1
    if args.profile_kernel:
        return profile_kernel_target(args.per_op, args.config)
    if args.phase_trace:
        return phase_trace(args)
    if args.config == "prefill":
        return bench_prefill(args)
    if args.config == "asr":
        return bench_asr(args)
    if args.config == "linear":
        return bench_linear(args)
    if args.model == "0.6b":
        return bench_c2(args)
    import torch

    from torch2vk_amd import kernels
    from torch2vk_amd.qwen3.config import QWEN3_1_7B, QWEN3_8B
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.qwen3.weights import synthetic_weights

    if not torch.cuda.is_available():
        print("no HIP device", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    cfg = QWEN3_8B if args.model == "8b" else QWEN3_1_7B
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

    # the persistent kernel's waits are bounded: one that gave up sets the status word and the tokens of that
    # launch are invalid, so a run with the word set reports nothing
    status_timed = decode_status(dec)
    if status_timed:
        print(f"[bench] persistent kernel status {status_timed:#x} after the timed steps: run invalid",
              file=sys.stderr, flush=True)
        return 3

    kern = kernel_timing(dec, weights, args.kernel_reps)
    print(f"[bench] kernel timing: {json.dumps(kern['per_launch_us'])}", file=sys.stderr, flush=True)
    status_kernels = decode_status(dec)
    if status_kernels:
        print(f"[bench] persistent kernel status {status_kernels:#x} after the kernel timing: run invalid",
              file=sys.stderr, flush=True)
        return 3

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
        "status": status_timed | status_kernels,
    }
    print(json.dumps(line), flush=True)
    return 0


def decode_status(dec) -> int:
    """The persistent kernel's status word (0 = every bounded wait ended in time; always 0 for per-op launches)."""
    return int(dec.status.item()) if dec.persistent else 0


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


def persistent_bytes(weights, c, kv_len: int, n_seq: int = 1) -> int:
    """Algorithmic bytes of one persistent decode launch: each layer's packed weights and norms (once, however
    many sequences share them), and per sequence the K/V rows 0 .. kv_len - 1 read and the new row written,
    and the residual stream in and out."""
    b = 0
    for i in range(c.layers):
        b += sum(weights.packed[f"layers.{i}.{n}"].numel() for n in ("q", "k", "v", "o", "gate", "up", "down"))
        b += sum(weights.norms[f"layers.{i}.{n}"].numel() * 4 for n in ("input_norm", "post_norm", "q_norm",
                                                                          "k_norm"))
    b += n_seq * (c.layers * (2 * kv_len * c.kv_dim * 2 + 2 * c.kv_dim * 2) + 2 * c.hidden * 4)
    return int(b)


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
        b = persistent_bytes(weights, c, kv_len)
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
    """The CPU oracle's decoder on whole tokens at full 8B shapes: every layer with its own KV cache at
    ``positions``, then the LM head and argmax.  The layers share one dequantized weight set (layer 0's: 773 MB
    of fp32 per layer, far past any CPU cache, so re-reading one set costs what 36 distinct ones would), which
    keeps the host memory at about 2 GB."""
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
    for i in range(1, c.layers):
        for name in ("q", "k", "v", "o", "gate", "up", "down", "input_norm", "post_norm", "q_norm", "k_norm"):
            dense[f"layers.{i}.{name}"] = dense[f"layers.0.{name}"]
    dense["norm"] = weights.norms["norm"].cpu()
    dense["embed"] = torch.zeros(8, c.hidden)
    lm = torch.from_numpy(getattr(oracle, f"dequant_{weights.types['lm_head']}")(
        weights.packed["lm_head"].cpu().numpy(), c.hidden))
    dense["lm_head"] = lm
    shape = Qwen3Shape(hidden=c.hidden, layers=c.layers, heads=c.heads, kv_heads=c.kv_heads, head_dim=c.head_dim,
                       mlp=c.mlp, vocab=c.vocab, rope_theta=c.rope_theta)
    model = Qwen3CpuModel(shape, dense, max_positions=positions + steps + 1)
    g = torch.Generator().manual_seed(1)
    model.k_cache[:, :positions].normal_(generator=g)
    model.v_cache[:, :positions].normal_(generator=g)
    token_times = []
    for step in range(steps):
        t0 = time.perf_counter()
        hidden = model.forward(torch.tensor([step % 8]), start=positions + step)
        int(torch.argmax(model.logits(hidden)))
        token_times.append(time.perf_counter() - t0)
    t_token = statistics.median(token_times)
    del np
    return {
        "value": round(1.0 / t_token, 4),
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "sample": f"CPU oracle decoder (torch {torch.__version__}, fp32 dense weights dequantized by the oracle, one "
                  f"weight set shared by the {c.layers} layers, each layer with its own KV cache): {steps} whole "
                  f"tokens from KV position {positions} (all {c.layers} layers, LM head, argmax), median "
                  f"{t_token * 1e3:.1f} ms per token",
    }


# ------------------------------------------------------------------ C1 linear --

LINEAR_COPIES = 256  # distinct weight copies streamed for GB/s: 453 MB, past the 256 MB MALL


def bench_linear(args) -> int:
    """y = x . deq(W)^T with x bf16 [1, 1024] ~ N(0, 1) and W fp32 [3072, 1024] ~ N(0, 0.02)
    quantized to Q4_K (seed 0).  Latency: one call on a hot weight, calls replayed back to back in a HIP graph.
    Bandwidth: one call on each of LINEAR_COPIES distinct weight copies in a graph (every copy cold), GB/s of
    the algorithmic bytes.  CPU: torch F.linear on the oracle-dequantized fp32 weight, median of 7 runs."""
    import numpy as np
    import torch

    import oracle
    from torch2vk_amd import kernels

    if not torch.cuda.is_available():
        print("no HIP device", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    n, k = 3072, 1024
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    x = torch.randn(1, k, generator=gen, device=dev).to(torch.bfloat16)
    w = kernels.quantize(torch.randn(n, k, generator=gen, device=dev) * 0.02, "q4_k")
    y = torch.empty(1, n, device=dev)
    kernels.q4k_matvec(x, w, out=y)
    torch.cuda.synchronize()
    w_deq = oracle.dequant_q4_k(w.cpu().numpy(), k)
    ref = x.float().cpu().numpy().astype(np.float64) @ w_deq.astype(np.float64).T
    err = float(np.abs(y.cpu().numpy() - ref).max() / np.abs(ref).max())
    reps = max(args.steps, 20)
    hot_us = _graph_us_per_call([lambda: kernels.q4k_matvec(x, w, out=y)] * 64, reps)
    eager_us = _events_us(lambda: kernels.q4k_matvec(x, w, out=y), 64 * reps)
    copies = [w.clone() for _ in range(LINEAR_COPIES)]
    ys = [torch.empty(1, n, device=dev) for _ in range(LINEAR_COPIES)]
    calls = [(lambda wc=wc, yc=yc: kernels.q4k_matvec(x, wc, out=yc)) for wc, yc in zip(copies, ys)]
    cold_us = _graph_us_per_call(calls, reps)
    call_bytes = w.numel() + k * 2 + n * 4
    gbs = call_bytes / (cold_us * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        threads = len(os.sched_getaffinity(0))
        torch.set_num_threads(threads)
        xc = x.float().cpu()
        wc = torch.from_numpy(w_deq)
        runs = []
        for _ in range(7):
            t0 = time.perf_counter()
            for _ in range(200):
                torch.nn.functional.linear(xc, wc)
            runs.append((time.perf_counter() - t0) / 200)
        cpu = {"value": round(statistics.median(runs) * 1e6, 2), "unit": "us/call", "cores": threads, "kind": "port",
               "sample": f"torch {torch.__version__} F.linear on the oracle-dequantized fp32 W, median of 7 runs of "
                         f"200 calls"}
    line = {
        "metric": "Q4_K linear x[1,1024] . W[3072,1024]^T latency (BASELINE configs[0])",
        "value": round(hot_us, 3),
        "unit": "us/call",
        "n_gpus": 1,
        "steps": reps,
        "warmup": 1,
        "ms_per_step": round(hot_us * 64 / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seed 0: x ~ N(0,1) bf16, W ~ N(0,0.02) quantized to Q4_K on the GPU)",
        "config": {"workload": "one Q4_K GEMV, x bf16 [1,1024], W [3072,1024] (1 769 472 B packed), fp32 out; "
                               "a step = 64 calls replayed in a HIP graph on the hot weight",
                   "batch": 1},
        "eager_us_per_call": round(eager_us, 3),
        "max_rel_error_vs_oracle": err,
        "roofline": {"bound": "hbm", "kernel": "q4k_gemv_kernel (K 1024)", "achieved": round(gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_launch": call_bytes, "avg_launch_us": round(cold_us, 3),
                     "note": f"one call on each of {LINEAR_COPIES} distinct weight copies per replay (cold weights)"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


# --------------------------------------------------------------- C2 0.6B decode --

C2_PROMPT = 128
C2_TOKENS = 128


def bench_c2(args) -> int:
    """the 28-layer Qwen3-0.6B shape, a prompt of 128 random token ids through the chunked
    matrix-core prefill (replayed from a HIP graph captured in the untimed first pass), then 128 greedy tokens
    (HIP graphs of 8 decode steps).  value = the 128 tokens over
    the time from the prompt's arrival to the last token; the decode-only rate is reported beside it."""
    import torch

    from torch2vk_amd.qwen3.config import QWEN3_0_6B
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.qwen3.weights import synthetic_weights

    if not torch.cuda.is_available():
        print("no HIP device", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    cfg = QWEN3_0_6B
    weights = synthetic_weights(cfg, device=dev, seed=0, policy=args.policy)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    prompt = torch.randint(0, cfg.vocab, (C2_PROMPT,), generator=gen, device=dev)
    dec = Qwen3Decoder(weights, max_positions=C2_PROMPT + C2_TOKENS + 16, max_new_tokens=C2_TOKENS + 8, device=dev)
    dec.stop_on_eos = False
    spg = args.steps_per_graph
    runs = []
    first_prefill = None
    for r in range(1 + max(1, args.kernel_reps)):   # the first pass warms the graphs and is not counted
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dec.prefill_graphed(prompt)  # the first pass captures the prefill's graph
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        dec.run_steps(C2_TOKENS - 1, steps_per_graph=spg, use_graph=not args.no_graph)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        status = decode_status(dec)
        if status:
            print(f"[bench] persistent kernel status {status:#x}: run invalid", file=sys.stderr, flush=True)
            return 3
        if r:
            runs.append((t1 - t0, t2 - t1))
        else:
            first_prefill = t1 - t0  # warm-up launch, capture and first replay of this prompt length
        print(f"[bench] pass {r}: prefill {1e3 * (t1 - t0):.2f} ms, {C2_TOKENS - 1} steps {1e3 * (t2 - t1):.2f} ms",
              file=sys.stderr, flush=True)
    pre = statistics.median(u for u, _ in runs)
    steps_s = statistics.median(v for _, v in runs)
    total = pre + steps_s
    tokens = [int(t) for t in dec.generated[:C2_TOKENS].tolist()]
    assert len(tokens) == C2_TOKENS and min(tokens) >= 0
    # the same prefill eager (no graph): what a prompt of a length not seen before costs after its first call
    eager = []
    for _ in range(max(3, args.kernel_reps)):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dec.prefill_chunked(prompt)
        torch.cuda.synchronize()
        eager.append(time.perf_counter() - t0)
    pre_eager = statistics.median(eager)
    kern = kernel_timing(dec, weights, args.kernel_reps)
    dom = kern["dominant"]
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_c2(cfg, weights, prompt.cpu(), args.cpu_sample_steps)
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)
    line = {
        "metric": "Qwen3-0.6B-shape int4 decode tok/s @bs1, 128-token prompt + 128 tokens (BASELINE configs[1])",
        "value": round(C2_TOKENS / total, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": C2_TOKENS,
        "warmup": 1,
        "ms_per_step": round(1e3 * total / C2_TOKENS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        # the reference's one published number: Qwen3-0.6B Q4_K_M greedy decode at 7.4 ms/token (~135 tok/s) on
        # its Radeon 890M (docs/torch2vk-introduction.md:676); comparable for the Q4_K_M policy only
        "vs_baseline": round((C2_TOKENS / total) / 135.0, 3) if args.policy == "q4_k_m" else None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) weights quantized on the GPU, "
                + ("Q4_K uniform int4" if args.policy == "uniform" else "Q4_K_M (Q4_K + Q6_K)") + "; random prompt ids)",
        "config": {"workload": f"qwen3-0.6b-shape greedy decode, batch 1: {C2_PROMPT}-token prompt through the "
                               f"chunked prefill (one HIP graph, captured in the untimed first pass for this prompt "
                               f"length), then {C2_TOKENS} tokens (HIP graphs of {spg} steps, "
                               + ("persistent layers kernel" if dec.persistent else "one launch per op") + ")",
                   "batch": 1, "prompt": C2_PROMPT, "new_tokens": C2_TOKENS},
        "prefill_ms": round(pre * 1e3, 3),
        "prefill_first_call_ms": round(first_prefill * 1e3, 3),
        "prefill_eager_ms": round(pre_eager * 1e3, 3),
        "value_eager_prefill": round(C2_TOKENS / (pre_eager + steps_s), 2),
        "decode_tok_s": round((C2_TOKENS - 1) / steps_s, 2),
        "roofline": {"bound": "hbm", "kernel": dom["kernel"], "achieved": round(dom["gbs"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": None, "bytes_per_launch": dom["bytes"], "avg_launch_us": round(dom["us"], 3)},
        "qmatmul_gbs": round(kern["qmatmul_gbs"], 1),
        "cpu_baseline": cpu,
        "status": 0,
    }
    print(json.dumps(line), flush=True)
    return 0


def cpu_baseline_c2(cfg, weights, prompt, runs: int) -> dict:
    """The CPU oracle's whole 0.6B decoder (torch, fp32 weights dequantized by the oracle): the 128-token
    prompt, then the median of ``runs`` single-token decode steps after it."""
    import torch

    import oracle
    from oracle.reference import Qwen3CpuModel, Qwen3Shape
    from torch2vk_amd.qwen3.weights import matrix_shapes

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    c = cfg
    shapes = matrix_shapes(c)
    dense = {name: torch.from_numpy(getattr(oracle, f"dequant_{weights.types[name]}")(
        weights.packed[name].cpu().numpy(), shapes[name][1])) for name in weights.packed}
    dense.update({name: t.cpu() for name, t in weights.norms.items()})
    shape = Qwen3Shape(hidden=c.hidden, layers=c.layers, heads=c.heads, kv_heads=c.kv_heads, head_dim=c.head_dim,
                       mlp=c.mlp, vocab=c.vocab, rope_theta=c.rope_theta)
    model = Qwen3CpuModel(shape, dense, max_positions=len(prompt) + runs + 2)
    t0 = time.perf_counter()
    hidden = model.forward(prompt.long(), start=0)
    t_prompt = time.perf_counter() - t0
    tok = int(torch.argmax(model.logits(hidden)))
    times = []
    for s in range(runs):
        t0 = time.perf_counter()
        hidden = model.forward(torch.tensor([tok]), start=len(prompt) + s)
        tok = int(torch.argmax(model.logits(hidden)))
        times.append(time.perf_counter() - t0)
    t_tok = statistics.median(times)
    return {"value": round(1.0 / t_tok, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"CPU oracle decoder (torch {torch.__version__}, all 28 layers, fp32 weights dequantized by the "
                      f"oracle): {len(prompt)}-token prompt in {t_prompt:.2f} s, then the median of {runs} decode "
                      f"steps ({t_tok * 1e3:.1f} ms)"}


# ----------------------------------------------------------------- prefill --

MFMA_BF16_PEAK_TFLOPS = 2500.0
PREFILL_SEQ = 2048  # tokens per sequence of configs[3]


def _events_us(fn, reps: int) -> float:
    """Average duration of ``fn`` (one launch) over ``reps`` back-to-back calls, HIP events on the current
    stream, which is the stream the launches go to."""
    import torch

    fn()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) * 1000.0 / reps


def _timed_steps(step, warmup: int, steps: int) -> float:
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def bench_prefill(args) -> int:
    """8 sequences x 2048 random token ids through the 36-layer Qwen3-8B shape, every
    linear weight Q8_0 (int8, group 32) dequantised into the bf16 MFMA GEMM, causal flash attention, then
    the final norm + LM head + greedy select of each sequence's first token.  A step is that whole prefill."""
    import torch

    from torch2vk_amd import kernels
    from torch2vk_amd.qwen3.config import QWEN3_8B

    if not torch.cuda.is_available():
        print("no HIP device", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    c = QWEN3_8B
    nb, tl = 8, PREFILL_SEQ
    m = nb * tl
    t_setup = time.time()
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)

    def packed(rows: int, cols: int, wtype: str) -> torch.Tensor:
        dense = torch.randn(rows, cols, generator=gen, device=dev).mul_(0.02)
        out = kernels.quantize(dense, wtype)
        del dense
        return out

    def norm(n: int) -> torch.Tensor:
        return torch.ones(n, device=dev).add_(torch.randn(n, generator=gen, device=dev).mul_(0.1))

    qkv_rows = c.q_dim + 2 * c.kv_dim
    layers = [dict(qkv=packed(qkv_rows, c.hidden, "q8_0"), o=packed(c.hidden, c.q_dim, "q8_0"),
                   gate=packed(c.mlp, c.hidden, "q8_0"), up=packed(c.mlp, c.hidden, "q8_0"),
                   down=packed(c.hidden, c.mlp, "q8_0"), input_norm=norm(c.hidden), post_norm=norm(c.hidden),
                   q_norm=norm(c.head_dim), k_norm=norm(c.head_dim)) for _ in range(c.layers)]
    embed = packed(c.vocab, c.hidden, "q8_0")
    lm_head = packed(c.vocab, c.hidden, "q4_k")
    final_norm = norm(c.hidden)
    ids = torch.randint(0, c.vocab, (m,), generator=gen, device=dev)
    bf, f32 = torch.bfloat16, torch.float32
    h = torch.empty(m, c.hidden, dtype=f32, device=dev)
    x = torch.empty(m, c.hidden, dtype=bf, device=dev)
    qkv = torch.empty(m, qkv_rows, dtype=f32, device=dev)
    qb = torch.empty(m, c.heads, c.head_dim, dtype=bf, device=dev)
    kc = torch.empty(nb, tl, c.kv_heads, c.head_dim, dtype=bf, device=dev)
    vc = torch.empty_like(kc)
    attn = torch.empty(nb, tl, c.heads, c.head_dim, dtype=bf, device=dev)
    up = torch.empty(m, c.mlp, dtype=f32, device=dev)
    act = torch.empty(m, c.mlp, dtype=bf, device=dev)
    ps = torch.empty(512, dtype=f32, device=dev)
    pt = torch.empty(512, dtype=torch.int32, device=dev)
    eos = torch.tensor(c.eos_token_ids, dtype=torch.int64, device=dev)
    next_tok = torch.zeros(nb, 1, dtype=torch.int64, device=dev)
    done = torch.zeros(nb, 1, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    print(f"[bench] prefill setup {time.time() - t_setup:.1f}s", file=sys.stderr, flush=True)

    def layer_pass(lw) -> None:
        kernels.rms_norm(h, lw["input_norm"], out=x)
        kernels.gemm(x, lw["qkv"], "q8_0", out=qkv)
        # the 8 sequences' q/k norm + RoPE + KV writes in one launch, each into its own cache
        kernels.qk_norm_rope_cache(qkv[:, :c.q_dim], qkv[:, c.q_dim:c.q_dim + c.kv_dim], qkv[:, c.q_dim + c.kv_dim:],
                                   qb, kc, vc, 0, q_norm_weight=lw["q_norm"], k_norm_weight=lw["k_norm"],
                                   theta=c.rope_theta)
        kernels.flash_attn_prefill(qb.view(nb, tl, c.heads, c.head_dim), kc, vc, out=attn, causal=True)
        kernels.gemm(attn.view(m, c.q_dim), lw["o"], "q8_0", out=h, residual=h)
        kernels.rms_norm(h, lw["post_norm"], out=x)
        kernels.gemm_swiglu(x, lw["gate"], lw["up"], "q8_0", out=act)
        kernels.gemm(act, lw["down"], "q8_0", out=h, residual=h)

    def step() -> None:
        kernels.embedding_q8_0(embed, ids, c.hidden, out=h)
        for lw in layers:
            layer_pass(lw)
        for b in range(nb):
            kernels.lm_head_argmax_partial(h[(b + 1) * tl - 1], lm_head, "q4_k", ps, pt, norm_weight=final_norm)
            kernels.token_select(ps, pt, eos, next_tok[b], done[b])

    per_step = _timed_steps(step, args.warmup, args.steps)
    tok_s = m / per_step
    params = qkv_rows * c.hidden + c.hidden * c.q_dim + 2 * c.mlp * c.hidden + c.hidden * c.mlp
    linear_flop = 2.0 * m * params * c.layers
    attn_flop = 4.0 * c.heads * c.head_dim * (tl * (tl + 1) / 2) * nb * c.layers
    total_flop = linear_flop + attn_flop + 2.0 * nb * c.vocab * c.hidden
    tflops = total_flop / per_step / 1e12
    print(f"[bench] prefill {per_step * 1e3:.1f} ms per 8 x 2048 tokens: {tok_s:.0f} tok/s, {tflops:.1f} TFLOP/s",
          file=sys.stderr, flush=True)

    # dominant kernel of the step: gate|up + SwiGLU in one GEMM (M 16384, K 4096, 2 x 12288 rows), HIP events
    # on its stream.  At these M the step dequantises each Q8_0 weight once to bf16 (kernels.DEQUANT_FIRST_ROWS)
    # and runs the tile loop on bf16 rows: the GEMM launch alone is the roofline kernel, the dequantisations
    # are timed beside it, and so is the same GEMM dequantising every tile in the loop (the split of the two).
    # The standalone up-projection GEMM the config names is timed the same ways.
    reps = args.kernel_reps * 4
    gate_b = kernels.dequantize_bf16(layers[0]["gate"], "q8_0", c.hidden)
    up_b = kernels.dequantize_bf16(layers[0]["up"], "q8_0", c.hidden)
    deq_us = _events_us(lambda: kernels.dequantize_bf16(layers[0]["up"], "q8_0", c.hidden, out=up_b), reps)
    gu_us = _events_us(lambda: kernels.gemm_swiglu(x, gate_b, up_b, "bf16", out=act), reps)
    gu_tflops = 2.0 * m * c.hidden * 2 * c.mlp / (gu_us * 1e-6) / 1e12
    gu_step_us = _events_us(lambda: kernels.gemm_swiglu(x, layers[0]["gate"], layers[0]["up"], "q8_0", out=act),
                            reps)
    gemm_us = _events_us(lambda: kernels.gemm(x, up_b, "bf16", out=up), reps)
    gemm_step_us = _events_us(lambda: kernels.gemm(x, layers[0]["up"], "q8_0", out=up), reps)
    saved = kernels.DEQUANT_FIRST_ROWS
    kernels.DEQUANT_FIRST_ROWS = 0
    try:
        gu_tile_us = _events_us(lambda: kernels.gemm_swiglu(x, layers[0]["gate"], layers[0]["up"], "q8_0", out=act),
                                reps)
        gemm_tile_us = _events_us(lambda: kernels.gemm(x, layers[0]["up"], "q8_0", out=up), reps)
    finally:
        kernels.DEQUANT_FIRST_ROWS = saved
    del gate_b, up_b
    up_flop = 2.0 * m * c.hidden * c.mlp
    gemm_tflops = up_flop / (gemm_step_us * 1e-6) / 1e12
    fa_us = _events_us(lambda: kernels.flash_attn_prefill(qb.view(nb, tl, c.heads, c.head_dim), kc, vc, out=attn,
                                                          causal=True), args.kernel_reps * 4)
    fa_tflops = 4.0 * c.heads * c.head_dim * (tl * (tl + 1) / 2) * nb / (fa_us * 1e-6) / 1e12
    cpu = None if args.no_cpu_baseline else cpu_baseline_prefill(layers[0], c)
    line = {
        "metric": "Qwen3-8B-shape int8 (Q8_0) prefill tok/s, 8 x 2048 tokens; MFMA utilisation vs bf16 dense peak",
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(per_step * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) weights quantized to Q8_0 on the GPU, random token ids)",
        "config": {
            "workload": "Qwen3-8B-shape prefill of 8 sequences x 2048 tokens: Q8_0 embedding, 36 layers (RMSNorm, "
                        "q|k|v GEMM, q/k norm + RoPE + KV write, causal flash attention, o GEMM + residual, "
                        "RMSNorm, gate|up GEMM with SwiGLU in its epilogue, down GEMM + residual; every GEMM "
                        "dequantises its Q8_0 weight to a bf16 scratch inside the step, then runs the bf16 tile "
                        "loop), final norm + Q4_K LM head + greedy select of each sequence's first token",
            "batch": nb, "seq_len": tl, "weights": "q8_0",
        },
        "mfma_utilisation": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "achieved_tflops": round(tflops, 1),
        "roofline": {
            "bound": "mfma",
            "kernel": "gemm_bf16_ring_kernel<SwiGLU epilogue> (gate|up over the Q8_0 weights dequantised to "
                      "bf16 once, M 16384 K 4096 N 2 x 12288)",
            "achieved": round(gu_tflops, 1),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(gu_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": profiled_traffic(TRAFFIC_PROFILES["prefill_gate_up_gemm"]),
            "traffic_source": TRAFFIC_PROFILES["prefill_gate_up_gemm"].name,
            "avg_launch_us": round(gu_us, 1),
        },
        "gate_up": {"with_dequant_us": round(gu_step_us, 1), "dequant_us_per_matrix": round(deq_us, 1),
                    "in_loop_dequant_us": round(gu_tile_us, 1),
                    "note": "with_dequant: the step's call (2 dequantisations + the bf16 GEMM); in_loop_dequant: "
                            "gemm_q_kernel<GemmQ80> dequantising every tile"},
        "up_projection_gemm": {"kernel": "t2h_dequantize_bf16 + gemm_bf16_ring_kernel (M 16384 K 4096 N 12288, "
                                         "fp32 out)",
                               "avg_launch_us": round(gemm_step_us, 1), "tflops": round(gemm_tflops, 1),
                               "gemm_alone_us": round(gemm_us, 1), "in_loop_dequant_us": round(gemm_tile_us, 1),
                               "in_loop_dequant_tflops": round(up_flop / (gemm_tile_us * 1e-6) / 1e12, 1)},
        "flash_attention": {"avg_launch_us": round(fa_us, 1), "tflops": round(fa_tflops, 1)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def cpu_baseline_prefill(lw, c) -> dict:
    """The CPU oracle's Qwen3 forward of all 36 8B-shape layers over one of the workload's 2048-token sequences:
    tokens/s of prefill on the host cores.  The layers share one weight set (layer 0's, dequantized from the same Q8_0 bytes; 773 MB of
    fp32 per layer, far past any CPU cache, so re-reading one set costs what 36 distinct ones would)."""
    import torch

    import oracle
    from oracle.reference import Qwen3CpuModel, Qwen3Shape

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    qkv = oracle.dequant_q8_0(lw["qkv"].cpu().numpy(), c.hidden)
    dense = {"layers.0.q": torch.from_numpy(qkv[:c.q_dim]),
             "layers.0.k": torch.from_numpy(qkv[c.q_dim:c.q_dim + c.kv_dim]),
             "layers.0.v": torch.from_numpy(qkv[c.q_dim + c.kv_dim:]),
             "layers.0.o": torch.from_numpy(oracle.dequant_q8_0(lw["o"].cpu().numpy(), c.q_dim)),
             "layers.0.gate": torch.from_numpy(oracle.dequant_q8_0(lw["gate"].cpu().numpy(), c.hidden)),
             "layers.0.up": torch.from_numpy(oracle.dequant_q8_0(lw["up"].cpu().numpy(), c.hidden)),
             "layers.0.down": torch.from_numpy(oracle.dequant_q8_0(lw["down"].cpu().numpy(), c.mlp))}
    for n in ("input_norm", "post_norm", "q_norm", "k_norm"):
        dense[f"layers.0.{n}"] = lw[n].cpu()
    for i in range(1, c.layers):
        for n in ("q", "k", "v", "o", "gate", "up", "down", "input_norm", "post_norm", "q_norm", "k_norm"):
            dense[f"layers.{i}.{n}"] = dense[f"layers.0.{n}"]
    n = PREFILL_SEQ
    dense["embed"] = torch.randn(n, c.hidden)
    dense["norm"] = torch.ones(c.hidden)
    dense["lm_head"] = torch.zeros(1, c.hidden)
    shape = Qwen3Shape(hidden=c.hidden, layers=c.layers, heads=c.heads, kv_heads=c.kv_heads, head_dim=c.head_dim,
                       mlp=c.mlp, vocab=c.vocab, rope_theta=c.rope_theta)
    model = Qwen3CpuModel(shape, dense, max_positions=n)
    t0 = time.perf_counter()
    model.forward(torch.arange(n), start=0)
    t_seq = time.perf_counter() - t0
    return {
        "value": round(n / t_seq, 2),
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "sample": f"CPU oracle Qwen3 forward (torch {torch.__version__}, fp32 dense weights dequantized from the "
                  f"Q8_0 bytes, one weight set shared by the {c.layers} layers) of all {c.layers} layers over one "
                  f"{n}-token sequence, causal ({t_seq:.2f} s); a CPU takes the batch's sequences one after another",
    }


# --------------------------------------------------------------------- asr --


def bench_asr(args) -> int:
    """the 24-layer, 1024-wide, 16-head audio encoder (Q8_0 linears, FFN 4096) over
    4 utterances x 1500 frames of N(0,1) features, attention within each utterance; then, per utterance, a
    Qwen3-0.6B-shape uniform-int4 decoder whose prompt embeddings carry that utterance's 1500 encoder states
    (injected at the audio placeholder positions), chunked prefill and 64 greedy tokens.  A step is the whole
    job; value = audio frames per second through it."""
    import torch

    from torch2vk_amd import kernels
    from torch2vk_amd.qwen3.config import QWEN3_0_6B
    from torch2vk_amd.qwen3.model import Qwen3Decoder, Qwen3DecoderGroup
    from torch2vk_amd.qwen3.weights import synthetic_weights
    from torch2vk_amd.qwen3_asr.config import ASR_C5_ENCODER
    from torch2vk_amd.qwen3_asr.encoder import (Qwen3AudioEncoder, quantize_audio_weights, run_audio_inject,
                                                synthetic_audio_dense)

    if not torch.cuda.is_available():
        print("no HIP device", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    ecfg, tcfg = ASR_C5_ENCODER, QWEN3_0_6B
    nb, frames, new_tokens = 4, 1500, 64
    t_setup = time.time()
    enc = Qwen3AudioEncoder(quantize_audio_weights(synthetic_audio_dense(ecfg, seed=0), ecfg, dev))
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    feats_in = torch.randn(nb * frames, ecfg.d_model, generator=gen, device=dev).to(torch.bfloat16).float()
    cu = kernels.segment_bounds([frames * i for i in range(nb + 1)], nb * frames, dev)
    tw = synthetic_weights(tcfg, device=dev, seed=2)
    prefix, suffix = [151644, 8948, 198, 151669], [151670, 151645, 198]
    prompt_len = len(prefix) + frames + len(suffix)
    # one decoder (KV cache) per utterance: their prompts prefill as one batch and their decode steps run
    # together, all 4 sequences' layers in one persistent launch
    group = Qwen3DecoderGroup.create(tw, nb, max_positions=prompt_len + new_tokens + 16,
                                     max_new_tokens=new_tokens + 8, device=dev)
    decs = group.decoders
    for dec in decs:
        dec.stop_on_eos = False
    ids = torch.tensor(prefix + [ecfg_audio_id()] * frames + suffix, device=dev)
    audio_pos = torch.arange(len(prefix), len(prefix) + frames, device=dev)
    h = torch.empty_like(feats_in)
    transcripts = []
    torch.cuda.synchronize()
    print(f"[bench] asr setup {time.time() - t_setup:.1f}s", file=sys.stderr, flush=True)

    def encode() -> torch.Tensor:
        h.copy_(feats_in)
        enc.encoder_layers(h, cu)
        return enc.head(h)

    def step() -> None:
        feats = encode()
        transcripts.clear()
        embs = []
        for b, dec in enumerate(decs):
            emb = dec.embed_tokens(ids)
            run_audio_inject(emb, audio_pos, feats[b * frames:(b + 1) * frames])
            embs.append(emb)
        group.prefill_chunked(embs, chunk=2048)
        transcripts.extend(group.finish(new_tokens))

    per_step = _timed_steps(step, args.warmup, args.steps)
    frames_s = nb * frames / per_step
    enc_s = _timed_steps(encode, 1, max(3, args.steps))
    d, f, lay = ecfg.d_model, ecfg.ffn, ecfg.layers
    enc_flop = 2.0 * nb * frames * lay * (4 * d * d + 2 * d * f) + 4.0 * nb * frames * frames * d * lay
    enc_flop += 2.0 * nb * frames * (d * d + d * ecfg.output_dim)
    enc_tflops = enc_flop / enc_s / 1e12
    x_ln = torch.randn(nb * frames, d, generator=gen, device=dev).to(torch.bfloat16)
    fc1 = enc.weights.packed["thinker.audio_tower.layers.0.fc1.weight"]
    b1 = enc.weights.vectors["thinker.audio_tower.layers.0.fc1.bias"]
    y = torch.empty(nb * frames, f, dtype=torch.bfloat16, device=dev)
    fc1_us = _events_us(lambda: kernels.q8_0_linear(x_ln, fc1, bias=b1, act="gelu", out=y), args.kernel_reps * 4)
    fc1_tflops = 2.0 * nb * frames * d * f / (fc1_us * 1e-6) / 1e12
    # dominant kernel of the step: the 4 decoders' persistent launch (all 28 layers of a token of each
    # utterance), timed at the middle of the generated span; its bytes are the shared weights once and each
    # sequence's KV rows (the 4 groups of blocks read the same weights, which L2 and the MALL serve after the
    # first: the counters measure 1.04x these bytes)
    for dec in decs:
        dec.position.fill_(prompt_len + new_tokens // 2)
    kv_len = prompt_len + new_tokens // 2 + 1
    dl_us = _graph_us_per_call([group.run_decode_layers] * 2, args.kernel_reps * 4)
    dl_bytes = persistent_bytes(tw, tcfg, kv_len, n_seq=nb)
    for dec in decs:
        dec.check_status()
    print(f"[bench] asr step {per_step * 1e3:.1f} ms ({frames_s:.0f} frames/s); encoder {enc_s * 1e3:.2f} ms, "
          f"{enc_tflops:.1f} TFLOP/s; fc1 {fc1_us:.1f} us {fc1_tflops:.1f} TFLOP/s; tokens {len(transcripts[0])}",
          file=sys.stderr, flush=True)
    cpu = None if args.no_cpu_baseline else cpu_baseline_asr(enc, ecfg, feats_in[:frames], tw, tcfg,
                                                             ids.tolist(), audio_pos.tolist(), new_tokens)
    line = {
        "metric": "Qwen3-ASR-shape audio frames/s: 24-layer 1024-wide encoder over 4 x 1500 frames, then a "
                  "0.6B-shape int4 decoder, 64 greedy tokens per utterance",
        "value": round(frames_s, 1),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(per_step * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (encoder input frames N(0,1) in bf16; seeded random-init weights: Q8_0 encoder, "
                "uniform Q4_K decoder)",
        "config": {
            "workload": "4 utterances x 1500 frames: encoder (24 layers, hidden 1024, 16 heads, FFN 4096, "
                        "attention within each utterance) + ln_post/proj1/proj2, then per utterance the audio "
                        "states injected into a 1507-position prompt, the 4 prompts prefilled as one batch, and 64 "
                        "greedy tokens of the 4 utterances decoded together (Qwen3-0.6B shape, uniform Q4_K, one "
                        "persistent launch for the 4 sequences' layers per step, HIP graphs of 8 steps)",
            "batch": nb, "frames": frames, "decoder_tokens": new_tokens,
        },
        "encoder_ms": round(enc_s * 1e3, 3),
        "encoder_tflops": round(enc_tflops, 1),
        "mfma_utilisation": round(enc_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": f"decode_layers_kernel<DlQwen3_0_6B_x4> (28 layers of a decoder token of each of the "
                      f"4 utterances, KV {kv_len})",
            "achieved": round(dl_bytes / (dl_us * 1e-6) / 1e9, 1) if dl_us else None,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dl_bytes / (dl_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if dl_us else None,
            "traffic": profiled_traffic(TRAFFIC_PROFILES["asr_decode_layers_0_6b"]),
            "traffic_source": TRAFFIC_PROFILES["asr_decode_layers_0_6b"].name,
            "avg_launch_us": round(dl_us, 1) if dl_us else None,
            "bytes_per_launch": dl_bytes,
        },
        "encoder_fc1": {"kernel": "gemm_q_kernel<GemmQ80> (fc1 + bias + GELU, M 6000 K 1024 N 4096)",
                        "avg_launch_us": round(fc1_us, 1), "tflops": round(fc1_tflops, 1),
                        "mfma_frac": round(fc1_tflops / MFMA_BF16_PEAK_TFLOPS, 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def ecfg_audio_id() -> int:
    from torch2vk_amd.qwen3_asr.config import AUDIO_TOKEN_ID

    return AUDIO_TOKEN_ID


def cpu_baseline_asr(enc, ecfg, feats: "torch.Tensor", tw, tcfg, ids: list[int], audio_pos: list[int],
                     new_tokens: int) -> dict:
    """One utterance's whole job on the host cores through the CPU oracle: the encoder (every layer, then the
    head) over its frames, its states injected into the prompt's embeddings, the prompt prefilled through every
    decoder layer, then ``new_tokens`` greedy tokens.  A CPU takes the utterances one after another, so
    frames/s = frames / the job's time."""
    import torch

    from oracle import asr as oasr
    from oracle.qwen3_check import dense_weights
    from oracle.reference import Qwen3CpuModel, Qwen3Shape
    from torch2vk_amd.qwen3.weights import matrix_shapes
    from torch2vk_amd.qwen3_asr.encoder import audio_tensor_shapes

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    frames = feats.shape[0]
    w = oasr.dense_from_packed({k: v.cpu().numpy() for k, v in enc.weights.packed.items()},
                               {k: v.cpu().numpy() for k, v in enc.weights.vectors.items()}, audio_tensor_shapes(ecfg))
    dense = dense_weights({k: v.cpu().numpy() for k, v in tw.packed.items()}, tw.types,
                          {k: v.cpu().numpy() for k, v in tw.norms.items()}, matrix_shapes(tcfg))
    shape = Qwen3Shape(hidden=tcfg.hidden, layers=tcfg.layers, heads=tcfg.heads, kv_heads=tcfg.kv_heads,
                       head_dim=tcfg.head_dim, mlp=tcfg.mlp, vocab=tcfg.vocab, rope_theta=tcfg.rope_theta)
    model = Qwen3CpuModel(shape, dense, max_positions=len(ids) + new_tokens + 1)
    tid = torch.tensor(ids)
    pos = torch.tensor(audio_pos)
    x = feats.float().cpu().clone()
    t0 = time.perf_counter()
    states = oasr.encoder_head_cpu(w, ecfg, oasr.encoder_layers_cpu(w, ecfg, x, cu_seqlens=[0, frames]))
    t_enc = time.perf_counter() - t0
    emb = dense["embed"][tid].clone()
    emb[pos] = states.to(emb.dtype)
    hidden = model.forward(tid, start=0, embeds=emb)
    tok = int(torch.argmax(model.logits(hidden)))
    t_prefill = time.perf_counter() - t0 - t_enc
    for s in range(new_tokens - 1):
        hidden = model.forward(torch.tensor([tok]), start=len(ids) + s)
        tok = int(torch.argmax(model.logits(hidden)))
    t_job = time.perf_counter() - t0
    return {
        "value": round(frames / t_job, 2),
        "unit": "frames/s",
        "cores": threads,
        "kind": "port",
        "sample": f"CPU oracle (torch {torch.__version__}, fp32 weights dequantized from the same Q8_0 / Q4_K bytes): "
                  f"one utterance's whole job, {t_job:.2f} s: the {ecfg.layers}-layer encoder and head over {frames} "
                  f"frames ({t_enc:.2f} s), the {len(ids)}-position prompt with its states through all "
                  f"{tcfg.layers} decoder layers ({t_prefill:.2f} s), {new_tokens} greedy tokens; a CPU runs the "
                  f"utterances one after another",
    }


if __name__ == "__main__":
    sys.exit(main())
