"""Headline benchmark: batch-1 greedy decode tok/s of the Llama-3-8B-shaped
4-bit codebook model (the reference's headline decode configuration) on one
MI355X, plus the dequant-GEMV HBM bandwidth as a fraction of peak.

    python bench.py [--steps K] [--warmup W] [--config llama3-8b|qwen3-1.7b]

One "step" is one decode token: a replay of the captured HIP graph of the
whole decode step -- the one-launch decode-step kernel (all 32 layers: fused
q|k|v dequant-GEMV with RMSNorm, attention, o GEMV, gate|up GEMV with
SwiGLU, down GEMV; phases hand over through tagged data, no grid barrier)
and the lm_head/argmax launch.  The prompt (128 random ids) is consumed
first, untimed; then W warm-up tokens, then K timed tokens, with the device
synchronised on both sides.  Weights are random-init in the packed format (synthetic data; no
checkpoints offline).  --per-layer times the five-launches-per-layer path
instead.

The roofline entry is for the dominant kernel, the decode-step kernel: it is
captured alone into a second graph (at the final position) and replayed K
times between HIP events on the launch stream; achieved = its algorithmic
bytes (packed indices + group scales + codebooks of the 224 linears, RMSNorm
weights, and the KV rows attention reads at that position) / time per
replay.  `traffic` is the HBM bytes per launch of the same replays from the
FETCH_SIZE/WRITE_SIZE passes summarised in
profiles/decode_step_llama3_8b_traffic.md (calibrated against a copy of
known size; `--copy-probe` runs that copy).  The CPU baseline is the C
restatement of the reference's Rust kernel (oracle/rowdot.c,
kernel/src/lib.rs semantics) on one layer's 7 linears, scaled to the 224
linears of a step.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "epure-runtime_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
METRIC = "batch-1 decode tok/s at 8B shape; dequant-GEMV HBM GB/s as % of peak"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", default="llama3-8b", choices=["llama3-8b", "qwen3-1.7b"])
    ap.add_argument("--prompt", type=int, default=None)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--per-layer", action="store_true",
                    help="five launches per layer instead of the one-launch step kernel")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only copy a BYTES-long device buffer 10 times (the known-size "
                         "kernel that calibrates rocprofv3's FETCH_SIZE/WRITE_SIZE)")
    return ap.parse_args()


def copy_probe(nbytes):
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": nbytes, "copies": 10}), flush=True)


def traffic_from_profile():
    """HBM bytes per launch of the step kernel, as measured by the
    FETCH_SIZE/WRITE_SIZE passes summarised in profiles/ (None if absent)."""
    path = os.path.join(ROOT, "profiles", "decode_step_llama3_8b_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def cpu_baseline(cfg, threads):
    """Reference Rust kernel semantics (C port) on one layer's 7 packed
    linears; tok/s ceiling = 1 / (time per layer * layers)."""
    import numpy as np
    from oracle import ref, rowdot
    shapes = cfg.packed_linear_shapes()
    data = []
    for j, (name, n, k) in enumerate(shapes):
        _, packed, scale, cb = ref.synth_linear(n, k, cfg.levels, cfg.group, seed=100 + j)
        x = ref.round_bf16(np.random.Generator(np.random.PCG64(j)).standard_normal(
            (1, k)).astype(np.float32))
        data.append((x, packed.reshape(n, k // 2), scale.astype(np.float32),
                     cb.astype(np.float32)))
    nt = threads or rowdot.threads()

    def layer():
        for x, p, s, c in data:
            rowdot.dequant_matmul(x, p, s, c, cfg.group, True, nthreads=nt)
    layer()                                       # warm-up
    times = []
    t_end = time.perf_counter() + 10.0
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 20):
        t0 = time.perf_counter()
        layer()
        times.append(time.perf_counter() - t0)
    t_layer = float(np.median(times))
    return {"value": round(1.0 / (t_layer * cfg.layers), 4), "unit": "tok/s", "cores": nt,
            "kind": "port",
            "sample": f"C port of kernel/src/lib.rs on one layer's 7 packed linears "
                      f"({sum(n * k for _, n, k in shapes) / 1e6:.0f}M weights, f32 x), median of "
                      f"{len(times)} runs = {t_layer * 1e3:.1f} ms, scaled x{cfg.layers} layers "
                      f"(linears only, lm_head excluded)"}


def main():
    args = parse()
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this build has "
              "no multi-GPU path: column-parallel linears would shard by rows with no "
              "exchange, row-parallel ones by K with one all-reduce).", file=sys.stderr)
        sys.exit(2)

    import torch
    from epure.decode import LLAMA3_8B, QWEN3_1_7B, Decoder, random_weights
    from epure.kernels import _abi

    cfg = {"llama3-8b": LLAMA3_8B, "qwen3-1.7b": QWEN3_1_7B}[args.config]
    n_prompt = args.prompt or (128 if args.config == "llama3-8b" else 32)
    dev = torch.device("cuda:0")
    print(f"# building {cfg.name} random weights (seed {args.seed})", file=sys.stderr, flush=True)
    w = random_weights(cfg, seed=args.seed, device=dev)
    total_steps = n_prompt - 1 + args.warmup + args.steps
    dec = Decoder(w, total_steps + 2, persistent=False if args.per_layer else None)
    import numpy as np
    prompt = np.random.Generator(np.random.PCG64(args.seed + 1)).integers(
        0, cfg.vocab, n_prompt).tolist()
    dec.reset(prompt)
    dec.capture()
    for _ in range(n_prompt - 1):
        dec.step()
    for _ in range(args.warmup):
        dec.step()
    torch.cuda.synchronize()
    print(f"# prompt + warm-up done; timing {args.steps} decode steps", file=sys.stderr,
          flush=True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        dec.step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    tok_s = args.steps / dt
    toks = dec.tokens[:n_prompt + args.warmup + args.steps].cpu().tolist()

    if dec.step_failed():
        raise RuntimeError("a grid barrier of the decode-step kernel timed out")

    # dominant kernel alone: the layers of one step (one launch, or the 160
    # per-layer launches), replayed at the final position between events on
    # the launch stream
    stream = torch.cuda.current_stream()
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        dec.layer_launches()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        for _ in range(args.steps):
            g.replay()
        e1.record(stream)
    e1.synchronize()
    kern_ms = e0.elapsed_time(e1) / args.steps
    pos = int(dec.state[0].item())
    packed = w.packed_bytes()
    norm_bytes = sum(t.numel() * 2 for L in w.layers
                     for t in (L.attn_norm, L.mlp_norm, L.q_norm, L.k_norm) if t is not None)
    kv_bytes = 2 * cfg.layers * cfg.n_kv * pos * cfg.head_dim * 2
    alg = packed + norm_bytes + kv_bytes
    kern_gbs = alg / (kern_ms * 1e-3) / 1e9
    resident = w.resident_bytes()
    step_ms = dt / args.steps * 1e3

    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": f"{cfg.name}-shaped batch-1 greedy decode, 4-bit codebook packed "
                        f"linears (16-entry cb, group {cfg.group}), bf16 embed/lm_head, "
                        f"prompt {n_prompt}",
            "layers": cfg.layers, "hidden": cfg.hidden, "intermediate": cfg.intermediate,
            "vocab": cfg.vocab, "prompt": n_prompt, "decoded": args.warmup + args.steps,
            "packed_linear_bytes": packed, "resident_weight_bytes": resident,
            "step_hbm_gbs_resident": round(resident / (step_ms * 1e-3) / 1e9, 1),
            "step_frac_resident": round(resident / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "step_frac_packed": round(packed / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "layers_path": "per-layer launches" if args.per_layer else "one-launch step kernel",
            "layers_ms_per_step": round(kern_ms, 4),
            "layers_alg_bytes": alg,
            "layers_kv_position": pos,
            "first_tokens": toks[n_prompt:n_prompt + 8],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_step_kernel" if not args.per_layer else "per-layer launches",
            "achieved": round(kern_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(kern_gbs / HBM_PEAK_GBS, 4),
            "traffic": None if args.per_layer else traffic_from_profile(),
        },
    }
    if not args.no_cpu_baseline:
        print("# CPU baseline (reference Rust semantics, C port)", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(cfg, args.cpu_threads)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
