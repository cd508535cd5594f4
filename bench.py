"""Headline benchmark: batch-1 greedy decode tok/s of the Llama-3-8B-shaped
4-bit codebook model (the reference's headline decode configuration) on one
MI355X, plus the dequant-GEMV HBM bandwidth as a fraction of peak.

    python bench.py [--steps K] [--warmup W] [--config llama3-8b|qwen3-1.7b|qwen3-8b|llama3.2-3b|qwen3-4b|
                                                       qwen3-0.6b|h2560-i6656]

One "step" is one decode token: a replay of the captured HIP graph of the
whole decode step -- the one-launch decode-step kernel (all 32 layers: fused
q|k|v dequant-GEMV with RMSNorm, attention, o GEMV, gate|up GEMV with
SwiGLU, down GEMV; phases hand over through tagged data, no grid barrier)
and the lm_head/argmax launch.  The run is config 2's: the prompt (128
random ids) is consumed first, untimed; then 256 tokens are decoded: W
warm-up tokens, K timed tokens (the device synchronised on both sides), and
the rest untimed (W + K > 256 decodes W + K).  The line reports the timed
KV positions.  Weights are random-init in the packed format (synthetic data; no
checkpoints offline).  --per-layer times the five-launches-per-layer path
instead.

The roofline entry is for the dominant kernel, the decode-step kernel: it is
captured alone into a second graph (at the position after the timed ones)
and replayed K times between HIP events on the launch stream; achieved = its algorithmic
bytes (packed indices + group scales + codebooks of the 224 linears, RMSNorm
weights, and the KV rows attention reads at that position) / time per
replay.  `traffic` is the HBM bytes per launch of the same replays from the
FETCH_SIZE/WRITE_SIZE passes summarised in
profiles/decode_step_llama3_8b_traffic.md (calibrated against a copy of
known size; `--copy-probe` runs that copy).  The CPU baseline is the C
restatement of the reference's Rust kernel (oracle/rowdot.c,
kernel/src/lib.rs semantics) on one layer's 7 linears, scaled to the 224
linears of a step.  The line also carries `gemv`: the config-0 dequant-GEMV
(4096x4096 4-bit, batch 1) over 64 rotating weight sets, GB/s per launch.

    python bench.py --workload gemv|prefill|backward|experts

prints one line for the other configurations instead: config 0 alone (GEMV
GB/s, with the C port timed on the same linear), config 3 (the 8-bit M sweep;
GB/s and MFMA utilisation per case) and config 4 (the compressed-state
backward; TFLOP/s against the dense bf16 MFMA peak, indices hashed before and
after).
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
    ap.add_argument("--config", default="llama3-8b",
                    choices=["llama3-8b", "qwen3-1.7b", "qwen3-8b", "llama3.2-3b", "qwen3-4b",
                             "qwen3-0.6b", "h2560-i6656"])
    ap.add_argument("--prompt", type=int, default=None)
    ap.add_argument("--decode", type=int, default=None,
                    help="tokens decoded after the prompt (default: the configuration's, "
                         "256 for the 8B shape, 128 for Qwen3-1.7B); the timed steps lie "
                         "inside them, after the warm-up")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--per-layer", action="store_true",
                    help="five launches per layer instead of the one-launch step kernel")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only copy a BYTES-long device buffer 10 times (the known-size "
                         "kernel that calibrates rocprofv3's FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "gemv", "prefill", "backward", "experts"],
                    help="decode: the headline (config 2); gemv: one 4096x4096 4-bit GEMV "
                         "over a rotating sweep (config 0); prefill: the 8-bit M sweep "
                         "(config 3); backward: the compressed-state backward (config 4); "
                         "experts: a stacked-expert linear grouped on the device")
    ap.add_argument("--fused-backward", action="store_true",
                    help="backward: keep every token count on the fused kernels "
                         "(EPURE_BWD_FUSED=1) instead of the library route from 512 tokens")
    ap.add_argument("--no-gemv", action="store_true",
                    help="decode: skip the config-0 GEMV sweep reported beside the step")
    ap.add_argument("--phases", action="store_true",
                    help="decode: also replay the step kernel with wall-clock stamps and "
                         "report where a layer's time goes (per-phase breakdown)")
    return ap.parse_args()


# ---------------------------------------------------------------- standalone linears
class _Linear:
    """One packed linear bound to the C ABI with preallocated buffers, so a
    launch is graph-capturable (ep_dequant_matmul / ep_dequant_matmul_bwd)."""

    def __init__(self, store, x, out_dtype=None, bwd_gy=None):
        import torch
        from epure.kernels import _abi, cuda
        self.h = cuda._hot(store)
        self.x = x
        M, K = x.shape
        self.y = torch.empty((M, self.h.N), device=x.device, dtype=out_dtype or x.dtype)
        nb = _abi.lib.ep_dequant_matmul_workspace(M, self.h.N, K, self.h.levels, self.h.group)
        self.ws = torch.empty(max(nb, 256), device=x.device, dtype=torch.uint8)
        self.gy = bwd_gy
        if bwd_gy is not None:
            G = (K + self.h.group - 1) // self.h.group
            self.gx = torch.empty((M, K), device=x.device, dtype=torch.bfloat16)
            self.gcb = torch.empty(self.h.levels, device=x.device, dtype=torch.float32)
            self.gsc = torch.empty((self.h.N, G), device=x.device, dtype=torch.float32)
            nb = _abi.lib.ep_dequant_matmul_bwd_workspace(M, self.h.N, K, self.h.levels,
                                                          self.h.group)
            self.bws = torch.empty(max(nb, 256), device=x.device, dtype=torch.uint8)

    def fwd(self, stream):
        from epure.kernels import _abi
        h, x, y = self.h, self.x, self.y
        rc = _abi.lib.ep_dequant_matmul(
            x.data_ptr(), _abi.dtype_code(x.dtype), x.stride(0),
            h.packed.data_ptr(), h.scale.data_ptr(), h.scale_dt, h.ld_scale,
            h.cb.data_ptr(), h.cb_dt, h.levels, h.group, x.shape[0], h.N, x.shape[1],
            y.data_ptr(), _abi.dtype_code(y.dtype), y.stride(0), 0,
            self.ws.data_ptr(), self.ws.numel(), stream)
        if rc != 0:
            raise RuntimeError(f"ep_dequant_matmul: {rc} {_abi.last_error()}")

    def bwd(self, stream):
        from epure.kernels import _abi
        h, x, gy = self.h, self.x, self.gy
        M, K = x.shape
        rc = _abi.lib.ep_dequant_matmul_bwd(
            gy.data_ptr(), _abi.dtype_code(gy.dtype), gy.stride(0),
            x.data_ptr(), _abi.dtype_code(x.dtype), x.stride(0),
            h.packed.data_ptr(), h.scale.data_ptr(), h.scale_dt, h.ld_scale,
            h.cb.data_ptr(), h.cb_dt, h.levels, h.group, M, h.N, K,
            self.gx.data_ptr(), _abi.BF16, K, self.gcb.data_ptr(), self.gsc.data_ptr(),
            self.gsc.shape[1], self.bws.data_ptr(), self.bws.numel(), stream)
        if rc != 0:
            raise RuntimeError(f"ep_dequant_matmul_bwd: {rc} {_abi.last_error()}")


def _graph_time(launches, replays):
    """Captures `launches` (callables taking the stream handle) into one HIP
    graph and returns the mean ms per replay, timed with HIP events on the
    capture stream."""
    import ctypes
    import torch
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        h = ctypes.c_void_p(stream.cuda_stream)
        for f in launches:          # eager pass: warms caches of launch parameters
            f(h)
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for f in launches:
                f(h)
        g.replay()
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(replays):
            g.replay()
        e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / replays


def _spec(levels):
    from epure.decode import DecoderConfig
    return DecoderConfig(0, 0, 0, 1, 1, 128, 0, 1.0, levels=levels, group=128)


def _weight_bytes(n, k, levels, group=128):
    idx = n * k // 2 if levels <= 16 else n * k
    return idx + n * ((k + group - 1) // group) * 2 + levels * 4


def gemv_sweep(seed=0, sets=64, replays=20):
    """Config 0: y = x.W^T, W 4096x4096 4-bit (16-entry codebook, group-128
    fp16 scales), x bf16 [1, 4096].  `sets` distinct weight sets (64 x 8.65 MB
    = 553 MB, more than the 256 MB MALL holds) are launched round-robin from
    one graph, so every launch streams its weights from HBM."""
    import torch
    from epure.decode import _gen, random_packed_linear
    dev = torch.device("cuda:0")
    n = k = 4096
    gen = _gen(seed, dev)
    x = torch.randn(1, k, generator=gen, device=dev).to(torch.bfloat16)
    lins = [_Linear(random_packed_linear(n, k, _spec(16), gen, dev), x) for _ in range(sets)]
    ms = _graph_time([L.fwd for L in lins], replays) / sets
    wb = _weight_bytes(n, k, 16)
    gbs = wb / (ms * 1e-3) / 1e9
    return {"kernel": "gemv_row_kernel", "shape": "4096x4096 4-bit, M=1, bf16 x/y",
            "rotating_sets": sets, "us_per_launch": round(ms * 1e3, 3),
            "alg_bytes_per_launch": wb, "achieved_gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


MFMA_PEAK_TFLOPS = 2500.0


def read_probe(replays=10):
    """The practical read ceiling (ep_read_probe, the dequant kernels' load
    shape), best over 1-8 resident workgroups per CU: one 1 GiB launch per
    replay -> GB/s; and a config-0-sized launch (8,650,816 bytes, the
    4096x4096 4-bit weights) over 64 rotating buffers in one graph ->
    microseconds per launch."""
    import torch
    from epure.kernels import _abi
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.zeros(8 * cus, dtype=torch.int32, device=dev)

    def launch(buf, nbytes, grid):
        def f(stream):
            rc = _abi.lib.ep_read_probe(buf.data_ptr(), nbytes, sink.data_ptr(), grid, stream)
            if rc != 0:
                raise RuntimeError(f"ep_read_probe: {rc} {_abi.last_error()}")
        return f
    grids = [cus, 2 * cus, 4 * cus, 8 * cus]
    big = torch.ones(1 << 28, dtype=torch.int32, device=dev)          # 1 GiB
    big_ms = {g: _graph_time([launch(big, big.numel() * 4, g)], replays) for g in grids}
    del big
    c0 = _weight_bytes(4096, 4096, 16) // 16 * 16
    bufs = [torch.ones(c0 // 4, dtype=torch.int32, device=dev) for _ in range(64)]
    c0_ms = {g: _graph_time([launch(b, c0, g) for b in bufs], replays) / len(bufs) for g in grids}
    del bufs
    torch.cuda.empty_cache()
    gb = min(big_ms, key=big_ms.get)
    gc = min(c0_ms, key=c0_ms.get)
    return {"kernel": "read_probe_kernel",
            "ceiling_gbs": round((1 << 30) / (big_ms[gb] * 1e-3) / 1e9, 1),
            "ceiling_workgroups_per_cu": gb // cus,
            "ceiling_gbs_by_wg_per_cu": {g // cus: round((1 << 30) / (ms * 1e-3) / 1e9, 1)
                                         for g, ms in big_ms.items()},
            "config0_launch_bytes": c0, "config0_launch_us": round(c0_ms[gc] * 1e3, 3),
            "config0_launch_workgroups_per_cu": gc // cus,
            "config0_launch_gbs": round(c0 / (c0_ms[gc] * 1e-3) / 1e9, 1)}


def _dense_time(stores, x, replays):
    """The route the caller takes above EPURE_DENSE_ABOVE (runtime.py:117-126):
    materialize(bf16) -- one ep_dequant_tile launch into a preallocated
    [N, K] bf16 tile -- then torch.matmul (hipBLASLt), for each rotating
    weight set; ms per linear."""
    import torch
    from epure.kernels import _abi, cuda
    hs = [cuda._hot(s) for s in stores]
    w = torch.empty((hs[0].N, hs[0].K), device=x.device, dtype=torch.bfloat16)
    y = torch.empty((x.shape[0], hs[0].N), device=x.device, dtype=torch.bfloat16)

    def one(h):
        def f(stream):
            rc = _abi.lib.ep_dequant_tile(
                h.packed.data_ptr(), h.scale.data_ptr(), h.scale_dt, h.ld_scale,
                h.cb.data_ptr(), h.cb_dt, h.levels, h.group, h.N, h.K, w.data_ptr(),
                _abi.BF16, w.stride(0), stream)
            if rc != 0:
                raise RuntimeError(f"ep_dequant_tile: {_abi.last_error()}")
            torch.matmul(x, w.t(), out=y)
        return f
    return _graph_time([one(h) for h in hs], replays) / len(hs)


def _sk1_serves(m, n, cus):
    """Whether the one-launch small-M kernel serves a config-3 linear (8-bit
    indices, bf16 x, group 128): enough 16-row tiles for 3/4 of the CUs, at
    most 4 per CU, and M <= 16 x the tiles per workgroup (skinny.hip
    sk1_tiles_per_wg)."""
    tiles = (n + 15) // 16
    if tiles * 4 < cus * 3 or tiles > 4 * cus:
        return False
    t = next(t for t in (1, 2, 4) if tiles <= t * cus)
    return m <= 16 * t


def _sk2_serves(m, n, k):
    """Whether the register-resident split-K kernel serves a config-3 linear
    (8-bit indices, bf16 x, group 128): 17 <= M <= 64, at M > 32 or on layers
    of at least 2^25 weights (skinny.hip sk2_serves); it takes the rows
    before the one-launch kernel does."""
    return 17 <= m <= 64 and (m > 32 or n * k >= 2 ** 25)


def _row_serves(k, bits=8):
    """Whether the batch-1 row GEMV takes a row of K indices (gemv.hip
    row_kernel_slabs): rows of 4, 8, 12, 16, 24, 28 or 32 slabs of 256
    bytes, and 56 with 8-bit indices."""
    rb = k * bits // 8
    if rb % 256:
        return False
    s = rb // 256
    return s in (4, 8, 12, 16, 24, 28, 32) or (bits == 8 and s == 56)


def prefill_sweep(seed=0, replays=10):
    """Config 3: 8-bit indices (256-entry fp16-valued codebook, group-128 fp16
    scales), (N, K) in {4096x4096, 14336x4096, 4096x14336}, bf16 x with M in
    {1, 4, 16, 64, 512, 2048}.  Weight sets rotate so at least ~512 MB are
    touched per replay (HBM, not the MALL, serves the small-M cases)."""
    import torch
    from epure.decode import _gen, random_packed_linear
    dev = torch.device("cuda:0")
    gen = _gen(seed, dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    rows = []
    for n, k in [(4096, 4096), (14336, 4096), (4096, 14336)]:
        wb = _weight_bytes(n, k, 256)
        sets = max(1, -(-512 * 2 ** 20 // wb))
        stores = [random_packed_linear(n, k, _spec(256), gen, dev) for _ in range(sets)]
        for m in (1, 4, 16, 64, 512, 2048):
            x = torch.randn(m, k, generator=gen, device=dev).to(torch.bfloat16)
            lins = [_Linear(s, x) for s in stores]
            ms = _graph_time([L.fwd for L in lins], replays) / sets
            dense_ms = _dense_time(stores, x, replays)
            byt = wb + m * k * 2 + m * n * 2
            flop = 2.0 * m * n * k
            rows.append({"N": n, "K": k, "M": m, "us": round(ms * 1e3, 2),
                         "dense_us": round(dense_ms * 1e3, 2),
                         "gbs": round(byt / (ms * 1e-3) / 1e9, 1),
                         "hbm_frac": round(byt / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                         "tflops": round(flop / (ms * 1e-3) / 1e12, 2),
                         "mfma_frac": round(flop / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4),
                         "kernel": (("gemv_row_kernel" if _row_serves(k) else "gemv_lut_kernel")
                                    if m == 1 else
                                    "sk2_kernel (+ sk_reduce_kernel when K is split)"
                                    if _sk2_serves(m, n, k) else
                                    "sk1_kernel" if _sk1_serves(m, n, cus) else
                                    "sk_kernel + sk_reduce_kernel" if m <= 64 else
                                    "pf_prep_kernel + pf_kernel (+ sk_reduce_kernel when K is split)")})
            del lins, x
        del stores
        torch.cuda.empty_cache()
    return rows


def experts_sweep(seed=0, replays=10):
    """A stacked-expert packed linear of the size of a Qwen3-30B-A3B layer's
    expert gate (or up) projections: E = 128 experts of 768 x 2048, 4-bit
    (16-entry codebook, group-128 fp16 scales, 100.7 MB), bf16 x, tokens
    routed top-8 (T = 8 x tokens rows, ids uniform over the experts).  The
    device-grouped call (ids sorted on the device, one grouped MFMA launch)
    is timed inside a captured graph; the host-grouped route (a host
    synchronization, one launch per expert) eagerly with events."""
    import torch
    from epure import PackedExperts, PackedWeight
    from epure.decode import _gen, random_packed_linear
    dev = torch.device("cuda:0")
    gen = _gen(seed, dev)
    E, n, k = 128, 768, 2048
    flat = random_packed_linear(E * n, k, _spec(16), gen, dev)
    store = PackedWeight((E, n, k), flat.packed, flat.scale, flat.cb, flat.group, flat.levels)
    wbytes = _weight_bytes(E * n, k, 16)
    rows = []
    for tokens in (16, 128, 512, 2048):
        T = 8 * tokens
        x = torch.randn(T, k, generator=gen, device=dev).to(torch.bfloat16)
        ids = torch.randint(0, E, (T,), generator=gen, device=dev, dtype=torch.int32)
        m = PackedExperts(store, check_ids=False)
        ms = _graph_time([lambda h: m(x, ids)], replays)
        host = PackedExperts(store, check_ids=False)
        host.GROUP_ON_DEVICE = False
        host(x, ids)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(replays):
            host(x, ids)
        e1.record()
        e1.synchronize()
        host_ms = e0.elapsed_time(e1) / replays
        used = int(torch.unique(ids).numel())
        flop = 2.0 * T * n * k
        byt = wbytes * used / E + T * k * 2 + T * n * 2
        rows.append({"tokens": tokens, "rows": T, "experts_used": used, "us": round(ms * 1e3, 2),
                     "host_grouped_us": round(host_ms * 1e3, 2),
                     "tflops": round(flop / (ms * 1e-3) / 1e12, 2),
                     "mfma_frac": round(flop / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4),
                     "gbs": round(byt / (ms * 1e-3) / 1e9, 1),
                     "hbm_frac": round(byt / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
        del x, ids
    return rows


def backward_sweep(seed=0, replays=10):
    """Config 4: grad_x, grad_codebook and grad_scales of one 2048x6144 and one
    6144x2048 packed linear (4-bit, 16 levels, group 128), x bf16 [2048, K]
    ~ N(0, 1), gy bf16 [2048, N] ~ N(0, 1e-2).  The indices are hashed before
    and after: they must be bit-identical."""
    import hashlib
    import torch
    from epure.decode import _gen, random_packed_linear
    dev = torch.device("cuda:0")
    gen = _gen(seed, dev)
    t = 2048
    rows = []
    for n, k in [(2048, 6144), (6144, 2048)]:
        s = random_packed_linear(n, k, _spec(16), gen, dev)
        x = torch.randn(t, k, generator=gen, device=dev).to(torch.bfloat16)
        gy = (torch.randn(t, n, generator=gen, device=dev) * 1e-2).to(torch.bfloat16)
        digest = lambda: hashlib.blake2b(s.packed.cpu().numpy().tobytes(),  # noqa: E731
                                         digest_size=16).hexdigest()
        before = digest()
        L = _Linear(s, x, bwd_gy=gy)
        ms = _graph_time([L.bwd], replays)
        flop = 4.0 * t * n * k
        rows.append({"N": n, "K": k, "T": t, "us": round(ms * 1e3, 2),
                     "tflops": round(flop / (ms * 1e-3) / 1e12, 2),
                     "mfma_frac": round(flop / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4),
                     "indices_frozen": digest() == before})
    return rows


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


# Wall-clock stamps decode_step_kernel writes when given a trace buffer
# (csrc/step.hip, stamp(a, layer, id)): [layers][24][workgroups] at 100 MHz.
_STAMPS = 24
_PHASE_EVENTS = [(1, "qkv done"), (10, "attention: q/k/v received"),
                 (11, "attention: item computed"), (12, "attention: output combined"),
                 (3, "o: activations staged"), (4, "o: done"),
                 (5, "gate|up: activations staged"), (6, "gate|up: done"),
                 (7, "down: activations staged"), (8, "down: done")]


def phase_breakdown(dec, cfg, replays=4):
    """One-launch step replayed with stamps at the current position: per
    event, the median over layers of (median and last workgroup's stamp)
    minus the layer's start (the last workgroup to begin it), in us; the
    layer period; and per hand-over, the last producer -> median consumer
    time and the producer skew (last minus median producer)."""
    import numpy as np
    import torch
    G = torch.cuda.get_device_properties(dec.device).multi_processor_count
    dec.step_trace = torch.zeros(cfg.layers * _STAMPS * G, dtype=torch.int64, device=dec.device)
    for _ in range(replays):  # the last replay's stamps are kept
        dec.step_trace.zero_()
        dec.layer_launches()
    torch.cuda.synchronize()
    tr = dec.step_trace.view(cfg.layers, _STAMPS, G).cpu().numpy().astype(np.float64) * 0.01
    dec.step_trace = None
    L = slice(2, cfg.layers - 1)  # steady-state layers
    start = tr[L, 0, :].max(axis=1, keepdims=True)

    def stat(ev, f):
        x = np.where(tr[L, ev, :] > 0, tr[L, ev, :] - start, np.nan)
        return float(np.nanmedian(f(x)))
    med = lambda x: np.nanmedian(x, axis=1)
    last = lambda x: np.nanmax(x, axis=1)
    out = {"position": int(dec.state[0].item()), "layers": [2, cfg.layers - 2],
           "layer_period_us": round(float(np.median(np.diff(tr[1:, 0, :].max(axis=1)))), 2),
           "events_us": {n: {"median_wg": round(stat(e, med), 2), "last_wg": round(stat(e, last), 2)}
                         for e, n in _PHASE_EVENTS}}
    hops = {}
    for name, pe, ce in [("q|k|v -> attention", 1, 10), ("attention -> o", 12, 3),
                         ("o -> gate|up", 4, 5), ("gate|up -> down", 6, 7)]:
        p = np.where(tr[L, pe, :] > 0, tr[L, pe, :], np.nan)
        c = np.where(tr[L, ce, :] > 0, tr[L, ce, :], np.nan)
        lp = np.nanmax(p, axis=1)
        hops[name] = {"last_producer_to_median_consumer_us": round(float(np.median(np.nanmedian(c, axis=1) - lp)), 2),
                      "last_producer_to_first_consumer_us": round(float(np.median(np.nanmin(c, axis=1) - lp)), 2),
                      "producer_skew_us": round(float(np.median(lp - np.nanmedian(p, axis=1))), 2)}
    out["hand_overs"] = hops
    return out


def cpu_model():
    """The host CPU's model name (Linux /proc/cpuinfo)."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, threads):
    """Reference Rust kernel semantics (C port) on one layer's 7 packed
    linears; tok/s ceiling = 1 / (time per layer * layers), on all host
    threads and on one."""
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

    def timed(threads_used, budget_s):
        def layer():
            for x, p, s, c in data:
                rowdot.dequant_matmul(x, p, s, c, cfg.group, True, nthreads=threads_used)
        layer()                                   # warm-up
        times = []
        t_end = time.perf_counter() + budget_s
        while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 20):
            t0 = time.perf_counter()
            layer()
            times.append(time.perf_counter() - t0)
        return float(np.median(times)), len(times)

    t_layer, runs = timed(nt, 10.0)
    t_one, runs_one = timed(1, 8.0)
    return {"value": round(1.0 / (t_layer * cfg.layers), 4), "unit": "tok/s", "cores": nt,
            "kind": "port", "cpu_model": cpu_model(),
            "value_1_thread": round(1.0 / (t_one * cfg.layers), 4),
            "sample": f"C port of kernel/src/lib.rs on one layer's 7 packed linears "
                      f"({sum(n * k for _, n, k in shapes) / 1e6:.0f}M weights, f32 x): median "
                      f"{t_layer * 1e3:.1f} ms over {runs} runs on {nt} threads, median "
                      f"{t_one * 1e3:.1f} ms over {runs_one} runs on 1 thread; scaled "
                      f"x{cfg.layers} layers (linears only, lm_head excluded)"}


def cpu_gemv_baseline(n, k, levels, ms, threads):
    """The C port of the reference Rust kernel (kernel/src/lib.rs) on one
    N x K linear with M rows of f32 x (bf16-valued): GB/s of packed weights."""
    import numpy as np
    from oracle import ref, rowdot
    _, packed, scale, cb = ref.synth_linear(n, k, levels, 128, seed=0)
    row = k // 2 if levels <= 16 else k
    rng = np.random.Generator(np.random.PCG64(1))
    nt = threads or rowdot.threads()
    out = []
    for m in ms:
        x = ref.round_bf16(rng.standard_normal((m, k)).astype(np.float32))
        args = (x, packed.reshape(n, row), scale.astype(np.float32), cb.astype(np.float32), 128,
                levels <= 16)
        rowdot.dequant_matmul(*args, nthreads=nt)
        times = []
        t_end = time.perf_counter() + 4.0
        while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 20):
            t0 = time.perf_counter()
            rowdot.dequant_matmul(*args, nthreads=nt)
            times.append(time.perf_counter() - t0)
        t = float(np.median(times))
        out.append((m, t, len(times)))
    wb = _weight_bytes(n, k, levels)
    m, t, runs = out[0]
    return {"value": round(wb / t / 1e9, 3), "unit": "GB/s", "cores": nt, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"C port of kernel/src/lib.rs, {n}x{k} {'4' if levels <= 16 else '8'}-bit "
                      f"linear, f32 x; " + "; ".join(
                          f"M={m_}: {t_ * 1e3:.2f} ms (median of {r_})" for m_, t_, r_ in out)}


def side_workload(args):
    """The non-headline configurations: one JSON line each."""
    base = {"n_gpus": 1, "steps": args.steps, "warmup": 2, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "data": "synthetic"}
    if args.workload == "gemv":
        g = gemv_sweep(args.seed, replays=args.steps)
        out = dict(metric="dequant-GEMV HBM GB/s (4096x4096 4-bit, batch 1)",
                   value=g["achieved_gbs"], unit="GB/s", ms_per_step=g["us_per_launch"] / 1e3,
                   dtype="f16", **base)
        out["config"] = {"workload": "config 0: one 4096x4096 4-bit packed linear, x bf16 [1,4096], "
                                     f"{g['rotating_sets']} rotating weight sets", **g}
        probe = read_probe()
        out["roofline"] = {"bound": "hbm", "kernel": g["kernel"], "achieved": g["achieved_gbs"],
                           "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": g["frac"],
                           "traffic": None, "probe": probe,
                           "frac_of_probe_launch": round(probe["config0_launch_us"]
                                                         / g["us_per_launch"], 4)}
        if not args.no_cpu_baseline:
            out["cpu_baseline"] = cpu_gemv_baseline(4096, 4096, 16, [1], args.cpu_threads)
    elif args.workload == "prefill":
        rows = prefill_sweep(args.seed, replays=min(args.steps, 20))
        top = max(rows, key=lambda r: r["tflops"])
        out = dict(metric="8-bit packed linear prefill sweep: TFLOP/s (large M), GB/s (small M)",
                   value=top["tflops"], unit="TFLOP/s", ms_per_step=top["us"] / 1e3,
                   dtype="f16", **base)
        # the smallest M from which the dense route wins at every shape
        ms_sorted = sorted({r["M"] for r in rows})
        cross = next((m for m in ms_sorted
                      if all(r["dense_us"] < r["us"] for r in rows if r["M"] >= m)), None)
        out["config"] = {"workload": "config 3: 8-bit codebook (256 levels), group 128; "
                                     "(N,K) in {4096x4096, 14336x4096, 4096x14336}, "
                                     "M in {1,4,16,64,512,2048}", "rows": rows,
                         "dense_route": "materialize(bf16) via ep_dequant_tile + torch.matmul",
                         "dense_wins_from_M": cross}
        out["roofline"] = {"bound": "mfma", "kernel": top["kernel"],
                           "achieved": top["tflops"], "peak": MFMA_PEAK_TFLOPS,
                           "unit": "TFLOP/s", "frac": top["mfma_frac"], "traffic": None,
                           "case": f"N={top['N']} K={top['K']} M={top['M']}"}
        if not args.no_cpu_baseline:
            out["cpu_baseline"] = cpu_gemv_baseline(4096, 4096, 256, [1, 4, 16],
                                                    args.cpu_threads)
    elif args.workload == "experts":
        rows = experts_sweep(args.seed, replays=min(args.steps, 20))
        top = max(rows, key=lambda r: r["tflops"])
        out = dict(metric="stacked-expert packed linear, device-grouped: TFLOP/s",
                   value=top["tflops"], unit="TFLOP/s", ms_per_step=top["us"] / 1e3,
                   dtype="f16", **base)
        out["config"] = {"workload": "128 experts x 768 x 2048 4-bit (Qwen3-30B-A3B expert gate/up "
                                     "size), bf16 x, top-8 routed rows, uniform ids",
                         "kernel": "expert_sort_kernel + row_exp_kernel + mm_kernel (grouped)",
                         "rows": rows}
        out["roofline"] = {"bound": "mfma", "kernel": "mm_kernel (grouped)", "achieved": top["tflops"],
                           "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": top["mfma_frac"],
                           "traffic": None, "case": f"rows={top['rows']}"}
        out["cpu_baseline"] = None  # the reference materializes the slab (no CPU expert kernel)
    else:
        rows = backward_sweep(args.seed, replays=min(args.steps, 20))
        flop = sum(4.0 * r["T"] * r["N"] * r["K"] for r in rows)
        us = sum(r["us"] for r in rows)
        tf = flop / (us * 1e-6) / 1e12
        out = dict(metric="compressed-state backward TFLOP/s (grad_x + implicit grad_W)",
                   value=round(tf, 2), unit="TFLOP/s", ms_per_step=round(us / 1e3, 4),
                   dtype="bf16", **base)
        out["config"] = {"workload": "config 4: 2048x6144 and 6144x2048 4-bit packed linears, "
                                     "T=2048, grad_x + grad_codebook + grad_scales",
                         "rows": rows,
                         "indices_frozen": all(r["indices_frozen"] for r in rows)}
        # T = 2048 takes the library route: two hipBLASLt GEMMs (grad_x, G = gy^T x)
        # around this library's prescale, materialize, finish and codebook-epilogue
        # kernels, the two chains on two streams; --fused-backward the fused kernels
        out["config"]["route"] = "fused" if args.fused_backward else "library"
        out["roofline"] = {"bound": "mfma",
                           "kernel": ("gy_prep_kernel + dx_kernel + dw_kernel + gc_final_kernel"
                                      if args.fused_backward else
                                      "hipBLASLt GEMMs + gy_prep/dequant_tile4/dx_finish/gw_epilogue/gc_final"),
                           "achieved": round(tf, 2), "peak": MFMA_PEAK_TFLOPS,
                           "unit": "TFLOP/s", "frac": round(tf / MFMA_PEAK_TFLOPS, 4),
                           "traffic": None}
        out["cpu_baseline"] = None  # the reference backward is torch autograd, no CPU kernel
    print(json.dumps(out), flush=True)


def main():
    args = parse()
    if args.fused_backward:
        os.environ["EPURE_BWD_FUSED"] = "1"  # read by the library on its first backward call
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this build has "
              "no multi-GPU path: column-parallel linears would shard by rows with no "
              "exchange, row-parallel ones by K with one all-reduce).", file=sys.stderr)
        sys.exit(2)
    if args.workload != "decode":
        side_workload(args)
        return

    import torch
    from epure.decode import CONFIGS, Decoder, random_weights

    cfg = CONFIGS[args.config]
    n_prompt = args.prompt or (32 if args.config == "qwen3-1.7b" else 128)
    # configs 1 and 2: the prompt, then 128 / 256 greedy tokens; W warm-up
    # and K timed tokens are the first W + K of them, the rest decoded after
    # (untimed), so the run is the configuration's whole decode
    n_decode = args.decode or (128 if args.config == "qwen3-1.7b" else 256)
    n_dec = max(n_decode, args.warmup + args.steps)
    dev = torch.device("cuda:0")
    print(f"# building {cfg.name} random weights (seed {args.seed})", file=sys.stderr, flush=True)
    w = random_weights(cfg, seed=args.seed, device=dev)
    total_steps = n_prompt - 1 + n_dec
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

    # dominant kernel alone: the layers of one step (one launch, or the 160
    # per-layer launches), replayed at the next position between events on
    # the launch stream.  The replays overwrite the residual input (the next
    # token's embedding) and that position's KV rows: the input is saved and
    # restored, and the next real step rewrites the rows.
    stream = torch.cuda.current_stream()
    h_saved = dec.h.clone()
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
    dec.h.copy_(h_saved)
    torch.cuda.synchronize()
    rest = n_dec - args.warmup - args.steps
    print(f"# decoding the remaining {rest} tokens (untimed)", file=sys.stderr, flush=True)
    for _ in range(rest):
        dec.step()
    torch.cuda.synchronize()
    toks = dec.tokens[:n_prompt + n_dec].cpu().tolist()
    if dec.step_failed():
        raise RuntimeError("a hand-over wait of the decode-step kernel timed out")
    packed = w.packed_bytes()
    norm_bytes = sum(t.numel() * 2 for L in w.layers
                     for t in (L.attn_norm, L.mlp_norm, L.q_norm, L.k_norm) if t is not None)
    # the replayed step reads KV rows 0..pos-1 from the f32 cache
    kv_bytes = 2 * cfg.layers * cfg.n_kv * pos * cfg.head_dim * 4
    alg = packed + norm_bytes + kv_bytes
    kern_gbs = alg / (kern_ms * 1e-3) / 1e9
    step_ms = dt / args.steps * 1e3
    # whole-model bytes a token must read: the packed linears, the bf16
    # lm_head (the tied embedding when tied), the norm weights and ONE
    # embedding row (the step gathers a single row of the table)
    lm_bytes = w.lm_head.numel() * 2
    model_bytes = packed + lm_bytes + norm_bytes + w.final_norm.numel() * 2 + cfg.hidden * 2
    first_pos = n_prompt - 1 + args.warmup
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
            "vocab": cfg.vocab, "prompt": n_prompt, "decoded": n_dec,
            "packed_linear_bytes": packed, "model_bytes_per_token": model_bytes,
            "step_gbs_model": round(model_bytes / (step_ms * 1e-3) / 1e9, 1),
            "step_frac_model": round(model_bytes / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "step_frac_packed": round(packed / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "timed_kv_positions": [first_pos, first_pos + args.steps - 1],
            "layers_path": "per-layer launches" if args.per_layer else "one-launch step kernel",
            "layers_ms_per_step": round(kern_ms, 4),
            "layers_alg_bytes": alg,
            "layers_kv_position": pos,
            "first_tokens": toks[n_prompt:n_prompt + 8],
            "last_tokens": toks[n_prompt + n_dec - 8:n_prompt + n_dec],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_step_kernel" if not args.per_layer else "per-layer launches",
            "achieved": round(kern_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(kern_gbs / HBM_PEAK_GBS, 4),
            "traffic": None if args.per_layer else traffic_from_profile(),
            "traffic_source": None if args.per_layer else
            "profiles/decode_step_llama3_8b_traffic.md: rocprofv3 FETCH_SIZE and WRITE_SIZE passes "
            "over this command's roofline replays (its final KV position is stated there), "
            "calibrated by bench.py --copy-probe; not measured in this run",
        },
    }
    if args.phases and dec.persistent:
        print("# per-phase breakdown (stamped replays)", file=sys.stderr, flush=True)
        out["phases"] = phase_breakdown(dec, cfg)
    del dec, w, g
    torch.cuda.empty_cache()
    print("# streaming-read probe", file=sys.stderr, flush=True)
    probe = read_probe()
    out["roofline"]["probe"] = probe
    out["roofline"]["frac_of_probe"] = round(kern_gbs / probe["ceiling_gbs"], 4)
    if not args.no_gemv:
        print("# config-0 GEMV sweep", file=sys.stderr, flush=True)
        out["gemv"] = gemv_sweep(args.seed)
        out["gemv"]["frac_of_probe_launch"] = round(probe["config0_launch_us"]
                                                    / out["gemv"]["us_per_launch"], 4)
    if not args.no_cpu_baseline:
        print("# CPU baseline (reference Rust semantics, C port)", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(cfg, args.cpu_threads)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
