"""Batch-1 greedy decode of a packed decoder on the gfx950 kernels.

This is the caller of the packed linears that the reference leaves to
transformers (epure/runtime.py:373-415 builds a LlamaForCausalLM /
Qwen3ForCausalLM whose linears are PackedLinear; generation runs through
``model.generate``, benchmarks/run.py:48-73).  Here one decode step is five
launches per layer, all through the C ABI of include/epure_decode.h:

    fused q|k|v GEMV   (RMSNorm of the residual fused into the activation load)
    attention          (q/k norm, RoPE, KV append, split-KV softmax)
    o GEMV             (accumulates into the f32 residual)
    fused gate|up GEMV (RMSNorm fused)
    down GEMV          (SwiGLU fused into the activation load; accumulates)

plus one lm_head launch (final norm, bf16 GEMV, greedy argmax, next-token
embedding).  The token position lives in device memory, so the step is
captured once as a HIP graph and replayed per token.

Weights are random-init (there is no network for checkpoints), seeded, in
the reference's packed format: 4-bit indices two per byte, a 16-entry
fp16-valued codebook per linear (16 sorted N(0, 1) draws, centred: their
mean is subtracted before the fp16 rounding; stored fp32 as the container
does), group-128 fp16 scales |N(0, 0.02)| + 1e-3; embeddings and lm_head
bf16 N(0, 0.02); norm weights 1.

Why the codebook is centred: with uniform indices and positive scales an
uncentred codebook gives every row the mean mean(cb) * scale, so each linear
maps the all-ones direction to itself with gain ~ mean(cb) * mean(scale) * K
(about 17 at K = 4096).  Within a few layers that one direction owns the
residual stream, every position produces the same logits and greedy decode
repeats one token -- a parity check on such a model compares a constant.
Centring keeps the bytes, the format and the kernels' work identical.
"""
import ctypes
import math
from dataclasses import dataclass, field

import torch

from .kernels import _abi
from .kernels import cuda as cuda_kernel
from .runtime import PackedWeight


@dataclass(frozen=True)
class DecoderConfig:
    hidden: int
    intermediate: int
    layers: int
    n_heads: int
    n_kv: int
    head_dim: int
    vocab: int
    rope_theta: float
    rms_eps: float = 1e-5
    qk_norm: bool = False
    tie_embeddings: bool = False
    levels: int = 16
    group: int = 128
    name: str = "decoder"

    def packed_linear_shapes(self):
        """(name, N, K) of the packed linears of one layer."""
        h, i, d = self.hidden, self.intermediate, self.head_dim
        return [("q", self.n_heads * d, h), ("k", self.n_kv * d, h), ("v", self.n_kv * d, h),
                ("o", h, self.n_heads * d), ("gate", i, h), ("up", i, h), ("down", h, i)]


# Decoder shapes with tuned one-launch variants: the two benchmark
# configurations (Llama-3-8B, Qwen3-1.7B), Qwen3-8B (the shape of the
# reference's own headline model, CHANGELOG.md:54-56: 36 layers,
# intermediate 12288), Llama-3.2-3B and Qwen3-4B (query width 4096 over
# hidden 2560).
LLAMA3_8B = DecoderConfig(4096, 14336, 32, 32, 8, 128, 128256, 5e5, 1e-5, name="llama3-8b")
QWEN3_1_7B = DecoderConfig(2048, 6144, 28, 16, 8, 128, 151936, 1e6, 1e-6, qk_norm=True,
                           tie_embeddings=True, name="qwen3-1.7b")
QWEN3_8B = DecoderConfig(4096, 12288, 36, 32, 8, 128, 151936, 1e6, 1e-6, qk_norm=True,
                         name="qwen3-8b")
LLAMA32_3B = DecoderConfig(3072, 8192, 28, 24, 8, 128, 128256, 5e5, 1e-5, tie_embeddings=True,
                           name="llama3.2-3b")
QWEN3_4B = DecoderConfig(2560, 9728, 36, 32, 8, 128, 151936, 1e6, 1e-6, qk_norm=True,
                         tie_embeddings=True, name="qwen3-4b")
# Shapes outside that list run the generic one-launch variants (hidden and
# query width up to 4096, intermediate up to 16384, multiples of 512, up to
# 8 query heads per kv head): e.g. the Qwen3-0.6B shape and a Llama-style
# 2560 / 6656 decoder with 5 query heads per kv head.
QWEN3_0_6B = DecoderConfig(1024, 3072, 28, 16, 8, 128, 151936, 1e6, 1e-6, qk_norm=True,
                           tie_embeddings=True, name="qwen3-0.6b")
H2560_I6656 = DecoderConfig(2560, 6656, 30, 20, 4, 128, 32000, 1e6, 1e-5, name="h2560-i6656")
CONFIGS = {c.name: c for c in (LLAMA3_8B, QWEN3_1_7B, QWEN3_8B, LLAMA32_3B, QWEN3_4B, QWEN3_0_6B,
                                H2560_I6656)}


def rope_tables(cfg, max_pos, device):
    """cos/sin [max_pos, head_dim/2] f32, computed as transformers does
    (LlamaRotaryEmbedding: inv_freq = theta^(-2i/d) in f32, freqs = pos * inv_freq)."""
    d = cfg.head_dim
    inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
    pos = torch.arange(max_pos, dtype=torch.int64).float()
    freqs = pos[:, None] * inv_freq[None, :]
    return freqs.cos().contiguous().to(device), freqs.sin().contiguous().to(device)


def _gen(seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def random_packed_linear(n, k, cfg, gen, device, center=True):
    """One packed weight: uniform indices, sorted N(0, 1) fp16-valued codebook
    (mean removed when ``center``), |N(0, 0.02)| + 1e-3 fp16 group scales."""
    nbytes = n * k // 2 if cfg.levels <= 16 else n * k
    hi = 256 if cfg.levels in (16, 256) else None
    if hi is None:
        raise ValueError("random weights are generated for 16 or 256 levels")
    packed = torch.randint(0, hi, (nbytes,), generator=gen, device=device, dtype=torch.uint8)
    cb = torch.sort(torch.randn(cfg.levels, generator=gen, device=device)).values
    if center:
        cb = cb - cb.mean()
    cb = cb.half().float()
    g = (k + cfg.group - 1) // cfg.group
    scale = (torch.randn(n, g, generator=gen, device=device).abs() * 0.02 + 1e-3).half()
    return PackedWeight((n, k), packed, scale, cb, cfg.group, cfg.levels)


@dataclass
class Layer:
    attn_norm: torch.Tensor
    mlp_norm: torch.Tensor
    lin: dict
    q_norm: torch.Tensor = None
    k_norm: torch.Tensor = None


@dataclass
class DecoderWeights:
    cfg: DecoderConfig
    embed: torch.Tensor
    lm_head: torch.Tensor
    final_norm: torch.Tensor
    layers: list = field(default_factory=list)

    def packed_bytes(self):
        return sum(s.packed.numel() + s.scale.numel() * s.scale.element_size()
                   + s.cb.numel() * s.cb.element_size()
                   for L in self.layers for s in L.lin.values())

    def resident_bytes(self):
        lm = 0 if self.cfg.tie_embeddings else self.lm_head.numel() * 2
        norms = sum(t.numel() * 2 for L in self.layers
                    for t in (L.attn_norm, L.mlp_norm, L.q_norm, L.k_norm) if t is not None)
        return self.packed_bytes() + lm + self.embed.numel() * 2 + norms + \
            self.final_norm.numel() * 2


def random_weights(cfg, seed=0, device="cuda", center=True):
    device = torch.device(device)
    gen = _gen(seed, device)
    h = cfg.hidden
    embed = (torch.randn(cfg.vocab, h, generator=gen, device=device) * 0.02).to(torch.bfloat16)
    lm_head = embed if cfg.tie_embeddings else \
        (torch.randn(cfg.vocab, h, generator=gen, device=device) * 0.02).to(torch.bfloat16)
    ones = lambda n: torch.ones(n, device=device, dtype=torch.bfloat16)  # noqa: E731
    layers = []
    for _ in range(cfg.layers):
        lin = {name: random_packed_linear(n, k, cfg, gen, device, center)
               for name, n, k in cfg.packed_linear_shapes()}
        layers.append(Layer(ones(h), ones(h), lin,
                            ones(cfg.head_dim) if cfg.qk_norm else None,
                            ones(cfg.head_dim) if cfg.qk_norm else None))
    return DecoderWeights(cfg, embed, lm_head, ones(h), layers)


def _ptrs(*tensors):
    return (ctypes.c_void_p * len(tensors))(*[t.data_ptr() for t in tensors])


class Decoder:
    """Device-resident greedy decoder over ``DecoderWeights``.

    ``persistent`` selects how the layers run: True = one launch per step
    (ep_decode_step, a resident workgroup per CU with grid barriers), False =
    five launches per layer (ep_fused_gemv / ep_decode_attention), None =
    the persistent kernel when it serves the shape.  Either way the step ends
    with ep_lm_head_argmax and is replayed from one captured graph."""

    def __init__(self, weights, max_pos, head_grid=None, persistent=None):
        if not cuda_kernel.available():
            raise RuntimeError("the gfx950 HIP backend is not available")
        self.w = weights
        cfg = self.cfg = weights.cfg
        dev = self.device = weights.embed.device
        if max_pos % 64:
            max_pos += 64 - max_pos % 64
        self.max_pos = max_pos
        f32, bf16, i32 = torch.float32, torch.bfloat16, torch.int32
        H, D = cfg.hidden, cfg.head_dim
        self.h = torch.zeros(H, device=dev, dtype=f32)
        self.q = torch.zeros(cfg.n_heads * D, device=dev, dtype=f32)
        self.k = torch.zeros(cfg.n_kv * D, device=dev, dtype=f32)
        self.v = torch.zeros(cfg.n_kv * D, device=dev, dtype=f32)
        self.attn = torch.zeros(cfg.n_heads * D, device=dev, dtype=f32)
        self.g = torch.zeros(cfg.intermediate, device=dev, dtype=f32)
        self.u = torch.zeros(cfg.intermediate, device=dev, dtype=f32)
        self.logits = torch.zeros(cfg.vocab, device=dev, dtype=f32)
        # float32 KV cache: the decoder computes in the reference model's
        # float32 precision (its CPU runtime dtype, runtime.py:_runtime_dtype)
        self.kcache = torch.zeros(cfg.layers, cfg.n_kv, max_pos, D, device=dev, dtype=f32)
        self.vcache = torch.zeros_like(self.kcache)
        self.cos, self.sin = rope_tables(cfg, max_pos, dev)
        self.state = torch.zeros(2, device=dev, dtype=i32)
        self.tokens = torch.zeros(max_pos + 1, device=dev, dtype=i32)
        self.argmax = torch.full((max_pos,), -1, device=dev, dtype=i32)
        self.prompt = torch.zeros(max_pos, device=dev, dtype=i32)
        self.n_prompt = 0
        ws = _abi.lib.ep_attention_workspace(cfg.n_heads, D, max_pos)
        self.attn_part = torch.zeros(ws // 4 + 1, device=dev, dtype=f32)
        self.attn_ctr = torch.zeros(cfg.n_heads, device=dev, dtype=i32)
        props = torch.cuda.get_device_properties(dev)
        self.head_grid = head_grid or props.multi_processor_count
        self.head_val = torch.zeros(self.head_grid, device=dev, dtype=f32)
        self.head_idx = torch.zeros(self.head_grid, device=dev, dtype=i32)
        self.head_ctr = torch.zeros(1, device=dev, dtype=i32)
        self._build_launch_args()
        served = bool(_abi.lib.ep_decode_step_serves(
            H, cfg.intermediate, cfg.n_heads, cfg.n_kv, D, max_pos, cfg.levels, cfg.group,
            self._step_dtype("scale"), self._step_dtype("cb")))
        if persistent and not served:
            raise RuntimeError(f"persistent decode step declined: {_abi.last_error()}")
        self.persistent = served if persistent is None else bool(persistent)
        if self.persistent:
            self._build_step_table()
        self.graph = None

    # ------------------------------------------------------------ launch args
    def _seg(self, names, outs, L):
        stores = [L.lin[n] for n in names]
        s0 = stores[0]
        return dict(
            K=s0.in_features, group=s0.group, levels=s0.levels,
            sdt=_abi.dtype_code(s0.scale.dtype), cdt=_abi.dtype_code(s0.cb.dtype),
            n=len(stores), packed=_ptrs(*[s.packed for s in stores]),
            scale=_ptrs(*[s.scale for s in stores]), cb=_ptrs(*[s.cb for s in stores]),
            y=_ptrs(*outs), N=(ctypes.c_int64 * len(stores))(*[s.out_features for s in stores]))

    def _build_launch_args(self):
        cfg = self.cfg
        self._layer_args = []
        for L in self.w.layers:
            self._layer_args.append(dict(
                qkv=self._seg(("q", "k", "v"), (self.q, self.k, self.v), L),
                o=self._seg(("o",), (self.h,), L),
                gu=self._seg(("gate", "up"), (self.g, self.u), L),
                down=self._seg(("down",), (self.h,), L),
                L=L))
        self.scale = 1.0 / math.sqrt(cfg.head_dim)

    def _step_dtype(self, which):
        s = self.w.layers[0].lin["q"]
        return _abi.dtype_code(s.scale.dtype if which == "scale" else s.cb.dtype)

    # Order of the 27 pointers of one layer descriptor (include/epure_decode.h).
    _STEP_LINEARS = ("q", "k", "v", "o", "gate", "up", "down")

    def _build_step_table(self):
        nbytes = _abi.lib.ep_decode_step_layer_bytes()
        if nbytes != 27 * 8:
            raise RuntimeError(f"unexpected decode-step layer descriptor size {nbytes}")
        rows = []
        self._cb16 = []  # 16-entry copies of shorter codebooks (the kernel reads 16)
        for li, L in enumerate(self.w.layers):
            st = [L.lin[n] for n in self._STEP_LINEARS]
            ptr = lambda t: 0 if t is None else t.data_ptr()  # noqa: E731
            cbs = []
            for s in st:
                cb = s.cb.reshape(-1)
                if cb.numel() < 16 or not cb.is_contiguous():
                    pad = torch.zeros(16, device=cb.device, dtype=cb.dtype)
                    pad[:cb.numel()] = cb
                    self._cb16.append(pad)
                    cb = pad
                cbs.append(cb.data_ptr())
            rows.append([s.packed.data_ptr() for s in st] + [s.scale.data_ptr() for s in st]
                        + cbs
                        + [ptr(L.attn_norm), ptr(L.mlp_norm), ptr(L.q_norm), ptr(L.k_norm),
                           self.kcache[li].data_ptr(), self.vcache[li].data_ptr()])
        self.step_table = torch.tensor(rows, dtype=torch.int64).to(self.device)
        cfg = self.cfg
        ws = _abi.lib.ep_decode_step_workspace(cfg.hidden, cfg.intermediate, cfg.n_heads,
                                               cfg.n_kv, cfg.head_dim, self.max_pos)
        self.step_ws = torch.zeros((ws + 15) // 16 * 4, device=self.device, dtype=torch.int32)
        self.step_trace = None

    def step_failed(self):
        """True if a hand-over wait of the persistent step timed out since
        the last ``reset()`` (every result from then on is garbage: the flag
        stays set and later waits give up at once).  Synchronizes.  Callers
        that drive ``step()`` themselves must check it; ``generate()``
        does."""
        return self.persistent and int(self.step_ws[2].item()) != 0

    def _step_kernel(self, stream):
        cfg = self.cfg
        rc = _abi.lib.ep_decode_step(
            self.step_table.data_ptr(), cfg.layers, self.h.data_ptr(), self.step_ws.data_ptr(),
            self.step_ws.numel() * 4, self.cos.data_ptr(),
            self.sin.data_ptr(), self.state.data_ptr(), cfg.hidden, cfg.intermediate,
            cfg.n_heads, cfg.n_kv, cfg.head_dim, self.max_pos, cfg.levels, cfg.group,
            self._step_dtype("scale"), self._step_dtype("cb"), cfg.rms_eps, cfg.rms_eps,
            self.scale,
            self.step_trace.data_ptr() if self.step_trace is not None else None, stream)
        _abi.check(rc, "ep_decode_step") or _raise_decline("ep_decode_step")

    def _gemv(self, a, xsrc, x, xdt, x_aux, accumulate, stream):
        rc = _abi.lib.ep_fused_gemv(
            xsrc, x.data_ptr(), xdt, x_aux.data_ptr() if x_aux is not None else None,
            self.cfg.rms_eps, a["K"], a["group"], a["levels"], a["sdt"], a["cdt"], a["n"],
            a["packed"], a["scale"], a["cb"], a["y"], a["N"], _abi.F32, int(accumulate), stream)
        _abi.check(rc, "ep_fused_gemv") or _raise_decline("ep_fused_gemv")

    # ------------------------------------------------------------ one step
    def step_launches(self):
        """Enqueue one decode step on the current stream (capturable)."""
        cfg, lib = self.cfg, _abi.lib
        stream = _abi.stream_handle(self.device)
        D = cfg.head_dim
        if self.persistent:
            self._step_kernel(stream)
        else:
            self._layers_multi(stream)
        rc = lib.ep_lm_head_argmax(
            self.h.data_ptr(), self.w.final_norm.data_ptr(), cfg.rms_eps,
            self.w.lm_head.data_ptr(), self.logits.data_ptr(), cfg.vocab, cfg.hidden,
            self.head_val.data_ptr(), self.head_idx.data_ptr(), self.head_ctr.data_ptr(),
            self.state.data_ptr(), self.prompt.data_ptr(), self.n_prompt,
            self.tokens.data_ptr(), self.argmax.data_ptr(), self.w.embed.data_ptr(),
            self.max_pos, self.head_grid, stream)
        _abi.check(rc, "ep_lm_head_argmax") or _raise_decline("ep_lm_head_argmax")

    def layer_launches(self):
        """Enqueue only the layers of one step (no lm_head): the persistent
        step kernel, or the 5 launches per layer.  The decode position is
        not advanced, so replays repeat the same position."""
        stream = _abi.stream_handle(self.device)
        if self.persistent:
            self._step_kernel(stream)
        else:
            self._layers_multi(stream)

    def _layers_multi(self, stream):
        cfg, lib = self.cfg, _abi.lib
        D = cfg.head_dim
        for li, a in enumerate(self._layer_args):
            L = a["L"]
            self._gemv(a["qkv"], _abi.XSRC_RMSNORM, self.h, _abi.F32, L.attn_norm, False, stream)
            rc = lib.ep_decode_attention(
                self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(),
                L.q_norm.data_ptr() if L.q_norm is not None else None,
                L.k_norm.data_ptr() if L.k_norm is not None else None, cfg.rms_eps,
                self.kcache[li].data_ptr(), self.vcache[li].data_ptr(), self.cos.data_ptr(),
                self.sin.data_ptr(), self.state.data_ptr(), self.attn_part.data_ptr(),
                self.attn_ctr.data_ptr(), self.attn.data_ptr(), cfg.n_heads, cfg.n_kv, D,
                self.max_pos, self.scale, stream)
            _abi.check(rc, "ep_decode_attention") or _raise_decline("ep_decode_attention")
            self._gemv(a["o"], _abi.XSRC_PLAIN, self.attn, _abi.F32, None, True, stream)
            self._gemv(a["gu"], _abi.XSRC_RMSNORM, self.h, _abi.F32, L.mlp_norm, False, stream)
            self._gemv(a["down"], _abi.XSRC_SWIGLU, self.g, _abi.F32, self.u, True, stream)

    def gemv_launches(self):
        """Enqueue only the step's packed GEMVs (4 launches per layer), for
        timing the dequant-GEMV on its own.  Reads and writes the same
        buffers as a step; the decode state is left untouched."""
        stream = _abi.stream_handle(self.device)
        for a in self._layer_args:
            L = a["L"]
            self._gemv(a["qkv"], _abi.XSRC_RMSNORM, self.h, _abi.F32, L.attn_norm, False, stream)
            self._gemv(a["o"], _abi.XSRC_PLAIN, self.attn, _abi.F32, None, True, stream)
            self._gemv(a["gu"], _abi.XSRC_RMSNORM, self.h, _abi.F32, L.mlp_norm, False, stream)
            self._gemv(a["down"], _abi.XSRC_SWIGLU, self.g, _abi.F32, self.u, True, stream)

    # ------------------------------------------------------------ driving
    def reset(self, prompt):
        """Start a new sequence: prompt tokens are forced, then greedy."""
        prompt = torch.as_tensor(prompt, dtype=torch.int32)
        n = int(prompt.numel())
        if n < 1 or n > self.max_pos:
            raise ValueError("prompt length must be 1..max_pos")
        if int(prompt.min()) < 0 or int(prompt.max()) >= self.cfg.vocab:
            raise ValueError(f"prompt token ids must lie in [0, {self.cfg.vocab})")
        self.prompt.zero_()
        self.prompt[:n].copy_(prompt.to(self.device))
        if self.n_prompt != n:
            self.n_prompt = n
            self.graph = None               # n_prompt is a launch argument
        if self.persistent:
            # hand-over words, tags and the time-out flag start clean
            self.step_ws.zero_()
        self.tokens.zero_()
        self.tokens[0] = int(prompt[0])
        self.argmax.fill_(-1)
        self.state.copy_(torch.tensor([0, int(prompt[0])], dtype=torch.int32))
        stream = _abi.stream_handle(self.device)
        _abi.check(_abi.lib.ep_embed_token(self.w.embed.data_ptr(), self.state.data_ptr(),
                                           self.h.data_ptr(), self.cfg.hidden, stream),
                   "ep_embed_token")

    def capture(self):
        """Capture one step as a HIP graph (warm-up launch first)."""
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step_launches()
        self.graph = g
        return g

    def step(self, use_graph=True):
        if use_graph:
            if self.graph is None:
                raise RuntimeError("call capture() after reset() before replaying")
            self.graph.replay()
        else:
            self.step_launches()

    def generate(self, prompt, n_new, use_graph=True):
        """Greedy decode: returns (tokens [n_prompt + n_new], argmax per position)."""
        self.reset(prompt)
        steps = self.n_prompt + n_new - 1
        if steps + 1 > self.max_pos:
            raise ValueError("max_pos too small for prompt + n_new")
        if use_graph and self.graph is None:
            # capture consumes no step: it records launches without running them
            self.capture()
        for _ in range(steps):
            self.step(use_graph)
        torch.cuda.synchronize(self.device)
        if self.step_failed():
            raise RuntimeError("decode step: a hand-over wait timed out; the tokens are invalid")
        n = self.n_prompt + n_new
        argmax = self.argmax[:n - 1].cpu().tolist()
        bad = [i for i, t in enumerate(argmax) if t < 0]
        if bad:
            raise RuntimeError(f"decode step: no finite logit at position {bad[0]} "
                               f"({len(bad)} positions); the tokens are invalid")
        return self.tokens[:n].cpu().tolist(), argmax


def _raise_decline(what):
    raise RuntimeError(f"{what} declined: {_abi.last_error()}")
