"""Packed store and packed linear -- the caller side of the fused kernels.

Mirrors the reference's resident representation and dispatch
(epure/runtime.py:34-160): ``PackedWeight`` owns ``packed`` / ``scale`` /
``cb`` buffers, ``PackedLinear.forward`` hands the call to a backend and
materializes when the backend declines, ``PackedEmbedding`` expands only the
rows a batch asks for, ``tie_packed_lm_head`` runs a tied lm_head through
the packed linear (runtime.py:289-300), ``ExpertHolder`` keeps a stacked
expert slab packed between calls (runtime.py:163-186) and ``PackedExperts``
runs expert-indexed linears without expanding the slab.  The ``.ebin``
loader is outside this build.
"""
import os

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from .kernels import cpu as cpu_kernel
from .kernels import cuda as cuda_kernel
from .kernels import _abi

_BUFFER_CACHE = {}

# Rows at or above which the GPU path materializes and calls a dense GEMM
# (reference runtime.py:26-31 defaults to 8).  The HIP backend serves every
# M itself, so the default keeps the fused path always.
_DENSE_ABOVE = int(os.environ.get("EPURE_DENSE_ABOVE", str(2**31 - 1)))


def _pack4(idx, levels):
    """Flat index stream -> bytes (runtime.py:34-45 layout).

    Up to 16 levels two indices share a byte, the even position in the low
    nibble; an odd count gets a zero pad.  Above 16 levels one index per byte.
    """
    flat = np.asarray(idx, dtype=np.uint8).reshape(-1)
    if levels > 16:
        return np.ascontiguousarray(flat)
    if flat.size & 1:
        flat = np.concatenate([flat, np.zeros(1, np.uint8)])
    pairs = flat.reshape(-1, 2)
    return np.ascontiguousarray((pairs[:, 0] & 0x0F) | (pairs[:, 1] << 4)).astype(np.uint8)


def _unpack4(packed, n, levels):
    """Bytes -> flat index stream of length n (runtime.py:48-54)."""
    if levels > 16:
        return packed[:n]
    if packed.is_cuda and cuda_kernel.available():
        out = torch.empty(n, dtype=torch.uint8, device=packed.device)
        rc = _abi.lib.ep_unpack_indices(packed.data_ptr(), n, levels, out.data_ptr(),
                                        _abi.stream_handle(packed.device))
        _abi.check(rc, "ep_unpack_indices")
        return out
    both = torch.stack((packed & 0x0F, packed >> 4), dim=-1)
    return both.reshape(-1)[:n]


def _as_tensor(a):
    return a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a))


class PackedWeight(nn.Module):
    """Indices, per-group scales and a codebook (runtime.py:57-89)."""

    def __init__(self, shape, packed, scale, cb, group, levels):
        super().__init__()
        self.levels, self.group = int(levels), int(group)
        self.shape = tuple(int(d) for d in shape)
        self.in_features = self.shape[-1]
        rows = 1
        for d in self.shape[:-1]:
            rows *= d
        self.out_features = rows
        self.register_buffer("packed", _as_tensor(packed), persistent=False)
        self.register_buffer("scale", _as_tensor(scale), persistent=False)
        self.register_buffer("cb", _as_tensor(cb), persistent=False)

    def packed_2d(self):
        cols = self.in_features if self.levels > 16 else (self.in_features + 1) // 2
        return self.packed.view(self.out_features, cols)

    def materialize(self, dtype=torch.float16):
        """Dense weight in ``dtype`` (runtime.py:78-89 semantics).

        ``dtype(cb)[idx] * dtype(scale)`` -- for fp16/bf16 both operands are
        rounded to ``dtype`` before the product, as the reference does.  On a
        gfx950 device without autograd this runs the library's dequant
        kernel; with gradients required it uses differentiable torch ops.
        """
        n = self.out_features * self.in_features
        needs_grad = torch.is_grad_enabled() and (self.cb.requires_grad
                                                  or self.scale.requires_grad)
        if (not needs_grad and self.packed.is_cuda and cuda_kernel.available()
                and dtype in (torch.float32, torch.float16, torch.bfloat16)):
            h = cuda_kernel._hot(self)
            if h.usable():
                w = torch.empty((self.out_features, self.in_features), dtype=dtype,
                                device=self.packed.device)
                rc = _abi.lib.ep_dequant_tile(
                    h.packed.data_ptr(), h.scale.data_ptr(), h.scale_dt, h.ld_scale,
                    h.cb.data_ptr(), h.cb_dt, h.levels, h.group, h.N, h.K,
                    w.data_ptr(), _abi.dtype_code(dtype), w.stride(0),
                    _abi.stream_handle(self.packed.device))
                if _abi.check(rc, "ep_dequant_tile"):
                    return w.reshape(self.shape) if len(self.shape) > 2 else w
        idx = _unpack4(self.packed, n, self.levels).view(self.out_features, self.in_features)
        table = self.cb.to(dtype).reshape(-1, 1)
        w = F.embedding(idx.int(), table).squeeze(-1)
        sc = self.scale.to(dtype).repeat_interleave(self.group, dim=1)[:, :self.in_features]
        w = w * sc
        return w.reshape(self.shape) if len(self.shape) > 2 else w


class PackedLinear(nn.Module):
    """Linear layer over a ``PackedWeight`` (runtime.py:92-126)."""

    def __init__(self, store, bias=None):
        super().__init__()
        self.store = store
        self.bias = bias

    def forward(self, x):
        s = self.store
        if len(s.shape) == 2 and not s.__dict__.get("_force_materialize", False):
            out = None
            if x.is_cuda:
                if x.reshape(-1, x.shape[-1]).shape[0] < _DENSE_ABOVE:
                    out = cuda_kernel.linear(x, s)
            elif s.levels <= 16:
                out = cpu_kernel.linear(x, s, _BUFFER_CACHE)
            if out is not None:
                return out + self.bias if self.bias is not None else out
        w = s.materialize(x.dtype)
        out = F.linear(x, w, self.bias)
        del w
        return out


class PackedEmbedding(nn.Module):
    """Embedding over a ``PackedWeight``: expands only the requested rows
    (runtime.py:129-160).

    ``forward(ids)`` returns ``[*ids.shape, in_features]`` in ``dtype`` with
    the reference's rounding, ``dtype(cb[idx]) * dtype(scale)`` per group --
    the rows of ``materialize(dtype)``.  On a gfx950 device the rows are
    expanded by the library's ``ep_embedding_rows`` kernel; CPU tensors take
    the reference's torch expression.  Ids outside ``[0, num_embeddings)``
    raise ``IndexError`` (checked on the host outside graph capture; a
    captured call writes zero rows for them).
    """

    def __init__(self, store, dtype=torch.float16):
        super().__init__()
        self.store = store
        self.dtype = dtype
        self.num_embeddings = store.out_features
        self.embedding_dim = store.in_features

    def forward(self, ids):
        s = self.store
        flat = ids.reshape(-1)
        n_in = s.in_features
        if (flat.is_cuda and s.packed.is_cuda and cuda_kernel.available()
                and self.dtype in (torch.float32, torch.float16, torch.bfloat16)):
            h = cuda_kernel._hot(s)
            if not h.usable():
                raise RuntimeError("PackedEmbedding: store buffers are not contiguous")
            flat = flat.to(torch.int64).contiguous()
            if flat.numel() and not torch.cuda.is_current_stream_capturing():
                lo, hi = int(flat.min()), int(flat.max())
                if lo < 0 or hi >= self.num_embeddings:
                    raise IndexError(f"embedding id out of range [0, {self.num_embeddings}): "
                                     f"{lo if lo < 0 else hi}")
            out = torch.empty((flat.numel(), n_in), dtype=self.dtype, device=flat.device)
            rc = _abi.lib.ep_embedding_rows(
                h.packed.data_ptr(), h.scale.data_ptr(), h.scale_dt, h.ld_scale,
                h.cb.data_ptr(), h.cb_dt, h.levels, h.group, h.N, h.K,
                flat.data_ptr(), flat.numel(), out.data_ptr(), _abi.dtype_code(self.dtype),
                out.stride(0), _abi.stream_handle(flat.device))
            _abi.check(rc, "ep_embedding_rows")
            return out.view(*ids.shape, n_in)
        if flat.numel() and (int(flat.min()) < 0 or int(flat.max()) >= self.num_embeddings):
            raise IndexError(f"embedding id out of range [0, {self.num_embeddings})")
        if s.levels > 16:
            idx = s.packed.view(self.num_embeddings, n_in)[flat].to(torch.long)
        else:
            rows = s.packed.view(self.num_embeddings, n_in // 2)[flat]
            lo, hi = (rows & 0x0F).to(torch.long), (rows >> 4).to(torch.long)
            idx = torch.empty(flat.numel(), n_in, dtype=torch.long, device=lo.device)
            idx[:, 0::2], idx[:, 1::2] = lo, hi
        cbt = torch.zeros(256, dtype=s.cb.dtype, device=s.cb.device)
        cbt[:s.cb.numel()] = s.cb.reshape(-1)  # indices >= levels read 0 (lib.rs:58-59)
        w = cbt[idx].to(self.dtype)
        sc = s.scale[flat].to(self.dtype)
        for gi, start in enumerate(range(0, n_in, s.group)):
            end = min(start + s.group, n_in)
            w[:, start:end] *= sc[:, gi:gi + 1]
        return w.view(*ids.shape, n_in)

    @property
    def weight(self):
        return self.store.materialize(self.dtype)


class ExpertHolder:
    """Keeps a stacked expert slab packed except while its module runs
    (runtime.py:163-186): a forward pre-hook attaches ``materialize(dtype)``
    as ``mod.<attr>`` (on a gfx950 device the library's dequant kernel), a
    forward hook drops it again."""

    def __init__(self, mod, attr, store, dtype=torch.float16):
        self.mod, self.attr, self.store = mod, attr, store
        self.dtype = dtype
        if attr in mod._parameters:
            del mod._parameters[attr]
        mod.register_forward_pre_hook(self._attach)
        mod.register_forward_hook(self._release)
        setattr(mod, attr, None)

    def _attach(self, mod, _a):
        setattr(mod, self.attr, self.store.materialize(self.dtype))

    def _release(self, mod, _a, _o):
        setattr(mod, self.attr, None)


class PackedExperts(nn.Module):
    """Expert-indexed linear over a stacked ``(E, N, K)`` store, kept packed.

    ``forward(x, expert_ids)`` returns ``y[t] = x[t] @ W[expert_ids[t]]^T``
    (``[T, N]`` in ``x.dtype``): the rows of one expert are a contiguous row
    range of the folded store (``out_features = E * N``, runtime.py:64-68),
    so each expert's tokens run the packed linear on that range -- the
    batch-1 GEMV, the small-M or the MFMA path by their count -- without
    expanding any expert (the reference's holder materializes the whole
    slab per call, runtime.py:163-186).  GPU tensors only.
    """

    def __init__(self, store):
        super().__init__()
        if len(store.shape) != 3:
            raise ValueError(f"expert store must be (E, N, K), got {store.shape}")
        self.store = store
        self.num_experts, self.out_features, self.in_features = store.shape

    def forward(self, x, expert_ids):
        s = self.store
        K, N = self.in_features, self.out_features
        x2 = x.reshape(-1, K)
        ids = expert_ids.reshape(-1).to(torch.int64)
        if ids.numel() != x2.shape[0]:
            raise ValueError("one expert id per row of x")
        if not (x2.is_cuda and cuda_kernel.available()):
            raise RuntimeError("PackedExperts runs on the gfx950 backend only")
        out = torch.empty((x2.shape[0], N), dtype=x2.dtype, device=x2.device)
        if ids.numel() == 0:
            return out
        order = torch.argsort(ids, stable=True)
        experts, counts = torch.unique_consecutive(ids[order], return_counts=True)
        experts, counts = experts.tolist(), counts.tolist()
        if experts[0] < 0 or experts[-1] >= self.num_experts:
            raise IndexError(f"expert id out of range [0, {self.num_experts})")
        h = cuda_kernel._hot(s)
        if not h.usable():
            raise RuntimeError("PackedExperts: store buffers are not contiguous")
        row_bytes = K if s.levels > 16 else K // 2
        if s.levels <= 16 and K % 2:
            raise ValueError("4-bit expert rows need an even K")
        esz = h.scale.element_size()
        start = 0
        for e, c in zip(experts, counts):
            rows = order[start:start + c]
            start += c
            xe = x2.index_select(0, rows).contiguous()
            ye = torch.empty((c, N), dtype=x2.dtype, device=x2.device)
            ws_bytes = _abi.lib.ep_dequant_matmul_workspace(c, N, K, h.levels, h.group)
            ws = torch.empty(ws_bytes, device=x2.device, dtype=torch.uint8) if ws_bytes else None
            rc = _abi.lib.ep_dequant_matmul(
                xe.data_ptr(), _abi.dtype_code(xe.dtype), xe.stride(0),
                h.packed.data_ptr() + e * N * row_bytes,
                h.scale.data_ptr() + e * N * h.ld_scale * esz, h.scale_dt, h.ld_scale,
                h.cb.data_ptr(), h.cb_dt, h.levels, h.group,
                c, N, K, ye.data_ptr(), _abi.dtype_code(ye.dtype), ye.stride(0), 0,
                ws.data_ptr() if ws is not None else None, ws_bytes,
                _abi.stream_handle(x2.device))
            if not _abi.check(rc, "ep_dequant_matmul"):
                raise RuntimeError(f"PackedExperts: shape declined: {_abi.last_error()}")
            out.index_copy_(0, rows, ye)
        return out


def tie_packed_lm_head(model, embed_store):
    """Run a tied lm_head through the packed embedding store
    (runtime.py:289-300): ``model.lm_head = PackedLinear(embed_store)`` and
    the config's ``tie_word_embeddings`` cleared, so a later
    ``tie_weights()`` does not look for a dense embedding Parameter."""
    model.lm_head = PackedLinear(embed_store)
    cfg = getattr(model, "config", None)
    if cfg is not None and getattr(cfg, "tie_word_embeddings", False):
        cfg.tie_word_embeddings = False
    return model


def apply_packed(model, stores):
    """Swap ``nn.Linear`` modules for ``PackedLinear`` (runtime.py:261-262).

    ``stores`` maps a module path (``"model.layers.0.mlp.up_proj"``) to a
    ``PackedWeight``; the linear's bias, if any, is kept.
    """
    for name, store in stores.items():
        parent_name, _, attr = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        target = getattr(parent, attr)
        if not isinstance(target, nn.Linear):
            raise TypeError(f"{name} is {type(target).__name__}, not nn.Linear")
        setattr(parent, attr, PackedLinear(store, getattr(target, "bias", None)))
    return model
