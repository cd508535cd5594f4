"""Packed stores and the modules that run them on the fused kernels.

Interface kept from the reference (epure/runtime.py:34-186, :289-300): a
``PackedWeight`` owns non-persistent ``packed`` / ``scale`` / ``cb`` buffers
and reports ``shape``, ``levels``, ``group``, ``in_features``,
``out_features`` and ``packed_2d()``; ``PackedLinear`` asks a backend for the
fused product and materializes the weight only when the backend declines;
``PackedEmbedding`` expands the rows a batch asks for; an expert holder keeps
a stacked slab packed between calls; a tied lm_head is a ``PackedLinear``
over the embedding store.

How this build does it:

* every dense expansion on the host goes through one helper, ``_expand``:
  a 256-entry level table in the target dtype (entries past ``levels`` are
  0, as the Rust kernel's zero-filled LUT makes them, kernel/src/lib.rs:58-59)
  gathered by index, then multiplied group-wise by the scales broadcast over
  a ``[rows, groups, group]`` view.  Both operands are in the target dtype
  before the product, which rounds once: the reference's
  ``dtype(cb)[idx] * dtype(scale)`` (runtime.py:78-89), and it is
  differentiable in ``cb`` and ``scale`` (the fine-tune path);
* indices of arbitrary rows are read straight from the flat packed stream
  (row r owns flat positions r*K .. r*K + K - 1; byte = position / 2, nibble
  = position & 1), so odd K needs no special case;
* on a gfx950 device without autograd, ``materialize`` and the embedding run
  the library's ``ep_dequant_tile`` / ``ep_embedding_rows`` kernels;
* ``PackedExperts`` (no counterpart in the reference, which expands the
  whole slab per call) runs expert-indexed rows packed.

The ``.ebin`` reader lives in ``epure.container``.
"""
import math
import os

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from .kernels import _abi
from .kernels import cpu as cpu_kernel
from .kernels import cuda as cuda_kernel

# Per-store host copies for the CPU backend, keyed by store identity
# (the reference's runtime.py:24 cache; the CPU backend drops an entry
# whose tensors were replaced).
_BUFFER_CACHE = {}

# Rows at or above which a GPU call skips the fused kernels and runs
# materialize + a dense GEMM (reference runtime.py:26-31 defaults to 8 on
# A100).  On MI355X the fused kernels win at every measured row count of
# the 8-bit config-3 sweep (M = 1..2048 at 4096x4096, 14336x4096,
# 4096x14336) but one near-tie (M = 2048 at 14336x4096: 386 vs 368 us), so
# unset every row count stays on the fused kernels.
_DENSE_ABOVE = int(os.environ.get("EPURE_DENSE_ABOVE", str(2**31 - 1)))

_TABLE = 256  # entries of the level table (the largest codebook an index can address)


# ---------------------------------------------------------------- packing
def _pack4(idx, levels):
    """Index stream -> the stored bytes (format of runtime.py:34-45).

    levels <= 16: two indices per byte over the flat stream, even position
    in the low nibble, a zero nibble pads an odd count.  levels > 16: one
    index per byte.  An index that does not fit a nibble is rejected rather
    than truncated.
    """
    flat = np.asarray(idx).reshape(-1)
    if levels > 16:
        return flat.astype(np.uint8)
    if flat.size and int(flat.max()) > 15:
        raise ValueError(f"index {int(flat.max())} does not fit 4 bits (levels={levels})")
    even = flat[0::2].astype(np.uint16)
    odd = np.zeros_like(even)
    odd[:flat.size // 2] = flat[1::2]
    return (even + odd * 16).astype(np.uint8)


def _unpack4(packed, n, levels):
    """Stored bytes -> the first ``n`` indices of the flat stream (uint8)."""
    if levels > 16:
        return packed.reshape(-1)[:n]
    if packed.is_cuda and cuda_kernel.available():
        out = torch.empty(n, dtype=torch.uint8, device=packed.device)
        rc = _abi.lib.ep_unpack_indices(packed.data_ptr(), n, levels, out.data_ptr(),
                                        _abi.stream_handle(packed.device))
        _abi.check(rc, "ep_unpack_indices")
        return out
    nib = torch.tensor([0, 4], dtype=torch.uint8, device=packed.device)
    both = (packed.reshape(-1, 1) >> nib) & 0x0F      # [bytes, 2]: low, high
    return both.reshape(-1)[:n]


def _row_indices(store, rows):
    """Indices (int64 ``[len(rows), K]``) of the given rows, read from the
    flat stream by position."""
    K = store.in_features
    pos = rows.reshape(-1, 1).to(torch.int64) * K + torch.arange(K, device=rows.device)
    flat = store.packed.reshape(-1)
    if store.levels > 16:
        return flat[pos].to(torch.int64)
    byte = flat[pos >> 1].to(torch.int64)
    return (byte >> ((pos & 1) * 4)) & 0x0F


def _level_table(cb, dtype):
    """cb in ``dtype``, zero-extended to 256 entries (differentiable)."""
    c = cb.reshape(-1).to(dtype)
    return F.pad(c, (0, _TABLE - c.numel())) if c.numel() < _TABLE else c[:_TABLE]


def _expand(store, idx, scale_rows, dtype):
    """``dtype(cb)[idx] * dtype(scale)`` for a block of rows.

    ``idx``: int64 ``[R, K]``; ``scale_rows``: ``[R, >= ceil(K/group)]``.
    """
    R, K = idx.shape
    g = store.group
    ng = -(-K // g)
    vals = _level_table(store.cb, dtype)[idx]
    if ng * g != K:
        vals = F.pad(vals, (0, ng * g - K))
    sc = scale_rows[:, :ng].to(dtype).unsqueeze(-1)
    return (vals.view(R, ng, g) * sc).view(R, ng * g)[:, :K]


def _tensor(a):
    return a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a))


def _needs_grad(store):
    return torch.is_grad_enabled() and (store.cb.requires_grad or store.scale.requires_grad)


# ---------------------------------------------------------------- store
class PackedWeight(nn.Module):
    """The resident form of one weight: indices, group scales, codebook
    (interface of runtime.py:57-89).

    ``shape`` is the logical weight shape; every axis but the last folds into
    rows (a stacked ``(E, N, K)`` expert slab has ``E*N`` rows).  ``packed``
    holds ``ceil(rows*K/2)`` bytes at 4-bit (levels <= 16) or ``rows*K`` at
    8-bit; ``scale`` is ``[rows, ceil(K/group)]`` (fp16, or fp32 once
    trained); ``cb`` holds ``levels`` values (f32 in the container, fp16
    accepted).
    """

    def __init__(self, shape, packed, scale, cb, group, levels):
        super().__init__()
        dims = tuple(int(d) for d in shape)
        if len(dims) < 2 or min(dims) < 0:
            raise ValueError(f"packed weight shape {shape} needs rank >= 2")
        self.shape = dims
        self.levels = int(levels)
        self.group = int(group)
        if not 1 <= self.levels <= _TABLE or self.group < 1:
            raise ValueError(f"levels {levels} / group {group} out of range")
        self.in_features = dims[-1]
        self.out_features = math.prod(dims[:-1])
        for name, value in (("packed", packed), ("scale", scale), ("cb", cb)):
            self.register_buffer(name, _tensor(value), persistent=False)
        want = self.out_features * self.row_bytes if self.levels > 16 else \
            -(-self.out_features * self.in_features // 2)
        if self.packed.numel() != want:
            raise ValueError(f"packed holds {self.packed.numel()} bytes, shape {dims} at "
                             f"levels {levels} needs {want}")

    @property
    def row_bytes(self):
        """Bytes of one row in the ``packed_2d`` view."""
        return self.in_features if self.levels > 16 else (self.in_features + 1) // 2

    def packed_2d(self):
        """``packed`` as ``[rows, row_bytes]`` (runtime.py:73-76); rows are
        byte-aligned in the flat stream only for even K at 4-bit."""
        return self.packed.view(self.out_features, self.row_bytes)

    def materialize(self, dtype=torch.float16):
        """The dense weight in ``dtype`` (``shape``-shaped).

        Without autograd on a gfx950 device this is one ``ep_dequant_tile``
        launch; otherwise the differentiable host expression (``_expand``).
        """
        rows, K = self.out_features, self.in_features
        w = None
        if (not _needs_grad(self) and self.packed.is_cuda and cuda_kernel.available()
                and dtype in (torch.float32, torch.float16, torch.bfloat16)):
            w = _dequant_on_device(self, dtype)
        if w is None:
            idx = _unpack4(self.packed, rows * K, self.levels).view(rows, K).to(torch.int64)
            w = _expand(self, idx, self.scale.reshape(rows, -1), dtype)
        return w.reshape(self.shape) if len(self.shape) > 2 else w


def _dequant_on_device(store, dtype):
    h = cuda_kernel._hot(store)
    if not h.usable():
        return None
    w = torch.empty((h.N, h.K), dtype=dtype, device=store.packed.device)
    rc = _abi.lib.ep_dequant_tile(
        h.packed.data_ptr(), h.scale.data_ptr(), h.scale_dt, h.ld_scale,
        h.cb.data_ptr(), h.cb_dt, h.levels, h.group, h.N, h.K,
        w.data_ptr(), _abi.dtype_code(dtype), w.stride(0), _abi.stream_handle(w.device))
    return w if _abi.check(rc, "ep_dequant_tile") else None


# ---------------------------------------------------------------- linear
class PackedLinear(nn.Module):
    """``y = x W^T (+ bias)`` over a ``PackedWeight`` (runtime.py:92-126).

    A fused backend serves the call when it can (GPU: fewer than
    ``_DENSE_ABOVE`` rows; CPU: levels <= 16); a ``None`` from it, a rank>2
    store, or a store flagged ``_force_materialize`` (``trainable_forward``)
    takes the dense route.
    """

    def __init__(self, store, bias=None):
        super().__init__()
        self.store = store
        self.bias = bias

    def _fused(self, x):
        s = self.store
        if len(s.shape) != 2 or s.__dict__.get("_force_materialize", False):
            return None
        if x.is_cuda:
            rows = x.numel() // x.shape[-1] if x.shape[-1] else 0
            return cuda_kernel.linear(x, s) if rows < _DENSE_ABOVE else None
        if s.levels > 16:
            return None
        return cpu_kernel.linear(x, s, _BUFFER_CACHE)

    def forward(self, x):
        y = self._fused(x)
        if y is None:
            # the dense route adds the bias inside the GEMM, as the reference does
            return F.linear(x, self.store.materialize(x.dtype), self.bias)
        return y if self.bias is None else y + self.bias


# ---------------------------------------------------------------- embedding
class PackedEmbedding(nn.Module):
    """Token embedding over a ``PackedWeight`` that expands only the rows a
    batch asks for (interface of runtime.py:129-160).

    ``forward(ids)`` is ``[*ids.shape, in_features]`` in ``dtype`` with the
    rounding of ``materialize(dtype)``.  Ids outside ``[0, num_embeddings)``
    raise ``IndexError`` (on the host; a call being captured into a HIP graph
    cannot look at the ids and writes zero rows for them instead).  With
    ``cb`` or ``scale`` requiring grad the expression is differentiable (a
    trained tied embedding gets its gradient).
    """

    def __init__(self, store, dtype=torch.float16):
        super().__init__()
        self.store = store
        self.dtype = dtype
        self.num_embeddings = store.out_features
        self.embedding_dim = store.in_features

    def _check_ids(self, flat):
        if flat.numel() == 0:
            return
        lo, hi = int(flat.min()), int(flat.max())
        if lo < 0 or hi >= self.num_embeddings:
            bad = lo if lo < 0 else hi
            raise IndexError(f"embedding id {bad} outside [0, {self.num_embeddings})")

    def forward(self, ids):
        s = self.store
        flat = ids.reshape(-1).to(torch.int64)
        on_device = (flat.is_cuda and s.packed.is_cuda and cuda_kernel.available()
                     and self.dtype in (torch.float32, torch.float16, torch.bfloat16))
        capturing = on_device and torch.cuda.is_current_stream_capturing()
        if not capturing:
            self._check_ids(flat)
        if on_device and not _needs_grad(s):
            out = _embedding_on_device(s, flat.contiguous(), self.dtype)
        else:
            out = _expand(s, _row_indices(s, flat), s.scale.reshape(s.out_features, -1)[flat],
                          self.dtype)
        return out.view(*ids.shape, s.in_features)

    @property
    def weight(self):
        return self.store.materialize(self.dtype)


def _embedding_on_device(store, flat, dtype):
    h = cuda_kernel._hot(store)
    if not h.usable():
        raise RuntimeError("PackedEmbedding: store buffers are not contiguous")
    out = torch.empty((flat.numel(), h.K), dtype=dtype, device=flat.device)
    rc = _abi.lib.ep_embedding_rows(
        h.packed.data_ptr(), h.scale.data_ptr(), h.scale_dt, h.ld_scale,
        h.cb.data_ptr(), h.cb_dt, h.levels, h.group, h.N, h.K,
        flat.data_ptr(), flat.numel(), out.data_ptr(), _abi.dtype_code(dtype),
        out.stride(0), _abi.stream_handle(flat.device))
    _abi.check(rc, "ep_embedding_rows")
    return out


# ---------------------------------------------------------------- experts
class ExpertHolder:
    """Keeps a module's stacked expert slab packed except while the module
    runs (the behaviour of the reference's runtime.py:163-186 holder).

    The parameter ``attr`` of ``mod`` is replaced by the store: a forward
    pre-hook sets ``mod.<attr>`` to ``materialize(dtype)`` (one dequant
    launch on a gfx950 device) and a forward hook clears it, so between calls
    only the packed form is resident.  ``remove()`` detaches both hooks.
    """

    def __init__(self, mod, attr, store, dtype=torch.float16):
        self.mod, self.attr, self.store, self.dtype = mod, attr, store, dtype
        mod._parameters.pop(attr, None)
        setattr(mod, attr, None)
        self._hooks = (mod.register_forward_pre_hook(lambda m, args: self._set(m, True)),
                       mod.register_forward_hook(lambda m, args, out: self._set(m, False)))

    def _set(self, mod, live):
        setattr(mod, self.attr, self.store.materialize(self.dtype) if live else None)

    def remove(self):
        for h in self._hooks:
            h.remove()
        self._hooks = ()


class PackedExperts(nn.Module):
    """Expert-indexed linear over a stacked ``(E, N, K)`` store, kept packed.

    ``forward(x, expert_ids)`` returns ``y[t] = x[t] @ W[expert_ids[t]]^T``
    (``[T, N]`` in ``x.dtype``): the rows of one expert are a contiguous row
    range of the folded store (``out_features = E * N``, runtime.py:64-68),
    so each expert's tokens run the packed linear on that range -- the
    batch-1 GEMV, the small-M or the MFMA path by their count -- without
    expanding any expert (the reference's holder materializes the whole
    slab per call, runtime.py:163-186).  GPU tensors only.

    Up to ``GATHER_MAX_TOKENS`` tokens (f16/bf16 ``x``) run one gathered
    launch that reads the ids on the device; more tokens are sorted by
    expert on the device and run one grouped MFMA launch over each expert's
    row tiles (``ep_expert_matmul_grouped``).  Neither synchronizes with the
    host when ``check_ids=False`` and both can be captured in a HIP graph
    (ids outside ``[0, E)`` are then clamped on the device).  With
    ``check_ids`` (the default) an eager call range-checks the ids on the
    host first and raises ``IndexError``.  Shapes the grouped kernel
    declines (K not a multiple of 64, more than 1024 experts) group per
    expert on the host.
    """

    def __init__(self, store, check_ids=True):
        super().__init__()
        if len(store.shape) != 3:
            raise ValueError(f"expert store must be (E, N, K), got {store.shape}")
        self.store = store
        self.check_ids = bool(check_ids)
        self.num_experts, self.out_features, self.in_features = store.shape

    # At most this many tokens run the gathered path (one launch, expert ids
    # read on the device, no host synchronization, capturable in a HIP
    # graph); it re-reads an expert's weights per token, so more tokens are
    # grouped per expert.
    GATHER_MAX_TOKENS = 8
    # Group larger token counts on the device (one sort and one grouped
    # launch); False groups them per expert on the host instead (one
    # ep_dequant_matmul per expert after a host synchronization).
    GROUP_ON_DEVICE = True

    def forward(self, x, expert_ids):
        s = self.store
        K, N = self.in_features, self.out_features
        x2 = x.reshape(-1, K)
        if expert_ids.numel() != x2.shape[0]:
            raise ValueError("one expert id per row of x")
        if not (x2.is_cuda and cuda_kernel.available()):
            raise RuntimeError("PackedExperts runs on the gfx950 backend only")
        out = torch.empty((x2.shape[0], N), dtype=x2.dtype, device=x2.device)
        if x2.shape[0] == 0:
            return out
        if x2.shape[0] <= self.GATHER_MAX_TOKENS and self._gathered(x2, expert_ids, out):
            return out
        if self.GROUP_ON_DEVICE and self._grouped(x2, expert_ids, out):
            return out
        ids = expert_ids.reshape(-1).to(torch.int64)
        order = torch.argsort(ids, stable=True)
        experts, counts = torch.unique_consecutive(ids[order], return_counts=True)
        experts, counts = experts.tolist(), counts.tolist()
        if experts[0] < 0 or experts[-1] >= self.num_experts:
            raise IndexError(f"expert id out of range [0, {self.num_experts})")
        h = cuda_kernel._hot(s)
        if not h.usable():
            raise RuntimeError("PackedExperts: store buffers are not contiguous")
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
                h.packed.data_ptr() + e * N * s.row_bytes,
                h.scale.data_ptr() + e * N * h.ld_scale * esz, h.scale_dt, h.ld_scale,
                h.cb.data_ptr(), h.cb_dt, h.levels, h.group,
                c, N, K, ye.data_ptr(), _abi.dtype_code(ye.dtype), ye.stride(0), 0,
                ws.data_ptr() if ws is not None else None, ws_bytes,
                _abi.stream_handle(x2.device))
            if not _abi.check(rc, "ep_dequant_matmul"):
                raise RuntimeError(f"PackedExperts: shape declined: {_abi.last_error()}")
            out.index_copy_(0, rows, ye)
        return out

    def _check_ids(self, ids32):
        """Host range check of the ids (eager calls with ``check_ids``)."""
        if self.check_ids and not torch.cuda.is_current_stream_capturing():
            lo, hi = int(ids32.min()), int(ids32.max())
            if lo < 0 or hi >= self.num_experts:
                raise IndexError(f"expert id out of range [0, {self.num_experts})")

    def _grouped(self, x2, expert_ids, out):
        """One device sort of the tokens by expert and one grouped MFMA
        launch (``ep_expert_matmul_grouped``); False where it declines the
        shape."""
        s = self.store
        K, N = self.in_features, self.out_features
        if x2.stride(1) != 1:
            return False
        h = cuda_kernel._hot(s)
        if not h.usable():
            return False
        T = x2.shape[0]
        ids32 = expert_ids.reshape(-1).to(device=x2.device, dtype=torch.int32).contiguous()
        self._check_ids(ids32)
        ws_bytes = _abi.lib.ep_expert_matmul_grouped_workspace(T, self.num_experts, K)
        ws = torch.empty(ws_bytes, device=x2.device, dtype=torch.uint8)
        rc = _abi.lib.ep_expert_matmul_grouped(
            x2.data_ptr(), _abi.dtype_code(x2.dtype), x2.stride(0), ids32.data_ptr(), T,
            h.packed.data_ptr(), h.scale.data_ptr(), h.scale_dt, h.ld_scale,
            h.cb.data_ptr(), h.cb_dt, h.levels, h.group,
            self.num_experts, N, K, out.data_ptr(), _abi.dtype_code(out.dtype), out.stride(0),
            ws.data_ptr(), ws_bytes, _abi.stream_handle(x2.device))
        if rc > 0:
            return False
        if not _abi.check(rc, "ep_expert_matmul_grouped"):
            raise RuntimeError(f"PackedExperts: {_abi.last_error()}")
        return True

    def _gathered(self, x2, expert_ids, out):
        """One ``ep_expert_matmul`` launch for every token; False where the
        kernel declines the shape.  With ``check_ids`` and outside stream
        capture the ids are range checked first (IndexError, as the grouped
        path); otherwise they are clamped on the device."""
        s = self.store
        K, N = self.in_features, self.out_features
        if x2.dtype not in (torch.float16, torch.bfloat16) or x2.stride(1) != 1:
            return False
        h = cuda_kernel._hot(s)
        if not h.usable():
            return False
        ids32 = expert_ids.reshape(-1).to(device=x2.device, dtype=torch.int32).contiguous()
        self._check_ids(ids32)
        rc = _abi.lib.ep_expert_matmul(
            x2.data_ptr(), _abi.dtype_code(x2.dtype), x2.stride(0), ids32.data_ptr(), x2.shape[0],
            h.packed.data_ptr(), h.scale.data_ptr(), h.scale_dt, h.ld_scale,
            h.cb.data_ptr(), h.cb_dt, h.levels, h.group,
            self.num_experts, N, K, out.data_ptr(), _abi.dtype_code(out.dtype), out.stride(0),
            _abi.stream_handle(x2.device))
        if rc > 0:
            return False
        if not _abi.check(rc, "ep_expert_matmul"):
            raise RuntimeError(f"PackedExperts: {_abi.last_error()}")
        return True


# ---------------------------------------------------------------- model surgery
def tie_packed_lm_head(model, embed_store):
    """Run a tied lm_head on the packed embedding store (runtime.py:289-300).

    ``model.lm_head`` becomes ``PackedLinear(embed_store)``; a config flag
    ``tie_word_embeddings`` is cleared (on ``model.config`` as well), since a
    later ``tie_weights()`` would look for a dense embedding Parameter.
    """
    model.lm_head = PackedLinear(embed_store)
    cfg = getattr(model, "config", None)
    if getattr(cfg, "tie_word_embeddings", False):
        cfg.tie_word_embeddings = False
    return model


def apply_packed(model, stores):
    """Replace ``nn.Linear`` modules by ``PackedLinear`` (what ``apply_to``
    does per packed record, runtime.py:261-262).

    ``stores`` maps a module path (``"model.layers.0.mlp.up_proj"``) to a
    ``PackedWeight``; the linear's bias is kept.
    """
    for path, store in stores.items():
        owner, _, leaf = path.rpartition(".")
        parent = model.get_submodule(owner) if owner else model
        old = getattr(parent, leaf)
        if not isinstance(old, nn.Linear):
            raise TypeError(f"{path} is {type(old).__name__}, not nn.Linear")
        if (old.out_features, old.in_features) != (store.out_features, store.in_features):
            raise ValueError(f"{path}: store is {store.out_features}x{store.in_features}, "
                             f"module {old.out_features}x{old.in_features}")
        setattr(parent, leaf, PackedLinear(store, old.bias))
    return model
