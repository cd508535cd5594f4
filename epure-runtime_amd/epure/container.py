"""`.ebin` container: reader, index decode, and packed stores from records.

Layout (the reference's epure/container.py:7-20, which this must read):

    MAGIC "EBIN0001" (8 bytes) | payload blobs | header JSON | u64 LE offset of the header

Header: ``format``, ``levels``, ``group``, ``tensors`` (records), optional
``extras`` (name -> [offset, length] of bundled config/tokenizer files).  A
record is ``kind == "raw"`` (an fp16 tensor: ``data`` blob, ``shape``) or
``kind == "epure"``: ``cb`` (f32 blob), ``scale`` (fp16 blob,
``scale_shape``), ``idx`` (rANS-coded index blob), ``chunks`` ([bytes,
symbols] per independently coded chunk), ``counts`` (symbol counts the coder
model was built from), ``shape``.  A blob reference is ``[offset, length]``.

The index stream decode (``rans_decode``) runs in libepure_cpu.so
(``ep_rans_decode``), chunks in parallel.  It restates the stack-ANS coder of
the `constriction` library the reference calls (container.py:28-51) -- 32-bit
words, 64-bit state, a categorical model quantized to 24 bits by the "fast"
rule (each symbol one unit plus floor(cumulative probability x (2^24 - n))).
constriction is not available here and no .ebin file exists to test
against, so bit-compatibility with files the reference's writer produced is
unpinned; the layout, the records and the decode's consistency with its
inverse are tested.
"""
import ctypes
import json
import os
import struct

import numpy as np
import torch
import torch.nn as nn

from .kernels import cpu as cpu_kernel
from .runtime import ExpertHolder, PackedEmbedding, PackedLinear, PackedWeight, _pack4

MAGIC = b"EBIN0001"
PRECISION = 24


# ---------------------------------------------------------------- reading
def read_header(path):
    """The header JSON of an .ebin file (container.py:54-62)."""
    with open(path, "rb") as f:
        if f.read(8) != MAGIC:
            raise ValueError(f"{path} is not an .ebin file (bad magic)")
        end = f.seek(0, os.SEEK_END) - 8
        if end < 8:
            raise ValueError(f"{path} is truncated")
        f.seek(end)
        (off,) = struct.unpack("<Q", f.read(8))
        if not 8 <= off <= end:
            raise ValueError(f"{path}: header offset {off} outside the file")
        f.seek(off)
        return json.loads(f.read(end - off))


def read_blob(f, rec):
    """Bytes of a blob reference ``[offset, length]`` (container.py:65-67)."""
    off, length = int(rec[0]), int(rec[1])
    f.seek(off)
    data = f.read(length)
    if len(data) != length:
        raise ValueError(f"blob [{off}, {length}] runs past the end of the file")
    return data


def extras(path):
    """Bundled config/tokenizer files by name (container.py:104-108)."""
    header = read_header(path)
    with open(path, "rb") as f:
        return {k: read_blob(f, rec) for k, rec in header.get("extras", {}).items()}


def describe(path):
    """Summary of a container (container.py:111-123)."""
    h = read_header(path)
    n_q = sum(1 for t in h["tensors"] if t["kind"] == "epure")
    return {"path": path, "format": h["format"], "levels": h["levels"], "group": h["group"],
            "compressed_tensors": n_q, "raw_tensors": len(h["tensors"]) - n_q,
            "size_bytes": os.path.getsize(path), "bundled": sorted(h.get("extras", {}))}


# ---------------------------------------------------------------- index decode
def symbol_cdf(counts):
    """Left-sided cumulative table (n + 1 entries, 2^24 total) of the coder
    model built from integer counts: probabilities max(count, 1) / total
    (container.py:31-37), quantized by the fast rule: entry i =
    floor(cum_i * (2^24 - n) / norm) + i with cum_i the float64 running sum
    of the first i probabilities, so every symbol keeps a nonzero share."""
    p = np.maximum(np.asarray(counts, dtype=np.float64), 1.0)
    p = p / p.sum()
    n = p.size
    if not 1 <= n <= 256:
        raise ValueError(f"{n} symbols (1..256 served)")
    run = np.cumsum(p)                        # sequential float64 sums
    scale = float(2 ** PRECISION - n) / float(run[-1])
    cum = np.concatenate(([0.0], run[:-1]))
    cdf = (cum * scale).astype(np.uint64) + np.arange(n, dtype=np.uint64)
    return np.concatenate((cdf, [2 ** PRECISION])).astype(np.uint32)


def rans_decode(blob, chunks, counts, nthreads=0):
    """Index stream of one tensor, decoded chunk by chunk (container.py:40-51);
    uint8 array of sum(symbols) indices."""
    lib = cpu_kernel._load()
    if lib is None:
        raise RuntimeError(f"libepure_cpu.so is not available: {cpu_kernel.LOAD_ERROR}")
    if not hasattr(lib, "_rans_bound"):
        lib.ep_rans_decode.restype = ctypes.c_int
        lib.ep_rans_decode.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                       ctypes.c_void_p, ctypes.c_int]
        lib._rans_bound = True
    chunks = np.asarray(chunks, dtype=np.int64).reshape(-1, 2)
    if np.any(chunks[:, 0] % 4):
        raise ValueError("chunk byte lengths must be whole 32-bit words")
    if int(chunks[:, 0].sum()) > len(blob):
        raise ValueError("chunks run past the index blob")
    words = np.frombuffer(blob, dtype=np.uint32, count=int(chunks[:, 0].sum()) // 4)
    cdf = symbol_cdf(counts)
    nwords = np.ascontiguousarray(chunks[:, 0] // 4)
    nsym = np.ascontiguousarray(chunks[:, 1])
    out = np.empty(int(nsym.sum()), dtype=np.uint8)
    rc = lib.ep_rans_decode(words.ctypes.data if words.size else None, nwords.ctypes.data,
                            nsym.ctypes.data, len(nsym), cdf.ctypes.data, cdf.size - 1,
                            out.ctypes.data if out.size else None, int(nthreads))
    if rc != 0:
        raise ValueError(f"ep_rans_decode failed ({rc})")
    return out


def dequantize(idx, scale, cb, shape, group):
    """float32 weights from indices, group scales and codebook
    (container.py:70-88): cb[idx] * scale per group, rank > 2 folded into
    rows; an index past the codebook reads 0."""
    shape = tuple(int(d) for d in shape)
    n_in = shape[-1]
    rows = int(np.prod(shape[:-1]))
    table = np.zeros(256, np.float32)
    cbf = np.asarray(cb, np.float32).reshape(-1)
    table[:cbf.size] = cbf
    w = table[np.asarray(idx).reshape(rows, n_in)]
    sc = np.asarray(scale, np.float32).reshape(rows, -1)
    ng = -(-n_in // group)
    full = np.repeat(sc[:, :ng], group, axis=1)[:, :n_in]
    return (w * full).reshape(shape)


# ---------------------------------------------------------------- stores
def read_stores(path, device="cpu", dtype=torch.float16):
    """``{name: PackedWeight | Tensor}`` for every record (runtime.py:225-249):
    epure records become packed stores on ``device`` (indices rANS-decoded
    and packed two per byte at <= 16 levels); raw records become dense
    tensors in ``dtype``."""
    header = read_header(path)
    group, levels = int(header["group"]), int(header["levels"])
    out = {}
    with open(path, "rb") as f:
        for t in header["tensors"]:
            if t["kind"] == "raw":
                arr = np.frombuffer(read_blob(f, t["data"]), np.float16).reshape(t["shape"])
                out[t["name"]] = torch.from_numpy(arr.copy()).to(device=device, dtype=dtype)
                continue
            if t["kind"] != "epure":
                raise ValueError(f"{t['name']}: unknown record kind {t['kind']!r}")
            cb = np.frombuffer(read_blob(f, t["cb"]), np.float32).copy()
            scale = np.frombuffer(read_blob(f, t["scale"]), np.float16).reshape(
                t["scale_shape"]).copy()
            idx = rans_decode(read_blob(f, t["idx"]), t["chunks"], t["counts"])
            n = int(np.prod(t["shape"]))
            if idx.size != n:
                raise ValueError(f"{t['name']}: {idx.size} indices decoded, shape needs {n}")
            out[t["name"]] = PackedWeight(t["shape"], _pack4(idx, levels), scale, cb, group,
                                          levels).to(device)
    return out, header


def _parent(root, dotted):
    owner, _, leaf = dotted.rpartition(".")
    return (root.get_submodule(owner) if owner else root), leaf


def apply_to(model, path, device="cpu", dtype=None, tie_lm_head=None):
    """Install an .ebin's weights into ``model`` with linears left packed
    (the reference's apply_to, runtime.py:214-305).

    ``nn.Linear`` -> ``PackedLinear`` (bias kept); an embedding ->
    ``PackedEmbedding`` in ``dtype``; a stacked 3-D expert parameter -> an
    ``ExpertHolder`` that keeps it packed between calls; anything else
    (routers, convolutions, norms) is restored dense.  ``dtype`` defaults to
    the model's floating-point dtype.  With a tied config (or
    ``tie_lm_head=True``) the lm_head runs on the embedding store.  Returns
    the model.
    """
    if dtype is None:
        dtype = next((p.dtype for p in model.parameters() if p.is_floating_point()),
                     torch.float16)
    stores, _ = read_stores(path, device=device, dtype=dtype)
    embed_store, holders = None, []
    for name, val in stores.items():
        mod_name = name[:-len(".weight")] if name.endswith(".weight") else name
        parent, leaf = _parent(model, mod_name)
        target = getattr(parent, leaf, None)
        if isinstance(val, torch.Tensor):
            p_parent, p_leaf = _parent(model, name)
            setattr(p_parent, p_leaf, nn.Parameter(val, requires_grad=False))
        elif type(target) is nn.Embedding or "embed_tokens" in name:
            embed_store = val
            setattr(parent, leaf, PackedEmbedding(val, dtype))
        elif isinstance(target, nn.Linear):
            setattr(parent, leaf, PackedLinear(val, target.bias))
        elif len(val.shape) == 3 and target is not None and not isinstance(target, nn.Module):
            holders.append(ExpertHolder(parent, leaf, val, dtype))
        else:
            p_parent, p_leaf = _parent(model, name)
            setattr(p_parent, p_leaf,
                    nn.Parameter(val.materialize(dtype).to(device), requires_grad=False))
    cfg = getattr(model, "config", None)
    tie = tie_lm_head if tie_lm_head is not None else bool(getattr(cfg, "tie_word_embeddings",
                                                                   False))
    if tie and embed_store is not None and hasattr(model, "lm_head"):
        from .runtime import tie_packed_lm_head
        tie_packed_lm_head(model, embed_store)
    if holders:
        model._epure_holders = holders
    return model
