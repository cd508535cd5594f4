"""numpy restatement of the reference's packed-linear arithmetic.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Each function cites the reference code it restates and the checks that pin
it (tests/test_oracle.py):

=========================  ====================================  ==========================================
function                   reference                             pinned by
=========================  ====================================  ==========================================
pack4 / unpack4            epure/runtime.py:34-54                per-element brute force, round trip,
                                                                 known bytes (0x21 -> [1, 2])
packed_2d                  epure/runtime.py:73-76                shape/stride identity
dequant_tile_f32           epure/container.py:70-88,             pure-Python double product rounded once
                           lib.rs:36-40 (LUT), runtime.py:78-89  to f32 (exact for fp16-valued inputs)
materialize                epure/runtime.py:78-89                torch CPU of the same expression
embedding_rows             epure/runtime.py:139-156              == materialize(dtype)[ids] (a second route),
                                                                 pure-Python brute force on a tiny store
rust_dequant_matmul        kernel/src/lib.rs:36-151              bit-exact vs oracle/rowdot.c, fp64 bound,
                                                                 single-term and power-of-two closed forms
linear_f64                 (mathematics)                         itself the brute force
backward_f64               fine-tuning/README.md:62-68,          torch autograd through materialize (f64)
                           runtime.py:84-88 autograd
snapshot_digest            epure/finetune.py:105-117             hashlib known answer
=========================  ====================================  ==========================================
"""
import hashlib

import numpy as np


# ---------------------------------------------------------------- packing
def pack4(idx, levels):
    """runtime.py:34-45: two indices per byte, even position in the low nibble.

    Packs the FLAT stream, pads an odd count with a zero, and is the identity
    above 16 levels.
    """
    idx = np.ascontiguousarray(idx, dtype=np.uint8).ravel()
    if levels > 16:
        return idx
    if idx.size % 2:
        idx = np.append(idx, np.uint8(0))
    return (idx[0::2] | (idx[1::2] << 4)).astype(np.uint8)


def unpack4(packed, n, levels):
    """runtime.py:48-54: interleave low/high nibbles, truncate to n."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8).ravel()
    if levels > 16:
        return packed[:n].copy()
    out = np.empty(packed.size * 2, dtype=np.uint8)
    out[0::2] = packed & 0x0F
    out[1::2] = packed >> 4
    return out[:n]


def packed_2d(packed, out_features, in_features, levels):
    """runtime.py:73-76: [N, ceil(K/2)] for 4-bit, [N, K] for 8-bit."""
    cols = in_features if levels > 16 else (in_features + 1) // 2
    return np.asarray(packed).reshape(out_features, cols)


def bits_for(levels):
    """cuda.py:82: 4-bit iff levels <= 16."""
    return 4 if levels <= 16 else 8


# ---------------------------------------------------------------- bf16 helpers
def f32_to_bf16_bits(a):
    """Round-to-nearest-even float32 -> bfloat16 bit pattern (uint16)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    rounding = ((u >> 16) & 1) + 0x7FFF
    r = ((u + rounding) >> 16).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        r = np.where(nan, np.uint16(0x7FC0), r)
    return r


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(a):
    """float32 values rounded (RNE) to the nearest bfloat16, returned as f32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


# ---------------------------------------------------------------- dequant
def dequant_tile_f32(idx2d, scale, cb, group):
    """container.py:70-88 / materialize(float32): w = f32(cb[idx]) * f32(scale).

    For fp16-valued cb and scale the f32 product is exact (<= 22 significant
    bits), so this is also the Rust LUT value (lib.rs:36-40).  Indices beyond
    len(cb) read 0, as the Rust LUT does (lib.rs:59).
    """
    idx2d = np.asarray(idx2d)
    rows, k = idx2d.shape
    cbf = np.zeros(256, np.float32)
    cbv = np.asarray(cb, np.float32).ravel()
    cbf[:cbv.size] = cbv
    scale = np.asarray(scale, np.float32).reshape(rows, -1)
    w = np.empty((rows, k), np.float32)
    for gi, start in enumerate(range(0, k, group)):
        end = min(start + group, k)
        w[:, start:end] = cbf[idx2d[:, start:end]] * scale[:, gi:gi + 1]
    return w


def materialize(packed, scale, cb, out_features, in_features, group, levels, dtype="f32"):
    """runtime.py:78-89 in the given dtype ("f32", "f16", "bf16").

    ``cb.to(dtype)[idx] * scale.to(dtype)`` -- for f16/bf16 each operand is
    rounded to the dtype and the product is rounded once more (the exact
    product of two such values fits f32, so rounding it once is what torch
    does).  Returns float32 values.
    """
    n = out_features * in_features
    idx = unpack4(packed, n, levels).reshape(out_features, in_features)
    cbv = np.asarray(cb, np.float32).ravel()
    sc = np.asarray(scale, np.float32).reshape(out_features, -1)
    if dtype == "f32":
        return dequant_tile_f32(idx, sc, cbv, group)
    if dtype == "f16":
        c = cbv.astype(np.float16).astype(np.float32)
        s = sc.astype(np.float16).astype(np.float32)
        w = dequant_tile_f32(idx, s, c, group)
        return w.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        c = round_bf16(cbv)
        s = round_bf16(sc)
        w = dequant_tile_f32(idx, s, c, group)
        return round_bf16(w)
    raise ValueError(dtype)


def embedding_rows(packed, scale, cb, out_features, in_features, group, levels, ids,
                   dtype="f16"):
    """runtime.py:139-156 PackedEmbedding.forward: for each id, that row's
    indices (positions id * K .. id * K + K - 1 of the flat stream), the
    codebook entries and the row's group scales each rounded to ``dtype``,
    their product rounded to ``dtype`` (an index >= levels reads 0, as the
    Rust LUT).  Only the requested rows are unpacked.  Returns float32
    values [len(ids), K]."""
    k = in_features
    packed = np.ascontiguousarray(packed, dtype=np.uint8).ravel()
    cbf = np.zeros(256, np.float32)
    cbv = np.asarray(cb, np.float32).ravel()
    cbf[:cbv.size] = cbv
    sc = np.asarray(scale, np.float32).reshape(out_features, -1)
    rnd = {"f32": lambda a: a.astype(np.float32),
           "f16": lambda a: a.astype(np.float16).astype(np.float32),
           "bf16": round_bf16}[dtype]
    out = np.empty((len(ids), k), np.float32)
    pos = np.arange(k, dtype=np.int64)
    for i, r in enumerate(np.asarray(ids, np.int64).ravel()):
        p = int(r) * k + pos
        if levels > 16:
            idx = packed[p]
        else:
            b = packed[p >> 1]
            idx = np.where(p & 1, b >> 4, b & 0x0F)
        w = rnd(cbf[idx]) * rnd(sc[int(r), pos // group])
        out[i] = rnd(w)
    return out


# ---------------------------------------------------------------- forward
def rust_dequant_matmul(x, packed2d, scales, cb, group, four_bit):
    """kernel/src/lib.rs:94-151, vectorised over output rows.

    Every output row runs the same float32 operation sequence as row_dot
    (lib.rs:47-88): per group a LUT cb*scale, per m an accumulator starting
    at 0, k ascending, product then add (no FMA), out += acc.  Vectorising
    across rows keeps each row's order, so the bits match the serial code.

    Kept quirk: when a group starts at an odd k (odd ``group`` with 4-bit
    indices) row_dot reads the LOW nibble of byte k>>1 for x[k]
    (lib.rs:71-77), i.e. it pairs the nibbles shifted by one.
    """
    x = np.ascontiguousarray(x, np.float32).ravel()
    packed2d = np.ascontiguousarray(packed2d, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    cbv = np.ascontiguousarray(cb, np.float32).ravel()
    n, row_bytes = packed2d.shape
    k = row_bytes * 2 if four_bit else row_bytes
    m = x.size // k if k else 0
    levels = cbv.size
    out = np.zeros((n, m), np.float32)
    rows = np.arange(n)
    lut = np.zeros((n, 256), np.float32)
    for gi, cs in enumerate(range(0, k, group)):
        ce = min(cs + group, k)
        lut[:, :levels] = cbv[None, :] * scales[:, gi:gi + 1]
        for mi in range(m):
            xr = x[mi * k:(mi + 1) * k]
            acc = np.zeros(n, np.float32)
            if four_bit:
                kk = cs
                while kk < ce:
                    byte = packed2d[:, kk >> 1]
                    acc = acc + xr[kk] * lut[rows, byte & 0x0F]
                    if kk + 1 < ce:
                        acc = acc + xr[kk + 1] * lut[rows, byte >> 4]
                    kk += 2
            else:
                for kk in range(cs, ce):
                    acc = acc + xr[kk] * lut[rows, packed2d[:, kk]]
            out[:, mi] = out[:, mi] + acc
    return np.ascontiguousarray(out.T)


def linear_f64(x, w):
    """Brute force y = x @ w.T in float64."""
    return np.asarray(x, np.float64) @ np.asarray(w, np.float64).T


# ---------------------------------------------------------------- backward
def backward_f64(gy, x, idx2d, scale, cb, group):
    """fine-tuning/README.md:62-68 closed forms, float64.

    grad_x = gy @ W; grad_W = gy^T @ x;
    grad_scale[n, g] = sum_{k in g} grad_W[n, k] * cb[idx[n, k]];
    grad_cb[l] = sum_{idx == l} grad_W[n, k] * scale[n, g(k)].
    """
    gy = np.asarray(gy, np.float64).reshape(-1, idx2d.shape[0])
    x = np.asarray(x, np.float64).reshape(gy.shape[0], -1)
    n, k = idx2d.shape
    cbv = np.asarray(cb, np.float64).ravel()
    sc = np.asarray(scale, np.float64).reshape(n, -1)
    g_of_k = np.arange(k) // group
    s_full = sc[:, g_of_k]
    w = cbv[idx2d] * s_full
    grad_x = gy @ w
    grad_w = gy.T @ x
    gsc = np.zeros_like(sc)
    np.add.at(gsc, (np.repeat(np.arange(n), k), np.tile(g_of_k, n)),
              (grad_w * cbv[idx2d]).ravel())
    gcb = np.zeros(cbv.size, np.float64)
    np.add.at(gcb, idx2d.ravel(), (grad_w * s_full).ravel())
    return grad_x, gcb, gsc


# ---------------------------------------------------------------- index freeze
def snapshot_digest(packed_bytes):
    """finetune.py:115-116: blake2b with a 16-byte digest, hex."""
    return hashlib.blake2b(np.ascontiguousarray(packed_bytes).tobytes(),
                           digest_size=16).hexdigest()


# ---------------------------------------------------------------- synthetic inputs
def synth_linear(n, k, levels=16, group=128, seed=0, cb_sorted=True):
    """Synthetic packed linear (numpy PCG64, machine-independent).

    idx uniform over 0..levels-1; cb = sort(N(0,1) draws) as fp16; scales
    |N(0, 0.02)| + 1e-3 as fp16 [n, ceil(k/group)].  Returns
    (idx2d u8, packed u8 flat, scale f16, cb f16).
    """
    rng = np.random.Generator(np.random.PCG64(seed))
    idx = rng.integers(0, levels, size=(n, k), dtype=np.uint8)
    cb = rng.standard_normal(levels)
    if cb_sorted:
        cb = np.sort(cb)
    cb = cb.astype(np.float16)
    g = (k + group - 1) // group
    scale = (np.abs(rng.normal(0.0, 0.02, size=(n, g))) + 1e-3).astype(np.float16)
    return idx, pack4(idx, levels), scale, cb
