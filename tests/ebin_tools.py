"""Test-side .ebin writer and rANS encoder (TEST INFRASTRUCTURE ONLY).

The reference ships no writer (epure/container.py:3-5) and no .ebin file;
these build containers to the layout container.py:7-20 reads, with index
streams coded by the exact inverse of the decode steps in csrc/rans.c, so
the reader, the records and the decoder can be checked end to end.
"""
import json
import struct

import numpy as np

from epure.container import MAGIC, PRECISION, symbol_cdf


def rans_encode(symbols, cdf):
    """32-bit words that decode (stack order) to ``symbols``."""
    bulk, state = [], 0
    for s in reversed([int(v) for v in symbols]):
        c, p = int(cdf[s]), int(cdf[s + 1]) - int(cdf[s])
        if (state >> (64 - PRECISION)) >= p:       # the next step would overflow 64 bits
            bulk.append(state & 0xFFFFFFFF)
            state >>= 32
        state = ((state // p) << PRECISION) | (c + state % p)
    lo, hi = state & 0xFFFFFFFF, state >> 32
    tail = [lo, hi] if hi else ([lo] if lo else [])
    return np.asarray(bulk + tail, dtype=np.uint32)


def encode_chunks(idx, counts, chunk):
    cdf = symbol_cdf(counts)
    blobs, chunks = [], []
    for i in range(0, len(idx), chunk):
        w = rans_encode(idx[i:i + chunk], cdf)
        blobs.append(w.tobytes())
        chunks.append([len(blobs[-1]), len(idx[i:i + chunk])])
    return b"".join(blobs), chunks


class Writer:
    """Blobs first, header JSON after them, its offset last."""

    def __init__(self, levels, group):
        self.buf = bytearray(MAGIC)
        self.header = {"format": "epure/1", "levels": levels, "group": group, "tensors": [],
                       "extras": {}}

    def blob(self, data):
        off = len(self.buf)
        self.buf += data
        return [off, len(data)]

    def raw(self, name, arr):
        a = np.asarray(arr, np.float16)
        self.header["tensors"].append({"name": name, "kind": "raw", "shape": list(a.shape),
                                       "data": self.blob(a.tobytes())})

    def packed(self, name, shape, idx, scale, cb, chunk=4096):
        counts = np.bincount(idx.reshape(-1), minlength=len(cb)).tolist()
        blob, chunks = encode_chunks(idx.reshape(-1), counts, chunk)
        self.header["tensors"].append({
            "name": name, "kind": "epure", "shape": list(shape),
            "cb": self.blob(np.asarray(cb, np.float32).tobytes()),
            "scale": self.blob(np.asarray(scale, np.float16).tobytes()),
            "scale_shape": list(np.asarray(scale).shape), "idx": self.blob(blob),
            "chunks": chunks, "counts": counts})

    def extra(self, name, data):
        self.header["extras"][name] = self.blob(data)

    def save(self, path):
        off = len(self.buf)
        out = self.buf + json.dumps(self.header).encode() + struct.pack("<Q", off)
        with open(path, "wb") as f:
            f.write(bytes(out))
