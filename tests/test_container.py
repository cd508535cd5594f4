"""The .ebin reader (reference epure/container.py:28-123, store building of
runtime.py:225-249) on containers written to its layout by tests/ebin_tools.

Pinned: the layout (magic, trailing header offset, blob references), raw and
packed records, the f32 dequantization's closed form, the rANS decode
against its exact inverse (round trips over skewed, uniform and
single-symbol streams, several chunks, empty chunks), and the packed stores
built from the records.  Not pinned: bit-compatibility of the index decode
with files the reference's `constriction` coder wrote (no such file or
library exists here)."""
import numpy as np
import pytest
import torch

from epure import PackedLinear, PackedWeight
from epure import container
from oracle import ref

from ebin_tools import Writer, encode_chunks, rans_encode


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def test_cdf_quantization_rule():
    cdf = container.symbol_cdf([0, 5, 1, 1000])       # a zero count still gets a share
    assert cdf[0] == 0 and cdf[-1] == 2 ** 24 and np.all(np.diff(cdf.astype(np.int64)) >= 1)
    p = np.array([1, 5, 1, 1000], np.float64) / 1007
    want = [int(np.float64(sum(p[:i])) * ((2 ** 24 - 4) / 1.0)) + i for i in range(4)]
    assert abs(int(cdf[3]) - want[3]) <= 1


@pytest.mark.parametrize("dist", ["uniform16", "skewed", "one", "levels256"])
def test_rans_round_trip(dist):
    r = rng(hash(dist) % 1000)
    if dist == "uniform16":
        idx = r.integers(0, 16, 20000).astype(np.uint8)
    elif dist == "skewed":
        idx = np.minimum(r.geometric(0.35, 30000) - 1, 15).astype(np.uint8)
    elif dist == "one":
        idx = np.full(5000, 3, np.uint8)
    else:
        idx = r.integers(0, 256, 9000).astype(np.uint8)
    levels = 256 if dist == "levels256" else 16
    counts = np.bincount(idx, minlength=levels)
    for chunk in (1, 777, 4096, 10 ** 6):
        blob, chunks = encode_chunks(idx, counts.tolist(), chunk)
        assert np.array_equal(container.rans_decode(blob, chunks, counts), idx)


def test_rans_empty_and_tiny_streams():
    counts = [3, 1]
    assert container.rans_decode(b"", [], counts).size == 0
    cdf = container.symbol_cdf(counts)
    for sym in ([0], [1], [1, 0, 1]):
        w = rans_encode(sym, cdf)
        got = container.rans_decode(w.tobytes(), [[w.nbytes, len(sym)]], counts)
        assert got.tolist() == sym


def test_rans_compresses_skewed_streams():
    idx = np.minimum(rng(3).geometric(0.6, 50000) - 1, 15).astype(np.uint8)
    blob, _ = encode_chunks(idx, np.bincount(idx, minlength=16).tolist(), 8192)
    assert len(blob) < 0.5 * idx.size / 2          # well under the 4-bit packing


def _write(path, n=48, k=256, levels=16, group=64):
    idx, packed, scale, cb = ref.synth_linear(n, k, levels, group, seed=n + k)
    w = Writer(levels, group)
    w.packed("model.layers.0.mlp.up_proj.weight", (n, k), idx.reshape(-1), scale, cb)
    raw = rng(5).standard_normal(k).astype(np.float16)
    w.raw("model.norm.weight", raw)
    w.extra("config.json", b'{"hidden_size": 256}')
    w.save(path)
    return idx, packed, scale, cb, raw


def test_header_blobs_and_extras(tmp_path):
    p = str(tmp_path / "m.ebin")
    _write(p)
    h = container.read_header(p)
    assert h["levels"] == 16 and h["group"] == 64 and len(h["tensors"]) == 2
    assert container.extras(p) == {"config.json": b'{"hidden_size": 256}'}
    d = container.describe(p)
    assert d["compressed_tensors"] == 1 and d["raw_tensors"] == 1 and d["bundled"] == ["config.json"]


def test_rejects_bad_files(tmp_path):
    p = tmp_path / "bad.ebin"
    p.write_bytes(b"NOTEBIN!" + b"\0" * 16)
    with pytest.raises(ValueError, match="magic"):
        container.read_header(str(p))
    p.write_bytes(container.MAGIC + b"\0" * 4 + (10 ** 6).to_bytes(8, "little"))
    with pytest.raises(ValueError):
        container.read_header(str(p))


def test_read_stores_builds_packed_weights(tmp_path):
    p = str(tmp_path / "m.ebin")
    idx, packed, scale, cb, raw = _write(p)
    stores, _ = container.read_stores(p, dtype=torch.float32)
    s = stores["model.layers.0.mlp.up_proj.weight"]
    assert isinstance(s, PackedWeight) and s.shape == (48, 256)
    assert np.array_equal(s.packed.numpy(), packed)           # same bytes as the packing rule
    assert np.array_equal(s.materialize(torch.float32).numpy(),
                          ref.dequant_tile_f32(idx.reshape(48, 256), scale, cb, 64))
    assert torch.equal(stores["model.norm.weight"], torch.from_numpy(raw.astype(np.float32)))


def test_dequantize_closed_form():
    idx, packed, scale, cb = ref.synth_linear(6, 100, 10, 32, seed=4)
    w = container.dequantize(idx, scale, cb, (2, 3, 100), 32)
    assert w.shape == (2, 3, 100)
    assert np.array_equal(w.reshape(6, 100), ref.dequant_tile_f32(idx.reshape(6, 100), scale,
                                                                   cb, 32))


def test_apply_to_tiny_llama(tmp_path):
    transformers = pytest.importorskip("transformers")
    torch.manual_seed(0)
    cfg = transformers.LlamaConfig(vocab_size=64, hidden_size=64, intermediate_size=128,
                                   num_hidden_layers=1, num_attention_heads=4,
                                   num_key_value_heads=2, max_position_embeddings=32,
                                   tie_word_embeddings=True)
    model = transformers.LlamaForCausalLM(cfg).float().eval()
    w = Writer(16, 32)
    dense = {}
    for name, prm in model.named_parameters():
        if prm.ndim == 2:
            n, k = prm.shape
            idx, packed, scale, cb = ref.synth_linear(n, k, 16, 32, seed=n * 3 + k)
            w.packed(name, (n, k), idx.reshape(-1), scale, cb)
            dense[name] = torch.from_numpy(ref.dequant_tile_f32(idx.reshape(n, k), scale, cb, 32))
        else:
            v = torch.ones_like(prm)
            w.raw(name, v.numpy())
            dense[name] = v
    p = str(tmp_path / "llama.ebin")
    w.save(p)
    ref_model = transformers.LlamaForCausalLM(cfg).float().eval()
    ref_model.load_state_dict({k: v for k, v in dense.items()}, strict=False)
    ref_model.tie_weights()
    container.apply_to(model, p, dtype=torch.float32)
    assert isinstance(model.model.layers[0].mlp.up_proj, PackedLinear)
    assert isinstance(model.lm_head, PackedLinear) and model.config.tie_word_embeddings is False
    ids = torch.randint(0, 64, (1, 9), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        got, want = model(ids).logits, ref_model(ids).logits
    assert torch.allclose(got, want, rtol=1e-4, atol=1e-4)
