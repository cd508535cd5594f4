"""Fine-tuning helpers on CPU (reference epure/finetune.py:42-176 behaviour):
which stores are trained, tied stores, the index freeze proof, the
trainable_forward route switch and the ScaleTuner loop on a tiny
transformers model.  Gradients are checked against float64 autograd of the
closed form W = cb[idx] * scale."""
import numpy as np
import pytest
import torch

from epure import (PackedEmbedding, PackedLinear, PackedWeight, ScaleTuner, make_trainable,
                   packed_weights, snapshot_indices, trainable_forward, verify_frozen)
from epure import runtime
from epure.kernels import cpu
from oracle import ref


def store(n, k, levels=16, group=32, seed=0):
    idx, packed, scale, cb = ref.synth_linear(n, k, levels, group, seed=seed)
    return idx, PackedWeight((n, k), packed, scale, cb.astype(np.float32), group, levels)


class Tied(torch.nn.Module):
    """Embedding and lm_head over one store (runtime.py:289-300 tying)."""

    def __init__(self, s, mid):
        super().__init__()
        self.embed = PackedEmbedding(s, torch.float32)
        self.mid = PackedLinear(mid)
        self.lm_head = PackedLinear(s)

    def forward(self, ids):
        return self.lm_head(self.mid(self.embed(ids)))


def test_packed_weights_includes_embeddings_and_shares_tied_store():
    _, s = store(40, 64)
    _, m = store(64, 64, seed=1)
    model = Tied(s, m)
    names = [n for n, _ in packed_weights(model)]
    assert names == ["embed", "mid", "lm_head"]
    params = make_trainable(model, "both", verbose=False)
    # the tied store is promoted once: 2 stores x (scale, cb)
    assert len(params) == 4
    assert model.embed.store.scale is model.lm_head.store.scale
    assert all(p.requires_grad and p.dtype == torch.float32 for p in params)
    snap = snapshot_indices(model)
    assert set(snap) == {"embed", "mid", "lm_head"}


@pytest.mark.parametrize("mode,attrs", [("scale", {"scale"}), ("codebook", {"cb"}),
                                        ("both", {"scale", "cb"})])
def test_make_trainable_modes(mode, attrs):
    _, s = store(16, 64)
    model = torch.nn.Sequential(PackedLinear(s))
    make_trainable(model, mode, verbose=False)
    trained = {a for a in ("scale", "cb") if isinstance(getattr(s, a), torch.nn.Parameter)}
    assert trained == attrs
    assert not s.packed.requires_grad


def _closed_form_grads(idx, scale, cb, group, fn):
    """float64 autograd of fn(W) with W = cb[idx] * scale (the closed form of
    fine-tuning/README.md:62-68); returns (grad_cb, grad_scale)."""
    cb64 = torch.tensor(cb, dtype=torch.float64, requires_grad=True)
    sc64 = torch.tensor(scale.astype(np.float64), requires_grad=True)
    w = cb64[torch.from_numpy(idx.astype(np.int64))] * sc64.repeat_interleave(group, 1)
    fn(w).backward()
    return cb64.grad, sc64.grad


def test_tied_embedding_gradients_match_float64():
    n, k, group = 40, 64, 32
    idx, s = store(n, k, group=group, seed=3)
    cb0, sc0 = s.cb.numpy().copy(), s.scale.numpy().astype(np.float32).copy()
    ids = torch.tensor([[3, 7, 3], [39, 0, 11]])
    model = torch.nn.Module()
    model.embed = PackedEmbedding(s, torch.float32)
    model.lm_head = PackedLinear(s)
    make_trainable(model, "both", verbose=False)
    h = model.embed(ids)                      # [2, 3, 64]
    logits = model.lm_head(h)                 # [2, 3, 40]
    (logits.square().sum() + 0.5 * h.sum()).backward()

    def f(w):
        e = w[ids.reshape(-1)].reshape(2, 3, k)
        return (e @ w.t()).square().sum() + 0.5 * e.sum()
    gcb, gsc = _closed_form_grads(idx.reshape(n, k), sc0, cb0, group, f)
    assert torch.allclose(s.cb.grad.double(), gcb, rtol=1e-4, atol=1e-4 * float(gcb.abs().max()))
    assert torch.allclose(s.scale.grad.double(), gsc, rtol=1e-4,
                          atol=1e-4 * float(gsc.abs().max()))


def test_trainable_forward_routes_through_materialize(monkeypatch):
    _, s = store(16, 64)
    lin = PackedLinear(s)
    calls = []
    monkeypatch.setattr(cpu, "linear", lambda x, st, cache=None: calls.append(1))
    x = torch.randn(2, 64)
    lin(x)
    assert calls == [1]                       # backend asked first
    model = torch.nn.Sequential(lin)
    trainable_forward(model, True)
    y = lin(x)
    assert calls == [1]                       # flag set: backend skipped
    assert torch.allclose(y, x @ s.materialize(torch.float32).t())
    trainable_forward(model, False)
    lin(x)
    assert calls == [1, 1]


def test_verify_frozen_names_changed_store():
    _, a = store(16, 64)
    _, b = store(16, 64, seed=2)
    model = torch.nn.Sequential(PackedLinear(a), PackedLinear(b))
    snap = snapshot_indices(model)
    assert verify_frozen(model, snap)
    b.packed[5] ^= 0x10
    with pytest.raises(RuntimeError, match="1 store"):
        verify_frozen(model, snap)


def test_scale_tuner_on_tiny_llama():
    transformers = pytest.importorskip("transformers")
    torch.manual_seed(0)
    cfg = transformers.LlamaConfig(vocab_size=96, hidden_size=64, intermediate_size=128,
                                   num_hidden_layers=2, num_attention_heads=4,
                                   num_key_value_heads=2, max_position_embeddings=64)
    model = transformers.LlamaForCausalLM(cfg).float()
    stores = {}
    for li in range(2):
        for name in ("self_attn.q_proj", "self_attn.k_proj", "mlp.up_proj", "mlp.down_proj"):
            path = f"model.layers.{li}.{name}"
            lin = model.get_submodule(path)
            n, k = lin.weight.shape
            _, s = store(n, k, group=32, seed=li * 10 + len(stores))
            stores[path] = s
    runtime.apply_packed(model, stores)
    ids = torch.randint(0, 96, (2, 16), generator=torch.Generator().manual_seed(1))
    tuner = ScaleTuner(model, "both", lr=1e-2)
    assert len(tuner.params) == 2 * len(stores)
    before = {p: s.packed.clone() for p, s in stores.items()}
    losses = [tuner.step(ids) for _ in range(8)]
    assert all(isinstance(v, float) for v in losses)
    assert losses[-1] < losses[0]
    tuner.finish()
    assert all(not p.requires_grad for p in tuner.params)
    assert all(torch.equal(before[p], s.packed) for p, s in stores.items())
    # only the packed stores' scale/cb were trained: dense weights untouched
    assert all(not p.requires_grad for p in model.parameters())
