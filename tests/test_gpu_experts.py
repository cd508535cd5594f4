"""Stacked experts (epure/runtime.py:163-186): the expert-indexed packed
linear (experts kept packed) and the reference-style holder that attaches
the dense slab only while its module runs.  Held to the packed-linear bar:
max relative error 2e-3 against the Rust-order float32 result per expert
(plus the output rounding)."""
import numpy as np
import pytest
import torch

from epure import ExpertHolder, PackedExperts, PackedWeight
from oracle import ref, rowdot

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def experts(E, n, k, levels, group, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    idx = rng.integers(0, levels, E * n * k).astype(np.uint8)
    packed = ref.pack4(idx, levels)
    cb = np.sort(rng.standard_normal(levels)).astype(np.float16).astype(np.float32)
    scale = (np.abs(rng.normal(0, 0.02, (E * n, k // group))) + 1e-3).astype(np.float16)
    s = PackedWeight((E, n, k), packed, scale, cb, group, levels).to(DEV)
    return s, packed, scale, cb


def want_rows(x32, ids, packed, scale, cb, E, n, k, group, levels):
    rb = k // 2 if levels <= 16 else k
    p2 = packed.reshape(E * n, rb)
    out = np.empty((len(ids), n), np.float32)
    for t, e in enumerate(ids):
        out[t] = rowdot.dequant_matmul(x32[t:t + 1], p2[e * n:(e + 1) * n],
                                       scale[e * n:(e + 1) * n].astype(np.float32), cb, group,
                                       levels <= 16)[0]
    return out


@pytest.mark.parametrize("E,n,k,levels,T", [(4, 256, 512, 16, 10), (8, 512, 1024, 16, 300),
                                            (3, 128, 256, 256, 7)])
def test_packed_experts_vs_oracle(E, n, k, levels, T):
    group = 128
    s, packed, scale, cb = experts(E, n, k, levels, group, seed=E + n)
    g = torch.Generator(device=DEV).manual_seed(T)
    x = torch.randn(T, k, generator=g, device=DEV).to(torch.bfloat16)
    ids = torch.randint(0, E - 1, (T,), generator=g, device=DEV)   # the last expert unused
    y = PackedExperts(s)(x, ids)
    assert y.shape == (T, n) and y.dtype == torch.bfloat16
    want = want_rows(x.float().cpu().numpy(), ids.cpu().tolist(), packed, scale, cb, E, n, k,
                     group, levels)
    got = y.float().cpu().numpy()
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < 2e-3 + 2.0 ** -8, err


def test_packed_experts_rejects_bad_ids():
    s, *_ = experts(2, 64, 128, 16, 128, seed=1)
    with pytest.raises(IndexError):
        PackedExperts(s)(torch.zeros(2, 128, device=DEV, dtype=torch.bfloat16),
                         torch.tensor([0, 2], device=DEV))


def test_expert_holder_attaches_only_during_forward():
    s, *_ = experts(4, 64, 128, 16, 64, seed=2)

    class Moe(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.weight = torch.nn.Parameter(torch.zeros(4, 64, 128))
            self.seen = None

        def forward(self, x):
            self.seen = self.weight
            # a plain reduction over the attached slab (no batched product)
            return x.float().sum(1)[:, None, None] * self.weight.float().sum(-1)[None]

    m = Moe().to(DEV)
    ExpertHolder(m, "weight", s, torch.bfloat16)
    assert m.weight is None
    y = m(torch.randn(3, 128, device=DEV))
    assert m.weight is None and y.shape == (3, 4, 64)
    assert torch.equal(m.seen, s.materialize(torch.bfloat16))
