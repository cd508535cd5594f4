"""Packed embedding (epure/runtime.py:129-160) and the tied lm_head through
the packed linear (runtime.py:289-300), on the gfx950 library.

Rows must be bit-exact against the oracle's restatement
(oracle/ref.py embedding_rows, pinned to materialize rows and brute force);
the tied lm_head is held to the packed-linear bar (max relative error 2e-3
against the Rust-order float32 result).
"""
import numpy as np
import pytest
import torch

from epure import PackedEmbedding, PackedLinear, PackedWeight, tie_packed_lm_head
from epure.kernels import cuda
from oracle import ref, rowdot

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def store(n, k, levels, group, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    idx = rng.integers(0, levels, n * k).astype(np.uint8)
    packed = ref.pack4(idx, levels)
    cb = np.sort(rng.standard_normal(levels)).astype(np.float16).astype(np.float32)
    scale = (np.abs(rng.normal(0, 0.02, (n, -(-k // group)))) + 1e-3).astype(np.float16)
    s = PackedWeight((n, k), packed, scale, cb, group, levels).to(DEV)
    return s, packed, scale, cb


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("n,k,levels,group", [(1000, 256, 16, 128), (300, 96, 256, 32),
                                              (77, 130, 16, 64), (50, 37, 16, 16)])
def test_embedding_rows_bitexact(dtype, n, k, levels, group):
    s, packed, scale, cb = store(n, k, levels, group, seed=n + k)
    ids = torch.tensor([[0, n - 1, 3], [3, n // 2, 1]], dtype=torch.int64, device=DEV)
    emb = PackedEmbedding(s, TDT[dtype])
    out = emb(ids)
    torch.cuda.synchronize()
    assert out.shape == (2, 3, k) and out.dtype == TDT[dtype]
    want = ref.embedding_rows(packed, scale.astype(np.float32), cb, n, k, group, levels,
                              ids.cpu().numpy().ravel(), dtype)
    assert np.array_equal(out.float().cpu().numpy().reshape(-1, k), want)


def test_embedding_matches_materialize_rows_and_weight():
    s, *_ = store(512, 512, 16, 128, seed=3)
    emb = PackedEmbedding(s, torch.bfloat16)
    ids = torch.randint(0, 512, (64,), device=DEV)
    assert torch.equal(emb(ids), s.materialize(torch.bfloat16)[ids])
    assert torch.equal(emb.weight, s.materialize(torch.bfloat16))


def test_embedding_cpu_path_matches_gpu():
    s, packed, scale, cb = store(200, 128, 16, 64, seed=4)
    s_cpu = PackedWeight((200, 128), packed, scale, cb, 64, 16)
    ids = torch.tensor([5, 199, 0, 5], dtype=torch.int64)
    a = PackedEmbedding(s_cpu, torch.float16)(ids)
    b = PackedEmbedding(s, torch.float16)(ids.to(DEV)).cpu()
    assert torch.equal(a, b)


def test_embedding_rejects_out_of_range_ids():
    s, *_ = store(100, 64, 16, 64, seed=5)
    emb = PackedEmbedding(s)
    with pytest.raises(IndexError):
        emb(torch.tensor([0, 100], device=DEV))
    with pytest.raises(IndexError):
        emb(torch.tensor([-1], device=DEV))


def test_embedding_graph_replay_matches_eager():
    s, *_ = store(4096, 1024, 16, 128, seed=6)
    emb = PackedEmbedding(s, torch.bfloat16)
    ids = torch.zeros(8, dtype=torch.int64, device=DEV)
    g = torch.cuda.CUDAGraph()
    emb(ids)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        out = emb(ids)
    for r in range(3):
        ids.copy_(torch.randint(0, 4096, (8,), device=DEV))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, emb(ids)), f"replay {r}"


def test_tied_lm_head_runs_the_packed_linear():
    # a tied vocab x hidden store used both as the embedding and as lm_head
    # (Qwen3-1.7B width, a 32768-row vocabulary slice)
    n, k, group = 32768, 2048, 128
    s, packed, scale, cb = store(n, k, 16, group, seed=7)

    class M(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.config = type("C", (), {"tie_word_embeddings": True})()
            self.lm_head = torch.nn.Linear(k, n, bias=False)

    m = tie_packed_lm_head(M(), s)
    assert isinstance(m.lm_head, PackedLinear) and m.lm_head.store is s
    assert m.config.tie_word_embeddings is False
    h = PackedEmbedding(s, torch.bfloat16)(torch.tensor([[11]], device=DEV))[0]  # [1, k]
    logits = m.lm_head(h)
    assert logits.shape == (1, n)
    x32 = h.float().cpu().numpy()
    want = rowdot.dequant_matmul(x32, packed.reshape(n, k // 2), scale.astype(np.float32),
                                 cb, group, True)
    got = logits.float().cpu().numpy()
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < 2e-3 + 2.0 ** -8, err   # bf16 output rounding
    assert cuda.available()
