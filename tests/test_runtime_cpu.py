"""Host logic of the drop-in package on CPU: packing helpers, the store, the
decline contract and the fine-tuning helpers (no GPU, no kernel launch)."""
import numpy as np
import pytest
import torch

from epure import PackedLinear, PackedWeight, make_trainable, snapshot_indices, verify_frozen
from epure import runtime
from epure.kernels import cpu, cuda
from oracle import ref


def store(n=16, k=256, levels=16, group=128, seed=0):
    idx, packed, scale, cb = ref.synth_linear(n, k, levels, group, seed=seed)
    return idx, PackedWeight((n, k), packed, scale, cb.astype(np.float32), group, levels)


@pytest.mark.parametrize("n", [1, 5, 64])
def test_pack4_matches_oracle(n):
    idx = np.random.Generator(np.random.PCG64(n)).integers(0, 16, n, dtype=np.uint8)
    assert np.array_equal(runtime._pack4(idx, 16), ref.pack4(idx, 16))
    assert np.array_equal(runtime._pack4(idx, 200), ref.pack4(idx, 200))


def test_unpack4_cpu_matches_oracle():
    b = np.random.Generator(np.random.PCG64(3)).integers(0, 256, 77, dtype=np.uint8)
    got = runtime._unpack4(torch.from_numpy(b), 153, 16).numpy()
    assert np.array_equal(got, ref.unpack4(b, 153, 16))


def test_store_shapes():
    _, s = store(n=12, k=64)
    assert s.in_features == 64 and s.out_features == 12
    assert tuple(s.packed_2d().shape) == (12, 32)


@pytest.mark.parametrize("dtype,name", [(torch.float32, "f32"), (torch.float16, "f16"),
                                        (torch.bfloat16, "bf16")])
def test_materialize_cpu_matches_oracle(dtype, name):
    idx, s = store()
    w = s.materialize(dtype).float().numpy()
    want = ref.materialize(s.packed.numpy(), s.scale.numpy(), s.cb.numpy(), 16, 256, 128, 16, name)
    assert np.array_equal(w, want)


def test_cpu_backend_declines_other_dtypes_and_linear_falls_back():
    _, s = store()
    x = torch.randn(3, 256).to(torch.bfloat16)
    assert cpu.available() is True and cpu.linear(x, s) is None   # bf16 x: decline
    assert cuda.linear(x, s) is None                    # CPU tensor: decline
    lin = PackedLinear(s, bias=torch.ones(16, dtype=torch.bfloat16))
    y = lin(x)
    want = torch.nn.functional.linear(x, s.materialize(torch.bfloat16), lin.bias)
    assert torch.equal(y, want)


def test_finetune_index_freeze_cycle():
    _, s = store()
    model = torch.nn.Sequential(PackedLinear(s))
    snap = snapshot_indices(model)
    params = make_trainable(model, "both", verbose=False)
    assert len(params) == 2 and all(p.dtype == torch.float32 for p in params)
    x = torch.randn(4, 256)
    model(x).square().sum().backward()       # materialize path: autograd reaches cb/scale
    assert s.cb.grad is not None and s.scale.grad is not None
    assert verify_frozen(model, snap)
    s.packed[0] ^= 1
    with pytest.raises(RuntimeError):
        verify_frozen(model, snap)


def test_make_trainable_rejects_mode():
    with pytest.raises(ValueError):
        make_trainable(torch.nn.Sequential(), "nope")


@pytest.mark.parametrize("dtype,name", [(torch.float32, "f32"), (torch.float16, "f16"),
                                        (torch.bfloat16, "bf16")])
@pytest.mark.parametrize("levels", [16, 256])
def test_packed_embedding_cpu_matches_oracle(dtype, name, levels):
    # the reference's torch expression (runtime.py:139-156) on CPU tensors
    idx, packed, scale, cb = ref.synth_linear(40, 128, levels, 32, seed=levels)
    s = PackedWeight((40, 128), packed, scale, cb.astype(np.float32), 32, levels)
    ids = torch.tensor([[3, 39], [0, 3]])
    out = runtime.PackedEmbedding(s, dtype)(ids)
    assert out.shape == (2, 2, 128) and out.dtype == dtype
    want = ref.embedding_rows(packed, scale.astype(np.float32), cb, 40, 128, 32, levels,
                              ids.numpy().ravel(), name)
    assert np.array_equal(out.float().numpy().reshape(-1, 128), want)


def test_packed_embedding_cpu_rejects_out_of_range():
    _, s = store(n=8, k=64)
    with pytest.raises(IndexError):
        runtime.PackedEmbedding(s)(torch.tensor([8]))


def test_tie_packed_lm_head_replaces_module_and_clears_flag():
    _, s = store(n=32, k=64)

    class M(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.config = type("C", (), {"tie_word_embeddings": True})()
            self.lm_head = torch.nn.Linear(64, 32, bias=False)

    m = runtime.tie_packed_lm_head(M(), s)
    assert isinstance(m.lm_head, PackedLinear) and m.lm_head.store is s
    assert m.config.tie_word_embeddings is False


def test_expert_holder_cpu_and_packed_experts_shape_checks():
    idx, packed, scale, cb = ref.synth_linear(3 * 8, 64, 16, 32, seed=9)
    s = PackedWeight((3, 8, 64), packed, scale, cb.astype(np.float32), 32, 16)

    class Moe(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.w = torch.nn.Parameter(torch.zeros(3, 8, 64))

        def forward(self, x):
            return self.w.sum() + x

    m = Moe()
    runtime.ExpertHolder(m, "w", s, torch.float32)
    assert m.w is None
    out = m(torch.zeros(1))
    want = ref.materialize(packed, scale, cb, 24, 64, 32, 16, "f32").sum()
    assert abs(float(out) - float(want)) < 1e-3 * max(1.0, abs(float(want)))
    assert m.w is None
    with pytest.raises(ValueError):
        runtime.PackedExperts(PackedWeight((24, 64), packed, scale, cb, 32, 16))
    with pytest.raises(RuntimeError):
        runtime.PackedExperts(s)(torch.zeros(2, 64), torch.tensor([0, 1]))


def test_pack4_rejects_wide_index_and_store_checks_bytes():
    with pytest.raises(ValueError):
        runtime._pack4(np.array([3, 16], np.uint8), 16)
    _, packed, scale, cb = ref.synth_linear(8, 64, 16, 32, seed=1)
    with pytest.raises(ValueError):
        PackedWeight((8, 64), packed[:-1], scale, cb, 32, 16)


@pytest.mark.parametrize("k", [7, 33])
def test_packed_embedding_odd_k_reads_flat_stream(k):
    # 4-bit rows with odd K are not byte-aligned: rows are read by flat position
    idx, packed, scale, cb = ref.synth_linear(9, k, 16, 4, seed=k)
    s = PackedWeight((9, k), packed, scale, cb.astype(np.float32), 4, 16)
    ids = torch.tensor([8, 0, 5, 5])
    got = runtime.PackedEmbedding(s, torch.float32)(ids)
    want = ref.dequant_tile_f32(idx.reshape(9, k), scale, cb, 4)[ids.numpy()]
    assert np.array_equal(got.numpy(), want)
