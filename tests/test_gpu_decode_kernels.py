"""Each decode-step kernel of include/epure_decode.h against a float32
reference of the same operation (the fused-prologue GEMVs, attention with
KV append, lm_head with greedy selection)."""
import ctypes
import math

import numpy as np
import pytest
import torch

from epure.decode import DecoderConfig, rope_tables
from epure.kernels import _abi
from oracle import ref
from oracle.decoder import dense_tile, rms, rotate_half

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def g(seed):
    return torch.Generator(device=DEV).manual_seed(seed)


def packed_store(n, k, seed, levels=16, group=128):
    _, packed, scale, cb = ref.synth_linear(n, k, levels, group, seed=seed)
    p = torch.from_numpy(packed).to(DEV)
    s = torch.from_numpy(scale).to(DEV)
    c = torch.from_numpy(cb.astype(np.float32)).to(DEV)
    return p, s, c, dense_tile(p, s, c, n, k, group, levels)


def normwise(y, r):
    return float((y - r).abs().max() / r.abs().max())


def fused(xsrc, x, x_aux, segs, ys, K, eps=1e-5, accumulate=False, x_dtype=_abi.F32):
    n = len(segs)
    P = lambda ts: (ctypes.c_void_p * n)(*[t.data_ptr() for t in ts])  # noqa: E731
    rc = _abi.lib.ep_fused_gemv(
        xsrc, x.data_ptr(), x_dtype, x_aux.data_ptr() if x_aux is not None else None, eps, K, 128,
        16, _abi.F16, _abi.F32, n, P([s[0] for s in segs]), P([s[1] for s in segs]),
        P([s[2] for s in segs]), P(ys), (ctypes.c_int64 * n)(*[y.numel() for y in ys]), _abi.F32,
        int(accumulate), _abi.stream_handle())
    assert rc == 0, _abi.last_error()
    torch.cuda.synchronize()


@pytest.mark.parametrize("K", [512, 2048, 4096, 14336])
def test_fused_rmsnorm_three_segments(K):
    segs = [packed_store(n, K, seed=K + i) for i, n in enumerate((1000, 64, 48))]
    h = torch.randn(K, generator=g(1), device=DEV) * 3
    w = (1 + 0.1 * torch.randn(K, generator=g(2), device=DEV)).to(torch.bfloat16)
    ys = [torch.zeros(s[3].shape[0], device=DEV) for s in segs]
    fused(_abi.XSRC_RMSNORM, h, w, segs, ys, K)
    xn = rms(h, w, 1e-5)
    for y, s in zip(ys, segs):
        assert normwise(y, s[3] @ xn) < 2e-5   # f32 activations as hi + lo fp16 terms


@pytest.mark.parametrize("K", [1024, 6144, 14336])
def test_fused_swiglu_accumulate(K):
    seg = packed_store(4096, K, seed=K)
    gt = torch.randn(K, generator=g(3), device=DEV) * 2
    ut = torch.randn(K, generator=g(4), device=DEV)
    y0 = torch.randn(4096, generator=g(5), device=DEV)
    y = y0.clone()
    fused(_abi.XSRC_SWIGLU, gt, ut, [seg], [y], K, accumulate=True)
    want = y0 + seg[3] @ (torch.nn.functional.silu(gt) * ut)
    assert normwise(y, want) < 2e-5


def test_fused_plain_bf16_accumulate():
    K = 4096
    seg = packed_store(4096, K, seed=9)
    x = torch.randn(K, generator=g(6), device=DEV).to(torch.bfloat16)
    y0 = torch.randn(4096, generator=g(7), device=DEV)
    y = y0.clone()
    fused(_abi.XSRC_PLAIN, x, None, [seg], [y], K, accumulate=True, x_dtype=_abi.BF16)
    assert normwise(y, y0 + seg[3] @ x.float()) < 2e-3


def attention_ref(q, k, v, kc, vc, cos, sin, pos, Hq, Hkv, D, qn, kn, eps):
    q = q.view(Hq, D)
    k = k.view(Hkv, D)
    v = v.view(Hkv, D)
    if qn is not None:
        q, k = rms(q, qn, eps), rms(k, kn, eps)
    c = torch.cat((cos[pos], cos[pos]))
    s = torch.cat((sin[pos], sin[pos]))
    q = q * c + rotate_half(q) * s
    k = k * c + rotate_half(k) * s
    K = kc[:, :pos + 1].float().clone()
    V = vc[:, :pos + 1].float().clone()
    K[:, pos], V[:, pos] = k, v
    grp = Hq // Hkv
    K, V = K.repeat_interleave(grp, 0), V.repeat_interleave(grp, 0)
    p = torch.softmax(torch.matmul(K, q.unsqueeze(-1)).squeeze(-1) / math.sqrt(D), -1)
    return torch.matmul(p.unsqueeze(1), V).reshape(-1), k, v


@pytest.mark.parametrize("qk_norm", [False, True])
@pytest.mark.parametrize("Hq,Hkv,D", [(32, 8, 128), (16, 8, 128), (8, 2, 64)])
@pytest.mark.parametrize("pos", [0, 1, 63, 64, 130, 255])
def test_decode_attention(qk_norm, Hq, Hkv, D, pos):
    max_pos = 256
    cfg = DecoderConfig(Hq * D, 1024, 1, Hq, Hkv, D, 100, 5e5)
    cos, sin = rope_tables(cfg, max_pos, DEV)
    q = torch.randn(Hq * D, generator=g(pos), device=DEV)
    k = torch.randn(Hkv * D, generator=g(pos + 1), device=DEV)
    v = torch.randn(Hkv * D, generator=g(pos + 2), device=DEV)
    kc = torch.randn(Hkv, max_pos, D, generator=g(3), device=DEV)
    vc = torch.randn(Hkv, max_pos, D, generator=g(4), device=DEV)
    qn = (1 + 0.1 * torch.randn(D, generator=g(5), device=DEV)).to(torch.bfloat16) \
        if qk_norm else None
    kn = (1 + 0.1 * torch.randn(D, generator=g(6), device=DEV)).to(torch.bfloat16) \
        if qk_norm else None
    want, kw, vw = attention_ref(q, k, v, kc, vc, cos, sin, pos, Hq, Hkv, D, qn, kn, 1e-6)
    state = torch.tensor([pos, 0], dtype=torch.int32, device=DEV)
    part = torch.zeros(_abi.lib.ep_attention_workspace(Hq, D, max_pos) // 4, device=DEV)
    ctr = torch.zeros(Hq, dtype=torch.int32, device=DEV)
    out = torch.zeros(Hq * D, dtype=torch.float32, device=DEV)
    for rep in range(2):                                 # second call: counters were reset
        rc = _abi.lib.ep_decode_attention(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), qn.data_ptr() if qk_norm else None,
            kn.data_ptr() if qk_norm else None, 1e-6, kc.data_ptr(), vc.data_ptr(),
            cos.data_ptr(), sin.data_ptr(), state.data_ptr(), part.data_ptr(), ctr.data_ptr(),
            out.data_ptr(), Hq, Hkv, D, max_pos, 1.0 / math.sqrt(D), _abi.stream_handle())
        assert rc == 0, _abi.last_error()
        torch.cuda.synchronize()
        assert not ctr.any()
        # float32 throughout: f32 rounding and summation order only
        assert normwise(out, want) < 2e-6
        assert normwise(kc[:, pos], kw) < 2e-6
        assert torch.equal(vc[:, pos], vw)


@pytest.mark.parametrize("V,H,n_prompt,pos", [(1000, 512, 1, 0), (128256, 4096, 10, 3),
                                              (50000, 2048, 4, 9)])
def test_lm_head_argmax(V, H, n_prompt, pos):
    W = (torch.randn(V, H, generator=g(1), device=DEV) * 0.02).to(torch.bfloat16)
    emb = (torch.randn(V, H, generator=g(2), device=DEV) * 0.02).to(torch.bfloat16)
    h = torch.randn(H, generator=g(3), device=DEV)
    nw = (1 + 0.1 * torch.randn(H, generator=g(4), device=DEV)).to(torch.bfloat16)
    xn = h * torch.rsqrt(h.square().mean() + 1e-5) * nw.float()
    want = W.float() @ xn
    am = int(want.argmax())
    grid = 1024
    logits = torch.zeros(V, device=DEV)
    pv = torch.zeros(grid, device=DEV)
    pi = torch.zeros(grid, dtype=torch.int32, device=DEV)
    ctr = torch.zeros(1, dtype=torch.int32, device=DEV)
    state = torch.tensor([pos, 7], dtype=torch.int32, device=DEV)
    prompt = torch.arange(100, 100 + max(n_prompt, 1), dtype=torch.int32, device=DEV)
    tokens = torch.zeros(64, dtype=torch.int32, device=DEV)
    amax = torch.full((63,), -1, dtype=torch.int32, device=DEV)
    rc = _abi.lib.ep_lm_head_argmax(
        h.data_ptr(), nw.data_ptr(), 1e-5, W.data_ptr(), logits.data_ptr(), V, H, pv.data_ptr(),
        pi.data_ptr(), ctr.data_ptr(), state.data_ptr(), prompt.data_ptr(), n_prompt,
        tokens.data_ptr(), amax.data_ptr(), emb.data_ptr(), 63, grid, _abi.stream_handle())
    assert rc == 0, _abi.last_error()
    torch.cuda.synchronize()
    assert normwise(logits, want) < 1e-5                   # f32 products, f32 sums
    assert int(amax[pos]) == am, (int(amax[pos]), am, float(torch.topk(want, 2).values.diff()))
    nxt = 100 + pos + 1 if pos + 1 < n_prompt else am
    assert int(tokens[pos + 1]) == nxt and state.tolist() == [pos + 1, nxt]
    assert torch.equal(h, emb[nxt].float())
    assert int(ctr) == 0
