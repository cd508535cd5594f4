"""Persistent decode step (ep_decode_step: every layer of a step in one
launch) against the per-layer launch sequence it replaces, and against the
dense float32 oracle through the greedy-decode tests of test_gpu_decode.py.

Both device paths compute in float32 (f32 KV cache and attention; GEMV
activations as hi + lo fp16 terms with per-32 power-of-two factors against
exact fp16 codebook entries, f32 accumulation); they differ in summation
order (the one-launch step's dot products run on the matrix cores, the
per-layer GEMV on v_dot2), the RMSNorm sum-of-squares grouping and the
attention's split over positions, i.e. in f32 rounding only.  Bars: the
normwise logit difference, plus argmax agreement wherever the difference
cannot reorder the top two.

Positions are taken past 512 so the attention's split-KV path (up to nine
64-position chunks per kv head, combined by chunk 0) runs, checked there
against the dense float32 oracle, and the hand-over time-out flag must stay
clear.
"""
import dataclasses

import numpy as np
import pytest
import torch

from epure.decode import (H2560_I6656, LLAMA3_8B, LLAMA32_3B, QWEN3_0_6B, QWEN3_1_7B, QWEN3_4B, QWEN3_8B,
                          Decoder, random_weights)
from oracle.decoder import RefDecoder

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
CFGS = {"qwen3-1.7b": QWEN3_1_7B, "llama3-8b": LLAMA3_8B}


def _ids(n, vocab, seed):
    return np.random.Generator(np.random.PCG64(seed)).integers(0, vocab, n).tolist()


@pytest.fixture(scope="module", params=list(CFGS))
def weights(request):
    cfg = CFGS[request.param]
    w = random_weights(cfg, seed=3, device=DEV)
    yield w
    del w
    torch.cuda.empty_cache()


def _pair(w, max_pos):
    p = Decoder(w, max_pos, persistent=True)
    m = Decoder(w, max_pos, persistent=False)
    assert p.persistent and not m.persistent
    return p, m


def test_persistent_matches_per_layer_launches(weights):
    """Both paths teacher-forced on the per-layer path's own greedy tokens:
    the argmax must agree wherever the two logit vectors' difference cannot
    reorder the top two, and the per-step normwise difference must stay at
    f32 rounding level (max < 5e-5)."""
    cfg = weights.cfg
    p, m = _pair(weights, 128)
    toks, _ = m.generate(_ids(20, cfg.vocab, 5), 40)
    p.reset(toks)
    m.reset(toks)
    p.capture()
    m.capture()
    diffs, mismatched = [], []
    for pos in range(len(toks) - 1):
        p.step()
        m.step()
        d = (p.logits - m.logits).abs().max()
        diffs.append(float(d / m.logits.abs().max()))
        top = torch.topk(m.logits, 2).values
        if int(p.logits.argmax()) != int(m.logits.argmax()) and float(top[0] - top[1]) > 2 * float(d):
            mismatched.append(pos)
    assert not p.step_failed(), "a grid barrier timed out"
    diffs = np.array(diffs)
    print(f"{cfg.name}: normwise difference median {np.median(diffs):.2e} "
          f"p95 {np.percentile(diffs, 95):.2e} max {diffs.max():.2e}")
    assert not mismatched, f"argmax differs beyond the logit difference at {mismatched}"
    assert diffs.max() < 5e-5


@pytest.mark.parametrize("name", list(CFGS))
def test_persistent_split_kv_long_context(name):
    """Positions 0..529 (one to nine 64-position chunks per kv head),
    teacher-forced with random tokens, against the dense float32 oracle, on
    a 2-layer model of the full shape (hidden, heads, intermediate: the same
    kernel variant; the layer count is a launch argument).

    Bars: median normwise error < 1e-5, 99th percentile < 5e-5, over all
    positions and over positions >= 256 (the split path) alone, and no worse
    than 2x the per-layer path's (plus f32 rounding slack)."""
    cfg = dataclasses.replace(CFGS[name], layers=2)
    w = random_weights(cfg, seed=4, device=DEV)
    p, m = _pair(w, 576)
    ref = RefDecoder.from_weights(w, p.max_pos)
    toks = _ids(530, cfg.vocab, 6)
    p.reset(toks)
    m.reset(toks)
    p.capture()
    m.capture()
    ep, em = [], []
    for pos in range(len(toks) - 1):
        p.step()
        m.step()
        want = ref.step(toks[pos], pos)
        n = want.abs().max()
        ep.append(float((p.logits - want).abs().max() / n))
        em.append(float((m.logits - want).abs().max() / n))
    assert not p.step_failed(), "a grid barrier timed out"
    ep, em = np.array(ep), np.array(em)
    for lo, label in ((0, "all positions"), (256, "positions >= 256")):
        a, b = ep[lo:], em[lo:]
        stats = (np.median(a), np.percentile(a, 99), np.median(b), np.percentile(b, 99))
        print(f"{cfg.name} x2 layers, {label}: one-launch median {stats[0]:.2e} p99 {stats[1]:.2e};"
              f" per-layer median {stats[2]:.2e} p99 {stats[3]:.2e}; max {a.max():.2e}/{b.max():.2e}")
        assert stats[0] < 1e-5 and stats[1] < 5e-5
        assert stats[0] <= 2 * stats[2] + 2e-6 and stats[1] <= 2 * stats[3] + 5e-6


def test_persistent_eager_equals_graph(weights):
    """The launch is replay-invariant: the barrier words and the attention
    counters are left ready for the next launch, eager or replayed."""
    cfg = weights.cfg
    d = Decoder(weights, 64, persistent=True)
    prompt = _ids(6, cfg.vocab, 7)
    a, _ = d.generate(prompt, 20, use_graph=False)
    la = d.logits.clone()
    b, _ = d.generate(prompt, 20, use_graph=True)
    assert a == b
    assert torch.equal(la, d.logits)
    assert not d.step_failed()


@pytest.mark.parametrize("base", [QWEN3_8B, LLAMA32_3B, QWEN3_4B],
                         ids=["qwen3-8b", "llama3.2-3b", "qwen3-4b"])
def test_more_shapes_one_launch_against_oracle(base):
    """The one-launch step at the Qwen3-8B, Llama-3.2-3B and Qwen3-4B shapes (full
    width, 3 layers: the layer count is a launch argument), teacher-forced
    over 140 random positions (three 64-position chunks) against the float32
    oracle, and 24 greedy tokens identical to the oracle's."""
    cfg = dataclasses.replace(base, layers=3)
    w = random_weights(cfg, seed=8, device=DEV)
    toks = _ids(140, cfg.vocab, 9)
    d = Decoder(w, len(toks) + 1, persistent=True)
    assert d.persistent
    ref = RefDecoder.from_weights(w, d.max_pos)
    d.reset(toks)
    d.capture()
    errs = []
    for pos in range(len(toks) - 1):
        d.step()
        want = ref.step(toks[pos], pos)
        errs.append(float((d.logits - want).abs().max() / want.abs().max()))
    assert not d.step_failed()
    errs = np.array(errs)
    print(f"{cfg.name} x3 layers: normwise median {np.median(errs):.2e} max {errs.max():.2e}")
    assert np.median(errs) < 1e-5 and errs.max() < 5e-5
    prompt = _ids(12, cfg.vocab, 10)
    got, _ = d.generate(prompt, 24)
    want, _, _ = ref.generate(prompt, 24)
    assert got == want


def _teacher_forced_and_greedy(w, n_pos=140, seed=9):
    """The one-launch step (it must serve the shape) teacher-forced over
    n_pos random positions against the float32 oracle, then 24 greedy
    tokens against the oracle's."""
    cfg = w.cfg
    toks = _ids(n_pos, cfg.vocab, seed)
    d = Decoder(w, len(toks) + 1, persistent=True)
    assert d.persistent
    ref = RefDecoder.from_weights(w, d.max_pos)
    d.reset(toks)
    d.capture()
    errs = []
    for pos in range(len(toks) - 1):
        d.step()
        want = ref.step(toks[pos], pos)
        errs.append(float((d.logits - want).abs().max() / want.abs().max()))
    assert not d.step_failed()
    errs = np.array(errs)
    print(f"{cfg.name} x{cfg.layers} layers: normwise median {np.median(errs):.2e} max {errs.max():.2e}")
    assert np.median(errs) < 1e-5 and errs.max() < 5e-5
    prompt = _ids(12, cfg.vocab, seed + 1)
    got, _ = d.generate(prompt, 24)
    want, _, _ = ref.generate(prompt, 24)
    assert got == want


@pytest.mark.parametrize("base", [QWEN3_0_6B, H2560_I6656], ids=["qwen3-0.6b", "h2560-i6656"])
def test_generic_shapes_one_launch_against_oracle(base):
    """Shapes outside the tuned list run the generic one-launch variant:
    the Qwen3-0.6B shape (hidden 1024, q/k norm, 2 query heads per kv head)
    and a Llama-style hidden 2560 / intermediate 6656 decoder with 20 query
    heads over 4 kv heads (GQ 5): 3 full-width layers, teacher-forced
    against the float32 oracle over 140 positions, 24 greedy tokens
    identical to the oracle's."""
    w = random_weights(dataclasses.replace(base, layers=3), seed=11, device=DEV)
    _teacher_forced_and_greedy(w)


def test_one_launch_f32_scales_against_oracle():
    """Group scales in f32 (as make_trainable leaves them, finetune.py:78),
    perturbed off the fp16 grid, at the Qwen3-1.7B shape: the one-launch
    step still serves it (the generic f32-scale variant) and matches the
    float32 oracle built from the same f32 scales."""
    w = random_weights(dataclasses.replace(QWEN3_1_7B, layers=3), seed=12, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(13)
    for L in w.layers:
        for s in L.lin.values():
            noise = torch.rand(s.scale.shape, generator=g, device=DEV) * 2.0 ** -10
            s.scale = (s.scale.float() * (1.0 + noise)).contiguous()
            assert s.scale.dtype == torch.float32
    _teacher_forced_and_greedy(w, seed=14)
