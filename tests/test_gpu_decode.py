"""Greedy-decode parity of the gfx950 decoder against the dense float32
oracle (oracle/decoder.py, itself pinned against transformers on CPU).

Bar: greedy decode gives identical argmax tokens
for 64 steps.  The oracle rounds to bf16 where the GPU decoder stores bf16
(KV rows, attention output, lm_head input); everything else is float32, so
the remaining differences are the GEMV's fp16 operands and summation order.
Each test prints the oracle's smallest top-1/top-2 logit margin so a flip
can be told apart from a near-tie.
"""
import numpy as np
import pytest
import torch

from epure.decode import LLAMA3_8B, QWEN3_1_7B, Decoder, DecoderConfig, random_weights
from oracle.decoder import RefDecoder

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

SMALL = {
    "llama": DecoderConfig(512, 1536, 3, 8, 2, 64, 1000, 1e4, 1e-5, name="small-llama"),
    "qwen3": DecoderConfig(512, 1024, 3, 8, 4, 64, 1003, 1e6, 1e-6, qk_norm=True,
                           tie_embeddings=True, name="small-qwen3"),
}


def prompt_ids(n, vocab, seed):
    return np.random.Generator(np.random.PCG64(seed)).integers(0, vocab, n).tolist()


@pytest.mark.parametrize("arch", ["llama", "qwen3"])
def test_small_decoder_logits_and_argmax(arch):
    cfg = SMALL[arch]
    w = random_weights(cfg, seed=11, device=DEV)
    dec = Decoder(w, 128)
    ref = RefDecoder.from_weights(w, dec.max_pos)
    prompt = prompt_ids(8, cfg.vocab, 12)
    toks, ref_arg, margins = ref.generate(prompt, 40)
    dec.reset(toks)
    dec.capture()
    ref2 = RefDecoder.from_weights(w, dec.max_pos)
    worst = 0.0
    for pos in range(len(toks) - 1):
        dec.step()
        want = ref2.step(toks[pos], pos)
        got = dec.logits
        err = float((got - want).abs().max() / want.abs().max())
        worst = max(worst, err)
    torch.cuda.synchronize()
    got_arg = dec.argmax[:len(toks) - 1].cpu().tolist()
    print(f"{arch}: worst normwise logit error {worst:.2e}, min margin {min(margins):.3e}")
    assert got_arg == ref_arg
    # Both sides round the KV rows and the attention output to bf16; a value
    # that lands on the other side of a bf16 rounding boundary moves by 2^-9
    # relative, so the logits are compared at 1e-2 (argmax must match).
    assert worst < 1e-2


def test_graph_replay_matches_eager():
    cfg = SMALL["llama"]
    w = random_weights(cfg, seed=21, device=DEV)
    dec = Decoder(w, 64)
    prompt = prompt_ids(5, cfg.vocab, 22)
    a, _ = dec.generate(prompt, 30, use_graph=False)
    la = dec.logits.clone()
    b, _ = dec.generate(prompt, 30, use_graph=True)
    assert a == b
    assert torch.equal(la, dec.logits)


@pytest.mark.parametrize("persistent", [True, False], ids=["one-launch", "per-layer"])
@pytest.mark.parametrize("cfg,n_prompt", [(QWEN3_1_7B, 32), (LLAMA3_8B, 128)],
                         ids=["qwen3-1.7b", "llama3-8b"])
def test_greedy_64_steps_identical(cfg, n_prompt, persistent):
    w = random_weights(cfg, seed=0, device=DEV)
    dec = Decoder(w, n_prompt + 64 + 1, persistent=persistent)
    prompt = prompt_ids(n_prompt, cfg.vocab, 1)
    toks, _ = dec.generate(prompt, 64)
    ref = RefDecoder.from_weights(w, dec.max_pos)
    want, _, margins = ref.generate(prompt, 64)
    gen_m = margins[n_prompt - 1:]
    print(f"{cfg.name}: min oracle margin over the 64 greedy steps {min(gen_m):.3e}")
    assert not dec.step_failed(), "a grid barrier of the one-launch step timed out"
    first = next((i for i, (x, y) in enumerate(zip(toks, want)) if x != y), None)
    assert first is None, (f"diverged at position {first}: got {toks[first]} want {want[first]}, "
                           f"oracle margin there {margins[first - 1]:.3e}")
