"""Pins oracle/decoder.py (the dense float32 decode restatement) against
transformers' own LlamaForCausalLM / Qwen3ForCausalLM -- the model classes the
reference's load() instantiates (epure/runtime.py:402-410) -- on tiny
configs with the same float32 weights (CPU, no network)."""
import pytest
import torch

from epure.decode import DecoderConfig, rope_tables
from oracle.decoder import RefDecoder, rope_tables_hf

transformers = pytest.importorskip("transformers")

TINY = {
    "llama": DecoderConfig(64, 128, 2, 4, 2, 16, 101, 5e5, 1e-5, name="tiny-llama"),
    "qwen3": DecoderConfig(64, 96, 2, 4, 2, 16, 97, 1e6, 1e-6, qk_norm=True,
                           tie_embeddings=True, name="tiny-qwen3"),
}


def hf_model(cfg, w):
    common = dict(hidden_size=cfg.hidden, intermediate_size=cfg.intermediate,
                  num_hidden_layers=cfg.layers, num_attention_heads=cfg.n_heads,
                  num_key_value_heads=cfg.n_kv, head_dim=cfg.head_dim, vocab_size=cfg.vocab,
                  rope_theta=cfg.rope_theta, rms_norm_eps=cfg.rms_eps,
                  tie_word_embeddings=cfg.tie_embeddings, max_position_embeddings=256)
    if cfg.qk_norm:
        model = transformers.Qwen3ForCausalLM(transformers.Qwen3Config(**common))
    else:
        model = transformers.LlamaForCausalLM(transformers.LlamaConfig(**common))
    sd = {"model.embed_tokens.weight": w["embed"], "model.norm.weight": w["final_norm"]}
    if not cfg.tie_embeddings:
        sd["lm_head.weight"] = w["lm_head"]
    for i, L in enumerate(w["layers"]):
        p = f"model.layers.{i}."
        for n in ("q", "k", "v", "o"):
            sd[p + f"self_attn.{n}_proj.weight"] = L[n]
        for n in ("gate", "up", "down"):
            sd[p + f"mlp.{n}_proj.weight"] = L[n]
        sd[p + "input_layernorm.weight"] = L["attn_norm"]
        sd[p + "post_attention_layernorm.weight"] = L["mlp_norm"]
        if cfg.qk_norm:
            sd[p + "self_attn.q_norm.weight"] = L["q_norm"]
            sd[p + "self_attn.k_norm.weight"] = L["k_norm"]
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in m or "lm_head" in m for m in missing), missing
    return model.float().eval()


def random_dense(cfg, seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g) * 0.2  # noqa: E731
    near1 = lambda n: 1 + 0.1 * torch.randn(n, generator=g)  # noqa: E731
    layers = []
    for _ in range(cfg.layers):
        L = {n: r(N, K) for n, N, K in cfg.packed_linear_shapes()}
        L["attn_norm"], L["mlp_norm"] = near1(cfg.hidden), near1(cfg.hidden)
        L["q_norm"] = near1(cfg.head_dim) if cfg.qk_norm else None
        L["k_norm"] = near1(cfg.head_dim) if cfg.qk_norm else None
        layers.append(L)
    embed = r(cfg.vocab, cfg.hidden)
    return {"embed": embed, "lm_head": embed if cfg.tie_embeddings else r(cfg.vocab, cfg.hidden),
            "final_norm": near1(cfg.hidden), "layers": layers}


def test_rope_tables_agree():
    cfg = TINY["llama"]
    a, b = rope_tables(cfg, 64, "cpu"), rope_tables_hf(cfg, 64, "cpu")
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("arch", ["llama", "qwen3"])
def test_oracle_decoder_matches_transformers(arch):
    cfg = TINY[arch]
    w = random_dense(cfg, 1)
    model = hf_model(cfg, w)
    ids = torch.randint(0, cfg.vocab, (1, 20), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        want = model(ids).logits[0]
    cos, sin = rope_tables_hf(cfg, 64, "cpu")
    ref = RefDecoder(cfg, w["embed"], w["lm_head"], w["final_norm"], w["layers"], cos, sin,
                     bf16_storage=False)
    got = torch.stack([ref.step(int(t), p) for p, t in enumerate(ids[0])])
    err = (got - want).abs().max() / want.abs().max()
    assert err < 1e-5, f"{arch}: normwise {err:.2e}"
    assert torch.equal(got.argmax(-1), want.argmax(-1))


def test_oracle_greedy_matches_transformers_generate():
    cfg = TINY["llama"]
    w = random_dense(cfg, 3)
    model = hf_model(cfg, w)
    prompt = [5, 17, 42, 7]
    with torch.no_grad():
        out = model.generate(torch.tensor([prompt]), max_new_tokens=12, do_sample=False,
                             pad_token_id=0)
    cos, sin = rope_tables_hf(cfg, 64, "cpu")
    ref = RefDecoder(cfg, w["embed"], w["lm_head"], w["final_norm"], w["layers"], cos, sin,
                     bf16_storage=False)
    toks, _, _ = ref.generate(prompt, 12)
    assert toks == out[0].tolist()
