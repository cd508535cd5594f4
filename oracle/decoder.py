"""Dense float32 restatement of the packed decoder (TEST INFRASTRUCTURE ONLY).

The reference decodes through transformers' LlamaForCausalLM /
Qwen3ForCausalLM with PackedLinear modules (epure/runtime.py:373-415,
:92-126).  This module restates one greedy decode step with dense float32
weights -- the exact f32 tile cb[idx] * scale (container.py:70-88) --
for the GPU decoder's parity tests.

The default is pure float32, the mode pinned against transformers itself
(tests/test_oracle_decoder.py) and the precision the GPU decoder computes
in.  ``bf16_storage=True`` additionally rounds to bf16 where a bf16 model
stores bf16 values (the KV cache rows, the attention output fed to o_proj,
the normalized lm_head input), for comparisons with a bf16-storage run.

Runs on whatever device its tensors live on (CPU for pinning, the GPU for
full-size parity runs, where a dense f32 copy of the weights fits).
"""
import math

import torch


def dense_tile(packed, scale, cb, n, k, group, levels):
    """f32(cb[idx]) * f32(scale) from the flat packed stream, in torch."""
    if levels <= 16:
        both = torch.stack((packed & 0x0F, packed >> 4), dim=-1).reshape(-1)[:n * k]
    else:
        both = packed[:n * k]
    idx = both.reshape(n, k).long()
    cbf = torch.zeros(256, dtype=torch.float32, device=packed.device)
    cbf[:cb.numel()] = cb.float().reshape(-1)
    sc = scale.float().reshape(n, -1).repeat_interleave(group, dim=1)[:, :k]
    return cbf[idx] * sc


def round_bf16(t):
    return t.to(torch.bfloat16).float()


def rms(x, w, eps):
    return x * torch.rsqrt(x.square().mean(-1, keepdim=True) + eps) * w.float()


def rope_tables_hf(cfg, max_pos, device):
    """cos/sin [max_pos, head_dim/2] the way transformers' LlamaRotaryEmbedding
    computes them (default rope type): inv_freq = 1 / theta^(2i/d) in f32,
    freqs = position * inv_freq in f32."""
    d = cfg.head_dim
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
    freqs = torch.arange(max_pos, dtype=torch.int64).float()[:, None] * inv[None, :]
    return freqs.cos().to(device), freqs.sin().to(device)


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


class RefDecoder:
    """Greedy decoder over dense f32 weights.

    ``layers``: list of dicts with dense f32 tensors q, k, v, o, gate, up,
    down ([N, K]), attn_norm, mlp_norm, and q_norm / k_norm (or None).
    """

    def __init__(self, cfg, embed, lm_head, final_norm, layers, cos, sin, bf16_storage=False):
        self.cfg, self.embed, self.lm_head, self.final_norm = cfg, embed, lm_head, final_norm
        self.layers, self.cos, self.sin = layers, cos.float(), sin.float()
        self.bf16 = bf16_storage
        self.max_pos = cos.shape[0]
        dev = embed.device
        D = cfg.head_dim
        self.kc = [torch.zeros(cfg.n_kv, self.max_pos, D, device=dev) for _ in layers]
        self.vc = [torch.zeros(cfg.n_kv, self.max_pos, D, device=dev) for _ in layers]

    @classmethod
    def from_weights(cls, w, max_pos, bf16_storage=False, device=None):
        """Build from epure.decode.DecoderWeights (packed) by dequantizing."""
        cfg = w.cfg
        dev = device or w.embed.device
        layers = []
        for L in w.layers:
            d = {}
            for name, s in L.lin.items():
                d[name] = dense_tile(s.packed.to(dev), s.scale.to(dev), s.cb.to(dev),
                                     s.out_features, s.in_features, s.group, s.levels)
            d["attn_norm"], d["mlp_norm"] = L.attn_norm.to(dev), L.mlp_norm.to(dev)
            d["q_norm"] = L.q_norm.to(dev) if L.q_norm is not None else None
            d["k_norm"] = L.k_norm.to(dev) if L.k_norm is not None else None
            layers.append(d)
        cos, sin = rope_tables_hf(cfg, max_pos, dev)
        return cls(cfg, w.embed.to(dev), w.lm_head.to(dev), w.final_norm.to(dev), layers, cos,
                   sin, bf16_storage)

    @torch.no_grad()
    def step(self, token, pos):
        """Logits (f32 [vocab]) after feeding `token` at position `pos`."""
        cfg, D = self.cfg, self.cfg.head_dim
        rnd = round_bf16 if self.bf16 else (lambda t: t)
        h = self.embed[token].float()
        cos = torch.cat((self.cos[pos], self.cos[pos]))
        sin = torch.cat((self.sin[pos], self.sin[pos]))
        group = cfg.n_heads // cfg.n_kv
        for li, L in enumerate(self.layers):
            xn = rms(h, L["attn_norm"], cfg.rms_eps)
            q = (L["q"] @ xn).view(cfg.n_heads, D)
            k = (L["k"] @ xn).view(cfg.n_kv, D)
            v = (L["v"] @ xn).view(cfg.n_kv, D)
            if L["q_norm"] is not None:
                q = rms(q, L["q_norm"], cfg.rms_eps)
                k = rms(k, L["k_norm"], cfg.rms_eps)
            q = q * cos + rotate_half(q) * sin
            k = k * cos + rotate_half(k) * sin
            self.kc[li][:, pos] = rnd(k)
            self.vc[li][:, pos] = rnd(v)
            K = self.kc[li][:, :pos + 1].repeat_interleave(group, dim=0)
            V = self.vc[li][:, :pos + 1].repeat_interleave(group, dim=0)
            s = torch.matmul(K, q.unsqueeze(-1)).squeeze(-1) / math.sqrt(D)
            p = torch.softmax(s, dim=-1)
            o = rnd(torch.matmul(p.unsqueeze(1), V).reshape(-1))
            h = h + L["o"] @ o
            xn = rms(h, L["mlp_norm"], cfg.rms_eps)
            g = L["gate"] @ xn
            u = L["up"] @ xn
            h = h + L["down"] @ (torch.nn.functional.silu(g) * u)
        rinv = torch.rsqrt(h.square().mean() + cfg.rms_eps)
        xn = rnd(rnd(h * rinv) * self.final_norm.float())
        return self.lm_head.float() @ xn

    def generate(self, prompt, n_new, teacher=None):
        """Greedy decode.  With ``teacher`` (a token list), feed those tokens
        instead of the argmax (teacher forcing).  Returns (tokens, argmax per
        position, top-1 minus top-2 logit margin per position)."""
        toks = list(prompt)
        argm, margins = [], []
        total = len(prompt) + n_new
        for pos in range(total - 1):
            logits = self.step(toks[pos], pos)
            top = torch.topk(logits, 2)
            a = int(top.indices[0])
            argm.append(a)
            margins.append(float(top.values[0] - top.values[1]))
            if pos + 1 < len(toks):
                continue
            toks.append(teacher[pos + 1] if teacher is not None else a)
        return toks, argm, margins
