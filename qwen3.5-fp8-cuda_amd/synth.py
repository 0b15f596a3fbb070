"""Seeded synthetic Qwen3.5-shaped weights and inputs.

There is no checkpoint in this environment; every benchmark and parity run
uses random-init weights of the real architecture, quantized exactly like the
reference's block quantizer (main.py:833-848): per 128x128 block,
s = max(amax / 448, 1e-12) and q = e4m3fn_RNE(W / s), with s kept in fp32
(the reference's checkpoints store fp32 `weight_scale_inv`; its quantizer rounds
s to bf16, which `scales_bf16()` reproduces for the reference ABI).

Draw order (one torch.Generator, seed `seed`): embed; per layer
input_layernorm, post_attention_layernorm, then the mixer
(full: q_proj, k_proj, v_proj, o_proj, q_norm, k_norm;
 linear: in_proj_qkv, in_proj_z, in_proj_b, in_proj_a, out_proj, conv1d,
 A_log, norm), then gate_proj, up_proj, down_proj; final norm; lm_head.
"""
import math

import torch

BLOCK = 128


def quantize_block_fp8(w, block=BLOCK):
    """fp32 [N, K] -> (uint8 E4M3FN bytes [N, K], fp32 scale_inv [ceil(N/128), ceil(K/128)])."""
    w = w.float()
    N, K = w.shape
    nb, kb = math.ceil(N / block), math.ceil(K / block)
    pad = torch.zeros(nb * block, kb * block, dtype=torch.float32, device=w.device)
    pad[:N, :K] = w
    blocks = pad.view(nb, block, kb, block)
    amax = blocks.abs().amax(dim=(1, 3))
    s = (amax / 448.0).clamp(min=1e-12)
    q = (blocks / s.view(nb, 1, kb, 1)).to(torch.float8_e4m3fn)
    q = q.reshape(nb * block, kb * block)[:N, :K].contiguous()
    return q.view(torch.uint8), s.contiguous()


class ModelWeights:
    """Weights in the reference's per-layer dict layout (main.py:614-688):
    FP8 linears are (uint8 bytes, fp32 scale_inv) tuples; norms fp32; the
    GatedDeltaNet norm, conv weights, embed and lm_head bf16."""

    LINEARS = ("q_proj", "k_proj", "v_proj", "o_proj", "in_proj_qkv", "in_proj_z",
               "in_proj_b", "in_proj_a", "out_proj", "gate_proj", "up_proj", "down_proj")

    def __init__(self, cfg, embed, lm_head, norm_f, layers):
        self.cfg = cfg
        self.embed = embed
        self.lm_head = lm_head
        self.norm_f = norm_f
        self.layers = layers

    def to(self, device):
        def mv(v):
            if isinstance(v, tuple):
                return tuple(t.to(device) for t in v)
            if isinstance(v, torch.Tensor):
                return v.to(device)
            return v
        layers = [{k: mv(v) for k, v in ly.items()} for ly in self.layers]
        return ModelWeights(self.cfg, mv(self.embed), mv(self.lm_head), mv(self.norm_f), layers)

    def nbytes_per_token(self):
        """Weight bytes a decode step streams: FP8 linears + scales + lm_head + one embed row."""
        n = 0
        for ly in self.layers:
            for k in self.LINEARS:
                if k in ly:
                    w, s = ly[k]
                    n += w.numel() + s.numel() * s.element_size()
        n += self.lm_head.numel() * 2 + self.cfg.hidden_size * 2
        return n


def make_weights(cfg, seed=0, device="cpu", std=0.02):
    g = torch.Generator(device=device)
    g.manual_seed(seed)

    def randn(*shape):
        return torch.randn(*shape, generator=g, device=device, dtype=torch.float32)

    def lin(n, k):
        return quantize_block_fp8(randn(n, k) * std)

    H, I, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    embed = (randn(V, H) * std).to(torch.bfloat16)
    layers = []
    for i in range(cfg.num_hidden_layers):
        ly = {"layer_type": cfg.layer_types[i]}
        ly["input_layernorm"] = randn(H) * std
        ly["post_attention_layernorm"] = randn(H) * std
        if cfg.is_full(i):
            ly["q_proj"] = lin(cfg.q_proj_rows, H)
            ly["k_proj"] = lin(cfg.kv_rows, H)
            ly["v_proj"] = lin(cfg.kv_rows, H)
            ly["o_proj"] = lin(H, cfg.attn_out_dim)
            ly["q_norm"] = randn(cfg.head_dim) * std
            ly["k_norm"] = randn(cfg.head_dim) * std
        else:
            Hv = cfg.linear_num_value_heads
            ly["in_proj_qkv"] = lin(cfg.conv_dim, H)
            ly["in_proj_z"] = lin(cfg.value_dim, H)
            ly["in_proj_b"] = lin(Hv, H)
            ly["in_proj_a"] = lin(Hv, H)
            ly["out_proj"] = lin(H, cfg.value_dim)
            ly["conv1d_w"] = (randn(cfg.conv_dim, cfg.linear_conv_kernel_dim) * std).to(torch.bfloat16)
            u = torch.rand(Hv, generator=g, device=device, dtype=torch.float32)
            ly["A_log"] = torch.log(1e-3 + u * (16.0 - 1e-3))
            ly["dt_bias"] = torch.ones(Hv, dtype=torch.float32, device=device)
            ly["norm_w"] = (1.0 + randn(cfg.linear_value_head_dim) * std).to(torch.bfloat16)
        ly["gate_proj"] = lin(I, H)
        ly["up_proj"] = lin(I, H)
        ly["down_proj"] = lin(H, I)
        layers.append(ly)
    norm_f = randn(H) * std
    lm_head = (randn(V, H) * std).to(torch.bfloat16)
    return ModelWeights(cfg, embed, lm_head, norm_f, layers)


def make_prompt(cfg, n=128, seed=1, device="cpu"):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.randint(0, cfg.vocab_size, (n,), generator=g, device=device, dtype=torch.int64)


def scales_bf16(weights):
    """Copy of `weights` with every scale_inv rounded to bf16 (the reference ABI)."""
    layers = []
    for ly in weights.layers:
        d = {}
        for k, v in ly.items():
            d[k] = (v[0], v[1].to(torch.bfloat16)) if isinstance(v, tuple) else v
        layers.append(d)
    return ModelWeights(weights.cfg, weights.embed, weights.lm_head, weights.norm_f, layers)
