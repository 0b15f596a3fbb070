"""Native block-FP8 Qwen3.5 checkpoints (safetensors) -> ModelWeights.

Mirrors the reference loader (main.py:326-353 config, 575-700 weights):
  * config.json, flat or wrapped in `text_config`; the checkpoint must declare
    quantization_config = {quant_method: "fp8", weight_block_size: [128, 128]}
    (main.py:336-340);
  * every *.safetensors shard of the directory;
  * key prefix `model.language_model.` (the released checkpoints) or `model.`;
  * FP8 linears: `*.weight` (float8_e4m3fn) + `*.weight_scale_inv`
    [ceil(N/128), ceil(K/128)], kept as raw bytes; the scales are converted to
    bf16 like the reference does (main.py:597) unless scale_dtype says fp32;
  * norms fp32 ((1+w) form), GatedDeltaNet norm / conv1d / embed / lm_head
    bf16, A_log / dt_bias fp32; conv1d [C, 1, 4] -> [C, 4];
  * lm_head: bf16 `lm_head.weight`, else tied to the embedding.
Linears stored in bf16 are not run by the E4M3 kernels: with quantize_bf16 they
are quantized with the reference's block quantizer (main.py:833-848),
otherwise loading fails and names them.
"""
import glob
import json
import os

import torch

from .config import Qwen35Config
from .synth import ModelWeights, quantize_block_fp8


class CheckpointError(ValueError):
    """The directory does not hold a loadable native block-FP8 checkpoint."""


def _quant_config(cfg_json):
    q = cfg_json.get("quantization_config")
    if q is None and "text_config" in cfg_json:
        q = cfg_json["text_config"].get("quantization_config")
    return q or {}


def load_checkpoint(model_dir, device="cuda", scale_dtype=torch.bfloat16, quantize_bf16=False):
    """Load a native block-FP8 checkpoint directory into ModelWeights on `device`."""
    path = os.path.join(model_dir, "config.json")
    if not os.path.isfile(path):
        raise CheckpointError(f"{model_dir}: config.json not found")
    with open(path) as f:
        cfg_json = json.load(f)
    q = _quant_config(cfg_json)
    if not (q.get("quant_method") == "fp8" and list(q.get("weight_block_size", [])) == [128, 128]):
        raise CheckpointError(f"{model_dir}: not a native 128x128 block-FP8 checkpoint "
                              f"(quantization_config={q})")
    cfg = Qwen35Config.from_dict(cfg_json)
    shards = sorted(glob.glob(os.path.join(model_dir, "*.safetensors")))
    if not shards:
        raise CheckpointError(f"{model_dir}: no *.safetensors files")

    from safetensors import safe_open
    raw = {}
    for fn in shards:
        with safe_open(fn, framework="pt") as f:
            for k in f.keys():
                raw[k] = f.get_tensor(k)

    prefix = "model.language_model." if any(k.startswith("model.language_model.") for k in raw) \
        else "model."

    def need(k):
        if k not in raw:
            raise CheckpointError(f"{model_dir}: missing tensor {k}")
        return raw[k]

    def f32(k):
        return need(k).to(torch.float32).contiguous().to(device)

    def b16(k):
        return need(k).to(torch.bfloat16).contiguous().to(device)

    bf16_linears = []

    def linear(k):
        t = need(k)
        sk = k.replace(".weight", ".weight_scale_inv")
        if t.dtype == torch.float8_e4m3fn and sk in raw:
            w = t.view(torch.uint8).contiguous()
            s = raw[sk].to(scale_dtype).contiguous()
            exp = ((w.shape[0] + 127) // 128, (w.shape[1] + 127) // 128)
            if tuple(s.shape) != exp:
                raise CheckpointError(f"{sk}: shape {tuple(s.shape)}, expected {exp}")
            return w.to(device), s.to(device)
        if not quantize_bf16:
            bf16_linears.append(k)
            return None
        w, s = quantize_block_fp8(t.float())
        return w.to(device), s.to(scale_dtype).to(device)

    embed = b16(prefix + "embed_tokens.weight")
    norm_f = f32(prefix + "norm.weight")
    if "lm_head.weight" in raw:
        if raw["lm_head.weight"].dtype == torch.float8_e4m3fn:
            raise CheckpointError("FP8 lm_head is not supported (the decode path streams a bf16 "
                                  "lm_head, like the reference's preferred path)")
        lm_head = b16("lm_head.weight")
    else:
        lm_head = embed   # tied (main.py:653-656)

    layers = []
    for i in range(cfg.num_hidden_layers):
        base = f"{prefix}layers.{i}."
        ly = {"input_layernorm": f32(base + "input_layernorm.weight"),
              "post_attention_layernorm": f32(base + "post_attention_layernorm.weight"),
              "layer_type": cfg.layer_types[i]}
        if cfg.is_full(i):
            for n in ("q_proj", "k_proj", "v_proj", "o_proj"):
                ly[n] = linear(base + f"self_attn.{n}.weight")
            ly["q_norm"] = f32(base + "self_attn.q_norm.weight")
            ly["k_norm"] = f32(base + "self_attn.k_norm.weight")
        else:
            for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj"):
                ly[n] = linear(base + f"linear_attn.{n}.weight")
            ly["A_log"] = f32(base + "linear_attn.A_log")
            ly["dt_bias"] = f32(base + "linear_attn.dt_bias")
            cw = need(base + "linear_attn.conv1d.weight")
            ly["conv1d_w"] = cw.reshape(cw.shape[0], -1).to(torch.bfloat16).contiguous().to(device)
            ly["norm_w"] = b16(base + "linear_attn.norm.weight")
        for n in ("gate_proj", "up_proj", "down_proj"):
            ly[n] = linear(base + f"mlp.{n}.weight")
        layers.append(ly)
    if bf16_linears:
        raise CheckpointError("linears stored in bf16 (pass quantize_bf16=True to quantize them "
                              f"with the 128x128 block quantizer): {bf16_linears[:6]}"
                              + (" ..." if len(bf16_linears) > 6 else ""))
    return ModelWeights(cfg, embed, lm_head, norm_f, layers)


def save_checkpoint(weights, model_dir, prefix="model.language_model.", tied=False):
    """Write ModelWeights as a native block-FP8 checkpoint in the released
    layout (the inverse of load_checkpoint; used to build test checkpoints)."""
    from safetensors.torch import save_file
    os.makedirs(model_dir, exist_ok=True)
    cfg = weights.cfg
    t = {prefix + "embed_tokens.weight": weights.embed.cpu(),
         prefix + "norm.weight": weights.norm_f.cpu()}
    if not tied:
        t["lm_head.weight"] = weights.lm_head.cpu()

    def put_linear(k, ws):
        w, s = ws
        t[k] = w.cpu().view(torch.float8_e4m3fn)
        t[k.replace(".weight", ".weight_scale_inv")] = s.cpu().float()

    for i, ly in enumerate(weights.layers):
        base = f"{prefix}layers.{i}."
        t[base + "input_layernorm.weight"] = ly["input_layernorm"].cpu()
        t[base + "post_attention_layernorm.weight"] = ly["post_attention_layernorm"].cpu()
        if cfg.is_full(i):
            for n in ("q_proj", "k_proj", "v_proj", "o_proj"):
                put_linear(base + f"self_attn.{n}.weight", ly[n])
            t[base + "self_attn.q_norm.weight"] = ly["q_norm"].cpu()
            t[base + "self_attn.k_norm.weight"] = ly["k_norm"].cpu()
        else:
            for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj"):
                put_linear(base + f"linear_attn.{n}.weight", ly[n])
            t[base + "linear_attn.A_log"] = ly["A_log"].cpu()
            t[base + "linear_attn.dt_bias"] = ly["dt_bias"].cpu()
            t[base + "linear_attn.conv1d.weight"] = ly["conv1d_w"].cpu().unsqueeze(1)
            t[base + "linear_attn.norm.weight"] = ly["norm_w"].cpu()
        for n in ("gate_proj", "up_proj", "down_proj"):
            put_linear(base + f"mlp.{n}.weight", ly[n])
    save_file({k: v.contiguous() for k, v in t.items()},
              os.path.join(model_dir, "model.safetensors"))
    tc = cfg.to_dict()
    tc["rope_parameters"] = {"rope_type": "default", "rope_theta": cfg.rope_theta,
                             "partial_rotary_factor": cfg.partial_rotary_factor}
    cfg_json = {"architectures": ["Qwen3_5ForConditionalGeneration"], "text_config": tc,
                "quantization_config": {"quant_method": "fp8", "weight_block_size": [128, 128]}}
    with open(os.path.join(model_dir, "config.json"), "w") as f:
        json.dump(cfg_json, f, indent=1)
