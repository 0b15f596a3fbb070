"""Golden vectors from transformers' Qwen3.5 implementation for the CPU oracle.

The reference engine takes its conv update and gated delta rule from the
third-party `transformers` package (main.py:21-26, unpinned `>=5.0`,
requirements.txt:3) and its model structure from the same model family.
This script runs that package's own functions on small seeded inputs and
stores inputs and outputs as data, so tests/test_golden_cpu.py can pin the
oracle's restatements without importing transformers at test time:

  * torch_chunk_gated_delta_rule / torch_recurrent_gated_delta_rule
    (T = 70 crosses a 64-chunk boundary; l2norm of q, k inside the rule);
  * causal_conv1d_update (torch path) and l2norm;
  * Qwen3_5RMSNorm ((1+w) form) and Qwen3_5RMSNormGated;
  * Qwen3_5TextRotaryEmbedding + apply_rotary_pos_emb (partial rotary);
  * a whole tiny Qwen3_5ForCausalLM (4 layers: 3 GatedDeltaNet + 1 gated
    attention) in fp32, loaded with the dequantized weights of
    synth.make_weights(tiny(), seed=0): logits of every position of an
    8-token prompt.

Run in the build container only (no network; Hub kernels disabled):
    python tests/golden/make_golden.py
Writes tests/golden/qwen35_hf_golden.safetensors (~60 KB).
"""
import os
import sys

os.environ.setdefault("HF_HUB_OFFLINE", "1")
os.environ.setdefault("TRANSFORMERS_OFFLINE", "1")
os.environ.setdefault("USE_HUB_KERNELS", "0")

import torch  # noqa: E402
import torch.nn.functional as F  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import transformers  # noqa: E402
from safetensors.torch import save_file  # noqa: E402
from transformers.models.qwen3_5 import modeling_qwen3_5 as hf  # noqa: E402
from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig  # noqa: E402

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()
from oracle import qwen35_oracle as orc  # noqa: E402
from qwen35_amd import config as qcfg, synth  # noqa: E402

OUT = os.path.join(HERE, "qwen35_hf_golden.safetensors")


def bf(x):
    return x.to(torch.bfloat16).float()


def hf_config(cfg):
    return Qwen3_5TextConfig(
        vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
        intermediate_size=cfg.intermediate_size, num_hidden_layers=cfg.num_hidden_layers,
        num_attention_heads=cfg.num_attention_heads, num_key_value_heads=cfg.num_key_value_heads,
        head_dim=cfg.head_dim, linear_num_key_heads=cfg.linear_num_key_heads,
        linear_num_value_heads=cfg.linear_num_value_heads,
        linear_key_head_dim=cfg.linear_key_head_dim,
        linear_value_head_dim=cfg.linear_value_head_dim,
        linear_conv_kernel_dim=cfg.linear_conv_kernel_dim, rms_norm_eps=cfg.rms_norm_eps,
        rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta,
                         "partial_rotary_factor": cfg.partial_rotary_factor},
        tie_word_embeddings=False, layer_types=list(cfg.layer_types))


def hf_state_dict(w):
    """Our synthetic weights in transformers' parameter names (fp32, FP8
    linears dequantized with their block scales)."""
    deq = lambda ws: orc.dequant(ws[0], ws[1]).float()
    sd = {"model.embed_tokens.weight": w.embed.float(), "lm_head.weight": w.lm_head.float(),
          "model.norm.weight": w.norm_f.float()}
    for i, ly in enumerate(w.layers):
        p = f"model.layers.{i}."
        sd[p + "input_layernorm.weight"] = ly["input_layernorm"].float()
        sd[p + "post_attention_layernorm.weight"] = ly["post_attention_layernorm"].float()
        for n in ("gate_proj", "up_proj", "down_proj"):
            sd[p + f"mlp.{n}.weight"] = deq(ly[n])
        if "q_proj" in ly:
            for n in ("q_proj", "k_proj", "v_proj", "o_proj"):
                sd[p + f"self_attn.{n}.weight"] = deq(ly[n])
            sd[p + "self_attn.q_norm.weight"] = ly["q_norm"].float()
            sd[p + "self_attn.k_norm.weight"] = ly["k_norm"].float()
        else:
            for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj"):
                sd[p + f"linear_attn.{n}.weight"] = deq(ly[n])
            sd[p + "linear_attn.conv1d.weight"] = ly["conv1d_w"].float().unsqueeze(1)
            sd[p + "linear_attn.A_log"] = ly["A_log"].float()
            sd[p + "linear_attn.dt_bias"] = ly["dt_bias"].float()
            sd[p + "linear_attn.norm.weight"] = ly["norm_w"].float()
    return sd


@torch.no_grad()
def main():
    g = torch.Generator().manual_seed(1234)
    r = lambda *s: torch.randn(*s, generator=g)
    out = {}

    # --- gated delta rule, chunked and recurrent ------------------------------
    T, H, dk, dv = 70, 2, 16, 16
    q, k, v = r(1, T, H, dk), r(1, T, H, dk), r(1, T, H, dv)
    gl = -F.softplus(r(1, T, H))
    beta = torch.sigmoid(r(1, T, H))
    oc, sc = hf.torch_chunk_gated_delta_rule(q, k, v, gl, beta, chunk_size=64,
                                             output_final_state=True, use_qk_l2norm_in_kernel=True)
    orr, sr = hf.torch_recurrent_gated_delta_rule(q, k, v, gl, beta, initial_state=None,
                                                  output_final_state=True,
                                                  use_qk_l2norm_in_kernel=True)
    out.update({"gdr.q": q[0], "gdr.k": k[0], "gdr.v": v[0], "gdr.g": gl[0], "gdr.beta": beta[0],
                "gdr.chunk_out": oc[0], "gdr.chunk_state": sc[0],
                "gdr.rec_out": orr[0], "gdr.rec_state": sr[0]})

    # --- conv update (one token, window 4) and l2norm -------------------------
    C = 24
    state = bf(r(1, C, 4))
    x = bf(r(1, C, 1))
    wc = bf(r(C, 4) * 0.5)
    st = state.clone()
    y = hf.causal_conv1d_update(x, st, wc, None, "silu")
    out.update({"conv.x": x[0, :, 0], "conv.state": state[0], "conv.w": wc,
                "conv.y": y[0, :, 0], "conv.state_out": st[0]})
    xl = r(3, 64).to(torch.bfloat16)
    out.update({"l2.x": xl.float(), "l2.y": hf.l2norm(xl).float()})

    # --- RMSNorm (1+w), RMSNormGated ------------------------------------------
    D = 256
    nrm = hf.Qwen3_5RMSNorm(D, eps=1e-6)
    nrm.weight.copy_(r(D) * 0.02)
    xn = r(2, D).to(torch.bfloat16)
    out.update({"rms.x": xn.float(), "rms.w": nrm.weight.detach().clone(),
                "rms.y": nrm(xn).float()})
    gn = hf.Qwen3_5RMSNormGated(128, eps=1e-6).to(torch.bfloat16)
    gn.weight.copy_((1 + r(128) * 0.02).to(torch.bfloat16))
    core, z = r(4, 128).to(torch.bfloat16), r(4, 128).to(torch.bfloat16)
    out.update({"rmsg.core": core.float(), "rmsg.z": z.float(), "rmsg.w": gn.weight.float(),
                "rmsg.y": gn(core, z).float()})

    # --- partial rotary embedding ------------------------------------------------
    cfg = qcfg.tiny()
    hcfg = hf_config(cfg)
    rot = hf.Qwen3_5TextRotaryEmbedding(hcfg)
    pos = torch.tensor([[0, 1, 5, 37, 1000]])
    xq = r(1, pos.shape[1], cfg.head_dim)
    cos, sin = rot(xq, pos)
    qh, kh = r(1, 2, pos.shape[1], cfg.head_dim), r(1, 1, pos.shape[1], cfg.head_dim)
    qo, ko = hf.apply_rotary_pos_emb(qh, kh, cos, sin)
    out.update({"rope.pos": pos[0].float(), "rope.cos": cos[0], "rope.sin": sin[0],
                "rope.q": qh[0], "rope.q_out": qo[0], "rope.k": kh[0], "rope.k_out": ko[0]})

    # --- whole tiny model -----------------------------------------------------------
    w = synth.make_weights(cfg, seed=0)
    model = hf.Qwen3_5ForCausalLM(hcfg).float().eval()
    missing, unexpected = model.load_state_dict(hf_state_dict(w), strict=False)
    assert not unexpected, unexpected
    assert not [m for m in missing if "rotary" not in m], missing
    prompt = synth.make_prompt(cfg, n=8, seed=1)
    logits = model(input_ids=prompt.view(1, -1), use_cache=False).logits[0]
    out.update({"model.prompt": prompt.float(), "model.logits": logits.float()})

    meta = {"transformers": transformers.__version__, "torch": torch.__version__,
            "model_cfg": "qwen35_amd.config.tiny()", "weights": "synth.make_weights(cfg, seed=0)",
            "prompt": "synth.make_prompt(cfg, n=8, seed=1)"}
    save_file({k: v.contiguous() for k, v in out.items()}, OUT, metadata=meta)
    print(f"wrote {OUT}: {len(out)} tensors, transformers {transformers.__version__}")


if __name__ == "__main__":
    main()
