"""Native block-FP8 checkpoint loader (main.py:326-353, 575-700 layout) on
synthetic checkpoints written in the released format (CPU only)."""
import json
import os

import pytest
import torch

from qwen35_amd import loader
from qwen35_amd.config import tiny
from qwen35_amd.synth import make_weights


def _same(a, b):
    if isinstance(a, tuple):
        return all(_same(x, y) for x, y in zip(a, b))
    if not isinstance(a, torch.Tensor):
        return a == b
    return a.dtype == b.dtype and a.shape == b.shape and torch.equal(a, b)


@pytest.mark.parametrize("prefix,tied", [("model.language_model.", False), ("model.", True)])
def test_round_trip_fp32_scales(tmp_path, prefix, tied):
    cfg = tiny(num_layers=4)
    w = make_weights(cfg, seed=5)
    if tied:
        w.lm_head = w.embed
    loader.save_checkpoint(w, str(tmp_path), prefix=prefix, tied=tied)
    got = loader.load_checkpoint(str(tmp_path), device="cpu", scale_dtype=torch.float32)
    assert got.cfg.to_dict() == cfg.to_dict()
    assert _same(got.embed, w.embed) and _same(got.lm_head, w.lm_head)
    assert _same(got.norm_f, w.norm_f)
    for a, b in zip(got.layers, w.layers):
        assert set(a) == set(b)
        for k in a:
            assert _same(a[k], b[k]), k


def test_reference_scale_rounding(tmp_path):
    """By default the scales are bf16, as the reference converts them (main.py:597)."""
    cfg = tiny(num_layers=4)
    w = make_weights(cfg, seed=6)
    loader.save_checkpoint(w, str(tmp_path))
    got = loader.load_checkpoint(str(tmp_path), device="cpu")
    ws, ss = got.layers[0]["gate_proj"]
    assert ss.dtype == torch.bfloat16
    assert torch.equal(ss, w.layers[0]["gate_proj"][1].to(torch.bfloat16))
    assert torch.equal(ws, w.layers[0]["gate_proj"][0])


def test_rejects_non_fp8_and_bf16_linears(tmp_path):
    cfg = tiny(num_layers=4)
    w = make_weights(cfg, seed=7)
    loader.save_checkpoint(w, str(tmp_path))
    p = os.path.join(str(tmp_path), "config.json")
    d = json.load(open(p))
    d["quantization_config"]["weight_block_size"] = [64, 64]
    json.dump(d, open(p, "w"))
    with pytest.raises(loader.CheckpointError, match="128x128"):
        loader.load_checkpoint(str(tmp_path), device="cpu")
    # a bf16 linear is refused unless quantize_bf16
    d["quantization_config"]["weight_block_size"] = [128, 128]
    json.dump(d, open(p, "w"))
    from safetensors.torch import load_file, save_file
    f = os.path.join(str(tmp_path), "model.safetensors")
    t = load_file(f)
    k = "model.language_model.layers.0.linear_attn.in_proj_a.weight"
    from oracle import qwen35_oracle as orc
    wq, sq = w.layers[0]["in_proj_a"]
    t[k] = orc.dequant(wq, sq).to(torch.bfloat16)
    del t[k.replace(".weight", ".weight_scale_inv")]
    save_file(t, f)
    with pytest.raises(loader.CheckpointError, match="in_proj_a"):
        loader.load_checkpoint(str(tmp_path), device="cpu")
    got = loader.load_checkpoint(str(tmp_path), device="cpu", quantize_bf16=True)
    wa, sa = got.layers[0]["in_proj_a"]
    assert wa.dtype == torch.uint8 and sa.shape == sq.shape
