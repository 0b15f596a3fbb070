"""The CPU oracle against golden vectors produced by transformers' own Qwen3.5
functions (tests/golden/make_golden.py, transformers 5.15.0; the version is
recorded in the fixture's metadata).  Pins the oracle's restatements of the
third-party pieces the reference imports (conv update, gated delta rule,
main.py:21-26) and, with a whole tiny model, its layer wiring: residuals,
(1+w) norms, the per-head [q | gate] split, GQA mapping, partial RoPE, conv
channel order, head repeat, A_log/dt_bias gates, gated RMSNorm."""
import math
import os

import pytest
import torch
from safetensors import safe_open

from oracle import qwen35_oracle as orc
from qwen35_amd import config as qcfg, synth

from _util import cos_sim

FIX = os.path.join(os.path.dirname(__file__), "golden", "qwen35_hf_golden.safetensors")


@pytest.fixture(scope="module")
def gold():
    with safe_open(FIX, framework="pt") as f:
        assert f.metadata()["transformers"] == "5.15.0"
        return {k: f.get_tensor(k) for k in f.keys()}


def _l2(x):
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + 1e-6)


def test_gated_delta_rule_chunked_and_recurrent(gold):
    q, k, v, g, beta = (gold[f"gdr.{n}"] for n in ("q", "k", "v", "g", "beta"))
    qn = _l2(q) / math.sqrt(q.shape[-1])
    kn = _l2(k)
    o, S = orc.chunk_gated_delta_rule(qn, kn, v, g, beta, chunk=64)
    torch.testing.assert_close(o, gold["gdr.chunk_out"], rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(S, gold["gdr.chunk_state"], rtol=1e-4, atol=1e-4)
    S2 = torch.zeros_like(S)
    o2 = orc.gated_delta_rule_seq(qn, kn, v, g, beta, S2)
    torch.testing.assert_close(o2, gold["gdr.rec_out"], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(S2, gold["gdr.rec_state"], rtol=1e-5, atol=1e-5)


def test_conv_update(gold):
    state = gold["conv.state"].clone()
    y = orc.conv_update(gold["conv.x"], state, gold["conv.w"])
    # the reference rounds the conv sum and the SiLU to bf16 (main.py:1097 on
    # bf16 tensors); transformers' fp32 path rounds nothing
    torch.testing.assert_close(y, gold["conv.y"], rtol=1e-2, atol=1e-3)
    assert torch.equal(state, gold["conv.state_out"])


def test_l2norm_on_bf16(gold):
    """Within one bf16 ulp: the fixture comes from torch's CPU kernels, whose
    bf16 rsqrt rounds twice (bf16(1 / bf16(sqrt(x)))); the reference runs the
    same op on CUDA, which rounds the fp32 rsqrt once -- the oracle follows
    the reference."""
    got, ref = orc.l2norm_bf16(gold["l2.x"]), gold["l2.y"]
    torch.testing.assert_close(got, ref, rtol=2.0 ** -7, atol=0)


def test_rmsnorm_one_plus_w(gold):
    y = orc.rmsnorm(gold["rms.x"], gold["rms.w"])
    torch.testing.assert_close(y, gold["rms.y"], rtol=0, atol=0)


def test_gated_rmsnorm(gold):
    y = orc.gated_rmsnorm(gold["rmsg.core"], gold["rmsg.z"], gold["rmsg.w"], bf16_steps=True)
    # same formula; the reference rounds silu(z) to bf16 before the product
    torch.testing.assert_close(y, gold["rmsg.y"], rtol=1e-2, atol=1e-3)


def test_partial_rope(gold):
    cfg = qcfg.tiny()
    rot = cfg.rotary_dim
    pos = gold["rope.pos"].long()
    cos, sin = orc.rope_tables(int(pos.max()) + 1, rot, cfg.rope_theta)
    # same fp32 construction as transformers (and main.py:527-533)
    torch.testing.assert_close(cos[pos], gold["rope.cos"][:, :rot], rtol=0, atol=1e-7)
    torch.testing.assert_close(sin[pos], gold["rope.sin"][:, :rot], rtol=0, atol=1e-7)
    for name in ("q", "k"):
        x = gold[f"rope.{name}"]
        y = orc.rope_rows(x, cos[pos], sin[pos], rot, round_out=False)
        torch.testing.assert_close(y, gold[f"rope.{name}_out"], rtol=1e-5, atol=1e-5)


def test_tiny_model_logits_match_transformers(gold):
    """The oracle (explicit bf16 rounding points of the reference engine) vs
    transformers' fp32 model on the same dequantized weights: every position
    of an 8-token prompt, decoded one token at a time."""
    cfg = qcfg.tiny()
    w = synth.make_weights(cfg, seed=0)
    prompt = synth.make_prompt(cfg, n=8, seed=1)
    assert torch.equal(prompt.float(), gold["model.prompt"])
    ref = gold["model.logits"]
    m = orc.OracleModel(w, max_seq_len=32, prefill="sequential")
    for t in range(len(prompt)):
        logits, _ = m.decode_token(int(prompt[t]), t)
        c = cos_sim(logits.view(-1), ref[t])
        assert c > 0.999, f"position {t}: cosine {c:.6f}"
        top = torch.topk(ref[t], 2).values
        if float(top[0] - top[1]) > 0.05:
            assert int(torch.argmax(logits)) == int(torch.argmax(ref[t])), f"position {t}"
    # and the batch prefill path on the whole prompt
    mp = orc.OracleModel(w, max_seq_len=32, prefill="reference")
    last = mp.forward(prompt.view(1, -1), 0).view(-1)
    assert cos_sim(last, ref[-1]) > 0.999
