"""The config-5 noise-floor fixture and the code that reads it (CPU)."""
import math

import torch

from oracle import parity_floor
from oracle import qwen35_oracle as orc
from qwen35_amd import config, synth


def test_summarize_closed_form():
    cos = [0.9995] * 120
    cos[7], cos[61] = 0.998, 0.9991
    agree = [True] * 120
    agree[3] = agree[90] = False
    margin = [5.0] * 120
    margin[3], margin[90], margin[10] = 2.0, 0.5, 1.0
    s = parity_floor.summarize(cos, agree, margin, window=50)
    assert s["rows"] == 120 and s["min_logit_cosine"] == 0.998
    assert s["window_min_logit_cosine"] == [0.998, 0.9991, 0.9995]
    assert s["free_running_identical_steps"] == 3
    assert s["disagreements_row_margin_ulps"] == [(3, 2.0), (90, 0.5)]
    assert s["largest_disagreeing_margin_ulps"] == 2.0
    # rows above 1 ulp: all but 90 (0.5) and 10 (exactly 1); row 3 disagrees
    assert s["argmax_agree_where_margin_gt_1ulp"] == "117/118"
    assert math.isclose(s["mean_logit_cosine"], (0.9995 * 118 + 0.998 + 0.9991) / 120)


def test_fixture_is_whole_and_consistent():
    fx = parity_floor.load()
    n = fx["rows"]
    assert n == 300 and fx["generator"] == "tests/golden/make_noise_floor.py"
    assert len(fx["fp32_greedy_tokens"]) == n and len(fx["fp32_margin_ulps"]) == n
    assert all(0 <= t < 248320 for t in fx["fp32_greedy_tokens"])
    assert all(m >= 0 for m in fx["fp32_margin_ulps"])
    assert set(fx["variants"]) == {"kblock", "fp64", "exact"}
    for name, v in fx["variants"].items():
        cs, ag = v["logit_cosine_vs_fp32"], v["argmax_agrees_with_fp32"]
        assert len(cs) == n and len(ag) == n, name
        assert v["min_logit_cosine"] == min(cs)
        first = next((j for j, ok in enumerate(ag) if not ok), n)
        assert v["free_running_identical_steps"] == first
        assert [d["row"] for d in v["disagreements"]] == [j for j, ok in enumerate(ag) if not ok]
        assert sorted(int(r) for r in v["layer_cosine_vs_fp32"]) == fx["trace_rows"]
        # every variant is a restatement of the same path: close, but not equal
        assert 0.998 < min(cs) < 1.0
    s = parity_floor.floor_summaries(fx)
    assert s["exact"]["rows"] == n and len(s["exact"]["window_min_logit_cosine"]) == 6


def test_oracle_rounding_modes_on_a_tiny_model():
    """fp32 (default), K-block and fp64 products and the exact (all fp64) path
    give logits within fp32 noise of one another; the exact path keeps its
    state in fp64; the modes are restored afterwards."""
    cfg = config.tiny(num_layers=4)
    w = synth.make_weights(cfg, seed=3)
    prompt = synth.make_prompt(cfg, n=7, seed=4)
    out = {}
    for mode, acc in [("fp32", torch.float32), ("kblock", torch.float32), ("fp64", torch.float32),
                      ("fp64", torch.float64)]:
        orc.MATMUL, orc.ACC = mode, acc
        try:
            ref = orc.OracleModel(w, max_seq_len=16)
            l0 = ref.forward(prompt, 0).view(-1)
            l1 = ref.decode_token(int(l0.argmax()), 7)[0].view(-1)
            states = [s for s in ref.rec_state if s is not None]
            assert states and all(s.dtype == acc for s in states)
        finally:
            orc.MATMUL, orc.ACC = "fp32", torch.float32
        out[(mode, acc)] = torch.cat([l0, l1]).double()
    base = out[("fp32", torch.float32)]
    for key, v in out.items():
        c = float(torch.nn.functional.cosine_similarity(v, base, dim=0))
        assert c > 0.9999, (key, c)
    assert not torch.equal(out[("fp64", torch.float64)], base)
    # x @ W^T in the three product modes, against a float64 product
    x, W = torch.randn(3, 384), torch.randn(50, 384)
    exact = x.double() @ W.double().t()
    for mode in ("fp32", "kblock", "fp64"):
        orc.MATMUL = mode
        try:
            y = orc.wmm(x, W)
        finally:
            orc.MATMUL = "fp32"
        assert y.dtype == torch.float32
        assert (y.double() - exact).abs().max() < 1e-4
