"""BASELINE config 5 at full size and full length (MI355X): the 32-layer
Qwen3.5-4B-shaped model, vocabulary 248,320, the bench's 128-token prompt
through the batch prefill, then 299 teacher-forced greedy decode steps against
the CPU oracle's explicit-dequant path (the reference harness's loop:
_benchmark_native_fp8.py:22-38; README.md:185).  300 logit rows in all, the
rows of tests/golden/config5_noise_floor.json.

The bars come from that fixture (tests/golden/make_noise_floor.py): on the same
model, prompt and teacher-forced tokens, the exact path (every intermediate in
fp64, bf16 only where the reference materialises bf16) sets how far the fp32
oracle itself lands from exact arithmetic, row by row.  The GPU is a second
fp32 evaluation of the same path with its own summation orders and
exponentials; if it is as accurate as the oracle and their rounding errors are
independent, its logit-cosine deficit against the oracle is twice the oracle's
deficit against the exact path (squared distances add).  So, per window of 50
rows:
  * 1 - min cosine(GPU, oracle) <= 2 * (1 - min cosine(oracle, exact));
and over all rows:
  * the argmax differs from the oracle's at rows whose top-2 margin exceeds 1
    bf16 ulp no more often than the K-block fp32 restatement's does (the
    reference kernels' summation order: a second fp32 implementation, two
    independent roundings like GPU vs oracle), n + 2 sqrt(n) for its count n
    (binomial spread);
  * every argmax difference sits at a top-2 margin no larger than sqrt(2) times
    the largest margin at which any fixture variant differs from the oracle.
(The fixture's figures: the oracle's deficit to the exact path 0.99891 at
worst, the GPU's to the oracle 0.87-1.11 times it per window when this test was
written; K-block 12 differences above 1 ulp, largest margin of any variant 4
ulps.)
Both sides read the RoPE tables the engine builds on the device (main.py:513-533
builds them on the device too).  Per-layer hidden-state cosines are compared
with the exact path's at rows 200..240, where the round-2 run's cosine fell.
"""
import math
import os

import pytest
import torch

from oracle import parity_floor
from oracle import qwen35_oracle as orc
from qwen35_amd import engine as eng_mod
from qwen35_amd.config import qwen35_4b
from qwen35_amd.synth import make_prompt, make_weights

from _util import cos_sim

pytestmark = pytest.mark.gpu

N_PROMPT = 128
FX = parity_floor.load()
N_ROWS = FX["rows"]
TRACE_ROWS = set(FX["trace_rows"])


def _ulp(x):
    return 2.0 ** (float(torch.floor(torch.log2(x.abs()))) - 7)


@pytest.fixture(scope="module")
def model(progress):
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    cfg = qwen35_4b()
    w = make_weights(cfg, seed=0, device="cuda")
    progress("\nconfig 5 weights drawn; building the oracle")
    max_seq = N_PROMPT + N_ROWS + 8
    eng = eng_mod.Qwen35FP8Engine(w, max_seq_len=max_seq)
    ref = orc.OracleModel(w.to("cpu"), max_seq_len=max_seq, prefill="reference")
    ref.cos, ref.sin = eng.rope_cos.cpu(), eng.rope_sin.cpu()
    progress("config 5 oracle built")
    prompt = make_prompt(cfg, n=N_PROMPT, seed=1)
    yield cfg, eng, ref, prompt
    del eng, ref


@pytest.mark.timeout(900)
def test_config5_full_length_within_noise_floor(model, progress):
    cfg, eng, ref, prompt = model
    g_tr, o_tr = [], []
    gl = eng.prefill_batch(prompt.cuda(), trace=g_tr).float().cpu().view(-1)
    rl = ref.prefill(prompt, trace=o_tr)[0].view(-1)
    progress("prefill per-layer cosine:", [round(cos_sim(a, b), 6) for a, b in zip(g_tr, o_tr)])
    rows = [(gl, rl)]
    toks, layer_cos = [], {}
    pos = N_PROMPT
    for j in range(1, N_ROWS):
        t = orc.argmax_first(rl)
        toks.append(t)
        if j in TRACE_ROWS:
            o_hs = []
            rl = ref.decode_token(t, pos, trace=o_hs)[0].view(-1)
            g_hs, gl = eng.decode_trace(t, pos)
            layer_cos[j] = [cos_sim(a, b) for a, b in zip(g_hs, o_hs)]
        else:
            rl = ref.decode_token(t, pos)[0].view(-1)
            gl = eng.forward(torch.tensor([[t]], device="cuda"), pos)
        rows.append((gl.float().cpu().view(-1), rl))
        pos += 1
        if j % 25 == 0:
            progress(f"row {j}/{N_ROWS - 1}: cosine {cos_sim(rows[-1][0], rl):.6f}")
    toks.append(orc.argmax_first(rl))
    cos, agree, margin = [], [], []
    for g, r in rows:
        top = torch.topk(r, 2)
        cos.append(cos_sim(g, r))
        agree.append(int(torch.argmax(g)) == int(top.indices[0]))
        margin.append(float(top.values[0] - top.values[1]) / _ulp(top.values[0]))
    gpu = parity_floor.summarize(cos, agree, margin)
    floor = parity_floor.floor_summaries(FX)
    exact = floor["exact"]
    print("GPU vs oracle:", {k: v for k, v in gpu.items() if k != "disagreements_row_margin_ulps"}, flush=True)
    print("GPU argmax differences (row, margin ulps):", [(j, round(m, 2)) for j, m in
                                                          gpu["disagreements_row_margin_ulps"]], flush=True)
    for name, f in floor.items():
        print(f"floor {name}:", {k: v for k, v in f.items() if k != "disagreements_row_margin_ulps"}, flush=True)
    same = toks == FX["fp32_greedy_tokens"]
    print(f"oracle tokens on this host equal the fixture's: {same}", flush=True)
    # where the deviation builds up: per layer, the largest deficit over rows
    # 200..240 of GPU vs oracle against twice that of oracle vs exact
    ex_layers = FX["variants"]["exact"]["layer_cosine_vs_fp32"]
    ratio = [max(1 - layer_cos[j][L] for j in layer_cos) /
             max(2 * max(1 - ex_layers[str(j)][L] for j in layer_cos), 1e-12)
             for L in range(cfg.num_hidden_layers)]
    print("per layer, max over rows 200..240 of (1 - cos GPU,oracle) / max of 2 (1 - cos oracle,exact):",
          [round(r, 2) for r in ratio], flush=True)

    # bars
    for w, (gc, ec) in enumerate(zip(gpu["window_min_logit_cosine"], exact["window_min_logit_cosine"])):
        assert 1 - gc <= 2 * (1 - ec), \
            f"rows {50 * w}..{50 * w + 49}: GPU min logit cosine {gc:.6f}, floor 1 - 2 (1 - {ec:.6f})"
    a_num, a_den = map(int, gpu["argmax_agree_where_margin_gt_1ulp"].split("/"))
    k_num, k_den = map(int, floor["kblock"]["argmax_agree_where_margin_gt_1ulp"].split("/"))
    n_k = k_den - k_num
    assert a_den - a_num <= n_k + 2 * math.sqrt(n_k), \
        f"argmax differs at {a_den - a_num} of {a_den} rows above 1 ulp; K-block floor {n_k} of {k_den}"
    m_floor = max(f["largest_disagreeing_margin_ulps"] for f in floor.values())
    big = [(j, m) for j, m in gpu["disagreements_row_margin_ulps"] if m > math.sqrt(2) * m_floor]
    assert not big, f"argmax differs at margins above sqrt(2) x {m_floor} ulps: {big}"
