"""BASELINE config 5 at full size (MI355X): the 32-layer Qwen3.5-4B-shaped
model, vocabulary 248,320, a 128-token prompt through the batch prefill, then
teacher-forced greedy decode against the CPU oracle's explicit-dequant path
(the reference harness: _benchmark_native_fp8.py:22-38; README.md:185)."""
import os

import pytest
import torch

from oracle import qwen35_oracle as orc
from qwen35_amd import engine as eng_mod
from qwen35_amd.config import qwen35_4b
from qwen35_amd.synth import make_prompt, make_weights

from _util import cos_sim

pytestmark = pytest.mark.gpu

N_PROMPT, N_STEPS = 128, 32


def _ulp(x):
    return 2.0 ** (float(torch.floor(torch.log2(x.abs()))) - 7)


@pytest.fixture(scope="module")
def model():
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    cfg = qwen35_4b()
    w = make_weights(cfg, seed=0, device="cuda")
    print("config 5 weights drawn; building the oracle", flush=True)
    eng = eng_mod.Qwen35FP8Engine(w, max_seq_len=N_PROMPT + N_STEPS + 8)
    ref = orc.OracleModel(w.to("cpu"), max_seq_len=N_PROMPT + N_STEPS + 8, prefill="reference")
    prompt = make_prompt(cfg, n=N_PROMPT, seed=1)
    yield cfg, eng, ref, prompt
    del eng, ref


@pytest.mark.timeout(900)
def test_config5_layer_trace_and_teacher_forced_tokens(model):
    """Per-layer hidden-state cosine (GPU vs oracle) of the prompt's last token
    and of the first decode step, then N_STEPS teacher-forced decode steps.

    The bar is the model's own rounding noise: two exact restatements of the
    reference (the oracle with fp32 vs fp64-accumulated matmuls,
    tests/parity_noise_floor.py) reach mean logit cosine 0.99943 and disagree
    on the argmax at 2 of 54 positions whose top-2 margin exceeds one bf16
    ulp, always at margins of at most 2 ulps.  So: the argmax agrees wherever
    the oracle's margin exceeds 4 bf16 ulps, at >= 90 % of the positions
    above 1 ulp, and the logit cosine stays above 0.999."""
    cfg, eng, ref, prompt = model
    g_tr, o_tr = [], []
    gl = eng.prefill_batch(prompt.cuda(), trace=g_tr).float().cpu().view(-1)
    rl = ref.prefill(prompt, trace=o_tr)[0].view(-1)
    prefill_cos = [round(cos_sim(a, b), 6) for a, b in zip(g_tr, o_tr)]
    print("prefill per-layer cosine:", prefill_cos, flush=True)
    assert cos_sim(gl, rl) > 0.999, f"prompt logits; layers {prefill_cos}"

    t = orc.argmax_first(rl)
    g_hs, g1 = eng.decode_trace(t, N_PROMPT)
    o_hs = []
    r1, _ = ref.decode_token(t, N_PROMPT, trace=o_hs)
    decode_cos = [round(cos_sim(a, b), 6) for a, b in zip(g_hs, o_hs)]
    print("decode per-layer cosine:", decode_cos, flush=True)
    assert min(decode_cos) > 0.999, f"decode layers {decode_cos}"

    rows = [(g1.view(-1), r1.view(-1))]
    pos = N_PROMPT + 1
    rl = r1.view(-1)
    for k in range(N_STEPS - 1):
        t = orc.argmax_first(rl)
        rl = ref.decode_token(t, pos)[0].view(-1)
        gl = eng.forward(torch.tensor([[t]], device="cuda"), pos).float().cpu().view(-1)
        rows.append((gl, rl))
        pos += 1
        print(f"teacher-forced step {k + 2}/{N_STEPS}: cosine {cos_sim(gl, rl):.6f}", flush=True)
    cos, decided, agree, missed = [], 0, 0, []
    for i, (g, r) in enumerate(rows):
        cos.append(cos_sim(g, r))
        top = torch.topk(r, 2)
        margin = float(top.values[0] - top.values[1])
        ulp = _ulp(top.values[0])
        ok = int(torch.argmax(g)) == int(top.indices[0])
        if margin > ulp:
            decided += 1
            agree += ok
        if not ok:
            missed.append((i, round(margin / ulp, 2)))
    print(f"teacher-forced: min cosine {min(cos):.6f}, argmax {agree}/{decided} above 1 ulp, "
          f"differences at (step, margin in ulps) {missed}", flush=True)
    assert all(m <= 4.0 for _, m in missed), f"argmax differs above 4 ulps: {missed}"
    assert agree >= 0.9 * decided, f"argmax agreement {agree}/{decided}"
    assert min(cos) > 0.999, f"logit cosines {[round(c, 5) for c in cos]}"
