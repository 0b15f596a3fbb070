"""Writes tests/golden/config5_noise_floor.json: the rounding noise floor of the
config-5 parity run (a CPU script for the build container, not a test; about
half an hour per variant on 8 cores:
`python tests/golden/make_noise_floor.py [rows] [variant ...]`, default all
three; variants already in the fixture are kept when only some are rerun).

Restatements of the reference's explicit-dequant decode path run on the same
full 4B-shaped model (seed-0 weights from the bench's CPU generator, the bench's
128-token prompt from seed 1, the reference's batch prefill, then greedy
decode) and differ from the fp32 oracle only in rounding (oracle/qwen35_oracle.py
MATMUL, ACC):
  fp32    one fp32 matmul: the oracle every GPU test compares with; its greedy
          tokens are the teacher-forced sequence of every run here and of the
          GPU's config-5 test (_benchmark_native_fp8.py:22-38 is the loop);
  kblock  fp32 partials per 128-wide K block added block by block, the order
          of the reference's own kernels (fused_kernels.cu:127-145): a second
          fp32 implementation;
  fp64    fp64 accumulation of the same operands;
  exact   every intermediate in fp64 (oracle ACC = float64, MATMUL = fp64),
          rounded to bf16 only where the reference materialises a bf16
          tensor, the recurrent state and KV cache in fp64: the path both
          fp32 implementations (the oracle, the GPU) approximate.
Per position (row 0 = the prompt's last token, row j = decode step j) the
fixture holds the fp32 oracle's greedy token and top-2 margin in bf16 ulps of
its top logit, and for each variant the logit cosine against fp32 and
whether its argmax agrees; per variant the number of greedy steps a
free-running run would share with the fp32 one (the first disagreement).  At
rows 200..240 it also holds the cosine of the hidden state after every layer
against the fp32 run.  The GPU's config-5 test reads its bars from here.
"""
import json
import os
import platform
import subprocess
import sys
import time

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import __graft_entry__  # noqa: E402

__graft_entry__.load_package()
from oracle import qwen35_oracle as orc  # noqa: E402
from qwen35_amd import config, synth  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "config5_noise_floor.json")
N_PROMPT = 128
TRACE_ROWS = range(200, 241)


def log(msg):
    print(f"noise floor: {msg}", file=sys.stderr, flush=True)


def bf16_ulp(x):
    return 2.0 ** (float(torch.floor(torch.log2(x.abs()))) - 7)


def cos(a, b):
    a, b = a.double().reshape(-1), b.double().reshape(-1)
    return float((a @ b) / (a.norm() * b.norm()))


def run(ref, prompt, n_rows, toks=None):
    """Logit rows 0..n_rows-1: the prompt (batch prefill), then decode steps fed
    `toks` (teacher forcing) or, when toks is None, the run's own greedy tokens.
    Returns (logits per row, tokens fed, hidden-state traces at TRACE_ROWS)."""
    logits = [ref.forward(prompt, 0).view(-1).clone()]
    fed, traces = [], {}
    pos = N_PROMPT
    t0 = time.time()
    for j in range(1, n_rows):
        tk = orc.argmax_first(logits[-1]) if toks is None else toks[j - 1]
        fed.append(tk)
        tr = [] if j in TRACE_ROWS else None
        logits.append(ref.decode_token(tk, pos, trace=tr)[0].view(-1).clone())
        if tr is not None:
            traces[j] = tr
        pos += 1
        if j % 25 == 0:
            log(f"{orc.MATMUL}: row {j}/{n_rows - 1} ({(time.time() - t0) / j:.2f} s per step)")
    return logits, fed, traces


def host():
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = {k.strip(): v.strip() for k, v in (ln.split(":", 1) for ln in out.splitlines() if ":" in ln)}
        return kv.get("Model name")
    except (OSError, ValueError):
        return platform.processor()


def main(n_rows, modes):
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    cfg = config.qwen35_4b()
    t0 = time.time()
    w = synth.make_weights(cfg, seed=0, device="cpu")
    prompt = synth.make_prompt(cfg, n=N_PROMPT, seed=1)
    ref = orc.OracleModel(w, max_seq_len=N_PROMPT + n_rows + 1, prefill="reference")
    log(f"model ready ({time.time() - t0:.0f} s)")
    orc.MATMUL = "fp32"
    l32, toks, tr32 = run(ref, prompt, n_rows)
    greedy = toks + [orc.argmax_first(l32[-1])]
    margins = []
    for r in l32:
        top = torch.topk(r, 2).values
        margins.append(round(float(top[0] - top[1]) / bf16_ulp(top[0]), 3))
    out = {
        "generator": "tests/golden/make_noise_floor.py",
        "model": "qwen35_4b, synth.make_weights(seed=0, device='cpu'), prompt synth.make_prompt(n=128, seed=1)",
        "host": {"cpu": host(), "threads": torch.get_num_threads(), "torch": torch.__version__},
        "rows": n_rows,
        "row_meaning": "row 0 = logits of the prompt's last token (batch prefill); row j = decode step j, "
                       "fed the fp32 oracle's greedy token of row j-1",
        "fp32_greedy_tokens": greedy,
        "fp32_margin_ulps": margins,
        "trace_rows": list(TRACE_ROWS),
        "variants": {},
    }
    if os.path.exists(OUT):
        with open(OUT) as f:
            old = json.load(f)
        if old.get("fp32_greedy_tokens") == greedy and old.get("rows") == n_rows:
            out["variants"] = {k: v for k, v in old["variants"].items() if k not in modes}
    for mode in modes:
        orc.MATMUL = "fp64" if mode == "exact" else mode
        orc.ACC = torch.float64 if mode == "exact" else torch.float32
        try:
            lv, _, trv = run(ref, prompt, n_rows, toks=toks)
        finally:
            orc.MATMUL, orc.ACC = "fp32", torch.float32
        cs = [round(cos(a, b), 7) for a, b in zip(lv, l32)]
        agree = [int(torch.argmax(a)) == greedy[j] for j, a in enumerate(lv)]
        first = next((j for j, ok in enumerate(agree) if not ok), None)
        out["variants"][mode] = {
            "logit_cosine_vs_fp32": cs,
            "argmax_agrees_with_fp32": agree,
            "free_running_identical_steps": n_rows if first is None else first,
            "disagreements": [{"row": j, "fp32_margin_ulps": margins[j]}
                              for j, ok in enumerate(agree) if not ok],
            "min_logit_cosine": min(cs),
            "mean_logit_cosine": round(sum(cs) / len(cs), 7),
            "layer_cosine_vs_fp32": {str(j): [round(cos(a, b), 7) for a, b in zip(trv[j], tr32[j])]
                                     for j in TRACE_ROWS if j in trv},
        }
        with open(OUT, "w") as f:
            json.dump(out, f, separators=(",", ":"))
        log(f"{mode}: min cosine {min(cs):.6f}, free-running identical {out['variants'][mode]['free_running_identical_steps']}, "
            f"disagreements {out['variants'][mode]['disagreements']}")
    log(f"wrote {OUT} ({time.time() - t0:.0f} s)")


if __name__ == "__main__":
    main(int(sys.argv[1]) if len(sys.argv) > 1 else 300,
         sys.argv[2:] or ["kblock", "fp64", "exact"])
