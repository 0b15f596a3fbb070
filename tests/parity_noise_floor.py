"""Noise floor of the config-5 parity (a CPU script, not a test: run it by
hand, `python tests/parity_noise_floor.py [steps]`, ~10 minutes on 8 cores).

Two exact restatements of the reference's explicit-dequant path on the full
4B-shaped model (seed 0 weights, the bench's 128-token prompt): the oracle
with fp32 matmuls (what the GPU is compared with) and the same oracle with
fp64-accumulated matmuls, teacher-forced on the fp32 oracle's greedy tokens.
Their logit cosine and argmax agreement (at positions whose top-2 margin
exceeds one bf16 ulp) are the level at which two correct implementations of
this random-init model differ; the GPU-vs-oracle parity leg of bench.py is
read against it.  Prints one JSON line.
"""
import json
import os
import sys
import time

import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import __graft_entry__  # noqa: E402

__graft_entry__.load_package()
from oracle import qwen35_oracle as orc  # noqa: E402
from qwen35_amd import config, synth  # noqa: E402


def linear_fp64(x, W):
    """orc.linear with fp64 accumulation (bf16 output, as the reference)."""
    return orc.bf16((x.double() @ W.double().t()).float())


def run(ref, prompt, toks):
    """Logits of the prompt and of each teacher-forced token."""
    out = [ref.forward(prompt, 0).view(-1).clone()]
    pos = len(prompt)
    for tk in toks:
        out.append(ref.decode_token(tk, pos)[0].view(-1).clone())
        pos += 1
    return out


def main(n_steps):
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    t0 = time.time()
    cfg = config.qwen35_4b()
    w = synth.make_weights(cfg, seed=0, device="cpu")
    prompt = synth.make_prompt(cfg, n=128, seed=1)
    ref = orc.OracleModel(w, max_seq_len=128 + n_steps + 1, prefill="reference")
    print(f"model ready ({time.time() - t0:.0f} s)", file=sys.stderr, flush=True)
    # fp32 oracle, free-running greedy: the token sequence both runs are fed
    logits = ref.forward(prompt, 0).view(-1)
    toks, l32 = [], [logits.clone()]
    pos = 128
    for k in range(n_steps):
        tk = orc.argmax_first(logits)
        toks.append(tk)
        if k == n_steps - 1:
            break
        logits = ref.decode_token(tk, pos)[0].view(-1)
        l32.append(logits.clone())
        pos += 1
    lin32, orc.linear = orc.linear, linear_fp64
    try:
        l64 = run(ref, prompt, toks[:-1])
    finally:
        orc.linear = lin32
    rows = []
    for a, b in zip(l32, l64):
        top = torch.topk(b, 2)
        margin = float(top.values[0] - top.values[1])
        ulp = 2.0 ** (float(torch.floor(torch.log2(top.values[0].abs()))) - 7)
        rows.append({"cos": float(torch.nn.functional.cosine_similarity(a.double(), b.double(), dim=0)),
                     "agree": int(torch.argmax(a)) == int(top.indices[0]), "margin": margin,
                     "decided": margin > ulp, "top": float(top.values[0])})
    dec = [r for r in rows if r["decided"]]
    print(json.dumps({
        "positions": len(rows), "min_cos": min(r["cos"] for r in rows),
        "mean_cos": sum(r["cos"] for r in rows) / len(rows),
        "agree_margin_gt_1ulp": f"{sum(r['agree'] for r in dec)}/{len(dec)}",
        "agree_all": f"{sum(r['agree'] for r in rows)}/{len(rows)}",
        "disagreements_position_margin_top": [(i, r["margin"], r["top"])
                                              for i, r in enumerate(rows) if not r["agree"]]}))


if __name__ == "__main__":
    main(int(sys.argv[1]) if len(sys.argv) > 1 else 40)
