"""Config-5 parity read against its rounding noise floor.

TEST INFRASTRUCTURE ONLY (used by tests/test_gpu_fullsize.py and bench.py's
parity leg, never by the product path).

tests/golden/config5_noise_floor.json (written by tests/golden/make_noise_floor.py)
holds, for the full 4B-shaped model, the bench prompt and 300 rows (row 0 =
the prompt's last token, row j = decode step j), how far two other exact fp32
/ fp64 restatements of the reference's explicit-dequant path land from the
fp32 oracle: per-row logit cosine and argmax agreement.  A GPU run is
summarised the same way (GPU vs the fp32 oracle, teacher-forced on the
oracle's greedy tokens) and its figures are set beside the floor's, window by
window.
"""
import json
import os

FIXTURE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "tests", "golden",
                       "config5_noise_floor.json")
WINDOW = 50


def load(path=FIXTURE):
    with open(path) as f:
        return json.load(f)


def summarize(cos, agree, margin_ulps, window=WINDOW):
    """Per-row logit cosine, argmax agreement and the fp32 oracle's top-2
    margin in bf16 ulps -> the figures every run is compared by."""
    n = len(cos)
    dis = [(j, margin_ulps[j]) for j in range(n) if not agree[j]]
    first = next((j for j in range(n) if not agree[j]), None)
    decided = [j for j in range(n) if margin_ulps[j] > 1.0]
    return {
        "rows": n,
        "min_logit_cosine": min(cos),
        "mean_logit_cosine": sum(cos) / n,
        "window_min_logit_cosine": [min(cos[w:w + window]) for w in range(0, n, window)],
        "argmax_agree_where_margin_gt_1ulp": f"{sum(agree[j] for j in decided)}/{len(decided)}",
        "argmax_disagreements": len(dis),
        "largest_disagreeing_margin_ulps": max((m for _, m in dis), default=0.0),
        "disagreements_row_margin_ulps": dis,
        "free_running_identical_steps": n if first is None else first,
    }


def floor_summaries(fx, rows=None):
    """The fixture's variants summarised over their first `rows` rows."""
    out = {}
    m = fx["fp32_margin_ulps"]
    for name, v in fx["variants"].items():
        n = rows or len(v["logit_cosine_vs_fp32"])
        out[name] = summarize(v["logit_cosine_vs_fp32"][:n], v["argmax_agrees_with_fp32"][:n], m[:n])
    return out
