"""Oracle pins for nucleus sampling (top_p_sample, main.py:49-87): closed
forms for the scaling, the penalty, the forced first token, ties and the
full-softmax fallback."""
import torch

from oracle import qwen35_oracle as orc


def _bf(x):
    return x.to(torch.bfloat16)


def test_scale_temperature_and_penalty_closed_form():
    x = _bf(torch.tensor([3.0, -2.0, 0.5, -0.25, 1.0]))
    # T = 0.5: a power-of-two reciprocal, so y = 2x exactly
    assert torch.equal(orc.sample_scale(x, 0.5), x.float() * 2)
    # T <= 0: no scaling (main.py:54)
    assert torch.equal(orc.sample_scale(x, 0.0), x.float())
    # penalty 2: negative values double, positive halve, each distinct id once
    y = orc.sample_scale(x, 1.0, rep_penalty=2.0, recent_ids=[0, 1, 1, 0, 3])
    assert torch.equal(y, torch.tensor([1.5, -4.0, 0.5, -0.5, 1.0]))
    # rep_penalty <= 1 or no window: unchanged
    assert torch.equal(orc.sample_scale(x, 1.0, rep_penalty=1.0, recent_ids=[0]), x.float())


def test_dominant_token_is_forced():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5000, generator=g)
    x[1234] = 30.0
    ids, probs, fb = orc.sample_nucleus(_bf(x), temperature=1.0, top_p=0.9)
    # its probability rounds to 1 > bf16(0.9): nothing passes, the first is kept
    assert ids.tolist() == [1234] and not fb


def test_ties_keep_lowest_indices():
    x = torch.full((3000,), -20.0)
    x[[7, 70, 700]] = 10.0
    ids, probs, fb = orc.sample_nucleus(_bf(x), temperature=1.0, top_p=0.9)
    # three near-equal thirds: running mass ~1/3, ~2/3 <= 0.898, then ~1 > 0.898
    assert ids.tolist() == [7, 70] and not fb
    # the log-partition is rounded to bf16 first (main.py:70-71):
    # bf16(10 + ln 3) = 11.125, so p = bf16(exp(10 - 11.125)) -- not 1/3
    assert torch.equal(probs, _bf(torch.exp(torch.tensor([-1.125, -1.125]))).float())


def test_flat_logits_fall_back_to_the_full_softmax():
    V = 4096
    ids, probs, fb = orc.sample_nucleus(_bf(torch.zeros(V)), temperature=0.7, top_p=0.9)
    # top-2000 mass is 2000/4096 < 0.9 -> full softmax, p = 2^-12 exactly; the
    # running mass k/4096 rounds to bf16 <= 0.8984375 up to k = 3688 (the tie at
    # 0.900390625 rounds to the even 0.8984375)
    assert fb
    assert len(ids) == 3688 and ids.tolist() == list(range(3688))
    assert torch.equal(probs, torch.full((3688,), 2.0 ** -12))


def test_penalty_moves_the_cut():
    x = torch.full((100,), -30.0)
    x[3], x[4] = 5.0, 4.0
    ids, _, _ = orc.sample_nucleus(_bf(x), temperature=1.0, top_p=0.9)
    assert ids.tolist() == [3]  # e / (1 + e) = 0.73 <= 0.898, then 1.0
    ids, _, _ = orc.sample_nucleus(_bf(x), temperature=1.0, top_p=0.9, rep_penalty=2.0,
                                   recent_ids=[3])
    assert ids.tolist() == [4]  # 3 -> 2.5 now ranks below 4
