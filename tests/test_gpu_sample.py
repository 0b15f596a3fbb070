"""On-device nucleus sampling (qh_sample_top_p, top_p_sample main.py:49-87)
against the CPU oracle's kept set, plus the draw's distribution (MI355X only)."""
import math
import struct

import pytest
import torch

from oracle import qwen35_oracle as orc
from qwen35_amd import abi
from qwen35_amd import engine as eng_mod
from qwen35_amd.config import tiny
from qwen35_amd.synth import make_prompt, make_weights

from _util import gen

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _f32(bits):
    return struct.unpack("<f", struct.pack("<I", int(bits) & 0xFFFFFFFF))[0]


class Sampler:
    def __init__(self, V, window_hist=None):
        self.lib = abi.load()
        self.V = V
        self.ws = torch.zeros(int(self.lib.qh_sample_workspace_size(V)), dtype=torch.uint8, device=DEV)
        self.ctr = torch.zeros(1, dtype=torch.int64, device=DEV)
        self.tok = torch.zeros(1, dtype=torch.int64, device=DEV)
        self.info = torch.zeros(16, dtype=torch.int64, device=DEV)
        self.hist = window_hist

    def __call__(self, logits, T, top_p, rp=1.0, slot=0, window=0, seed=7):
        hist = self.hist
        rc = self.lib.qh_sample_top_p(
            abi.ptr(logits), self.V, T, top_p, rp, abi.ptr(hist) if hist is not None else None,
            hist.numel() if hist is not None else 0, None, slot, 0, None, window, seed,
            abi.ptr(self.ctr), abi.ptr(self.ws), abi.ptr(self.tok), None, None, 0,
            abi.ptr(self.info), abi.stream_handle())
        abi.check(rc, "sample")
        torch.cuda.synchronize()
        info = self.info.cpu().tolist()
        return int(self.tok.item()), info


def _check_cut(s, x_cpu, T, top_p, rp=1.0, recent=None, slot=0, window=0):
    """One call: the device's kept count, fallback flag and log-partition agree
    with the oracle; the drawn token is in the kept set."""
    tok, info = s(x_cpu.to(DEV), T, top_p, rp, slot=slot, window=window)
    M, Z, logz_b = _f32(info[9]), _f32(info[10]), _f32(info[11])
    ref_logz = orc.bf16(torch.logsumexp(orc.sample_scale(x_cpu, T, rp, recent), 0)).item()
    assert abs(logz_b - ref_logz) <= 2 ** -7 * max(1.0, abs(ref_logz)), (logz_b, ref_logz)
    # the cut itself, given the device's fp32 sums (a summation order may move a
    # bf16 rounding of the log-partition)
    ids, probs, fb = orc.sample_nucleus(x_cpu, T, top_p, rp, recent, logz_b=logz_b, soft_mz=(M, Z))
    assert bool(info[3]) == fb, "fallback decision"
    assert info[2] == len(ids), f"kept {info[2]} vs oracle {len(ids)}"
    assert tok in set(ids.tolist())
    return ids, probs, tok, info


def test_peaked_and_forced():
    g = gen(61)
    V = 248320
    s = Sampler(V)
    x = torch.randn(V, generator=g)
    x[4321] = 40.0
    ids, _, tok, info = _check_cut(s, x.bfloat16(), 1.0, 0.9)
    assert ids.tolist() == [4321] and tok == 4321


def test_ties_and_lowest_index_order():
    V = 3000
    s = Sampler(V)
    x = torch.full((V,), -20.0)
    x[[700, 7, 70]] = 10.0
    ids, _, tok, _ = _check_cut(s, x.bfloat16(), 1.0, 0.9)
    assert ids.tolist() == [7, 70]


def test_flat_fallback_full_vocabulary():
    for V in (4096, 248320):
        s = Sampler(V)
        ids, _, _, info = _check_cut(s, torch.zeros(V).bfloat16(), 0.7, 0.9)
        assert info[3] == 1  # full-softmax fallback


@pytest.mark.parametrize("T,top_p,scale", [(0.7, 0.9, 4.0), (1.0, 0.5, 3.0), (0.3, 0.95, 1.0),
                                           (0.0, 0.9, 6.0)])
def test_random_logits_vocab_sized(T, top_p, scale):
    g = gen(62)
    V = 248320
    s = Sampler(V)
    x = (torch.randn(V, generator=g) * scale).bfloat16()
    for _ in range(3):
        _check_cut(s, x, T, top_p)


def test_repetition_penalty_window():
    g = gen(63)
    V = 50000
    x = torch.randn(V, generator=g) * 2
    top = torch.topk(x, 6).indices.tolist()
    hist = torch.zeros(64, dtype=torch.int64)
    recent = [top[0], top[1], top[0], 17, 23]  # a duplicate: penalised once
    hist[10:15] = torch.tensor(recent)
    s = Sampler(V, window_hist=hist.to(DEV))
    # window hist[max(0, 15 - 5) .. 15)
    ids, _, _, info = _check_cut(s, x.bfloat16(), 0.7, 0.9, rp=1.3, recent=recent, slot=15, window=5)
    assert info[14] == 5
    assert int(s.hist[15].item()) == int(s.tok.item())  # the history slot is written


def test_draw_distribution():
    """Many draws over a small nucleus: frequencies match the renormalised kept
    probabilities (5 sigma per token)."""
    g = gen(64)
    V = 20000
    x = torch.randn(V, generator=g) * 0.5
    x[:6] = torch.tensor([6.0, 5.5, 5.2, 5.0, 4.5, 4.0])
    xb = x.bfloat16()
    s = Sampler(V)
    ids, probs, _, _ = _check_cut(s, xb, 1.0, 0.9)
    p = probs.double() / probs.double().sum()
    n = 3000
    counts = {}
    xd = xb.to(DEV)
    for _ in range(n):
        t, _ = s(xd, 1.0, 0.9)
        counts[t] = counts.get(t, 0) + 1
    assert set(counts) <= set(ids.tolist())
    for i, pi in zip(ids.tolist(), p.tolist()):
        f = counts.get(i, 0) / n
        assert abs(f - pi) <= 5 * math.sqrt(pi * (1 - pi) / n) + 1e-3, (i, f, pi)


def test_engine_sampling_graph_matches_eager_and_is_seeded():
    cfg = tiny(num_layers=4)
    w = make_weights(cfg, seed=0)
    prompt = make_prompt(cfg, n=6, seed=1)

    def run(graph, seed):
        eng = eng_mod.Qwen35FP8Engine(w, max_seq_len=64)
        eng.set_sampling(temperature=0.8, top_p=0.9, rep_penalty=1.1, window=50, seed=seed)
        if graph:
            eng.capture()
        eng.forward(prompt.view(1, -1).cuda(), 0)
        eng.generate(10)
        torch.cuda.synchronize()
        return eng.tokens(len(prompt) - 1, len(prompt) + 10).cpu().tolist()

    a = run(False, 5)
    b = run(True, 5)
    assert a == b, "graph replay draws the same tokens as eager launches"
    assert all(0 <= t < cfg.vocab_size for t in a)
