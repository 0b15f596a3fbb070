"""Drift over many consecutive decode steps (MI355X): the recurrent
GatedDeltaNet state and the attention over a growing KV cache, each carried by
the GPU through its own earlier results and compared with the CPU oracle at
every step.

One-step parity cannot see an error that accumulates (a biased exponential in
the state decay, a cache row written slightly differently and re-read by
every later step).  The recurrent state's error is measured against the same
recurrence in fp64 (oracle/qwen35_oracle.py delta_rule_step's arithmetic
restated in double precision): fed the same bf16 inputs, the GPU's fp32 state
may drift from exact arithmetic no more than the fp32 oracle itself does, up
to a factor of 2 and an absolute floor of 2e-7 of the state's scale.
"""
import math

import pytest
import torch

from oracle import qwen35_oracle as orc
from qwen35_amd import abi
from qwen35_amd import engine as eng_mod

from _util import assert_close, bf, cos_sim, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
N_STEPS = 300


def _delta_rule_fp64(q, k, v, g, beta, S):
    """orc.delta_rule_step in float64 (S updated in place, fp64)."""
    q, k, v = q.double(), k.double(), v.double()
    dk = q.shape[-1]
    qn = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6) * (1.0 / math.sqrt(dk))
    kn = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    Sd = S * torch.exp(g.double()).view(-1, 1, 1)
    pred = (Sd * kn.unsqueeze(-1)).sum(dim=-2)
    delta = (v - pred) * beta.double().view(-1, 1)
    S.copy_(Sd + kn.unsqueeze(-1) * delta.unsqueeze(-2))
    return (S * qn.unsqueeze(-1)).sum(dim=-2)


def _rel(a, b):
    return float((a.double() - b.double()).abs().max() / b.double().abs().max())


def _away_from_bf16_ties(x, f):
    """x (bf16 values) moved by whole bf16 steps until f(x), evaluated in fp64,
    rounds to the same bf16 value as f(x) (1 +- 2^-16): then any evaluation of f
    within a few fp32 ulps (the GPU's, the oracle's) rounds to that value too."""
    x = x.to(torch.bfloat16)
    for _ in range(64):
        y = f(x.double())
        lo = y.to(torch.bfloat16)
        bad = ((y * (1 + 2.0 ** -16)).to(torch.bfloat16) != lo) | ((y * (1 - 2.0 ** -16)).to(torch.bfloat16) != lo)
        if not bool(bad.any()):
            return x
        x = torch.where(bad, (x.view(torch.int16) + 1).view(torch.bfloat16), x)
    raise AssertionError("could not move the inputs away from bf16 rounding boundaries")


def _gdn_drift(clean):
    g = gen(4242 + clean)
    Hk, Hv, dk, dv = 16, 32, 128, 128
    kd, C = Hk * dk, 2 * Hk * dk + Hv * dv
    if clean:
        conv_w = torch.zeros(C, 4)
        conv_w[:, 3] = 1.0
        conv_w = bf(conv_w)
    else:
        conv_w = bf(randn(g, C, 4, std=0.5))
    A_log = torch.log(1e-3 + torch.rand(Hv, generator=g) * 16)
    dt_bias = torch.ones(Hv)
    S32 = randn(g, Hv, dk, dv, std=0.1)
    S64 = S32.double().clone()
    st = torch.zeros(C, 4)                         # ordered conv state, oldest first
    lib = abi.load()
    ring = torch.zeros(C, 4, dtype=torch.bfloat16, device=DEV)
    Sg = S32.clone().to(DEV)
    dw, dA, ddt = conv_w.to(DEV), A_log.to(DEV), dt_bias.to(DEV)
    coreg = torch.empty(Hv * dv, dtype=torch.bfloat16, device=DEV)
    silu = lambda x: x * torch.sigmoid(x)
    worst, errs = 0.0, []
    for t in range(N_STEPS):
        mixed, a, b = bf(randn(g, C)), bf(randn(g, Hv)), bf(randn(g, Hv))
        if clean:
            mixed = _away_from_bf16_ties(mixed, silu)
            b = _away_from_bf16_ties(b, torch.sigmoid)
        dm, da, db = mixed.to(DEV), a.to(DEV), b.to(DEV)
        abi.check(lib.qh_gdn_decode_core(abi.ptr(dm), abi.ptr(da), abi.ptr(db), abi.ptr(ring),
                                         abi.ptr(dw), abi.ptr(dA), abi.ptr(ddt), abi.ptr(Sg),
                                         abi.ptr(coreg), None, t, Hk, Hv, dk, dv,
                                         abi.stream_handle()), "gdn_core")
        y = orc.conv_update(mixed.float(), st, conv_w.float())
        q = y[:kd].view(Hk, dk).repeat_interleave(Hv // Hk, 0)
        k = y[kd:2 * kd].view(Hk, dk).repeat_interleave(Hv // Hk, 0)
        v = y[2 * kd:].view(Hv, dv)
        gg, beta = orc.linear_gates(a.float(), b.float(), A_log, dt_bias)
        core = orc.delta_rule_step(q, k, v, gg, beta, S32)
        _delta_rule_fp64(q, k, v, gg, beta, S64)
        torch.cuda.synchronize()
        assert_close(coreg, orc.bf16(core.reshape(-1)), atol_frac=1e-3, what=f"core, step {t}")
        ring_ref = torch.empty(C, 4)
        for i in range(4):
            ring_ref[:, (t - 3 + i) % 4] = st[:, i]
        assert torch.equal(ring.cpu().float()[:, t % 4], ring_ref[:, t % 4]), f"conv ring, step {t}"
        Sc = Sg.cpu()
        e_gpu, e_32, e_go = _rel(Sc, S64), _rel(S32, S64), _rel(Sc, S32)
        errs.append((e_gpu, e_32, e_go))
        if clean:
            worst = max(worst, e_gpu / max(e_32, 2e-7))
            assert e_gpu <= max(2.0 * e_32, 2e-7), \
                f"step {t}: GPU state error {e_gpu:.3g} vs the fp32 oracle's {e_32:.3g} (fp64 reference)"
        else:
            assert e_go <= 1e-4, f"step {t}: GPU state off the fp32 oracle's by {e_go:.3g} of its scale"
        if t % 50 == 49:
            print(f"step {t + 1}: state error vs fp64: GPU {e_gpu:.3g}, fp32 oracle {e_32:.3g}; "
                  f"GPU vs oracle {e_go:.3g}", flush=True)
    if clean:
        print(f"largest GPU / oracle error ratio {worst:.3f}", flush=True)
    # no trend: the last 50 steps' mean deviation is no larger than twice the
    # 50 before them (a drift would keep growing)
    late = sum(e[2] for e in errs[-50:]) / 50
    mid = sum(e[2] for e in errs[-100:-50]) / 50
    assert late <= 2 * max(mid, 1e-7), f"GPU - oracle state deviation grows: {mid:.3g} -> {late:.3g}"


def test_gdn_decode_core_300_steps_recurrence_no_drift():
    """BASELINE config 4a shapes (16 key / 32 value heads, dk = dv = 128):
    N_STEPS consecutive qh_gdn_decode_core steps from a state ~ N(0, 0.1), the
    conv ring and the state carried on the GPU.  The conv taps pass x_t
    through and the inputs keep SiLU(x) and sigmoid(b) away from bf16
    rounding boundaries, so GPU and oracle feed the recurrence identical bf16
    q, k, v and beta and only its arithmetic (l2norm, the exponential decay,
    the fp32 sums) differs.  Every step: the bf16 core against the fp32
    oracle (rtol 1e-2, cosine >= 0.99999), the conv ring exactly, and the
    state's error against the fp64 recurrence no larger than twice the fp32
    oracle's own (or 2e-7 of the state's scale)."""
    _gdn_drift(clean=True)


def test_gdn_decode_core_300_steps_random_inputs():
    """The same N_STEPS steps with unrestricted random inputs and conv taps:
    here the GPU's fp32 conv + SiLU can round a channel to the other bf16
    neighbour than the oracle's (a one-ulp input difference that the state
    then carries and decays).  Every step: the core within the kernel parity
    bar, the state within 1e-4 of the oracle's scale, and no growth of the
    deviation over the run."""
    _gdn_drift(clean=False)


def test_attention_decode_over_growing_context():
    """BASELINE config 4b shapes (16 query / 4 KV heads, head dim 256, RoPE on
    64 dims, theta 1e7) decoded for N_STEPS consecutive positions from a
    128-token cache, the position read from device memory and 64 splits as the
    engine runs them (4096-slot cache).  GPU and oracle each keep their own
    cache (each writes its own normed, rotated K at every step); both read the
    device-built RoPE tables.  Every step: the output against the oracle
    (rtol 1e-2, atol 1e-3 of the largest value, cosine >= 0.99999) and the
    cache row just written; at the end, the whole written cache."""
    g = gen(777)
    Hq, Hkv, D, rot, max_seq, ctx0 = 16, 4, 256, 64, 4096, 128
    splits = eng_mod.default_attn_splits(max_seq)
    kc = torch.zeros(Hkv, max_seq, D)
    vc = torch.zeros(Hkv, max_seq, D)
    kc[:, :ctx0] = bf(randn(g, Hkv, ctx0, D)).float()
    vc[:, :ctx0] = bf(randn(g, Hkv, ctx0, D)).float()
    qn, kn = randn(g, D, std=0.02), randn(g, D, std=0.02)
    gcos, gsin = eng_mod.rope_tables(max_seq, rot, 1e7, device=DEV)
    cos, sin = gcos.cpu(), gsin.cpu()
    lib = abi.load()
    kcg, vcg = bf(kc).to(DEV), bf(vc).to(DEV)
    dqn, dkn = qn.to(DEV), kn.to(DEV)
    out = torch.empty(Hq * D, dtype=torch.bfloat16, device=DEV)
    scratch = torch.zeros(int(lib.qh_attn_scratch_bytes(Hkv, splits, D)) + 4, dtype=torch.uint8,
                          device=DEV)
    counters = torch.zeros(Hkv, dtype=torch.int32, device=DEV)
    posd = torch.zeros(1, dtype=torch.int32, device=DEV)
    min_cos = 1.0
    for step in range(N_STEPS):
        pos = ctx0 + step
        q_all, k_new, v_new = bf(randn(g, Hq * 2 * D)), bf(randn(g, Hkv * D)), bf(randn(g, Hkv * D))
        qa, dk_, dv_ = q_all.to(DEV), k_new.to(DEV), v_new.to(DEV)
        posd.fill_(pos)
        abi.check(lib.qh_attn_decode(abi.ptr(qa), 2 * D, abi.ptr(qa[D:]), 2 * D, abi.ptr(dk_), abi.ptr(dv_),
                                     abi.ptr(dqn), abi.ptr(dkn), abi.ptr(gcos), abi.ptr(gsin),
                                     abi.ptr(kcg), abi.ptr(vcg), max_seq, D, rot, Hq, Hkv,
                                     abi.ptr(posd), 0, splits, abi.ptr(scratch), abi.ptr(counters),
                                     abi.ptr(out), 1e-6, abi.stream_handle()), "attn_decode")
        ref = orc.attn_decode(q_all.float(), k_new.float(), v_new.float(), qn, kn, cos, sin, kc, vc,
                              pos, Hq, Hkv, D, rot)
        torch.cuda.synchronize()
        min_cos = min(min_cos, assert_close(out, ref, atol_frac=1e-3, what=f"attention at position {pos}"))
        assert_close(kcg[:, pos], kc[:, pos], rtol=2 ** -7, atol_frac=0, min_cos=0.99999,
                     what=f"K row {pos}")
        assert torch.equal(vcg[:, pos].cpu().float(), vc[:, pos]), f"V row {pos}"
    last = ctx0 + N_STEPS
    assert_close(kcg[:, :last], kc[:, :last], rtol=2 ** -7, atol_frac=0, min_cos=0.999999,
                 what="whole K cache")
    assert torch.equal(vcg[:, :last].cpu().float(), vc[:, :last]), "whole V cache"
    assert int(counters.abs().sum()) == 0
    print(f"attention over positions {ctx0}..{last - 1}: min output cosine {min_cos:.8f}", flush=True)
