"""Batch prefill (the reference's s > 1 path, main.py:1550-1566) on the GPU
against the CPU oracle's prefill restatement (MI355X only)."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import qwen35_oracle as orc
from qwen35_amd import abi
from qwen35_amd import engine as eng_mod
from qwen35_amd.config import tiny
from qwen35_amd.synth import make_prompt, make_weights

from _util import assert_close, bf, cos_sim, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def cu(t):
    return t.to(DEV).contiguous()


# (tokens, past): positions 0 .. past-1 are cached by an earlier prep call,
# positions past .. tokens-1 are the prefill.  Prefills of 256 or more tokens
# run the matrix-core kernel (300: a ragged last 32-token block; 330 - 70 =
# 260 after a cached prefix), shorter ones the per-token kernel.
# The last two cases take the per-token kernel with two query heads per wave
# (8 per KV head, head dim 128) and with an idle wave (3 per KV head).
@pytest.mark.parametrize("M,past,Hq,Hkv,D", [(37, 0, 8, 2, 256), (70, 0, 8, 2, 256), (100, 20, 8, 2, 256),
                                             (256, 0, 8, 2, 256), (300, 0, 8, 2, 256), (330, 70, 8, 2, 256),
                                             (45, 10, 16, 2, 128), (50, 13, 6, 2, 256)])
def test_attention_prefill(M, past, Hq, Hkv, D):
    g = gen(21)
    rot, max_seq = 64, 512
    q_all = bf(randn(g, M, Hq, 2 * D))
    k, v = bf(randn(g, M, Hkv, D)), bf(randn(g, M, Hkv, D))
    qn_w, kn_w = randn(g, D, std=0.1), randn(g, D, std=0.1)
    cos, sin = orc.rope_tables(max_seq, rot, 1e7)
    lib = abi.load()
    dq, dk_, dv_ = cu(q_all), cu(k), cu(v)
    q32 = torch.empty(M, Hq, D, dtype=torch.float32, device=DEV)
    kc = torch.zeros(Hkv, max_seq, D, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    n = M - past
    out = torch.empty(n, Hq * D, dtype=torch.bfloat16, device=DEV)
    dcos, dsin, dqn, dkn = cu(cos), cu(sin), cu(qn_w), cu(kn_w)
    st = abi.stream_handle()
    for p0, cnt in ((0, past), (past, n)):
        if cnt:
            abi.check(lib.qh_attn_prep(abi.ptr(dq[p0:]), abi.ptr(dk_[p0:]), abi.ptr(dv_[p0:]), abi.ptr(dqn),
                                       abi.ptr(dkn), abi.ptr(dcos), abi.ptr(dsin), abi.ptr(q32[p0:]),
                                       abi.ptr(kc), abi.ptr(vc), cnt, Hq, Hkv, D, rot, p0, max_seq, 1e-6, st))
    abi.check(lib.qh_attn_prefill(abi.ptr(q32[past:]), abi.ptr(dq[past:, :, D:]), Hq * 2 * D, 2 * D,
                                  abi.ptr(kc), abi.ptr(vc), abi.ptr(out), n, Hq, Hkv, D, past, max_seq,
                                  st))
    torch.cuda.synchronize()
    # oracle: the attention part of OracleModel._full_prefill
    q = orc.rmsnorm(q_all[..., :D].float(), qn_w)
    kk = orc.rmsnorm(k.float(), kn_w)
    q = orc.rope_rows(q, cos[:M].view(M, 1, -1), sin[:M].view(M, 1, -1), rot, round_out=False)
    kk = orc.rope_rows(kk, cos[:M].view(M, 1, -1), sin[:M].view(M, 1, -1), rot, round_out=False)
    # the head norm rounds to bf16 before RoPE: a different fp32 summation order
    # may move that rounding by one bf16 ulp
    assert_close(q32.view(M, Hq, D), q, rtol=2 ** -7, atol_frac=1e-6, what="q (fp32, rotated)")
    assert_close(kc[:, :M], orc.bf16(kk).transpose(0, 1), rtol=2 ** -7, atol_frac=0,
                 what="k cache rows")
    assert torch.equal(vc[:, :M].cpu(), v.transpose(0, 1))
    K, V = orc.bf16(kk).transpose(0, 1), v.float().transpose(0, 1)
    mask = torch.triu(torch.full((M, M), float("-inf")), diagonal=1)
    ref = torch.empty(M, Hq, D)
    for h in range(Hq):
        kv = h * Hkv // Hq
        sc = (q[:, h] @ K[kv].t()) * (D ** -0.5) + mask
        ref[:, h] = orc.bf16(torch.softmax(sc, dim=-1) @ V[kv])
    ref = orc.bf16(ref.reshape(M, -1) * orc.bf16(torch.sigmoid(q_all[..., D:].float().reshape(M, -1))))
    assert_close(out, ref[past:], atol_frac=1e-3, what="prefill attention")


# M = 45: five full 8-token blocks of the scan plus a tail; M = 3: fewer
# tokens than the conv window (the ring supplies them all); past > 0 with a
# filled ring and state: the conv reads positions before the prompt.
# algo "chunk" (qh_gdn_chunk): M = 64 one full chunk, 130 two chunks and a
# 2-token tail, 200 from a stored state over four chunks, 600 (from a stored
# state) the 8-channel conv kernel of prompts of 512+ tokens.  Hv = 8 and 32
# (Hv % 8 == 0) place the state kernel's 8 workgroups of a head on one XCD.
@pytest.mark.parametrize("M,past,algo,Hk,Hv", [
    (45, 0, "scan", 2, 4), (3, 0, "scan", 2, 4), (8, 6, "scan", 2, 4), (21, 6, "scan", 2, 4),
    (45, 0, "chunk", 2, 4), (3, 0, "chunk", 2, 4), (21, 6, "chunk", 2, 4), (64, 0, "chunk", 2, 4),
    (130, 0, "chunk", 2, 4), (200, 6, "chunk", 2, 4), (600, 6, "chunk", 2, 4),
    (130, 6, "chunk", 4, 8), (70, 6, "chunk", 16, 32), (130, 0, "scan", 16, 32)])
def test_gdn_prefill(M, past, algo, Hk, Hv):
    g = gen(22 + M + past + Hv)
    dk, dv = 128, 128
    C = 2 * Hk * dk + Hv * dv
    mixed = bf(randn(g, M, C))
    a, b = bf(randn(g, M, Hv)), bf(randn(g, M, Hv))
    z = bf(randn(g, M, Hv * dv))
    conv_w = bf(randn(g, C, 4, std=0.3))
    A_log = torch.log(1e-3 + torch.rand(Hv, generator=g) * 16)
    dt_bias = torch.ones(Hv)
    norm_w = bf(1 + randn(g, dv, std=0.02))
    lib = abi.load()
    ring0 = bf(randn(g, C, 4)) if past else torch.zeros(C, 4)
    state0 = randn(g, Hv, dk, dv, std=0.1) if past else torch.zeros(Hv, dk, dv)
    ring = cu(ring0).to(torch.bfloat16)
    state = cu(state0).float()
    y = torch.empty(M, C, dtype=torch.bfloat16, device=DEV)
    qn = torch.empty(M, Hk * dk, dtype=torch.bfloat16, device=DEV)
    kn = torch.empty_like(qn)
    gg = torch.empty(M, Hv, dtype=torch.float32, device=DEV)
    beta = torch.empty(M, Hv, dtype=torch.bfloat16, device=DEV)
    out = torch.empty(M, Hv * dv, dtype=torch.bfloat16, device=DEV)
    dm, da, db, dz, dw = cu(mixed), cu(a), cu(b), cu(z), cu(conv_w)
    dA, ddt, dnw = cu(A_log), cu(dt_bias), cu(norm_w)
    st = abi.stream_handle()
    abi.check(lib.qh_gdn_prep(abi.ptr(dm), abi.ptr(ring), abi.ptr(dw), abi.ptr(da), abi.ptr(db),
                              abi.ptr(dA), abi.ptr(ddt), abi.ptr(y), abi.ptr(qn), abi.ptr(kn),
                              abi.ptr(gg), abi.ptr(beta), M, Hk, Hv, dk, dv, past, st))
    if algo == "scan":
        abi.check(lib.qh_gdn_scan(abi.ptr(qn), abi.ptr(kn), abi.ptr(y), abi.ptr(gg), abi.ptr(beta),
                                  abi.ptr(dz), abi.ptr(dnw), abi.ptr(state), abi.ptr(out), M, Hk, Hv,
                                  dk, dv, 1e-6, st))
    else:
        nws = int(lib.qh_gdn_chunk_workspace_size(M, Hv))
        assert nws == Hv * ((M + 63) // 64) * 99328
        ws = torch.empty(nws, dtype=torch.uint8, device=DEV)
        abi.check(lib.qh_gdn_chunk(abi.ptr(qn), abi.ptr(kn), abi.ptr(y), abi.ptr(gg), abi.ptr(beta),
                                   abi.ptr(dz), abi.ptr(dnw), abi.ptr(state), abi.ptr(out), M, Hk, Hv,
                                   dk, dv, 1e-6, abi.ptr(ws), nws, st))
    torch.cuda.synchronize()
    # oracle: OracleModel._gdn_prefill after the projections
    # window history: slot (past - 3 + i) % 4 of the ring holds position past - 3 + i
    cs = torch.zeros(C, 4)
    for i in range(3):
        cs[:, 1 + i] = ring0.float()[:, (past - 3 + i) % 4]
    xt = torch.cat([cs, mixed.float().t()], dim=1)
    conv = torch.stack([(conv_w.float() * xt[:, j + 1:j + 5]).sum(1) for j in range(M)], dim=0)
    yr = orc.bf16(F.silu(orc.bf16(conv)))
    assert_close(y, yr, atol_frac=1e-3, what="conv")
    ring_ref = ring0.float().clone()
    for mm in range(max(0, M - 4), M):
        ring_ref[:, (past + mm) % 4] = mixed[mm].float()
    assert torch.equal(ring.cpu().float(), ring_ref)
    yg = y.cpu().float()   # continue from the GPU conv output (isolates the later stages)
    kd, r = Hk * dk, Hv // Hk
    q = orc.l2norm_bf16(yg[:, :kd].reshape(M, Hk, dk))
    k = orc.l2norm_bf16(yg[:, kd:2 * kd].reshape(M, Hk, dk))
    assert_close(qn.view(M, Hk, dk), q, rtol=2 ** -7, atol_frac=0, what="l2norm q")
    assert_close(kn.view(M, Hk, dk), k, rtol=2 ** -7, atol_frac=0, what="l2norm k")
    gr, br = orc.linear_gates(a, b, A_log, dt_bias)
    assert_close(gg, gr, rtol=1e-5, atol_frac=1e-6, what="g")
    assert torch.equal(beta.cpu().float(), br)
    qh = qn.cpu().float().view(M, Hk, dk).repeat_interleave(r, dim=1)
    kh = kn.cpu().float().view(M, Hk, dk).repeat_interleave(r, dim=1)
    vh = yg[:, 2 * kd:].reshape(M, Hv, dv)
    S = state0.clone()
    o = orc.gated_delta_rule_seq(qh * (1.0 / math.sqrt(dk)), kh, vh, gg.cpu(), beta.cpu().float(), S)
    gated = orc.gated_rmsnorm(orc.bf16(o), z.float().view(M, Hv, dv), norm_w, 1e-6, bf16_steps=True)
    assert_close(out.view(M, Hv, dv), gated, atol_frac=1e-3, what="gated output")
    assert_close(state, S, rtol=1e-3, atol_frac=1e-4, what="final state")
    if algo == "chunk":
        # the reference's own (chunked) algorithm from the same state
        o_c, S_c = orc.chunk_gated_delta_rule(qh * (1.0 / math.sqrt(dk)), kh, vh, gg.cpu(),
                                              beta.cpu().float(), S0=state0)
        gated_c = orc.gated_rmsnorm(orc.bf16(o_c), z.float().view(M, Hv, dv), norm_w, 1e-6,
                                    bf16_steps=True)
        assert_close(out.view(M, Hv, dv), gated_c, atol_frac=1e-3, what="gated output (chunked)")
        assert_close(state, S_c, rtol=1e-3, atol_frac=1e-4, what="final state (chunked)")


# n % 8 == 0 takes the 16-byte kernel, 10007 the element kernel
@pytest.mark.parametrize("n", [10007, 10000, 3 * 9216])
def test_silu_mul_exact(n):
    g = gen(23)
    a, b = bf(randn(g, n)), bf(randn(g, n))
    lib = abi.load()
    da, db = cu(a), cu(b)
    out = torch.empty(n, dtype=torch.bfloat16, device=DEV)
    abi.check(lib.qh_silu_mul(abi.ptr(da), abi.ptr(db), abi.ptr(out), n, abi.stream_handle()))
    torch.cuda.synchronize()
    ref = orc.bf16(orc.bf16(F.silu(a.float())) * b.float())
    assert torch.equal(out.cpu().float(), ref)


def test_engine_batch_prefill_chunked_gdn_matches_oracle():
    """A 150-token prompt: the engine's GatedDeltaNet layers take the chunked
    (WY) matrix-core path (qh_gdn_chunk); logits against the oracle's reference
    prefill (recurrent rule), then a second batch prefill continuing at
    past_len 150 from the stored state."""
    cfg = tiny(num_layers=4)
    w = make_weights(cfg, seed=0)
    prompt = make_prompt(cfg, n=150, seed=3)
    more = make_prompt(cfg, n=100, seed=4)
    assert prompt.numel() >= eng_mod.GDN_CHUNK_MIN_TOKENS and more.numel() >= eng_mod.GDN_CHUNK_MIN_TOKENS
    eng = eng_mod.Qwen35FP8Engine(w, max_seq_len=256)
    ref = orc.OracleModel(w, max_seq_len=256, prefill="reference")
    l1 = eng.forward(prompt.view(1, -1).cuda(), 0).float().cpu().view(-1)
    r1 = ref.forward(prompt.view(1, -1), 0).view(-1)
    assert cos_sim(l1, r1) > 0.9999
    l2 = eng.forward(more.view(1, -1).cuda(), 150).float().cpu().view(-1)
    r2 = ref.forward(more.view(1, -1), 150).view(-1)
    assert cos_sim(l2, r2) > 0.9999


def test_engine_batch_prefill_matches_oracle_reference_prefill():
    """Whole-model batch prefill (FP8 GEMMs + batch kernels) against the oracle's
    reference prefill path, then greedy decode continuing from its state."""
    cfg = tiny(num_layers=4)
    w = make_weights(cfg, seed=0)
    prompt = make_prompt(cfg, n=9, seed=1)
    eng = eng_mod.Qwen35FP8Engine(w, max_seq_len=64)
    logits = eng.forward(prompt.view(1, -1).cuda(), 0).float().cpu().view(-1)
    ref = orc.OracleModel(w, max_seq_len=64, prefill="reference")
    rl = ref.forward(prompt.view(1, -1), 0).view(-1)
    assert cos_sim(logits, rl) > 0.9999
    assert int(eng.pos.item()) == len(prompt)
    n_steps = 8
    eng.generate(n_steps - 1)
    torch.cuda.synchronize()
    toks = eng.tokens(len(prompt) - 1, len(prompt) - 1 + n_steps).cpu().tolist()
    pos, lg = len(prompt), rl
    for i in range(n_steps):
        t = orc.argmax_first(lg)
        top = torch.topk(lg, 2).values
        if toks[i] != t:
            assert float(top[0] - top[1]) <= 2 ** -6, f"step {i}: {toks[i]} vs oracle {t}"
            break
        lg, _ = ref.decode_token(t, pos)
        lg = lg.view(-1)
        pos += 1


def test_engine_batch_prefill_4b_widths_matches_oracle():
    """Batch prefill at the 4B layer widths (hidden 2560, MLP 9216, 16x256
    attention, 32x128 GatedDeltaNet; 4 layers, small vocabulary): the grouped
    GEMMs, split-K (out_proj / o_proj / down at M = 40 have fewer tiles than
    CUs), the wave-per-columns scan and the batch attention, against the
    oracle's reference prefill."""
    import dataclasses
    from qwen35_amd.config import qwen35_4b
    cfg = dataclasses.replace(qwen35_4b(), num_hidden_layers=4, vocab_size=4096, layer_types=None)
    w = make_weights(cfg, seed=5)
    prompt = make_prompt(cfg, n=40, seed=6)
    eng = eng_mod.Qwen35FP8Engine(w, max_seq_len=64)
    logits = eng.forward(prompt.view(1, -1).cuda(), 0).float().cpu().view(-1)
    ref = orc.OracleModel(w, max_seq_len=64, prefill="reference")
    rl = ref.forward(prompt.view(1, -1), 0).view(-1)
    # At these widths the oracle's two exact restatements of the prompt pass
    # (the reference's chunked prefill and the token-by-token recurrence)
    # already disagree at the 1e-4 level of logit cosine (0.99982 at 4 layers,
    # measured): the GPU path must agree with the reference prefill as well as
    # they agree with each other.
    rs = orc.OracleModel(w, max_seq_len=64, prefill="sequential").forward(prompt.view(1, -1), 0).view(-1)
    c, c_oracle = cos_sim(logits, rl), cos_sim(rs, rl)
    assert c > 0.9995 and c >= c_oracle - 1e-4, f"logit cosine {c} (oracle paths: {c_oracle})"
    top = torch.topk(rl, 2).values
    if float(top[0] - top[1]) > 2 ** -6:
        assert int(torch.argmax(logits)) == orc.argmax_first(rl)
