"""Pins of the CPU oracle (no GPU): library routines, closed forms, invariants
and brute force on tiny inputs, chosen so a dropped term, wrong sign or index,
or a transposed operand fails at least one of them."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import qwen35_oracle as orc

from _util import bf, cos_sim, gen, randn


# ------------------------------------------------------------------ A0
def test_e4m3_table_matches_torch_float8():
    codes = torch.arange(256, dtype=torch.uint8)
    lib = codes.view(torch.float8_e4m3fn).float()
    tab = orc.e4m3_table()
    nan = torch.isnan(lib)
    assert torch.equal(nan, torch.isnan(tab))
    assert nan.sum() == 2 and nan[0x7F] and nan[0xFF]
    assert torch.equal(lib[~nan], tab[~nan])


def test_e4m3_special_values():
    assert orc.e4m3_decode(0x7E) == 448.0
    assert orc.e4m3_decode(0xFE) == -448.0
    assert orc.e4m3_decode(0x01) == 2.0 ** -9
    assert orc.e4m3_decode(0x08) == 2.0 ** -6
    assert orc.e4m3_decode(0x38) == 1.0
    assert orc.e4m3_decode(0x80) == 0.0 and math.copysign(1, orc.e4m3_decode(0x80)) == -1


# ------------------------------------------------------------------ A10 / A1
def test_block_quantizer_closed_form():
    g = gen(0)
    W = randn(g, 300, 260, std=0.02)
    q, s = orc.quantize_block_fp8(W)
    assert q.dtype == torch.uint8 and s.shape == (3, 3)
    # s = amax/448 per block; the block max maps to +-448
    for bi in range(3):
        for bk in range(3):
            blk = W[bi * 128:(bi + 1) * 128, bk * 128:(bk + 1) * 128]
            assert torch.isclose(s[bi, bk], blk.abs().max() / 448, rtol=1e-7)
            qb = orc.e4m3_table()[q[bi * 128:(bi + 1) * 128, bk * 128:(bk + 1) * 128].long()]
            assert qb.abs().max() == 448.0
    # dequant error bounded by half an E4M3 ulp (relative 2^-4) or the subnormal step
    D = orc.dequant(q, s)
    full = s.repeat_interleave(128, 0).repeat_interleave(128, 1)[:300, :260]
    err = (D - W).abs()
    assert (err <= W.abs() * 2 ** -4 + full * 2 ** -10 + 1e-12).all()


def test_dequant_modes_brute_force():
    g = gen(1)
    N, K = 130, 256
    q = torch.randint(0, 256, (N, K), generator=g, dtype=torch.uint8)
    q[q == 0x7F] = 0
    q[q == 0xFF] = 0
    tab = orc.e4m3_table()
    sb = torch.rand(2, 2, generator=g) + 0.5
    sr = torch.rand(N, generator=g) + 0.5
    srb = torch.rand(N, 2, generator=g) + 0.5
    Db, Dr, Drb = orc.dequant(q, sb), orc.dequant(q, sr.view(N, 1), 1), orc.dequant(q, srb)
    for n in (0, 127, 128, 129):
        for k in (0, 127, 128, 255):
            v = tab[int(q[n, k])]
            assert Db[n, k] == v * sb[n // 128, k // 128]
            assert Dr[n, k] == v * sr[n]
            assert Drb[n, k] == v * srb[n, k // 128]
    assert orc.scale_code(q, sb) == 2 and orc.scale_code(q, srb) == -2


def test_gemv_exact_integer_case():
    """s = 1 and small integer weights/activations: the fp32 GEMV is exact."""
    g = gen(2)
    N, K = 64, 256
    ints = torch.randint(-8, 9, (N, K), generator=g).float()
    q = ints.to(torch.float8_e4m3fn).view(torch.uint8)
    s = torch.ones(1, 2)
    x = torch.randint(-4, 5, (K,), generator=g).float()
    y = orc.linear(x, orc.dequant(q, s))
    assert torch.equal(y, orc.bf16(ints @ x))   # exact sum, one bf16 rounding
    # one-hot x selects a dequantised column
    e = torch.zeros(K)
    e[17] = 1.0
    assert torch.equal(orc.linear(e, orc.dequant(q, s)), ints[:, 17])


def test_gemv_fp32_vs_fp64_brute_force():
    g = gen(3)
    q, s = orc.quantize_block_fp8(randn(g, 256, 384, std=0.02))
    x = bf(randn(g, 384)).float()
    y = orc.linear(x, orc.dequant(q, s))
    y64 = orc.gemv_fp64(x, q, s)
    assert (y.double() - y64).abs().max() <= 2 ** -8 * y64.abs().max()


# ------------------------------------------------------------------ A3
def test_rmsnorm_invariants():
    g = gen(4)
    x = bf(randn(g, 4, 2560) * 5)
    y = orc.rmsnorm(x.float(), torch.zeros(2560))
    rms = y.pow(2).mean(-1).sqrt()
    assert torch.allclose(rms, torch.ones(4), atol=1e-2)
    w = torch.full((2560,), 1.0)          # (1 + w) = 2 doubles the output
    assert torch.allclose(orc.rmsnorm(x.float(), w), orc.bf16(2 * y), rtol=0, atol=0)


# ------------------------------------------------------------------ A4
def test_rope_identity_at_pos0_and_pair_norm():
    cos, sin = orc.rope_tables(64, 64, 1e7)
    g = gen(5)
    x = randn(g, 3, 256)
    assert torch.equal(orc.rope_rows(x, cos[0], sin[0], 64, False), x)
    y = orc.rope_rows(x, cos[37], sin[37], 64, False)
    assert torch.equal(y[:, 64:], x[:, 64:])                     # pass-through dims
    n0 = x[:, :32] ** 2 + x[:, 32:64] ** 2                       # pair (c, c+32) norm kept
    n1 = y[:, :32] ** 2 + y[:, 32:64] ** 2
    assert torch.allclose(n0, n1, rtol=1e-5)
    # inv_freq denominator is the rotary dim: channel 1 rotates by pos * theta^(-2/64)
    ang = 37 * 1e7 ** (-2 / 64)
    assert math.isclose(float(cos[37, 1]), math.cos(ang), rel_tol=1e-6)


def test_attention_single_position_returns_v_and_gqa_mapping():
    g = gen(6)
    Hq, Hkv, D = 16, 4, 256
    kc = randn(g, Hkv, 8, D)
    vc = randn(g, Hkv, 8, D)
    q = randn(g, Hq * D)
    out = orc.attn_only(q, kc, vc, 1, Hq, Hkv)
    for h in range(Hq):
        assert torch.equal(out.view(Hq, D)[h], orc.bf16(vc[h // 4, 0]))
    # brute force softmax for ctx 8 against float64
    out8 = orc.attn_only(q, kc, vc, 8, Hq, Hkv).view(Hq, D)
    for h in (0, 5, 15):
        kv = h // 4
        s = (q.view(Hq, D)[h].double() @ kc[kv].double().t()) / 16.0
        ref = torch.softmax(s, -1) @ vc[kv].double()
        assert torch.allclose(out8[h].double(), ref, rtol=1e-2, atol=1e-2)


# ------------------------------------------------------------------ A5
def test_conv_update_closed_form():
    g = gen(7)
    C = 16
    st = bf(randn(g, C, 4)).float()
    w = bf(randn(g, C, 4)).float()
    x = bf(randn(g, C)).float()
    st0 = st.clone()
    y = orc.conv_update(x, st, w)
    assert torch.equal(st[:, :3], st0[:, 1:]) and torch.equal(st[:, 3], x)
    manual = w[:, 0] * st0[:, 1] + w[:, 1] * st0[:, 2] + w[:, 2] * st0[:, 3] + w[:, 3] * x
    assert torch.allclose(y, orc.bf16(F.silu(orc.bf16(manual))), atol=1e-6)


def test_delta_rule_invariants():
    g = gen(8)
    H, d = 4, 16
    q, k, v = randn(g, H, d), randn(g, H, d), randn(g, H, d)
    S0 = randn(g, H, d, d, std=0.1)
    gl = -torch.rand(H, generator=g)
    # beta = 0: pure decay
    S = S0.clone()
    orc.delta_rule_step(q, k, v, gl, torch.zeros(H), S)
    assert torch.allclose(S, S0 * torch.exp(gl).view(-1, 1, 1), rtol=1e-6, atol=1e-7)
    # g = 0, beta = 1: the state now maps k^ to v exactly (delta rule writes v)
    S = S0.clone()
    orc.delta_rule_step(q, k, v, torch.zeros(H), torch.ones(H), S)
    kn = k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    recalled = (S * kn.unsqueeze(-1)).sum(-2)
    assert torch.allclose(recalled, v, atol=1e-4)


def test_recurrent_equals_chunked_rule():
    g = gen(9)
    T, H, dk, dv = 150, 3, 32, 24
    q = F.normalize(randn(g, T, H, dk), dim=-1) / math.sqrt(dk)
    k = F.normalize(randn(g, T, H, dk), dim=-1)
    v = randn(g, T, H, dv)
    gl = -torch.rand(T, H, generator=g) * 0.5
    beta = torch.sigmoid(randn(g, T, H))
    S = torch.zeros(H, dk, dv)
    o_rec = orc.gated_delta_rule_seq(q, k, v, gl, beta, S)
    o_chk, S_chk = orc.chunk_gated_delta_rule(q, k, v, gl, beta)
    assert torch.allclose(o_rec, o_chk, rtol=1e-4, atol=1e-4)
    assert torch.allclose(S, S_chk, rtol=1e-4, atol=1e-4)


def test_chunked_rule_from_initial_state_equals_recurrent():
    """The initial-state path of the chunked rule (prefill at past_len > 0)
    against the recurrence from the same state, over 2.5 chunks."""
    g = gen(19)
    T, H, dk, dv = 160, 2, 32, 24
    q = F.normalize(randn(g, T, H, dk), dim=-1) / math.sqrt(dk)
    k = F.normalize(randn(g, T, H, dk), dim=-1)
    v = randn(g, T, H, dv)
    gl = -torch.rand(T, H, generator=g) * 0.5
    beta = torch.sigmoid(randn(g, T, H))
    S0 = randn(g, H, dk, dv, std=0.3)
    S = S0.clone()
    o_rec = orc.gated_delta_rule_seq(q, k, v, gl, beta, S)
    o_chk, S_chk = orc.chunk_gated_delta_rule(q, k, v, gl, beta, S0=S0)
    assert torch.allclose(o_rec, o_chk, rtol=1e-4, atol=1e-4)
    assert torch.allclose(S, S_chk, rtol=1e-4, atol=1e-4)
    # a wrong initial state is detected: zero start differs
    o_zero, _ = orc.chunk_gated_delta_rule(q, k, v, gl, beta)
    assert (o_zero - o_rec).abs().max() > 1e-2


def test_l2norm_bf16_and_gates():
    g = gen(10)
    x = bf(randn(g, 5, 128)).float()
    y = orc.l2norm_bf16(x)
    assert torch.allclose(y.norm(dim=-1), torch.ones(5), atol=2e-2)
    a = torch.tensor([0.0, 25.0, -3.0])
    gg, beta = orc.linear_gates(a, torch.zeros(3), torch.zeros(3), torch.zeros(3))
    assert torch.allclose(gg, -torch.tensor([math.log(2.0), 25.0, math.log1p(math.exp(-3.0))]))
    assert torch.equal(beta, torch.full((3,), 0.5))


# ------------------------------------------------------------------ A6
def test_argmax_first_on_ties():
    x = torch.tensor([1.0, 3.0, 2.0, 3.0, 3.0])
    assert orc.argmax_first(x) == 1
    assert orc.argmax_first(torch.tensor([-1.0, -1.0])) == 0


# ------------------------------------------------------------------ model
def test_prefill_close_to_sequential_decode():
    """Batch prefill and token-by-token decode are the same function up to the
    bf16 rounding points that differ between the two reference paths."""
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    cfg = pkg.config.tiny(num_layers=4)
    w = pkg.synth.make_weights(cfg, seed=0)
    prompt = pkg.synth.make_prompt(cfg, n=9, seed=1)
    a = orc.OracleModel(w, 64, prefill="reference").forward(prompt, 0).view(-1)
    b = orc.OracleModel(w, 64, prefill="sequential").forward(prompt, 0).view(-1)
    assert cos_sim(a, b) > 0.999


def test_prefill_continues_from_cache():
    """A prompt prefilled in two pieces (the second at past_len > 0, which
    continues from the stored KV cache, conv state and recurrent state,
    main.py:1130-1131) gives the logits of the one-piece prefill; the
    recurrent GatedDeltaNet part is the same computation token by token."""
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    cfg = pkg.config.tiny(num_layers=4)
    w = pkg.synth.make_weights(cfg, seed=0)
    prompt = pkg.synth.make_prompt(cfg, n=12, seed=3)
    m = orc.OracleModel(w, 64, prefill="reference")
    whole = m.forward(prompt, 0, logits_to_keep=0)
    assert whole.shape == (12, cfg.vocab_size)
    first = m.forward(prompt[:7], 0, logits_to_keep=0)
    second = m.forward(prompt[7:], 7, logits_to_keep=0)
    pieces = torch.cat([first, second])
    for j in range(12):
        assert cos_sim(pieces[j], whole[j]) > 0.9999, j
    # logits_to_keep=k keeps the last k rows of the same computation
    last2 = m.forward(prompt, 0, logits_to_keep=2)
    assert torch.equal(last2, whole[-2:])


def test_forward_at_zero_starts_a_new_sequence():
    """forward(ids, 0) ignores whatever an earlier sequence left in the
    caches: the same prompt gives the same logits after another prompt."""
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    cfg = pkg.config.tiny(num_layers=4)
    w = pkg.synth.make_weights(cfg, seed=0)
    a = pkg.synth.make_prompt(cfg, n=5, seed=4)
    b = pkg.synth.make_prompt(cfg, n=1, seed=5)
    for mode in ("reference", "sequential"):
        m = orc.OracleModel(w, 64, prefill=mode)
        fresh = m.forward(b, 0)
        m.forward(a, 0)
        assert torch.equal(m.forward(b, 0), fresh), mode
