"""Per-kernel parity of the HIP library against the CPU oracle (MI355X only).

Every call goes through the C-ABI (ctypes), the reference symbols with bf16
scales and the native qh_* entry points with fp32 scales.
"""
import math

import numpy as np
import pytest
import torch

from oracle import qwen35_oracle as orc
from qwen35_amd import abi, ops
from qwen35_amd import engine as eng_mod

from _util import assert_close, bf, cos_sim, gen, quant, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"

# Device copies made by cu() stay referenced until the test ends: a pointer
# taken from a temporary tensor would be freed (and its memory reused by the
# caching allocator) before the kernel reads it.
_KEEP = []


@pytest.fixture(autouse=True)
def _keep_alive():
    abi.load().qh_clear_error()   # the error string is per thread and persists
    yield
    torch.cuda.synchronize()
    _KEEP.clear()


def cu(t):
    d = t.to(DEV).contiguous()
    _KEEP.append(d)
    return d


def sync():
    torch.cuda.synchronize()


# ------------------------------------------------------------------ E4M3
def test_e4m3_decode_all_codes(lib):
    """Every E4M3FN code through the GEMV with s = 1 and a one-hot x equals the
    OCP closed form (NaN codes stay NaN)."""
    N, K = 256, 128
    w = torch.arange(256, dtype=torch.uint8).view(N, 1).expand(N, K).contiguous()
    s = torch.ones(N)          # one scale per row (K_blocks == 1)
    x = torch.zeros(K, dtype=torch.bfloat16)
    x[0] = 1.0
    y = ops.fp8_linear(cu(x).view(1, K), cu(w), cu(s)).cpu().float()
    ref = orc.e4m3_table()
    nan = torch.isnan(ref)
    assert torch.isnan(y.view(-1)[nan]).all()
    assert torch.equal(y.view(-1)[~nan], bf(ref[~nan]).float())


# ------------------------------------------------------------------ GEMV
@pytest.mark.parametrize("N,K", [(256, 384), (9216, 2560), (2560, 9216), (32, 2560), (2560, 4096),
                                 (200, 1000), (1, 128)])
@pytest.mark.parametrize("mode", ["block", "row", "row_block"])
def test_gemv_fp32_scales(N, K, mode):
    g = gen(N * 7 + K)
    W = randn(g, N, K, std=0.02)
    if K % 128 and mode != "row":
        pytest.skip("block scales need K % 128 == 0")
    if mode == "block":
        w, s = orc.quantize_block_fp8(W)
    elif mode == "row":
        amax = W.abs().amax(1, keepdim=True)
        s = (amax / 448).clamp(min=1e-12)
        w = (W / s).to(torch.float8_e4m3fn).view(torch.uint8)
        s = s.view(N)
    else:
        kb = K // 128
        blk = W.view(N, kb, 128)
        s = (blk.abs().amax(2) / 448).clamp(min=1e-12)
        w = (blk / s.unsqueeze(2)).to(torch.float8_e4m3fn).view(N, K).view(torch.uint8)
    x = bf(randn(g, K))
    code = orc.scale_code(w, s) if s.dim() == 2 else 1
    ref = orc.linear(x.float(), orc.dequant(w, s, code))
    lib = abi.load()
    y = torch.empty(N, dtype=torch.bfloat16, device=DEV)
    abi.check(lib.qh_gemv_e4m3(abi.ptr(cu(x)), None, None, 1e-6, K, None, None, 1,
                               abi.ptr(cu(w)), abi.ptr(cu(s.float())), abi.ptr(y), N, code,
                               None, None, None, 0, 0, None, None, None, 0, 0,
                               None, None, None, 0, 0, 0, abi.stream_handle()))
    sync()
    assert_close(y, ref, what=f"gemv {N}x{K} {mode}")


# 9216 x 2560, 2560 x 4096 and 4096 x 2560 take the 128-bit paced kernel with
# bf16 scales (5, 2 and 2 row slots per wave); 256 x 384 the generic kernel.
@pytest.mark.parametrize("N,K", [(256, 384), (9216, 2560), (2560, 4096), (4096, 2560)])
def test_gemv_reference_abi_bf16_scales(N, K):
    """launch_gemv_v4_extern / v3 with bf16 scale_inv, via the reference-named wrapper."""
    g = gen(3)
    w, s = quant(g, N, K)
    s16 = s.to(torch.bfloat16)
    x = bf(randn(g, K))
    ref = orc.linear(x.float(), orc.dequant(w, s16.float()))
    y = ops.fp8_linear(cu(x).view(1, 1, K), cu(w), cu(s16))
    sync()
    assert y.shape == (1, 1, N)
    assert_close(y, ref, what="gemv bf16 scales")
    lib = abi.load()
    y3 = torch.empty(N, dtype=torch.bfloat16, device=DEV)
    lib.launch_gemv_v3_extern(abi.ptr(cu(x)), abi.ptr(cu(w)), abi.ptr(cu(s16)), abi.ptr(y3),
                              N, K, K // 128, abi.stream_handle())
    sync()
    assert torch.equal(y3.cpu(), y.view(-1).cpu())


def test_grouped_projections_match_single():
    """launch_linear_in_proj4, launch_fused_qkv and launch_fused_gate_up equal
    separate GEMVs (one launch over concatenated row spaces)."""
    g = gen(11)
    K = 2560
    segs = [quant(g, n, K) for n in (8192, 32, 32, 4096)]
    x = bf(randn(g, K))
    xs = cu(x)
    lib = abi.load()
    ys = [torch.empty(w.shape[0], dtype=torch.bfloat16, device=DEV) for w, _ in segs]
    args = []
    for (w, s), y in zip(segs, ys):
        args += [abi.ptr(cu(w)), abi.ptr(cu(s.to(torch.bfloat16))), abi.ptr(y), w.shape[0], K // 128]
    lib.qh_clear_error()
    lib.launch_linear_in_proj4(abi.ptr(xs), *args, K, abi.stream_handle())
    sync()
    assert abi.last_error() == ""
    for (w, s), y in zip(segs, ys):
        ref = orc.linear(x.float(), orc.dequant(w, s.to(torch.bfloat16).float()))
        assert_close(y, ref, what="in_proj4")
    (wq, sq), (wk, sk), (wv, sv) = [quant(g, n, K) for n in (1024, 256, 256)]
    q, k, v = ops.fused_qkv(xs, cu(wq), cu(sq), cu(wk), cu(sk), cu(wv), cu(sv))
    gg, uu = ops.fused_gate_up(xs, cu(wq), cu(sq.to(torch.bfloat16)), cu(wk), cu(sk.to(torch.bfloat16)))
    sync()
    for y, (w, s) in ((q, (wq, sq)), (k, (wk, sk)), (v, (wv, sv))):
        assert_close(y, orc.linear(x.float(), orc.dequant(w, s)), what="fused_qkv")
    assert_close(gg, orc.linear(x.float(), orc.dequant(wq, sq.to(torch.bfloat16).float())), what="gate")
    assert_close(uu, orc.linear(x.float(), orc.dequant(wk, sk.to(torch.bfloat16).float())), what="up")


# The first three take the 128-bit paced kernel (2, 2 and 7 row slots per
# wave); 16384 x 2560 (8 slots per wave) falls back to the register pipeline.
@pytest.mark.parametrize("N,K", [(2560, 2560), (2560, 9216), (12352, 2560), (16384, 2560)])
def test_gemv_norm_prologue_and_residual_epilogue(N, K):
    g = gen(5)
    w, s = quant(g, N, K)
    x = bf(randn(g, K))
    nw = randn(g, K, std=0.02)
    res = bf(randn(g, N))
    lib = abi.load()
    y = torch.empty(N, dtype=torch.bfloat16, device=DEV)
    abi.check(lib.qh_gemv_e4m3(abi.ptr(cu(x)), None, abi.ptr(cu(nw)), 1e-6, K, abi.ptr(cu(res)),
                               None, 1, abi.ptr(cu(w)), abi.ptr(cu(s)), abi.ptr(y), N, K // 128,
                               None, None, None, 0, 0, None, None, None, 0, 0,
                               None, None, None, 0, 0, 0, abi.stream_handle()))
    sync()
    xn = orc.rmsnorm(x.float(), nw)
    ref = orc.bf16(res.float() + orc.linear(xn, orc.dequant(w, s)))
    assert_close(y, ref, atol_frac=1e-3, what="norm+gemv+res")


# The 128-bit paced kernels take every K % 512 == 0 up to 9216 (KC = 1..9 one-KB
# chunks per row, a half chunk when K % 1024 == 512) with 2, 5 or 7 row slots
# per wave: 1, 33 and 50 rows per CU on a 256-CU part exercise each slot count,
# with the (1+w) norm prologue and the residual epilogue.
@pytest.mark.parametrize("K", [512, 1536, 2048, 3072, 4608, 6144, 8192, 9216])
@pytest.mark.parametrize("rows_per_cu", [1, 33, 50])
def test_gemv_b128_chunk_counts_and_slots(K, rows_per_cu):
    g = gen(K + rows_per_cu)
    N = rows_per_cu * 256 + 3
    w, s = quant(g, N, K)
    x = bf(randn(g, K))
    nw = randn(g, K, std=0.02)
    res = bf(randn(g, N))
    lib = abi.load()
    y = torch.empty(N, dtype=torch.bfloat16, device=DEV)
    abi.check(lib.qh_gemv_e4m3(abi.ptr(cu(x)), None, abi.ptr(cu(nw)), 1e-6, K, abi.ptr(cu(res)),
                               None, 1, abi.ptr(cu(w)), abi.ptr(cu(s)), abi.ptr(y), N, K // 128,
                               None, None, None, 0, 0, None, None, None, 0, 0,
                               None, None, None, 0, 0, 0, abi.stream_handle()))
    sync()
    xn = orc.rmsnorm(x.float(), nw)
    ref = orc.bf16(res.float() + orc.linear(xn, orc.dequant(w, s)))
    assert_close(y, ref, atol_frac=1e-3, what=f"b128 gemv {N}x{K}")


def test_gemv_rejects_bad_args(lib):
    y = torch.empty(8, dtype=torch.bfloat16, device=DEV)
    rc = lib.qh_gemv_e4m3(None, None, None, 1e-6, 100, None, None, 1, None, None, abi.ptr(y), 8, 1,
                          None, None, None, 0, 0, None, None, None, 0, 0, None, None, None, 0, 0,
                          0, abi.stream_handle())
    assert rc != 0 and "multiple of 8" in abi.last_error()


# ------------------------------------------------------------------ norm
def test_rmsnorm_reference_abi():
    g = gen(7)
    for N, D in ((1, 2560), (16, 256), (4, 256)):
        x = bf(randn(g, N, D) * 3)
        w = randn(g, D, std=0.02)
        ref = orc.rmsnorm(x.float(), w)
        xg = cu(x)
        out = torch.empty_like(xg)
        lib = abi.load()
        lib.launch_rmsnorm_out(abi.ptr(xg), abi.ptr(cu(w)), abi.ptr(out), N, D, 1e-6, abi.stream_handle())
        lib.launch_rmsnorm_ip(abi.ptr(xg), abi.ptr(cu(w)), N, D, 1e-6, abi.stream_handle())
        sync()
        assert_close(out, ref, what="rmsnorm_out")
        assert torch.equal(xg.cpu(), out.cpu())


@pytest.mark.parametrize("M,D", [(128, 2560), (3, 256), (5, 8192), (7, 1000), (4, 100)])
def test_add_rmsnorm(M, D):
    """qh_add_rmsnorm (the batch prefill's residual add + (1+w) RMSNorm after
    every output projection): h = bf16(h + o) bit for bit, out against the
    oracle's rmsnorm of that sum.  D = 2560 / 256 / 8192 / 1000 take the 16-byte
    vector kernel (1, 2 or 4 vectors per thread, a partial last vector row);
    D = 100 (not a multiple of 8) the scalar fallback."""
    g = gen(M * 31 + D)
    h = bf(randn(g, M, D) * 2)
    o = bf(randn(g, M, D))
    w = randn(g, D, std=0.02)
    want_h = bf(h.float() + o.float())
    ref = orc.rmsnorm(want_h.float(), w)
    hg, og, wg = cu(h), cu(o), cu(w)
    out = torch.empty_like(hg)
    lib = abi.load()
    abi.check(lib.qh_add_rmsnorm(abi.ptr(hg), abi.ptr(og), abi.ptr(wg), abi.ptr(out), M, D, 1e-6,
                                 abi.stream_handle()), "add_rmsnorm")
    sync()
    assert torch.equal(hg.cpu(), want_h), "residual sum differs from the bf16 add"
    assert_close(out, ref, what="add_rmsnorm")
    # the plain norm on the same rows goes through the same kernel (o = null)
    out2 = torch.empty_like(hg)
    abi.check(lib.qh_rmsnorm(abi.ptr(hg), abi.ptr(wg), abi.ptr(out2), M, D, 1e-6, abi.stream_handle()),
              "rmsnorm")
    sync()
    assert torch.equal(out2.cpu(), out.cpu())


# ------------------------------------------------------------------ MLP
# (2560, 16384): 64 gate/up pairs per CU, more than the 128-bit paced kernel's
# 7 per wave, so the register pipeline runs gate/up, and down (K = 16384) the
# generic kernel.
@pytest.mark.parametrize("H,I", [(2560, 9216), (256, 512), (2560, 16384)])
def test_mlp_decode(H, I):
    """fused (1+w) RMSNorm -> gate/up SiLU -> down (+residual)."""
    g = gen(2)
    ln = randn(g, H, std=0.02)
    wg, sg = quant(g, I, H)
    wu, su = quant(g, I, H)
    wd, sd = quant(g, H, I)
    h = bf(randn(g, H))
    o = bf(randn(g, H))
    ref, mref = orc.mlp_decode(h.float(), o.float(), ln, orc.dequant(wg, sg), orc.dequant(wu, su),
                               orc.dequant(wd, sd))
    lib = abi.load()
    m = torch.empty(I, dtype=torch.bfloat16, device=DEV)
    out = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    abi.check(lib.qh_mlp_decode(abi.ptr(cu(h)), abi.ptr(cu(o)), abi.ptr(cu(ln)), 1e-6, H,
                                abi.ptr(cu(wg)), abi.ptr(cu(sg)), abi.ptr(cu(wu)), abi.ptr(cu(su)), I,
                                H // 128, abi.ptr(cu(wd)), abi.ptr(cu(sd)), I // 128, abi.ptr(m),
                                abi.ptr(out), 0, abi.stream_handle()))
    sync()
    assert_close(m, mref, atol_frac=1e-3, what="mlp m")
    assert_close(out, ref, atol_frac=1e-3, what="mlp out")


def test_layer_post_o_fp8_mlp_reference_abi():
    g = gen(9)
    H, I = 2560, 9216
    ln = randn(g, H, std=0.02)
    (wg, sg), (wu, su), (wd, sd) = quant(g, I, H), quant(g, I, H), quant(g, H, I)
    sg, su, sd = (s.to(torch.bfloat16) for s in (sg, su, sd))
    h, o = bf(randn(g, H)), bf(randn(g, H))
    ref, mref = orc.mlp_decode(h.float(), o.float(), ln, orc.dequant(wg, sg.float()),
                               orc.dequant(wu, su.float()), orc.dequant(wd, sd.float()))
    bufs = [torch.empty(n, dtype=torch.bfloat16, device=DEV) for n in (H, I, I, I, I)]
    out, ws, gb, ub, sb = bufs
    lib = abi.load()
    lib.launch_rmsnorm_ip  # noqa: B018  (symbol present)
    lib.layer_post_o_fp8_mlp(abi.ptr(cu(h)), abi.ptr(cu(o)), abi.ptr(cu(ln)), abi.ptr(cu(wg)),
                             abi.ptr(cu(sg)), I, abi.ptr(cu(wu)), abi.ptr(cu(su)), I, abi.ptr(cu(wd)),
                             abi.ptr(cu(sd)), H, abi.ptr(out), abi.ptr(ws), abi.ptr(gb), abi.ptr(ub),
                             abi.ptr(sb), H, H // 128, I // 128, abi.stream_handle())
    sync()
    assert abi.last_error() == ""
    assert_close(sb, mref, atol_frac=1e-3, what="silu_buf")
    assert_close(out, ref, atol_frac=1e-3, what="post_o_mlp")


# ------------------------------------------------------------------ attention
def _attn_case(g, ctx, Hq=16, Hkv=4, D=256, rot=64, max_seq=None):
    max_seq = max_seq or ctx
    kc = bf(randn(g, Hkv, max_seq, D)).float()
    vc = bf(randn(g, Hkv, max_seq, D)).float()
    q_all = bf(randn(g, Hq * 2 * D))
    k_new = bf(randn(g, Hkv * D))
    v_new = bf(randn(g, Hkv * D))
    qn = randn(g, D, std=0.02)
    kn = randn(g, D, std=0.02)
    return kc, vc, q_all, k_new, v_new, qn, kn


# (4096, 64), (2049, 64), (300, 64): the engine's split count for a 4096-slot
# cache (engine.default_attn_splits).  Above 8 active splits the merge runs in
# two levels (groups of 8, then the group records): 4096/64 has 8 full groups,
# 2049/64 33 active splits (a last group of 1), 300/64 and 427/32 10 and 14
# (8 + 2, 8 + 6), 288/64 9 (8 + 1), 512/64 16 (8 + 8), 545/64 18 (8 + 8 + 2).
@pytest.mark.parametrize("ctx,splits", [(1, 1), (17, 1), (130, 4), (4096, 32), (427, 32),
                                        (4096, 64), (2049, 64), (300, 64), (288, 64), (512, 64),
                                        (545, 64)])
def test_attn_decode(ctx, splits):
    """BASELINE config 4b (ctx 4096): q/k norm, partial RoPE (theta 1e7, 64 of
    256 dims), KV write at slot ctx-1, GQA 16/4, sigmoid gate."""
    _check_attn_decode(ctx, splits, 16, 4)


# Groups of 5..8 query heads per KV head run the two-heads-per-wave form of
# the kernel (a wave holds two query heads' q and P.V accumulators).
@pytest.mark.parametrize("Hq,Hkv,ctx,splits", [(8, 1, 700, 16), (16, 2, 4096, 64), (6, 1, 300, 8),
                                               (12, 2, 129, 4), (5, 1, 33, 2)])
def test_attn_decode_group_sizes(Hq, Hkv, ctx, splits):
    _check_attn_decode(ctx, splits, Hq, Hkv)


def _check_attn_decode(ctx, splits, Hq, Hkv):
    g = gen(ctx + 1000 * Hq + Hkv)
    D, rot, max_seq = 256, 64, 4096
    kc, vc, q_all, k_new, v_new, qn, kn = _attn_case(g, ctx, Hq=Hq, Hkv=Hkv, max_seq=max_seq)
    # Cache rows past the context hold NaN: no split may read a row it does
    # not own into the result.
    kc[:, ctx:] = float("nan")
    vc[:, ctx:] = float("nan")
    # Tables built on the device, as the reference builds them (main.py:527-533)
    # and the engine does; the oracle reads the same values (host-built ones
    # can differ in the last bit at large angles).
    gcos, gsin = eng_mod.rope_tables(max_seq, rot, 1e7, device=DEV)
    cos, sin = gcos.cpu(), gsin.cpu()
    pos = ctx - 1
    kc_ref, vc_ref = kc.clone(), vc.clone()
    ref = orc.attn_decode(q_all.float(), k_new.float(), v_new.float(), qn, kn, cos, sin, kc_ref,
                          vc_ref, pos, Hq, Hkv, D, rot)
    lib = abi.load()
    kcg, vcg = cu(bf(kc)), cu(bf(vc))
    out = torch.empty(Hq * D, dtype=torch.bfloat16, device=DEV)
    scratch = torch.zeros(int(lib.qh_attn_scratch_bytes(Hkv, splits, D)) + 4, dtype=torch.uint8, device=DEV)
    counters = torch.zeros(Hkv, dtype=torch.int32, device=DEV)
    posd = torch.tensor([pos], dtype=torch.int32, device=DEV)
    qa = cu(q_all)
    for use_dev_pos in (True, False):
        abi.check(lib.qh_attn_decode(abi.ptr(qa), 2 * D, abi.ptr(qa[D:]), 2 * D, abi.ptr(cu(k_new)),
                                     abi.ptr(cu(v_new)), abi.ptr(cu(qn)), abi.ptr(cu(kn)), abi.ptr(gcos),
                                     abi.ptr(gsin), abi.ptr(kcg), abi.ptr(vcg), max_seq, D, rot, Hq, Hkv,
                                     abi.ptr(posd) if use_dev_pos else None, pos, splits,
                                     abi.ptr(scratch), abi.ptr(counters), abi.ptr(out), 1e-6,
                                     abi.stream_handle()))
        sync()
        assert_close(out, ref, atol_frac=1e-3,
                     what=f"attn {Hq}/{Hkv} ctx={ctx} splits={splits} dev_pos={use_dev_pos}")
        assert torch.equal(kcg[:, pos].cpu().float(), kc_ref[:, pos]), "K cache slot"
        assert torch.equal(vcg[:, pos].cpu().float(), vc_ref[:, pos]), "V cache slot"
        assert int(counters.abs().sum()) == 0, "arrival counters must self-reset"
        # the two-level merge's group counters open the scratch ([Hkv][8] words)
        assert int(scratch[:Hkv * 8 * 4].abs().sum()) == 0, "group counters must self-reset"


def test_layer_mid_attn_reference_abi():
    g = gen(21)
    Hq, Hkv, D, rot, max_seq, past = 16, 4, 256, 64, 512, 99
    kc, vc, q_all, k_new, v_new, qn, kn = _attn_case(g, past + 1, max_seq=max_seq)
    cos, sin = orc.rope_tables(max_seq, rot, 1e7)
    q = q_all.float().view(Hq, 2 * D)[:, :D].reshape(-1)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    qr = orc.rope_rows(orc.rmsnorm(q.view(Hq, D), qn), cos[past], sin[past], rot, True)
    kr = orc.rope_rows(orc.rmsnorm(k_new.float().view(Hkv, D), kn), cos[past], sin[past], rot, True)
    kc_ref[:, past] = kr
    vc_ref[:, past] = v_new.float().view(Hkv, D)
    ref = orc.attn_only(qr, kc_ref, vc_ref, past + 1, Hq, Hkv)
    lib = abi.load()
    qb, kb = cu(bf(q)), cu(k_new)
    kcg, vcg = cu(bf(kc)), cu(bf(vc))
    out = torch.empty(Hq * D, dtype=torch.bfloat16, device=DEV)
    lib.layer_mid_attn(abi.ptr(qb), abi.ptr(kb), abi.ptr(cu(v_new)), abi.ptr(out), abi.ptr(cu(qn)),
                       abi.ptr(cu(kn)), abi.ptr(cu(cos)), abi.ptr(cu(sin)), abi.ptr(kcg), abi.ptr(vcg),
                       past, past, past + 1, max_seq, D, rot, Hq, Hkv, abi.stream_handle())
    sync()
    assert abi.last_error() == ""
    assert_close(out, ref, atol_frac=1e-3, what="layer_mid_attn")
    assert torch.equal(qb.cpu().float().view(Hq, D), qr), "q written back normalised + rotated"
    assert torch.equal(kb.cpu().float().view(Hkv, D), kr)
    # launch_fused_attn_v2 on the updated cache with the rotated q
    out2 = torch.empty_like(out)
    lib.launch_fused_attn_v2(abi.ptr(qb), abi.ptr(kcg), abi.ptr(vcg), abi.ptr(out2), past + 1, max_seq,
                             D, Hq, Hkv, abi.stream_handle())
    sync()
    assert_close(out2, ref, atol_frac=1e-3, what="fused_attn_v2")


# ------------------------------------------------------------------ GDN
def _gdn_inputs(g, Hk=16, Hv=32, dk=128, dv=128):
    C = 2 * Hk * dk + Hv * dv
    return dict(
        mixed=bf(randn(g, C)), a=bf(randn(g, Hv)), b=bf(randn(g, Hv)), z=bf(randn(g, Hv * dv)),
        conv_state=bf(randn(g, C, 4, std=1.0)), conv_w=bf(randn(g, C, 4, std=0.5)),
        A_log=torch.log(1e-3 + torch.rand(Hv, generator=g) * 16), dt_bias=torch.ones(Hv),
        norm_w=bf(1 + randn(g, dv, std=0.02)), S=randn(g, Hv, dk, dv, std=0.1))


def _ring_from_ordered(state, t):
    """Ordered conv state [C, 4] (oldest..newest = x_{t-4..t-1}) -> ring with
    slot j holding x_j mod 4."""
    ring = torch.empty_like(state)
    for i in range(4):
        ring[:, (t - 4 + i) % 4] = state[:, i]
    return ring


@pytest.mark.parametrize("t", [7, 4096])
def test_gdn_decode(t):
    """BASELINE config 4a: conv update + gates + l2norm + delta rule + gated RMSNorm."""
    g = gen(t)
    Hk, Hv, dk, dv = 16, 32, 128, 128
    d = _gdn_inputs(g, Hk, Hv, dk, dv)
    kd = Hk * dk
    st = d["conv_state"].float().clone()
    y = orc.conv_update(d["mixed"].float(), st, d["conv_w"].float())
    q = y[:kd].view(Hk, dk).repeat_interleave(2, 0)
    k = y[kd:2 * kd].view(Hk, dk).repeat_interleave(2, 0)
    v = y[2 * kd:].view(Hv, dv)
    gg, beta = orc.linear_gates(d["a"].float(), d["b"].float(), d["A_log"], d["dt_bias"])
    S = d["S"].clone()
    core = orc.delta_rule_step(q, k, v, gg, beta, S)
    ref = orc.gated_rmsnorm(core, d["z"].float().view(Hv, dv), d["norm_w"].float())
    lib = abi.load()
    ring = cu(bf(_ring_from_ordered(d["conv_state"].float(), t)))
    Sg = cu(d["S"])
    coreg = torch.empty(Hv * dv, dtype=torch.float32, device=DEV)
    out = torch.empty(Hv * dv, dtype=torch.bfloat16, device=DEV)
    counters = torch.zeros(Hv, dtype=torch.int32, device=DEV)
    abi.check(lib.qh_gdn_decode(abi.ptr(cu(d["mixed"])), abi.ptr(cu(d["a"])), abi.ptr(cu(d["b"])),
                                abi.ptr(cu(d["z"])), abi.ptr(ring), abi.ptr(cu(d["conv_w"])),
                                abi.ptr(cu(d["A_log"])), abi.ptr(cu(d["dt_bias"])), abi.ptr(cu(d["norm_w"])),
                                abi.ptr(Sg), abi.ptr(coreg), abi.ptr(out), abi.ptr(counters), None, t,
                                Hk, Hv, dk, dv, 1e-6, abi.stream_handle()))
    sync()
    assert_close(coreg, core, atol_frac=1e-3, what="gdn core")
    assert_close(out, ref, atol_frac=2e-3, what="gdn gated out")
    c = cos_sim(Sg.cpu(), S)
    assert c > 0.999999, f"state cosine {c}"
    assert torch.allclose(Sg.cpu(), S, rtol=1e-4, atol=1e-5)
    assert torch.equal(ring.cpu().float(), _ring_from_ordered(st, t + 1)), "conv ring update"
    assert int(counters.abs().sum()) == 0


@pytest.mark.parametrize("t", [7, 4096])
def test_gdn_decode_core_and_gated_out_proj(t):
    """The split decode step: qh_gdn_decode_core (one wave per head and 8
    columns, bf16 core, conv ring and state updated) against the oracle, then
    qh_gemv_e4m3_gated (gated RMSNorm prologue + out_proj + residual) against
    the oracle from the GPU's own core."""
    g = gen(t + 5)
    Hk, Hv, dk, dv, H = 16, 32, 128, 128, 2560
    d = _gdn_inputs(g, Hk, Hv, dk, dv)
    kd = Hk * dk
    st = d["conv_state"].float().clone()
    y = orc.conv_update(d["mixed"].float(), st, d["conv_w"].float())
    q = y[:kd].view(Hk, dk).repeat_interleave(2, 0)
    k = y[kd:2 * kd].view(Hk, dk).repeat_interleave(2, 0)
    v = y[2 * kd:].view(Hv, dv)
    gg, beta = orc.linear_gates(d["a"].float(), d["b"].float(), d["A_log"], d["dt_bias"])
    S = d["S"].clone()
    core = orc.delta_rule_step(q, k, v, gg, beta, S)
    lib = abi.load()
    ring = cu(bf(_ring_from_ordered(d["conv_state"].float(), t)))
    Sg = cu(d["S"])
    coreg = torch.empty(Hv * dv, dtype=torch.bfloat16, device=DEV)
    abi.check(lib.qh_gdn_decode_core(abi.ptr(cu(d["mixed"])), abi.ptr(cu(d["a"])), abi.ptr(cu(d["b"])),
                                     abi.ptr(ring), abi.ptr(cu(d["conv_w"])), abi.ptr(cu(d["A_log"])),
                                     abi.ptr(cu(d["dt_bias"])), abi.ptr(Sg), abi.ptr(coreg), None, t,
                                     Hk, Hv, dk, dv, abi.stream_handle()), "gdn_core")
    sync()
    assert_close(coreg, orc.bf16(core.reshape(-1)), atol_frac=1e-3, what="gdn core (bf16)")
    c = cos_sim(Sg.cpu(), S)
    assert c > 0.999999, f"state cosine {c}"
    assert torch.allclose(Sg.cpu(), S, rtol=1e-4, atol=1e-5)
    assert torch.equal(ring.cpu().float(), _ring_from_ordered(st, t + 1)), "conv ring update"
    # out_proj with the gated RMSNorm prologue and the residual
    wo, so = quant(g, H, Hv * dv)
    h = bf(randn(g, H))
    h2 = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    dwo, dso = cu(wo), cu(so)
    abi.check(lib.qh_gemv_e4m3_gated(abi.ptr(coreg), abi.ptr(cu(d["z"])), abi.ptr(cu(d["norm_w"])), dv,
                                     1e-6, Hv * dv, abi.ptr(cu(h)), abi.ptr(dwo), abi.ptr(dso),
                                     abi.ptr(h2), H, ops.scale_mode(dwo, dso), 0,
                                     abi.stream_handle()), "gemv_gated")
    sync()
    gated = orc.gated_rmsnorm(coreg.cpu().float().view(Hv, dv), d["z"].float().view(Hv, dv),
                              d["norm_w"].float())
    ref = orc.bf16(h.float() + orc.linear(gated.reshape(-1), orc.dequant(wo, so)))
    assert_close(h2, ref, atol_frac=1e-3, what="gated out_proj + residual")


def test_delta_rule_and_gates_reference_abi():
    g = gen(31)
    H, hd = 32, 128
    q, k, v = bf(randn(g, H, hd)), bf(randn(g, H, hd)), bf(randn(g, H, hd))
    a, b = bf(randn(g, H)), bf(randn(g, H))
    A_log = torch.log(1e-3 + torch.rand(H, generator=g) * 16)
    dt = torch.ones(H)
    gg, beta = orc.linear_gates(a.float(), b.float(), A_log, dt)
    S = randn(g, H, hd, hd, std=0.1)
    Sr = S.clone()
    ref = orc.delta_rule_step(q.float(), k.float(), v.float(), gg, beta, Sr)
    lib = abi.load()
    gd = torch.empty(H, device=DEV)
    bd = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    lib.launch_prepare_linear_gates(abi.ptr(cu(a)), abi.ptr(cu(b)), abi.ptr(cu(A_log)), abi.ptr(cu(dt)),
                                    abi.ptr(gd), abi.ptr(bd), H, abi.stream_handle())
    Sg = cu(S)
    out = torch.empty(H * hd, dtype=torch.bfloat16, device=DEV)
    lib.launch_delta_rule_decode(abi.ptr(cu(q)), abi.ptr(cu(k)), abi.ptr(cu(v)), abi.ptr(gd), abi.ptr(bd),
                                 abi.ptr(Sg), abi.ptr(out), H, hd, abi.stream_handle())
    z = bf(randn(g, H * hd))
    w = bf(1 + randn(g, hd, std=0.02))
    gated = torch.empty_like(out)
    lib.launch_rmsnorm_gated_decode(abi.ptr(out), abi.ptr(cu(z)), abi.ptr(cu(w)), abi.ptr(gated), H, hd,
                                    1e-6, abi.stream_handle())
    sync()
    assert abi.last_error() == ""
    assert torch.allclose(gd.cpu(), gg, rtol=1e-5, atol=1e-6)
    assert torch.equal(bd.cpu().float(), beta)
    assert_close(out, ref, atol_frac=1e-3, what="delta rule")
    assert torch.allclose(Sg.cpu(), Sr, rtol=1e-4, atol=1e-5)
    gref = orc.gated_rmsnorm(out.cpu().float().view(H, hd), z.float().view(H, hd), w.float(), bf16_steps=False)
    assert_close(gated, gref, atol_frac=1e-3, what="rmsnorm_gated_decode")


# ------------------------------------------------------------------ lm_head
@pytest.mark.parametrize("nbytes,n_out", [(16, 512), (4096 * 3 + 48, 512), (10 * 2 ** 20 + 16 * 7, 512),
                                          (2560 * 9216, 512), (2560 * 9216, 3), (2560 * 9216, 256),
                                          (12352 * 2560, 1024), (12352 * 2560, 4096)])
def test_read_stream_reads_every_word_once(nbytes, n_out):
    """qh_read_stream (the measured read floor): the XOR of its per-workgroup
    checksums equals the XOR of all 32-bit words of the buffer, so every word
    is read exactly once, whatever the size and grid; workgroups past the grid
    leave their output words untouched."""
    g = gen(nbytes % 1000 + n_out)
    words = torch.randint(-2 ** 31, 2 ** 31, (nbytes // 4,), generator=g, dtype=torch.int64).to(torch.int32)
    src = words.to(DEV)
    out = torch.full((n_out + 1,), 0x5A5A5A5A, dtype=torch.int32, device=DEV)
    lib = abi.load()
    abi.check(lib.qh_read_stream(abi.ptr(src), nbytes, abi.ptr(out), n_out, abi.stream_handle()), "read_stream")
    sync()
    got = out.cpu()
    grid = min(n_out, 4 * torch.cuda.get_device_properties(0).multi_processor_count)
    expect = int(np.bitwise_xor.reduce(words.numpy().view(np.uint32)))
    have = int(np.bitwise_xor.reduce(got[:grid].numpy().view(np.uint32)))
    assert have == expect
    assert (got[grid:] == 0x5A5A5A5A).all()


@pytest.mark.parametrize("V,K", [(1000, 256), (248320, 2560)])
def test_lm_head_argmax(V, K):
    g = gen(V)
    W = bf(randn(g, V, K, std=0.02))
    h = bf(randn(g, K) * 4)
    nf = randn(g, K, std=0.02)
    logits_ref, tok_ref = orc.lm_head_argmax(h.float(), nf, W.float())
    lib = abi.load()
    logits = torch.empty(V, dtype=torch.bfloat16, device=DEV)
    scratch = torch.zeros(int(lib.qh_lm_head_scratch_bytes(V)), dtype=torch.uint8, device=DEV)
    counter = torch.zeros(1, dtype=torch.int32, device=DEV)
    tok = torch.zeros(1, dtype=torch.int64, device=DEV)
    hist = torch.full((8,), -1, dtype=torch.int64, device=DEV)
    pos = torch.tensor([3], dtype=torch.int32, device=DEV)
    emb = cu(W)
    nxt = torch.empty(K, dtype=torch.bfloat16, device=DEV)
    for rep in range(2):
        abi.check(lib.qh_lm_head_argmax(abi.ptr(cu(h)), abi.ptr(cu(nf)), 1e-6, K, abi.ptr(cu(W)), V,
                                        abi.ptr(logits), abi.ptr(scratch), abi.ptr(counter), abi.ptr(tok),
                                        abi.ptr(hist), 8, abi.ptr(pos), abi.ptr(emb), abi.ptr(nxt),
                                        abi.stream_handle()))
    sync()
    assert_close(logits, logits_ref, atol_frac=1e-3, what="logits")
    got = int(tok.item())
    lg = logits.cpu().float()
    assert got == orc.argmax_first(lg), "argmax of the GPU's own bf16 logits"
    if got != tok_ref:  # only allowed on a bf16 near-tie
        assert abs(float(logits_ref[got]) - float(logits_ref[tok_ref])) <= 2 ** -7 * abs(float(logits_ref[tok_ref]))
    assert int(pos.item()) == 5 and int(hist[3]) == got and int(hist[4]) == got
    assert torch.equal(nxt.cpu(), W[got])
    assert int(counter.item()) == 0


def test_argmax_ties_lowest_index():
    V, K = 4096, 128
    W = torch.zeros(V, K, dtype=torch.bfloat16)
    for r in (4000, 77, 2048, 3999):
        W[r, 0] = 1.0
    h = torch.zeros(K, dtype=torch.bfloat16)
    h[0] = 1.0
    lib = abi.load()
    logits = torch.empty(V, dtype=torch.bfloat16, device=DEV)
    scratch = torch.zeros(int(lib.qh_lm_head_scratch_bytes(V)), dtype=torch.uint8, device=DEV)
    counter = torch.zeros(1, dtype=torch.int32, device=DEV)
    tok = torch.zeros(1, dtype=torch.int64, device=DEV)
    abi.check(lib.qh_lm_head_argmax(abi.ptr(cu(h)), None, 1e-6, K, abi.ptr(cu(W)), V, abi.ptr(logits),
                                    abi.ptr(scratch), abi.ptr(counter), abi.ptr(tok), None, 0, None, None,
                                    None, abi.stream_handle()))
    sync()
    assert int(tok.item()) == 77


def test_argmax_nan_logits_stay_in_bounds():
    """Regression: all-NaN logits once left the argmax at its INT_MAX sentinel
    and the next-token embedding copy read far out of bounds.  NaN now ranks
    highest (torch.argmax order) and the index is clamped into the vocabulary."""
    V, K = 1000, 128
    W = torch.ones(V, K, dtype=torch.bfloat16)
    W[5:, 0] = float("nan")
    h = torch.ones(K, dtype=torch.bfloat16)
    lib = abi.load()
    logits = torch.empty(V, dtype=torch.bfloat16, device=DEV)
    scratch = torch.zeros(int(lib.qh_lm_head_scratch_bytes(V)), dtype=torch.uint8, device=DEV)
    counter = torch.zeros(1, dtype=torch.int32, device=DEV)
    tok = torch.zeros(1, dtype=torch.int64, device=DEV)
    emb, nxt = cu(W), torch.empty(K, dtype=torch.bfloat16, device=DEV)
    abi.check(lib.qh_lm_head_argmax(abi.ptr(cu(h)), None, 1e-6, K, abi.ptr(emb), V, abi.ptr(logits),
                                    abi.ptr(scratch), abi.ptr(counter), abi.ptr(tok), None, 0, None,
                                    abi.ptr(emb), abi.ptr(nxt), abi.stream_handle()))
    sync()
    assert int(tok.item()) == 5


# ------------------------------------------------------------------ prefill GEMM
# Every shape runs the persistent ring kernel, on the plan its cost model
# picks (tile shape, workgroups per CU, K slices):
# - (512, 9216, 2560) and (512, 2560, 9216): config 3a, 64 x 64 tiles (with a
#   workspace the second splits K in 2);
# - (5, 256, 384) an odd K-block count; (130, 200, 256), (2000, 4100, 384)
#   ragged M and N (rows past M / N read as zeros);
# - (700, 9000, 2560), (200, 12352, 384): 64 x 128 tiles; (300, 2560, 2560)
#   with a workspace: 64 x 128 tiles, K split in 4;
# - (1100, 9000, 384), (1500, 3000, 2560): 128 x 192 tiles, the second in
#   groups of 2 row tiles; (2200, 1000, 4096): 64 x 64 tiles in groups of 3
#   row tiles (35 = 11 x 3 + 2);
# - with a workspace, (128, 2560, 4096), (37, 1000, 9216) and (128, 32, 2560)
#   split K in 8, 8 and 5 (split-K items + reduction).
@pytest.mark.parametrize("M,N,K", [(512, 9216, 2560), (512, 2560, 9216), (5, 256, 384), (130, 200, 256),
                                   (700, 9000, 2560), (2000, 4100, 384), (2048, 4160, 1024),
                                   (1100, 9000, 384), (128, 2560, 4096), (37, 1000, 9216), (128, 32, 2560),
                                   (200, 12352, 384), (300, 2560, 2560), (1500, 3000, 2560), (2200, 1000, 4096)])
def test_gemm_e4m3(M, N, K):
    """BASELINE config 3a: X bf16 [M, K] . deq(W)^T through the fp8 matrix cores."""
    g = gen(M + N + K)
    w, s = quant(g, N, K)
    x = bf(randn(g, M, K))
    ref = x.float() @ orc.dequant(w, s).t()
    y = ops.fp8_linear(cu(x), cu(w), cu(s))
    sync()
    c = cos_sim(y.cpu().float(), ref)
    assert c >= 0.99999, f"gemm cosine {c}"
    assert_close(y, orc.bf16(ref), rtol=2e-2, atol_frac=5e-3, min_cos=0.99999, what="gemm")
    y16 = ops.fp8_linear(cu(x), cu(w), cu(s.to(torch.bfloat16)))   # bf16 scales: fp8_gemm_batch
    sync()
    ref16 = x.float() @ orc.dequant(w, s.to(torch.bfloat16).float()).t()
    assert cos_sim(y16.cpu().float(), ref16) >= 0.99999
    lib = abi.load()
    ws = torch.empty(int(lib.qh_gemm_workspace_size(M, K)), dtype=torch.uint8, device=DEV)
    yw = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    abi.check(lib.qh_gemm_e4m3(abi.ptr(cu(x)), abi.ptr(cu(w)), abi.ptr(cu(s)), abi.ptr(yw), M, N, K,
                               K // 128, 0, abi.ptr(ws), ws.numel(), abi.stream_handle()), "gemm with workspace")
    sync()
    assert cos_sim(yw.cpu().float(), ref) >= 0.99999
    assert_close(yw, orc.bf16(ref), rtol=2e-2, atol_frac=5e-3, min_cos=0.99999, what="gemm, workspace")


@pytest.mark.parametrize("M,N,K,norm", [(128, 2560, 4096, True), (128, 2560, 9216, True),
                                         (37, 1000, 9216, False), (512, 2560, 9216, True),
                                         (5, 256, 384, True), (64, 100, 256, True)])
def test_gemm_add_rmsnorm_matches_separate_steps(M, N, K, norm):
    """qh_gemm_e4m3_add_rmsnorm (the batch prefill's output projection +
    residual + norm) against qh_gemm_e4m3 then qh_add_rmsnorm / qh_add_bf16
    with the same workspace, bit for bit.  (128, 2560, 4096 / 9216) and
    (37, 1000, 9216) split K and take the fused split-K finish; (512, 2560,
    9216) is unsplit and (5, 256, 384) too short to split; (64, 100, 256) has
    N % 8 != 0.  The sum is also checked against the fp32 oracle product."""
    g = gen(M + N + K + norm)
    w, s = quant(g, N, K)
    x = bf(randn(g, M, K))
    h0 = bf(randn(g, M, N))
    nw = randn(g, N, std=0.02)
    lib = abi.load()
    ws = torch.empty(int(lib.qh_gemm_workspace_size(M, K)), dtype=torch.uint8, device=DEV)
    dx, dw, ds, dnw = cu(x), cu(w), cu(s), cu(nw)
    # separate steps
    o1 = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    h1 = cu(h0)
    hn1 = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    abi.check(lib.qh_gemm_e4m3(abi.ptr(dx), abi.ptr(dw), abi.ptr(ds), abi.ptr(o1), M, N, K, K // 128, 0,
                               abi.ptr(ws), ws.numel(), abi.stream_handle()), "gemm")
    if norm:
        abi.check(lib.qh_add_rmsnorm(abi.ptr(h1), abi.ptr(o1), abi.ptr(dnw), abi.ptr(hn1), M, N, 1e-6,
                                     abi.stream_handle()), "add_rmsnorm")
    else:
        abi.check(lib.qh_add_bf16(abi.ptr(h1), abi.ptr(o1), abi.ptr(h1), M * N, abi.stream_handle()), "add")
    # fused
    o2 = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    h2 = cu(h0)
    hn2 = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    abi.check(lib.qh_gemm_e4m3_add_rmsnorm(abi.ptr(dx), abi.ptr(dw), abi.ptr(ds), abi.ptr(o2), M, N, K,
                                           K // 128, 0, abi.ptr(h2), abi.ptr(dnw) if norm else None,
                                           abi.ptr(hn2), 1e-6, abi.ptr(ws), ws.numel(), abi.stream_handle()),
              "gemm_add_rmsnorm")
    sync()
    assert torch.equal(h1.cpu(), h2.cpu()), "residual stream differs from the separate steps"
    if norm:
        assert torch.equal(hn1.cpu(), hn2.cpu()), "normed rows differ from the separate steps"
    ref = h0.float() + orc.bf16(x.float() @ orc.dequant(w, s).t()).float()
    assert cos_sim(h2.cpu().float(), ref) >= 0.99999


@pytest.mark.parametrize("M", [128, 37])
def test_gemm_grouped_matches_single_launches(M):
    """qh_gemm_e4m3_grouped (the prefill's in_proj shape: 8192 / 4096 / 32 / 32
    rows of one activation) against one qh_gemm_e4m3 per segment and against
    the fp32 reference.  The two calls may split K differently (the split
    count follows the tile count), so they agree to one bf16 ulp, not bit for
    bit."""
    g = gen(40 + M)
    K, ns = 2560, (8192, 4096, 32, 32)
    x = bf(randn(g, M, K))
    ws_ = [quant(g, n, K) for n in ns]
    lib = abi.load()
    ws = torch.empty(int(lib.qh_gemm_workspace_size(M, K)), dtype=torch.uint8, device=DEV)
    dx = cu(x)
    dw = [(cu(w), cu(s)) for w, s in ws_]
    yg = [torch.empty(M, n, dtype=torch.bfloat16, device=DEV) for n in ns]
    args = []
    for (w, s), y, n in zip(dw, yg, ns):
        args += [abi.ptr(w), abi.ptr(s), abi.ptr(y), n, ops.scale_mode(w, s)]
    abi.check(lib.qh_gemm_e4m3_grouped(abi.ptr(dx), M, K, 4, *args, 0, abi.ptr(ws), ws.numel(),
                                       abi.stream_handle()), "grouped")
    ys = [ops.fp8_linear(dx, w, s) for w, s in dw]
    sync()
    for a, b, (w, s), n in zip(yg, ys, ws_, ns):
        assert_close(a, b, rtol=2 ** -7, atol_frac=1e-6, what=f"grouped vs single, {n} rows")
        ref = x.float() @ orc.dequant(w, s).t()
        assert cos_sim(a.cpu().float(), ref) >= 0.99999


# ------------------------------------------------- reference ABI, called directly
def _ref_kb(w, s):
    """main.py:249-251: the K_blocks code main.py passes for a scale tensor."""
    k_blocks = s.shape[1]
    return -k_blocks if s.shape[0] == w.shape[0] and k_blocks > 1 else k_blocks


@pytest.mark.parametrize("M,N,K,mode", [(40, 2560, 2560, "block"), (7, 1000, 384, "block"),
                                        (33, 256, 1024, "row"), (19, 384, 512, "row_block")])
def test_fp8_gemm_batch_reference_abi(M, N, K, mode):
    """fp8_gemm_batch exactly as main.py:262-269 calls it: bf16 scale_inv, the
    K_blocks code of main.py:249-251, the null stream, no workspace."""
    import ctypes
    g = gen(M * 7 + N + K)
    W = randn(g, N, K, std=0.02)
    if mode == "block":
        w, s = orc.quantize_block_fp8(W)
    elif mode == "row":
        s = (W.abs().amax(dim=1, keepdim=True) / 448.0).clamp(min=1e-12)
        w = (W / s).to(torch.float8_e4m3fn).view(torch.uint8)
    else:
        s = (W.view(N, K // 128, 128).abs().amax(dim=2) / 448.0).clamp(min=1e-12)
        w = (W.view(N, K // 128, 128) / s.unsqueeze(-1)).to(torch.float8_e4m3fn).view(
            torch.uint8).reshape(N, K)
    s16 = s.to(torch.bfloat16)
    x = bf(randn(g, M, K))
    ref = x.float() @ orc.dequant(w, s16.float()).t()
    lib = abi.load()
    dx, dw, ds = cu(x), cu(w.contiguous()), cu(s16.contiguous())
    y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    lib.qh_clear_error()
    lib.fp8_gemm_batch(abi.ptr(dx), abi.ptr(dw), abi.ptr(ds), abi.ptr(y), M, N, K,
                       _ref_kb(w, s16), ctypes.c_void_p(0))
    sync()
    assert abi.last_error() == ""
    c = cos_sim(y.cpu().float(), ref)
    assert c >= 0.99999, f"fp8_gemm_batch cosine {c}"
    assert_close(y, orc.bf16(ref), rtol=2e-2, atol_frac=5e-3, min_cos=0.99999, what="fp8_gemm_batch")


@pytest.mark.parametrize("path", ["fp8_gemm_batch", "qh_gemm_e4m3_ws"])
def test_gemm_activation_outlier_channels(path):
    """Channels 100-3000x larger than the rest sit in the same 32-element runs
    as ordinary values.  Their weight columns are zero, so the output is the
    ordinary channels' product alone: any precision the outliers cost their
    neighbours in the activation split shows up in full."""
    M, N, K = 64, 512, 1024
    g = gen(77)
    w, s = quant(g, N, K)
    cols = torch.tensor([3, 77, 500, 901, 902])
    w = w.clone()
    w[:, cols] = 0                                  # E4M3 +0
    x = randn(g, M, K)
    x[:, cols] = torch.tensor([1000.0, -300.0, 100.0, 3000.0, -1500.0])
    x[::3, 40] = 2000.0                             # row-dependent outliers too
    w[:, 40] = 0
    x = bf(x)
    ref = x.float() @ orc.dequant(w, s).t()
    lib = abi.load()
    dx, dw = cu(x), cu(w)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    if path == "fp8_gemm_batch":
        s16 = s.to(torch.bfloat16)
        ref = x.float() @ orc.dequant(w, s16.float()).t()
        lib.fp8_gemm_batch(abi.ptr(dx), abi.ptr(dw), abi.ptr(cu(s16)), abi.ptr(y), M, N, K, K // 128,
                           abi.stream_handle())
    else:
        ws = torch.empty(int(lib.qh_gemm_workspace_size(M, K)), dtype=torch.uint8, device=DEV)
        abi.check(lib.qh_gemm_e4m3(abi.ptr(dx), abi.ptr(dw), abi.ptr(cu(s)), abi.ptr(y), M, N, K,
                                   K // 128, 0, abi.ptr(ws), ws.numel(), abi.stream_handle()), "gemm")
    sync()
    assert abi.last_error() == ""
    c = cos_sim(y.cpu().float(), ref)
    assert c >= 0.99999, f"{path}: cosine {c} with outlier channels"
    assert_close(y, orc.bf16(ref), rtol=2e-2, atol_frac=5e-3, min_cos=0.99999, what=path)


def test_launch_fused_qkv_reference_abi():
    """launch_fused_qkv with main.py:281-298's arguments: bf16 scale_inv, K_blk =
    s_q.shape[1] and the N_*_blk row-block counts."""
    g = gen(31)
    K, Nq, Nkv = 2560, 8192, 1024
    x = bf(randn(g, K))
    mats = [quant(g, n, K) for n in (Nq, Nkv, Nkv)]
    mats = [(w, s.to(torch.bfloat16)) for w, s in mats]
    refs = [orc.linear(x.float(), orc.dequant(w, s.float())) for w, s in mats]
    lib = abi.load()
    outs = [torch.empty(w.shape[0], dtype=torch.bfloat16, device=DEV) for w, _ in mats]
    (wq, sq), (wk, sk), (wv, sv) = [(cu(w), cu(s)) for w, s in mats]
    lib.qh_clear_error()
    lib.launch_fused_qkv(abi.ptr(cu(x)), abi.ptr(wq), abi.ptr(wk), abi.ptr(wv), abi.ptr(sq),
                         abi.ptr(sk), abi.ptr(sv), *[abi.ptr(o) for o in outs], K, Nq, Nkv, Nkv,
                         sq.shape[1], sq.shape[0], sk.shape[0], sv.shape[0], abi.stream_handle())
    sync()
    assert abi.last_error() == ""
    for o, r, name in zip(outs, refs, "qkv"):
        assert_close(o, r, what=f"launch_fused_qkv {name}")


@pytest.mark.parametrize("D,seq", [(256, 999), (128, 300)])
def test_launch_fused_attn_reference_abi(D, seq):
    """launch_fused_attn (fused_kernels.cu:1027-1043): attention of already
    normalised, rotated query heads over the cache, no cache write."""
    g = gen(D + seq)
    Hq, Hkv, max_seq = 16, 4, 1024
    kc = bf(randn(g, Hkv, max_seq, D)).float()
    vc = bf(randn(g, Hkv, max_seq, D)).float()
    q = bf(randn(g, Hq * D))
    ref = orc.attn_only(q.float(), kc, vc, seq, Hq, Hkv)
    lib = abi.load()
    kcg, vcg = cu(bf(kc)), cu(bf(vc))
    out = torch.empty(Hq * D, dtype=torch.bfloat16, device=DEV)
    lib.qh_clear_error()
    lib.launch_fused_attn(abi.ptr(cu(q)), abi.ptr(kcg), abi.ptr(vcg), abi.ptr(out), seq, max_seq, D,
                          Hq, Hkv, abi.stream_handle())
    sync()
    assert abi.last_error() == ""
    assert_close(out, ref, atol_frac=1e-3, what=f"launch_fused_attn D={D}")
    assert torch.equal(kcg.cpu().float(), kc), "launch_fused_attn must not write the cache"
