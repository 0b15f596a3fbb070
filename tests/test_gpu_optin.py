"""The reference's opt-in fused decode path on this library (MI355X only).

main.py:1263-1361 (QWEN_NATIVE_FP8_FUSED) runs a full-attention layer as
layer_pre_attn -> host-side q/k norm, RoPE, KV write, attention and sigmoid
gate -> layer_post_attn.  Its host code splits layer_pre_attn's q output as
[first half | second half] (main.py:1292-1294) although the checkpoint's
q_proj rows are per-head [q_h | gate_h] (main.py:1001).  With the q/gate head
dim set, this library's layer_pre_attn writes q de-interleaved, and the whole
opt-in layer then matches the oracle's decode layer."""
import pytest
import torch

from oracle import qwen35_oracle as orc
from qwen35_amd import abi

from _util import assert_close, bf, gen, quant, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def cu(t):
    return t.to(DEV).contiguous()


def _bf16_scales(s):
    """The reference converts scale_inv to bf16 at load (main.py:597)."""
    return bf(s)


def _layer(g, hidden=512, inter=1024, H=4, Hkv=2, D=128):
    L = {"H": H, "Hkv": Hkv, "D": D, "hidden": hidden, "inter": inter}
    for name, n, k in (("q", 2 * H * D, hidden), ("k", Hkv * D, hidden), ("v", Hkv * D, hidden),
                       ("o", hidden, H * D), ("g", inter, hidden), ("u", inter, hidden),
                       ("d", hidden, inter)):
        w, s = quant(g, n, k)
        L[name] = (w, _bf16_scales(s))
    L["ln"] = randn(g, hidden, std=0.02)
    L["ln2"] = randn(g, hidden, std=0.02)
    L["qn"] = randn(g, D, std=0.1)
    L["kn"] = randn(g, D, std=0.1)
    return L


def _pre_attn(lib, L, hidden_bf, d):
    H, Hkv, D, hd = L["H"], L["Hkv"], L["D"], L["hidden"]
    (wq, sq), (wk, sk), (wv, sv) = L["q"], L["k"], L["v"]
    q = torch.empty(2 * H * D, dtype=torch.bfloat16, device=DEV)
    k = torch.empty(Hkv * D, dtype=torch.bfloat16, device=DEV)
    v = torch.empty_like(k)
    ws = torch.empty(hd, dtype=torch.bfloat16, device=DEV)
    args = [cu(wq), cu(sq), cu(wk), cu(sk), cu(wv), cu(sv)]
    lib.qh_clear_error()
    assert lib.qh_set_qgate_head_dim(d) == 0
    try:
        lib.layer_pre_attn(abi.ptr(hidden_bf), abi.ptr(cu(L["ln"])), abi.ptr(args[0]), abi.ptr(args[1]),
                           wq.shape[0], sq.shape[1], abi.ptr(args[2]), abi.ptr(args[3]), wk.shape[0],
                           sk.shape[1], abi.ptr(args[4]), abi.ptr(args[5]), wv.shape[0], sv.shape[1],
                           abi.ptr(q), abi.ptr(k), abi.ptr(v), abi.ptr(ws), hd, hd // 128,
                           abi.stream_handle())
        torch.cuda.synchronize()
    finally:
        lib.qh_set_qgate_head_dim(-1)
    assert abi.last_error() == ""
    return q.cpu(), k.cpu(), v.cpu()


def test_layer_pre_attn_qgate_deinterleave():
    g = gen(41)
    L = _layer(g)
    H, D = L["H"], L["D"]
    hidden = bf(randn(g, L["hidden"]))
    lib = abi.load()
    dh = cu(hidden)
    q0, k0, v0 = _pre_attn(lib, L, dh, 0)
    q1, k1, v1 = _pre_attn(lib, L, dh, D)
    # the checkpoint order matches the oracle's projection ...
    hn = orc.rmsnorm(hidden.float(), L["ln"])
    assert_close(q0, orc.linear(hn, orc.dequant(*L["q"])), what="q_proj (checkpoint order)")
    # ... and the de-interleaved output is exactly its [q heads | gate heads] permutation
    assert torch.equal(q1, q0.view(H, 2, D).transpose(0, 1).reshape(-1))
    assert torch.equal(k1, k0) and torch.equal(v1, v0)
    assert lib.qh_set_qgate_head_dim(-2) == -1  # rejected
    assert "qh_set_qgate_head_dim" in abi.last_error()
    lib.qh_clear_error()


def _optin_layer(lib, L, hidden, pos, kc, vc, cos, sin, rot, d):
    """main.py:1263-1361 with this library: returns the layer output (bf16)."""
    H, Hkv, D, hd, inter = L["H"], L["Hkv"], L["D"], L["hidden"], L["inter"]
    dh = cu(hidden)
    q_buf, k_buf, v_buf = _pre_attn(lib, L, dh, d)
    # host side, as main.py:1290-1327 (decode: per-head norm in bf16, RoPE in fp32)
    q = orc.rmsnorm(q_buf[:H * D].float().view(H, D), L["qn"])
    gate = q_buf[H * D:].float()
    k = orc.rmsnorm(k_buf.float().view(Hkv, D), L["kn"])
    q = orc.rope_rows(q, cos[pos], sin[pos], rot, round_out=False)
    k = orc.rope_rows(k, cos[pos], sin[pos], rot, round_out=False)
    kc[:, pos] = orc.bf16(k)
    vc[:, pos] = v_buf.float().view(Hkv, D)
    att = torch.empty(H, D)
    for h in range(H):
        kv = h * Hkv // H
        att[h] = orc.bf16(orc.attn_core(q[h], kc[kv, :pos + 1], vc[kv, :pos + 1]))
    attn_1d = orc.bf16(att.reshape(-1) * orc.bf16(torch.sigmoid(gate)))
    # layer_post_attn: o_proj + residual + norm + gate/up SiLU + down + residual
    (wo, so), (wg, sg), (wu, su), (wd, sd) = L["o"], L["g"], L["u"], L["d"]
    t = {n: cu(x) for n, x in (("wo", wo), ("so", so), ("wg", wg), ("sg", sg), ("wu", wu),
                               ("su", su), ("wd", wd), ("sd", sd), ("ln2", L["ln2"]))}
    out = torch.empty(hd, dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(max(hd, inter), dtype=torch.bfloat16, device=DEV)
    gb, ub, sb = (torch.empty(inter, dtype=torch.bfloat16, device=DEV) for _ in range(3))
    da = cu(bf(attn_1d))
    lib.layer_post_attn(abi.ptr(dh), abi.ptr(da), abi.ptr(t["wo"]), abi.ptr(t["so"]), hd, so.shape[1],
                        abi.ptr(t["ln2"]), abi.ptr(t["wg"]), abi.ptr(t["sg"]), inter, sg.shape[1],
                        abi.ptr(t["wu"]), abi.ptr(t["su"]), inter, su.shape[1], abi.ptr(t["wd"]),
                        abi.ptr(t["sd"]), hd, sd.shape[1], abi.ptr(out), abi.ptr(ws), abi.ptr(gb),
                        abi.ptr(ub), abi.ptr(sb), hd, H * D, so.shape[1], sg.shape[1], sd.shape[1],
                        abi.stream_handle())
    torch.cuda.synchronize()
    assert abi.last_error() == ""
    return out.cpu()


def test_reference_optin_full_attention_layer_matches_oracle():
    g = gen(42)
    L = _layer(g)
    H, Hkv, D = L["H"], L["Hkv"], L["D"]
    rot, max_seq, pos = D // 4, 64, 37
    cos, sin = orc.rope_tables(max_seq, rot, 1e7)
    kc0 = orc.bf16(randn(g, Hkv, max_seq, D))
    vc0 = orc.bf16(randn(g, Hkv, max_seq, D))
    hidden = bf(randn(g, L["hidden"]))
    # oracle: the generic decode layer (main.py:981-1059, 1519-1541)
    hn = orc.rmsnorm(hidden.float(), L["ln"])
    q_all = orc.linear(hn, orc.dequant(*L["q"]))
    k_new = orc.linear(hn, orc.dequant(*L["k"]))
    v_new = orc.linear(hn, orc.dequant(*L["v"]))
    kc, vc = kc0.clone(), vc0.clone()
    att = orc.attn_decode(q_all, k_new, v_new, L["qn"], L["kn"], cos, sin, kc, vc, pos, H, Hkv, D, rot)
    o = orc.linear(att, orc.dequant(*L["o"]))
    ref, _ = orc.mlp_decode(hidden.float(), o, L["ln2"], orc.dequant(*L["g"]), orc.dequant(*L["u"]),
                            orc.dequant(*L["d"]))
    lib = abi.load()
    got = _optin_layer(lib, L, hidden, pos, kc0.clone(), vc0.clone(), cos, sin, rot, D)
    assert_close(got, ref, atol_frac=2e-3, min_cos=0.9999, what="opt-in layer, de-interleaved q/gate")
    # without the de-interleave the reference's split mixes q and gate heads
    bad = _optin_layer(lib, L, hidden, pos, kc0.clone(), vc0.clone(), cos, sin, rot, 0)
    assert (bad.float() - ref.float()).abs().max() > 10 * (got.float() - ref.float()).abs().max()
