"""Chained decode phases (qh_chain) against the same phases launched one by
one (each of which is pinned to the CPU oracle in test_gpu_kernels.py), and
against the oracle directly.  MI355X only."""
import pytest
import torch

from oracle import qwen35_oracle as orc
from qwen35_amd import abi, ops

from _util import assert_close, bf, gen, quant, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, I, KO = 2560, 9216, 4096
SEGS = (8192, 4096, 32, 32)   # in_proj qkv / z / b / a rows


def _layer(seed):
    g = gen(seed)
    d = {
        "mix": bf(randn(g, KO)), "h": bf(randn(g, H)),
        "o": quant(g, H, KO), "gate": quant(g, I, H), "up": quant(g, I, H), "down": quant(g, H, I),
        "ln2": randn(g, H, std=0.02), "ln1": randn(g, H, std=0.02),
        "inp": [quant(g, n, H) for n in SEGS],
    }
    return {k: ([(w.to(DEV), s.to(DEV)) for w, s in v] if k == "inp" else
                (tuple(t.to(DEV) for t in v) if isinstance(v, tuple) else v.to(DEV)))
            for k, v in d.items()}


def _bufs():
    e = lambda n: torch.empty(n, dtype=torch.bfloat16, device=DEV)
    return {"h2": e(H), "m": e(I), "hout": e(H), "ys": [e(n) for n in SEGS]}


def _phases(L, B, h_in):
    return [
        ops.chain_gemv_phase(L["mix"], [(L["o"], B["h2"])], res=h_in),
        ops.chain_mlp_phase(B["h2"], L["ln2"], L["gate"], L["up"], B["m"]),
        ops.chain_gemv_phase(B["m"], [(L["down"], B["hout"])], res=B["h2"]),
        ops.chain_gemv_phase(B["hout"], list(zip(L["inp"], B["ys"])), norm_w=L["ln1"]),
    ]


def _separate(L, B, h_in):
    lib, st = abi.load(), abi.stream_handle()

    def gemv(x, segs, norm_w=None, res=None):
        args = []
        for i in range(4):
            if i < len(segs):
                (w, s), y = segs[i]
                args += [abi.ptr(w), abi.ptr(s), abi.ptr(y), w.shape[0], ops.scale_mode(w, s)]
            else:
                args += [None, None, None, 0, 0]
        abi.check(lib.qh_gemv_e4m3(abi.ptr(x), None, abi.ptr(norm_w), 1e-6, x.numel(),
                                   abi.ptr(res), None, len(segs), *args, 0, st), "gemv")

    gemv(L["mix"], [(L["o"], B["h2"])], res=h_in)
    (wg, sg), (wu, su) = L["gate"], L["up"]
    abi.check(lib.qh_mlp_gate_up(abi.ptr(B["h2"]), None, abi.ptr(L["ln2"]), 1e-6, H, abi.ptr(wg),
                                 abi.ptr(sg), abi.ptr(wu), abi.ptr(su), I, ops.scale_mode(wg, sg),
                                 abi.ptr(B["m"]), None, None, 0, st), "mlp")
    gemv(B["m"], [(L["down"], B["hout"])], res=B["h2"])
    gemv(B["hout"], list(zip(L["inp"], B["ys"])), norm_w=L["ln1"])


def _counts(sync, nphase=4):
    """Finished-workgroup count of each phase (16 64-bit parts, 128 B apart)."""
    words = sync.cpu().view(torch.int64)   # pairs of uint32 words -> one 64-bit part
    return [int(sum(words[(32 * 16 * k + 32 * j) // 2] for j in range(16))) for k in range(nphase)]


def _outs(B):
    return [B["h2"].clone(), B["m"].clone(), B["hout"].clone()] + [y.clone() for y in B["ys"]]


def test_chain_matches_separate_launches_and_oracle():
    L = _layer(11)
    sync = torch.zeros(abi.load().qh_chain_sync_words(), dtype=torch.int32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    Bc, Bs = _bufs(), _bufs()
    ops.launch_chain(_phases(L, Bc, L["h"]), sync, err)
    _separate(L, Bs, L["h"])
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    counts = _counts(sync)
    assert all(c > 0 for c in counts), counts
    for a, b, name in zip(_outs(Bc), _outs(Bs), ["h2", "m", "h", "qkv", "z", "b", "a"]):
        assert torch.equal(a, b), f"chain vs separate launches differ in {name}"
    # and the oracle, phase by phase from the chain's own inputs
    cpu = lambda t: t.float().cpu()
    deq = lambda ws: orc.dequant(ws[0].cpu(), ws[1].cpu())
    h2 = orc.bf16(cpu(L["h"]) + orc.linear(cpu(L["mix"]), deq(L["o"])))
    assert_close(Bc["h2"], h2, atol_frac=1e-3, what="o_proj+res")
    xn = orc.rmsnorm(cpu(Bc["h2"]), cpu(L["ln2"]))
    gg, uu = xn @ deq(L["gate"]).T, xn @ deq(L["up"]).T
    assert_close(Bc["m"], orc.bf16(torch.nn.functional.silu(gg) * uu), atol_frac=1e-3, what="mlp")
    hh = orc.bf16(cpu(Bc["h2"]) + orc.linear(cpu(Bc["m"]), deq(L["down"])))
    assert_close(Bc["hout"], hh, atol_frac=1e-3, what="down+res")
    xn1 = orc.rmsnorm(cpu(Bc["hout"]), cpu(L["ln1"]))
    for ws, y, n in zip(L["inp"], Bc["ys"], SEGS):
        assert_close(y, orc.linear(xn1, deq(ws)), atol_frac=1e-3, what=f"in_proj {n}")


def test_chain_repeats_and_graph_replays():
    """The counters only grow (compared against the launch epoch): back-to-back
    launches and replays of a captured graph keep giving the eager result."""
    L = _layer(12)
    sync = torch.zeros(abi.load().qh_chain_sync_words(), dtype=torch.int32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    B = _bufs()
    ph = _phases(L, B, L["h"])
    ops.launch_chain(ph, sync, err)
    torch.cuda.synchronize()
    ref = _outs(B)
    for _ in range(3):
        for t in [B["h2"], B["m"], B["hout"]] + B["ys"]:
            t.fill_(0)
        ops.launch_chain(ph, sync, err)
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(_outs(B), ref))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        ops.launch_chain(ph, sync, err)
        ops.launch_chain(ph, sync, err)
    torch.cuda.synchronize()
    for _ in range(3):
        for t in [B["h2"], B["m"], B["hout"]] + B["ys"]:
            t.fill_(0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(_outs(B), ref))
    # 1 + 3 eager launches, then 3 replays of a graph holding 2 launches
    assert int(err.item()) == 0
    counts = _counts(sync)
    assert all(c > 0 and c % 10 == 0 for c in counts), counts


def test_chain_rejects_bad_phases(lib):
    sync = torch.zeros(8, dtype=torch.int32, device=DEV)
    x = torch.zeros(1000, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(64, 1000, dtype=torch.uint8, device=DEV)
    s = torch.ones(1, 8, device=DEV)
    y = torch.empty(64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(abi.QhError):
        ops.launch_chain([ops.chain_gemv_phase(x, [((w, s), y)])], sync)
    with pytest.raises(abi.QhError):
        ops.launch_chain([], sync)
