"""Allocation-free decode attention (qh_attn_decode_noalloc, partials and
counters in the library's fixed device array) against qh_attn_decode with
caller scratch, through the C-ABI: two calls in a row, the second smaller."""
import pytest
import torch

from oracle import qwen35_oracle as orc
from qwen35_amd import abi

from _util import assert_close, bf, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _args(q_all, k_new, v_new, qn, kn, cos, sin, kc, vc, max_seq, D, rot, Hq, Hkv, pos, nsplit):
    return [abi.ptr(q_all), 2 * D, abi.ptr(q_all[D:]), 2 * D, abi.ptr(k_new), abi.ptr(v_new),
            abi.ptr(qn), abi.ptr(kn), abi.ptr(cos), abi.ptr(sin), abi.ptr(kc), abi.ptr(vc),
            max_seq, D, rot, Hq, Hkv, None, pos, nsplit]


# (Hq, Hkv, D, ctx, max_seq, nsplit) of the two calls.  At head_dim 256, 16 KV
# heads x (55 split + 8 level-2 records) x 8 x 258 floats + 16 x 8 counters =
# 2,080,640 words is the largest 16-KV-head shape that fits the fixed 2^21-float
# array; 55 splits also leave a ragged last merge group (7 of 8).
@pytest.mark.parametrize("first,second", [((16, 4, 256, 4096, 4096, 64), (8, 2, 128, 300, 512, 16)),
                                          ((64, 16, 256, 4096, 4096, 55), (16, 4, 256, 700, 1024, 8)),
                                          ((32, 8, 256, 4096, 4096, 64), (16, 4, 256, 700, 1024, 12))])
def test_noalloc_attention_matches_scratch_entry_point(first, second):
    lib = abi.load()
    for step, (Hq, Hkv, D, ctx, max_seq, nsplit) in enumerate((first, second)):
        g = gen(100 + step)
        rot = 64 if D == 256 else 32
        kc = bf(randn(g, Hkv, max_seq, D))
        vc = bf(randn(g, Hkv, max_seq, D))
        q_all = bf(randn(g, Hq * 2 * D))
        k_new, v_new = bf(randn(g, Hkv * D)), bf(randn(g, Hkv * D))
        qn, kn = randn(g, D, std=0.02), randn(g, D, std=0.02)
        cos, sin = orc.rope_tables(max_seq, rot, 1e7)
        pos = ctx - 1
        dev = [t.to(DEV) for t in (q_all, k_new, v_new, qn, kn, cos, sin)]
        caches = [(kc.to(DEV), vc.to(DEV)) for _ in range(2)]
        outs = [torch.empty(Hq * D, dtype=torch.bfloat16, device=DEV) for _ in range(2)]
        scratch = torch.zeros(int(lib.qh_attn_scratch_bytes(Hkv, nsplit, D)) + 4, dtype=torch.uint8,
                              device=DEV)
        counters = torch.zeros(Hkv, dtype=torch.int32, device=DEV)
        a = _args(*dev, *caches[0], max_seq, D, rot, Hq, Hkv, pos, nsplit)
        abi.check(lib.qh_attn_decode(*a, abi.ptr(scratch), abi.ptr(counters), abi.ptr(outs[0]), 1e-6,
                                     abi.stream_handle()), "qh_attn_decode")
        b = _args(*dev, *caches[1], max_seq, D, rot, Hq, Hkv, pos, nsplit)
        abi.check(lib.qh_attn_decode_noalloc(*b, abi.ptr(outs[1]), 1e-6, abi.stream_handle()),
                  "qh_attn_decode_noalloc")
        torch.cuda.synchronize()
        # same kernel, same splits: identical results and cache writes
        assert torch.equal(outs[1], outs[0]), f"call {step}: outputs differ"
        assert torch.equal(caches[1][0], caches[0][0]) and torch.equal(caches[1][1], caches[0][1])
        kr, vr = kc.float().clone(), vc.float().clone()
        ref = orc.attn_decode(q_all.float(), k_new.float(), v_new.float(), qn, kn, cos, sin, kr, vr,
                              pos, Hq, Hkv, D, rot)
        assert_close(outs[1], ref, atol_frac=1e-3, what=f"noalloc attention, call {step}")


@pytest.mark.parametrize("n_kv,nsplit", [(64, 64), (16, 56)])
def test_noalloc_attention_rejects_shapes_beyond_its_scratch(n_kv, nsplit):
    """A shape whose scratch is above 2^21 words (16 x 56: 16 x 8 + 16 x 64 x
    8 x 258 = 2,113,664, one split more than the accepted 16 x 55) is refused
    before any launch."""
    lib = abi.load()
    assert lib.qh_attn_scratch_bytes(n_kv, nsplit, 256) > 8 << 20
    assert lib.qh_attn_scratch_bytes(16, 55, 256) <= 8 << 20
    x = torch.zeros(16, dtype=torch.bfloat16, device=DEV)
    rc = lib.qh_attn_decode_noalloc(abi.ptr(x), 512, None, 0, abi.ptr(x), abi.ptr(x), None, None,
                                    None, None, abi.ptr(x), abi.ptr(x), 4096, 256, 64, 4 * n_kv, n_kv,
                                    None, 0, nsplit, abi.ptr(x), 1e-6, abi.stream_handle())
    assert rc == -1
    assert "fixed scratch" in abi.last_error()
