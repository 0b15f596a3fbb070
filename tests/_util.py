"""Shared helpers for the parity tests."""
import torch

from oracle import qwen35_oracle as orc


def gen(seed=0):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def randn(g, *shape, std=1.0):
    return torch.randn(*shape, generator=g) * std


def bf(x):
    return x.to(torch.bfloat16)


def cos_sim(a, b):
    a = a.double().reshape(-1)
    b = b.double().reshape(-1)
    return float((a @ b) / (a.norm() * b.norm() + 1e-300))


def assert_close(got, ref, rtol=1e-2, atol_frac=1e-4, min_cos=0.99999, what=""):
    """bf16-output parity: |got - ref| <= rtol*|ref| + atol_frac*max|ref|
    elementwise, and cosine similarity >= min_cos."""
    got = got.detach().float().cpu().reshape(-1)
    ref = ref.detach().float().cpu().reshape(-1)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    tol = rtol * ref.abs() + atol_frac * ref.abs().max()
    bad = (got - ref).abs() > tol
    nbad = int(bad.sum())
    c = cos_sim(got, ref)
    if nbad or c < min_cos:
        i = int(((got - ref).abs() - tol).argmax())
        raise AssertionError(f"{what}: {nbad}/{ref.numel()} outside tolerance, cos={c:.8f}; "
                             f"worst i={i} got={got[i].item():.6g} ref={ref[i].item():.6g}")
    return c


def quant(g, n, k, std=0.02):
    return orc.quantize_block_fp8(randn(g, n, k, std=std))
