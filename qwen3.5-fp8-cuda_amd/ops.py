"""Reference-named operator wrappers over the HIP library.

Same names, argument meaning and dispatch as the reference's host wrappers
(main.py:242-323): ``fp8_linear`` (M == 1 -> GEMV, M > 1 -> GEMM),
``maybe_fp8_linear`` (FP8 tuple vs bf16 tensor), ``fused_qkv`` and
``fused_gate_up``.  Scales may be bf16 (the reference's ABI: routed to the
reference symbols) or fp32 (the native entry points).  Every launch goes on
the current torch stream, never the legacy null stream, so the calls can be
captured in a HIP graph.
"""
import torch
import torch.nn.functional as F

from . import abi


def scale_mode(w_bytes, scale):
    """Reference `K_blocks` encoding (main.py:249-251): negative marks
    [N, K_blocks] per-row-per-block scales."""
    n_out = w_bytes.shape[0]
    k_blocks = scale.shape[1] if scale.dim() == 2 else 1
    if scale.dim() == 2 and scale.shape[0] == n_out and k_blocks > 1:
        return -k_blocks
    return k_blocks


def _check_linear(x2d, w_bytes, w_scale):
    if not (x2d.is_cuda and w_bytes.is_cuda and w_scale.is_cuda):
        raise ValueError("fp8_linear: tensors must be on the GPU")
    if x2d.dtype != torch.bfloat16 or w_bytes.dtype != torch.uint8:
        raise TypeError("fp8_linear: expects bf16 input and uint8 (E4M3FN) weight bytes")
    if w_scale.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("fp8_linear: scale_inv must be bf16 or fp32")
    if not (x2d.is_contiguous() and w_bytes.is_contiguous() and w_scale.is_contiguous()):
        raise ValueError("fp8_linear: tensors must be contiguous")
    if w_bytes.shape[1] != x2d.shape[1]:
        raise ValueError(f"fp8_linear: K mismatch {x2d.shape[1]} vs {w_bytes.shape[1]}")


def fp8_linear(input_bf16, w_bytes, w_scale_inv, out=None):
    """FP8 linear y = x W^T (main.py:242-270).  bf16 scales go to the
    reference symbols (launch_gemv_v4_extern for M == 1, fp8_gemm_batch for
    M > 1), fp32 scales to the native entry points."""
    lib = abi.load()
    orig = input_bf16.shape
    K = orig[-1]
    N = w_bytes.shape[0]
    x2d = input_bf16.reshape(-1, K)
    if not x2d.is_contiguous():
        x2d = x2d.contiguous()
    _check_linear(x2d, w_bytes, w_scale_inv)
    M = x2d.shape[0]
    kb = scale_mode(w_bytes, w_scale_inv)
    y = out if out is not None else torch.empty(M, N, dtype=torch.bfloat16, device=x2d.device)
    st = abi.stream_handle()
    bf16_scales = w_scale_inv.dtype == torch.bfloat16
    if M == 1:
        if bf16_scales:
            lib.qh_clear_error()
            lib.launch_gemv_v4_extern(abi.ptr(x2d), abi.ptr(w_bytes), abi.ptr(w_scale_inv),
                                      abi.ptr(y), N, K, kb, st)
            err = abi.last_error(lib)
            if err:
                raise abi.QhError(err)
        else:
            abi.check(lib.qh_gemv_e4m3(abi.ptr(x2d), None, None, 1e-6, K, None, None, 1,
                                       abi.ptr(w_bytes), abi.ptr(w_scale_inv), abi.ptr(y), N, kb,
                                       None, None, None, 0, 0, None, None, None, 0, 0,
                                       None, None, None, 0, 0, 0, st), "fp8_linear")
    elif bf16_scales:
        lib.qh_clear_error()
        lib.fp8_gemm_batch(abi.ptr(x2d), abi.ptr(w_bytes), abi.ptr(w_scale_inv), abi.ptr(y),
                           M, N, K, kb, st)
        err = abi.last_error(lib)
        if err:
            raise abi.QhError(err)
    else:
        abi.check(lib.qh_gemm_e4m3(abi.ptr(x2d), abi.ptr(w_bytes), abi.ptr(w_scale_inv),
                                   abi.ptr(y), M, N, K, kb, 0, None, 0, st), "fp8_linear")
    return y.reshape(*orig[:-1], N)


def maybe_fp8_linear(input_bf16, weight):
    """FP8 tuple (bytes, scale) -> fp8_linear; bf16 tensor -> F.linear (main.py:273-279)."""
    if isinstance(weight, tuple):
        return fp8_linear(input_bf16, weight[0], weight[1])
    return F.linear(input_bf16, weight)


def fused_qkv(x_bf16, w_q, s_q, w_k, s_k, w_v, s_v):
    """Three projections sharing one input in one launch (main.py:281-298)."""
    lib = abi.load()
    K = x_bf16.shape[-1]
    N_q, N_k, N_v = w_q.shape[0], w_k.shape[0], w_v.shape[0]
    dev = x_bf16.device
    q = torch.empty(N_q, dtype=torch.bfloat16, device=dev)
    k = torch.empty(N_k, dtype=torch.bfloat16, device=dev)
    v = torch.empty(N_v, dtype=torch.bfloat16, device=dev)
    st = abi.stream_handle()
    if s_q.dtype == torch.bfloat16:
        lib.qh_clear_error()
        lib.launch_fused_qkv(abi.ptr(x_bf16), abi.ptr(w_q), abi.ptr(w_k), abi.ptr(w_v),
                             abi.ptr(s_q), abi.ptr(s_k), abi.ptr(s_v), abi.ptr(q), abi.ptr(k),
                             abi.ptr(v), K, N_q, N_k, N_v, scale_mode(w_q, s_q),
                             s_q.shape[0], s_k.shape[0], s_v.shape[0], st)
        err = abi.last_error(lib)
        if err:
            raise abi.QhError(err)
    else:
        abi.check(lib.qh_gemv_e4m3(abi.ptr(x_bf16), None, None, 1e-6, K, None, None, 3,
                                   abi.ptr(w_q), abi.ptr(s_q), abi.ptr(q), N_q, scale_mode(w_q, s_q),
                                   abi.ptr(w_k), abi.ptr(s_k), abi.ptr(k), N_k, scale_mode(w_k, s_k),
                                   abi.ptr(w_v), abi.ptr(s_v), abi.ptr(v), N_v, scale_mode(w_v, s_v),
                                   None, None, None, 0, 0, 0, st), "fused_qkv")
    return q, k, v


def fused_gate_up(x_bf16, w_g, s_g, w_u, s_u):
    """Gate and up projections in one launch (main.py:301-323)."""
    lib = abi.load()
    K = x_bf16.shape[-1]
    N_g, N_u = w_g.shape[0], w_u.shape[0]
    dev = x_bf16.device
    g = torch.empty(N_g, dtype=torch.bfloat16, device=dev)
    u = torch.empty(N_u, dtype=torch.bfloat16, device=dev)
    st = abi.stream_handle()
    kb = scale_mode(w_g, s_g)
    if s_g.dtype == torch.bfloat16:
        lib.qh_clear_error()
        lib.launch_fused_gate_up(abi.ptr(x_bf16), abi.ptr(w_g), abi.ptr(w_u), abi.ptr(s_g),
                                 abi.ptr(s_u), abi.ptr(g), abi.ptr(u), K, N_g, N_u, kb,
                                 s_g.shape[0], s_u.shape[0], st)
        err = abi.last_error(lib)
        if err:
            raise abi.QhError(err)
    else:
        abi.check(lib.qh_gemv_e4m3(abi.ptr(x_bf16), None, None, 1e-6, K, None, None, 2,
                                   abi.ptr(w_g), abi.ptr(s_g), abi.ptr(g), N_g, kb,
                                   abi.ptr(w_u), abi.ptr(s_u), abi.ptr(u), N_u, scale_mode(w_u, s_u),
                                   None, None, None, 0, 0, None, None, None, 0, 0, 0, st),
                  "fused_gate_up")
    return g, u


def rmsnorm(x, weight, eps=1e-6, out=None):
    """(1+w) RMSNorm over the last dim; in place unless `out` is given
    (main.py:898-933 decode path / launch_rmsnorm_ip)."""
    lib = abi.load()
    D = x.shape[-1]
    rows = x.numel() // D
    dst = x if out is None else out
    abi.check(lib.qh_rmsnorm(abi.ptr(x), abi.ptr(weight), abi.ptr(dst), rows, D, eps,
                             abi.stream_handle()), "rmsnorm")
    return dst
