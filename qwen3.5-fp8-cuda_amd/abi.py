"""ctypes binding of libqwen35_fp8_hip.so.

The reference loads two DLLs with ``ctypes.CDLL`` and declares argtypes for
each export (main.py:103-240).  This module does the same for the single
gfx950 library: the reference symbols keep their exact argtypes, the native
``qh_*`` entry points return ``int`` status with ``qh_last_error()`` for the
message.

The library binds to the HIP runtime already loaded by torch (both carry the
soname ``libamdhip64.so.7``), so torch is imported first and torch streams can
be passed straight through.
"""
import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL: shares torch's HIP runtime)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libqwen35_fp8_hip.so"

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t
_u64 = ctypes.c_uint64

# Reference ABI (fused_kernels.cu:940-1356, fp8_kernels.cu:68-91); argtypes as
# declared by main.py:108-240.
REFERENCE_ARGTYPES = {
    "fp8_gemm_batch": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp],
    "launch_gemv_v4_extern": [_vp, _vp, _vp, _vp, _i, _i, _i, _vp],
    "launch_gemv_v3_extern": [_vp, _vp, _vp, _vp, _i, _i, _i, _vp],
    "launch_linear_in_proj4": [_vp] + [_vp, _vp, _vp, _i, _i] * 4 + [_i, _vp],
    "launch_fused_qkv": [_vp] + [_vp] * 3 + [_vp] * 3 + [_vp] * 3 + [_i] * 4 + [_i] * 4 + [_vp],
    "launch_fused_gate_up": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp],
    "launch_rmsnorm_ip": [_vp, _vp, _i, _i, _f, _vp],
    "launch_rmsnorm_out": [_vp, _vp, _vp, _i, _i, _f, _vp],
    "launch_fused_attn_v2": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "launch_fused_attn": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "layer_mid_attn": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                       _i, _i, _i, _i, _i, _i, _i, _i, _vp],
    "layer_pre_attn": [_vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _i, _i, _vp, _vp, _i, _i,
                       _vp, _vp, _vp, _vp, _i, _i, _vp],
    "layer_post_attn": [_vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _i, _i, _vp, _vp, _i, _i,
                        _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "layer_post_o_fp8_mlp": [_vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _i,
                             _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp],
    "launch_prepare_linear_gates": [_vp, _vp, _vp, _vp, _vp, _vp, _i, _vp],
    "launch_rmsnorm_gated_decode": [_vp, _vp, _vp, _vp, _i, _i, _f, _vp],
    "launch_delta_rule_decode": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp],
}

# Native entry points: (restype, argtypes).
NATIVE_SIGNATURES = {
    "qh_last_error": (ctypes.c_char_p, []),
    "qh_clear_error": (None, []),
    "qh_abi_version": (_i, []),
    "qh_set_qgate_head_dim": (_i, [_i]),
    "qh_gemv_e4m3": (_i, [_vp, _vp, _vp, _f, _i, _vp, _vp, _i]
                     + [_vp, _vp, _vp, _i, _i] * 4 + [_i, _vp]),
    "qh_mlp_gate_up": (_i, [_vp, _vp, _vp, _f, _i, _vp, _vp, _vp, _vp, _i, _i,
                            _vp, _vp, _vp, _i, _vp]),
    "qh_mlp_decode": (_i, [_vp, _vp, _vp, _f, _i, _vp, _vp, _vp, _vp, _i, _i,
                           _vp, _vp, _i, _vp, _vp, _i, _vp]),
    "qh_rmsnorm": (_i, [_vp, _vp, _vp, _i, _i, _f, _vp]),
    "qh_add_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f, _vp]),
    "qh_attn_scratch_bytes": (_sz, [_i, _i, _i]),
    "qh_attn_decode": (_i, [_vp, _i, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                            _i, _i, _i, _i, _i, _vp, _i, _i, _vp, _vp, _vp, _f, _vp]),
    "qh_attn_decode_noalloc": (_i, [_vp, _i, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                    _i, _i, _i, _i, _i, _vp, _i, _i, _vp, _f, _vp]),
    "qh_gdn_decode": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                           _vp, _i, _i, _i, _i, _i, _f, _vp]),
    "qh_gdn_decode_core": (_i, [_vp] * 10 + [_i] * 5 + [_vp]),
    "qh_gemv_e4m3_gated": (_i, [_vp, _vp, _vp, _i, _f, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "qh_read_stream": (_i, [_vp, _sz, _vp, _i, _vp]),
    "qh_lm_head_scratch_bytes": (_sz, [_i]),
    "qh_lm_head_argmax": (_i, [_vp, _vp, _f, _i, _vp, _i, _vp, _vp, _vp, _vp, _vp, _i,
                               _vp, _vp, _vp, _vp]),
    "qh_sample_workspace_size": (_sz, [_i]),
    "qh_sample_top_p": (_i, [_vp, _i, _f, _f, _f, _vp, _i, _vp, _i, _i, _vp, _i, _u64, _vp, _vp,
                             _vp, _vp, _vp, _i, _vp, _vp]),
    "qh_embed": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "qh_add_bf16": (_i, [_vp, _vp, _vp, _i, _vp]),
    "qh_linear_gates": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _vp]),
    "qh_gated_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f, _i, _vp]),
    "qh_gemm_workspace_size": (_sz, [_i, _i]),
    "qh_gemm_e4m3": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "qh_gemm_e4m3_add_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _f, _vp, _sz, _vp]),
    "qh_gemm_e4m3_grouped": (_i, [_vp, _i, _i, _i] + [_vp, _vp, _vp, _i, _i] * 4 + [_i, _vp, _sz, _vp]),
    "qh_attn_prep": (_i, [_vp] * 10 + [_i] * 7 + [_f, _vp]),
    "qh_attn_prefill": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp] + [_i] * 6 + [_vp]),
    "qh_gdn_prep": (_i, [_vp] * 12 + [_i] * 6 + [_vp]),
    "qh_gdn_scan": (_i, [_vp] * 9 + [_i] * 5 + [_f, _vp]),
    "qh_gdn_chunk_workspace_size": (_sz, [_i, _i]),
    "qh_gdn_chunk": (_i, [_vp] * 9 + [_i] * 5 + [_f, _vp, _sz, _vp]),
    "qh_silu_mul": (_i, [_vp, _vp, _vp, _sz, _vp]),
}


class QhError(RuntimeError):
    """A native entry point rejected its arguments or failed to launch."""


_LIB = None


def library_path():
    return os.environ.get("QH_LIB", os.path.join(_HERE, LIB_NAME))


def load(path=None):
    """Load the library once and declare every signature.  Raises if missing:
    there is no fallback implementation."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = path or library_path()
    if not os.path.exists(p):
        raise FileNotFoundError(
            f"{p} not found: build it with `python qwen3.5-fp8-cuda_amd/build.py` "
            "(there is no non-HIP fallback)")
    lib = ctypes.CDLL(p)
    for name, argt in REFERENCE_ARGTYPES.items():
        fn = getattr(lib, name)
        fn.argtypes = argt
        fn.restype = None
    for name, (rest, argt) in NATIVE_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argt
        fn.restype = rest
    if path is None:
        _LIB = lib
    return lib


def last_error(lib=None):
    lib = lib or load()
    msg = lib.qh_last_error()
    return msg.decode() if msg else ""


def check(rc, what=""):
    """Raise QhError when a native entry point returned non-zero."""
    if rc != 0:
        raise QhError(f"{what}: {last_error()}" if what else last_error())
    return rc


def ptr(t):
    """Device pointer of a tensor (or None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)
