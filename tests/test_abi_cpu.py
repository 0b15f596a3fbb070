"""C-ABI checks that need no GPU: the library loads, exports every symbol the
public header declares, and rejects invalid arguments before touching HIP."""
import ctypes
import os
import re

import pytest

from qwen35_amd import abi, config, ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qwen35_fp8_hip.h")

# Every symbol the reference's main.py binds (main.py:108-240).
REFERENCE_SYMBOLS = [
    "fp8_gemm_batch", "launch_gemv_v4_extern", "launch_linear_in_proj4", "launch_fused_qkv",
    "launch_fused_gate_up", "launch_rmsnorm_ip", "launch_rmsnorm_out", "launch_fused_attn_v2",
    "launch_fused_attn", "layer_mid_attn", "layer_pre_attn", "layer_post_attn",
    "layer_post_o_fp8_mlp", "launch_prepare_linear_gates", "launch_rmsnorm_gated_decode",
    "launch_delta_rule_decode",
]


def header_symbols():
    """Function names declared in the public header (comments stripped)."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    decls = re.findall(r"^(?:const\s+)?(?:void|int|size_t|char)\s*\*?\s*(\w+)\s*\(", text, re.M)
    return sorted(set(decls))


def exported(path):
    lib = ctypes.CDLL(path)
    return lambda name: hasattr(lib, name)


def test_header_declares_every_reference_symbol():
    decl = header_symbols()
    for s in REFERENCE_SYMBOLS + ["launch_gemv_v3_extern"]:
        assert s in decl, s


def test_library_exports_every_declared_symbol():
    has = exported(abi.library_path())
    missing = [s for s in header_symbols() if not has(s)]
    assert not missing, missing


def test_binding_covers_reference_argtypes():
    lib = abi.load()
    for s in REFERENCE_SYMBOLS:
        assert s in abi.REFERENCE_ARGTYPES
        assert getattr(lib, s).argtypes == abi.REFERENCE_ARGTYPES[s]
    # spot-check arities against the reference declarations (main.py)
    assert len(abi.REFERENCE_ARGTYPES["launch_gemv_v4_extern"]) == 8
    assert len(abi.REFERENCE_ARGTYPES["layer_mid_attn"]) == 19
    assert len(abi.REFERENCE_ARGTYPES["layer_post_attn"]) == 30
    assert len(abi.REFERENCE_ARGTYPES["layer_post_o_fp8_mlp"]) == 21
    assert len(abi.REFERENCE_ARGTYPES["launch_linear_in_proj4"]) == 23


def test_validation_errors_need_no_gpu():
    lib = abi.load()
    rc = lib.qh_gemv_e4m3(None, None, None, 1e-6, 2560, None, None, 5, *([None, None, None, 0, 0] * 4),
                          0, None)
    assert rc == -1 and "nseg" in abi.last_error()
    rc = lib.qh_gemv_e4m3(None, None, None, 1e-6, 100, None, None, 1, *([None, None, None, 0, 0] * 4),
                          0, None)
    assert rc == -1 and "multiple of 8" in abi.last_error()
    rc = lib.qh_rmsnorm(None, None, None, 1, 0, 1e-6, None)
    assert rc == -1 and "bad shape" in abi.last_error()
    rc = lib.qh_add_rmsnorm(None, None, None, None, -1, 2560, 1e-6, None)
    assert rc == -1 and "bad shape" in abi.last_error()
    rc = lib.qh_add_rmsnorm(None, None, None, None, 4, 2560, 1e-6, None)
    assert rc == -1 and "null pointer" in abi.last_error()
    p = ctypes.c_void_p(4096)
    rc = lib.qh_add_rmsnorm(p, ctypes.c_void_p(8192), ctypes.c_void_p(12288), p, 4, 2560, 1e-6, None)
    assert rc == -1 and "alias" in abi.last_error()
    rc = lib.qh_gemm_e4m3_add_rmsnorm(None, None, None, None, 4, 2560, 100, 1, 0, None, None, None, 1e-6,
                                      None, 0, None)
    assert rc == -1 and "multiple of 128" in abi.last_error()
    rc = lib.qh_gemm_e4m3_add_rmsnorm(None, None, None, None, 4, 2560, 256, 2, 0, None, None, None, 1e-6,
                                      None, 0, None)
    assert rc == -1 and "null pointer" in abi.last_error()
    q = [ctypes.c_void_p(4096 * k) for k in range(1, 6)]
    rc = lib.qh_gemm_e4m3_add_rmsnorm(q[0], q[1], q[2], q[3], 4, 2560, 256, 2, 0, q[3], q[4], q[0], 1e-6,
                                      None, 0, None)
    assert rc == -1 and "distinct" in abi.last_error()
    rc = lib.qh_gated_rmsnorm(None, None, None, None, 4, 512, 1e-6, 1, None)
    assert rc == -1 and "head_dim" in abi.last_error()
    rc = lib.qh_attn_decode(None, 512, None, 512, None, None, None, None, None, None, None, None,
                            4096, 96, 64, 16, 4, None, 0, 1, None, None, None, 1e-6, None)
    assert rc == -1 and "head_dim" in abi.last_error()
    rc = lib.qh_attn_decode(None, 512, None, 512, None, None, None, None, None, None, None, None,
                            4096, 256, 64, 16, 3, None, 0, 1, None, None, None, 1e-6, None)
    assert rc == -1 and "n_kv_heads" in abi.last_error()
    rc = lib.qh_attn_decode(None, 512, None, 512, None, None, None, None, None, None, None, None,
                            16, 256, 64, 16, 4, None, 16, 1, None, None, None, 1e-6, None)
    assert rc == -1 and "out of range" in abi.last_error()
    rc = lib.qh_gdn_decode(None, None, None, None, None, None, None, None, None, None, None, None, None,
                           None, 0, 16, 32, 64, 128, 1e-6, None)
    assert rc == -1 and "dk" in abi.last_error()
    # the plain-read floor: alignment, size and output checks before any launch
    for src, nbytes, n_out in [(4096, 100, 8), (4100, 4096, 8), (4096, 0, 8), (4096, 4096, 0),
                               (4096, (1 << 31) + 16, 8)]:
        rc = lib.qh_read_stream(ctypes.c_void_p(src), nbytes, ctypes.c_void_p(8192), n_out, None)
        assert rc == -1 and "read_stream" in abi.last_error(), (src, nbytes, n_out)
    # chunked GatedDeltaNet prefill: shape and workspace checks before any launch
    rc = lib.qh_gdn_chunk(None, None, None, None, None, None, None, None, None, 64, 16, 32, 64, 128,
                          1e-6, None, 0, None)
    assert rc == -1 and "unsupported shape" in abi.last_error()
    for Hk, Hv in [(16, 0), (16, -16), (0, 32)]:
        rc = lib.qh_gdn_chunk(None, None, None, None, None, None, None, None, None, 130, Hk, Hv, 128, 128,
                              1e-6, ctypes.c_void_p(256), 1 << 30, None)
        assert rc == -1 and "unsupported shape" in abi.last_error(), (Hk, Hv)
    need = int(lib.qh_gdn_chunk_workspace_size(130, 32))
    assert need == 32 * 3 * 99328
    rc = lib.qh_gdn_chunk(None, None, None, None, None, None, None, None, None, 130, 16, 32, 128, 128,
                          1e-6, None, need, None)
    assert rc == -1 and "workspace" in abi.last_error()
    rc = lib.qh_gdn_chunk(None, None, None, None, None, None, None, None, None, 130, 16, 32, 128, 128,
                          1e-6, ctypes.c_void_p(256), need - 1, None)
    assert rc == -1 and "workspace" in abi.last_error()
    rc = lib.qh_gemm_e4m3(None, None, None, None, 4, 4, 100, 1, 0, None, 0, None)
    assert rc == -1
    # grouped GEMM: every check runs before anything touches a device pointer
    none4 = [None, None, None, 0, 0] * 4
    rc = lib.qh_gemm_e4m3_grouped(None, 4, 2560, 1, *none4, 0, None, 0, None)
    assert rc == -1 and "null activation" in abi.last_error()
    fake = ctypes.c_void_p(256)
    rc = lib.qh_gemm_e4m3_grouped(fake, 4, 2560, 5, *none4, 0, None, 0, None)
    assert rc == -1 and "nseg=5" in abi.last_error()
    rc = lib.qh_gemm_e4m3_grouped(fake, 4, 2560, 1, *none4, 0, None, 0, None)
    assert rc == -1 and "segment 0" in abi.last_error()
    rc = lib.qh_gemm_e4m3_grouped(fake, 4, 100, 1, *none4, 0, None, 0, None)
    assert rc == -1
    # split-K workspace: a buffer smaller than qh_gemm_workspace_size, or
    # misaligned, is refused before anything touches the device
    need = int(lib.qh_gemm_workspace_size(512, 2560))
    assert need == 16 << 20
    ws = ctypes.c_void_p(1 << 20)
    x4 = [ctypes.c_void_p(4096 * k) for k in range(1, 5)]
    for nbytes, addr, msg in [(need - 1, ws, "smaller than"), (0, ws, "smaller than"),
                              (need, ctypes.c_void_p((1 << 20) + 16), "256-byte aligned")]:
        lib.qh_clear_error()
        rc = lib.qh_gemm_e4m3(*x4, 512, 9216, 2560, 20, 0, addr, nbytes, None)
        assert rc == -1 and msg in abi.last_error(), abi.last_error()
        lib.qh_clear_error()
        rc = lib.qh_gemm_e4m3_grouped(x4[0], 512, 2560, 1, x4[1], x4[2], x4[3], 9216, 20,
                                      *([None, None, None, 0, 0] * 3), 0, addr, nbytes, None)
        assert rc == -1 and msg in abi.last_error(), abi.last_error()
        lib.qh_clear_error()
        rc = lib.qh_gemm_e4m3_add_rmsnorm(x4[0], x4[1], x4[2], x4[3], 512, 2560, 9216, 72, 0,
                                          ctypes.c_void_p(1 << 24), None, None, 1e-6, addr, nbytes, None)
        assert rc == -1 and msg in abi.last_error(), abi.last_error()
    # reference symbols: no error channel in the reference; ours records one
    lib.qh_clear_error()
    lib.launch_gemv_v4_extern(None, None, None, None, 16, 12, 1, None)
    assert "multiple of 8" in abi.last_error()


def test_attention_scratch_layout():
    """qh_attn_scratch_bytes: n_kv x 8 group-counter words, then the split
    records [n_kv][nsplit][8][D + 2] and, above 8 splits, the level-2 records
    [n_kv][8][8][D + 2] (4-byte words).  Split-K with no scratch, and more than
    8 splits with scratch but no room for the group counters, are refused."""
    lib = abi.load()
    for n_kv, nsplit, D in [(4, 1, 256), (4, 8, 256), (4, 9, 256), (4, 64, 256), (2, 16, 128), (16, 55, 256)]:
        words = n_kv * 8 + n_kv * (nsplit + (8 if nsplit > 8 else 0)) * 8 * (D + 2)
        assert lib.qh_attn_scratch_bytes(n_kv, nsplit, D) == 4 * words, (n_kv, nsplit, D)
    rc = lib.qh_attn_decode(None, 512, None, 512, None, None, None, None, None, None, None, None,
                            4096, 256, 64, 16, 4, None, 100, 16, None, ctypes.c_void_p(4096), None, 1e-6,
                            None)
    assert rc == -1 and "scratch" in abi.last_error()


def test_scale_mode_encoding():
    import torch
    w = torch.zeros(256, 512, dtype=torch.uint8)
    assert ops.scale_mode(w, torch.zeros(2, 4)) == 4            # block
    assert ops.scale_mode(w, torch.zeros(256, 1)) == 1          # per row
    assert ops.scale_mode(w, torch.zeros(256, 4)) == -4         # per row and K block
    assert ops.scale_mode(torch.zeros(1, 128, dtype=torch.uint8), torch.zeros(1, 1)) == 1


def test_config_shapes():
    c = config.qwen35_4b()
    assert c.layer_types.count("full_attention") == 8
    assert [i for i in range(32) if c.is_full(i)] == list(range(3, 32, 4))
    assert c.q_proj_rows == 8192 and c.kv_rows == 1024 and c.conv_dim == 8192
    assert c.rotary_dim == 64 and c.value_dim == 4096
    nested = {"text_config": {"hidden_size": 2560, "num_hidden_layers": 32,
                              "rope_parameters": {"rope_theta": 1e7, "partial_rotary_factor": 0.25}}}
    c2 = config.Qwen35Config.from_dict(nested)
    assert c2.rope_theta == 1e7 and c2.rotary_dim == 64


def test_engine_refuses_without_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    from qwen35_amd import engine, synth
    w = synth.make_weights(config.tiny(num_layers=1, vocab=256), seed=0)
    with pytest.raises(RuntimeError, match="needs a GPU"):
        engine.Qwen35FP8Engine(w, max_seq_len=16)
