"""MI355X-native batch-1 FP8 decode path for Qwen3.5-shaped hybrid models.

The package directory is named after the reference it replaces
(`qwen3.5-fp8-cuda_amd/`), which is not a valid module name; it is imported as
``qwen35_amd`` through ``load_package()`` in the repository's
``__graft_entry__.py`` (tests and bench.py do the same).

Modules:
  abi     ctypes binding of libqwen35_fp8_hip.so (reference symbols + qh_*)
  ops     reference-named wrappers: fp8_linear, maybe_fp8_linear, fused_qkv, ...
  config  model shape (config.json keys)
  synth   seeded synthetic weights, reference block quantizer
  engine  decode engine: per-token launch sequence and HIP-graph replay
  build   hipcc build of the shared library
"""
from . import abi, config, ops, synth  # noqa: F401

__all__ = ["abi", "config", "ops", "synth", "engine"]
