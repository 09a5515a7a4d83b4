"""hilda-vllm_amd: MI355X-native speculative-decoding verify path.

The package is imported by path name (it contains a hyphen):
    import importlib; hv = importlib.import_module("hilda-vllm_amd")
Kernels live in libhilda_spec.so (csrc/, C ABI in include/hilda_spec.h); the
Python modules mirror the reference interfaces they replace.
"""
from . import _lib, ops, synthetic  # noqa: F401

__all__ = ["_lib", "ops", "synthetic"]
