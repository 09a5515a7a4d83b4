"""The C-ABI library loads and exports every entry point of include/hilda_spec.h.

Runs without a GPU: only host-side argument validation is exercised (every
call below returns before touching a device).
"""
import ctypes
import re
from pathlib import Path

import pytest

HEADER = Path(__file__).resolve().parents[1] / "include" / "hilda_spec.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hs_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    for n in ["hs_spec_accept", "hs_sampler", "hs_status_string"]:
        assert n in names


def test_every_declared_symbol_is_exported(hv):
    lib = hv._lib.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_symbol(hv):
    assert sorted(hv._lib.SIGNATURES) == declared_functions()


def test_status_strings(hv):
    lib = hv._lib.lib()
    assert lib.hs_status_string(0) == b"ok"
    assert lib.hs_status_string(-1) == b"invalid argument"
    assert lib.hs_version() >= 1


def test_workspace_sizes(hv):
    lib = hv._lib.lib()
    assert lib.hs_spec_accept_workspace_size(1, 3, 151936) > 0
    assert lib.hs_spec_accept_workspace_size(0, 3, 151936) == 0
    assert lib.hs_sampler_workspace_size(4, 151936) > lib.hs_sampler_workspace_size(1, 151936)


def test_spec_accept_rejects_bad_arguments_on_host(hv):
    lib = hv._lib.lib()
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p).value
    common = dict(B=1, g=3, V=100)

    def call(B=1, g=3, V=100, mode=0, dtype=1, ws=1 << 20, logits=p, stride=100):
        return lib.hs_spec_accept(logits, dtype, stride, p, V, p, p, p, p, p, p, B, g, V, mode,
                                  p, p, p, None, p, ws, None)

    assert call(B=0) == -1
    assert call(g=0) == -1
    assert call(g=33) == -1
    assert call(mode=7) == -1
    assert call(dtype=5) == -1
    assert call(logits=None) == -1
    assert call(stride=50) == -1
    assert call(ws=16) == -2
    del common


def test_sampler_rejects_bad_arguments_on_host(hv):
    lib = hv._lib.lib()
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p).value
    # uniforms without tokens
    assert lib.hs_sampler(p, 0, 100, 2, 100, p, None, None, 0, None, 0, 0, p, None, None, p,
                          1 << 20, None) == -1
    # greedy with a probability output
    assert lib.hs_sampler(p, 0, 100, 2, 100, None, None, None, 2, p, 100, 0, None, p, None, p,
                          1 << 20, None) == -1
    # bad out_kind
    assert lib.hs_sampler(p, 0, 100, 2, 100, p, None, None, 0, p, 100, 3, None, None, None, p,
                          1 << 20, None) == -1


@pytest.mark.parametrize("fn", ["hs_spec_accept", "hs_sampler"])
def test_no_cpu_fallback_symbol(hv, fn):
    # the product library contains no oracle code
    lib = hv._lib.lib()
    assert not hasattr(lib, "or_spec_accept")
    assert hasattr(lib, fn)
