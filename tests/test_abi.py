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


def test_accept_commit_next_rejects_bad_arguments_on_host(hv):
    """hs_spec_accept_commit_next checks the bookkeeping arguments as
    hs_spec_commit_next does, then the acceptance's as hs_spec_accept does, before
    any launch."""
    L = hv._lib
    lib = L.lib()
    buf = ctypes.create_string_buffer(4096)
    p = ctypes.cast(buf, ctypes.c_void_p).value
    st = L.SpecState(*([p] * 11), 1, 4, 64, 8, 16, 0, 2)  # B=1, W=4, T=64, 8 blocks of 16

    def args(lookback=1, elig=p, ws_bytes=1 << 20, vids=None, next_gamma=3):
        return L.CommitNextArgs(ctypes.pointer(st), elig, p, ws_bytes, next_gamma, lookback, None,
                                p, p, p, p, p, vids, None, None, None, None)

    def call(na, B=1, g=3):
        return lib.hs_spec_accept_commit_next(p, 1, 100, p, 100, p, p, p, p, p, p, B, g, 100, 0,
                                              p, p, p, None, p, 1 << 20,
                                              None if na is None else ctypes.byref(na), None)

    assert call(None) == -1  # no bookkeeping arguments
    assert call(args(), B=2) == -1  # a state of another batch
    assert call(args(lookback=2)) == -1
    assert call(args(elig=None)) == -1
    assert call(args(next_gamma=-1)) == -1
    assert call(args(vids=p)) == -1  # the verify staging outputs: all five or none
    assert call(args(ws_bytes=8)) == -2
    assert call(args(), g=0) == -1  # the acceptance's own checks


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


def test_linear_rmsnorm_rejects_overlapping_residual_on_host(hv):
    """Workgroup 0 writes residual_out while the other workgroups still read x and
    residual_in, so any overlap is refused before a launch."""
    lib = hv._lib.lib()
    buf = ctypes.create_string_buffer(1 << 16)
    base = (ctypes.cast(buf, ctypes.c_void_p).value + 255) // 256 * 256
    x, res, w, nw, out = base, base + 8192, base + 16384, base + 24576, base + 32768
    K, N = 512, 4

    def call(r_out, r_in=res, rows=2):
        return lib.hs_linear_rmsnorm(x, K, r_in, K, r_out, K, nw, 1e-6, w, rows, K, N, 0, out, N,
                                     None)
    assert call(res) == -1          # residual_out == residual_in
    assert call(x) == -1            # residual_out == x
    assert call(res + 2 * K) == -1  # overlaps the second residual row
    assert call(x, r_in=None) == -1
    # shape limits: 9 rows, K not a multiple of 512
    assert lib.hs_linear_rmsnorm(x, K, None, 0, None, 0, nw, 1e-6, w, 9, K, N, 0, out, N,
                                 None) == -4
    assert lib.hs_linear_rmsnorm(x, K, None, 0, None, 0, nw, 1e-6, w, 1, 500, N, 0, out, N,
                                 None) == -4
    assert lib.hs_linear_rmsnorm(x, K, None, 0, None, 0, None, 1e-6, w, 1, K, N, 0, out, N,
                                 None) == -1


def test_qk_norm_rope_store_rejects_bad_arguments_on_host(hv):
    lib = hv._lib.lib()
    buf = ctypes.create_string_buffer(256)
    p = (ctypes.cast(buf, ctypes.c_void_p).value + 15) // 16 * 16

    def call(hd=128, dtype=1, ks=1.0, ts=(4 + 2 * 2) * 128, bs=16):
        return lib.hs_qk_norm_rope_store(p, ts, 4, 2, hd, p, p, p, p, 1e-6, p, p, p, dtype, 0, 0, 0,
                                         ks, 1.0, p, bs, 8, 3, None)
    assert call(hd=64) == -4
    assert call(dtype=7) == -1
    assert call(dtype=2, ks=0.0) == -1
    assert call(ts=100) == -1
    assert call(bs=0) == -1


def test_qk_norm_rope_attend_rejects_bad_arguments_on_host(hv):
    lib = hv._lib.lib()
    buf = ctypes.create_string_buffer(256)
    p = (ctypes.cast(buf, ctypes.c_void_p).value + 15) // 16 * 16

    def call(hd=128, dtype=1, ks=1.0, ts=(4 + 2 * 2) * 128, n=3, qkv=p):
        return lib.hs_qk_norm_rope_attend(qkv, ts, n, p, p, p, 64, p, 1e-6, p, p, p, p, dtype, 0,
                                          0, 0, ks, 1.0, p, 8, 8, 8, p, p, 1, 4, 64, 4, 2, hd,
                                          16, 0.1, p, 512, 128, None, 0, None)
    assert call(n=0) == 0
    assert call(n=-1) == -1
    assert call(qkv=None) == -1
    assert call(hd=64) == -4
    assert call(dtype=7) == -1
    assert call(dtype=2, ks=0.0) == -1
    assert call(ts=100) == -1
