"""numpy/ctypes front end of the CPU oracle (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module; the product path (hilda-vllm_amd) never does. The arithmetic
lives in spec_oracle.c / attn_oracle.c, which restate the reference files
cited in their headers.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"

MODE_REFERENCE, MODE_FILTERED, MODE_GREEDY = 0, 1, 2
_MODES = {"reference": 0, "filtered": 1, "greedy": 2}

_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")


def build() -> Path:
    res = subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp = ctypes.c_void_p
        L.or_exp_f32.argtypes = [ctypes.c_float]
        L.or_exp_f32.restype = ctypes.c_float
        L.or_fx44.argtypes = [ctypes.c_float]
        L.or_fx44.restype = ctypes.c_uint64
        L.or_f32_of_u64.argtypes = [ctypes.c_uint64]
        L.or_f32_of_u64.restype = ctypes.c_float
        L.or_key_f32.argtypes = [ctypes.c_float]
        L.or_key_f32.restype = ctypes.c_uint32
        L.or_spec_accept.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, vp, vp,
                                     vp, vp, vp, ctypes.c_int, vp, vp, vp, vp, vp]
        L.or_spec_accept.restype = ctypes.c_int
        L.or_sampler.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, vp, vp, ctypes.c_int, vp, vp,
                                 vp, vp]
        L.or_sampler.restype = ctypes.c_int
        L.or_filter_keep.argtypes = [_f32p, ctypes.c_int, ctypes.c_float, ctypes.c_int,
                                     ctypes.c_float, _u8p, ctypes.POINTER(ctypes.c_float),
                                     ctypes.POINTER(ctypes.c_float)]
        L.or_filter_keep.restype = ctypes.c_int
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact bf16 -> f32 from raw uint16 bit patterns."""
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounding = ((u >> 16) & 1) + 0x7FFF
    return ((u + rounding) >> 16).astype(np.uint16)


def exp_f32(y: float) -> float:
    return lib().or_exp_f32(float(y))


def fx44(v: float) -> int:
    return int(lib().or_fx44(float(v)))


def f32_of_u64(n: int) -> float:
    return lib().or_f32_of_u64(int(n))


def key_f32(x: float) -> int:
    return int(lib().or_key_f32(float(x)))


def spec_accept(logits, draft_probs, draft_tokens, temperatures, u_accept, u_resample,
                mode="reference", top_ks=None, top_ps=None, want_probs=False):
    """Oracle of the fused acceptance sampler.

    logits [B, gamma+1, V] f32 (bf16 inputs must be converted exactly first),
    draft_probs [B, gamma, V] f32, draft_tokens [B, gamma] int64.
    Returns dict(num_accepted, out_tokens, out_len, row_stats[, probs]).
    """
    m = _MODES[mode] if isinstance(mode, str) else int(mode)
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    B, R, V = logits.shape
    gamma = R - 1
    q = np.ascontiguousarray(draft_probs, dtype=np.float32) if draft_probs is not None else \
        np.zeros((B, gamma, V), np.float32)
    dtok = np.ascontiguousarray(draft_tokens, dtype=np.int64)
    temps = np.ascontiguousarray(temperatures if temperatures is not None else np.ones(B),
                                 dtype=np.float32)
    tk = None if top_ks is None else np.ascontiguousarray(top_ks, dtype=np.int32)
    tp = None if top_ps is None else np.ascontiguousarray(top_ps, dtype=np.float32)
    ua = np.ascontiguousarray(u_accept if u_accept is not None else np.zeros((B, gamma)),
                              dtype=np.float32)
    ur = np.ascontiguousarray(u_resample if u_resample is not None else np.zeros(B),
                              dtype=np.float32)
    nacc = np.zeros(B, np.int32)
    out = np.zeros((B, R), np.int64)
    olen = np.zeros(B, np.int32)
    stats = np.zeros((B * R, 2), np.float32)
    probs = np.zeros((B, R, V), np.float32) if want_probs else None
    rc = lib().or_spec_accept(_ptr(logits), B, gamma, V, _ptr(q), _ptr(dtok), _ptr(temps),
                              _ptr(tk), _ptr(tp), _ptr(ua), _ptr(ur), m, _ptr(nacc), _ptr(out),
                              _ptr(olen), _ptr(stats), _ptr(probs))
    assert rc == 0
    res = dict(num_accepted=nacc, out_tokens=out, out_len=olen, row_stats=stats)
    if want_probs:
        res["probs"] = probs
    return res


def sampler(logits, temperatures=None, top_ks=None, top_ps=None, mode="reference",
            uniforms=None, want_probs=True):
    m = _MODES[mode] if isinstance(mode, str) else int(mode)
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    rows, V = logits.shape
    temps = np.ascontiguousarray(temperatures if temperatures is not None else np.ones(rows),
                                 dtype=np.float32)
    tk = None if top_ks is None else np.ascontiguousarray(top_ks, dtype=np.int32)
    tp = None if top_ps is None else np.ascontiguousarray(top_ps, dtype=np.float32)
    probs = np.zeros((rows, V), np.float32) if (want_probs and m != MODE_GREEDY) else None
    un = None if uniforms is None else np.ascontiguousarray(uniforms, dtype=np.float32)
    toks = np.zeros(rows, np.int64) if (un is not None or m == MODE_GREEDY) else None
    stats = np.zeros((rows, 2), np.float32)
    rc = lib().or_sampler(_ptr(logits), rows, V, _ptr(temps), _ptr(tk), _ptr(tp), m, _ptr(probs),
                          _ptr(un), _ptr(toks), _ptr(stats))
    assert rc == 0
    return dict(probs=probs, tokens=toks, row_stats=stats)


def filter_keep(logits_row, temperature=1.0, top_k=0, top_p=1.0):
    """Kept mask of Sampler's top-k then top-p filters on one row."""
    x = np.ascontiguousarray(logits_row, dtype=np.float32)
    keep = np.zeros(x.shape[0], np.uint8)
    M = ctypes.c_float()
    S = ctypes.c_float()
    n = lib().or_filter_keep(x, x.shape[0], float(temperature), int(top_k), float(top_p), keep,
                             ctypes.byref(M), ctypes.byref(S))
    return keep.astype(bool), n, M.value, S.value
