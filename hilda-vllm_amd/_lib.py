"""ctypes binding of libhilda_spec.so (the C ABI declared in include/hilda_spec.h).

The library is built in-tree by build_lib.py. There is no fallback: if the
library is missing or a call fails, a RuntimeError is raised.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libhilda_spec.so"

HS_OK = 0
HS_ERR_SCRATCH_LIMIT = -5
HS_F32, HS_BF16, HS_FP8_E4M3 = 0, 1, 2
HS_ACCEPT_REFERENCE, HS_ACCEPT_FILTERED, HS_ACCEPT_GREEDY = 0, 1, 2
HS_ACCEPT_TOPK_LE64 = 0x100
HS_ACCEPT_CHAIN = 0x200

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t
_f32 = ctypes.c_float

# name -> (restype, argtypes); every symbol declared in include/hilda_spec.h
SIGNATURES: dict[str, tuple] = {
    "hs_status_string": (ctypes.c_char_p, [_i32]),
    "hs_version": (_i32, []),
    "hs_spec_accept_workspace_size": (_sz, [_i32, _i32, _i32]),
    "hs_spec_accept": (_i32, [_vp, _i32, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp,
                              _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "hs_sampler_workspace_size": (_sz, [_i32, _i32]),
    "hs_sampler": (_i32, [_vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp, _i32, _vp, _i64, _i32,
                          _vp, _vp, _vp, _vp, _sz, _vp]),
    "hs_verify_attention_workspace_size": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "hs_verify_attention": (_i32, [_vp, _i64, _i64, _vp, _vp, _i32, _i64, _i64, _i64, _f32, _f32,
                                   _vp, _i64, _i32, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _i32,
                                   _i32, _i32, _f32, _vp, _i64, _i64, _vp, _sz, _vp]),
    "hs_verify_attention_noalloc": (_i32, [_vp, _i64, _i64, _vp, _vp, _i32, _i64, _i64, _i64,
                                           _f32, _f32, _vp, _i64, _i32, _i32, _vp, _vp, _i32,
                                           _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp, _i64,
                                           _i64, _vp]),
    "hs_verify_attention_noalloc_scratch_bytes": (_sz, []),
    "hs_store_kvcache": (_i32, [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i32, _i64, _i64,
                                _i64, _f32, _f32, _vp, _i32, _i32, _i32, _i32, _i32, _vp]),
}



class SpecState(ctypes.Structure):
    """Mirror of hs_spec_state (include/hilda_spec.h)."""
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "context_lens", "num_prompt", "max_tokens", "ignore_eos", "finished", "block_tables",
        "num_seq_blocks", "tokens", "free_ring", "free_hdr", "ref_count")] + [
        ("B", ctypes.c_int32), ("W", ctypes.c_int32), ("T", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32), ("block_size", ctypes.c_int32), ("pad", ctypes.c_int32),
        ("eos", ctypes.c_int64), ("block_hash", ctypes.c_void_p)]


_sp = ctypes.POINTER(SpecState)


class CommitNextArgs(ctypes.Structure):
    """Mirror of hs_commit_next_args (include/hilda_spec.h)."""
    _fields_ = [("state", _sp), ("eligible", _vp), ("workspace", _vp),
                ("workspace_bytes", ctypes.c_size_t), ("next_gamma", ctypes.c_int32),
                ("lookback", ctypes.c_int32)] + [(n, _vp) for n in (
        "status", "input_ids", "positions", "slot_mapping", "cu_seqlens_q", "cu_seqlens_k",
        "v_input_ids", "v_positions", "v_slot_mapping", "v_cu_seqlens_q", "v_cu_seqlens_k")]


SIGNATURES.update({
    "hs_spec_accept_commit_next": (_i32, [_vp, _i32, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _vp,
                                          _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp,
                                          _sz, ctypes.POINTER(CommitNextArgs), _vp]),
    "hs_spec_prealloc": (_i32, [_sp, _i32, _vp, _vp, _vp]),
    "hs_verify_prepare": (_i32, [_sp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "hs_draft_prepare": (_i32, [_sp, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "hs_spec_commit_workspace_size": (_sz, [_i32, _i32, _i32]),
    "hs_spec_commit": (_i32, [_sp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _sz, _vp]),
    "hs_spec_commit_next": (_i32, [_sp, _i32, _vp, _vp, _vp, _vp, _sz, _i32, _vp, _i32, _vp, _vp,
                                   _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "hs_zero_kv_slots": (_i32, [_vp, _i64, _i32, _i64, _i64, _i64, _vp, _i32, _vp]),
    "hs_linear": (_i32, [_vp, _i64, _vp, _i32, _i32, _i32, _i32, _vp, _i64, _vp]),
    "hs_rmsnorm": (_i32, [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i32, _i32, _f32, _vp]),
    "hs_qk_norm_rope": (_i32, [_vp, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _f32, _vp, _vp,
                               _i32, _vp]),
    "hs_silu_mul": (_i32, [_vp, _i64, _i32, _vp, _i64, _i32, _vp]),
    "hs_linear_rmsnorm": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _f32, _vp, _i32, _i32,
                                 _i32, _i32, _vp, _i64, _vp]),
    "hs_qk_norm_rope_store": (_i32, [_vp, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _f32, _vp,
                                     _vp, _vp, _i32, _i64, _i64, _i64, _f32, _f32, _vp, _i32,
                                     _i32, _i32, _vp]),
    "hs_qk_norm_rope_attend": (_i32, [_vp, _i64, _i32, _vp, _vp, _vp, _i32, _vp, _f32, _vp, _vp,
                                      _vp, _vp, _i32, _i64, _i64, _i64, _f32, _f32, _vp, _i64,
                                      _i32, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32,
                                      _i32, _f32, _vp, _i64, _i64, _vp, _sz, _vp]),
})

_lib = None


def lib() -> ctypes.CDLL:
    """Loads the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run `python hilda-vllm_amd/build_lib.py` "
                "(or __graft_entry__.build())")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int, what: str) -> None:
    if status != HS_OK:
        msg = lib().hs_status_string(status).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {status})")
