"""ctypes binding of the C ABI in ``include/delta_hip.h`` (``delta_amd/_delta_hip.so``).

There is no fallback: if the library is missing every kernel call raises.
"""
from __future__ import annotations

import ctypes
from ctypes import c_double, c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_delta_hip.so"

DELTA_BF16 = 0
DELTA_FP16 = 1
ABI_VERSION = 202  # delta_abi_version() of the library these signatures describe

_P = c_void_p


class DecodeAppendC(ctypes.Structure):
    """``delta_decode_append_t``: the new decode token's RoPE + KV append."""
    _fields_ = [("k", c_void_p), ("k_stride", c_int64), ("v", c_void_p), ("v_stride", c_int64),
                ("offsets", c_void_p), ("kv_indptr", c_void_p), ("kv_indices", c_void_p),
                ("kv_indices_len", c_int64), ("rope_scale", c_float), ("rope_theta", c_float),
                ("llama31", c_int), ("low_freq_factor", c_float), ("high_freq_factor", c_float),
                ("old_context_len", c_float)]


_AP = ctypes.POINTER(DecodeAppendC)


class BudgetRuleC(ctypes.Structure):
    """``delta_budget_rule_t``: per-row budgets max(min_tokens, kv_len / divisor) tokens."""
    _fields_ = [("min_tokens", c_int), ("divisor", c_int), ("out", c_void_p)]


_BR = ctypes.POINTER(BudgetRuleC)
# name -> (restype, argtypes); one entry per function declared in include/delta_hip.h
SIGNATURES = {
    "delta_last_error": (ctypes.c_char_p, []),
    "delta_abi_version": (c_int, []),
    "delta_decode_num_splits": (c_int, [c_int, c_int, c_int]),
    "delta_paged_decode_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "delta_paged_prefill": (c_int, [
        _P, c_int64, c_int64, _P, c_int64, _P, _P, _P, c_int64, _P, _P, c_int64, c_int64, _P,
        c_int, c_int, c_int, c_int, c_int, c_float, c_int, _P]),
    "delta_paged_decode": (c_int, [
        _P, c_int64, c_int64,                 # q, strides
        _P, c_int64,                          # kv_cache, num_pages
        _P, _P, c_int64, _P,                  # indptr, indices, indices_len, last_page_len
        _P, c_int64, c_int64, _P,             # o, strides, lse
        _P, c_int64, c_int64,                 # dump, strides
        c_int, c_int, c_int, c_int, c_int,    # batch, hq, hkv, head_dim, dtype
        c_float, c_int,                       # sm_scale, max_pages_per_row
        _P, c_size_t, _P]),                   # workspace, bytes, stream
    "delta_paged_decode_noalloc": (c_int, [
        _P, c_int64, c_int64, _P, c_int64, _P, _P, c_int64, _P, _P, c_int64, c_int64, _P, _P, c_int64, c_int64,
        c_int, c_int, c_int, c_int, c_int, c_float, c_int, _P]),
    "delta_paged_decode_append": (c_int, [
        _AP, _P, c_int64, c_int64, _P, c_int64, _P, _P, c_int64, _P, _P, c_int64, c_int64, _P, _P, c_int64,
        c_int64, c_int, c_int, c_int, c_int, c_int, c_float, c_int, _P, c_size_t, _P]),
    "delta_paged_decode_subset_append": (c_int, [
        _AP, _P, c_int64, c_int64, _P, c_int64, _P, _P, c_int64, _P, _P, c_int64, c_int64, _P,
        c_int, c_int, c_int, c_int, c_int, c_float, c_int, _P, c_size_t, _P]),
    "delta_paged_decode_subset": (c_int, [
        _P, c_int64, c_int64, _P, c_int64, _P, _P, c_int64, _P, _P, c_int64, c_int64, _P,
        c_int, c_int, c_int, c_int, c_int, c_float, c_int, _P, c_size_t, _P]),
    "delta_page_score_workspace_bytes": (c_size_t, [c_int, c_int]),
    "delta_page_scores_from_logits": (c_int, [
        _P, c_int64, c_int64, _P, _P, _P, _P, c_int64, c_int, c_int, c_int, _P, c_size_t, _P]),
    "delta_page_score_kv_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "delta_page_score_needs_dump": (c_int, [c_int, c_int, c_int, c_int]),
    "delta_page_score": (c_int, [
        _P, c_int64, c_int64, _P, c_int64, _P, _P, c_int64, _P,
        _P, c_int64, c_int64, _P, c_int64,
        c_int, c_int, c_int, c_int, c_int, c_float, c_int, _P, c_size_t, _P]),
    "delta_paged_decode_scores_supported": (c_int, [c_int, c_int, c_int, c_int, c_int]),
    "delta_paged_decode_scores_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "delta_paged_decode_scores": (c_int, [
        _P, c_int64, c_int64, _P, c_int64, _P, _P, c_int64, _P, _P, c_int64, c_int64, _P, _P, c_int64,
        c_int, c_int, c_int, c_int, c_int, c_float, c_int, _P, c_size_t, _P]),
    "delta_paged_decode_scores_append": (c_int, [
        _AP, _P, c_int64, c_int64, _P, c_int64, _P, _P, c_int64, _P, _P, c_int64, c_int64, _P, _P, c_int64,
        c_int, c_int, c_int, c_int, c_int, c_float, c_int, _P, c_size_t, _P]),
    "delta_select_pages": (c_int, [
        _P, c_int64, _P, _P, c_int64, c_int, c_int, c_int, _P, c_int, c_float, c_int, _P,
        _P, c_int64, _P, _P]),
    "delta_pack_page_indices": (c_int, [
        _P, c_int, _P, _P, _P, _P, _P, c_int64, _P, c_int, c_int, c_int, c_int, _P]),
    "delta_decode_page_info": (c_int, [
        _P, _P, _P, c_int, c_int, c_int, _P, _BR, c_double, c_int, _P, _P, _P, _P, _P, _P, _P, _P]),
    "delta_append_kv": (c_int, [
        _P, c_int64, _P, c_int64, _P, _P, c_int64, _P, c_int64, _P, _P, c_int, c_int, c_int,
        c_int, c_int, _P]),
    "delta_argmax_workspace_bytes": (c_size_t, [c_int]),
    "delta_argmax_rows": (c_int, [_P, c_int64, c_int, c_int, c_int, _P, c_int64, _P, c_size_t, _P]),
    "delta_add_rmsnorm": (c_int, [_P, c_int64, _P, c_int64, _P, c_float, _P, c_int64, _P, c_int64, c_int, c_int,
                                  c_int, _P]),
    "delta_add_rmsnorm_partials": (c_int, [_P, c_int64, _P, c_int, _P, c_float, _P, c_int64, _P, c_int64, c_int,
                                           c_int, c_int, _P]),
    "delta_silu_mul": (c_int, [_P, c_int64, _P, c_int64, c_int, c_int, c_int, _P]),
    "delta_gemm_skinny": (c_int, [_P, c_int64, _P, c_int64, _P, _P, c_int64, c_int, c_int, c_int, c_int, _P]),
    "delta_gemm_rows32_splits": (c_int, [c_int, c_int, c_int]),
    "delta_gemm_rows32": (c_int, [_P, c_int64, _P, c_int64, _P, _P, c_int64, _P, c_int, c_int, c_int, c_int, _P]),
    "delta_gemm_rows32_silu": (c_int, [_P, c_int64, _P, c_int64, _P, c_int64, c_int, c_int, c_int, c_int, _P]),
    "delta_gemm_skinny_silu": (c_int, [_P, c_int64, _P, c_int64, _P, c_int64, c_int, c_int, c_int, c_int, _P]),
    "delta_rope": (c_int, [
        _P, c_int64, _P, c_int64, _P, c_int64, _P, c_int64, _P, _P, c_int, c_int, c_int, c_int,
        c_int, c_int, c_float, c_float, c_int, c_float, c_float, c_float, _P]),
    "delta_rope_append": (c_int, [
        _P, c_int64, _P, c_int64, _P, c_int64, _P, c_int64, _P, _P, _P, c_int64, _P, c_int64, _P, _P,
        c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_float, c_int, c_float, c_float, c_float, _P]),
}

_lib = None


class DeltaHipError(RuntimeError):
    """A C-ABI call returned a non-zero status."""


def load() -> ctypes.CDLL:
    """Load the HIP library (raises if it was never built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"delta_amd HIP library missing at {LIB_PATH}; build it with "
                "`python -m delta_amd.build` (there is no CPU fallback)")
        lib = ctypes.CDLL(str(LIB_PATH))
        # The version first: a stale library may lack entry points these bindings name.
        ver_fn = getattr(lib, "delta_abi_version", None)
        ver = None
        if ver_fn is not None:
            ver_fn.restype = c_int
            ver_fn.argtypes = []
            ver = ver_fn()
        if ver != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {ver}, these bindings expect {ABI_VERSION}: rebuild it "
                               "with `python -m delta_amd.build`")
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Invoke a status-returning entry point; raise DeltaHipError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.delta_last_error().decode(errors="replace")
        raise DeltaHipError(f"{name} failed (status {rc}): {msg}")


def query(name: str, *args):
    """Invoke a sizing / version query that returns a plain value."""
    return getattr(load(), name)(*args)
