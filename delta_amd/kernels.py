"""Torch-tensor wrappers over the C ABI (device memory and streams come from torch).

Every wrapper validates shapes, dtypes, devices and strides on the host before
it launches, so a kernel never sees an operand that disagrees with its grid.
All outputs and workspaces are caller-provided or allocated here *outside*
any graph capture; the kernels themselves never allocate or synchronise.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib

PAGE_SIZE = 16
HEAD_DIM = 128

_DTYPES = {torch.bfloat16: _lib.DELTA_BF16, torch.float16: _lib.DELTA_FP16}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected bfloat16 or float16") from None


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(device: torch.device):
    return torch.cuda.current_stream(device).cuda_stream


def _check_cuda(*tensors, device=None):
    dev = device
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("delta_amd kernels need GPU tensors")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {t.device} vs {dev}")
    return dev


def _check_i32(name: str, t: torch.Tensor, min_numel: int = 0):
    if t.dtype != torch.int32:
        raise TypeError(f"{name} must be int32, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.numel() < min_numel:
        raise ValueError(f"{name} needs >= {min_numel} entries, has {t.numel()}")


def _check_cache(kv_cache: torch.Tensor):
    if kv_cache.dim() != 5 or kv_cache.shape[1] != 2 or kv_cache.shape[2] != PAGE_SIZE \
            or kv_cache.shape[4] != HEAD_DIM:
        raise ValueError(f"kv_cache must be [pages, 2, 16, Hkv, 128], got {tuple(kv_cache.shape)}")
    if not kv_cache.is_contiguous():
        raise ValueError("kv_cache must be contiguous")
    _dtype_code(kv_cache)


def _check_heads(q: torch.Tensor, kv_cache: torch.Tensor):
    if q.dim() != 3 or q.shape[2] != HEAD_DIM:
        raise ValueError(f"q must be [batch, Hq, 128], got {tuple(q.shape)}")
    if q.stride(2) != 1 or q.stride(1) % 8 or q.stride(0) % 8:
        raise ValueError("q needs a unit inner stride and strides in multiples of 8 elements")
    if q.dtype != kv_cache.dtype:
        raise TypeError(f"q dtype {q.dtype} != kv_cache dtype {kv_cache.dtype}")
    hq, hkv = q.shape[1], kv_cache.shape[3]
    if hq % hkv or hq // hkv > 8:
        raise ValueError(f"num_qo_heads={hq} must be a multiple of num_kv_heads={hkv}, group <= 8")
    return hq, hkv


class Workspace:
    """Grow-only device scratch buffer (allocate before any graph capture).  A buffer that a
    larger request replaces is kept alive, not freed: a graph captured earlier still holds its
    address and may be replayed."""

    def __init__(self):
        self._buf: dict = {}
        self._retired: list = []

    def get(self, nbytes: int, device: torch.device) -> torch.Tensor:
        nbytes = max(int(nbytes), 256)
        key = (device.type, device.index)
        buf = self._buf.get(key)
        if buf is None or buf.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("workspace must be sized before graph capture")
            if buf is not None:
                self._retired.append(buf)
            buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
            self._buf[key] = buf
        return buf


_default_ws = Workspace()


def decode_workspace_bytes(batch: int, hq: int, hkv: int, max_pages: int) -> int:
    return int(_lib.query("delta_paged_decode_workspace_bytes", batch, hq, hkv, max_pages))


@dataclass
class DecodeAppend:
    """The decode token's RoPE and KV append, fused into a ``paged_decode`` launch
    (``delta_decode_append_t``): q is then the un-rotated query, and row b's new token (k, v
    rows b, position ``offsets[b]`` for the rotation) is written at ``kv_len_b - 1`` of the
    cache's full CSR ``(kv_indptr, kv_indices)``, sharing ``kv_last_page_len`` with the
    attention.  Bit-identical to ``rope_append`` followed by the plain attention."""
    k: torch.Tensor
    v: torch.Tensor
    offsets: torch.Tensor
    kv_indptr: torch.Tensor
    kv_indices: torch.Tensor
    rope_scale: float = 1.0
    rope_theta: float = 1e4
    low_freq_factor: Optional[float] = None
    high_freq_factor: Optional[float] = None
    old_context_len: Optional[float] = None


def _append_struct(ap: "DecodeAppend", B: int, hkv: int, kv_cache: torch.Tensor):
    for name, t in (("k", ap.k), ("v", ap.v)):
        if t.dim() != 3 or tuple(t.shape) != (B, hkv, HEAD_DIM) or t.stride(2) != 1 or t.stride(1) != HEAD_DIM \
                or t.stride(0) % 2 or t.dtype != kv_cache.dtype or not t.is_cuda:
            raise ValueError(f"append.{name} must be [{B}, {hkv}, 128] of the cache dtype with contiguous heads")
    _check_i32("append.offsets", ap.offsets, B)
    _check_i32("append.kv_indptr", ap.kv_indptr, B + 1)
    _check_i32("append.kv_indices", ap.kv_indices)
    llama31 = ap.low_freq_factor is not None and ap.high_freq_factor is not None
    return _lib.DecodeAppendC(
        ap.k.data_ptr(), ap.k.stride(0), ap.v.data_ptr(), ap.v.stride(0), ap.offsets.data_ptr(),
        ap.kv_indptr.data_ptr(), ap.kv_indices.data_ptr(), ap.kv_indices.numel(), float(ap.rope_scale),
        float(ap.rope_theta), int(llama31), float(ap.low_freq_factor or 0.0), float(ap.high_freq_factor or 0.0),
        float(ap.old_context_len or 0.0))


def paged_decode(q: torch.Tensor, kv_cache: torch.Tensor, kv_indptr: torch.Tensor,
                 kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor, *,
                 max_pages_per_row: int, sm_scale: Optional[float] = None,
                 out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None,
                 logits_dump: Optional[torch.Tensor] = None,
                 workspace: Optional[torch.Tensor] = None, subset: bool = False,
                 append: Optional[DecodeAppend] = None) -> torch.Tensor:
    """Paged decode attention (``delta_paged_decode``); returns ``out`` [B, Hq, 128].

    ``logits_dump`` (fp32, [B_max, Hq, S] or any view with unit last stride)
    receives the planner-layer logits for ``t < kv_len``.  ``subset=True``
    runs the same attention through ``delta_paged_decode_subset`` (selected
    pages; no dump).  ``append`` fuses the decode token's RoPE and KV append in
    (``delta_paged_decode[_subset]_append``).
    """
    if subset and logits_dump is not None:
        raise ValueError("the subset attention writes no logits dump")
    dev = _check_cuda(q, kv_cache, kv_indptr, kv_indices, kv_last_page_len, out, lse, logits_dump)
    _check_cache(kv_cache)
    hq, hkv = _check_heads(q, kv_cache)
    B = q.shape[0]
    _check_i32("kv_indptr", kv_indptr, B + 1)
    _check_i32("kv_indices", kv_indices)
    _check_i32("kv_last_page_len", kv_last_page_len, B)
    if out is None:
        out = torch.empty_like(q)
    if out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1:
        raise ValueError("out must match q's shape/dtype with unit inner stride")
    if lse is not None and (lse.dtype != torch.float32 or lse.shape[0] < B or lse.shape[1] != hq
                            or not lse.is_contiguous()):
        raise ValueError("lse must be contiguous fp32 [>=B, Hq]")
    dsb = dsh = 0
    if logits_dump is not None:
        if logits_dump.dtype != torch.float32 or logits_dump.dim() != 3 or logits_dump.stride(2) != 1:
            raise ValueError("logits_dump must be fp32 [B, Hq, S] with unit last stride")
        if logits_dump.shape[0] < B or logits_dump.shape[1] != hq \
                or logits_dump.shape[2] < max_pages_per_row * PAGE_SIZE:
            raise ValueError(f"logits_dump {tuple(logits_dump.shape)} too small for "
                             f"B={B}, Hq={hq}, {max_pages_per_row} pages")
        dsb, dsh = logits_dump.stride(0), logits_dump.stride(1)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(HEAD_DIM)
    need = decode_workspace_bytes(B, hq, hkv, max_pages_per_row)
    if workspace is None:
        workspace = _default_ws.get(need, dev)
    elif workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace too small: {need} bytes needed")
    common_head = (q.data_ptr(), q.stride(0), q.stride(1), kv_cache.data_ptr(), kv_cache.shape[0],
                   kv_indptr.data_ptr(), kv_indices.data_ptr(), kv_indices.numel(), kv_last_page_len.data_ptr(),
                   out.data_ptr(), out.stride(0), out.stride(1), _ptr(lse))
    common_tail = (B, hq, hkv, HEAD_DIM, _dtype_code(q), float(sm_scale), int(max_pages_per_row),
                   workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream(dev))
    if append is not None:
        ap = ctypes.byref(_append_struct(append, B, hkv, kv_cache))
        if subset:
            _lib.call("delta_paged_decode_subset_append", ap, *common_head, *common_tail)
        else:
            _lib.call("delta_paged_decode_append", ap, *common_head, _ptr(logits_dump), dsb, dsh, *common_tail)
    elif subset:
        _lib.call("delta_paged_decode_subset", *common_head, *common_tail)
    else:
        _lib.call("delta_paged_decode", *common_head, _ptr(logits_dump), dsb, dsh, *common_tail)
    return out


def paged_decode_scores_supported(batch: int, num_qo_heads: int, num_kv_heads: int, max_pages_per_row: int,
                                  with_append: bool = False) -> bool:
    """True when ``paged_decode_scores`` applies to this shape (the rows' logits fit on chip)."""
    return bool(_lib.query("delta_paged_decode_scores_supported", int(batch), int(num_qo_heads),
                           int(num_kv_heads), int(max_pages_per_row), int(bool(with_append))))


def paged_decode_scores_workspace_bytes(batch: int, num_kv_heads: int, max_pages_per_row: int) -> int:
    """Workspace bytes of ``paged_decode_scores`` (its per-token maxima)."""
    return int(_lib.query("delta_paged_decode_scores_workspace_bytes", int(batch), int(num_kv_heads),
                          int(max_pages_per_row)))


def paged_decode_scores(q: torch.Tensor, kv_cache: torch.Tensor, kv_indptr: torch.Tensor,
                        kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor, *,
                        max_pages_per_row: int, sm_scale: Optional[float] = None,
                        out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None,
                        scores: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
                        append: Optional[DecodeAppend] = None):
    """The planner layer without a logits dump (``delta_paged_decode_scores[_append]``): full
    attention and the del3_legacy_softmax page scores in one pass; returns ``(out, scores)``,
    scores fp32 [B, max_pages_per_row].  Only where ``paged_decode_scores_supported``."""
    dev = _check_cuda(q, kv_cache, kv_indptr, kv_indices, kv_last_page_len, out, lse, scores)
    _check_cache(kv_cache)
    hq, hkv = _check_heads(q, kv_cache)
    B = q.shape[0]
    _check_i32("kv_indptr", kv_indptr, B + 1)
    _check_i32("kv_indices", kv_indices)
    _check_i32("kv_last_page_len", kv_last_page_len, B)
    if out is None:
        out = torch.empty_like(q)
    if out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1:
        raise ValueError("out must match q's shape/dtype with unit inner stride")
    if lse is not None and (lse.dtype != torch.float32 or lse.shape[0] < B or lse.shape[1] != hq
                            or not lse.is_contiguous()):
        raise ValueError("lse must be contiguous fp32 [>=B, Hq]")
    if scores is None:
        scores = torch.empty((B, max_pages_per_row), dtype=torch.float32, device=dev)
    if scores.dtype != torch.float32 or scores.stride(1) != 1 or scores.shape[0] < B \
            or scores.shape[1] < max_pages_per_row:
        raise ValueError("scores must be fp32 [>=B, >=max_pages_per_row]")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(HEAD_DIM)
    need = paged_decode_scores_workspace_bytes(B, hkv, max_pages_per_row)
    if workspace is None:
        workspace = _default_ws.get(need, dev)
    elif workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace too small: {need} bytes needed")
    args = (q.data_ptr(), q.stride(0), q.stride(1), kv_cache.data_ptr(), kv_cache.shape[0],
            kv_indptr.data_ptr(), kv_indices.data_ptr(), kv_indices.numel(), kv_last_page_len.data_ptr(),
            out.data_ptr(), out.stride(0), out.stride(1), _ptr(lse), scores.data_ptr(), scores.stride(0),
            B, hq, hkv, HEAD_DIM, _dtype_code(q), float(sm_scale), int(max_pages_per_row),
            workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream(dev))
    if append is not None:
        _lib.call("delta_paged_decode_scores_append",
                  ctypes.byref(_append_struct(append, B, hkv, kv_cache)), *args)
    else:
        _lib.call("delta_paged_decode_scores", *args)
    return out, scores


def paged_prefill(q: torch.Tensor, kv_cache: torch.Tensor, qo_indptr: torch.Tensor,
                  kv_indptr: torch.Tensor, kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor, *,
                  max_qo_len: int, sm_scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                  lse: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal paged prefill attention (``delta_paged_prefill``); q/out [nnz, Hq, 128]."""
    dev = _check_cuda(q, kv_cache, qo_indptr, kv_indptr, kv_indices, kv_last_page_len, out, lse)
    _check_cache(kv_cache)
    hq, hkv = _check_heads(q, kv_cache)
    B = qo_indptr.numel() - 1
    _check_i32("qo_indptr", qo_indptr, B + 1)
    _check_i32("kv_indptr", kv_indptr, B + 1)
    _check_i32("kv_indices", kv_indices)
    _check_i32("kv_last_page_len", kv_last_page_len, B)
    if out is None:
        out = torch.empty_like(q)
    if out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1:
        raise ValueError("out must match q's shape/dtype with unit inner stride")
    if lse is not None and (lse.dtype != torch.float32 or tuple(lse.shape) != (q.shape[0], hq)
                            or not lse.is_contiguous()):
        raise ValueError("lse must be contiguous fp32 [nnz, Hq]")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(HEAD_DIM)
    _lib.call("delta_paged_prefill", q.data_ptr(), q.stride(0), q.stride(1), kv_cache.data_ptr(),
              kv_cache.shape[0], qo_indptr.data_ptr(), kv_indptr.data_ptr(), kv_indices.data_ptr(),
              kv_indices.numel(), kv_last_page_len.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1),
              _ptr(lse), int(B), hq, hkv, HEAD_DIM, _dtype_code(q), float(sm_scale), int(max_qo_len), _stream(dev))
    return out


def page_scores_from_logits(logits_dump: torch.Tensor, kv_indptr: torch.Tensor,
                            kv_last_page_len: torch.Tensor, max_pages: int, *,
                            lse: Optional[torch.Tensor] = None,
                            scores: Optional[torch.Tensor] = None,
                            batch: Optional[int] = None,
                            workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """del3_legacy_softmax page scores from a logits dump; returns fp32 [B, max_pages]."""
    dev = _check_cuda(logits_dump, kv_indptr, kv_last_page_len, lse, scores)
    if logits_dump.dtype != torch.float32 or logits_dump.dim() != 3 or logits_dump.stride(2) != 1:
        raise ValueError("logits_dump must be fp32 [B, Hq, S] with unit last stride")
    B = int(batch if batch is not None else kv_indptr.numel() - 1)
    hq = logits_dump.shape[1]
    if logits_dump.shape[0] < B or logits_dump.shape[2] < max_pages * PAGE_SIZE:
        raise ValueError("logits_dump too small")
    _check_i32("kv_indptr", kv_indptr, B + 1)
    _check_i32("kv_last_page_len", kv_last_page_len, B)
    if scores is None:
        scores = torch.empty((B, max_pages), dtype=torch.float32, device=dev)
    if scores.dtype != torch.float32 or scores.stride(1) != 1 or scores.shape[0] < B \
            or scores.shape[1] < max_pages:
        raise ValueError("scores must be fp32 [>=B, >=max_pages] with unit inner stride")
    if lse is not None and (lse.dtype != torch.float32 or not lse.is_contiguous()
                            or lse.shape[0] < B or lse.shape[1] != hq):
        raise ValueError("lse must be contiguous fp32 [>=B, Hq]")
    need = int(_lib.query("delta_page_score_workspace_bytes", B, hq))
    if workspace is None:
        workspace = _default_ws.get(need, dev)
    _lib.call("delta_page_scores_from_logits",
              logits_dump.data_ptr(), logits_dump.stride(0), logits_dump.stride(1), _ptr(lse),
              kv_indptr.data_ptr(), kv_last_page_len.data_ptr(), scores.data_ptr(), scores.stride(0),
              B, hq, int(max_pages), workspace.data_ptr(),
              workspace.numel() * workspace.element_size(), _stream(dev))
    return scores


def page_score(q: torch.Tensor, kv_cache: torch.Tensor, kv_indptr: torch.Tensor,
               kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor, max_pages: int, *,
               sm_scale: Optional[float] = None, logits_dump: Optional[torch.Tensor] = None,
               scores: Optional[torch.Tensor] = None,
               workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Standalone scorer (K read once): returns fp32 page scores [B, max_pages].

    Without ``logits_dump`` the scorer keeps each row's logits on chip when the shape allows
    (``delta_page_score_needs_dump`` == 0: no dump written); otherwise a dump buffer is used."""
    dev = _check_cuda(q, kv_cache, kv_indptr, kv_indices, kv_last_page_len, logits_dump, scores)
    _check_cache(kv_cache)
    hq, hkv = _check_heads(q, kv_cache)
    B = q.shape[0]
    _check_i32("kv_indptr", kv_indptr, B + 1)
    _check_i32("kv_indices", kv_indices)
    _check_i32("kv_last_page_len", kv_last_page_len, B)
    if logits_dump is None and int(_lib.query("delta_page_score_needs_dump", B, hq, hkv, max_pages)):
        logits_dump = torch.empty((B, hq, max_pages * PAGE_SIZE), dtype=torch.float32, device=dev)
    if logits_dump is not None and (
            logits_dump.dtype != torch.float32 or logits_dump.dim() != 3 or logits_dump.stride(2) != 1
            or logits_dump.shape[0] < B or logits_dump.shape[1] != hq
            or logits_dump.shape[2] < max_pages * PAGE_SIZE):
        raise ValueError("logits_dump must be fp32 [>=B, Hq, >=max_pages*16] with unit last stride")
    if scores is None:
        scores = torch.empty((B, max_pages), dtype=torch.float32, device=dev)
    if scores.dtype != torch.float32 or scores.stride(1) != 1 or scores.shape[0] < B \
            or scores.shape[1] < max_pages:
        raise ValueError("scores must be fp32 [>=B, >=max_pages]")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(HEAD_DIM)
    need = int(_lib.query("delta_page_score_kv_workspace_bytes", B, hq, hkv, max_pages))
    if workspace is None:
        workspace = _default_ws.get(need, dev)
    _lib.call("delta_page_score",
              q.data_ptr(), q.stride(0), q.stride(1), kv_cache.data_ptr(), kv_cache.shape[0],
              kv_indptr.data_ptr(), kv_indices.data_ptr(), kv_indices.numel(),
              kv_last_page_len.data_ptr(), _ptr(logits_dump), 0 if logits_dump is None else logits_dump.stride(0),
              0 if logits_dump is None else logits_dump.stride(1), scores.data_ptr(), scores.stride(0),
              B, hq, hkv, HEAD_DIM, _dtype_code(q), float(sm_scale), int(max_pages),
              workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream(dev))
    return scores


def select_pages(scores: torch.Tensor, kv_indptr: torch.Tensor, block_table: torch.Tensor,
                 k: int, L: int, *, pos_bias_scale: float = 1e-7, fixed_count: bool = False,
                 batch: Optional[int] = None, max_pages: Optional[int] = None,
                 k_per_row: Optional[torch.Tensor] = None,
                 use_subset: Optional[torch.Tensor] = None,
                 out_indices: Optional[torch.Tensor] = None,
                 out_indptr: Optional[torch.Tensor] = None):
    """PageSelectorV2 selection (``delta_select_pages``) -> (indices, indptr) int32.

    ``out_indices`` is returned whole (callers slice with ``indptr[-1]``); when
    allocated here it holds ``batch * k`` entries (or the full page count when
    ``use_subset`` may be 0).
    """
    dev = _check_cuda(scores, kv_indptr, block_table, k_per_row, use_subset, out_indices, out_indptr)
    B = int(batch if batch is not None else kv_indptr.numel() - 1)
    n = int(max_pages if max_pages is not None else scores.shape[1])
    if scores.dtype != torch.float32 or scores.stride(1) != 1 or scores.shape[0] < B or scores.shape[1] < n:
        raise ValueError("scores must be fp32 [>=B, >=max_pages] with unit inner stride")
    _check_i32("kv_indptr", kv_indptr, B + 1)
    if block_table.dtype != torch.int32 or block_table.stride(1) != 1 or block_table.shape[0] < B \
            or block_table.shape[1] < n:
        raise ValueError("block_table must be int32 [>=B, >=max_pages] with unit inner stride")
    if k_per_row is not None:
        _check_i32("k_per_row", k_per_row, B)
    if use_subset is not None:
        _check_i32("use_subset", use_subset, 1)
    if k_per_row is None and k > n:
        raise RuntimeError("selected index k out of range")
    if out_indptr is None:
        out_indptr = torch.empty(B + 1, dtype=torch.int32, device=dev)
    _check_i32("out_indptr", out_indptr, B + 1)
    if out_indices is None:
        cap = B * max(int(k), 1) if k_per_row is None else int(k_per_row.sum())
        if use_subset is not None:
            cap = max(cap, B * n)
        out_indices = torch.empty(max(cap, 1), dtype=torch.int32, device=dev)
    _check_i32("out_indices", out_indices)
    _lib.call("delta_select_pages",
              scores.data_ptr(), scores.stride(0), kv_indptr.data_ptr(), block_table.data_ptr(),
              block_table.stride(0), B, n, int(k), _ptr(k_per_row), int(L), float(pos_bias_scale),
              int(bool(fixed_count)), _ptr(use_subset), out_indices.data_ptr(), out_indices.numel(),
              out_indptr.data_ptr(), _stream(dev))
    return out_indices, out_indptr


def pack_page_indices(slot_block_table: torch.Tensor, active_slots: torch.Tensor,
                      start_cols: torch.Tensor, counts: torch.Tensor, indptr: torch.Tensor,
                      out_indices: torch.Tensor, row_block_table: torch.Tensor, n_rows: int,
                      max_count: int, *, write_row_block: bool) -> None:
    """In-place page-list pack (``delta_pack_page_indices``, page_metadata.py:42-70)."""
    if n_rows <= 0 or max_count <= 0:
        return
    dev = _check_cuda(slot_block_table, active_slots, start_cols, counts, indptr, out_indices,
                      row_block_table)
    for name, t in (("slot_block_table", slot_block_table), ("active_slots", active_slots),
                    ("start_cols", start_cols), ("counts", counts), ("indptr", indptr),
                    ("out_indices", out_indices)):
        _check_i32(name, t)
    if write_row_block:
        _check_i32("row_block_table", row_block_table)
    if write_row_block and row_block_table.numel() < n_rows * slot_block_table.shape[1]:
        raise ValueError("row_block_table too small")
    if active_slots.numel() < n_rows or start_cols.numel() < n_rows or counts.numel() < n_rows \
            or indptr.numel() < n_rows:
        raise ValueError("metadata arrays shorter than n_rows")
    _lib.call("delta_pack_page_indices",
              slot_block_table.data_ptr(), int(slot_block_table.shape[0]), active_slots.data_ptr(),
              start_cols.data_ptr(), counts.data_ptr(), indptr.data_ptr(), out_indices.data_ptr(),
              out_indices.numel(), _ptr(row_block_table) if write_row_block else None, int(n_rows),
              int(slot_block_table.shape[1]), int(max_count), int(bool(write_row_block)),
              _stream(dev))


def decode_page_info(cachelens: torch.Tensor, slot_block_table: torch.Tensor, batch: int, k: int,
                     compression_ratio: float, selective: bool, kv_indptr: torch.Tensor,
                     kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor,
                     row_block_table: Optional[torch.Tensor] = None,
                     subset_indices: Optional[torch.Tensor] = None,
                     subset_indptr: Optional[torch.Tensor] = None,
                     use_subset: Optional[torch.Tensor] = None,
                     active: Optional[torch.Tensor] = None,
                     k_per_row: Optional[torch.Tensor] = None,
                     budget_rule: Optional[tuple] = None) -> None:
    """Device-side decode page info for rows 0..batch-1 (``delta_decode_page_info``).

    ``active`` (int32 [batch], optional) marks the rows the ``use_subset`` gate counts; idle
    rows still get their CSR entries.  ``k_per_row`` (int32 [batch], optional) gives each row
    its own subset budget in place of ``k``.  ``budget_rule`` = ``(min_tokens, divisor, out)``
    derives each row's budget from its length instead, ``max(min_tokens, kv_len // divisor) // 16``
    pages clamped to [1, k], and writes them to ``out`` (int32 [batch]) for ``select_pages``."""
    rule_out = budget_rule[2] if budget_rule is not None else None
    dev = _check_cuda(cachelens, slot_block_table, kv_indptr, kv_indices, kv_last_page_len,
                      row_block_table, subset_indices, subset_indptr, use_subset, active, k_per_row, rule_out)
    pps = slot_block_table.shape[1]
    _check_i32("cachelens", cachelens, batch)
    if active is not None:
        _check_i32("active", active, batch)
    _check_i32("slot_block_table", slot_block_table, batch * pps)
    _check_i32("kv_indptr", kv_indptr, batch + 1)
    _check_i32("kv_indices", kv_indices, batch * pps)
    _check_i32("kv_last_page_len", kv_last_page_len, batch)
    if row_block_table is not None:
        _check_i32("row_block_table", row_block_table, batch * pps)
        if row_block_table.shape[-1] != pps:
            raise ValueError("row_block_table must have pages_per_slot columns")
    if subset_indices is not None:
        _check_i32("subset_indices", subset_indices, batch * pps)
        _check_i32("subset_indptr", subset_indptr, batch + 1)
    if use_subset is not None:
        _check_i32("use_subset", use_subset, 1)
    if k_per_row is not None:
        _check_i32("k_per_row", k_per_row, batch)
    rule = None
    if budget_rule is not None:
        if k_per_row is not None:
            raise ValueError("budget_rule and k_per_row are exclusive")
        min_tokens, divisor, out = budget_rule
        _check_i32("budget_rule out", out, batch)
        rule = ctypes.byref(_lib.BudgetRuleC(int(min_tokens), int(divisor), out.data_ptr()))
    _lib.call("delta_decode_page_info",
              cachelens.data_ptr(), _ptr(active), slot_block_table.data_ptr(), int(batch), int(pps), int(k),
              _ptr(k_per_row), rule, float(compression_ratio), int(bool(selective)), kv_indptr.data_ptr(),
              kv_indices.data_ptr(), kv_last_page_len.data_ptr(), _ptr(row_block_table),
              _ptr(subset_indices), _ptr(subset_indptr), _ptr(use_subset), _stream(dev))


def append_kv(k: torch.Tensor, v: torch.Tensor, kv_append_indptr: torch.Tensor,
              kv_cache: torch.Tensor, kv_indices: torch.Tensor, kv_indptr: torch.Tensor,
              kv_last_page_len: torch.Tensor) -> None:
    """In-place KV append (``delta_append_kv``, utils.py:31-79)."""
    dev = _check_cuda(k, v, kv_append_indptr, kv_cache, kv_indices, kv_indptr, kv_last_page_len)
    _check_cache(kv_cache)
    hkv = kv_cache.shape[3]
    for name, t in (("k", k), ("v", v)):
        if t.dim() != 3 or t.shape[1] != hkv or t.shape[2] != HEAD_DIM or t.stride(2) != 1 \
                or t.stride(1) != HEAD_DIM or t.stride(0) % 8:
            raise ValueError(f"{name} must be [nnz, {hkv}, 128] with contiguous heads")
        if t.dtype != kv_cache.dtype:
            raise TypeError(f"{name} dtype must match kv_cache")
    nnz = k.shape[0]
    if v.shape[0] != nnz:
        raise ValueError("k and v token counts differ")
    B = kv_append_indptr.numel() - 1
    _check_i32("kv_append_indptr", kv_append_indptr)
    _check_i32("kv_indices", kv_indices)
    _check_i32("kv_indptr", kv_indptr, B + 1)
    _check_i32("kv_last_page_len", kv_last_page_len, B)
    _lib.call("delta_append_kv",
              k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0), kv_append_indptr.data_ptr(),
              kv_cache.data_ptr(), kv_cache.shape[0], kv_indices.data_ptr(), kv_indices.numel(),
              kv_indptr.data_ptr(), kv_last_page_len.data_ptr(), int(nnz), int(B), int(hkv),
              HEAD_DIM, _dtype_code(kv_cache), _stream(dev))


def rope(q: torch.Tensor, k: torch.Tensor, indptr: torch.Tensor, offsets: torch.Tensor, *,
         rope_scale: float = 1.0, rope_theta: float = 1e4,
         low_freq_factor: Optional[float] = None, high_freq_factor: Optional[float] = None,
         old_context_len: Optional[float] = None,
         q_out: Optional[torch.Tensor] = None, k_out: Optional[torch.Tensor] = None):
    """Interleaved RoPE (``delta_rope``); returns (q_rope, k_rope)."""
    dev = _check_cuda(q, k, indptr, offsets, q_out, k_out)
    for name, t in (("q", q), ("k", k)):
        if t.dim() != 3 or t.shape[2] != HEAD_DIM or t.stride(2) != 1 or t.stride(1) != HEAD_DIM:
            raise ValueError(f"{name} must be [nnz, H, 128] with contiguous heads")
    if k.dtype != q.dtype or k.shape[0] != q.shape[0]:
        raise ValueError("q/k mismatch")
    q_out = torch.empty_like(q) if q_out is None else q_out
    k_out = torch.empty_like(k) if k_out is None else k_out
    for name, t, ref in (("q_out", q_out, q), ("k_out", k_out, k)):
        if t.shape != ref.shape or t.dtype != ref.dtype or t.stride(2) != 1 or t.stride(1) != HEAD_DIM:
            raise ValueError(f"{name} must match its input's shape with contiguous heads")
    B = indptr.numel() - 1
    _check_i32("indptr", indptr, B + 1)
    _check_i32("offsets", offsets, B)
    llama31 = low_freq_factor is not None and high_freq_factor is not None
    _lib.call("delta_rope",
              q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), q_out.data_ptr(),
              q_out.stride(0), k_out.data_ptr(), k_out.stride(0), indptr.data_ptr(),
              offsets.data_ptr(), int(q.shape[0]), int(B), int(q.shape[1]), int(k.shape[1]),
              HEAD_DIM, _dtype_code(q), float(rope_scale), float(rope_theta), int(llama31),
              float(low_freq_factor or 0.0), float(high_freq_factor or 0.0),
              float(old_context_len or 0.0), _stream(dev))
    return q_out, k_out


def rope_append(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_append_indptr: torch.Tensor,
                offsets: torch.Tensor, kv_cache: torch.Tensor, kv_indices: torch.Tensor,
                kv_indptr: torch.Tensor, kv_last_page_len: torch.Tensor, *, rope_scale: float = 1.0,
                rope_theta: float = 1e4, low_freq_factor: Optional[float] = None,
                high_freq_factor: Optional[float] = None, old_context_len: Optional[float] = None,
                q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``rope`` then ``append_kv`` in one launch (``delta_rope_append``); returns the rotated q."""
    dev = _check_cuda(q, k, v, kv_append_indptr, offsets, kv_cache, kv_indices, kv_indptr, kv_last_page_len, q_out)
    _check_cache(kv_cache)
    hkv = kv_cache.shape[3]
    if q.dim() != 3 or q.shape[2] != HEAD_DIM or q.stride(2) != 1 or q.stride(1) != HEAD_DIM:
        raise ValueError("q must be [nnz, Hq, 128] with contiguous heads")
    for name, t in (("k", k), ("v", v)):
        if t.dim() != 3 or t.shape[1] != hkv or t.shape[2] != HEAD_DIM or t.stride(2) != 1 \
                or t.stride(1) != HEAD_DIM or (name == "v" and t.stride(0) % 8) or t.shape[0] != q.shape[0]:
            raise ValueError(f"{name} must be [nnz, {hkv}, 128] with contiguous heads (v rows 16-byte aligned)")
        if t.dtype != kv_cache.dtype or q.dtype != kv_cache.dtype:
            raise TypeError("q, k, v and kv_cache must share a dtype")
    q_out = torch.empty_like(q) if q_out is None else q_out
    if q_out.shape != q.shape or q_out.dtype != q.dtype or q_out.stride(2) != 1 or q_out.stride(1) != HEAD_DIM:
        raise ValueError("q_out must match q's shape with contiguous heads")
    B = kv_append_indptr.numel() - 1
    _check_i32("kv_append_indptr", kv_append_indptr, B + 1)
    _check_i32("offsets", offsets, B)
    _check_i32("kv_indices", kv_indices)
    _check_i32("kv_indptr", kv_indptr, B + 1)
    _check_i32("kv_last_page_len", kv_last_page_len, B)
    llama31 = low_freq_factor is not None and high_freq_factor is not None
    _lib.call("delta_rope_append",
              q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0), q_out.data_ptr(),
              q_out.stride(0), kv_append_indptr.data_ptr(), offsets.data_ptr(), kv_cache.data_ptr(),
              kv_cache.shape[0], kv_indices.data_ptr(), kv_indices.numel(), kv_indptr.data_ptr(),
              kv_last_page_len.data_ptr(), int(q.shape[0]), int(B), int(q.shape[1]), int(hkv), HEAD_DIM,
              _dtype_code(q), float(rope_scale), float(rope_theta), int(llama31), float(low_freq_factor or 0.0),
              float(high_freq_factor or 0.0), float(old_context_len or 0.0), _stream(dev))
    return q_out


def argmax_rows(logits: torch.Tensor, out: Optional[torch.Tensor] = None,
                workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """First index of each row's maximum (``delta_argmax_rows``); logits [rows, cols]."""
    dev = _check_cuda(logits, out, workspace)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [rows, cols] with unit inner stride")
    rows, cols = logits.shape
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=dev)
    if out.dtype != torch.int64 or out.dim() != 1 or out.shape[0] < rows:
        raise ValueError("out must be int64 [>=rows]")
    need = int(_lib.query("delta_argmax_workspace_bytes", rows))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    nbytes = workspace.numel() * workspace.element_size()
    _lib.call("delta_argmax_rows", logits.data_ptr(), logits.stride(0), int(rows), int(cols),
              _dtype_code(logits), out.data_ptr(), out.stride(0), workspace.data_ptr(), nbytes, _stream(dev))
    return out


def _rows2d(name: str, t: torch.Tensor, dim: int) -> torch.Tensor:
    t2 = t.reshape(-1, dim)
    if t2.stride(1) != 1 or t2.stride(0) % 8 or t2.data_ptr() % 16:
        raise ValueError(f"{name} must have 16-byte aligned contiguous rows")
    return t2


def add_rmsnorm(x: torch.Tensor, residual: Optional[torch.Tensor], weight: torch.Tensor, eps: float,
                out: Optional[torch.Tensor] = None):
    """(x + residual, RMSNorm(x + residual) * weight) in one kernel (``delta_add_rmsnorm``).

    ``residual`` may also be the fp32 partials ``[S, rows, dim]`` of a split-K
    ``gemm_rows32`` (``delta_add_rmsnorm_partials``: summed and rounded to x's dtype first).
    Returns ``(h, y)``; ``h`` is ``x`` itself when ``residual`` is None."""
    dev = _check_cuda(x, residual, weight, out)
    dim = x.shape[-1]
    _dtype_code(x)
    if weight.dtype != x.dtype or weight.numel() != dim or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous [dim] tensor of x's dtype")
    x2 = _rows2d("x", x, dim)
    rows = x2.shape[0]
    if residual is not None and residual.dtype == torch.float32 and x.dtype != torch.float32:
        if residual.dim() != 3 or tuple(residual.shape[1:]) != (rows, dim) or not residual.is_contiguous():
            raise ValueError(f"partials must be contiguous fp32 [S, {rows}, {dim}]")
        h = torch.empty_like(x)
        h2 = _rows2d("h", h, dim)
        if out is None:
            out = torch.empty_like(x)
        o2 = _rows2d("out", out, dim)
        _lib.call("delta_add_rmsnorm_partials", x2.data_ptr(), x2.stride(0), residual.data_ptr(),
                  int(residual.shape[0]), weight.data_ptr(), float(eps), h2.data_ptr(), h2.stride(0),
                  o2.data_ptr(), o2.stride(0), int(rows), int(dim), _dtype_code(x), _stream(dev))
        return h, out
    h = x if residual is None else torch.empty_like(x)
    r2 = None if residual is None else _rows2d("residual", residual, dim)
    h2 = None if residual is None else _rows2d("h", h, dim)
    if out is None:
        out = torch.empty_like(x)
    o2 = _rows2d("out", out, dim)
    _lib.call("delta_add_rmsnorm", x2.data_ptr(), x2.stride(0), _ptr(r2), 0 if r2 is None else r2.stride(0),
              weight.data_ptr(), float(eps), _ptr(h2), 0 if h2 is None else h2.stride(0), o2.data_ptr(),
              o2.stride(0), int(rows), int(dim), _dtype_code(x), _stream(dev))
    return h, out


def silu_mul(gate_up: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """silu(gate) * up of a ``[..., 2 * inter]`` gate|up tensor (``delta_silu_mul``)."""
    dev = _check_cuda(gate_up, out)
    inter = gate_up.shape[-1] // 2
    g2 = _rows2d("gate_up", gate_up, 2 * inter)
    if out is None:
        out = torch.empty(*gate_up.shape[:-1], inter, dtype=gate_up.dtype, device=dev)
    o2 = _rows2d("out", out, inter)
    _lib.call("delta_silu_mul", g2.data_ptr(), g2.stride(0), o2.data_ptr(), o2.stride(0), int(g2.shape[0]),
              int(inter), _dtype_code(gate_up), _stream(dev))
    return out


def gemm_skinny_ok(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """True when ``delta_gemm_skinny`` takes ``x @ weight.T``: decode-sized rows, K % 64 == 0,
    N % 16 == 0, 16-byte aligned rows of a bf16/fp16 weight of x's dtype."""
    if x.dtype not in _DTYPES or weight.dtype != x.dtype or weight.dim() != 2 or not x.is_cuda:
        return False
    N, Kd = weight.shape
    rows = x.numel() // max(x.shape[-1], 1)
    return (x.shape[-1] == Kd and Kd % 64 == 0 and N % 16 == 0 and 0 < rows <= 32
            and weight.stride(1) == 1 and weight.stride(0) % 8 == 0 and weight.data_ptr() % 16 == 0)


def gemm_rows32_splits(M: int, N: int, K: int) -> int:
    """K splits ``delta_gemm_rows32`` uses for this shape (1: rounded output; > 1: fp32 partials)."""
    return int(_lib.query("delta_gemm_rows32_splits", int(M), int(N), int(K)))


def gemm_rows32(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None, partials: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``x @ weight.T (+ bias)`` for <= 32 token rows on ``delta_gemm_rows32``.

    Returns the rounded output ``[..., N]`` when the shape runs unsplit, else the fp32 partials
    ``[S, M, N]`` whose sum over S is the product (bias included once)."""
    dev = _check_cuda(x, weight, bias, out, partials)
    N, Kd = weight.shape
    if x.shape[-1] != Kd:
        raise ValueError(f"x has {x.shape[-1]} features, weight expects {Kd}")
    if weight.dtype != x.dtype or (bias is not None and (bias.dtype != x.dtype or bias.numel() != N
                                                         or not bias.is_contiguous())):
        raise TypeError("x, weight and bias must share a dtype; bias must be contiguous [N]")
    if weight.stride(1) != 1:
        raise ValueError("weight rows must be contiguous")
    x2 = _rows2d("x", x, Kd)
    M = x2.shape[0]
    S = gemm_rows32_splits(M, N, Kd)
    if S < 1:
        raise ValueError(f"delta_gemm_rows32 does not take [{M}, {Kd}] x [{N}, {Kd}]^T")
    o2 = None
    if S == 1:
        if out is None:
            out = torch.empty(*x.shape[:-1], N, dtype=x.dtype, device=dev)
        o2 = out.reshape(-1, N)
        if o2.stride(1) != 1 or o2.shape[0] != M:
            raise ValueError("out must be [..., N] with contiguous rows")
    else:
        if partials is None:
            partials = torch.empty(S, M, N, dtype=torch.float32, device=dev)
        if partials.dtype != torch.float32 or not partials.is_contiguous() or tuple(partials.shape) != (S, M, N):
            raise ValueError(f"partials must be contiguous fp32 [{S}, {M}, {N}]")
    _lib.call("delta_gemm_rows32", x2.data_ptr(), x2.stride(0), weight.data_ptr(), weight.stride(0), _ptr(bias),
              o2.data_ptr() if o2 is not None else None, o2.stride(0) if o2 is not None else 0,
              partials.data_ptr() if S > 1 else None, int(M), int(N), int(Kd), _dtype_code(x), _stream(dev))
    return out if S == 1 else partials


def gemm_rows32_silu(x: torch.Tensor, w13: torch.Tensor, out: Optional[torch.Tensor] = None,
                     _entry: str = "delta_gemm_rows32_silu") -> torch.Tensor:
    """``silu(x @ w1.T) * (x @ w3.T)`` for <= 32 token rows in one launch (``delta_gemm_rows32_silu``);
    ``w13`` is the row-major merged ``[2 * inter, dim]`` weight (w1 rows, then w3 rows)."""
    dev = _check_cuda(x, w13, out)
    N2, Kd = w13.shape
    inter = N2 // 2
    if x.shape[-1] != Kd or N2 % 2:
        raise ValueError("x must be [..., dim] and w13 [2 * inter, dim]")
    if w13.dtype != x.dtype or w13.stride(1) != 1:
        raise ValueError("w13 must share x's dtype and have contiguous rows")
    x2 = _rows2d("x", x, Kd)
    M = x2.shape[0]
    if out is None:
        out = torch.empty(*x.shape[:-1], inter, dtype=x.dtype, device=dev)
    o2 = out.reshape(-1, inter)
    if o2.stride(1) != 1 or o2.shape[0] != M:
        raise ValueError("out must be [..., inter] with contiguous rows")
    _lib.call(_entry, x2.data_ptr(), x2.stride(0), w13.data_ptr(), w13.stride(0), o2.data_ptr(),
              o2.stride(0), int(M), int(inter), int(Kd), _dtype_code(x), _stream(dev))
    return out


def gemm_skinny_silu(x: torch.Tensor, w13: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The same fused gate/up GEMM + SiLU-mul for <= 8 token rows (``delta_gemm_skinny_silu``)."""
    return gemm_rows32_silu(x, w13, out, _entry="delta_gemm_skinny_silu")


def gemm_skinny(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``F.linear(x, weight, bias)`` for decode-sized x on ``delta_gemm_skinny``."""
    dev = _check_cuda(x, weight, bias, out)
    N, Kd = weight.shape
    if x.shape[-1] != Kd:
        raise ValueError(f"x has {x.shape[-1]} features, weight expects {Kd}")
    if weight.dtype != x.dtype or (bias is not None and (bias.dtype != x.dtype or bias.numel() != N
                                                         or not bias.is_contiguous())):
        raise TypeError("x, weight and bias must share a dtype; bias must be contiguous [N]")
    if weight.stride(1) != 1:
        raise ValueError("weight rows must be contiguous")
    x2 = _rows2d("x", x, Kd)
    M = x2.shape[0]
    if out is None:
        out = torch.empty(*x.shape[:-1], N, dtype=x.dtype, device=dev)
    o2 = out.reshape(-1, N)
    if o2.stride(1) != 1 or o2.shape[0] != M:
        raise ValueError("out must be [..., N] with contiguous rows")
    _lib.call("delta_gemm_skinny", x2.data_ptr(), x2.stride(0), weight.data_ptr(), weight.stride(0),
              _ptr(bias), o2.data_ptr(), o2.stride(0), int(M), int(N), int(Kd), _dtype_code(x), _stream(dev))
    return out
