"""CPU oracle for DELTA's selective-KV decode hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``delta_amd/`` imports this module; only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker / the timed CPU baseline.

Every function restates, in plain PyTorch-CPU tensor math, one step of the
reference path (hoenza/DELTA, read as text under /root/reference).  The cited
``file:line`` is the reference code the function follows:

* paged KV layout and ``kv_len``      DELTA/Engine/DELTA/model.py:99-103,
                                      DELTA/Engine/DELTA/scheduler.py:60-74
* planner logits dump                 DELTA/Engine/DELTA/backend.py:175-222, 542
* del3_legacy_softmax page score      DELTA/Engine/DELTA/backend.py:887-904
* PageSelectorV2 prepare / select     DELTA/Engine/DELTA/page_selector_v2.py:49-69, 113-212
* paged decode attention (qo_len=1)   DELTA/Engine/DELTA/backend.py:461-512, 1091-1105
* page-index packer                   DELTA/Engine/DELTA/page_metadata.py:6-70
* KV append                           DELTA/Engine/utils.py:31-79
* RoPE (interleaved)                  DELTA/Engine/DELTA/model.py:152-175

Third-party arithmetic the reference calls but does not ship: FlashInfer 0.5.2
(README.md:47).  The dump, attention, append and RoPE steps restate FlashInfer's
published semantics at those call sites.

Pinning (the checks that make this restatement trustworthy) lives in
``tests/test_oracle_pinning.py``:
  - dump logits: pure-Python brute force on tiny shapes;
  - page score: pure-Python brute force, the closed forms sum(score)=1 for one
    head and sum(score) in [1, Hq], zero score past kv_len, invariance to the
    physical page permutation and to V;
  - selector: brute-force sort on (value desc, page asc), the structural
    invariants (row counts, forced last-L, ascending order, physical-id gather),
    fixed == general, monotonicity;
  - attention: torch SDPA on CPU, sparse == full when every page is selected,
    physical-permutation invariance;
  - packer / append: brute force over Python lists;
  - RoPE: closed forms (identity at position 0, pair norms kept, explicit
    angles) and, for the Llama-3.1 frequencies, Meta's published wavelength
    rule written independently in pure Python, inside the blend band, on both
    edges and outside it (a wrong smoothing coefficient fails it).
No reference test or golden vector exists for FlashInfer's RoPE kernel itself;
the published formula is what is pinned.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np
import torch

PAGE_SIZE = 16


# ---------------------------------------------------------------------------
# Page-table semantics
# ---------------------------------------------------------------------------

def kv_lengths(kv_indptr: torch.Tensor, kv_last_page_len: torch.Tensor,
               page_size: int = PAGE_SIZE) -> torch.Tensor:
    """Tokens held by each row: (pages - 1) * page_size + last_page_len.

    Follows scheduler.py:60-66 (``page_lastlen`` grows by qo_len; a full page
    allocates a fresh, empty one) and FlashInfer's ``get_seq_lens`` used at
    utils.py:49.  A row with zero pages holds ``last_page_len`` tokens.
    """
    indptr = kv_indptr.to(torch.int64)
    npages = indptr[1:] - indptr[:-1]
    return torch.clamp(npages - 1, min=0) * page_size + kv_last_page_len.to(torch.int64)


def gather_row_kv(kv_cache: torch.Tensor, kv_indptr: torch.Tensor,
                  kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor,
                  row: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """K and V of one row in logical token order, each [kv_len, Hkv, d].

    Cache layout ``[num_pages, 2, page_size, Hkv, d]`` (model.py:102): K at
    ``[:, 0]``, V at ``[:, 1]``.
    """
    page_size = kv_cache.shape[2]
    start, end = int(kv_indptr[row]), int(kv_indptr[row + 1])
    pages = kv_indices[start:end].to(torch.int64)
    n = int(kv_lengths(kv_indptr[row:row + 2], kv_last_page_len[row:row + 1], page_size)[0])
    if pages.numel() == 0:
        shape = (0,) + tuple(kv_cache.shape[3:])
        return kv_cache.new_zeros(shape), kv_cache.new_zeros(shape)
    k = kv_cache[pages, 0].reshape(-1, *kv_cache.shape[3:])[:n]
    v = kv_cache[pages, 1].reshape(-1, *kv_cache.shape[3:])[:n]
    return k, v


# ---------------------------------------------------------------------------
# Planner layer: logits dump + del3_legacy_softmax page score
# ---------------------------------------------------------------------------

def dump_logits(q: torch.Tensor, kv_cache: torch.Tensor, kv_indptr: torch.Tensor,
                kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor,
                sm_scale: float, max_len: int,
                compute_dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """fp32 ``x[b, h, t] = (q[b,h] . K[b, t, h // G]) * sm_scale``; -inf past kv_len.

    Restates the ``BatchDumpAttentionWeights`` logits transform
    (backend.py:175-222): for the last query row it stores ``logits * sm_scale``
    at ``b*H*S + h*S + t`` for ``t < kv_len``; the buffer is -inf filled
    (backend.py:384-389), so every other position reads -inf.  ``sm_scale`` is
    ``1/sqrt(head_dim)`` at the call site (backend.py:542).  The dot product is
    taken in ``compute_dtype`` (float64 by default) and rounded once to fp32.
    """
    B, Hq, d = q.shape
    Hkv = kv_cache.shape[3]
    G = Hq // Hkv
    out = torch.full((B, Hq, max_len), float("-inf"), dtype=torch.float32)
    for b in range(B):
        k, _ = gather_row_kv(kv_cache, kv_indptr, kv_indices, kv_last_page_len, b)
        n = k.shape[0]
        if n == 0:
            continue
        kk = k.to(compute_dtype).repeat_interleave(G, dim=1)          # [n, Hq, d]
        s = torch.einsum("hd,nhd->hn", q[b].to(compute_dtype), kk) * float(sm_scale)
        out[b, :, :n] = s.to(torch.float32)
    return out


def legacy_softmax_page_scores(logits: torch.Tensor, active_bsz: int, max_pages: int,
                               page_size: int = PAGE_SIZE,
                               compute_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``del3_legacy_softmax`` page scores, fp32 ``[active_bsz, max_pages]``.

    backend.py:898-904: take the dump view ``[:B, :, :, :max_pages*16]``,
    ``softmax`` over tokens, ``amax`` over *all* q heads, ``sum`` over the
    (size-1) query axis, then sum each run of 16 tokens into its page.
    ``compute_dtype`` float32 is the reference's own precision; float64 gives a
    tighter value for pinning.
    """
    x = logits[:active_bsz, :, : max_pages * page_size].to(compute_dtype)
    probs = torch.softmax(x, dim=-1)
    head_max = probs.amax(dim=1)                                    # [B, T]
    return head_max.reshape(active_bsz, max_pages, page_size).sum(dim=-1).to(torch.float32)


# ---------------------------------------------------------------------------
# PageSelectorV2
# ---------------------------------------------------------------------------

def position_bias(n: int, scale: float) -> np.ndarray:
    """fp32 ``-arange(n) * scale`` as built at page_selector_v2.py:52-55.

    torch multiplies an fp32 tensor by a Python scalar in fp32, so both factors
    are fp32 and the product is rounded once to fp32.
    """
    return (-np.arange(n, dtype=np.float32)) * np.float32(scale)


def prepare_scores(page_scores: torch.Tensor, page_counts: torch.Tensor, L: int,
                   pos_bias_scale: float = 1e-7) -> torch.Tensor:
    """Selection keys exactly as ``PageSelectorV2._prepare_scores``.

    page_selector_v2.py:113-130, all in fp32:
      1. ``nan_to_num(nan=-inf, neginf=-inf)``: NaN -> -inf, +inf -> FLT_MAX;
      2. add the position bias ``-j * scale`` (skipped when scale == 0);
      3. pages ``j`` in ``[max(tp - L, 0), tp)`` -> +inf (always kept);
      4. pages ``j >= tp`` -> -inf.
    """
    s = page_scores.detach().to(torch.float32).cpu().numpy().copy()
    B, n = s.shape
    with np.errstate(invalid="ignore", over="ignore"):
        s = np.nan_to_num(s, nan=-np.inf, neginf=-np.inf, posinf=np.finfo(np.float32).max)
        s = s.astype(np.float32)
        if pos_bias_scale != 0.0:
            s = (s + position_bias(n, pos_bias_scale)[None, :]).astype(np.float32)
    tp = page_counts.to(torch.int64).cpu().numpy()
    j = np.arange(n)[None, :]
    last_start = np.maximum(tp - L, 0)[:, None]
    s[(j >= last_start) & (j < tp[:, None])] = np.inf
    s[j >= tp[:, None]] = -np.inf
    return torch.from_numpy(s)


def topk_positions(keys: torch.Tensor, k: int) -> torch.Tensor:
    """Top-k columns of each row ordered by (key desc, column asc), then sorted asc.

    ``torch.topk`` (page_selector_v2.py:144, 171-178) leaves the order of equal
    keys unspecified; this restatement fixes it to the smaller page index first
    (the deterministic tie-break the GPU selector implements).  ``-0.0`` and
    ``+0.0`` compare equal, as in ``torch.topk``.  Positions are then sorted
    ascending (page_selector_v2.py:132-134).
    """
    B, n = keys.shape
    if k > n:
        raise RuntimeError("selected index k out of range")
    out = np.empty((B, k), dtype=np.int64)
    kn = keys.numpy()
    cols = np.arange(n)
    for b in range(B):
        # lexsort: last key is primary -> (-value, column)
        vals = kn[b].astype(np.float64) + 0.0    # -0.0 + 0.0 == +0.0
        order = np.lexsort((cols, -vals))
        out[b] = np.sort(order[:k])
    return torch.from_numpy(out)


def select_pages(page_scores: torch.Tensor, page_counts: torch.Tensor,
                 block_table: torch.Tensor, k: int, L: int,
                 pos_bias_scale: float = 1e-7,
                 fixed_count: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """``PageSelectorV2.select`` -> (int32 physical indices, int32 indptr).

    General path (page_selector_v2.py:136-164): top-k, sort ascending, gather
    physical ids from the row-major block table, keep the first ``min(tp, k)``
    per row, ``indptr = cumsum``.  Fixed path (166-188): every row contributes
    ``k`` pages and ``indptr = arange(B+1) * k``.  ``k <= 0`` returns an empty
    selection (139-141, 168-169).
    """
    B, n = page_scores.shape
    if k <= 0:
        return torch.zeros(0, dtype=torch.int32), torch.zeros(B + 1, dtype=torch.int32)
    keys = prepare_scores(page_scores, page_counts, L, pos_bias_scale)
    pos = topk_positions(keys, k)
    bt = block_table[:B, :n].to(torch.int64)
    selected = torch.gather(bt, 1, pos).to(torch.int32)
    if fixed_count:
        return selected.reshape(-1), torch.arange(B + 1, dtype=torch.int32) * k
    valid = torch.clamp(page_counts.to(torch.int64), max=k)
    indptr = torch.zeros(B + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(valid, 0).to(torch.int32)
    keep = torch.arange(k)[None, :] < valid[:, None]
    return selected[keep].to(torch.int32), indptr


def block_table_from_csr(kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
                         pages_per_slot: int) -> torch.Tensor:
    """Row-major block table from CSR, zero padded (page_selector_v2.py:102-111)."""
    B = kv_indptr.numel() - 1
    bt = torch.zeros((B, pages_per_slot), dtype=torch.int32)
    for b in range(B):
        s, e = int(kv_indptr[b]), int(kv_indptr[b + 1])
        bt[b, : e - s] = kv_indices[s:e]
    return bt


# ---------------------------------------------------------------------------
# Paged decode attention
# ---------------------------------------------------------------------------

def paged_decode_attention(q: torch.Tensor, kv_cache: torch.Tensor,
                           kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
                           kv_last_page_len: torch.Tensor, sm_scale: float,
                           compute_dtype: torch.dtype = torch.float64
                           ) -> Tuple[torch.Tensor, torch.Tensor]:
    """One-token decode attention over a paged CSR; returns (o fp32, lse fp32).

    The FlashInfer paged prefill the reference plans with ``causal=True`` and
    one query per row (backend.py:1091-1105) reduces to
    ``o[b,h] = softmax(q[b,h] . K[b,:,h//G] * sm_scale) @ V[b,:,h//G]`` over the
    row's ``kv_len`` tokens.  ``target_subset_decode`` (backend.py:487-512) is
    the same over the subset CSR with the shared ``last_page_len``.  ``lse`` is
    the natural-log log-sum-exp of the scaled logits (-inf, o = 0 for an empty
    row).
    """
    B, Hq, d = q.shape
    Hkv = kv_cache.shape[3]
    G = Hq // Hkv
    o = torch.zeros((B, Hq, d), dtype=torch.float32)
    lse = torch.full((B, Hq), float("-inf"), dtype=torch.float32)
    for b in range(B):
        k, v = gather_row_kv(kv_cache, kv_indptr, kv_indices, kv_last_page_len, b)
        if k.shape[0] == 0:
            continue
        kk = k.to(compute_dtype).repeat_interleave(G, dim=1)       # [n, Hq, d]
        vv = v.to(compute_dtype).repeat_interleave(G, dim=1)
        s = torch.einsum("hd,nhd->hn", q[b].to(compute_dtype), kk) * float(sm_scale)
        m = s.amax(dim=-1, keepdim=True)
        e = torch.exp(s - m)
        den = e.sum(dim=-1, keepdim=True)
        o[b] = (torch.einsum("hn,nhd->hd", e, vv) / den).to(torch.float32)
        lse[b] = (m + torch.log(den)).squeeze(-1).to(torch.float32)
    return o, lse


def paged_prefill_attention(q: torch.Tensor, qo_indptr: torch.Tensor, kv_cache: torch.Tensor,
                            kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
                            kv_last_page_len: torch.Tensor, sm_scale: float,
                            compute_dtype: torch.dtype = torch.float64
                            ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Causal attention of several query tokens per row over a paged CSR; (o, lse) fp32.

    The FlashInfer paged prefill the reference plans with ``causal=True``
    (backend.py:1091-1105) for rows with ``qo_len_b = qo_indptr[b+1] - qo_indptr[b]``
    query tokens: the KV cache already holds the row's new tokens (update_kv runs
    before attention, model.py:413-418), so query i of row b sits at position
    ``kv_len_b - qo_len_b + i`` and attends the tokens ``0 .. position``.
    ``q`` is ``[nnz, Hq, d]`` with rows ``qo_indptr[b] ..``.
    """
    nnz, Hq, d = q.shape
    Hkv = kv_cache.shape[3]
    G = Hq // Hkv
    o = torch.zeros((nnz, Hq, d), dtype=torch.float32)
    lse = torch.full((nnz, Hq), float("-inf"), dtype=torch.float32)
    for b in range(len(qo_indptr) - 1):
        q0, q1 = int(qo_indptr[b]), int(qo_indptr[b + 1])
        if q1 <= q0:
            continue
        k, v = gather_row_kv(kv_cache, kv_indptr, kv_indices, kv_last_page_len, b)
        n = k.shape[0]
        kk = k.to(compute_dtype).repeat_interleave(G, dim=1)
        vv = v.to(compute_dtype).repeat_interleave(G, dim=1)
        s = torch.einsum("ihd,nhd->ihn", q[q0:q1].to(compute_dtype), kk) * float(sm_scale)  # [qo, Hq, n]
        pos = n - (q1 - q0) + torch.arange(q1 - q0)
        mask = torch.arange(n)[None, :] > pos[:, None]                                   # [qo, n]
        s = s.masked_fill(mask[:, None, :], float("-inf"))
        m = s.amax(dim=-1, keepdim=True)
        ok = torch.isfinite(m)
        e = torch.where(ok, torch.exp(s - torch.where(ok, m, 0.0)), 0.0)
        den = e.sum(dim=-1, keepdim=True)
        o[q0:q1] = torch.where(den > 0, torch.einsum("ihn,nhd->ihd", e, vv) / den.clamp_min(1e-300), 0.0).to(torch.float32)
        lse[q0:q1] = torch.where(den > 0, m + torch.log(den.clamp_min(1e-300)), float("-inf")).squeeze(-1).to(torch.float32)
    return o, lse


# ---------------------------------------------------------------------------
# Host/device metadata helpers
# ---------------------------------------------------------------------------

def pack_page_indices(slot_block_table: torch.Tensor, active_slots: torch.Tensor,
                      start_cols: torch.Tensor, counts: torch.Tensor,
                      indptr: torch.Tensor, out_indices: torch.Tensor,
                      row_block_table: Optional[torch.Tensor], n_rows: int,
                      write_row_block: bool) -> None:
    """In-place restatement of ``_pack_page_indices_kernel`` (page_metadata.py:6-35).

    Row ``r`` copies ``slot_block_table[active_slots[r], start_cols[r]:+counts[r]]``
    to ``out_indices[indptr[r]:]`` and, when ``write_row_block``, to
    ``row_block_table[r, :counts[r]]``.  ``n_rows <= 0`` is a no-op (55-56).
    """
    for r in range(max(n_rows, 0)):
        slot = int(active_slots[r])
        start = int(start_cols[r])
        c = int(counts[r])
        if c <= 0:
            continue
        vals = slot_block_table[slot, start:start + c]
        dst = int(indptr[r])
        out_indices[dst:dst + c] = vals
        if write_row_block:
            row_block_table[r, :c] = vals


def decode_page_info(cachelens: torch.Tensor, pages_per_row_alloc: int, k,
                     page_size: int = PAGE_SIZE):
    """Per-row page counts for one decode step, as ``_collect_decode_page_info_fast``.

    backend.py:2047-2067 with scheduler.py:60-66: before the step each row
    holds ``cachelens[b]`` tokens; ``plan(1, 16)`` adds the decode token, so
    ``kv_len = cachelens + 1``, ``page_count = kv_len // 16 + 1`` and
    ``last_page_len = kv_len % 16`` (a full page leaves a fresh empty page).
    ``subset_count = min(page_count, k)``, ``subset_start = page_count - subset_count``.
    ``k`` is the global ``subset_cache_size`` or, for this build's per-row budgets (an
    extension), one budget per row (negative budgets count as 0).
    """
    kv_len = cachelens.to(torch.int64) + 1
    page_count = kv_len // page_size + 1
    if int(page_count.max()) > pages_per_row_alloc:
        raise RuntimeError("row outgrew its page allocation")
    last = kv_len % page_size
    kk = torch.clamp(torch.as_tensor(k, dtype=torch.int64), min=0)
    subset_count = torch.minimum(page_count, kk)
    subset_start = page_count - subset_count
    return page_count, last, subset_count, subset_start


def budget_rule_pages(cachelens: torch.Tensor, min_tokens: int, divisor: int, k_cap: int,
                      page_size: int = PAGE_SIZE) -> torch.Tensor:
    """Per-row subset budgets in pages under a length rule (an extension, no reference code).

    Config 5's "per-sequence budget of max(512, len/8) tokens" read
    at each decode step: ``len`` is the row's length after the decode token, ``kv_len =
    cachelens + 1`` (backend.py:2047-2067's plan(1, 16)); the budget is ``max(min_tokens,
    kv_len // divisor)`` tokens in whole pages (``// page_size``), clamped to ``[1, k_cap]``.
    """
    kv_len = cachelens.to(torch.int64) + 1
    tokens = torch.clamp(kv_len // int(divisor), min=int(min_tokens))
    return torch.clamp(tokens // page_size, min=1, max=int(k_cap)).to(torch.int32)


def use_subset_decision(full_total: int, subset_total: int, compression_ratio: float,
                        enable_selective_cache: bool = True) -> bool:
    """``use_subset`` gate (backend.py:2104-2109): full/subset page ratio above threshold."""
    return bool(enable_selective_cache and subset_total > 0
                and (full_total / subset_total) > compression_ratio)


def decode_step_gate(cachelens, active, k, compression_ratio: float,
                     enable_selective_cache: bool = True, page_size: int = PAGE_SIZE) -> bool:
    """The decode step's ``use_subset`` decision over its active rows only.

    backend.py:2047-2067 loops over ``active_slots``: each row's ``page_count`` (after
    ``plan(1, 16)``) goes into ``full_total`` and ``min(page_count, subset_cache_size)``
    into ``subset_total``; backend.py:2104-2109 then compares their ratio.  Slots with
    ``active[b] == 0`` take no part.  ``k`` is the global budget or one budget per row (this
    build's per-row extension: row b then adds ``min(page_count, k[b])``).
    """
    per_row = not isinstance(k, (int, float))
    full_total = subset_total = 0
    for b in range(len(cachelens)):
        if int(active[b]) == 0:
            continue
        pc = (int(cachelens[b]) + 1) // page_size + 1
        kb = max(int(k[b]) if per_row else int(k), 0)
        full_total += pc
        subset_total += min(pc, kb)
    return use_subset_decision(full_total, subset_total, compression_ratio, enable_selective_cache)


def append_kv(k: torch.Tensor, v: torch.Tensor, kv_append_indptr: torch.Tensor,
              kv_cache: torch.Tensor, kv_indices: torch.Tensor, kv_indptr: torch.Tensor,
              kv_last_page_len: torch.Tensor) -> None:
    """In-place ``mylib::update_kv`` (utils.py:31-66, FlashInfer semantics).

    ``seq_len`` comes from the page table *after* the new tokens were planned
    (``get_seq_lens``); appended token ``i`` of row ``b`` lands at position
    ``seq_len - append_len + i``: page ``kv_indices[kv_indptr[b] + pos // 16]``,
    slot ``pos % 16``.
    """
    page_size = kv_cache.shape[2]
    seq = kv_lengths(kv_indptr, kv_last_page_len, page_size)
    B = kv_append_indptr.numel() - 1
    for b in range(B):
        a0, a1 = int(kv_append_indptr[b]), int(kv_append_indptr[b + 1])
        n = a1 - a0
        for i in range(n):
            pos = int(seq[b]) - n + i
            page = int(kv_indices[int(kv_indptr[b]) + pos // page_size])
            kv_cache[page, 0, pos % page_size] = k[a0 + i]
            kv_cache[page, 1, pos % page_size] = v[a0 + i]


def rope_frequencies(head_dim: int, rope_scale: float, rope_theta: float,
                     low_freq_factor: Optional[float] = None,
                     high_freq_factor: Optional[float] = None,
                     old_context_len: Optional[int] = None) -> torch.Tensor:
    """Per-pair angular frequency of FlashInfer's interleaved RoPE (fp64).

    model.py:152-175 calls ``apply_rope`` / ``apply_llama31_rope`` with
    ``interleave=True``.  Published formula: pair ``j`` (elements 2j, 2j+1)
    rotates at ``theta**(-2j/d)``; plain RoPE divides by ``rope_scale``;
    Llama-3.1 blends ``f/rope_scale`` and ``f`` with
    ``smooth = clamp(f * old_ctx / (2*pi*(hi - lo)) - 1/(hi/lo - 1), 0, 1)``,
    which is Meta's wavelength rule ``(old_ctx / wavelen - lo) / (hi - lo)`` with
    ``wavelen = 2*pi / f`` (pinned against that form in the tests).
    """
    j = torch.arange(head_dim // 2, dtype=torch.float64)
    f = rope_theta ** (-(2.0 * j) / head_dim)
    if low_freq_factor is None or high_freq_factor is None:
        return f / rope_scale
    a = old_context_len / (2.0 * math.pi * high_freq_factor - 2.0 * math.pi * low_freq_factor)
    c = -1.0 / (high_freq_factor / low_freq_factor - 1.0)
    smooth = torch.clamp(f * a + c, 0.0, 1.0)
    return (1.0 - smooth) * (f / rope_scale) + smooth * f


def apply_rope(x: torch.Tensor, indptr: torch.Tensor, offsets: torch.Tensor,
               freqs: torch.Tensor) -> torch.Tensor:
    """Interleaved RoPE of ``x`` [nnz, H, d] (fp64 math, returned as fp32).

    Token ``i`` of row ``b`` sits at ``offsets[b] + i - indptr[b]``;
    ``out[2j] = x[2j] cos - x[2j+1] sin``, ``out[2j+1] = x[2j+1] cos + x[2j] sin``.
    """
    nnz = x.shape[0]
    pos = torch.empty(nnz, dtype=torch.float64)
    for b in range(indptr.numel() - 1):
        s, e = int(indptr[b]), int(indptr[b + 1])
        pos[s:e] = float(offsets[b]) + torch.arange(e - s, dtype=torch.float64)
    ang = pos[:, None] * freqs[None, :]                      # [nnz, d/2]
    c, s = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
    xf = x.to(torch.float64)
    x0, x1 = xf[..., 0::2], xf[..., 1::2]
    out = torch.empty_like(xf)
    out[..., 0::2] = x0 * c - x1 * s
    out[..., 1::2] = x1 * c + x0 * s
    return out.to(torch.float32)


# ---------------------------------------------------------------------------
# One selective planner step (scores -> selection -> sparse attention)
# ---------------------------------------------------------------------------

def selective_step(q: torch.Tensor, kv_cache: torch.Tensor, kv_indptr: torch.Tensor,
                   kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor,
                   k: int, L: int, sm_scale: Optional[float] = None,
                   pos_bias_scale: float = 1e-7, pages_per_slot: Optional[int] = None,
                   score_dtype: torch.dtype = torch.float32):
    """Planner score -> v2 selection -> sparse attention of the same layer's q/KV.

    Chains backend.py:787-853 (``_replan``) with the subset decode of
    backend.py:487-512.  Returns a dict with ``scores``, ``indices``,
    ``indptr``, ``o_full``, ``o_sparse``.
    """
    B, Hq, d = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    counts = (kv_indptr[1:] - kv_indptr[:-1]).to(torch.int64)
    max_pages = int(counts.max())
    page_size = kv_cache.shape[2]
    x = dump_logits(q, kv_cache, kv_indptr, kv_indices, kv_last_page_len, sm_scale,
                    max_pages * page_size)
    scores = legacy_softmax_page_scores(x, B, max_pages, page_size, score_dtype)
    bt = block_table_from_csr(kv_indptr, kv_indices, pages_per_slot or max_pages)
    indices, indptr = select_pages(scores, counts, bt, k, L, pos_bias_scale)
    o_full, _ = paged_decode_attention(q, kv_cache, kv_indptr, kv_indices, kv_last_page_len, sm_scale)
    o_sparse, _ = paged_decode_attention(q, kv_cache, indptr, indices, kv_last_page_len, sm_scale)
    return {"scores": scores, "indices": indices, "indptr": indptr,
            "o_full": o_full, "o_sparse": o_sparse, "logits": x}
