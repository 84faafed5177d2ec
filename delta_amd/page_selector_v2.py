"""PageSelectorV2 with the reference's constructor, buffers and methods, selecting on gfx950.

Mirrors DELTA/Engine/DELTA/page_selector_v2.py:4-212.  ``select`` runs the
radix-select kernel (``delta_select_pages``): same keys (nan_to_num, fp32
position bias, forced last-L, invalid tail), top-k with ties broken by the
smaller page index, ascending logical order, physical ids from the row-major
block table.  The fixed-count path returns the static CSR without a host
sync; the general path, like the reference's boolean-mask compaction, syncs
once to size its result.
"""
from __future__ import annotations

import torch

from . import kernels as K


class PageSelectorV2:
    def __init__(self, max_batch_size, pages_per_slot, enable_selective_cache, subset_cache_size,
                 compression_ratio, L, device, position_bias_scale: float = 1e-7):
        self.max_batch_size = max_batch_size
        self.pages_per_slot = pages_per_slot
        self.enable_selective_cache = enable_selective_cache
        self.subset_cache_size = subset_cache_size
        self.compression_ratio = compression_ratio
        self.max_num_pages = pages_per_slot * max_batch_size
        self.max_num_subset_pages = subset_cache_size * max_batch_size
        self.L = L
        self.device = device
        self.position_bias_scale = float(position_bias_scale)

        i32 = dict(dtype=torch.int32, device=device)
        self.qo_indptr = torch.arange(max_batch_size + 1, **i32)
        self.paged_kv_indices = torch.zeros(self.max_num_pages, **i32)
        self.paged_kv_indptr = torch.arange(max_batch_size + 1, **i32)
        self.paged_kv_last_page_len = torch.zeros(max_batch_size, **i32)
        self.paged_subset_kv_indices = torch.zeros(self.max_num_pages, **i32)
        self.paged_subset_kv_indptr = torch.arange(max_batch_size + 1, **i32)
        self._active_B = max_batch_size
        if self.enable_selective_cache:
            self._block_table = torch.zeros((max_batch_size, pages_per_slot), **i32)
            self._selected_pages_flat = torch.zeros(max(self.max_num_pages, 1), **i32)
            self._selected_indptr = torch.zeros(max_batch_size + 1, **i32)
            self._fixed_selected_indptr = torch.arange(max_batch_size + 1, **i32) * subset_cache_size
            self.tp = self.paged_kv_indptr[1:] - self.paged_kv_indptr[:-1]
            self.base_offsets = self.paged_kv_indptr[:-1]

    def plan(self, qo_indptr, paged_kv_indices, paged_kv_indptr, paged_kv_last_page_len,
             paged_subset_kv_indices, paged_subset_kv_indptr, L=None, block_table_prebuilt=False):
        """Bind this step's CSR tensors (page_selector_v2.py:74-111)."""
        self.qo_indptr = qo_indptr
        self.paged_kv_indices = paged_kv_indices
        self.paged_kv_indptr = paged_kv_indptr
        self.paged_kv_last_page_len = paged_kv_last_page_len
        self.paged_subset_kv_indices = paged_subset_kv_indices
        self.paged_subset_kv_indptr = paged_subset_kv_indptr
        if not self.enable_selective_cache or paged_kv_indices is paged_subset_kv_indices:
            return
        if L is not None:
            self.L = int(L)
        B = paged_kv_indptr.numel() - 1
        self._active_B = B
        self.tp = paged_kv_indptr[1:] - paged_kv_indptr[:-1]
        self.base_offsets = paged_kv_indptr[:-1]
        if block_table_prebuilt:
            return
        # Row-major block table from the CSR (zero padded).
        n_total = paged_kv_indices.numel()
        bt = self._block_table[:B]
        bt.zero_()
        if n_total > 0:
            rows = torch.repeat_interleave(torch.arange(B, device=paged_kv_indptr.device),
                                           self.tp.long(), output_size=n_total)
            cols = torch.arange(n_total, device=paged_kv_indptr.device) - self.base_offsets[rows].long()
            bt[rows, cols] = paged_kv_indices.to(torch.int32)

    def select(self, page_scores: torch.Tensor, *, fixed_count: bool = False, debug_compare: bool = False):
        """Top-k pages per row -> (int32 physical indices, int32 indptr) (page_selector_v2.py:190-212)."""
        B, nmax = page_scores.shape
        k = self.subset_cache_size
        if k <= 0:
            return (self.paged_subset_kv_indices[:0],
                    self._fixed_selected_indptr[:B + 1] if fixed_count
                    else torch.zeros(B + 1, dtype=torch.int32, device=page_scores.device))
        idx, ip = K.select_pages(page_scores, self.paged_kv_indptr, self._block_table, k, self.L,
                                 pos_bias_scale=self.position_bias_scale, fixed_count=fixed_count,
                                 batch=B, max_pages=nmax, out_indices=self._selected_pages_flat,
                                 out_indptr=self._selected_indptr)
        if fixed_count:
            sel = idx[:B * k]
            if debug_compare:
                gi, gp = self._select_general(page_scores, B, nmax)
                if not torch.equal(ip[:B + 1], gp) or not torch.equal(sel, gi):
                    raise RuntimeError("PageSelectorV2 fixed-count fast path mismatch against general selector")
            return sel, ip[:B + 1]
        return idx[:int(ip[B])], ip[:B + 1]

    def _select_general(self, page_scores, B, nmax):
        out = torch.empty(max(B * nmax, 1), dtype=torch.int32, device=page_scores.device)
        ip = torch.empty(B + 1, dtype=torch.int32, device=page_scores.device)
        K.select_pages(page_scores, self.paged_kv_indptr, self._block_table, self.subset_cache_size,
                       self.L, pos_bias_scale=self.position_bias_scale, batch=B, max_pages=nmax,
                       out_indices=out, out_indptr=ip)
        return out[:int(ip[B])], ip
