"""LMBackend: DELTA's engine surface, with the selective decode step on gfx950.

Public surface mirrors DELTA/Engine/DELTA/backend.py: the constructor and its
validation (29-168), ``load_model`` (227), ``setup_caches`` (247-593),
``add_requests`` (1480), ``run_scheduler_loop`` (1486-1553) and the
``mylib::target_*`` attention ops bound per layer.  What differs is where the
work runs:

* Decode metadata is derived on the device (``delta_decode_page_info``) from
  ``cachelens`` and a slot block table that holds every page a slot owns, so
  a decode step needs no host planning (the reference rebuilds it on the host
  each step, backend.py:2040-2172).
* The planner layer's attention writes the logits dump and lse, then page
  scores and the v2 selection run on the device straight into the subset CSR
  (the reference runs them eagerly between graph segments, 1432-1447), so the
  *whole* decode step -- metadata, every layer, argmax, the token feedback and
  the ``cachelens`` advance -- is one hipGraph.
* Idle slots point at a private scratch page with ``cachelens = 0`` so the
  graph also covers partial batches.
* Prefill / mixed steps run eagerly: all new tokens are appended, then the
  causal paged prefill kernel attends each row's pages.

Out of scope on this build (raise): tensor parallelism, ``torch.compile``
(no Triton), the v1 selector, the ``delta_lse`` scorer and an fp16 dump.
"""
from __future__ import annotations

import json
import os
import time
from collections import defaultdict
from pathlib import Path
from typing import List, Optional

import torch

from . import kernels as K
from . import ops
from . import model as model_mod
from .model import Transformer, build_random_model
from .page_selector_v2 import PageSelectorV2
from .public_config import FINAL_PUBLIC_DELTA_BACKEND_CONFIG as _CFG
from .scheduler import BatchSlots, PagePool, ServingRequest

PAGE_SIZE = 16


class _StepCSR:
    """Page tables the attention ops read during one forward (prefill steps also carry the
    query-token CSR of the rows)."""

    __slots__ = ("mode", "kv_indptr", "kv_indices", "kv_last", "max_pages", "qo_indptr", "max_qo")

    def __init__(self, mode, kv_indptr, kv_indices, kv_last, max_pages, qo_indptr=None, max_qo=1):
        self.mode = mode
        self.kv_indptr = kv_indptr
        self.kv_indices = kv_indices
        self.kv_last = kv_last
        self.max_pages = max_pages
        self.qo_indptr = qo_indptr
        self.max_qo = max_qo


class LMBackend:
    def __init__(
        self,
        dtype=torch.bfloat16,
        device: str = "cuda:0",
        dec_len: int = 1,
        draft_dec_len: int = None,
        cuda_graph_decode: bool = False,
        cuda_graph_delta_subset_segments: bool = _CFG["cuda_graph_delta_subset_segments"],
        delta_impl_profile: bool = _CFG["delta_impl_profile"],
        delta_fused_page_scores: bool = _CFG["delta_fused_page_scores"],
        delta_fixed_selector: bool = _CFG["delta_fixed_selector"],
        delta_fast_decode_page_info: bool = _CFG["delta_fast_decode_page_info"],
        delta_v2_position_bias: bool = _CFG["delta_v2_position_bias"],
        delta_debug_page_selection_parity: bool = False,
        delta_debug_fast_decode_page_info_parity: bool = False,
        delta_subset_plan_reuse: bool = _CFG["delta_subset_plan_reuse"],
        delta_dump_buffer_dtype: str = _CFG["delta_dump_buffer_dtype"],
        delta_page_score_impl: str = _CFG["delta_page_score_impl"],
        page_selector_version: str = _CFG["page_selector_version"],
    ) -> None:
        # Same validation and messages as backend.py:49-64.
        page_selector_version = str(page_selector_version).lower()
        if page_selector_version not in {"v1", "v2"}:
            raise ValueError(f"Unsupported page_selector_version={page_selector_version!r}; expected 'v1' or 'v2'")
        delta_dump_buffer_dtype = str(delta_dump_buffer_dtype).lower()
        if delta_dump_buffer_dtype not in {"fp16", "fp32"}:
            raise ValueError(
                f"Unsupported delta_dump_buffer_dtype={delta_dump_buffer_dtype!r}; expected 'fp16' or 'fp32'")
        delta_page_score_impl = str(delta_page_score_impl).lower()
        if delta_page_score_impl not in {"delta_lse", "del3_legacy_softmax"}:
            raise ValueError("Unsupported delta_page_score_impl="
                             f"{delta_page_score_impl!r}; expected 'delta_lse' or 'del3_legacy_softmax'")
        # The public release path is the only one built for gfx950.
        if page_selector_version != "v2":
            raise NotImplementedError("page_selector_version='v1' is not built on this path (v2 only)")
        if delta_dump_buffer_dtype != "fp32":
            raise NotImplementedError("delta_dump_buffer_dtype='fp16' is not built on this path (fp32 only)")
        if delta_page_score_impl != "del3_legacy_softmax":
            raise NotImplementedError("delta_page_score_impl='delta_lse' is not built on this path")
        if dec_len != 1 or draft_dec_len is not None:
            raise NotImplementedError("speculative decoding (dec_len != 1) is not part of this path")

        self.dtype = dtype
        self.device = torch.device(device)
        self.dec_len = dec_len
        self.enable_cuda_graph_decode = bool(cuda_graph_decode)
        self.enable_cuda_graph_delta_subset_segments = cuda_graph_delta_subset_segments
        self.enable_delta_impl_profile = delta_impl_profile
        self.enable_delta_fused_page_scores = delta_fused_page_scores
        self.enable_delta_fixed_selector = delta_fixed_selector
        self.enable_delta_fast_decode_page_info = delta_fast_decode_page_info
        self.enable_delta_v2_position_bias = delta_v2_position_bias
        self.enable_delta_debug_page_selection_parity = delta_debug_page_selection_parity
        self.enable_delta_debug_fast_decode_page_info_parity = delta_debug_fast_decode_page_info_parity
        self.enable_delta_subset_plan_reuse = delta_subset_plan_reuse
        self.delta_dump_buffer_dtype = delta_dump_buffer_dtype
        self.delta_page_score_impl = delta_page_score_impl
        self.page_selector_version = page_selector_version

        self.model: Optional[Transformer] = None
        self.cachelens = None
        self.is_main_process = True
        self.tokenizer = None
        self.scheduler = None
        self.throughput_mode = False
        self.timer = None
        self._compiled = False
        self._step: Optional[_StepCSR] = None
        self._decode_graph: Optional[torch.cuda.CUDAGraph] = None
        self._decode_graph_on_chip = False  # the planner path the captured step runs
        self._decode_graph_failed: Optional[str] = None
        self._decode_graph_stats = defaultdict(int)
        self._decode_graph_fallback_reasons = defaultdict(int)
        self._decode_graph_capture_errors = {}
        self._decode_graph_capture_time_s = defaultdict(float)
        # delta_impl_profile: named device sections timed with HIP events (backend.py:105-107)
        self._delta_impl_profile_ms = defaultdict(float)
        self._delta_impl_profile_counts = defaultdict(int)
        self._delta_impl_profile_pending = []
        self._profile_paused = False  # the capture's warm-up bodies are not steps
        self._pending_events = []
        self._step_records = []
        self._using_subset_cache_this_step = False

    # ------------------------------------------------------------------ setup
    def set_tokenizer(self, tokenizer):
        self.tokenizer = tokenizer

    def load_model(self, checkpoints, use_tp: bool = False, rank_group=None, group=None, seed: int = 0,
                   **shape_overrides):
        """Load a model (backend.py:227-228 -> utils.py:209-231).

        ``checkpoints`` is either a ``model.pth`` state dict (loaded with
        ``weights_only=True``; its parent directory names the shape, as in the
        reference) or ``"random:<shape>"`` for a seeded random-init model, whose
        ``ModelArgs`` fields ``shape_overrides`` may change (e.g. ``n_layer``).  A state dict
        loads strictly, as the reference's does (utils.py:217-221): separate wq/wk/wv and
        w1/w3 tensors are merged by the modules' load hooks, and a missing or unknown key
        raises instead of leaving a parameter at its random init.
        """
        if use_tp:
            raise NotImplementedError("tensor parallelism is out of scope for this one-GPU path")
        ck = str(checkpoints)
        if ck.startswith("random:"):
            self.model = build_random_model(ck[len("random:"):], self.device, self.dtype, seed=seed,
                                            **shape_overrides)
            return
        if shape_overrides:
            raise ValueError("shape overrides apply to random-init models only; a checkpoint names its shape")
        path = Path(ck)
        model = build_random_model(path.parent.name, self.device, self.dtype, seed=seed)
        state = torch.load(str(path), mmap=True, weights_only=True)
        if "model" in state and "stories" in ck:  # nested checkpoints (utils.py:218-219)
            state = state["model"]
        model.load_state_dict(state, strict=True)
        self.model = model.to(self.dtype)

    def compile(self):
        """torch.compile is not used on this path (it would need Triton); graphs replace it."""
        self.enable_cuda_graph_decode = True

    @torch.inference_mode()
    def setup_caches(self, max_batch_size: int = 1, max_seq_length: int = 2048,
                     kv_cache_pool: Optional[int] = None):
        """Allocate the paged caches, page tables, planner buffers and workspaces (backend.py:247-593).
        ``kv_cache_pool`` = n shares n physical KV caches among the layers round robin (layer i
        uses cache i % n): a benchmark aid for shapes whose KV exceeds HBM (
        ~425 GB), where every layer still reads and appends its own pages at the real shape but
        the layers of one cache share its values, so the outputs are not a model's."""
        if self.model is None:
            raise RuntimeError("load_model() first")
        cfg = self.model.config
        dev = self.device
        self.max_length = max_seq_length
        self.batch_size = max_batch_size
        if max_batch_size <= model_mod._ROWS32_MAX:
            # the gate|up GEMM of this engine's decode steps runs on delta_gemm_skinny (<= 8
            # rows) or delta_gemm_rows32_silu, both on the row-major merged weight
            for layer in self.model.layers:
                layer.feed_forward.use_row_major_w13()
        self.page_size = PAGE_SIZE
        self.pages_per_slot = (max_seq_length + PAGE_SIZE - 1) // PAGE_SIZE + 1  # +1: trailing empty page
        self.max_num_pages = self.pages_per_slot * max_batch_size
        # one private scratch page per slot: idle slots append/read only there
        self.num_pages = self.max_num_pages + max_batch_size
        self.scratch_pages = torch.arange(self.max_num_pages, self.num_pages, dtype=torch.int32)
        self.page_pool = PagePool(self.max_num_pages, seed=0)
        self._synthetic_pages: List[int] = []  # held by prepare_synthetic_decode
        self.scheduler = BatchSlots(max_batch_size, self.page_pool, verbose=self.is_main_process)

        self.enable_selective_cache = bool(getattr(cfg, "enable_selective_cache", False))
        self.subset_cache_size = int(getattr(cfg, "subset_cache_size", 64))
        self.compression_ratio = float(getattr(cfg, "compression_ratio", 1.0))
        self.L = int(getattr(cfg, "L", 8))
        self.k_eff = max(1, min(self.subset_cache_size, self.pages_per_slot))

        i32 = dict(dtype=torch.int32, device=dev)
        B = max_batch_size
        self.cachelens = torch.zeros(B, **i32)
        self.active = torch.zeros(B, **i32)
        # Host mirror of cachelens / active and the pages each slot's table holds, so a decode
        # step that would take a row past its pages is refused before it runs (the device
        # metadata clamps such a row to a full table, which would overwrite its last slot).
        self._host_lens = [0] * B
        self._host_active = [0] * B
        self._slot_pages = [self.pages_per_slot] * B
        self.slot_block_table = self.scratch_pages.to(dev)[:, None].repeat(1, self.pages_per_slot).contiguous()
        self.page_selector = PageSelectorV2(B, self.pages_per_slot, True, self.k_eff,
                                           self.compression_ratio, self.L, dev,
                                           position_bias_scale=1e-7 if self.enable_delta_v2_position_bias else 0.0)
        # Per-row subset budgets (``set_subset_budgets``): read by the metadata and selection
        # launches when switched on, so a captured step takes new values on every replay.
        self.k_per_row = torch.full((B,), self.k_eff, **i32)
        self._per_row_budgets = False
        # Or a length rule (``set_subset_budget_rule``): the metadata launch derives each row's
        # budget from its length at every step and writes it into k_per_row for the selection.
        self._budget_rule = None
        self.use_subset_flag = torch.zeros(1, **i32)
        self.qo_indptr = torch.arange(B + 1, **i32)
        self.static_tokens = torch.zeros((1, B), dtype=torch.long, device=dev)
        hq = cfg.n_head
        hkv = cfg.n_local_heads
        self.dump = torch.full((B, hq, self.pages_per_slot * PAGE_SIZE), float("-inf"), dtype=torch.float32,
                               device=dev)
        self.lse = torch.zeros((B, hq), dtype=torch.float32, device=dev)
        self.page_scores = torch.zeros((B, self.pages_per_slot), dtype=torch.float32, device=dev)
        # The planner keeps its logits on chip (attention and page scores in one pass, no dump)
        # where the shape allows it; the dump path stays for the selection parity check.
        self.plan_scores_on_chip = (K.paged_decode_scores_supported(B, hq, hkv, self.pages_per_slot, True)
                                    and K.paged_decode_scores_supported(B, hq, hkv, self.pages_per_slot, False))
        ws = max(K.decode_workspace_bytes(B, hq, hkv, self.pages_per_slot),
                 K.decode_workspace_bytes(B, hq, hkv, self.k_eff),
                 K.paged_decode_scores_workspace_bytes(B, hkv, self.pages_per_slot), 256)
        self.workspace = torch.empty(ws, dtype=torch.uint8, device=dev)
        self._pinned_tokens = torch.zeros(B, dtype=torch.long).pin_memory()
        with torch.device(dev):
            self.model.setup_caches(num_pages=self.num_pages, page_size=PAGE_SIZE, kv_cache_pool=kv_cache_pool)
        self.layer_roles = list(self.model.layer_roles)
        ops.set_active_backend(self)
        self._decode_graph = None

    def set_subset_budgets(self, pages=None) -> None:
        """Give each slot its own subset budget in pages, or go back to the global
        ``subset_cache_size`` with ``None``.  An extension: the reference selects one global k
        per step, ``min(pages, k)`` per row (page_selector_v2.py:136-164); a per-row budget is
        what BASELINE config 5's ``max(512, len/8)``-token rule needs.  Each budget lies in
        [1, subset_cache_size] (the cap the subset attention launch is planned for).  Row b's
        subset is then min(pages_b, budget_b) pages, in the ``use_subset`` gate's totals, the
        default subset CSR and the selection.  New values take effect on the next step, replayed
        or eager; switching the per-row budgets on or off captures the step again."""
        if self.cachelens is None:
            raise RuntimeError("setup_caches() first")
        if pages is None:  # also ends a budget rule
            if self._per_row_budgets:
                self._decode_graph = None
            self._per_row_budgets = False
            self._budget_rule = None
            return
        vals = [int(x) for x in (pages.tolist() if isinstance(pages, torch.Tensor) else pages)]
        if len(vals) != self.batch_size:
            raise ValueError(f"need {self.batch_size} per-row budgets, got {len(vals)}")
        bad = [v for v in vals if v < 1 or v > self.k_eff]
        if bad:
            raise ValueError(f"per-row budgets must lie in [1, {self.k_eff}] pages (the subset_cache_size cap); "
                             f"got {bad[0]}")
        with torch.inference_mode():
            self.k_per_row.copy_(torch.tensor(vals, dtype=torch.int32))
        if not self._per_row_budgets or self._budget_rule is not None:
            self._decode_graph = None
        self._budget_rule = None
        self._per_row_budgets = True

    def set_subset_budget_rule(self, min_tokens: Optional[int] = 512, divisor: int = 8) -> None:
        """Per-row budgets from each row's length, recomputed on the device at every decode step:
        row b selects ``max(min_tokens, kv_len_b // divisor)`` tokens in whole 16-token pages,
        clamped to [1, subset_cache_size], where ``kv_len_b`` is its length after the step's
        token.  The defaults are BASELINE config 5's ``max(512, len/8)``-token budget.  An
        extension like ``set_subset_budgets`` (the reference has one global k), but a captured
        step keeps applying the rule as the rows grow.  ``min_tokens=None`` goes back to the
        global ``subset_cache_size``; setting fixed budgets replaces the rule."""
        if self.cachelens is None:
            raise RuntimeError("setup_caches() first")
        if min_tokens is None:
            if self._budget_rule is not None:
                self._decode_graph = None
            self._budget_rule = None
            self._per_row_budgets = False
            return
        if int(divisor) < 1 or int(min_tokens) < 0:
            raise ValueError(f"budget rule needs divisor >= 1 and min_tokens >= 0, got {divisor}, {min_tokens}")
        rule = (int(min_tokens), int(divisor))
        if rule != self._budget_rule:  # the rule's constants are baked into the captured launch
            self._decode_graph = None
        self._budget_rule = rule
        self._per_row_budgets = True

    def _row_budgets(self):
        """The per-row budget tensor when per-row budgets (fixed or by rule) are on, else None
        (global k).  Under a rule the step's metadata launch has just written it."""
        return self.k_per_row if self._per_row_budgets else None

    def _page_info_budgets(self) -> dict:
        """Budget arguments of the step's metadata launch: the rule with k_per_row as its output,
        or the fixed per-row budgets, or neither."""
        if self._budget_rule is not None:
            return dict(budget_rule=(*self._budget_rule, self.k_per_row))
        return dict(k_per_row=self._row_budgets())

    # ----------------------------------------------------------- op bodies
    def rope_params(self) -> dict:
        c = self.model.config
        p = dict(rope_scale=float(c.scaling_factor), rope_theta=float(c.rope_base))
        if c.high_freq_factor is not None and c.low_freq_factor is not None:
            p.update(low_freq_factor=float(c.low_freq_factor), high_freq_factor=float(c.high_freq_factor),
                     old_context_len=float(c.original_max_position_embeddings))
        return p

    def _decode_mode(self) -> bool:
        return self._step is not None and self._step.mode == "decode"

    def decode_append_ok(self) -> bool:
        """Decode steps (one new token per row) fuse RoPE and the KV append into the attention."""
        return self._decode_mode()

    def attn_append(self, role, q, k, v, offsets, kv_cache, ap_indices, ap_indptr):
        """A decode layer's attention with the new token's RoPE and KV append in the same launch
        (model.py:413-418 rope -> update_kv -> attention op); q, k are un-rotated."""
        ap = K.DecodeAppend(k, v, offsets, ap_indptr, ap_indices, **self.rope_params())
        if role == "subset":
            return self.attn_subset(q, kv_cache, append=ap)
        if role == "plan":
            return self.attn_plan(q, kv_cache, append=ap)
        return self.attn_full(q, kv_cache, append=ap)

    def attn_full(self, q, kv_cache, append=None):
        st = self._step
        if st.mode == "prefill":  # several query tokens per row: causal prefill kernel
            return self._profile_cuda_section("delta_prefill_attention", lambda: K.paged_prefill(
                q, kv_cache, st.qo_indptr, st.kv_indptr, st.kv_indices, st.kv_last, max_qo_len=st.max_qo))
        return self._profile_cuda_section("delta_full_attention", lambda: K.paged_decode(
            q, kv_cache, st.kv_indptr, st.kv_indices, st.kv_last, max_pages_per_row=st.max_pages,
            workspace=self.workspace, append=append))

    def attn_subset(self, q, kv_cache, append=None):
        if not (self.enable_selective_cache and self._decode_mode()):
            return self.attn_full(q, kv_cache, append=append)
        sel = self.page_selector
        return self._profile_cuda_section("delta_subset_attention", lambda: K.paged_decode(
            q, kv_cache, sel.paged_subset_kv_indptr, sel.paged_subset_kv_indices, self._step.kv_last,
            max_pages_per_row=self.k_eff, workspace=self.workspace, subset=True, append=append))

    def _plan_on_chip(self) -> bool:
        return self.plan_scores_on_chip and not self.enable_delta_debug_page_selection_parity

    def attn_plan(self, q, kv_cache, append=None):
        """Planner layer: full attention, page scores (logits kept on chip, or through the
        logits dump), v2 selection into the subset CSR."""
        if not (self.enable_selective_cache and self._decode_mode()):
            return self.attn_full(q, kv_cache, append=append)
        st = self._step
        sel = self.page_selector
        B = q.shape[0]
        prof = self._profile_cuda_section
        if self._plan_on_chip():
            # attention and page scores in one pass: one section for both
            o, _ = prof("delta_planner_attention_scores", lambda: K.paged_decode_scores(
                q, kv_cache, st.kv_indptr, st.kv_indices, st.kv_last, max_pages_per_row=st.max_pages, lse=self.lse,
                scores=self.page_scores, workspace=self.workspace, append=append))
        else:
            o = prof("delta_planner_attention_dump", lambda: K.paged_decode(
                q, kv_cache, st.kv_indptr, st.kv_indices, st.kv_last, max_pages_per_row=st.max_pages, lse=self.lse,
                logits_dump=self.dump, workspace=self.workspace, append=append))

        def replan():  # backend.py:787-853: page scores (dump path), then the v2 selection
            if not self._plan_on_chip():
                prof("delta_page_score", lambda: K.page_scores_from_logits(
                    self.dump, st.kv_indptr, st.kv_last, self.pages_per_slot, lse=self.lse, scores=self.page_scores,
                    batch=B, workspace=self.workspace))
            prof("delta_page_select", lambda: K.select_pages(
                self.page_scores, st.kv_indptr, sel._block_table, self.k_eff, self.L,
                pos_bias_scale=sel.position_bias_scale, batch=B, max_pages=self.pages_per_slot,
                k_per_row=self._row_budgets(), use_subset=self.use_subset_flag,
                out_indices=sel.paged_subset_kv_indices, out_indptr=sel.paged_subset_kv_indptr))

        prof("delta_replan_total", replan)
        return o

    def _debug_check_selection(self, st, B):
        """Selection from the two-pass (dump-only) scores must equal the planner's (backend.py:812-819)."""
        ref_scores = K.page_scores_from_logits(self.dump, st.kv_indptr, st.kv_last, self.pages_per_slot,
                                               batch=B)
        sel = self.page_selector
        ri, rp = K.select_pages(ref_scores, st.kv_indptr, sel._block_table, self.k_eff, self.L,
                                pos_bias_scale=sel.position_bias_scale, batch=B, max_pages=self.pages_per_slot,
                                k_per_row=self._row_budgets(), use_subset=self.use_subset_flag,
                                out_indices=torch.empty_like(sel.paged_subset_kv_indices))
        n = int(rp[B])
        if not torch.equal(rp[:B + 1], sel.paged_subset_kv_indptr[:B + 1]) or \
                not torch.equal(ri[:n], sel.paged_subset_kv_indices[:n]):
            raise RuntimeError("DELTA page selection mismatch against torch-score reference path")

    def _debug_checks_after_step(self, cachelens_before: torch.Tensor):
        """The reference's debug parity checks, run after a decode step (eager or replayed) on
        the tables and buffers that step left: the fast page info against a host rebuild
        (backend.py:1966-2012) and the planner's selection against a selection from two-pass
        scores of the same dump (backend.py:812-819)."""
        B = self.batch_size
        if self.enable_delta_debug_fast_decode_page_info_parity:
            self._debug_check_decode_page_info(cachelens_before)
        if self.enable_delta_debug_page_selection_parity and self.enable_selective_cache and "plan" in self.layer_roles:
            self._debug_check_selection(self._decode_csr(), B)

    def _debug_check_decode_page_info(self, cachelens_before: torch.Tensor):
        """Device decode metadata vs the same tables rebuilt on the host from ``cachelens`` and
        the slot block table (what ``Request.plan(1, 16)`` and the generic snapshot give,
        scheduler.py:60-66, backend.py:1850-1936); raises on the first difference."""
        B, pps, k = self.batch_size, self.pages_per_slot, self.k_eff
        lens = [int(x) for x in cachelens_before.tolist()]
        act = [int(x) for x in self.active.tolist()]
        bt = self.slot_block_table.cpu()
        counts = [(n + 1) // PAGE_SIZE + 1 for n in lens]
        last = [(n + 1) % PAGE_SIZE for n in lens]
        ks = self.k_per_row.tolist() if self._per_row_budgets else [k] * B
        if self._budget_rule is not None:  # the rule's budgets for the step's lengths
            mt, dv = self._budget_rule
            want = [min(max(max(mt, (n + 1) // dv) // PAGE_SIZE, 1), k) for n in lens]
            if ks != want:
                raise RuntimeError("DELTA fast decode page-info mismatch in k_per_row (budget rule)")
        full_tot = sum(c for c, a in zip(counts, act) if a)
        sub_tot = sum(min(c, kb) for c, kb, a in zip(counts, ks, act) if a)
        use = bool(self.enable_selective_cache and sub_tot > 0 and full_tot / sub_tot > self.compression_ratio)
        sub_counts = [min(c, kb) if use else c for c, kb in zip(counts, ks)]
        ip, sub_ip = [0], [0]
        ind, sub_ind = [], []
        for b in range(B):
            row = bt[b, :counts[b]].tolist()
            ind += row
            sub_ind += row[counts[b] - sub_counts[b]:]
            ip.append(len(ind))
            sub_ip.append(len(sub_ind))
        sel = self.page_selector
        rbt = torch.zeros((B, pps), dtype=torch.int32)
        for b in range(B):
            rbt[b, :counts[b]] = bt[b, :counts[b]]
        i32 = dict(dtype=torch.int32)
        checks = [
            ("use_subset", self.use_subset_flag.cpu(), torch.tensor([int(use)], **i32)),
            ("paged_kv_indptr", sel.paged_kv_indptr[:B + 1].cpu(), torch.tensor(ip, **i32)),
            ("paged_kv_indices", sel.paged_kv_indices[:ip[-1]].cpu(), torch.tensor(ind, **i32)),
            ("paged_kv_last_page_len", sel.paged_kv_last_page_len[:B].cpu(), torch.tensor(last, **i32)),
            ("block_table", sel._block_table[:B].cpu(), rbt),
        ]
        if not use or "plan" not in self.layer_roles:  # a planner step rewrites the subset CSR
            checks += [("paged_subset_kv_indptr", sel.paged_subset_kv_indptr[:B + 1].cpu(), torch.tensor(sub_ip, **i32)),
                       ("paged_subset_kv_indices", sel.paged_subset_kv_indices[:sub_ip[-1]].cpu(),
                        torch.tensor(sub_ind, **i32))]
        for name, got, want in checks:
            if not torch.equal(got, want):
                raise RuntimeError(f"DELTA fast decode page-info mismatch in {name}")

    # --------------------------------------------------------- planner scores
    def _compute_page_scores_from_attention_buffer(self) -> torch.Tensor:
        """del3_legacy_softmax page scores of the last decode step's planner layer
        (backend.py:887-913): fp32 ``[batch, pages_per_slot]``, ``score[b, j] = sum over the
        tokens t of page j of max_h softmax_t(logits[b, h, :])``; pages past a row's end score 0.
        From the dump with the planner's lse for the normaliser, or, when the planner kept its
        logits on chip, the scores it wrote."""
        if self._plan_on_chip():
            return self.page_scores
        st = self._decode_csr()
        return K.page_scores_from_logits(self.dump, st.kv_indptr, st.kv_last, self.pages_per_slot, lse=self.lse,
                                         scores=self.page_scores, batch=self.batch_size, workspace=self.workspace)

    def _compute_page_scores_reference(self) -> torch.Tensor:
        """The same scores from the dump alone (softmax normaliser recomputed, no lse): the
        reference's torch-score path used by its selection parity check (backend.py:906-909)."""
        if self._plan_on_chip():
            raise RuntimeError("the planner kept its logits on chip (no dump); set plan_scores_on_chip = False "
                               "or enable delta_debug_page_selection_parity for the dump")
        st = self._decode_csr()
        return K.page_scores_from_logits(self.dump, st.kv_indptr, st.kv_last, self.pages_per_slot,
                                         batch=self.batch_size)

    # ------------------------------------------------------------ decode step
    def _decode_csr(self) -> _StepCSR:
        sel = self.page_selector
        return _StepCSR("decode", sel.paged_kv_indptr, sel.paged_kv_indices, sel.paged_kv_last_page_len,
                        self.pages_per_slot)

    def _decode_body(self, advance: bool):
        """One decode step for all slots; only device work (capturable)."""
        B = self.batch_size
        sel = self.page_selector
        self._profile_cuda_section("delta_decode_page_info", lambda: K.decode_page_info(
            self.cachelens, self.slot_block_table, B, self.k_eff, self.compression_ratio, self.enable_selective_cache,
            sel.paged_kv_indptr, sel.paged_kv_indices, sel.paged_kv_last_page_len, row_block_table=sel._block_table,
            subset_indices=sel.paged_subset_kv_indices, subset_indptr=sel.paged_subset_kv_indptr,
            use_subset=self.use_subset_flag, active=self.active, **self._page_info_budgets()))
        self._step = self._decode_csr()
        try:
            tokens = self.model(self.static_tokens, self.cachelens, self.qo_indptr, sel.paged_kv_indices,
                                sel.paged_kv_indptr, sel.paged_kv_last_page_len)
        finally:
            self._step = None
        self.static_tokens.copy_(tokens)
        if advance:
            self.cachelens.add_(self.active)
        return tokens

    def _capture_decode_graph(self):
        t0 = time.perf_counter()
        stream = torch.cuda.Stream(device=self.device)
        saved_tokens = self.static_tokens.clone()
        stream.wait_stream(torch.cuda.current_stream(self.device))
        self._profile_paused = True
        try:
            with torch.cuda.stream(stream):
                for _ in range(2):  # warm-up (workspaces, BLAS handles); no cachelens advance
                    self._decode_body(advance=False)
                    self.static_tokens.copy_(saved_tokens)
        finally:
            self._profile_paused = False
        torch.cuda.current_stream(self.device).wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self._decode_body(advance=True)
        self._decode_graph = graph
        self._decode_graph_on_chip = self._plan_on_chip()
        self._decode_graph_stats["captures"] += 1
        self._decode_graph_capture_time_s["decode_step"] += time.perf_counter() - t0

    def sync_host_lens(self):
        """Re-read ``cachelens`` / ``active`` from the device into the host mirror (after a
        caller wrote them directly)."""
        self._host_lens = [int(x) for x in self.cachelens.tolist()]
        self._host_active = [int(x) for x in self.active.tolist()]

    def _check_decode_budget(self, n: int):
        if self.enable_delta_debug_fast_decode_page_info_parity:
            # the guard trusts the host mirror; in debug mode check it against the device first
            lens, act = self.cachelens.tolist(), self.active.tolist()
            if lens != self._host_lens or act != self._host_active:
                raise RuntimeError("host copy of cachelens/active differs from the device: call sync_host_lens() "
                                   "after writing them directly")
        for b in range(self.batch_size):
            if self._host_active[b]:
                need = (self._host_lens[b] + n) // PAGE_SIZE + 1
                if need > self._slot_pages[b]:
                    raise RuntimeError(
                        f"decode budget exhausted: slot {b} holds {self._host_lens[b]} tokens and "
                        f"{self._slot_pages[b]} pages; {n} more decode step(s) need {need} pages")

    @torch.inference_mode()
    def decode_steps(self, n: int = 1, use_graph: Optional[bool] = None):
        """Run ``n`` decode steps for every slot, feeding tokens back on the device.  Raises
        before running when a row would need more pages than its slot holds."""
        self._check_decode_budget(n)
        use_graph = self.enable_cuda_graph_decode if use_graph is None else use_graph
        if self._decode_graph is not None and self._decode_graph_on_chip != self._plan_on_chip():
            self._decode_graph = None  # captured with the other planner path (the debug flag moved)
        if use_graph and self._decode_graph is None and self._decode_graph_failed is None:
            try:
                self._capture_decode_graph()
            except Exception as exc:  # capture failure -> eager fallback (backend.py:1138-1150)
                self._decode_graph_failed = repr(exc)
                self._decode_graph_stats["capture_failures"] += 1
                self._decode_graph_fallback_reasons["capture_failed"] += 1
                self._decode_graph_capture_errors["decode_step"] = repr(exc)
                if self.is_main_process:
                    print(f"[hip graph decode] capture failed, running eagerly: {exc}")
        debug = self.enable_delta_debug_fast_decode_page_info_parity or (
            self.enable_delta_debug_page_selection_parity and self.enable_selective_cache)
        for _ in range(n):
            before = self.cachelens.clone() if debug else None
            if use_graph and self._decode_graph is not None:
                try:
                    # one section per replay: a replayed step cannot be split into its parts
                    self._profile_cuda_section("delta_decode_step_graph", self._decode_graph.replay)
                    self._decode_graph_stats["replays"] += 1
                except Exception as exc:  # replay failure -> eager from here on (backend.py:1172-1181)
                    self._decode_graph = None
                    self._decode_graph_failed = repr(exc)
                    self._decode_graph_stats["replay_failures"] += 1
                    self._decode_graph_fallback_reasons["replay_failed"] += 1
                    self._decode_graph_capture_errors["replay"] = repr(exc)
                    if self.is_main_process:
                        print(f"[hip graph decode] replay failed, running eagerly: {exc}")
                    self._decode_body(advance=True)
            else:
                if use_graph:  # the graph is off for this engine (capture failed or disabled)
                    self._decode_graph_fallback_reasons["no_graph_eager_step"] += 1
                self._profile_cuda_section("delta_decode_step_eager", lambda: self._decode_body(advance=True))
            if debug:
                self._debug_checks_after_step(before)
        for b in range(self.batch_size):
            if self._host_active[b]:
                self._host_lens[b] += n
        return self.static_tokens

    # --------------------------------------------------- synthetic contexts
    @torch.inference_mode()
    def prepare_synthetic_decode(self, kv_len, decode_budget: int = 256, seed: int = 0,
                                 fill_std: float = 1.0, k_outlier_channels: int = 0,
                                 k_outlier_scale: float = 8.0):
        """Put every slot in the state "``kv_len`` tokens cached, decoding" (``kv_len`` an int
        or one length per slot): pages for ``kv_len + decode_budget`` tokens from the page
        pool, seeded N(0, fill_std) K/V in every layer, random current tokens.  With
        ``k_outlier_channels`` = n, n seeded head-dim channels of every layer's K are scaled by
        ``k_outlier_scale`` (per-channel outliers).  The pages an earlier call took go back to
        the pool first.  Used by the benchmark and tests (no prompts, no prefill)."""
        B = self.batch_size
        lens = [int(kv_len)] * B if isinstance(kv_len, int) else [int(x) for x in kv_len]
        if len(lens) != B:
            raise ValueError(f"need {B} context lengths, got {len(lens)}")
        for n in lens:
            need = (n + decode_budget) // PAGE_SIZE + 1
            if need > self.pages_per_slot:
                raise ValueError(f"{n} + {decode_budget} tokens need {need} pages > {self.pages_per_slot}")
        if self._synthetic_pages:
            self.page_pool.give_back(self._synthetic_pages)
            self._synthetic_pages = []
        bt = self.slot_block_table.cpu()
        for b, n in enumerate(lens):
            need = (n + decode_budget) // PAGE_SIZE + 1
            pages = self.page_pool.take(need)
            self._synthetic_pages.extend(pages)
            bt[b, :need] = torch.tensor(pages, dtype=torch.int32)
        self.slot_block_table.copy_(bt)
        self._slot_pages = [(n + decode_budget) // PAGE_SIZE + 1 for n in lens]
        self._host_lens = list(lens)
        self._host_active = [1] * B
        gen = torch.Generator(device=self.device)
        gen.manual_seed(seed)
        outl = None
        if k_outlier_channels:
            g2 = torch.Generator()
            g2.manual_seed(seed + 2)
            outl = torch.randperm(self.model.config.head_dim, generator=g2)[:k_outlier_channels].to(self.device)
        seen = set()
        for layer in self.model.layers:
            cache = layer.attention.kv_cache.kv_cache
            if cache.data_ptr() in seen:  # a shared cache (kv_cache_pool) is filled once
                continue
            seen.add(cache.data_ptr())
            cache.normal_(0.0, fill_std, generator=gen)
            if outl is not None:
                cache[:, 0, :, :, outl] *= k_outlier_scale
        self.cachelens.copy_(torch.tensor(lens, dtype=torch.int32))
        self.active.fill_(1)
        vocab = self.model.config.vocab_size
        self.static_tokens.copy_(torch.randint(0, vocab, (1, B), generator=gen, device=self.device))
        self._decode_graph = None

    # ------------------------------------------------------ request serving
    def add_requests(self, input_ids_list: list, max_lengths: list, eot_token_ids: list):
        if self.scheduler is None:
            raise RuntimeError("Backend not initialized. Call setup_caches first.")
        self.scheduler.submit(input_ids_list, max_lengths, eot_token_ids)

    @torch.inference_mode()
    def _sync_slot_block_table(self, slot_id: int, request: ServingRequest, old_page_count: int):
        new = len(request.pages)
        if new > old_page_count:
            self.slot_block_table[slot_id, old_page_count:new].copy_(
                torch.tensor(request.pages[old_page_count:new], dtype=torch.int32))
        self._slot_pages[slot_id] = new

    @torch.inference_mode()
    def _release_slot(self, slot_id: int):
        self.cachelens[slot_id].fill_(0)
        self.active[slot_id].fill_(0)
        self.slot_block_table[slot_id].fill_(int(self.scratch_pages[slot_id]))
        self._host_lens[slot_id] = 0
        self._host_active[slot_id] = 0
        self._slot_pages[slot_id] = self.pages_per_slot  # the scratch page in every column

    @torch.inference_mode()
    def run_scheduler_loop(self):
        """Serve queued requests until done (backend.py:1486-1553)."""
        torch.cuda.synchronize(self.device)
        self.scheduler.t_start = time.perf_counter()
        self._step_records = []
        i = 0
        while True:
            i += 1
            finished = self.scheduler.release_finished()
            if finished and self.throughput_mode:
                if self.is_main_process:
                    print(f"\n[throughput_mode] {len(finished)} request(s) finished -- stopping all")
                self._force_finish_all_requests()
                break
            for slot_id in finished:
                self._release_slot(slot_id)
            for slot_id, req in self.scheduler.fill_free_slots():
                req.admit()
                self.slot_block_table[slot_id].fill_(int(self.scratch_pages[slot_id]))
                self._sync_slot_block_table(slot_id, req, 0)
            if not self.scheduler.any_active():
                break
            self._forward(i)
            if self.enable_delta_impl_profile:
                self._flush_delta_impl_profile_events()
        if self.is_main_process:
            self._print_final_stats()
        return self.get_detailed_results()

    def _force_finish_all_requests(self):
        """Throughput mode: end every running request now (backend.py:1555-1563)."""
        for slot_id in self.scheduler.occupied():
            req = self.scheduler.request_in(slot_id)
            if not req.finished:
                req.state = ServingRequest.FINISHED
                req.t_end = time.perf_counter()
                self.page_pool.give_back(req.pages)
            self.scheduler.slots[slot_id] = None
            self._release_slot(slot_id)

    def _active_slots(self) -> List[int]:
        return self.scheduler.occupied()

    def _record_event(self):
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        return ev

    def _profile_cuda_section(self, name: str, fn):
        """Run ``fn``; with ``delta_impl_profile`` on, time its device work between two HIP events
        on the current stream under ``name`` (backend.py:1570-1578).  While a decode step is
        being captured the section runs untimed (events recorded into a capture would become
        graph nodes); a replayed step is timed whole as ``delta_decode_step_graph``, so the
        per-section breakdown of a decode step comes from eager steps (``cuda_graph_decode``
        off)."""
        if not self.enable_delta_impl_profile or self._profile_paused or torch.cuda.is_current_stream_capturing():
            return fn()
        start = self._record_event()
        out = fn()
        end = self._record_event()
        self._delta_impl_profile_pending.append((name, start, end))
        self._delta_impl_profile_counts[name] += 1
        return out

    def _flush_delta_impl_profile_events(self):
        """Add the finished sections' times into the totals (backend.py:1580-1585); waits for
        the device."""
        if not self._delta_impl_profile_pending:
            return
        torch.cuda.synchronize(self.device)
        for name, start, end in self._delta_impl_profile_pending:
            self._delta_impl_profile_ms[name] += start.elapsed_time(end)
        self._delta_impl_profile_pending.clear()

    def delta_impl_profile_summary(self) -> dict:
        """``{section: {"count", "total_ms", "avg_ms"}}`` of the sections timed so far."""
        self._flush_delta_impl_profile_events()
        out = {}
        for name in sorted(self._delta_impl_profile_counts):
            n = self._delta_impl_profile_counts[name]
            tot = self._delta_impl_profile_ms.get(name, 0.0)
            out[name] = {"count": n, "total_ms": tot, "avg_ms": tot / n if n else 0.0}
        return out

    def _forward(self, step_index: int):
        slots = self._active_slots()
        if not slots:
            return
        reqs = [self.scheduler.request_in(s) for s in slots]
        ev0 = self._record_event()
        decode_only = all(len(r.generated) > 0 for r in reqs)
        if decode_only:
            self._using_subset_cache_this_step = self.enable_selective_cache
            for s, r in zip(slots, reqs):
                old = len(r.pages)
                r.reserve(1)
                self._sync_slot_block_table(s, r, old)
                self._pinned_tokens[s] = r.generated[-1]
            mask = torch.zeros(self.batch_size, dtype=torch.int32)
            mask[slots] = 1
            self.active.copy_(mask)
            self._host_active = mask.tolist()
            self.static_tokens[0].copy_(self._pinned_tokens, non_blocking=True)
            ev1 = self._record_event()
            tokens = self.decode_steps(1)
            ev2 = self._record_event()
            nxt = tokens[0].cpu().tolist()
            next_tokens = [nxt[s] for s in slots]
            qo_lengths = [1] * len(slots)
        else:
            self._using_subset_cache_this_step = False
            ev1 = self._record_event()
            next_tokens, qo_lengths = self._profile_cuda_section("delta_prefill_step",
                                                                 lambda: self._prefill_forward(slots, reqs))
            ev2 = self._record_event()
        for r, t in zip(reqs, next_tokens):
            r.record(int(t))
        self.scheduler.tokens_generated += sum(qo_lengths)
        ev3 = self._record_event()
        self._pending_events.append((step_index, ev0, ev1, ev2, ev3, len(slots)))

    @torch.inference_mode()
    def _prefill_forward(self, slots, reqs):
        """Eager step for rows with several query tokens (prompts): KV append of all new tokens,
        then causal paged prefill attention over each row's pages."""
        dev = self.device
        toks, qo_lens, rows_pages, rows_last, offsets = [], [], [], [], []
        for s, r in zip(slots, reqs):
            q_tokens = r.next_input()
            old = len(r.pages)
            start = r.kv_len(PAGE_SIZE)
            r.reserve(len(q_tokens))
            self._sync_slot_block_table(s, r, old)
            toks.append(q_tokens.to(torch.long))
            qo_lens.append(len(q_tokens))
            rows_pages.append(list(r.pages))
            rows_last.append(r.fill)
            offsets.append(start)
        # the rows' page CSR (after planning, it covers the new tokens)
        kv_indptr, kv_indices = [0], []
        for pages in rows_pages:
            kv_indices.extend(pages)
            kv_indptr.append(len(kv_indices))
        i32 = dict(dtype=torch.int32, device=dev)
        tokens = torch.cat(toks).view(1, -1).to(dev)
        qo_indptr = torch.tensor([0] + list(torch.cumsum(torch.tensor(qo_lens), 0).tolist()), **i32)
        row_ip = torch.tensor(kv_indptr, **i32)
        row_ind = torch.tensor(kv_indices, **i32)
        row_last = torch.tensor(rows_last, **i32)
        self._step = _StepCSR("prefill", row_ip, row_ind, row_last, max(len(p) for p in rows_pages),
                              qo_indptr=qo_indptr, max_qo=max(qo_lens))
        try:
            out = self.model(tokens, torch.tensor(offsets, **i32), qo_indptr, row_ind, row_ip, row_last)
        finally:
            self._step = None
        for s, q_len, start in zip(slots, qo_lens, offsets):
            self.cachelens[s].fill_(start + q_len)
            self.active[s].fill_(1)
            self._host_lens[s] = start + q_len
            self._host_active[s] = 1
        last_pos = (qo_indptr[1:] - 1).long()
        next_tokens = out[0].index_select(0, last_pos).cpu().tolist()
        return next_tokens, qo_lens

    # ------------------------------------------------------------- reporting
    def _print_final_stats(self):
        torch.cuda.synchronize(self.device)
        total_time = time.perf_counter() - self.scheduler.t_start
        total_tokens = self.scheduler.tokens_generated
        for step, e0, e1, e2, e3, bsz in self._pending_events:
            self._step_records.append({"step": step, "collect_pages_ms": e0.elapsed_time(e1),
                                       "model_forward_ms": e1.elapsed_time(e2),
                                       "postprocess_ms": e2.elapsed_time(e3), "step_total_ms": e0.elapsed_time(e3),
                                       "active_bsz": bsz})
        self._pending_events.clear()
        print(f"\n{'=' * 60}\nSCHEDULER PERFORMANCE SUMMARY\n{'=' * 60}")
        print(f"Total time: {total_time:.2f}s")
        print(f"Total requests: {len(self.scheduler.requests)}")
        print(f"Total tokens: {total_tokens:,}")
        print(f"Tokens per second: {total_tokens / max(total_time, 1e-9):.2f}")
        if self.enable_cuda_graph_decode:  # backend.py:2199-2215
            st = self._decode_graph_stats
            print("\nHIP Graph Decode:")
            for key in ("captures", "replays", "capture_failures", "replay_failures"):
                print(f"  {key.replace('_', ' ')}: {st.get(key, 0)}")
            if self._decode_graph_capture_time_s:
                print(f"  capture time by graph: "
                      f"{ {k: round(v, 3) for k, v in self._decode_graph_capture_time_s.items()} }")
            if self._decode_graph_fallback_reasons:
                print(f"  fallback reasons: {dict(self._decode_graph_fallback_reasons)}")
            if self._decode_graph_capture_errors:
                print(f"  capture errors: {self._decode_graph_capture_errors}")
        prof = self.delta_impl_profile_summary() if self.enable_delta_impl_profile else {}
        if prof:  # backend.py:2232-2238
            print("\nDELTA Implementation Profile:")
            for name, r in prof.items():
                print(f"  {name:<32s} avg {r['avg_ms']:8.3f} ms  total {r['total_ms']:10.1f} ms  ({r['count']} calls)")
        if self._step_records:
            n = len(self._step_records)
            for key in ("collect_pages_ms", "model_forward_ms", "postprocess_ms", "step_total_ms"):
                avg = sum(r[key] for r in self._step_records) / n
                print(f"  {key[:-3]:<20s} avg {avg:8.3f} ms  ({n} steps)")
            log_dir = os.environ.get("DELTA_STEP_LOG_DIR")
            if log_dir:
                path = Path(log_dir) / f"step_timings_{time.strftime('%Y%m%d_%H%M%S')}.json"
                path.parent.mkdir(parents=True, exist_ok=True)
                meta = {"total_time_s": total_time, "total_tokens": total_tokens,
                        "tokens_per_second": total_tokens / max(total_time, 1e-9), "batch_size": self.batch_size,
                        "max_length": self.max_length, "page_size": PAGE_SIZE,
                        "selective_cache": self.enable_selective_cache, "num_steps": n,
                        "cuda_graph_decode": self.enable_cuda_graph_decode,
                        "cuda_graph_decode_stats": dict(self._decode_graph_stats),
                        "cuda_graph_decode_fallback_reasons": dict(self._decode_graph_fallback_reasons),
                        "cuda_graph_decode_capture_errors": dict(self._decode_graph_capture_errors),
                        "cuda_graph_decode_capture_time_s": dict(self._decode_graph_capture_time_s),
                        "delta_impl_profile": bool(self.enable_delta_impl_profile),
                        "delta_impl_profile_ms": dict(self._delta_impl_profile_ms),
                        "delta_impl_profile_counts": dict(self._delta_impl_profile_counts),
                        "delta_fused_page_scores": self.enable_delta_fused_page_scores,
                        "delta_fixed_selector": self.enable_delta_fixed_selector,
                        "delta_debug_page_selection_parity": self.enable_delta_debug_page_selection_parity,
                        "delta_subset_plan_reuse": self.enable_delta_subset_plan_reuse,
                        "delta_dump_buffer_dtype": self.delta_dump_buffer_dtype,
                        "delta_page_score_impl": self.delta_page_score_impl,
                        "planner_logits_on_chip": self._plan_on_chip() if self.enable_selective_cache else False,
                        "per_row_budgets": self._per_row_budgets,
                        "subset_budget_rule": list(self._budget_rule) if self._budget_rule else None}
                path.write_text(json.dumps({"meta": meta, "steps": self._step_records}, indent=2))
                print(f"  Step timings saved to: {path}")
        print("=" * 60)

    def get_detailed_results(self):
        if self.scheduler is None:
            return []
        return self.scheduler.report(self.tokenizer)
