"""Seeded synthetic inputs for the selective-KV decode hot path.

One layer's planner/selective inputs -- q, a paged KV cache, the CSR page
table, a row-major block table and the selection budget -- for the five
benchmark configurations (and scaled-down variants for parity tests):

  1  B=1,  32q/8kv, 4096 tokens, identity page table, q/K/V ~ N(0,1), k=32, L=8
  2  B=8,  32q/8kv, 16384 tokens, fp16, random page permutation, 8 planted
     pages per row whose K is shifted toward the group's mean query (+2 logit),
     k=128 pages (2048 tokens)
  3  B=32, 32q/8kv, 8192 tokens, bf16, shuffled page pool, k=128, L=8
  4  B=4,  28q/4kv, 65536 tokens, bf16, 4 K channels scaled x8, k=256
  5  B=128, 40q/8kv, lengths ~ U[1024, 32768], bf16, random pages,
     per-row budget max(512, len/8) tokens

Row lengths follow FlashInfer's page-table convention (last page holds
1..16 tokens) unless ``trailing_empty_page`` asks for the DELTA scheduler's
convention (scheduler.py:60-66: a full page is followed by an empty one).
"""
from __future__ import annotations

import math
import random
from dataclasses import dataclass
from typing import List, Optional

import torch

PAGE_SIZE = 16
HEAD_DIM = 128


@dataclass
class LayerCase:
    q: torch.Tensor                 # [B, Hq, 128]
    kv_cache: torch.Tensor          # [num_pages, 2, 16, Hkv, 128]
    kv_indptr: torch.Tensor         # int32 [B+1]
    kv_indices: torch.Tensor        # int32 [sum pages]
    kv_last_page_len: torch.Tensor  # int32 [B]
    block_table: torch.Tensor       # int32 [B, max_pages] (zero padded)
    kv_lens: List[int]
    k: int                          # page budget (global)
    k_per_row: Optional[torch.Tensor]
    L: int
    planted: Optional[torch.Tensor]  # int64 [B, n_planted] logical page ids
    name: str = ""

    @property
    def batch(self) -> int:
        return self.q.shape[0]

    @property
    def max_pages(self) -> int:
        return int((self.kv_indptr[1:] - self.kv_indptr[:-1]).max())

    @property
    def sm_scale(self) -> float:
        return 1.0 / math.sqrt(HEAD_DIM)

    def to(self, device) -> "LayerCase":
        mv = lambda t: None if t is None else t.to(device)
        return LayerCase(mv(self.q), mv(self.kv_cache), mv(self.kv_indptr), mv(self.kv_indices),
                         mv(self.kv_last_page_len), mv(self.block_table), list(self.kv_lens),
                         self.k, mv(self.k_per_row), self.L, mv(self.planted), self.name)


def pages_for(kv_len: int, trailing_empty_page: bool) -> tuple:
    """(pages, last_page_len) of a row holding kv_len tokens."""
    if trailing_empty_page:
        return kv_len // PAGE_SIZE + 1, kv_len % PAGE_SIZE
    n = max(1, -(-kv_len // PAGE_SIZE))
    return n, kv_len - (n - 1) * PAGE_SIZE


def make_case(*, batch: int, hq: int, hkv: int, kv_lens, dtype=torch.bfloat16, seed: int = 0,
              page_order: str = "randperm", k: int = 32, L: int = 8, n_planted: int = 0,
              outlier_channels: int = 0, k_per_row=None, trailing_empty_page: bool = False,
              device="cpu", name: str = "") -> LayerCase:
    """Build one seeded layer case; random tensors are drawn on ``device``."""
    if isinstance(kv_lens, int):
        kv_lens = [kv_lens] * batch
    kv_lens = [int(x) for x in kv_lens]
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    counts, lasts = zip(*(pages_for(n, trailing_empty_page) for n in kv_lens))
    total = int(sum(counts))
    q = torch.randn((batch, hq, HEAD_DIM), generator=gen, device=device, dtype=torch.float32)
    kv = torch.randn((total, 2, PAGE_SIZE, hkv, HEAD_DIM), generator=gen, device=device,
                     dtype=torch.float32)
    if page_order == "identity":
        perm = list(range(total))
    elif page_order == "randperm":
        g2 = torch.Generator()
        g2.manual_seed(seed)
        perm = torch.randperm(total, generator=g2).tolist()
    elif page_order == "shuffle":  # PageManager-style pool: shuffled list, pages popped off the end
        pool = list(range(total))
        random.Random(seed).shuffle(pool)
        perm = [pool.pop() for _ in range(total)]
    else:
        raise ValueError(page_order)
    indptr = [0]
    for c in counts:
        indptr.append(indptr[-1] + c)
    kv_indices = torch.tensor(perm, dtype=torch.int32)
    kv_indptr = torch.tensor(indptr, dtype=torch.int32)
    last = torch.tensor(lasts, dtype=torch.int32)
    max_pages = max(counts)
    bt = torch.zeros((batch, max_pages), dtype=torch.int32)
    for b in range(batch):
        bt[b, :counts[b]] = kv_indices[indptr[b]:indptr[b + 1]]

    planted = None
    G = hq // hkv
    if n_planted:
        g3 = torch.Generator()
        g3.manual_seed(seed + 1)
        planted = torch.zeros((batch, n_planted), dtype=torch.int64)
        qd = q.to(dtype).to(torch.float32)
        for b in range(batch):
            cand = counts[b] - L
            planted[b] = torch.randperm(cand, generator=g3)[:n_planted].sort().values
            for h in range(hkv):
                qbar = qd[b, h * G:(h + 1) * G].mean(dim=0)
                shift = 2.0 * math.sqrt(HEAD_DIM) * qbar / (qbar @ qbar)
                phys = kv_indices[indptr[b] + planted[b]].to(torch.int64).to(device)
                kv[phys, 0, :, h, :] += shift.to(device)
    if outlier_channels:
        g4 = torch.Generator()
        g4.manual_seed(seed + 2)
        ch = torch.randperm(HEAD_DIM, generator=g4)[:outlier_channels].to(device)
        kv[:, 0, :, :, ch] *= 8.0

    kpr = None
    if k_per_row is not None:
        kpr = torch.tensor(list(k_per_row), dtype=torch.int32)
    return LayerCase(q.to(dtype), kv.to(dtype), kv_indptr.to(device), kv_indices.to(device),
                     last.to(device), bt.to(device), kv_lens, int(k), kpr if kpr is None else kpr.to(device),
                     int(L), planted, name)


def config_case(config: int, *, device="cpu", dtype=None, scale: float = 1.0,
                batch: Optional[int] = None) -> LayerCase:
    """The benchmark configuration ``config`` (1-5); ``scale`` < 1 shrinks the context
    (and budget) for oracle-sized parity runs, ``batch`` overrides the row count."""
    def ctx(n):
        return max(PAGE_SIZE * 2, int(n * scale))

    def budget(tokens):
        return max(1, int(tokens * scale) // PAGE_SIZE)

    if config == 1:
        return make_case(batch=batch or 1, hq=32, hkv=8, kv_lens=ctx(4096), dtype=dtype or torch.float32,
                         seed=0, page_order="identity", k=budget(512), L=8, device=device, name="config1")
    if config == 2:
        return make_case(batch=batch or 8, hq=32, hkv=8, kv_lens=ctx(16384), dtype=dtype or torch.float16,
                         seed=0, page_order="randperm", k=budget(2048), L=8, n_planted=8, device=device,
                         name="config2")
    if config == 3:
        return make_case(batch=batch or 32, hq=32, hkv=8, kv_lens=ctx(8192), dtype=dtype or torch.bfloat16,
                         seed=0, page_order="shuffle", k=budget(2048), L=8, device=device, name="config3")
    if config == 4:
        return make_case(batch=batch or 4, hq=28, hkv=4, kv_lens=ctx(65536), dtype=dtype or torch.bfloat16,
                         seed=0, page_order="randperm", k=budget(4096), L=8, outlier_channels=4,
                         device=device, name="config4")
    if config == 5:
        B = batch or 128
        rng = random.Random(0)
        lens = [ctx(rng.randint(1024, 32768)) for _ in range(B)]
        kpr = [max(1, max(int(512 * scale), n // 8) // PAGE_SIZE) for n in lens]
        return make_case(batch=B, hq=40, hkv=8, kv_lens=lens, dtype=dtype or torch.bfloat16, seed=0,
                         page_order="randperm", k=max(kpr), L=8, k_per_row=kpr, device=device,
                         name="config5")
    raise ValueError(f"unknown config {config}")
