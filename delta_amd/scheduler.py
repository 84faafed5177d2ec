"""Serving-loop bookkeeping: the physical page pool, each request's pages, the batch slots.

The engine derives every decode step's page tables on the device from two things this module
owns on the host: which physical pages a slot's request holds (copied into the slot block
table) and how many tokens it holds.  Three rules of DELTA/Engine/DELTA/scheduler.py decide
both, and are kept exactly:

* Pool order (scheduler.py:8-30): the page ids ``0..n-1`` are shuffled once by a generator
  seeded with ``seed`` (the same permutation ``random.seed(seed); random.shuffle(ids)``
  gives) and handed out from the end of that order.
* Page growth (scheduler.py:60-74): a request starts on one empty page; adding ``n`` tokens
  raises the last page's fill by ``n`` and takes a fresh page each time the fill reaches 16,
  so a full page is always followed by an empty one and ``kv_len = (pages - 1) * 16 + fill``.
* Completion (scheduler.py:83-90): a request ends on a stop token or once prompt plus output
  reach ``max_length``, and its pages go back to the pool.

Everything else is this build's own: requests live in a flat list indexed by id, slots hold
request ids (``None`` when free), waiting ids sit in a deque, and the pool reshuffles its
free ids with its own generator when pages come back (the reference reshuffles with the
process-wide one, so only the order after a release may differ).
"""
from __future__ import annotations

import random
import time
from collections import deque
from typing import Deque, Dict, List, Optional, Sequence, Tuple

import torch

PAGE_SIZE = 16


class PagePool:
    """Shuffled pool of physical KV page ids."""

    def __init__(self, total_pages: int, seed: Optional[int] = None):
        self.total_pages = int(total_pages)
        self._rng = random.Random(seed)
        ids = list(range(self.total_pages))
        self._rng.shuffle(ids)
        self._free: List[int] = ids          # handed out from the end
        self._held = set()

    @property
    def available(self) -> int:
        return len(self._free)

    def take(self, n: int = 1) -> List[int]:
        """``n`` pages from the end of the free order (all or none)."""
        if n > len(self._free):
            raise RuntimeError(f"Out of KV pages: {n} wanted, {len(self._free)} free")
        got = [self._free.pop() for _ in range(n)]
        self._held.update(got)
        return got

    def give_back(self, pages: Sequence[int]) -> None:
        back = [p for p in pages if p in self._held]
        self._held.difference_update(back)
        self._free.extend(back)
        self._rng.shuffle(self._free)


class ServingRequest:
    """One prompt being served: its tokens, its pages and its timing."""

    WAITING, ACTIVE, FINISHED = "waiting", "active", "finished"

    def __init__(self, rid: int, prompt: torch.Tensor, max_length: int, stop_ids: Sequence[int],
                 pool: PagePool):
        self.rid = rid
        self.prompt = prompt
        self.max_length = int(max_length)
        self.stop_ids = set(int(t) for t in stop_ids)
        self.generated: List[int] = []
        self.pages: List[int] = []
        self.fill = 0                  # tokens in the last page
        self.state = self.WAITING
        self.t_start: Optional[float] = None
        self.t_end: Optional[float] = None
        self._pool = pool

    # -- pages
    def admit(self) -> None:
        """Start serving: one empty page."""
        self.state = self.ACTIVE
        self.t_start = time.perf_counter()
        self.pages = self._pool.take(1)
        self.fill = 0

    def reserve(self, n_tokens: int, page_size: int = PAGE_SIZE) -> None:
        """Account for ``n_tokens`` new tokens (the page-growth rule above)."""
        self.fill += int(n_tokens)
        grow = self.fill // page_size
        if grow:
            self.pages.extend(self._pool.take(grow))
            self.fill -= grow * page_size

    def kv_len(self, page_size: int = PAGE_SIZE) -> int:
        return (len(self.pages) - 1) * page_size + self.fill

    # -- tokens
    def next_input(self) -> torch.Tensor:
        """The tokens of this request's next forward: the prompt, then the last output."""
        return self.prompt if not self.generated else torch.tensor([self.generated[-1]], dtype=torch.long)

    def record(self, token: int) -> bool:
        """Append an output token; True when the request is now finished."""
        self.generated.append(int(token))
        if int(token) in self.stop_ids or len(self.prompt) + len(self.generated) >= self.max_length:
            self._pool.give_back(self.pages)
            self.state = self.FINISHED
            self.t_end = time.perf_counter()
            return True
        return False

    @property
    def finished(self) -> bool:
        return self.state == self.FINISHED

    def summary(self, tokenizer=None) -> Dict:
        """The per-request record the reference's result consumers read (same keys)."""
        elapsed = (self.t_end - self.t_start) if (self.t_end and self.t_start) else 0
        n_out = len(self.generated)
        rec = {"request_id": self.rid, "status": self.state, "input_length": len(self.prompt),
               "output_length": n_out, "tokens_generated": n_out, "total_time": elapsed,
               "tokens_per_second": n_out / elapsed if elapsed > 0 else 0}
        if tokenizer is not None:
            rec["input_text"] = _decode_or_placeholder(tokenizer, self.prompt)
            rec["output_text"] = _decode_or_placeholder(tokenizer, self.generated)
        return rec


def _decode_or_placeholder(tokenizer, ids) -> str:
    try:
        return tokenizer.decode(ids, skip_special_tokens=True)
    except Exception:  # a tokenizer that cannot take these ids still yields a record
        return f"[{len(ids)} tokens]"


class BatchSlots:
    """Fixed batch slots over a queue of requests (free slots take waiting requests in order)."""

    def __init__(self, batch_size: int, pool: PagePool, verbose: bool = True):
        self.pool = pool
        self.verbose = verbose
        self.slots: List[Optional[int]] = [None] * int(batch_size)
        self.requests: List[ServingRequest] = []
        self.waiting: Deque[int] = deque()
        self.tokens_generated = 0
        self.t_start: Optional[float] = None

    def submit(self, prompts: Sequence[torch.Tensor], max_lengths, stop_ids: Sequence[int]) -> None:
        for i, prompt in enumerate(prompts):
            cap = max_lengths[i] if isinstance(max_lengths, (list, tuple)) else max_lengths
            req = ServingRequest(len(self.requests), prompt, cap, stop_ids, self.pool)
            self.requests.append(req)
            self.waiting.append(req.rid)
        if self.verbose:
            print(f"queued {len(prompts)} request(s); {len(self.waiting)} waiting")

    def fill_free_slots(self) -> List[Tuple[int, ServingRequest]]:
        """Place waiting requests into free slots (lowest slot first); returns (slot, request)."""
        placed = []
        for s, rid in enumerate(self.slots):
            if rid is None and self.waiting:
                req = self.requests[self.waiting.popleft()]
                self.slots[s] = req.rid
                placed.append((s, req))
        return placed

    def release_finished(self) -> List[int]:
        """Free the slots whose request finished; returns those slot ids."""
        done = [s for s, rid in enumerate(self.slots) if rid is not None and self.requests[rid].finished]
        for s in done:
            self.slots[s] = None
        return done

    def occupied(self) -> List[int]:
        return [s for s, rid in enumerate(self.slots) if rid is not None]

    def request_in(self, slot: int) -> ServingRequest:
        return self.requests[self.slots[slot]]

    def any_active(self) -> bool:
        return any(rid is not None for rid in self.slots)

    def report(self, tokenizer=None) -> List[Dict]:
        return [r.summary(tokenizer) for r in self.requests if r.finished]
