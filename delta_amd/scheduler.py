"""Host request bookkeeping with DELTA's page-table semantics.

Mirrors DELTA/Engine/DELTA/scheduler.py:8-186: a shuffled global page pool
(``PageManager``, ``random.seed(seed)`` then ``random.shuffle``; pages are
popped off the end), requests that grow their page list as tokens are planned
(``Request.plan``: ``page_lastlen += qo_len``; every time it reaches 16 a
fresh page is taken, so a full page is followed by an empty one) and a
slot-based batch scheduler.
"""
from __future__ import annotations

import random
import time
from typing import List, Optional, Tuple

import torch


class PageManager:
    """Randomised pool of physical KV pages (scheduler.py:8-40)."""

    def __init__(self, total_pages: int, seed: Optional[int] = None):
        self.total_pages = int(total_pages)
        self.free: List[int] = list(range(self.total_pages))
        self.in_use = set()
        if seed is not None:
            random.seed(seed)
        random.shuffle(self.free)

    def alloc_one(self) -> int:
        if not self.free:
            raise RuntimeError("Out of KV pages: pool is empty")
        p = self.free.pop()
        self.in_use.add(p)
        return p

    def alloc(self, n: int) -> List[int]:
        if n > len(self.free):
            raise RuntimeError(f"Out of KV pages: need {n}, have {len(self.free)} left")
        return [self.alloc_one() for _ in range(n)]

    def free_pages(self, pages: List[int]):
        for p in pages:
            if p in self.in_use:
                self.in_use.remove(p)
                self.free.append(p)
        random.shuffle(self.free)


class Request:
    """One generation request (scheduler.py:43-93)."""

    def __init__(self, id: int, input_ids: torch.Tensor, max_length: int, eot_token_ids: list,
                 page_manager: PageManager) -> None:
        self.id = id
        self.input_ids = input_ids
        self.max_length = max_length
        self.eot_token_ids = eot_token_ids
        self.output_ids: List[int] = []
        self.page_manager = page_manager
        self.status = "waiting"
        self.page_indices: List[int] = []
        self.page_lastlen = 0
        self.start_time = None
        self.end_time = None

    def plan(self, qo_len: int, page_size: int):
        """Account for ``qo_len`` new tokens, taking pages as they fill."""
        self.page_lastlen += qo_len
        while self.page_lastlen >= page_size:
            self.page_indices.append(self.page_manager.alloc_one())
            self.page_lastlen -= page_size

    def initialize_pages(self, slot_id: int, pages_per_slot: int):
        self.status = "active"
        self.start_time = time.perf_counter()
        self.page_indices = [self.page_manager.alloc_one()]
        self.page_lastlen = 0

    def kv_len(self, page_size: int = 16) -> int:
        return (len(self.page_indices) - 1) * page_size + self.page_lastlen

    def get_qo_tokens(self):
        if len(self.output_ids) == 0:
            return self.input_ids
        return torch.tensor([self.output_ids[-1]], dtype=torch.long)

    def append_output(self, token_id: int):
        self.output_ids.append(token_id)
        if token_id in self.eot_token_ids or (len(self.input_ids) + len(self.output_ids)) >= self.max_length:
            self.page_manager.free_pages(self.page_indices)
            self.status = "finished"
            self.end_time = time.perf_counter()
            return True
        return False

    def is_finished(self):
        return self.status == "finished"


class BatchScheduler:
    """Slot scheduler (scheduler.py:96-186)."""

    def __init__(self, batch_size: int, device, is_main_process: bool, pages_per_slot: int,
                 page_size: int, page_manager: PageManager):
        self.is_main_process = is_main_process
        self.pages_per_slot = pages_per_slot
        self.page_size = page_size
        self.page_manager = page_manager
        self.max_pages = 0
        self.active_bsz = 0
        self.request_queue: List[Request] = []
        self.waiting_queue_ids: List[int] = []
        self.runner_slots = torch.tensor([-1] * batch_size)
        self.stats = {"total_tokens_generated": 0, "start_time": None, "encode_steps": 0, "decode_steps": 0}

    def add_requests(self, input_ids_list: list, max_lengths, eot_token_ids: list):
        for i, input_ids in enumerate(input_ids_list):
            max_length = max_lengths[i] if isinstance(max_lengths, list) else max_lengths
            rid = len(self.request_queue)
            self.request_queue.append(Request(rid, input_ids, max_length, eot_token_ids, self.page_manager))
            self.waiting_queue_ids.append(rid)
        if self.is_main_process:
            print(f"Added {len(input_ids_list)} requests. Total waiting: {len(self.waiting_queue_ids)}")

    def schedule_requests(self) -> Tuple[List[int], List[Request]]:
        slots, reqs = [], []
        for slot_id in range(len(self.runner_slots)):
            if self.runner_slots[slot_id] == -1 and self.waiting_queue_ids:
                rid = self.waiting_queue_ids.pop(0)
                self.runner_slots[slot_id] = rid
                slots.append(slot_id)
                reqs.append(self.request_queue[rid])
        return slots, reqs

    def check_finished_requests(self) -> List[int]:
        finished = []
        for slot_id in range(len(self.runner_slots)):
            rid = int(self.runner_slots[slot_id])
            if rid != -1 and self.request_queue[rid].is_finished():
                finished.append(slot_id)
                self.runner_slots[slot_id] = -1
        return finished

    def has_active_requests(self) -> bool:
        return any(int(x) != -1 for x in self.runner_slots)

    def get_detailed_results(self, tokenizer=None):
        results = []
        for r in self.request_queue:
            if not r.is_finished():
                continue
            total = r.end_time - r.start_time if r.end_time and r.start_time else 0
            res = {"request_id": r.id, "status": r.status, "input_length": len(r.input_ids),
                   "output_length": len(r.output_ids), "tokens_generated": len(r.output_ids),
                   "total_time": total,
                   "tokens_per_second": len(r.output_ids) / total if total > 0 else 0}
            if tokenizer:
                try:
                    res["input_text"] = tokenizer.decode(r.input_ids, skip_special_tokens=True)
                    res["output_text"] = tokenizer.decode(r.output_ids, skip_special_tokens=True)
                except Exception:
                    res["input_text"] = f"[{len(r.input_ids)} tokens]"
                    res["output_text"] = f"[{len(r.output_ids)} tokens]"
            results.append(res)
        return sorted(results, key=lambda x: x["request_id"])
