"""``mylib::*`` torch.library ops with the reference's names and schemas, on the HIP kernels.

Reference registrations: ``mylib::target_decode`` / ``target_subset_decode`` /
``target_decode_plan`` (backend.py:461-585), ``mylib::update_kv``
(utils.py:31-79), ``mylib::rope`` (model.py:152-175).  As in the reference the
page tables are a side channel: the active ``LMBackend`` owns the step's CSR
buffers, and the attention ops read them from it.  Each op has a fake
(meta) implementation returning ``empty_like`` like the reference.
"""
from __future__ import annotations

import torch

from . import kernels as K

_ACTIVE = {"backend": None}


def set_active_backend(backend) -> None:
    """Route the attention / rope ops to ``backend`` (done by LMBackend.setup_caches)."""
    _ACTIVE["backend"] = backend


def active_backend():
    b = _ACTIVE["backend"]
    if b is None:
        raise RuntimeError("no active LMBackend: call setup_caches() before running the model")
    return b


def _defined(name: str) -> bool:
    try:
        getattr(torch.ops.mylib, name)
        return True
    except (AttributeError, RuntimeError):
        return False


def _register():
    if not _defined("target_decode"):
        for op in ("target_decode", "target_subset_decode", "target_decode_plan"):
            torch.library.define(f"mylib::{op}", "(Tensor q, Tensor kv_cache) -> Tensor")

        @torch.library.impl("mylib::target_decode", "cuda")
        def target_decode(q, kv_cache):
            return active_backend().attn_full(q, kv_cache)

        @torch.library.impl("mylib::target_subset_decode", "cuda")
        def target_subset_decode(q, kv_cache):
            return active_backend().attn_subset(q, kv_cache)

        @torch.library.impl("mylib::target_decode_plan", "cuda")
        def target_decode_plan(q, kv_cache):
            return active_backend().attn_plan(q, kv_cache)

        for op in ("target_decode", "target_subset_decode", "target_decode_plan"):
            torch.library.register_fake(f"mylib::{op}")(lambda q, kv_cache: torch.empty_like(q))

    if not _defined("update_kv"):
        torch.library.define(
            "mylib::update_kv",
            "(Tensor k, Tensor v, Tensor kv_append_indptr, Tensor(a!) kv_cache, Tensor kv_page_indices, "
            "Tensor kv_page_indptr, Tensor cachelen) -> ()")

        @torch.library.impl("mylib::update_kv", "cuda")
        def update_kv(k, v, kv_append_indptr, kv_cache, kv_page_indices, kv_page_indptr, kv_page_last_len):
            K.append_kv(k, v, kv_append_indptr, kv_cache, kv_page_indices, kv_page_indptr, kv_page_last_len)

        @torch.library.register_fake("mylib::update_kv")
        def update_kv_fake(k, v, kv_append_indptr, kv_cache, kv_page_indices, kv_page_indptr, kv_page_last_len):
            return None

    if not _defined("rope"):
        torch.library.define("mylib::rope",
                             "(Tensor q, Tensor k, Tensor indptr, Tensor offsets) -> (Tensor ropeq, Tensor ropek)")

        @torch.library.impl("mylib::rope", "cuda")
        def rope(q, k, indptr, offsets):
            return K.rope(q, k, indptr, offsets, **active_backend().rope_params())

        @torch.library.register_fake("mylib::rope")
        def rope_fake(q, k, indptr, offsets):
            return torch.empty_like(q), torch.empty_like(k)


_register()
