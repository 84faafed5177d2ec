"""Host-side logic of the engine surface (no GPU): config, validation, scheduling, layer roles."""
import random

import pytest
import torch

from delta_amd.public_config import FINAL_PUBLIC_DELTA_BACKEND_CONFIG
from delta_amd.scheduler import BatchScheduler, PageManager, Request


def test_public_config_matches_reference_release():
    # DELTA/Engine/DELTA/public_config.py:9-20
    assert FINAL_PUBLIC_DELTA_BACKEND_CONFIG == {
        "page_selector_version": "v2",
        "delta_dump_buffer_dtype": "fp32",
        "delta_page_score_impl": "del3_legacy_softmax",
        "cuda_graph_delta_subset_segments": True,
        "delta_fused_page_scores": True,
        "delta_fixed_selector": True,
        "delta_fast_decode_page_info": True,
        "delta_v2_position_bias": True,
        "delta_subset_plan_reuse": True,
        "delta_impl_profile": False,
    }


def test_backend_validation_messages():
    from delta_amd.backend import LMBackend
    with pytest.raises(ValueError, match="page_selector_version"):
        LMBackend(device="cpu", page_selector_version="v3")
    with pytest.raises(ValueError, match="delta_dump_buffer_dtype"):
        LMBackend(device="cpu", delta_dump_buffer_dtype="bf16")
    with pytest.raises(ValueError, match="delta_page_score_impl"):
        LMBackend(device="cpu", delta_page_score_impl="foo")
    # accepted by the reference but not built here: fail loudly
    for kw in (dict(page_selector_version="v1"), dict(delta_dump_buffer_dtype="fp16"),
               dict(delta_page_score_impl="delta_lse")):
        with pytest.raises(NotImplementedError):
            LMBackend(device="cpu", **kw)
    b = LMBackend(device="cpu", cuda_graph_decode=True, **FINAL_PUBLIC_DELTA_BACKEND_CONFIG)
    assert b.enable_cuda_graph_decode and b.page_selector_version == "v2"
    with pytest.raises(NotImplementedError):
        b.load_model("random:tiny-test", use_tp=True)


def test_page_manager_is_the_seeded_shuffled_pool():
    pm = PageManager(100, seed=0)
    pool = list(range(100))
    random.seed(0)
    random.shuffle(pool)
    assert [pm.alloc_one() for _ in range(5)] == pool[::-1][:5]
    with pytest.raises(RuntimeError, match="Out of KV pages"):
        pm.alloc(1000)


def test_request_plan_page_growth():
    pm = PageManager(64, seed=1)
    r = Request(0, torch.tensor([1, 2, 3, 4]), 100, [], pm)
    r.initialize_pages(0, 8)
    assert len(r.page_indices) == 1 and r.page_lastlen == 0
    r.plan(4, 16)
    assert (len(r.page_indices), r.page_lastlen, r.kv_len()) == (1, 4, 4)
    r.plan(12, 16)  # exactly full: a fresh empty page follows
    assert (len(r.page_indices), r.page_lastlen, r.kv_len()) == (2, 0, 16)
    r.plan(1, 16)
    assert (len(r.page_indices), r.page_lastlen, r.kv_len()) == (2, 1, 17)
    # finishing returns the pages to the pool
    free_before = len(pm.free)
    r.max_length = 5
    assert r.append_output(7)
    assert r.is_finished() and len(pm.free) == free_before + 2


def test_batch_scheduler_slots():
    pm = PageManager(64, seed=0)
    s = BatchScheduler(2, "cpu", False, 8, 16, pm)
    s.add_requests([torch.tensor([1]), torch.tensor([2]), torch.tensor([3])], 10, [])
    slots, reqs = s.schedule_requests()
    assert slots == [0, 1] and [r.id for r in reqs] == [0, 1]
    reqs[1].status = "finished"
    assert s.check_finished_requests() == [1]
    slots, reqs = s.schedule_requests()
    assert slots == [1] and reqs[0].id == 2 and s.has_active_requests()


def test_layer_roles_follow_full_cache_layers():
    # model.py:177-196: full -> target_decode, last full before a non-full -> plan, else subset
    from delta_amd.model import ModelArgs, Transformer
    cfg = ModelArgs.from_name("tiny-test")
    cfg.n_layer = 6
    cfg.full_cache_layers = [0, 1, 4]
    m = Transformer(cfg)
    m.setup_caches(num_pages=2, page_size=16)
    assert m.layer_roles == ["full", "plan", "subset", "subset", "plan", "subset"]
    cfg2 = ModelArgs.from_name("tiny-test")
    m2 = Transformer(cfg2)
    m2.setup_caches(num_pages=2, page_size=16)
    assert m2.layer_roles == ["full"] * 4


def test_ops_registered_with_reference_schemas():
    import delta_amd.ops  # noqa: F401
    s = str(torch.ops.mylib.update_kv.default._schema)
    assert "Tensor(a!) kv_cache" in s and s.endswith("-> ()")
    assert "(Tensor q, Tensor kv_cache) -> Tensor" in str(torch.ops.mylib.target_decode_plan.default._schema)
    assert "-> (Tensor ropeq, Tensor ropek)" in str(torch.ops.mylib.rope.default._schema)


def test_workload_shapes():
    from delta_amd.workloads import config_case
    c = config_case(1)
    assert tuple(c.q.shape) == (1, 32, 128) and c.kv_cache.shape[0] == 256 and c.k == 32
    assert c.kv_last_page_len.tolist() == [16] and torch.equal(c.kv_indices, torch.arange(256, dtype=torch.int32))
    c2 = config_case(2, scale=1 / 16)
    assert c2.planted.shape == (8, 8) and c2.q.dtype == torch.float16
    assert bool((c2.planted < c2.max_pages - c2.L).all())
    c5 = config_case(5, scale=1 / 64, batch=6)
    assert c5.k_per_row.numel() == 6 and len(set(c5.kv_lens)) > 1
