"""Host-side logic of the engine surface (no GPU): config, validation, scheduling, layer roles."""
import random

import pytest
import torch

from delta_amd.public_config import FINAL_PUBLIC_DELTA_BACKEND_CONFIG
from delta_amd.scheduler import BatchSlots, PagePool, ServingRequest


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


def test_page_pool_is_the_seeded_shuffled_pool():
    """Pool order is the reference's (scheduler.py:8-30): ids shuffled by the process-wide
    generator seeded with `seed`, handed out from the end."""
    pool = PagePool(100, seed=0)
    want = list(range(100))
    random.seed(0)
    random.shuffle(want)
    assert pool.take(5) == want[::-1][:5]
    assert pool.available == 95
    with pytest.raises(RuntimeError, match="Out of KV pages"):
        pool.take(1000)
    assert pool.available == 95          # a failed take takes nothing
    pool.give_back([want[-1], 12345])    # unknown ids are ignored
    assert pool.available == 96


def test_request_page_growth():
    """scheduler.py:60-74: one empty page to start; a full page is followed by an empty one."""
    pool = PagePool(64, seed=1)
    r = ServingRequest(0, torch.tensor([1, 2, 3, 4]), 100, [], pool)
    r.admit()
    assert len(r.pages) == 1 and r.fill == 0 and r.kv_len() == 0
    r.reserve(4)
    assert (len(r.pages), r.fill, r.kv_len()) == (1, 4, 4)
    r.reserve(12)  # exactly full: a fresh empty page follows
    assert (len(r.pages), r.fill, r.kv_len()) == (2, 0, 16)
    r.reserve(1)
    assert (len(r.pages), r.fill, r.kv_len()) == (2, 1, 17)
    r.reserve(40)  # several pages at once, in pool order
    assert (len(r.pages), r.fill, r.kv_len()) == (4, 9, 57)
    # a loop over single-token steps lands on the same pages/fill
    sim_pages, sim_fill = 1, 0
    for n in (4, 12, 1, 40):
        sim_fill += n
        while sim_fill >= 16:
            sim_pages += 1
            sim_fill -= 16
    assert (sim_pages, sim_fill) == (len(r.pages), r.fill)
    assert r.next_input().tolist() == [1, 2, 3, 4]
    # finishing returns the pages to the pool
    free_before = pool.available
    r.max_length = 6
    assert not r.record(7)
    assert r.next_input().tolist() == [7]
    assert r.record(8)
    assert r.finished and pool.available == free_before + 4
    # a stop token ends a request too
    r2 = ServingRequest(1, torch.tensor([1]), 100, [2], pool)
    r2.admit()
    assert r2.record(2) and r2.finished


def test_batch_slots():
    pool = PagePool(64, seed=0)
    s = BatchSlots(2, pool, verbose=False)
    s.submit([torch.tensor([1]), torch.tensor([2]), torch.tensor([3])], 10, [])
    placed = s.fill_free_slots()
    assert [slot for slot, _ in placed] == [0, 1] and [r.rid for _, r in placed] == [0, 1]
    for _, r in placed:
        r.admit()
    placed[1][1].record(2)  # not finished yet
    placed[1][1].max_length = 1
    placed[1][1].record(3)
    assert s.release_finished() == [1] and s.occupied() == [0]
    placed = s.fill_free_slots()
    assert [slot for slot, _ in placed] == [1] and placed[0][1].rid == 2 and s.any_active()
    assert [rec["request_id"] for rec in s.report()] == [1]
    rec = s.report()[0]
    assert {"request_id", "status", "input_length", "output_length", "tokens_generated", "total_time",
            "tokens_per_second"} <= set(rec) and rec["output_length"] == 2


def test_request_summary_with_tokenizer():
    class Tok:
        def decode(self, ids, skip_special_tokens=True):
            if len(ids) > 2:
                raise ValueError("too long")
            return "|".join(str(int(i)) for i in ids)

    pool = PagePool(8, seed=0)
    r = ServingRequest(0, torch.tensor([5, 6, 7]), 4, [], pool)
    r.admit()
    r.record(9)
    rec = r.summary(Tok())
    assert rec["output_text"] == "9" and rec["input_text"] == "[3 tokens]"


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


def _reference_style_state(model):
    """A state dict in the reference checkpoint's naming: separate wq/wk/wv (+ biases) and
    w1/w3 (model.py:392-405; FeedForward w1/w2/w3)."""
    cfg = model.config
    q, kv = cfg.n_head * cfg.head_dim, cfg.n_local_heads * cfg.head_dim
    out = {}
    for name, t in model.state_dict().items():
        t = t.clone()
        if name.endswith("attention.wqkv.weight") or name.endswith("attention.wqkv.bias"):
            stem, kind = name.rsplit(".wqkv.", 1)
            for w, part in zip(("wq", "wk", "wv"), t.split([q, kv, kv])):
                out[f"{stem}.{w}.{kind}"] = part.clone()
        elif name.endswith("feed_forward.w13_t"):
            w13 = t.t()
            out[name[:-len("w13_t")] + "w1.weight"] = w13[:cfg.intermediate_size].contiguous()
            out[name[:-len("w13_t")] + "w3.weight"] = w13[cfg.intermediate_size:].contiguous()
        else:
            out[name] = t
    return out


def test_checkpoint_with_separate_projections_loads_every_parameter(tmp_path):
    from delta_amd.backend import LMBackend
    from delta_amd.model import build_random_model
    src = build_random_model("tiny-test", "cpu", torch.bfloat16, seed=5)
    path = tmp_path / "tiny-test" / "model.pth"
    path.parent.mkdir()
    torch.save(_reference_style_state(src), str(path))
    be = LMBackend(device="cpu")
    be.load_model(path, seed=0)          # a different random init underneath
    got = dict(be.model.named_parameters())
    for name, p in src.named_parameters():
        assert torch.equal(got[name], p), name
    # strict, as the reference: a missing or an unknown key raises
    state = _reference_style_state(src)
    state.pop("layers.1.attention.wk.weight")
    torch.save(state, str(path))
    with pytest.raises(Exception):
        LMBackend(device="cpu").load_model(path)
    state = _reference_style_state(src)
    state["layers.0.attention.extra.weight"] = torch.zeros(2)
    torch.save(state, str(path))
    with pytest.raises(RuntimeError, match="Unexpected key"):
        LMBackend(device="cpu").load_model(path)


def test_qkv_bias_and_row_major_gate_up_merge_on_load():
    from delta_amd.model import build_random_model
    src = build_random_model("tiny-test", "cpu", torch.float32, seed=3, qkv_bias=True)
    with torch.no_grad():
        for layer in src.layers:
            layer.attention.wqkv.bias.normal_()
    state = _reference_style_state(src)
    assert "layers.0.attention.wq.bias" in state and "layers.0.feed_forward.w1.weight" in state
    dst = build_random_model("tiny-test", "cpu", torch.float32, seed=4, qkv_bias=True)
    for layer in dst.layers:
        layer.feed_forward.use_row_major_w13()
    dst.load_state_dict(state, strict=True)
    for a, b in zip(src.layers, dst.layers):
        assert torch.equal(a.attention.wqkv.weight, b.attention.wqkv.weight)
        assert torch.equal(a.attention.wqkv.bias, b.attention.wqkv.bias)
        assert torch.equal(a.feed_forward.w13_t.t(), b.feed_forward.w13)
