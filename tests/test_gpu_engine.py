"""GPU engine tests: the LMBackend decode step wires the right tables into the kernels.

Each layer's recorded (q, o) is checked against the CPU oracle on the layer's
own cache after the step: full layers over the full CSR, the planner layer's
selection against the oracle's selection from the same q/K, subset layers over
the engine's subset CSR.  The captured hipGraph must reproduce eager steps bit
for bit, with eager work between replays.
"""
import pytest
import torch

from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def make_engine(selective=True, graph=False, B=3, max_len=512, full_layers=(0, 1), k=6, L=2, ratio=1.0,
                n_layer=None, dtype=torch.bfloat16, **backend_kw):
    from delta_amd.backend import LMBackend
    eng = LMBackend(dtype=dtype, device=DEV, cuda_graph_decode=graph, **backend_kw)
    eng.load_model("random:tiny-test", seed=1, **({} if n_layer is None else {"n_layer": n_layer}))
    cfg = eng.model.config
    cfg.enable_selective_cache = selective
    cfg.full_cache_layers = list(full_layers)
    cfg.subset_cache_size = k
    cfg.compression_ratio = ratio
    cfg.L = L
    eng.setup_caches(max_batch_size=B, max_seq_length=max_len)
    return eng


def assert_close(got, want, what):
    got = got.float().cpu()
    want = want.float().cpu()
    err = (got - want).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(got.flatten(), want.flatten(), dim=0).item()
    assert err <= 2e-2 and cos > 0.999, f"{what}: err {err} cos {cos}"


def _csr(eng):
    sel = eng.page_selector
    B = eng.batch_size
    ip = sel.paged_kv_indptr[:B + 1].cpu()
    return (ip, sel.paged_kv_indices[:int(ip[-1])].cpu(), sel.paged_kv_last_page_len[:B].cpu(),
            sel.paged_subset_kv_indptr[:B + 1].cpu())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("lens", [[100, 257, 400], [300, 300, 300]])
def test_decode_step_layers_match_oracle(lens, dtype):
    eng = make_engine(dtype=dtype)
    eng.prepare_synthetic_decode(lens, decode_budget=16, seed=3)
    for layer in eng.model.layers:
        layer.attention.record = []
    eng.decode_steps(1, use_graph=False)
    torch.cuda.synchronize()
    ip, ind, last, sip = _csr(eng)
    sind = eng.page_selector.paged_subset_kv_indices[:int(sip[-1])].cpu()
    assert last.tolist() == [(n + 1) % 16 for n in lens]
    assert eng.cachelens.cpu().tolist() == [n + 1 for n in lens]
    scale = 1 / 128 ** 0.5
    for li, (role, layer) in enumerate(zip(eng.layer_roles, eng.model.layers)):
        (q, o), = layer.attention.record
        cache = layer.attention.kv_cache.kv_cache.cpu()
        qc = q.cpu()
        if role in ("full", "plan"):
            ref, _ = O.paged_decode_attention(qc, cache, ip, ind, last, scale)
            assert_close(o, ref, f"layer {li} ({role})")
        if role == "plan":
            counts = ip[1:] - ip[:-1]
            bt = O.block_table_from_csr(ip, ind, int(counts.max()))
            x = O.dump_logits(qc, cache, ip, ind, last, scale, int(counts.max()) * 16)
            scores = O.legacy_softmax_page_scores(x, len(lens), int(counts.max()))
            want_i, want_p = O.select_pages(scores, counts, bt, eng.k_eff, eng.L)
            assert sip.tolist() == want_p.tolist()
            if sind.tolist() != want_i.tolist():  # allowed only for near-threshold pages
                keys = O.prepare_scores(scores, counts, eng.L)
                for b in range(len(lens)):
                    got = set(sind[int(sip[b]):int(sip[b + 1])].tolist())
                    want = set(want_i[int(want_p[b]):int(want_p[b + 1])].tolist())
                    thr = sorted(keys[b].tolist(), reverse=True)[eng.k_eff - 1]
                    for p in got ^ want:
                        j = bt[b].tolist().index(p)
                        assert abs(float(keys[b, j]) - thr) <= 2e-4 * abs(thr)
        if role == "subset":
            ref, _ = O.paged_decode_attention(qc, cache, sip, sind, last, scale)
            assert_close(o, ref, f"layer {li} (subset)")


def test_gate_off_subset_layers_attend_everything():
    eng = make_engine(ratio=1e9)
    eng.prepare_synthetic_decode([100, 200, 300], decode_budget=16, seed=4)
    eng.decode_steps(1, use_graph=False)
    torch.cuda.synchronize()
    ip, ind, last, sip = _csr(eng)
    assert int(eng.use_subset_flag) == 0
    assert torch.equal(sip, ip)
    assert torch.equal(eng.page_selector.paged_subset_kv_indices[:int(ip[-1])].cpu(), ind)


def _snapshot(eng):
    return ([l.attention.kv_cache.kv_cache.clone() for l in eng.model.layers], eng.cachelens.clone(),
            eng.static_tokens.clone())


@torch.inference_mode()
def _restore(eng, snap):
    caches, cl, tok = snap
    for l, c in zip(eng.model.layers, caches):
        l.attention.kv_cache.kv_cache.copy_(c)
    eng.cachelens.copy_(cl)
    eng.static_tokens.copy_(tok)
    eng.sync_host_lens()


@pytest.mark.parametrize("selective,dtype", [(True, torch.bfloat16), (False, torch.bfloat16),
                                             (True, torch.float16)], ids=["selective", "full", "selective_fp16"])
def test_graph_replays_match_eager_steps(selective, dtype):
    eng = make_engine(selective=selective, graph=True, B=4, dtype=dtype)
    eng.prepare_synthetic_decode([15, 16, 31, 200], decode_budget=40, seed=5)  # crosses page boundaries
    snap = _snapshot(eng)
    eager = []
    for _ in range(20):
        eager.append(eng.decode_steps(1, use_graph=False).clone())
    eager_caches = [l.attention.kv_cache.kv_cache.clone() for l in eng.model.layers]
    _restore(eng, snap)
    for i in range(20):
        tok = eng.decode_steps(1, use_graph=True).clone()
        # unrelated eager work between replays
        a = torch.randn(256, 256, device=DEV)
        (a @ a).sum().item()
        assert torch.equal(tok, eager[i]), f"replay {i} differs from the eager step"
    assert eng._decode_graph is not None and eng._decode_graph_stats["replays"] == 20
    for l, c in zip(eng.model.layers, eager_caches):
        assert torch.equal(l.attention.kv_cache.kv_cache, c)


def test_partial_batch_idle_slots_untouched():
    eng = make_engine(B=3)
    eng.prepare_synthetic_decode([50, 60, 70], decode_budget=16, seed=6)
    eng._release_slot(1)
    caches = [l.attention.kv_cache.kv_cache.clone() for l in eng.model.layers]
    owned = eng.slot_block_table[[0, 2]].flatten().long()
    eng.decode_steps(3, use_graph=False)
    torch.cuda.synchronize()
    assert eng.cachelens.cpu().tolist() == [53, 0, 73]
    scratch = int(eng.scratch_pages[1])
    for l, c in zip(eng.model.layers, caches):
        cur = l.attention.kv_cache.kv_cache
        changed = (cur != c).flatten(1).any(1).nonzero().flatten().tolist()
        assert all(p == scratch or p in set(owned.tolist()) for p in changed)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_serving_loop_with_prefill(dtype):
    """Three requests through two slots (prefill, decode, a slot reused): every request gets
    its full output, every page returns to the pool, and the token streams are identical with
    the decode steps eager or replayed from the captured graph."""
    prompts = [torch.tensor([1, 2, 3, 4]), torch.tensor([5, 6, 7, 8, 9, 10, 11]), torch.tensor([12] * 20)]
    caps = [90, 80, 100]
    streams = []
    for graph in (False, True):
        eng = make_engine(B=2, max_len=256, k=4, graph=graph, dtype=dtype)
        eng.add_requests(prompts, caps, [])
        results = eng.run_scheduler_loop()
        assert len(results) == 3
        for r, p, ml in zip(results, prompts, caps):
            assert r["output_length"] == ml - len(p) and r["status"] == "finished"
        assert eng.page_pool.available == eng.page_pool.total_pages
        assert not eng.scheduler.any_active()
        if graph:
            assert eng._decode_graph_stats["replays"] > 0 and eng._decode_graph_failed is None
        streams.append([list(r.generated) for r in eng.scheduler.requests])
    assert streams[0] == streams[1]
    assert all(len(s) > 0 for s in streams[0])


def test_prefill_rows_are_causal():
    eng = make_engine(B=1, max_len=256)
    for layer in eng.model.layers:
        layer.attention.record = []
    prompt = torch.arange(1, 41)
    eng.add_requests([prompt], [41], [])
    eng.run_scheduler_loop()
    (q, o), = eng.model.layers[0].attention.record[:1]
    req = eng.scheduler.requests[0]
    cache = eng.model.layers[0].attention.kv_cache.kv_cache.cpu()
    pages = torch.tensor(req.pages, dtype=torch.int32)
    n = 40
    ip = torch.zeros(n + 1, dtype=torch.int32)
    ind, lastl = [], []
    for i in range(n):
        cnt = i // 16 + 1
        ind.extend(pages[:cnt].tolist())
        ip[i + 1] = len(ind)
        lastl.append(i % 16 + 1)
    ref, _ = O.paged_decode_attention(q.cpu(), cache, ip, torch.tensor(ind, dtype=torch.int32),
                                      torch.tensor(lastl, dtype=torch.int32), 1 / 128 ** 0.5)
    assert_close(o, ref, "prefill layer 0")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_two_row_prefill_step_matches_oracle(dtype):
    """One eager prompt step for two rows of different lengths: layer 0's attention output
    equals the oracle's causal prefill over each row's own pages."""
    eng = make_engine(B=2, max_len=256, dtype=dtype)
    for layer in eng.model.layers:
        layer.attention.record = []
    prompts = [torch.arange(1, 24), torch.arange(30, 39)]
    eng.add_requests(prompts, [60, 60], [])
    with torch.inference_mode():  # the first iteration of run_scheduler_loop
        placed = eng.scheduler.fill_free_slots()
        new_slots = [slot for slot, _ in placed]
        for slot_id, req in placed:
            req.admit()
            eng.slot_block_table[slot_id].fill_(int(eng.scratch_pages[slot_id]))
            eng._sync_slot_block_table(slot_id, req, 0)
        eng._forward(1)
    torch.cuda.synchronize()
    (q, o), = eng.model.layers[0].attention.record[:1]
    cache = eng.model.layers[0].attention.kv_cache.kv_cache.cpu()
    reqs = [eng.scheduler.request_in(s) for s in new_slots]
    lens = [len(p) for p in prompts]
    pages = [r.pages[:(n + 15) // 16] for r, n in zip(reqs, lens)]
    ip = torch.tensor([0, len(pages[0]), len(pages[0]) + len(pages[1])], dtype=torch.int32)
    ind = torch.tensor(pages[0] + pages[1], dtype=torch.int32)
    last = torch.tensor([n - ((n + 15) // 16 - 1) * 16 for n in lens], dtype=torch.int32)
    qo_indptr = torch.tensor([0, lens[0], lens[0] + lens[1]], dtype=torch.int32)
    ref, _ = O.paged_prefill_attention(q.cpu(), qo_indptr, cache, ip, ind, last, 1 / 128 ** 0.5)
    assert_close(o, ref, "two-row prefill layer 0")


def test_fused_dense_path_matches_reference_structure():
    """The fused element-wise kernels give the same logits as the reference's op-by-op blocks."""
    eng = make_engine(B=3)
    eng.prepare_synthetic_decode([100, 200, 300], decode_budget=16, seed=7)
    sel = eng.page_selector
    outs = []
    with torch.inference_mode():
        for fused in (True, False):
            eng.model.fused = fused
            eng._step = eng._decode_csr()
            import delta_amd.kernels as K
            K.decode_page_info(eng.cachelens, eng.slot_block_table, eng.batch_size, eng.k_eff,
                               eng.compression_ratio, True, sel.paged_kv_indptr, sel.paged_kv_indices,
                               sel.paged_kv_last_page_len, row_block_table=sel._block_table,
                               subset_indices=sel.paged_subset_kv_indices,
                               subset_indptr=sel.paged_subset_kv_indptr, use_subset=eng.use_subset_flag)
            outs.append(eng.model.forward_logits(eng.static_tokens, eng.cachelens, eng.qo_indptr,
                                                 sel.paged_kv_indices, sel.paged_kv_indptr,
                                                 sel.paged_kv_last_page_len).float())
            eng._step = None
    a, b = outs
    cos = torch.nn.functional.cosine_similarity(a.flatten(), b.flatten(), dim=0).item()
    assert cos > 0.999, cos
    assert (a - b).abs().max().item() < 0.05 * b.abs().max().item()


def test_synthetic_fill_outlier_channels():
    """prepare_synthetic_decode(k_outlier_channels=n): n channels of every layer's K scaled by
    k_outlier_scale, V and the other K channels untouched (config 4's per-channel outliers)."""
    eng = make_engine()
    eng.prepare_synthetic_decode([200, 200, 200], decode_budget=16, seed=3)
    ref = [l.attention.kv_cache.kv_cache.clone() for l in eng.model.layers]
    eng.prepare_synthetic_decode([200, 200, 200], decode_budget=16, seed=3, k_outlier_channels=2,
                                 k_outlier_scale=8.0)
    for layer, r in zip(eng.model.layers, ref):
        c = layer.attention.kv_cache.kv_cache
        assert torch.equal(c[:, 1], r[:, 1])                    # V untouched
        ratio = (c[:, 0].float().abs().sum(dim=(0, 1, 2)) / r[:, 0].float().abs().sum(dim=(0, 1, 2))).cpu()
        scaled = (ratio - 8.0).abs() < 1e-2
        assert int(scaled.sum()) == 2 and bool(((ratio - 1.0).abs() < 1e-6)[~scaled].all())


def test_row_major_gate_up_matches_transposed():
    """use_row_major_w13 (small-batch engines: the gate|up GEMM on delta_gemm_skinny) keeps the
    FFN's values: same output as the transposed layout on hipBLASLt, to bf16 rounding."""
    from delta_amd.model import FeedForward, ModelArgs
    torch.manual_seed(5)
    ff = FeedForward(ModelArgs(dim=512, intermediate_size=1024, n_head=4, n_local_heads=2))
    with torch.no_grad():
        ff.w13_t.normal_(0, 0.05)
        ff.w2.weight.normal_(0, 0.05)
    ff = ff.to(device=DEV, dtype=torch.bfloat16)
    x = torch.randn(3, 512, device=DEV, dtype=torch.bfloat16)
    with torch.inference_mode():
        y_t = ff.forward_fused(x).float()
        ff.use_row_major_w13()
        assert not hasattr(ff, "w13_t") and tuple(ff.w13.shape) == (2048, 512)
        y_r = ff.forward_fused(x).float()
        y_plain = ff(x).float()
    for y in (y_r, y_plain):
        assert (y - y_t).abs().max().item() <= 2e-2 * y_t.abs().max().item()


def test_decode_budget_is_enforced_before_the_step():
    """A decode step that would take a row past the pages its slot holds is refused on the
    host before anything runs (the device metadata would clamp the row and overwrite its
    last slot).  Row 2 holds 120 tokens and (120 + 16) // 16 + 1 = 9 pages: 23 more decode
    steps fit ((120 + 23) // 16 + 1 = 9), the 24th does not; rows 0 and 1 (96 tokens, 8 pages)
    have room for 31."""
    eng = make_engine(B=3, max_len=512)
    eng.prepare_synthetic_decode([96, 96, 120], decode_budget=16, seed=2)
    with pytest.raises(RuntimeError, match="decode budget exhausted: slot 2"):
        eng.decode_steps(24, use_graph=False)
    assert eng.cachelens.tolist() == [96, 96, 120]        # nothing ran
    eng.decode_steps(23, use_graph=False)
    assert eng.cachelens.tolist() == [119, 119, 143]
    with pytest.raises(RuntimeError, match="decode budget exhausted"):
        eng.decode_steps(1, use_graph=False)


def test_debug_parity_checks_run_after_eager_and_replayed_steps():
    """delta_debug_fast_decode_page_info_parity / delta_debug_page_selection_parity (the
    reference's in-engine checks, backend.py:812-819, 1966-2012) run after every step, eager or
    replayed, and raise on a table that differs from the host rebuild."""
    eng = make_engine(B=4, graph=True, delta_debug_fast_decode_page_info_parity=True,
                      delta_debug_page_selection_parity=True)
    eng.prepare_synthetic_decode([15, 100, 250, 31], decode_budget=40, seed=8)
    eng.decode_steps(3, use_graph=False)
    eng.decode_steps(5, use_graph=True)
    assert eng._decode_graph_stats["replays"] == 5
    before = eng.cachelens.clone()
    eng.decode_steps(1, use_graph=False)
    eng._debug_check_decode_page_info(before)          # consistent tables pass
    with torch.inference_mode():
        eng.page_selector.paged_kv_indices[3] += 1
    with pytest.raises(RuntimeError, match="page-info mismatch in paged_kv_indices"):
        eng._debug_check_decode_page_info(before)
    # a partial batch near the gate's threshold: row 0 alone has 8 pages, 8 / min(8, 4) = 2 >
    # 1.8 (on); counting the 3 idle slots' pages would give 11 / 7 = 1.57 (off)
    eng2 = make_engine(B=4, ratio=1.8, k=4, delta_debug_fast_decode_page_info_parity=True,
                       delta_debug_page_selection_parity=True)
    eng2.prepare_synthetic_decode([119, 300, 300, 300], decode_budget=16, seed=9)
    with torch.inference_mode():
        eng2.active.copy_(torch.tensor([1, 0, 0, 0], dtype=torch.int32))
        eng2.cachelens.copy_(torch.tensor([119, 0, 0, 0], dtype=torch.int32))
    eng2.sync_host_lens()
    eng2.decode_steps(2, use_graph=False)
    assert int(eng2.use_subset_flag) == 1
    # in debug mode the decode-budget guard checks its host copy of cachelens against the device
    with torch.inference_mode():
        eng2.cachelens[0] += 1
    with pytest.raises(RuntimeError, match="host copy of cachelens"):
        eng2.decode_steps(1, use_graph=False)
    eng2.sync_host_lens()
    eng2.decode_steps(1, use_graph=False)


def test_replay_failure_falls_back_to_eager():
    """A failing graph replay is counted and the step runs eagerly (backend.py:1172-1181)."""
    eng = make_engine(B=3, graph=True)
    eng.prepare_synthetic_decode([50, 60, 70], decode_budget=16, seed=10)
    snap = _snapshot(eng)
    want = eng.decode_steps(2, use_graph=False).clone()
    _restore(eng, snap)
    eng.decode_steps(1, use_graph=True)                 # captures, then replays once

    class _Broken:
        def replay(self):
            raise RuntimeError("replay refused")

    eng._decode_graph = _Broken()
    got = eng.decode_steps(1, use_graph=True).clone()
    assert torch.equal(got, want)
    assert eng._decode_graph_stats["replay_failures"] == 1 and eng._decode_graph is None
    assert "replay refused" in eng._decode_graph_failed
    assert eng.cachelens.tolist() == [52, 62, 72]


def test_planner_on_chip_matches_dump_path_in_the_engine():
    """With >= 256 (row, kv head) blocks the engine's planner keeps its logits on chip
    (delta_paged_decode_scores_append).  From the same state, one decode step each way: the
    planner layer's output within the attention tolerance, page scores within 1e-5 relative,
    the subset selection identical (a page may differ only where the two keys at the k-th
    boundary are within that tolerance); ragged rows and idle slots.  And a graph replay of the
    on-chip step equals the eager step bit for bit."""
    B = 128  # tiny-test has 2 kv heads: 256 blocks
    eng = make_engine(graph=True, B=B, max_len=512, k=6, L=2)
    assert eng.plan_scores_on_chip
    lens = [20 + (37 * i) % 400 for i in range(B)]
    eng.prepare_synthetic_decode(lens, decode_budget=16, seed=21)
    eng._release_slot(5)
    eng._release_slot(77)
    plan = eng.model.layers[1].attention
    snap = _snapshot(eng)
    runs = {}
    for on_chip in (True, False):
        _restore(eng, snap)
        eng.plan_scores_on_chip = on_chip
        plan.record = []
        tok = eng.decode_steps(1, use_graph=False).clone()
        sip = eng.page_selector.paged_subset_kv_indptr[:B + 1].clone()
        runs[on_chip] = (tok, sip, eng.page_selector.paged_subset_kv_indices[:int(sip[-1])].clone(),
                         eng.page_scores.clone(), plan.record[0][1].clone())
    plan.record = None
    t1, p1, i1, s1, o1 = runs[True]
    t0, p0, i0, s0, o0 = runs[False]
    assert_close(o1, o0, "planner layer output, on chip vs dump")
    rel = ((s1 - s0).abs() / s0.abs().clamp_min(1e-30)).max().item()
    assert rel < 1e-5, rel
    assert torch.equal(p1, p0)
    if not torch.equal(i1, i0):  # only near-ties at the k-th key may swap
        for b in range(B):
            a, c = i1[int(p1[b]):int(p1[b + 1])].tolist(), i0[int(p0[b]):int(p0[b + 1])].tolist()
            if a != c:
                ks = s0[b, :eng.pages_per_slot]
                diff = set(a) ^ set(c)
                bt = eng.slot_block_table[b].tolist()
                vals = [float(ks[bt.index(p)]) for p in diff]
                assert max(vals) - min(vals) <= 1e-5 * max(abs(v) for v in vals), f"row {b}"
    # graph replay of the on-chip step from the same state
    _restore(eng, snap)
    eng.plan_scores_on_chip = True
    eng._decode_graph = None
    tok_g = eng.decode_steps(1, use_graph=True).clone()
    sip_g = eng.page_selector.paged_subset_kv_indptr[:B + 1].clone()
    assert torch.equal(tok_g, t1)
    assert torch.equal(sip_g, p1)
    assert torch.equal(eng.page_selector.paged_subset_kv_indices[:int(sip_g[-1])], i1)
    # the selection parity check needs the dump: the step is captured again on the dump path
    eng.enable_delta_debug_page_selection_parity = True
    eng.decode_steps(1, use_graph=True)
    assert eng._decode_graph_stats["captures"] == 2 and not eng._decode_graph_on_chip


def test_page_scores_from_attention_buffer_api():
    """LMBackend._compute_page_scores_from_attention_buffer (backend.py:911-913) returns the
    last planner step's del3_legacy_softmax scores: equal to the oracle's from the same dump
    within 1e-4 relative, and to the two-pass reference route."""
    eng = make_engine(B=3)
    eng.prepare_synthetic_decode([100, 257, 400], decode_budget=16, seed=11)
    eng.decode_steps(1, use_graph=False)
    torch.cuda.synchronize()
    B, mp = eng.batch_size, eng.pages_per_slot
    got = eng._compute_page_scores_from_attention_buffer().clone().cpu().double()
    ref_route = eng._compute_page_scores_reference().cpu().double()
    ip = eng.page_selector.paged_kv_indptr[:B + 1].cpu()
    last = eng.page_selector.paged_kv_last_page_len[:B].cpu()
    lens = O.kv_lengths(ip, last).tolist()
    logits = eng.dump.cpu().double().clone()
    for b in range(B):
        logits[b, :, lens[b]:] = float("-inf")
    want = O.legacy_softmax_page_scores(logits, B, mp, compute_dtype=torch.float64).double()
    assert got.shape == (B, mp)
    rel = ((got - want).abs() / want.abs().clamp_min(1e-30)).max().item()
    assert rel < 1e-4, rel
    assert ((ref_route - got).abs() / got.abs().clamp_min(1e-30)).max().item() < 1e-4
    # a row's pages past its end score 0
    pages = (ip[1:] - ip[:-1]).tolist()
    for b in range(B):
        assert got[b, pages[b]:].abs().max().item() == 0.0


def test_config3_llama3_8b_engine_step_matches_oracle():
    """The benchmark's own workload: Llama-3-8B shape (32 layers, 32 q / 8 kv heads), B = 32,
    8192-token context, 128-page budget, L = 8, layers 0-1 full (layer 1 the planner).  One
    recorded eager step is checked on sampled rows against the oracle, reading each layer's
    own cache after the step: layer 0's full attention; layer 1's full attention and its page
    selection (the oracle's own chain from the same rotated q and cache; a page may differ only
    within twice the row's measured score error of the k-th key); layers 2 and 31's subset
    attention over the step's subset CSR.  Then the same step replayed from a captured graph,
    from the same state, equals the eager step bit for bit: tokens, selection, appended K/V
    (backend.py:1449-1478, model.py:177-196)."""
    import math
    from delta_amd import ops
    from delta_amd.backend import LMBackend
    B, ctx, k, L = 32, 8192, 128, 8
    scale = 1 / math.sqrt(128)
    eng = LMBackend(dtype=torch.bfloat16, device=DEV, cuda_graph_decode=True)
    eng.load_model("random:llama-3-8b", seed=0)
    cfg = eng.model.config
    cfg.enable_selective_cache = True
    cfg.full_cache_layers = [0, 1]
    cfg.subset_cache_size = k
    cfg.compression_ratio = 1.0
    cfg.L = L
    eng.setup_caches(max_batch_size=B, max_seq_length=ctx + 64)
    eng.prepare_synthetic_decode(ctx, decode_budget=32, seed=0)
    assert eng.layer_roles[:3] == ["full", "plan", "subset"] and eng.layer_roles[-1] == "subset"
    watch = (0, 1, 2, 31)
    for i in watch:
        eng.model.layers[i].attention.record = []
    lens0, tok0 = eng.cachelens.clone(), eng.static_tokens.clone()
    eager_tok = eng.decode_steps(1, use_graph=False).clone()
    torch.cuda.synchronize()
    rec = {i: eng.model.layers[i].attention.record[0] for i in watch}
    for i in watch:
        eng.model.layers[i].attention.record = None
    sel = eng.page_selector
    full_ip = sel.paged_kv_indptr[:B + 1].cpu()
    full_ind = sel.paged_kv_indices[:int(full_ip[-1])].cpu()
    last = sel.paged_kv_last_page_len[:B].cpu()
    sub_ip = sel.paged_subset_kv_indptr[:B + 1].clone()
    sub_ind = sel.paged_subset_kv_indices[:int(sub_ip[-1])].clone()
    assert int(eng.use_subset_flag) == 1 and (sub_ip[1:] - sub_ip[:-1]).eq(k).all()
    gpu_scores = eng.page_scores.cpu().double()

    def row_kv(layer, pages):
        cache = eng.model.layers[layer].attention.kv_cache.kv_cache
        kv = cache[pages.to(DEV).long()].cpu()
        n = pages.numel()
        return kv, torch.tensor([0, n], dtype=torch.int32), torch.arange(n, dtype=torch.int32)

    for b in (0, 13, 31):
        pages = full_ind[int(full_ip[b]):int(full_ip[b + 1])]
        n = pages.numel()
        for layer in (0, 1):
            q, o = rec[layer]
            kv, ip1, ind1 = row_kv(layer, pages)
            o_ref, _ = O.paged_decode_attention(q[b:b + 1].cpu(), kv, ip1, ind1, last[b:b + 1], scale)
            assert_close(o[b:b + 1], o_ref, f"layer {layer} row {b} full attention")
        q1 = rec[1][0][b:b + 1].cpu()
        kv, ip1, ind1 = row_kv(1, pages)
        x = O.dump_logits(q1, kv, ip1, ind1, last[b:b + 1], scale, n * 16)
        s_ref = O.legacy_softmax_page_scores(x, 1, n, compute_dtype=torch.float64).double()
        cnt = torch.tensor([n], dtype=torch.int32)
        want_i, _ = O.select_pages(s_ref.float(), cnt, pages[None, :], k, L)
        got = set(sub_ind[int(sub_ip[b]):int(sub_ip[b + 1])].cpu().tolist())
        err = (gpu_scores[b, :n] - s_ref[0]).abs().max().item()
        keys = O.prepare_scores(s_ref.float(), cnt, L)[0]
        thr = sorted(keys.tolist(), reverse=True)[k - 1]
        for page in got ^ set(want_i.tolist()):
            j = pages.tolist().index(page)
            assert abs(float(keys[j]) - thr) <= 2 * err + 1e-6 * abs(thr), f"row {b}: page {j} far from the k-th key"
        sub_pages = sub_ind[int(sub_ip[b]):int(sub_ip[b + 1])].cpu()
        for layer in (2, 31):
            q, o = rec[layer]
            kv, ip1, ind1 = row_kv(layer, sub_pages)
            o_ref, _ = O.paged_decode_attention(q[b:b + 1].cpu(), kv, ip1, ind1, last[b:b + 1], scale)
            assert_close(o[b:b + 1], o_ref, f"layer {layer} row {b} subset attention")

    # the new token's cache slot of every row, in three layers, after the eager step
    pos = lens0.cpu()
    slot_pages = torch.tensor([int(full_ind[int(full_ip[b]) + int(pos[b]) // 16]) for b in range(B)])
    def slots():
        return [eng.model.layers[i].attention.kv_cache.kv_cache[slot_pages.to(DEV).long(), :,
                                                                 (pos % 16).to(DEV).long()].clone() for i in (0, 1, 31)]
    eager_slots = slots()
    with torch.inference_mode():
        eng.cachelens.copy_(lens0)
        eng.static_tokens.copy_(tok0)
    eng.sync_host_lens()
    replay_tok = eng.decode_steps(1, use_graph=True).clone()
    torch.cuda.synchronize()
    assert eng._decode_graph_failed is None and eng._decode_graph_stats["replays"] == 1
    assert torch.equal(replay_tok, eager_tok)
    assert torch.equal(sel.paged_subset_kv_indptr[:B + 1], sub_ip)
    assert torch.equal(sel.paged_subset_kv_indices[:int(sub_ip[-1])], sub_ind)
    for a, b_ in zip(slots(), eager_slots):
        assert torch.equal(a, b_)
    assert eng.cachelens.cpu().tolist() == (lens0.cpu() + 1).tolist()
    ops.set_active_backend(None)
    del eng
    torch.cuda.empty_cache()


# ------------------------------------------------------------------ several planner layers
# The reference's speed recipe makes several planners per step (run_reasoni_speed_compare.sh:
# full layers 0 1 2 14 22 -> planners 2, 14, 22; model.py:177-196): each one rewrites the subset
# CSR, which the subset layers after it read.  Full layers (0, 1, 3) of a 6-layer model give the
# roles full / plan / subset / plan / subset / subset.
MULTI_ROLES = ["full", "plan", "subset", "plan", "subset", "subset"]
SCALE = 1 / 128 ** 0.5


def _spy_planner_selections(eng):
    """Wrap ``attn_plan`` so each planner layer's selection (the subset CSR right after the
    layer) is copied as it is made; eager steps only."""
    taken = []
    orig = eng.attn_plan
    B = eng.batch_size

    def spy(q, kv_cache, append=None):
        o = orig(q, kv_cache, append=append)
        sel = eng.page_selector
        ip = sel.paged_subset_kv_indptr[:B + 1].cpu()
        taken.append((ip, sel.paged_subset_kv_indices[:int(ip[-1])].cpu()))
        return o

    eng.attn_plan = spy
    return taken


def _oracle_chain_selection(q, cache, ip, ind, last, k, L):
    """The oracle's own chain for one planner layer: fp64 logits rounded to fp32, fp64
    del3_legacy_softmax scores, v2 selection (backend.py:887-904, page_selector_v2.py:113-188)."""
    counts = ip[1:] - ip[:-1]
    mp = int(counts.max())
    bt = O.block_table_from_csr(ip, ind, mp)
    x = O.dump_logits(q, cache, ip, ind, last, SCALE, mp * 16)
    s = O.legacy_softmax_page_scores(x, q.shape[0], mp, compute_dtype=torch.float64)
    want_i, want_p = O.select_pages(s.float(), counts, bt, k, L)
    return want_i, want_p, s, bt


@pytest.mark.parametrize("B,on_chip", [(5, False), (128, True)])
def test_multi_planner_step_matches_oracle(B, on_chip):
    """One eager decode step with two planner layers: each planner's selection equals the
    oracle's chain from that layer's own rotated q and cache, bit for bit; each subset layer
    attends the selection of the planner before it (layer 2 planner 1's, layers 4 and 5 planner
    3's), within the attention tolerance; the two selections differ, so the second one is what
    layers 4 and 5 read.  Both planner routes: the logits dump (B = 5) and logits on chip (B =
    128: 256 (row, kv head) blocks, with two idle slots)."""
    eng = make_engine(B=B, max_len=512, k=6, L=2, full_layers=(0, 1, 3), n_layer=6)
    assert eng.layer_roles == MULTI_ROLES
    assert eng._plan_on_chip() == on_chip
    lens = [20 + (97 * i) % 420 for i in range(B)]
    eng.prepare_synthetic_decode(lens, decode_budget=16, seed=31)
    if B > 8:
        eng._release_slot(3)
        eng._release_slot(64)
    for layer in eng.model.layers:
        layer.attention.record = []
    taken = _spy_planner_selections(eng)
    eng.decode_steps(1, use_graph=False)
    torch.cuda.synchronize()
    assert len(taken) == 2 and int(eng.use_subset_flag) == 1
    ip, ind, last, _ = _csr(eng)
    rec = [l.attention.record[0] for l in eng.model.layers]
    caches = [l.attention.kv_cache.kv_cache.cpu() for l in eng.model.layers]
    for li in range(6):
        if MULTI_ROLES[li] in ("full", "plan"):
            ref, _ = O.paged_decode_attention(rec[li][0].cpu(), caches[li], ip, ind, last, SCALE)
            assert_close(rec[li][1], ref, f"layer {li} ({MULTI_ROLES[li]})")
    for t, li in enumerate((1, 3)):
        want_i, want_p, s, bt = _oracle_chain_selection(rec[li][0].cpu(), caches[li], ip, ind, last, eng.k_eff, eng.L)
        got_p, got_i = taken[t]
        assert got_p.tolist() == want_p.tolist(), f"planner layer {li}: indptr"
        if got_i.tolist() != want_i.tolist():
            keys = O.prepare_scores(s.float(), ip[1:] - ip[:-1], eng.L)
            msg = []
            for b in range(B):
                a = set(got_i[int(got_p[b]):int(got_p[b + 1])].tolist())
                r = set(want_i[int(want_p[b]):int(want_p[b + 1])].tolist())
                if a != r:
                    thr = sorted(keys[b].tolist(), reverse=True)[eng.k_eff - 1]
                    gaps = [abs(float(keys[b, bt[b].tolist().index(p)]) - thr) for p in a ^ r]
                    msg.append(f"row {b} gap {max(gaps):.3e} (k-th key {thr:.6e})")
            raise AssertionError(f"planner layer {li}: selection differs from the oracle chain: " + "; ".join(msg))
    assert not torch.equal(taken[0][1], taken[1][1]), "the two planners chose the same pages"
    for li, t in ((2, 0), (4, 1), (5, 1)):
        sp, si = taken[t]
        ref, _ = O.paged_decode_attention(rec[li][0].cpu(), caches[li], sp, si, last, SCALE)
        assert_close(rec[li][1], ref, f"layer {li} (subset after planner {(1, 3)[t]})")
    # what the step leaves in the subset CSR is the last planner's selection
    sel = eng.page_selector
    assert torch.equal(sel.paged_subset_kv_indptr[:B + 1].cpu(), taken[1][0])
    assert torch.equal(sel.paged_subset_kv_indices[:int(taken[1][0][-1])].cpu(), taken[1][1])


@pytest.mark.parametrize("B,ratio", [(4, 1.0), (4, 1e9), (128, 1.0)])
def test_multi_planner_graph_replays_match_eager(B, ratio):
    """Two planner layers inside one captured step: 12 graph replays, with eager work between
    them, equal 12 eager steps from the same state bit for bit -- tokens, the subset CSR the
    step leaves, and every layer's cache (the appended K/V).  With the gate off (ratio 1e9) the
    planners select nothing, the subset CSR is the full CSR and the subset layers attend every
    page, as the reference's unplanned step does (backend.py:560-580, 2104-2109).  B = 128 (256
    (row, kv head) blocks) runs both planners with their logits on chip."""
    eng = make_engine(graph=True, B=B, k=6, L=2, full_layers=(0, 1, 3), n_layer=6, ratio=ratio)
    assert eng.layer_roles == MULTI_ROLES
    assert eng._plan_on_chip() == (B == 128)
    lens = [15, 16, 31, 200] if B == 4 else [10 + (53 * i) % 300 for i in range(B)]
    eng.prepare_synthetic_decode(lens, decode_budget=40, seed=32)
    snap = _snapshot(eng)
    sel = eng.page_selector

    def subset_csr():
        ip = sel.paged_subset_kv_indptr[:B + 1].clone()
        return ip, sel.paged_subset_kv_indices[:int(ip[-1])].clone()

    eager = []
    for _ in range(12):
        tok = eng.decode_steps(1, use_graph=False).clone()
        eager.append((tok, *subset_csr()))
    eager_caches = [l.attention.kv_cache.kv_cache.clone() for l in eng.model.layers]
    assert int(eng.use_subset_flag) == (1 if ratio == 1.0 else 0)
    if ratio != 1.0:
        ip, ind, _, _ = _csr(eng)
        assert torch.equal(eager[-1][1].cpu(), ip) and torch.equal(eager[-1][2].cpu(), ind)
    _restore(eng, snap)
    for i in range(12):
        tok = eng.decode_steps(1, use_graph=True).clone()
        a = torch.randn(256, 256, device=DEV)
        (a @ a).sum().item()
        ip, ind = subset_csr()
        assert torch.equal(tok, eager[i][0]), f"replay {i}: tokens differ from the eager step"
        assert torch.equal(ip, eager[i][1]) and torch.equal(ind, eager[i][2]), f"replay {i}: subset CSR differs"
    assert eng._decode_graph_failed is None and eng._decode_graph_stats["replays"] == 12
    for li, (l, c) in enumerate(zip(eng.model.layers, eager_caches)):
        assert torch.equal(l.attention.kv_cache.kv_cache, c), f"layer {li} cache differs"
    if ratio != 1.0:  # gate off: every subset layer attends the full CSR
        for layer in eng.model.layers:
            layer.attention.record = []
        eng.decode_steps(1, use_graph=False)
        torch.cuda.synchronize()
        ip, ind, last, _ = _csr(eng)
        for li in (2, 4, 5):
            q, o = eng.model.layers[li].attention.record[0]
            ref, _ = O.paged_decode_attention(q.cpu(), eng.model.layers[li].attention.kv_cache.kv_cache.cpu(), ip,
                                              ind, last, SCALE)
            assert_close(o, ref, f"layer {li} with the gate off")


# ------------------------------------------------------------------ aux surface
def test_delta_impl_profile_sections():
    """delta_impl_profile (backend.py:1570-1585, call sites 537-578, 789-853): every eager decode
    step times its named device sections with HIP events; a replayed step is timed whole (its
    parts cannot be split) and the capture's warm-up bodies are not counted.  Two planners and
    three subset layers per step (full layers 0, 1, 3 of 6)."""
    eng = make_engine(B=5, k=6, L=2, full_layers=(0, 1, 3), n_layer=6, graph=True, delta_impl_profile=True)
    eng.prepare_synthetic_decode([40, 150, 260, 370, 480], decode_budget=16, seed=51)
    eng.decode_steps(2, use_graph=False)
    prof = eng.delta_impl_profile_summary()
    want = {"delta_decode_step_eager": 2, "delta_decode_page_info": 2, "delta_full_attention": 2,
            "delta_planner_attention_dump": 4, "delta_page_score": 4, "delta_page_select": 4,
            "delta_replan_total": 4, "delta_subset_attention": 6}
    assert {k: v["count"] for k, v in prof.items()} == want
    assert all(v["total_ms"] > 0 for v in prof.values())
    assert prof["delta_replan_total"]["total_ms"] >= prof["delta_page_select"]["total_ms"]
    parts = sum(prof[n]["total_ms"] for n in ("delta_decode_page_info", "delta_full_attention",
                                              "delta_planner_attention_dump", "delta_replan_total",
                                              "delta_subset_attention"))
    assert parts <= prof["delta_decode_step_eager"]["total_ms"]
    eng.decode_steps(3, use_graph=True)
    prof = eng.delta_impl_profile_summary()
    assert prof["delta_decode_step_graph"]["count"] == 3
    assert prof["delta_subset_attention"]["count"] == 6 and prof["delta_decode_step_eager"]["count"] == 2
    # the on-chip planner (B * Hkv >= 256) times attention and scores as one section
    eng2 = make_engine(B=128, k=6, L=2, delta_impl_profile=True)
    eng2.prepare_synthetic_decode([30 + i for i in range(128)], decode_budget=16, seed=52)
    eng2.decode_steps(1, use_graph=False)
    prof2 = eng2.delta_impl_profile_summary()
    assert prof2["delta_planner_attention_scores"]["count"] == 1 and "delta_page_score" not in prof2
    assert prof2["delta_page_select"]["count"] == 1


def test_final_stats_report_graph_fallbacks_and_profile(tmp_path, monkeypatch, capsys):
    """_print_final_stats prints and saves what the reference does (backend.py:2199-2238,
    2251-2275): captures, replays, capture time, fallback reasons and capture errors, and the
    delta_impl_profile table; here the capture fails, so every decode step falls back to eager
    and says so."""
    import json
    monkeypatch.setenv("DELTA_STEP_LOG_DIR", str(tmp_path))
    eng = make_engine(B=2, max_len=256, k=4, graph=True, delta_impl_profile=True)

    def refuse():
        raise RuntimeError("capture refused")

    eng._capture_decode_graph = refuse
    eng.add_requests([torch.tensor([1, 2, 3, 4]), torch.tensor([5, 6, 7])], [40, 30], [])
    eng.run_scheduler_loop()
    out = capsys.readouterr().out
    for text in ("HIP Graph Decode:", "capture failures: 1", "fallback reasons", "capture errors",
                 "DELTA Implementation Profile:", "delta_decode_step_eager", "delta_prefill_step"):
        assert text in out, text
    meta = json.loads(next(tmp_path.glob("step_timings_*.json")).read_text())["meta"]
    assert meta["cuda_graph_decode_fallback_reasons"]["capture_failed"] == 1
    assert meta["cuda_graph_decode_fallback_reasons"]["no_graph_eager_step"] > 0
    assert "capture refused" in meta["cuda_graph_decode_capture_errors"]["decode_step"]
    assert meta["delta_impl_profile"] is True
    assert meta["delta_impl_profile_counts"]["delta_prefill_step"] >= 1
    assert meta["delta_impl_profile_counts"]["delta_decode_step_eager"] > 0
    assert set(meta["delta_impl_profile_ms"]) == set(meta["delta_impl_profile_counts"])
    # a healthy graph engine reports its capture time
    eng2 = make_engine(B=2, max_len=256, k=4, graph=True)
    eng2.add_requests([torch.tensor([1, 2, 3, 4])], [30], [])
    eng2.run_scheduler_loop()
    out = capsys.readouterr().out
    assert "capture time by graph" in out and eng2._decode_graph_capture_time_s["decode_step"] > 0


# ------------------------------------------------------------------ per-row budgets
def test_per_row_budgets_through_the_engine():
    """set_subset_budgets (an extension: the reference's k is global, page_selector_v2.py:136-164):
    each row keeps min(pages, budget) pages.  One eager step with two planners is checked row by
    row against the oracle chain with each row's own k; the gate counts the per-row totals
    (O.decode_step_gate); then 10 graph replays equal 10 eager steps bit for bit, with the
    budgets changed between steps 4 and 5 (values only: the captured step reads them live)."""
    B = 6
    eng = make_engine(graph=True, B=B, k=8, L=2, full_layers=(0, 1, 3), n_layer=6, ratio=1.0)
    lens = [30, 120, 210, 300, 390, 470]
    eng.prepare_synthetic_decode(lens, decode_budget=24, seed=41)
    budgets = [1, 8, 3, 5, 8, 2]
    with pytest.raises(ValueError, match="per-row budgets must lie in"):
        eng.set_subset_budgets([0, 8, 3, 5, 8, 2])
    with pytest.raises(ValueError, match="per-row budgets must lie in"):
        eng.set_subset_budgets([9, 8, 3, 5, 8, 2])
    eng.set_subset_budgets(budgets)
    for layer in eng.model.layers:
        layer.attention.record = []
    taken = _spy_planner_selections(eng)
    cl0 = eng.cachelens.cpu().tolist()
    eng.decode_steps(1, use_graph=False)
    torch.cuda.synchronize()
    assert int(eng.use_subset_flag) == int(O.decode_step_gate(cl0, [1] * B, budgets, 1.0))
    ip, ind, last, _ = _csr(eng)
    counts = ip[1:] - ip[:-1]
    rec = [l.attention.record[0] for l in eng.model.layers]
    caches = [l.attention.kv_cache.kv_cache.cpu() for l in eng.model.layers]
    for t, li in enumerate((1, 3)):
        got_p, got_i = taken[t]
        assert (got_p[1:] - got_p[:-1]).tolist() == [min(int(c), kb) for c, kb in zip(counts, budgets)]
        q = rec[li][0].cpu()
        bt = O.block_table_from_csr(ip, ind, int(counts.max()))
        x = O.dump_logits(q, caches[li], ip, ind, last, SCALE, int(counts.max()) * 16)
        s = O.legacy_softmax_page_scores(x, B, int(counts.max()), compute_dtype=torch.float64).float()
        for b in range(B):
            wi, _ = O.select_pages(s[b:b + 1], counts[b:b + 1], bt[b:b + 1], budgets[b], eng.L)
            assert got_i[int(got_p[b]):int(got_p[b + 1])].tolist() == wi.tolist(), f"planner {li} row {b}"
    for li, t in ((2, 0), (4, 1), (5, 1)):
        sp, si = taken[t]
        ref, _ = O.paged_decode_attention(rec[li][0].cpu(), caches[li], sp, si, last, SCALE)
        assert_close(rec[li][1], ref, f"layer {li} over per-row budgets")
    eng.attn_plan = type(eng).attn_plan.__get__(eng)  # drop the spy
    for layer in eng.model.layers:
        layer.attention.record = None
    # graph replays == eager steps, budgets changed mid-way
    snap = _snapshot(eng)
    sel = eng.page_selector
    budgets2 = [8, 2, 2, 7, 1, 4]

    def run(use_graph):
        eng.set_subset_budgets(budgets)
        outs = []
        for i in range(10):
            if i == 5:
                eng.set_subset_budgets(budgets2)
            tok = eng.decode_steps(1, use_graph=use_graph).clone()
            p = sel.paged_subset_kv_indptr[:B + 1].clone()
            outs.append((tok, p, sel.paged_subset_kv_indices[:int(p[-1])].clone()))
        return outs, [l.attention.kv_cache.kv_cache.clone() for l in eng.model.layers]

    eager, eager_caches = run(False)
    _restore(eng, snap)
    replay, replay_caches = run(True)
    assert eng._decode_graph_stats["captures"] == 1 and eng._decode_graph_stats["replays"] == 10
    for i, (a, b) in enumerate(zip(eager, replay)):
        assert all(torch.equal(x, y) for x, y in zip(a, b)), f"step {i}: replay differs from eager"
    last_counts = (eager[-1][1][1:] - eager[-1][1][:-1]).tolist()
    assert all(c <= kb for c, kb in zip(last_counts, budgets2))
    for x, y in zip(eager_caches, replay_caches):
        assert torch.equal(x, y)
    eng.set_subset_budgets(None)
    assert not eng._per_row_budgets and eng._decode_graph is None


def test_budget_rule_through_the_engine():
    """set_subset_budget_rule (an extension): each row's budget, max(min_tokens, kv_len //
    divisor) tokens in pages, is recomputed on the device at every step.  With min 32 tokens,
    divisor 2 and k = 8, rows of 30, 94, 125, 160, 190 and 470 cached tokens start at 2, 2, 3, 5,
    5 and 8 pages; rows 1 and 4 cross to 3 and 6 pages at step 1 and row 2 to 4 at step 2.  The
    first eager step's selections are checked row by row against the oracle chain; then 10
    graph replays equal 10 eager steps bit for bit, the budgets after each step equal
    O.budget_rule_pages of the step's lengths, and the debug page-info check (which rebuilds
    the budgets on the host) passes on every step."""
    B, k = 6, 8
    eng = make_engine(graph=True, B=B, k=k, L=2, full_layers=(0, 1, 3), n_layer=6, ratio=1.0)
    lens = [30, 94, 125, 160, 190, 470]
    eng.prepare_synthetic_decode(lens, decode_budget=24, seed=43)
    for bad in ((32, 0), (-1, 2)):
        with pytest.raises(ValueError, match="budget rule needs"):
            eng.set_subset_budget_rule(*bad)
    eng.set_subset_budget_rule(32, 2)
    assert eng._per_row_budgets and eng._budget_rule == (32, 2)
    for layer in eng.model.layers:
        layer.attention.record = []
    taken = _spy_planner_selections(eng)
    cl0 = eng.cachelens.cpu()
    budgets = O.budget_rule_pages(cl0, 32, 2, k).tolist()
    assert budgets == [2, 2, 3, 5, 5, 8]
    eng.decode_steps(1, use_graph=False)
    torch.cuda.synchronize()
    assert eng.k_per_row.cpu().tolist() == budgets
    assert int(eng.use_subset_flag) == int(O.decode_step_gate(cl0.tolist(), [1] * B, budgets, 1.0))
    ip, ind, last, _ = _csr(eng)
    counts = ip[1:] - ip[:-1]
    rec = [l.attention.record[0] for l in eng.model.layers]
    caches = [l.attention.kv_cache.kv_cache.cpu() for l in eng.model.layers]
    for t, li in enumerate((1, 3)):
        got_p, got_i = taken[t]
        assert (got_p[1:] - got_p[:-1]).tolist() == [min(int(c), kb) for c, kb in zip(counts, budgets)]
        q = rec[li][0].cpu()
        bt = O.block_table_from_csr(ip, ind, int(counts.max()))
        x = O.dump_logits(q, caches[li], ip, ind, last, SCALE, int(counts.max()) * 16)
        s = O.legacy_softmax_page_scores(x, B, int(counts.max()), compute_dtype=torch.float64).float()
        for b in range(B):
            wi, _ = O.select_pages(s[b:b + 1], counts[b:b + 1], bt[b:b + 1], budgets[b], eng.L)
            assert got_i[int(got_p[b]):int(got_p[b + 1])].tolist() == wi.tolist(), f"planner {li} row {b}"
    eng.attn_plan = type(eng).attn_plan.__get__(eng)  # drop the spy
    for layer in eng.model.layers:
        layer.attention.record = None
    snap = _snapshot(eng)
    sel = eng.page_selector
    eng.enable_delta_debug_fast_decode_page_info_parity = True

    def run(use_graph):
        outs, seen = [], []
        for _ in range(10):
            before = eng.cachelens.cpu()
            tok = eng.decode_steps(1, use_graph=use_graph).clone()
            p = sel.paged_subset_kv_indptr[:B + 1].clone()
            outs.append((tok, p, sel.paged_subset_kv_indices[:int(p[-1])].clone()))
            got = eng.k_per_row.cpu().tolist()
            assert got == O.budget_rule_pages(before, 32, 2, k).tolist()
            seen.append(got)
        return outs, seen, [l.attention.kv_cache.kv_cache.clone() for l in eng.model.layers]

    eager, seen, eager_caches = run(False)
    assert seen[0] == [2, 3, 3, 5, 6, 8] and seen[1] == [2, 3, 4, 5, 6, 8]  # rows 1, 4, then 2 grew
    _restore(eng, snap)
    replay, seen_r, replay_caches = run(True)
    assert seen_r == seen
    assert eng._decode_graph_stats["captures"] == 1 and eng._decode_graph_stats["replays"] == 10
    for i, (a, b) in enumerate(zip(eager, replay)):
        assert all(torch.equal(x, y) for x, y in zip(a, b)), f"step {i}: replay differs from eager"
        counts_i = (a[1][1:] - a[1][:-1]).tolist()
        assert all(c <= kb for c, kb in zip(counts_i, seen[i]))
    for x, y in zip(eager_caches, replay_caches):
        assert torch.equal(x, y)
    eng.set_subset_budgets([1] * B)  # fixed budgets replace the rule (and the captured step)
    assert eng._budget_rule is None and eng._decode_graph is None
    eng.set_subset_budget_rule(32, 2)
    eng.set_subset_budget_rule(None)
    assert not eng._per_row_budgets and eng._budget_rule is None and eng._decode_graph is None


def test_speed_recipe_shape_three_planners_match_oracle():
    """The reference's speed recipe (run_reasoni_speed_compare.sh:16-28) at a 2048-token context:
    DeepSeek-R1-Distill-Qwen-1.5B shape (28 layers, 12 q / 2 kv heads, qkv bias), B = 64, subset
    64 pages, L = 8, full layers 0 1 2 14 22, so layers 2, 14 and 22 are planners (model.py:177-
    196).  One eager step, sampled rows: each planner's selection equals the oracle chain from its
    own layer's rotated q and cache, bit for bit; the first subset layer after each planner (3,
    15, 23) and the last layer attend that planner's selection.  Then the same step replayed from
    a captured graph, from the same state, equals the eager step: tokens, the subset CSR it
    leaves, the appended K/V of every layer's new token."""
    import math
    from delta_amd import ops
    from delta_amd.backend import LMBackend
    B, ctx, k, L = 64, 2048, 64, 8
    scale = 1 / math.sqrt(128)
    eng = LMBackend(dtype=torch.bfloat16, device=DEV, cuda_graph_decode=True)
    eng.load_model("random:DeepSeek-R1-Distill-Qwen-1.5B", seed=0)
    cfg = eng.model.config
    cfg.enable_selective_cache = True
    cfg.full_cache_layers = [0, 1, 2, 14, 22]
    cfg.subset_cache_size = k
    cfg.compression_ratio = 1.0
    cfg.L = L
    eng.setup_caches(max_batch_size=B, max_seq_length=ctx + 64)
    eng.prepare_synthetic_decode(ctx, decode_budget=32, seed=0)
    planners = [i for i, r in enumerate(eng.layer_roles) if r == "plan"]
    assert planners == [2, 14, 22]
    watch = (2, 3, 14, 15, 22, 23, 27)
    for i in watch:
        eng.model.layers[i].attention.record = []
    taken = _spy_planner_selections(eng)
    lens0, tok0 = eng.cachelens.clone(), eng.static_tokens.clone()
    eager_tok = eng.decode_steps(1, use_graph=False).clone()
    torch.cuda.synchronize()
    assert len(taken) == 3 and int(eng.use_subset_flag) == 1
    rec = {i: eng.model.layers[i].attention.record[0] for i in watch}
    for i in watch:
        eng.model.layers[i].attention.record = None
    eng.attn_plan = type(eng).attn_plan.__get__(eng)
    sel = eng.page_selector
    full_ip = sel.paged_kv_indptr[:B + 1].cpu()
    full_ind = sel.paged_kv_indices[:int(full_ip[-1])].cpu()
    last = sel.paged_kv_last_page_len[:B].cpu()

    def row_kv(layer, pages):
        cache = eng.model.layers[layer].attention.kv_cache.kv_cache
        kv = cache[pages.to(DEV).long()].cpu()
        n = pages.numel()
        return kv, torch.tensor([0, n], dtype=torch.int32), torch.arange(n, dtype=torch.int32)

    for t, layer in enumerate(planners):
        sp, si = taken[t]
        assert (sp[1:] - sp[:-1]).eq(k).all()
        for b in (0, 31, 63):
            pages = full_ind[int(full_ip[b]):int(full_ip[b + 1])]
            n = pages.numel()
            q = rec[layer][0][b:b + 1].cpu()
            kv, ip1, ind1 = row_kv(layer, pages)
            x = O.dump_logits(q, kv, ip1, ind1, last[b:b + 1], scale, n * 16)
            s_ref = O.legacy_softmax_page_scores(x, 1, n, compute_dtype=torch.float64).float()
            want_i, _ = O.select_pages(s_ref, torch.tensor([n], dtype=torch.int32), pages[None, :], k, L)
            got = si[int(sp[b]):int(sp[b + 1])]
            assert got.tolist() == want_i.tolist(), f"planner {layer} row {b}: selection differs from the oracle"
            o_ref, _ = O.paged_decode_attention(q, kv, ip1, ind1, last[b:b + 1], scale)
            assert_close(rec[layer][1][b:b + 1], o_ref, f"planner {layer} row {b} attention")
            for sub in {2: (3,), 14: (15,), 22: (23, 27)}[layer]:
                qs, os_ = rec[sub]
                kv, ip1, ind1 = row_kv(sub, got)
                o_ref, _ = O.paged_decode_attention(qs[b:b + 1].cpu(), kv, ip1, ind1, last[b:b + 1], scale)
                assert_close(os_[b:b + 1], o_ref, f"layer {sub} row {b} over planner {layer}'s selection")
    assert not torch.equal(taken[0][1], taken[1][1]) and not torch.equal(taken[1][1], taken[2][1])

    pos = lens0.cpu()
    slot_pages = torch.tensor([int(full_ind[int(full_ip[b]) + int(pos[b]) // 16]) for b in range(B)])

    def slots():
        return [eng.model.layers[i].attention.kv_cache.kv_cache[slot_pages.to(DEV).long(), :,
                                                                 (pos % 16).to(DEV).long()].clone()
                for i in range(len(eng.model.layers))]

    eager_slots = slots()
    sub_ip = sel.paged_subset_kv_indptr[:B + 1].clone()
    sub_ind = sel.paged_subset_kv_indices[:int(sub_ip[-1])].clone()
    with torch.inference_mode():
        eng.cachelens.copy_(lens0)
        eng.static_tokens.copy_(tok0)
    eng.sync_host_lens()
    replay_tok = eng.decode_steps(1, use_graph=True).clone()
    torch.cuda.synchronize()
    assert eng._decode_graph_failed is None and eng._decode_graph_stats["replays"] == 1
    assert torch.equal(replay_tok, eager_tok)
    assert torch.equal(sel.paged_subset_kv_indptr[:B + 1], sub_ip)
    assert torch.equal(sel.paged_subset_kv_indices[:int(sub_ip[-1])], sub_ind)
    for i, (a, b_) in enumerate(zip(slots(), eager_slots)):
        assert torch.equal(a, b_), f"layer {i}: appended K/V differs"
    ops.set_active_backend(None)
    del eng
    torch.cuda.empty_cache()


def test_kv_cache_pool_shares_caches_round_robin():
    """setup_caches(kv_cache_pool=n) (a benchmark aid for shapes whose KV exceeds HBM): layer i
    uses physical cache i % n, prepare_synthetic_decode fills each physical cache once, and a
    step over the shared caches replays from its graph bit for bit like the eager step."""
    from delta_amd.backend import LMBackend
    eng = LMBackend(dtype=torch.bfloat16, device=DEV, cuda_graph_decode=True)
    eng.load_model("random:tiny-test", seed=1, n_layer=6)
    cfg = eng.model.config
    cfg.enable_selective_cache = True
    cfg.full_cache_layers = [0, 1]
    cfg.subset_cache_size = 6
    cfg.L = 2
    eng.setup_caches(max_batch_size=3, max_seq_length=512, kv_cache_pool=2)
    ptrs = [l.attention.kv_cache.kv_cache.data_ptr() for l in eng.model.layers]
    assert len(set(ptrs)) == 2 and all(ptrs[i] == ptrs[i % 2] for i in range(6))
    eng.prepare_synthetic_decode([100, 257, 400], decode_budget=16, seed=3)
    snap = _snapshot(eng)
    eager = [eng.decode_steps(1, use_graph=False).clone() for _ in range(4)]
    _restore(eng, snap)
    replay = [eng.decode_steps(1, use_graph=True).clone() for _ in range(4)]
    assert all(torch.equal(a, b) for a, b in zip(eager, replay))
    with pytest.raises(ValueError, match="kv_cache_pool"):
        eng.setup_caches(max_batch_size=3, max_seq_length=512, kv_cache_pool=0)
