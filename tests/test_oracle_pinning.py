"""Pins the CPU oracle (oracle/delta_oracle.py) to brute force, closed forms and invariants.

The reference ships no golden vectors for this path (its tests are end-to-end
runners), so each oracle function is pinned here by an independent route:
pure-Python loops on tiny inputs, closed forms the math fixes, and invariants a
plausible mistake (wrong head map, missing bias, wrong tie order, off-by-one
in kv_len, transposed operand) would break.
"""
import math
import random

import numpy as np
import pytest
import torch

from oracle import delta_oracle as O

F32_MAX = float(np.finfo(np.float32).max)


def tiny_case(seed=0, B=3, hq=4, hkv=2, lens=(20, 33, 16), dtype=torch.float64, trailing=False):
    from delta_amd.workloads import make_case
    return make_case(batch=B, hq=hq, hkv=hkv, kv_lens=list(lens), dtype=dtype, seed=seed,
                     page_order="randperm", k=2, L=1, trailing_empty_page=trailing)


# ---------------------------------------------------------------- page tables

def test_kv_lengths_flashinfer_convention():
    indptr = torch.tensor([0, 3, 3, 5, 6], dtype=torch.int32)
    last = torch.tensor([16, 0, 1, 0], dtype=torch.int32)
    assert O.kv_lengths(indptr, last).tolist() == [48, 0, 17, 0]


def _request_plan_sim(n_tokens_per_step):
    """scheduler.py:60-74 restated as a loop: pages/last after each plan()."""
    pages, last = 1, 0  # initialize_pages
    out = []
    for q in n_tokens_per_step:
        last += q
        while last >= 16:
            pages += 1
            last -= 16
        out.append((pages, last))
    return out


def test_decode_page_info_matches_request_plan():
    steps = [4] + [1] * 60  # dummy4tok prompt, then decode steps
    sim = _request_plan_sim(steps)
    # before decode step i the row holds cachelens = 4 + (i - 1) tokens
    for i in range(1, len(steps)):
        cl = torch.tensor([4 + i - 1], dtype=torch.int32)
        pc, last, sc, ss = O.decode_page_info(cl, 100, k=3)
        assert (int(pc[0]), int(last[0])) == sim[i]
        assert int(sc[0]) == min(sim[i][0], 3) and int(ss[0]) == sim[i][0] - int(sc[0])


def test_use_subset_gate():
    assert O.use_subset_decision(100, 20, 1.0)
    assert not O.use_subset_decision(20, 20, 1.0)       # ratio 1 is not > 1
    assert not O.use_subset_decision(100, 20, 5.0)
    assert not O.use_subset_decision(100, 0, 1.0)
    assert not O.use_subset_decision(100, 20, 1.0, enable_selective_cache=False)


def test_decode_step_gate_counts_active_rows_only():
    """4 active rows of 4097 pages (kv_len 65537), k = 256, ratio 16, 28 idle slots: the
    totals are 4 * 4097 = 16388 and 4 * 256 = 1024, 16388 / 1024 = 16.0039 > 16, so the
    subset is on; counting each idle slot's one page would give 16416 / 1052 = 15.6 (off)."""
    B = 32
    cl = [65536] * 4 + [0] * (B - 4)
    act = [1] * 4 + [0] * (B - 4)
    assert O.decode_step_gate(cl, act, 256, 16.0)
    assert not O.decode_step_gate(cl, [1] * B, 256, 16.0)   # idle slots counted: 15.6
    assert not O.decode_step_gate(cl, act, 256, 16.004)      # just above 16.0039
    assert not O.decode_step_gate(cl, [0] * B, 256, 0.0)     # nothing active: subset_total 0
    assert not O.decode_step_gate(cl, act, 256, 1.0, enable_selective_cache=False)
    # the per-row count is Request.plan's: kv_len // 16 + 1 pages
    assert O.decode_step_gate([15], [1], 1, 1.5)             # 16 tokens -> 2 pages, 2 / 1 > 1.5
    assert not O.decode_step_gate([14], [1], 1, 1.5)         # 15 tokens -> 1 page


def test_per_row_budgets_in_page_info_and_gate():
    """Per-row budgets (this build's extension): each row's subset count is min(pages, k_b).
    Hand-counted: rows of 15, 40, 300 and 95 cached tokens hold 2, 3, 19 and 7 pages after the
    decode token (kv_len // 16 + 1); budgets 1, 8, 4, 0 give subset counts 1, 3, 4, 0 and
    starts 1, 0, 15, 7.  Gate: 31 pages over 8 subset pages = 3.875."""
    cl = torch.tensor([15, 40, 300, 95], dtype=torch.int32)
    pc, last, sc, ss = O.decode_page_info(cl, 100, k=torch.tensor([1, 8, 4, 0]))
    assert pc.tolist() == [2, 3, 19, 7] and last.tolist() == [0, 9, 13, 0]
    assert sc.tolist() == [1, 3, 4, 0] and ss.tolist() == [1, 0, 15, 7]
    assert O.decode_page_info(cl, 100, k=torch.tensor([-5, 8, 4, 0]))[2].tolist() == [0, 3, 4, 0]
    act = [1, 1, 1, 1]
    assert O.decode_step_gate(cl.tolist(), act, [1, 8, 4, 0], 3.87)
    assert not O.decode_step_gate(cl.tolist(), act, [1, 8, 4, 0], 3.875)
    # row 2 idle: 12 pages over 4 = 3.0
    assert O.decode_step_gate(cl.tolist(), [1, 1, 0, 1], [1, 8, 4, 0], 2.99)
    assert not O.decode_step_gate(cl.tolist(), [1, 1, 0, 1], [1, 8, 4, 0], 3.0)
    # a global budget equal for every row matches the per-row form
    assert O.decode_step_gate(cl.tolist(), act, [5] * 4, 2.0) == O.decode_step_gate(cl.tolist(), act, 5, 2.0)


def test_budget_rule_pages_hand_counted():
    """Config 5's max(512, len/8)-token budget, len = cachelens + 1 after the decode token.
    Hand-counted: 1024 and 4096 tokens sit on the 512-token floor (32 pages); 4223 tokens give
    527 tokens (32 pages) and 4224 give 528 (33 pages), the first step the share passes a page;
    32768 tokens give 4096 tokens (256 pages), 100 under a cap of 100; one token with no floor
    gives 0 tokens, raised to the 1-page minimum."""
    cl = torch.tensor([1023, 4095, 4222, 4223, 32767], dtype=torch.int32)
    assert O.budget_rule_pages(cl, 512, 8, 2048).tolist() == [32, 32, 32, 33, 256]
    assert O.budget_rule_pages(cl, 512, 8, 100).tolist() == [32, 32, 32, 33, 100]
    assert O.budget_rule_pages(torch.tensor([0, 15, 16]), 0, 8, 64).tolist() == [1, 1, 1]
    assert O.budget_rule_pages(torch.tensor([0, 255, 256]), 0, 1, 64).tolist() == [1, 16, 16]
    # fed to decode_page_info as per-row budgets: 4224 tokens hold 265 pages, 33 of them selected
    pc, _, sc, ss = O.decode_page_info(cl, 2049, k=O.budget_rule_pages(cl, 512, 8, 2048))
    assert pc.tolist() == [65, 257, 264, 265, 2049] and sc.tolist() == [32, 32, 32, 33, 256]
    assert ss.tolist() == [33, 225, 232, 232, 1793]


# ---------------------------------------------------------------- dump logits

def test_dump_logits_bruteforce():
    c = tiny_case(seed=3)
    d = 128
    scale = 1.0 / math.sqrt(d)
    S = 48
    x = O.dump_logits(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, scale, S)
    G = c.q.shape[1] // c.kv_cache.shape[3]
    for b in range(c.batch):
        pages = c.kv_indices[int(c.kv_indptr[b]):int(c.kv_indptr[b + 1])].tolist()
        n = c.kv_lens[b]
        for h in range(c.q.shape[1]):
            for t in range(S):
                if t >= n:
                    assert x[b, h, t] == float("-inf")
                    continue
                page, slot = pages[t // 16], t % 16
                krow = c.kv_cache[page, 0, slot, h // G].tolist()
                want = math.fsum(a * bb for a, bb in zip(c.q[b, h].tolist(), krow)) * scale
                assert abs(float(x[b, h, t]) - want) <= 1e-6 * max(1.0, abs(want))


def test_dump_uses_gqa_head_map():
    # A map h % Hkv instead of h // G would pair head 1 with kv head 1: make them differ.
    c = tiny_case(seed=4, B=1, hq=4, hkv=2, lens=(16,))
    x = O.dump_logits(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, 1.0, 16)
    page = int(c.kv_indices[0])
    k0 = c.kv_cache[page, 0, 0, 0]
    assert torch.allclose(x[0, 1, 0].double(), (c.q[0, 1] @ k0).double(), rtol=1e-6)


# ---------------------------------------------------------------- page scores

def _scores_bruteforce(x, B, max_pages):
    hq = x.shape[1]
    out = [[0.0] * max_pages for _ in range(B)]
    for b in range(B):
        probs = []
        for h in range(hq):
            row = x[b, h, :max_pages * 16].tolist()
            m = max(row)
            e = [0.0 if v == float("-inf") else math.exp(v - m) for v in row]
            s = math.fsum(e)
            probs.append([v / s for v in e])
        for j in range(max_pages):
            out[b][j] = math.fsum(max(probs[h][t] for h in range(hq)) for t in range(16 * j, 16 * j + 16))
    return torch.tensor(out, dtype=torch.float64)


def test_page_scores_bruteforce():
    torch.manual_seed(0)
    B, hq, S = 2, 5, 80
    x = torch.randn(B, hq, S, dtype=torch.float32) * 3
    x[0, :, 70:] = float("-inf")
    x[1, :, 41:] = float("-inf")
    want = _scores_bruteforce(x.double(), B, 5)
    got64 = O.legacy_softmax_page_scores(x, B, 5, compute_dtype=torch.float64)
    got32 = O.legacy_softmax_page_scores(x, B, 5)
    assert torch.allclose(got64.double(), want, rtol=1e-6, atol=0)
    assert torch.allclose(got32.double(), want, rtol=1e-5, atol=1e-9)


def test_page_scores_closed_forms():
    c = tiny_case(seed=5, B=2, hq=4, hkv=2, lens=(37, 64))
    mp = 4
    x = O.dump_logits(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, 0.1, mp * 16)
    s = O.legacy_softmax_page_scores(x, 2, mp, compute_dtype=torch.float64).double()
    # every head's softmax sums to 1: the head-max sum lies in [1, Hq]
    assert (s.sum(1) >= 1 - 1e-6).all() and (s.sum(1) <= 4 + 1e-6).all()
    # row 0 holds 37 tokens = 3 pages: page 3 scores exactly 0
    assert s[0, 3] == 0.0
    # one head: sum of scores == 1
    s1 = O.legacy_softmax_page_scores(x[:, :1], 2, mp, compute_dtype=torch.float64).double()
    assert torch.allclose(s1.sum(1), torch.ones(2, dtype=torch.float64), atol=1e-12)
    # identical heads: head-max == that head
    xr = x[:, :1].repeat(1, 3, 1)
    s3 = O.legacy_softmax_page_scores(xr, 2, mp, compute_dtype=torch.float64).double()
    assert torch.allclose(s3, s1, atol=1e-15)


def test_scores_invariant_to_page_permutation_and_v():
    c = tiny_case(seed=6, B=2, lens=(40, 60))
    mp = 4
    x = O.dump_logits(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, 0.2, mp * 16)
    # move every page to a new physical slot; same logical content
    n = c.kv_cache.shape[0]
    perm = torch.randperm(n, generator=torch.Generator().manual_seed(1))
    cache2 = torch.empty_like(c.kv_cache)
    cache2[perm] = c.kv_cache
    idx2 = perm[c.kv_indices.long()].to(torch.int32)
    cache2[:, 1] = torch.randn_like(cache2[:, 1])  # V must not matter
    x2 = O.dump_logits(c.q, cache2, c.kv_indptr, idx2, c.kv_last_page_len, 0.2, mp * 16)
    assert torch.equal(x, x2)


# ---------------------------------------------------------------- selector

def _select_bruteforce(scores, counts, bt, k, L, bias):
    B, n = scores.shape
    idx, indptr = [], [0]
    for b in range(B):
        tp = int(counts[b])
        keyed = []
        for j in range(n):
            s = float(scores[b, j])
            if s != s:
                s = float("-inf")
            elif s == float("inf"):
                s = F32_MAX
            if bias:
                bj = float(np.float32(float(j) * float(np.float32(bias))))  # exact product, one rounding
                s = float(np.float32(-bj + s)) if s not in (float("-inf"), F32_MAX) else s
            if max(tp - L, 0) <= j < tp:
                s = float("inf")
            if j >= tp:
                s = float("-inf")
            keyed.append((-s, j))
        chosen = sorted(sorted(keyed)[:k], key=lambda p: p[1])
        keep = [j for _, j in chosen][:min(tp, k)]
        idx.extend(int(bt[b, j]) for j in keep)
        indptr.append(indptr[-1] + len(keep))
    return idx, indptr


@pytest.mark.parametrize("seed", range(6))
def test_selector_bruteforce(seed):
    rng = np.random.default_rng(seed)
    B, n, k, L = 4, 24, 6, 2
    scores = torch.tensor(rng.random((B, n)), dtype=torch.float32)
    # quantised values so exact ties (and bias-broken ties) happen often
    scores = torch.round(scores * 8) / 8
    scores[0, 3] = float("nan")
    scores[1, 5] = float("inf")
    scores[2, 7] = float("-inf")
    counts = torch.tensor([24, 10, 5, 17])
    bt = torch.tensor(rng.permutation(B * n).reshape(B, n), dtype=torch.int32)
    for bias in (1e-7, 0.0):
        got_i, got_p = O.select_pages(scores, counts, bt, k, L, bias)
        want_i, want_p = _select_bruteforce(scores, counts, bt, k, L, bias)
        assert got_i.tolist() == want_i and got_p.tolist() == want_p


def test_selector_bias_rounding_is_fp32():
    b = O.position_bias(1000, 1e-7)
    for j in (1, 3, 7, 999):
        assert b[j] == np.float32(-(np.float64(j) * np.float64(np.float32(1e-7))))
    # bias breaks exact ties toward the lower page index
    scores = torch.ones(1, 10)
    counts = torch.tensor([10])
    bt = torch.arange(10, dtype=torch.int32)[None]
    idx, _ = O.select_pages(scores, counts, bt, 4, 1, 1e-7)
    assert idx.tolist() == [0, 1, 2, 9]


def test_selector_invariants():
    rng = np.random.default_rng(7)
    B, n, k, L = 5, 40, 12, 4
    scores = torch.tensor(rng.random((B, n)), dtype=torch.float32)
    counts = torch.tensor([40, 13, 12, 3, 31])
    bt = torch.tensor(rng.permutation(B * n).reshape(B, n), dtype=torch.int32)
    idx, indptr = O.select_pages(scores, counts, bt, k, L)
    for b in range(B):
        tp = int(counts[b])
        row = idx[indptr[b]:indptr[b + 1]].tolist()
        assert len(row) == min(tp, k)
        pos = [list(bt[b]).index(v) for v in row]
        assert pos == sorted(pos) and all(p < tp for p in pos)
        assert set(range(max(tp - L, 0), tp)) <= set(pos)
    # fixed path == general path when every row has >= k pages
    full = torch.full((B,), n)
    fi, fp = O.select_pages(scores, full, bt, k, L, fixed_count=True)
    gi, gp = O.select_pages(scores, full, bt, k, L)
    assert torch.equal(fi, gi) and torch.equal(fp, gp)
    assert fp.tolist() == [k * b for b in range(B + 1)]


def test_selector_monotone():
    rng = np.random.default_rng(8)
    scores = torch.tensor(rng.random((1, 30)), dtype=torch.float32)
    counts = torch.tensor([30])
    bt = torch.arange(30, dtype=torch.int32)[None]
    idx, _ = O.select_pages(scores, counts, bt, 8, 2)
    sel = set(idx.tolist())
    s2 = scores.clone()
    j_in = min(sel)
    s2[0, j_in] += 10.0            # raising a selected page keeps it
    j_out = next(j for j in range(30) if j not in sel)
    s2[0, j_out] -= 10.0           # lowering an unselected page keeps it out
    idx2, _ = O.select_pages(s2, counts, bt, 8, 2)
    assert set(idx2.tolist()) == sel


def test_selector_k_out_of_range_raises():
    with pytest.raises(RuntimeError):
        O.select_pages(torch.zeros(1, 4), torch.tensor([4]), torch.zeros(1, 4, dtype=torch.int32), 5, 1)


# ---------------------------------------------------------------- attention

def test_attention_matches_sdpa():
    c = tiny_case(seed=9, B=3, hq=8, hkv=2, lens=(19, 48, 5))
    o, lse = O.paged_decode_attention(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, 0.09)
    G = 4
    for b in range(3):
        k, v = O.gather_row_kv(c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, b)
        kk = k.double().repeat_interleave(G, 1).transpose(0, 1)  # [Hq, n, d]
        vv = v.double().repeat_interleave(G, 1).transpose(0, 1)
        ref = torch.nn.functional.scaled_dot_product_attention(
            c.q[b].double()[:, None, :], kk, vv, scale=0.09)[:, 0]
        assert torch.allclose(o[b].double(), ref, atol=1e-6)
        s = (c.q[b].double()[:, None, :] * kk).sum(-1) * 0.09
        assert torch.allclose(lse[b].double(), torch.logsumexp(s, -1), atol=1e-5)


def virtual_decode_rows(qo_lens, kv_indptr, kv_indices, kv_last_page_len, page_size=16):
    """One decode row per prefill query token, over its causal prefix (an independent
    construction: page lists cut from the row's CSR, last_page_len from the position)."""
    ip, ind, last = [0], [], []
    for b, qo in enumerate(qo_lens):
        n = int(O.kv_lengths(kv_indptr[b:b + 2], kv_last_page_len[b:b + 1], page_size)[0])
        pages = kv_indices[int(kv_indptr[b]):int(kv_indptr[b + 1])].tolist()
        for i in range(qo):
            pos = n - qo + i
            npg = pos // page_size + 1
            ind.extend(pages[:npg])
            ip.append(len(ind))
            last.append(pos % page_size + 1)
    return (torch.tensor(ip, dtype=torch.int32), torch.tensor(ind, dtype=torch.int32),
            torch.tensor(last, dtype=torch.int32))


def test_prefill_equals_causal_virtual_rows():
    """Causal prefill == one decode row per query token over its prefix, and == decode when
    every row has one query token."""
    c = tiny_case(seed=12, B=3, hq=8, hkv=2, lens=(40, 17, 64))
    qo = [5, 1, 16]
    gen = torch.Generator().manual_seed(3)
    q = torch.randn(sum(qo), 8, 128, generator=gen, dtype=torch.float64)
    qo_indptr = torch.tensor([0, 5, 6, 22], dtype=torch.int32)
    o, lse = O.paged_prefill_attention(q, qo_indptr, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, 0.088)
    vip, vind, vlast = virtual_decode_rows(qo, c.kv_indptr, c.kv_indices, c.kv_last_page_len)
    o2, lse2 = O.paged_decode_attention(q, c.kv_cache, vip, vind, vlast, 0.088)
    assert torch.allclose(o, o2, atol=1e-6) and torch.allclose(lse, lse2, atol=1e-6)
    # first query of row 0 (position 35) must not see token 36+: changing them leaves it unchanged
    cache = c.kv_cache.clone()
    pages0 = c.kv_indices[int(c.kv_indptr[0]):int(c.kv_indptr[1])].long()
    cache[pages0[2], :, 4:] += 100.0  # tokens 36..47 of row 0
    o3, _ = O.paged_prefill_attention(q, qo_indptr, cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, 0.088)
    assert torch.equal(o3[0], o[0]) and not torch.allclose(o3[4], o[4])
    # one query per row: exactly the decode attention
    q1 = q[[4, 5, 21]]
    o4, lse4 = O.paged_prefill_attention(q1, torch.arange(4, dtype=torch.int32), c.kv_cache, c.kv_indptr,
                                         c.kv_indices, c.kv_last_page_len, 0.088)
    o5, lse5 = O.paged_decode_attention(q1, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, 0.088)
    assert torch.allclose(o4, o5, atol=1e-7) and torch.allclose(lse4, lse5, atol=1e-7)


def test_sparse_equals_full_when_all_pages_selected():
    c = tiny_case(seed=10, B=2, lens=(40, 70))
    res = O.selective_step(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, k=5, L=2)
    assert torch.equal(res["indices"], c.kv_indices) and torch.equal(res["indptr"], c.kv_indptr)
    assert torch.allclose(res["o_full"], res["o_sparse"], atol=0)


def test_attention_empty_row_and_permutation():
    c = tiny_case(seed=11, B=2, lens=(33, 20))
    last = c.kv_last_page_len.clone()
    indptr = c.kv_indptr.clone()
    indptr[2] = indptr[1]  # row 1 has no pages
    last[1] = 0
    o, lse = O.paged_decode_attention(c.q, c.kv_cache, indptr, c.kv_indices, last, 0.1)
    assert torch.all(o[1] == 0) and torch.all(torch.isinf(lse[1]))
    n = c.kv_cache.shape[0]
    perm = torch.randperm(n, generator=torch.Generator().manual_seed(2))
    cache2 = torch.empty_like(c.kv_cache)
    cache2[perm] = c.kv_cache
    o2, _ = O.paged_decode_attention(c.q, cache2, c.kv_indptr, perm[c.kv_indices.long()].int(),
                                     c.kv_last_page_len, 0.1)
    o1, _ = O.paged_decode_attention(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, 0.1)
    assert torch.allclose(o1, o2, atol=1e-7)


def test_trailing_empty_page_contributes_nothing():
    c = tiny_case(seed=12, B=1, lens=(32,), trailing=True)
    assert c.kv_last_page_len.tolist() == [0] and int(c.kv_indptr[1]) == 3
    x = O.dump_logits(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, 0.1, 48)
    s = O.legacy_softmax_page_scores(x, 1, 3)
    assert s[0, 2] == 0
    idx, _ = O.select_pages(s, torch.tensor([3]), c.block_table, 2, 1)
    assert int(idx[-1]) == int(c.kv_indices[2])  # the empty last page is forced in


# ---------------------------------------------------------------- metadata, append, rope

def test_pack_page_indices_bruteforce():
    rng = random.Random(0)
    pps = 9
    slot_bt = torch.tensor([[rng.randrange(1000) for _ in range(pps)] for _ in range(5)], dtype=torch.int32)
    active = torch.tensor([3, 0, 4], dtype=torch.int32)
    starts = torch.tensor([2, 0, 5], dtype=torch.int32)
    counts = torch.tensor([4, 9, 0], dtype=torch.int32)
    indptr = torch.tensor([0, 4, 13, 13], dtype=torch.int32)
    out = torch.full((13,), -1, dtype=torch.int32)
    row_bt = torch.full((3, pps), -1, dtype=torch.int32)
    O.pack_page_indices(slot_bt, active, starts, counts, indptr, out, row_bt, 3, True)
    want = slot_bt[3, 2:6].tolist() + slot_bt[0, :9].tolist()
    assert out.tolist() == want
    assert row_bt[0, :4].tolist() == slot_bt[3, 2:6].tolist() and row_bt[0, 4:].tolist() == [-1] * 5
    assert row_bt[2].tolist() == [-1] * pps


def test_append_then_gather_round_trip():
    c = tiny_case(seed=13, B=2, lens=(17, 40))
    cache = c.kv_cache.clone()
    k = torch.randn(3, 2, 128, dtype=torch.float64)
    v = torch.randn(3, 2, 128, dtype=torch.float64)
    app = torch.tensor([0, 1, 3], dtype=torch.int32)  # 1 token for row 0, 2 for row 1
    O.append_kv(k, v, app, cache, c.kv_indices, c.kv_indptr, c.kv_last_page_len)
    k0, v0 = O.gather_row_kv(cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, 0)
    k1, v1 = O.gather_row_kv(cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, 1)
    assert torch.equal(k0[-1], k[0]) and torch.equal(v0[-1], v[0])
    assert torch.equal(k1[-2:], k[1:]) and torch.equal(v1[-2:], v[1:])
    # nothing else moved
    ka, _ = O.gather_row_kv(c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, 1)
    assert torch.equal(k1[:-2], ka[:-2])


def test_rope_closed_forms():
    torch.manual_seed(1)
    x = torch.randn(4, 3, 128, dtype=torch.float64)
    f = O.rope_frequencies(128, 1.0, 1e4)
    assert f[0] == 1.0 and abs(float(f[1]) - 1e4 ** (-2 / 128)) < 1e-15
    indptr = torch.tensor([0, 4], dtype=torch.int32)
    # position 0 is the identity
    y0 = O.apply_rope(x[:1], torch.tensor([0, 1], dtype=torch.int32), torch.tensor([0], dtype=torch.int32), f)
    assert torch.allclose(y0.double(), x[:1], atol=1e-6)
    # rotation preserves every pair's norm
    y = O.apply_rope(x, indptr, torch.tensor([100], dtype=torch.int32), f).double()
    n0 = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    n1 = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
    assert torch.allclose(n0, n1, rtol=1e-5)
    # token i of the row sits at offset + i: pair 0 of token 1 turned by (offset+1) * f0
    a = 101.0
    want0 = x[1, 0, 0] * math.cos(a) - x[1, 0, 1] * math.sin(a)
    assert abs(float(y[1, 0, 0]) - float(want0)) < 1e-5
    # rope_scale divides the frequencies; llama3.1 keeps high frequencies unscaled
    f2 = O.rope_frequencies(128, 8.0, 5e5, 1.0, 4.0, 8192)
    assert abs(float(f2[0]) - 1.0) < 1e-12
    assert abs(float(f2[-1]) - float(O.rope_frequencies(128, 8.0, 5e5)[-1])) < 1e-18


def _llama31_by_wavelength(head_dim, scale, theta, lo, hi, old_ctx):
    """Meta's published Llama-3.1 frequency rule, written from wavelengths in pure Python
    (no shared code with the oracle): keep f when its wavelength 2*pi/f is shorter than
    old_ctx/hi, divide by ``scale`` when it is longer than old_ctx/lo, else blend
    (1 - s) f/scale + s f with s = (old_ctx/wavelength - lo) / (hi - lo)."""
    out = []
    for j in range(head_dim // 2):
        f = theta ** (-(2.0 * j) / head_dim)
        wavelen = 2.0 * math.pi / f
        if wavelen < old_ctx / hi:
            out.append(f)
        elif wavelen > old_ctx / lo:
            out.append(f / scale)
        else:
            s = (old_ctx / wavelen - lo) / (hi - lo)
            out.append((1.0 - s) * f / scale + s * f)
    return out


def _blend_weights(head_dim, theta, lo, hi, old_ctx):
    return [(old_ctx * theta ** (-(2.0 * j) / head_dim) / (2.0 * math.pi) - lo) / (hi - lo)
            for j in range(head_dim // 2)]


@pytest.mark.parametrize("scale,theta,lo,hi,old_ctx", [
    (8.0, 5e5, 1.0, 4.0, 8192),    # Llama-3.1-8B (model.py:87)
    (32.0, 5e5, 1.0, 4.0, 8192),   # the 3.2 family's scale
    (4.0, 1e4, 2.0, 8.0, 4096),    # band moved: other factors and base
])
def test_rope_llama31_blend_band_matches_published_rule(scale, theta, lo, hi, old_ctx):
    got = O.rope_frequencies(128, scale, theta, lo, hi, old_ctx).tolist()
    want = _llama31_by_wavelength(128, scale, theta, lo, hi, old_ctx)
    inside = [j for j, s in enumerate(_blend_weights(128, theta, lo, hi, old_ctx)) if 0.0 < s < 1.0]
    assert len(inside) >= 3, "the case must put pairs inside the blend band"
    for j in range(64):
        assert abs(got[j] - want[j]) <= 1e-12 * want[j], (j, got[j], want[j])
    # both sides of the band take the plain rules
    assert any(got[j] == 1.0 * theta ** (-(2.0 * j) / 128) for j in range(64))
    assert any(abs(got[j] - theta ** (-(2.0 * j) / 128) / scale) < 1e-18 for j in range(64))


@pytest.mark.parametrize("j", [9, 17, 25])
def test_rope_llama31_band_edges(j):
    """old_ctx chosen so pair j sits exactly on an edge: wavelength = old_ctx / hi gives f, =
    old_ctx / lo gives f / scale (the blend is continuous there)."""
    theta, scale, lo, hi = 5e5, 8.0, 1.0, 4.0
    f = theta ** (-(2.0 * j) / 128)
    wavelen = 2.0 * math.pi / f
    hi_edge = O.rope_frequencies(128, scale, theta, lo, hi, hi * wavelen)
    lo_edge = O.rope_frequencies(128, scale, theta, lo, hi, lo * wavelen)
    assert abs(float(hi_edge[j]) - f) <= 1e-12 * f
    assert abs(float(lo_edge[j]) - f / scale) <= 1e-12 * f
    # one pair further in either direction is past the edge
    assert abs(float(hi_edge[j - 1]) - theta ** (-(2.0 * (j - 1)) / 128)) <= 1e-12
    assert abs(float(lo_edge[j + 1]) * scale - theta ** (-(2.0 * (j + 1)) / 128)) <= 1e-12 * f


def test_rope_llama31_check_detects_a_wrong_coefficient():
    """The blend check above is sensitive: a plausible slip in the smoothing coefficient
    (hi + lo for hi - lo, or the offset's ratio inverted) moves the band's frequencies by far
    more than its tolerance."""
    d, scale, theta, lo, hi, old = 128, 8.0, 5e5, 1.0, 4.0, 8192
    want = _llama31_by_wavelength(d, scale, theta, lo, hi, old)

    def slipped(variant):
        j = torch.arange(d // 2, dtype=torch.float64)
        f = theta ** (-(2.0 * j) / d)
        a = old / (2.0 * math.pi * (hi + lo)) if variant == "sum" else old / (2.0 * math.pi * (hi - lo))
        c = -1.0 / (hi / lo - 1.0) if variant == "sum" else -1.0 / (lo / hi - 1.0)
        s = torch.clamp(f * a + c, 0.0, 1.0)
        return ((1.0 - s) * (f / scale) + s * f).tolist()

    for variant in ("sum", "ratio"):
        bad = slipped(variant)
        assert max(abs(x - y) / y for x, y in zip(bad, want)) > 1e-3, variant
