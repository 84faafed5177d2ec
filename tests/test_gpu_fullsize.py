"""GPU parity at the BASELINE configurations' full sizes.

Configs 2 (8 rows x 16 k tokens, fp16, planted pages) and 4 (4 rows x 64 k tokens, G = 7,
outlier channels) hold ~0.5 GB of KV, so the CPU oracle runs on them whole: logits dump,
page scores (planner and K-only routes), full attention, selection and sparse attention
are compared with it directly.  Config 5 (128 ragged rows of 1 k-32 k tokens, per-row
budgets, ~10 GB of KV) is checked through size-independent properties -- score sums,
counts, forced last pages, ascending order, determinism -- plus bit-exact selection for
every row and the oracle's scores and sparse attention for sampled rows.

Tolerances as in test_gpu_kernels: scores 1e-4 relative, dump 1e-4 * (1 + |x|), attention
2e-2 absolute with cosine > 0.999, selection bit-exact.
"""
import pytest
import torch

from delta_amd import kernels as K
from delta_amd.workloads import config_case
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def assert_attn_close(got, want, what):
    got = got.float().cpu()
    want = want.float().cpu()
    err = (got - want).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(got.flatten(), want.flatten(), dim=0).item()
    assert err <= 2e-2, f"{what}: max abs err {err}"
    assert cos > 0.999, f"{what}: cosine {cos}"


def assert_scores_close(got, ref, what):
    got, ref = got.double(), ref.double()
    rel = (got - ref).abs() / ref.abs().clamp_min(1e-30)
    rel[ref == 0] = got[ref == 0].abs()
    assert rel.max().item() < 1e-4, f"{what}: rel err {rel.max().item()}"


def rows_case(c, rows, indptr, indices):
    """CPU copy of the pages that ``rows`` hold under (indptr, indices), renumbered 0..n-1."""
    ip = indptr.cpu().to(torch.int64)
    idx = indices.cpu().to(torch.int64)
    pages = torch.cat([idx[ip[b]:ip[b + 1]] for b in rows])
    counts = torch.tensor([int(ip[b + 1] - ip[b]) for b in rows])
    sub_ip = torch.zeros(len(rows) + 1, dtype=torch.int32)
    sub_ip[1:] = torch.cumsum(counts, 0).to(torch.int32)
    kv = c.kv_cache[pages.to(DEV)].cpu()
    return (c.q[list(rows)].cpu(), kv, sub_ip, torch.arange(pages.numel(), dtype=torch.int32),
            c.kv_last_page_len[list(rows)].cpu())


@pytest.mark.parametrize("config", [2, 4])
def test_full_size_chain_matches_oracle(config):
    c = config_case(config, device=DEV)
    B, hq = c.q.shape[:2]
    mp, k, L = c.max_pages, c.k, c.L
    dump = torch.full((B, hq, mp * 16), 12345.0, device=DEV)
    lse = torch.empty(B, hq, device=DEV)
    o_full = K.paged_decode(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len,
                            max_pages_per_row=mp, lse=lse, logits_dump=dump)
    s = K.page_scores_from_logits(dump, c.kv_indptr, c.kv_last_page_len, mp, lse=lse)
    s_kv = K.page_score(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, mp)
    idx, ip = K.select_pages(s, c.kv_indptr, c.block_table, k, L)
    o_sp = K.paged_decode(c.q, c.kv_cache, ip, idx, c.kv_last_page_len, max_pages_per_row=k, subset=True)
    torch.cuda.synchronize()

    cc = c.to("cpu")
    x = O.dump_logits(cc.q, cc.kv_cache, cc.kv_indptr, cc.kv_indices, cc.kv_last_page_len, cc.sm_scale, mp * 16)
    d = dump.cpu()
    valid = torch.isfinite(x)
    assert ((d[valid] - x[valid]).abs() / (1 + x[valid].abs())).max().item() < 1e-4
    ref_s = O.legacy_softmax_page_scores(x, B, mp, compute_dtype=torch.float64)
    del x, d
    assert_scores_close(s.cpu(), ref_s, f"config {config} planner scores")
    assert_scores_close(s_kv.cpu(), ref_s, f"config {config} K-only scores")

    o_ref, lse_ref = O.paged_decode_attention(cc.q, cc.kv_cache, cc.kv_indptr, cc.kv_indices,
                                              cc.kv_last_page_len, cc.sm_scale)
    assert_attn_close(o_full, o_ref, f"config {config} full attention")
    assert torch.allclose(lse.cpu(), lse_ref, atol=1e-3, rtol=1e-4)

    counts = cc.kv_indptr[1:] - cc.kv_indptr[:-1]
    want_i, want_p = O.select_pages(s.cpu(), counts, cc.block_table, k, L)
    assert ip.cpu().tolist() == want_p.tolist()
    assert idx[:int(want_p[-1])].cpu().tolist() == want_i.tolist()
    o_sp_ref, _ = O.paged_decode_attention(cc.q, cc.kv_cache, want_p, want_i, cc.kv_last_page_len, cc.sm_scale)
    assert_attn_close(o_sp, o_sp_ref, f"config {config} sparse attention")

    if cc.planted is not None:  # config 2: the 8 planted pages of every row are selected
        got = want_i.tolist()
        for b in range(B):
            sel = set(got[int(want_p[b]):int(want_p[b + 1])])
            assert {int(cc.block_table[b, int(j)]) for j in cc.planted[b]} <= sel, f"row {b}: planted recall < 8/8"


def _ulp32(x: float) -> float:
    import numpy as np
    return float(np.spacing(np.float32(abs(x))))


# (config, planner route): the dump route (planner launch with the logits dump, then the
# two-pass score kernel) everywhere, and the on-chip route (attention and page scores in one
# pass, plain and with the decode token's RoPE + append fused in, the launch the engine's
# config-3 step makes) where the rows' logits fit on chip.
SELECTION_ROUTES = [(2, "dump"), (3, "dump"), (4, "dump"), (3, "on_chip"), (3, "on_chip_append")]


def _planner_scores(c, route):
    """Page scores of ``c``'s planner layer through ``route``; returns (scores, q the scores
    were computed from, the cache after the launch)."""
    B, hq = c.q.shape[:2]
    hkv = c.kv_cache.shape[3]
    mp = c.max_pages
    lse = torch.empty(B, hq, device=DEV)
    if route == "dump":
        dump = torch.empty((B, hq, mp * 16), device=DEV)
        K.paged_decode(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, max_pages_per_row=mp,
                       lse=lse, logits_dump=dump)
        s = K.page_scores_from_logits(dump, c.kv_indptr, c.kv_last_page_len, mp, lse=lse)
        return s, c.q
    append = route.endswith("append")
    assert K.paged_decode_scores_supported(B, hq, hkv, mp, append), f"{route} does not apply at this shape"
    ap, q_ref = None, c.q
    if append:
        # the decode token of every row at its last position: rotated k and v written into the
        # slot, q rotated in the launch (the same rotation as delta_rope, tested bit for bit)
        g = torch.Generator(device=DEV).manual_seed(77)
        kn = torch.randn((B, hkv, 128), generator=g, device=DEV).to(c.q.dtype)
        vn = torch.randn((B, hkv, 128), generator=g, device=DEV).to(c.q.dtype)
        offs = torch.tensor([n - 1 for n in c.kv_lens], dtype=torch.int32, device=DEV)
        ap = K.DecodeAppend(kn, vn, offs, c.kv_indptr, c.kv_indices, rope_scale=1.0, rope_theta=500000.0)
        q_ref = K.rope(c.q, kn, torch.arange(B + 1, dtype=torch.int32, device=DEV), offs, rope_scale=1.0,
                       rope_theta=500000.0)[0]
    _, s = K.paged_decode_scores(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len,
                                 max_pages_per_row=mp, lse=lse, append=ap)
    return s, q_ref


@pytest.mark.parametrize("config,route", SELECTION_ROUTES)
def test_full_size_selection_matches_oracle_chain(config, route):
    """End-to-end selection parity at the full BASELINE size, bit-exact: the GPU chain (planner
    scores through ``route`` -> radix select) against the oracle's own chain (fp64 logits rounded
    to fp32 -> fp64 del3_legacy_softmax scores -> v2 selection), backend.py:887-904 and
    page_selector_v2.py:113-188.  Every row's selected pages must be identical.  Should a row
    differ, the message says how far each differing page's key lies from the k-th key relative
    to the row's score error (two fp32 summation orders can only swap pages closer than that).
    Sparse attention is always checked: the kernel over the oracle's selection against the
    oracle's sparse attention."""
    import math
    c = config_case(config, device=DEV)
    B, hq = c.q.shape[:2]
    mp, k, L = c.max_pages, c.k, c.L
    s, q_ref = _planner_scores(c, route)
    idx, ip = K.select_pages(s, c.kv_indptr, c.block_table, k, L)
    torch.cuda.synchronize()
    cc = c.to("cpu")
    q_ref = q_ref.cpu()
    x = O.dump_logits(q_ref, cc.kv_cache, cc.kv_indptr, cc.kv_indices, cc.kv_last_page_len, cc.sm_scale, mp * 16)
    ref_s = O.legacy_softmax_page_scores(x, B, mp, compute_dtype=torch.float64).double()
    del x
    got_s = s.cpu().double()
    assert_scores_close(got_s, ref_s, f"config {config} {route} scores")
    counts = cc.kv_indptr[1:] - cc.kv_indptr[:-1]
    want_i, want_p = O.select_pages(ref_s.float(), counts, cc.block_table, k, L)
    keys = O.prepare_scores(ref_s.float(), counts, L)
    got_i, got_p = idx.cpu(), ip.cpu()
    assert got_p.tolist() == want_p.tolist()
    report = []
    pages_diff = 0
    for b in range(B):
        a = set(got_i[int(got_p[b]):int(got_p[b + 1])].tolist())
        r = set(want_i[int(want_p[b]):int(want_p[b + 1])].tolist())
        if a == r:
            continue
        pages_diff += len(a - r)
        err = (got_s[b] - ref_s[b]).abs().max().item()
        kb = sorted(keys[b].tolist(), reverse=True)
        thr = kb[min(k, int(counts[b])) - 1]
        bt = cc.block_table[b].tolist()
        gaps = [abs(float(keys[b, bt.index(p)]) - thr) for p in a ^ r]
        report.append(f"row {b}: {len(a - r)} pages, gaps to the k-th key {max(gaps):.3e} "
                      f"(score error {err:.3e}, {max(gaps) / max(err, 1e-30):.2f}x; fp32 ulp {_ulp32(thr):.1e}; "
                      f"k-th key finite: {math.isfinite(thr)})")
    assert pages_diff == 0, (f"config {config} {route}: {pages_diff} of {int(want_p[-1])} selected pages differ "
                             f"from the oracle's own chain: " + "; ".join(report))
    o_sp = K.paged_decode(q_ref.to(DEV), c.kv_cache, want_p.to(DEV), want_i.to(DEV), c.kv_last_page_len,
                          max_pages_per_row=k, subset=True)
    o_ref, _ = O.paged_decode_attention(q_ref, cc.kv_cache, want_p, want_i, cc.kv_last_page_len, cc.sm_scale)
    assert_attn_close(o_sp, o_ref, f"config {config} sparse attention over the oracle's selection")


def test_full_size_config5_ragged_properties():
    c = config_case(5, device=DEV)
    B, hq = c.q.shape[:2]
    mp, L = c.max_pages, c.L
    kpr = c.k_per_row.to(DEV)
    kmax = int(kpr.max())
    dump = torch.empty((B, hq, mp * 16), device=DEV)
    lse = torch.empty(B, hq, device=DEV)
    K.paged_decode(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len,
                   max_pages_per_row=mp, lse=lse, logits_dump=dump)
    s = K.page_scores_from_logits(dump, c.kv_indptr, c.kv_last_page_len, mp, lse=lse)
    idx, ip = K.select_pages(s, c.kv_indptr, c.block_table, kmax, L, k_per_row=kpr)
    o_sp = K.paged_decode(c.q, c.kv_cache, ip, idx, c.kv_last_page_len, max_pages_per_row=kmax, subset=True)
    o_sp2 = K.paged_decode(c.q, c.kv_cache, ip, idx, c.kv_last_page_len, max_pages_per_row=kmax, subset=True)
    s_kv = K.page_score(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, mp)
    torch.cuda.synchronize()
    assert torch.equal(o_sp, o_sp2)

    counts = (c.kv_indptr[1:] - c.kv_indptr[:-1]).cpu()
    sc = s.cpu()
    tot = sc.sum(1)
    assert bool((tot > 1 - 1e-3).all()) and bool((tot < hq + 1e-3).all())
    for b in range(B):  # nothing scored past a row's pages
        assert bool((sc[b, int(counts[b]):] == 0).all())
    assert_scores_close(s_kv.cpu(), sc, "config 5 K-only vs planner scores")

    # Selection: bit-exact against the oracle row by row (per-row budgets), and its invariants.
    kc = kpr.cpu()
    bt = c.block_table.cpu()
    got_p = ip.cpu()
    got_i = idx[:int(got_p[-1])].cpu()
    for b in range(B):
        wi, _ = O.select_pages(sc[b:b + 1], counts[b:b + 1], bt[b:b + 1], int(kc[b]), L)
        row = got_i[int(got_p[b]):int(got_p[b + 1])]
        assert row.tolist() == wi.tolist(), f"row {b}: selection differs from the oracle"
        n = int(counts[b])
        assert row.numel() == min(n, int(kc[b]))
        pos = {int(p): j for j, p in enumerate(bt[b, :n].tolist())}
        logical = [pos[int(p)] for p in row.tolist()]
        assert logical == sorted(logical) and len(set(logical)) == len(logical)
        assert set(range(max(0, n - L), n)) <= set(logical)

    # Oracle scores and sparse attention for sampled rows (shortest, longest, two others).
    lens = torch.tensor(c.kv_lens)
    sample = sorted({int(lens.argmin()), int(lens.argmax()), 0, B // 2})
    q, kv, sip, sidx, slast = rows_case(c, sample, c.kv_indptr, c.kv_indices)
    for r, b in enumerate(sample):
        n = int(counts[b])
        x = O.dump_logits(q[r:r + 1], kv, sip[r:r + 2] - sip[r], sidx[int(sip[r]):int(sip[r + 1])],
                          slast[r:r + 1], c.sm_scale, n * 16)
        ref = O.legacy_softmax_page_scores(x, 1, n, compute_dtype=torch.float64)
        assert_scores_close(sc[b:b + 1, :n], ref, f"config 5 row {b} scores")
    q, kv, sip, sidx, slast = rows_case(c, sample, ip, idx)
    o_ref, _ = O.paged_decode_attention(q, kv, sip, sidx, slast, c.sm_scale)
    assert_attn_close(o_sp[sample], o_ref, "config 5 sparse attention (sampled rows)")
