"""The planner's Python boundary: PageSelectorV2.plan / .select (page_selector_v2.py:74-212)
driven as the reference drives them, checked against the CPU oracle."""
import pytest
import torch

from delta_amd.page_selector_v2 import PageSelectorV2
from delta_amd.workloads import make_case
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _scores(B, n, seed):
    g = torch.Generator().manual_seed(seed)
    s = torch.rand((B, n), generator=g, dtype=torch.float32)
    s[0, 3] = float("nan")
    s[1, 2] = s[1, 5] = s[1, 9] = 0.25          # ties: the smaller page index wins
    s[2, 1] = float("inf")                       # nan_to_num: +inf -> FLT_MAX
    return s


@pytest.mark.parametrize("prebuilt", [False, True])
def test_plan_then_select_general(prebuilt):
    """Ragged rows (some shorter than k): plan() binds the step's CSR and builds the row-major
    block table (or takes a prebuilt one); select(fixed_count=False) equals the oracle."""
    c = make_case(batch=5, hq=8, hkv=2, kv_lens=[40, 700, 1000, 96, 333], seed=3, k=12, L=3,
                  trailing_empty_page=True)
    g = c.to(DEV)
    B, pps = 5, 80
    sel = PageSelectorV2(8, pps, True, c.k, 1.0, 8, DEV)
    qo = torch.arange(B + 1, dtype=torch.int32, device=DEV)
    sub_i = torch.zeros(B * pps, dtype=torch.int32, device=DEV)
    sub_p = torch.zeros(B + 1, dtype=torch.int32, device=DEV)
    if prebuilt:
        sel._block_table.zero_()
        sel._block_table[:B, :g.block_table.shape[1]] = g.block_table
    sel.plan(qo, g.kv_indices, g.kv_indptr, g.kv_last_page_len, sub_i, sub_p, L=c.L,
             block_table_prebuilt=prebuilt)
    assert sel.L == c.L and sel.paged_kv_indptr is g.kv_indptr
    want_bt = O.block_table_from_csr(c.kv_indptr, c.kv_indices, pps)
    assert torch.equal(sel._block_table[:B].cpu(), want_bt)
    n = c.max_pages
    scores = _scores(B, n, seed=5)
    idx, ip = sel.select(scores.to(DEV), fixed_count=False)
    counts = c.kv_indptr[1:] - c.kv_indptr[:-1]
    wi, wp = O.select_pages(scores, counts, want_bt, c.k, c.L)
    assert ip.cpu().tolist() == wp.tolist()
    assert idx.cpu().tolist() == wi.tolist()
    # the rows shorter than k emit all their pages
    assert (ip[1:] - ip[:-1]).cpu().tolist() == torch.clamp(counts, max=c.k).tolist()


def test_select_fixed_count_with_debug_compare():
    """Every row has >= k pages: the fixed-count path returns the static indptr b * k and the
    same pages as the general path (its debug_compare runs the general selector)."""
    c = make_case(batch=4, hq=8, hkv=2, kv_lens=[512, 600, 1000, 777], seed=4, k=16, L=4)
    g = c.to(DEV)
    B, pps = 4, 64
    sel = PageSelectorV2(B, pps, True, c.k, 1.0, c.L, DEV)
    sel.plan(torch.arange(B + 1, dtype=torch.int32, device=DEV), g.kv_indices, g.kv_indptr,
             g.kv_last_page_len, torch.zeros(B * pps, dtype=torch.int32, device=DEV),
             torch.zeros(B + 1, dtype=torch.int32, device=DEV))
    n = c.max_pages
    scores = _scores(B, n, seed=6)
    idx, ip = sel.select(scores.to(DEV), fixed_count=True, debug_compare=True)
    counts = c.kv_indptr[1:] - c.kv_indptr[:-1]
    wi, wp = O.select_pages(scores, counts, O.block_table_from_csr(c.kv_indptr, c.kv_indices, pps), c.k, c.L,
                            fixed_count=True)
    assert ip.cpu().tolist() == wp.tolist() == [b * c.k for b in range(B + 1)]
    assert idx.cpu().tolist() == wi.tolist()
    gi, gp = sel.select(scores.to(DEV), fixed_count=False)
    assert torch.equal(gi, idx) and torch.equal(gp, ip)


def test_select_with_zero_budget_and_plan_on_shared_lists():
    """k = 0 selects nothing; a plan() whose subset lists are the full lists (the gate-off step,
    backend.py:2111-2150) binds them and leaves the block table alone."""
    B, pps = 3, 16
    sel = PageSelectorV2(B, pps, True, 0, 1.0, 2, DEV)
    idx, ip = sel.select(torch.rand((B, 5), device=DEV), fixed_count=False)
    assert idx.numel() == 0 and ip.cpu().tolist() == [0, 0, 0, 0]
    sel2 = PageSelectorV2(B, pps, True, 4, 1.0, 2, DEV)
    sel2._block_table.fill_(7)
    ind = torch.arange(10, dtype=torch.int32, device=DEV)
    ipt = torch.tensor([0, 3, 6, 10], dtype=torch.int32, device=DEV)
    sel2.plan(torch.arange(B + 1, dtype=torch.int32, device=DEV), ind, ipt,
              torch.ones(B, dtype=torch.int32, device=DEV), ind, ipt)
    assert sel2.paged_subset_kv_indices is ind and sel2._block_table.eq(7).all()
