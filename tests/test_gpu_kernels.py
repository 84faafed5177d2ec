"""GPU parity: every HIP kernel against the CPU oracle on the same seeded inputs.

Tolerances (north star): selected page sets bit-exact; page scores within 1e-4
relative (fp32); attention outputs within 2e-2 absolute with cosine > 0.999
(bf16/fp16).  Logits dump within 1e-4 * (1 + |x|) (fp32 accumulation order).
"""

import pytest
import torch

from delta_amd import _lib, kernels as K
from delta_amd.workloads import config_case, make_case
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def cases():
    return {
        "cfg1_bf16": lambda: config_case(1, dtype=torch.bfloat16),
        "cfg2_fp16_small": lambda: config_case(2, scale=0.125),
        "cfg3_bf16_small": lambda: config_case(3, scale=0.125, batch=6),
        "cfg4_g7_small": lambda: config_case(4, scale=1 / 64),
        "cfg5_g5_ragged_small": lambda: config_case(5, scale=1 / 32, batch=12),
        "ragged_g1": lambda: make_case(batch=5, hq=8, hkv=8, kv_lens=[1, 15, 16, 17, 300], seed=3, k=4, L=2),
        "ragged_g8_trailing": lambda: make_case(batch=4, hq=16, hkv=2, kv_lens=[32, 48, 7, 129], seed=4,
                                                k=3, L=1, trailing_empty_page=True, dtype=torch.float16),
        # 36 rows x 8 kv heads >= 256 blocks and <= 65536 page-heads: the head-major mapping
        "head_major_ragged_g2": lambda: make_case(batch=36, hq=16, hkv=8,
                                                  kv_lens=[1 + (37 * i) % 900 for i in range(36)], seed=5,
                                                  page_order="shuffle", k=8, L=2),
        # one long row: 8 (row, head) pairs split 32 ways (merge of 32 units), 1501 pages for
        # the 1024-thread selector, a 384-page subset
        "long_row_b1": lambda: make_case(batch=1, hq=32, hkv=8, kv_lens=[24007], seed=7,
                                         page_order="shuffle", k=384, L=8),
    }


CASES = cases()


def assert_attn_close(got, want, what=""):
    got = got.float().cpu()
    want = want.float().cpu()
    err = (got - want).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(got.flatten(), want.flatten(), dim=0).item()
    assert err <= 2e-2, f"{what}: max abs err {err}"
    assert cos > 0.999, f"{what}: cosine {cos}"


def gpu(c):
    return c.to(DEV)


def assert_variant_close(a, b):
    """Launches with and without the logits dump compute the same math but may cut a row's
    pages into different work units (small attention launches split head-major, dump
    launches page-major), so the fp32 sums run in another order and P (rounded to the KV
    dtype for the P.V MFMA, +-2^-8 relative) can round the other way.  The output then moves
    by ~2^-8 of its typical magnitude: allowed, a few ulp of each output plus two ulp of the
    largest output of its (row, head)."""
    ulp = torch.finfo(a.dtype).eps
    a, b = a.float(), b.float()
    scale = b.abs().amax(dim=-1, keepdim=True)
    assert ((a - b).abs() <= 4 * ulp * b.abs() + 2 * ulp * scale + 1e-6).all()


@pytest.mark.parametrize("name", list(CASES))
def test_decode_attention_and_dump(name):
    c = CASES[name]()
    g = gpu(c)
    B, hq = c.q.shape[:2]
    mp = c.max_pages
    dump = torch.full((B, hq, mp * 16 + 5), 12345.0, device=DEV)
    lse = torch.empty(B, hq, device=DEV)
    o = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len,
                       max_pages_per_row=mp, lse=lse, logits_dump=dump)
    torch.cuda.synchronize()
    o_ref, lse_ref = O.paged_decode_attention(c.q, c.kv_cache, c.kv_indptr, c.kv_indices,
                                              c.kv_last_page_len, c.sm_scale)
    assert_attn_close(o, o_ref, name)
    assert torch.allclose(lse.cpu(), lse_ref, atol=1e-3, rtol=1e-4)
    x_ref = O.dump_logits(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len,
                          c.sm_scale, mp * 16 + 5)
    d = dump.cpu()
    valid = torch.isfinite(x_ref)
    # Whole pages are written: past kv_len inside the row's last page the dump may hold -inf
    # (what the reference's -inf-filled buffer holds there); nothing past that page is touched.
    npages = (c.kv_indptr[1:] - c.kv_indptr[:-1]).tolist()
    for b in range(B):
        kv_len = int(valid[b, 0].sum())
        end = min(npages[b], mp) * 16
        tail = d[b, :, kv_len:end]
        assert torch.all((tail == 12345.0) | (tail == float("-inf"))), f"row {b}: bad values past kv_len"
        assert torch.all(d[b, :, end:] == 12345.0), f"row {b}: dump wrote past the last page"
    err = (d[valid] - x_ref[valid]).abs() / (1 + x_ref[valid].abs())
    assert err.max().item() < 1e-4
    # the no-dump variant agrees to rounding and each variant is deterministic
    o2 = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, max_pages_per_row=mp)
    o3 = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, max_pages_per_row=mp)
    assert torch.equal(o2, o3)
    assert_variant_close(o, o2)


@pytest.mark.parametrize("name", list(CASES))
def test_page_scores(name):
    c = CASES[name]()
    g = gpu(c)
    B, hq = c.q.shape[:2]
    mp = c.max_pages
    dump = torch.empty((B, hq, mp * 16), device=DEV)
    lse = torch.empty(B, hq, device=DEV)
    K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len,
                   max_pages_per_row=mp, lse=lse, logits_dump=dump)
    s_lse = K.page_scores_from_logits(dump, g.kv_indptr, g.kv_last_page_len, mp, lse=lse)
    s_2pass = K.page_scores_from_logits(dump, g.kv_indptr, g.kv_last_page_len, mp)
    s_kv = K.page_score(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, mp)
    # A dump at a 4-byte offset with odd row strides (no alignment assumed by the scorer).
    dump_u = torch.full((B, hq, mp * 16 + 1), float("nan"), device=DEV)[:, :, 1:]
    dump_u.copy_(dump)
    s_unal = K.page_scores_from_logits(dump_u, g.kv_indptr, g.kv_last_page_len, mp, lse=lse)
    torch.cuda.synchronize()
    x = O.dump_logits(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, c.sm_scale, mp * 16)
    ref = O.legacy_softmax_page_scores(x, B, mp, compute_dtype=torch.float64).double()
    for what, s in (("planner", s_lse), ("two-pass", s_2pass), ("kv-only", s_kv), ("unaligned dump", s_unal)):
        s = s.cpu().double()
        rel = ((s - ref).abs() / ref.abs().clamp_min(1e-30))
        rel[ref == 0] = s[ref == 0].abs()
        assert rel.max().item() < 1e-4, f"{name}/{what}: rel err {rel.max().item()}"


@pytest.mark.parametrize("name", ["cfg2_fp16_small", "cfg3_bf16_small", "long_row_b1"])
def test_planner_dump_at_unaligned_address(name):
    """The planner's dump stores (16-byte buffer stores) into a dump view at a 4-byte offset
    with odd row strides, as the C ABI allows: the dump, lse and o equal those of an aligned
    dump, and nothing is written outside the view."""
    c = CASES[name]()
    g = gpu(c)
    B, hq = c.q.shape[:2]
    mp = c.max_pages
    dump_a = torch.full((B, hq, mp * 16), float("-inf"), device=DEV)
    lse_a = torch.empty(B, hq, device=DEV)
    o_a = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, max_pages_per_row=mp,
                         lse=lse_a, logits_dump=dump_a)
    base = torch.full((B, hq, mp * 16 + 1), 7.0, device=DEV)
    dump_u = base[:, :, 1:]
    dump_u.fill_(float("-inf"))
    lse_u = torch.empty(B, hq, device=DEV)
    o_u = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, max_pages_per_row=mp,
                         lse=lse_u, logits_dump=dump_u)
    torch.cuda.synchronize()
    assert torch.equal(dump_u, dump_a) and torch.equal(lse_u, lse_a) and torch.equal(o_u, o_a)
    assert bool((base[:, :, 0] == 7.0).all())


@pytest.mark.parametrize("hq", [4, 12, 20, 24, 40, 44, 48, 56, 64, 72, 96])
def test_page_scores_from_logits_head_counts(hq):
    """The score kernel's head passes (hq rounded up to a multiple of 8 up to 64 heads, several
    passes above) on synthetic logits: rows of 1, 333 and 640 tokens (-inf past kv_len), with the
    planner's lse and with the two-pass normaliser, within 1e-4 of the fp64 oracle."""
    gen = torch.Generator().manual_seed(hq)
    kv_lens = [1, 333, 640]
    B = len(kv_lens)
    pages = [n // 16 + (n % 16 > 0) for n in kv_lens]
    mp = max(pages)
    indptr = torch.zeros(B + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(torch.tensor(pages), 0)
    last = torch.tensor([n - 16 * (p - 1) for n, p in zip(kv_lens, pages)], dtype=torch.int32)
    x = torch.randn(B, hq, mp * 16, generator=gen) * 3
    for b, n in enumerate(kv_lens):
        x[b, :, n:] = float("-inf")
    lse = torch.logsumexp(x.double(), dim=-1).float()
    ref = O.legacy_softmax_page_scores(x, B, mp, compute_dtype=torch.float64).double()
    xd = x.to(DEV)
    for what, kw in (("planner lse", dict(lse=lse.to(DEV))), ("two-pass", {})):
        s = K.page_scores_from_logits(xd, indptr.to(DEV), last.to(DEV), mp, **kw).cpu().double()
        rel = (s - ref).abs() / ref.abs().clamp_min(1e-30)
        rel[ref == 0] = s[ref == 0].abs()
        assert rel.max().item() < 1e-4, f"hq={hq} {what}: rel err {rel.max().item()}"


@pytest.mark.parametrize("name", list(CASES))
def test_selection_bit_exact_on_gpu_scores(name):
    c = CASES[name]()
    g = gpu(c)
    mp = c.max_pages
    s = K.page_score(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, mp)
    counts = (c.kv_indptr[1:] - c.kv_indptr[:-1])
    k = min(c.k, mp)
    kpr = c.k_per_row
    if kpr is not None:
        kpr = torch.clamp(kpr, max=mp)
    idx, indptr = K.select_pages(s, g.kv_indptr, g.block_table, k, c.L,
                                 k_per_row=None if kpr is None else kpr.to(DEV))
    torch.cuda.synchronize()
    sc = s.cpu()
    if kpr is None:
        want_i, want_p = O.select_pages(sc, counts, c.block_table, k, c.L)
    else:  # per-row budgets: the oracle row by row
        wi, wp = [], [0]
        for b in range(c.batch):
            ii, _ = O.select_pages(sc[b:b + 1], counts[b:b + 1], c.block_table[b:b + 1], int(kpr[b]), c.L)
            wi.append(ii)
            wp.append(wp[-1] + ii.numel())
        want_i, want_p = torch.cat(wi), torch.tensor(wp, dtype=torch.int32)
    assert indptr.cpu().tolist() == want_p.tolist()
    assert idx[:int(want_p[-1])].cpu().tolist() == want_i.tolist()


# Row lengths for each selection launch: 256-thread blocks (<= 1024 pages), 512-thread blocks
# with 4 or 8 keys per thread (<= 2048, <= 4096), 1024-thread blocks with the keys in registers
# (<= 8192; 4097 is config 4's row after its decode token) and with the keys re-read every pass
# (longer).
@pytest.mark.parametrize("n", [300, 1500, 2500, 4097, 5000, 9000])
def test_selection_adversarial_scores(n):
    gen = torch.Generator().manual_seed(5)
    B = 6
    s = torch.round(torch.rand(B, n, generator=gen) * 4) / 4  # heavy ties
    s[0, :50] = float("nan")
    s[1, 10:20] = float("inf")
    s[2, ::3] = float("-inf")
    s[3] = 0.0
    s[3, ::2] = -0.0
    s[4, 5] = 3.4e38
    counts = torch.tensor([n, n - 1, 2 * n // 3, n, 17, 64])
    indptr = torch.zeros(B + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(counts, 0)
    bt = torch.randperm(B * n, generator=gen).reshape(B, n).to(torch.int32)
    for k, L, bias in ((40, 8, 1e-7), (40, 8, 0.0), (64, 0, 1e-7), (1, 1, 1e-7), (300, 3, 1e-7)):
        idx, ip = K.select_pages(s.to(DEV), indptr.to(DEV), bt.to(DEV), k, L, pos_bias_scale=bias)
        wi, wp = O.select_pages(s, counts, bt, k, L, bias)
        assert ip.cpu().tolist() == wp.tolist(), (k, L, bias)
        assert idx[:int(wp[-1])].cpu().tolist() == wi.tolist(), (k, L, bias)


def test_selection_fixed_and_use_subset():
    gen = torch.Generator().manual_seed(6)
    B, n, k = 4, 50, 16
    s = torch.rand(B, n, generator=gen)
    counts = torch.tensor([50, 50, 40, 30])
    indptr = torch.zeros(B + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(counts, 0)
    bt = torch.randperm(B * n, generator=gen).reshape(B, n).to(torch.int32)
    idx, ip = K.select_pages(s.to(DEV), indptr.to(DEV), bt.to(DEV), k, 4, fixed_count=True)
    wi, wp = O.select_pages(s, counts, bt, k, 4, fixed_count=True)
    assert ip.cpu().tolist() == wp.tolist() and idx.cpu().tolist() == wi.tolist()
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    idx, ip = K.select_pages(s.to(DEV), indptr.to(DEV), bt.to(DEV), k, 4, use_subset=flag)
    assert ip.cpu().tolist() == indptr.tolist()
    full = torch.cat([bt[b, :int(counts[b])] for b in range(B)])
    assert idx[:int(indptr[-1])].cpu().tolist() == full.tolist()


@pytest.mark.parametrize("seed", range(12))
def test_selection_random_shapes(seed):
    """Seeded random selections against the oracle, bit for bit: row counts over both launch
    sizes and the register-held / re-read paths (max pages 3 .. 9500), ragged rows, random k, L
    and position bias, quantised scores (ties) with NaN / +-inf sprinkled in, and per-row
    budgets on every other seed (each row against the oracle's single-row selection)."""
    g = torch.Generator().manual_seed(1000 + seed)
    ri = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=g))
    B = ri(1, 24)
    n = [ri(3, 300), ri(300, 1024), ri(1025, 4096), ri(4097, 8192), ri(8193, 9500)][seed % 5]
    counts = torch.randint(1, n + 1, (B,), generator=g)
    counts[0] = n
    s = torch.round(torch.rand(B, n, generator=g) * ri(4, 4096)) / 1024.0
    s[torch.rand(B, n, generator=g) < 0.01] = float("nan")
    s[torch.rand(B, n, generator=g) < 0.005] = float("inf")
    s[torch.rand(B, n, generator=g) < 0.01] = float("-inf")
    indptr = torch.zeros(B + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(counts, 0)
    bt = torch.randperm(B * n, generator=g).reshape(B, n).to(torch.int32)
    k, L = ri(1, min(n, 300)), ri(0, 10)
    bias = [0.0, 1e-7, 1e-3][seed % 3]
    sd, ipd, btd = s.to(DEV), indptr.to(DEV), bt.to(DEV)
    if seed % 2 == 0:
        idx, ip = K.select_pages(sd, ipd, btd, k, L, pos_bias_scale=bias)
        wi, wp = O.select_pages(s, counts, bt, k, L, bias)
        assert ip.cpu().tolist() == wp.tolist()
        assert idx[:int(wp[-1])].cpu().tolist() == wi.tolist()
    else:
        kpr = torch.randint(1, k + 1, (B,), generator=g).to(torch.int32)
        idx, ip = K.select_pages(sd, ipd, btd, k, L, pos_bias_scale=bias, k_per_row=kpr.to(DEV))
        got_p = ip.cpu()
        for b in range(B):
            wi, wp = O.select_pages(s[b:b + 1], counts[b:b + 1], bt[b:b + 1], int(kpr[b]), L, bias)
            assert int(got_p[b + 1] - got_p[b]) == int(wp[-1]), b
            assert idx[int(got_p[b]):int(got_p[b + 1])].cpu().tolist() == wi.tolist(), b


@pytest.mark.parametrize("n", [1500, 3000, 4097, 8192, 9000])
def test_selection_long_rows_fixed_per_row_and_gate_off(n):
    """The 512- and 1024-thread launches (each thread a contiguous run of ceil(n / threads)
    keys, up to 8192 pages; longer rows re-read their scores every pass): the fixed path,
    per-row budgets over ragged rows (each against the oracle's single-row selection with its
    own k) and the gate off (every row's pages in order)."""
    gen = torch.Generator().manual_seed(16)
    B, k, L = 5, 96, 8
    s = torch.rand(B, n, generator=gen) * 1e-3
    s[1, ::7] = s[1, 3]  # ties
    counts = torch.tensor([n, n, n - 5, n // 2, 200])
    indptr = torch.zeros(B + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(counts, 0)
    bt = torch.randperm(B * n, generator=gen).reshape(B, n).to(torch.int32)
    sd, ipd, btd = s.to(DEV), indptr.to(DEV), bt.to(DEV)
    idx, ip = K.select_pages(sd, ipd, btd, k, L, fixed_count=True)
    wi, wp = O.select_pages(s, counts, bt, k, L, fixed_count=True)
    assert ip.cpu().tolist() == wp.tolist() and idx.cpu().tolist() == wi.tolist()
    kpr = torch.tensor([1, k, 37, k // 2, 200], dtype=torch.int32)  # row 4 (200 pages) takes them all
    idx, ip = K.select_pages(sd, ipd, btd, 200, L, k_per_row=kpr.to(DEV))
    got_p = ip.cpu()
    for b in range(B):
        kb = int(kpr[b])
        wi, wp = O.select_pages(s[b:b + 1], counts[b:b + 1], bt[b:b + 1], kb, L)
        assert int(got_p[b + 1] - got_p[b]) == int(wp[-1]), b
        assert idx[int(got_p[b]):int(got_p[b + 1])].cpu().tolist() == wi.tolist(), b
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    idx, ip = K.select_pages(sd, ipd, btd, k, L, use_subset=flag)
    assert ip.cpu().tolist() == indptr.tolist()
    full = torch.cat([bt[b, :int(counts[b])] for b in range(B)])
    assert idx[:int(indptr[-1])].cpu().tolist() == full.tolist()


@pytest.mark.parametrize("name", list(CASES))
def test_selective_step_end_to_end(name):
    """Planner score -> selection -> sparse attention, against the oracle's own chain."""
    c = CASES[name]()
    if c.k_per_row is not None:
        pytest.skip("per-row budgets checked in test_selection_bit_exact_on_gpu_scores")
    g = gpu(c)
    B, hq = c.q.shape[:2]
    mp = c.max_pages
    k = min(c.k, mp)
    dump = torch.empty((B, hq, mp * 16), device=DEV)
    lse = torch.empty(B, hq, device=DEV)
    o_full = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len,
                            max_pages_per_row=mp, lse=lse, logits_dump=dump)
    s = K.page_scores_from_logits(dump, g.kv_indptr, g.kv_last_page_len, mp, lse=lse)
    idx, ip = K.select_pages(s, g.kv_indptr, g.block_table, k, c.L)
    o_sp = K.paged_decode(g.q, g.kv_cache, ip, idx, g.kv_last_page_len, max_pages_per_row=k, subset=True)
    torch.cuda.synchronize()
    ref = O.selective_step(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, k=k, L=c.L)
    assert_attn_close(o_full, ref["o_full"], name + "/full")
    got = idx[:int(ip[-1])].cpu()
    counts = (c.kv_indptr[1:] - c.kv_indptr[:-1])
    # Exact equality unless two pages straddle the threshold closer than the score error.
    keys = O.prepare_scores(ref["scores"], counts, c.L)
    mism = 0
    for b in range(B):
        a = set(got[int(ip[b]):int(ip[b + 1])].tolist())
        r = set(ref["indices"][int(ref["indptr"][b]):int(ref["indptr"][b + 1])].tolist())
        if a == r:
            continue
        mism += 1
        kb = sorted(keys[b].tolist(), reverse=True)
        thr = kb[k - 1]
        bt = c.block_table[b].tolist()
        for p in a ^ r:
            j = bt.index(p)
            assert abs(float(keys[b, j]) - thr) <= 2e-4 * abs(thr), f"{name}: row {b} page {j} far from threshold"
    if mism == 0:
        assert_attn_close(o_sp, ref["o_sparse"], name + "/sparse")
    else:
        # the kernel over the oracle's own selection, against the oracle's sparse attention
        o_sp_r = K.paged_decode(g.q, g.kv_cache, ref["indptr"].to(DEV), ref["indices"].to(DEV), g.kv_last_page_len,
                                max_pages_per_row=k, subset=True)
        assert_attn_close(o_sp_r, ref["o_sparse"], name + "/sparse over the oracle's selection")
    if c.planted is not None:
        for b in range(B):
            sel = set(got[int(ip[b]):int(ip[b + 1])].tolist())
            planted_phys = {int(c.block_table[b, int(j)]) for j in c.planted[b]}
            assert planted_phys <= sel, f"row {b}: planted-page recall < 100%"


@pytest.mark.parametrize("plan_pages", ["exact", "short"])
def test_ragged_work_units(plan_pages):
    """Rows of very different lengths in one split launch: each row is cut into work units of
    at most 128 pages, packed at the front of the grid.  "short" plans for fewer pages than
    the longest row holds: that row's last unit takes the remainder.  Attention, lse and the
    dump must still cover every page of every row."""
    lens = [1, 16, 17, 2500 * 16 + 3, 40, 900 * 16, 5, 3000]
    c = make_case(batch=len(lens), hq=16, hkv=8, kv_lens=lens, seed=11, page_order="randperm", k=4, L=2)
    g = gpu(c)
    B, hq = c.q.shape[:2]
    mp = c.max_pages if plan_pages == "exact" else 100
    assert K._lib.query("delta_decode_num_splits", B, 8, mp) > 1  # a split (work-unit) launch
    dump = torch.full((B, hq, c.max_pages * 16), 12345.0, device=DEV)
    lse = torch.empty(B, hq, device=DEV)
    o = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len,
                       max_pages_per_row=mp, lse=lse, logits_dump=dump)
    o2 = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, max_pages_per_row=mp)
    torch.cuda.synchronize()
    o_ref, lse_ref = O.paged_decode_attention(c.q, c.kv_cache, c.kv_indptr, c.kv_indices,
                                              c.kv_last_page_len, c.sm_scale)
    assert_attn_close(o, o_ref, "ragged units")
    assert_attn_close(o2, o_ref, "ragged units, no dump")
    assert_variant_close(o, o2)
    assert torch.allclose(lse.cpu(), lse_ref, atol=1e-3, rtol=1e-4)
    x_ref = O.dump_logits(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len,
                          c.sm_scale, c.max_pages * 16)
    d = dump.cpu()
    written = min(mp, c.max_pages) * 16  # the dump holds max_pages_per_row pages per row
    valid = torch.isfinite(x_ref)
    valid[:, :, written:] = False
    err = (d[valid] - x_ref[valid]).abs() / (1 + x_ref[valid].abs())
    assert err.max().item() < 1e-4
    assert torch.all(d[:, :, written:] == 12345.0)


@pytest.mark.parametrize("batch,hq,hkv,trailing,lo,hi", [
    (40, 40, 8, False, 1, 60),    # 320 blocks: rounds of 32 rows, the second one partial and reversed
    (96, 8, 4, True, 1, 60),      # rounds of 64 rows, trailing empty pages
    (300, 2, 1, False, 1, 60),    # rounds of 256 rows, a partial reversed round of 44
    (500, 1, 1, False, 32, 33),   # two page counts (ties everywhere); the row tables outgrow the
                                  # scorers' own LDS
])
def test_balanced_row_order(batch, hq, hkv, trailing, lo, hi):
    """Unsplit head-major launches whose (row, kv head) blocks outnumber the CUs (B * Hkv > 256
    on MI355X) and whose rows reach 32 pages take their rows in a balanced order: rows ranked by
    page count (ties by row) and dealt in rounds of CUs / Hkv, every other round reversed, each
    block reading its row's bounds from the ranking's LDS tables.  Every row must still be
    attended exactly once, so every row's output, lse, dump and page scores are checked against
    the oracle: the attention launch with and without the dump, the subset launch over the same
    pages, the planner and the K-only scorer with their logits on chip."""
    gen = torch.Generator().manual_seed(61)
    lens = (torch.randint(lo - 1, hi, (batch,), generator=gen) * 16
            + torch.randint(1, 17, (batch,), generator=gen)).tolist()
    lens[0] = 1 if lo == 1 else lens[0]
    lens[1] = hi * 16  # the longest row: max_pages >= 32
    c = make_case(batch=batch, hq=hq, hkv=hkv, kv_lens=lens, seed=62, page_order="randperm", k=4, L=2,
                  trailing_empty_page=trailing)
    g = gpu(c)
    B, mp = batch, c.max_pages
    dump = torch.full((B, hq, mp * 16), 12345.0, device=DEV)
    lse = torch.empty(B, hq, device=DEV)
    o = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, max_pages_per_row=mp,
                       lse=lse, logits_dump=dump)
    o_nd = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, max_pages_per_row=mp)
    o_sub = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, max_pages_per_row=mp,
                           subset=True)
    o_chip, s_chip = K.paged_decode_scores(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len,
                                           max_pages_per_row=mp)
    s_k = K.page_score(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, mp)
    torch.cuda.synchronize()
    o_ref, lse_ref = O.paged_decode_attention(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len,
                                              c.sm_scale)
    for b in range(B):
        for what, got in (("dump launch", o), ("no dump", o_nd), ("subset", o_sub), ("planner on chip", o_chip)):
            assert_attn_close(got[b], o_ref[b], f"{what}, row {b}")
    assert torch.equal(o_nd, o_sub)
    assert torch.allclose(lse.cpu(), lse_ref, atol=1e-3, rtol=1e-4)
    x_ref = O.dump_logits(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, c.sm_scale, mp * 16)
    valid = torch.isfinite(x_ref)
    d = dump.cpu()
    assert ((d[valid] - x_ref[valid]).abs() / (1 + x_ref[valid].abs())).max().item() < 1e-4
    ref = O.legacy_softmax_page_scores(x_ref, B, mp, compute_dtype=torch.float64).double()
    for what, s in (("planner on chip", s_chip), ("K-only scorer", s_k)):
        s = s.cpu().double()
        rel = (s - ref).abs() / ref.abs().clamp_min(1e-30)
        rel[ref == 0] = s[ref == 0].abs()
        assert rel.max().item() < 1e-4, f"{what}: rel err {rel.max().item()}"


def test_sparse_equals_full_when_budget_covers_all():
    c = config_case(3, scale=0.25, batch=4)
    g = gpu(c)
    mp = c.max_pages
    dump = torch.empty((4, 32, mp * 16), device=DEV)
    lse = torch.empty(4, 32, device=DEV)
    o_full = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len,
                            max_pages_per_row=mp, lse=lse, logits_dump=dump)
    s = K.page_scores_from_logits(dump, g.kv_indptr, g.kv_last_page_len, mp, lse=lse)
    idx, ip = K.select_pages(s, g.kv_indptr, g.block_table, mp, 8)
    assert torch.equal(ip, g.kv_indptr) and torch.equal(idx[:int(ip[-1])], g.kv_indices)
    o_sp = K.paged_decode(g.q, g.kv_cache, ip, idx, g.kv_last_page_len, max_pages_per_row=mp, subset=True)
    o_nd = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, max_pages_per_row=mp)
    assert torch.equal(o_sp, o_nd)
    assert_variant_close(o_sp, o_full)


def test_pack_page_indices():
    gen = torch.Generator().manual_seed(7)
    pps = 40
    slot_bt = torch.randint(0, 10000, (6, pps), generator=gen, dtype=torch.int32)
    active = torch.tensor([5, 1, 2, 0], dtype=torch.int32)
    starts = torch.tensor([0, 10, 3, 39], dtype=torch.int32)
    counts = torch.tensor([40, 30, 0, 1], dtype=torch.int32)
    indptr = torch.tensor([0, 40, 70, 70, 71], dtype=torch.int32)
    out = torch.full((71,), -1, dtype=torch.int32)
    row = torch.full((4, pps), -1, dtype=torch.int32)
    out_g, row_g = out.to(DEV), row.to(DEV)
    K.pack_page_indices(slot_bt.to(DEV), active.to(DEV), starts.to(DEV), counts.to(DEV), indptr.to(DEV),
                        out_g, row_g, 4, 40, write_row_block=True)
    O.pack_page_indices(slot_bt, active, starts, counts, indptr, out, row, 4, True)
    assert torch.equal(out_g.cpu(), out) and torch.equal(row_g.cpu(), row)


def test_decode_page_info():
    gen = torch.Generator().manual_seed(8)
    B, pps, k = 7, 64, 9
    cachelens = torch.tensor([0, 14, 15, 16, 31, 200, 1100], dtype=torch.int32)  # last row overflows
    slot_bt = torch.randint(0, 99999, (B, pps), generator=gen, dtype=torch.int32)
    ind = torch.zeros(B * pps, dtype=torch.int32, device=DEV)
    ip = torch.zeros(B + 1, dtype=torch.int32, device=DEV)
    last = torch.zeros(B, dtype=torch.int32, device=DEV)
    rbt = torch.full((B, pps), -7, dtype=torch.int32, device=DEV)
    sub_i = torch.zeros(B * pps, dtype=torch.int32, device=DEV)
    sub_p = torch.zeros(B + 1, dtype=torch.int32, device=DEV)
    flag = torch.full((1,), -1, dtype=torch.int32, device=DEV)
    K.decode_page_info(cachelens.to(DEV), slot_bt.to(DEV), B, k, 1.0, True, ip, ind, last, rbt, sub_i, sub_p, flag)
    torch.cuda.synchronize()
    pc, lp, sc, ss = O.decode_page_info(cachelens[:-1], pps, k)
    pc = torch.cat([pc, torch.tensor([pps])])     # the overflowing row is clamped to a full table
    lp = torch.cat([lp, torch.tensor([16])])
    sc = torch.clamp(pc, max=k)
    ss = pc - sc
    assert last.cpu().tolist() == lp.tolist()
    want_ip = [0] + torch.cumsum(pc, 0).tolist()
    assert ip.cpu().tolist() == want_ip
    for b in range(B):
        row = slot_bt[b, :int(pc[b])]
        assert ind[want_ip[b]:want_ip[b + 1]].cpu().tolist() == row.tolist()
        assert rbt[b, :int(pc[b])].cpu().tolist() == row.tolist()
        assert rbt[b, int(pc[b]):].cpu().eq(0).all()
    sp = [0] + torch.cumsum(sc, 0).tolist()
    assert sub_p.cpu().tolist() == sp
    for b in range(B):
        assert sub_i[sp[b]:sp[b + 1]].cpu().tolist() == slot_bt[b, int(ss[b]):int(pc[b])].tolist()
    assert int(flag) == int(O.use_subset_decision(int(pc.sum()), int(sc.sum()), 1.0)) == 1
    # gate off (ratio too high): the subset CSR is the full CSR
    K.decode_page_info(cachelens.to(DEV), slot_bt.to(DEV), B, k, 1e9, True, ip, ind, last, rbt, sub_i, sub_p, flag)
    torch.cuda.synchronize()
    assert int(flag) == 0
    assert sub_p.cpu().tolist() == want_ip
    assert torch.equal(sub_i[:want_ip[-1]], ind[:want_ip[-1]])


@pytest.mark.parametrize("active_rows", [[0, 1, 2, 3], [3, 10, 17, 30], list(range(32))])
def test_decode_page_info_gate_counts_active_rows(active_rows):
    """Partial batches near the gate's threshold: the device gate sums page totals over the
    active rows only, as the reference does (backend.py:2047-2067, 2104-2109)."""
    B, pps, k = 32, 4100, 256
    gen = torch.Generator().manual_seed(9)
    cachelens = torch.zeros(B, dtype=torch.int32)
    active = torch.zeros(B, dtype=torch.int32)
    for r in active_rows:
        cachelens[r] = 65536          # 4097 pages after the decode token
        active[r] = 1
    slot_bt = torch.randint(0, 1 << 20, (B, pps), generator=gen, dtype=torch.int32).to(DEV)
    ind = torch.zeros(B * pps, dtype=torch.int32, device=DEV)
    ip = torch.zeros(B + 1, dtype=torch.int32, device=DEV)
    last = torch.zeros(B, dtype=torch.int32, device=DEV)
    sub_i = torch.zeros(B * pps, dtype=torch.int32, device=DEV)
    sub_p = torch.zeros(B + 1, dtype=torch.int32, device=DEV)
    flag = torch.full((1,), -1, dtype=torch.int32, device=DEV)
    for ratio in (15.9, 16.0, 16.0039, 16.004, 16.5):
        for act in (active, None):
            K.decode_page_info(cachelens.to(DEV), slot_bt, B, k, ratio, True, ip, ind, last, None, sub_i, sub_p,
                               flag, active=None if act is None else act.to(DEV))
            torch.cuda.synchronize()
            want = O.decode_step_gate(cachelens.tolist(), [1] * B if act is None else act.tolist(), k, ratio)
            assert int(flag) == int(want), (active_rows, ratio, act is None)
            # the CSR covers every slot either way; the subset CSR follows the gate
            pc = [(int(c) + 1) // 16 + 1 for c in cachelens]
            want_ip = [0] + torch.cumsum(torch.tensor(pc), 0).tolist()
            assert ip.cpu().tolist() == want_ip
            sc = [min(n, k) if want else n for n in pc]
            assert sub_p.cpu().tolist() == [0] + torch.cumsum(torch.tensor(sc), 0).tolist()


def test_decode_page_info_per_row_budgets():
    """k_per_row (an extension of the reference's global k): row b's subset is its last
    min(pages_b, k_b) pages and the gate sums min(pages_b, k_b) over the active rows, as
    O.decode_page_info / O.decode_step_gate count them; budgets clamp to [0, pages_per_slot]
    as the selector clamps them; idle rows keep their entries but leave the totals."""
    gen = torch.Generator().manual_seed(10)
    B, pps = 6, 40
    cachelens = torch.tensor([15, 40, 300, 95, 0, 500], dtype=torch.int32)
    kpr = torch.tensor([1, 8, 4, 0, 3, 99], dtype=torch.int32)     # 99 clamps to pages_per_slot
    active = torch.tensor([1, 1, 1, 1, 0, 1], dtype=torch.int32)
    slot_bt = torch.randint(0, 1 << 20, (B, pps), generator=gen, dtype=torch.int32)
    ind = torch.zeros(B * pps, dtype=torch.int32, device=DEV)
    ip = torch.zeros(B + 1, dtype=torch.int32, device=DEV)
    last = torch.zeros(B, dtype=torch.int32, device=DEV)
    sub_i = torch.zeros(B * pps, dtype=torch.int32, device=DEV)
    sub_p = torch.zeros(B + 1, dtype=torch.int32, device=DEV)
    flag = torch.full((1,), -1, dtype=torch.int32, device=DEV)
    pc, lp, sc, ss = O.decode_page_info(cachelens, pps, torch.clamp(kpr, max=pps))
    for ratio in (1.0, 1.57, 1.58, 1e9):  # active totals 63 / 40 = 1.575
        K.decode_page_info(cachelens.to(DEV), slot_bt.to(DEV), B, 7, ratio, True, ip, ind, last, None, sub_i,
                           sub_p, flag, active=active.to(DEV), k_per_row=kpr.to(DEV))
        torch.cuda.synchronize()
        want = O.decode_step_gate(cachelens.tolist(), active.tolist(), torch.clamp(kpr, max=pps).tolist(), ratio)
        assert int(flag) == int(want), ratio
        assert last.cpu().tolist() == lp.tolist()
        cnt = sc.tolist() if want else pc.tolist()
        start = ss.tolist() if want else [0] * B
        sp = [0] + torch.cumsum(torch.tensor(cnt), 0).tolist()
        assert sub_p.cpu().tolist() == sp, ratio
        for b in range(B):
            assert sub_i[sp[b]:sp[b + 1]].cpu().tolist() == slot_bt[b, start[b]:int(pc[b])].tolist(), (ratio, b)


@pytest.mark.parametrize("min_tokens,divisor,k", [(512, 8, 256), (64, 8, 20), (0, 1, 1000)])
def test_decode_page_info_budget_rule(min_tokens, divisor, k):
    """budget_rule (an extension): every row's budget comes from its length on the device,
    written out equal to O.budget_rule_pages, and the gate's totals and the default subset CSR
    use it as they use fixed per-row budgets.  300 rows (more than one 256-thread pass of the
    totals loop) of ragged lengths in [0, 8000], a few idle; the gate is checked on and off."""
    gen = torch.Generator().manual_seed(12)
    B = 300
    cachelens = torch.randint(0, 8001, (B,), generator=gen, dtype=torch.int32)
    cachelens[:4] = torch.tensor([0, 15, 4223, 8000], dtype=torch.int32)
    pps = 8001 // 16 + 1
    active = (torch.rand(B, generator=gen) > 0.1).to(torch.int32)
    slot_bt = torch.randint(0, 1 << 20, (B, pps), generator=gen, dtype=torch.int32)
    want_k = O.budget_rule_pages(cachelens, min_tokens, divisor, k)
    pc, lp, sc, ss = O.decode_page_info(cachelens, pps, want_k)
    ip = torch.zeros(B + 1, dtype=torch.int32, device=DEV)
    ind = torch.zeros(B * pps, dtype=torch.int32, device=DEV)
    last = torch.zeros(B, dtype=torch.int32, device=DEV)
    sub_i = torch.zeros(B * pps, dtype=torch.int32, device=DEV)
    sub_p = torch.zeros(B + 1, dtype=torch.int32, device=DEV)
    flag = torch.full((1,), -1, dtype=torch.int32, device=DEV)
    full_tot = int(pc[active.bool()].sum())
    sub_tot = int(sc[active.bool()].sum())
    for ratio in (1.0, full_tot / sub_tot - 1e-6, full_tot / sub_tot + 1e-6):
        out = torch.full((B,), -7, dtype=torch.int32, device=DEV)
        K.decode_page_info(cachelens.to(DEV), slot_bt.to(DEV), B, k, ratio, True, ip, ind, last, None, sub_i,
                           sub_p, flag, active=active.to(DEV), budget_rule=(min_tokens, divisor, out))
        torch.cuda.synchronize()
        assert out.cpu().tolist() == want_k.tolist()
        want = O.decode_step_gate(cachelens.tolist(), active.tolist(), want_k.tolist(), ratio)
        assert int(flag) == int(want), ratio
        cnt = sc.tolist() if want else pc.tolist()
        start = ss.tolist() if want else [0] * B
        sp = [0] + torch.cumsum(torch.tensor(cnt), 0).tolist()
        assert sub_p.cpu().tolist() == sp, ratio
        got = sub_i.cpu()
        for b in range(B):
            assert got[sp[b]:sp[b + 1]].tolist() == slot_bt[b, start[b]:int(pc[b])].tolist(), (ratio, b)
    out = torch.zeros(B, dtype=torch.int32, device=DEV)
    with pytest.raises(K._lib.DeltaHipError, match="budget rule needs"):
        K.decode_page_info(cachelens.to(DEV), slot_bt.to(DEV), B, k, 1.0, True, ip, ind, last, None, sub_i,
                           sub_p, flag, budget_rule=(min_tokens, 0, out))
    with pytest.raises(ValueError, match="exclusive"):
        K.decode_page_info(cachelens.to(DEV), slot_bt.to(DEV), B, k, 1.0, True, ip, ind, last, None, sub_i,
                           sub_p, flag, k_per_row=out, budget_rule=(min_tokens, divisor, out))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_append_kv(dtype):
    c = make_case(batch=3, hq=8, hkv=4, kv_lens=[17, 32, 50], seed=9, dtype=dtype, trailing_empty_page=True)
    gen = torch.Generator().manual_seed(1)
    nnz = 6
    app = torch.tensor([0, 1, 1, 6], dtype=torch.int32)  # row 1 appends nothing; row 2 appends 5 (prefill-like)
    qkv = torch.randn(nnz, 16, 128, generator=gen).to(dtype)  # strided k/v views like wqkv(x).split
    k, v = qkv[:, 8:12], qkv[:, 12:16]
    cache = c.kv_cache.clone()
    O.append_kv(k.float(), v.float(), app, cache, c.kv_indices, c.kv_indptr, c.kv_last_page_len)
    gcache = c.kv_cache.to(DEV)
    K.append_kv(k.to(DEV), v.to(DEV), app.to(DEV), gcache, c.kv_indices.to(DEV), c.kv_indptr.to(DEV),
                c.kv_last_page_len.to(DEV))
    assert torch.equal(gcache.cpu(), cache)


@pytest.mark.parametrize("llama31", [False, True])
def test_rope(llama31):
    gen = torch.Generator().manual_seed(2)
    nnz, hq, hkv = 7, 32, 8
    q = torch.randn(nnz, hq, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(nnz, hkv, 128, generator=gen).to(torch.bfloat16)
    indptr = torch.tensor([0, 1, 5, 7], dtype=torch.int32)
    offsets = torch.tensor([8191, 0, 123], dtype=torch.int32)
    kw = dict(rope_scale=8.0 if llama31 else 1.0, rope_theta=5e5)
    if llama31:
        kw.update(low_freq_factor=1.0, high_freq_factor=4.0, old_context_len=8192)
    qo, ko = K.rope(q.to(DEV), k.to(DEV), indptr.to(DEV), offsets.to(DEV), **kw)
    f = O.rope_frequencies(128, kw["rope_scale"], kw["rope_theta"], kw.get("low_freq_factor"),
                           kw.get("high_freq_factor"), kw.get("old_context_len"))
    qr = O.apply_rope(q.float(), indptr, offsets, f)
    kr = O.apply_rope(k.float(), indptr, offsets, f)
    # fp32 angles at positions ~8k are good to ~1e-3 rad; bf16 output rounding ~4e-3 relative
    assert (qo.float().cpu() - qr).abs().max().item() < 3e-2
    assert (ko.float().cpu() - kr).abs().max().item() < 3e-2


def test_decode_is_deterministic_full_size():
    """Config 3 at full size: two runs are bit-identical; score sums lie in [1, Hq]."""
    c = config_case(3, device=DEV)
    mp = c.max_pages
    B, hq = c.q.shape[:2]
    dump = torch.empty((B, hq, mp * 16), device=DEV)
    lse = torch.empty(B, hq, device=DEV)
    o1 = K.paged_decode(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len,
                        max_pages_per_row=mp, lse=lse, logits_dump=dump)
    o2 = K.paged_decode(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len,
                        max_pages_per_row=mp, lse=lse, logits_dump=dump)
    s = K.page_scores_from_logits(dump, c.kv_indptr, c.kv_last_page_len, mp, lse=lse)
    idx, ip = K.select_pages(s, c.kv_indptr, c.block_table, c.k, c.L)
    idx2, ip2 = K.select_pages(s, c.kv_indptr, c.block_table, c.k, c.L)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    tot = s.sum(1)
    assert bool((tot > 1 - 1e-3).all()) and bool((tot < hq + 1e-3).all())
    assert torch.equal(idx, idx2) and torch.equal(ip, ip2)
    assert ip.cpu().tolist() == [c.k * b for b in range(B + 1)]
    # ascending logical order, forced last L pages
    inv = torch.empty(c.kv_cache.shape[0], dtype=torch.int64, device=DEV)
    inv[c.block_table.flatten().long()] = torch.arange(mp, device=DEV).repeat(B)
    pos = inv[idx.long()].view(B, c.k)
    assert bool((pos[:, 1:] > pos[:, :-1]).all())
    assert bool((pos[:, -c.L:] == torch.arange(mp - c.L, mp, device=DEV)).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dense_step_helpers_match_torch(dtype):
    """add_rmsnorm / silu_mul / argmax against the torch ops they replace (model.py:320-323, 509-532)."""
    gen = torch.Generator(device=DEV).manual_seed(3)
    rows, dim, inter = 32, 4096, 1024
    x = torch.randn(rows, dim, generator=gen, device=DEV).to(dtype)
    r = torch.randn(rows, dim, generator=gen, device=DEV).to(dtype)
    w = (1 + 0.1 * torch.randn(dim, generator=gen, device=DEV)).to(dtype)
    h, y = K.add_rmsnorm(x, r, w, 1e-5)
    h_ref = x + r
    hf = h_ref.float()
    y_ref = (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(dtype) * w
    assert torch.equal(h, h_ref)
    ulp = torch.finfo(dtype).eps
    assert ((y.float() - y_ref.float()).abs() <= 2 * ulp * y_ref.float().abs() + 1e-6).all()
    _, y0 = K.add_rmsnorm(x, None, w, 1e-5)
    xf = x.float()
    y0_ref = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(dtype) * w
    assert ((y0.float() - y0_ref.float()).abs() <= 2 * ulp * y0_ref.float().abs() + 1e-6).all()
    gu = torch.randn(rows, 2 * inter, generator=gen, device=DEV).to(dtype) * 3
    s = K.silu_mul(gu)
    s_ref = torch.nn.functional.silu(gu[:, :inter]) * gu[:, inter:]
    assert ((s.float() - s_ref.float()).abs() <= 2 * ulp * s_ref.float().abs() + 1e-6).all()
    logits = torch.randn(rows, 128256, generator=gen, device=DEV).to(dtype)
    logits[3, 77] = logits[3].max() + 1
    logits[4, 10] = logits[4, 20] = logits[4].max() + 1   # tie: first index wins
    logits[5, 1000] = float("nan")                         # NaN ranks highest, as torch.argmax
    assert torch.equal(K.argmax_rows(logits), torch.argmax(logits, -1))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,Kd,bias", [(32, 4096, 4096, False), (1, 48, 64, True), (5, 6144, 4160, True),
                                        (32, 272, 14336, False), (40, 64, 1024, False), (4, 3584, 18944, False),
                                        (8, 4608, 3584, True), (2, 152064, 3584, False), (3, 16, 640, True)])
def test_gemm_skinny_matches_fp32_reference(dtype, M, N, Kd, bias):
    """delta_gemm_skinny against x.float() @ w.float().T (+ b): fp32 accumulation then one
    rounding, so the error is one output ulp plus fp32 summation-order noise."""
    gen = torch.Generator(device=DEV).manual_seed(M * 7 + N + Kd)
    x = torch.randn(M, Kd, generator=gen, device=DEV).to(dtype)
    w = (torch.randn(N, Kd, generator=gen, device=DEV) * 0.05).to(dtype)
    b = (torch.randn(N, generator=gen, device=DEV) * 0.1).to(dtype) if bias else None
    out = K.gemm_skinny(x, w, b)
    torch.cuda.synchronize()
    ref = x.float() @ w.float().T + (b.float() if bias else 0.0)
    mag = x.float().abs() @ w.float().abs().T
    eps = torch.finfo(dtype).eps
    err = (out.float() - ref).abs()
    assert torch.all(err <= eps * ref.abs() + 1e-5 * mag + 1e-6), f"max err {err.max().item()}"
    # deterministic
    assert torch.equal(out, K.gemm_skinny(x, w, b))


@pytest.mark.parametrize("llama31,hq,hkv,dtype,misalign,qo", [
    (False, 16, 4, torch.bfloat16, False, [1, 2, 1, 1]),
    (True, 16, 4, torch.bfloat16, False, [1, 2, 1, 1]),
    (True, 64, 8, torch.float16, False, [1, 0, 2, 1]),   # > 3 chunks per thread; an empty row
    (False, 40, 8, torch.bfloat16, True, [2, 1, 0, 1]),  # 4-byte aligned q/k: the pairwise kernel
])
def test_rope_append_equals_rope_then_append(llama31, hq, hkv, dtype, misalign, qo):
    """The fused launch writes the same q and the same cache bytes as delta_rope followed by
    delta_append_kv (same per-element arithmetic), including a 2-token append, a row whose
    append lands on a fresh page and a row with nothing to append."""
    gen = torch.Generator().manual_seed(21)
    B = len(qo)
    lens_after = [17, 33, 16, 300]  # tokens cached after the append
    pages = [(n + 15) // 16 for n in lens_after]
    num_pages = sum(pages) + 5
    perm = torch.randperm(num_pages, generator=gen)[:sum(pages)].to(torch.int32)
    indptr = torch.tensor([0] + list(torch.cumsum(torch.tensor(pages), 0)), dtype=torch.int32)
    last = torch.tensor([n - (p - 1) * 16 for n, p in zip(lens_after, pages)], dtype=torch.int32)
    app = torch.tensor([0] + list(torch.cumsum(torch.tensor(qo), 0)), dtype=torch.int32)
    offsets = torch.tensor([n - a for n, a in zip(lens_after, qo)], dtype=torch.int32)
    nnz = sum(qo)
    pad = 2 if misalign else 0
    qk = torch.randn(nnz, pad + (hq + hkv) * 128, generator=gen).to(dtype).to(DEV)
    q, k = qk[:, pad:].split([hq * 128, hkv * 128], dim=-1)
    v = torch.randn(nnz, hkv * 128, generator=gen).to(dtype).to(DEV)
    q, k, v = q.view(nnz, hq, 128), k.view(nnz, hkv, 128), v.view(nnz, hkv, 128)
    cache = torch.randn(num_pages, 2, 16, hkv, 128, generator=gen).to(dtype).to(DEV)
    cache2 = cache.clone()
    p = dict(rope_scale=8.0 if llama31 else 1.0, rope_theta=5e5)
    if llama31:
        p.update(low_freq_factor=1.0, high_freq_factor=4.0, old_context_len=8192.0)
    g = lambda t: t.to(DEV)
    q1, k1 = K.rope(q, k, g(app), g(offsets), **p)
    K.append_kv(k1, v, g(app), cache, g(perm), g(indptr), g(last))
    q2 = K.rope_append(q, k, v, g(app), g(offsets), cache2, g(perm), g(indptr), g(last), **p)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2)
    assert torch.equal(cache, cache2)


@pytest.mark.parametrize("hq,hkv,dtype", [(32, 8, torch.bfloat16), (28, 4, torch.bfloat16), (8, 8, torch.float16),
                                          (40, 8, torch.bfloat16), (16, 2, torch.float16)])
def test_paged_prefill_matches_oracle(hq, hkv, dtype):
    """Causal prefill (several query tokens per row) against the oracle: ragged rows, a row
    with one query token, a prompt longer than one block of waves, shuffled pages."""
    kv_lens = [70, 16, 300, 33]
    qo = [37, 1, 300, 9]
    c = make_case(batch=4, hq=hq, hkv=hkv, kv_lens=kv_lens, seed=31, page_order="randperm", k=4, L=2,
                  dtype=dtype)
    gen = torch.Generator().manual_seed(32)
    nnz = sum(qo)
    q = torch.randn(nnz, hq, 128, generator=gen).to(dtype)
    qo_indptr = torch.tensor([0] + list(torch.cumsum(torch.tensor(qo), 0)), dtype=torch.int32)
    g = gpu(c)
    lse = torch.empty(nnz, hq, device=DEV)
    o = K.paged_prefill(q.to(DEV), g.kv_cache, qo_indptr.to(DEV), g.kv_indptr, g.kv_indices, g.kv_last_page_len,
                        max_qo_len=max(qo), lse=lse)
    torch.cuda.synchronize()
    o_ref, lse_ref = O.paged_prefill_attention(q, qo_indptr, c.kv_cache, c.kv_indptr, c.kv_indices,
                                               c.kv_last_page_len, c.sm_scale)
    assert_attn_close(o, o_ref, f"prefill G={hq // hkv}")
    assert torch.allclose(lse.cpu(), lse_ref, atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("seed", range(8))
def test_paged_prefill_random_shapes(seed):
    """Seeded random prefill shapes against the oracle: group sizes 1-8, 1-8 kv heads, 1-6 rows
    of 1-700 cached tokens with prompts of 1..kv_len tokens (chunked prefill: the prompt's first
    token sits past the row's start), trailing empty pages and both dtypes; o and lse."""
    g = torch.Generator().manual_seed(2000 + seed)
    ri = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=g))
    G, hkv = ri(1, 8), [1, 2, 4, 8][ri(0, 3)]
    hq = G * hkv
    B = ri(1, 6)
    kv_lens = [ri(1, 700) for _ in range(B)]
    qo = [ri(1, n) for n in kv_lens]
    dtype = [torch.bfloat16, torch.float16][seed % 2]
    c = make_case(batch=B, hq=hq, hkv=hkv, kv_lens=kv_lens, seed=50 + seed, page_order="randperm", k=4, L=2,
                  dtype=dtype, trailing_empty_page=bool(seed % 3 == 0))
    q = torch.randn(sum(qo), hq, 128, generator=g).to(dtype)
    qo_indptr = torch.tensor([0] + list(torch.cumsum(torch.tensor(qo), 0)), dtype=torch.int32)
    gc = gpu(c)
    lse = torch.empty(sum(qo), hq, device=DEV)
    o = K.paged_prefill(q.to(DEV), gc.kv_cache, qo_indptr.to(DEV), gc.kv_indptr, gc.kv_indices,
                        gc.kv_last_page_len, max_qo_len=max(qo), lse=lse)
    torch.cuda.synchronize()
    o_ref, lse_ref = O.paged_prefill_attention(q, qo_indptr, c.kv_cache, c.kv_indptr, c.kv_indices,
                                               c.kv_last_page_len, c.sm_scale)
    assert_attn_close(o, o_ref, f"random prefill seed {seed}: G={G} hkv={hkv} kv={kv_lens} qo={qo}")
    assert torch.allclose(lse.cpu(), lse_ref, atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_paged_prefill_long_rows_growing_scores(sign):
    """Prompts of 1100 and 300 tokens (more than 64 pages: the page-id window moves), K scaled
    up along each row so the running maximum keeps growing (the accumulators are rescaled many
    times), and a negative scale (q's signs flipped in the kernel): o and lse against the oracle.
    The scores are peaked, so o is close to single V rows; V is halved (exact) so that o's own
    bf16 rounding stays well inside the 2e-2 bar."""
    hq, hkv = 32, 8
    kv_lens, qo = [1100, 700], [1100, 300]
    c = make_case(batch=2, hq=hq, hkv=hkv, kv_lens=kv_lens, seed=33, page_order="randperm", k=4, L=2,
                  dtype=torch.bfloat16)
    cache = c.kv_cache.float()
    for b, n in enumerate(kv_lens):
        pages = c.kv_indices[int(c.kv_indptr[b]):int(c.kv_indptr[b + 1])].long()
        ramp = 1.0 + torch.arange(len(pages) * 16, dtype=torch.float32).view(-1, 16) / 48.0
        cache[pages, 0] *= ramp[:, :, None, None]
        cache[pages, 1] *= 0.5
    cache = cache.to(torch.bfloat16)
    gen = torch.Generator().manual_seed(34)
    q = torch.randn(sum(qo), hq, 128, generator=gen).to(torch.bfloat16)
    qo_indptr = torch.tensor([0, qo[0], qo[0] + qo[1]], dtype=torch.int32)
    scale = sign / 128 ** 0.5
    lse = torch.empty(sum(qo), hq, device=DEV)
    o = K.paged_prefill(q.to(DEV), cache.to(DEV), qo_indptr.to(DEV), c.kv_indptr.to(DEV), c.kv_indices.to(DEV),
                        c.kv_last_page_len.to(DEV), max_qo_len=max(qo), sm_scale=scale, lse=lse)
    torch.cuda.synchronize()
    o_ref, lse_ref = O.paged_prefill_attention(q, qo_indptr, cache, c.kv_indptr, c.kv_indices,
                                               c.kv_last_page_len, scale)
    assert_attn_close(o, o_ref, f"long prefill, scale sign {sign}")
    assert torch.allclose(lse.cpu(), lse_ref, atol=2e-3, rtol=1e-4)


@pytest.mark.parametrize("hq,hkv,dtype,batch,max_len", [
    (32, 8, torch.bfloat16, 32, 1500),    # config-3 heads, 256 (row, kv head) blocks
    (40, 8, torch.bfloat16, 32, 700),     # G = 5
    (16, 2, torch.float16, 128, 400),     # G = 8
    (32, 8, torch.bfloat16, 32, 9500),    # 594 pages: near the LDS limit with the append slots
])
def test_planner_scores_on_chip_match_dump_path_and_oracle(hq, hkv, dtype, batch, max_len):
    """The planner without a dump (delta_paged_decode_scores[_append]): o and lse against the
    dump launch and the oracle, page scores against delta_page_scores_from_logits of that dump
    and the oracle's del3_legacy_softmax (1e-4 relative), and with the fused append the cache
    bytes equal delta_rope_append's and o equals the fused dump launch's to rounding.  Ragged
    rows: one page, a partial last page, a row at max_len."""
    gen = torch.Generator().manual_seed(51)
    lens = torch.randint(1, max_len, (batch,), generator=gen).tolist()
    lens[0], lens[1], lens[2] = 1, 17, max_len
    c = make_case(batch=batch, hq=hq, hkv=hkv, kv_lens=lens, seed=52, page_order="randperm", k=4, L=2,
                  dtype=dtype)
    g = gpu(c)
    B, mp = batch, c.max_pages
    assert K.paged_decode_scores_supported(B, hq, hkv, mp, True)
    lse_d = torch.empty(B, hq, device=DEV)
    dump = torch.full((B, hq, mp * 16), float("-inf"), device=DEV)
    o_d = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, max_pages_per_row=mp,
                         lse=lse_d, logits_dump=dump)
    s_d = K.page_scores_from_logits(dump, g.kv_indptr, g.kv_last_page_len, mp, lse=lse_d)
    lse = torch.empty(B, hq, device=DEV)
    o, s = K.paged_decode_scores(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len,
                                 max_pages_per_row=mp, lse=lse)
    torch.cuda.synchronize()
    assert_attn_close(o, o_d.float(), "on-chip planner vs dump launch")
    assert torch.allclose(lse, lse_d, atol=1e-4, rtol=1e-5)
    rel = ((s - s_d).abs() / s_d.abs().clamp_min(1e-30)).max().item()
    assert rel < 1e-5, rel
    o_ref, lse_ref = O.paged_decode_attention(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len,
                                              c.sm_scale)
    assert_attn_close(o, o_ref, "on-chip planner vs oracle")
    assert torch.allclose(lse.cpu(), lse_ref, atol=1e-4, rtol=1e-5)
    x = O.dump_logits(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, c.sm_scale, mp * 16)
    want = O.legacy_softmax_page_scores(x, B, mp, compute_dtype=torch.float64).double()
    got = s.cpu().double()
    assert ((got - want).abs() / want.abs().clamp_min(1e-30)).max().item() < 1e-4
    pages = (c.kv_indptr[1:] - c.kv_indptr[:-1]).tolist()
    for b in range(B):
        if pages[b] < mp:  # a row's pages past its end score 0
            assert got[b, pages[b]:].abs().max().item() == 0.0

    # fused RoPE + append: cache bytes as delta_rope_append, o and scores as the fused dump launch
    kn = torch.randn(B, hkv, 128, generator=gen).to(dtype).to(DEV)
    vn = torch.randn(B, hkv, 128, generator=gen).to(dtype).to(DEV)
    offsets = torch.tensor([n - 1 for n in lens], dtype=torch.int32, device=DEV)
    ap = K.DecodeAppend(kn, vn, offsets, g.kv_indptr, g.kv_indices, rope_scale=8.0, rope_theta=5e5,
                        low_freq_factor=1.0, high_freq_factor=4.0, old_context_len=8192.0)
    c1, c2 = g.kv_cache.clone(), g.kv_cache.clone()
    lse1 = torch.empty(B, hq, device=DEV)
    dump1 = torch.full((B, hq, mp * 16), float("-inf"), device=DEV)
    o1 = K.paged_decode(g.q, c1, g.kv_indptr, g.kv_indices, g.kv_last_page_len, max_pages_per_row=mp, lse=lse1,
                        logits_dump=dump1, append=ap)
    s1 = K.page_scores_from_logits(dump1, g.kv_indptr, g.kv_last_page_len, mp, lse=lse1)
    o2, s2 = K.paged_decode_scores(g.q, c2, g.kv_indptr, g.kv_indices, g.kv_last_page_len, max_pages_per_row=mp,
                                   append=ap)
    torch.cuda.synchronize()
    assert torch.equal(c1, c2)
    assert_attn_close(o2, o1.float(), "fused on-chip planner vs fused dump launch")
    assert ((s2 - s1).abs() / s1.abs().clamp_min(1e-30)).max().item() < 1e-5


def test_planner_scores_on_chip_refuses_unsupported_shapes():
    """Fewer than 256 (row, kv head) blocks, or rows whose logits do not fit in LDS: a clear
    error (the caller keeps the dump path)."""
    c = make_case(batch=4, hq=32, hkv=8, kv_lens=[300] * 4, seed=53, k=4, L=2)
    g = gpu(c)
    assert not K.paged_decode_scores_supported(4, 32, 8, c.max_pages, False)
    with pytest.raises(_lib.DeltaHipError, match="does not fit the on-chip planner"):
        K.paged_decode_scores(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len,
                              max_pages_per_row=c.max_pages)
    assert not K.paged_decode_scores_supported(32, 32, 8, 700, False)


@pytest.mark.parametrize("hq,hkv,dtype,llama31,batch", [
    (32, 8, torch.bfloat16, False, 6),    # page-major split launches
    (32, 8, torch.bfloat16, True, 36),    # head-major subset (36 rows x 8 kv heads)
    (28, 4, torch.float16, True, 5),      # G = 7
    (16, 2, torch.bfloat16, False, 3),    # G = 8
])
def test_decode_append_equals_rope_append_then_decode(hq, hkv, dtype, llama31, batch):
    """The fused decode launch (RoPE + append + attention) against delta_rope_append followed by
    the plain attention: o, lse, logits dump and every cache byte identical -- full, planner
    and subset kernels; rows whose new token opens a page, fills one (trailing empty page) or
    lands on a page the subset does not hold."""
    gen = torch.Generator().manual_seed(41)
    lens = [1 + (97 * i + 31) % 700 for i in range(batch)]
    lens[0] = 16   # new token fills page 0; trailing empty page
    lens[1] = 17   # new token opens page 1
    c = make_case(batch=batch, hq=hq, hkv=hkv, kv_lens=lens, seed=42, page_order="randperm", k=4, L=2,
                  trailing_empty_page=True, dtype=dtype)
    g = gpu(c)
    B = batch
    mp = c.max_pages
    q = torch.randn(B, hq, 128, generator=gen).to(dtype).to(DEV)
    kn = torch.randn(B, hkv, 128, generator=gen).to(dtype).to(DEV)
    vn = torch.randn(B, hkv, 128, generator=gen).to(dtype).to(DEV)
    kv_len = torch.tensor(lens, dtype=torch.int32)
    offsets = (kv_len - 1).to(DEV)
    app = torch.arange(B + 1, dtype=torch.int32, device=DEV)
    p = dict(rope_scale=8.0 if llama31 else 1.0, rope_theta=5e5)
    if llama31:
        p.update(low_freq_factor=1.0, high_freq_factor=4.0, old_context_len=8192.0)
    ap = K.DecodeAppend(kn, vn, offsets, g.kv_indptr, g.kv_indices, **p)

    def unfused(cache, **kw):
        qr = K.rope_append(q, kn, vn, app, offsets, cache, g.kv_indices, g.kv_indptr, g.kv_last_page_len, **p)
        return K.paged_decode(qr, cache, **kw)

    # full + planner (dump, lse)
    for dump_on in (False, True):
        outs = []
        for fused in (False, True):
            cache = g.kv_cache.clone()
            lse = torch.full((B, hq), 7.0, device=DEV)
            dump = torch.full((B, hq, mp * 16), 12345.0, device=DEV) if dump_on else None
            kw = dict(kv_indptr=g.kv_indptr, kv_indices=g.kv_indices, kv_last_page_len=g.kv_last_page_len,
                      max_pages_per_row=mp, lse=lse, logits_dump=dump)
            o = K.paged_decode(q, cache, append=ap, **kw) if fused else unfused(cache, **kw)
            outs.append((o, lse, dump, cache))
        torch.cuda.synchronize()
        (o1, l1, d1, c1), (o2, l2, d2, c2) = outs
        assert torch.equal(o1, o2) and torch.equal(l1, l2) and torch.equal(c1, c2)
        if dump_on:
            assert torch.equal(d1, d2)

    # subset: every row keeps its first and last pages; row 0's new token sits on page 0
    # (the last page is the empty trailing one), so drop page 0 there: the token is appended
    # but not attended, as in the two-call path.
    counts = (c.kv_indptr[1:] - c.kv_indptr[:-1]).tolist()
    sub, sptr = [], [0]
    for b in range(B):
        row = c.kv_indices[int(c.kv_indptr[b]):int(c.kv_indptr[b + 1])].tolist()
        keep = sorted({0, counts[b] - 1, counts[b] // 2}) if counts[b] > 1 else [0]
        if b == 0:
            keep = [j for j in keep if j != 0]
        sub += [row[j] for j in keep]
        sptr.append(len(sub))
    s_idx = torch.tensor(sub, dtype=torch.int32, device=DEV)
    s_ptr = torch.tensor(sptr, dtype=torch.int32, device=DEV)
    outs = []
    for fused in (False, True):
        cache = g.kv_cache.clone()
        kw = dict(kv_indptr=s_ptr, kv_indices=s_idx, kv_last_page_len=g.kv_last_page_len, max_pages_per_row=3,
                  subset=True)
        o = K.paged_decode(q, cache, append=ap, **kw) if fused else unfused(cache, **kw)
        outs.append((o, cache))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,Kd,bias", [(32, 4096, 4096, False), (32, 6144, 4096, True), (17, 4096, 14336, False),
                                        (32, 28672, 4096, False), (1, 64, 64, True), (32, 128256, 1024, False),
                                        (9, 192, 640, True)])
def test_gemm_rows32_matches_fp32_reference(dtype, M, N, Kd, bias):
    """delta_gemm_rows32 (x staged in LDS, K split across the grid) against x.float() @ w.float().T
    (+ b): the fp32 partials sum to the product; the unsplit output is it rounded once."""
    gen = torch.Generator(device=DEV).manual_seed(M * 3 + N + Kd)
    x = torch.randn(M, Kd, generator=gen, device=DEV).to(dtype)
    w = (torch.randn(N, Kd, generator=gen, device=DEV) * 0.05).to(dtype)
    b = (torch.randn(N, generator=gen, device=DEV) * 0.1).to(dtype) if bias else None
    S = K.gemm_rows32_splits(M, N, Kd)
    r = K.gemm_rows32(x, w, b)
    r2 = K.gemm_rows32(x, w, b)
    torch.cuda.synchronize()
    ref = x.float() @ w.float().T + (b.float() if bias else 0.0)
    mag = x.float().abs() @ w.float().abs().T
    if S == 1:
        assert r.dtype == dtype and tuple(r.shape) == (M, N)
        err = (r.float() - ref).abs()
        assert torch.all(err <= torch.finfo(dtype).eps * ref.abs() + 1e-5 * mag + 1e-6), f"max err {err.max().item()}"
    else:
        assert r.dtype == torch.float32 and tuple(r.shape) == (S, M, N)
        err = (r.sum(0) - ref).abs()
        assert torch.all(err <= 1e-5 * mag + 1e-6), f"max err {err.max().item()}"
    assert torch.equal(r, r2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_add_rmsnorm_over_partials_equals_rounded_sum(dtype):
    """delta_add_rmsnorm_partials (the norm after a split-K projection) gives bit for bit what
    delta_add_rmsnorm gives on the partials' sum (split order) rounded to the dtype."""
    gen = torch.Generator(device=DEV).manual_seed(11)
    M, N, Kd = 32, 4096, 4096
    xin = torch.randn(M, Kd, generator=gen, device=DEV).to(dtype)
    w = (torch.randn(N, Kd, generator=gen, device=DEV) * 0.02).to(dtype)
    x = torch.randn(M, N, generator=gen, device=DEV).to(dtype)
    nw = (1 + 0.1 * torch.randn(N, generator=gen, device=DEV)).to(dtype)
    parts = K.gemm_rows32(xin, w)
    assert parts.dtype == torch.float32 and parts.shape[0] > 1
    h, y = K.add_rmsnorm(x, parts, nw, 1e-5)
    r = parts[0].clone()
    for s in range(1, parts.shape[0]):
        r += parts[s]
    h2, y2 = K.add_rmsnorm(x, r.to(dtype), nw, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(h, h2) and torch.equal(y, y2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,inter,Kd", [(32, 14336, 4096), (13, 1024, 640), (32, 18944, 3584)])
def test_gemm_rows32_silu_equals_gemm_then_silu_mul(dtype, M, inter, Kd):
    """The fused gate/up GEMM + SiLU-mul writes the bits of delta_gemm_rows32 (unsplit, the same
    per-column sums) followed by delta_silu_mul."""
    gen = torch.Generator(device=DEV).manual_seed(M + inter + Kd)
    x = torch.randn(M, Kd, generator=gen, device=DEV).to(dtype)
    w13 = (torch.randn(2 * inter, Kd, generator=gen, device=DEV) * 0.03).to(dtype)
    fused = K.gemm_rows32_silu(x, w13)
    gu = K.gemm_rows32(x, w13) if K.gemm_rows32_splits(M, 2 * inter, Kd) == 1 else None
    ref = K.silu_mul((x.float() @ w13.float().T).to(dtype))
    torch.cuda.synchronize()
    if gu is not None:
        assert torch.equal(fused, K.silu_mul(gu))
    err = (fused.float() - ref.float()).abs()
    assert err.max().item() <= 0.02 * ref.float().abs().max().item() + 1e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,inter,Kd", [(4, 18944, 3584), (1, 64, 128), (8, 14336, 4096), (3, 1040, 640)])
def test_gemm_skinny_silu_equals_gemm_then_silu_mul(dtype, M, inter, Kd):
    """The fused gate/up GEMM + SiLU-mul at <= 8 rows writes the bits of delta_gemm_skinny over the
    merged weight followed by delta_silu_mul."""
    gen = torch.Generator(device=DEV).manual_seed(M * 5 + inter + Kd)
    x = torch.randn(M, Kd, generator=gen, device=DEV).to(dtype)
    w13 = (torch.randn(2 * inter, Kd, generator=gen, device=DEV) * 0.03).to(dtype)
    fused = K.gemm_skinny_silu(x, w13)
    two = K.silu_mul(K.gemm_skinny(x, w13))
    torch.cuda.synchronize()
    assert torch.equal(fused, two)


@pytest.mark.parametrize("ragged", [False, True])
def test_page_score_on_chip_matches_oracle_and_dump_path(ragged):
    """The K-only scorer without a dump (the row's logits kept in LDS, per-(kv head, token) maxima,
    then page sums) against the oracle's del3_legacy_softmax scores (1e-4 relative) and the dump
    path on the same inputs.  B * Hkv = 256 (row, head) blocks, rows of up to 300 pages."""
    lens = [300 * 16] * 32 if not ragged else [16 * (1 + (37 * i) % 300) + (i % 16) for i in range(32)]
    c = make_case(batch=32, hq=32, hkv=8, kv_lens=lens, seed=5, page_order="randperm", k=4, L=2,
                  trailing_empty_page=ragged)
    g = gpu(c)
    mp = c.max_pages
    assert K._lib.query("delta_page_score_needs_dump", 32, 32, 8, mp) == 0
    s_chip = K.page_score(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, mp)
    dump = torch.empty((32, 32, mp * 16), device=DEV)
    s_dump = K.page_score(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, mp, logits_dump=dump)
    torch.cuda.synchronize()
    x = O.dump_logits(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, c.sm_scale, mp * 16)
    ref = O.legacy_softmax_page_scores(x, 32, mp, compute_dtype=torch.float64).double()
    for what, s in (("on chip", s_chip), ("dump", s_dump)):
        s = s.cpu().double()
        rel = (s - ref).abs() / ref.abs().clamp_min(1e-30)
        rel[ref == 0] = s[ref == 0].abs()
        assert rel.max().item() < 1e-4, f"{what}: rel err {rel.max().item()}"
