"""Seeded random shapes through the whole decode chain on the GPU, against the oracle.

Each case draws a dtype, the kv-head count and group size (1..8), a batch of ragged rows
(1..1200 tokens, some ending on a page boundary with a trailing empty page), a page order, a
budget and L, then checks: the planner launch (attention within 2e-2 abs / cos > 0.999, lse,
logits dump within 1e-4 * (1 + |x|)), the page scores (1e-4 relative), the selection (bit-exact
against the oracle fed the same scores), the sparse attention over that selection, and the
fused RoPE + append launch against the two-step path (bit-identical).
"""
import random

import pytest
import torch

from delta_amd import kernels as K
from delta_amd.workloads import make_case
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def close_attn(got, want, what):
    got, want = got.float().cpu(), want.float().cpu()
    err = (got - want).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(got.flatten(), want.flatten(), dim=0).item()
    assert err <= 2e-2 and cos > 0.999, f"{what}: err {err} cos {cos}"


def draw(seed, large=False):
    r = random.Random(seed)
    hkv = r.choice([1, 2, 4, 8])
    G = r.randint(1, 8)
    # large: more (row, kv head) blocks than CUs, so unsplit launches take the balanced row order
    lo = -(-257 // hkv)
    B = r.randint(lo, max(200, lo + 40)) if large else r.randint(1, 40)
    lens = []
    for _ in range(B):
        n = r.randint(1, 1200)
        if r.random() < 0.2:
            n = 16 * max(1, n // 16)
        lens.append(n)
    return dict(dtype=r.choice([torch.bfloat16, torch.float16]), hkv=hkv, hq=hkv * G, batch=B, kv_lens=lens,
                page_order=r.choice(["randperm", "shuffle", "identity"]), trailing_empty_page=r.random() < 0.5,
                k_frac=r.random(), L=r.randint(0, 8), seed=seed)


@pytest.mark.parametrize("seed", range(16))
def test_random_decode_chain(seed):
    _decode_chain(draw(1000 + seed), seed)


@pytest.mark.parametrize("seed", range(6))
def test_random_decode_chain_large_batch(seed):
    """The same chain with 257 to 1600 (row, kv head) blocks: the planner, full and subset
    launches take the balanced row order wherever their rows reach 32 pages."""
    _decode_chain(draw(3000 + seed, large=True), 3000 + seed)


def _decode_chain(p, seed):
    c = make_case(batch=p["batch"], hq=p["hq"], hkv=p["hkv"], kv_lens=p["kv_lens"], dtype=p["dtype"], seed=p["seed"],
                  page_order=p["page_order"], trailing_empty_page=p["trailing_empty_page"], k=1, L=p["L"])
    g = c.to(DEV)
    B, hq = c.q.shape[:2]
    mp = c.max_pages
    k = max(1, int(p["k_frac"] * mp))
    L = min(p["L"], k)
    what = f"seed {seed}: B={B} hq={hq} hkv={p['hkv']} {p['dtype']} k={k} L={L}"

    dump = torch.full((B, hq, mp * 16), 12345.0, device=DEV)
    lse = torch.empty(B, hq, device=DEV)
    o = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, max_pages_per_row=mp,
                       lse=lse, logits_dump=dump)
    s = K.page_scores_from_logits(dump, g.kv_indptr, g.kv_last_page_len, mp, lse=lse)
    idx, ip = K.select_pages(s, g.kv_indptr, g.block_table, k, L)
    o_sp = K.paged_decode(g.q, g.kv_cache, ip, idx, g.kv_last_page_len, max_pages_per_row=k, subset=True)
    torch.cuda.synchronize()

    o_ref, lse_ref = O.paged_decode_attention(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len,
                                              c.sm_scale)
    close_attn(o, o_ref, what + " planner attention")
    assert torch.allclose(lse.cpu(), lse_ref, atol=1e-3, rtol=1e-4), what
    x = O.dump_logits(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, c.sm_scale, mp * 16)
    d = dump.cpu()
    valid = torch.isfinite(x)
    assert ((d[valid] - x[valid]).abs() / (1 + x[valid].abs())).max().item() < 1e-4, what
    ref_s = O.legacy_softmax_page_scores(x, B, mp, compute_dtype=torch.float64).double()
    got_s = s.cpu().double()
    rel = (got_s - ref_s).abs() / ref_s.abs().clamp_min(1e-30)
    rel[ref_s == 0] = got_s[ref_s == 0].abs()
    assert rel.max().item() < 1e-4, what + f" scores rel {rel.max().item()}"

    counts = c.kv_indptr[1:] - c.kv_indptr[:-1]
    want_i, want_p = O.select_pages(s.cpu(), counts, c.block_table, k, L)
    assert ip.cpu().tolist() == want_p.tolist(), what
    assert idx[:int(want_p[-1])].cpu().tolist() == want_i.tolist(), what
    o_sp_ref, _ = O.paged_decode_attention(c.q, c.kv_cache, want_p, want_i, c.kv_last_page_len, c.sm_scale)
    close_attn(o_sp, o_sp_ref, what + " sparse attention")

    # Fused RoPE + append (the rows' last token is the new one) against the two-step path.
    gen = torch.Generator().manual_seed(seed)
    kn = torch.randn(B, p["hkv"], 128, generator=gen).to(p["dtype"]).to(DEV)
    vn = torch.randn(B, p["hkv"], 128, generator=gen).to(p["dtype"]).to(DEV)
    offsets = torch.tensor([n - 1 for n in p["kv_lens"]], dtype=torch.int32, device=DEV)
    app = torch.arange(B + 1, dtype=torch.int32, device=DEV)
    rp = dict(rope_scale=1.0, rope_theta=1e4)
    outs = []
    for fused in (False, True):
        cache = g.kv_cache.clone()
        if fused:
            ap = K.DecodeAppend(kn, vn, offsets, g.kv_indptr, g.kv_indices, **rp)
            oo = K.paged_decode(g.q, cache, ip, idx, g.kv_last_page_len, max_pages_per_row=k, subset=True, append=ap)
        else:
            qr = K.rope_append(g.q, kn, vn, app, offsets, cache, g.kv_indices, g.kv_indptr, g.kv_last_page_len, **rp)
            oo = K.paged_decode(qr, cache, ip, idx, g.kv_last_page_len, max_pages_per_row=k, subset=True)
        outs.append((oo, cache))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1]), what + " fused append"


@pytest.mark.parametrize("seed", range(8))
def test_random_planner_on_chip(seed):
    """The planner without a dump (delta_paged_decode_scores) on seeded random shapes with
    >= 256 (row, kv head) blocks: o and lse against the dump launch and the oracle, page scores
    against delta_page_scores_from_logits of that dump (1e-5 relative) and the oracle (1e-4),
    the selection from both score routes identical."""
    r = random.Random(2000 + seed)
    hkv = r.choice([2, 4, 8])
    G = r.randint(1, 8)
    B = -(-256 // hkv) + r.randint(0, 16)
    lens = [r.randint(1, 1200) for _ in range(B)]
    dtype = r.choice([torch.bfloat16, torch.float16])
    c = make_case(batch=B, hq=hkv * G, hkv=hkv, kv_lens=lens, dtype=dtype, seed=2000 + seed,
                  page_order=r.choice(["randperm", "shuffle"]), trailing_empty_page=r.random() < 0.5, k=1, L=2)
    g = c.to(DEV)
    hq, mp = hkv * G, c.max_pages
    what = f"seed {seed}: B={B} hq={hq} hkv={hkv} {dtype} pages {mp}"
    assert K.paged_decode_scores_supported(B, hq, hkv, mp, False), what
    dump = torch.full((B, hq, mp * 16), float("-inf"), device=DEV)
    lse_d = torch.empty(B, hq, device=DEV)
    o_d = K.paged_decode(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len, max_pages_per_row=mp,
                         lse=lse_d, logits_dump=dump)
    s_d = K.page_scores_from_logits(dump, g.kv_indptr, g.kv_last_page_len, mp, lse=lse_d)
    lse = torch.empty(B, hq, device=DEV)
    o, s = K.paged_decode_scores(g.q, g.kv_cache, g.kv_indptr, g.kv_indices, g.kv_last_page_len,
                                 max_pages_per_row=mp, lse=lse)
    k = max(1, mp // 3)
    i1, p1 = K.select_pages(s, g.kv_indptr, g.block_table, k, 2)
    i0, p0 = K.select_pages(s_d, g.kv_indptr, g.block_table, k, 2)
    torch.cuda.synchronize()
    close_attn(o, o_d, what + " vs dump launch")
    assert torch.allclose(lse, lse_d, atol=1e-4, rtol=1e-5), what
    rel = ((s - s_d).abs() / s_d.abs().clamp_min(1e-30)).max().item()
    assert rel < 1e-5, what + f" scores vs dump path {rel}"
    o_ref, lse_ref = O.paged_decode_attention(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len,
                                              c.sm_scale)
    close_attn(o, o_ref, what + " vs oracle")
    x = O.dump_logits(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, c.sm_scale, mp * 16)
    ref_s = O.legacy_softmax_page_scores(x, B, mp, compute_dtype=torch.float64).double()
    got = s.cpu().double()
    rel = (got - ref_s).abs() / ref_s.abs().clamp_min(1e-30)
    rel[ref_s == 0] = got[ref_s == 0].abs()
    assert rel.max().item() < 1e-4, what + f" scores vs oracle {rel.max().item()}"
    assert torch.equal(p1, p0), what
    n = int(p1[-1].item())
    if not torch.equal(i1[:n], i0[:n]):  # only keys equal to within the scores' 1e-5 may swap
        sc = s_d.cpu()
        for b in range(B):
            a = i1[int(p1[b]):int(p1[b + 1])].tolist()
            z = i0[int(p0[b]):int(p0[b + 1])].tolist()
            if a != z:
                bt = c.block_table[b].tolist()
                vals = [float(sc[b, bt.index(pg)]) for pg in set(a) ^ set(z)]
                assert max(vals) - min(vals) <= 1e-5 * max(abs(v) for v in vals), what + f" row {b}"
