"""The allocation-free decode entry point (delta_paged_decode_noalloc, static device scratch)
against delta_paged_decode with a caller workspace, through the C ABI: bit-identical outputs,
lse and logits dump on two calls in a row (the second smaller), for every split plan that uses
the scratch (page-major planner splits, head-major small-batch splits of one-wave and four-wave
blocks); the same call captured in a hipGraph and replayed; and a clear refusal of a shape whose
split partials exceed the static scratch."""
import math

import pytest
import torch

from delta_amd import _lib
from delta_amd import kernels as K
from delta_amd.workloads import make_case

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _args(c, mp, out, lse, dump):
    B, hq = c.q.shape[:2]
    return [c.q.data_ptr(), c.q.stride(0), c.q.stride(1), c.kv_cache.data_ptr(), c.kv_cache.shape[0],
            c.kv_indptr.data_ptr(), c.kv_indices.data_ptr(), c.kv_indices.numel(), c.kv_last_page_len.data_ptr(),
            out.data_ptr(), out.stride(0), out.stride(1), lse.data_ptr(),
            None if dump is None else dump.data_ptr(), 0 if dump is None else dump.stride(0),
            0 if dump is None else dump.stride(1), B, hq, c.kv_cache.shape[3], 128, _lib.DELTA_BF16,
            1 / math.sqrt(128), mp]


def _buffers(c, with_dump):
    B, hq = c.q.shape[:2]
    out = torch.full_like(c.q, 3.0)
    lse = torch.full((B, hq), 5.0, device=DEV)
    dump = torch.full((B, hq, c.max_pages * 16), 7.0, device=DEV) if with_dump else None
    return out, lse, dump


def _workspace_call(c, out, lse, dump):
    B, hq = c.q.shape[:2]
    need = K.decode_workspace_bytes(B, hq, c.kv_cache.shape[3], c.max_pages)
    assert need > 0, "the case must run split, so the scratch is used"
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    _lib.call("delta_paged_decode", *_args(c, c.max_pages, out, lse, dump), ws.data_ptr(), need,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()


def _run(c, noalloc, with_dump=True):
    out, lse, dump = _buffers(c, with_dump)
    if noalloc:
        _lib.call("delta_paged_decode_noalloc", *_args(c, c.max_pages, out, lse, dump),
                  torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
    else:
        _workspace_call(c, out, lse, dump)
    return (out, lse) if dump is None else (out, lse, dump)


def test_noalloc_entry_point_matches_workspace_entry_point():
    cases = [
        # a 16-row planner launch at the config-3 row shape (page-major split, logits dump), then a
        # smaller ragged one
        make_case(batch=16, hq=32, hkv=8, kv_lens=8192, dtype=torch.bfloat16, seed=21, page_order="shuffle",
                  device=DEV),
        make_case(batch=3, hq=28, hkv=4, kv_lens=[5000, 777, 12000], dtype=torch.bfloat16, seed=22, device=DEV),
    ]
    for c in cases:
        want = _run(c, noalloc=False)
        got = _run(c, noalloc=True)
        for name, a, b in zip(("o", "lse", "dump"), got, want):
            assert torch.equal(a, b), f"B={c.q.shape[0]}: {name} differs from delta_paged_decode"


def test_noalloc_small_batch_split_plans_match_workspace_entry_point():
    """Attention launches of fewer than 256 (row, kv head) pairs split head-major, and their
    partials reach the scratch differently: B = 8, Hkv = 8, 128 pages per row runs one-wave
    blocks of 16 splits storing partials from registers; then (the scratch holding the first
    call's partials) B = 4, Hkv = 4, 4096 pages per row runs four-wave blocks, one block per
    (row, split)."""
    cases = [
        make_case(batch=8, hq=32, hkv=8, kv_lens=2048, dtype=torch.bfloat16, seed=24, page_order="shuffle",
                  device=DEV),
        make_case(batch=4, hq=28, hkv=4, kv_lens=[65536, 60001, 65536, 33333], dtype=torch.bfloat16, seed=25,
                  page_order="shuffle", device=DEV),
    ]
    for c in cases:
        want = _run(c, noalloc=False, with_dump=False)
        got = _run(c, noalloc=True, with_dump=False)
        for name, a, b in zip(("o", "lse"), got, want):
            assert torch.equal(a, b), f"B={c.q.shape[0]}: {name} differs from delta_paged_decode"


def test_noalloc_entry_point_in_a_captured_graph():
    """The documented use: delta_paged_decode_noalloc recorded in a hipGraph (no allocation, no
    memset inside) and replayed.  Two replays equal the eager workspace call bit for bit; a third,
    after new q values are copied into the captured q buffer, equals the workspace call on those
    values (the graph reads its inputs live)."""
    c = make_case(batch=8, hq=32, hkv=8, kv_lens=[2048, 1000, 3000, 17, 2048, 2500, 999, 1600],
                  dtype=torch.bfloat16, seed=26, page_order="shuffle", device=DEV)
    want = _run(c, noalloc=False, with_dump=False)
    out, lse, _ = _buffers(c, with_dump=False)
    args = _args(c, c.max_pages, out, lse, None)  # read on the host before the capture
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # first call outside the capture: the scratch address lookup
        _lib.call("delta_paged_decode_noalloc", *args, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    # captured under inference mode, as the engine captures its step: an earlier test may have
    # created the CUDA generator's state there, which capture_begin then updates in place
    with torch.inference_mode(), torch.cuda.graph(g):
        _lib.call("delta_paged_decode_noalloc", *args, torch.cuda.current_stream().cuda_stream)
    for i in range(2):
        out.fill_(3.0)
        lse.fill_(5.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want[0]) and torch.equal(lse, want[1]), f"replay {i} differs from the eager call"
        a = torch.randn(128, 128, device=DEV)  # unrelated eager work between replays
        (a @ a).sum().item()
    q2 = torch.randn_like(c.q.float()).to(c.q.dtype)
    c.q.copy_(q2)
    want2 = _run(c, noalloc=False, with_dump=False)
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want2[0]) and torch.equal(lse, want2[1]), "replay on new q differs"
    del g


def test_noalloc_refuses_a_shape_beyond_its_scratch():
    B, hq, hkv, mp = 128, 64, 8, 200000
    need = int(_lib.query("delta_paged_decode_workspace_bytes", B, hq, hkv, mp))
    assert need > 64 << 20
    q = torch.zeros((B, hq, 128), dtype=torch.bfloat16, device=DEV)
    cache = torch.zeros((2, 2, 16, hkv, 128), dtype=torch.bfloat16, device=DEV)
    ip = torch.zeros(B + 1, dtype=torch.int32, device=DEV)
    last = torch.zeros(B, dtype=torch.int32, device=DEV)
    with pytest.raises(_lib.DeltaHipError, match="static scratch"):
        _lib.call("delta_paged_decode_noalloc", q.data_ptr(), q.stride(0), q.stride(1), cache.data_ptr(), 2,
                  ip.data_ptr(), ip.data_ptr(), 0, last.data_ptr(), q.data_ptr(), q.stride(0), q.stride(1), None,
                  None, 0, 0, B, hq, hkv, 128, _lib.DELTA_BF16, 0.088, mp, torch.cuda.current_stream().cuda_stream)
