"""The allocation-free decode entry point (delta_paged_decode_noalloc, static device scratch)
against delta_paged_decode with a caller workspace, through the C ABI: bit-identical outputs,
lse and logits dump on two calls in a row (the second smaller), and a clear refusal of a shape
whose split partials exceed the static scratch."""
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
            out.data_ptr(), out.stride(0), out.stride(1), lse.data_ptr(), dump.data_ptr(), dump.stride(0),
            dump.stride(1), B, hq, c.kv_cache.shape[3], 128, _lib.DELTA_BF16, 1 / math.sqrt(128), mp]


def _run(c, noalloc):
    B, hq = c.q.shape[:2]
    mp = c.max_pages
    out = torch.full_like(c.q, 3.0)
    lse = torch.full((B, hq), 5.0, device=DEV)
    dump = torch.full((B, hq, mp * 16), 7.0, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        _lib.call("delta_paged_decode_noalloc", *_args(c, mp, out, lse, dump), stream)
    else:
        need = K.decode_workspace_bytes(B, hq, c.kv_cache.shape[3], mp)
        assert need > 0, "the case must run split, so the scratch is used"
        ws = torch.empty(need, dtype=torch.uint8, device=DEV)
        _lib.call("delta_paged_decode", *_args(c, mp, out, lse, dump), ws.data_ptr(), need, stream)
    torch.cuda.synchronize()
    return out, lse, dump


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
