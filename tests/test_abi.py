"""The C-ABI library builds, loads without a GPU and exports what include/delta_hip.h declares."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "delta_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"\b(delta_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    from delta_amd import _lib
    if not _lib.LIB_PATH.exists():
        from delta_amd import build
        build.build()
    return _lib.load()


def test_header_declares_the_hot_path():
    names = declared_functions()
    for must in ("delta_paged_decode", "delta_page_score", "delta_page_scores_from_logits",
                 "delta_select_pages", "delta_pack_page_indices", "delta_decode_page_info",
                 "delta_append_kv", "delta_rope", "delta_last_error"):
        assert must in names


def test_every_declared_symbol_is_exported(lib):
    from delta_amd import _lib
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_no_undeclared_exports(lib):
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", str(ROOT / "delta_amd" / "_delta_hip.so")],
                         capture_output=True, text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l and l.split()[-1].startswith("delta_")}
    assert exported == set(declared_functions())


def test_queries_without_gpu(lib):
    assert lib.delta_abi_version() == 202
    assert lib.delta_last_error() == b""
    # split heuristic: deterministic, >= 1; the larger of the attention and the dump plans.
    # Page-major splits are sized for 16-wave blocks (Hkv heads x R waves): up to 4096 waves in
    # total, >= 2 pages per wave; head-major blocks (one kv head) when batch*Hkv >= 256 and
    # batch*Hkv*max_pages <= 262144 never split; attention launches with batch*Hkv < 256 use
    # head-major blocks split to 256 blocks (fewer splits than page-major).
    assert lib.delta_decode_num_splits(32, 8, 128) == 1        # config 3 subset: head-major
    assert lib.delta_decode_num_splits(64, 4, 128) == 1        # head-major
    assert lib.delta_decode_num_splits(32, 8, 513) == 1        # config 3 full: head-major
    # past the head-major size: page-major, 8 splits (256 blocks) of 129 pages, over the 128-page unit: 9
    assert lib.delta_decode_num_splits(32, 8, 1025) == 9
    assert lib.delta_decode_num_splits(1024, 8, 2048) == 1
    assert lib.delta_decode_num_splits(8, 8, 128) == 32        # config 2
    assert lib.delta_decode_num_splits(4, 4, 4096) == 64       # config 4: R = 4
    assert lib.delta_decode_num_splits(4, 4, 256) == 32        # >= 2 pages per wave
    assert lib.delta_decode_num_splits(1, 8, 4) == 1           # unsplit: no one-wave conversion
    assert lib.delta_paged_decode_workspace_bytes(1024, 32, 8, 2048) == 0
    assert lib.delta_paged_decode_workspace_bytes(32, 32, 8, 128) == 0
    # partials (m, l, acc[128]) per (row, split, q head), 256-byte aligned
    assert lib.delta_paged_decode_workspace_bytes(32, 32, 8, 1025) == 32 * 32 * 9 * 130 * 4
    # config 5 (ragged up to 2049 pages): units of at most 128 pages, 17 for the longest row
    assert lib.delta_decode_num_splits(128, 8, 2049) == 17
    assert lib.delta_page_score_workspace_bytes(32, 32) == 32 * 32 * 4
    # the larger of: (m, l) per (row, split, q head) + the lse buffer (dump path),
    # and the LDS scorer's per-(kv head, token) maxima [B][Hkv][max_pages*16] (config 3 fits)
    assert lib.delta_page_score_needs_dump(32, 32, 8, 513) == 0
    assert lib.delta_page_score_kv_workspace_bytes(32, 32, 8, 513) == 32 * 8 * 513 * 16 * 4
    assert lib.delta_page_score_needs_dump(8, 32, 8, 1024) == 1      # config 2: 64 (row, head) pairs
    assert lib.delta_page_score_needs_dump(32, 64, 8, 513) == 1      # G = 8: 263 KB of logits per row
    assert lib.delta_page_score_kv_workspace_bytes(8, 32, 8, 1024) == 8 * 32 * 32 * 2 * 4 + 8 * 32 * 4
    assert lib.delta_page_score_kv_workspace_bytes(1024, 32, 8, 2048) == 1024 * 32 * 4


def test_argument_errors_reported_without_launch(lib):
    from delta_amd import _lib
    # head_dim 64 is rejected before any launch; the message is kept per thread
    with pytest.raises(_lib.DeltaHipError, match="head_dim"):
        _lib.call("delta_paged_decode", 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, None, None, 0, 0,
                  1, 8, 8, 64, 0, 1.0, 1, None, 0, None)
    with pytest.raises(_lib.DeltaHipError, match="k out of range"):
        _lib.call("delta_select_pages", 8, 4, 8, 8, 4, 1, 4, 5, None, 1, 1e-7, 0, None, 8, 4, 8, None)
    # the dump writer's offsets must stay below 2^31 bytes: max_pages * 16 <= 2^28 floats
    # (aligned stand-in addresses; rejected before any launch)
    with pytest.raises(_lib.DeltaHipError, match="max_pages \\* 16 <= 2\\^28"):
        _lib.call("delta_paged_decode", 256, 1024, 128, 256, 100, 256, 256, 100, 256, 256, 1024, 128, None,
                  256, 1 << 30, 1 << 28, 1, 8, 8, 128, 0, 1.0, (1 << 24) + 1, None, 0, None)
    # a budget rule needs divisor > 0, an output array and no fixed per-row budgets
    import ctypes
    for rule, kpr in (((512, 0, 8), None), ((512, 8, None), None), ((-1, 8, 8), None), ((512, 8, 8), 8)):
        with pytest.raises(_lib.DeltaHipError, match="budget rule needs"):
            _lib.call("delta_decode_page_info", 8, None, 8, 4, 16, 8, kpr, ctypes.byref(_lib.BudgetRuleC(*rule)),
                      1.0, 1, 8, 8, 8, None, 8, 8, 8, None)


def test_gemm_rows32_plan_and_errors_without_launch(lib):
    from delta_amd import _lib
    # splits: enough (N / 64 NB) x S blocks for 256 CUs, S dividing K / 64; 0 = shape not taken
    assert lib.delta_gemm_rows32_splits(32, 4096, 4096) == 4      # Llama-3-8B wo
    assert lib.delta_gemm_rows32_splits(32, 4096, 14336) == 8     # w2: two column groups per wave
    assert lib.delta_gemm_rows32_splits(32, 28672, 4096) == 1     # w1|w3: 448 blocks, unsplit
    assert lib.delta_gemm_rows32_splits(32, 4100, 4096) == 0      # N % 64
    assert lib.delta_gemm_rows32_splits(32, 4096, 4000) == 0      # K % 64
    # rejected before any launch (null x / w are checked after the shape)
    with pytest.raises(_lib.DeltaHipError, match="M .* must be <= 32"):
        _lib.call("delta_gemm_rows32", 16, 4096, 16, 4096, None, 16, 4096, 16, 33, 4096, 4096, 0, None)
    with pytest.raises(_lib.DeltaHipError, match="multiple of 64"):
        _lib.call("delta_gemm_rows32", 16, 4096, 16, 4096, None, 16, 4100, 16, 32, 4100, 4096, 0, None)
    with pytest.raises(_lib.DeltaHipError, match="fp32 partials"):
        _lib.call("delta_gemm_rows32", 16, 4096, 16, 4096, None, 16, 4096, None, 32, 4096, 4096, 0, None)
    with pytest.raises(_lib.DeltaHipError, match="nsplit must be 2, 4, 8 or 16"):
        _lib.call("delta_add_rmsnorm_partials", 16, 4096, 16, 0, 16, 1e-5, 16, 4096, 16, 4096, 32, 4096, 0, None)


@pytest.mark.skipif(torch.cuda.is_available(), reason="stand-in addresses: validation-only, run where no GPU is visible")
def test_append_descriptor_errors_reported_without_launch(lib):
    from delta_amd import _lib
    # The fused decode entry points check their append descriptor before any launch; the
    # non-null 16-byte-aligned stand-in addresses below are never dereferenced.
    with pytest.raises(_lib.DeltaHipError, match="null append"):
        _lib.call("delta_paged_decode_append", None, 16, 0, 0, 16, 1, 16, 16, 0, 16, 16, 0, 0, None, None, 0, 0,
                  1, 8, 8, 128, 0, 1.0, 1, None, 0, None)
    bad_theta = _lib.DecodeAppendC(16, 1024, 16, 1024, 16, 16, 16, 1, 1.0, -1.0, 0, 0.0, 0.0, 0.0)
    with pytest.raises(_lib.DeltaHipError, match="rope"):
        _lib.call("delta_paged_decode_subset_append", ctypes.byref(bad_theta), 16, 0, 0, 16, 1, 16, 16, 0, 16, 16,
                  0, 0, None, 1, 8, 8, 128, 0, 1.0, 1, None, 0, None)
    odd_stride = _lib.DecodeAppendC(16, 1023, 16, 1024, 16, 16, 16, 1, 1.0, 1e4, 0, 0.0, 0.0, 0.0)
    with pytest.raises(_lib.DeltaHipError, match="even row strides"):
        _lib.call("delta_paged_decode_append", ctypes.byref(odd_stride), 16, 0, 0, 16, 1, 16, 16, 0, 16, 16, 0, 0,
                  None, None, 0, 0, 1, 8, 8, 128, 0, 1.0, 1, None, 0, None)


def _rejects(name, args, match):
    from delta_amd import _lib
    with pytest.raises(_lib.DeltaHipError, match=match):
        _lib.call(name, *args)


def test_empty_calls_return_before_touching_pointers(lib):
    from delta_amd import _lib
    # batch / row count 0: nothing to do, success, even with every pointer null
    _lib.call("delta_paged_prefill", None, 0, 0, None, 0, None, None, None, 0, None, None, 0, 0, None,
              0, 32, 8, 128, 0, 1.0, 0, None)
    _lib.call("delta_append_kv", None, 0, None, 0, None, None, 0, None, 0, None, None, 0, 0, 8, 128, 0, None)
    _lib.call("delta_rope", None, 0, None, 0, None, 0, None, 0, None, None, 0, 0, 32, 8, 128, 0,
              1.0, 5e5, 0, 1.0, 4.0, 8192.0, None)
    _lib.call("delta_pack_page_indices", None, 0, None, None, None, None, None, 0, None, 0, 16, 0, 0, None)
    _lib.call("delta_page_scores_from_logits", None, 0, 0, None, None, None, None, 0, 0, 32, 16, None, 0, None)
    _lib.call("delta_page_score", None, 0, 0, None, 0, None, None, 0, None, None, 0, 0, None, 0,
              0, 32, 8, 128, 0, 1.0, 16, None, 0, None)
    _lib.call("delta_select_pages", None, 0, None, None, 0, 0, 16, 4, None, 2, 1e-7, 0, None, None, 0, None, None)
    _lib.call("delta_decode_page_info", None, None, None, 0, 16, 4, None, None, 1.0, 1,
              None, None, None, None, None, None, None, None)


def test_argument_errors_of_every_hot_path_entry_point(lib):
    """Each entry point's first-line checks (reference behaviour: a RuntimeError naming the bad
    argument) fire before anything touches the pointers; null pointers only, so the calls are
    safe wherever they run."""
    # causal prefill
    pf = lambda hq, hkv, hd, dt, q=None: (q, 0, 0, None, 16, None, None, None, 0, None, None, 0, 0, None,
                                           1, hq, hkv, hd, dt, 1.0, 4, None)
    _rejects("delta_paged_prefill", pf(32, 8, 64, 0), "head_dim must be 128")
    _rejects("delta_paged_prefill", pf(12, 8, 128, 0), "multiple of num_kv_heads")
    _rejects("delta_paged_prefill", pf(72, 8, 128, 0), "group size 9 > 8")
    _rejects("delta_paged_prefill", pf(32, 8, 128, 7), "bad dtype")
    _rejects("delta_paged_prefill", pf(32, 8, 128, 0), "null pointer")
    # KV append and RoPE
    ak = lambda hd, dt: (None, 0, None, 0, None, None, 16, None, 0, None, None, 1, 1, 8, hd, dt, None)
    _rejects("delta_append_kv", ak(64, 0), "head_dim must be 128")
    _rejects("delta_append_kv", ak(128, 9), "bad dtype")
    _rejects("delta_append_kv", ak(128, 1), "null pointer")
    rp = lambda hd, dt: (None, 0, None, 0, None, 0, None, 0, None, None, 1, 1, 32, 8, hd, dt,
                         1.0, 5e5, 0, 1.0, 4.0, 8192.0, None)
    _rejects("delta_rope", rp(96, 0), "head_dim must be 128")
    _rejects("delta_rope", rp(128, 3), "bad dtype")
    _rejects("delta_rope", rp(128, 0), "null pointer")
    # page-index packer (page_metadata.py:42-70)
    _rejects("delta_pack_page_indices", (None, 4, None, None, None, None, None, 0, None, 2, 16, 8, 1, None),
             "null pointer")
    # page scores from a logits dump
    sl = lambda dump, hq, sstride, dstride_h: (dump, 0, dstride_h, None, None, None, None, sstride, 2, hq, 16,
                                               None, 0, None)
    _rejects("delta_page_scores_from_logits", sl(None, 32, 16, 256), "null pointer")
    # K-only scorer
    ps = lambda scores, hq, hkv, sstride: (None, 0, 0, None, 16, None, None, 0, None, None, 0, 0, scores,
                                          sstride, 2, hq, hkv, 128, 0, 1.0, 16, None, 0, None)
    _rejects("delta_page_score", ps(None, 32, 8, 16), "null output pointer")
    # selection
    sp = lambda scores, sstride, bt_stride, mp, k, kpr, L, fixed: (scores, sstride, None, None, bt_stride, 2, mp, k,
                                                                    kpr, L, 1e-7, fixed, None, None, 0, None, None)
    _rejects("delta_select_pages", sp(None, 16, 16, 16, 4, None, 2, 0), "null pointer")
    # decode metadata
    _rejects("delta_decode_page_info", (None, None, None, 2, 16, 4, None, None, 1.0, 1,
                                        None, None, None, None, None, None, None, None), "null pointer")


@pytest.mark.skipif(torch.cuda.is_available(), reason="stand-in addresses: validation-only, run where no GPU is visible")
def test_argument_errors_past_the_null_checks(lib):
    """The checks after the null-pointer ones, with non-null 256-byte aligned stand-in addresses
    that are never dereferenced (each call fails validation before any launch)."""
    A = 1 << 20  # stand-in address
    _rejects("delta_paged_prefill", (A + 8, 1024, 128, A, 16, A, A, A, 16, A, A, 4096, 128, None,
                                     1, 32, 8, 128, 0, 1.0, 4, None), "16-byte aligned")
    _rejects("delta_paged_prefill", (A, 4096, 128, A, 16, A, A, A, 16, A, A + 2, 4096, 128, None,
                                     1, 32, 8, 128, 0, 1.0, 4, None), "o 8-byte aligned")
    _rejects("delta_paged_prefill", (A, 4096, 128, A, 0, A, A, A, 16, A, A, 4096, 128, None,
                                     1, 32, 8, 128, 0, 1.0, 4, None), "empty cache")
    _rejects("delta_append_kv", (A + 4, 1024, A, 1024, A, A, 16, A, 16, A, A, 1, 1, 8, 128, 0, None),
             "16-byte aligned")
    _rejects("delta_rope", (A, 4096, A, 1024, A, 4096, A, 1024, A, A, 1, 1, 32, 8, 128, 0,
                            0.0, 5e5, 0, 1.0, 4.0, 8192.0, None), "bad rope params")
    _rejects("delta_rope", (A, 4096, A, 1024, A, 4096, A, 1024, A, A, 1, 1, 32, 8, 128, 0,
                            8.0, 5e5, 1, 4.0, 1.0, 8192.0, None), "llama3.1 frequency factors")
    _rejects("delta_pack_page_indices", (A, 4, A, A, A, A, A, 64, None, 2, 16, 8, 1, None), "null row block table")
    sl = lambda hq, sstride, dstride_h: (A, 32 * 256, dstride_h, None, A, A, A, sstride, 2, hq, 16, None, 0, None)
    _rejects("delta_page_scores_from_logits", sl(0, 16, 256), r"num_qo_heads must be in \[1, 256\]")
    _rejects("delta_page_scores_from_logits", sl(32, 8, 256), "score_stride < max_pages")
    _rejects("delta_page_scores_from_logits", sl(32, 16, 255), "dump rows shorter than max_pages\\*16")
    ps = lambda hq, hkv, sstride, dump=None, dstride_h=0, ws=None, wsb=0: (
        A, 4096, 128, A, 16, A, A, 16, A, dump, 0, dstride_h, A, sstride, 2, hq, hkv, 128, 0, 1.0, 16, ws, wsb, None)
    _rejects("delta_page_score", ps(300, 10, 16), "too many heads")
    _rejects("delta_page_score", ps(12, 8, 16), "multiple of num_kv_heads")
    _rejects("delta_page_score", ps(32, 8, 8), "score_stride < max_pages")
    _rejects("delta_page_score", ps(32, 8, 16, dump=A, dstride_h=100), "dump rows shorter")
    _rejects("delta_page_score", ps(32, 8, 16), "needs a logits dump buffer")  # 2 x 8 (row, kv head) pairs
    _rejects("delta_page_score", ps(32, 8, 16, dump=A, dstride_h=256), "workspace of .* bytes needed")
    sp = lambda sstride, bt_stride, mp, k, kpr, L, fixed: (A, sstride, A, A, bt_stride, 2, mp, k, kpr, L, 1e-7,
                                                           fixed, None, A, 64, A, None)
    _rejects("delta_select_pages", sp(16, 16, 0, 4, None, 2, 0), "max_pages must be positive")
    _rejects("delta_select_pages", sp(8, 16, 16, 4, None, 2, 0), "row strides must be >= max_pages")
    _rejects("delta_select_pages", sp(16, 16, 16, 4, A, 2, 1), "fixed_count needs a global k")
    _rejects("delta_select_pages", sp(16, 16, 16, 4, None, -1, 0), "L must be >= 0")
    pi = lambda pps, si, sip: (A, None, A, 2, pps, 4, None, None, 1.0, 1, A, A, A, None, si, sip, None, None)
    _rejects("delta_decode_page_info", pi(0, None, None), "pages_per_slot <= 0")
    _rejects("delta_decode_page_info", pi(16, A, None), "go together")


def test_wrappers_reject_cpu_tensors():
    from delta_amd import kernels
    q = torch.zeros(1, 8, 128, dtype=torch.bfloat16)
    cache = torch.zeros(2, 2, 16, 8, 128, dtype=torch.bfloat16)
    i32 = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU"):
        kernels.paged_decode(q, cache, i32, i32, i32, max_pages_per_row=1)
