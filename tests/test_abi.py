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


def test_wrappers_reject_cpu_tensors():
    from delta_amd import kernels
    q = torch.zeros(1, 8, 128, dtype=torch.bfloat16)
    cache = torch.zeros(2, 2, 16, 8, 128, dtype=torch.bfloat16)
    i32 = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU"):
        kernels.paged_decode(q, cache, i32, i32, i32, max_pages_per_row=1)
