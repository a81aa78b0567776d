"""The C-ABI library loads and exports what include/cvmm_hip.h declares.

Runs without a GPU: only host-side functions are called (workspace queries,
argument validation that fails before any launch)."""
import ctypes
import os
import re

import pytest

from cvmm_codex_amd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cvmm_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cvmm_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not N.available():
        from cvmm_codex_amd import build
        build.build(verbose=False)
    return N.lib()


def test_header_declares_the_bound_symbols():
    assert set(_declared()) == set(N.EXPORTED)


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(N.LIB_PATH)
    for name in _declared():
        assert hasattr(raw, name), name


def test_abi_version(lib):
    assert lib.cvmm_abi_version() == 13


def test_workspace_queries(lib):
    assert lib.cvmm_sort_workspace_bytes(65536, 64) > 0
    # the no-alloc sort's 1 MiB static scratch holds the sort's workspace at
    # every accepted size (<= 32767 experts, < 2^31 routes)
    worst = max(lib.cvmm_sort_workspace_bytes(R, E) for E in (1, 63, 64, 255, 1000, 8191, 8192, 16383, 32746, 32767)
                for R in (1, 1024, 65535, 65537, 1 << 20, (1 << 31) - 1))
    assert worst <= 1 << 20
    # no workspace needed for an unweighted forward with offsets given
    assert lib.cvmm_fwd_workspace_bytes(65536, 64, 1024, 128, 65536, N.BF16, N.BF16, 1, 0, 0) == 0
    # weighted combine: route-ordered buffer or fp32 token accumulator
    assert lib.cvmm_fwd_workspace_bytes(65536, 64, 128, 1024, 8192, N.BF16, N.BF16, 1, 1, 0) >= 65536 * 1024 * 2
    assert (lib.cvmm_fwd_workspace_bytes(65536, 64, 128, 1024, 8192, N.BF16, N.BF16, 1, 1, N.FLAG_ATOMIC_REDUCE)
            >= 8192 * 1024 * 4)
    # token-input grad (top-64 sum) with the routed path: the route-ordered [R, d_in] buffer
    R, T, E = 524288, 8192, 256
    assert lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 1) == 0
    try:
        assert lib.cvmm_bwd_x_workspace_bytes(R, E, 2048, 64, T, 1, 0, 1, 64, N.BF16, N.BF16, 0, 0) >= R * 2048 * 2
    finally:
        lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 0)
    # weight grad: counters + bounded partial slots
    assert lib.cvmm_bwd_w_workspace_bytes(65536, 64, 1024, 128, N.BF16, 1) > 64 * 8 * 4
    # room for the scaled route rows of a weighted route-input selection
    base = lib.cvmm_bwd_w_workspace_bytes(65536, 64, 128, 1024, N.BF16, 1)
    assert lib.cvmm_bwd_w_workspace_bytes_ex(65536, 64, 128, 1024, N.BF16, 1, 0) == base
    assert lib.cvmm_bwd_w_workspace_bytes_ex(65536, 64, 128, 1024, N.BF16, 1, 1) >= base + 65536 * 128 * 2
    assert lib.cvmm_bwd_w_workspace_bytes_ex(65536, 64, 128, 1024, N.F32, 1, 1) == \
        lib.cvmm_bwd_w_workspace_bytes(65536, 64, 128, 1024, N.F32, 1)


def test_invalid_arguments_fail_before_launch(lib):
    rc = lib.cvmm_sort_routes(None, 0, 10, 0, 1, None, None, None, None, None, None, None, 0, None)
    assert rc == 1 and b"n_experts" in lib.cvmm_last_error()
    rc = lib.cvmm_sort_routes(None, 0, 10, 100000, 1, None, None, None, None, None, None, None, 0, None)
    assert rc == 2
    # the no-alloc sort names a bad argument before any HIP call, like the sort
    rc = lib.cvmm_sort_routes_noalloc(None, 0, 10, 0, 1, None, None, None, None, None, None, None)
    assert rc == 1 and b"n_experts" in lib.cvmm_last_error()
    rc = lib.cvmm_sort_routes_noalloc(None, 0, 10, 100000, 1, None, None, None, None, None, None, None)
    assert rc == 2
    # the id copy with the sort's histogram: expert count, workspace; the sort with unknown flags
    assert lib.cvmm_copy_ids_count(None, 0, 10, 0, None, None, 0, None) == 1
    assert lib.cvmm_copy_ids_count(ctypes.c_void_p(16), 0, 10, 8, ctypes.c_void_p(16), None, 0, None) == 3
    assert lib.cvmm_sort_routes_cast_keys_ex(None, 0, 10, 8, 1, None, None, None, None, None, None, None, 0, None,
                                             0, 0, 0, 0, 0, 0, 0, None, None, 0, 64, None) == 1
    args = [None, 7, 1, 16, None, 0, 4, 16, 8, 128, 8, 1, None, None, None, 1, None, None, None, 0, 1,
            0, None, 0, 1, 8, 0, None, 0, None]
    assert lib.cvmm_fwd(*args) == 1 and b"dtype" in lib.cvmm_last_error()
    args[1] = 0
    args[-4] = 0
    args[2] = 1
    args[24] = 2   # out_rows != R
    assert lib.cvmm_fwd(*args) == 1
    # weighted forward without workspace
    wargs = [None, 0, 8, 16, None, 0, 4, 16, 8, 128, 8, 1, None, None, None, 8, None, None, ctypes.c_void_p(16),
             0, 4, 0, None, 0, 2, 8, 0, None, 0, None]
    assert lib.cvmm_fwd(*wargs) == 3


def test_kept_scaled_rows_arguments_fail_before_launch(lib):
    """cvmm_fwd_keep_scaled needs its written flag (cleared on any error);
    cvmm_bwd_w takes CVMM_FLAG_ROWS_SCALED only for a weighted route-input
    selection whose x is in the 16-bit op dtype."""
    fake = ctypes.c_void_p(256)
    args = [None, 7, 1, 16, None, 0, 4, 16, 8, 128, 8, 1, None, None, None, 1, None, None, None, 0, 1,
            2, None, 2, 1, 8]
    assert lib.cvmm_fwd_keep_scaled(*args, None, None, 0, None, 0, None) == 1
    written = ctypes.c_int32(5)
    assert lib.cvmm_fwd_keep_scaled(*args, None, ctypes.addressof(written), 0, None, 0, None) == 1
    assert written.value == 0 and b"dtype" in lib.cvmm_last_error()

    def bwd_w(x_dtype, out_index, rw, flags):
        return lib.cvmm_bwd_w(fake, x_dtype, 8, 16, fake, N.BF16, 2, 8, 4, 16, 8, fake, fake, out_index, 8, fake,
                              rw, N.F32, 4, N.BF16, fake, N.F32, 128, 8, 1, flags, fake, 1 << 30, None)
    assert bwd_w(N.BF16, fake, fake, N.FLAG_ROWS_SCALED) == 1          # token input
    assert b"ROWS_SCALED" in lib.cvmm_last_error()
    assert bwd_w(N.BF16, None, None, N.FLAG_ROWS_SCALED) == 1          # unweighted
    assert bwd_w(N.F32, None, fake, N.FLAG_ROWS_SCALED) == 1           # rows not in the op dtype


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(N, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(N, "_lib", None)
    with pytest.raises(N.NativeLibraryMissing):
        N.lib()


def test_tuning_knob_rejects_bad_values(lib):
    assert lib.cvmm_tuning_set(N.TUNE_PANEL_TILES_PER_WG, -1) != 0
    assert lib.cvmm_tuning_set(N.TUNE_PANEL_TILES_PER_WG, 5000) != 0
    assert lib.cvmm_tuning_set(99, 1) != 0
    assert lib.cvmm_tuning_set(N.TUNE_PANEL_TILES_PER_WG, 0) == 0
    assert lib.cvmm_tuning_set(N.TUNE_WGRAD_ORDER, 4) != 0
    assert lib.cvmm_tuning_set(N.TUNE_WGRAD_ORDER, -1) != 0
    assert lib.cvmm_tuning_set(N.TUNE_WGRAD_ORDER, 3) == 0
    assert lib.cvmm_tuning_set(N.TUNE_WGRAD_ORDER, 0) == 0
    assert lib.cvmm_tuning_set(N.TUNE_WGRAD_TILE, 6) != 0
    assert lib.cvmm_tuning_set(N.TUNE_WGRAD_TILE, -1) != 0
    assert lib.cvmm_tuning_set(N.TUNE_WGRAD_TILE, 5) == 0
    assert lib.cvmm_tuning_set(N.TUNE_WGRAD_TILE, 0) == 0
    assert lib.cvmm_tuning_set(N.TUNE_GEMM_ORDER, 3) != 0
    assert lib.cvmm_tuning_set(N.TUNE_GEMM_ORDER, 0) == 0
    assert lib.cvmm_tuning_set(N.TUNE_RING_TILE, 4) != 0
    assert lib.cvmm_tuning_set(N.TUNE_RING_TILE, 3) == 0
    assert lib.cvmm_tuning_set(N.TUNE_RING_TILE, 2) == 0
    assert lib.cvmm_tuning_set(N.TUNE_RING_TILE, 0) == 0
    assert lib.cvmm_tuning_set(N.TUNE_WGRAD_CHUNK, -1) != 0
    assert lib.cvmm_tuning_set(N.TUNE_WGRAD_CHUNK, 1 << 31) != 0
    assert lib.cvmm_tuning_set(N.TUNE_WGRAD_CHUNK, 2048) == 0
    assert lib.cvmm_tuning_set(N.TUNE_WGRAD_CHUNK, 0) == 0
    assert lib.cvmm_tuning_set(4, 32) != 0               # the retired reduce-GEMM threshold knob


def test_router_arguments_fail_before_launch(lib):
    assert lib.cvmm_route_topk_workspace_bytes(16384, 128, 8) > 129 * 4
    # k > E, E > 1024, k > 64, bad dtype, missing workspace
    assert lib.cvmm_route_topk(None, 0, 16, 8, 8, 9, 1, None, None, None, None, None, None, None, None, 0, None) == 1
    assert lib.cvmm_route_topk(None, 0, 16, 2048, 2048, 8, 1, None, None, None, None, None, None, None, None, 0,
                               None) == 2
    assert lib.cvmm_route_topk(None, 0, 16, 128, 128, 65, 1, None, None, None, None, None, None, None, None, 0,
                               None) == 2
    assert lib.cvmm_route_topk(None, 7, 16, 128, 128, 8, 1, None, None, None, None, None, None, None, None, 0,
                               None) == 1
    assert lib.cvmm_route_topk(None, 0, 16, 128, 128, 8, 1, None, None, None, None, None, None, None, None, 0,
                               None) == 3
    assert lib.cvmm_route_topk_backward(None, 0, 16, 128, 128, 8, 1, None, None, None, 64, None) == 1


def test_dense_topk_choice(lib):
    """The top-k sum's dense form is chosen at SwitchHead fan-out (64 of 256
    experts, K = 64, N = 2048), not at top-8 of 64 (ff_up / ff_down) or of 128
    (the FFN stack); only for 16-bit ops, 2 <= top_k <= 64, K % 8 == 0,
    N % 8 == 0 and at most 1024 experts;
    the knob forces either way."""
    BF, F32 = N.BF16, N.F32
    assert lib.cvmm_topk_dense(8192, 256, 64, 2048, 64, BF) == 1        # switch_v grad-input, switch_o forward
    assert lib.cvmm_topk_dense(8192, 64, 128, 1024, 8, BF) == 0          # ff_up grad-input, ff_down forward
    assert lib.cvmm_topk_dense(16384, 128, 512, 2048, 8, BF) == 0        # the FFN stack's down projection
    assert lib.cvmm_topk_dense(8192, 256, 64, 2048, 64, F32) == 0        # fp32 op: routed path
    assert lib.cvmm_topk_dense(8192, 256, 60, 2048, 64, BF) == 0         # K % 8 != 0
    assert lib.cvmm_topk_dense(8192, 256, 64, 2048, 65, BF) == 0         # top_k > 64
    assert lib.cvmm_topk_dense(8192, 5000, 64, 2048, 64, BF) == 0        # too many experts for the slot table
    try:
        assert lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 2) == 0
        assert lib.cvmm_topk_dense(8192, 64, 128, 1024, 8, BF) == 1
        assert lib.cvmm_topk_dense(100, 7, 16, 24, 2, N.F16) == 1
        assert lib.cvmm_topk_dense(100, 7, 16, 24, 1, N.F16) == 0        # top-1 has no sum
        # the GEMM addresses weights, operand rows and table with 32-bit offsets
        assert lib.cvmm_topk_dense(8192, 1024, 1024, 2048, 8, BF) == 0   # 4 GiB of weights
        assert lib.cvmm_topk_dense(1 << 20, 16, 1024, 512, 64, BF) == 0  # 128 GiB of operand rows
        assert lib.cvmm_topk_dense(1 << 20, 1024, 8, 512, 2, BF) == 0    # 4 GiB slot table
        assert lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 1) == 0
        assert lib.cvmm_topk_dense(8192, 256, 64, 2048, 64, BF) == 0
        assert lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 3) != 0
    finally:
        lib.cvmm_tuning_set(N.TUNE_DENSE_TOPK, 0)
    assert lib.cvmm_topk_dense(8192, 2000, 64, 2048, 64, BF) == 0        # more experts than the table's rows hold
    assert lib.cvmm_topk_dense(8192, 256, 64, 2044, 64, BF) == 0         # N % 8 != 0
    # workspace: the dense form needs a weight copy, the slot tables (5 bytes
    # per token and expert) and an operand copy (each at most E*K*N or R*K
    # values), not the [R, N] route buffer
    R, T, E = 524288, 8192, 256
    ws = lib.cvmm_bwd_x_workspace_bytes(R, E, 2048, 64, T, 1, 0, 1, 64, BF, BF, 0, 0)
    assert E * 64 * 2048 * 2 + T * E * 5 <= ws < R * 2048 * 2 // 4
    ws = lib.cvmm_fwd_workspace_bytes(R, E, 64, 2048, T, BF, BF, 1, 1, 0)
    assert E * 64 * 2048 * 2 + T * E * 5 + R * 64 * 2 <= ws < R * 2048 * 2 // 4
