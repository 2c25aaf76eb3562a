"""The C-ABI library loads on a host without a GPU, exports every symbol
include/*.h declares, and validates arguments before touching the device."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from jeeves_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> set[str]:
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(jv_\w+)\s*\(", text))
    return names


def test_header_declares_the_path():
    names = declared_functions()
    for required in ("jv_fp8_linear", "jv_fp8_gemm", "jv_fp8_quantize_rows_bf16", "jv_fp8_quantize_rows_f32",
                     "jv_fp8_swiglu_quantize", "jv_device_cu_count", "jv_fp8_last_error", "jv_w8a16_linear"):
        assert required in names


def test_library_exports_every_declared_symbol(product_lib):
    for name in declared_functions():
        assert hasattr(product_lib, name), name


def test_python_binding_matches_header():
    assert set(_lib.SIGNATURES) == declared_functions()


def test_library_is_gfx950_only():
    data = _lib.LIB_PATH.read_bytes()
    assert b"gfx950" in data
    for other in (b"gfx942", b"gfx90a", b"sm_"):
        assert other + b"\x00" not in data or other == b"sm_"


def test_value_errors_need_no_device(product_lib):
    L = product_lib
    assert L.jv_fp8_quantize_rows_bf16(None, 0, 4, 7, None, 0, None, None) == _lib.JV_ERR_VALUE
    assert b"divisible by 8" in L.jv_fp8_last_error()
    rc = L.jv_fp8_linear(None, 0, None, 0, None, None, None, None, 0, 0.0, None, 0, 4, 64, 100, None, 0, None, 0, None)
    assert rc == _lib.JV_ERR_VALUE
    assert b"divisible by 128" in L.jv_fp8_last_error()
    rc = L.jv_fp8_gemm(None, 0, None, None, 0, None, None, None, None, 8, 0.0, None, 0, 4, 64, 128, None, 0, None, 0, None)
    assert rc == _lib.JV_ERR_VALUE and b"rank 8" in L.jv_fp8_last_error()
    rc = L.jv_fp8_swiglu_quantize(None, 0, None, 0, 4, 20000, None, 0, None, None, 0, None, 0, None, None)
    assert rc == _lib.JV_ERR_VALUE
    rc = L.jv_w8a16_linear(None, 0, None, 0, None, None, None, 0, 4, 64, 100, None, 0, None, 0, None)
    assert rc == _lib.JV_ERR_VALUE and b"divisible by 128" in L.jv_fp8_last_error()
    rc = L.jv_w8a16_linear(None, 3, None, 0, None, None, None, 0, 4, 64, 128, None, 0, None, 0, None)
    assert rc == _lib.JV_ERR_VALUE and b"aligned" in L.jv_fp8_last_error()
    # M = 0 is a no-op that succeeds
    assert L.jv_w8a16_linear(None, 0, None, 0, None, None, None, 0, 0, 64, 128, None, 0, None, 0, None) == 0
    assert L.jv_fp8_linear(None, 0, None, 0, None, None, None, None, 0, 0.0, None, 0, 0, 64, 128, None, 0, None, 0, None) == 0


def test_error_mapping():
    with pytest.raises(ValueError):
        _lib.lib().jv_fp8_quantize_rows_bf16(None, 0, 1, 3, None, 0, None, None) and _lib.check(_lib.JV_ERR_VALUE)
    with pytest.raises(RuntimeError):
        _lib.check(_lib.JV_ERR_RUNTIME)
    _lib.check(_lib.JV_OK)


def test_split_for_is_pure_host_logic(product_lib):
    L = product_lib
    # decode, 256 CUs: every 9B projection has enough 16-row tiles (k/v: 64) to
    # skip split-K; only N < 512 (fewer than 32 tiles) splits K across workgroups
    assert L.jv_fp8_split_for(16, 4096, 4096, 256) == 1
    assert L.jv_fp8_split_for(16, 1024, 4096, 256) == 1
    assert L.jv_fp8_split_for(16, 24576, 4096, 256) == 1
    assert L.jv_fp8_split_for(16, 256, 4096, 256) == 8   # 16 tiles, capped at K/128/4
    assert L.jv_fp8_split_for(16, 128, 12288, 256) == 12  # 8 tiles; K=12288 runs 8 waves: capped at K/128/8
    assert L.jv_fp8_counters_needed(16, 256, 4096, 256) == 16
    assert L.jv_fp8_counters_needed(16, 4096, 4096, 256) == 0
    # 17-128 tokens on the batch-decode kernel: no K split, no counters
    assert L.jv_fp8_split_for(96, 4096, 4096, 256) == 1
    assert L.jv_fp8_counters_needed(96, 4096, 4096, 256) == 0
    # 17-128 tokens on the prefill kernel: 64x64 tiles (5 stages) split K
    # until tiles x splits reach the CUs, at most 4 ways, none from 0.625
    # rounds of tiles; longer rows take 64 tokens x 64 channels per tile too
    assert L.jv_fp8_split_for(96, 4096, 12288, 256) == 2     # 128 tiles of 64x64
    assert L.jv_fp8_counters_needed(96, 4096, 12288, 256) == 128
    assert L.jv_fp8_split_for(96, 6144, 4096, 256) == 1     # 192 tiles
    assert L.jv_fp8_split_for(64, 4096, 12288, 256) == 4    # down from 32 tokens: 64 tiles of 64x64
    assert L.jv_fp8_counters_needed(64, 4096, 12288, 256) == 64
    assert L.jv_fp8_split_for(31, 4096, 12288, 256) == 1    # below 32 tokens: the batch-decode kernel
    # above 128 tokens: the lockstep tile and K split of least modelled time; a
    # split keeps at least four 128-deep stages, at most 8
    assert L.jv_fp8_split_for(256, 4096, 12288, 256) == 2   # 128 tiles of 64x128
    assert L.jv_fp8_counters_needed(256, 4096, 12288, 256) == 128
    assert L.jv_fp8_split_for(512, 4096, 12288, 256) == 2   # 128 tiles of 128x128
    assert L.jv_fp8_split_for(128, 1024, 8192, 256) == 4    # 32 tiles
    assert L.jv_fp8_split_for(256, 1024, 512, 256) == 1     # 4 stages of 128 leave no room to split
    assert L.jv_fp8_split_for(512, 1024, 4096, 256) == 2    # 128 tiles of 64x64
    assert L.jv_fp8_split_for(512, 4096, 4096, 256) == 1    # 256 tiles of 64x128 fill the CUs
    assert L.jv_fp8_split_for(1040, 2048, 4096, 256) == 1
    assert L.jv_fp8_split_for(2048, 4096, 4096, 256) == 1   # 256x128 tiles
    assert L.jv_fp8_counters_needed(2048, 4096, 4096, 256) == 0
    assert L.jv_fp8_split_for(65, 24576, 4096, 256) == 1    # 192 tiles of 128x128
    assert L.jv_fp8_split_for(4096, 24576, 4096, 256) == 1  # 256x256 ping-pong tiles never split


def launch_shape(L, M, N, K, cus=256):
    shape = (ctypes.c_int32 * 4)()
    _lib.check(L.jv_fp8_launch_shape(M, N, K, cus, shape))
    return list(shape)


def test_batch_decode_plans_are_host_logic(product_lib):
    """17-128 tokens on K = 4096 (4 waves of 8 steps) or K = 12288 (8 waves of
    12): the batch-decode kernel (kind 3) where at most one workgroup per CU,
    at least half the CUs and at most 6 tiles per workgroup (576 KiB of
    operands) allow it; one workgroup per weight group and token part."""
    L = product_lib
    assert launch_shape(L, 32, 1024, 4096) == [3, 128, 256, 1]     # k/v: 64 groups x 2 token parts
    assert launch_shape(L, 64, 1024, 4096) == [3, 256, 256, 1]     # 64 x 4 parts of one tile
    assert launch_shape(L, 128, 1024, 4096) == [3, 256, 256, 1]    # 64 x 4 parts of two tiles
    assert launch_shape(L, 64, 4096, 4096) == [3, 256, 256, 1]     # q/o: 128 pairs of tiles x 2 parts
    assert launch_shape(L, 64, 6144, 4096) == [3, 192, 256, 1]     # merged q/k/v: 192 pairs, 4 token tiles
    assert launch_shape(L, 32, 4096, 12288) == [3, 256, 512, 1]    # down, 8 waves
    assert launch_shape(L, 16, 1024, 4096)[0] == 0                 # 16 tokens: the decode kernel
    assert launch_shape(L, 129, 1024, 4096)[0] == 1                # past 128 tokens: prefill tiles
    assert launch_shape(L, 64, 1024, 2048)[0] != 3                 # other row lengths
    assert launch_shape(L, 48, 4096, 12288)[0] == 1                # 3 token tiles of K = 12288 exceed 576 KiB
    assert launch_shape(L, 96, 6144, 4096)[0] == 1                 # 6 token tiles: 7+ tiles a workgroup
    assert launch_shape(L, 32, 10240, 4096)[0] == 1                # 320 pairs exceed the CUs
    assert launch_shape(L, 64, 24576, 4096)[0] == 1                # gate+up
    assert launch_shape(L, 64, 512, 4096)[0] == 0                  # 32 tiles: decode kernel, K split
    for M in range(17, 129):
        for N, K in ((1024, 4096), (4096, 4096), (6144, 4096), (4096, 12288)):
            kind, wgs, threads, splits = launch_shape(L, M, N, K)
            if kind == 3:
                assert wgs <= 256 and 2 * wgs >= 256 and splits == 1, (M, N, K)
                assert L.jv_fp8_counters_needed(M, N, K, 256) == 0 and L.jv_fp8_split_for(M, N, K, 256) == 1


def test_batch_decode_plans_stay_within_their_bounds(product_lib):
    """Over CU counts, weights and batch sizes: the batch-decode kernel runs
    only at 17-128 tokens on K = 4096 / 12288 weights of at least 64 tiles,
    with one workgroup per CU at most and half the CUs at least, 4 waves for
    K = 4096 and 8 for K = 12288, and needs no K split, counters or partials."""
    L = product_lib
    seen = 0
    for cus in (64, 80, 104, 120, 228, 256, 304):
        for K in (2048, 4096, 8192, 12288):
            for N in (256, 1008, 1024, 1040, 2048, 4096, 4112, 6144, 8192, 10240, 12288, 24576):
                for M in (1, 16, 17, 31, 32, 33, 48, 50, 64, 65, 80, 96, 100, 112, 127, 128, 129, 256):
                    kind, wgs, threads, splits = launch_shape(L, M, N, K, cus)
                    if kind != 3:
                        continue
                    seen += 1
                    assert 17 <= M <= 128 and K in (4096, 12288) and (N + 15) // 16 >= 64, (cus, M, N, K)
                    assert wgs <= cus and 2 * wgs >= cus and splits == 1, (cus, M, N, K, wgs)
                    assert threads == (256 if K == 4096 else 512), (cus, M, N, K)
                    assert L.jv_fp8_split_for(M, N, K, cus) == 1 and L.jv_fp8_counters_needed(M, N, K, cus) == 0
    assert seen > 100, seen


def test_prefill_plans_stay_within_their_bounds(product_lib):
    """Over CU counts, weights and batch sizes above the decode regimes: a
    ping-pong plan (kind 2) is one workgroup of 512 threads per 256x256 or
    128x384 tile and never splits K; a lockstep plan (kind 1) runs 4 or 8
    waves, and a K split keeps its tiles x splits within one round of
    workgroups (at most two per CU) and needs one counter per tile."""
    L = product_lib
    seen_pp = seen_split = 0
    for cus in (64, 80, 104, 120, 228, 256, 304):
        for K in (2048, 4096, 12288):
            for N in (1024, 1040, 4096, 6144, 10240, 12288, 24576):
                for M in (129, 192, 300, 512, 777, 1024, 1536, 2048, 3000, 8192):
                    kind, wgs, threads, splits = launch_shape(L, M, N, K, cus)
                    assert kind in (1, 2), (cus, M, N, K, kind)
                    if kind == 2:
                        seen_pp += 1
                        assert threads == 512 and splits == 1, (cus, M, N, K)
                        assert wgs in (-(-M // 256) * -(-N // 256), -(-M // 128) * -(-N // 384)), (cus, M, N, K, wgs)
                        continue
                    assert threads in (256, 512) and 1 <= splits <= 8, (cus, M, N, K)
                    if splits > 1:
                        seen_split += 1
                        assert wgs <= 2 * cus and wgs % splits == 0, (cus, M, N, K, wgs, splits)
                        assert L.jv_fp8_counters_needed(M, N, K, cus) == wgs // splits
                    else:
                        assert L.jv_fp8_counters_needed(M, N, K, cus) == 0
    assert seen_pp > 100 and seen_split > 20, (seen_pp, seen_split)


def test_lockstep_model_picks_the_measured_fastest_tiles(product_lib):
    """Above 128 tokens the lockstep tile of least modelled time: the 5-stage
    64x128 / 64x64 rings where one round of small tiles is bound by the bytes
    each CU keeps in flight (q/o at 256-512 tokens, k/v at 768-2048), 128x128
    and 256x128 where whole rounds of larger tiles fit; the fastest choices
    in alternating A/B timings on MI355X (256 CUs). Workgroups and threads
    name the tile: 64x64 runs 4 waves, 64x128 and 256x128 run 8."""
    L = product_lib
    # (M, N, K): (workgroups, threads, splits)
    want = {(256, 4096, 4096): (256, 256, 1),     # 64x64, 5 stages: 12.2 us vs 14.7 on 64x64 split 2
            (512, 4096, 4096): (256, 512, 1),     # 64x128, 5 stages: 16.2 vs 18.6 on 64x64
            (512, 1024, 4096): (256, 256, 2),     # 64x64, 5 stages, 2 splits: 10.1 vs 11.0
            (1024, 1024, 4096): (256, 256, 1),    # 64x64, 5 stages: 11.7 vs 13.4
            (2048, 1024, 4096): (256, 512, 1),    # 64x128, 5 stages: 15.7 vs 17.6
            (256, 8192, 4096): (256, 512, 1),     # 64x128, 5 stages: 17.5 vs 20.4
            (1024, 4096, 4096): (256, 256, 1),    # 128x128
            (2048, 4096, 4096): (256, 512, 1),    # 256x128
            (512, 4096, 12288): (256, 256, 2)}    # 128x128, 2 splits
    for (M, N, K), (wgs, threads, splits) in want.items():
        kind, got_wgs, got_threads, got_splits = launch_shape(L, M, N, K)
        assert (kind, got_wgs, got_threads, got_splits) == (1, wgs, threads, splits), (M, N, K)


def test_wide_weights_never_split_k(product_lib):
    """On weights wide enough for 1.5 rounds of 64-channel tiles the FP8 GEMM
    (from 17 tokens) and the W8A16 GEMM (from 32) leave the decode kernel at
    different batch sizes; the decode plan never splits K there, so neither
    choice needs a workspace or tile counters. The split depends on N, K and
    the CU count only: 16 tokens (always the decode kernel) stand for every
    batch."""
    L = product_lib
    for cus in (32, 80, 104, 256, 304):
        n_wide = 64 * (-(-3 * cus // 2) - 1) + 1  # smallest N with 2 * ceil(N / 64) >= 3 * cus
        for N in (n_wide, 24576, 248320):
            if N < n_wide:
                continue
            for K in (128, 4096, 12288, 16384, 65536):
                assert L.jv_fp8_split_for(16, N, K, cus) == 1, (cus, N, K)
                assert L.jv_fp8_counters_needed(16, N, K, cus) == 0, (cus, N, K)


def test_packed_layout_sizes_are_host_logic(product_lib):
    L = product_lib
    assert L.jv_fp8_packed_codes_bytes(16, 4096) == 16 * 4096
    assert L.jv_fp8_packed_codes_bytes(17, 4096) == 32 * 4096   # rows pad to 16
    assert L.jv_fp8_packed_codes_bytes(1, 128) == 16 * 128
    assert L.jv_fp8_packed_codes_bytes(65, 4096) == 80 * 4096   # prefill batches too
    assert L.jv_fp8_packed_codes_bytes(2048, 12288) == 2048 * 12288
    assert L.jv_fp8_packed_codes_bytes(-1, 4096) == -1
    assert L.jv_fp8_packed_codes_bytes(16, 100) == -1           # K must be a multiple of 128


def test_hook_library_exports(hooks_lib):
    for name in ("th_encode", "th_encode_sweep", "th_quotient_sweep", "th_mfma32", "th_mfma16", "th_silu_sweep", "th_gemm_form"):
        assert hasattr(hooks_lib, name)
