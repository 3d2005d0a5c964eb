"""Launch plans of the tile kernels checked on the CPU (qlinear_check_launch_plan, no GPU): for
ragged M and N, every kernel configuration, split count and several CU counts, every workgroup of
every launch maps through the kernels' own xcd_remap / tile_coords to a tile that starts inside
M x N (or to a 256 x 256 half wholly past M, which the kernel leaves before any memory access),
every tile part is covered exactly once, and the workspace holds every split-K partial.

Guards the fault class of a workgroup whose tile lies past the edge of its operands (once: a
128-row half wholly past M built an activation buffer descriptor with a wrapped range).
"""
import itertools
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "comfy_ui_gfx906_tools_amd", "libqlinear.so")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.skip("libqlinear.so not built (python -m comfy_ui_gfx906_tools_amd.build)")
    from comfy_ui_gfx906_tools_amd import _lib
    return _lib.load_library(LIB)


def _check(lib, *args):
    rc = lib.qlinear_check_launch_plan(*args)
    assert rc == 0, f"{args}: {lib.qlinear_last_error().decode()}"


MS = [1, 2, 5, 16, 17, 63, 64, 65, 127, 128, 129, 200, 255, 256, 257, 383, 384, 385, 512, 513, 640, 1000, 2049, 4608]
NS = [16, 100, 255, 256, 257, 520, 777, 3072, 12288]
CUS = [8, 80, 256, 304]


@pytest.mark.parametrize("cus", CUS)
def test_w4a16_plans_every_configuration(lib, cus):
    flags_cfg = lambda c: (c + 1) << 8  # noqa: E731 - QL_W4A16_CFG(c)
    for M, N in itertools.product(MS, NS):
        for K in (64, 640, 3072):
            for xdt in (1, 2):  # fp16 / bf16 x
                _check(lib, 0, xdt, M, N, K, 0, 0, cus)              # automatic choice
                for c in range(7):
                    for splits in ((0, 1) if c in (4, 6) else (0, 1, 2, 7)):
                        _check(lib, 0, xdt, M, N, K, splits, flags_cfg(c), cus)


def test_w4a16_plans_k_tails_and_bf16_mode(lib):
    for M, N, K in itertools.product([3, 130, 300, 513], [200, 777], [32, 96, 160, 4160]):
        for flags in (0, 1, 1 | (1 + 1) << 8, (0 + 1) << 8):
            _check(lib, 0, 2, M, N, K, 0, flags, 256)


@pytest.mark.parametrize("cus", CUS)
def test_w8a8_and_w4a4_plans(lib, cus):
    for M, N in itertools.product(MS, NS):
        _check(lib, 1, 0, M, N, 3072, 0, 0, cus)
        for splits in (1, 2, 3, 8):
            _check(lib, 2, 0, M, N, 1024, splits, 0, cus)


def test_plan_check_reports_violations(lib):
    """The check itself rejects what it must: a bad op or CU count."""
    assert lib.qlinear_check_launch_plan(3, 0, 64, 64, 64, 0, 0, 256) != 0
    assert "op must be" in lib.qlinear_last_error().decode()
    assert lib.qlinear_check_launch_plan(0, 2, 64, 64, 64, 0, 0, 0) != 0



def test_describe_plan():
    """qlinear_w4a16_describe_plan reports the plan the GEMM makes: the C2 shapes on 256 CUs."""
    from comfy_ui_gfx906_tools_amd import _lib
    if not os.path.exists(LIB):
        pytest.skip("libqlinear.so not built")
    fc1 = _lib.w4a16_describe_plan(4608, 12288, 3072, cus=256)
    assert (fc1["config"], fc1["tile_rows"], fc1["tiles"], fc1["whole_tiles"], fc1["staged"]) == (5, 256, 864, 768, True)
    fc2 = _lib.w4a16_describe_plan(4608, 3072, 12288, cus=256, x_dtype=__import__("torch").float16)
    # 216 tiles of 256 rows would leave 40 CUs idle: 252 tiles of 224 rows, one round
    assert (fc2["config"], fc2["tile_rows"], fc2["tiles"], fc2["whole_tiles"], fc2["staged"]) == (5, 224, 252, 252, False)
    assert _lib.w4a16_describe_plan(4608, 3072, 12288, cus=256, splits=1)["tile_rows"] == 256
    assert _lib.w4a16_describe_plan(1, 10240, 4096, cus=256)["config"] == 7
    assert _lib.w4a16_describe_plan(16, 10240, 4096, cus=256)["config"] == 8
    assert _lib.w4a16_describe_plan(64, 10240, 4096, cus=256)["config"] == 2
    assert _lib.w4a16_describe_plan(100, 10240, 4032, cus=256)["config"] == 1
    assert _lib.w4a16_describe_plan(256, 10240, 4096, cus=256)["config"] == 1


def test_describe_plan_row_tiles():
    """Configuration 5 forced at small M: the shortest tile height that covers M (64 / 128 / 256),
    and K pieces enough for one per CU when the tiles fill fewer than half of them (each piece at
    least 4 stages of 64); an explicit split count is taken as given (up to the stage count)."""
    from comfy_ui_gfx906_tools_amd import _lib
    if not os.path.exists(LIB):
        pytest.skip("libqlinear.so not built")
    d = _lib.w4a16_describe_plan(64, 10240, 4096, config=5, cus=256)
    assert (d["tile_rows"], d["tiles"], d["whole_tiles"], d["k_pieces"]) == (64, 40, 0, 6)
    d = _lib.w4a16_describe_plan(100, 10240, 4096, config=5, cus=256)
    assert (d["tile_rows"], d["k_pieces"]) == (128, 6)
    d = _lib.w4a16_describe_plan(256, 10240, 4096, config=5, cus=256)
    assert (d["tile_rows"], d["k_pieces"]) == (256, 6)
    d = _lib.w4a16_describe_plan(64, 10240, 512, config=5, cus=256)  # 8 stages: 2 pieces of 4
    assert d["k_pieces"] == 2
    d = _lib.w4a16_describe_plan(64, 40960, 4096, config=5, cus=256)  # 160 tiles: whole
    assert (d["tile_rows"], d["whole_tiles"], d["k_pieces"]) == (64, 160, 1)
    d = _lib.w4a16_describe_plan(64, 10240, 4096, config=5, splits=3, cus=256)
    assert (d["whole_tiles"], d["k_pieces"]) == (0, 3)
    d = _lib.w4a16_describe_plan(64, 10240, 4096, config=5, splits=1, cus=256)
    assert (d["whole_tiles"], d["k_pieces"]) == (40, 1)


@pytest.mark.parametrize("cus", [80, 256, 304])
def test_w4a16_k_pieces_fit_one_round(cus):
    """Automatic plans (splits 0): the K pieces of the cut tiles fit one round of workgroups after
    the whole rounds, on both tile kernels (a second round of pieces measured 20-35% slower)."""
    from comfy_ui_gfx906_tools_amd import _lib
    if not os.path.exists(LIB):
        pytest.skip("libqlinear.so not built")
    import torch
    for M, N, K in itertools.product([17, 64, 100, 128, 200, 512, 768, 1024, 2049], [3072, 9216, 18432, 21504],
                                     [1024, 3072, 12288]):
        for xdt in (torch.float16, torch.bfloat16):
            d = _lib.w4a16_describe_plan(M, N, K, x_dtype=xdt, cus=cus)
            if d["config"] > 6 or d["k_pieces"] == 1:
                continue
            cut = d["tiles"] - d["whole_tiles"]
            assert cut * d["k_pieces"] <= cus, (M, N, K, xdt, cus, d)
