"""The fp32 tile planner (ml-edsl_amd/csrc/plan_f32.cpp), on the CPU.

plan_f32.cpp holds the shipped tile table and the planner and needs no HIP,
so it is built here with g++ beside a small driver (tests/plan/plan_driver.cpp)
and asked for the plans of the BASELINE layers, their 8-way column shards and
the shapes the GPU tests pin (tests/test_gpu_edge_tiles.py). The GPU tests
check the same plans through the library on the device.
"""
from __future__ import annotations

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "ml-edsl_amd", "csrc")
CUS = 256  # MI355X


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("plan") / "plan_driver")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-o", exe,
                    os.path.join(ROOT, "tests", "plan", "plan_driver.cpp"), os.path.join(CSRC, "plan_f32.cpp")],
                   check=True)
    return exe


def plans(driver, queries):
    text = "".join(f"{M} {N} {K} {int(al)} {cus}\n" for M, N, K, al, cus in queries)
    out = subprocess.run([driver], input=text, capture_output=True, text=True, check=True).stdout
    return out.split()


def table(driver):
    out = subprocess.run([driver], input="table\n", capture_output=True, text=True, check=True).stdout
    return [line.split() for line in out.splitlines()]


# (M, K, N), aligned operands, the plan
PINNED = [
    # BASELINE layers that take the tiles (C4 takes the small-M kernel)
    ((256, 256, 256), True, "f32_16x16x64_direct_k4"),             # C1
    ((1024, 1024, 1024), True, "f32_64x64x64_direct_rc"),          # C2
    ((4096, 4096, 4096), True, "f32_128x128x16_direct"),           # C3
    ((2048, 2048, 2048), True, "f32_64x64x16_direct"),
    ((4096, 4096, 512), True, "f32_64x64x64_direct_k4"),           # C3 column shard (N = 512)
    # tests/test_gpu_edge_tiles.py
    ((1000, 1000, 1000), True, "f32_64x64x64_direct_k4_edge"),
    ((4000, 256, 4000), True, "f32_128x128x16_direct_edge"),
    ((4097, 256, 4096), True, "f32_64x64x64_mfma16_edge"),
    ((512, 1000, 512), True, "f32_32x32x64_direct_rc_edge"),
    ((4096, 1024, 4096), True, "f32_128x128x16_direct"),
    ((3072, 512, 3072), True, "f32_64x64x64_direct_k4"),
    ((2001, 2001, 2001), True, "f32_128x128x32_mfma16_anyshape"),  # K % 4 != 0
    ((1025, 1025, 1025), True, "f32_64x64x64_w2x2_k2_pf2_anyshape"),
    ((2048, 2048, 2048), False, "f32_128x128x32_mfma16_anyshape"),
    ((4001, 1001, 4001), True, "f32_256x256x16_w4x4_anyshape"),
    # layers of at most 64 rows the small-M kernel does not take
    ((16, 4096, 50257), False, "f32_32x32x64_w1x1_k4_pf4_anyshape"),
    ((64, 256, 4096), True, "f32_32x32x64_w1x1_k4_pf4"),
    ((70, 37, 50), True, "f32_32x32x64_w1x1_k4_pf4_anyshape"),
    # exactly one 64x64 tile per CU, any shape: loads four K steps ahead
    ((1024, 1025, 1024), True, "f32_64x64x32_w2x2_k2_pf4_anyshape"),
    # K = 0: the element-checked tile writes the epilogue of the bias
    ((100, 0, 100), True, "f32_64x64x16_w2x2_guard"),
    # 2304 one-wave 128x128 tiles would leave the last round three quarters empty
    ((6144, 6144, 6144), True, "f32_64x64x64_direct_k4"),
    # short K stays on the LDS-staged tiles: one 128x128 tile per CU, then 64x64
    ((2048, 128, 2048), True, "f32_128x128x32_mfma16_w8"),
    ((1024, 128, 1024), True, "f32_64x64x64_mfma16"),
    # R x C one-wave tiles, K split four ways: one round of workgroups ...
    ((512, 512, 512), True, "f32_32x32x64_direct_rc"),
    ((768, 768, 768), True, "f32_48x48x64_direct_rc"),
    ((720, 768, 720), True, "f32_48x48x64_direct_rc"),
    ((768, 784, 768), True, "f32_48x48x64_direct_rc"),      # K a multiple of 16, not of 64
    # ... and their edge twins
    ((1500, 1500, 1500), True, "f32_96x96x64_direct_rc_edge"),
    ((760, 760, 760), True, "f32_48x48x64_direct_rc_edge"),
    ((500, 500, 500), True, "f32_32x32x64_direct_rc_edge"),
    ((1200, 1204, 1200), True, "f32_80x80x64_direct_rc_edge"),  # K a multiple of 4 only
    # two rounds of partial 64x64 tiles against one of 80x80
    ((1500, 1000, 1000), True, "f32_80x80x64_direct_rc_edge"),
    ((1200, 1024, 1200), True, "f32_80x80x64_direct_rc"),
    ((1536, 512, 1536), True, "f32_96x96x64_direct_rc"),
    ((1536, 1024, 720), True, "f32_96x48x64_direct_rc"),
    ((720, 1024, 1536), True, "f32_48x96x64_direct_rc"),
    # ... or several, with tiles of 64 and more that read no more per output than 64x64
    ((2304, 2304, 2304), True, "f32_64x64x64_direct_k4"),    # 48x96 over 4.5 rounds: not taken
    ((2560, 1024, 2560), True, "f32_80x80x64_direct_rc"),
    # too few tiles for half the CUs, and even cost against 64x64
    ((256, 1024, 256), True, "f32_32x32x64_w1x1_k4_pf4"),
    # two rounds of 32x32 at half the cost of a half-full round of 64x64
    ((128, 4096, 4096), True, "f32_32x32x64_direct_rc"),
    # edge twins need K >= 384
    ((96, 256, 4096), True, "f32_32x32x64_w1x1_k4_pf4"),
    ((96, 4096, 4096), True, "f32_48x48x64_direct_rc_edge"),
    ((500, 512, 2304), True, "f32_80x80x64_direct_rc_edge"),
    # 48x96 over three rounds lost to 64x64 (79.6 against 72.2 us)
    ((1536, 1024, 2304), True, "f32_64x64x64_direct_k4"),
    # a round three quarters full of 64x64 beats three rounds of 32x32
    ((192, 4096, 4096), True, "f32_64x64x64_direct_rc"),
    ((3072, 3072, 3072), True, "f32_64x64x64_direct_k4"),
]


def test_pinned_plans(driver):
    got = plans(driver, [(M, N, K, al, CUS) for (M, K, N), al, _ in PINNED])
    want = [p for _, _, p in PINNED]
    assert got == want, [(s, g, w) for (s, _, w), g in zip(PINNED, got) if g != w]


def test_table_is_named_and_every_tile_is_planned(driver):
    """Names are unique and every shipped configuration is the plan of some
    layer: the table holds no configuration the planner cannot reach."""
    rows = table(driver)
    names = [r[1] for r in rows]
    assert len(names) == len(set(names)) == 34
    dims = [1, 4, 17, 64, 65, 100, 128, 256, 257, 500, 512, 720, 768, 1000, 1024, 1025, 1536, 2000, 2048, 2304,
            3000, 4096, 4097, 6000, 6144]
    queries = [(M, N, K, al, CUS) for M in dims for N in dims for K in dims + [0] for al in (0, 1)]
    reached = set(plans(driver, queries))
    assert reached == set(names), set(names) - reached


def test_plans_follow_the_bounds_rules(driver):
    """A plan's bounds variant always fits the operands: exact tiles only
    where the tile divides the layer, 16-byte tiles only on aligned rows with
    K and N multiples of 4."""
    rows = {r[1]: tuple(int(v) for v in r[2:]) for r in table(driver)}
    dims = [3, 16, 65, 96, 128, 255, 256, 1000, 1024, 1030, 4096]
    queries = [(M, N, K, al, CUS) for M in dims for N in dims for K in dims for al in (0, 1)]
    for (M, N, K, al, _), name in zip(queries, plans(driver, queries)):
        bm, bn, bk, guard = rows[name]
        if guard == 0:  # exact
            assert al and M % bm == 0 and N % bn == 0 and K % bk == 0, (M, N, K, name)
        elif guard == 1:  # edge tiles
            assert al and K % 4 == 0 and N % 4 == 0 and K >= 4 and N >= 4, (M, N, K, name)


def test_one_wave_tiles_need_32_bit_buffer_offsets(driver):
    """The one-wave tiles address A and B through buffer descriptors with
    32-bit byte offsets: a row stride that puts K rows of B (or 128 rows of
    A) past 2^31 bytes must plan an LDS-staged tile instead."""
    def plan(M, N, K, lda, ldb):
        out = subprocess.run([driver], input=f"{M} {N} {K} 1 {CUS} {lda} {ldb}\n", capture_output=True,
                             text=True, check=True).stdout
        return out.split()[0]
    assert plan(4096, 4096, 4096, 4096, 4096) == "f32_128x128x16_direct"
    assert plan(1024, 1024, 1024, 1024, 1024) == "f32_64x64x64_direct_rc"
    # K rows of B past 2^31 bytes: 4096 rows of 2^17 floats = 2 GiB
    big_ldb = 1 << 17
    assert "direct" not in plan(4096, 4096, 4096, 4096, big_ldb)
    assert "direct" not in plan(1024, 1024, 1024, 1024, 1 << 19)
    # 128 rows of A past 2^31 bytes
    assert "direct" not in plan(4096, 4096, 4096, 1 << 22, 4096)
    # just inside: (K + 16) * ldb * 4 + 1024 <= 2^31 - 1
    ldb_ok = ((2**31 - 1 - 1024) // ((4096 + 16) * 4)) // 4 * 4
    assert plan(4096, 4096, 4096, 4096, ldb_ok) == "f32_128x128x16_direct"
    assert "direct" not in plan(4096, 4096, 4096, 4096, ldb_ok + 4 * 64)
