"""The prefill GEMM planner (host logic, no GPU): the launch forms it picks for the measured
shapes, and the invariants every pick keeps (kq4_gemm_plan_info, include/kq4.h). Planned for a
256-CU MI355X."""
import os

import pytest

CU = 256
Q4_STAGE, Q8_STAGE = 16, 8          # stream-layout blocks per stage
PART_MAX = 24 << 20                  # partial-sum bytes of the planner's splits, at most


@pytest.fixture(scope="module")
def kq4():
    import kq4 as m
    if not os.path.exists(m.LIB_PATH):
        pytest.fail(f"{m.LIB_PATH} not built (run `make -C kestrel-llm_amd`)")
    return m


# (rows, cols, tokens) -> (tile, K slices), tile 1 / 2 / 3 / 4 = 128x128 / 64x128 / 64x64 /
# 128x64: the choices the forced (tile, slices) sweeps on MI355X measured fastest or within the
# spread (Qwen3-8B gate 12288 x 4096, down 4096 x 12288, QKV 6144 x 4096; Qwen3-VL-2B QKV
# 4096 x 2048, gate 6144 x 2048, down 2048 x 6144)
PLANS = [
    ((12288, 4096), 32, (3, 4)), ((12288, 4096), 128, (2, 4)), ((12288, 4096), 256, (2, 2)),
    ((12288, 4096), 320, (2, 1)), ((12288, 4096), 512, (2, 1)), ((12288, 4096), 640, (1, 1)),
    ((12288, 4096), 768, (2, 1)),
    ((12288, 4096), 1536, (2, 1)), ((12288, 4096), 2048, (1, 1)), ((6144, 4096), 1536, (2, 1)),
    ((4096, 12288), 32, (3, 8)), ((4096, 12288), 128, (2, 8)), ((4096, 12288), 256, (2, 6)),
    ((4096, 12288), 512, (1, 4)), ((4096, 12288), 768, (2, 2)), ((4096, 12288), 1024, (1, 2)),
    ((4096, 12288), 1152, (2, 1)), ((4096, 12288), 1536, (2, 1)), ((4096, 12288), 1792, (1, 1)),
    ((4096, 12288), 2048, (1, 1)),
    ((6144, 4096), 512, (2, 2)),
    ((4096, 2048), 24, (3, 4)), ((4096, 2048), 256, (3, 1)),
    ((6144, 2048), 128, (3, 1)), ((6144, 2048), 768, (2, 1)),
    ((2048, 6144), 512, (2, 6)),
]


@pytest.mark.parametrize("shape,n,want", PLANS)
def test_measured_plans(kq4, shape, n, want):
    rows, cols = shape
    assert kq4.gemm_plan(n, rows, cols, chain=kq4.CHAIN_ASM, ncu=CU) == want


def test_small_batches_on_the_gemv(kq4):
    for n in (1, 8, 9, 16):
        assert kq4.gemm_plan(n, 4096, 12288, ncu=CU) == (0, 0)
    assert kq4.gemm_plan(17, 4096, 12288, ncu=CU) != (0, 0)
    with kq4.options(gemv_chunk_max=8):
        assert kq4.gemm_plan(12, 4096, 12288, chain=kq4.CHAIN_ASM, ncu=CU) == (3, 8)
    assert kq4.gemm_plan(12, 4096, 12288, q8=True, ncu=CU) != (0, 0)   # Q8_0: the GEMM


def test_forced_forms(kq4):
    with kq4.options(gemm_split=1):
        assert kq4.gemm_plan(128, 4096, 12288, chain=kq4.CHAIN_ASM, ncu=CU) == (3, 1)
    with kq4.options(gemm_tile=2, gemm_split=8):
        assert kq4.gemm_plan(300, 2000, 4096, ncu=CU) == (2, 8)
    with kq4.options(gemm_tile=2):      # the planner's slices for the forced tile
        assert kq4.gemm_plan(128, 4096, 12288, chain=kq4.CHAIN_ASM, ncu=CU) == (2, 8)
    with kq4.options(gemm_split=7):     # 384 blocks do not fill 7 whole-stage slices: none
        assert kq4.gemm_plan(2048, 4096, 12288, chain=kq4.CHAIN_ASM, ncu=CU)[1] == 1


def split_ok(nb, cb, k):
    """k slices of whole stages that all hold blocks (the launcher's condition)."""
    ks = (-(-nb // k) + cb - 1) // cb * cb
    return (k - 1) * ks < nb


@pytest.mark.parametrize("q8", [False, True])
def test_plan_invariants(kq4, q8):
    chains = (kq4.CHAIN_AUTO, kq4.CHAIN_GEMV32, kq4.CHAIN_Q8GEMM) if q8 else \
        (kq4.CHAIN_AUTO, kq4.CHAIN_CTILE, kq4.CHAIN_ASM)
    cb = Q8_STAGE if q8 else Q4_STAGE
    seen = set()
    for n in (17, 24, 33, 64, 100, 128, 200, 256, 384, 512, 640, 768, 1024, 1536, 2048, 4096):
        for rows in (64, 256, 1000, 2048, 4096, 6144, 12288, 32768):
            for cols in (256, 1024, 2016, 2048, 2080, 4096, 6144, 8192, 12288, 24576):
                for chain in chains:
                    tile, k = kq4.gemm_plan(n, rows, cols, q8=q8, chain=chain, ncu=CU)
                    seen.add((tile, k))
                    main = n & ~3 if (not q8 and chain == kq4.CHAIN_AUTO) else n
                    assert 1 <= tile <= 4 and 1 <= k <= 8, (n, rows, cols, chain, tile, k)
                    if chain == kq4.CHAIN_CTILE:          # two accumulator sets: never split,
                        assert k == 1 and tile in (2, 3)  # 64 x 128 at most
                    if cols < 2048:                       # below K = 2048 never split
                        assert k == 1, (n, rows, cols)
                    if k > 1:
                        assert split_ok(cols // 32, cb, k), (n, rows, cols, k)
                        assert (k - 1) * main * rows * 4 <= PART_MAX, (n, rows, cols, tile, k)
    assert {t for t, _ in seen} == {1, 2, 3}      # 128 x 64 only when forced
    assert max(k for _, k in seen) == 8
