"""Host emulation of the GEMM kernels' workgroup decomposition (no GPU).

Every GEMM kernel in miori_amd/csrc/gemm.hip maps its workgroup index the
same way: with `remap` on and a grid that is a multiple of 8, the hardware
index (dealt round-robin over the 8 XCDs) becomes pid = (b % 8) * (nwg / 8)
+ b / 8, so each XCD gets a contiguous run of tiles; then tile = pid %
ntiles, ksp = pid / ntiles, tm = tile % tiles_m, tn = tile / tiles_m, and
split ksp takes K tiles [KT_ALL * ksp / SK, KT_ALL * (ksp + 1) / SK). The
checks: the remap is a bijection, and every (row tile, column tile, K tile)
of the padded grid is computed by exactly one workgroup, for each tile shape
the dispatcher uses (the 192x128 tiles included) at the BASELINE config-3/4
shapes, ragged shapes and the K splits the cost model can pick."""
import pytest

BK = 64
TILES = [(256, 128), (192, 128), (128, 128), (64, 128), (64, 64), (192, 256), (256, 256)]
SHAPES = [(256, 8192, 2048), (256, 2048, 8192), (256, 2560, 2048), (1024, 8192, 2048),
          (1024, 2048, 8192), (1024, 2560, 2048), (1472, 8192, 2048), (1472, 2048, 8192),
          (1472, 2560, 2048), (1400, 8000, 2048), (1500, 8208, 2048), (300, 2048, 8192)]


def remap(b, nwg, on=True):
    if on and nwg % 8 == 0:
        return (b & 7) * (nwg >> 3) + (b >> 3)
    return b


@pytest.mark.parametrize("nwg", [8, 16, 96, 192, 256, 384, 512, 768, 1000, 7])
def test_remap_is_a_bijection(nwg):
    assert sorted(remap(b, nwg) for b in range(nwg)) == list(range(nwg))


@pytest.mark.parametrize("BM,BN", TILES)
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_grid_covers_every_tile_and_k_tile_once(BM, BN, M, N, K):
    tiles_m = (M + BM - 1) // BM
    tiles_n = (N + BN - 1) // BN
    ntiles = tiles_m * tiles_n
    kt_all = K // BK
    for SK in (1, 2, 3, 4, 8):
        if kt_all // SK < 1:
            continue
        nwg = ntiles * SK
        seen = {}
        for b in range(nwg):
            pid = remap(b, nwg)
            tile, ksp = pid % ntiles, pid // ntiles
            tm, tn = tile % tiles_m, tile // tiles_m
            kt0 = kt_all * ksp // SK
            kt1 = kt_all * (ksp + 1) // SK
            assert kt1 > kt0
            for kt in range(kt0, kt1):
                key = (tm, tn, kt)
                assert key not in seen, (key, b, seen.get(key))
                seen[key] = b
        assert len(seen) == tiles_m * tiles_n * kt_all
        # the padded grid covers the output
        assert tiles_m * BM >= M and tiles_n * BN >= N


def _nbw_of(K, kb, nw):
    per = (K // kb + nw - 1) // nw
    return 1 if per <= 1 else 2 if per <= 2 else 4 if per <= 4 else 8


@pytest.mark.parametrize("K,KB", [(2048, 128), (8192, 128), (2048, 64), (4096, 64), (1024, 128),
                                  (8704, 128), (8448, 64), (384, 128)])
@pytest.mark.parametrize("SK", [1, 2, 4])
@pytest.mark.parametrize("NWV", [4, 8])
def test_skinny_k_blocks_covered_once(K, KB, SK, NWV):
    """skinny.hip: K is cut into nblk = K / KB blocks, split SK ways over
    gridDim.y (nloc = nblk / SK each, kb0 = y * nloc); wave w of a workgroup
    takes blocks [kb0 + w*nloc/NWV, kb0 + (w+1)*nloc/NWV), in NBW slots
    (nbw_of rounding) of which those past its count are padding (masked).
    Every block is computed once, and no wave has more blocks than slots."""
    nblk = K // KB
    if nblk % SK:
        pytest.skip("the launcher only splits K into whole blocks")
    nloc = nblk // SK
    nbw = _nbw_of(K // SK, KB, NWV)
    if nbw * NWV < nloc:
        pytest.skip("shape outside the kernel's 8-blocks-per-wave limit (rejected)")
    seen = []
    for y in range(SK):
        kb0 = y * nloc
        for w in range(NWV):
            b0, b1 = kb0 + w * nloc // NWV, kb0 + (w + 1) * nloc // NWV
            assert b1 - b0 <= nbw
            for i in range(nbw):
                if i < b1 - b0:
                    seen.append(min(b0 + i, nblk - 1))
    assert sorted(seen) == list(range(nblk))


@pytest.mark.parametrize("M", [5, 8, 9, 16, 17, 24, 31, 32])
def test_skinny_m_split_covers_rows_once(M):
    """The M split over gridDim.z (two workgroups of one 16-row m-tile each
    above M = 8): z takes rows [z * ceil(M / 2), min(M, (z + 1) * ceil(M / 2)))
    and stores only those; every row once."""
    for gz in (1, 2):
        mstep = M if gz == 1 else (M + gz - 1) // gz
        rows = []
        for z in range(gz):
            m0 = z * mstep
            rows += list(range(m0, min(M, m0 + mstep)))
        assert sorted(rows) == list(range(M))
        # one 16-row m-tile per workgroup when split (MT = 1), two otherwise
        assert mstep <= (16 if gz == 2 else 32)
