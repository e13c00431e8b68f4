"""Host emulation of the LDS address maps of the GEMM and skinny kernels (no
GPU): every DMA'd 16-byte chunk lands in one slot of its stage, each slot is
written once, every fragment read finds the k chunk the MFMA lane map asks
for, reads stay inside their operand's region, and the 16 lanes that LDS
serves together hit 16 distinct 16-byte bank groups. The formulas restate
the index arithmetic of gemm_w8_kernel, gemm_pc_kernel (miori_amd/csrc/
gemm.hip) and the skinny kernel's x tile (miori_amd/csrc/skinny.hip); a
change to one of them that breaks a mapping fails here before any GPU run."""
import numpy as np
import pytest

ROWB = 128  # bytes per LDS row of a bf16 K tile (64 elements)


def _swz_chunk(r, c):
    """Logical 16-byte chunk stored at physical chunk c of LDS row r."""
    return c ^ (r & 7) ^ ((r >> 3) & 1)


def _check_frag_reads(addr_of, rows_of, region, want_chunk):
    """addr_of(lane) -> byte address; rows_of(lane) -> tile row; checks the
    chunk read, the region bound and banks for one 64-lane read."""
    lo, hi = region
    for grp in range(4):
        banks = set()
        for lane in range(16 * grp, 16 * grp + 16):
            a = addr_of(lane)
            assert lo <= a and a + 16 <= hi, (lane, a, region)
            r = rows_of(lane)
            assert a - lo == r * ROWB + (a - lo) % ROWB
            phys = ((a - lo) % ROWB) // 16
            assert _swz_chunk(r, phys) == want_chunk(lane), (lane, r, phys)
            banks.add((a // 16) % 16)
        assert len(banks) == 16, f"bank groups {sorted(banks)}"


def _check_dma(writes, size):
    """writes: iterable of (slot byte address, row, logical chunk); every
    16-byte slot of [0, size) written once, holding the chunk its swizzle
    position says."""
    seen = {}
    for a, r, kb in writes:
        assert 0 <= a < size and a % 16 == 0
        assert a not in seen, f"slot {a} written twice"
        seen[a] = (r, kb)
    assert len(seen) == size // 16, "every slot of the stage is written"
    for a, (r, kb) in seen.items():
        assert _swz_chunk(r, (a % ROWB) // 16) == kb


@pytest.mark.parametrize("BM,BN", [(192, 256), (256, 256)])
def test_eight_wave_maps(BM, BN):
    WM, WN = BM // 2, BN // 4
    A_ST, B_ST = BM * ROWB, BN * ROWB
    PW = (BM + BN) // 8 // 8
    writes = []
    for w in range(8):
        for p in range(PW):
            g = w * PW + p
            is_a = g < BM // 8
            base = g * 8 * ROWB if is_a else A_ST + (g - BM // 8) * 8 * ROWB
            for lane in range(64):
                r = (g if is_a else g - BM // 8) * 8 + (lane >> 3)
                kb = (lane & 7) ^ (r & 7) ^ ((r >> 3) & 1)
                writes.append((base + lane * 16, r + (0 if is_a else BM), kb))
    # rows of B follow A's in one stage: row index counted over the stage
    _check_dma(((a, a // ROWB, kb) for a, _, kb in writes), A_ST + B_ST)
    for wave in range(8):
        wm, wn = wave >> 2, wave & 3
        for ks in range(2):
            def c0(lane):
                return (2 * (lane >> 4)) ^ ((lane & 7) ^ ((lane >> 3) & 1))
            for i in range(WM // 16):
                _check_frag_reads(
                    lambda lane: wm * WM * ROWB + ((c0(lane) ^ ks) << 4) + (lane & 15) * ROWB + i * 16 * ROWB,
                    lambda lane: wm * WM + 16 * i + (lane & 15), (0, A_ST),
                    lambda lane: 2 * (lane >> 4) + ks)
            for j in range(WN // 16):
                _check_frag_reads(
                    lambda lane: A_ST + wn * WN * ROWB + ((c0(lane) ^ ks) << 4) + (lane & 15) * ROWB + j * 16 * ROWB,
                    lambda lane: wn * WN + 16 * j + (lane & 15), (A_ST, A_ST + B_ST),
                    lambda lane: 2 * (lane >> 4) + ks)
    # epilogue staging of 8 waves x 32 rows x (WN + 8) floats inside the ring
    assert 8 * 32 * (WN + 8) * 4 <= 2 * (A_ST + B_ST)


@pytest.mark.parametrize("BM,BN", [(256, 128), (192, 128), (128, 128)])
def test_producer_consumer_maps(BM, BN):
    WM, WN = BM // 2, BN // 2
    A_ST, B_ST = BM * ROWB, BN * ROWB
    PA, PB = BM // 32, BN // 32
    for is_a, PX, ST in ((True, PA, A_ST), (False, PB, B_ST)):
        writes = []
        for w4 in range(4):
            for p in range(PX):
                r0 = (w4 * PX + p) * 8
                for lane in range(64):
                    r = r0 + (lane >> 3)
                    kb = (lane & 7) ^ (r & 7) ^ ((r >> 3) & 1)
                    writes.append((r0 * ROWB + lane * 16, r, kb))
        _check_dma(writes, ST)
    for w4 in range(4):
        wm, wn = w4 >> 1, w4 & 1
        for ks in range(2):
            def c0(lane):
                return (2 * (lane >> 4)) ^ ((lane & 7) ^ ((lane >> 3) & 1))
            for i in range(WM // 16):
                _check_frag_reads(
                    lambda lane: wm * WM * ROWB + ((c0(lane) ^ ks) << 4) + (lane & 15) * ROWB + i * 16 * ROWB,
                    lambda lane: wm * WM + 16 * i + (lane & 15), (0, A_ST),
                    lambda lane: 2 * (lane >> 4) + ks)
            for j in range(WN // 16):
                _check_frag_reads(
                    lambda lane: wn * WN * ROWB + ((c0(lane) ^ ks) << 4) + (lane & 15) * ROWB + j * 16 * ROWB,
                    lambda lane: wn * WN + 16 * j + (lane & 15), (0, B_ST),
                    lambda lane: 2 * (lane >> 4) + ks)


@pytest.mark.parametrize("KB,nloc,xrows", [
    (128, 16, 8), (128, 16, 32), (128, 17, 9), (64, 33, 12), (64, 32, 32), (128, 4, 5),
    (64, 40, 7), (128, 64, 16),
])
def test_skinny_x_tile_map(KB, nloc, xrows):
    """The x tile: row r at r * rsb bytes, chunk ch of row r at chunk
    ch ^ (r & 15); DMA u fills bytes [1024u, 1024u + 1024), lane -> its slot's
    source chunk (clamped into the row)."""
    kw = nloc * KB                    # elements of the workgroup's K range
    rsb = ((kw + 127) // 128) * 128 * 2
    nch = kw // 8
    nins = (xrows * rsb + 1023) // 1024
    tile = nins * 1024
    held = {}
    inv_d = np.float32(1.0) / np.float32(rsb >> 8)
    for u in range(nins):
        for lane in range(64):
            p = u * 1024 + lane * 16
            # the kernel's division-free row: trunc((a + 1/2) * (1/d)) in fp32
            a = u * 4 + (lane >> 4)
            r = int((np.float32(a) + np.float32(0.5)) * inv_d)
            assert r == p // rsb
            rr = min(r, xrows - 1)
            ch = min(((p - r * rsb) >> 4) ^ (r & 15), nch - 1)
            assert p + 16 <= tile
            held[p] = (rr, ch, r)
    # every valid (row, chunk) is read from the slot that holds it
    for row in range(xrows):
        for ch in range(nch):
            a = row * rsb + ((ch ^ (row & 15)) << 4)
            assert a + 16 <= tile
            rr, hch, r = held[a]
            assert r == row and rr == row and hch == ch, (row, ch, held[a])
    # a fragment read: lanes j = 0..15 of one quarter read rows j at one chunk
    if xrows >= 16:
        for ch in range(0, nch, 3):
            banks = {((j * rsb + ((ch ^ j) << 4)) // 16) % 16 for j in range(16)}
            assert len(banks) == 16


@pytest.mark.parametrize("rows,nfrag", [(256, 8), (192, 6), (128, 4), (64, 2)])
def test_mfma32_fragment_map(rows, nfrag):
    """The 32x32x16 fragment reads of gemm_kernel and gemm_pcq_kernel: in
    k-step ks (four per 64-deep K tile) lane half h = lane / 32 reads chunk
    4h + ks of row (lane % 32) + 32 i, at chunk (4h ^ f) ^ ks with f the
    row's swizzle term. LDS serves 16 lanes at a time; each group of 16
    reads 16 rows of one chunk column."""
    region = (0, rows * ROWB)
    for ks in range(4):
        def c0(lane):
            return (4 * (lane >> 5)) ^ ((lane & 7) ^ ((lane >> 3) & 1))
        for i in range(nfrag):
            _check_frag_reads(
                lambda lane: ((c0(lane) ^ ks) << 4) + (lane & 31) * ROWB + i * 32 * ROWB,
                lambda lane: 32 * i + (lane & 31), region,
                lambda lane: 4 * (lane >> 5) + ks)


@pytest.mark.parametrize("K,rows", [(2048, 16), (2048, 32), (1024, 9), (4096, 16)])
def test_lm_head_x_tile_map(K, rows):
    """The persistent 8-bit lm_head kernel's x tile (skinny.hip lmh_kernel):
    row r at r * 2K bytes, 1 KiB DMA ch of row r fills chunks ch*64 .. +63,
    lane l fetching logical chunk ch*64 + (l ^ (r & 15)); a read of logical
    chunk L (a block's base, a multiple of 16 chunks, plus an offset below
    16) addresses chunk L ^ (r & 15)."""
    XR = 2 * K
    held = {}
    for r in range(rows):
        for ch in range(K // 512):
            for lane in range(64):
                held[r * XR + ch * 1024 + lane * 16] = (r, ch * 64 + (lane ^ (r & 15)))
    assert len(held) == rows * K // 8
    for r in range(rows):
        for L in range(K // 8):
            a = r * XR + ((L ^ (r & 15)) << 4)
            assert held[a] == (r, L)
    if rows >= 16:
        for L in range(0, K // 8, 5):
            banks = {((j * XR + ((L ^ j) << 4)) // 16) % 16 for j in range(16)}
            assert len(banks) == 16


@pytest.mark.parametrize("nins,grid", [(128, 256), (33, 256), (7, 64), (128, 8), (5, 3)])
def test_rotated_x_dma_order_covers_tile(nins, grid):
    """MIORI_SKINNY_XROT: the skinny kernel's x-tile DMAs in rotated order
    (start r0 = (blockIdx / 8) % per_xcd * nins / per_xcd, wave w taking
    v = w, w + 8, ... and DMA u = (v + r0) mod nins), and lmh_kernel's
    (r0 = blockIdx * 37 mod nx): every DMA of the tile issued exactly once
    per workgroup, so the tile's contents do not depend on the order."""
    per_xcd = max(1, grid >> 3)
    for bid in range(grid):
        for r0 in ((bid >> 3) % per_xcd * nins // per_xcd, (bid * 37) % nins):
            assert 0 <= r0 < nins
            us = []
            for w in range(8):
                for v in range(w, nins, 8):
                    us.append(v + r0 if v + r0 < nins else v + r0 - nins)
            assert sorted(us) == list(range(nins))


def test_fp32_row_division_exhaustive():
    """The skinny kernel's x-tile DMA loop takes a slot's row as
    trunc((a + 1/2) * fp32(1/d)) instead of a // d (a = slot / 256 bytes,
    d = row bytes / 256). Every a < 2^11 and d <= 64 the kernel can see
    (x tile <= 32 rows of <= 16 KiB) gives the integer quotient."""
    a = np.arange(1 << 11, dtype=np.int64)
    for d in range(1, 65):
        inv = np.float32(1.0) / np.float32(d)
        q = ((a.astype(np.float32) + np.float32(0.5)) * inv).astype(np.int64)
        assert np.array_equal(q, a // d), d


@pytest.mark.parametrize("BM,EPR", [(256, 128), (192, 64), (128, 128)])
def test_fused_epilogue_passes_cover_the_wave_tile(BM, EPR):
    """gemm_pcq_kernel's epilogue (gemm.hip store_wave_tile / store_wave_rows
    with the fused form's wave tile, BM rows x 32 columns of 32x32 MFMA
    tiles): pass ps stages MFMA tiles [ps*EPR/32, (ps+1)*EPR/32) into rows
    (i - ps*EPR/32)*32 + 8*(e/4) + 4*(lane/32) + e%4 of an EPR x (32 + 8)
    fp32 region, column lane % 32; the read-back stores row ps*EPR + r.
    Every element of the BM x 32 tile is staged once and lands on its own
    output row and column; the four waves' regions fit the kernel's LDS
    (three stages of BM x 128 bytes of A and of 128 x 128 bytes)."""
    WN, RS = 32, 40
    TM = BM // 32
    assert BM % EPR == 0 and EPR % 32 == 0
    assert 4 * EPR * RS * 4 <= 3 * BM * 128 + 3 * 128 * 128
    seen = {}
    for ps in range(BM // EPR):
        region = {}
        for i in range(TM):
            if i < ps * (EPR // 32) or i >= (ps + 1) * (EPR // 32):
                continue
            for lane in range(64):
                for e in range(16):
                    r = (i - ps * (EPR // 32)) * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)
                    assert 0 <= r < EPR
                    key = (r, lane & 31)
                    assert key not in region
                    # the MFMA element's true position in the wave tile
                    region[key] = (32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3), lane & 31)
        for (r, c), src in region.items():
            out = (ps * EPR + r, c)
            assert out == src
            assert out not in seen
            seen[out] = True
    assert len(seen) == BM * WN


@pytest.mark.parametrize("BM,BN", [(256, 128), (192, 128), (128, 128)])
def test_producer_consumer_epilogue_covers_the_wave_tile(BM, BN):
    """gemm_pc_kernel's epilogue (store_wave_tile16): each consumer wave's
    (BM/2) x (BN/2) tile of 16x16 MFMA tiles is staged EPR rows per pass
    (EPR = BM/2 when the four waves' regions of EPR x (BN/2 + 8) floats fit
    the kernel's LDS, else 32), element e of lane l of tile (i, j) at row
    (i - ps*EPR/16)*16 + 4*(l/16) + e, column 16j + l%16, and read back as
    row ps*EPR + r. Every element lands once, on its own row and column."""
    WM, WN = BM // 2, BN // 2
    RS = WN + 8
    lds = 3 * BM * 128 + 3 * BN * 128
    EPR = WM if 4 * WM * RS * 4 <= lds else 32
    assert WM % EPR == 0 and EPR % 32 == 0
    seen = set()
    for ps in range(WM // EPR):
        region = {}
        for i in range(WM // 16):
            if i < ps * (EPR // 16) or i >= (ps + 1) * (EPR // 16):
                continue
            for j in range(WN // 16):
                for lane in range(64):
                    for e in range(4):
                        r = (i - ps * (EPR // 16)) * 16 + 4 * (lane >> 4) + e
                        c = j * 16 + (lane & 15)
                        assert 0 <= r < EPR and (r, c) not in region
                        region[(r, c)] = (16 * i + 4 * (lane >> 4) + e, c)
        for (r, c), src in region.items():
            assert (ps * EPR + r, c) == src and src not in seen
            seen.add(src)
    assert len(seen) == WM * WN


@pytest.mark.parametrize("depth,nbpt", [(16, 16), (16, 32), (32, 32), (32, 64)])
def test_lm_head_xsum_reads_the_block_fragments(depth, nbpt):
    """MIORI_LMH_XSUM: the x sums of block kb are made from the x-tile bytes
    at (kb & ~1) * 128 + xa[kb & 1] (xa the per-lane row and swizzled chunk
    offset), while the per-block code reads block i of the chunk starting
    at kb0 (a multiple of DEPTH) at kb0 * 128 + (i / 2) * 256 + xa[i % 2]:
    the same bytes for every kb; and the sums' slots ((kb * MT + mt) * 4 + c)
    * 16 bytes, read at xsum + kb0 * MT * 64 + ((i * MT + mt) * 4 + c) * 16,
    agree too."""
    for MT in (1, 2):
        for kb0 in range(0, nbpt, depth):
            for i in range(depth):
                kb = kb0 + i
                assert kb0 * 128 + (i // 2) * 256 == (kb & ~1) * 128 and i % 2 == kb & 1
                for mt in range(MT):
                    for c in range(4):
                        assert (kb0 * MT * 64 + ((i * MT + mt) * 4 + c) * 16
                                == ((kb * MT + mt) * 4 + c) * 16)
