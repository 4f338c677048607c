"""Host-side model of the fast kernels' LDS layouts (no GPU).

The gfx950 fast path copies operands into LDS with buffer-to-LDS DMA (lane l of
a wave instruction writes 16-byte slot l of a 1 KB block) under an XOR
swizzle, and reads MFMA fragments back with ds_read_b128 (K-contiguous
operands) or two ds_read_b64_tr_b16 (M/N-contiguous operands).  This test
replays that address arithmetic on a labelled tile and checks that every
lane's fragment holds exactly the (row, k) elements the 32x32x16 MFMA
expects: lane (l32, g) of K step kk needs k = 16*kk + 8*g + e, e = 0..7, of
row (or column) l32 of its 32-wide sub-tile.

ds_read_b64_tr_b16 semantics (measured on gfx950 with an in-bounds LDS probe):
within each 16-lane group, lane i receives element i % 4 of the 8-byte pieces
addressed by lanes 4*r + i // 4, r = 0..3.
"""
import numpy as np
import pytest

# ---- the kernel's swizzles and address formulas (gemm_gfx950.hip) ----------
def fk(row, bk=32):
    return ((row >> 1) ^ (row >> 3)) & 3 if bk == 32 else (row >> 1) & 7


def fm(k, granules):
    return ((0x7520 >> ((k & 3) * 4)) & 0xF) & (granules - 1)


def dma_kmajor(rows, waves, bk=32):
    """LDS byte -> (row, kcol) for the K-contiguous stage written by DMA."""
    lds = {}
    chunks = bk // 8
    instr = rows * bk * 2 // 1024 // waves
    for wave in range(waves):
        for i in range(instr):
            q = i * waves + wave
            for lane in range(64):
                r = (64 // chunks) * q + lane // chunks
                c = (lane % chunks) ^ fk(r, bk)
                for e in range(8):
                    lds[q * 1024 + lane * 16 + 2 * e] = (r, c * 8 + e)
    return lds


def dma_mnmajor(rows, waves, bk=32):
    """LDS byte -> (row, kcol) for the M/N-contiguous stage written by DMA."""
    lds = {}
    row_bytes = rows * 2
    granules = rows // 16
    instr = bk * row_bytes // 1024 // waves
    for wave in range(waves):
        for i in range(instr):
            base = (i * waves + wave) * 1024
            for lane in range(64):
                pos = base + lane * 16
                k = pos // row_bytes
                slot = (pos % row_bytes) // 16
                lg = (slot >> 1) ^ fm(k, granules)
                for e in range(8):
                    lds[pos + 2 * e] = (lg * 16 + (slot & 1) * 8 + e, k)
    return lds


def frag_kmajor(lds, wrow, sub, kk, bk=32):
    out = {}
    for lane in range(64):
        l32, g = lane & 31, lane >> 5
        row = wrow + l32
        ch = ((2 * kk + g) ^ fk(row, bk)) << 4
        addr = row * bk * 2 + sub * 32 * bk * 2 + ch
        out[lane] = [lds[addr + 2 * e] for e in range(8)]
    return out


def frag_mnmajor(lds, rows, wrow, sub, kk):
    """Two ds_read_b64_tr_b16 per fragment, addresses as in the kernel."""
    row_bytes = rows * 2
    granules = rows // 16
    addr = {}
    for h in range(2):
        for lane in range(64):
            r, q, gp, g = (lane >> 2) & 3, lane & 3, (lane >> 4) & 1, lane >> 5
            k = kk * 16 + 8 * g + 4 * h + r
            f = fm(k, granules)
            granule = (wrow >> 4) + 2 * sub + gp
            addr[(h, lane)] = k * row_bytes + ((granule ^ f) << 5) + q * 8
    out = {}
    for lane in range(64):
        grp, i = lane // 16, lane % 16
        vals = []
        for h in range(2):
            for r in range(4):
                src = 16 * grp + 4 * r + i // 4
                vals.append(lds[addr[(h, src)] + 2 * (i % 4)])
        out[lane] = vals
    return out


def expected(wrow, sub, kk):
    return {lane: [(wrow + sub * 32 + (lane & 31), 16 * kk + 8 * (lane >> 5) + e) for e in range(8)]
            for lane in range(64)}


# (rows, K per stage): 256x256 stages hold 64 K values, the smaller tiles 32
SHAPES = [(64, 32), (128, 32), (256, 32), (256, 64)]


@pytest.mark.parametrize("rows,bk", SHAPES)
def test_kmajor_dma_and_fragments(rows, bk):
    lds = dma_kmajor(rows, 4, bk)
    assert len(lds) == rows * bk                      # every element written once
    for wrow in range(0, rows, rows // 2 if rows >= 64 else 32):
        for sub in range(min(4, (rows // 2) // 32)):
            for kk in range(bk // 16):
                assert frag_kmajor(lds, wrow, sub, kk, bk) == expected(wrow, sub, kk)


@pytest.mark.parametrize("rows,bk", SHAPES)
def test_mnmajor_dma_and_transposed_fragments(rows, bk):
    lds = dma_mnmajor(rows, 4, bk)
    assert len(lds) == rows * bk
    wave_rows = rows // 2
    for wrow in (0, wave_rows):
        for sub in range(wave_rows // 32):
            for kk in range(bk // 16):
                assert frag_mnmajor(lds, rows, wrow, sub, kk) == expected(wrow, sub, kk)


def _banks(addrs, width):
    """Max accesses to one 4-byte bank among `addrs` (each a (byte, size) pair) per `width`-byte cycle."""
    hits = {}
    for a, size in addrs:
        for b in range(a, a + size, 4):
            bank = (b // 4) % (width // 4)
            hits.setdefault(bank, set()).add(b // width)
    return max(len(v) for v in hits.values())


@pytest.mark.parametrize("rows,bk", [(128, 32), (256, 32), (256, 64)])
def test_fragment_reads_are_bank_conflict_free(rows, bk):
    # ds_read_b128, K-contiguous: 16-lane phases over 256 bytes of banks
    for lane0 in range(0, 64, 16):
        for kk in range(bk // 16):
            addrs = []
            for lane in range(lane0, lane0 + 16):
                row = (lane & 31)
                addrs.append((row * bk * 2 + (((2 * kk + (lane >> 5)) ^ fk(row, bk)) << 4), 16))
            assert _banks(addrs, 256) == 1
    # ds_read_b64_tr_b16, M/N-contiguous: 32-lane phases over 256 bytes of banks
    row_bytes, granules = rows * 2, rows // 16
    for half in range(2):
        for sub in range(2):
            for kk in range(bk // 16):
                addrs = []
                for lane in range(32 * half, 32 * half + 32):
                    r, q, gp, g = (lane >> 2) & 3, lane & 3, (lane >> 4) & 1, lane >> 5
                    k = kk * 16 + 8 * g + r
                    addrs.append((k * row_bytes + (((2 * sub + gp) ^ fm(k, granules)) << 5) + q * 8, 8))
                assert _banks(addrs, 256) == 1


# ---- 16x16x32 MFMA fragments (256x256 tile, 64 K values per stage) ----------
# Lane (l16 = lane % 16, q = lane // 16) of K step kk (32 wide) needs row (or
# column) l16 of its 16-wide sub-tile and k = 32*kk + 8*q + e, e = 0..7.
def fm16(k, granules):
    return (((0x7520 >> ((k & 3) * 4)) & 0xF) ^ ((k >> 3) & 1)) & (granules - 1)


def dma_mnmajor16(rows, waves, bk=64):
    lds = {}
    row_bytes = rows * 2
    granules = rows // 16
    instr = bk * row_bytes // 1024 // waves
    for wave in range(waves):
        for i in range(instr):
            base = (i * waves + wave) * 1024
            for lane in range(64):
                pos = base + lane * 16
                k = pos // row_bytes
                slot = (pos % row_bytes) // 16
                lg = (slot >> 1) ^ fm16(k, granules)
                for e in range(8):
                    lds[pos + 2 * e] = (lg * 16 + (slot & 1) * 8 + e, k)
    return lds


def frag16_kmajor(lds, wrow, sub, kk, bk=64):
    out = {}
    for lane in range(64):
        l16, q = lane & 15, lane >> 4
        row = wrow + l16
        addr = row * bk * 2 + sub * 16 * bk * 2 + (((4 * kk + q) ^ fk(row, bk)) << 4)
        out[lane] = [lds[addr + 2 * e] for e in range(8)]
    return out


def frag16_mnmajor_addrs(rows, wcol, sub, kk, h):
    row_bytes = rows * 2
    granules = rows // 16
    addr = {}
    for lane in range(64):
        q, r, c = lane >> 4, (lane >> 2) & 3, lane & 3
        k = 32 * kk + 8 * q + 4 * h + r
        gi = (wcol >> 4) + sub
        addr[lane] = k * row_bytes + ((gi ^ fm16(k, granules)) << 5) + c * 8
    return addr


def frag16_mnmajor(lds, rows, wcol, sub, kk):
    a = [frag16_mnmajor_addrs(rows, wcol, sub, kk, h) for h in range(2)]
    out = {}
    for lane in range(64):
        grp, i = lane // 16, lane % 16
        vals = []
        for h in range(2):
            for r in range(4):
                src = 16 * grp + 4 * r + i // 4
                vals.append(lds[a[h][src] + 2 * (i % 4)])
        out[lane] = vals
    return out


def expected16(wrow, sub, kk):
    return {lane: [(wrow + sub * 16 + (lane & 15), 32 * kk + 8 * (lane >> 4) + e) for e in range(8)]
            for lane in range(64)}


def test_mfma16_kmajor_fragments():
    lds = dma_kmajor(256, 4, 64)
    for wrow in (0, 128):
        for sub in range(8):
            for kk in range(2):
                assert frag16_kmajor(lds, wrow, sub, kk) == expected16(wrow, sub, kk)


def test_mfma16_mnmajor_fragments():
    lds = dma_mnmajor16(256, 4, 64)
    assert len(lds) == 256 * 64
    for wcol in (0, 128):
        for sub in range(8):
            for kk in range(2):
                assert frag16_mnmajor(lds, 256, wcol, sub, kk) == expected16(wcol, sub, kk)


def test_mfma16_reads_are_bank_conflict_free():
    # ds_read_b128 (K-contiguous): 16-lane phases
    for lane0 in range(0, 64, 16):
        for kk in range(2):
            addrs = []
            for lane in range(lane0, lane0 + 16):
                row = lane & 15
                addrs.append((row * 128 + (((4 * kk + (lane >> 4)) ^ fk(row, 64)) << 4), 16))
            assert _banks(addrs, 256) == 1
    # ds_read_b64_tr_b16 (M/N-contiguous): 32-lane phases
    for sub in range(8):
        for kk in range(2):
            for h in range(2):
                a = frag16_mnmajor_addrs(256, 0, sub, kk, h)
                for half in range(2):
                    assert _banks([(a[l], 8) for l in range(32 * half, 32 * half + 32)], 256) == 1


# ---- kernel address formulas of the 16x16 operands, 4 and 8 waves -----------
def dma_kmajor16_kernel(waves):
    """LDS byte -> (row, k) as the K-major 16x16 operand issues its DMA:
    one offset register per wave, instruction i adds 8*waves rows."""
    lds = {}
    for wave in range(waves):
        for lane in range(64):
            r0 = 8 * wave + (lane >> 3)
            c = (lane & 7) ^ fk(r0, 64)
            for i in range(256 * 128 // 1024 // waves):
                r = r0 + 8 * waves * i
                assert fk(r, 64) == fk(r0, 64)          # one K column per lane
                m0 = (i * waves + wave) * 1024
                for e in range(8):
                    lds[m0 + lane * 16 + 2 * e] = (r, c * 8 + e)
    return lds


def dma_mnmajor16_kernel(waves):
    """Same for the M/N-major operand: two offset registers (i even / odd)."""
    lds = {}
    for wave in range(waves):
        for lane in range(64):
            k0, slot = 2 * wave + (lane >> 5), lane & 31
            lg = [(slot >> 1) ^ fm16(k0 + 2 * waves * j, 16) for j in range(2)]
            for i in range(64 * 512 // 1024 // waves):
                k = k0 + 2 * waves * i
                assert (slot >> 1) ^ fm16(k, 16) == lg[i & 1]
                m0 = (i * waves + wave) * 1024
                for e in range(8):
                    lds[m0 + lane * 16 + 2 * e] = (lg[i & 1] * 16 + (slot & 1) * 8 + e, k)
    return lds


def frag16_mnmajor_kernel(lds, wcol, sub, kk, stage=0):
    """ds_read_b64_tr_b16 addresses as the kernel forms them: (stage + frag0) ^ (sub << 5)."""
    a = [{}, {}]
    for lane in range(64):
        q, r, c = lane >> 4, (lane >> 2) & 3, lane & 3
        k0 = 8 * q + r
        frag0 = k0 * 512 + c * 8 + (((wcol >> 4) ^ fm16(k0, 16)) << 5)
        base = (stage + frag0) ^ (sub << 5)
        for h in range(2):
            a[h][lane] = base + (32 * kk + 4 * h) * 512 - stage
    out = {}
    for lane in range(64):
        grp, i = lane // 16, lane % 16
        out[lane] = [lds[a[h][16 * grp + 4 * r + i // 4] + 2 * (i % 4)] for h in range(2) for r in range(4)]
    return out


@pytest.mark.parametrize("waves", [4, 8])
def test_mfma16_kernel_dma_matches_layout(waves):
    assert dma_kmajor16_kernel(waves) == dma_kmajor(256, waves, 64)
    assert dma_mnmajor16_kernel(waves) == dma_mnmajor16(256, waves, 64)


@pytest.mark.parametrize("waves,wtn", [(4, 128), (8, 64)])
def test_mfma16_kernel_mnmajor_fragments(waves, wtn):
    lds = dma_mnmajor16_kernel(waves)
    for wcol in range(0, 256, wtn):
        for sub in range(wtn // 16):
            for kk in range(2):
                for stage in (0, 65536):
                    assert frag16_mnmajor_kernel(lds, wcol, sub, kk, stage) == expected16(wcol, sub, kk)


# ---- wide kernels (_x): descriptor offsets stay below 2 GiB -------------------
# The host sends an aligned operand of 2^30 elements or more to the _x kernels when
# its leading dimension is below 2^22 (K-contiguous) or 2^24 - 256 (M/N-contiguous)
# elements (test_host_api.py::test_operand_size_limits).  Their descriptors start
# at the tile's first row (K-contiguous) or the stage's first k row (M/N-contiguous)
# and span at most 2 GiB, with 0x80000000 reserved as the out-of-range offset: every
# 16-byte piece a lane fetches must end at or below 2^31 bytes from that start, and
# rebasing must not move any piece.
KMAJOR_LD_BOUND, MNMAJOR_LD_BOUND = 1 << 22, (1 << 24) - 256


@pytest.mark.parametrize("waves", [4, 8])
def test_wide_kmajor_offsets(waves):
    ld = KMAJOR_LD_BOUND - 8                      # largest allowed (rows stay 16-byte aligned)
    step = 16 * waves * ld                        # bytes between a wave's DMA instructions
    worst = 0
    for wave in range(waves):
        for lane in range(64):
            r0 = 8 * wave + (lane >> 3)
            c = (lane & 7) ^ fk(r0, 64)
            off0 = (r0 * ld + c * 8) * 2          # from the tile's first row
            for i in range(256 * 128 // 1024 // waves):
                off = off0 + i * step
                worst = max(worst, off + 16)
                for row0, k0 in ((0, 0), (256 * 12345, 64 * 7)):     # rebasing moves nothing
                    rowb = row0 * ld * 2
                    assert rowb + k0 * 2 + off == ((row0 + r0 + 8 * waves * i) * ld + k0 + c * 8) * 2
    assert worst <= 1 << 31


@pytest.mark.parametrize("waves", [4, 8])
def test_wide_mnmajor_offsets(waves):
    ld = MNMAJOR_LD_BOUND - 8
    row0 = (ld - 1) // 256 * 256                  # the last tile of a row, ending up to 255 past it
    step = 4 * waves * ld
    worst = 0
    for wave in range(waves):
        for lane in range(64):
            k0, slot = 2 * wave + (lane >> 5), lane & 31
            for i in range(64 * 512 // 1024 // waves):
                k = k0 + 2 * waves * i
                lg = (slot >> 1) ^ fm16(k, 16)
                off = (k * ld + row0 + lg * 16 + (slot & 1) * 8) * 2   # from the stage's first k row
                assert off == (k0 * ld + row0 + lg * 16 + (slot & 1) * 8) * 2 + i * step
                worst = max(worst, off + 16)
    assert worst <= 1 << 31
