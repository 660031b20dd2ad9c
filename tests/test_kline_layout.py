"""Lane arithmetic of the K whole-line loads and the V-row LDS swizzle, on the CPU.

pd_device.h loads each 16-row group of K as whole 128-byte lines (kline_offset:
lane S gets row 8sh + S/8, 16-byte chunk S%8 of line h, rotated by two in the
upper half-wavefront), then lines_to_mfma turns each pair of loads into the
MFMA A-operand registers with two bank-masked DPP moves (row_shr:4 on banks 1
and 3, row_shl:4 on banks 0 and 2 of every 16-lane row), an exchange of the
pair on upper lanes with S & 2 = 0, and one ds_bpermute per dword from lane
kline_source(L).  This test runs the same index arithmetic on NumPy lanes and
checks the result against the operand layout the QK MFMA reads (lane 16g + r:
row r, chunk 4ch + g), for every head dim, and that each half-wavefront's 32
ds_bpermute sources are distinct modulo 32 (no bank conflicts).  On the GPU the kernel's outputs are bit-identical to loads made
directly in the operand layout (tests/test_gpu_matched.py and the paged tests).
The V-row swizzle test at the end checks the LDS copy/read round trip and the
bank spread of the transposed reads.
"""
import numpy as np
import pytest

LANES = np.arange(64)


def dpp_row_shift(old, src, shift, bank_mask):
    """update_dpp(old, src, row_shr:shift (shift > 0) or row_shl:-shift, row_mask 0xf,
    bank_mask): lanes of the enabled banks (4-lane groups of each 16-lane row) read src
    from lane - shift within their row; the others keep old."""
    out = old.copy()
    for lane in LANES:
        bank = (lane & 15) >> 2
        if not (bank_mask >> bank) & 1:
            continue
        src_lane = lane - shift
        assert (src_lane >> 4) == (lane >> 4), "source outside the 16-lane row"
        out[lane] = src[src_lane]
    return out


def kline_chunk(lane):
    p = lane & 7
    return (p - 2) & 7 if lane >= 32 else p


def kline_source(lane):
    r, g = lane & 15, lane >> 4
    k = r & 7
    return 4 * (8 * k + (4 if r >= 8 else 0) + (((g + 2) & 3) if k >= 4 else g))


EXCHANGE = np.array([lane >= 32 and not lane & 2 for lane in LANES])


def bpermute(src, byte_index):
    return src[byte_index // 4]


@pytest.mark.parametrize("dim", [64, 128, 256])
def test_whole_line_loads_rearrange_into_the_operand_layout(dim):
    chunks = dim // 8                      # 16-byte chunks per K row
    # K rows of one 16-row group; each chunk is labelled (row, chunk)
    label = lambda row, chunk: 1000 * row + chunk
    lines = chunks // 8                    # 128-byte lines per row
    regs = {}
    for h in range(lines):
        for sh in range(2):                # kline_offset + 128 h, rows + 8 sh
            regs[(h, sh)] = np.array([label(8 * sh + s // 8, 8 * h + kline_chunk(int(s)))
                                      for s in LANES])
    idx = np.array([kline_source(int(lane)) for lane in LANES])
    for h in range(lines):
        a, b = regs[(h, 0)], regs[(h, 1)]
        u = dpp_row_shift(a, b, 4, 0xA)
        v = dpp_row_shift(b, a, -4, 0x5)
        u, v = np.where(EXCHANGE, v, u), np.where(EXCHANGE, u, v)
        got = {2 * h: bpermute(u, idx), 2 * h + 1: bpermute(v, idx)}
        for ch, reg in got.items():
            want = np.array([label(lane & 15, 4 * ch + (lane >> 4)) for lane in LANES])
            np.testing.assert_array_equal(reg, want)


def test_bpermute_sources_are_distinct_modulo_32_in_each_half():
    """ds_bpermute reads its source lanes through 32 banks; the rotation of the upper
    half's chunks gives each half-wavefront 32 sources in distinct banks (the
    unrotated layout put rows k and k + 4 on lanes 32 apart: 16 banks, 2-way)."""
    src = [kline_source(int(lane)) // 4 for lane in LANES]
    for half in (range(0, 32), range(32, 64)):
        assert len({src[lane] % 32 for lane in half}) == 32
    unrotated = [8 * (lane & 15) + (lane >> 4) if (lane & 15) < 8 else
                 8 * ((lane & 15) - 8) + (lane >> 4) + 4 for lane in range(64)]
    assert len({unrotated[lane] % 32 for lane in range(32)}) == 16


def test_whole_line_loads_still_cover_one_line_per_eight_lanes():
    row_bytes = 512
    addr = [(lane // 8) * row_bytes + 16 * kline_chunk(lane) for lane in range(64)]
    for start in range(0, 64, 8):
        assert sorted(a % 128 for a in addr[start:start + 8]) == list(range(0, 128, 16))
        assert len({a // 128 for a in addr[start:start + 8]}) == 1


def test_operand_layout_loads_touch_half_lines_and_whole_line_loads_whole_ones():
    """What the rearrangement is for: a load in the operand layout covers 64 bytes of
    each of 16 rows (no 8 consecutive lanes share a line), a whole-line load covers 8
    full lines with 8 consecutive lanes each."""
    row_bytes = 512
    operand = [(lane & 15) * row_bytes + 16 * (lane >> 4) for lane in LANES]
    whole = [(lane // 8) * row_bytes + 16 * (lane % 8) for lane in LANES]
    line_of = lambda addr: addr // 128
    assert len({line_of(a) for a in operand}) == 16
    assert len({line_of(a) for a in whole}) == 8
    for start in range(0, 64, 8):
        assert len({line_of(a) for a in whole[start:start + 8]}) == 1
        assert len({line_of(a) for a in operand[start:start + 8]}) == 8


def vswz(dim, row):
    if dim >= 128:
        return 2 * (row & 3) + 8 * ((row >> 3) & 1)
    return 2 * (((row >> 1) & 1) | (((row >> 3) & 1) << 1))


def v_read_offset(dim, col0, lane, row):
    b = lane & 3
    return 16 * (((col0 >> 3) + (b >> 1)) ^ vswz(dim, row)) + 8 * (b & 1)


def read_row(lane, step, second):
    """Tile row that `lane` reads in a transposed read of the column-split P V: rows
    8(L/16) + (L%16)/4 (+4 in the second read) of 32-row k-step `step`."""
    return 32 * step + 8 * (lane >> 4) + ((lane & 15) >> 2) + (4 if second else 0)


@pytest.mark.parametrize("dim", [64, 128, 256])
def test_v_rows_swizzle_round_trips_and_transposed_reads_are_conflict_free(dim):
    """pd_device.h stores V rows in LDS unpadded, 16-byte piece p of row r at position
    p ^ vswz(r) (v_copy_offset), and reads them back with v_read_offset.  Every copy
    lane fills one distinct position and every transposed read finds the logical columns
    it asks for.  The LDS serves 32 lanes of a read per clock over 64 four-byte banks
    (256 bytes); the 32 lanes of each half-wavefront hit 256 distinct bytes for the
    column-split reads of the tile and loader kernels.  (A 4-row swizzle gave 2-way
    conflicts here, which SQ_LDS_BANK_CONFLICT showed on MI355X.)"""
    pieces = dim // 8
    pitch = 16 * pieces
    tile = 16384 // dim
    tw = tile // 4                         # rows per wavefront
    copies = tw * pitch // 1024
    stored = {}
    for i in range(copies):
        for lane in range(64):
            slot = 64 * i + lane
            row, pos = divmod(slot, pieces)
            stored[(row, pos)] = (row, pos ^ vswz(dim, row))
    assert len(stored) == tw * pieces
    assert sorted(stored.values()) == [(r, p) for r in range(tw) for p in range(pieces)]

    def address(row):
        """Byte address of `row` of the tile: wavefront row // tw's slot, then the row."""
        return (row // tw) * tw * pitch + (row % tw) * pitch

    for step in range(tile // 32):
        for second in (False, True):
            for col0 in range(0, dim, 16):
                for half in (0, 32):
                    chunks = set()
                    for lane in range(half, half + 32):
                        row = read_row(lane, step, second)
                        local = row % tw
                        off = v_read_offset(dim, col0, lane, local % 16)
                        pos, within = divmod(off, 16)
                        b = lane & 3
                        assert stored[(local, pos)] == (local, (col0 + 4 * b) // 8)
                        assert within == 8 * (b & 1)
                        chunks.add(((address(row) + off) % 256) // 8)
                    assert len(chunks) == 32, (step, second, col0, half)


def vswz_rows(row):
    """vswz<64, true>: the V swizzle of the D 64 kernels that multiply P V by rows."""
    return 2 * (((row >> 1) & 1) | (((row >> 2) & 1) << 1))


def rows_read_row(lane, step, second):
    """Row of its wavefront's 64 that `lane` reads in a transposed read of the row-wise
    P V (pv_tile_rows): rows 4(L/16) + (L%16)/4 (+16 in the second read) of k-step
    `step`, in the k order of the probabilities left in the score registers."""
    return 32 * step + 4 * (lane >> 4) + ((lane & 15) >> 2) + (16 if second else 0)


def _rows_chunks(swizzle, read):
    """8-byte LDS chunks (mod 256 bytes) per half-wavefront read of the row-wise P V,
    after checking that every read finds the logical columns it asks for."""
    pitch, rows = 128, 64
    stored = {(r, p ^ swizzle(r)): p for r in range(rows) for p in range(8)}
    assert len(stored) == rows * 8
    out = []
    for step in range(2):
        for second in (False, True):
            for col0 in range(0, 64, 16):
                for half in (0, 32):
                    chunks = set()
                    for lane in range(half, half + 32):
                        row = read(lane, step, second)
                        b = lane & 3
                        pos = ((col0 >> 3) + (b >> 1)) ^ swizzle(row)
                        assert stored[(row, pos)] == (col0 + 4 * b) // 8
                        chunks.add(((row * pitch + 16 * pos + 8 * (b & 1)) % 256) // 8)
                    out.append(len(chunks))
    return out


def test_row_wise_v_swizzle_is_conflict_free_where_the_column_swizzle_is_not():
    """The row-wise reads put rows 0-7 of a 16-row group in one half-wavefront (the
    column-split reads put rows 0-3 and 8-11 there): with bit 2 of the row in the
    swizzle every half-wavefront read hits 32 distinct 8-byte chunks of the 256 bytes
    the LDS serves per clock; the column swizzle (bit 3) would give 2-way conflicts."""
    assert set(_rows_chunks(vswz_rows, rows_read_row)) == {32}
    assert set(_rows_chunks(lambda r: vswz(64, r), rows_read_row)) == {16}
    # The operand k order: lane (qg, qh) supplies k = 8 qg + e for rows 4 qg + e
    # (e < 4) and 16 + 4 qg + e - 4, which is where the scores of 16-row groups 2s and
    # 2s + 1 left that lane's probabilities (rows 16 g + 4 qg + r).
    for lane in range(64):
        qg, c = lane >> 4, (lane & 15) >> 2
        assert rows_read_row(lane, 0, False) == 16 * 0 + 4 * qg + c
        assert rows_read_row(lane, 1, True) == 16 * 3 + 4 * qg + c


def kswz(dim, row):
    return row & 15 if dim >= 128 else (row >> 1) & 7


@pytest.mark.parametrize("dim,heads", [(64, 1), (64, 2), (128, 1), (256, 1)])
def test_loader_k_stage_layout(dim, heads):
    """cols_loader_kernel's K stage: loader w's copy i (1 KiB, lane l at byte 16 l)
    fills position 64 (8 w + i) + l, i.e. row pos // (D/8), piece (pos % (D/8)) ^
    kswz(row), read from global memory at that row's offset; compute wavefront w's lane
    (qh, qg) reads piece qg + 4 ch of row kTW w + 16 g + qh with one ds_read_b128.
    Every position is filled once, every read finds its logical piece, the 16 lanes a
    ds_read_b128 serves per clock (256 bytes over 64 banks) hit 16 distinct 16-byte
    groups, and every 8 consecutive lanes of a copy read one 128-byte line of K.  With
    kv-head pairs (D 64) tile row R is token R // 2 of kv head R % 2: a token's two
    rows are adjacent 128-byte lines."""
    pieces = dim // 8
    tile = 16384 // dim
    tw = tile // 4
    hkv = 4 if heads == 2 else 1
    row_stride = hkv * dim * 2                  # bytes between tokens in the pool

    def source(row, piece):
        return (row // heads) * row_stride + (row % heads) * dim * 2 + 16 * piece

    stage = {}
    for w in range(4):
        for i in range(8):
            lines = []
            for lane in range(64):
                pos = 64 * (8 * w + i) + lane
                row, ph = divmod(pos, pieces)
                assert (row, ph) not in stage
                stage[(row, ph)] = ph ^ kswz(dim, row)      # logical piece held there
                lines.append(source(row, ph ^ kswz(dim, row)) // 128)
            for start in range(0, 64, 8):
                assert len(set(lines[start:start + 8])) == 1, (w, i, start)
    assert len(stage) == tile * pieces
    for w in range(4):
        for g in range(tw // 16):
            for ch in range(dim // 32):
                for qg in range(4):
                    banks = set()
                    for qh in range(16):
                        row = tw * w + 16 * g + qh
                        ph = (qg + 4 * ch) ^ kswz(dim, row)
                        assert stage[(row, ph)] == qg + 4 * ch
                        banks.add(((row * 2 * dim + 16 * ph) % 256) // 16)
                    assert len(banks) == 16, (w, g, ch, qg)
