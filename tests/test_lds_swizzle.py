"""The LDS pipeline's address arithmetic (paged_decode.hip, mfma_segment with
dma_staged), checked on the CPU by its properties rather than by retyping it:

* the direct-to-LDS loads place every (token, 16-byte chunk) of a 16-token
  block exactly once, and each 16-lane row of a load still reads one whole,
  contiguous 256-byte token row from memory;
* every lane's K read (A operand of S = K Q^T: token `row`, dims
  32c + 8grp .. +7) and V^T read (ds_read_b64_tr_b16: token 4grp + row/4,
  dims 16dt + 4(row % 4) .. +3) lands on the logical element the MFMA layout
  needs;
* no 16-lane phase of those reads hits one LDS bank twice (64 banks of
  4 bytes), while unpadded rows without the swizzle would.

The formulas below are the kernel's, written once here; what is checked is
what they must satisfy, so a dropped XOR term, a wrong shift or a swapped
row/group index fails.
"""

from __future__ import annotations

D = 128  # head_dim of the LDS pipeline (16-bit elements)
ROW_BYTES = D * 2  # one staged token row
BANKS = 64  # gfx950 LDS: 64 banks of 4 bytes


def dma_lane(c: int, lane: int, tile: str) -> tuple[int, int, int]:
    """Load c, lane l of the K or V tile: (token, chunk read from memory, LDS
    byte offset)."""
    tok = 4 * c + (lane >> 4)
    slot = lane & 15
    chunk = slot ^ tok if tile == "k" else slot ^ (2 * (tok & 7))
    return tok, chunk, c * 1024 + 16 * lane


def stored_at(tile: str) -> dict[int, tuple[int, int]]:
    """LDS byte offset of each stored 16-byte chunk -> (token, logical chunk)."""
    placed = {}
    for c in range(4):
        for lane in range(64):
            tok, chunk, off = dma_lane(c, lane, tile)
            assert off not in placed
            placed[off] = (tok, chunk)
    return placed


def k_read(lane: int, c: int) -> int:
    """Element offset of lane's K read for chunk c (k_rd ^ (c << 5))."""
    row, grp = lane & 15, lane >> 4
    k_rd = row * D + ((grp ^ (row & 3)) << 3) + ((row >> 2) << 5)
    return k_rd ^ (c << 5)


def v_read(lane: int, dt: int) -> int:
    """Element offset of lane's transposing V read for tile dt (v_rd ^ (dt << 4))."""
    row, grp = lane & 15, lane >> 4
    tok = 4 * grp + (row >> 2)
    v_rd = tok * D + (((row & 3) >> 1) << 3) + 4 * (row & 1) + ((tok & 7) << 4)
    return v_rd ^ (dt << 4)


def logical(placed: dict[int, tuple[int, int]], elem: int) -> tuple[int, int]:
    """(token, dim) held at element offset `elem` of a staged block."""
    byte = 2 * elem
    tok, chunk = placed[byte - byte % 16]
    return tok, 8 * chunk + (byte % 16) // 2


def banks(byte: int, size: int) -> set[int]:
    return {((byte + i) // 4) % BANKS for i in range(0, size, 4)}


def test_loads_place_every_chunk_once_and_read_whole_rows():
    for tile in ("k", "v"):
        placed = stored_at(tile)
        assert sorted(placed.values()) == [(t, ch) for t in range(16) for ch in range(16)]
        for c in range(4):
            for r in range(4):  # each 16-lane row of the load
                toks = {dma_lane(c, 16 * r + i, tile)[0] for i in range(16)}
                chunks = sorted(dma_lane(c, 16 * r + i, tile)[1] for i in range(16))
                assert len(toks) == 1 and chunks == list(range(16)), "a row must read one whole token row"


def test_k_reads_are_the_mfma_a_operand():
    placed = stored_at("k")
    for lane in range(64):
        row, grp = lane & 15, lane >> 4
        for c in range(D // 32):
            e = k_read(lane, c)
            assert e % 8 == 0
            for j in range(8):
                assert logical(placed, e + j) == (row, 32 * c + 8 * grp + j), (lane, c, j)


def test_v_reads_are_the_transposed_tiles():
    placed = stored_at("v")
    for lane in range(64):
        row, grp = lane & 15, lane >> 4
        for dt in range(D // 16):
            e = v_read(lane, dt)
            assert e % 4 == 0
            for j in range(4):
                assert logical(placed, e + j) == (4 * grp + (row >> 2), 16 * dt + 4 * (row & 3) + j), (lane, dt, j)


def test_reads_are_bank_conflict_free_per_16_lane_phase():
    for c in range(D // 32):  # K: 16 lanes x 16 bytes = one full pass over the banks
        for phase in range(4):
            hit = [b for lane in range(16 * phase, 16 * phase + 16) for b in banks(2 * k_read(lane, c), 16)]
            assert len(hit) == len(set(hit)) == 64, (c, phase)
    for dt in range(D // 16):  # V^T: 16 lanes x 8 bytes = half a pass
        for phase in range(4):
            hit = [b for lane in range(16 * phase, 16 * phase + 16) for b in banks(2 * v_read(lane, dt), 8)]
            assert len(hit) == len(set(hit)) == 32, (dt, phase)


def test_without_the_permutation_the_reads_would_conflict():
    # The same reads on unpadded rows in memory order: 16 K rows at a
    # 256-byte stride share their banks, and so do the 4 V rows of a phase.
    for c in range(D // 32):
        hit = [b for lane in range(16) for b in banks((lane & 15) * ROW_BYTES + 2 * (32 * c), 16)]
        assert len(set(hit)) < len(hit)
    for dt in range(D // 16):
        hit = [b for lane in range(16)
               for b in banks((lane >> 2) * ROW_BYTES + 2 * (16 * dt + 4 * (lane & 3)), 8)]
        assert len(set(hit)) < len(hit)
