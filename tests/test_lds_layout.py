"""The backward kernel's Q / dO tile layout at head_dim 64 (`bq_swz` in
`csrc/attn_mfma.hip`): a permutation of each 128-byte row's eight 16-byte
pieces, chosen so that the kernel's two read patterns are free of LDS bank
conflicts. The permutation is read from the source and checked here on the
host against gfx950's read banking: 64 four-byte banks, `ds_read_b128`
served 16 lanes at a time, `ds_read_b64_tr_b16` 32 lanes at a time.
"""

import re
from pathlib import Path

SRC = Path(__file__).resolve().parents[1] / "moba-triton_amd" / "csrc" / "attn_mfma.hip"
ROWS = 64    # query rows of one step's tile (NQ)
PIECES = 8   # 16-byte pieces of a 128-byte row (head_dim 64, 16-bit elements)


def swz():
    """bq_swz's return expression, evaluated as Python (same operators)."""
    text = SRC.read_text()
    m = re.search(r"int bq_swz\(int row\) \{\s*return (.*?);\s*\}", text, re.S)
    assert m, "bq_swz not found"
    expr = m.group(1)
    return lambda row: eval(expr, {}, {"row": row})


def group(row, piece, f):
    """4-bank group (0..15) of a piece: even rows start at bank 0, odd rows at
    bank 32 (128-byte rows); a piece is four banks."""
    return (row & 1) * 8 + (piece ^ f(row))


def test_permutation_is_a_bijection_within_every_row():
    f = swz()
    for row in range(ROWS):
        assert sorted(p ^ f(row) for p in range(PIECES)) == list(range(PIECES))


def test_row_reads_are_conflict_free():
    """S / dP operands: lanes 16i .. 16i + 15 read one piece of 16
    consecutive rows of a 32-row tile (ds_read_b128)."""
    f = swz()
    for r0 in range(0, ROWS, 16):
        for piece in range(PIECES):
            groups = {group(r, piece, f) for r in range(r0, r0 + 16)}
            assert len(groups) == 16, (r0, piece)


def test_transposing_reads_are_conflict_free():
    """dV / dK operands: 32 lanes read 4 consecutive rows (4a .. 4a + 3) x
    the 4 pieces of one 32-feature tile (ds_read_b64_tr_b16, 8 bytes a lane,
    two lanes a piece)."""
    f = swz()
    for a in range(ROWS // 4):
        for dt in range(2):
            groups = [group(r, p, f) for r in range(4 * a, 4 * a + 4)
                      for p in range(4 * dt, 4 * dt + 4)]
            assert len(set(groups)) == 16, (a, dt)


def test_padded_rows_conflicted_before():
    """The layout it replaced (rows padded to 144 bytes, no permutation)
    folds rows r and r + 2 of a transposing read onto the same banks."""
    def banks(row, piece):
        start = (row * 144 + piece * 16) // 4
        return {(start + i) % 64 for i in range(4)}
    seen = [banks(r, p) for r in range(4) for p in range(4)]
    assert sum(len(b) for b in seen) > len(set().union(*seen))
