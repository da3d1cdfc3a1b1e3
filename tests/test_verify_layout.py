"""The verify's LDS staging of non-temporal state blocks (csrc/verify_kernel.cuh,
`stage_write` / `stage_read`), restated on the CPU for every chunk count J the
kernel is instantiated with: a block is 16 rows x CPR = 4J chunks of 16 bytes;
load j of lane l reads chunk (row j*RPL + l // CPR, chunk l % CPR) and stores
it at slot r*CPR + (c ^ swz(r)); the read-back gives lane (li, ls) chunk
4j + ls of row li. Checked: every operand register receives exactly the chunk
the matrix-core layout assigns it (the layout the ordinary loads produce
directly), each write covers 64 consecutive slots, and the 16 lanes of a read
that share ls hit 16 distinct 16-byte bank groups. The GPU tests compare the
two load bodies' results bit for bit."""

import pytest


def _swz(cpr: int):
    mask = (cpr if cpr < 16 else 16) - 1
    sh = 0 if cpr >= 16 else (1 if cpr == 8 else 2)
    return lambda r: (r >> sh) & mask


@pytest.mark.parametrize("J", [1, 2, 4, 8, 16])
def test_staging_maps_whole_rows_to_the_operand_layout(J):
    cpr = 4 * J
    rpl = 64 // cpr
    swz = _swz(cpr)
    stage = {}
    for j in range(J):
        slots = set()
        for lane in range(64):
            chunk, row = lane & (cpr - 1), j * rpl + lane // cpr
            assert row < 16
            slot = row * cpr + (chunk ^ swz(row))
            assert slot not in stage
            stage[slot] = (row, chunk)
            slots.add(slot)
        assert slots == set(range(64 * j, 64 * j + 64)), "a write must cover 64 consecutive slots"
    assert len(stage) == 16 * cpr
    for j in range(J):
        for ls in range(4):
            groups = set()
            for li in range(16):
                c = 4 * j + ls
                slot = li * cpr + (c ^ swz(li))
                assert stage[slot] == (li, c), "operand register got another chunk"
                groups.add(slot % 16)
            assert len(groups) == 16, "bank conflict among the lanes of one read"


@pytest.mark.parametrize("J", [1, 2, 4, 8, 16])
def test_whole_row_loads_cover_the_block_once(J):
    """The non-temporal body's loads read every chunk of a 16-row block once,
    each load 64 consecutive chunks in row-major order (whole rows)."""
    cpr = 4 * J
    rpl = 64 // cpr
    seen = []
    for j in range(J):
        offs = [(j * rpl + lane // cpr) * cpr + (lane & (cpr - 1)) for lane in range(64)]
        assert offs == list(range(64 * j, 64 * j + 64))
        seen += offs
    assert sorted(seen) == list(range(16 * cpr))
