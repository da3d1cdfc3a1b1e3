"""The verify's LDS staging of non-temporal state blocks (csrc/verify_kernel.cuh,
`row_slot` / `op_slot` and the loads' `c_voff` / `c_soff`), restated on the CPU
for every chunk count J the kernel is instantiated with. A block is 16 rows x
CPR = 4J chunks of 16 bytes, staged in ROUNDS rounds of SC = CPR / ROUNDS
chunks per row (two rounds for J >= 2). Load j (round g = j // JR) gives lane
l the chunk (row (j % JR) * RPL + l // SC, chunk g * SC + l % SC) and writes
it to slot r * SC + (c ^ swz(r)) of its round; operand register j of lane
(li, ls) reads chunk 4j + ls of row li back. Checked: every operand register
receives exactly the chunk the matrix-core layout assigns it (the layout the
ordinary loads produce directly), the loads cover the block once in runs of
SC consecutive chunks, each write covers 64 consecutive slots, and the 16
lanes of a read that share ls hit 16 distinct 16-byte bank groups. The GPU
tests compare the two load bodies' results bit for bit."""

import pytest


def _geometry(J):
    cpr = 4 * J
    rounds = 2 if J >= 2 else 1
    sc = cpr // rounds
    jr = J // rounds
    rpl = 64 // sc
    mask = (sc if sc < 16 else 16) - 1
    sh = 0 if sc >= 16 else (1 if sc == 8 else 2)
    return cpr, rounds, sc, jr, rpl, (lambda r: (r >> sh) & mask)


@pytest.mark.parametrize("J", [1, 2, 4, 8, 16])
def test_staging_rounds_map_row_runs_to_the_operand_layout(J):
    cpr, rounds, sc, jr, rpl, swz = _geometry(J)
    assert rounds * jr == J and sc == 4 * jr
    for g in range(rounds):
        stage = {}
        for j in range(g * jr, (g + 1) * jr):
            slots = set()
            for lane in range(64):
                r, c = (j % jr) * rpl + lane // sc, lane % sc
                assert r < 16
                slot = r * sc + (c ^ swz(r))
                assert slot not in stage
                stage[slot] = (r, g * sc + c)
                slots.add(slot)
            jj = j % jr
            assert slots == set(range(64 * jj, 64 * jj + 64)), "a write must cover 64 consecutive slots"
        assert len(stage) == 16 * sc, "a round's stage must be filled exactly once"
        for j in range(g * jr, (g + 1) * jr):
            for ls in range(4):
                groups = set()
                for li in range(16):
                    slot = li * sc + ((4 * (j % jr) + ls) ^ swz(li))
                    assert stage[slot] == (li, 4 * j + ls), "operand register got another chunk"
                    groups.add(slot % 16)
                assert len(groups) == 16, "bank conflict among the lanes of one read"


@pytest.mark.parametrize("J", [1, 2, 4, 8, 16])
def test_row_run_loads_cover_the_block_once(J):
    """Every chunk of a 16-row block is loaded once; each load reads SC
    consecutive chunks of each of its rows (row-major within the round)."""
    cpr, rounds, sc, jr, rpl, _ = _geometry(J)
    seen = []
    for j in range(J):
        g = j // jr
        offs = [((j % jr) * rpl + lane // sc) * cpr + g * sc + lane % sc for lane in range(64)]
        for k in range(0, 64, sc):
            assert offs[k:k + sc] == list(range(offs[k], offs[k] + sc))
        seen += offs
    assert sorted(seen) == list(range(16 * cpr))
