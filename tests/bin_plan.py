"""Checks of a decode plan (pc_attn_plan) against the lengths and tables it was built from,
restating what the attention kernel reads from each plan row and which workspace slots it
touches, so that every index the kernel derives from a plan is shown in range on the CPU.

Plan row (pc_attn_plan_record_ints() int32): {segments, blocks, plan epoch, 0 x 5}, then 4 segments of
{sequence, length, first block, blocks, first bin, part, parts, first slot}, then the
bin's block ids (up to 256). Row r belongs to group r % 8; the bins of a cut sequence are
rows first bin + 8 k of one group; parts 0 .. parts - 2 have workspace slots
first slot + k (the last part is folded in registers). Every live row of one plan carries the
same nonzero 22-bit epoch. The workspace is a 256-byte header (the fault word), then the
partial slots.
"""

from __future__ import annotations

from typing import Dict, List

import numpy as np

HEADER = 8
SEG = 8
MAX_SEGS = 4
RECORD = HEADER + MAX_SEGS * SEG
MAX_UNITS = 256
ROW = RECORD + MAX_UNITS
GROUPS = 8
HEADS = 4
SLOT_BYTES = 2176
WORKSPACE_HEADER = 256
EPOCH_LIMIT = 1 << 22


def check_decode_plan(plan: np.ndarray, lengths: np.ndarray, tables: np.ndarray, num_blocks: int,
                      workspace_bytes: int) -> Dict[str, int]:
    """Assert the plan covers every cached block of every sequence exactly once with the
    right ids, and that every row, slot and flag the kernel would touch is in range.
    Returns a few statistics (rows, live rows, cut sequences, slots, max blocks per row)."""
    plan = np.asarray(plan)
    assert plan.ndim == 2 and plan.shape[1] == ROW and plan.dtype == np.int32
    rows = plan.shape[0]
    assert rows % GROUPS == 0
    batch = len(lengths)
    nblk = [(int(x) + 15) // 16 if x > 0 else 0 for x in lengths]
    parts: Dict[int, List[tuple]] = {}
    slots_needed = (workspace_bytes - WORKSPACE_HEADER) // (HEADS * SLOT_BYTES)
    used_slots = set()
    epochs = set()
    live = most = 0
    for r in range(rows):
        row = plan[r]
        nseg, nunits = int(row[0]), int(row[1])
        if nseg <= 0:
            assert not row.any(), f"padding row {r} is not empty"
            continue
        live += 1
        assert 1 <= nseg <= MAX_SEGS and 1 <= nunits <= MAX_UNITS and not row[3:HEADER].any()
        assert 0 < int(row[2]) < EPOCH_LIMIT
        epochs.add(int(row[2]))
        most = max(most, nunits)
        u = 0
        for s in range(nseg):
            b, length, j0, n, k0, kidx, nspan, slot = (int(v) for v in row[HEADER + SEG * s: HEADER + SEG * (s + 1)])
            assert 0 <= b < batch and length == int(lengths[b]) and n >= 1 and 0 <= j0 and j0 + n <= nblk[b]
            assert np.array_equal(row[RECORD + u: RECORD + u + n], tables[b, j0: j0 + n]), f"row {r} segment {s} ids"
            assert (row[RECORD + u: RECORD + u + n] >= 0).all() and (row[RECORD + u: RECORD + u + n] < num_blocks).all()
            u += n
            assert 0 <= kidx < nspan and r == k0 + GROUPS * kidx and k0 % GROUPS == r % GROUPS
            if nspan > 1:
                # a cut part is the first segment of its row (a later part) or the last (an earlier part)
                assert (kidx == 0 or s == 0) and (kidx == nspan - 1 or s == nseg - 1)
                assert slot >= 0 and slot + nspan - 1 <= slots_needed, "partial slots outside the workspace"
                if kidx < nspan - 1:
                    assert (slot + kidx) not in used_slots
                    used_slots.add(slot + kidx)
            else:
                assert slot == -1 or slot == 0
            parts.setdefault(b, []).append((j0, n, r, kidx, nspan, k0, slot))
        assert u == nunits and not row[RECORD + nunits:].any()
        for s in range(nseg, MAX_SEGS):
            assert not row[HEADER + SEG * s: HEADER + SEG * (s + 1)].any()
    assert len(epochs) <= 1, "live rows of one plan carry different epochs"
    cut = 0
    for b in range(batch):
        got = sorted(parts.get(b, []))
        if nblk[b] == 0:
            assert not got
            continue
        assert got, f"sequence {b} not planned"
        pos = 0
        for k, (j0, n, r, kidx, nspan, k0, slot) in enumerate(got):
            assert j0 == pos and kidx == k and nspan == len(got) and k0 == got[0][5] and slot == got[0][6]
            pos += n
        assert pos == nblk[b]
        cut += len(got) > 1
    return {"rows": rows, "live": live, "cut": cut, "slots": len(used_slots), "most": most}


def regrouped_plan(plan: np.ndarray, perm) -> np.ndarray:
    """The same bins with group x's rows moved to group perm[x] (row r -> 8 (r // 8) +
    perm[r % 8]) and every segment's first-bin field renamed the same way: each bin runs
    on another XCD, the spans stay in one group, their parts in the same order. The
    attention output must not change by a bit."""
    plan = np.asarray(plan)
    out = np.zeros_like(plan)
    for r in range(plan.shape[0]):
        row = plan[r].copy()
        for s in range(min(int(row[0]), MAX_SEGS)):
            k0 = int(row[HEADER + SEG * s + 4])
            row[HEADER + SEG * s + 4] = GROUPS * (k0 // GROUPS) + perm[k0 % GROUPS]
        out[GROUPS * (r // GROUPS) + perm[r % GROUPS]] = row
    return out
