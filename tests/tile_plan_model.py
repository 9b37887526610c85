"""Host model of the tiled expert path's work decomposition (tiles.hip, expert_items.h,
routing.hip), used to show on the CPU that every intermediate row a kernel reads was written by
an earlier kernel of the same call, for a given routing.

It restates, from the device code:
  - the routing's work-range records (align_block: per active expert, in expert order, off =
    exclusive prefix of the counts, cnt, key = active experts before it, j0 = exclusive prefix
    of the range counts, nr = ceil(cnt / span); one record per range);
  - the sorted positions (ascending f within each expert, experts ascending);
  - work_item + range_group: workgroup b -> (shared or routed, token range, weight group);
  - tile_gateup_kernel: act rows [off, off+m) x the group's owned 16-column tiles;
  - tile_down_kernel: reads act rows off + min(q, m-1) over its split's K slice, writes
    part[split][f][owned 16-row tiles] for q < m;
  - combine: reads part[split][t*k+j][:] for every split and every contributing assignment
    (and the shared expert's part_s[split][t][:]).
Grid sizes, span, splits and split steps come from the library's own host plan
(smx_moe_plan_info), so the model checks the plan the library launches.
"""
from __future__ import annotations

import numpy as np

ROW_TILE = 16
TILE_TOK = 128          # sorted positions per range (kTileTok)
GATE_COLS = 128         # intermediate columns per gate/up workgroup (kTileGateCols)
DOWN_ROWS = 256         # W2 rows per down workgroup (kTileDownRows)
WAVES = 4
STEP_BYTES = 64         # unit of split_steps


def range_group(local: int, per_item: int, nr: int):
    """expert_items.h range_group: item `local` of an expert's nr * per_item items."""
    full = per_item // 8 * 8 * nr
    if local < full:
        blk, inn = divmod(local, 8 * nr)
        r = inn // 8
        return r, blk * 8 + (inn - r * 8)
    rem = per_item % 8
    inn = local - full
    r = inn // rem
    return r, per_item // 8 * 8 + (inn - r * rem)


def routing_records(ids: np.ndarray, routable: np.ndarray, E: int, span: int):
    """Records and sorted positions of a routing: ids [N] (flat f = t*k + j), routable [N]."""
    counts = np.zeros(E, dtype=np.int64)
    for f, e in enumerate(ids):
        if routable[f]:
            counts[e] += 1
    sorted_f = []
    recs = []
    off = key = j0 = 0
    for e in range(E):
        c = int(counts[e])
        sorted_f.extend(int(f) for f in np.nonzero((ids == e) & routable)[0])
        if c == 0:
            continue
        nr = -(-c // span)
        for _ in range(nr):
            recs.append(dict(off=off, cnt=c, key=key, j0=j0, nr=nr, expert=e))
        off += c
        key += 1
        j0 += nr
    return recs, np.array(sorted_f, dtype=np.int64), counts


def _routed_item(rb: int, per_item: int, recs, span: int):
    """work_item's routed branch for routed workgroup index rb (None: past the ranges)."""
    j = rb // per_item
    if j >= len(recs):
        return None
    rr = recs[j]
    local = rb - rr["j0"] * per_item
    assert 0 <= local < rr["nr"] * per_item, (rb, rr)
    r, g = (0, local) if rr["nr"] == 1 else range_group(local, per_item, rr["nr"])
    off = rr["off"] + r * span
    m = min(span, rr["cnt"] - r * span)
    assert m >= 1, (rb, rr, r)
    return off, m, g


def _shared_item(b: int, per_item: int, tok_groups: int, T: int, span: int):
    nr = tok_groups if tok_groups > 1 else 1
    if nr > 1:
        v, g = range_group(b, per_item, nr)
    else:
        v, g = divmod(b, per_item)
    off = v * span
    return off, min(span, T - off), g


def _owned_tiles(first_tile: int, count: int, last: int):
    return [t for t in range(first_tile, first_tile + count) if t <= last]


def check_tiled_coverage(T: int, H: int, I: int, k: int, eb: int, ids: np.ndarray,
                         routable: np.ndarray, E: int, plan: dict, Is: int = 0) -> dict:
    """Raise AssertionError if any act/part element a kernel of the tiled path reads was not
    written (or was written twice) for this routing. ids/routable: [T, k]. Returns counts."""
    assert plan["tiled"] == 1, plan
    span = plan["span"]
    assert span == TILE_TOK
    N = T * k
    flat = ids.reshape(-1).astype(np.int64)
    ok = routable.reshape(-1).astype(bool)
    recs, sorted_f, _ = routing_records(flat, ok, E, span)
    nranges = len(recs)
    assert nranges <= plan["max_ranges"], f"{nranges} ranges, grid sized for {plan['max_ranges']}"

    s_blocks_gu = plan["shared_gateup_blocks"]
    s_blocks_dn = plan["shared_down_blocks"]
    groups_r = -(-I // GATE_COLS)
    groups_s = -(-Is // GATE_COLS) if Is else 0
    rgroups = -(-H // DOWN_ROWS)
    assert plan["tile_gateup_grid"] == s_blocks_gu + plan["max_ranges"] * groups_r
    assert plan["tile_down_grid"] == s_blocks_dn + plan["max_ranges"] * rgroups * plan["splits"]

    # gate/up: act [N, I/16] and act_s [T, Is/16] written
    act = np.zeros((N, I // ROW_TILE), dtype=np.int32)
    act_s = np.zeros((T, max(Is, ROW_TILE) // ROW_TILE), dtype=np.int32)
    items = 0
    for b in range(plan["tile_gateup_grid"]):
        if b < s_blocks_gu:
            off, m, g = _shared_item(b, groups_s, plan["shared_tok_groups"], T, span)
            tiles = [t for w in range(WAVES) for t in
                     _owned_tiles(g * GATE_COLS // ROW_TILE + 2 * w, 2, Is // ROW_TILE - 1)]
            act_s[off:off + m, tiles] += 1
        else:
            it = _routed_item(b - s_blocks_gu, groups_r, recs, span)
            if it is None:
                continue
            off, m, g = it
            tiles = [t for w in range(WAVES) for t in
                     _owned_tiles(g * GATE_COLS // ROW_TILE + 2 * w, 2, I // ROW_TILE - 1)]
            act[off:off + m, tiles] += 1
        items += 1
    routed_rows = len(sorted_f)
    assert (act[:routed_rows] == 1).all(), "an act element of a routed row written 0 or 2+ times"
    if Is:
        assert (act_s[:T] == 1).all(), "an act element of the shared expert written 0 or 2+ times"

    # down: reads act over its K slice, writes part[split][f][H/16]
    def k_cols(sp: int, steps: int, width: int):
        c0 = sp * steps * STEP_BYTES // eb
        c1 = c0 + steps * STEP_BYTES // eb
        assert c1 <= width, (sp, steps, width)
        return c0 // ROW_TILE, c1 // ROW_TILE

    splits, s_splits = plan["splits"], plan["shared_splits"]
    assert splits * plan["split_steps"] * STEP_BYTES == I * eb, "routed K splits do not tile I"
    if Is:
        assert s_splits * plan["shared_split_steps"] * STEP_BYTES == Is * eb, "shared K splits do not tile Is"
    part = np.zeros((splits, N, H // ROW_TILE), dtype=np.int32)
    part_s = np.zeros((max(s_splits, 1), T, H // ROW_TILE), dtype=np.int32)
    for b in range(plan["tile_down_grid"]):
        if b < s_blocks_dn:
            off, m, g = _shared_item(b, rgroups * s_splits, plan["shared_tok_groups"], T, span)
            sp, rg = divmod(g, rgroups)
            c0, c1 = k_cols(sp, plan["shared_split_steps"], Is)
            assert (act_s[off:off + m, c0:c1] == 1).all(), "shared down reads an unwritten act row"
            tiles = [t for w in range(WAVES) for t in _owned_tiles(rg * DOWN_ROWS // ROW_TILE + 4 * w, 4, H // ROW_TILE - 1)]
            for q in range(m):
                part_s[sp, off + q, tiles] += 1
        else:
            it = _routed_item(b - s_blocks_dn, rgroups * splits, recs, span)
            if it is None:
                continue
            off, m, g = it
            sp, rg = divmod(g, rgroups)
            c0, c1 = k_cols(sp, plan["split_steps"], I)
            # token rows off + min(q, m - 1), q < 128: exactly rows [off, off + m)
            assert (act[off:off + m, c0:c1] == 1).all(), "down reads an unwritten act row"
            tiles = [t for w in range(WAVES) for t in _owned_tiles(rg * DOWN_ROWS // ROW_TILE + 4 * w, 4, H // ROW_TILE - 1)]
            for q in range(m):
                part[sp, sorted_f[off + q], tiles] += 1
    assert (part <= 1).all() and (part_s <= 1).all(), "a partial written twice"

    # combine: every split of every contributing assignment (and of the shared expert)
    for f in range(N):
        if ok[f]:
            assert (part[:, f, :] == 1).all(), f"combine reads an unwritten partial of f={f}"
        else:
            assert (part[:, f, :] == 0).all(), f"a dropped assignment f={f} was computed"
    if Is:
        assert (part_s[:s_splits] == 1).all(), "combine reads an unwritten shared partial"
    return dict(ranges=nranges, gateup_items=items, sorted=routed_rows)
