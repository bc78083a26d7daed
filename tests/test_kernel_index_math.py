"""CPU emulation of the HIP kernels' index math (no GPU).

Each kernel's work decomposition is replayed on the host with the kernel's
own formulas, and every index it forms is checked against the buffer it
addresses, before any of it runs on a GPU:

  * permute (count_kernel + scatter_kernel, reframework_amd/csrc/permute.hip):
    the scatter's LDS tables (`total`, `base`, the per-wave `wave_cnt`, the
    per-part prefix sums over the count table) are replayed per block, round
    and wave with every LDS word poisoned at kernel start, so a read of a word
    the kernel never wrote fails; the ballot ranking
    is replayed bit by bit. Every slot_to_row / row_src write must stay in
    bounds, every row must be written once, and the result must equal the
    oracle's stable grouping. A planted mistake (the per-round zeroing of
    `wave_cnt` covering only wave 0's row, which once sent row_src out of
    bounds on the GPU) must be caught.
  * the tiled grouped GEMM (ffn_tiled.h): the persistent schedule (XCD
    remap, work_split's K-split tail, decode_tile's per-expert item groups)
    must cover every (K-split, permuted row, weight tile) exactly once, by a
    whole item or by all S K-parts of a split item, whose partial tiles stay
    within the workspace; every token row the MFMAs read (all 256 rows of a
    256-row tile; on 128-row tiles the 128 rows of the compact token buffer
    that the two token-loading waves fill) is a loaded row of the tile or a
    zero-filled padding row, and every valid row is read; token and weight
    offsets stay in their 32-bit buffer ranges.
  * the weight-streaming kernel's in-kernel grouping (ffn_skinny.hip,
    group_slots): its outputs must equal the permute's, every LDS, meta and
    global index must stay in its array, and every tile it hands a workgroup
    must lie inside one expert's rows.

Shapes: the workloads the throughput figures are quoted on (Mixtral 1, 16,
256 and 4096 tokens; Phi-3.5 2048 with Zipf-skewed routing; the fine-grained
layer at 8 and 4096 tokens with its two shared columns) plus ragged and
dropped-slot cases.
"""

from __future__ import annotations

import numpy as np
import pytest

from _helpers import skewed_ids, tile_height, tile_order
from oracle import oracle
from reframework_amd import _capi

WAVE, THREADS = 64, 256
WAVES = THREADS // WAVE
CHUNK = 256           # kPermuteChunk: slots per block of the count + scatter launches
SINGLE_MAX = 1024     # kPermuteSingleMax: up to this many slots one block permutes
POISON = -(1 << 40)   # an LDS word nobody wrote


# ------------------------------------------------------------------ permute
def _routed(ids_flat, emap, E):
    """routed_expert(): the local expert of each slot, -1 when dropped."""
    out = np.empty(len(ids_flat), np.int64)
    for s, g in enumerate(ids_flat):
        if emap:
            out[s] = emap[g] if 0 <= g < len(emap) else -1
        else:
            out[s] = g if 0 <= g < E else -1
        if out[s] >= E:
            out[s] = -1
    return out


def _emulate_prefix(counts, b, E, parts_overrun=False):
    """The scatter's per-block prefix over the count table: thread tid sums
    expert tid % E over block part tid // E of P = min(256 // E, 8) parts,
    and the parts are added in LDS. Checks every count-table read and LDS
    index."""
    n_blocks = counts.shape[0]
    table = counts.reshape(-1)
    P = min(THREADS // E, 8)
    ptot = np.full(THREADS, POISON, np.int64)
    ppre = np.full(THREADS, POISON, np.int64)
    for tid in range(THREADS):
        e, p = tid % E, tid // E
        tot = pre = 0
        if p < P:
            per = -(-n_blocks // P)
            for bb in range(p * per, min(n_blocks, (p + 1) * per)):
                idx = bb * E + e
                assert 0 <= idx < table.size, f"count-table read {idx} outside [0, {table.size})"
                tot += int(table[idx])
                pre += int(table[idx]) if bb < b else 0
        ptot[tid], ppre[tid] = tot, pre
    total = np.zeros(E, np.int64)
    base = np.zeros(E, np.int64)
    for x in range(E):
        for q in range(P + 1 if parts_overrun else P):
            i = q * E + x
            assert 0 <= i < THREADS and ptot[i] != POISON, f"LDS part {i} unwritten or out of range"
            total[x] += ptot[i]
            base[x] += ppre[i]
    return total, base


def emulate_permute(ids, E, tile_rows, max_tiles, emap=None, zero_first_row_only=False):
    """Replays count_kernel / scatter_kernel. Returns (offsets, slot_to_row,
    row_src, tile_map); raises AssertionError on an out-of-bounds index, a
    row written twice or a read of unwritten LDS."""
    T, K = ids.shape
    R = T * K
    e_of = _routed(ids.reshape(-1), emap, E)
    n_blocks = 1 if R <= SINGLE_MAX else -(-R // CHUNK)
    rounds = SINGLE_MAX // THREADS if n_blocks == 1 else CHUNK // THREADS
    counts = np.zeros((n_blocks, E), np.int64)  # count_kernel (or the one block's own count)
    for s in range(R):
        if e_of[s] >= 0:
            counts[0 if n_blocks == 1 else s // CHUNK, e_of[s]] += 1
    slot_to_row = np.full(R, POISON, np.int64)
    row_src = np.full(R, POISON, np.int64)
    offsets = tile_map = None
    for b in range(n_blocks):
        if n_blocks > 1:
            total, base = _emulate_prefix(counts, b, E)
        else:
            total, base = counts[0].copy(), np.zeros(E, np.int64)
        start = np.concatenate([[0], np.cumsum(total)])
        tiles = -(-total // tile_rows)
        tile_start = np.concatenate([[0], np.cumsum(tiles)])
        tile_start[E] = min(tile_start[E], max_tiles)
        base = base + start[:E]
        if b == 0:
            offsets = start.copy()
            nt = int(tile_start[E])
            tile_map = [nt, tile_rows]
            # the kernel's place of each expert: its rank r by (rows desc, id)
            # at 2 r in the first half, 2 (E - 1 - r) + 1 in the second
            order = np.full(E, POISON, np.int64)
            for e in range(E):
                r = sum(1 for f in range(E) if total[f] > total[e] or (total[f] == total[e] and f < e))
                p = 2 * r if 2 * r < E else 2 * (E - 1 - r) + 1
                assert 0 <= p < E and order[p] == POISON
                order[p] = e
            place_start = np.concatenate([[0], np.cumsum(tiles[order])])
            for j in range(nt):
                lo = int(np.searchsorted(place_start[:E], j, side="right") - 1)
                e = int(order[lo])
                h = tile_height(int(start[e + 1] - start[e]), tile_rows)
                tile_map += [e, int(start[e] + (j - place_start[lo]) * h)]
        wave_cnt = np.full((WAVES, 256), POISON, np.int64)  # LDS at kernel start
        r = 0
        while r < rounds and b * CHUNK + r * THREADS < R:
            # per-round zeroing, as the kernel indexes it
            for i in range(WAVES * E):
                if zero_first_row_only:
                    wave_cnt.reshape(-1)[i] = 0  # the flat-index mistake
                else:
                    wave_cnt[i // E, i % E] = 0
            slots = b * CHUNK + r * THREADS + np.arange(THREADS)
            es = np.array([e_of[s] if s < R else -1 for s in slots])
            rank = np.zeros(THREADS, np.int64)
            for w in range(WAVES):
                lanes = es[w * WAVE:(w + 1) * WAVE]
                routed = lanes >= 0
                bits = [((lanes >> bit) & 1).astype(bool) for bit in range(8)]
                for ln in range(WAVE):
                    if not routed[ln]:
                        continue
                    same = routed.copy()
                    for bit in range(8):
                        same &= bits[bit] if bits[bit][ln] else ~bits[bit]
                    rank[w * WAVE + ln] = int(same[:ln].sum())
                    if rank[w * WAVE + ln] == 0:
                        wave_cnt[w, lanes[ln]] = int(same.sum())
            for t in range(THREADS):
                s = slots[t]
                if s >= R:
                    continue
                e = es[t]
                if e < 0:
                    slot_to_row[s] = -1
                    continue
                w = t // WAVE
                assert all(wave_cnt[v, e] != POISON for v in range(w)), "unwritten LDS read"
                row = int(base[e] + rank[t] + sum(wave_cnt[v, e] for v in range(w)))
                assert 0 <= row < R, f"row {row} outside [0, {R})"
                assert row_src[row] == POISON, f"row {row} written twice"
                slot_to_row[s] = row
                row_src[row] = s // K
            for ee in range(E):
                col = wave_cnt[:, ee]
                assert (col != POISON).all(), "unwritten LDS read"
                base[ee] += int(col.sum())
            r += 1
    return offsets, slot_to_row, row_src, tile_map


def _mixtral_ids(T, seed=0):
    return skewed_ids(T, 2, 8, seed=seed, skew=0.5)


def _finegrained_ids(T, seed=0):
    routed = np.argsort(np.random.default_rng(seed).random((T, 64)), axis=1)[:, :6]
    return np.concatenate([routed, np.full((T, 1), 64), np.full((T, 1), 65)], 1).astype(np.int64)


PERMUTE_CASES = [
    ("mixtral_t1", lambda: _mixtral_ids(1), 8, None),
    ("mixtral_t16", lambda: _mixtral_ids(16), 8, None),
    ("mixtral_t256", lambda: _mixtral_ids(256), 8, None),
    ("mixtral_t4096", lambda: _mixtral_ids(4096), 8, None),
    ("phi35_t2048", lambda: skewed_ids(2048, 2, 16, seed=3, skew=1.1), 16, None),
    ("finegrained_t8", lambda: _finegrained_ids(8), 66, None),
    ("finegrained_t4096", lambda: _finegrained_ids(4096), 66, None),
    ("experts256_t1500_k8", lambda: skewed_ids(1500, 8, 256, seed=5, skew=0.8), 256, None),
    ("finegrained_t700_dropped", lambda: _finegrained_ids(700, 1), 66,
     [(-1 if e % 5 == 3 else e) for e in range(66)]),
]


@pytest.mark.parametrize("name,make,E,emap", PERMUTE_CASES, ids=[c[0] for c in PERMUTE_CASES])
def test_permute_emulation_in_bounds_and_equal_to_oracle(name, make, E, emap):
    ids = make()
    T, K = ids.shape
    plan = _capi.make_plan(T, 4096, 14336, E, K, _capi.BF16)
    assert plan.n_blocks == (1 if T * K <= SINGLE_MAX else -(-T * K // CHUNK))
    offsets, s2r, src, tile_map = emulate_permute(ids, E, plan.tile_rows, plan.max_tiles, emap)
    o_off, o_s2r, o_src = oracle.permute(ids, E, emap)
    assert np.array_equal(offsets, o_off)
    assert np.array_equal(s2r, o_s2r)
    n = int(offsets[-1])
    assert np.array_equal(src[:n], o_src[:n])
    assert (src[n:] == POISON).all()  # rows past the routed ones are never written
    assert tile_map[0] <= plan.max_tiles
    # every expert's tiles, its tile height apart, in the interleaved size order
    counts = np.diff(o_off)
    want = [(e, int(o_off[e]) + j * tile_height(int(counts[e]), plan.tile_rows))
            for e in tile_order(counts) for j in range(-(-int(counts[e]) // plan.tile_rows))]
    assert tile_map[0] == len(want)
    assert [tuple(tile_map[2 + 2 * j:4 + 2 * j]) for j in range(len(want))] == want


def test_permute_emulation_catches_partial_wave_table_zeroing():
    """The planted mistake: clearing the first 4*E flat words of
    wave_cnt[4][256] clears only wave 0's row; a multi-wave round must then
    read stale (here: unwritten) counts."""
    ids = _finegrained_ids(700, 1)
    with pytest.raises(AssertionError):
        emulate_permute(ids, 66, 256, 10_000, zero_first_row_only=True)


def test_permute_prefix_emulation_catches_part_overrun():
    """Planted mistake: summing one part too many reads past the 256 LDS
    partial sums for 32 experts (8 parts)."""
    counts = np.ones((40, 32), np.int64)
    assert _emulate_prefix(counts, 3, 32)[0].tolist() == [40] * 32
    assert _emulate_prefix(counts, 3, 32)[1].tolist() == [3] * 32
    with pytest.raises(AssertionError):
        _emulate_prefix(counts, 3, 32, parts_overrun=True)


# ------------------------------------------------------------- tiled GEMM
def xcd_remap(pid, nwg):
    xcd, slot = pid & 7, pid >> 3
    q, rem = nwg >> 3, nwg & 7
    base = xcd * (q + 1) if xcd < rem else rem * (q + 1) + (xcd - rem) * q
    return base + slot


def work_split(n_work, G, nk, cap):
    """(n_full, n_units, S) as dma_pipe.h work_split derives it."""
    Rr = n_work // G if G > 0 else 0
    tail = n_work - Rr * G
    if cap <= 0 or tail == 0:
        return n_work, 0, 1
    cap = min(cap, G)
    best, S, s = 14 * nk, 1, 2
    while s <= 16 and s * tail <= cap and nk % s == 0:
        c = 14 * nk // s + s * tail
        if c < best:
            best, S = c, s
        s *= 2
    return (Rr * G, tail * S, S) if S > 1 else (n_work, 0, 1)


def emulate_tiled(counts, plan, gate_up, cus=256, T=None):
    """Replays one tiled launch (gate_up or down) over per-expert row counts;
    returns the number of work sequence entries. Asserts exactly-once
    coverage, ragged-tile row coverage and buffer bounds."""
    E, H, I = plan.E, plan.H, plan.I
    tile_rows = plan.tile_rows
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    R = int(offs[-1])

    def height(e):
        # full tiles share the expert's rows evenly, in heights rounded up to
        # 32 rows (1085 rows: 5 tiles of 224 and 189 rows)
        return tile_height(int(counts[e]), tile_rows)

    # the permute's tile map: an expert's tiles its tile height apart, the
    # experts in the interleaved size order
    tiles = [(e, int(offs[e] + j * height(e))) for e in tile_order(counts)
             for j in range(-(-int(counts[e]) // tile_rows))]
    n_t = len(tiles)
    assert n_t <= plan.max_tiles
    S_d = 1 if gate_up else plan.down_splits
    n_wt = I // 128 if gate_up else H // 256
    per_split = n_wt * n_t
    n_work = S_d * per_split
    G = min(n_wt * plan.max_tiles * S_d, cus)
    k_per_split = H if gate_up else I // S_d
    nk = k_per_split // 64
    if gate_up:
        cap = min((plan.workspace_bytes - plan.off_y) // (256 * 256 * 4), 4096)
    else:
        cap = (plan.workspace_bytes - plan.off_part) // (256 * 256 * 4)
    n_full, n_units, S = work_split(n_work, G, nk, cap)

    def decode_tile(L):
        split = L // per_split
        rem = L - split * per_split
        t0 = rem // n_wt
        e = tiles[t0][0]
        eb, ee = int(offs[e]), int(offs[e + 1])
        b = t0 - (tiles[t0][1] - eb) // height(e)
        ne = (ee - eb + tile_rows - 1) // tile_rows
        r2 = rem - b * n_wt
        wt = r2 // ne
        tt = b + (r2 - wt * ne)
        assert tiles[tt][0] == e
        row0 = tiles[tt][1]
        assert row0 == eb + (tt - b) * height(e)
        return split, wt, e, row0, min(row0 + height(e), ee)

    whole = np.zeros((S_d, R, n_wt), np.int64)
    parts, kcover = {}, {}
    n_seq = n_full + n_units
    lds_rows = np.arange(256)
    # ragged launches (full tiles, <= 512 routed rows per active expert):
    # per-item token-block count and rotated XCD slots
    act = min(E, plan.rows)
    ragged = tile_rows == 256 and act > 0 and plan.rows // act <= 512

    def next_item(pid, L):
        # the full-tile kernel's item sequence: in ragged launches rotated
        # slots in whole rounds of full items, else (and in the other rounds)
        # slot s; the 128-row kernel steps by G
        if not ragged:
            return L + G
        slot = pid >> 3
        n_x = (G >> 3) + (1 if (pid & 7) < (G & 7) else 0)
        base = xcd_remap(pid, G) - slot
        k = L // G + 1
        rot = (slot + 13 * k) % n_x if (k + 1) * G <= n_full else slot
        return k * G + base + rot

    for pid in range(G):
        L = xcd_remap(pid, G)
        while L < n_seq:
            if L < n_full:
                split, wt, e, r0, r1 = decode_tile(L)
                whole[split, r0:r1, wt] += 1
            else:
                u = L - n_full
                assert u < cap, f"partial tile {u} past the {cap} the workspace holds"
                it = n_full + u // S
                split, wt, e, r0, r1 = decode_tile(it)
                kb = (u % S) * (nk // S)  # decode_work's step range
                kcover.setdefault(it, []).append((kb, kb + nk // S))
                parts.setdefault(it, []).append(u % S)
            n = r1 - r0
            assert 1 <= n <= tile_rows
            half = tile_rows < 256
            # tile row held by each row of the token buffer: 256 rows of the
            # full-tile buffer; the 128 rows of the compact half-tile buffer
            # (ffn_tiled_half_kernel), which its two token waves fill, 8 loads
            # of 8 rows each: rows (8 w + q) * 8 + lane / 8
            if half:
                held = np.array(sorted((8 * w + q) * 8 + ln // 8 for w in range(2)
                                       for q in range(8) for ln in range(0, 64, 8)))
                assert np.array_equal(held, np.arange(128))
            else:
                held = lds_rows
            # tile rows the MFMAs read: on half tiles token half h (64 rows),
            # two 32-row blocks j of v_mfma_f32_32x32x16; on full tiles 16-row
            # blocks of v_mfma_f32_16x16x32, interleaved between the token waves
            if half:
                read = {h * 64 + j * 32 + lr for h in range(2) for j in range(2) for lr in range(32)}
                used = read
            else:
                # token wave h's block j is tile rows 16 (2 j + h) ..; the
                # LDS reads cover all 8 blocks, the MFMAs blocks j < J (ragged:
                # J = ceil(n / 32), else the expert's tile height / 32)
                read = {(2 * j + h) * 16 + lr for h in range(2) for j in range(8) for lr in range(16)}
                J = min(8, -(-(n if ragged else height(e)) // 32))
                assert n <= height(e) <= tile_rows
                used = {(2 * j + h) * 16 + lr for h in range(2) for j in range(J) for lr in range(16)}
            assert set(range(n)) <= used <= read and max(read) < tile_rows
            assert read <= set(held.tolist())
            # every LDS row is loaded from a valid row or zero-filled
            valid = r0 + held < r1
            src_rows = np.minimum(r0 + np.minimum(held, tile_rows - 1), r1 - 1)
            assert (src_rows >= 0).all() and (src_rows < R).all()
            pitch = (H if gate_up else I) * 2
            if not gate_up:
                assert ((held[valid]) * pitch + 7 * 16 + (nk - 1) * 128 < 2 ** 31).all()
            # weight rows of the tile and their 32-bit offsets
            if gate_up:
                wr = np.concatenate([wt * 128 + np.arange(128), I + wt * 128 + np.arange(128)])
                assert wr.max() < 2 * I
                assert int(wr.max()) * pitch + 128 * nk <= 2 ** 32
            else:
                wr = wt * 256 + np.arange(256)
                assert wr.max() < H
            L = next_item(pid, L)
    for it, ks in parts.items():
        assert sorted(ks) == list(range(S)), f"item {it}: K-parts {ks}"
        # the parts' step ranges tile [0, nk) without gap or overlap
        rng = sorted(kcover[it])
        assert rng[0][0] == 0 and rng[-1][1] == nk and all(a[1] == b[0] for a, b in zip(rng, rng[1:]))
        split, wt, e, r0, r1 = decode_tile(it)
        whole[split, r0:r1, wt] += 1
    assert (whole == 1).all(), "a (split, row, weight tile) is not covered exactly once"
    # fix-up tasks cover the split items' rows once: per item, gate blocks x
    # token blocks (gate_up) or weight blocks x groups of 4 token blocks (down)
    per_item = 32 if gate_up else 16
    tasks = n_units // S * per_item
    assert tasks == len(parts) * per_item
    return n_seq


def _counts(ids, E):
    return np.bincount(ids.reshape(-1), minlength=E)[:E]


TILED_CASES = [
    ("mixtral_t4096", 4096, 4096, 14336, 8, lambda: _mixtral_ids(4096)),
    ("mixtral_t256", 256, 4096, 14336, 8, lambda: _mixtral_ids(256)),
    ("mixtral_t1536", 1536, 4096, 14336, 8, lambda: _mixtral_ids(1536, 2)),
    ("phi35_t2048", 2048, 4096, 6400, 16, lambda: skewed_ids(2048, 2, 16, seed=3, skew=1.1)),
    ("finegrained_t4096", 4096, 2048, 1408, 66, lambda: _finegrained_ids(4096)),
    ("ragged_e64", 1000, 4096, 256, 64, lambda: skewed_ids(1000, 1, 64, seed=5, skew=1.5)),
    # the counts of the GPU balanced-tile-height tests (every token-block count)
    ("balanced_e8", 3083, 512, 2048, 8, lambda: _ids_of([257, 300, 513, 700, 1025, 1, 32, 255])),
    ("balanced_e11", 6683, 512, 2048, 11,
     lambda: _ids_of([257, 300, 513, 700, 1025, 1, 32, 255, 1200, 1200, 1200])),
    ("balanced_e16", 3078, 512, 1536, 16,
     lambda: _ids_of([29, 94, 140, 187, 257, 281, 369, 514, 1, 33, 64, 97, 128, 160, 224, 500])),
    # the many-expert top-8 cases of the GPU expert tests (same routing)
    ("e128_k8_prefill", 2048, 512, 256, 128, lambda: skewed_ids(2048, 8, 128, seed=2048, skew=1.0)),
    ("e128_k8_half_tiles", 600, 512, 256, 128, lambda: skewed_ids(600, 8, 128, seed=600, skew=1.0)),
    ("e256_k8_half_tiles", 1024, 256, 256, 256,
     lambda: skewed_ids(1024, 8, 256, seed=1024, skew=1.0)),
]


def _ids_of(counts):
    return np.repeat(np.arange(len(counts)), counts)[:, None]


@pytest.mark.parametrize("gate_up", [True, False], ids=["gate_up", "down"])
@pytest.mark.parametrize("name,T,H,I,E,make", TILED_CASES, ids=[c[0] for c in TILED_CASES])
def test_tiled_schedule_covers_once_in_bounds(name, T, H, I, E, make, gate_up):
    ids = make()
    K = ids.shape[1]
    plan = _capi.make_plan(T, H, I, E, K, _capi.BF16)
    assert plan.path in (_capi.PATH_MFMA_TILED, _capi.PATH_MFMA_TILED128)
    emulate_tiled(_counts(ids, E), plan, gate_up)
    # the same routing on a forced 256-row tile map and a 128-row one
    for path in (_capi.PATH_MFMA_TILED, _capi.PATH_MFMA_TILED128):
        emulate_tiled(_counts(ids, E), _capi.make_plan(T, H, I, E, K, _capi.BF16, path), gate_up)


@pytest.mark.parametrize("cus", [256, 80, 304])
def test_tiled_schedule_on_other_cu_counts(cus):
    """Workgroups per launch follow the device's CU count: the decomposition
    holds for other counts too (the workspace is planned for 256 here)."""
    ids = skewed_ids(3000, 2, 16, seed=8, skew=1.2)
    plan = _capi.make_plan(3000, 4096, 2048, 16, 2, _capi.BF16)
    for gate_up in (True, False):
        emulate_tiled(_counts(ids, 16), plan, gate_up, cus=cus)


# --------------------------------------------------- skinny in-kernel grouping
GROUP_PER_LANE = 4  # kGroupExpertsPerLane


def emulate_group_slots(ids, E, max_tiles, emap=None, rows=16, ttile=0):
    """Replays group_slots: one wave groups <= 64 slots (lane s = slot s)
    through per-expert 64-bit slot masks in LDS, lane l owning experts
    4 l .. 4 l + 3, with every LDS, meta and global index checked against
    its array."""
    T, K = ids.shape
    R = T * K
    assert R <= WAVE and E <= GROUP_PER_LANE * WAVE
    emask = [None] * (GROUP_PER_LANE * WAVE)   # LDS: unset until zeroed
    estart = [None] * (GROUP_PER_LANE * WAVE)
    rowsrc = [None] * WAVE
    for lane in range(WAVE):
        for i in range(GROUP_PER_LANE):
            emask[GROUP_PER_LANE * lane + i] = 0
    e = np.full(WAVE, -1, np.int64)
    e[:R] = _routed(ids.reshape(-1), emap, E)
    for lane in range(WAVE):
        if e[lane] >= 0:
            assert 0 <= e[lane] < len(emask)
            emask[e[lane]] |= 1 << lane
    cnt = np.zeros((WAVE, GROUP_PER_LANE), np.int64)
    for lane in range(WAVE):
        for i in range(GROUP_PER_LANE):
            x = GROUP_PER_LANE * lane + i
            cnt[lane, i] = bin(emask[x]).count("1") if x < E else 0
    nt = -(-cnt // rows)
    rows_l, tiles_l = cnt.sum(1), nt.sum(1)
    rstart0 = np.concatenate([[0], np.cumsum(rows_l)[:-1]])
    tstart0 = np.concatenate([[0], np.cumsum(tiles_l)[:-1]])
    total_rows, total_tiles = int(rows_l.sum()), int(tiles_l.sum())
    assert total_tiles <= max_tiles
    offsets = np.full(E + 1, POISON, np.int64)
    tile_map = {}
    meta = [total_tiles, -1, 0, 0]
    hits = 0
    for lane in range(WAVE):
        rs, ts = int(rstart0[lane]), int(tstart0[lane])
        for i in range(GROUP_PER_LANE):
            x = GROUP_PER_LANE * lane + i
            if x < E:
                estart[x] = rs
                if ts <= ttile < ts + nt[lane, i]:
                    r0 = rs + (ttile - ts) * rows
                    meta[1:] = [x, r0, min(r0 + rows, rs + int(cnt[lane, i]))]
                    hits += 1
                offsets[x] = rs
                for j in range(int(nt[lane, i])):
                    assert 2 + 2 * (ts + j) + 1 < 2 + 2 * max_tiles
                    tile_map[ts + j] = (x, rs + j * rows)
            rs += int(cnt[lane, i])
            ts += int(nt[lane, i])
    assert hits == (1 if ttile < total_tiles else 0)
    offsets[E] = total_rows
    slot_to_row = np.full(R, -1, np.int64)
    row_src = {}
    for lane in range(WAVE):
        if e[lane] < 0:
            continue
        assert estart[e[lane]] is not None
        below = emask[e[lane]] & ((1 << lane) - 1)
        row = estart[e[lane]] + bin(below).count("1")
        assert 0 <= row < total_rows <= R <= len(rowsrc)
        assert row not in row_src
        rowsrc[row] = lane // K
        row_src[row] = lane // K
        slot_to_row[lane] = row
    return offsets, slot_to_row, row_src, [tile_map[j] for j in range(total_tiles)], meta


@pytest.mark.parametrize("T,K,E,drop", [(1, 2, 8, False), (8, 2, 8, True), (4, 4, 32, True),
                                        (2, 8, 32, False), (5, 3, 16, False), (16, 2, 8, False),
                                        (32, 2, 8, True), (8, 6, 64, False), (8, 8, 256, True),
                                        (3, 6, 64, True), (20, 3, 8, False), (64, 1, 8, False),
                                        (16, 4, 16, True)])
def test_skinny_grouping_equals_permute_and_stays_in_bounds(T, K, E, drop):
    ids = skewed_ids(T, K, E, seed=T * E + K, skew=1.2)
    emap = [(-1 if x % 5 == 3 else x) for x in range(E)] if drop else None
    plan = _capi.make_plan(T, 4096, 14336, E, K, _capi.BF16)
    assert plan.path == _capi.PATH_MFMA_SKINNY and plan.rows <= 64
    o_off, o_s2r, o_src = oracle.permute(ids, E, emap)
    for ttile in range(plan.max_tiles):
        offsets, s2r, rsrc, tmap, meta = emulate_group_slots(ids, E, plan.max_tiles, emap,
                                                             ttile=ttile)
        assert np.array_equal(offsets, o_off) and np.array_equal(s2r, o_s2r)
        assert all(o_src[r] == t for r, t in rsrc.items()) and len(rsrc) == o_off[-1]
        for (e, row0) in tmap:  # each tile inside its expert's rows, in expert order
            assert o_off[e] <= row0 < o_off[e + 1]
        assert [e for e, _ in tmap] == sorted(e for e, _ in tmap)
        if ttile < meta[0]:  # the workgroup's tile is the map's
            e, r0, r1 = meta[1:]
            assert tmap[ttile] == (e, r0) and r0 < r1 <= o_off[e + 1]


def test_skinny_grouping_fine_grained_decode_with_shared_columns():
    """The fine-grained layer at 8 tokens: 6 routed slots and the 2 shared
    columns per token, 64 slots over 66 experts (one wave's worth)."""
    ids = _finegrained_ids(8)
    plan = _capi.make_plan(8, 2048, 1408, 66, 8, _capi.BF16)
    assert plan.path == _capi.PATH_MFMA_SKINNY and plan.rows == 64
    o_off, o_s2r, o_src = oracle.permute(ids, 66)
    for ttile in range(plan.max_tiles):
        offsets, s2r, rsrc, tmap, meta = emulate_group_slots(ids, 66, plan.max_tiles, ttile=ttile)
        assert np.array_equal(offsets, o_off) and np.array_equal(s2r, o_s2r)
        assert all(o_src[r] == t for r, t in rsrc.items())


# ------------------------------------------------ random shapes (CPU replay)
import _random_shapes  # noqa: E402


@pytest.mark.parametrize("c", _random_shapes.ALL, ids=_random_shapes.name)
def test_random_shapes_index_math_in_bounds(c):
    """The configurations of tests/test_gpu_random_shapes.py, replayed here
    first: the permute (or the in-kernel grouping at <= 64 slots) equal to the
    oracle's grouping and in bounds, and the tiled schedules covering every
    item once within their buffers."""
    T, K, E = c["T"], c["K"], c["E"]
    ids = skewed_ids(T, K, E, c["seed"], c["skew"])
    emap = c["emap"]
    plan = _capi.make_plan(T, c["H"], c["I"], E, K, _random_shapes.DTYPES[c["dt"]])
    o_off, o_s2r, _ = oracle.permute(ids, E, emap)
    if plan.path == _capi.PATH_MFMA_SKINNY and plan.rows <= 64:
        for t in range(plan.max_tiles):
            offsets, s2r, _, _, _ = emulate_group_slots(ids, E, plan.max_tiles, emap, ttile=t)
            assert np.array_equal(offsets, o_off) and np.array_equal(s2r, o_s2r)
    else:
        offsets, s2r, _, _ = emulate_permute(ids, E, plan.tile_rows, plan.max_tiles, emap)
        assert np.array_equal(offsets, o_off) and np.array_equal(s2r, o_s2r)
    if plan.path in (_capi.PATH_MFMA_TILED, _capi.PATH_MFMA_TILED128):
        counts = np.diff(o_off)
        emulate_tiled(counts, plan, True)
        emulate_tiled(counts, plan, False)


def emulate_norm_router_tile(H, E, T, t0):
    """add_rmsnorm_router_mfma_kernel's addressing (norm.hip) for the
    workgroup of rows t0.., restated: returns the tile byte offsets written
    per (row, chunk), the logical (row, chunk) behind each MFMA A fragment,
    and the gate element offsets of the B fragments. Checks bounds as it goes."""
    N, TOK = 8, 8       # kNormRouterRows rows per workgroup
    cpt = 1 if H <= 2048 else 2
    max_h = cpt * THREADS * N
    tile_bytes = TOK * max_h * 2
    chunks, pitch = H // N, max_h * 2
    ntok = min(TOK, T - t0)
    assert ntok >= 1
    slot = lambda t, ch: t * pitch + ((ch ^ t) << 4)
    # direct-to-LDS loads: lane `lane` of wave w, pass c, row t writes the 16
    # bytes at t * pitch + (64 w + 256 c) * 16 + 16 lane, holding x chunk s ^ t
    # of row min(t, ntok - 1) (s = its thread's slot), or zeros past the row
    loaded, filler = {}, {}
    for t in range(TOK):
        src = min(t, ntok - 1)
        assert 0 <= t0 + src < T
        for tid in range(THREADS):
            w, lane = divmod(tid, WAVE)
            for c in range(cpt):
                s = tid + c * THREADS
                dst = t * pitch + (w * WAVE + c * THREADS) * 16 + 16 * lane
                assert 0 <= dst and dst + 16 <= tile_bytes and dst not in loaded
                if s < chunks:
                    assert (s ^ t) < chunks and src * H * 2 + ((s ^ t) << 4) + 16 <= H * 2 * ntok
                    loaded[dst], filler[dst] = (t, s ^ t), tid
                else:
                    loaded[dst], filler[dst] = None, tid
    written = {}
    for t in range(TOK):
        for tid in range(THREADS):
            for c in range(cpt):
                ch = tid + c * THREADS
                if ch >= chunks:
                    continue
                off = slot(t, ch)
                assert 0 <= off and off + 16 <= tile_bytes
                # the slot holds this chunk, loaded by a lane of the same wave
                assert loaded[off] == (t, ch) and filler[off] // WAVE == tid // WAVE
                written[(t, ch)] = off
    assert len(written) == TOK * chunks and len(set(written.values())) == len(written)
    nb = H // 256
    reads, gate = [], []
    for wave in range(WAVES):
        cbase = wave * (H // 32)
        for b in range(nb):
            for u in range(2):
                offs = []
                for lane in range(WAVE):
                    r16, kq = lane & 15, lane >> 4
                    C = cbase + 8 * b + 4 * u + kq
                    assert C < chunks
                    off = slot(r16 % TOK, C)  # fragment rows TOK.. repeat rows 0..
                    assert off == written[(r16 % TOK, C)]
                    if r16 < TOK:
                        reads.append((r16, C))
                    offs.append(off)
                    g0 = min(r16, E - 1) * H + wave * (H // 4) + kq * 8 + b * 64 + u * 32
                    assert min(r16, E - 1) < E and wave * (H // 4) + kq * 8 + b * 64 + u * 32 + 8 <= H
                    gate.append(g0)
                # the rows of one k group sit in distinct 16-byte slots of one
                # 128-byte span (lanes of a repeated row read the same address)
                for kq in range(4):
                    grp = offs[16 * kq:16 * kq + TOK]
                    assert len({(o % 128) // 16 for o in grp}) == TOK
                    assert len({o // 128 % (pitch // 128) for o in grp}) == 1
    return written, reads, gate


@pytest.mark.parametrize("H,E,T,t0", [(4096, 8, 4096, 4088), (2048, 16, 2054, 2048),
                                      (256, 5, 2000, 1992), (3072, 12, 2048, 0),
                                      (512, 9, 2051, 2048), (1024, 16, 4096, 16)])
def test_norm_router_mfma_tile_addressing(H, E, T, t0):
    written, reads, gate = emulate_norm_router_tile(H, E, T, t0)
    # every chunk of every row is read exactly once, by the wave owning its quarter
    assert sorted(reads) == sorted(written)
    # the A fragment of lane (r, kq), step (b, u) of wave w holds k = w H/4 +
    # 64 b + 32 u + 8 kq .. + 7 of row r; the B fragment the same k of its gate
    # row: per gate row, every k exactly once
    k_of = sorted(g % H for g in gate)
    assert k_of == sorted(list(range(0, H, 8)) * 16)
