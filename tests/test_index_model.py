"""Host replica of the backward kernels' index arithmetic (csrc/moc_mfma.h
bwd_tile, csrc/moc_bwd_lean.h bwd_lean_tile, csrc/moc_mfma_launch.h grids):

  * every LDS index a lane forms (routing-weight rows and swizzled columns, m
    tile slots written and read transposed, dalpha operand rows, dalpha tiles)
    lies inside its array, and the transposed reads fetch exactly the slots the
    writers filled (each slot written by one lane, read back by the lanes that
    want its tokens and channels);
  * over the whole grid (route halves of the taps pass, two-tier token ranges)
    every dalpha / dbasis partial that stage 2 sums is written exactly once.

Pure integer arithmetic on the CPU, for the shapes whose kernels run on the GPU
(the 8-tap 64-route prefill taps pass included).  The formulas restate the
kernels' own; the point is the exhaustive extent and coverage check over every
lane, wave, workgroup and super-block, which no GPU test can observe directly.
"""
from __future__ import annotations

import itertools

import pytest


def cdiv(a, b):
    return -(-a // b)


# ---------------------------------------------------------------------------
# grids (csrc/moc_mfma_launch.h)

def bwd_eown(S, taps=False):
    """Own rows per 32-row super-block: all of them in the taps pass, the first
    32 - (S-1) elsewhere."""
    return 32 if taps else 32 - (S - 1)


def bwd_grid_gx(N, gx, D, S, target, taps=False):
    eown = bwd_eown(S, taps)
    n_super = cdiv(N, eown)
    gy_target = max(target // gx, 1)
    n_sb = cdiv(n_super, gy_target)
    max_sb = ((1 << 30) // (D * 4) - 32) // eown
    if n_sb > max_sb:
        n_sb = max(max_sb, 1)
    gy = cdiv(n_super, n_sb)
    return dict(gx=gx, gy=gy, n_sb=n_sb, gy1=gy, n_old=n_sb * gy, n_total=n_sb * gy)


def tiered(N, gx, D, S, n_cu, share=62):
    g = bwd_grid_gx(N, gx, D, S, 512)
    if n_cu % g["gx"]:
        return g
    gy1 = n_cu // g["gx"]
    if g["gy"] != 2 * gy1:
        return g
    eown = 32 - (S - 1)
    n_super = cdiv(N, eown)
    n_old = (n_super * share + 50) // 100
    n1, n2 = cdiv(n_old, gy1), cdiv(n_super - n_old, g["gy"] - gy1)
    if n2 < 1 or n2 > n1:
        return g
    return dict(g, n_sb=n1, gy1=gy1, n_old=n_old, n_total=n_super)


def sb_range(by, g):
    gy, gy1, n_old, n_total = g["gy"], g["gy1"], g["n_old"], g["n_total"]
    if by < gy1:
        return by * n_old // gy1, (by + 1) * n_old // gy1
    return (n_old + (by - gy1) * (n_total - n_old) // (gy - gy1),
            n_old + (by + 1 - gy1) * (n_total - n_old) // (gy - gy1))


def blocks(g, nz):
    """(bx, by, zh) of every live workgroup; nz route parts on a 1-D grid with
    the parts of a tile 8 ids apart (bwd_block)."""
    gx, gy = g["gx"], g["gy"]
    if nz == 1:
        return [(bx, by, 0) for by in range(gy) for bx in range(gx)]
    out = []
    for L in range(8 * nz * cdiv(gx * gy, 8)):
        t = (L // (8 * nz)) * 8 + (L & 7)
        if t >= gx * gy:
            continue
        out.append((t % gx, t // gx, (L >> 3) % nz))
    return out


# ---------------------------------------------------------------------------
# LDS layouts

def acol(r, col, KP):
    if KP == 16:
        sw = (r >> 3) & 3
    else:
        sw = ((r >> 1) & 1) | (((r >> 3) & 3) << 1)
    return (col & 3) | (((col >> 2) ^ sw) << 2)


def tr_read(group_slots, slot_tokens):
    """ds_read_b64_tr_b16 of one 16-lane group: lane i gets element i % 4 of the
    slots read by lanes i // 4 + {0, 4, 8, 12}; returns per lane the 4 (slot,
    element) pairs."""
    return [[(group_slots[i // 4 + 4 * e], i % 4) for e in range(4)] for i in range(16)]


def check_trtile_nc2(NB=2):
    """bwd_tile's TrTile<NB, 2>: slots cover [0, kSlots) once, and the transposed
    read of (rb, cg) returns m[token 16 rb + i][channel 16 cg + 4 qq + e]."""
    GB = 4 * NB
    kslots = 2 * GB * 16
    owner = {}
    for j, q, b, c in itertools.product(range(16), range(4), range(NB), range(2)):
        g = NB * q + b
        sl = (c * GB + g) * 16 + (j ^ (2 * c + 4 * (g & 3)))
        assert 0 <= sl < kslots
        assert sl not in owner
        owner[sl] = (2 * j + c, g)  # (channel, token group)
    assert len(owner) == kslots
    for rb, cg, qq in itertools.product(range(NB), range(2), range(4)):
        slots = []
        for i in range(16):
            e, a = i >> 2, i & 3
            c = e & 1
            sl = (c * GB + a) * 16 + ((8 * cg + 2 * qq + (e >> 1)) ^ (2 * c + 4 * a)) + 64 * rb
            assert 0 <= sl < kslots
            slots.append(sl)
        for i, parts in enumerate(tr_read(slots, None)):
            for e, (sl, el) in enumerate(parts):
                ch, g = owner[sl]
                assert ch == 16 * cg + 4 * qq + e and 4 * g + el == 16 * rb + i


def check_trtile_nc1():
    """bwd_lean_tile's TrTile1: one channel per lane."""
    owner = {}
    for j, q, b in itertools.product(range(16), range(4), range(2)):
        g = 2 * q + b
        sl = g * 16 + (j ^ (4 * (g & 3)))
        assert 0 <= sl < 128 and sl not in owner
        owner[sl] = (j, g)
    for rb, qq in itertools.product(range(2), range(4)):
        slots = []
        for i in range(16):
            e, a = i >> 2, i & 3
            g = 4 * rb + a
            slots.append(g * 16 + ((4 * qq + e) ^ (4 * a)))
        for i, parts in enumerate(tr_read(slots, None)):
            for e, (sl, el) in enumerate(parts):
                ch, g = owner[sl]
                assert ch == 4 * qq + e and 4 * g + el == 16 * rb + i


def test_transposed_m_tiles():
    check_trtile_nc2()
    check_trtile_nc1()


@pytest.mark.parametrize("S,KC,MODE,SPLIT", [
    (4, 1, "fused", False), (8, 2, "taps", False), (8, 4, "taps", True), (7, 4, "taps", True),
    (5, 2, "taps", False), (2, 2, "fused", True), (8, 4, "fused", True)])
def test_bwd_tile_lds_extents(S, KC, MODE, SPLIT):
    """bwd_tile (NB 2, NC 2): routing-weight rows and columns, the dalpha B
    operand rows, the dalpha tiles and the staging chunks stay inside their
    arrays for every lane, wave and tap."""
    NB, NC, R, TB = 2, 2, 8, 32
    KP = 16 * KC
    WPG = 8 if MODE == "taps" else 4
    KX = (2 if MODE == "taps" else 1) if SPLIT else KC
    ST = (S + 1) // 2 if MODE == "taps" else S
    AROWS = TB + S - 1
    zhs = range((KC // KX) if SPLIT else 1)
    for zh in zhs:
        kc0 = zh * KX
        for j, q in itertools.product(range(16), range(4)):
            # W operand rows (aop): row R (j/4) + 4 b + j % 4 + e, e < S
            if MODE != "taps":
                for b, e, kc in itertools.product(range(NB), range(S), range(KC)):
                    r = R * (j >> 2) + 4 * b + (j & 3) + e
                    assert r < AROWS and acol(r, 16 * kc + 4 * q, KP) + 4 <= KP
            # alpha^T operands (transposed rows of the own tokens)
            for b, kx in itertools.product(range(NB), range(KX)):
                r = R * q + 4 * b + (j >> 2)
                assert r < AROWS and acol(r, 16 * (kc0 + kx) + 4 * (j & 3), KP) + 4 <= KP
            # dalpha B operand rows (b_lds, rows (s, k)) and columns
            for s, kx, cg in itertools.product(range(ST), range(KX), range(NC)):
                assert s * 16 * KX + 16 * kx + j < 16 * KX * ST
                assert 16 * cg + 4 * q + 4 <= 16 * NC + 4
            # dalpha tile writes [NB][KX][16][17]
            for rb, kx, v in itertools.product(range(NB), range(KX), range(4)):
                assert 4 * q + v < 16 and j < 17
        # staging: chunk c of 4 elements, row c / (KP / 4)
        achunks = AROWS * KP // 4
        aper = cdiv(achunks, 64 * WPG)
        for tid, i in itertools.product(range(64 * WPG), range(aper)):
            ch = tid + i * 64 * WPG
            if ch < achunks:
                row, col = ch // (KP // 4), (ch % (KP // 4)) * 4
                assert row < AROWS and acol(row, col, KP) + 4 <= KP
    # the dalpha sum: every (rb, kx, row, col) once per super-block
    nsum = NB * KX * 256 // (64 * WPG)
    seen = set()
    for tid, i in itertools.product(range(64 * WPG), range(nsum)):
        idx = tid + i * 64 * WPG
        seen.add((idx // (KX * 256), (idx // 256) % KX, (idx >> 4) & 15, idx & 15))
    assert len(seen) == NB * KX * 256


def test_lean_lds_extents():
    """bwd_lean_tile: the two row-shifted copies of the routing weights (W
    operand reads at shift e < 4 stay within an 8-row group, so the swizzle of
    the row equals that of the lane's base row), transposed alpha reads, m tile
    and dalpha tiles."""
    R, TB, KP = 8, 32, 16
    for S in (2, 3, 4):
        AROWS = TB + S - 1
        for j, q in itertools.product(range(16), range(4)):
            base = R * (j >> 2) + (j & 3)
            for b, e in itertools.product(range(2), range(S)):  # shifts e < S
                r = base + e
                assert r < AROWS - 4 * b  # rows of copy b that were staged
                assert (r >> 3) == (j >> 2)  # one swizzle over the shifts
                assert acol(r, 4 * q, KP) == ((q ^ (j >> 2)) << 2)
            for b in range(2):
                r = R * q + 4 * b + (j >> 2)
                assert r < AROWS
        for tid in range(512):
            if tid < AROWS * KP // 4:
                row = tid >> 2
                assert row < AROWS and (row < 4 or row - 4 < AROWS)


def coverage(N, D, S, KC, mode, SPLIT, n_cu=256):
    """Writes of part_da [gx][N][KP] and part_db [gy][KP][S][D] over the grid
    the launch uses; each entry stage 2 reads must be written exactly once."""
    KP = 16 * KC
    eown = bwd_eown(S, mode == "taps")
    if mode == "taps":
        nz = 2 if SPLIT else 1
        g = bwd_grid_gx(N, cdiv(D, 128), D, S, (n_cu // nz) * 1, taps=True)
        WCH, ST, KX = 4, (S + 1) // 2, (2 if SPLIT else KC)
    else:
        nz = KC if SPLIT else 1
        g = tiered(N, cdiv(D, 128), D, S, n_cu) if not SPLIT else bwd_grid_gx(N, cdiv(D, 128), D, S, 512)
        WCH, ST, KX = 4, S, (1 if SPLIT else KC)
    da, db = {}, {}
    for bx, by, zh in blocks(g, nz):
        kc0 = zh * KX
        lo, hi = sb_range(by, g)
        for sb in range(lo, hi):
            t0 = sb * eown
            if t0 >= N:
                break
            own = min(t0 + eown, N) - t0
            for row, kx, col in itertools.product(range(own), range(KX), range(16)):
                key = (bx, t0 + row, 16 * (kc0 + kx) + col)
                da[key] = da.get(key, 0) + 1
        for w in range(WCH * (2 if mode == "taps" else 1)):
            th = w // WCH if mode == "taps" else 0
            d0 = (bx * WCH + w % WCH) * 32
            if d0 >= D:
                continue
            for kx, s, j, q, v, c in itertools.product(range(KX), range(ST), range(16), range(4),
                                                       range(4), range(2)):
                tap = th * ST + s
                ch = d0 + 2 * (4 * q + v) + c
                if ch < D and tap < S:
                    key = (by, 16 * (kc0 + kx) + j, tap, ch)
                    db[key] = db.get(key, 0) + 1
    assert all(n == 1 for n in da.values()) and all(n == 1 for n in db.values())
    assert len(da) == g["gx"] * N * KP
    assert len(db) == g["gy"] * KP * S * D
    return g


@pytest.mark.parametrize("N,D,S,KC,mode,SPLIT,n_cu", [
    (120, 192, 8, 4, "taps", True, 256),     # the 8-tap 64-route prefill taps pass (T 40)
    (210, 192, 8, 4, "taps", True, 256),     # T 70
    (999, 192, 8, 4, "taps", True, 256),
    (2 * 4096, 192, 8, 4, "taps", True, 16),  # ranges of many super-blocks
    (300, 256, 8, 2, "taps", False, 256),
    (464, 256, 4, 1, "fused", False, 16),    # two-tier ranges (gy = 2 n_cu / gx)
    (999, 192, 4, 4, "fused", True, 256),
])
def test_partials_written_once(N, D, S, KC, mode, SPLIT, n_cu):
    g = coverage(N, D, S, KC, mode, SPLIT, n_cu)
    if mode == "fused" and not SPLIT and n_cu == 16:
        assert g["gy1"] * 2 == g["gy"] and g["n_old"] < g["n_total"]  # tiers in use


def test_lean_partials_written_once():
    """bwd_lean_tile on the fused pass's (two-tier) grid: 8 waves of 16 channels
    per 128-channel group, dalpha rows of the own tokens, dbasis (k, s, 4
    channels per lane)."""
    for N, D, S, n_cu in ((464, 256, 4, 16), (999, 196, 3, 256), (77, 64, 2, 256)):
        KP, eown = 16, 32 - (S - 1)
        g = tiered(N, cdiv(D, 128), D, S, n_cu)
        da, db = {}, {}
        for bx, by, _ in blocks(g, 1):
            lo, hi = sb_range(by, g)
            for sb in range(lo, hi):
                t0 = sb * eown
                if t0 >= N:
                    break
                own = min(t0 + eown, N) - t0
                for tl in range(512):
                    r2, row, c = tl >> 8, (tl >> 4) & 15, tl & 15
                    if 16 * r2 + row < own:
                        key = (bx, t0 + 16 * r2 + row, c)
                        da[key] = da.get(key, 0) + 1
            for wave, j, q, s, v in itertools.product(range(8), range(16), range(4), range(S),
                                                      range(4)):
                d0 = (bx * 8 + wave) * 16
                if d0 < D and d0 + 4 * q < D:
                    key = (by, j, s, d0 + 4 * q + v)
                    db[key] = db.get(key, 0) + 1
        assert all(n == 1 for n in da.values()) and len(da) == g["gx"] * N * KP
        assert all(n == 1 for n in db.values()) and len(db) == g["gy"] * KP * S * D


# ---------------------------------------------------------------------------
# grouped launches (csrc/moc_mfma_launch.h bwd_layers_one, csrc/moc_mfma.h
# layer_index / bwd_layers_kernel)

def layers_grid(layer_grids, nz):
    """blk0 of each layer and the launch's block count: a layer's grid is its
    gx gy tiles, or with nz route parts the 1-D split grid of 8 nz ids per 8
    tiles (the taps pass in route halves, the fused pass split in chunks)."""
    blk0, blk = [], 0
    for g in layer_grids:
        blk0.append(blk)
        tiles = g["gx"] * g["gy"]
        blk += 8 * nz * cdiv(tiles, 8) if nz > 1 else tiles
    return blk0, blk


def layers_blocks(layer_grids, nz):
    """(layer, bx, by, zh) of every live block id of the grouped launch, mapped
    as the kernel maps it: the owning layer is the last whose blk0 <= id; the
    local id is split into (bx, row) by the layer's gx (no route parts) or
    through bwd_block's split mapping."""
    blk0, blk = layers_grid(layer_grids, nz)
    out = []
    for b in range(blk):
        li = max(i for i in range(len(blk0)) if blk0[i] <= b)
        g = layer_grids[li]
        local = b - blk0[li]
        if nz == 1:
            out.append((li, local % g["gx"], local // g["gx"], 0))
            continue
        t = (local // (8 * nz)) * 8 + (local & 7)
        if t >= g["gx"] * g["gy"]:
            continue
        out.append((li, t % g["gx"], t // g["gx"], (local >> 3) % nz))
    return out


@pytest.mark.parametrize("dims,S,KC,mode,n_cu", [
    ([512, 256, 128], 6, 2, "dx", 256),      # SiLU two passes, 32 routes: dx pass
    ([512, 256, 128], 6, 2, "taps", 256),
    ([256, 128], 4, 4, "taps", 256),         # 64 routes: taps pass in route halves
    ([4096, 1024, 1024], 8, 2, "dx", 256),   # configs[4]
    ([256, 192], 8, 4, "fused", 256),        # fused pass split in route chunks
])
def test_grouped_grid_covers_each_layer_once(dims, S, KC, mode, n_cu):
    """Every block of a layer's single launch runs exactly once in the grouped
    launch, and no block id maps past a layer's tiles (a block with by >= gy
    would take a token range past the layer's last)."""
    N = 999
    if mode == "taps":
        nz = 2 if KC == 4 else 1
        grids = [bwd_grid_gx(N, cdiv(D, 128), D, S, n_cu // nz, taps=True) for D in dims]
    elif mode == "dx":
        nz = 1
        grids = [bwd_grid_gx(N, cdiv(D, 128), D, S, 512) for D in dims]
    else:
        nz = KC
        grids = [bwd_grid_gx(N, cdiv(D, 128), D, S, 512) for D in dims]
    got = layers_blocks(grids, nz)
    want = [(li,) + blk for li, g in enumerate(grids) for blk in blocks(g, nz)]
    assert sorted(got) == sorted(want)
    assert len(set(got)) == len(got)
    assert all(by < grids[li]["gy"] for li, _, by, _ in got)
