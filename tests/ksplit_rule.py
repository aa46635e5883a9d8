"""Restatement of the K-split choice, for tests that need to know which
matrices of a call split: pan2_amd/csrc/pm_tiles.hpp::k_split (the rule;
tests/native/tile_order_check.cpp pins the C++ itself) applied per call as
pan2_amd/csrc/panmuon.hip::split_call does. A stage splits only when the
call's engine matrices (short side > 128) together hold at most 128 of its
tiles (two chunks) or 64 (four), and each matrix as far as its shape allows.
(A matrix whose partials would take its workspace past the 256 MiB scratch of
the allocation-free step also stays unsplit; no shape the tests give this
restatement comes near that.)
"""


def up(x, m=256):
    return (x + m - 1) // m * m


def k_split(mp, tiles, kt):
    if mp < 512 or tiles <= 0 or kt % 4:
        return 1
    s = 1
    while 2 * s <= 4 and (kt // 4) % (2 * s) == 0 and kt // (2 * s) >= 16 and tiles * 2 * s <= 256:
        s *= 2
    return s


def stage_tiles(shape):
    """(GRAM, symmetric products, UPDATE / FINAL) tiles of an engine matrix, and its Mp, Np."""
    mp, np_ = up(min(shape)), up(max(shape))
    nt = mp // 256
    tri = nt * (nt + 1) // 2
    return (tri, tri, nt * (np_ // 256)), mp, np_


def call_splits(shapes):
    """Chunks per tile of (GRAM, the symmetric products, UPDATE / FINAL) for
    every matrix of one call; (1, 1, 1) for small matrices."""
    engine = [s for s in shapes if min(s) > 128]
    total = [sum(stage_tiles(s)[0][st] for s in engine) for st in range(3)]
    out = []
    for s in shapes:
        if min(s) <= 128:
            out.append((1, 1, 1))
            continue
        _, mp, np_ = stage_tiles(s)
        out.append((k_split(mp, total[0], np_ // 64), k_split(mp, total[1], mp // 64), k_split(mp, total[2], mp // 64)))
    return out
