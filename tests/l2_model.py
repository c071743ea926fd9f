"""A model of the tile GEMM's operand traffic past the L2, for CPU checks of the tile
order against the measured FETCH_SIZE.

Test infrastructure. MI355X dispatches workgroups to its 8 XCDs in turn (workgroup b
to XCD b mod 8), and each XCD has its own 4 MiB L2. The model runs the launch round by
round (one workgroup per CU: `cus` concurrent tiles, `cus / 8` per XCD), with the
concurrent tiles of an XCD stepping through K together (128 bytes per step), and counts
the 128-byte lines that miss an LRU L2 of each XCD. The tile of workgroup b is the
kernel's `tile_of` (krea2-hrx_amd/csrc/k2w8_gemm_common.hpp), restated here.
"""

from __future__ import annotations

from collections import OrderedDict

XCDS = 8
L2_BYTES = 4 << 20
LINE = 128


def tile_of(bid: int, tiles_m: int, tiles_n: int, m_group: int):
    """gemm::tile_of: XCD-major renumbering, then m_group m-tiles per n sweep."""
    total = tiles_m * tiles_n
    per_xcd = total // XCDS
    if bid < per_xcd * XCDS:
        bid = (bid % XCDS) * per_xcd + bid // XCDS
    span = m_group * tiles_n
    group, in_group = divmod(bid, span)
    first_m = group * m_group
    rows = min(tiles_m - first_m, m_group)
    return first_m + in_group % rows, in_group // rows


def fetch_bytes(m, n, k, bm, bn, cus=256, m_group=4, order=tile_of, reverse_odd_rounds=False):
    """Bytes of A and W that miss the XCDs' L2s over one launch."""
    tiles_m, tiles_n = (m + bm - 1) // bm, n // bn
    total, steps = tiles_m * tiles_n, k // 128
    lines = L2_BYTES // LINE
    caches = [OrderedDict() for _ in range(XCDS)]
    misses = 0
    for r in range((total + cus - 1) // cus):
        per_xcd = [[] for _ in range(XCDS)]
        for b in range(r * cus, min(total, (r + 1) * cus)):
            per_xcd[b % XCDS].append(order(b, tiles_m, tiles_n, m_group))
        for x, tiles in enumerate(per_xcd):
            cache = caches[x]
            a_rows = [row for tm in sorted({t[0] for t in tiles}) for row in range(tm * bm, min(m, (tm + 1) * bm))]
            w_rows = [row for tn in sorted({t[1] for t in tiles}) for row in range(tn * bn, (tn + 1) * bn)]
            for s in range(steps):
                step = steps - 1 - s if (reverse_odd_rounds and r % 2) else s
                for key in [(0, row, step) for row in a_rows] + [(1, row, step) for row in w_rows]:
                    if key in cache:
                        cache.move_to_end(key)
                    else:
                        misses += 1
                        cache[key] = True
                        if len(cache) > lines:
                            cache.popitem(last=False)
    return misses * LINE
