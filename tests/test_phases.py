"""CPU checks of the phase-timeline summary (transfer_station_amd/phases.py): the restated item
mapping of the persistent prefill and the arithmetic of the phase split, on synthetic stamps."""
import collections

import numpy as np

from transfer_station_amd import phases


def test_item_mapping_covers_every_item_once():
    # non-causal: Hq heads x nqt tiles, every (head, tile) exactly once over the workgroups
    for Hq, Hkv, nqt, nwg in ((128, 32, 4, 256), (131, 131, 4, 256), (64, 16, 8, 256)):
        got = collections.Counter()
        for b in range(nwg):
            got.update(phases.items_of(b, nwg, Hq * nqt, Hq // Hkv, nqt, False))
        assert got == collections.Counter({qt: Hq for qt in range(nqt)})
    # causal pairs: items alternate a heavy and a light tile whose key tiles add up the same
    Hq, Hkv, nqt, nwg = 128, 32, 16, 256
    got = collections.Counter()
    for b in range(nwg):
        qts = phases.items_of(b, nwg, Hq * nqt // 2, Hq // Hkv, nqt, True)
        assert all(qts[k] + qts[k + 1] == nqt - 1 for k in range(0, len(qts), 2))
        got.update(qts)
    assert got == collections.Counter({qt: Hq for qt in range(nqt)})


def test_summary_of_synthetic_stamps():
    # 16 workgroups (R = 2 per XCD), 8 heads x 4 tiles of 256 rows, 8 key tiles per item: two
    # items per workgroup. Model: entry at 10 ticks per workgroup index, a 4 us prologue, 3 us per
    # steady tile, first and last tiles 1 and 2 us longer, a 5 us tail.
    Hq, Hkv, Sq, Sk, nwg, slots = 8, 2, 1024, 1024, 16, 64
    st = np.zeros((nwg, slots), np.uint64)
    tick = lambda us: int(round(us / phases.TICK_US))
    for b in range(nwg):
        t = 1000 + 10 * b
        st[b, 0] = t
        t += tick(4)
        st[b, 1] = t
        for k in range(2):
            st[b, 2 + 4 * k] = t
            t += tick(3 + 1)
            st[b, 3 + 4 * k] = t
            t += tick(3 * 6)
            st[b, 4 + 4 * k] = t
            t += tick(3 + 2)
            st[b, 5 + 4 * k] = t
        st[b, slots - 1] = t + tick(5)
    s = phases.summarize(st, slots, Hq, Hkv, Sq, Sk, 0)
    assert s["workgroups"] == nwg
    assert abs(s["entry_spread_us"] - 1.5) < 1e-9
    assert s["prologue_us"]["median"] == 4.0 and s["key_tile_us"]["median"] == 3.0
    assert s["first_tile_extra_us"]["median"] == 1.0 and s["last_tile_extra_us"]["median"] == 2.0
    assert s["between_items_us"]["max"] == 0.0 and s["tail_us"]["median"] == 5.0
    assert abs(s["span_us"] - (1.5 + 4 + 2 * 27 + 5)) < 1e-9
    assert [it["item"] for it in s["items"]] == [0, 1]
    assert all(it["key_tiles"] == 8 and it["first_tile_extra_us"]["median"] == 1.0 and
               it["last_tile_extra_us"]["median"] == 2.0 for it in s["items"])


def test_key_halves_pairs_run_the_even_count_first():
    # The key-halves variant runs one pair of 128-row tiles per workgroup, the tile of even
    # key-tile count first, so that its LDS buffer order is fixed at compile time: with whole
    # tiles (Sq % 128 == 0) every pair holds one tile of even and one of odd count.
    for Hq, Hkv, Sq, Sk in ((16, 8, 4096, 4096), (32, 8, 2048, 2048), (64, 16, 1024, 1536),
                            (64, 8, 1024, 1100), (128, 1, 512, 512)):
        nqt, nwg = Sq // 128, 256
        units = Hq * nqt // 2
        assert units == nwg

        def swap(qt):
            return phases.key_tiles(qt, Sq, Sk, True, 128) % 2 == 1

        got = collections.Counter()
        for b in range(nwg):
            qts = phases.items_of(b, nwg, units, Hq // Hkv, nqt, True, swap)
            assert len(qts) == 2 and qts[0] + qts[1] == nqt - 1
            n0, n1 = (phases.key_tiles(q, Sq, Sk, True, 128) for q in qts)
            assert n0 % 2 == 0 and n1 % 2 == 1, (Hq, Sq, Sk, qts)
            got.update(qts)
        assert got == collections.Counter({qt: Hq for qt in range(nqt)})
