"""CPU checks of the stream-K work split and combine protocol (csrc/mi_streamk.hpp).

* The split: a small C++ program compiled here with g++ from the header
  itself prints, for many (tiles, K tiles, grid) cases, each workgroup's
  first unit and each tile's owner and early-part count.  They are checked
  against a brute-force walk over the units: the ranges tile the units
  exactly, no range is empty, first_wg holds the tile's K tile 0, the
  later parts are the workgroups whose ranges start strictly inside the
  tile, the kernel's reverse walk runs a tile's head first and a tail last,
  and the whole grid reads K on at most two fronts.
* The protocol: every interleaving of the parts' counter updates (the
  checker and up to three storers) is run on a model of the atomic counter with
  the header's constants.  In each, exactly one part combines, and every
  partial sum it reads from the workspace was stored before the counter
  update that it read, and the counter ends at zero for the next launch.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "nki-autotune_amd", "csrc", "mi_streamk.hpp")

CASES = [(224, 128, 256), (224, 64, 256), (224, 128, 224), (1, 128, 128), (4, 64, 256), (7, 3, 5), (13, 17, 11),
         (128, 128, 256), (3, 1000, 256), (224, 100, 256), (60, 64, 49), (100, 1, 64), (21, 8, 168), (5, 7, 35), (2, 50, 37)]


def _constants() -> dict:
    text = open(HEADER).read()
    out = {}
    for name in ("kSkLastArrived", "kSkLastReady", "kSkCounterBytes"):
        m = re.search(rf"constexpr int {name} = ([^;]+);", text)
        out[name] = int(eval(m.group(1).replace("kSkLastArrived", str(out.get("kSkLastArrived", 0)))))  # noqa: S307
    out["kSkStoredMask"] = out["kSkLastArrived"] - 1
    return out


@pytest.fixture(scope="module")
def plan_tool(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    d = tmp_path_factory.mktemp("sk")
    src = d / "plan.cpp"
    src.write_text(
        '#define MI_HD\n#include "' + HEADER + '"\n#include <cstdio>\n#include <cstdlib>\n'
        "int main(int argc, char** argv) {\n"
        "  long long T = atoll(argv[1]), KT = atoll(argv[2]), G = atoll(argv[3]);\n"
        "  mi::StreamKPlan p(T, KT, G);\n"
        "  for (long long w = 0; w <= G; ++w) printf(\"b %lld %lld\\n\", w, p.begin(w));\n"
        "  for (long long t = 0; t < T; ++t) printf(\"t %lld %lld %lld\\n\", t, p.first_wg(t), p.later_parts(t));\n"
        "  printf(\"g %lld\\n\", mi::streamk_grid(256, T, KT));\n"
        "  return 0;\n}\n")
    exe = d / "plan"
    subprocess.run([gxx, "-std=c++17", "-O1", "-o", str(exe), str(src)], check=True)
    return str(exe)


def _run(tool, T, KT, G):
    out = subprocess.run([tool, str(T), str(KT), str(G)], check=True, capture_output=True, text=True).stdout
    begin, tiles, grid = {}, {}, None
    for line in out.splitlines():
        f = line.split()
        if f[0] == "b":
            begin[int(f[1])] = int(f[2])
        elif f[0] == "t":
            tiles[int(f[1])] = (int(f[2]), int(f[3]))
        else:
            grid = int(f[1])
    return begin, tiles, grid


@pytest.mark.parametrize("T,KT,G", CASES)
def test_split_covers_every_unit_once(plan_tool, T, KT, G):
    begin, tiles, grid = _run(plan_tool, T, KT, G)
    total = T * KT
    assert grid == min(256, total)
    assert begin[0] == 0 and begin[G] == total
    owner_of = {}
    for w in range(G):
        assert begin[w] < begin[w + 1], (w, "empty range")          # grid <= total
        for u in range(begin[w], begin[w + 1]):
            owner_of[u] = w
    assert sorted(owner_of) == list(range(total))
    for t in range(T):
        ow, ne = tiles[t]
        assert owner_of[t * KT] == ow
        starts_inside = [w for w in range(G) if t * KT < begin[w] < (t + 1) * KT]
        assert starts_inside == list(range(ow + 1, ow + 1 + ne)), (t, starts_inside, ow, ne)
        parts = sorted({owner_of[u] for u in range(t * KT, (t + 1) * KT)})
        assert parts == [ow] + starts_inside
    # The kernel's segment walk, in reverse unit order: the head of the last
    # tile first (K from 0), then whole tiles, then the tail of the first tile
    # (the part holding K tile KT-1 that does not start the tile: a checker).
    fronts = set()
    for w in range(G):
        u, start, segs = begin[w + 1], begin[w], []
        while u > start:
            t = (u - 1) // KT
            kb = max(t * KT, start) - t * KT
            segs.append((t, kb, u - t * KT))
            u = t * KT + kb
        assert sum(ke - kb for _, kb, ke in segs) == begin[w + 1] - begin[w]
        for i, (t, kb, ke) in enumerate(segs):
            if kb > 0:
                assert i == len(segs) - 1, (w, segs)     # a part not starting its tile runs last
            if ke < KT:
                assert i == 0, (w, segs)                 # a part ending before the tile's end runs first
        tau = 0
        for t, kb, ke in segs:
            for kt in range(kb, ke):
                fronts.add(kt - tau)
                tau += 1
    share = total // G
    if KT <= 2 * share <= 2 * KT:
        # Shares of half a tile to one tile (every range holds a tile's start
        # or its end): every workgroup reads K tile tau or tau + (KT - share)
        # at time tau (shares differ by one unit when G does not divide T*KT).
        assert fronts <= {0, KT - share, KT - share - 1}, (fronts, share)


def _interleavings(seqs):
    """Every merge of the per-part operation sequences (order within a part kept)."""
    if all(not s for s in seqs):
        yield []
        return
    for i, s in enumerate(seqs):
        if s:
            rest = list(seqs)
            rest[i] = s[1:]
            for tail in _interleavings(rest):
                yield [(i, s[0])] + tail


def _simulate(order, n, c):
    """Run one interleaving: part 0 is the checker ("arrive", "store", "ready"), parts 1..n the storers
    ("store", "add").  ``published`` holds the slots whose part stored them and then updated the counter; a
    combiner may read only those (and its registers).  The combiner resets the counter."""
    ctr, stored, published, combiners, checker = 0, set(), set(), [], "arrive"
    mask = c["kSkStoredMask"]
    for part, op in order:
        if part == 0:
            if op == "arrive":
                old, ctr = ctr, ctr + c["kSkLastArrived"]
                if (old & mask) == n:
                    combiners.append((0, set(published)))
                    ctr, checker = 0, "done"
                else:
                    checker = "store"
            elif checker != "store":
                continue                       # combined at arrival: no store, no second update
            elif op == "store":
                stored.add("c")
            else:
                assert "c" in stored
                published.add("c")
                old, ctr = ctr, ctr + c["kSkLastReady"]
                if (old & mask) == n:
                    combiners.append((0, set(published)))
                    ctr = 0
        elif op == "store":
            stored.add(part)
        else:
            assert part in stored
            published.add(part)
            old, ctr = ctr, ctr + 1
            if (old & c["kSkLastReady"]) and (old & mask) == n - 1:
                combiners.append((part, set(published)))
                ctr = 0
    return combiners, ctr


@pytest.mark.parametrize("n", [1, 2, 3])
def test_exactly_one_part_combines_in_every_order(n):
    c = _constants()
    assert c["kSkLastReady"] > c["kSkLastArrived"] > n
    seqs = [["arrive", "store", "ready"]] + [["store", "add"] for _ in range(n)]
    count = 0
    for order in _interleavings(seqs):
        combiners, ctr = _simulate(order, n, c)
        assert len(combiners) == 1, (order, combiners)
        who, published = combiners[0]
        reads = set(range(1, n + 1)) | ({"c"} if who != 0 else set())
        assert reads <= published, (order, who, published)
        assert ctr == 0, (order, ctr)          # nothing touches the counter after the reset
        count += 1
    expected = 1
    for k in range(1, 3 + 2 * n + 1):
        expected *= k
    assert count == expected // (6 * 2 ** n)


def test_counter_region_holds_every_tile():
    c = _constants()
    assert c["kSkCounterBytes"] % 256 == 0 and c["kSkCounterBytes"] // 4 >= 4096
