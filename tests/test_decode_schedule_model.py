"""Host-side model of the packed decode kernel's tile pipeline (CPU only).

``decode_packed_kernel`` (fade_amd/csrc/decode_packed.h) streams tiles into NS
LDS ring stages per wave with direct-to-LDS loads that the compiler does not
track, and waits for them with its own ``s_waitcnt vmcnt(c)``: c is the number
of loads issued after the ones the next stage read needs.  The counts are
right only if every path through the prologue, the tile claims, the mid-tile
refill of a stage's K part and the split ends issues exactly what the waits
assume.  This model replays that control flow -- the same tile bounds, claim
order, issue split (K part after the tile's K reads, the rest after its V
reads) and wait arguments -- with adversarial completion: a wait retires only
the oldest loads, down to c outstanding.  It checks, over many tile mixes,
formats, wave counts and claim interleavings:

- every read of a stage finds all loads of its tile and region retired;
- every load into a region is issued after the reads of the tile it replaces;
- every wait count is one of the immediates the kernel can encode (any other
  value would fall through to its last branch);
- the tiles of a split are each taken by exactly one wave;
- no load is in flight when a wave leaves the loop (the wave merge reuses
  ring 0 right after).
"""

import random
from dataclasses import dataclass

import pytest

# (K-part loads, V-part loads incl. metadata) per packed tile and per fp16
# tile, for the kernel's format instances: Stage<KB, VB, FMT>::kOps = KB + VB
# + (ASYM ? 8 : 1), kOpsF16 = SYM ? 9 : 8; the K part of a packed tile is 4
# (4-bit) or 2 (2-bit) 1 KB loads, of an fp16 tile 4 row loads.
FORMATS = {
    "sym44": dict(KB=4, VB=4, meta=1, sym=True),
    "sym22": dict(KB=2, VB=2, meta=1, sym=True),
    "lit48": dict(KB=4, VB=8, meta=1, sym=False),
    "asym44": dict(KB=4, VB=4, meta=8, sym=False),
    "asym42": dict(KB=4, VB=2, meta=8, sym=False),
    "asym22": dict(KB=2, VB=2, meta=8, sym=False),
    "asym24": dict(KB=2, VB=4, meta=8, sym=False),
}


@dataclass
class Fmt:
    k_packed: int
    v_packed: int
    k_f16: int
    v_f16: int

    @property
    def A(self):
        return self.k_packed + self.v_packed

    @property
    def F(self):
        return self.k_f16 + self.v_f16


def fmt_ops(name: str) -> Fmt:
    f = FORMATS[name]
    k_loads = 4 if f["KB"] == 4 else 2
    v_loads = {8: 8, 4: 4, 2: 2}[f["VB"]]
    return Fmt(k_loads, v_loads + f["meta"], 4, 4 + (1 if f["sym"] else 0))


class Wave:
    """One wave's outstanding loads (oldest first), as (tile, stage, part)."""

    def __init__(self):
        self.q = []
        self.loaded = {}  # (stage, part) -> tile whose loads into it were issued last

    def issue(self, tile, stage, part, n):
        self.q.extend([(tile, stage, part)] * n)
        self.loaded[(stage, part)] = tile

    def wait(self, c, fmt: Fmt, ns: int = 2):
        allowed = {i * fmt.A + j * fmt.F for i in range(ns + 1) for j in range(ns + 1 - i)}
        assert c in allowed, f"wait count {c} has no immediate (kernel falls through to vmcnt(0))"
        assert c <= 63, "more loads in flight than vmcnt counts"
        while len(self.q) > c:  # adversarial: retire only the oldest
            self.q.pop(0)

    def read(self, tile, stage, part):
        assert self.loaded.get((stage, part)) == tile, f"stage {stage} {part} holds another tile than {tile}"
        pending = [x for x in self.q if x[1] == stage and x[2] == part]
        assert not pending, f"read of tile {tile} stage {stage} {part} with loads in flight: {pending[:2]}"


def run_workgroup(fmt: Fmt, NW: int, t0: int, t1: int, nFt: int, det: bool, rng: random.Random, q_loads=2,
                  NS: int = 2):
    """Replays one workgroup (NS ring stages per wave); returns the tiles each wave processed."""
    claim = [0]
    taken = [[] for _ in range(NW)]

    def ops(t):
        return 0 if t >= t1 else (fmt.F if t < nFt else fmt.A)

    def parts(t):
        return (fmt.k_f16, fmt.v_f16) if t < nFt else (fmt.k_packed, fmt.v_packed)

    def wave_prog(w):
        wv = Wave()
        wv.q.extend([("query", -1, "q")] * q_loads)  # query row (+ K scales, + R rows) ahead of the tiles
        ta, tb = t0 + w, t0 + NW + w

        def issue(t, st, k, v):
            kp, vp = parts(t)
            if k:
                wv.issue(t, st, "K", kp)
            if v:
                wv.issue(t, st, "V", vp)

        tq = [t0 + s * NW + w for s in range(NS)]  # the ring, oldest first from stage 0
        for s in range(NS):
            if tq[s] < t1:
                issue(tq[s], s, True, True)
        wv.wait(sum(ops(t) for t in tq), fmt, NS)
        assert not [x for x in wv.q if x[0] == "query"], "query loads still in flight after the prologue wait"

        def step(s):
            cur = tq[s]
            if cur >= t1:
                return False
            if det:
                nt = cur + NS * NW
            else:
                yield "claim"  # the only point where other waves can interleave meaningfully
                nt = t0 + NS * NW + claim[0]
                claim[0] += 1
            wv.wait(sum(ops(tq[(s + j) % NS]) for j in range(1, NS)), fmt, NS)
            wv.read(cur, s, "K")
            if nt < t1:
                issue(nt, s, True, False)  # refill_k: after the K reads (lgkmcnt(0))
            wv.read(cur, s, "V")
            taken[w].append(cur)
            if nt < t1:
                issue(nt, s, False, True)
            tq[s] = nt
            return True

        more = True
        while more:
            for s in range(NS):
                if more:
                    more = yield from step(s)
        assert not wv.q, f"wave {w} leaves the loop with loads in flight: {wv.q[:2]}"

    progs = [wave_prog(w) for w in range(NW)]
    live = list(range(NW))
    while live:
        w = rng.choice(live)
        try:
            next(progs[w])
        except StopIteration:
            live.remove(w)
    return taken


def split_bounds(split, tps, nT, nFt, rot):
    t0 = split * tps if not rot else (0 if split == 0 else nFt + (split - 1) * tps)
    t1 = nFt if (rot and split == 0) else min(t0 + tps, nT)
    return t0, t1


@pytest.mark.parametrize("NS", [2, 3, 4])
@pytest.mark.parametrize("fmt_name", sorted(FORMATS))
def test_schedule_model(fmt_name, NS):
    fmt = fmt_ops(fmt_name)
    if NS * max(fmt.A, fmt.F) > 63:
        pytest.skip("more loads in flight than vmcnt counts: the kernel does not build this stage count")
    rng = random.Random((hash(fmt_name) & 0xFFFF) + NS)
    for trial in range(300):
        NW = rng.choice([4, 6, 8])
        nFt = rng.randrange(0, 7)
        nMt = rng.randrange(1 if nFt == 0 else 0, 40)
        nT = nFt + nMt
        rot = fmt_name in ("sym44", "sym22") and nMt > 0 and rng.random() < 0.3
        det = rng.random() < 0.3
        if rot:
            ms = rng.randrange(1, nMt + 1)
            tps = -(-nMt // ms)
            n = 1 + -(-nMt // tps)
        else:
            want = rng.randrange(1, nT + 1)
            tps = -(-nT // want)
            n = -(-nT // tps)
        # per-row lengths: this row may have fewer tiles than the plan's capacity
        row_nT = nT if rng.random() < 0.7 else rng.randrange(0, nT + 1)
        row_nFt = min(nFt, row_nT)
        seen = []
        for split in range(n):
            t0, t1 = split_bounds(split, tps, row_nT, row_nFt if rot else nFt, rot)
            if not rot:
                t1 = min(t1, row_nT)
            taken = run_workgroup(fmt, NW, t0, t1, row_nFt if rot else nFt, det, rng,
                                  q_loads=2 + (8 if rot and split > 0 else 0), NS=NS)
            flat = sorted(t for ts in taken for t in ts)
            assert flat == list(range(t0, max(t0, t1))), (fmt_name, trial, split, flat, t0, t1)
            seen += flat
        assert sorted(seen) == list(range(row_nT)), (fmt_name, trial, sorted(seen), row_nT)


def test_model_catches_a_short_wait():
    """Planted mistakes: a wait that counts a packed tile's loads behind the stage
    while an fp16 tile (fewer loads) is in flight, and a count with no immediate."""
    fmt = fmt_ops("asym44")  # A = 16 loads per packed tile, F = 8 per fp16 tile
    wv = Wave()
    wv.issue(0, 0, "K", fmt.k_packed)
    wv.issue(0, 0, "V", fmt.v_packed)
    wv.issue(1, 1, "K", fmt.k_f16)
    wv.issue(1, 1, "V", fmt.v_f16)
    wv.wait(fmt.A, fmt)  # should be wait(F)
    with pytest.raises(AssertionError):
        wv.read(0, 0, "V")
    with pytest.raises(AssertionError):
        Wave().wait(fmt.A + 1, fmt)
