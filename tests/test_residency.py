"""Host-side residency planning (crates/model/src/moe.rs:692-880) with the
reference's own popularity fixture, tests/golden/route_hist_30b.csv (copied
from the reference's tests/golden/, 48 layers x 128 experts).  No GPU."""
from __future__ import annotations

import csv
import ctypes as C
from pathlib import Path

import numpy as np

from styx_amd._lib import load

HIST = Path(__file__).resolve().parent / "golden" / "route_hist_30b.csv"
SKIP = 0xFFFFFFFF
SLAB_30B = 884736 + 1081344 + 1290240  # q4_K + q5_K + q6_K slabs of one (layer, expert)


def plan(hist, L, E, slab, budget_mb):
    remap = np.empty(L * E, np.uint32)
    n = C.c_uint64()
    slabs = np.full(L, slab, np.uint64)
    rc = load().styx_residency_plan(str(hist).encode() if hist else None, L, E, slabs.ctypes.data,
                                    budget_mb, remap.ctypes.data, C.byref(n))
    assert rc == 0
    return remap.reshape(L, E), n.value


def read_hits():
    rows = list(csv.reader(open(HIST)))[1:]
    hits = np.zeros((48, 128), np.int64)
    for l, e, h in rows:
        hits[int(l), int(e)] = int(h)
    return hits


def test_fixture_shape():
    hits = read_hits()
    assert hits.shape == (48, 128) and (hits >= 0).all() and hits.sum() > 0


def test_6gib_budget_pins_the_hottest_slabs():
    """config 3: a 6 GiB budget over 3,256,320-byte slabs holds
    floor(6 GiB / slab) = 1978 slabs (about 41 of 128 per layer)."""
    remap, n = plan(HIST, 48, 128, SLAB_30B, 6144)
    assert n == (6144 << 20) // SLAB_30B == 1978
    hot = remap != SKIP
    assert hot.sum() == n
    hits = read_hits()
    # every pinned slab is at least as popular as every unpinned one
    assert hits[hot].min() >= hits[~hot].max()
    # hot slots are dense per layer and ordered by expert id
    for l in range(48):
        ids = np.nonzero(hot[l])[0]
        assert np.array_equal(remap[l, ids], np.arange(len(ids)))


def test_budget_edges():
    remap, n = plan(HIST, 48, 128, SLAB_30B, 0)
    assert n == 0 and (remap == SKIP).all()
    remap, n = plan(HIST, 48, 128, SLAB_30B, 1 << 30)  # everything fits
    assert n == 48 * 128 and np.array_equal(remap, np.tile(np.arange(128), (48, 1)))


def test_without_histogram_whole_layers_in_order():
    layer = SLAB_30B * 128
    remap, n = plan(None, 48, 128, SLAB_30B, (3 * layer + layer // 2) >> 20)
    assert n == 3 * 128
    assert (remap[:3] != SKIP).all() and (remap[3:] == SKIP).all()


def test_zipf_bias_table_gives_zipf_popularity():
    """The configs[2] router bias (styx_zipf_bias_table): on an independent
    sample of router logit noise N(0, (0.02 sqrt(2048))^2), top-8 routing
    over 128 experts picks rank r with a frequency that falls as r^-1.1
    (least-squares exponent over the ranks picked on fewer than half the
    tokens), rank 1 on every token, and the 41 most popular experts (a
    6 GiB budget at the 30B shape) take 0.81 of the picks, the capped-Zipf
    value; biases fall with rank, and the table is deterministic."""
    E, k, s, sd = 128, 8, 1.1, 0.02 * 2048 ** 0.5
    t = np.empty(E, np.float32)
    assert load().styx_zipf_bias_table(E, k, C.c_float(s), C.c_float(sd), 77, t.ctypes.data) == 0
    t2 = np.empty(E, np.float32)
    load().styx_zipf_bias_table(E, k, C.c_float(s), C.c_float(sd), 77, t2.ctypes.data)
    assert np.array_equal(t, t2) and t[0] == 0 and (np.diff(t) <= 0).all()
    rng = np.random.default_rng(2024)
    n = 20000
    lg = t + (sd * rng.standard_normal((n, E))).astype(np.float32)
    top = np.argpartition(-lg, k, axis=1)[:, :k]
    freq = np.bincount(top.ravel(), minlength=E) / n
    r = np.arange(1, E + 1)
    m = freq < 0.5
    slope = np.polyfit(np.log(r[m]), np.log(freq[m]), 1)[0]
    assert abs(slope + 1.1) < 0.1, slope
    assert freq[0] > 0.98
    assert abs(freq[:41].sum() / k - 0.812) < 0.02


def test_hud_lines_match_reference_format():
    """generate_moe.rs:87-119: totals, shares, cold PCIe bytes, the
    per-layer heatmap (. = no cold slot, digit = tenths of k slots cold,
    capped at 9) and the repin line."""
    from styx_amd import Hud
    slab = 3256320
    h = Hud(4, 8, slab)
    h.tick(np.array([[8, 0], [4, 4], [0, 8], [7, 1]]))
    h.tick(np.array([[8, 0], [6, 2], [0, 8], [8, 0]]))
    lines = h.lines(2, repin_swaps=3)
    # hot 8+4+0+7 + 8+6+0+8 = 41, cold 0+4+8+1 + 0+2+8+0 = 23 of 64 slots;
    # 23 cold slabs of 3256320 B = 0.07 GiB, 35.7 MiB per token
    assert lines[0] == ("hud: hot 64.1% (41) | cold 35.9% (23) | cold PCIe ~0.07 GiB total, "
                        "~35.7 MiB/tok")
    # layer cold shares over 2 tokens x 8 slots: 0, 6/16, 16/16, 1/16
    assert lines[1] == "hud: cold/layer [.390] (.=0%, 9=90%+ of k=8 slots)"
    assert lines[2] == f"hud: repin 3 slab swaps (~{3 * slab / 2**30:.2f} GiB copied)"
    assert len(Hud(48, 8, slab).lines(1)) == 2  # no repin line without swaps
