"""The per-world statistics and body checksums that the full-size parity
tests take after every vector step (tests/b3test.py stats_of_block and
body_hash in numpy, oracle/stats.c in C for the oracle's side,
stats_of_device_block and device_body_hash in torch for the device's):
closed forms for single bodies, agreement of the three implementations on
stepped scene worlds, and the checksum's response to one changed word."""
import math

import numpy as np
import pytest

from b3test import (body_block, body_hash, clone, device_body_hash, oracle_run, oracle_stats, stats_of_block,
                    stats_of_device_block)
from puffysics_amd import scenes


def _one_body(scene=2):
    """A stacks world with only body 1 dynamic: every other body static."""
    w = clone(scenes.build(scene, 1))
    b = w["bodies"]
    b["type"][0, :] = 0
    b["type"][0, 1] = 2
    return w


def test_closed_forms():
    w = _one_body()
    b = w["bodies"]
    b["inv_mass"][0, 1] = 0.5                          # m = 2
    b["center"]["y"][0, 1] = 3.0
    for a in "xyz":
        b["lin_vel"][a][0, 1] = 0.0
        b["ang_vel"][a][0, 1] = 0.0
    b["rotation"]["v"]["x"][0, 1] = 0.0
    b["rotation"]["v"]["y"][0, 1] = 0.0
    b["rotation"]["v"]["z"][0, 1] = 0.0
    b["rotation"]["s"][0, 1] = 1.0
    h, e = stats_of_block(body_block(w))
    assert h[0] == 3.0 and math.isclose(e[0], 2 * 9.81 * 3.0)
    b["lin_vel"]["x"][0, 1] = 3.0
    b["lin_vel"]["z"][0, 1] = -4.0                     # |v|^2 = 25
    b["inv_inertia"]["x"][0, 1] = 0.25                 # I_x = 4
    b["ang_vel"]["x"][0, 1] = 2.0                      # 0.5 * 4 * 4
    h, e = stats_of_block(body_block(w))
    assert math.isclose(e[0], 0.5 * 2 * 25 + 8.0 + 2 * 9.81 * 3.0)
    # a body turned 90 degrees about z: world x rate is body -y rate
    s = math.sqrt(0.5)
    b["rotation"]["v"]["z"][0, 1] = s
    b["rotation"]["s"][0, 1] = s
    b["inv_inertia"]["x"][0, 1] = 1.0
    b["inv_inertia"]["y"][0, 1] = 0.125                # I_y = 8
    h2, e2 = stats_of_block(body_block(w))
    assert math.isclose(e2[0], 0.5 * 2 * 25 + 0.5 * 8 * 4 + 2 * 9.81 * 3.0, rel_tol=1e-6)
    o = oracle_stats(w)
    assert math.isclose(o[0][0], h2[0]) and math.isclose(o[1][0], e2[0], rel_tol=1e-12)


@pytest.mark.parametrize("scene", [1, 2, 3, 4, 5])
def test_three_implementations_agree(scene):
    torch = pytest.importorskip("torch")
    worlds = scenes.build(scene, 96)
    oracle_run(scene, worlds, clone(worlds), 0, 25, threads=4)
    worlds["bodies"]["lin_vel"]["y"][5, 0] = np.float32("nan")
    blk = body_block(worlds)
    h, e = stats_of_block(blk)
    o = oracle_stats(worlds)
    d = stats_of_device_block(torch.from_numpy(blk.view(np.int32).copy())).numpy()
    for got in (o[:2], d):
        for k, ref in enumerate((h, e)):
            ok = np.isclose(got[k], ref, rtol=1e-12, atol=1e-12) | (np.isnan(got[k]) & np.isnan(ref))
            assert ok.all()
    hh = body_hash(blk)
    assert np.array_equal(o[2], hh)
    assert np.array_equal(device_body_hash(torch.from_numpy(blk.view(np.int32).copy())).numpy(), hh)


def test_checksum_sees_one_word_and_not_nan_bits():
    worlds = scenes.build(5, 8)
    base = oracle_stats(worlds)[2]
    w2 = clone(worlds)
    w2["bodies"]["position"]["x"][3, 16] = np.nextafter(w2["bodies"]["position"]["x"][3, 16], np.float32(9))
    c = oracle_stats(w2)[2]
    assert c[3] != base[3] and np.array_equal(np.delete(c, 3), np.delete(base, 3))
    w3, w4 = clone(worlds), clone(worlds)
    blk3, blk4 = body_block(w3), body_block(w4)
    blk3[2, 4, 13] = 0x7FC00000                        # two NaNs with other bits
    blk4[2, 4, 13] = 0xFFC00001
    assert np.array_equal(oracle_stats(w3)[2], oracle_stats(w4)[2])
    assert np.array_equal(body_hash(blk3), body_hash(blk4))
