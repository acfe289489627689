"""The engine's per-lane step code, built for the host, against the oracle.

The lane code (puffysics_amd/csrc/b3d_lane.h, b3d_inputs.h) is what the
gfx950 step kernel runs per world.  Compiled with g++ -ffp-contract=off and
the same libm, it must reproduce the oracle bit for bit: this pins the
word-transposed tile layout, the restore ranges, the merge-pointer warm
start and every index the kernels compute, without a GPU.
"""
import numpy as np
import pytest

from b3test import EmuBatch, clone, diff_words, oracle_run
from puffysics_amd import scenes

CASES = [(1, 70, 40), (2, 70, 65), (3, 70, 25), (4, 66, 12), (5, 130, 40)]


@pytest.mark.parametrize("scene,count,steps", CASES)
def test_lane_code_matches_oracle(scene, count, steps):
    worlds = scenes.build(scene, count)
    initial = clone(worlds)
    emu = EmuBatch(scene, worlds)
    ref = clone(worlds)
    oracle_run(scene, ref, initial, 0, steps)
    emu.run(0, steps)
    got = emu.worlds()
    bad = diff_words(got, ref, scenes.SCENES[scene].sig)
    assert len(bad) == 0, "first differences (world, word): %s" % bad[:10].tolist()
    # the run did something: contacts exist where the scene has any
    if scene != 3:
        assert ref["contact_count"].sum() > 0
