"""Parity at the benchmark's full sizes, over the benchmarks' full runs.

The other GPU tests compare against the oracle at sizes it finishes in
seconds.  These run the five benchmark workloads at their own sizes (4,096
worlds; 65,536 for the arm) for their whole length (1,000 vector steps;
2,000 for the bin), with the scenes' masks, resets and inputs, on two
engines side by side: one with B3_ENGINE_KEEP_SOLVER_FIELDS and one with the
default options, which is the configuration bench.py times (on the arm,
the one-wave kernel b3k_step, whose contacts warm-start inside their
preparation).  Against the oracle stepping the same worlds:
  - after every vector step, each world's mean height and mean energy over
    its dynamic bodies, taken on the device from the engines' tiles; over
    the run their time means agree within 1% (the contract's long-run bar)
    and in fact to float64 rounding;
  - every 10th vector step, an exact checksum of every body word of every
    world (tests/b3test.py body_hash);
  - at the end of each segment (the arm: at steps 500 and 1,000), every
    live word of every world: bit-identical with KEEP; with the default
    options bit-identical except the contacts' prepared solver fields,
    which that mode does not write back.
Each workload's run is split into segments, one test each, run in order; a
segment run on its own steps through the earlier ones first.

Also one step of all 65,536 arm worlds from the same device state, on both
option sets, against the oracle stepping the downloaded worlds.
"""
import numpy as np
import pytest

from b3test import (clone, device_body_block, device_body_hash, diff_words, oracle_run, oracle_stats,
                    solver_field_words, stats_of_device_block)
from puffysics_amd import scenes

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

RUN_STEPS = {1: 1000, 2: 1000, 3: 1000, 4: 2000, 5: 1000}
SEGMENT = {1: 500, 2: 500, 3: 500, 4: 500, 5: 125}
FULL_DIFF_EVERY = {1: 500, 2: 500, 3: 500, 4: 500, 5: 500}
HASH_EVERY = 10
ORACLE_THREADS = 16


def _engines(worlds, scene):
    """(keep, default-options) engines on the same worlds."""
    from puffysics_amd.engine import B3_ENGINE_KEEP_SOLVER_FIELDS, B3Engine
    keep = B3Engine(worlds, scenes.SCENES[scene].sig)
    keep.set_options(B3_ENGINE_KEEP_SOLVER_FIELDS)
    lean = B3Engine(worlds, scenes.SCENES[scene].sig)
    return keep, lean


def bad_words(got, ref, sig, keep):
    """Differing live words; with the default options the contacts'
    prepared solver fields are left out."""
    bad = diff_words(got, ref, sig)
    if not keep and len(bad):
        allowed = solver_field_words(ref)
        bad = bad[~allowed[bad[:, 0], bad[:, 1]]]
    return bad


class FullRun:
    """One workload at its benchmark size on both engines and the oracle."""

    def __init__(self, scene):
        sc = scenes.SCENES[scene]
        self.scene, self.sc, self.count = scene, sc, sc.worlds
        worlds = scenes.build(scene, self.count)
        self.dtype = worlds.dtype
        self.engines = _engines(worlds, scene)
        self.tiles = [e.tiles() for e in self.engines]
        self.ref = clone(worlds)
        self.initial = worlds
        self.t = 0
        self.reset = torch.zeros(self.count, dtype=torch.uint8, device="cuda")
        self.stepm = torch.zeros(self.count, dtype=torch.uint8, device="cuda")
        self.acc_dev = torch.zeros((2, 2, self.count), dtype=torch.float64, device="cuda")
        self.acc_ref = np.zeros((2, self.count))
        self.hashes = 0

    def step(self):
        t, sc = self.t, self.sc
        oracle_run(self.scene, self.ref, self.initial, t, 1, threads=ORACLE_THREADS)
        hashed = t % HASH_EVERY == HASH_EVERY - 1
        st = oracle_stats(self.ref, checksum=hashed)
        self.acc_ref += st[:2]
        self.engines[0].scene_masks(self.scene, scenes.SEED, t, self.reset, self.stepm)
        for k, eng in enumerate(self.engines):
            eng.restore(self.reset)
            eng.scene_inputs(self.scene, scenes.SEED, t, self.stepm)
            eng.step(sc.dt, sc.substeps, self.stepm)
            blk = device_body_block(self.tiles[k], self.dtype, self.count)
            self.acc_dev[k] += stats_of_device_block(blk)
            if hashed:
                h = device_body_hash(blk).cpu().numpy()
                bad = np.flatnonzero(h != st[2])
                assert len(bad) == 0, "%s engine: body words differ after step %d in worlds %s" % (
                    ("keep", "default")[k], t, bad[:10].tolist())
        if hashed:
            self.hashes += 1
        self.t += 1

    def compare_all_words(self):
        torch.cuda.synchronize()
        for k, eng in enumerate(self.engines):
            bad = bad_words(eng.download(), self.ref, self.sc.sig, keep=(k == 0))
            assert len(bad) == 0, "%s engine after step %d: %d differing words in worlds %s, first %s" % (
                ("keep", "default")[k], self.t - 1, len(bad), np.unique(bad[:, 0])[:10].tolist(), bad[:4].tolist())

    def check_aggregates(self):
        """Time means over the run within 1% per world (NaN on both sides
        agrees: the reference's own capsule-box manifold can produce a NaN
        normal, and the engine reproduces it)."""
        ref = self.acc_ref / self.t
        for k in range(2):
            dev = self.acc_dev[k].cpu().numpy() / self.t
            for i, name in enumerate(("mean height", "mean energy")):
                g, r = dev[i], ref[i]
                floor = 1e-2 * np.nanmedian(np.abs(r)) + 1e-12
                ok = (np.abs(g - r) <= 0.01 * np.maximum(np.abs(r), floor)) | (np.isnan(g) & np.isnan(r))
                assert ok.all(), "%s differs in worlds %s" % (name, np.flatnonzero(~ok)[:10].tolist())
                tight = (np.abs(g - r) <= 1e-9 * np.maximum(np.abs(r), floor)) | (np.isnan(g) & np.isnan(r))
                assert tight.all(), "%s beyond float64 rounding in worlds %s" % (
                    name, np.flatnonzero(~tight)[:10].tolist())
        # the workloads move: energy changes over the run in most worlds
        start = oracle_stats(self.initial, checksum=False)[1]
        assert np.nanmedian(np.abs(ref[1] - start)) > 0

    def close(self):
        for e in self.engines:
            e.close()


_runs = {}


def _run_to(scene, end):
    run = _runs.get(scene)
    if run is None or run.t > end - SEGMENT[scene]:
        if run is not None:
            run.close()
        run = _runs[scene] = FullRun(scene)
    while run.t < end:
        run.step()
        if run.t % FULL_DIFF_EVERY[scene] == 0 and run.t < end:
            run.compare_all_words()
    return run


@pytest.mark.timeout(600)
@pytest.mark.parametrize("scene,segment", [(s, k) for s in (1, 2, 3, 4, 5) for k in range(RUN_STEPS[s] // SEGMENT[s])])
def test_full_run(scene, segment):
    """Segment `segment` of the workload's full run; see the module
    docstring for what is compared when."""
    end = (segment + 1) * SEGMENT[scene]
    run = _run_to(scene, end)
    assert run.t == end
    if end % FULL_DIFF_EVERY[scene] == 0:
        run.compare_all_words()
    if end == RUN_STEPS[scene]:
        assert run.hashes == RUN_STEPS[scene] // HASH_EVERY
        try:
            run.check_aggregates()
            if scene in (3, 5):                     # the hinges' spring / motor / limit rows ran
                j = run.ref["joints"]
                assert np.abs(j["spring_impulse"]).max() + np.abs(j["motor_impulse"]).max() > 0
            assert scene in (1, 3) or run.ref["contact_count"].mean() > 1
        finally:
            run.close()
            del _runs[scene]


def _gpu_run(eng, scene, t0, nsteps):
    sc = scenes.SCENES[scene]
    reset = torch.zeros(eng.count, dtype=torch.uint8, device="cuda")
    stepm = torch.zeros(eng.count, dtype=torch.uint8, device="cuda")
    for t in range(t0, t0 + nsteps):
        eng.scene_masks(scene, scenes.SEED, t, reset, stepm)
        eng.restore(reset)
        eng.scene_inputs(scene, scenes.SEED, t, stepm)
        eng.step(sc.dt, sc.substeps, stepm)
    torch.cuda.synchronize()


def _assert_same_contacts(got, ref):
    """Contact count, shape pair, point count and feature ids of every live
    contact, vectorised over the batch."""
    assert (got["contact_count"] == ref["contact_count"]).all()
    cg, cr = got["contacts"], ref["contacts"]
    live = np.arange(cg.shape[1])[None, :] < ref["contact_count"][:, None]
    for f in ("shape_a", "shape_b", "body_a", "body_b", "point_count"):
        bad = (cg[f] != cr[f]) & live
        assert not bad.any(), "%s differs at %s" % (f, np.argwhere(bad)[:5].tolist())
    pc = np.where(live, cr["point_count"], 0)
    for p in range(cg["points"].shape[2]):
        on = pc > p
        bad = (cg["points"]["feature"][:, :, p] != cr["points"]["feature"][:, :, p]) & on
        assert not bad.any(), "feature %d differs at %s" % (p, np.argwhere(bad)[:5].tolist())


@pytest.mark.timeout(600)
@pytest.mark.parametrize("keep", [True, False], ids=["keep", "default"])
def test_arm_65536_one_step_from_the_same_state(keep):
    """The 65,536-world arm batch after 40 vector steps on the device, then
    one more step on the device and on the oracle from that same state:
    identical contacts and identical worlds, word for word, in every world
    (with the default options, all but the prepared solver fields)."""
    from puffysics_amd.engine import B3_ENGINE_KEEP_SOLVER_FIELDS, B3Engine
    scene, count, warm = 5, 65536, 40
    sig = scenes.SCENES[scene].sig
    worlds = scenes.build(scene, count)
    eng = B3Engine(worlds, sig)
    if keep:
        eng.set_options(B3_ENGINE_KEEP_SOLVER_FIELDS)
    _gpu_run(eng, scene, 0, warm)
    state = eng.download()
    ref = clone(state)
    oracle_run(scene, ref, worlds, warm, 1, threads=ORACLE_THREADS)
    _gpu_run(eng, scene, warm, 1)
    got = eng.download()
    eng.close()
    assert ref["contact_count"].mean() > 8          # a contact-rich state
    _assert_same_contacts(got, ref)
    bad = bad_words(got, ref, sig, keep)
    assert len(bad) == 0, "%d differing words in worlds %s" % (len(bad), np.unique(bad[:, 0])[:10].tolist())
