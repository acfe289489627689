"""Boundary behaviour of the device engine beyond single-scene parity:
  - the step, restore and scene inputs captured into a HIP graph replay
    bit-identically to the same calls made eagerly ("enqueues on stream
    without allocation or synchronization; safe in capture",
    b3_batch.cuh:77-80), on both step kernels;
  - a kernel's dynamic-LDS limit, one setting shared by every engine in the
    process, is not lowered by an engine created later;
  - idle lanes of a shared tile (worlds outside the step mask, or past the
    end of the batch) stay untouched while the tile's other worlds step;
  - an empty batch validates its arguments and then succeeds without a
    launch (b3_batch.cuh:81-101).
"""
import numpy as np
import pytest

from b3test import clone, diff_words, gpu_run, oracle_run
from puffysics_amd import scenes

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _engine(worlds, scene, options=1):
    from puffysics_amd.engine import B3Engine
    eng = B3Engine(worlds, scenes.SCENES[scene].sig)
    eng.set_options(options)
    return eng


def _vector_step(eng, scene, t, reset, stepm):
    sc = scenes.SCENES[scene]
    eng.scene_masks(scene, scenes.SEED, t, reset, stepm)
    eng.scene_inputs(scene, scenes.SEED, t, stepm)
    eng.step(sc.dt, sc.substeps, stepm, reset)


@pytest.mark.parametrize("scene,count,options", [(5, 4096, 1), (5, 300, 1), (4, 130, 1), (5, 300, 4), (5, 17000, 0),
                                                 (1, 4096, 0)],
                         ids=["arm4096-shared-keep", "arm300-shared-keep", "bin130-shared-keep",
                              "arm300-one_wave", "arm17000-one_wave-default", "hover4096-kept_row-default"])
def test_graph_replay_equals_eager(scene, count, options):
    """Masks, inputs and the fused restore + step of one vector step are
    captured once; each replay is checked against the same calls made
    eagerly on a twin engine, with downloads (eager work and
    synchronisation) between replays.  Batches of at most one tile per CU
    (4,096 and 300 arm worlds, 130 bin worlds) take the shared-tile kernel;
    the one-wave kernel b3k_step runs when forced (option
    B3_ENGINE_ONE_WAVE_PER_TILE = 4) and for 17,000 arm worlds (266 tiles)
    with the default options, the configuration of the 65,536-world
    benchmark; the hover's worlds (two shapes) take the one-wave kernel that
    keeps their contact row, b3k_step<JI, true>, at any batch size."""
    sc = scenes.SCENES[scene]
    worlds = scenes.build(scene, count)
    graphed, eager = _engine(worlds, scene, options), _engine(worlds, scene, options)
    reset_g = torch.zeros(count, dtype=torch.uint8, device="cuda")
    stepm_g = torch.zeros(count, dtype=torch.uint8, device="cuda")
    reset_e = torch.zeros_like(reset_g)
    stepm_e = torch.zeros_like(stepm_g)
    t = 7                                  # a step whose masks reset some worlds
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _vector_step(graphed, scene, t, reset_g, stepm_g)
    torch.cuda.synchronize()
    assert len(diff_words(graphed.download(), worlds, sc.sig)) == 0   # capture ran nothing
    for r in range(4):
        graph.replay()
        _vector_step(eager, scene, t, reset_e, stepm_e)
        torch.cuda.synchronize()
        a, b = graphed.download(), eager.download()
        bad = diff_words(a, b, sc.sig)
        assert len(bad) == 0, "replay %d: %d differing words" % (r, len(bad))
    if scene == 5:                         # the arm scene's masks reset and skip worlds
        assert int(reset_e.sum()) > 0 and int(stepm_e.sum()) < count
    graphed.close()
    eager.close()


def test_lds_limit_survives_a_later_engine():
    """The bin's shared tiles take 150 KiB of LDS.  Creating a stacks engine
    (less LDS) afterwards must not lower the kernels' limit below what the
    bin launches with."""
    worlds = scenes.build(4, 130)
    ref = clone(worlds)
    bin_eng = _engine(worlds, 4)
    stacks = _engine(scenes.build(2, 64), 2)
    gpu_run(bin_eng, 4, 0, 5)
    oracle_run(4, ref, clone(worlds), 0, 5)
    bad = diff_words(bin_eng.download(), ref, scenes.SCENES[4].sig)
    assert len(bad) == 0
    stacks.close()
    bin_eng.close()


@pytest.mark.parametrize("scene,count", [(5, 200), (4, 100), (2, 70)])
def test_shared_tile_with_sparse_step_mask(scene, count):
    """Shared tiles where only every ninth world steps and one whole tile
    steps none: idle worlds keep every word, the stepping ones equal the
    oracle's."""
    from b3test import oracle_step_batch
    sc = scenes.SCENES[scene]
    worlds = scenes.build(scene, count)
    oracle_run(scene, worlds, clone(worlds), 0, 10)
    active = (np.arange(count) % 9 == 4).astype(np.uint8)
    active[64:128] = 0
    ref = clone(worlds)
    eng = _engine(worlds, scene)
    d_active = torch.from_numpy(active).cuda()
    for _ in range(6):
        oracle_step_batch(ref, sc.sig, sc.dt, sc.substeps, active)
        eng.step(sc.dt, sc.substeps, d_active)
    torch.cuda.synchronize()
    got = eng.download()
    eng.close()
    bad = diff_words(got, ref, sc.sig)
    assert len(bad) == 0, "%d differing words, first %s" % (len(bad), bad[:4].tolist())
    idle = active == 0
    assert len(diff_words(got[idle], worlds[idle], sc.sig)) == 0


def test_empty_batch():
    """Zero worlds: every entry point succeeds with nothing to do, while the
    step still refuses an invalid dt or substep count first (the reference's
    b3_batch_step_gpu validates, then returns cudaSuccess for an empty
    batch, b3_batch.cuh:83-86; b3_batch_restore_gpu likewise, :95-98)."""
    from puffysics_amd.engine import (HIP_ERROR_INVALID_VALUE, b3_batch_apply_gpu, b3_batch_restore_gpu,
                                      b3_batch_step_gpu)
    for scene in (1, 5):
        sc = scenes.SCENES[scene]
        empty = scenes.build(scene, 64)[:0].copy()
        eng = _engine(empty, scene)
        assert eng.count == 0
        assert b3_batch_step_gpu(eng.handle, sc.dt, sc.substeps) == 0
        assert b3_batch_step_gpu(eng.handle, 0.0, sc.substeps) == 0
        for dt, subs in ((float("nan"), 4), (-1.0, 4), (sc.dt, 0)):
            assert b3_batch_step_gpu(eng.handle, dt, subs) == HIP_ERROR_INVALID_VALUE
        assert b3_batch_restore_gpu(eng.handle) == 0
        force = torch.zeros(3, device="cuda")
        assert b3_batch_apply_gpu(eng.handle, force=force) == 0
        eng.set_snapshots(empty)
        eng.upload(empty)
        assert len(eng.download()) == 0
        assert len(eng.stats()) == 0
        torch.cuda.synchronize()
        eng.close()
