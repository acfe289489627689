"""Write the golden fixtures of the five scenes from the reference's own
CPU path.

Runs only where the reference tree is present: oracle/Makefile compiles
the reference's b3_batch.cuh / puffysics.cuh CPU path from its sources
into oracle/_ref/libb3ref_<n>.so (`make -C oracle ref`).  For each scene a
few worlds are built through the reference's creation API and driven
through the scene's workload loop (masks, restore, inputs, b3_batch_step);
their raw B3World bytes are saved at several step counts.  The fixtures
are data: inputs and the reference's outputs.

    python tests/golden/make_golden.py
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

from b3test import hover_actions, hover_cpu_run, hover_ref_lib, ref_lib  # noqa: E402
from puffysics_amd import scenes  # noqa: E402

# scene -> (worlds, checkpoints in vector steps)
PLAN = {1: (4, (1, 10, 60)), 2: (4, (1, 10, 61)), 3: (4, (1, 10, 60)), 4: (2, (1, 10, 30)), 5: (6, (1, 10, 60))}


def main():
    for scene, (count, checkpoints) in PLAN.items():
        ref = ref_lib(scene)
        if ref is None:
            raise SystemExit("oracle/_ref/libb3ref_%d.so missing: run make -C oracle ref" % scene)
        sc = scenes.SCENES[scene]
        ws = ref.ref_world_size()
        worlds = np.zeros(count * ws, np.uint8)
        ref.ref_build_batch(scene, worlds.ctypes.data, count, scenes.SEED, 0)
        initial = worlds.copy()
        out = {"initial": initial.reshape(count, ws).copy()}
        t = 0
        for cp in checkpoints:
            ref.ref_run(scene, worlds.ctypes.data, initial.ctypes.data, count, scenes.SEED, t, cp - t, sc.dt,
                        sc.substeps, 1, None)
            t = cp
            out["step%d" % cp] = worlds.reshape(count, ws).copy()
        out["signature"] = np.array([ref.ref_sig()], np.uint64)
        out["checkpoints"] = np.array(checkpoints, np.int32)
        path = os.path.join(HERE, "scene%d.npz" % scene)
        np.savez_compressed(path, **out)
        print("%s: %d worlds, checkpoints %s, %d bytes" % (path, count, checkpoints, os.path.getsize(path)))


# hover: envs, steps, observation checkpoints (every OBS_EVERY steps)
HOVER = (32, 300)
OBS_EVERY = 25


def hover():
    """The reference's hover task (oracle/_ref/libhover_ref.so) driven like
    its PufferLib adapter: init with seed 1, reset, 300 steps of seeded
    actions.  Rewards and terminals of every step, observations every 25
    steps, the summed log and the final worlds."""
    lib = hover_ref_lib()
    if lib is None:
        raise SystemExit("oracle/_ref/libhover_ref.so missing: run make -C oracle ref")
    n, steps = HOVER
    actions = hover_actions(n, steps)
    obs, rew, term, log, worlds = hover_cpu_run(lib, "rhover", n, actions)
    keep = np.arange(0, steps + 1, OBS_EVERY)
    path = os.path.join(HERE, "hover.npz")
    np.savez_compressed(path, actions=actions, rewards=rew, terminals=term, obs_steps=keep, observations=obs[keep],
                        log=log, worlds=worlds.view(np.uint8).reshape(n, -1))
    print("%s: %d envs, %d steps, %d episode ends, %d bytes" % (path, n, steps, int(term.sum()), os.path.getsize(path)))


if __name__ == "__main__":
    main()
    hover()
