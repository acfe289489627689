"""Counted algorithmic flops per env-step of the five benchmark workloads.

Runs each workload (masks, restore, inputs, step: the scene's own loop) on
a sample of its worlds with the counting build of the oracle
(oracle/liboracle_flops.so: b3cpu.c with every fp32 +, -, *, /, sqrt
counted), and records, for every vector step t, the flops of that step
divided by the worlds it stepped.  bench.py averages these over the steps
it times.  Writes tests/golden/flops.json; run after changing the oracle:
    python tests/golden/make_flops.py
"""
import ctypes as C
import json
import os
import sys
from concurrent.futures import ProcessPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

# (scene, sample worlds, vector steps): the benchmark's warm-up of 50 steps
# and its timed steps (1000; 2000 for the bin) are both covered.
PLAN = [(1, 256, 1050), (2, 128, 1050), (3, 128, 1050), (4, 32, 2050), (5, 128, 1050)]


def count_scene(scene, count, steps):
    import numpy as np
    from puffysics_amd import scenes
    lib = C.CDLL(os.path.join(ROOT, "oracle", "liboracle_flops.so"))
    fn = lib.ocount_batch_step
    fn.restype = C.c_longlong
    fn.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_int, C.c_ulonglong, C.c_float, C.c_int, C.c_void_p]
    sc = scenes.SCENES[scene]
    worlds = scenes.build(scene, count)
    initial = worlds.copy()
    per_step = []
    for t in range(steps):
        reset, stepm = scenes.masks(scene, count, t)
        r = reset.astype(bool)
        worlds[r] = initial[r]
        scenes.apply_inputs(scene, worlds, t, stepm)
        flops = fn(worlds.ctypes.data, worlds.dtype.itemsize, 0, count, sc.sig, sc.dt, sc.substeps,
                   stepm.ctypes.data)
        assert flops >= 0
        per_step.append(flops / max(int(stepm.sum()), 1))
    return scene, {"worlds_sampled": count, "steps": steps, "flops_per_env_step": [round(v, 1) for v in per_step],
                   "mean_contacts_end": float(worlds["contact_count"].mean())}


def main():
    out = {"counting": "oracle/liboracle_flops.so: fp32 +, -, *, / and sqrt count 1 each, the twist's atan2f 33, "
                       "negation / fabs / comparisons 0; no fused multiply-add exists in the step",
           "scenes": {}}
    with ProcessPoolExecutor(max_workers=len(PLAN)) as ex:
        for scene, res in ex.map(count_scene, *zip(*PLAN)):
            out["scenes"][str(scene)] = res
            v = res["flops_per_env_step"]
            print("scene %d: %.0f flops per env-step over steps 50..%d" % (scene, sum(v[50:]) / len(v[50:]),
                                                                             len(v) - 1))
    with open(os.path.join(HERE, "flops.json"), "w") as f:
        json.dump(out, f, separators=(",", ":"))


if __name__ == "__main__":
    main()
