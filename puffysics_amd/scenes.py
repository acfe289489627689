"""The five synthetic workloads and their host builders.

Each scene is a world family built through the public creation API
(include/b3_setup.h, the reference's src/puffysics/04_world.inl and
06_joints.inl) by puffysics_amd/scenes/b3_scenes.h, with fixed compile-time
capacities, a step size and a substep count:

  1 hover   one sphere (r 0.5, mass 1) above a ground box, random thrust
  2 stack   five unit cubes on a ground box, an impulse every 60 steps
  3 chain   eight capsules hanging from hinges with spring, motor, limits
  4 bin     32 spheres / boxes / capsules dropped into a five-box bin
  5 arm     a four-link hinged arm plus 12 free bodies on a ground box,
            2% random resets and a 90% random step mask per vector step
"""
import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _native
from .b3types import signature, world_dtype


@dataclass(frozen=True)
class Scene:
    id: int
    name: str
    worlds: int        # batch size of the workload
    caps: tuple        # (bodies, shapes, contacts, joints)
    dt: float
    substeps: int
    steps: int         # vector steps of the workload

    @property
    def sig(self):
        return signature(*self.caps)


SCENES = {
    1: Scene(1, "hover", 4096, (2, 2, 4, 2), 1.0 / 60.0, 4, 1000),
    2: Scene(2, "stack", 4096, (6, 6, 16, 1), 1.0 / 60.0, 4, 1000),
    3: Scene(3, "chain", 4096, (9, 8, 32, 8), 1.0 / 120.0, 8, 1000),
    4: Scene(4, "bin", 4096, (33, 37, 128, 1), 1.0 / 60.0, 4, 2000),
    5: Scene(5, "arm", 65536, (17, 17, 64, 4), 1.0 / 60.0, 4, 1000),
}
SEED = 1


def build(scene, count, seed=SEED, first=0):
    """`count` fresh worlds of a scene (world indices first .. first+count-1)."""
    sc = SCENES[scene]
    lib = _native.scenes_lib()
    assert getattr(lib, "b3s_signature_%d" % scene)() == sc.sig
    worlds = np.zeros(count, dtype=world_dtype(sc.sig))
    assert worlds.dtype.itemsize == getattr(lib, "b3s_world_size_%d" % scene)()
    if count and not getattr(lib, "b3s_build_batch_%d" % scene)(worlds.ctypes.data, count, seed, first):
        raise ValueError("unknown scene %d" % scene)
    return worlds


def apply_inputs(scene, worlds, step, step_mask=None, seed=SEED, first=0):
    """Host application of step `step`'s scene inputs (b3s_apply_inputs)."""
    lib = _native.scenes_lib()
    mask = None if step_mask is None else np.ascontiguousarray(step_mask, dtype=np.uint8)
    getattr(lib, "b3s_apply_inputs_batch_%d" % scene)(
        worlds.ctypes.data, len(worlds), seed, first, step, None if mask is None else mask.ctypes.data)


def masks(scene, count, step, seed=SEED, first=0):
    """(reset, step) masks of a vector step, as uint8 arrays."""
    reset = np.zeros(count, np.uint8)
    stepm = np.zeros(count, np.uint8)
    _native.scenes_lib().b3s_masks(scene, seed, first, count, step, reset.ctypes.data, stepm.ctypes.data)
    return reset, stepm
