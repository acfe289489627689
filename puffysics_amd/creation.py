"""Building worlds from Python with the reference's creation API.

libb3scenes.so exports the creation calls of include/b3_setup.h (the
reference's src/puffysics/04_world.inl and 06_joints.inl) for one capacity
set, CUSTOM_SIG = 16 bodies, 16 shapes, 32 contacts, 8 joints.  Worlds are
numpy structured arrays of that B3World layout; every call takes the world
array and an index.
"""
import ctypes as C

import numpy as np

from . import _native
from .b3types import signature, world_dtype

CUSTOM_SIG = signature(16, 16, 32, 8)
_f = C.c_float


def _lib():
    lib = _native.scenes_lib()
    if not getattr(lib, "_b3c_ready", False):
        vp, i = C.c_void_p, C.c_int
        lib.b3c_world_init.argtypes = [vp, _f, _f, _f]
        lib.b3c_body.argtypes = [vp, i] + [_f] * 13
        lib.b3c_sphere.argtypes = [vp, i, _f, _f, _f, _f, _f, _f, _f]
        lib.b3c_box.argtypes = [vp, i] + [_f] * 9
        lib.b3c_capsule.argtypes = [vp, i, _f, _f, _f, _f, _f]
        lib.b3c_finalize_mass.argtypes = [vp, i]
        lib.b3c_set_inertial.argtypes = [vp, i, _f, _f, _f, _f]
        lib.b3c_revolute.argtypes = [vp, i, i] + [_f] * 9
        lib.b3c_weld.argtypes = [vp, i, i] + [_f] * 6
        lib.b3c_joint_limits.argtypes = [vp, i, i, _f, _f]
        lib.b3c_joint_motor.argtypes = [vp, i, i, _f, _f]
        lib.b3c_joint_spring.argtypes = [vp, i, i, _f, _f, _f]
        lib._b3c_ready = True
    return lib


def new_worlds(count, gravity=(0.0, -10.0, 0.0)):
    """`count` empty worlds (b3_world_init) with the given gravity."""
    worlds = np.zeros(count, dtype=world_dtype(CUSTOM_SIG))
    for k in range(count):
        _lib().b3c_world_init(_ptr(worlds, k), *gravity)
    return worlds


def _ptr(worlds, k):
    return worlds.ctypes.data + k * worlds.dtype.itemsize


def body(worlds, k, type, pos, rot=(0.0, 0.0, 0.0, 1.0), lin_vel=(0.0, 0.0, 0.0), ang_vel=(0.0, 0.0, 0.0)):
    """b3_create_body; quaternions are (x, y, z, s)."""
    return _lib().b3c_body(_ptr(worlds, k), type, *pos, *rot, *lin_vel, *ang_vel)


def sphere(worlds, k, b, radius, center=(0.0, 0.0, 0.0), density=1000.0, friction=0.6, restitution=0.0):
    return _lib().b3c_sphere(_ptr(worlds, k), b, *center, radius, density, friction, restitution)


def box(worlds, k, b, half, pos=(0.0, 0.0, 0.0), density=1000.0, friction=0.6, restitution=0.0):
    return _lib().b3c_box(_ptr(worlds, k), b, *half, *pos, density, friction, restitution)


def capsule(worlds, k, b, half_len, radius, density=1000.0, friction=0.6, restitution=0.0):
    return _lib().b3c_capsule(_ptr(worlds, k), b, half_len, radius, density, friction, restitution)


def finalize_mass(worlds, k, b):
    _lib().b3c_finalize_mass(_ptr(worlds, k), b)


def set_inertial(worlds, k, b, mass, inertia):
    _lib().b3c_set_inertial(_ptr(worlds, k), b, mass, *inertia)


def revolute(worlds, k, a, b, anchor_a, anchor_b, axis):
    return _lib().b3c_revolute(_ptr(worlds, k), a, b, *anchor_a, *anchor_b, *axis)


def weld(worlds, k, a, b, anchor_a, anchor_b):
    return _lib().b3c_weld(_ptr(worlds, k), a, b, *anchor_a, *anchor_b)


def joint_limits(worlds, k, j, lower, upper, enable=1):
    _lib().b3c_joint_limits(_ptr(worlds, k), j, enable, lower, upper)


def joint_motor(worlds, k, j, speed, max_torque, enable=1):
    _lib().b3c_joint_motor(_ptr(worlds, k), j, enable, speed, max_torque)


def joint_spring(worlds, k, j, target, hertz, damping, enable=1):
    _lib().b3c_joint_spring(_ptr(worlds, k), j, enable, target, hertz, damping)
