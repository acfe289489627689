"""ctypes / numpy mirrors of the plain-data world model (include/b3_types.h).

The structs are byte-for-byte the reference's (src/puffysics/02_types.inl:
55-142, 306-346); a whole batch of worlds is a numpy structured array whose
dtype is built for one capacity signature (B3_CONFIG_SIGNATURE,
src/puffysics/01_config.inl:70-74).
"""
import ctypes as C

import numpy as np

B3_STATIC, B3_KINEMATIC, B3_DYNAMIC = 0, 1, 2
B3_SPHERE, B3_CAPSULE, B3_BOX = 0, 1, 2
B3_JOINT_WELD, B3_JOINT_REVOLUTE = 0, 1
B3_MAX_MANIFOLD = 4


class B3Vec3(C.Structure):
    _fields_ = [("x", C.c_float), ("y", C.c_float), ("z", C.c_float)]


class B3Vec2(C.Structure):
    _fields_ = [("x", C.c_float), ("y", C.c_float)]


class B3Quat(C.Structure):
    _fields_ = [("v", B3Vec3), ("s", C.c_float)]


class B3Mat3(C.Structure):
    _fields_ = [("cx", B3Vec3), ("cy", B3Vec3), ("cz", B3Vec3)]


class B3Mat2(C.Structure):
    _fields_ = [("cx", B3Vec2), ("cy", B3Vec2)]


class B3Soft(C.Structure):
    _fields_ = [("bias_rate", C.c_float), ("mass_scale", C.c_float), ("impulse_scale", C.c_float)]


class B3Body(C.Structure):
    _fields_ = [("position", B3Vec3), ("rotation", B3Quat), ("center", B3Vec3), ("local_center", B3Vec3),
                ("lin_vel", B3Vec3), ("ang_vel", B3Vec3), ("force", B3Vec3), ("torque", B3Vec3),
                ("delta_pos", B3Vec3), ("delta_rot", B3Quat), ("inv_mass", C.c_float),
                ("inv_inertia", B3Vec3), ("inv_i_world", B3Mat3), ("linear_damping", C.c_float),
                ("angular_damping", C.c_float), ("gravity_scale", C.c_float), ("type", C.c_int),
                ("flags", C.c_uint32)]


class B3Shape(C.Structure):
    _fields_ = [("body", C.c_int), ("type", C.c_int), ("local_pos", B3Vec3), ("local_rot", B3Quat),
                ("radius", C.c_float), ("half", B3Vec3), ("friction", C.c_float), ("restitution", C.c_float),
                ("rolling", C.c_float), ("density", C.c_float), ("category", C.c_uint64), ("mask", C.c_uint64)]


class B3Point(C.Structure):
    _fields_ = [("r_a", B3Vec3), ("r_b", B3Vec3), ("base_sep", C.c_float), ("rel_vel", C.c_float),
                ("normal_impulse", C.c_float), ("total_normal", C.c_float), ("normal_mass", C.c_float),
                ("lever", C.c_float), ("feature", C.c_uint32)]


class B3Contact(C.Structure):
    _fields_ = [("shape_a", C.c_int), ("shape_b", C.c_int), ("body_a", C.c_int), ("body_b", C.c_int),
                ("point_count", C.c_int), ("static_contact", C.c_int), ("normal", B3Vec3),
                ("tangent1", B3Vec3), ("tangent2", B3Vec3), ("points", B3Point * B3_MAX_MANIFOLD),
                ("center_a", B3Vec3), ("center_b", B3Vec3), ("friction", C.c_float), ("restitution", C.c_float),
                ("rolling", C.c_float), ("twist_mass", C.c_float), ("twist_impulse", C.c_float),
                ("friction_impulse", B3Vec2), ("rolling_impulse", B3Vec3), ("tangent_mass", B3Mat2),
                ("rolling_mass", B3Mat3), ("inv_mass_a", C.c_float), ("inv_mass_b", C.c_float),
                ("inv_i_a", B3Mat3), ("inv_i_b", B3Mat3), ("softness", B3Soft)]


class B3Joint(C.Structure):
    _fields_ = [("type", C.c_int), ("body_a", C.c_int), ("body_b", C.c_int), ("collide_connected", C.c_int),
                ("fixed_rotation", C.c_int), ("local_anchor_a", B3Vec3), ("local_anchor_b", B3Vec3),
                ("local_rot_a", B3Quat), ("local_rot_b", B3Quat), ("constraint_hertz", C.c_float),
                ("constraint_damping", C.c_float), ("softness", B3Soft), ("inv_mass_a", C.c_float),
                ("inv_mass_b", C.c_float), ("inv_i_a", B3Mat3), ("inv_i_b", B3Mat3), ("frame_p_a", B3Vec3),
                ("frame_p_b", B3Vec3), ("frame_q_a", B3Quat), ("frame_q_b", B3Quat), ("delta_center", B3Vec3),
                ("linear_impulse", B3Vec3), ("angular_impulse", B3Vec3), ("angular_mass", B3Mat3),
                ("linear_hertz", C.c_float), ("linear_damping", C.c_float), ("angular_hertz", C.c_float),
                ("angular_damping", C.c_float), ("linear_spring", B3Soft), ("angular_spring", B3Soft),
                ("perp_impulse", B3Vec2), ("spring_impulse", C.c_float), ("motor_impulse", C.c_float),
                ("lower_impulse", C.c_float), ("upper_impulse", C.c_float), ("hertz", C.c_float),
                ("damping_ratio", C.c_float), ("max_motor_torque", C.c_float), ("motor_speed", C.c_float),
                ("target_angle", C.c_float), ("lower_angle", C.c_float), ("upper_angle", C.c_float),
                ("enable_spring", C.c_int), ("enable_motor", C.c_int), ("enable_limit", C.c_int),
                ("rotation_axis", B3Vec3), ("perp_x", B3Vec3), ("perp_y", B3Vec3), ("axial_mass", C.c_float),
                ("spring_softness", B3Soft)]


HEADER_FIELDS = [("gravity", B3Vec3), ("contact_hertz", C.c_float), ("contact_damping", C.c_float),
                 ("contact_speed", C.c_float), ("restitution_threshold", C.c_float),
                 ("max_linear_speed", C.c_float), ("body_count", C.c_int), ("shape_count", C.c_int),
                 ("contact_count", C.c_int), ("joint_count", C.c_int), ("body_overflow", C.c_int),
                 ("shape_overflow", C.c_int), ("joint_overflow", C.c_int), ("contact_overflow", C.c_int),
                 ("contacts_dropped", C.c_int)]


class B3StepStats(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("body_count", "shape_count", "contact_count", "joint_count",
                                        "body_overflow", "shape_overflow", "joint_overflow",
                                        "contact_overflow", "contacts_dropped")]


class B3Batch(C.Structure):
    _fields_ = [("data", C.c_void_p), ("stride", C.c_size_t), ("world_offset", C.c_size_t), ("count", C.c_int)]


class B3GravityLaw(C.Structure):
    """Pairwise gravity law of b3_batch_step_gravity_gpu (NbodyConfig, nbody.cuh:40-46)."""
    _fields_ = [("gravity", C.c_float), ("softening", C.c_float)]


def signature(bodies, shapes, contacts, joints):
    """B3_CONFIG_SIGNATURE for a capacity set."""
    return bodies | (shapes << 16) | (contacts << 32) | (joints << 48)


def capacities(sig):
    return sig & 0xFFFF, (sig >> 16) & 0xFFFF, (sig >> 32) & 0xFFFF, (sig >> 48) & 0xFFFF


_world_types = {}


def world_ctype(sig):
    """The ctypes B3World of a capacity signature (compiler layout)."""
    if sig not in _world_types:
        b, s, c, j = capacities(sig)
        if min(b, s, c, j) < 1:
            raise ValueError("invalid capacity signature %#x" % sig)
        _world_types[sig] = type("B3World_%x" % sig, (C.Structure,), {
            "_fields_": HEADER_FIELDS + [("bodies", B3Body * b), ("shapes", B3Shape * s),
                                         ("contacts", B3Contact * c), ("joints", B3Joint * j)]})
    return _world_types[sig]


def world_dtype(sig):
    return np.dtype(world_ctype(sig))


def world_size(sig):
    return C.sizeof(world_ctype(sig))


def empty_worlds(sig, count):
    return np.zeros(count, dtype=world_dtype(sig))


def batch_of(worlds):
    """A B3Batch viewing a contiguous numpy array of worlds."""
    assert worlds.flags["C_CONTIGUOUS"]
    return B3Batch(worlds.ctypes.data, worlds.dtype.itemsize, 0, len(worlds))
