"""Loading of the in-tree native libraries.

libb3engine.so is the product (gfx950 kernels behind the C ABI of
include/b3_engine.h and include/b3_workload.h); libb3scenes.so holds the
host world builders of the benchmark scenes.  Both are built by
__graft_entry__.build() (make -C puffysics_amd).  There is no fallback: a
missing library raises.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
ENGINE_PATH = os.path.join(HERE, "libb3engine.so")
SCENES_PATH = os.path.join(HERE, "libb3scenes.so")

# (name, restype, argtypes) of every C-ABI entry point in include/b3_engine.h
# and include/b3_workload.h; None and strings stand for the structs of
# b3types.py passed by value (None: B3Batch).
_vp, _i, _ull, _f, _sz = C.c_void_p, C.c_int, C.c_ulonglong, C.c_float, C.c_size_t
ENGINE_SYMBOLS = [
    ("b3_engine_create", _i, [C.POINTER(C.c_void_p), None, _ull]),
    ("b3_engine_destroy", _i, [_vp]),
    ("b3_engine_count", _i, [_vp]),
    ("b3_engine_set_snapshots", _i, [_vp, _vp]),
    ("b3_engine_upload", _i, [_vp, None]),
    ("b3_engine_download", _i, [_vp, None]),
    ("b3_batch_restore_gpu", _i, [_vp, _vp, _vp]),
    ("b3_batch_step_gpu", _i, [_vp, _f, _i, _vp, _vp, _vp]),
    ("b3_batch_art_step_gpu", _i, [_vp, _f, _i, _vp, _vp, _vp]),
    ("b3_batch_apply_gpu", _i, [_vp, _vp, _vp, _vp, _vp, _vp]),
    ("b3_batch_stats_gpu", _i, [_vp, _vp, _vp]),
    ("b3_engine_device_view", _i, [_vp, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]),
    ("b3_engine_set_options", _i, [_vp, C.c_uint]),
    ("b3_batch_step_gravity_gpu", _i, [_vp, _f, _i, _vp, _vp, "B3GravityLaw", _vp, _vp]),
    ("b3_batch_step_worlds_gpu", _i, [None, _ull, _f, _i, _vp, _vp]),
    ("b3_host_step", None, [_vp, _ull, _f, _i]),
    ("b3_host_batch_step", _i, [None, _ull, _f, _i, _vp]),
    ("b3w_masks_gpu", _i, [_i, _ull, _i, _i, _vp, _vp, _vp]),
    ("b3w_inputs_gpu", _i, [_vp, _i, _ull, _i, _vp, _vp]),
]

_engine = None
_scenes = None


def _torch_runtime_first():
    """Initialise torch's HIP runtime before a library of this package loads
    the system one.  PyTorch ships its own copy of the HIP runtime; when the
    system runtime is loaded into the process first, calls through it fail
    with hipErrorNoDevice once torch has initialised the GPU.  Without a GPU
    (or without torch) this does nothing."""
    try:
        import torch
    except ImportError:
        return
    if torch.cuda.is_available():
        torch.cuda.init()


def engine_lib():
    """The engine library, loaded once; raises if it has not been built."""
    global _engine
    if _engine is None:
        if not os.path.exists(ENGINE_PATH):
            raise RuntimeError("%s is missing: run __graft_entry__.build()" % ENGINE_PATH)
        from . import b3types
        _torch_runtime_first()
        lib = C.CDLL(ENGINE_PATH)
        for name, res, args in ENGINE_SYMBOLS:
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = [b3types.B3Batch if a is None else getattr(b3types, a) if isinstance(a, str) else a
                           for a in args]
        _engine = lib
    return _engine


def scenes_lib():
    global _scenes
    if _scenes is None:
        if not os.path.exists(SCENES_PATH):
            raise RuntimeError("%s is missing: run __graft_entry__.build()" % SCENES_PATH)
        lib = C.CDLL(SCENES_PATH)
        for n in range(1, 6):
            getattr(lib, "b3s_signature_%d" % n).restype = C.c_ulonglong
            getattr(lib, "b3s_world_size_%d" % n).restype = C.c_size_t
            getattr(lib, "b3s_build_batch_%d" % n).argtypes = [_vp, _i, _ull, _i]
            getattr(lib, "b3s_apply_inputs_batch_%d" % n).argtypes = [_vp, _i, _ull, _i, _i, _vp]
        lib.b3s_masks.argtypes = [_i, _ull, _i, _i, _i, _vp, _vp]
        _scenes = lib
    return _scenes
