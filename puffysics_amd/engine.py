"""Python binding of the engine's C ABI (include/b3_engine.h).

Mirrors the reference's batch interface (b3_batch.cuh:12-99): the
module-level b3_batch_* functions take the same arguments with the same
meaning and return the hipError_t code (0 = hipSuccess), never raising;
`B3Engine` wraps them for Python callers and raises `B3Error` instead.
Masks and input arrays are torch tensors on the engine's device (or raw
device pointers); `stream` is a torch.cuda.Stream, a raw hipStream_t, or
None for the current torch stream.  PyTorch only supplies device memory
and streams: every physics operation runs in libb3engine.so.
"""
import ctypes as C

import numpy as np

from . import _native
from .b3types import B3GravityLaw, B3StepStats, batch_of, world_dtype

HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1


class B3Error(RuntimeError):
    def __init__(self, call, code):
        super().__init__("%s failed with hipError_t %d" % (call, code))
        self.code = code


def _ptr(x):
    """Device pointer of a tensor / integer / None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _stream(s):
    if s is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(s, int):
        return s
    return s.cuda_stream


def b3_engine_create(worlds, sig):
    """(code, handle) for a contiguous numpy array of host worlds."""
    h = C.c_void_p()
    code = _native.engine_lib().b3_engine_create(C.byref(h), batch_of(worlds), sig)
    return code, h


def b3_batch_step_gpu(engine, dt, substeps, step_mask=None, reset_mask=None, stream=None):
    """Fused masked restore + masked step (b3_batch_step_gpu, b3_batch.cuh:81-89)."""
    return _native.engine_lib().b3_batch_step_gpu(engine, dt, substeps, _ptr(step_mask), _ptr(reset_mask),
                                                  _stream(stream))


def b3_batch_art_step_gpu(engine, dt, substeps, step_mask=None, reset_mask=None, stream=None):
    """b3_art_step, the reduced-coordinate integrator (09_step.inl:266-323),
    over the masked batch with the fused restore; the engine needs
    B3_ENGINE_ART_CONTACTS."""
    return _native.engine_lib().b3_batch_art_step_gpu(engine, dt, substeps, _ptr(step_mask), _ptr(reset_mask),
                                                      _stream(stream))


def b3_batch_restore_gpu(engine, reset=None, stream=None):
    """Masked snapshot restore (b3_batch_restore_gpu, b3_batch.cuh:91-99)."""
    return _native.engine_lib().b3_batch_restore_gpu(engine, _ptr(reset), _stream(stream))


def b3_batch_apply_gpu(engine, force=None, torque=None, linear_impulse=None, mask=None, stream=None):
    """Dense b3_apply_force / b3_apply_torque / b3_apply_linear_impulse (09_step.inl:132-146)."""
    return _native.engine_lib().b3_batch_apply_gpu(engine, _ptr(force), _ptr(torque), _ptr(linear_impulse),
                                                   _ptr(mask), _stream(stream))


def b3_batch_step_gravity_gpu(engine, dt, substeps, gravity, softening, masses=None, step_mask=None,
                              reset_mask=None, stream=None):
    """b3_batch_step_gpu with Plummer-softened pairwise gravity between each
    world's bodies in the per-substep force hook (B3_USER_FORCES,
    01_config.inl:189-198; nbody_rigid.cuh:15-66).  `masses` is None or a
    [worlds, max_bodies] float32 device tensor of gravitational masses."""
    return _native.engine_lib().b3_batch_step_gravity_gpu(engine, dt, substeps, _ptr(step_mask), _ptr(reset_mask),
                                                          B3GravityLaw(gravity, softening), _ptr(masses),
                                                          _stream(stream))


class _DLDevice(C.Structure):
    _fields_ = [("device_type", C.c_int32), ("device_id", C.c_int32)]


class _DLDataType(C.Structure):
    _fields_ = [("code", C.c_uint8), ("bits", C.c_uint8), ("lanes", C.c_uint16)]


class _DLTensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("device", _DLDevice), ("ndim", C.c_int32), ("dtype", _DLDataType),
                ("shape", C.POINTER(C.c_int64)), ("strides", C.POINTER(C.c_int64)), ("byte_offset", C.c_uint64)]


class _DLManagedTensor(C.Structure):
    _fields_ = [("dl_tensor", _DLTensor), ("manager_ctx", C.c_void_p), ("deleter", C.c_void_p)]


_DL_ROCM, _DL_CPU, _DL_INT = 10, 1, 0
_dl_keep = []


def device_tensor(ptr, shape, device_type=_DL_ROCM, device_id=None):
    """A torch int32 tensor of `shape` over memory the caller owns (the
    engine's device tiles), through a DLPack capsule: no copy, no
    allocation.  The memory must outlive the tensor."""
    import torch
    if device_id is None:
        device_id = torch.cuda.current_device() if device_type == _DL_ROCM else 0
    shp = (C.c_int64 * len(shape))(*shape)
    m = _DLManagedTensor()
    m.dl_tensor = _DLTensor(ptr, _DLDevice(device_type, device_id), len(shape), _DLDataType(_DL_INT, 32, 1), shp,
                            None, 0)
    m.manager_ctx = None
    m.deleter = None
    _dl_keep.append((m, shp))         # the capsule's struct and shape stay valid for the process
    new = C.pythonapi.PyCapsule_New
    new.restype = C.py_object
    new.argtypes = [C.c_void_p, C.c_char_p, C.c_void_p]
    return torch.utils.dlpack.from_dlpack(new(C.addressof(m), b"dltensor", None))


B3_ENGINE_KEEP_SOLVER_FIELDS = 1
B3_ENGINE_ART_CONTACTS = 2
B3_ENGINE_ONE_WAVE_PER_TILE = 4


class B3Engine:
    """A batch of worlds resident on the current HIP device."""

    def __init__(self, worlds, sig):
        worlds = np.ascontiguousarray(worlds)
        if worlds.dtype != world_dtype(sig):
            raise ValueError("worlds do not have the B3World layout of signature %#x" % sig)
        self.sig = sig
        self.dtype = worlds.dtype
        self.count = len(worlds)
        code, self._h = b3_engine_create(worlds, sig)
        if code != HIP_SUCCESS:
            raise B3Error("b3_engine_create", code)
        self._lib = _native.engine_lib()

    @property
    def handle(self):
        return self._h

    def _check(self, name, code):
        if code != HIP_SUCCESS:
            raise B3Error(name, code)

    def close(self):
        if self._h:
            code = self._lib.b3_engine_destroy(self._h)
            self._h = C.c_void_p()
            self._check("b3_engine_destroy", code)

    def __del__(self):
        try:
            if getattr(self, "_h", None):
                self._lib.b3_engine_destroy(self._h)
                self._h = C.c_void_p()
        except Exception:
            pass

    def set_options(self, options):
        """B3_ENGINE_* option bits (KEEP_SOLVER_FIELDS)."""
        self._check("b3_engine_set_options", self._lib.b3_engine_set_options(self._h, options))

    def set_snapshots(self, worlds):
        worlds = np.ascontiguousarray(worlds, dtype=self.dtype)
        if len(worlds) != self.count:
            raise ValueError("need %d snapshots" % self.count)
        self._check("b3_engine_set_snapshots", self._lib.b3_engine_set_snapshots(self._h, worlds.ctypes.data))

    def upload(self, worlds):
        worlds = np.ascontiguousarray(worlds, dtype=self.dtype)
        self._check("b3_engine_upload", self._lib.b3_engine_upload(self._h, batch_of(worlds)))

    def download(self):
        out = np.zeros(self.count, dtype=self.dtype)
        self._check("b3_engine_download", self._lib.b3_engine_download(self._h, batch_of(out)))
        return out

    def step(self, dt, substeps, step_mask=None, reset_mask=None, stream=None):
        self._check("b3_batch_step_gpu", b3_batch_step_gpu(self._h, dt, substeps, step_mask, reset_mask, stream))

    def art_step(self, dt, substeps, step_mask=None, reset_mask=None, stream=None):
        self._check("b3_batch_art_step_gpu", b3_batch_art_step_gpu(self._h, dt, substeps, step_mask, reset_mask,
                                                                   stream))

    def step_gravity(self, dt, substeps, gravity, softening, masses=None, step_mask=None, reset_mask=None,
                     stream=None):
        self._check("b3_batch_step_gravity_gpu", b3_batch_step_gravity_gpu(
            self._h, dt, substeps, gravity, softening, masses, step_mask, reset_mask, stream))

    def restore(self, reset=None, stream=None):
        self._check("b3_batch_restore_gpu", b3_batch_restore_gpu(self._h, reset, stream))

    def apply(self, force=None, torque=None, linear_impulse=None, mask=None, stream=None):
        self._check("b3_batch_apply_gpu", b3_batch_apply_gpu(self._h, force, torque, linear_impulse, mask, stream))

    def stats(self, stream=None):
        """Per-world B3StepStats as a numpy structured array (synchronises)."""
        import torch
        out = torch.zeros(self.count * C.sizeof(B3StepStats), dtype=torch.uint8, device="cuda")
        self._check("b3_batch_stats_gpu", self._lib.b3_batch_stats_gpu(self._h, out.data_ptr(), _stream(stream)))
        torch.cuda.synchronize()
        return out.cpu().numpy().view(np.dtype(B3StepStats))

    def scene_masks(self, scene, seed, step, reset_out, step_out, stream=None):
        self._check("b3w_masks_gpu", self._lib.b3w_masks_gpu(scene, seed, step, self.count, _ptr(reset_out),
                                                             _ptr(step_out), _stream(stream)))

    def tiles(self):
        """The live world state as a torch int32 tensor [tiles, world_words,
        64] sharing the engine's device memory (b3_engine_device_view): word
        k of world w is tiles[w // 64, k, w % 64].  Valid until close()."""
        ptr, words = C.c_void_p(), C.c_size_t()
        self._check("b3_engine_device_view", self._lib.b3_engine_device_view(self._h, C.byref(ptr), C.byref(words)))
        ntiles = (self.count + 63) // 64
        return device_tensor(ptr.value, (ntiles, words.value, 64))

    def scene_inputs(self, scene, seed, step, step_mask=None, stream=None):
        self._check("b3w_inputs_gpu", self._lib.b3w_inputs_gpu(self._h, scene, seed, step, _ptr(step_mask),
                                                               _stream(stream)))
