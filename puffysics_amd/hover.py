"""The PufferLib hover environment on the engine (include/b3_hover.h).

Mirrors the reference adapter's vector API
(examples/pufferlib/puffysics_hover/puffysics_hover.cu:44-79):
`HoverEnvs(n, seed)` is puf_vec_create, `reset()` puf_reset, `step()`
puf_step, `log()` puf_log, `close()` puf_close.  Observations, actions,
rewards and terminals are torch CUDA tensors owned by the object (the
reference takes the trainer's buffers; `HoverEnvs` accepts them too).
"""
import ctypes as C
import os

from . import _native

HOVER_PATH = os.path.join(_native.HERE, "libb3hover.so")


class B3HoverConfig(C.Structure):
    _fields_ = [("target_height", C.c_float), ("thrust", C.c_float), ("dt", C.c_float), ("substeps", C.c_int),
                ("horizon", C.c_int)]


class B3HoverLog(C.Structure):
    _fields_ = [("perf", C.c_float), ("score", C.c_float), ("episode_return", C.c_float),
                ("episode_length", C.c_float), ("n", C.c_float)]


_vp, _i = C.c_void_p, C.c_int
HOVER_SYMBOLS = [
    ("b3_hover_default_config", B3HoverConfig, []),
    ("b3_hover_create", _i, [C.POINTER(_vp), _i, B3HoverConfig, C.c_uint32, _vp, _vp, _vp, _vp]),
    ("b3_hover_reset", _i, [_vp, _vp]),
    ("b3_hover_step", _i, [_vp, _vp]),
    ("b3_hover_log", _i, [_vp, C.POINTER(B3HoverLog), _vp]),
    ("b3_hover_engine", _vp, [_vp]),
    ("b3_hover_destroy", _i, [_vp]),
]

_lib = None


def hover_lib():
    """libb3hover.so, loaded once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(HOVER_PATH):
            raise RuntimeError("%s is missing: run __graft_entry__.build()" % HOVER_PATH)
        _native.engine_lib()   # the adapter links the engine library
        lib = C.CDLL(HOVER_PATH)
        for name, res, args in HOVER_SYMBOLS:
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def default_config():
    return hover_lib().b3_hover_default_config()


class HoverEnvs:
    """n hover envs on the current device."""

    def __init__(self, n, seed=1, config=None, observations=None, actions=None, rewards=None, terminals=None):
        import torch
        from .engine import B3Error
        lib = hover_lib()
        self.n = n
        self.config = config if config is not None else lib.b3_hover_default_config()
        self.observations = observations if observations is not None else torch.zeros((n, 3), device="cuda")
        self.actions = actions if actions is not None else torch.zeros(n, device="cuda")
        self.rewards = rewards if rewards is not None else torch.zeros(n, device="cuda")
        self.terminals = terminals if terminals is not None else torch.zeros(n, device="cuda")
        self._h = _vp()
        code = lib.b3_hover_create(C.byref(self._h), n, self.config, seed, self.observations.data_ptr(),
                                   self.actions.data_ptr(), self.rewards.data_ptr(), self.terminals.data_ptr())
        if code != 0:
            raise B3Error("b3_hover_create", code)

    def _check(self, name, code):
        from .engine import B3Error
        if code != 0:
            raise B3Error(name, code)

    def _stream(self, stream):
        import torch
        s = stream if stream is not None else torch.cuda.current_stream()
        return s.cuda_stream

    def reset(self, stream=None):
        self._check("b3_hover_reset", hover_lib().b3_hover_reset(self._h, self._stream(stream)))

    def step(self, stream=None):
        self._check("b3_hover_step", hover_lib().b3_hover_step(self._h, self._stream(stream)))

    def log(self, stream=None):
        out = B3HoverLog()
        self._check("b3_hover_log", hover_lib().b3_hover_log(self._h, C.byref(out), self._stream(stream)))
        return {f: getattr(out, f) for f, _ in B3HoverLog._fields_}

    def engine_handle(self):
        return hover_lib().b3_hover_engine(self._h)

    def close(self):
        if self._h:
            self._check("b3_hover_destroy", hover_lib().b3_hover_destroy(self._h))
            self._h = _vp()

    def __del__(self):
        try:
            if getattr(self, "_h", None):
                hover_lib().b3_hover_destroy(self._h)
                self._h = _vp()
        except Exception:
            pass
