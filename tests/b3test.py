"""Shared helpers of the test suite: the oracle (CPU restatement of the
reference b3_step), the host build of the engine's lane code, and world
comparisons.  The oracle and the emulation library are test
infrastructure; the engine never loads them."""
import ctypes as C
import os

import numpy as np

from puffysics_amd import scenes
from puffysics_amd.b3types import B3Contact, B3Point, world_ctype, world_dtype

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_PATH = os.path.join(ROOT, "oracle", "liboracle.so")
REF_DIR = os.path.join(ROOT, "oracle", "_ref")
EMU_PATH = os.path.join(ROOT, "tests", "emu", "libb3emu.so")
GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")

_vp, _i, _ull, _f = C.c_void_p, C.c_int, C.c_ulonglong, C.c_float
_oracle = None
_emu = None
_refs = {}


def oracle():
    global _oracle
    if _oracle is None:
        lib = C.CDLL(ORACLE_PATH)
        lib.ocpu_world_size.restype = C.c_size_t
        lib.ocpu_world_size.argtypes = [_ull]
        lib.ocpu_step.argtypes = [_vp, _ull, _f, _i]
        lib.ocpu_find_contacts.argtypes = [_vp, _ull]
        for n in range(1, 6):
            fn = getattr(lib, "ocpu_run_%d" % n)
            fn.restype = C.c_longlong
            fn.argtypes = [_vp, _vp, _i, _ull, _i, _i, _f, _i, _i, _vp]
        _oracle = lib
    return _oracle


def ref_lib(scene):
    """The reference's own CPU path compiled from its sources, or None."""
    path = os.path.join(REF_DIR, "libb3ref_%d.so" % scene)
    if not os.path.exists(path):
        return None
    if scene not in _refs:
        lib = C.CDLL(path)
        lib.ref_sig.restype = C.c_ulonglong
        lib.ref_world_size.restype = C.c_size_t
        lib.ref_build.argtypes = [_i, _vp, _ull, _i]
        lib.ref_build_batch.argtypes = [_i, _vp, _i, _ull, _i]
        lib.ref_step.argtypes = [_vp, _f, _i]
        lib.ref_run.restype = C.c_longlong
        lib.ref_run.argtypes = [_i, _vp, _vp, _i, _ull, _i, _i, _f, _i, _i, _vp]
        _refs[scene] = lib
    return _refs[scene]


def emu():
    global _emu
    if _emu is None:
        lib = C.CDLL(EMU_PATH)
        lib.emu_upload.argtypes = [_vp, _i, _ull, _vp]
        lib.emu_download.argtypes = [_vp, _i, _ull, _vp]
        lib.emu_restore.argtypes = [_vp, _vp, _i, _ull, _vp]
        lib.emu_step.argtypes = [_vp, _i, _ull, _f, _i, _vp]
        lib.emu_inputs.argtypes = [_vp, _i, _ull, _i, _ull, _i, _vp]
        lib.emu_world_words.argtypes = [_ull]
        _emu = lib
    return _emu


def oracle_run(scene, worlds, initial, t0, nsteps, seed=scenes.SEED, threads=1):
    """Steps [t0, t0+nsteps) of a scene's workload on the oracle, in place:
    masks, restore, inputs, step (puffysics_amd/scenes/b3_workload.h)."""
    sc = scenes.SCENES[scene]
    fn = getattr(oracle(), "ocpu_run_%d" % scene)
    return fn(worlds.ctypes.data, initial.ctypes.data, len(worlds), seed, t0, nsteps, sc.dt, sc.substeps,
              threads, None)


class EmuBatch:
    """Word-transposed tiles stepped by the host build of the lane code."""

    def __init__(self, scene, worlds):
        self.scene = scene
        self.sc = scenes.SCENES[scene]
        self.count = len(worlds)
        self.dtype = worlds.dtype
        words = emu().emu_world_words(self.sc.sig)
        ntiles = (self.count + 63) // 64
        self.tiles = np.zeros(ntiles * words * 64, np.uint32)
        self.snap = np.zeros_like(self.tiles)
        w = np.ascontiguousarray(worlds)
        emu().emu_upload(w.ctypes.data, self.count, self.sc.sig, self.tiles.ctypes.data)
        emu().emu_upload(w.ctypes.data, self.count, self.sc.sig, self.snap.ctypes.data)

    def run(self, t0, nsteps, seed=scenes.SEED):
        e = emu()
        for t in range(t0, t0 + nsteps):
            reset, stepm = scenes.masks(self.scene, self.count, t, seed)
            if reset.any():
                e.emu_restore(self.tiles.ctypes.data, self.snap.ctypes.data, self.count, self.sc.sig,
                              reset.ctypes.data)
            e.emu_inputs(self.tiles.ctypes.data, self.count, self.sc.sig, self.scene, seed, t, stepm.ctypes.data)
            e.emu_step(self.tiles.ctypes.data, self.count, self.sc.sig, self.sc.dt, self.sc.substeps,
                       stepm.ctypes.data)

    def worlds(self):
        out = np.zeros(self.count, dtype=self.dtype)
        emu().emu_download(self.tiles.ctypes.data, self.count, self.sc.sig, out.ctypes.data)
        return out


# B3Shape has 4 bytes of padding before its 8-aligned category field.
SHAPE_PAD_WORD = 17


def clone(worlds):
    """Byte-exact copy.  numpy copies structured arrays field by field and
    leaves padding bytes of the copy as the allocator returned them."""
    out = np.empty_like(worlds)
    out.view(np.uint8)[:] = np.ascontiguousarray(worlds).view(np.uint8)
    return out


def live_word_mask(worlds, sig):
    """Boolean [count, words] mask of the words b3_step defines: header,
    live bodies / shapes / joints, live contacts without their unused
    point slots.  Struct padding is left out."""
    W = world_ctype(sig)
    nwords = C.sizeof(W) // 4
    mask = np.zeros((len(worlds), nwords), bool)
    bo, so, co, jo = (W.bodies.offset // 4, W.shapes.offset // 4, W.contacts.offset // 4, W.joints.offset // 4)
    bw, sw, cw, jw = 50, 22, C.sizeof(B3Contact) // 4, 115
    pts = B3Contact.points.offset // 4
    pw = C.sizeof(B3Point) // 4
    mask[:, :17] = True
    for i, w in enumerate(worlds):
        mask[i, bo:bo + bw * int(w["body_count"])] = True
        mask[i, so:so + sw * int(w["shape_count"])] = True
        mask[i, so + SHAPE_PAD_WORD:so + sw * int(w["shape_count"]):sw] = False
        mask[i, jo:jo + jw * int(w["joint_count"])] = True
        for c in range(int(w["contact_count"])):
            base = co + c * cw
            pc = int(w["contacts"][c]["point_count"])
            mask[i, base:base + pts + pw * pc] = True
            mask[i, base + pts + pw * 4:base + cw] = True
    return mask


def words(worlds):
    return np.ascontiguousarray(worlds).view(np.uint32).reshape(len(worlds), -1)


def diff_words(a, b, sig):
    """Indices (world, word) where two batches differ on live words."""
    m = live_word_mask(a, sig) & live_word_mask(b, sig)
    d = (words(a) != words(b)) & m
    return np.argwhere(d)
