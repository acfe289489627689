"""The PufferLib hover environment (§8 f1): the oracle against the
reference's own hover task and its fixture on the CPU, and the engine's
adapter (libb3hover.so, include/b3_hover.h) against both on the GPU.

The hover world has no contacts and no hinges, so the adapter's
observations, rewards, terminals, logs and worlds must equal the
reference's bit for bit."""
import ctypes as C
import os

import numpy as np
import pytest

from b3test import ROOT, hover_actions, hover_cpu_run, hover_ref_lib, oracle

FIXTURE = os.path.join(ROOT, "tests", "golden", "hover.npz")


def bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


def test_oracle_matches_reference_task():
    """The oracle's hover env restates hover_task.h and the environment
    step; the reference's task compiled from its sources must agree bit for
    bit over several episodes (failures and horizons)."""
    ref = hover_ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref/libhover_ref.so not built (reference tree absent)")
    actions = hover_actions(48, 600, seed=9)
    a = hover_cpu_run(oracle(), "ohover", 48, actions, seed=7)
    b = hover_cpu_run(ref, "rhover", 48, actions, seed=7)
    for x, y in zip(a[:4], b[:4]):
        assert np.array_equal(bits(x), bits(y))
    assert np.array_equal(a[4].view(np.uint8), b[4].view(np.uint8))
    assert b[2].sum() > 48          # episodes ended more than once per env on average
    assert b[3][0] > 0 and b[3][4] > b[3][0]   # some by the horizon, some by failure


def test_oracle_matches_fixture():
    d = np.load(FIXTURE)
    n = d["actions"].shape[1]
    obs, rew, term, log, worlds = hover_cpu_run(oracle(), "ohover", n, d["actions"])
    assert np.array_equal(bits(rew), bits(d["rewards"]))
    assert np.array_equal(bits(term), bits(d["terminals"]))
    assert np.array_equal(bits(obs[d["obs_steps"]]), bits(d["observations"]))
    assert np.array_equal(bits(log), bits(d["log"]))
    assert np.array_equal(worlds.view(np.uint8).reshape(n, -1), d["worlds"])


def test_hover_library_exports_the_header():
    from puffysics_amd.hover import HOVER_SYMBOLS, hover_lib
    lib = hover_lib()
    hdr = open(os.path.join(ROOT, "include", "b3_hover.h")).read()
    for name, _, _ in HOVER_SYMBOLS:
        assert name in hdr
        assert getattr(lib, name) is not None


def test_default_config_is_the_reference_default():
    from puffysics_amd.hover import default_config
    c = default_config()
    assert (c.target_height, c.thrust, c.substeps, c.horizon) == (2.0, 10.0, 4, 256)
    assert c.dt == np.float32(1.0 / 60.0)


# ---- GPU ----

def _gpu_run(n, actions, seed=1):
    import torch
    from puffysics_amd.hover import HoverEnvs
    envs = HoverEnvs(n, seed=seed)
    steps = len(actions)
    obs = np.zeros((steps + 1, n, 3), np.float32)
    rew = np.zeros((steps + 1, n), np.float32)
    term = np.zeros((steps + 1, n), np.float32)
    envs.reset()
    obs[0], rew[0], term[0] = envs.observations.cpu().numpy(), envs.rewards.cpu().numpy(), envs.terminals.cpu().numpy()
    for t in range(steps):
        envs.actions.copy_(torch.from_numpy(np.ascontiguousarray(actions[t])))
        envs.step()
        obs[t + 1] = envs.observations.cpu().numpy()
        rew[t + 1] = envs.rewards.cpu().numpy()
        term[t + 1] = envs.terminals.cpu().numpy()
    lg = envs.log()
    log = np.array([lg[k] for k in ("perf", "score", "episode_return", "episode_length", "n")], np.float32)
    worlds = download(envs.engine_handle(), n)
    envs.close()
    return obs, rew, term, log, worlds


def download(handle, n):
    from puffysics_amd import _native
    from puffysics_amd.b3types import batch_of, world_dtype
    from b3test import oracle
    lib = oracle()
    lib.ohover_signature.restype = C.c_ulonglong
    out = np.zeros(n, world_dtype(lib.ohover_signature()))
    assert _native.engine_lib().b3_engine_download(handle, batch_of(out)) == 0
    return out


@pytest.mark.gpu
def test_adapter_matches_reference_fixture():
    d = np.load(FIXTURE)
    n = d["actions"].shape[1]
    obs, rew, term, log, worlds = _gpu_run(n, d["actions"])
    assert np.array_equal(bits(rew), bits(d["rewards"]))
    assert np.array_equal(bits(term), bits(d["terminals"]))
    assert np.array_equal(bits(obs[d["obs_steps"]]), bits(d["observations"]))
    assert np.array_equal(bits(log), bits(d["log"]))
    from b3test import live_word_mask
    from b3test import oracle as _o
    lib = _o()
    lib.ohover_signature.restype = C.c_ulonglong
    m = live_word_mask(worlds, lib.ohover_signature())
    ref = d["worlds"].view(np.uint32).reshape(n, -1)
    assert np.array_equal(worlds.view(np.uint32).reshape(n, -1)[m], ref[m])


@pytest.mark.gpu
def test_adapter_matches_oracle_many_envs():
    """300 envs over 700 steps: every observation, reward and terminal."""
    n, steps = 300, 700
    actions = hover_actions(n, steps, seed=21)
    g = _gpu_run(n, actions, seed=3)
    o = hover_cpu_run(oracle(), "ohover", n, actions, seed=3)
    for x, y in zip(g[:4], o[:4]):
        assert np.array_equal(bits(x), bits(y))
    assert o[2].sum() > n


@pytest.mark.gpu
def test_adapter_rejects_bad_arguments():
    import torch
    from puffysics_amd.hover import B3HoverConfig, default_config, hover_lib
    lib = hover_lib()
    h = C.c_void_p()
    buf = torch.zeros(16, device="cuda")
    p = buf.data_ptr()
    assert lib.b3_hover_create(C.byref(h), 0, default_config(), 1, p, p, p, p) != 0
    bad = default_config()
    bad.substeps = 0
    assert lib.b3_hover_create(C.byref(h), 4, bad, 1, p, p, p, p) != 0
    assert lib.b3_hover_create(C.byref(h), 4, default_config(), 1, None, p, p, p) != 0
    assert not h
    assert lib.b3_hover_step(None, None) != 0
    assert lib.b3_hover_destroy(None) == 0
    assert isinstance(B3HoverConfig(), B3HoverConfig)
