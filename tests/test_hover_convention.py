"""The done-step convention of the hover environment step
(examples/pufferlib/puffysics_hover/puffysics_hover.h:38-56), checked
step by step without the restatements of that step (oracle/hover.c,
oracle/hover_ref.c or the adapter's kernels).

Before every step the test takes each env's world, applies the action's
force (hover_apply_action, hover_task.h:68-73) and runs one b3_step of its
own (the library's CPU step); from that pre-reset state it evaluates the
task's reward and terminal (hover_task.h:83-93).  The environment must then
report:
  - that reward, bit for bit, on every step including the terminal one
    (the reward is the pre-reset reward);
  - that terminal flag;
  - on a terminal step, the observation of a freshly reset world (at rest,
    height target + jitter with |jitter| <= 0.5, tick 0) and a world that is
    exactly that; on any other step the observation of the stepped world;
  - log.n, episode_length, perf, score and episode_return incremented once
    per done, by 1, the episode's tick count, tick >= horizon and the sum of
    the episode's rewards (so tick and return restart from zero).
"""
import ctypes as C

import numpy as np
import pytest

from b3test import _hover_bind, hover_actions, hover_ref_lib, oracle
from puffysics_amd import _native
from puffysics_amd.b3types import world_dtype

TARGET, THRUST, DT, SUBSTEPS, HORIZON = 2.0, 10.0, 1.0 / 60.0, 4, 256
f32 = np.float32


def _reward(y, vy):
    """hover_reward (hover_task.h:83-87) in float32, in its operation order."""
    err = np.abs(y - f32(TARGET))
    return f32(1.0) - np.minimum(err + f32(0.1) * np.abs(vy), f32(2.0))


def _expected_step(world, action, sig):
    """The world after hover_step (hover_task.h:95-99) on a copy."""
    w = world.copy()
    level = f32(2.0) if action >= 1.5 else (f32(1.0) if action >= 0.5 else f32(0.0))
    b = w["bodies"]
    fy = level * f32(THRUST) / b["inv_mass"][0, 0]
    b["force"]["y"][0, 0] = b["force"]["y"][0, 0] + fy
    _native.engine_lib().b3_host_step(w.ctypes.data, sig, f32(DT), SUBSTEPS)
    return w


def check_convention(n, steps, actions, step_fn, world_fn, log_fn, obs0, sig):
    """Drive `step_fn(t) -> (obs, rewards, terminals)` and compare with the
    convention; `world_fn(i)` gives env i's world, `log_fn()` the summed log."""
    ticks = np.rint(obs0[:, 2] * HORIZON).astype(int)
    assert (ticks == 0).all()
    ret = np.zeros(n, np.float32)
    log = log_fn()
    dones = 0
    for t in range(steps):
        pre = [_expected_step(world_fn(i), actions[t][i], sig) for i in range(n)]
        obs, rew, term = step_fn(t)
        new_log = log_fn()
        dlog = new_log - log
        want_log = np.zeros(5, np.float64)
        for i in range(n):
            y = pre[i]["bodies"]["position"]["y"][0, 0]
            vy = pre[i]["bodies"]["lin_vel"]["y"][0, 0]
            r = _reward(y, vy)
            tick = ticks[i] + 1
            done = (not np.isfinite(y)) or np.abs(y - f32(TARGET)) > f32(3.0) or tick >= HORIZON
            assert rew[i].view(np.uint32) == r.view(np.uint32), (t, i, rew[i], r)
            assert term[i] == (1.0 if done else 0.0), (t, i)
            ret[i] = ret[i] + r
            if done:
                w = world_fn(i)
                b = w["bodies"]
                y0 = b["position"]["y"][0, 0]
                assert abs(float(y0) - TARGET) <= 0.5 and w["body_count"][0] == 1
                for f in ("lin_vel", "ang_vel", "force", "torque"):
                    assert all(b[f][a][0, 0] == 0 for a in "xyz"), f
                assert obs[i][0].view(np.uint32) == (y0 - f32(TARGET)).view(np.uint32)
                assert obs[i][1] == 0.0 and obs[i][2] == 0.0
                want_log += [tick >= HORIZON, ret[i], ret[i], tick, 1]
                ret[i] = 0.0
                ticks[i] = 0
                dones += 1
            else:
                assert obs[i][0].view(np.uint32) == (y - f32(TARGET)).view(np.uint32)
                assert obs[i][1].view(np.uint32) == vy.view(np.uint32)
                assert obs[i][2] == f32(tick) / f32(HORIZON)
                ticks[i] = tick
        assert np.allclose(dlog, want_log, rtol=1e-6, atol=1e-4), (t, dlog, want_log)
        assert dlog[4] == want_log[4] and dlog[3] == want_log[3] and dlog[0] == want_log[0]
        log = new_log
    return dones


def _cpu_env(lib, prefix, n, seed):
    _hover_bind(lib, prefix)
    f = lambda s: getattr(lib, prefix + s)
    envs = np.zeros(f("_env_bytes")() * n, np.uint8)
    f("_init")(envs.ctypes.data, n, TARGET, THRUST, DT, SUBSTEPS, HORIZON, seed)
    sig = f("_signature")()
    dtype = world_dtype(sig)
    obs = np.zeros((n, 3), np.float32)
    rew = np.zeros(n, np.float32)
    term = np.zeros(n, np.float32)
    f("_reset")(envs.ctypes.data, n, obs.ctypes.data, rew.ctypes.data, term.ctypes.data)

    def world(i):
        w = np.zeros(1, dtype)
        f("_world")(envs.ctypes.data, i, w.ctypes.data)
        return w

    def log():
        out = np.zeros(5, np.float32)
        f("_log")(envs.ctypes.data, n, out.ctypes.data)
        return out.astype(np.float64)
    return f, envs, sig, obs.copy(), world, log


@pytest.mark.parametrize("which", ["oracle", "reference"])
def test_cpu_env_step_convention(which):
    lib = oracle() if which == "oracle" else hover_ref_lib()
    if lib is None:
        pytest.skip("oracle/_ref/libhover_ref.so not built (reference tree absent)")
    prefix = "ohover" if which == "oracle" else "rhover"
    n, steps = 24, 320
    actions = hover_actions(n, steps, seed=5)
    actions[:, ::3] = 2.0                     # some envs fly off and fail early
    f, envs, sig, obs0, world, log = _cpu_env(lib, prefix, n, seed=11)

    def step(t):
        obs = np.zeros((n, 3), np.float32)
        rew = np.zeros(n, np.float32)
        term = np.zeros(n, np.float32)
        a = np.ascontiguousarray(actions[t], np.float32)
        f("_step")(envs.ctypes.data, n, a.ctypes.data, obs.ctypes.data, rew.ctypes.data, term.ctypes.data)
        return obs, rew, term
    dones = check_convention(n, steps, actions, step, world, log, obs0, sig)
    assert dones > n // 3


@pytest.mark.gpu
def test_gpu_adapter_step_convention():
    import torch
    from puffysics_amd.b3types import batch_of
    from puffysics_amd.hover import HoverEnvs
    n, steps = 24, 320
    actions = hover_actions(n, steps, seed=5)
    actions[:, ::3] = 2.0
    envs = HoverEnvs(n, seed=11)
    lib = oracle()
    lib.ohover_signature.restype = C.c_ulonglong
    sig = lib.ohover_signature()
    dtype = world_dtype(sig)
    envs.reset()
    obs0 = envs.observations.cpu().numpy().copy()

    def worlds():
        out = np.zeros(n, dtype)
        torch.cuda.synchronize()
        assert _native.engine_lib().b3_engine_download(envs.engine_handle(), batch_of(out)) == 0
        return out
    cache = {}

    def world(i):
        if "w" not in cache:
            cache["w"] = worlds()
        return cache["w"][i:i + 1].copy()

    def step(t):
        envs.actions.copy_(torch.from_numpy(np.ascontiguousarray(actions[t])))
        envs.step()
        torch.cuda.synchronize()
        cache.clear()
        return (envs.observations.cpu().numpy(), envs.rewards.cpu().numpy(), envs.terminals.cpu().numpy())

    def log():
        lg = envs.log()
        return np.array([lg[k] for k in ("perf", "score", "episode_return", "episode_length", "n")], np.float64)
    dones = check_convention(n, steps, actions, step, world, log, obs0, sig)
    envs.close()
    assert dones > n // 3
