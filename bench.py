"""Physics-only env-steps/s of the batched stepping engine on one MI355X.

Measures the five benchmark workloads (scenes built by
puffysics_amd/scenes/b3_scenes.h, inputs drawn by a counter-based RNG):
  hover   4,096 worlds: a sphere over a ground box, random thrust; dt 1/60, 4 substeps
  stacks  4,096 worlds: 5 jittered unit cubes, periodic impulses; dt 1/60, 4 substeps
  chains  4,096 worlds: 8 capsules on sprung, motorised, limited hinges; dt 1/120, 8 substeps
  bin     4,096 worlds: 32 mixed bodies in a 5-box bin; dt 1/60, 4 substeps
  arm    65,536 worlds: a 4-link hinged arm with motors and 12 free bodies,
                        2% reset and 90% step masks per vector step; dt 1/60, 4 substeps
The headline (`value`, `config`, `roofline`, `cpu_baseline`) is the arm at
65,536 worlds; every workload's own figures are under `configs`.

One vector step = masked restore + scene inputs + masked step on one HIP
stream, with the worlds resident in HBM; an env-step is one world stepped
(substeps not counted).  Each workload is first settled untimed to W vector
steps before its window start (vector step 500; 1000 for the bin: halfway
through the benchmark run, once the stacks stand, the bin's bodies have
landed and the arm's resets run at their steady rate), and its device state
is saved.  Each repeat (3, median) restores that state, runs the W untimed
warm-up steps and times the window of K vector steps from the window start
(defaults: W = 50, K to the end of the benchmark run: 500; 1000 for the
bin), so every repeat times the same work.  The step kernel's own duration
is timed with HIP events on its stream around every 8th launch.

Per workload, all over the same window:
  roofline   algorithmic bytes per launch (the byte model below on each
             stepped world's live contact count after each step of the
             window, from one more untimed pass of it) / kernel time,
             against 8 TB/s; counted flops per launch
             (tests/golden/flops.json: the oracle's fp32 operations on the
             same workload and steps) / kernel time, against the fp32 vector
             peak (157.3 TFLOP/s with packed FMA, 78.6 without); measured HBM
             bytes (rocprofv3 FETCH_SIZE / WRITE_SIZE in profiles/) only
             when that profile was taken of this source tree over launches
             of a window with the same start.
  cpu        the reference's own CPU path (b3_batch_step / b3_batch_restore,
             oracle/_ref) built -O3 for this host's x86-64 level, one pinned
             thread per physical core available to the process, on the
             workload's full world count, started from the device's state at
             the window start (bit-identical to the reference's) and run
             over the window's first steps, repeated for a bounded time.
`--profile-commands DIR` / `--profile-summary DIR` (with --scene) give the
rocprofv3 runs of the same window and reduce them to profiles/.

Two more measurements, each its own JSON line and not the headline:
`--scene N --art` steps the workload with articulated contacts
(B3_ENGINE_ART_CONTACTS, the reference's B3_ART_CONTACTS=1 step), and
`--hover-env N` times the PufferLib hover adapter's vector step on N envs.
"""
import argparse
import ctypes as C
import hashlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "physics env-steps/sec at 4096 and 65536 worlds, 1 MI355X; % HBM/VALU roofline"
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3          # 256 CUs x 4 SIMDs x 16 lanes x 2 (packed) x 2 (FMA) x 2.4 GHz
FP32_NONPACKED_TFLOPS = 78.6
HEADLINE = 5
NAMES = {1: "hover", 2: "stacks", 3: "chains", 4: "bin", 5: "arm"}

# Algorithmic bytes of one env-step, per item: the minimal persistent-state
# traffic of a step with all scratch on chip.
BYTES_DYNAMIC_BODY = 212   # 76 read + 64 written + 24 force/torque clear + 48 constants
BYTES_STATIC_BODY = 36
BYTES_SHAPE = 80
BYTES_CONTACT = 136        # 68-byte warm cache read and written
BYTES_JOINT = 192          # 120 constants + 36 impulses read + 36 written
BYTES_WORLD = 58           # 56 header + step and reset mask bytes

# Each workload's timed window starts at this vector step, halfway through
# its benchmark run (1,000 vector steps; 2,000 for the bin): the stacks stand,
# the bin's bodies have landed and the arm's resets run at their steady
# rate.  The default window runs to the end of the benchmark run.
WINDOW_START = {1: 500, 2: 500, 3: 500, 4: 1000, 5: 500}
RUN_LENGTH = {1: 1000, 2: 1000, 3: 1000, 4: 2000, 5: 1000}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def physical_cpus():
    """One logical CPU per physical core among those this process may use,
    capped by the cgroup's CPU quota; and the uncapped count."""
    allowed = sorted(os.sched_getaffinity(0))
    seen, cpus = set(), []
    for cpu in allowed:
        base = "/sys/devices/system/cpu/cpu%d/topology/" % cpu
        try:
            key = (open(base + "physical_package_id").read().strip(), open(base + "core_id").read().strip())
        except OSError:
            key = ("?", str(cpu))
        if key in seen:
            continue
        seen.add(key)
        cpus.append(cpu)
    quota = None
    try:
        q, period = open("/sys/fs/cgroup/cpu.max").read().split()
        if q != "max":
            quota = max(1, int(int(q) / int(period)))
    except (OSError, ValueError):
        pass
    n = len(cpus) if quota is None else min(len(cpus), quota)
    return cpus[:n], len(cpus), quota


def engine_source_digest():
    """Digest of the engine's sources: the build a counter profile came from."""
    h = hashlib.sha256()
    d = os.path.join(ROOT, "puffysics_amd", "csrc")
    for name in sorted(os.listdir(d)):
        with open(os.path.join(d, name), "rb") as f:
            h.update(name.encode() + b"\0" + f.read())
    with open(os.path.join(ROOT, "puffysics_amd", "Makefile"), "rb") as f:
        h.update(f.read())
    return h.hexdigest()[:16]


def world_bytes_model(worlds, contacts):
    """Per-world algorithmic bytes of one step, given live contact counts."""
    import numpy as np
    b = worlds["bodies"]
    live = np.arange(b.shape[1])[None, :] < worlds["body_count"][:, None]
    n_dyn = ((b["type"] == 2) & live).sum(axis=1)
    n_static = live.sum(axis=1) - n_dyn
    return (BYTES_DYNAMIC_BODY * n_dyn + BYTES_STATIC_BODY * n_static + BYTES_SHAPE * worlds["shape_count"]
            + BYTES_CONTACT * contacts + BYTES_JOINT * worlds["joint_count"] + BYTES_WORLD).astype(np.float64)


def counted_flops(scene, first, count):
    """Mean counted flops per env-step over vector steps [first, first+count)
    of the workload (tests/golden/flops.json), and the window used."""
    with open(os.path.join(ROOT, "tests", "golden", "flops.json")) as f:
        per_step = json.load(f)["scenes"][str(scene)]["flops_per_env_step"]
    lo, hi = first, first + count
    if hi > len(per_step):            # past the counted run: its last 500 steps
        lo, hi = max(0, len(per_step) - 500), len(per_step)
    window = per_step[lo:hi]
    return sum(window) / len(window), [lo, hi]


def joint_rows_fit(max_b, max_s, max_c, max_j):
    """Whether a shared tile keeps its joint rows in LDS (joint_rows_fit in
    puffysics_amd/csrc/b3d_lane.h): the velocity or contact-generation
    rows, the contact levels, 52 words per joint and the joint levels within
    640 words per lane."""
    lds_rows = max(7 * max_b, 48 + 6 * max_s if 48 + 6 * max_s <= 160 else 48)
    words = lds_rows + 2 + max_b + 2 * max_c + 52 * max_j + 1 + 4 * max_j + max_b
    return max_j > 0 and words <= 640


def joint_impulses_fit(max_b, max_s, max_c, max_j):
    """Whether the one-wave step keeps the joint impulses in LDS (ji_fit in
    puffysics_amd/csrc/b3d_lane.h): 7 velocity words per body and 9 impulse
    words per joint within 160 words per lane."""
    return max_j > 0 and 7 * max_b + 9 * max_j <= 160


def kernel_name(scene, count):
    """The step kernel a batch launches (b3_engine_create): b3k_step<JI, true>
    for worlds of at most two shapes; else b3k_step_shared<Masks, JL> when
    the tiles fit one per CU, b3k_step<JI, false> when they do not."""
    import torch
    from puffysics_amd import scenes
    tiles = (count + 63) // 64
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    caps = scenes.SCENES[scene].caps
    if caps[1] <= 2:                 # one candidate pair: b3k_step<JI, true> at any batch size
        return "b3k_step<%s, true>" % ("true" if joint_impulses_fit(*caps) else "false")
    if tiles > cus:
        return "b3k_step<%s, false>" % ("true" if joint_impulses_fit(*caps) else "false")
    masks = 12 <= caps[1] <= 64
    return "b3k_step_shared<%s, %s>" % ("true" if masks else "false", "true" if joint_rows_fit(*caps) else "false")


def load_counters(kernel, scene, count, digest, start, end):
    """Per-launch counter figures of a kernel on a workload from the committed
    rocprofv3 summary, if it was taken of this source tree over launches of
    the window [start, end) (same start: every window from a start is the
    same stationary run); else None."""
    path = os.path.join(ROOT, "profiles", "counters_%s%d.json" % (NAMES[scene], count))
    if not os.path.exists(path):
        return None
    with open(path) as f:
        c = json.load(f)
    if c.get("source_digest") != digest or c.get("kernel") != kernel:
        return None
    w = c.get("window")
    if not w or w[0] != start or w[1] > end:
        return None
    return c


def cpu_baseline(scene, count, state, initial, start, end, seconds):
    """The reference's CPU path on the workload's worlds over the GPU's timed
    window: from `state` (the worlds at vector step `start`, downloaded from
    the device, bit-identical to what the reference computes), vector steps
    [start, end) or the first of them, repeated from `state` until about
    `seconds` of stepping have been timed."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from b3test import fast_levels_supported, oracle, ref_fast_lib, ref_lib
    from puffysics_amd import scenes
    sc = scenes.SCENES[scene]
    cpus, affinity_cores, quota = physical_cpus()
    nthreads = max(1, len(cpus))
    cpu_arr = (C.c_int * nthreads)(*cpus)
    lib, flags = None, None
    for level, cflags in fast_levels_supported():
        lib = ref_fast_lib(scene, level)
        if lib is not None:
            flags = cflags
            break
    if lib is None and ref_lib(scene) is not None:
        lib, flags = ref_lib(scene), "-O2 -ffp-contract=off -fno-fast-math"
    src = np.ascontiguousarray(state).view(np.uint8).ravel()
    init = np.ascontiguousarray(initial).view(np.uint8).ravel().copy()
    worlds = np.empty_like(src)
    if lib is not None:
        kind = "reference"
        assert lib.ref_world_size() * count == src.size
        fn = lib.ref_run
        args = lambda t0, n: (scene, worlds.ctypes.data, init.ctypes.data, count, scenes.SEED, t0, n, sc.dt,
                              sc.substeps, nthreads, cpu_arr)
    else:
        kind, flags = "port", "-O2 -ffp-contract=off -fno-fast-math"
        fn = getattr(oracle(), "ocpu_run_%d" % scene)
        args = lambda t0, n: (worlds.ctypes.data, init.ctypes.data, count, scenes.SEED, t0, n, sc.dt, sc.substeps,
                              nthreads, cpu_arr)
    worlds[:] = src
    t0 = time.perf_counter()
    fn(*args(start, 1))
    first = time.perf_counter() - t0
    per_pass = int(max(1, min(end - start, seconds / max(first, 1e-6))))
    env_steps, el, passes = 0, 0.0, 0
    while passes == 0 or el < seconds:
        worlds[:] = src
        t0 = time.perf_counter()
        env_steps += fn(*args(start, per_pass))
        el += time.perf_counter() - t0
        passes += 1
    return {"value": round(env_steps / el, 1), "unit": "env-steps/s", "cores": nthreads, "kind": kind,
            "flags": flags, "affinity_physical_cores": affinity_cores, "cgroup_cpu_quota": quota,
            "window": [start, start + per_pass],
            "sample": "all %d worlds from the device's state at vector step %d, vector steps %d..%d of the same "
                      "workload (inside the GPU's timed window %d..%d), %d pass%s, %d pinned threads (one per "
                      "physical core available), %.1f s" % (count, start, start, start + per_pass, start, end, passes,
                                                          "" if passes == 1 else "es", nthreads, el)}


def window_of(scene, steps, warmup):
    """The vector steps a workload's run covers: untimed settling [0, settle),
    then per repeat `warmup` untimed steps [settle, start) and the timed
    window [start, start + steps), every repeat from the same saved state."""
    start = WINDOW_START[scene]
    w = min(warmup, start)
    return start - w, start, start + steps


def run_workload(scene, count, steps, warmup, repeats, event_every, digest, cpu_seconds=None, art=False):
    import numpy as np
    import torch
    from puffysics_amd import scenes
    from puffysics_amd.engine import B3Engine

    sc = scenes.SCENES[scene]
    log("%s: building %d worlds" % (NAMES[scene], count))
    worlds = scenes.build(scene, count)
    eng = B3Engine(worlds, sc.sig)
    if art:
        from puffysics_amd.engine import B3_ENGINE_ART_CONTACTS
        eng.set_options(B3_ENGINE_ART_CONTACTS)
    tiles = eng.tiles()
    stream = torch.cuda.current_stream()
    settle, start, end = window_of(scene, steps, warmup)
    reset = torch.empty((end, count), dtype=torch.uint8, device="cuda")
    stepm = torch.empty((end, count), dtype=torch.uint8, device="cuda")
    for t in range(end):
        eng.scene_masks(scene, scenes.SEED, t, reset[t], stepm[t])
    step_counts = stepm.sum(dim=1, dtype=torch.int64).cpu().numpy()
    reset_any = reset.amax(dim=1).cpu().numpy()

    def vector_step(t):
        if reset_any[t]:
            eng.restore(reset[t])
        eng.scene_inputs(scene, scenes.SEED, t, stepm[t])

    log("  settling: vector steps 0..%d untimed" % settle)
    for t in range(settle):
        vector_step(t)
        eng.step(sc.dt, sc.substeps, stepm[t])
    saved = tiles.clone()                      # the state every repeat starts from
    torch.cuda.synchronize()

    def warm_up():
        tiles.copy_(saved)
        for t in range(settle, start):
            vector_step(t)
            eng.step(sc.dt, sc.substeps, stepm[t])

    rates, ms, kernel_ms = [], [], []
    timed = range(0, steps, max(1, event_every))
    for r in range(repeats):
        warm_up()
        k_start = {i: torch.cuda.Event(enable_timing=True) for i in timed}
        k_end = {i: torch.cuda.Event(enable_timing=True) for i in timed}
        t_begin, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t_begin.record(stream)
        for i in range(steps):
            t = start + i
            vector_step(t)
            if i in k_start:
                k_start[i].record(stream)
            eng.step(sc.dt, sc.substeps, stepm[t])
            if i in k_end:
                k_end[i].record(stream)
        t_end.record(stream)
        torch.cuda.synchronize()
        el_ms = t_begin.elapsed_time(t_end)
        env = int(step_counts[start:end].sum())
        rates.append(env / (el_ms * 1e-3))
        ms.append(el_ms / steps)
        kernel_ms.append(sum(k_start[i].elapsed_time(k_end[i]) for i in timed) / len(timed))
        log("  repeat %d: vector steps %d..%d, %.4f ms/step, %.4g env-steps/s, step kernel %.4f ms" % (
            r, start, end, ms[-1], rates[-1], kernel_ms[-1]))
    med = sorted(range(repeats), key=lambda i: rates[i])[repeats // 2]

    # The byte model over the same window, untimed: the same steps again from
    # the saved state, with each stepped world's live contact count after
    # each step.  The state at the window's start seeds the CPU baseline.
    warm_up()
    torch.cuda.synchronize()
    state_at_start = eng.download() if cpu_seconds else None
    base = torch.from_numpy(world_bytes_model(worlds, np.zeros(count))).cuda()
    cc_word = worlds.dtype.fields["contact_count"][1] // 4
    bytes_sum = torch.zeros((), dtype=torch.float64, device="cuda")
    contact_sum = torch.zeros((), dtype=torch.float64, device="cuda")
    for t in range(start, end):
        vector_step(t)
        eng.step(sc.dt, sc.substeps, stepm[t])
        cc = tiles[:, cc_word, :].reshape(-1)[:count].double()
        on = stepm[t].double()
        bytes_sum += (on * (base + BYTES_CONTACT * cc)).sum()
        contact_sum += cc.mean()
    torch.cuda.synchronize()
    eng.close()
    stepped = float(step_counts[start:end].sum())
    bytes_launch = float(bytes_sum) / steps
    mean_stepped = stepped / steps
    bytes_env = float(bytes_sum) / stepped
    k_ms = kernel_ms[med]
    kernel = "b3k_step_art<false>" if art else kernel_name(scene, count)
    hbm_gbs = bytes_launch / (k_ms * 1e-3) / 1e9
    flops_env, counted = counted_flops(scene, start, steps)
    tflops = flops_env * mean_stepped / (k_ms * 1e-3) / 1e12
    counters = load_counters(kernel, scene, count, digest, start, end)
    traffic = None
    if counters:
        traffic = counters["fetch_bytes_per_launch"] + counters["write_bytes_per_launch"]
    roofline = {"bound": "hbm", "achieved": round(hbm_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(hbm_gbs / HBM_PEAK_GBS, 5), "traffic": traffic,
                "kernel": kernel, "kernel_ms": round(k_ms, 5), "kernel_launches_timed": len(timed),
                "window": [start, end],
                "bytes_per_launch": round(bytes_launch, 1),
                "bytes_per_env_step": round(bytes_env, 1),
                "mean_contacts_per_world": round(float(contact_sum) / steps, 2),
                "mean_stepped_worlds": round(mean_stepped, 1),
                "valu": {"achieved": round(tflops, 3), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops / FP32_PEAK_TFLOPS, 5),
                         "frac_nonpacked": round(tflops / FP32_NONPACKED_TFLOPS, 5),
                         "flops_per_env_step": round(flops_env, 1), "counted_steps": counted,
                         "source": "tests/golden/flops.json (oracle fp32 operations counted on the workload)"}}
    if art:
        # the counted flops are the independent-body step's: no VALU figure
        roofline["valu"] = {"note": "tests/golden/flops.json counts the independent-body step, not this one"}
    # the lower of the two ceilings, and the fraction of it reached
    ceil_hbm = HBM_PEAK_GBS * 1e9 / bytes_env
    ceil_valu = float("inf") if art else FP32_PEAK_TFLOPS * 1e12 / flops_env
    attainable = min(ceil_hbm, ceil_valu)
    roofline["attainable_env_steps_per_s"] = round(attainable, 1)
    roofline["binding"] = "hbm" if ceil_hbm <= ceil_valu else "valu"
    roofline["attainable_frac"] = round(rates[med] / attainable, 5)
    if traffic:
        roofline["traffic_gbs"] = round(traffic / (k_ms * 1e-3) / 1e9, 1)
        roofline["traffic_frac"] = round(traffic / (k_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        roofline["traffic_profile"] = "profiles/counters_%s%d.json" % (NAMES[scene], count)
        roofline["traffic_window"] = counters["window"]
    else:
        roofline["traffic_note"] = ("no rocprofv3 counter profile of this source tree (%s) over a window inside "
                                    "[%d, %d) in profiles/" % (digest, start, end))
    masks = "2% reset / 90% step" if scene == 5 else ("impulse every 60 steps" if scene == 2 else "none")
    config = {"workload": "%s%d: %d worlds of the %s scene, dt %.6g, %d substeps, masks %s" % (
                  NAMES[scene], count, count, NAMES[scene], sc.dt, sc.substeps, masks),
              "worlds": count, "scene": NAMES[scene], "dt": sc.dt, "substeps": sc.substeps, "repeats": repeats,
              "window": [start, end], "settled_untimed": settle}
    if art:
        config["contacts"] = "articulated (B3_ENGINE_ART_CONTACTS: the reference's B3_ART_CONTACTS=1 step)"
    out = {"value": round(rates[med], 1), "unit": "env-steps/s", "steps": steps, "warmup": start - settle,
           "ms_per_step": round(ms[med], 5), "config": config, "roofline": roofline,
           "repeat_values": [round(v, 1) for v in rates]}
    if cpu_seconds:
        log("%s%d: cpu baseline from vector step %d" % (NAMES[scene], count, start))
        out["cpu_baseline"] = cpu_baseline(scene, count, state_at_start, worlds, start, end, cpu_seconds)
        out["gpu_over_cpu"] = round(out["value"] / out["cpu_baseline"]["value"], 1)
    return out


def run_hover_env(n, steps, warmup, repeats):
    """The PufferLib hover environment on the engine (include/b3_hover.h,
    puffysics_amd/hover.py): env-steps/s of its vector step (actions to
    forces, the engine step with the previous step's terminals reset, then
    observations, rewards and terminals), with the trainer's action write
    (a device copy of pre-drawn actions in [-1, 1]) inside each timed step."""
    import torch
    from puffysics_amd.hover import HoverEnvs
    env = HoverEnvs(n, seed=1)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1)
    acts = torch.rand((warmup + steps, n), generator=gen, device="cuda") * 2.0 - 1.0
    stream = torch.cuda.current_stream()
    rates, ms = [], []
    for r in range(repeats):
        env.reset()
        for i in range(warmup):
            env.actions.copy_(acts[i])
            env.step()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(steps):
            env.actions.copy_(acts[warmup + i])
            env.step()
        b.record(stream)
        torch.cuda.synchronize()
        el = a.elapsed_time(b)
        rates.append(n * steps / (el * 1e-3))
        ms.append(el / steps)
        log("  hover env repeat %d: %.4f ms/step, %.4g env-steps/s" % (r, ms[-1], rates[-1]))
    stats = env.log()
    env.close()
    med = sorted(range(repeats), key=lambda i: rates[i])[repeats // 2]
    return {"metric": "hover env-steps/sec (PufferLib adapter on the engine), 1 MI355X", "value": round(rates[med], 1),
            "unit": "env-steps/s", "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(ms[med], 5),
            "higher_is_better": True, "dtype": "f32", "data": "synthetic (seeded envs, pre-drawn uniform actions)",
            "config": {"workload": "hover env: %d envs, one vector step = actions, physics step with resets, "
                                   "observations" % n, "envs": n, "repeats": repeats},
            "repeat_values": [round(v, 1) for v in rates], "episodes_logged": stats.get("n")}


# ---- rocprofv3 summaries of the step kernel over the timed window ----
# Each profile run is `bench.py --scene N --no-cpu` with the same --steps,
# --warmup and --repeats under rocprofv3 (one run per counter set, as the
# tool collects no more than one hardware pass at a time).  The step kernel
# is launched once per vector step in the bench's fixed order (settling,
# then per repeat the warm-up and the timed window, then the byte model's
# pass), so its timed launches are known by their position.

PROFILE_RUNS = [("trace", "--kernel-trace --stats"),
                ("fetch", "--pmc FETCH_SIZE"),
                ("write", "--pmc WRITE_SIZE"),
                ("sq1", "--pmc SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_INSTS_VALU SQ_ACTIVE_INST_VALU SQ_INSTS_LDS "
                        "SQ_LDS_BANK_CONFLICT SQ_INSTS_VMEM_RD"),
                ("sq2", "--pmc SQ_INSTS_VMEM_WR SQ_INSTS_SALU SQ_WAIT_INST_ANY SQ_ACTIVE_INST_ANY "
                        "SQ_INST_CYCLES_VMEM_RD GRBM_GUI_ACTIVE")]
COPY_MIB = 1024


def timed_step_launches(scene, steps, warmup, repeats):
    """Positions, among a bench run's step-kernel launches, of the timed ones."""
    settle, start, end = window_of(scene, steps, warmup)
    w = start - settle
    out = []
    for r in range(repeats):
        first = settle + r * (w + steps) + w
        out.extend(range(first, first + steps))
    return out


def profile_commands(scene, steps, warmup, repeats, outdir):
    bench = "python3 bench.py --scene %d --no-cpu --steps %d --warmup %d --repeats %d" % (scene, steps, warmup,
                                                                                          repeats)
    cmds = []
    for name, opts in PROFILE_RUNS:
        flt = "" if name == "trace" else " --kernel-include-regex b3k_step"
        cmds.append("timeout -s KILL 300 rocprofv3 %s%s -d %s/%s -o run -f csv -- %s" % (opts, flt, outdir, name,
                                                                                          bench))
    for name, counter in (("copy_fetch", "FETCH_SIZE"), ("copy_write", "WRITE_SIZE")):
        cmds.append("timeout -s KILL 120 rocprofv3 --pmc %s -d %s/%s -o run -f csv -- python3 bench.py "
                    "--copy-calibration %d" % (counter, outdir, name, COPY_MIB))
    return cmds


def _csv_rows(d, suffix):
    import csv
    import glob
    paths = sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True))
    if not paths:
        raise SystemExit("no %s under %s" % (suffix, d))
    with open(paths[0], newline="") as f:
        return list(csv.DictReader(f))


def _short(name):
    name = name.replace("(anonymous namespace)::", "").replace("void ", "")
    return name.split("(")[0] if name.startswith("b3k_") else name[:150]


def _step_kernel(names):
    """The workload's step kernel: the launched kernel named b3k_step<JI> or
    b3k_step_shared<...>."""
    cands = [n for n in names if _short(n).startswith("b3k_step<") or _short(n).startswith("b3k_step_shared<")]
    if len(set(cands)) != 1:
        raise SystemExit("expected one step kernel, found %s" % sorted(set(cands)))
    return cands[0]


def _counter_means(rows, picks):
    """Per-counter mean over the step kernel's launches at positions `picks`."""
    step = _step_kernel({r["Kernel_Name"] for r in rows})
    by_dispatch = {}
    for r in rows:
        if r["Kernel_Name"] == step:
            by_dispatch.setdefault(int(r["Dispatch_Id"]), {})[r["Counter_Name"]] = float(r["Counter_Value"])
    order = sorted(by_dispatch)
    sel = [by_dispatch[order[i]] for i in picks]
    names = sorted({k for d in sel for k in d})
    return {k: sum(d[k] for d in sel) / len(sel) for k in names}, len(order)


def code_object_resources(kernel):
    """Registers and static memory of a kernel (its short name) from the
    AMDGPU metadata notes of the gfx950 code object in the in-tree
    puffysics_amd/libb3engine.so (llvm-readelf --notes of the object that
    clang-offload-bundler takes out of the library's .hip_fatbin section);
    None when the tools or the kernel are missing.  .vgpr_count counts the
    AGPRs too."""
    import subprocess
    import tempfile
    llvm = "/opt/rocm/llvm/bin"
    lib = os.path.join(ROOT, "puffysics_amd", "libb3engine.so")
    try:
        with tempfile.TemporaryDirectory() as tmp:
            fat, co = os.path.join(tmp, "fat.bin"), os.path.join(tmp, "co.elf")
            subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", lib, fat], check=True)
            subprocess.run([os.path.join(llvm, "clang-offload-bundler"), "--unbundle", "--type=o",
                            "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", "--input=" + fat, "--output=" + co],
                           check=True)
            notes = subprocess.run([os.path.join(llvm, "llvm-readelf"), "--notes", co], check=True,
                                   capture_output=True, text=True).stdout
    except (OSError, subprocess.CalledProcessError):
        return None
    blocks, cur = [], None
    for line in notes.splitlines():
        t = line.strip()
        if t.startswith("- .agpr_count:"):
            cur = {}
            blocks.append(cur)
            t = t[2:]
        if cur is not None and t.startswith(".") and ":" in t:
            k, v = t.split(":", 1)
            cur[k[1:]] = v.strip()
    names = [b.get("name", "") for b in blocks]
    try:
        dem = subprocess.run(["c++filt"], input="\n".join(names), check=True,
                             capture_output=True, text=True).stdout.splitlines()
    except (OSError, subprocess.CalledProcessError):
        return None
    for b, d in zip(blocks, dem):
        if _short(d) == kernel:
            return {"vgpr_total": int(b["vgpr_count"]), "agpr": int(b["agpr_count"]), "sgpr": int(b["sgpr_count"]),
                    "lds_static_bytes": int(b["group_segment_fixed_size"]),
                    "scratch_bytes": int(b["private_segment_fixed_size"])}
    return None


def profile_summary(root, scene, count, steps, warmup, repeats, digest):
    """Writes profiles/<kernel>_<workload>.md and profiles/counters_<workload>.json
    from the runs of profile_commands under `root`."""
    settle, start, end = window_of(scene, steps, warmup)
    picks = timed_step_launches(scene, steps, warmup, repeats)
    trace = _csv_rows(os.path.join(root, "trace"), "kernel_trace.csv")
    step = _step_kernel({r["Kernel_Name"] for r in trace})
    launches = sorted((r for r in trace if r["Kernel_Name"] == step), key=lambda r: int(r["Dispatch_Id"]))
    expect = settle + (repeats + 1) * (start - settle + steps)
    if len(launches) != expect:
        raise SystemExit("%d step launches traced, the bench's plan has %d" % (len(launches), expect))
    dur = [(int(launches[i]["End_Timestamp"]) - int(launches[i]["Start_Timestamp"])) / 1e3 for i in picks]
    avg_us = sum(dur) / len(dur)
    # every kernel over the timed repeats' span of time
    spans = []
    for r in range(repeats):
        a, b = picks[r * steps], picks[r * steps + steps - 1]
        spans.append((int(launches[a]["Start_Timestamp"]), int(launches[b]["End_Timestamp"])))
    table = {}
    for row in trace:
        t0, t1 = int(row["Start_Timestamp"]), int(row["End_Timestamp"])
        if any(a <= t0 and t1 <= b for a, b in spans):
            table.setdefault(_short(row["Kernel_Name"]), []).append((t1 - t0) / 1e3)
    fetch, nf = _counter_means(_csv_rows(os.path.join(root, "fetch"), "counter_collection.csv"), picks)
    write, _ = _counter_means(_csv_rows(os.path.join(root, "write"), "counter_collection.csv"), picks)
    sq = {}
    for name in ("sq1", "sq2"):
        sq.update(_counter_means(_csv_rows(os.path.join(root, name), "counter_collection.csv"), picks)[0])
    copy_bytes = COPY_MIB << 20
    scale = {}
    for name, counter in (("copy_fetch", "FETCH_SIZE"), ("copy_write", "WRITE_SIZE")):
        rows = [r for r in _csv_rows(os.path.join(root, name), "counter_collection.csv")
                if r["Counter_Name"] == counter and float(r["Counter_Value"]) > 0]
        kib = sorted(float(r["Counter_Value"]) for r in rows)[len(rows) // 2]
        scale[counter] = round(copy_bytes / (kib * 1024), 3)
    fetch_b = fetch["FETCH_SIZE"] * 1024 * scale["FETCH_SIZE"]
    write_b = write["WRITE_SIZE"] * 1024 * scale["WRITE_SIZE"]
    l0 = launches[0]
    kernel = _short(step)
    regs = code_object_resources(kernel)
    if regs is None:
        raise SystemExit("no code-object metadata for %s in puffysics_amd/libb3engine.so" % kernel)
    regs.update(wg=int(l0["Workgroup_Size_X"]), grid=int(l0["Grid_Size_X"]))
    workload = "%s%d" % (NAMES[scene], count)
    counters = {"kernel": kernel.replace(",", ", ").replace(",  ", ", "),
                "workload": workload, "source_digest": digest, "window": [start, start + steps],
                "timed_launches": len(picks), "launches_profiled": nf,
                "fetch_bytes_per_launch": round(fetch_b), "write_bytes_per_launch": round(write_b),
                "trace_avg_us": round(avg_us, 2), "fetch_scale": scale["FETCH_SIZE"],
                "write_scale": scale["WRITE_SIZE"], "sq": {k: round(v, 1) for k, v in sq.items()}, "registers": regs}
    os.makedirs(os.path.join(ROOT, "profiles"), exist_ok=True)
    with open(os.path.join(ROOT, "profiles", "counters_%s.json" % workload), "w") as f:
        json.dump(counters, f, indent=1)
        f.write("\n")
    cmds = profile_commands(scene, steps, warmup, repeats, "gpurun_out/prof_%s" % workload)
    tag = kernel.replace("<", "_").replace(">", "").replace(", ", "_").replace(",", "_")
    lines = ["# %s on the %s workload (%d worlds), one MI355X" % (kernel, NAMES[scene], count), "",
             "Source digest `%s` (`bench.engine_source_digest()`: the engine sources this profile was taken of)."
             % digest, "",
             "Commands (each its own run, from the repository root, with `export TMPDIR=/tmp` for the tool), then "
             "this summary:", ""]
    lines += ["    " + c for c in cmds]
    lines += ["    python3 bench.py --profile-summary gpurun_out/prof_%s --scene %d --steps %d --warmup %d "
              "--repeats %d" % (workload, scene, steps, warmup, repeats), "",
              "Every run is the bench's own run of this workload: settled untimed to vector step %d, then per "
              "repeat %d untimed warm-up steps and the timed window of vector steps %d..%d, all %d repeats from the "
              "same saved state, then one more pass of the window for the byte model.  The figures below are the "
              "step kernel's %d launches inside the timed windows (positions known from that order; %d launches "
              "of it in all)." % (settle, start - settle, start, start + steps, repeats, len(picks), len(launches)),
              "", "## Kernel trace, timed windows", "",
              "| kernel | calls | avg us | min us | max us |", "|---|---|---|---|---|"]
    for name, d in sorted(table.items(), key=lambda kv: -sum(kv[1])):
        lines.append("| %s | %d | %.2f | %.2f | %.2f |" % (name, len(d), sum(d) / len(d), min(d), max(d)))
    wc = sq.get("SQ_WAVE_CYCLES", 0) or 1
    lines += ["", "Step kernel over its timed launches: **%.2f us** average." % avg_us, "",
              "## Counters of `%s` (mean per timed launch)" % kernel, "",
              "Registers (the AMDGPU metadata of the kernel in the gfx950 code object of "
              "puffysics_amd/libb3engine.so, `llvm-readelf --notes`): %d VGPRs in all, %d of them AGPRs, %d SGPRs; "
              "static LDS %d bytes (the step's LDS is dynamic, sized at launch), private segment %d bytes; "
              "workgroup %d threads, grid %d (the dispatch records)." % (
                  regs["vgpr_total"], regs["agpr"], regs["sgpr"], regs["lds_static_bytes"], regs["scratch_bytes"],
                  regs["wg"], regs["grid"]), "",
              "| counter | value |", "|---|---|"]
    for k in sorted(sq):
        lines.append("| %s | %.4g |" % (k, sq[k]))
    lines += ["| FETCH_SIZE (KiB) | %.4g |" % fetch["FETCH_SIZE"], "| WRITE_SIZE (KiB) | %.4g |" % write["WRITE_SIZE"],
              "", "## Derived", "",
              "- HBM bytes per launch: fetch %.3g + write %.3g = %.3g B, each counter scaled by what it reads for "
              "a plain %d MiB device copy (x%.3f fetch, x%.3f write). Over the %.2f us average: %.0f GB/s, %.1f%% "
              "of 8 TB/s." % (fetch_b, write_b, fetch_b + write_b, COPY_MIB, scale["FETCH_SIZE"],
                              scale["WRITE_SIZE"], avg_us, (fetch_b + write_b) / (avg_us * 1e-6) / 1e9,
                              (fetch_b + write_b) / (avg_us * 1e-6) / 1e9 / 80.0),
              "- VALU active %.1f%% and any instruction active %.1f%% of wave cycles (SQ_ACTIVE_INST_VALU, "
              "SQ_ACTIVE_INST_ANY over SQ_WAVE_CYCLES); waiting on any instruction %.1f%%." % (
                  100 * sq.get("SQ_ACTIVE_INST_VALU", 0) / wc, 100 * sq.get("SQ_ACTIVE_INST_ANY", 0) / wc,
                  100 * sq.get("SQ_WAIT_INST_ANY", 0) / wc),
              "- Waves %d; VALU instructions per wave %.3g; LDS instructions %.3g with %.0f bank-conflict cycles."
              % (sq.get("SQ_WAVES", 0), sq.get("SQ_INSTS_VALU", 0) / max(1.0, sq.get("SQ_WAVES", 1)),
                 sq.get("SQ_INSTS_LDS", 0), sq.get("SQ_LDS_BANK_CONFLICT", 0)), ""]
    path = os.path.join(ROOT, "profiles", "%s_%s.md" % (tag, workload))
    with open(path, "w") as f:
        f.write("\n".join(lines))
    log("wrote %s and profiles/counters_%s.json" % (os.path.relpath(path, ROOT), workload))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed vector steps per repeat of every workload (default: from the window start to the "
                         "end of the benchmark run: 500; 1000 for the bin)")
    ap.add_argument("--warmup", type=int, default=50,
                    help="untimed vector steps before each repeat's window (after settling to the window start "
                         "less these)")
    ap.add_argument("--repeats", type=int, default=3)
    ap.add_argument("--event-every", type=int, default=8, metavar="N",
                    help="time every N-th step launch with a pair of HIP events (each pair is a gap in the "
                         "stream: on the small scenes, timing every launch costs up to 15%% of the throughput)")
    ap.add_argument("--scene", type=int, default=0, help="only this workload (1-5)")
    ap.add_argument("--worlds", type=int, default=0, help="with --scene: another world count")
    ap.add_argument("--cpu-seconds", type=float, default=5.0, help="timed CPU work per workload")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only copy MIB MiB device-to-device 10 times with a plain copy kernel (for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    ap.add_argument("--profile-commands", metavar="DIR",
                    help="with --scene: print the rocprofv3 runs whose outputs --profile-summary reads, and exit")
    ap.add_argument("--art", action="store_true",
                    help="with --scene: the step with articulated contacts (B3_ENGINE_ART_CONTACTS), no CPU leg")
    ap.add_argument("--hover-env", type=int, default=0, metavar="N",
                    help="the PufferLib hover adapter's vector step on N envs, one JSON line, and exit")
    ap.add_argument("--profile-summary", metavar="DIR",
                    help="with --scene: summarise those runs under DIR into profiles/ and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_per_launch": n * 4}))
        return
    if args.gpus != 1:
        print("bench.py: the engine runs on one GPU; worlds are independent and would shard by world index "
              "with no exchange, but only --gpus 1 is measured here", file=sys.stderr)
        sys.exit(2)

    def steps_of(scene):
        return args.steps if args.steps is not None else RUN_LENGTH[scene] - WINDOW_START[scene]

    if args.profile_commands or args.profile_summary:
        if not args.scene:
            raise SystemExit("--profile-commands / --profile-summary need --scene")
        from puffysics_amd import scenes
        count = args.worlds or scenes.SCENES[args.scene].worlds
        if args.profile_commands:
            print("\n".join(profile_commands(args.scene, steps_of(args.scene), args.warmup, args.repeats,
                                             args.profile_commands)))
        else:
            profile_summary(args.profile_summary, args.scene, count, steps_of(args.scene), args.warmup,
                            args.repeats, engine_source_digest())
        return

    import torch
    from puffysics_amd import scenes
    torch.cuda.set_device(0)
    if args.hover_env:
        steps = args.steps if args.steps is not None else 1000
        print(json.dumps(run_hover_env(args.hover_env, steps, args.warmup, args.repeats)), flush=True)
        return
    if args.art and not args.scene:
        raise SystemExit("--art needs --scene")
    digest = engine_source_digest()
    todo = [args.scene] if args.scene else [1, 2, 3, 4, 5]
    results = {}
    for scene in todo:
        count = (args.worlds if args.scene and args.worlds else scenes.SCENES[scene].worlds)
        res = run_workload(scene, count, steps_of(scene), args.warmup, args.repeats, args.event_every, digest,
                           None if args.no_cpu or args.art else args.cpu_seconds, art=args.art)
        results["%s%d" % (NAMES[scene], count)] = (scene, count, res)
    head_key = next((k for k, v in results.items() if v[0] == HEADLINE), next(iter(results)))
    head = results[head_key][2]
    out = {"metric": METRIC, "value": head["value"], "unit": "env-steps/s", "n_gpus": 1, "steps": head["steps"],
           "warmup": head["warmup"], "ms_per_step": head["ms_per_step"], "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "f32",
           "data": "synthetic (seeded scene builders, counter-based per-step inputs)",
           "config": head["config"], "roofline": head["roofline"], "cpu_baseline": head.get("cpu_baseline"),
           "engine_source_digest": digest,
           "configs": {k: v[2] for k, v in results.items()}}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
