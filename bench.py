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
(substeps not counted).  Each workload runs W untimed vector steps, then K
timed ones per repeat (default: 50, then 1000; 2000 for the bin; 3
repeats, median).  The step kernel's own duration is timed with HIP events
on its stream around every 8th launch.

Per workload:
  roofline   algorithmic bytes per launch (the byte model below on the live
             contact counts) / kernel time, against 8 TB/s; counted flops per
             launch (tests/golden/flops.json: the oracle's fp32 operations
             on the same workload) / kernel time, against the fp32 vector
             peak (157.3 TFLOP/s with packed FMA, 78.6 without); measured HBM
             bytes (rocprofv3 FETCH_SIZE / WRITE_SIZE in profiles/) only
             when that profile was taken of this source tree.
  cpu        the reference's own CPU path (b3_batch_step / b3_batch_restore,
             oracle/_ref) built -O3 for this host's x86-64 level, one pinned
             thread per physical core available to the process, on the
             workload's full world count over a bounded number of steps.
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


def kernel_name(scene, count):
    """The step kernel a batch launches: b3k_step_shared<Masks, JL> when its
    tiles fit one per CU (b3_engine_create), else b3k_step."""
    import torch
    from puffysics_amd import scenes
    tiles = (count + 63) // 64
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if tiles > cus:
        return "b3k_step"
    caps = scenes.SCENES[scene].caps
    masks = 12 <= caps[1] <= 64
    return "b3k_step_shared<%s, %s>" % ("true" if masks else "false", "true" if joint_rows_fit(*caps) else "false")


def load_counters(kernel, scene, count, digest):
    """Per-launch counter figures of a kernel on a workload from the committed
    rocprofv3 summary, if it was taken of this source tree; else None."""
    path = os.path.join(ROOT, "profiles", "counters_%s%d.json" % (NAMES[scene], count))
    if not os.path.exists(path):
        return None
    with open(path) as f:
        c = json.load(f)
    if c.get("source_digest") != digest or c.get("kernel") != kernel:
        return None
    return c


def cpu_baseline(scene, count, warmup, seconds):
    """The reference's CPU path on the workload's worlds: `warmup` untimed
    vector steps, then as many as fit in about `seconds` (at least 3)."""
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
    if lib is not None:
        kind = "reference"
        ws = lib.ref_world_size()
        worlds = np.zeros(count * ws, np.uint8)
        lib.ref_build_batch(scene, worlds.ctypes.data, count, scenes.SEED, 0)
        initial = worlds.copy()

        def run(t0, n):
            return lib.ref_run(scene, worlds.ctypes.data, initial.ctypes.data, count, scenes.SEED, t0, n, sc.dt,
                               sc.substeps, nthreads, cpu_arr)
    else:
        kind, flags = "port", "-O2 -ffp-contract=off -fno-fast-math"
        worlds = scenes.build(scene, count)
        initial = worlds.copy()
        fn = getattr(oracle(), "ocpu_run_%d" % scene)

        def run(t0, n):
            return fn(worlds.ctypes.data, initial.ctypes.data, count, scenes.SEED, t0, n, sc.dt, sc.substeps,
                      nthreads, cpu_arr)
    if warmup:
        run(0, warmup)
    t0 = time.perf_counter()
    done = run(warmup, 1)
    first = time.perf_counter() - t0
    nsteps = int(max(3, min(2000, seconds / max(first, 1e-6))))
    t0 = time.perf_counter()
    env_steps = run(warmup + 1, nsteps)
    el = time.perf_counter() - t0
    del done
    return {"value": round(env_steps / el, 1), "unit": "env-steps/s", "cores": nthreads, "kind": kind,
            "flags": flags, "affinity_physical_cores": affinity_cores, "cgroup_cpu_quota": quota,
            "sample": "all %d worlds, vector steps %d..%d of the same workload (after %d untimed), %d pinned threads "
                      "(one per physical core available), %.1f s" % (count, warmup + 1, warmup + nsteps, warmup + 1,
                                                                     nthreads, el)}


def run_workload(scene, count, steps, warmup, repeats, event_every, digest):
    import numpy as np
    import torch
    from puffysics_amd import scenes
    from puffysics_amd.engine import B3Engine

    sc = scenes.SCENES[scene]
    log("%s: building %d worlds" % (NAMES[scene], count))
    worlds = scenes.build(scene, count)
    eng = B3Engine(worlds, sc.sig)
    stream = torch.cuda.current_stream()
    total = warmup + steps * repeats
    reset = torch.empty((total, count), dtype=torch.uint8, device="cuda")
    stepm = torch.empty((total, count), dtype=torch.uint8, device="cuda")
    for t in range(total):
        eng.scene_masks(scene, scenes.SEED, t, reset[t], stepm[t])
    step_counts = stepm.sum(dim=1, dtype=torch.int64).cpu().numpy()
    reset_any = reset.amax(dim=1).cpu().numpy()

    for t in range(warmup):
        if reset_any[t]:
            eng.restore(reset[t])
        eng.scene_inputs(scene, scenes.SEED, t, stepm[t])
        eng.step(sc.dt, sc.substeps, stepm[t])
    torch.cuda.synchronize()

    rates, ms, kernel_ms = [], [], []
    t = warmup
    timed = range(0, steps, max(1, event_every))
    for r in range(repeats):
        k_start = {i: torch.cuda.Event(enable_timing=True) for i in timed}
        k_end = {i: torch.cuda.Event(enable_timing=True) for i in timed}
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        t_begin = t
        for i in range(steps):
            if reset_any[t]:
                eng.restore(reset[t])
            eng.scene_inputs(scene, scenes.SEED, t, stepm[t])
            if i in k_start:
                k_start[i].record(stream)
            eng.step(sc.dt, sc.substeps, stepm[t])
            if i in k_end:
                k_end[i].record(stream)
            t += 1
        end.record(stream)
        torch.cuda.synchronize()
        el_ms = start.elapsed_time(end)
        env = int(step_counts[t_begin:t].sum())
        rates.append(env / (el_ms * 1e-3))
        ms.append(el_ms / steps)
        kernel_ms.append(sum(k_start[i].elapsed_time(k_end[i]) for i in timed) / len(timed))
        log("  repeat %d: %.4f ms/step, %.4g env-steps/s, step kernel %.4f ms" % (r, ms[-1], rates[-1],
                                                                                 kernel_ms[-1]))
    med = sorted(range(repeats), key=lambda i: rates[i])[repeats // 2]

    st = eng.stats()
    eng.close()
    per_world = world_bytes_model(worlds, st["contact_count"])
    mean_stepped = float(step_counts[warmup:].mean())
    k_ms = kernel_ms[med]
    kernel = kernel_name(scene, count)
    bytes_env = float(per_world.mean())
    hbm_gbs = bytes_env * mean_stepped / (k_ms * 1e-3) / 1e9
    # the median repeat's window of vector steps
    first = warmup + med * steps
    flops_env, window = counted_flops(scene, first, steps)
    tflops = flops_env * mean_stepped / (k_ms * 1e-3) / 1e12
    counters = load_counters(kernel, scene, count, digest)
    traffic = None
    if counters:
        traffic = counters["fetch_bytes_per_launch"] + counters["write_bytes_per_launch"]
    roofline = {"bound": "hbm", "achieved": round(hbm_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(hbm_gbs / HBM_PEAK_GBS, 5), "traffic": traffic,
                "kernel": kernel, "kernel_ms": round(k_ms, 5), "kernel_launches_timed": len(timed),
                "bytes_per_env_step": round(bytes_env, 1),
                "mean_contacts_per_world": round(float(st["contact_count"].mean()), 2),
                "mean_stepped_worlds": round(mean_stepped, 1),
                "valu": {"achieved": round(tflops, 3), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops / FP32_PEAK_TFLOPS, 5),
                         "frac_nonpacked": round(tflops / FP32_NONPACKED_TFLOPS, 5),
                         "flops_per_env_step": round(flops_env, 1), "counted_steps": window,
                         "source": "tests/golden/flops.json (oracle fp32 operations counted on the workload)"}}
    # the lower of the two ceilings, and the fraction of it reached
    ceil_hbm = HBM_PEAK_GBS * 1e9 / bytes_env
    ceil_valu = FP32_PEAK_TFLOPS * 1e12 / flops_env
    attainable = min(ceil_hbm, ceil_valu)
    roofline["attainable_env_steps_per_s"] = round(attainable, 1)
    roofline["binding"] = "hbm" if ceil_hbm <= ceil_valu else "valu"
    roofline["attainable_frac"] = round(rates[med] / attainable, 5)
    if traffic:
        roofline["traffic_gbs"] = round(traffic / (k_ms * 1e-3) / 1e9, 1)
        roofline["traffic_frac"] = round(traffic / (k_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        roofline["traffic_profile"] = "profiles/counters_%s%d.json" % (NAMES[scene], count)
    else:
        roofline["traffic_note"] = "no rocprofv3 counter profile of this source tree (%s) in profiles/" % digest
    masks = "2% reset / 90% step" if scene == 5 else ("impulse every 60 steps" if scene == 2 else "none")
    config = {"workload": "%s%d: %d worlds of the %s scene, dt %.6g, %d substeps, masks %s" % (
                  NAMES[scene], count, count, NAMES[scene], sc.dt, sc.substeps, masks),
              "worlds": count, "scene": NAMES[scene], "dt": sc.dt, "substeps": sc.substeps, "repeats": repeats}
    return {"value": round(rates[med], 1), "unit": "env-steps/s", "steps": steps, "warmup": warmup,
            "ms_per_step": round(ms[med], 5), "config": config, "roofline": roofline,
            "repeat_values": [round(v, 1) for v in rates]}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed vector steps per repeat of every workload (default: 1000; 2000 for the bin)")
    ap.add_argument("--warmup", type=int, default=50)
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

    import torch
    from puffysics_amd import scenes
    torch.cuda.set_device(0)
    digest = engine_source_digest()
    todo = [args.scene] if args.scene else [1, 2, 3, 4, 5]
    results = {}
    for scene in todo:
        count = (args.worlds if args.scene and args.worlds else scenes.SCENES[scene].worlds)
        steps = args.steps if args.steps is not None else (2000 if scene == 4 else 1000)
        res = run_workload(scene, count, steps, args.warmup, args.repeats, args.event_every, digest)
        results["%s%d" % (NAMES[scene], count)] = (scene, count, res)
    if not args.no_cpu:
        for key, (scene, count, res) in results.items():
            log("%s: cpu baseline" % key)
            res["cpu_baseline"] = cpu_baseline(scene, count, args.warmup, args.cpu_seconds)
            res["gpu_over_cpu"] = round(res["value"] / res["cpu_baseline"]["value"], 1)
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
