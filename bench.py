"""Physics-only env-steps/s of the batched stepping engine on one MI355X.

Workload (default): the arm scene at 65,536 worlds: each world is a ground
box, a 4-link hinged capsule arm (motors, limits, random torques) and 12
free spheres / boxes; every vector step draws a 2% reset mask and a 90% step
mask; dt 1/60, 4 substeps.  One vector step = masked restore + scene inputs
(forces / torques) + masked step, all on one HIP stream; an env-step is one
world stepped (substeps are not counted).  Masks for every step are drawn
on the device before the timed region; the worlds stay resident in HBM.

Prints one JSON line with the throughput, the roofline of the step kernel
(algorithmic bytes per launch / its event-timed average duration, against
8 TB/s; with the committed counter summary of the workload, also its HBM
traffic and its VALU issue rate against the fp32 vector rate) and a CPU
baseline: the reference's own CPU path compiled from its sources
(oracle/_ref) when present, else the oracle, on a bounded sample of the
same workload with one thread per physical core.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "physics env-steps/sec at 4096 and 65536 worlds, 1 MI355X; % HBM/VALU roofline"
HBM_PEAK_GBS = 8000.0
# fp32 vector issue rate: 256 CUs x 4 SIMDs x 16 lanes x 2.4 GHz (an FMA would count twice; the
# step is built without contraction)
VALU_PEAK_TLANE = 39.32
VALU_FP32_PEAK_TFLOPS = 157.3

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


def physical_cpus(limit):
    """One logical CPU per physical core, among those this process may use."""
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
    return cpus[:limit]


def world_bytes_model(worlds, contacts):
    """Per-world algorithmic bytes of one step, given live contact counts."""
    import numpy as np
    b = worlds["bodies"]
    live = np.arange(b.shape[1])[None, :] < worlds["body_count"][:, None]
    n_dyn = ((b["type"] == 2) & live).sum(axis=1)
    n_static = live.sum(axis=1) - n_dyn
    return (BYTES_DYNAMIC_BODY * n_dyn + BYTES_STATIC_BODY * n_static + BYTES_SHAPE * worlds["shape_count"]
            + BYTES_CONTACT * contacts + BYTES_JOINT * worlds["joint_count"] + BYTES_WORLD).astype(np.float64)


def cpu_baseline(scene, seconds_target, threads_limit):
    """Time the reference CPU path (or the oracle) on a bounded sample."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from b3test import oracle, ref_lib
    from puffysics_amd import scenes
    sc = scenes.SCENES[scene]
    cpus = physical_cpus(threads_limit)
    nthreads = max(1, len(cpus))
    cpu_arr = (C.c_int * nthreads)(*cpus) if cpus else None
    ref = ref_lib(scene)
    count = 512 * nthreads
    if ref is not None:
        kind = "reference"
        ws = ref.ref_world_size()
        worlds = np.zeros(count * ws, np.uint8)
        ref.ref_build_batch(scene, worlds.ctypes.data, count, scenes.SEED, 0)
        initial = worlds.copy()

        def run(t0, n):
            return ref.ref_run(scene, worlds.ctypes.data, initial.ctypes.data, count, scenes.SEED, t0, n, sc.dt,
                               sc.substeps, nthreads, cpu_arr)
    else:
        kind = "port"
        worlds = scenes.build(scene, count)
        initial = worlds.copy()
        fn = getattr(oracle(), "ocpu_run_%d" % scene)

        def run(t0, n):
            return fn(worlds.ctypes.data, initial.ctypes.data, count, scenes.SEED, t0, n, sc.dt, sc.substeps,
                      nthreads, cpu_arr)
    run(0, 5)  # warm caches and page in
    t0 = time.perf_counter()
    done = run(5, 5)
    per_step = (time.perf_counter() - t0) / 5
    nsteps = max(5, min(800, int(seconds_target / max(per_step, 1e-6))))
    t0 = time.perf_counter()
    env_steps = run(10, nsteps)
    el = time.perf_counter() - t0
    del done
    return {"value": env_steps / el, "unit": "env-steps/s", "cores": nthreads, "kind": kind,
            "sample": "%d worlds x %d vector steps (steps 10..%d) of the same workload, %d pinned threads, "
                      "%.1f s" % (count, nsteps, 9 + nsteps, nthreads, el)}


def load_counters(scene, worlds):
    """Per-launch counter figures of the step kernel from a committed rocprofv3
    summary (HBM bytes, VALU instructions), or {}."""
    path = os.path.join(ROOT, "profiles", "b3k_step_%s%d_traffic.json" % (scene, worlds))
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--repeats", type=int, default=3)
    ap.add_argument("--event-every", type=int, default=8, metavar="N",
                    help="time every N-th step launch of the timed region with a pair of HIP events (each pair "
                         "is a gap in the stream: on the small scenes, timing every launch costs up to 15%% "
                         "of the throughput)")
    ap.add_argument("--scene", type=int, default=5)
    ap.add_argument("--worlds", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--art", action="store_true",
                    help="step with articulation-aware contacts (B3_ENGINE_ART_CONTACTS); not the headline mode")
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

    import numpy as np
    import torch
    from puffysics_amd import scenes
    from puffysics_amd.engine import B3Engine

    sc = scenes.SCENES[args.scene]
    count = args.worlds or sc.worlds
    torch.cuda.set_device(0)
    log("building %d %s worlds" % (count, sc.name))
    worlds = scenes.build(args.scene, count)
    eng = B3Engine(worlds, sc.sig)
    if args.art:
        from puffysics_amd.engine import B3_ENGINE_ART_CONTACTS
        eng.set_options(B3_ENGINE_ART_CONTACTS)
    stream = torch.cuda.current_stream()
    total = args.warmup + args.steps * args.repeats
    reset = torch.empty((total, count), dtype=torch.uint8, device="cuda")
    stepm = torch.empty((total, count), dtype=torch.uint8, device="cuda")
    for t in range(total):
        eng.scene_masks(args.scene, scenes.SEED, t, reset[t], stepm[t])
    step_counts = stepm.sum(dim=1, dtype=torch.int64).cpu().numpy()
    reset_any = reset.amax(dim=1).cpu().numpy()

    def vector_step(t):
        if reset_any[t]:
            eng.restore(reset[t])
        eng.scene_inputs(args.scene, scenes.SEED, t, stepm[t])
        eng.step(sc.dt, sc.substeps, stepm[t])

    log("warmup %d steps" % args.warmup)
    for t in range(args.warmup):
        vector_step(t)
    torch.cuda.synchronize()

    rates, ms, kernel_ms = [], [], []
    t = args.warmup
    for r in range(args.repeats):
        timed = range(0, args.steps, max(1, args.event_every))
        k_start = {i: torch.cuda.Event(enable_timing=True) for i in timed}
        k_end = {i: torch.cuda.Event(enable_timing=True) for i in timed}
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        t_begin = t
        for i in range(args.steps):
            if reset_any[t]:
                eng.restore(reset[t])
            eng.scene_inputs(args.scene, scenes.SEED, t, stepm[t])
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
        ms.append(el_ms / args.steps)
        kernel_ms.append(sum(k_start[i].elapsed_time(k_end[i]) for i in timed) / len(timed))
        log("repeat %d: %.3f ms/step, %.4g env-steps/s, step kernel %.3f ms" % (r, ms[-1], rates[-1], kernel_ms[-1]))
    med = sorted(range(args.repeats), key=lambda i: rates[i])[args.repeats // 2]

    # algorithmic bytes per step launch, from the live contact counts now
    st = eng.stats()
    per_world = world_bytes_model(worlds, st["contact_count"])
    mean_stepped = float(step_counts[args.warmup:].mean())
    bytes_per_launch = float(per_world.mean()) * mean_stepped
    k_ms = kernel_ms[med]
    achieved = bytes_per_launch / (k_ms * 1e-3) / 1e9
    counters = {} if args.art else load_counters(sc.name, count)
    traffic = counters.get("bytes_per_launch")
    valu = None
    if counters.get("valu_insts_per_launch"):
        # wave64 VALU instructions x 64 lanes over the measured launch time,
        # against the fp32 vector issue rate
        lane_ops = counters["valu_insts_per_launch"] * 64
        rate = lane_ops / (k_ms * 1e-3) / 1e12
        valu = {"achieved": round(rate, 3), "peak": VALU_PEAK_TLANE, "unit": "T lane-ops/s",
                "frac": round(rate / VALU_PEAK_TLANE, 4), "insts_per_launch": counters["valu_insts_per_launch"]}
    roofline = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": traffic,
                "kernel": "b3k_step_art" if args.art else "b3k_step", "kernel_ms": round(k_ms, 4),
                "kernel_launches_timed": len(timed),
                "bytes_per_env_step": round(float(per_world.mean()), 1),
                "mean_contacts_per_world": round(float(st["contact_count"].mean()), 2), "valu": valu}
    if traffic:
        # the measured HBM bytes of a launch over the same launch time
        roofline["traffic_gbs"] = round(traffic / (k_ms * 1e-3) / 1e9, 1)
        roofline["traffic_frac"] = round(traffic / (k_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    eng.close()
    del worlds

    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline(args.scene, args.cpu_seconds, 16)

    out = {"metric": METRIC, "value": round(rates[med], 1), "unit": "env-steps/s", "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms[med], 4),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
           "data": "synthetic (seeded scene builders, counter-based per-step inputs)",
           "config": {"workload": "%s%d: %d worlds of the %s scene, dt %.6g, %d substeps, masks %s" % (
               sc.name, count, count, sc.name, sc.dt, sc.substeps,
               "2% reset / 90% step" if args.scene == 5 else "none"),
               "worlds": count, "scene": sc.name, "dt": sc.dt, "substeps": sc.substeps,
               "repeats": args.repeats, "mean_stepped_worlds": round(mean_stepped, 1),
               "contacts": "articulated (B3_ENGINE_ART_CONTACTS)" if args.art else "independent-body (default)"},
           "roofline": roofline, "cpu_baseline": cpu}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
