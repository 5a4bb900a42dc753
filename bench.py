#!/usr/bin/env python3
"""Throughput benchmark of the batched physics step on one MI355X.

Workload: Ant, 4096 envs, MJCF timestep 0.01, substeps 1,
4 solver iterations, 64 contacts per env; actions i.i.d. U[-1,1] per env and step (seed 0),
torso height 0.75 + U[-0.1,0.1] and hinge noise U[-0.1,0.1] applied with reset_to_state.

A "step" is one zeno_world_step call over all envs on that step's host actions, the
reference's own method (benchmarks/bench_full_physics.zig:67-83). W untimed warm-up steps,
a reset, and untimed steps until every contact list is full precede K timed steps,
bracketed by a stream synchronisation on both sides. Beside value: the same steps with the
actions resident in HBM, replayed from one HIP graph, and the caller's per-step loop
(step + observations, rewards, dones).

Printed: one JSON line with value = env-steps/s, a roofline object for the step kernel
(HIP events on the library's stream over the timed region; algorithmic bytes per env-step
from the buffer sizes the step must read and write) and a CPU baseline (the scalar C oracle
on this host's cores over a bounded sample of the same workload).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0


def algorithmic_bytes_per_env_step(model: dict, max_contacts: int) -> int:
    """Minimum HBM bytes one env-step must move in the reference layout: actions (R),
    body pos/quat/vel/angvel (R+W) + accel (W), joint q/qd/tau (W), lambda (R+W), contact
    slots (R+W), contact count and previous count, observations (W)."""
    A, B, J = model["num_actuators"], model["num_bodies"], model["num_joints"]
    N, obs = model["num_constraints"], model["obs_dim"]
    return 4 * A + 144 * B + 12 * J + 8 * N + 128 * max_contacts + 8 + 4 * obs


def hip_device_buffer(host: np.ndarray):
    """Copies host into a new device allocation (libamdhip64 via ctypes). Returns (ptr, free)."""
    hip = C.CDLL("libamdhip64.so")
    ptr = C.c_void_p()
    if hip.hipMalloc(C.byref(ptr), C.c_size_t(host.nbytes)) != 0:
        raise RuntimeError("hipMalloc failed")
    if hip.hipMemcpy(ptr, C.c_void_p(host.ctypes.data), C.c_size_t(host.nbytes), 1) != 0:
        raise RuntimeError("hipMemcpy failed")
    return ptr.value, (lambda: hip.hipFree(ptr))


def calibrate_copy(nbytes: int) -> None:
    hip = C.CDLL("libamdhip64.so")
    a, b = C.c_void_p(), C.c_void_p()
    if hip.hipMalloc(C.byref(a), C.c_size_t(nbytes)) or hip.hipMalloc(C.byref(b), C.c_size_t(nbytes)):
        raise RuntimeError("hipMalloc failed")
    hip.hipMemset(a, 1, C.c_size_t(nbytes))
    for _ in range(3):
        if hip.hipMemcpy(b, a, C.c_size_t(nbytes), 3) != 0:
            raise RuntimeError("hipMemcpy D2D failed")
    hip.hipDeviceSynchronize()
    hip.hipFree(a)
    hip.hipFree(b)


def load_traffic(profile_json: Path):
    try:
        d = json.loads(profile_json.read_text())
        return d.get("hbm_bytes_per_launch")
    except Exception:
        return None


def cpu_baseline(model, state, acts, num_envs: int, budget_s: float, workload: str = "ant",
                 max_contacts: int = 64, extended: bool = False) -> dict:
    from oracle.oracle import OracleWorld

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    o = OracleWorld(model, num_envs, max_contacts_per_env=max_contacts)
    o.extended_contacts = extended
    o.reset_to_state(*state)
    o.step(acts[0], nthreads=threads)  # warm-up
    # The pregenerated action rows are reused cyclically so that the sample runs for the
    # whole time budget; the trajectory continues, it is not restarted.
    steps = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        o.step(acts[1 + steps % (acts.shape[0] - 1)], nthreads=threads)
        steps += 1
    dt = time.perf_counter() - t0
    return {
        "value": num_envs * steps / dt,
        "unit": "env-steps/s",
        "cores": threads,
        "kind": "port",
        "sample": f"scalar C oracle (restatement of the reference MSL step), {workload} {num_envs} envs x "
                  f"{steps} steps of the same seeded inputs (action rows reused cyclically), OpenMP over "
                  f"envs, {dt:.1f} s",
    }


# The reference's published step numbers (README.md:56-59, docs/reference/performance.md:13-16
# of the reference): 1024 envs x 1000 steps on an Apple M4 Pro.
PUBLISHED = {"pendulum": 4.97e6, "cartpole": 6.52e6, "ant": 5.89e6, "humanoid": 5.95e6}


def published_configs() -> dict:
    """The reference's own benchmark (benchmarks/bench_full_physics.zig:37-83) on this build:
    1024 envs, timestep 0.002, 4 contact iterations, 64 contacts, 1 substep; one action array
    U[-1, 1] drawn once and reused; 10 warm-up steps, reset, then 1000 zeno_world_step calls
    on host actions timed by wall clock."""
    from zeno_amd.scenes import ASSETS
    from zeno_amd.world import ZenoWorld

    out = {}
    for name, ref in PUBLISHED.items():
        w = ZenoWorld(mjcf_path=str(ASSETS / f"{name}.xml"), num_envs=1024, timestep=0.002,
                      contact_iterations=4, max_contacts_per_env=64, substeps=1)
        acts = np.random.default_rng(42).uniform(-1.0, 1.0, (1024, max(w.action_dim, 1))).astype(np.float32)
        acts = acts[:, : w.action_dim]
        for _ in range(10):
            w.step(acts)
        w.reset()
        w.synchronize()
        t0 = time.perf_counter()
        for _ in range(1000):
            w.step(acts)
        w.synchronize()
        v = 1024 * 1000 / (time.perf_counter() - t0)
        out[name] = {"value": v, "unit": "env-steps/s", "published": ref, "ratio": v / ref}
        w.close()
    return out


def collide_pairs_inputs(n: int, seed: int = 0):
    """n operand pairs for the extended narrow phase: types uniform over sphere, capsule, box
    and plane on both sides, sizes U[0.05, 0.6], positions U[-0.7, 0.7]^3 (about a third of
    the pairs touch), random rotations."""
    from zeno_amd.collision import COLLIDER_DTYPE

    rng = np.random.default_rng(seed)
    sides = []
    for _ in range(2):
        r = np.zeros(n, COLLIDER_DTYPE)
        r["type"] = rng.integers(0, 4, n)
        r["size"] = rng.uniform(0.05, 0.6, (n, 3))
        r["position"][:, :3] = rng.uniform(-0.7, 0.7, (n, 3))
        q = rng.normal(size=(n, 4))
        r["quaternion"] = q / np.linalg.norm(q, axis=1, keepdims=True)
        sides.append(r)
    return sides[0], sides[1]


def bench_collide(n: int, steps: int, warmup: int, cpu_seconds: float, no_cpu: bool) -> dict:
    """zeno_amd_detect_collisions over n resident pairs: HIP events on the null stream around
    each launch; 192 algorithmic bytes per pair (two 64-B operands read, one 64-B result
    written)."""
    from zeno_amd import _lib as L
    from zeno_amd.collision import CONTACT_RESULT_DTYPE

    a, b = collide_pairs_inputs(n)
    hip = C.CDLL("libamdhip64.so")
    pa, fa = hip_device_buffer(a)
    pb, fb = hip_device_buffer(b)
    po, fo = hip_device_buffer(np.zeros(n, CONTACT_RESULT_DTYPE))
    lib = L.load()
    ev = [C.c_void_p() for _ in range(2 * steps)]
    for e in ev:
        hip.hipEventCreate(C.byref(e))
    for _ in range(warmup):
        if lib.zeno_amd_detect_collisions(C.c_void_p(pa), C.c_void_p(pb), n, C.c_void_p(po), None) != 0:
            raise RuntimeError("detect_collisions failed")
    hip.hipDeviceSynchronize()
    t0 = time.perf_counter()
    for k in range(steps):
        hip.hipEventRecord(ev[2 * k], None)
        lib.zeno_amd_detect_collisions(C.c_void_p(pa), C.c_void_p(pb), n, C.c_void_p(po), None)
        hip.hipEventRecord(ev[2 * k + 1], None)
    hip.hipDeviceSynchronize()
    elapsed = time.perf_counter() - t0
    ms = C.c_float()
    total_ms = 0.0
    for k in range(steps):
        hip.hipEventElapsedTime(C.byref(ms), ev[2 * k], ev[2 * k + 1])
        total_ms += ms.value
    for e in ev:
        hip.hipEventDestroy(e)
    fa(); fb(); fo()
    kernel_s = total_ms / 1e3 / steps
    achieved = 192.0 * n / kernel_s / 1e9
    result = {
        "metric": "contact pairs/sec (narrow_phase.detectCollision, batched)",
        "value": n * steps / elapsed, "unit": "pairs/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": 1e3 * elapsed / steps, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic: uniform random type pairs, sizes, poses (seed 0)",
        "config": {"workload": f"collide_pairs {n} pairs per launch (operands resident in HBM)", "pairs": n},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS,
                     "traffic": load_traffic(ROOT / "profiles" / "collide_pairs_hbm_traffic.json") if n == 8388608 else None,
                     "kernel": "detect_collisions_kernel",
                     "kernel_avg_us": kernel_s * 1e6, "algorithmic_bytes_per_pair": 192,
                     "algorithmic_bytes_per_launch": 192 * n},
    }
    if not no_cpu:
        from oracle.oracle import detect_collisions as cpu_detect

        threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
        m = min(n, 1 << 20)
        done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < cpu_seconds:
            cpu_detect(a[:m], b[:m], nthreads=threads)
            done += m
        dt = time.perf_counter() - t0
        result["cpu_baseline"] = {"value": done / dt, "unit": "pairs/s", "cores": threads, "kind": "port",
                                  "sample": f"C oracle of detectCollision, OpenMP over pairs, {done} pairs "
                                            f"(the first {m} of the same inputs, repeated), {dt:.1f} s"}
    return result


def settle_steps(w, acts, limit: int = 64) -> int:
    """Untimed steps after a reset until every env's contact list is full (the reference
    never clears the count between steps, all_shaders.metal:765-766, so the list saturates at
    max_contacts within a few steps and the step then does the same work every call); scenes
    whose counts stop growing stop early.
    Returns the number of steps taken (actions acts[0..n))."""
    M = w.max_contacts_per_env
    prev = None
    for k in range(limit):
        # The previous count (a copy: hands out no view) equals the current one once a step
        # has run since the reset, which zeroed the current counts but not the previous ones.
        counts = w.get_prev_contact_counts() if k > 0 else None
        if counts is not None and (counts.min() >= M or (prev is not None and np.array_equal(counts, prev))):
            return k
        prev = counts
        w.step(acts[k])
    return limit


def main() -> int:
    from zeno_amd.scenes import WORKLOADS, workload_inputs

    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="ant", choices=sorted(WORKLOADS))
    ap.add_argument("--envs", type=int, default=0, help="override the workload's env count")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline time budget")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--max-contacts", type=int, default=64, help="max_contacts_per_env of the world")
    ap.add_argument("--extended-contacts", action="store_true",
                    help="extended-contact mode: box and capsule pairs through detectCollision in the step")
    ap.add_argument("--no-legs", action="store_true",
                    help="skip the device-action, HIP-graph, env-loop and published-config legs")
    ap.add_argument("--no-graph", action="store_true", help="skip the HIP-graph replay leg")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="first run 3 device-to-device copies of this many MiB (a plain copy kernel "
                         "of known size, used to scale rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--collide-pairs", type=int, default=0,
                    help="instead of the step, time the batched extended narrow phase on this many pairs")
    args = ap.parse_args()
    if args.calibrate_copy_mib > 0:
        calibrate_copy(args.calibrate_copy_mib << 20)
    if args.collide_pairs > 0:
        print(json.dumps(bench_collide(args.collide_pairs, min(args.steps, 200), max(args.warmup, 1),
                                       min(args.cpu_seconds, 10.0), args.no_cpu)), flush=True)
        return 0

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the step shards by environment with no cross-GPU "
              "traffic, and this build targets a single MI355X. Run with --gpus 1.", file=sys.stderr)
        return 2

    from zeno_amd.world import ZenoWorld

    wl = WORKLOADS[args.workload]
    E = args.envs or wl.num_envs
    settle_max = 64
    total = max(args.warmup, 1) + settle_max + args.steps
    path, xml, model, state, acts = workload_inputs(args.workload, E, total, seed=0)
    w = ZenoWorld(mjcf_path=path, mjcf_string=xml, num_envs=E, max_contacts_per_env=args.max_contacts)
    if args.extended_contacts:
        w.set_extended_contacts(True)
    epw, lds = w.launch_config()

    # Warm-up, then reset to the seeded initial state (bench_full_physics.zig:67-72), then
    # untimed steps until the contact lists are full, so that a short run times the steady
    # state. Every leg below starts from the same reset and the same settling steps.
    w.reset_to_state(*state)
    for k in range(args.warmup):
        w.step(acts[k])
    w.reset_to_state(*state)
    S = settle_steps(w, acts)
    timed = acts[S:S + args.steps]

    def restart():
        w.reset_to_state(*state)
        for k in range(S):
            w.step(acts[k])
        w.synchronize()

    # Timed region (value): the reference's own method, bench_full_physics.zig:67-83: K
    # zeno_world_step calls on host actions (the kernel reads them in place from a pinned
    # ring), wall clock between two stream synchronisations. HIP events on the world's
    # stream around every 8th launch give the step kernel's average duration (an event pair
    # costs a few us of queue time, so timing every launch, or every second one, slows the
    # loop it measures: 70.5 -> 73.8 us per step at K = 20 when every second launch was timed).
    w.synchronize()
    w.set_kernel_timing(True, every=8)
    w.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        w.step(timed[k])
    w.synchronize()
    elapsed = time.perf_counter() - t0
    kernel_ms, launches = w.get_kernel_timing()
    w.set_kernel_timing(False)
    value = E * args.steps / elapsed
    kernel_avg_s = (kernel_ms / 1e3) / max(launches, 1)
    # No getter touches this world before the legs are done: a getter hands its array out,
    # and every later step would then store that array to host memory as well.

    legs = {}
    finite = True
    if not args.no_legs:
        # Device-resident actions (zeno_amd_world_step_device): no host ring.
        A = model["num_actuators"]
        flat = np.ascontiguousarray(timed).reshape(-1)
        if flat.size == 0:
            flat = np.zeros(1, np.float32)
        dptr, dfree = hip_device_buffer(flat)
        stride = E * A * 4
        restart()
        t1 = time.perf_counter()
        for k in range(args.steps):
            rc = w._lib.zeno_amd_world_step_device(w.handle, C.c_void_p(dptr + k * stride), 0)
            if rc != 0:
                raise RuntimeError(f"step_device failed: {rc}")
        w.synchronize()
        el = time.perf_counter() - t1
        legs["device_actions"] = {"value": E * args.steps / el, "ms_per_step": 1e3 * el / args.steps,
                                  "method": "zeno_amd_world_step_device with the actions resident in HBM"}
        # The same K steps captured into one HIP graph and replayed with one call.
        if not args.no_graph:
            restart()
            w.capture_steps(dptr, stride, args.steps)
            t2 = time.perf_counter()
            w.graph_launch()
            w.synchronize()
            el = time.perf_counter() - t2
            w.release_graph()
            legs["hip_graph"] = {"value": E * args.steps / el, "ms_per_step": 1e3 * el / args.steps,
                                 "method": "the timed steps captured into one HIP graph, replayed with one launch call"}
        dfree()
        # The caller's per-step loop (ZenoEnv.reset, then ZenoEnv.step: python/zeno/env.py:
        # 103-178): the reset returns the observations, which hands the observation mirror out,
        # so every step returns with it current (the kernel stores the rows to host memory and
        # the call waits); then step, observations, rewards and dones every step. Timed over
        # at least 200 steps (the actions cycle), so that one slow call of a short run does not
        # stand for the loop.
        K2 = max(args.steps, 200)
        restart()
        obs = w.get_observations()
        t3 = time.perf_counter()
        for k in range(K2):
            w.step(timed[k % len(timed)])
            obs = w.get_observations()
            w.get_rewards()
            w.get_dones()
        el = time.perf_counter() - t3
        legs["env_loop"] = {"value": E * K2 / el, "ms_per_step": 1e3 * el / K2, "steps": K2,
                            "extra_us_per_step_over_value": 1e6 * (el / K2 - elapsed / args.steps),
                            "obs_bytes_per_step": int(obs.nbytes),
                            "method": "after a reset that returns the observations: zeno_world_step on host "
                                      "actions + get_observations (copy) + get_rewards + get_dones every step"}
        finite = bool(np.isfinite(obs).all())
    finite = finite and bool(np.isfinite(w.get_body_positions(zero_copy=False)).all())

    bytes_env_step = algorithmic_bytes_per_env_step(model, w.max_contacts_per_env)
    bytes_launch = bytes_env_step * E
    achieved = bytes_launch / kernel_avg_s / 1e9
    tag = f"{args.workload}{E}" + (f"_m{args.max_contacts}" if args.max_contacts != 64 else "") + \
        ("_ext" if args.extended_contacts else "")
    prof = ROOT / "profiles" / f"{tag}_hbm_traffic.json"
    traffic = load_traffic(prof)

    metric = (f"env-steps/sec at Ant 4096 envs × {args.steps} steps; achieved HBM GB/s"
              if args.workload == "ant" and E == 4096 else f"env-steps/sec at {args.workload} {E} envs × {args.steps} steps")
    result = {
        "metric": metric,
        "value": value,
        "unit": "env-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": 1e3 * elapsed / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded initial-state noise and i.i.d. actions on the reference's MJCF model",
        "config": {
            "workload": f"{args.workload} {E} envs x {args.steps} steps, zeno_world_step on host actions",
            "model": wl.mjcf, "num_envs": E, "timestep": w.timestep, "substeps": 1,
            "contact_iterations": 4, "max_contacts_per_env": w.max_contacts_per_env,
            "settle_steps": S, "envs_per_wave": epw, "lds_bytes_per_workgroup": lds,
            "extended_contacts": bool(args.extended_contacts), "placement": w.modes()["placement"],
        },
        "hbm_gbps": bytes_env_step * value / 1e9,
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBPS,
            "traffic": traffic,
            "kernel": "step_kernel",
            "kernel_avg_us": kernel_avg_s * 1e6,
            "kernel_launches_timed": launches,
            "algorithmic_bytes_per_env_step": bytes_env_step,
            "algorithmic_bytes_per_launch": bytes_launch,
        },
        **legs,
        "finite": finite,
    }
    if args.workload == "ant" and not args.no_legs:
        result["published_configs"] = {
            "note": "the reference's own benchmark method and configs (1024 envs, dt 0.002, host actions, "
                    "1000 steps) on this GPU, beside its published Apple M4 Pro numbers",
            **published_configs(),
        }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(model, state, acts, E, args.cpu_seconds, args.workload,
                                              args.max_contacts, args.extended_contacts)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
