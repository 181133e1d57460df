#!/usr/bin/env python3
"""Headline benchmark: FP32 MACE energy + forces + stress per call on one
MI355X, medium configuration.

Workload: random-init MACE of the medium shape (2 layers, 128x0e+128x1o,
l_max 3, correlation 3, 89-element embedding, 8 Bessel functions, radial MLP
[64,64,64], r_cut 6.0 A) on a perturbed cubic SrTiO3 10x10x10 supercell
(5,000 atoms, sigma 0.05 A, seed 0), neighbour graph at r_cut + 0.5 A skin
built once on the device and retained (the reference protocol,
benchmarks/mace_torch_comparison_protocol.md:65-90).

One step = one complete E+F+S call with the positions already resident in
HBM: edge geometry, both interaction layers forward and reverse, FP64 atom
forces, stress and the total energy on the device.  W untimed warm-up steps,
then exactly K timed steps between device synchronisations.

Also reported: per-kernel HIP-event timing of the dominant kernel on the
evaluator stream (roofline), the PCIe-inclusive host-positions call, the cold
call (graph rebuild) and the CPU oracle on a bounded sample (cpu_baseline).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "symmetrix-xl_amd"))
sys.path.insert(0, ROOT)

PEAK_FP32_TFLOPS = 157.3  # MI355X dense FP32 (matrix and packed vector)
PEAK_HBM_GBS = 8000.0
DOMINANT = "r1_reverse"


def r1_reverse_flops_per_edge_channel(num_paths, num_terms, num_rows):
    """Algorithmic FLOPs of the layer-2 reverse per active edge and channel:
    edge-force part E_a*C*(12P + 2T + 14 rows) plus source-adjoint part
    E_a*C*(6P + 2 rows + 2T) (FMA = 2 flops)."""
    return (12 * num_paths + 2 * num_terms + 14 * num_rows) + (6 * num_paths + 2 * num_rows + 2 * num_terms)


def model_counts(path):
    """Paths, CG terms and rows of the model file (for the roofline)."""
    with open(path) as f:
        j = json.load(f)
    P = len(j["Phi1_l"])
    T = len(j["Phi1_clebsch_gordan"])
    rows = sum((2 * a + 1) * (2 * b + 1) for a, b in zip(j["Phi1_l1"], j["Phi1_l2"]))
    return P, T, rows, j["num_channels"]


def hip_lib():
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipFree.argtypes = [ctypes.c_void_p]
    hip.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
    return hip


def device_copy_of(hip, a):
    p = ctypes.c_void_p()
    if hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(a.nbytes)) != 0:
        raise RuntimeError("hipMalloc failed")
    if hip.hipMemcpy(p, a.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(a.nbytes), 1) != 0:
        raise RuntimeError("hipMemcpy failed")
    return p


def load_traffic():
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE), if present."""
    path = os.path.join(ROOT, "profiles", "r1_reverse_medium_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def cpu_baseline(model_path, system, cutoff, skin, max_seconds=25.0):
    """The CPU oracle (FP32 C++/OpenMP restatement of the reference CPU path)
    on the same workload: warm calls with the graph retained."""
    from oracle import oracle as ora
    om = ora.OracleModel(model_path)
    graph = ora.neighbor_graph(system["positions"], system["cell"], cutoff + skin)
    cell = np.asarray(system["cell"], float)
    vol = abs(np.linalg.det(cell))
    types = om.types_of(system["numbers"])
    nt = types[graph["sources"]]

    def call():
        xyz, r = ora.prepared_geometry(graph, cell, system["positions"], system["positions"], om.r_cut)
        e, f = om.evaluate(types, graph["num_neigh"], graph["sources"], nt, xyz, r)
        ora.reduce_forces(len(types), graph["receivers"], graph["sources"], f)
        ora.reduce_stress(f, xyz, vol)
        return float(np.sum(e))

    def median_us_per_atom(seconds, most):
        times = []
        t_start = time.perf_counter()
        while True:
            t0 = time.perf_counter()
            call()
            times.append(time.perf_counter() - t0)
            if time.perf_counter() - t_start > seconds or len(times) >= most:
                break
        return round(statistics.median(times) * 1e6 / len(types), 3), len(times)

    call()  # warm-up (radial tabulation for the active types)
    cores = int(ora.lib().oracle_num_threads())
    value, calls = median_us_per_atom(max_seconds, 5)
    out = {"value": value, "unit": "us/atom", "cores": cores, "kind": "port",
           "sample": "medium workload (5000 atoms, 496k edges), %d warm call(s) after 1 warm-up, median" % calls,
           "cpu": cpu_model()}
    # the reference quotes its CPU path on 8 cores: the same sample on 8 threads
    if cores > 8:
        ora.lib().oracle_set_num_threads(8)
        v8, calls8 = median_us_per_atom(max_seconds / 2, 3)
        ora.lib().oracle_set_num_threads(cores)
        out["cores_8"] = {"value": v8, "unit": "us/atom", "cores": 8, "calls": calls8}
    return out


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def capacity(n, md_steps, tile_receivers):
    """the medium model in the tiled plan on an n^3
    SrTiO3 supercell; a velocity-Verlet NVE run of md_steps at 1 fs."""
    from symmetrix import md, random_model, systems
    from symmetrix.mace_kokkos import MACEKokkosFloat

    hip = hip_lib()
    free0, total = ctypes.c_size_t(), ctypes.c_size_t()
    hip.hipMemGetInfo(ctypes.byref(free0), ctypes.byref(total))
    def note(msg):
        print("[capacity] %s" % msg, file=sys.stderr, flush=True)

    model_path = random_model.cached_model("medium")
    system = systems.srtio3_supercell(n, sigma=0.05, seed=0)
    note("system n=%d: %d atoms" % (n, len(system["numbers"])))
    ev = MACEKokkosFloat(model_path)
    ev.set_execution_plan_request("capacity", tile_receivers)
    t0 = time.perf_counter()
    run = md.NVE(ev, system, skin=0.5, temperature=300.0, seed=0)
    first_s = time.perf_counter() - t0
    note("graph + first call %.1f s, %d edges, %s" % (first_s, run.num_edges, ev.execution_plan))
    free1 = ctypes.c_size_t()
    hip.hipMemGetInfo(ctypes.byref(free1), ctypes.byref(total))
    per_step, trace = run.run(md_steps, dt_fs=1.0,
                              progress=lambda k, e: note("step %d total energy %.6f eV" % (k, e)))
    n_atoms = len(system["numbers"])
    out = {
        "metric": "tiled capacity: atoms evaluated (FP32 E+F, 1 MI355X) and us/atom/step of 1 fs NVE",
        "atoms": n_atoms, "supercell": n, "edges": int(run.num_edges), "plan": ev.execution_plan,
        "md_steps": md_steps, "us_per_atom_step": round(per_step * 1e6 / n_atoms, 4),
        "first_call_s": round(first_s, 2), "graph_rebuilds": run.rebuilds,
        "device_memory_used_GiB": round((free0.value - free1.value) / 2**30, 2),
        "device_memory_total_GiB": round(total.value / 2**30, 2),
        "energy_drift_eV_per_atom": (trace[-1] - trace[0]) / n_atoms,
        "reference": {"atoms": 11240455, "hardware": "A100 80 GB", "mode": "tiled streaming"},
    }
    print(json.dumps(out), flush=True)


def copy_calibration(nbytes, repeats=5):
    """A plain device-to-device copy of nbytes (hipMemcpy, one copy kernel
    per call): the reference point that scales the rocprofv3 FETCH_SIZE /
    WRITE_SIZE counters to bytes."""
    hip = hip_lib()
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    if hip.hipMalloc(ctypes.byref(src), ctypes.c_size_t(nbytes)) or hip.hipMalloc(ctypes.byref(dst), ctypes.c_size_t(nbytes)):
        raise RuntimeError("hipMalloc failed")
    for _ in range(repeats):
        if hip.hipMemcpy(dst, src, ctypes.c_size_t(nbytes), 3) != 0:
            raise RuntimeError("hipMemcpy failed")
    hip.hipFree(src)
    hip.hipFree(dst)
    print(json.dumps({"copy_calibration_bytes": nbytes, "copies": repeats}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--capacity", type=int, default=0, metavar="N",
                    help="run the tiled capacity config on an N^3 SrTiO3 supercell instead")
    ap.add_argument("--md-steps", type=int, default=20)
    ap.add_argument("--tile-receivers", type=int, default=32768)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run device-to-device copies of BYTES (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures the single-GPU path only: this build runs on one MI355X and "
              "has no multi-GPU (halo-exchange) path; run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.capacity:
        capacity(args.capacity, args.md_steps, args.tile_receivers)
        return

    from symmetrix import random_model, systems
    from symmetrix.mace_kokkos import MACEKokkosFloat

    model_path = random_model.cached_model("medium")
    system = systems.srtio3_supercell(10, sigma=0.05, seed=0)
    skin = 0.5
    ev = MACEKokkosFloat(model_path)
    lut = {z: i for i, z in enumerate(ev.atomic_numbers)}
    types = np.array([lut[int(z)] for z in system["numbers"]], np.int32)
    cell = np.asarray(system["cell"], float)
    inv = np.linalg.inv(cell)
    vol = abs(float(np.linalg.det(cell)))
    n_atoms = len(types)

    t0 = time.perf_counter()
    g = ev._prepare_periodic_factorized_graph(types, system["positions"], cell, inv, ev.r_cut + skin)
    ev._compute_prepared_factorized_positions(g["generation"], system["positions"])
    cold_ms = (time.perf_counter() - t0) * 1e3
    gen = g["generation"]

    hip = hip_lib()
    d_pos = device_copy_of(hip, np.ascontiguousarray(system["positions"], dtype=np.float64))

    from symmetrix._native import check, lib

    def step():
        ev._compute_prepared_factorized_positions_device(gen, d_pos.value)
        check(lib.smx_reduce_prepared_node_forces(ev._h, gen, None))
        check(lib.smx_reduce_prepared_stress(ev._h, gen, vol, None))
        check(lib.smx_total_energy_device(ev._h, None))
        ev.synchronize()

    for _ in range(args.warmup):
        step()
    # HIP events around the dominant kernel on the evaluator's own stream
    ev.set_kernel_timing(True)
    ev.set_kernel_timing_filter(DOMINANT)
    ev.reset_kernel_timing()
    per_call = []
    ev.synchronize()
    t_all = time.perf_counter()
    for _ in range(args.steps):
        t0 = time.perf_counter()
        step()
        per_call.append(time.perf_counter() - t0)
    ev.synchronize()
    elapsed = time.perf_counter() - t_all
    timing = ev.kernel_timing()
    ev.set_kernel_timing(False)

    ms_per_step = elapsed * 1e3 / args.steps
    us_per_atom = elapsed * 1e6 / (args.steps * n_atoms)
    median_us_per_atom = statistics.median(per_call) * 1e6 / n_atoms

    # PCIe-inclusive call: positions from host memory, results copied back
    t0 = time.perf_counter()
    host_calls = 3
    for _ in range(host_calls):
        ev._compute_prepared_factorized_positions(gen, system["positions"])
        e = ev.node_energies
        ev._reduce_atom_forces(n_atoms, None, None, gen)
        ev._reduce_stress(vol, None, gen)
    host_us_per_atom = (time.perf_counter() - t0) * 1e6 / (host_calls * n_atoms)
    energy = float(np.sum(e))

    # roofline of the dominant kernel
    P, T, rows, C = model_counts(model_path)
    rec = ev._stage("edge_records")
    E_active = int(np.count_nonzero(rec.reshape(g["num_edges"], -1)[:, 2].view(np.int32)))
    ms_r1, launches = timing.get(DOMINANT, (float("nan"), 0))
    avg_ms = ms_r1 / max(launches, 1)
    flops = E_active * C * r1_reverse_flops_per_edge_channel(P, T, rows)
    achieved = flops / (avg_ms * 1e-3) / 1e12
    traffic = load_traffic()

    out = {
        "metric": "us/atom per E+F+stress call (FP32, 1 MI355X) at 5k atoms",
        "value": round(us_per_atom, 4),
        "unit": "us/atom",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (random-init medium MACE, perturbed SrTiO3 supercell, seed 0)",
        "config": {"workload": "medium: SrTiO3 10x10x10 (5000 atoms), MACE 128x0e+128x1o l_max 3 corr 3, "
                               "r_cut 6.0 A + 0.5 A skin, graph retained",
                   "atoms": n_atoms, "edges": int(g["num_edges"]), "active_edges": E_active,
                   "positions": "device-resident"},
        "roofline": {"bound": "mfma", "kernel": DOMINANT, "achieved": round(achieved, 3),
                     "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_TFLOPS, 4),
                     "traffic": traffic, "avg_launch_ms": round(avg_ms, 4),
                     "flops_per_launch": flops,
                     "compute": "FP32 VALU (edge-wise channel products; packed FP32 disabled, so 78.6 "
                                "TFLOP/s is the attainable issue rate)",
                     "traffic_source": "profiles/hbm_traffic_medium_5k.md (FETCH_SIZE+WRITE_SIZE, copy-scaled)"},
        "median_us_per_atom": round(median_us_per_atom, 4),
        "host_positions_us_per_atom": round(host_us_per_atom, 4),
        "cold_call_ms": round(cold_ms, 2),
        "energy_eV": energy,
        "baseline_reference": {"value": 1.922, "hardware": "RTX 5090", "note": "published, trained OMAT-0 medium"},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(model_path, system, ev.r_cut, skin)
    hip.hipFree(d_pos)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
