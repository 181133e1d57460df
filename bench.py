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

Also reported (extra keys, each measured in the same run):
* roofline of the dominant kernel from HIP events on the evaluator stream:
  executed flops (VALU op counters) over the non-packed FP32 VALU ceiling,
  the published FP32 peak beside it, and the algorithmic-equivalent rate;
* the reference protocol (3 warm-ups, median of 10) with device-resident
  positions, through the host-positions call, and through the Symmetrix
  calculator (the reference's ASE-call boundary), plus the cold call;
* the wide (30,000-atom water) and irregular (20,000 atoms, 10 species)
  configs: median us/atom and the dominant kernel's fraction;
* the tiled capacity config at 11.5M atoms (20 NVE steps at 1 fs);
* the MH-1 (MACE_Nonlinear) family member on the same 5,000-atom cell, at
  the reference's MH-1 boundary and through the calculator;
* the CPU oracle on the box's host cores (3 warm-ups, median of 10, OMP
  threads bound to cores), on all allowed cores and on 8 of them.
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
VALU_FP32_TFLOPS = 78.6   # FP32 VALU without packed FP32 (256 CUs x 4 SIMD x 16 lanes x 2 x 2.4 GHz)
PEAK_HBM_GBS = 8000.0
DOMINANT = "r1_reverse"
# FP32 operations the R1 reverse executes per active edge and channel, all
# source-group passes of one call: the coupled adjoints are contracted once
# per receiver, leaving per edge T = Y G, s = G h, W = sum_p R T,
# A = sum_p dR h T, SB = sum_p R s and f = u A + dY SB.  Measured with the
# VALU counters (64 x (ADD_F32 + MUL_F32 + 2 FMA_F32) per dispatch over
# E_active x C; profiles/executed_flops_r1.md), keyed by the model's
# (paths, coupling terms, rows): medium and wide shapes.
R1_REVERSE_EXECUTED_FLOPS_PER_EDGE_CHANNEL = {(10, 86, 88): 692.5, (17, 215, 243): 1565.8}


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


CPU_WORKER = r"""
import json, statistics, sys, time
import numpy as np
sys.path[:0] = [sys.argv[1], sys.argv[1] + "/symmetrix-xl_amd"]
from oracle import oracle as ora
from symmetrix import systems
om = ora.OracleModel(sys.argv[2])
system = systems.srtio3_supercell(10, sigma=0.05, seed=0)
skin = float(sys.argv[3])
graph = ora.neighbor_graph(system["positions"], system["cell"], om.r_cut + skin)
cell = np.asarray(system["cell"], float)
vol = abs(np.linalg.det(cell))
types = om.types_of(system["numbers"])
nt = types[graph["sources"]]
def call():
    xyz, r = ora.prepared_geometry(graph, cell, system["positions"], system["positions"], om.r_cut)
    e, f = om.evaluate(types, graph["num_neigh"], graph["sources"], nt, xyz, r)
    ora.reduce_forces(len(types), graph["receivers"], graph["sources"], f)
    ora.reduce_stress(f, xyz, vol)
for _ in range(3):
    call()
times = []
for _ in range(10):
    t0 = time.perf_counter()
    call()
    times.append(time.perf_counter() - t0)
print(json.dumps({"us_per_atom": statistics.median(times) * 1e6 / len(types),
                  "threads": int(ora.lib().oracle_num_threads())}))
"""


def cpu_baseline(model_path, skin):
    """The CPU oracle (FP32 C++/OpenMP restatement of the reference CPU path)
    on the headline workload in child processes (no GPU use), with the
    reference protocol (3 warm-ups, median of 10 calls, graph retained) and
    threads bound to cores as in benchmarks/openmp_full_property_qualification.py:319-322:
    run A on every core this process may use (capped at 16, the box's CPU
    share), run B on 8 of them (the reference's published 8-core figures)."""
    import subprocess
    allowed = sorted(os.sched_getaffinity(0))
    runs = {}
    for label, cores in (("all", allowed[:16]), ("8_cores", allowed[:8])):
        env = dict(os.environ, OMP_NUM_THREADS=str(len(cores)), OMP_PROC_BIND="close", OMP_PLACES="cores")
        cmd = ["taskset", "-c", ",".join(map(str, cores)), sys.executable, "-c", CPU_WORKER, ROOT, model_path,
               str(skin)]
        out = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=300)
        if out.returncode != 0:
            raise RuntimeError("CPU baseline worker failed: " + out.stderr[-2000:])
        runs[label] = json.loads(out.stdout.strip().splitlines()[-1])
        runs[label]["cpus"] = cores
    a = runs["all"]
    return {"value": round(a["us_per_atom"], 3), "unit": "us/atom", "cores": a["threads"], "kind": "port",
            "sample": "medium workload (5000 atoms, 496k edges, graph retained): 3 warm-up calls, median of 10, "
                      "OMP_PROC_BIND=close OMP_PLACES=cores, taskset to the listed CPUs",
            "cpu": cpu_model(), "cpus": a["cpus"],
            "cores_8": {"value": round(runs["8_cores"]["us_per_atom"], 3), "unit": "us/atom",
                        "cores": runs["8_cores"]["threads"], "cpus": runs["8_cores"]["cpus"]}}


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
    SrTiO3 supercell; a velocity-Verlet NVE run of md_steps at 1 fs.
    Returns the result record."""
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
    ev.close()
    return out


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
    ap.add_argument("--no-calculator", action="store_true", help="skip the calculator-boundary timing")
    ap.add_argument("--no-configs", action="store_true", help="skip the wide, irregular and one-interaction configs")
    ap.add_argument("--no-lammps", action="store_true", help="skip the LAMMPS pair-style step timing")
    ap.add_argument("--only-config", choices=("wide", "irregular", "single", "field", "mh1"),
                    help="run only that config (3 warm-ups, median of 10) and print its summary")
    ap.add_argument("--capacity-steps", type=int, default=20,
                    help="NVE steps of the tiled 11.5M-atom capacity extra key (0 skips it)")
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
        print(json.dumps(capacity(args.capacity, args.md_steps, args.tile_receivers)), flush=True)
        return

    from symmetrix import random_model, systems
    if args.only_config == "field":
        print(json.dumps(field_response_protocol(hip_lib(), 0.5)), flush=True)
        return
    if args.only_config == "mh1":
        print(json.dumps(mh1_protocol()), flush=True)
        return
    if args.only_config:
        model_path, system, workload = config_case(args.only_config)
        print(json.dumps(summary(run_config(hip_lib(), model_path, system, 0.5, 3, 10), workload)), flush=True)
        return

    def note(msg):
        print("[bench] %s" % msg, file=sys.stderr, flush=True)

    model_path = random_model.cached_model("medium")
    system = systems.srtio3_supercell(10, sigma=0.05, seed=0)
    skin = 0.5
    hip = hip_lib()
    head = run_config(hip, model_path, system, skin, args.warmup, args.steps, timed_steps=True)
    n_atoms = head["atoms"]
    note("medium: %.4f us/atom (mean of %d), median %.4f" % (head["us_per_atom"], args.steps,
                                                           head["median_us_per_atom"]))
    out = {
        "metric": "us/atom per E+F+stress call (FP32, 1 MI355X) at 5k atoms",
        "value": round(head["us_per_atom"], 4),
        "unit": "us/atom",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (random-init medium MACE, perturbed SrTiO3 supercell, seed 0)",
        "config": {"workload": "medium: SrTiO3 10x10x10 (5000 atoms), MACE 128x0e+128x1o l_max 3 corr 3, "
                               "r_cut 6.0 A + 0.5 A skin, graph retained",
                   "atoms": n_atoms, "edges": head["edges"], "active_edges": head["active_edges"],
                   "positions": "device-resident"},
        "roofline": dict(head["roofline"], traffic=load_traffic(),
                         traffic_source="profiles/hbm_traffic_medium_5k.md (FETCH_SIZE+WRITE_SIZE, copy-scaled)"),
        "median_us_per_atom": round(head["median_us_per_atom"], 4),
        "protocol": head["protocol"],
        "host_positions_us_per_atom": round(head["host_us_per_atom"], 4),
        "cold_call_ms": round(head["cold_ms"], 2),
        "energy_eV": head["energy"],
        "baseline_reference": {"value": 1.922, "hardware": "RTX 5090", "note": "published, trained OMAT-0 medium"},
    }
    if not args.no_calculator:
        out["calculator_us_per_atom"] = calculator_protocol(model_path, system, skin)
        note("calculator: %s" % out["calculator_us_per_atom"])
    out["model_load_s"] = model_load_seconds(model_path)
    note("model load: %s" % out["model_load_s"])
    if not args.no_lammps:
        out["lammps_step"] = lammps_step_protocol(hip, model_path, system, skin)
        note("lammps step: %s" % out["lammps_step"])
        out["split_phases"] = split_phase_protocol(hip, model_path, system, skin)
        note("split phases: %s" % out["split_phases"])
    if not args.no_configs:
        out["configs"] = {}
        for name in ("wide", "irregular", "single"):
            cfg_model, cfg_system, workload = config_case(name)
            out["configs"][name] = summary(run_config(hip, cfg_model, cfg_system, skin, 3, 10), workload)
            note("%s: %s" % (name, out["configs"][name]))
        out["field_response"] = field_response_protocol(hip, skin)
        note("field response: %s" % out["field_response"])
        out["configs"]["mh1"] = mh1_protocol()
        note("mh1: %s" % out["configs"]["mh1"])
    if args.capacity_steps > 0:
        try:
            out["capacity"] = capacity(132, args.capacity_steps, args.tile_receivers)
        except Exception as exc:  # reported, never hidden
            out["capacity"] = {"error": "%s: %s" % (type(exc).__name__, exc)}
        note("capacity: %s" % out["capacity"])
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(model_path, skin)
    print(json.dumps(out), flush=True)


def mh1_protocol():
    """MH-1 (MACE_Nonlinear) on SrTiO3 10x10x10: the 64/32-channel l_max-3
    family member (random init), the reference's MH-1 boundary
    (compute_node_energies_forces with the CSR graph inside r_cut in host
    memory, node energies and per-edge forces back; mace_nonlinear.hpp:44-51),
    3 warm-ups then the median of 10; per-kernel device time of one call; and
    the calculator boundary (positions in, E/F/S out, graph retained)."""
    from symmetrix import random_mh1, systems
    from symmetrix.calculator import Symmetrix
    from symmetrix.mace_nonlinear import MACENonlinearKokkosFloat
    from symmetrix.neighbors import neighbor_list_ijS
    model = random_mh1.cached_mh1("mh1_medium")
    system = systems.srtio3_supercell(10, sigma=0.05, seed=0)
    pos, cell = np.asarray(system["positions"]), np.asarray(system["cell"])
    ev = MACENonlinearKokkosFloat(model)
    lut = {z: i for i, z in enumerate(ev.atomic_numbers)}
    types = np.array([lut[int(z)] for z in system["numbers"]], np.int32)
    recv, src, shifts = neighbor_list_ijS(pos, cell, np.array([True] * 3), ev.r_cut)
    xyz = pos[src] - pos[recv] + shifts @ cell
    r = np.sqrt(np.einsum("ij,ij->i", xyz, xyz))
    keep = r < ev.r_cut
    recv, src, xyz, r = recv[keep], src[keep], np.ascontiguousarray(xyz[keep]), r[keep]
    n = len(types)
    args = (n, types, np.bincount(recv, minlength=n).astype(np.int32), src, types[src], xyz.reshape(-1), r)
    for _ in range(3):
        ev.compute_node_energies_forces(*args)
    ts = []
    for _ in range(10):
        t0 = time.perf_counter()
        ev.compute_node_energies_forces(*args)
        _ = ev.node_forces
        ts.append(time.perf_counter() - t0)
    ev._set_kernel_timing(True)
    ev.compute_node_energies_forces(*args)
    kt = ev._kernel_timing()
    ev._set_kernel_timing(False)
    top = sorted(kt.items(), key=lambda kv: -kv[1][0])[:6]
    calc = Symmetrix(model)
    for _ in range(3):
        calc.calculate(system, ["energy", "forces", "stress"])
    cs = []
    for _ in range(10):
        t0 = time.perf_counter()
        calc.calculate(system, ["energy", "forces", "stress"])
        cs.append(time.perf_counter() - t0)
    return {"workload": "mh1: MACE_Nonlinear (MH-1 family) 64x(0e..3o) nodes, 32 edge channels, l_max 3, corr 3, "
                        "r_cut 6.0 A, on SrTiO3 10x10x10 (5000 atoms)",
            "atoms": n, "edges": int(len(r)), "median_us_per_atom": round(statistics.median(ts) * 1e6 / n, 4),
            "protocol": "3 warm-ups, median of 10 compute_node_energies_forces calls (host graph in, "
                        "per-edge forces out)",
            "device_ms_per_call": round(sum(v[0] for v in kt.values()), 3),
            "top_kernels_ms": {k: round(v[0], 3) for k, v in top},
            "calculator_us_per_atom": round(statistics.median(cs) * 1e6 / n, 4)}


def field_response_protocol(hip, skin):
    """The MACEField path at the benchmark size: the field_l2 model (128
    channels, 0e+1o+2e hidden, l_max 3, correlation 3, a first-interaction
    residual) on the medium SrTiO3 system in a graph field; the evaluation
    (E, F, S and dE/dE, device positions) and then its response (the field
    Hessian and the Born charge bins: three tangent passes), 3 warm-ups and
    the median of 10 of each."""
    from symmetrix import random_model, systems
    from symmetrix.mace_kokkos import MACEKokkosFloat
    from symmetrix._native import check, lib
    model_path = random_model.cached_model("field_l2")
    system = systems.srtio3_supercell(10, sigma=0.05, seed=0)
    field = np.array([0.12, -0.21, 0.27])
    ev = MACEKokkosFloat(model_path)
    lut = {z: i for i, z in enumerate(ev.atomic_numbers)}
    types = np.array([lut[int(z)] for z in system["numbers"]], np.int32)
    cell = np.asarray(system["cell"], float)
    vol = abs(float(np.linalg.det(cell)))
    n = len(types)
    g = ev._prepare_periodic_factorized_graph(types, system["positions"], cell, np.linalg.inv(cell), ev.r_cut + skin)
    gen = g["generation"]
    ev._set_electric_field(field)
    d_pos = device_copy_of(hip, np.ascontiguousarray(system["positions"], dtype=np.float64))

    def evaluation():
        ev._compute_prepared_factorized_positions_device(gen, d_pos.value)
        check(lib.smx_reduce_prepared_node_forces(ev._h, gen, None))
        check(lib.smx_reduce_prepared_stress(ev._h, gen, vol, None))
        ev.synchronize()

    def response():
        ev._compute_prepared_factorized_field_response(gen, field, True, scatter_bec_bins=True)

    out = {"workload": "field_l2 MACEField model (128x(0e+1o+2e), l_max 3, corr 3, residual) on SrTiO3 10x10x10 "
                       "(5000 atoms), graph field, r_cut 5.0 A + 0.5 A skin",
           "atoms": n, "edges": int(g["num_edges"])}
    for key, fn in (("evaluation_ms", evaluation), ("response_ms", response)):
        for _ in range(3):
            fn()
        times = []
        for _ in range(10):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        out[key] = round(statistics.median(times) * 1e3, 3)
    out["response_per_component_us_per_atom"] = round(out["response_ms"] * 1e3 / 3 / n, 4)
    hip.hipFree(d_pos)
    ev.close()
    return out


def config_case(name):
    """(model path, system, workload text) of the wide, irregular and
    one-interaction configs."""
    from symmetrix import random_model, systems
    if name == "single":
        return (random_model.cached_model("medium_single"), systems.srtio3_supercell(10, sigma=0.05, seed=0),
                "single: one-interaction MACE 128x0e+128x1o l_max 3 corr 3, readout corr 2, A0-scaled "
                "(single_layer_readout), SrTiO3 10x10x10 (5000 atoms), r_cut 6.0 A + 0.5 A skin")
    if name == "wide":
        return (random_model.cached_model("wide"), systems.water_box(10000, seed=0),
                "wide: 10,000 rigid waters (30,000 atoms), MACE 256x(0e+1o+2e) l_max 3 corr 3, "
                "r_cut 5.0 A + 0.5 A skin")
    return (random_model.cached_model("medium"),
            systems.irregular_box(20000, density=0.08, min_distance=1.8, seed=0),
            "irregular: 20,000 atoms uniform at 0.08/A^3, 1.8 A minimum separation, 10 species, medium model")


def summary(r, workload):
    return {"workload": workload, "atoms": r["atoms"], "edges": r["edges"], "active_edges": r["active_edges"],
            "median_us_per_atom": round(r["median_us_per_atom"], 4), "protocol": "3 warm-ups, median of 10",
            "roofline": None if r["roofline"] is None else {
                k: r["roofline"][k] for k in ("kernel", "avg_launch_ms", "achieved", "frac",
                                              "algorithmic_equivalent_tflops", "unit")}}


def run_config(hip, model_path, system, skin, warmup, steps, timed_steps=False):
    """One configuration on the device-resident positions path: cold call,
    warm-ups, then `steps` calls with the dominant kernel timed by HIP
    events on the evaluator stream."""
    from symmetrix._native import check, lib
    from symmetrix.mace_kokkos import MACEKokkosFloat
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
    d_pos = device_copy_of(hip, np.ascontiguousarray(system["positions"], dtype=np.float64))

    def step():
        ev._compute_prepared_factorized_positions_device(gen, d_pos.value)
        check(lib.smx_reduce_prepared_node_forces(ev._h, gen, None))
        check(lib.smx_reduce_prepared_stress(ev._h, gen, vol, None))
        check(lib.smx_total_energy_device(ev._h, None))
        ev.synchronize()

    for _ in range(warmup):
        step()
    ev.set_kernel_timing(True)
    ev.set_kernel_timing_filter(DOMINANT)
    ev.reset_kernel_timing()
    per_call = []
    ev.synchronize()
    t_all = time.perf_counter()
    for _ in range(steps):
        t0 = time.perf_counter()
        step()
        per_call.append(time.perf_counter() - t0)
    ev.synchronize()
    elapsed = time.perf_counter() - t_all
    timing = ev.kernel_timing()
    ev.set_kernel_timing(False)
    out = {"atoms": n_atoms, "edges": int(g["num_edges"]), "cold_ms": cold_ms,
           "ms_per_step": elapsed * 1e3 / steps, "us_per_atom": elapsed * 1e6 / (steps * n_atoms),
           "median_us_per_atom": statistics.median(per_call) * 1e6 / n_atoms}
    if timed_steps:
        # the reference protocol on the same path: 3 warm-ups, median of 10
        for _ in range(3):
            step()
        med = []
        for _ in range(10):
            t0 = time.perf_counter()
            step()
            med.append(time.perf_counter() - t0)
        out["protocol"] = {"warmup": 3, "calls": 10, "median_us_per_atom": round(
            statistics.median(med) * 1e6 / n_atoms, 4), "positions": "device-resident"}
        # PCIe-inclusive call: positions from host memory, node energies,
        # atom forces and stress copied back (the one-call form)
        for _ in range(3):
            ev._compute_prepared_factorized_positions_results(gen, system["positions"], vol)
        host = []
        for _ in range(10):
            t0 = time.perf_counter()
            e, _, _ = ev._compute_prepared_factorized_positions_results(gen, system["positions"], vol)
            host.append(time.perf_counter() - t0)
        out["host_us_per_atom"] = statistics.median(host) * 1e6 / n_atoms
        out["energy"] = float(np.sum(e))
    # roofline of the dominant kernel: algorithmic flops of the active edges
    P, T, rows, C = model_counts(model_path)
    rec = ev._stage("edge_records")
    E_active = int(np.count_nonzero(rec.reshape(g["num_edges"], -1)[:, 2].view(np.int32)))
    out["active_edges"] = E_active
    out["roofline"] = None
    if P == 0:
        # a one-interaction model has no R1 reverse
        hip.hipFree(d_pos)
        ev.close()
        return out
    ms_r1, launches = timing.get(DOMINANT, (float("nan"), 0))
    avg_ms = ms_r1 / max(launches, 1)
    per_call = max(launches // max(steps, 1), 1)   # the wide shape runs one launch per source-component group
    flops = E_active * C * r1_reverse_flops_per_edge_channel(P, T, rows) / per_call
    achieved = flops / (avg_ms * 1e-3) / 1e12
    executed = R1_REVERSE_EXECUTED_FLOPS_PER_EDGE_CHANNEL.get((P, T, rows))
    # achieved/peak/frac: the algorithmic-equivalent rate (the survey's flop
    # count of the R1 reverse over the published FP32 peak); the kernel
    # executes fewer flops than that count (the coupling is contracted once
    # per receiver), so its hardware efficiency is executed_frac, executed
    # flops over the 78.6 TFLOP/s this VALU code can issue
    # achieved/peak/frac: executed flops (VALU op counters per edge-channel)
    # over the FP32 VALU issue rate without packed FP32 (this build compiles
    # packed FP32 out), the kernel's attainable ceiling; the published FP32
    # peak (157.3, packed/MFMA) is reported beside it.  The survey's
    # algorithmic count is an equivalent rate only (the kernel contracts the
    # coupling once per receiver), never a fraction of a peak.
    roof = {"bound": "valu", "kernel": DOMINANT, "achieved": None, "peak": VALU_FP32_TFLOPS, "unit": "TFLOP/s",
            "frac": None, "achieved_kind": "executed flops (VALU op counters)",
            "peak_kind": "FP32 VALU issue rate without packed FP32 (256 CUs x 4 SIMD x 16 lanes x 2 x 2.4 GHz)",
            "published_fp32_peak": PEAK_FP32_TFLOPS, "frac_of_published_fp32_peak": None,
            "avg_launch_ms": round(avg_ms, 4), "launches_per_call": per_call,
            "algorithmic_flops_per_launch": int(flops), "algorithmic_equivalent_tflops": round(achieved, 3),
            "compute": "FP32 VALU: edge-wise channel products, no MFMA",
            "executed_flops_per_launch": None, "executed_frac": None}
    if executed:
        ex = E_active * C * executed / per_call
        rate = ex / (avg_ms * 1e-3) / 1e12
        roof["executed_flops_per_launch"] = int(ex)
        roof["achieved"] = round(rate, 3)
        roof["frac"] = roof["executed_frac"] = round(rate / VALU_FP32_TFLOPS, 4)
        roof["frac_of_published_fp32_peak"] = round(rate / PEAK_FP32_TFLOPS, 4)
    out["roofline"] = roof
    hip.hipFree(d_pos)
    ev.close()
    return out


def lammps_arrays(system, cutoff):
    """The arrays pair_style symmetrix/mace/kk holds on one rank
    (pair_symmetrix_mace_kokkos.cpp:1010-1282): local atoms, the ghost images
    within `cutoff` of the (orthorhombic) box, atom->map(tag) as owner, and a
    full neighbour list (cutoff = r_cut + skin, LAMMPS's list cutoff) in a
    column-major array, as Kokkos lays it out on the device."""
    from scipy.spatial import cKDTree
    pos = np.asarray(system["positions"], float)
    cell = np.asarray(system["cell"], float)
    if np.count_nonzero(cell - np.diag(np.diag(cell))):
        raise ValueError("lammps_arrays expects an orthorhombic box")
    n = len(pos)
    L = np.diag(cell)
    frac = pos / L
    frac -= np.floor(frac)
    local = frac * L
    allpos, owner = [local], [np.arange(n)]
    for a in (-1, 0, 1):
        for b in (-1, 0, 1):
            for c in (-1, 0, 1):
                if (a, b, c) == (0, 0, 0):
                    continue
                img = local + np.array([a, b, c]) * L
                keep = np.all((img > -cutoff) & (img < L + cutoff), axis=1)
                allpos.append(img[keep])
                owner.append(np.nonzero(keep)[0])
    allpos = np.concatenate(allpos)
    owner = np.concatenate(owner).astype(np.int32)
    rows = cKDTree(allpos).query_ball_point(local, cutoff)
    rows = [np.array(sorted(j for j in r if j != i), np.int32) for i, r in enumerate(rows)]
    maxn = max(len(r) for r in rows)
    nb = np.zeros((maxn, n), np.int32)
    for i, r in enumerate(rows):
        nb[:len(r), i] = r
    numneigh = np.array([len(r) for r in rows], np.int32)
    return allpos, owner, nb, numneigh


def lammps_step_protocol(hip, model_path, system, skin):
    """smx_lammps_compute, the pair style's compute(), on device-resident
    LAMMPS arrays of the medium system: 3 warm-ups, median of 10 calls, once
    on a retained neighbour list (rebuild = 0, the steps between LAMMPS
    rebuilds) and once rebuilding the graph on every call (rebuild = 1).
    The reference's 2.559 us/atom/step (RTX 5090, README.md:101-110) is a
    whole LAMMPS step (integrator, communication and its own neighbour list
    included); this is the pair-style part of one."""
    from symmetrix._native import SmxLammpsArgsV2
    from symmetrix.mace_kokkos import MACEKokkosFloat
    ev = MACEKokkosFloat(model_path)
    lut = {int(z): i for i, z in enumerate(ev.atomic_numbers)}
    species = sorted(set(int(z) for z in system["numbers"]))
    type_of_z = {z: t + 1 for t, z in enumerate(species)}
    allpos, owner, nb, numneigh = lammps_arrays(system, ev.r_cut + skin)
    n, nall = len(numneigh), len(allpos)
    types = np.array([type_of_z[int(z)] for z in system["numbers"]], np.int32)[owner]
    a = SmxLammpsArgsV2()
    a.inum, a.nall, a.ntypes = n, nall, len(species)
    a.ilist = device_copy_of(hip, np.arange(n, dtype=np.int32))
    a.numneigh = device_copy_of(hip, numneigh)
    a.neighbors = device_copy_of(hip, nb)
    a.stride_atom, a.stride_neighbor = 1, n
    a.x = device_copy_of(hip, np.ascontiguousarray(allpos))
    a.type = device_copy_of(hip, types)
    a.type_to_model = device_copy_of(hip, np.array([lut[z] for z in species], np.int32))
    a.owner = device_copy_of(hip, owner)
    a.f = device_copy_of(hip, np.zeros((nall, 3)))
    a.eatom = None
    a.stream = None
    out = {"atoms": n, "ghosts": nall - n, "neighbors": int(numneigh.sum())}
    for key, rebuild in (("retained_list_us_per_atom", 0), ("rebuild_every_call_us_per_atom", 1)):
        a.rebuild = 1
        ev._lammps_compute(a)
        a.rebuild = rebuild
        for _ in range(3):
            ev._lammps_compute(a)
        times = []
        for _ in range(10):
            t0 = time.perf_counter()
            ev._lammps_compute(a)
            times.append(time.perf_counter() - t0)
        out[key] = round(statistics.median(times) * 1e6 / n, 4)
    out["reference"] = {"value": 2.559, "hardware": "RTX 5090", "note": "whole LAMMPS step, trained model"}
    for p in (a.ilist, a.numneigh, a.neighbors, a.x, a.type, a.type_to_model, a.owner, a.f):
        hip.hipFree(ctypes.c_void_p(p))
    ev.close()
    return out


def split_phase_protocol(hip, model_path, system, skin, parts=2):
    """One rank's share of the medium system cut into `parts` slabs along x
    (the split-phase evaluation a domain-decomposed LAMMPS run makes per
    step): each slab's begin, continue and finish with device edge vectors
    and device exchange rows (3 warm-ups, median of 10).  The inter-rank
    copies themselves are the caller's (MPI/RCCL) and not timed; the rows
    handed to continue are the slab's from a first full exchange."""
    from symmetrix._native import check, lib
    from symmetrix.mace_kokkos import MACEKokkosFloat, neighbor_list
    probe = MACEKokkosFloat(model_path)
    lut = {int(z): i for i, z in enumerate(probe.atomic_numbers)}
    r_cut = probe.r_cut
    probe.close()
    pos = np.asarray(system["positions"], float)
    cell = np.asarray(system["cell"], float)
    g = neighbor_list(pos, cell, r_cut + skin)
    types = np.array([lut[int(z)] for z in system["numbers"]], np.int32)
    xyz_all = g["fractional_xyz"] @ cell
    d = np.linalg.norm(xyz_all, axis=1)
    scale = np.where(d >= r_cut, r_cut / d, 1.0)
    xyz_all, r_all = xyz_all * scale[:, None], d * scale
    frac = (pos @ np.linalg.inv(cell))[:, 0] % 1.0
    owner = np.minimum((frac * parts).astype(int), parts - 1)
    off, src = g["offsets"], g["sources"]
    n = len(types)
    slabs, held = [], []

    def dev(a):
        p = device_copy_of(hip, np.ascontiguousarray(a))
        held.append(p)
        return p
    for dd in range(parts):
        recv = np.flatnonzero(owner == dd)
        edges = np.concatenate([np.arange(off[i], off[i + 1]) for i in recv])
        feats = np.concatenate([recv, np.setdiff1d(np.unique(src[edges]), recv)])
        index = np.full(n, -1, np.int64)
        index[feats] = np.arange(len(feats))
        ev = MACEKokkosFloat(model_path)
        gen = ev._prepare_factorized_feature_graph(len(recv), len(feats), index[recv], types[recv], types[feats],
                                                   (off[recv + 1] - off[recv]).astype(np.int32),
                                                   index[src[edges]].astype(np.int32), types[src[edges]])
        slabs.append(dict(ev=ev, gen=gen, recv=recv, feats=feats, E=len(edges),
                          xyz=dev(xyz_all[edges]), r=dev(r_all[edges])))
    # one full exchange on the host gives every slab its feature rows
    for sl in slabs:
        check(lib.smx_begin_factorized_distributed_evaluation(sl["ev"]._h, sl["gen"], len(sl["recv"]),
                                                              len(sl["feats"]), sl["xyz"], sl["r"], 1))
    H1 = None
    for sl in slabs:
        h = sl["ev"]._distributed_h1()
        H1 = np.zeros((n, h.shape[1]), np.float32) if H1 is None else H1
        H1[sl["recv"]] = h
    for sl in slabs:
        sl["rows"] = dev(H1[sl["feats"]])
        check(lib.smx_continue_factorized_distributed_evaluation(sl["ev"]._h, sl["rows"], len(sl["feats"]), 1))
        check(lib.smx_finish_factorized_distributed_evaluation(sl["ev"]._h, None, 0, 1))
    sl = slabs[0]
    h = sl["ev"]._h

    def step():
        check(lib.smx_begin_factorized_distributed_evaluation(h, sl["gen"], len(sl["recv"]), len(sl["feats"]),
                                                              sl["xyz"], sl["r"], 1))
        check(lib.smx_continue_factorized_distributed_evaluation(h, sl["rows"], len(sl["feats"]), 1))
        check(lib.smx_finish_factorized_distributed_evaluation(h, None, 0, 1))
    for _ in range(3):
        step()
    times = []
    for _ in range(10):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    out = {"slabs": parts, "receivers": int(len(sl["recv"])), "feature_nodes": int(len(sl["feats"])),
           "edges": int(sl["E"]), "ms_per_step": round(statistics.median(times) * 1e3, 4),
           "us_per_receiver": round(statistics.median(times) * 1e6 / len(sl["recv"]), 4),
           "note": "begin + continue + finish of one slab; the inter-rank row copies are not timed"}
    for s_ in slabs:
        s_["ev"].close()
    for p in held:
        hip.hipFree(p)
    return out


def model_load_seconds(model_path):
    """Evaluator construction (model file read, tables built, device upload)
    from the JSON file and from its SMXB binary form."""
    import tempfile
    from symmetrix import model_format
    from symmetrix.mace_kokkos import MACEKokkosFloat
    out = {}
    with tempfile.TemporaryDirectory() as d:
        binary = os.path.join(d, "model.smxb")
        model_format.convert(model_path, binary)
        for key, path in (("json", model_path), ("binary", binary)):
            t0 = time.perf_counter()
            MACEKokkosFloat(path).close()
            out[key] = round(time.perf_counter() - t0, 3)
        out["json_bytes"] = os.path.getsize(model_path)
        out["binary_bytes"] = os.path.getsize(binary)
    return out


def calculator_protocol(model_path, system, skin):
    """The reference's timing boundary: Symmetrix.calculate with host
    positions in and energy, forces and stress out, graph retained (3
    warm-ups, median of 10; benchmarks/mace_torch_comparison_protocol.md:65-90)."""
    from symmetrix.calculator import Symmetrix
    calc = Symmetrix(model_path, neighbor_skin=skin)
    atoms = {"numbers": system["numbers"], "positions": system["positions"], "cell": system["cell"],
             "pbc": [True, True, True]}
    for _ in range(3):
        calc.calculate(atoms, ["energy", "forces", "stress"])
    times = []
    for _ in range(10):
        t0 = time.perf_counter()
        calc.calculate(atoms, ["energy", "forces", "stress"])
        times.append(time.perf_counter() - t0)
    calc.evaluator.close()
    return round(statistics.median(times) * 1e6 / len(system["numbers"]), 4)


if __name__ == "__main__":
    main()
