"""Benchmark: TACE energy + conservative forces on the 12,288-atom water box.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

One step = one MD-step evaluation on one GPU: GPU cell-list neighbour list
from positions resident in HBM, the model forward (edge featurisation, 3
interaction + product layers, readout) and the backward for F = -dE/dr.
Workload: 4,096 H2O, 49.7 A periodic cube, r_c = 6,
Cartesian-TACE architecture C=128, L=3, nu=3, 3 layers, random-init weights
(seed 0), float32.  Prints one JSON line on stdout.

``roofline`` is for the kernel with the largest share of the timed region,
bracketed with HIP events on the stream it runs on; its algorithmic bytes
per launch follow the formulas in DESIGN.md.  ``cpu_baseline`` times the
CPU oracle (a restatement of the reference algorithm) on a bounded sample of
the same workload on this host.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "atom-steps/sec (E+F, fp32) at 12k atoms; % HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0
DT_FS = 0.5  # water with H


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algorithmic_bytes(name: str, info, var, s: int) -> float:
    """Bytes a kernel must move at minimum (each operand read / written once)."""
    from tace_amd import ops

    if name.startswith("edge_tp_fwd"):
        n, E, C = info
        return s * (E * (var.npath * C + var.d2) + n * C * (var.d1 + var.dout)) + 4 * (E + n + 1)
    if name.startswith("edge_tp_bwd"):
        n, E, C, need_x = info
        return s * (E * (2 * var.npath * C + 2 * var.d2) + n * C * (var.d1 * (2 if need_x else 1) + var.dout)) \
            + 4 * (E + n + 1)
    if name.startswith("uuu_fwd"):
        n, C = info
        return s * n * C * (var.d1 + var.d2 + var.dout)
    if name.startswith("uuu_bwd"):
        n, C = info
        return s * n * C * (2 * var.d1 + 2 * var.d2 + var.dout)
    if name.startswith("edge_basis_fwd"):
        (E,) = info
        return s * E * (3 + 8 + 16)
    if name.startswith("edge_basis_bwd"):
        (E,) = info
        return s * E * (3 + 8 + 16 + 3)
    return float("nan")


def measured_traffic(entry: str):
    """HBM bytes per call of ``entry`` from the rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary committed under profiles/ (None when not measured)."""
    path = os.path.join(ROOT, "profiles", "water12k_hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        line = line.strip()
        if line.startswith("traffic ") and "=" in line:
            name, val = line[len("traffic "):].rsplit("=", 1)
            if name.strip() == entry:
                return float(val)
    return None


def cpu_baseline(preset_cfg_fn, n_side=5, reps=3):
    """CPU oracle on a 125-molecule slice of the same water model (float32)."""
    from oracle import model as om
    from oracle import neighbours as onl
    from tace_amd import data, structures

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    s = structures.water_box(n_side=n_side, box=49.7 / 16 * n_side, seed=1)
    ei, S = onl.neighbour_list(s["positions"], s["cell"], s["pbc"], 6.0)
    cfg = preset_cfg_fn(ei.shape[1] / len(s["numbers"]))
    torch.manual_seed(0)
    m = om.TACE(cfg).float()
    for prm in m.parameters():  # frozen, as in the reference calculators
        prm.requires_grad_(False)
    d = data.collate([s], [(ei, S)], cfg["atomic_numbers"], dtype=torch.float32)
    om.compute(m, d, forces=True)  # warm-up
    t0 = time.perf_counter()
    for _ in range(reps):
        t_nl = time.perf_counter()
        ei, S = onl.neighbour_list(s["positions"], s["cell"], s["pbc"], 6.0)
        d = data.collate([s], [(ei, S)], cfg["atomic_numbers"], dtype=torch.float32)
        om.compute(m, d, forces=True)
    dt = time.perf_counter() - t0
    n = len(s["numbers"])
    return dict(value=n * reps / dt, unit="atom-steps/s", cores=threads, kind="port",
                sample=f"{n}-atom water slice ({n_side}^3 H2O, same C=128/L=3/3-layer model, float32), "
                       f"{reps} timed E+F steps incl. brute-force NL after 1 warm-up; {dt:.1f} s")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--n-side", type=int, default=16, help="water molecules per box edge (16 -> 12,288 atoms)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernels", action="store_true", help="print the per-kernel breakdown to stderr")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a device copy of 1 GiB five times (reference for the HBM byte counters)")
    args = ap.parse_args()
    if args.calibrate_copy:
        a = torch.empty(1 << 28, dtype=torch.float32, device="cuda:0").fill_(1.0)
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        log("[bench] copied 1 GiB x5")
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one MI355X; runs on more than one GPU are not part of it "
              "(see DESIGN.md for how the path would shard).", file=sys.stderr)
        sys.exit(2)

    from tace_amd import configs, data, model as pm, ops, structures

    dev = torch.device("cuda:0")
    box = 49.7 / 16 * args.n_side
    s = structures.water_box(n_side=args.n_side, box=box, seed=0)
    nat = len(s["numbers"])
    pos64 = torch.as_tensor(s["positions"], dtype=torch.float64, device=dev)
    g0 = data.resident_graph(pos64, s["cell"], s["pbc"], torch.zeros(nat, 2, device=dev), 6.0)
    E0 = g0["edge_index"].shape[1]
    avg = E0 / nat

    def cfg_fn(a):
        return configs.model_cfg("water12k", [1, 8], a)

    cfg = cfg_fn(avg)
    torch.manual_seed(0)
    model = pm.create_model(cfg).to(dev)
    model.reset_target_property(["energy", "forces"])
    # inference set-up of the reference calculators (ase/calculator.py:100-102,
    # torchsim.py:142, lammps/mliap.py:38): eval mode, parameters frozen
    model.eval()
    for prm in model.parameters():
        prm.requires_grad_(False)
    attrs = data.one_hot(s["numbers"], cfg["atomic_numbers"], torch.float32).to(dev)

    def step():
        g = data.resident_graph(pos64, s["cell"], s["pbc"], attrs, 6.0)
        return model(g)

    log(f"[bench] water box: {nat} atoms, {E0} edges (avg {avg:.1f}), warm-up {args.warmup}")
    for _ in range(args.warmup):
        out = step()
    torch.cuda.synchronize()
    log(f"[bench] warm-up done, E = {out['energy'].item():.6f}; timing {args.steps} steps")

    ops.TIMER = ops.KernelTimer()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    timer, ops.TIMER = ops.TIMER, None
    ms = dt / args.steps * 1e3
    summ = timer.summary()
    log(f"[bench] {ms:.2f} ms/step")

    # dominant native kernel -> roofline
    name, (cnt, tot_ms, infos) = max(summ.items(), key=lambda kv: kv[1][1])
    key = name.split(":", 1)[1] if ":" in name else None
    var = ops.find_variant(key) if key else None
    byts = sum(algorithmic_bytes(name, i, var, 4) for i in infos)
    achieved = byts / (tot_ms * 1e-3) / 1e9
    traffic = measured_traffic(name)
    roof = dict(kernel=name, bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                frac=round(achieved / HBM_PEAK_GBS, 4), traffic=traffic,
                algorithmic_bytes=round(byts / cnt),
                avg_launch_us=round(tot_ms / cnt * 1e3, 1), share_of_step=round(tot_ms / (dt * 1e3), 3))
    if args.kernels:
        for k, (c, t, _) in sorted(summ.items(), key=lambda kv: -kv[1][1]):
            log(f"  {t / args.steps:8.3f} ms/step  {c // args.steps:3d} launches/step  {k}")

    res = dict(metric=METRIC, value=round(nat * args.steps / dt, 1), unit="atom-steps/s", n_gpus=1,
               steps=args.steps, warmup=args.warmup, ms_per_step=round(ms, 3), higher_is_better=True,
               scaling="weak", vs_baseline=None, dtype="fp32", data="synthetic",
               config=dict(workload=f"water box {nat} atoms (configs[2]), E+F, NL rebuilt every step",
                           atoms=nat, edges=int(E0), channels=128, L=3, correlation=3, layers=3, cutoff=6.0,
                           parallelism="single GPU"),
               ns_per_day=round(1e3 / ms * 86400 * DT_FS * 1e-6, 4), roofline=roof)
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle) ...")
        res["cpu_baseline"] = cpu_baseline(cfg_fn)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
