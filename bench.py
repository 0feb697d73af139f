"""Benchmark: TACE energy + conservative forces on the 12,288-atom water box.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                    [--workload water12k|fcc1024|ragged128|fe101k] [--kernels]

One step = one MD-step evaluation on one GPU: GPU cell-list neighbour list
from positions resident in HBM, the model forward (edge featurisation, 3
interaction + product layers, readout) and the backward for F = -dE/dr.
Workload: 4,096 H2O, 49.7 A periodic cube, r_c = 6,
Cartesian-TACE architecture C=128, L=3, nu=3, 3 layers, random-init weights
(seed 0), float32.  Prints one JSON line on stdout.  The other configurations
have their own workloads: ``fcc1024`` (configs[1], 1,024-atom FCC alloy),
``ragged128`` (configs[3], 128 random crystals, 89 species, with stress) and
``fe101k`` (configs[4], TECE: bcc Fe 37^3 cells, 101,306 atoms, r_c = 5, C=128,
L=2, 4 heads, 2 layers, bf16 channel mixing).

``roofline`` is for the kernel with the largest share of the step, bracketed
with HIP events on the stream it runs on in a second timed pass of the same
K steps (every native launch instrumented; the first pass, which gives
``value``, runs without the per-launch events); its algorithmic bytes per
launch follow ``section8d_bytes`` / ``algorithmic_bytes`` below.  ``cpu_baseline`` times the
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
FP32_PEAK_TFS = 157.3    # MI355X dense fp32 (matrix and vector)
BF16_PEAK_TFS = 2500.0   # MI355X dense bf16 MFMA
# float32 GEMMs on the bf16 MFMA: six bf16 products per float32 product
BF16X3_PRODUCTS = 6
DT_FS = 0.5  # water with H


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algorithmic_bytes(name: str, info, var, s: int) -> float:
    """Bytes a kernel must move at minimum (each operand read / written once)."""
    from tace_amd import ops

    if name.startswith("edge_tp_fwd"):
        # with edge pairs (a 4th item) the weights are one row per pair
        n, E, C = info[:3]
        rows = info[3] if len(info) > 3 else E
        return s * (rows * var.npath * C + E * var.d2 + n * C * (var.d1 + var.dout)) + 4 * (E + n + 1) \
            + (4 * E if len(info) > 3 else 0)
    if name.startswith("edge_tp_bwd"):
        n, E, C, need_x = info[:4]
        rows = info[4] if len(info) > 4 else E
        return s * (rows * var.npath * C + E * (var.npath * C + 2 * var.d2)
                    + n * C * (var.d1 * (2 if need_x else 1) + var.dout)) + 4 * (E + n + 1) \
            + (4 * E if len(info) > 4 else 0)
    if name.startswith("edge_rtp_fwd"):
        # h instead of w: x, y, h read (the last radial layer's 64 x W weights
        # once), out written
        n, E, C = info
        return s * (E * (64 + var.d2) + n * C * (var.d1 + var.dout) + 64 * var.npath * C) + 4 * (E + n + 1)
    if name.startswith("edge_rtp_bwd"):
        # x, y, h, g_out read; g_w, g_y (and g_x) written
        n, E, C, need_x = info
        return s * (E * (64 + var.npath * C + 2 * var.d2) + n * C * (var.d1 * (2 if need_x else 1) + var.dout)
                    + 64 * var.npath * C) + 4 * (E + n + 1)
    if name.startswith("uuu_fwd"):
        n, C = info
        return s * n * C * (var.d1 + var.d2 + var.dout)
    if name.startswith("uuu_bwd"):
        n, C = info
        return s * n * C * (2 * var.d1 + 2 * var.d2 + var.dout)
    if name.startswith("edge_wigner_fwd"):
        E, K = info
        return s * E * (3 + K * K)
    if name.startswith("edge_wigner_bwd"):
        E, K = info
        return s * E * (3 + K * K + 3)
    if name.startswith("tece_score_fwd"):
        E, K, C, H = info
        return s * E * (2 * K * C + 2 * H + H) + s * H
    if name.startswith("tece_score_bwd"):
        E, K, C, H, b16 = info
        return s * E * (2 * K * C + 4 * H + H) + (2 if b16 else s) * E * 2 * K * C + s * H
    if name.startswith("so2_gemm_bf16"):
        # bf16 A [m, k] and B [k, n] read once, float32 out [m, n] written
        m, n, k = info
        return 2 * m * k + 2 * k * n + 4 * m * n
    if name.startswith("graph_softmax_fwd"):
        E, H, n = info
        return s * E * H * 2 + 4 * (E + n + 1)
    if name.startswith("graph_softmax_bwd"):
        E, H, n = info
        return s * E * H * 3 + 4 * (E + n + 1)
    if name.startswith("tece_rotate_out_fwd"):
        n, E, C, K, H = info
        return s * (E * (K * C + H + K * K) + n * K * C) + 4 * (E + 2 * n + 1)
    if name.startswith("tece_rotate_out_bwd"):
        n, E, C, K, H, b16 = info
        return s * (E * (K * C + 2 * H + 2 * K * K) + n * K * C) + (2 if b16 else s) * E * K * C + 8 * E
    if name.startswith("edge_rotate_in_fwd"):
        E, K, C, has_w, b16 = info
        nc = (int(math.isqrt(K)) * (int(math.isqrt(K)) + 1)) // 2
        so = 2 if b16 else s
        # x_src, x_dst and W read; m_src, m_dst (and w read, m_w written) out
        return s * E * (2 * K * C + K * K + (2 * nc * C if has_w else 0)) + so * E * (2 * K * C + (2 * K * C if has_w else 0)) \
            + 16 * E
    if name.startswith("edge_rotate_in_bwd"):
        E, K, C, has_w = info[:4]
        runs = len(info) > 4 and info[4]
        nc = (int(math.isqrt(K)) * (int(math.isqrt(K)) + 1)) // 2
        # x_src, x_dst, g_m_src, g_m_dst, W read; per-edge sender grad_x rows
        # and g_W written, receiver grad_x rows per edge or (runs) one per run
        # of a workgroup's four edges, counted as a quarter row per edge; with
        # radial weights also g_m_w and w read, g_w written
        return s * E * ((5.25 if runs else 6) * K * C + 2 * K * K + (2 * K * C + 4 * nc * C if has_w else 0)) + 16 * E
    if name.startswith("tece_edge_ace_fwd") or name.startswith("tece_edge_ace_bwd"):
        E, A, L, b16 = info
        n, P = L + 1, len(ops.edge_ace_paths(L))
        ys = E * ((P * n * A + n * A + (n * (L + 1) + n) * A) + L * 4 * n * A)   # y0 [E, .], y_m [2E, 2nA]
        os_ = E * (n * A + L * 2 * n * A)                                       # o0 [E, nA], o_m [2E, nA]
        so = 2 if b16 else s
        if name.startswith("tece_edge_ace_fwd"):
            return s * ys + so * os_
        return s * (ys + os_) + so * ys
    if name.startswith("radial_mlp_out"):
        E, n_out = info
        return s * (E * (64 + n_out) + 64 * n_out)
    if name.startswith("rows_accumulate"):
        n_rows, width, n_out = info
        return s * width * (n_rows + 2 * n_out) + 4 * (n_rows + n_out)
    if name.startswith("seg_linear"):
        x_numel, y_numel, w_numel, _flops = info
        return s * (x_numel + y_numel + w_numel)
    if name.startswith("edge_basis_fwd"):
        (E,) = info
        return s * E * (3 + 8 + 16)
    if name.startswith("edge_basis_bwd"):
        (E,) = info
        return s * E * (3 + 8 + 16 + 3)
    return float("nan")


def section8d_bytes(name: str, info, var, s: int) -> float:
    """The per-edge algorithmic bytes of an edge-TP launch as the hot-path
    measurement contract defines them (every per-edge operand counted per
    edge, the weights included; int32 CSR src + perm = 8 B per edge):
      forward   s [E (W + d_Y) + N (d_x + d_out)] + 8 E
      backward  s [E (2 W + 2 d_Y) + N (2 d_x + d_out)] + 8 E
                (without grad_x, as in layer 0: N (d_x + d_out))
    with W = P C, d_x = d1 C, d_out = dout C per node, d_Y = d2."""
    n, E, C = info[:3]
    W, dY, dx, do = var.npath * C, var.d2, var.d1 * C, var.dout * C
    if name.startswith("edge_tp_fwd"):
        return s * (E * (W + dY) + n * (dx + do)) + 8 * E
    if name.startswith("edge_tp_bwd"):
        need_x = info[3]
        return s * (E * (2 * W + 2 * dY) + n * ((2 if need_x else 1) * dx + do)) + 8 * E
    return float("nan")


def measured_traffic(workload: str, entry: str):
    """HBM bytes per call of ``entry`` from the rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary committed under profiles/ for this workload (None when not measured)."""
    path = os.path.join(ROOT, "profiles", f"{workload}_hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        line = line.strip()
        if line.startswith("traffic ") and "=" in line:
            name, val = line[len("traffic "):].rsplit("=", 1)
            if name.strip() == entry:
                return float(val)
    return None


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


MFMA_KERNELS = ("seg_linear", "so2_gemm_bf16")


def mfma_roofline(summ, wall_ms: float):
    """MFMA-bound kernel with the largest share: the segmented per-species GEMM
    (the product basis's Coef contractions and the element-aware linears), on
    the bf16 MFMA with float32 split into three bf16 terms.  ``achieved`` is
    its algorithmic float32 flops (tile rows x columns x k, summed over the
    tile table) over its HIP-event time, against the fp32 peak;
    ``bf16_pipe_frac`` counts the six bf16 products per float32 product
    against the bf16 peak."""
    if "seg_linear" not in summ:
        return None
    cnt, tot_ms, infos = summ["seg_linear"]
    flops = sum(i[3] for i in infos)
    tfs = flops / (tot_ms * 1e-3) / 1e12
    return dict(kernel="seg_linear (k_seg_linear_bx3f + k_seg_linear_ks)", bound="mfma", achieved=round(tfs, 1),
                peak=FP32_PEAK_TFS, unit="TFLOP/s", frac=round(tfs / FP32_PEAK_TFS, 4),
                bf16_pipe_frac=round(BF16X3_PRODUCTS * tfs / BF16_PEAK_TFS, 4),
                flops_per_step=None, launches=cnt, avg_launch_us=round(tot_ms / cnt * 1e3, 1),
                share_of_step=round(tot_ms / wall_ms, 3))


def _lscpu() -> dict:
    """Model name, sockets, cores and threads of this host (lscpu)."""
    import subprocess
    out = {}
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        return out
    want = {"Model name": "model", "Vendor ID": "vendor", "CPU family": "family", "Model": "model_id",
            "Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket", "Thread(s) per core": "threads_per_core",
            "CPU(s)": "cpus", "CPU max MHz": "max_mhz"}
    for line in txt.splitlines():
        if ":" in line:
            k, v = line.split(":", 1)
            if k.strip() in want:
                out[want[k.strip()]] = v.strip()
    return out


def cpu_baseline(wl, reps=3, dtype=torch.float32):
    """CPU oracle on a bounded slice of the workload's structure (same model)."""
    from oracle import model as om
    from oracle import neighbours as onl
    from tace_amd import data

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    structs, what = wl["cpu_slice"]()
    rc = wl["cutoff"]
    stress = "stress" in wl["targets"]

    def graph():
        edges = [onl.neighbour_list(s["positions"], s["cell"], s["pbc"], rc) for s in structs]
        return edges, data.collate(structs, edges, cfg["atomic_numbers"], dtype=dtype)

    n = sum(len(s["numbers"]) for s in structs)
    edges = [onl.neighbour_list(s["positions"], s["cell"], s["pbc"], rc) for s in structs]
    cfg = wl["cfg"](sum(e[0].shape[1] for e in edges) / n)
    torch.manual_seed(0)
    m = om.TACE(cfg).to(dtype)
    for prm in m.parameters():  # frozen, as in the reference calculators
        prm.requires_grad_(False)
    om.compute(m, graph()[1], forces=True, stress=stress)  # warm-up
    t0 = time.perf_counter()
    for _ in range(reps):
        om.compute(m, graph()[1], forces=True, stress=stress)
    dt = time.perf_counter() - t0
    prec = "float32" if dtype == torch.float32 else "float64"
    return dict(value=n * reps / dt, unit="atom-steps/s", cores=threads, kind="port", cpu=_cpu_model(),
                precision=prec,
                sample=f"{n}-atom {what} (same model, {prec}), "
                       f"{reps} timed {'E+F+S' if stress else 'E+F'} steps incl. brute-force NL after 1 warm-up; "
                       f"{dt:.1f} s")


def workloads(args):
    """The bench workloads: the headline water box (configs[2], default), the
    FCC alloy, the ragged crystal batch and the TECE
    bcc Fe box."""
    from tace_amd import configs, structures

    box = 49.7 / 16 * args.n_side
    water = dict(
        metric=METRIC, cutoff=6.0, dt_fs=DT_FS, species=[1, 8], targets=["energy", "forces"],
        structs=lambda: [structures.water_box(n_side=args.n_side, box=box, seed=0)],
        cfg=lambda a: configs.model_cfg("water12k", [1, 8], a),
        describe=lambda nat: f"water box {nat} atoms (configs[2]), E+F, NL rebuilt every step",
        arch=dict(channels=128, L=3, correlation=3, layers=3, cutoff=6.0),
        cpu_slice=lambda: ([structures.water_box(n_side=5, box=49.7 / 16 * 5, seed=1)], "water slice (5^3 H2O)"))
    fcc = dict(
        metric="atom-steps/sec (E+F, fp32) at 1,024 atoms FCC alloy (configs[1])", cutoff=5.0, dt_fs=1.0,
        species=[26, 27, 28, 29], targets=["energy", "forces"],
        structs=lambda: [structures.fcc_alloy(seed=0)],
        cfg=lambda a: configs.model_cfg("fcc1024", [26, 27, 28, 29], a),
        describe=lambda nat: f"4-species FCC alloy {nat} atoms (configs[1]), E+F, NL rebuilt every step",
        arch=dict(channels=128, L=3, correlation=3, layers=2, cutoff=5.0),
        cpu_slice=lambda: ([structures.fcc_alloy(reps=(4, 4, 2), seed=1)], "FCC alloy slice (4x4x2 cells)"))
    ragged = dict(
        metric="atom-steps/sec (E+F+S, fp32) on a 128-crystal ragged batch, 89 species (configs[3])", cutoff=6.0,
        dt_fs=1.0, species=list(structures.MPTRJ_ELEMENTS), targets=["energy", "forces", "stress"],
        structs=lambda: structures.ragged_batch(128, seed=0),
        cfg=lambda a: configs.model_cfg("ragged128", list(structures.MPTRJ_ELEMENTS), a),
        describe=lambda nat: f"128 random triclinic crystals, {nat} atoms (configs[3]), E+F+S, batched GPU NL "
                             f"every step",
        arch=dict(channels=256, L=3, correlation=3, layers=2, cutoff=6.0, species=89),
        cpu_slice=lambda: (structures.ragged_batch(3, nmin=8, nmax=40, seed=1), "3-crystal ragged slice"))
    r = args.fe_reps
    fe = dict(
        metric=f"atom-steps/sec (E+F, fp32) at {2 * r ** 3} atoms bcc Fe, TECE (configs[4])", cutoff=5.0,
        dt_fs=1.0, species=[26], targets=["energy", "forces"],
        structs=lambda: [structures.bcc_fe(reps=(r, r, r), seed=0)],
        cfg=lambda a: configs.model_cfg("tece", [26], a),
        describe=lambda nat: f"bcc Fe {r}^3 box {nat} atoms (configs[4]), TECE E+F, NL rebuilt every step",
        arch=dict(channels=128, L=2, mmax=2, heads=4, edge_ace_hidden=32, correlation=2, layers=2, cutoff=5.0,
                  layer_types="cgtp, uv_so2", product="silu_bilineargate"),
        cpu_slice=lambda: ([structures.bcc_fe(reps=(4, 4, 4), seed=1)], "bcc Fe slice (4^3 cells)"))
    return dict(water12k=water, fcc1024=fcc, ragged128=ragged, fe101k=fe)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="water12k", choices=["water12k", "fcc1024", "ragged128", "fe101k"],
                    help="water12k: the headline water box (configs[2]); fcc1024: FCC alloy (configs[1]); "
                         "ragged128: 128-crystal batch with stress (configs[3]); fe101k: TECE on bcc Fe (configs[4])")
    ap.add_argument("--n-side", type=int, default=16, help="water molecules per box edge (16 -> 12,288 atoms)")
    ap.add_argument("--fe-reps", type=int, default=37, help="bcc cells per box edge (37 -> 101,306 atoms)")
    ap.add_argument("--fe-fp32-mixing", action="store_true",
                    help="fe101k: SO(2) channel mixing in fp32 instead of the configuration's bf16")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernels", action="store_true", help="print the per-kernel breakdown to stderr")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a device copy of 1 GiB five times (reference for the HBM byte counters)")
    args = ap.parse_args()
    if args.steps < 1 or args.warmup < 0:
        ap.error("--steps must be at least 1 and --warmup at least 0")
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
              "(the one-GPU line is the per-GPU share of a spatially decomposed run).", file=sys.stderr)
        sys.exit(2)

    from tace_amd import data, model as pm, ops

    wl = workloads(args)[args.workload]
    dev = torch.device("cuda:0")
    structs = wl["structs"]()
    rc = wl["cutoff"]
    nat = sum(len(s["numbers"]) for s in structs)
    single = len(structs) == 1
    if single:
        s = structs[0]
        pos64 = torch.as_tensor(s["positions"], dtype=torch.float64, device=dev)
        g0 = data.resident_graph(pos64, s["cell"], s["pbc"], torch.zeros(nat, len(wl["species"]), device=dev), rc)
    else:
        g0 = data.gpu_graph(structs, wl["species"], rc, dtype=torch.float32, device=dev)
    E0 = g0["edge_index"].shape[1]
    avg = E0 / nat
    del g0

    cfg = wl["cfg"](avg)
    torch.manual_seed(0)
    model = pm.create_model(cfg).to(dev)
    model.reset_target_property(wl["targets"])
    # inference set-up of the reference calculators (ase/calculator.py:100-102,
    # torchsim.py:142, lammps/mliap.py:38): eval mode, parameters frozen
    model.eval()
    for prm in model.parameters():
        prm.requires_grad_(False)
    mixing = None
    if args.workload == "fe101k" and not args.fe_fp32_mixing:
        mixing = torch.bfloat16  # "fp32 with bf16 channel mixing on MFMA"
        pm.set_tece_channel_mixing(model, mixing)
    if single:
        attrs = data.one_hot(s["numbers"], cfg["atomic_numbers"], torch.float32).to(dev)

        def step():
            return model(data.resident_graph(pos64, s["cell"], s["pbc"], attrs, rc))
    else:
        def step():
            return model(data.gpu_graph(structs, cfg["atomic_numbers"], rc, dtype=torch.float32, device=dev))

    log(f"[bench] {args.workload}: {nat} atoms, {E0} edges (avg {avg:.1f}), warm-up {args.warmup}")
    out = None
    for _ in range(args.warmup):
        out = step()
    torch.cuda.synchronize()
    e_w = "n/a" if out is None else f"{out['energy'].sum().item():.6f}"
    log(f"[bench] warm-up done, E = {e_w}; timing {args.steps} steps")

    # timed region: K steps; a HIP event pair per step (current stream) gives
    # the median, the wall clock around all K the throughput
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        ev[i][0].record()
        out = step()
        ev[i][1].record()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt / args.steps * 1e3
    step_ms = sorted(a.elapsed_time(b) for a, b in ev)
    med = step_ms[len(step_ms) // 2] if len(step_ms) % 2 else 0.5 * sum(step_ms[len(step_ms) // 2 - 1:][:2])
    log(f"[bench] {ms:.2f} ms/step (median {med:.2f}, min {step_ms[0]:.2f}, max {step_ms[-1]:.2f})")

    # the same K steps again, timed the same way, with every native launch
    # bracketed by HIP events on its stream (ops.KernelTimer): the per-kernel
    # times of the roofline objects.  Kept out of the first pass, whose
    # throughput it would lower on launch-bound sizes (two events and their
    # Python per launch: ~1 ms per step at 1,024 atoms)
    ops.TIMER = ops.KernelTimer()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    dt_timed = time.perf_counter() - t1
    timer, ops.TIMER = ops.TIMER, None
    summ = timer.summary()
    log(f"[bench] instrumented pass: {dt_timed / args.steps * 1e3:.2f} ms/step")

    # model only: the same forward + force backward on a graph built once
    if single:
        g_fixed = data.resident_graph(pos64, s["cell"], s["pbc"], attrs, rc)
    else:
        g_fixed = data.gpu_graph(structs, cfg["atomic_numbers"], rc, dtype=torch.float32, device=dev)
    model(g_fixed)
    mev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    for i in range(args.steps):
        mev[i][0].record()
        model(g_fixed)
        mev[i][1].record()
    torch.cuda.synchronize()
    model_ms = sorted(a.elapsed_time(b) for a, b in mev)
    model_med = model_ms[len(model_ms) // 2]
    del g_fixed
    log(f"[bench] model only (graph built once): median {model_med:.2f} ms/step")

    # dominant native entry point -> roofline
    # the matrix-core GEMMs have their own roofline (roofline_mfma)
    phases = timer.phases()
    hbm_kernels = {k: v for k, v in summ.items() if k not in MFMA_KERNELS}
    name, (cnt, tot_ms, infos) = max(hbm_kernels.items(), key=lambda kv: kv[1][1])
    key = name.split(":", 1)[1] if ":" in name else None
    var = ops.find_variant(key) if key else None
    traffic = measured_traffic(args.workload, name)
    src = (f"profiles/{args.workload}_hbm_traffic.md (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)")
    if name.startswith("edge_tp_") and name in phases:
        # the edge-TP backward: its product kernel alone (HIP events around
        # the kernel inside the entry point, tace_mark_phase_event), by the
        # per-edge bytes; the entry point (kernel + grad_y and grad_x sums) and
        # the bytes with the weights counted once per edge pair beside it
        k_cnt, k_ms = phases[name]
        b8d = sum(section8d_bytes(name, i, var, 4) for i in infos)
        bpair = sum(algorithmic_bytes(name, i, var, 4) for i in infos)
        kern = b8d / (k_ms * 1e-3) / 1e9
        entry = b8d / (tot_ms * 1e-3) / 1e9
        roof = dict(kernel=f"{name} (product kernel k_uvu_*_bwd alone)", bound="hbm", achieved=round(kern, 1),
                    peak=HBM_PEAK_GBS, unit="GB/s", frac=round(kern / HBM_PEAK_GBS, 4),
                    traffic=measured_traffic(args.workload, name + " kernel"),
                    traffic_source=src, algorithmic_bytes=round(b8d / cnt),
                    bytes_definition="per edge: s[E(2W+2dY) + N(2dx+dout)] + 8E",
                    avg_launch_us=round(k_ms / k_cnt * 1e3, 1), share_of_step=round(k_ms / (dt_timed * 1e3), 3),
                    entry_point=dict(what="tace_edge_tp_bwd: kernel + grad_y part sum + grad_x sender sum",
                                     achieved=round(entry, 1), frac=round(entry / HBM_PEAK_GBS, 4),
                                     avg_launch_us=round(tot_ms / cnt * 1e3, 1), traffic=traffic,
                                     traffic_over_algorithmic=(round(traffic / (b8d / cnt), 3)
                                                               if traffic is not None else None)),
                    pair_rows=dict(what="weights counted once per edge pair (the model's pair-shared radial "
                                        "weights), entry point time",
                                   algorithmic_bytes=round(bpair / cnt),
                                   frac=round(bpair / (tot_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)))
    else:
        byts = sum(algorithmic_bytes(name, i, var, 4) for i in infos)
        achieved = byts / (tot_ms * 1e-3) / 1e9
        roof = dict(kernel=name, bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(achieved / HBM_PEAK_GBS, 4), traffic=traffic,
                    traffic_source=src if traffic is not None else None,
                    algorithmic_bytes=round(byts / cnt),
                    avg_launch_us=round(tot_ms / cnt * 1e3, 1), share_of_step=round(tot_ms / (dt_timed * 1e3), 3))
    # every edge / scatter kernel of the step: all edge-TP entry points (their
    # grad_y and grad_x sums included) against the per-edge bytes
    agg_b, agg_ms = 0.0, 0.0
    for k, (c, t, inf) in summ.items():
        if k.startswith("edge_tp_fwd") or k.startswith("edge_tp_bwd"):
            v = ops.find_variant(k.split(":", 1)[1])
            agg_b += sum(section8d_bytes(k, i, v, 4) for i in inf)
            agg_ms += t
    if agg_ms > 0:
        a = agg_b / (agg_ms * 1e-3) / 1e9
        roof["aggregate_edge_scatter"] = dict(
            what="all edge-TP forward and backward entry points of the step (every layer; grad_y / grad_x sums "
                 "included), per-edge bytes", bytes_per_step=round(agg_b / args.steps),
            ms_per_step=round(agg_ms / args.steps, 3), achieved=round(a, 1), frac=round(a / HBM_PEAK_GBS, 4),
            target_frac=0.60)
    roof_mfma = mfma_roofline(summ, dt_timed * 1e3)
    if roof_mfma is not None:
        roof_mfma["flops_per_step"] = round(sum(i[3] for i in summ["seg_linear"][2]) / args.steps)
    if args.kernels:
        for k, (c, t, _) in sorted(summ.items(), key=lambda kv: -kv[1][1]):
            log(f"  {t / args.steps:8.3f} ms/step  {c // args.steps:3d} launches/step  {k}")

    res = dict(metric=wl["metric"], value=round(nat * args.steps / dt, 1), unit="atom-steps/s", n_gpus=1,
               steps=args.steps, warmup=args.warmup, ms_per_step=round(ms, 3), higher_is_better=True,
               scaling="weak", vs_baseline=None, dtype="fp32" if mixing is None else "fp32, bf16 channel mixing",
               data="synthetic",
               config=dict(workload=wl["describe"](nat), atoms=nat, edges=int(E0), **wl["arch"],
                           parallelism="single GPU"),
               ms_per_step_median=round(med, 3), model_only_ms_per_step=round(model_med, 3),
               instrumented_ms_per_step=round(dt_timed / args.steps * 1e3, 3),
               ns_per_day=round(1e3 / ms * 86400 * wl["dt_fs"] * 1e-6, 4), dt_fs=wl["dt_fs"], roofline=roof,
               roofline_mfma=roof_mfma,
               peak_mem_gb=round(torch.cuda.max_memory_allocated(dev) / 2 ** 30, 1))
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle) ...")
        res["cpu_baseline"] = cpu_baseline(wl)
        res["cpu_baseline"]["fp64"] = {k: v for k, v in cpu_baseline(wl, dtype=torch.float64).items()
                                       if k in ("value", "unit", "precision", "sample")}
        res["cpu_baseline"]["host"] = _lscpu()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
