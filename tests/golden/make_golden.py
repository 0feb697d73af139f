"""Writes the golden fixtures of the energy/force path from the CPU oracle.

    python tests/golden/make_golden.py [name ...]

Each fixture ``<name>.npz`` holds the structure seed, the model preset and
weight seed, a checksum of the weights, and float64 oracle outputs (energy,
forces, stress where the configuration asks for it).  Weights are not stored:
they are regenerated with ``torch.manual_seed(weight_seed)`` by constructing
the oracle model, and the checksum guards that this reproduces them.

The reference (xvzemin/tace) ships no golden vectors for this path and cannot
be imported here (e3nn / torch_geometric / matscipy absent), so these vectors
come from the oracle, whose own pins are in tests/test_oracle_pins.py.
"""

import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import model as om  # noqa: E402
from oracle import neighbours as onl  # noqa: E402
from tace_amd import configs, data, structures  # noqa: E402


def cases():
    return {
        "si64_fp64": dict(structs=lambda: [structures.si_diamond(seed=1)], preset="si64", stress=True, over={}),
        "fcc1024": dict(structs=lambda: [structures.fcc_alloy(seed=1)], preset="fcc1024", stress=False, over={}),
        "water375": dict(structs=lambda: [structures.water_box(n_side=5, box=49.7 / 16 * 5, seed=2)],
                         preset="water12k", stress=False, over={}),
        # config-5 architecture (TECE) on a 128-atom bcc Fe slice
        "fe128_tece": dict(structs=lambda: [structures.bcc_fe(reps=(4, 4, 4), seed=3)], preset="tece", stress=False,
                           over={}),
        # config-4 architecture (89-species embedding over the MPTrj elements,
        # 256 channels, L = 3, nu = 3, 2 layers, r_c = 6) on four small
        # random triclinic crystals, with stress
        "ragged89_c256": dict(structs=lambda: _ragged(4, (8, 40), seed=5), preset="ragged128", stress=True,
                              over={}, zs=list(structures.MPTRJ_ELEMENTS)),
    }


def _ragged(n_structs, size_range, seed):
    rng = np.random.default_rng(seed)
    return [structures.random_crystal(rng, int(rng.integers(size_range[0], size_range[1] + 1)),
                                      structures.MPTRJ_ELEMENTS) for _ in range(n_structs)]


def weight_checksum(model) -> np.ndarray:
    s1 = sum(p.detach().double().sum().item() for p in model.parameters())
    s2 = sum(p.detach().double().pow(2).sum().item() for p in model.parameters())
    return np.array([s1, s2])


def build(name, spec, weight_seed=0):
    structs = spec["structs"]()
    rc = configs.PRESETS[spec["preset"]]["cutoff"]
    edges = [onl.neighbour_list(s["positions"], s["cell"], s["pbc"], rc) for s in structs]
    zs = spec.get("zs") or sorted({int(z) for s in structs for z in s["numbers"]})
    nat = sum(len(s["positions"]) for s in structs)
    avg = sum(e[0].shape[1] for e in edges) / nat
    cfg = configs.model_cfg(spec["preset"], zs, avg, **spec["over"])
    torch.manual_seed(weight_seed)
    model = om.TACE(cfg).double()
    d = data.collate(structs, edges, cfg["atomic_numbers"], dtype=torch.float64)
    return structs, edges, cfg, model, d


def main(names):
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    for name, spec in cases().items():
        if names and name not in names:
            continue
        t0 = time.time()
        structs, edges, cfg, model, d = build(name, spec)
        out = om.compute(model, d, forces=True, stress=spec["stress"])
        arrays = dict(energy=out["energy"].numpy(), forces=out["forces"].numpy(),
                      weight_checksum=weight_checksum(model), num_edges=np.array([d["edge_index"].shape[1]]),
                      avg_num_neighbors=np.array([cfg["avg_num_neighbors"]]), weight_seed=np.array([0]))
        if spec["stress"]:
            arrays["stress"] = out["stress"].numpy()
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)
        print(f"{name}: E={out['energy'].tolist()} edges={d['edge_index'].shape[1]} in {time.time() - t0:.1f}s",
              flush=True)


if __name__ == "__main__":
    main(sys.argv[1:])
