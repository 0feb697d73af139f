"""End-to-end parity of the MI355X model against the CPU oracle (GPU).

Same seeded structure and the same weights (the oracle's state_dict loaded
into the HIP model).  Bars: float64 energies to 1e-10
relative and forces to 1e-8 eV/A; float32 energies to 1e-5 relative and
forces to 1e-4 eV/A (float32 GPU against the float64 oracle).
"""

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import neighbours as onl
from tace_amd import configs, data, model as pm, structures

pytestmark = pytest.mark.gpu

BARS = {torch.float64: (1e-10, 1e-8, 1e-8), torch.float32: (1e-5, 1e-4, 1e-4)}


def _run_pair(structs, preset, cuda, dtype, seed=0, stress=False, avg=None, keep=None, frozen=True, **over):
    edges = [onl.neighbour_list(s["positions"], s["cell"], s["pbc"], configs.PRESETS[preset]["cutoff"])
             for s in structs]
    zs = sorted({int(z) for s in structs for z in s["numbers"]})
    nat = sum(len(s["positions"]) for s in structs)
    if avg is None:
        avg = sum(e[0].shape[1] for e in edges) / nat
    cfg = configs.model_cfg(preset, zs, avg, **over)
    torch.manual_seed(seed)
    ref = om.TACE(cfg).double()
    d64 = data.collate(structs, edges, cfg["atomic_numbers"], dtype=torch.float64)
    want = om.compute(ref, d64, forces=True, stress=stress)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(dtype)
    try:
        gpu = pm.create_model(cfg)
    finally:
        torch.set_default_dtype(prev)
    pm.load_reference_state_dict(gpu.readout_fn, {k: (v.to(dtype) if v.is_floating_point() else v)
                                                  for k, v in ref.state_dict().items()})
    gpu = gpu.to(cuda).eval()   # inference, as the calculators set it
    if frozen:   # the calculators freeze the parameters too
        for prm in gpu.parameters():
            prm.requires_grad_(False)
    if not stress:
        gpu.reset_target_property(["energy", "forces"])
    dg = data.collate(structs, edges, cfg["atomic_numbers"], dtype=dtype, device=cuda)
    got = gpu(dg)
    if keep is not None:
        keep.update(model=gpu, cfg=cfg)
    return got, want


def _check(got, want, dtype, stress=False):
    e_rel, f_abs, s_abs = BARS[dtype]
    E, E0 = got["energy"].double().cpu(), want["energy"]
    assert ((E - E0).abs() / E0.abs()).max().item() < e_rel, (E, E0)
    F, F0 = got["forces"].double().cpu(), want["forces"]
    assert (F - F0).abs().max().item() < f_abs, (F - F0).abs().max().item()
    # the model's forces are small at random init: also require relative agreement
    assert (F - F0).abs().max().item() <= 1e-3 * F0.abs().max().item() + f_abs * 1e-2
    if stress:
        S, S0 = got["stress"].double().cpu(), want["stress"]
        assert (S - S0).abs().max().item() < s_abs


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_si64_energy_forces_stress(cuda, dtype):
    """Config 1 architecture: C=64, L=2, 2 layers, correlation 3, E/F/S."""
    got, want = _run_pair([structures.si_diamond(seed=1)], "si64", cuda, dtype, stress=True)
    _check(got, want, dtype, stress=True)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("frozen", [True, False])
def test_fcc_alloy_slice(cuda, dtype, frozen):
    """Config 2 architecture (C=128, L=3, 2 layers) on a 4x4x2 slice (128 atoms, 4 species);
    frozen parameters run the product basis and the interaction's input linears
    as single autograd nodes with gradient sums in the kernel epilogues,
    trainable ones as one node per operator."""
    got, want = _run_pair([structures.fcc_alloy(reps=(4, 4, 2), seed=2)], "fcc1024", cuda, dtype, frozen=frozen)
    _check(got, want, dtype)


@pytest.mark.parametrize("dtype", [torch.float32])
def test_water_slice(cuda, dtype):
    """Config 3 architecture (C=128, L=3, 3 layers, r_c=6) on 64 molecules."""
    got, want = _run_pair([structures.water_box(n_side=4, box=12.425, seed=3)], "water12k", cuda, dtype)
    _check(got, want, dtype)


def _edge_cases():
    box = np.eye(3) * 20.0
    single = dict(positions=np.zeros((1, 3)), cell=box, numbers=np.array([14]), pbc=(True,) * 3)
    apart = dict(positions=np.array([[1.0, 1.0, 1.0], [8.5, 1.2, 0.9]]), cell=box, numbers=np.array([14, 14]),
                 pbc=(True,) * 3)
    dimer = dict(positions=np.array([[1.0, 1.0, 1.0], [3.2, 1.3, 0.8]]), cell=box, numbers=np.array([14, 14]),
                 pbc=(True,) * 3)
    return single, apart, dimer


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_batch_with_isolated_atoms_and_edgeless_structures(cuda, dtype):
    """The readout's batch rules (tace/models/_e3nn/tace.py:356-418) in one
    ragged batch with stress: a single atom without neighbours (scale and
    shift 0), two atoms beyond the cutoff (no edges, scale and shift kept), a
    close dimer and a crystal, against the oracle at the model bars."""
    single, apart, dimer = _edge_cases()
    structs = [structures.si_diamond(seed=4), single, apart, dimer]
    keep = {}
    got, want = _run_pair(structs, "si64", cuda, dtype, stress=True, keep=keep)
    # the same batch through the batched GPU neighbour search (what the calculators run)
    cfg = keep["cfg"]
    g2 = keep["model"](data.gpu_graph(structs, cfg["atomic_numbers"], configs.PRESETS["si64"]["cutoff"],
                                      dtype=dtype, device=cuda))
    tol = 1e-12 if dtype == torch.float64 else 1e-5
    for k in ("energy", "forces", "stress"):
        d = (g2[k] - got[k]).abs().max().item()
        assert d <= tol * max(got[k].abs().max().item(), 1.0), (k, d)
    e_rel, f_abs, s_abs = BARS[dtype]
    E, E0 = got["energy"].double().cpu(), want["energy"]
    assert ((E - E0).abs() <= e_rel * E0.abs().clamp_min(1.0)).all(), (E, E0)
    F, F0 = got["forces"].double().cpu(), want["forces"]
    assert (F - F0).abs().max().item() < f_abs
    assert F[64:66].abs().max().item() == 0.0   # the single atom and the pair beyond the cutoff feel no force
    S, S0 = got["stress"].double().cpu(), want["stress"]
    assert (S - S0).abs().max().item() < s_abs
    assert S[1:3].abs().max().item() == 0.0


def test_batch_without_any_edge(cuda):
    """A batch whose structures have no edge at all (every kernel launch
    with zero edges): energies equal the oracle's, forces and stress zero."""
    single, apart, _ = _edge_cases()
    got, want = _run_pair([single, apart], "si64", cuda, torch.float64, stress=True, avg=28.0)
    E, E0 = got["energy"].double().cpu(), want["energy"]
    assert ((E - E0).abs() <= 1e-10 * E0.abs().clamp_min(1.0)).all(), (E, E0)
    assert got["forces"].abs().max().item() == 0.0 and want["forces"].abs().max().item() == 0.0
    assert got["stress"].abs().max().item() == 0.0


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_ragged_batch_with_stress(cuda, dtype):
    """Config 4 shape on a small ragged batch: triclinic cells, several species, E/F/S per crystal."""
    rng = np.random.default_rng(5)
    structs = [structures.random_crystal(rng, int(rng.integers(8, 30)), [3, 8, 14, 26, 29]) for _ in range(3)]
    got, want = _run_pair(structs, "ragged128", cuda, dtype, stress=True, num_channel=32)
    _check(got, want, dtype, stress=True)


def test_gpu_neighbour_list_feeds_model(cuda):
    """The GPU-built graph (receiver-grouped edges) gives the oracle-NL energies."""
    s = structures.fcc_alloy(reps=(3, 3, 2), seed=6)
    edges = [onl.neighbour_list(s["positions"], s["cell"], s["pbc"], 5.0)]
    cfg = configs.model_cfg("fcc1024", sorted(set(s["numbers"].tolist())), edges[0][0].shape[1] / len(s["numbers"]),
                            num_channel=32)
    torch.manual_seed(1)
    gpu = pm.create_model(cfg).double().to(cuda).eval()
    gpu.reset_target_property(["energy", "forces"])
    a = gpu(data.collate([s], edges, cfg["atomic_numbers"], dtype=torch.float64, device=cuda))
    g = data.gpu_graph([s], cfg["atomic_numbers"], 5.0, dtype=torch.float64, device=cuda)
    assert bool((g["edge_index"][1][1:] >= g["edge_index"][1][:-1]).all())
    b = gpu(g)
    assert abs(a["energy"] - b["energy"]).max().item() < 1e-10 * abs(a["energy"]).max().item()
    assert (a["forces"] - b["forces"]).abs().max().item() < 1e-10


def test_batched_gpu_neighbour_list_feeds_model(cuda):
    """The batched GPU graph of several crystals (one neighbour search pass)
    gives the oracle-NL energies, forces and stresses of the same batch."""
    rng = np.random.default_rng(8)
    structs = [structures.random_crystal(rng, int(rng.integers(4, 30)), [1, 8, 26, 29]) for _ in range(6)]
    structs.append(structures.si_diamond(seed=3))
    zs = sorted({int(z) for s in structs for z in s["numbers"]})
    edges = [onl.neighbour_list(s["positions"], s["cell"], s["pbc"], 5.0) for s in structs]
    nat = sum(len(s["positions"]) for s in structs)
    cfg = configs.model_cfg("si64", zs, sum(e[0].shape[1] for e in edges) / nat, num_channel=16)
    torch.manual_seed(4)
    gpu = pm.create_model(cfg).double().to(cuda).eval()
    a = gpu(data.collate(structs, edges, cfg["atomic_numbers"], dtype=torch.float64, device=cuda))
    g = data.gpu_graph(structs, cfg["atomic_numbers"], 5.0, dtype=torch.float64, device=cuda)
    assert g["edge_index"].shape[1] == sum(e[0].shape[1] for e in edges)
    assert bool((g["edge_index"][1][1:] >= g["edge_index"][1][:-1]).all())
    b = gpu(g)
    assert (a["energy"] - b["energy"]).abs().max().item() < 1e-10 * a["energy"].abs().max().item()
    assert (a["forces"] - b["forces"]).abs().max().item() < 1e-10
    assert (a["stress"] - b["stress"]).abs().max().item() < 1e-10


@pytest.mark.parametrize("which", ["water", "ragged"])
def test_energies_forces_stress_repeat_bit_for_bit(cuda, which):
    """Every reduction on the path runs in a fixed order (receiver and sender
    CSR sums, per-graph sums of the energies and of the strain gradient), so
    repeated evaluations give the same bits: a water box and a ragged batch
    with stress, float32."""
    if which == "water":
        structs, preset, over = [structures.water_box(n_side=6, box=49.7 / 16 * 6, seed=7)], "water12k", {}
    else:
        rng = np.random.default_rng(9)
        structs = [structures.random_crystal(rng, int(rng.integers(8, 60)), [1, 8, 14, 26, 29]) for _ in range(12)]
        preset, over = "ragged128", dict(num_channel=32)
    zs = sorted({int(z) for s in structs for z in s["numbers"]})
    rc = configs.PRESETS[preset]["cutoff"]
    cfg = configs.model_cfg(preset, zs, 40.0, **over)
    torch.manual_seed(2)
    gpu = pm.create_model(cfg).to(cuda).eval()
    for prm in gpu.parameters():
        prm.requires_grad_(False)
    if which == "water":
        gpu.reset_target_property(["energy", "forces"])
    g = data.gpu_graph(structs, cfg["atomic_numbers"], rc, dtype=torch.float32, device=cuda)
    runs = [gpu(g) for _ in range(3)]
    keys = ["energy", "forces"] + (["stress"] if which == "ragged" else [])
    for r in runs[1:]:
        for k in keys:
            assert torch.equal(r[k], runs[0][k]), k


def test_graph_sum_and_gather(cuda):
    """``ops.graph_sum`` (``tace_graph_sum``) against float64 sums, with empty
    graphs and graphs of one and of several thousand nodes; ``graph_gather``
    and the two backward directions against torch's index_add / index_select."""
    from tace_amd import ops
    counts = torch.tensor([0, 1, 5000, 0, 37, 300, 1])
    ptr = torch.zeros(len(counts) + 1, dtype=torch.int64)
    ptr[1:] = torch.cumsum(counts, 0)
    batch = torch.repeat_interleave(torch.arange(len(counts)), counts)
    g = torch.Generator().manual_seed(3)
    for dtype, w in ((torch.float32, 2), (torch.float64, 9), (torch.float32, 1)):
        v = torch.randn(int(ptr[-1]), w, generator=g, dtype=torch.float64)
        want = torch.zeros(len(counts), w, dtype=torch.float64).index_add_(0, batch, v)
        vg = v.to(dtype).to(cuda).requires_grad_(True)
        got = ops.graph_sum(vg, ptr.to(cuda), batch.to(cuda))
        tol = 1e-12 if dtype == torch.float64 else 1e-5
        assert (got.double().cpu() - want).abs().max().item() <= tol * max(1.0, want.abs().max().item())
        assert torch.equal(got, ops.graph_sum(vg, ptr.to(cuda), batch.to(cuda)))
        up = torch.randn(len(counts), w, generator=g, dtype=torch.float64).to(dtype).to(cuda)
        (gv,) = torch.autograd.grad(got, vg, up)
        assert torch.equal(gv, up.index_select(0, batch.to(cuda)))
        per = up.clone().requires_grad_(True)
        gat = ops.graph_gather(per, ptr.to(cuda), batch.to(cuda))
        assert torch.equal(gat, up.index_select(0, batch.to(cuda)))
        (gp,) = torch.autograd.grad(gat, per, vg.detach())
        assert (gp.double().cpu() - want).abs().max().item() <= tol * max(1.0, want.abs().max().item())
