"""LAMMPS ML-IAP mode (GPU): pair vectors in, local energies and
edge_forces = dE/d(edge_vector) out (``adapter.py:140-149, 286-312``,
``interface/lammps/mliap.py:25-151``), on a periodic cell presented the way
LAMMPS does: local atoms plus ghost images, edges [neighbour j, local i], a
ghost exchange object.  Checked against the CPU oracle's energy and its
gradient with respect to the edge vectors (float64 bars: 1e-10 relative
energy, 1e-8 eV/A)."""

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import neighbours as onl
from tace_amd import configs, data, model as pm, structures

pytestmark = pytest.mark.gpu


class _Exchange:
    """Single-domain stand-in for LAMMPS's KOKKOS ML-IAP data: ghost rows are
    copies of their owners' rows; the reverse pass sums them back."""

    def __init__(self, owner: torch.Tensor):
        self.owner = owner

    def forward_exchange(self, inp, out, n):
        out.copy_(inp[self.owner])

    def reverse_exchange(self, gout, gin, n):
        gin.zero_()
        gin.index_add_(0, self.owner, gout)


def _lammps_inputs(s, rc, zs, device):
    ei, S = onl.neighbour_list(s["positions"], s["cell"], s["pbc"], rc)
    pos = torch.as_tensor(np.asarray(s["positions"]), dtype=torch.float64)
    cell = torch.as_tensor(np.asarray(s["cell"]), dtype=torch.float64)
    ei = torch.as_tensor(np.asarray(ei), dtype=torch.int64)
    S = torch.as_tensor(np.asarray(S), dtype=torch.float64)
    n = pos.shape[0]
    vec = pos[ei[1]] - pos[ei[0]] + S @ cell
    ghosts, sender = {}, []
    for k in range(ei.shape[1]):
        j, sh = int(ei[0, k]), tuple(int(v) for v in S[k].tolist())
        if sh == (0, 0, 0):
            sender.append(j)
        else:
            sender.append(ghosts.setdefault((j, sh), n + len(ghosts)))
    owner = torch.cat([torch.arange(n), torch.tensor([j for (j, _) in ghosts], dtype=torch.int64)])
    attrs = data.one_hot(s["numbers"], zs, torch.float64)
    lmp = dict(edge_vector=vec.to(device).requires_grad_(True), node_attrs=attrs[owner].to(device),
               edge_index=torch.stack([torch.tensor(sender), ei[1]]).to(device),
               batch=torch.zeros(n, dtype=torch.int64, device=device),
               ptr=torch.tensor([0, n], dtype=torch.int64, device=device),
               lmp_data=_Exchange(owner.to(device)), natoms=(n, len(ghosts)))
    return lmp, (ei, S, vec, attrs, len(ghosts))


@pytest.mark.parametrize("preset,over", [("si64", {}), ("tece", dict(num_channel=32, edge_ace_hidden=16, num_head=2))])
def test_lammps_edge_forces_match_oracle(cuda, preset, over):
    s = structures.bcc_fe(reps=(2, 2, 2), seed=11)
    rc = configs.PRESETS[preset]["cutoff"]
    zs = [26]
    lmp, (ei, S, vec, attrs, nghost) = _lammps_inputs(s, rc, zs, cuda)
    assert nghost > 0
    cfg = configs.model_cfg(preset, zs, ei.shape[1] / len(s["numbers"]), **over)
    torch.manual_seed(9)
    ref = om.TACE(cfg).double()
    v = vec.clone().requires_grad_(True)
    n = attrs.shape[0]
    E0, e0 = ref.energy(attrs, ei, v, (v ** 2).sum(1, keepdim=True).sqrt() + 1e-9, torch.zeros(n, dtype=torch.int64),
                        torch.tensor([0, n]), 1)
    (gv0,) = torch.autograd.grad(E0.sum(), v)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    try:
        model = pm.create_model(cfg)
    finally:
        torch.set_default_dtype(prev)
    pm.load_reference_state_dict(model.readout_fn, ref.state_dict())
    model = model.to(cuda)
    # what interface/lammps/mliap.py:25-37 does to the model
    model.lmp = True
    model.flags.compute_forces = False
    model.flags.compute_edge_forces = True
    for p in model.parameters():
        p.requires_grad = False
    out = model(lmp)
    E = out["energy"].cpu()
    assert abs(E[0] - E0[0]).item() < 1e-10 * abs(E0[0]).item(), (E, E0)
    assert (out["node_energy"].cpu() - e0.detach()).abs().max().item() < 1e-10 * e0.abs().max().item()
    ef = out["edge_forces"].cpu()
    assert ef.shape == vec.shape
    assert (ef - gv0).abs().max().item() < 1e-8, (ef - gv0).abs().max().item()


def test_lammps_mode_rejects_ghost_receivers(cuda):
    s = structures.bcc_fe(reps=(2, 2, 2), seed=11)
    lmp, _ = _lammps_inputs(s, 5.0, [26], cuda)
    ei = lmp["edge_index"].clone()
    ei[1, 0] = lmp["natoms"][0]  # a ghost as receiver
    lmp["edge_index"] = ei
    cfg = configs.model_cfg("si64", [26], 50.0, num_channel=16)
    model = pm.create_model(cfg).double().to(cuda)
    model.flags.compute_edge_forces = True
    with pytest.raises(ValueError):
        model(lmp)


def test_atomic_virials_sum_to_the_virial(cuda):
    """Per-atom virials (utils.py:82-115) from the edge forces add up to the
    strain-derivative virial of each structure, and the edge forces are the
    oracle's dE/d(edge vector)."""
    rng = np.random.default_rng(21)
    structs = [structures.random_crystal(rng, int(rng.integers(6, 14)), [3, 8, 26]) for _ in range(2)]
    edges = [onl.neighbour_list(s["positions"], s["cell"], s["pbc"], 5.0) for s in structs]
    zs = sorted({int(z) for s in structs for z in s["numbers"]})
    nat = sum(len(s["positions"]) for s in structs)
    cfg = configs.model_cfg("si64", zs, sum(e[0].shape[1] for e in edges) / nat, num_channel=16)
    torch.manual_seed(2)
    ref = om.TACE(cfg).double()
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    try:
        model = pm.create_model(cfg)
    finally:
        torch.set_default_dtype(prev)
    pm.load_reference_state_dict(model.readout_fn, ref.state_dict())
    model = model.to(cuda)
    model.reset_target_property(["energy", "forces", "virials", "atomic_virials", "atomic_stresses"])
    d = data.collate(structs, edges, cfg["atomic_numbers"], dtype=torch.float64, device=cuda)
    out = model(d)
    av = out["atomic_virials"].cpu()
    V = out["virials"].cpu()
    b = d["batch"].cpu()
    for g in range(len(structs)):
        Vg = av[b == g].sum(0)
        assert (Vg - V[g]).abs().max().item() < 1e-9 * max(1.0, V[g].abs().max().item()), (Vg, V[g])
    assert (av - av.transpose(-1, -2)).abs().max().item() == 0.0
    # edge forces against the oracle
    d64 = data.collate(structs, edges, cfg["atomic_numbers"], dtype=torch.float64)
    src, dst = d64["edge_index"]
    vec = (d64["positions"][dst] - d64["positions"][src]
           + torch.einsum("ni,nij->nj", d64["edge_shifts"], d64["lattice"][d64["batch"][src]])).requires_grad_(True)
    n = d64["node_attrs"].shape[0]
    E0, _ = ref.energy(d64["node_attrs"], d64["edge_index"], vec, (vec ** 2).sum(1, keepdim=True).sqrt() + 1e-9,
                       d64["batch"], d64["ptr"], 2)
    (gv,) = torch.autograd.grad(E0.sum(), vec)
    assert (out["edge_forces"].cpu() - gv).abs().max().item() < 1e-8



@pytest.mark.parametrize("preset", ["si64", "tece"])
def test_lammps_two_domains_match_single_domain(cuda, tmp_path, preset):
    """The periodic cell split into two LAMMPS domains (x < L/2 and the rest),
    each with its own ghosts, run by two processes (one per domain, as MPI
    ranks would be) on the one GPU with the per-layer ghost exchange over a
    gloo stand-in for LAMMPS's communication: the two local energies add up
    to the oracle's energy and every edge's dE/d(edge vector) equals the
    oracle's (float64 bars)."""
    import os
    import socket
    import sys

    import torch.multiprocessing as mp

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import _lammps_domains as ld

    setup = ld.setup(preset)
    with socket.socket() as sk:
        sk.bind(("127.0.0.1", 0))
        port = sk.getsockname()[1]
    mp.spawn(ld.worker, args=(port, str(tmp_path), preset), nprocs=2, join=True)
    ei, vec, E0, gv0, dom = setup["ei"], setup["vec"], setup["E0"], setup["gv0"], setup["dom"]
    E = 0.0
    for d in (0, 1):
        r = np.load(tmp_path / f"dom{d}.npz")
        E += float(r["energy"][0])
        mine = (dom[ei[1]] == d).nonzero().squeeze(1).numpy()
        assert (r["mine"] == mine).all()
        assert np.abs(r["edge_forces"] - gv0.numpy()[mine]).max() < 1e-8
        assert int(r["n_ghost_foreign"][0]) > 0   # the exchange really crossed domains
    assert abs(E - float(E0[0])) < 1e-10 * abs(float(E0[0])), (E, E0)
