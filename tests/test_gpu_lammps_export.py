"""LAMMPS-mode export (GPU): the edge-forces program of
``export.save_lammps_program`` (``export_lammps_aotinductor``,
``tace/models/compile/aot.py:291-350``, with dynamic pair, atom and local-atom
counts), reloaded and run through ``lammps.TACEProgramLammpsCalc`` (the
reference's ``TACEAOTILammpsCalc``, ``interface/lammps/mliap.py:154-218``) on
LAMMPS-style data of another size: local energies and dE/d(edge vector) equal
the CPU oracle's at the float64 bars (1e-10 relative energy, 1e-8 eV/A).  The
cgtp (L = 2) and the TECE architecture; the TECE program runs the
convolution's HIP kernels."""

import pickle

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import neighbours as onl
from tace_amd import configs, data, export, lammps, model as pm, ops, structures

pytestmark = pytest.mark.gpu


class _MliapData:
    """Single-domain stand-in for LAMMPS's KOKKOS ML-IAP data object: pair
    arrays, element types, per-atom energies, and the ghost exchange (ghost
    rows are copies of their owners' rows; the reverse pass sums them back)."""

    def __init__(self, s, rc, zs, device):
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
            sender.append(j if sh == (0, 0, 0) else ghosts.setdefault((j, sh), n + len(ghosts)))
        self.owner = torch.cat([torch.arange(n), torch.tensor([j for (j, _) in ghosts], dtype=torch.int64)]).to(device)
        species = torch.tensor([zs.index(int(z)) for z in s["numbers"]], dtype=torch.int64)
        self.elems = species[self.owner.cpu()].to(device)
        self.rij = vec.to(device)
        self.pair_j = torch.tensor(sender, dtype=torch.int64, device=device)
        self.pair_i = ei[1].to(device)
        self.nlocal, self.ntotal, self.npairs = n, n + len(ghosts), ei.shape[1]
        self.eatoms = torch.zeros(n, dtype=torch.float64, device=device)
        self.energy = None
        self.pair_forces = None
        self.host = (ei, vec, data.one_hot(s["numbers"], zs, torch.float64))

    def forward_exchange(self, inp, out, n):
        out.copy_(inp[self.owner])

    def reverse_exchange(self, gout, gin, n):
        gin.zero_()
        gin.index_add_(0, self.owner, gout)

    def update_pair_forces(self, f):
        self.pair_forces = f.clone()

    def batch(self):
        """The batch dict of TACELammpsCalc._prepare_batch (mliap.py:123-143)."""
        n = self.nlocal
        return {"edge_vector": self.rij.clone(),
                "node_attrs": torch.nn.functional.one_hot(self.elems, num_classes=int(self.elems.max()) + 1)
                .to(torch.float64),
                "edge_index": torch.stack([self.pair_j, self.pair_i]),
                "batch": torch.zeros(n, dtype=torch.int64, device=self.rij.device),
                "ptr": torch.tensor([0, n], dtype=torch.int64, device=self.rij.device)}


def _oracle(ref, d: _MliapData):
    ei, vec, attrs = d.host
    v = vec.clone().requires_grad_(True)
    n = attrs.shape[0]
    E0, e0 = ref.energy(attrs, ei, v, (v ** 2).sum(1, keepdim=True).sqrt() + 1e-9, torch.zeros(n, dtype=torch.int64),
                        torch.tensor([0, n]), 1)
    (gv0,) = torch.autograd.grad(E0.sum(), v)
    return E0.detach(), e0.detach(), gv0


@pytest.mark.parametrize("preset,over", [("si64", dict(num_channel=16)),
                                         ("tece", dict(num_channel=32, edge_ace_hidden=16, num_head=2))])
def test_lammps_program_matches_oracle(cuda, tmp_path, preset, over):
    zs = [26]
    rc = configs.PRESETS[preset]["cutoff"]
    sample = _MliapData(structures.bcc_fe(reps=(2, 2, 2), seed=11), rc, zs, cuda)
    cfg = configs.model_cfg(preset, zs, sample.npairs / sample.nlocal, **over)
    torch.manual_seed(9)
    ref = om.TACE(cfg).double()
    with torch.no_grad():
        for name, prm in ref.named_parameters():   # a non-zero radial phase (zero-initialised in the reference)
            if "radial_proj" in name:
                prm.normal_(0.0, 0.3)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    try:
        model = pm.create_model(cfg)
    finally:
        torch.set_default_dtype(prev)
    pm.load_reference_state_dict(model.readout_fn, ref.state_dict())
    model = model.to(cuda)
    print(f"[lammps export] {preset}: exporting", flush=True)
    path = export.save_lammps_program(model, sample.batch(), str(tmp_path / "lmp.pt2"))
    calc = lammps.TACEProgramLammpsCalc(path, zs, rc, torch.float64)
    calc = pickle.loads(pickle.dumps(calc))   # the package bytes travel, the loaded program does not
    for st in (structures.bcc_fe(reps=(2, 2, 2), seed=11), structures.bcc_fe(reps=(3, 2, 2), seed=13)):
        d = _MliapData(st, rc, zs, cuda)
        assert d.ntotal > d.nlocal
        E0, e0, gv0 = _oracle(ref, d)
        ops.TIMER = ops.KernelTimer()
        try:
            calc.compute_forces(d)
            launched = set(ops.TIMER.summary())
        finally:
            ops.TIMER = None
        assert abs(d.energy - E0[0].item()) < 1e-10 * abs(E0[0].item()), (d.energy, E0)
        assert (d.eatoms.cpu() - e0).abs().max().item() < 1e-10 * e0.abs().max().item()
        f = d.pair_forces.cpu()
        assert f.shape == gv0.shape and (f - gv0).abs().max().item() < 1e-8, (f - gv0).abs().max().item()
        assert any(k.startswith("edge_tp_fwd") for k in launched)
        if preset == "tece":
            # the convolution on its kernels inside the program
            for k in ("edge_rotate_in_fwd", "edge_rotate_in_bwd", "tece_score_fwd", "tece_rotate_out_fwd",
                      "tece_rotate_out_bwd", "tece_edge_ace_fwd"):
                assert k in launched, (k, sorted(launched))


def test_lammps_program_loader_interface(cuda, tmp_path):
    """``load_lammps_program`` returns the (energy, node_energy, edge_forces)
    call of ``AOTICompiledLammpsModel`` with its metadata."""
    zs = [26]
    d = _MliapData(structures.bcc_fe(reps=(2, 2, 2), seed=3), 5.0, zs, cuda)
    cfg = configs.model_cfg("si64", zs, d.npairs / d.nlocal, num_channel=16)
    torch.manual_seed(2)
    model = pm.create_model(cfg).double().to(cuda)
    path = export.save_lammps_program(model, d.batch(), str(tmp_path / "lmp.pt2"))
    prog = export.load_lammps_program(path)
    assert prog.input_keys == export.LAMMPS_INPUT_KEYS and prog.atomic_numbers == zs and prog.cutoff == 5.0
    b = d.batch()
    b["lmp_data"] = d
    E, e, f = prog(b)
    assert E.shape == (1,) and e.shape == (d.nlocal,) and f.shape == (d.npairs, 3)
    with pytest.raises(ValueError):
        export.load_program(path)   # not a graph program
