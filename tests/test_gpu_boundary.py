"""The reference callers' forward calls, replayed on the GPU model.

``TACETorchSimCalc.forward`` (``tace/interface/torchsim/torchsim.py:194-306``)
and ``TACEAseCalc.calculate`` (``tace/interface/ase/calculator.py:129-178``)
line by line, on this build's ``TensorModel``, against the CPU oracle on the
same structures and weights (float64 bars: energy 1e-10 relative, forces and
stress 1e-8).  The TorchSim replay runs an energy+forces model with the
caller's ``compute_stress=True`` override (torchsim.py:131-137), the edge list
in an arbitrary (not receiver-sorted) order with integer unit shifts; the ASE
replay feeds a batch object that, like a torch_geometric ``Batch``, has item
access and ``in`` but no ``get``.
"""

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import neighbours as onl
from tace_amd import configs, data, model as pm, structures

pytestmark = pytest.mark.gpu


class _Batch:
    """Item access and membership only (the subset of torch_geometric's
    ``Batch`` the model path may rely on)."""

    def __init__(self, d):
        self._d = dict(d)

    def __getitem__(self, k):
        return self._d[k]

    def __contains__(self, k):
        return k in self._d


def _setup(seed, targets):
    rng = np.random.default_rng(seed)
    structs = [structures.random_crystal(rng, int(rng.integers(4, 16)), [1, 8, 14]) for _ in range(3)]
    rc = configs.PRESETS["si64"]["cutoff"]
    edges = [onl.neighbour_list(s["positions"], s["cell"], s["pbc"], rc) for s in structs]
    zs = sorted({int(z) for s in structs for z in s["numbers"]})
    nat = sum(len(s["positions"]) for s in structs)
    cfg = configs.model_cfg("si64", zs, sum(e[0].shape[1] for e in edges) / nat, num_channel=16)
    cfg["target_property"] = list(targets)
    torch.manual_seed(seed)
    ref = om.TACE(cfg).double()
    want = om.compute(ref, data.collate(structs, edges, cfg["atomic_numbers"], dtype=torch.float64), forces=True,
                      stress=True)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)  # load_tace builds the model in the checkpoint's dtype
    try:
        model = pm.create_model(cfg)
    finally:
        torch.set_default_dtype(prev)
    model.load_state_dict({f"readout_fn.{k}": v for k, v in ref.state_dict().items()}, strict=True)
    return structs, edges, model, want


def test_torchsim_forward_replay_with_stress_override(cuda):
    structs, edges, model, want = _setup(31, ["energy", "forces"])
    model = model.to(device=cuda, dtype=torch.float64)
    # __init__ (torchsim.py:131-153)
    model.flags.compute_forces = True
    model.flags.compute_stress = True
    model.compute_first_derivative = True
    model.reset_fidelity_idx(None)
    model.eval()
    for p in model.parameters():
        p.requires_grad = False
    torch_element = model.get_torch_element()
    model.atomic_numbers = torch.tensor(model.get_atomic_numbers(), dtype=torch.int64, device=cuda)
    # forward (torchsim.py:233-306): inputs as torch_sim hands them over
    z = torch.as_tensor(np.concatenate([s["numbers"] for s in structs]), device=cuda)
    sys_idx = torch.repeat_interleave(torch.arange(len(structs), device=cuda),
                                      torch.tensor([len(s["numbers"]) for s in structs], device=cuda))
    counts = torch.bincount(sys_idx)
    ptr = torch.cat([counts.new_zeros(1), counts.cumsum(0)])
    node_attrs = torch_element.z2onehot(z).to(torch.float64)
    eis, shs, a = [], [], 0
    for s, (ei, S) in zip(structs, edges):
        eis.append(ei + a)
        shs.append(S)
        a += len(s["positions"])
    ei = torch.as_tensor(np.concatenate(eis, axis=1))
    sh = torch.as_tensor(np.concatenate(shs)).to(torch.int64)  # integer unit shifts
    perm = torch.randperm(ei.shape[1], generator=torch.Generator().manual_seed(4))
    data_dict = dict(ptr=ptr, node_attrs=node_attrs, batch=sys_idx,
                     pbc=torch.tensor([True, True, True], device=cuda),
                     lattice=torch.as_tensor(np.stack([np.asarray(s["cell"]).reshape(3, 3) for s in structs]),
                                             device=cuda),
                     positions=torch.as_tensor(np.concatenate([s["positions"] for s in structs]), device=cuda),
                     edge_index=ei[:, perm].to(cuda), edge_shifts=sh[perm].to(cuda))
    out = model(data_dict)
    results = {"energy": out["energy"].detach(), "forces": out["forces"].detach(), "stress": out["stress"].detach()}
    for key, val in out.items():
        if key not in ("energy", "forces", "stress") and isinstance(val, torch.Tensor):
            results[key] = val.detach()
    E0 = want["energy"]
    assert ((results["energy"].cpu() - E0).abs() / E0.abs()).max().item() < 1e-10
    assert (results["forces"].cpu() - want["forces"]).abs().max().item() < 1e-8
    assert results["stress"].shape == (len(structs), 3, 3)
    assert (results["stress"].cpu() - want["stress"]).abs().max().item() < 1e-8
    assert "virials" in results  # the reference returns virials with stress (adapter.py:106-111)
    # the override off again: no stress
    model.flags.compute_stress = False
    assert model(data_dict)["stress"] is None


def test_ase_calculate_replay(cuda):
    structs, edges, model, want = _setup(32, ["energy", "forces", "stress"])
    model = model.to(device=cuda, dtype=torch.float64)
    model.eval()
    for p in model.parameters():
        p.requires_grad = False
    element = model.get_torch_element()
    target_property = model.get_target_property()
    for g, (s, (ei, S)) in enumerate(zip(structs, edges)):
        # from_atoms (dataset/graph.py:36-161) for one structure, batch_size=1
        n = len(s["positions"])
        batch = _Batch(dict(
            positions=torch.as_tensor(s["positions"], device=cuda),
            node_attrs=element.z2onehot(torch.as_tensor(s["numbers"])).to(torch.float64).to(cuda),
            edge_index=torch.as_tensor(ei, device=cuda),
            edge_shifts=torch.as_tensor(S, dtype=torch.float64, device=cuda),
            lattice=torch.as_tensor(np.asarray(s["cell"]).reshape(1, 3, 3), device=cuda),
            batch=torch.zeros(n, dtype=torch.int64, device=cuda),
            ptr=torch.tensor([0, n], device=cuda),
            fidelity_idx=torch.tensor([0], device=cuda)))
        outs = model(batch)
        results = {}
        for p in target_property:
            if p == "energy":
                results["energy"] = outs[p].detach().cpu().item()
            elif p == "stress":
                results["stress"] = outs[p].detach().cpu().numpy().squeeze(0)
            else:
                results[p] = outs[p].detach().cpu().numpy()
        lo, hi = int(sum(len(x["positions"]) for x in structs[:g])), None
        hi = lo + n
        assert abs(results["energy"] - want["energy"][g].item()) < 1e-10 * abs(want["energy"][g].item())
        assert np.abs(results["forces"] - want["forces"][lo:hi].numpy()).max() < 1e-8
        assert results["stress"].shape == (3, 3)
        assert np.abs(results["stress"] - want["stress"][g].numpy()).max() < 1e-8
