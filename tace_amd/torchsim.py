"""TorchSim calculator over the MI355X model.

``TACETorchSimCalc`` mirrors the reference's TorchSim ``ModelInterface``
(``tace/interface/torchsim/torchsim.py:28-306``): the same constructor
arguments, the same per-call inputs (a TorchSim ``SimState``: ``positions``
[N, 3], ``row_vector_cell`` [B, 3, 3], ``pbc``, ``atomic_numbers`` [N],
``system_idx`` [N]) and the same result dict (``energy`` [B], ``forces``
[N, 3], ``stress`` [B, 3, 3], plus any further model outputs), all detached.

Differences, each forced by this build's scope: ``model`` must be a
``tace_amd`` model instance (the reference's ``load_tace`` package loader is
not part of the hot path; checkpoints load through
``tace_amd.model.load_reference_state_dict``), the acceleration switches
(``enable_oeq`` ...) do not exist (the HIP kernels always run), and the
default neighbour list is the batched HIP cell-list search on the GPU
(``ops.neighbour_list_batch``) instead of ``torch_sim.neighbors.torchsim_nl``
-- the same edge set, built without leaving the device except for the cells.
``torch_sim`` itself is not needed: any object with the ``SimState`` fields
above works.  A ``neighbor_list_fn`` with TorchSim's signature
``(positions, row_vector_cell, pbc, cutoff, system_idx) -> (edge_index,
mapping_system, unit_shifts)`` replaces the default, as in the reference.
"""

from __future__ import annotations

from typing import Callable, Dict, List, Optional

import torch

from . import data as tdata

__all__ = ["TACETorchSimCalc"]


class TACETorchSimCalc(torch.nn.Module):
    """TorchSim model interface over a ``tace_amd.model.TensorModel``."""

    def __init__(self, model: torch.nn.Module, *, device: Optional[torch.device] = None,
                 dtype: torch.dtype = torch.float32, neighbor_list_fn: Optional[Callable] = None,
                 compute_forces: bool = True, compute_stress: bool = True,
                 atomic_numbers: Optional[torch.Tensor] = None, system_idx: Optional[torch.Tensor] = None,
                 fidelity_idx: Optional[int] = None, target_property: Optional[List[str]] = None) -> None:
        super().__init__()
        if not isinstance(model, torch.nn.Module):
            raise TypeError("TACETorchSimCalc takes a tace_amd model instance (load checkpoints with "
                            "tace_amd.model.load_reference_state_dict)")
        self._device = torch.device(device) if device is not None else (
            torch.device("cuda") if torch.cuda.is_available() else torch.device("cpu"))
        self._compute_forces = compute_forces
        self._compute_stress = compute_stress
        self.neighbor_list_fn = neighbor_list_fn
        self._memory_scales_with = "n_atoms_x_density"
        model = model.to(device=self._device, dtype=dtype)
        if target_property:  # load_tace(..., target_property=...), lit_model.py:639-661
            model.reset_target_property(list(target_property))
        # torchsim.py:131-137: the caller's switches override the targets'
        model.flags.compute_forces = self._compute_forces
        model.flags.compute_stress = self._compute_stress
        model.compute_first_derivative = self._compute_forces or self._compute_stress
        model.reset_fidelity_idx(fidelity_idx)
        model.eval()
        for param in model.parameters():
            param.requires_grad = False
        self.model = model
        self._dtype = model.get_model_dtype()
        self.r_max = model.get_cutoff()
        self.torch_element = model.get_torch_element()
        self.atomic_numbers_in_init = atomic_numbers is not None
        self.system_idx_in_init = system_idx is not None
        if (atomic_numbers is not None and system_idx is not None
                and system_idx.shape[0] != atomic_numbers.shape[0]):
            raise ValueError(f"system_idx length {system_idx.shape[0]} must match "
                             f"atomic_numbers length {atomic_numbers.shape[0]}.")
        if atomic_numbers is not None:
            self.atomic_numbers = atomic_numbers.to(device=self._device, dtype=torch.int64)
            self._setup_node_attrs(self.atomic_numbers)
        if system_idx is not None:
            self.system_idx = system_idx.to(device=self._device, dtype=torch.int64)
            self._setup_ptr(self.system_idx)

    @property
    def device(self) -> torch.device:
        return self._device

    @property
    def dtype(self) -> torch.dtype:
        return self._dtype

    @property
    def compute_forces(self) -> bool:
        return self._compute_forces

    @property
    def compute_stress(self) -> bool:
        return self._compute_stress

    def _setup_ptr(self, system_idx: torch.Tensor) -> None:
        counts = torch.bincount(system_idx)
        self.n_systems = len(counts)
        self.n_atoms_per_system = counts.tolist()
        self.ptr = torch.cat([counts.new_zeros(1), counts.cumsum(0)])

    def _setup_node_attrs(self, atomic_numbers: torch.Tensor) -> None:
        zs = self.torch_element.zs
        if int(atomic_numbers.max()) > max(zs) or bool((self.torch_element.z2idx(atomic_numbers.cpu()) < 0).any()):
            raise ValueError("atomic number outside the model's element table")
        self.node_attrs = self.torch_element.z2onehot(atomic_numbers).to(self._dtype)

    def _graph(self, state) -> Dict[str, torch.Tensor]:
        cell = state.row_vector_cell.to(self._device)
        pos = state.positions.to(self._device)
        B = self.n_systems
        pbc = torch.as_tensor(state.pbc).reshape(-1).cpu()
        pbcs = [[bool(v) for v in (pbc.tolist() * 3 if pbc.numel() == 1 else pbc.tolist())]] * B
        if self.neighbor_list_fn is not None:
            edge_index, _mapping, unit_shifts = self.neighbor_list_fn(pos, cell, state.pbc, self.r_max,
                                                                      self.system_idx)
            return dict(edge_index=edge_index.to(self._device), edge_shifts=unit_shifts.to(self._device, self._dtype))
        cells_host = cell.detach().to(torch.float64).reshape(B, 3, 3).cpu().numpy()
        g = tdata.device_graph(pos.detach().to(torch.float64).contiguous(), self.n_atoms_per_system,
                               list(cells_host), pbcs, self.r_max)
        g["edge_shifts"] = g["edge_shifts"].to(self._dtype)
        return g

    def forward(self, state, **_kwargs: object) -> Dict[str, torch.Tensor]:
        """Energies [B], forces [N, 3] and stresses [B, 3, 3] of the systems of
        ``state`` (``torchsim.py:194-306``)."""
        if self.atomic_numbers_in_init:
            if state.positions.shape[0] != self.atomic_numbers.shape[0]:
                raise ValueError(f"Expected {self.atomic_numbers.shape[0]} atoms, got {state.positions.shape[0]}.")
        else:
            atomic_numbers = state.atomic_numbers.to(device=self._device, dtype=torch.int64)
            if not hasattr(self, "atomic_numbers") or not torch.equal(atomic_numbers, self.atomic_numbers):
                self._setup_node_attrs(atomic_numbers)
                self.atomic_numbers = atomic_numbers
        if self.system_idx_in_init:
            if state.system_idx.shape[0] != self.system_idx.shape[0]:
                raise ValueError(f"Expected system_idx of length {self.system_idx.shape[0]}, "
                                 f"got {state.system_idx.shape[0]}.")
        else:
            system_idx = state.system_idx.to(device=self._device, dtype=torch.int64)
            if not hasattr(self, "system_idx") or not torch.equal(system_idx, self.system_idx):
                self._setup_ptr(system_idx)
                self.system_idx = system_idx
        d = dict(ptr=self.ptr, node_attrs=self.node_attrs, batch=self.system_idx,
                 lattice=state.row_vector_cell.to(self._device, self._dtype).reshape(-1, 3, 3),
                 positions=state.positions.to(self._device, self._dtype), **self._graph(state))
        out = self.model(d)
        results: Dict[str, torch.Tensor] = {}
        energy = out.get("energy")
        results["energy"] = energy.detach() if energy is not None else torch.zeros(self.n_systems,
                                                                                    device=self._device)
        if self.compute_forces and out.get("forces") is not None:
            results["forces"] = out["forces"].detach()
        if self.compute_stress and out.get("stress") is not None:
            results["stress"] = out["stress"].detach()
        for key, val in out.items():
            if key not in ("energy", "forces", "stress") and isinstance(val, torch.Tensor):
                results[key] = val.detach()
        return results
