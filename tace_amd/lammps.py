"""LAMMPS ML-IAP calculator for exported LAMMPS programs.

``TACEProgramLammpsCalc`` is ``TACEAOTILammpsCalc``
(``tace/interface/lammps/mliap.py:154-218``) for the programs of
``tace_amd.export.save_lammps_program``: the same constructor, pickling
(the program's bytes travel, the loaded program does not) and
``compute_forces(data)`` on LAMMPS's KOKKOS ML-IAP data -- pair vectors
``rij``, ``pair_i`` / ``pair_j``, ``elems``, ``nlocal`` / ``ntotal`` /
``npairs``, ``forward_exchange`` / ``reverse_exchange`` for the per-layer
ghost exchange -- writing ``eatoms``, ``energy`` and the pair forces back.
It derives from LAMMPS's ``MLIAPUnified`` when the LAMMPS Python module is
importable (as the reference's class does), else from ``object``.
"""

from __future__ import annotations

import os
import tempfile
from pathlib import Path
from typing import Sequence, Union

import torch

from . import export, library

try:
    from lammps.mliap.mliap_unified_abc import MLIAPUnified
except ImportError:   # LAMMPS not installed: the class still runs on any data object
    MLIAPUnified = object

_SYMBOLS = ("X H He Li Be B C N O F Ne Na Mg Al Si P S Cl Ar K Ca Sc Ti V Cr Mn Fe Co Ni Cu Zn Ga Ge As Se Br Kr "
            "Rb Sr Y Zr Nb Mo Tc Ru Rh Pd Ag Cd In Sn Sb Te I Xe Cs Ba La Ce Pr Nd Pm Sm Eu Gd Tb Dy Ho Er Tm Yb "
            "Lu Hf Ta W Re Os Ir Pt Au Hg Tl Pb Bi Po At Rn Fr Ra Ac Th Pa U Np Pu Am Cm Bk Cf Es Fm Md No Lr Rf "
            "Db Sg Bh Hs Mt Ds Rg Cn Nh Fl Mc Lv Ts Og").split()


class TACEProgramLammpsCalc(MLIAPUnified):
    def __init__(self, package_path: Union[str, Path], atomic_numbers: Sequence[int], cutoff: float,
                 dtype: torch.dtype) -> None:
        if MLIAPUnified is not object:
            MLIAPUnified.__init__(self)
        package_path = Path(package_path)
        self.package_bytes = package_path.read_bytes()
        self.package_filename = package_path.name
        self.element_types = [_SYMBOLS[int(z)] for z in atomic_numbers]
        self.num_species = len(self.element_types)
        self.rcutfac = 0.5 * float(cutoff)
        self.nparams = 1
        self.ndescriptors = 1
        self.dtype = dtype
        self.device = torch.device("cpu")
        self.model = None
        self.initialized = False

    def __getstate__(self):
        state = dict(self.__dict__)
        state["model"] = None
        state["device"] = torch.device("cpu")
        state["initialized"] = False
        return state

    @staticmethod
    def _validate_lammps_data(data, device):
        if not all(hasattr(data, m) for m in ("forward_exchange", "reverse_exchange")):
            raise RuntimeError("TACE requires the KOKKOS ML-IAP interface for ghost exchange. "
                               "Run LAMMPS with '-k on g <Ng> -sf kk'.")
        if device.type != "cuda":
            raise RuntimeError("the MI355X program runs on the GPU (KOKKOS device data)")

    def _initialize_device(self, data):
        device = torch.as_tensor(data.elems).device
        self._validate_lammps_data(data, device)
        self.device = device
        with tempfile.TemporaryDirectory(prefix="tace-amd-lammps-") as tmp:
            path = os.path.join(tmp, self.package_filename)
            with open(path, "wb") as f:
                f.write(self.package_bytes)
            self.model = export.load_lammps_program(path)
        self.initialized = True

    def _prepare_batch(self, data, nlocal, nghosts, species):
        vec = torch.as_tensor(data.rij).to(self.dtype).to(self.device)
        return {
            "edge_vector": vec,
            "node_attrs": torch.nn.functional.one_hot(species.to(self.device), num_classes=self.num_species)
            .to(self.dtype),
            "edge_index": torch.stack([torch.as_tensor(data.pair_j, dtype=torch.int64).to(self.device),
                                       torch.as_tensor(data.pair_i, dtype=torch.int64).to(self.device)], dim=0),
            "batch": torch.zeros(nlocal, dtype=torch.int64, device=self.device),
            "ptr": torch.tensor([0, nlocal], dtype=torch.int64, device=self.device),
        }

    @staticmethod
    def _update_lammps_data(data, node_energy, pair_forces, nlocal):
        pair_forces = pair_forces.to(dtype=torch.float64).contiguous()
        node_energy = node_energy.to(dtype=torch.float64).contiguous()
        eatoms = torch.as_tensor(data.eatoms)
        eatoms.copy_(node_energy[:nlocal])
        data.energy = node_energy[:nlocal].sum().item()
        data.update_pair_forces(pair_forces)

    def compute_forces(self, data):
        nlocal, ntotal, npairs = data.nlocal, data.ntotal, data.npairs
        species = torch.as_tensor(data.elems, dtype=torch.int64)
        if not self.initialized:
            self._initialize_device(data)
        if nlocal == 0 or npairs <= 1:
            return
        torch.cuda.synchronize(self.device)
        batch = self._prepare_batch(data, nlocal, ntotal - nlocal, species)
        with library.use_lammps_data(data):
            _, node_energy, pair_forces = self.model(batch)
        torch.cuda.synchronize(self.device)
        self._update_lammps_data(data, node_energy, pair_forces, nlocal)

    def compute_descriptors(self, data):
        pass

    def compute_gradients(self, data):
        pass
