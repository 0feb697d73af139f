"""Whole-model export: ``TensorModel`` energy + forces (+ stress), or its
LAMMPS ML-IAP form (energies + dE/d(edge vector)), as one ``torch.export``
program.

The reference packages its model for deployment by tracing the forward with
its force derivatives (``make_fx``, symbolic shapes), exporting it with
dynamic atom, edge and graph counts and compiling the program with AOTInductor
(``tace/models/compile/aot.py:206-273`` for the graph model,
``aot.py:291-350`` for LAMMPS; loaded by ``load_aotinductor`` /
``load_lammps_aotinductor``, ``aot.py:276-289, 353-365``, and by the LAMMPS
interface, ``interface/lammps/mliap.py:154-218``).  Here the model is traced
in ``ops.export_mode``: every kernel is a ``tace_amd::`` ``torch.library``
operator with a fake implementation and a registered backward (tensor
products, per-species linears, per-graph sums, the TECE convolution's
kernels, the LAMMPS ghost exchange), the host-side plans are made inside
those operators, and everything else is torch operations, so
``autograd.grad`` for the forces stays inside the graph.  The saved program
(``torch.export.save``) runs the HIP kernels through ``tace_amd.library``
when loaded.

AOTInductor compilation is not applied: on ROCm it generates the
non-operator parts of the graph as Triton kernels, which this build does not
ship.  ``load_program`` / ``load_lammps_program`` return modules with the
call and getters of the reference's ``AOTICompiledTensorModel`` /
``AOTICompiledLammpsModel`` (``aot.py:46-209``), and
``tace_amd.lammps.TACEProgramLammpsCalc`` is ``TACEAOTILammpsCalc`` for these
programs.
"""

from __future__ import annotations

import contextlib
import json
from typing import Dict, List, Optional, Tuple

import torch
from torch.fx.experimental.proxy_tensor import make_fx

from . import library  # noqa: F401  (registers the tace_amd:: operators)
from . import ops

# tace/models/compile/aot.py:23-43
INPUT_KEYS = ("positions", "node_attrs", "edge_index", "edge_shifts", "lattice", "batch", "ptr", "fidelity_idx")
LAMMPS_INPUT_KEYS = ("edge_vector", "node_attrs", "edge_index", "batch", "ptr", "fidelity_idx")
LAMMPS_OUTPUT_KEYS = ("energy", "node_energy", "edge_forces")
GRAPH_FORMAT = "tace_amd.graph.pt2"
LAMMPS_FORMAT = "tace_amd.lammps.pt2"


def _output_keys(model) -> List[str]:
    fl = model.flags
    keys = ["energy", "node_energy"]
    if fl.compute_forces:
        keys.append("forces")
    if fl.compute_stress or fl.compute_virials:
        keys += ["virials", "stress"]
    return keys


def _canonical(data: Dict[str, torch.Tensor], keys) -> Dict[str, torch.Tensor]:
    """``_canonicalize_inputs`` (``aot.py:626-644``): fidelity_idx filled with
    fidelity 0 per graph when absent, tensors contiguous."""
    d = dict(data)
    if "fidelity_idx" in keys and "fidelity_idx" not in d:
        d["fidelity_idx"] = torch.zeros(d["ptr"].numel() - 1, dtype=torch.int64, device=d["ptr"].device)
    return {k: (v.contiguous() if torch.is_tensor(v) else v) for k, v in d.items()}


def _freeze(model):
    model.eval()
    for p in model.parameters():
        p.requires_grad_(False)


def _size_oblivious():
    # sizes treated as >= 2 whatever the sample's, and shape facts the
    # symbolic solver cannot prove (e.g. min(3E, 9E) == 3E) kept as run-time
    # assertions of the program instead of failing the export; no duck sizing
    # (a sample whose graph count + 1 equals 3 would otherwise tie ptr's length
    # to the 3 x 3 lattice dimensions and specialise it)
    cfg = torch.fx.experimental._config
    opts = {k: v for k, v in (("backed_size_oblivious", True), ("use_duck_shape", False)) if hasattr(cfg, k)}
    return cfg.patch(**opts) if opts else contextlib.nullcontext()


def _export(fn, inputs, dyn) -> torch.export.ExportedProgram:
    with _size_oblivious():
        traced = make_fx(fn, tracing_mode="symbolic", _allow_non_fake_inputs=True)(*inputs)
        return torch.export.export(traced, inputs, dynamic_shapes=dyn, strict=False,
                                   prefer_deferred_runtime_asserts_over_guards=True)


def export_program(model, sample_data: Dict[str, torch.Tensor]) -> torch.export.ExportedProgram:
    """``torch.export`` program of ``model`` (a ``TensorModel``, parameters
    frozen, eval mode) on ``sample_data`` (the data dict ``forward`` takes),
    with dynamic numbers of atoms and edges, and of graphs when the sample
    holds more than one (``_graph_dynamic_shapes``, ``aot.py:513-530``).
    Program inputs are the tensors of ``INPUT_KEYS`` in that order (one
    fidelity: ``fidelity_idx`` is accepted and not read); outputs the tensors
    of the model's outputs (energy, node_energy, forces, virials and stress as
    its flags ask)."""
    if getattr(model, "lmp", False):
        raise NotImplementedError("graph export of a model in LAMMPS mode: use export_lammps_program")
    _freeze(model)
    keys = _output_keys(model)

    def fn(*args):
        with ops.export_mode():
            out = model(dict(zip(INPUT_KEYS, args)))
        return tuple(out[k] for k in keys)

    sample = _canonical(sample_data, INPUT_KEYS)
    inputs = tuple(sample[k] for k in INPUT_KEYS)
    atoms = torch.export.Dim("num_atoms", min=2)
    edges = torch.export.Dim("num_edges", min=1)
    if sample["ptr"].numel() - 1 != 1:
        graphs = torch.export.Dim("num_graphs", min=1)
        g, p = {0: graphs}, {0: graphs + 1}
    else:
        g, p = None, None
    dyn = ({0: atoms}, {0: atoms}, {1: edges}, {0: edges}, g, {0: atoms}, p, g)
    return _export(fn, inputs, dyn)


def export_lammps_program(model, sample_data: Dict[str, torch.Tensor]) -> torch.export.ExportedProgram:
    """``export_lammps_aotinductor`` (``aot.py:291-350``) as a ``torch.export``
    program: inputs ``LAMMPS_INPUT_KEYS`` (pair vectors [E, 3], node_attrs of
    the nlocal + nghosts LAMMPS atoms, edge_index [neighbour j, local i],
    batch [nlocal], ptr, fidelity_idx), outputs ``LAMMPS_OUTPUT_KEYS`` (energy
    [1], local node energies [nlocal], edge_forces = dE/d(edge_vector)).
    Dynamic pair, atom and local-atom counts (``_lammps_dynamic_shapes``,
    ``aot.py:542-553``).  The program runs on all nlocal + nghosts rows and
    exchanges ghost rows before every interaction layer >= 1 through the
    LAMMPS data made current with ``library.use_lammps_data``."""
    # what EdgeForcesWrapper does to the model (interface/lammps/mliap.py:25-37)
    model.lmp = True
    model.flags.compute_forces = False
    model.flags.compute_stress = False
    model.flags.compute_virials = False
    model.flags.compute_edge_forces = True
    _freeze(model)

    def fn(*args):
        with ops.export_mode():
            out = model(dict(zip(LAMMPS_INPUT_KEYS, args)))
        return tuple(out[k] for k in LAMMPS_OUTPUT_KEYS)

    sample = _canonical(sample_data, LAMMPS_INPUT_KEYS)
    inputs = tuple(sample[k] for k in LAMMPS_INPUT_KEYS)
    edges = torch.export.Dim("num_edges", min=2)
    total = torch.export.Dim("num_total", min=2)
    local = torch.export.Dim("num_local", min=1)
    dyn = ({0: edges}, {0: total}, {1: edges}, {0: local}, None, None)
    return _export(fn, inputs, dyn)


def _metadata(model, fmt: str, inputs, outputs) -> Dict[str, str]:
    """The reference's package metadata (``_export_metadata``, ``aot.py``)."""
    rf = model.readout_fn
    return {"tace_format": fmt, "tace_input_keys": json.dumps(list(inputs)),
            "tace_output_keys": json.dumps(list(outputs)),
            "tace_atomic_numbers": json.dumps([int(z) for z in model.get_atomic_numbers()]),
            "tace_cutoff": repr(float(model.get_cutoff())),
            "tace_dtype": str(model.get_model_dtype()).replace("torch.", ""),
            "tace_target_property": json.dumps(list(model.get_target_property())),
            "tace_embedding_property": json.dumps(list(getattr(model, "get_embedding_property", lambda: [])())),
            "tace_fidelity_idx": "0", "tace_layers": str(getattr(rf, "num_layers", ""))}


def save_program(model, sample_data: Dict[str, torch.Tensor], path: str) -> str:
    """Exports ``model`` (``export_program``) and writes it to ``path`` (.pt2)
    with the package metadata in its extra files."""
    ep = export_program(model, sample_data)
    meta = _metadata(model, GRAPH_FORMAT, INPUT_KEYS, _output_keys(model))
    torch.export.save(ep, path, extra_files={"tace_metadata": json.dumps(meta)})
    return path


def save_lammps_program(model, sample_data: Dict[str, torch.Tensor], path: str) -> str:
    """``export_lammps_program`` written to ``path`` (.pt2) with its metadata."""
    ep = export_lammps_program(model, sample_data)
    meta = _metadata(model, LAMMPS_FORMAT, LAMMPS_INPUT_KEYS, LAMMPS_OUTPUT_KEYS)
    torch.export.save(ep, path, extra_files={"tace_metadata": json.dumps(meta)})
    return path


def _load(path: str, fmt: str):
    extra = {"tace_metadata": ""}
    ep = torch.export.load(path, extra_files=extra)
    meta = json.loads(extra["tace_metadata"] or "{}")
    if meta.get("tace_format") != fmt:
        raise ValueError(f"{path} is not a {fmt} package ({meta.get('tace_format')!r})")
    return ep, meta


class ExportedTensorModel(torch.nn.Module):
    """A loaded graph program with ``AOTICompiledTensorModel``'s call and
    getters (``aot.py:46-149``): ``forward(data) -> dict``."""

    def __init__(self, program: torch.export.ExportedProgram, metadata: Dict[str, str]):
        super().__init__()
        self.program = program
        self.module_ = program.module()
        self.metadata = metadata
        self.input_keys = tuple(json.loads(metadata["tace_input_keys"]))
        self.output_keys = list(json.loads(metadata["tace_output_keys"]))
        self.atomic_numbers = [int(z) for z in json.loads(metadata["tace_atomic_numbers"])]
        self.cutoff = float(metadata["tace_cutoff"])
        self.model_dtype = getattr(torch, metadata["tace_dtype"])
        self.exported_target_property = list(json.loads(metadata["tace_target_property"]))
        self.target_property = list(self.exported_target_property)
        self.embedding_property = list(json.loads(metadata["tace_embedding_property"]))
        self.fidelity_idx = int(metadata["tace_fidelity_idx"])

    def forward(self, data: Dict[str, torch.Tensor]) -> Dict[str, Optional[torch.Tensor]]:
        d = _canonical(data, self.input_keys)
        missing = [k for k in self.input_keys if k not in d]
        if missing:
            raise KeyError(f"missing program inputs: {missing}")
        outs = self.module_(*[d[k] for k in self.input_keys])
        res: Dict[str, Optional[torch.Tensor]] = dict(energy=None, node_energy=None, forces=None, virials=None,
                                                      stress=None)
        res.update(zip(self.output_keys, outs))
        return res

    def reset_target_property(self, target_property: List[str]) -> None:
        missing = set(target_property) - set(self.exported_target_property)
        if missing:
            raise ValueError(f"the program was not exported with target properties {sorted(missing)}")
        self.target_property = list(target_property)

    def reset_fidelity_idx(self, fidelity_idx: Optional[int] = 0) -> None:
        if fidelity_idx not in (None, 0):
            raise NotImplementedError("one fidelity on the MI355X path")

    def get_fidelity_idx(self) -> int:
        return self.fidelity_idx

    def get_embedding_property(self) -> List[str]:
        return list(self.embedding_property)

    def get_target_property(self) -> List[str]:
        return list(self.target_property)

    def get_model_dtype(self) -> torch.dtype:
        return self.model_dtype

    def get_cutoff(self) -> float:
        return self.cutoff

    def get_atomic_numbers(self) -> List[int]:
        return list(self.atomic_numbers)


class ExportedLammpsModel(torch.nn.Module):
    """A loaded LAMMPS program with ``AOTICompiledLammpsModel``'s call
    (``aot.py:152-209``): ``forward(data) -> (energy, node_energy,
    edge_forces)``; ``data["lmp_data"]`` (or the data made current with
    ``library.use_lammps_data``) serves the ghost exchange."""

    def __init__(self, program: torch.export.ExportedProgram, metadata: Dict[str, str]):
        super().__init__()
        self.program = program
        self.module_ = program.module()
        self.metadata = metadata
        self.input_keys = tuple(json.loads(metadata["tace_input_keys"]))
        self.output_keys = tuple(json.loads(metadata["tace_output_keys"]))
        self.atomic_numbers = [int(z) for z in json.loads(metadata["tace_atomic_numbers"])]
        self.cutoff = float(metadata["tace_cutoff"])
        self.model_dtype = getattr(torch, metadata["tace_dtype"])
        self.fidelity_idx = int(metadata["tace_fidelity_idx"])

    def forward(self, data: Dict[str, torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        d = _canonical(data, self.input_keys)
        missing = [k for k in self.input_keys if k not in d]
        if missing:
            raise KeyError(f"missing LAMMPS program inputs: {missing}")
        args = [d[k].detach() if k == "edge_vector" else d[k] for k in self.input_keys]
        lmp = d.get("lmp_data")
        ctx = library.use_lammps_data(lmp) if lmp is not None else contextlib.nullcontext()
        with ctx:
            outs = self.module_(*args)
        res = dict(zip(self.output_keys, outs))
        return res["energy"], res["node_energy"], res["edge_forces"]


def load_program(path: str) -> ExportedTensorModel:
    """``load_aotinductor`` (``aot.py:276-289``) for a program of ``save_program``."""
    return ExportedTensorModel(*_load(path, GRAPH_FORMAT))


def load_lammps_program(path: str) -> ExportedLammpsModel:
    """``load_lammps_aotinductor`` (``aot.py:353-365``) for a program of
    ``save_lammps_program``."""
    return ExportedLammpsModel(*_load(path, LAMMPS_FORMAT))
