"""Whole-model export: ``TensorModel`` energy + forces (+ stress) as one
``torch.export`` program.

The reference packages its model for deployment by tracing the forward with
its force derivatives (``make_fx``, symbolic shapes), exporting it with
dynamic atom and edge counts and compiling the program with AOTInductor
(``tace/models/compile/aot.py:206-273``; loaded by ``load_aotinductor``,
``aot.py:275-290``, and by the LAMMPS interface, ``interface/lammps/mliap.py:154-218``).
Here the model is traced in ``ops.export_mode``: every kernel is a
``tace_amd::`` ``torch.library`` operator with a fake implementation and a
registered backward (tensor products, per-species linears), the host-side
plans are made inside those operators, and everything else is torch
operations, so ``autograd.grad`` for the forces stays inside the graph.  The
saved program (``torch.export.save``) runs the HIP kernels through
``tace_amd.library`` when loaded.  AOTInductor compilation is not applied: on
ROCm it would generate the non-operator parts of the graph as Triton kernels.
"""

from __future__ import annotations

import contextlib
from typing import Dict, List, Optional

import torch
from torch.fx.experimental.proxy_tensor import make_fx

from . import library  # noqa: F401  (registers the tace_amd:: operators)
from . import ops

INPUT_KEYS = ("positions", "node_attrs", "edge_index", "edge_shifts", "lattice", "batch", "ptr")


def _output_keys(model) -> List[str]:
    fl = model.flags
    keys = ["energy", "node_energy"]
    if fl.compute_forces:
        keys.append("forces")
    if fl.compute_stress or fl.compute_virials:
        keys += ["virials", "stress"]
    return keys


def export_program(model, sample_data: Dict[str, torch.Tensor]) -> torch.export.ExportedProgram:
    """``torch.export`` program of ``model`` (a ``TensorModel``, parameters
    frozen, eval mode) on ``sample_data`` (the data dict ``forward`` takes),
    with dynamic numbers of atoms, edges and graphs.  Program inputs are the
    tensors of ``INPUT_KEYS`` in that order; outputs the tensors of the
    model's outputs (energy, node_energy, forces, virials and stress as its
    flags ask)."""
    if getattr(model, "lmp", False):
        raise NotImplementedError("export the model before switching it to LAMMPS mode")
    model.eval()
    for p in model.parameters():
        p.requires_grad_(False)
    keys = _output_keys(model)

    def fn(*args):
        with ops.export_mode():
            out = model(dict(zip(INPUT_KEYS, args)))
        return tuple(out[k] for k in keys)

    inputs = tuple(sample_data[k] for k in INPUT_KEYS)
    atoms = torch.export.Dim("num_atoms", min=2)
    edges = torch.export.Dim("num_edges", min=2)
    dyn = ({0: atoms}, {0: atoms}, {1: edges}, {0: edges}, None, {0: atoms}, None)
    # sizes treated as >= 2 whatever the sample's, and shape facts the
    # symbolic solver cannot prove (e.g. min(3E, 9E) == 3E) kept as run-time
    # assertions of the program instead of failing the export
    cfg = torch.fx.experimental._config
    ctx = cfg.patch(backed_size_oblivious=True) if hasattr(cfg, "backed_size_oblivious") else contextlib.nullcontext()
    with ctx:
        traced = make_fx(fn, tracing_mode="symbolic", _allow_non_fake_inputs=True)(*inputs)
        return torch.export.export(traced, inputs, dynamic_shapes=dyn, strict=False,
                                   prefer_deferred_runtime_asserts_over_guards=True)


class ExportedTensorModel(torch.nn.Module):
    """A loaded program with ``TensorModel``'s call: ``forward(data) -> dict``."""

    def __init__(self, program: torch.export.ExportedProgram, output_keys: List[str]):
        super().__init__()
        self.program = program
        self.module_ = program.module()
        self.output_keys = list(output_keys)

    def forward(self, data: Dict[str, torch.Tensor]) -> Dict[str, Optional[torch.Tensor]]:
        outs = self.module_(*[data[k] for k in INPUT_KEYS])
        return dict(zip(self.output_keys, outs))


def save_program(model, sample_data: Dict[str, torch.Tensor], path: str) -> str:
    """Exports ``model`` (``export_program``) and writes it to ``path`` (.pt2);
    the output names go into the package's extra files."""
    ep = export_program(model, sample_data)
    torch.export.save(ep, path, extra_files={"tace_outputs": ",".join(_output_keys(model))})
    return path


def load_program(path: str) -> ExportedTensorModel:
    extra = {"tace_outputs": ""}
    ep = torch.export.load(path, extra_files=extra)
    return ExportedTensorModel(ep, extra["tace_outputs"].split(","))
