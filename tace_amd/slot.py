"""Adapters for the reference's tensor-product plug-in slot.

The reference fills ``self.fused_tp`` of ``O3ScatterTensorProduct``
(``tace/models/_e3nn/fused.py:218-257``) and of ``uuuTensorProduct``
(``fused.py:61-71``) with an accelerated module when an acceleration flag is
set (``tace/utils/env.py:9-64``).  These classes have the same constructor and
``forward`` contract as the OEQ adapter (``tace/models/oeq/_tp_scatter.py:53-93``)
and run the MI355X HIP kernels; ``INTEGRATION.md`` shows the lines a
maintainer adds to ``fused.py`` / ``env.py`` to select them with
``TACE_USE_HIP=1``.

Contract (``fused.py:259-271``): ``forward(x [N, irreps_in1.dim], y [E,
irreps_in2.dim], w [E, weight_numel], edge_index [2, E] int64)`` returns
``scatter_sum(tp(x[edge_index[0]], y, w), edge_index[1], dim_size=N)``, with
gradients for x, y and w.  Edges may come in any order.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import ops
from .so3 import Irreps, generate_paths

ACCELERATION_ENV_NAME = "TACE_USE_HIP"


def _irreps(x) -> Irreps:
    return Irreps(str(x).replace(" ", ""))


def _ls(irreps: Irreps):
    return [ir.l for _, ir in irreps]


class e3nnHipScatterTensorProduct(torch.nn.Module):
    """Fused uvu tensor product + receiver scatter on the HIP kernels."""

    def __init__(self, irreps_in1, irreps_in2, irreps_out, instructions: Optional[Sequence[tuple]] = None):
        super().__init__()
        self.irreps_in1, self.irreps_in2 = _irreps(irreps_in1), _irreps(irreps_in2)
        out = _irreps(irreps_out)
        # with explicit instructions the caller passes the per-path output
        # irreps (fused.py:200-201); the targets are their distinct irreps
        target = out.regroup() if instructions is not None else out
        paths, self.irreps_out = generate_paths(target, self.irreps_in1, self.irreps_in2, "uvu")
        if instructions is not None:
            got = [(int(i[0]), int(i[1]), int(i[2])) for i in instructions]
            if got != [tuple(p) for p in paths] or any(i[3] != "uvu" for i in instructions):
                raise ValueError("e3nnHipScatterTensorProduct: instructions differ from generate_paths(mode='uvu') "
                                 "(tace/models/_e3nn/paths.py:30-71); only that path order is compiled")
            if str(self.irreps_out) != str(out):
                raise ValueError(f"irreps_out {out} does not match the path outputs {self.irreps_out}")
        muls = {m for m, _ in self.irreps_in1}
        if len(muls) != 1 or any(m != 1 for m, _ in self.irreps_in2):
            raise ValueError("the HIP uvu kernels need one multiplicity for irreps_in1 and 1 for irreps_in2")
        self.C = muls.pop()
        self.weight_numel = self.C * len(paths)
        lout = sorted({ir.l for _, ir in self.irreps_out})
        self.key = ops.variant_key("uvu", _ls(self.irreps_in1), _ls(self.irreps_in2), lout)
        ops.find_variant(self.key)  # raises if this variant is not compiled in

    def forward(self, x: torch.Tensor, y: torch.Tensor, w: torch.Tensor, edge_index: torch.Tensor) -> torch.Tensor:
        plan = ops.EdgePlan.from_edge_index(edge_index, x.shape[0])
        return ops.edge_tp_scatter(x, y, w, plan, ops.find_variant(self.key), self.C)


class e3nnHipUuuTensorProduct(torch.nn.Module):
    """Weightless uuu tensor product (``uuuTensorProduct.fused_tp(x, y, ws=None)``)."""

    def __init__(self, irreps_in1, irreps_in2, irreps_out, identical_inputs: bool = False):
        super().__init__()
        self.irreps_in1, self.irreps_in2 = _irreps(irreps_in1), _irreps(irreps_in2)
        out = _irreps(irreps_out)
        paths, self.irreps_out = generate_paths(out, self.irreps_in1, self.irreps_in2, "uuu", identical_inputs)
        muls = {m for m, _ in self.irreps_in1} | {m for m, _ in self.irreps_in2}
        if len(muls) != 1:
            raise ValueError("the HIP uuu kernels need one multiplicity across both inputs")
        self.C = muls.pop()
        self.key = ops.variant_key("uuu", _ls(self.irreps_in1), _ls(self.irreps_in2),
                                   sorted({ir.l for _, ir in out}))
        ops.find_variant(self.key)

    def forward(self, x: torch.Tensor, y: torch.Tensor, ws: Optional[torch.Tensor] = None) -> torch.Tensor:
        if ws is not None:
            raise ValueError("the weighted (bilinear-gate) uuu product is not on the MI355X path")
        return ops.uuu_tp(x, y, ops.find_variant(self.key), self.C)
