"""Adapters for the reference's tensor-product plug-in slot.

The reference fills ``self.fused_tp`` of ``O3ScatterTensorProduct``
(``tace/models/_e3nn/fused.py:218-257``) and of ``uuuTensorProduct``
(``fused.py:61-71``) with an accelerated module when an acceleration flag is
set (``tace/utils/env.py:9-64``).  These classes have the same constructor and
``forward`` contract as the OEQ adapter (``tace/models/oeq/_tp_scatter.py:53-93``)
and run the MI355X HIP kernels.  ``HipTeceConvolution`` replaces the TECE
convolution module (``OAM20260705Convolution``) the same way.  A maintainer
selects them with ``TACE_USE_HIP=1`` by adding a few lines to ``fused.py`` /
``inter.py`` / ``env.py``.

Contract (``fused.py:259-271``): ``forward(x [N, irreps_in1.dim], y [E,
irreps_in2.dim], w [E, weight_numel], edge_index [2, E] int64)`` returns
``scatter_sum(tp(x[edge_index[0]], y, w), edge_index[1], dim_size=N)``, with
gradients for x, y and w.  Edges may come in any order.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import library, ops
from .model import e3nn_to_gm, gm_to_e3nn
from .so3 import Irrep, Irreps, generate_paths
from .tece import TeceConvolution

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
        # a registered custom operator (tace_amd.library): traceable by
        # make_fx / torch.export, backward included
        return library.uvu_scatter(x, y, w, edge_index, self.key, self.C)


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
        # ws [N, paths*C]: the per-node weights of the trainable (bilinear-gate)
        # product; only the variants compiled as weighted accept them (the ABI
        # rejects a mismatch)
        return library.uuu(x, y, ws, self.key, self.C)


class HipTeceConvolution(TeceConvolution):
    """Drop-in for ``OAM20260705Convolution``
    (``tace/models/_e3nn/archive/oam_2026_07_05.py:547-823``) as
    ``OAM20260705Interaction._build_rejector`` (``inter.py:469-498``) builds
    it: same constructor arguments, parameters (names, shapes) and
    ``forward(x, w, edge_index, cutoff, wigner, wigner_inv, radial_basis)``,
    x and the result in the e3nn ``mul_ir`` layout of C x (0..lmax).  Runs the
    HIP kernels of ``tace_amd.tece``.  Supported: the interaction's flags
    (``inter.py:450-454``), gate_m0, mmax == lmax, edge_wise_hidden == C and
    ``cutoff`` None (radial basis with ``apply_cutoff``); anything else raises."""

    def __init__(self, mmax: int, lmax: int, num_channel: int, num_head: int, use_temperature: bool,
                 edge_ace_hidden: int, edge_wise_hidden: Optional[int], num_radial_basis: int, so2_linear_type: str,
                 gate_m0: bool, use_so2_edge_ace: bool, use_graph_softmax: bool, reshape_in=None, reshape_out=None,
                 scalar_act=None, tensor_act=None, use_radial_phase: bool = True):
        flags = dict(use_temperature=use_temperature, use_so2_edge_ace=use_so2_edge_ace,
                     use_graph_softmax=use_graph_softmax, use_radial_phase=use_radial_phase, gate_m0=gate_m0)
        if so2_linear_type != "w1" or not all(flags.values()):
            raise NotImplementedError(f"HipTeceConvolution covers so2_linear_type='w1' with {sorted(flags)} all True")
        if edge_wise_hidden not in (None, num_channel):
            raise NotImplementedError("HipTeceConvolution needs edge_wise_hidden == num_channel")
        super().__init__(mmax, lmax, num_channel, num_head, edge_ace_hidden, num_radial_basis)

    def forward(self, x, w, edge_index, cutoff, wigner, wigner_inv, radial_basis):
        if cutoff is not None:
            raise NotImplementedError("HipTeceConvolution: per-edge cutoff rescaling (apply_cutoff=False) is not "
                                      "on the MI355X path")
        Nn, C, L, H = x.shape[0], self.C, self.lmax, self.H
        n = L + 1
        irreps = Irreps([(C, Irrep(l, (-1) ** l)) for l in range(L + 1)])
        x_lc = self.node_components(e3nn_to_gm(x.contiguous(), irreps))
        # the kernels as registered custom operators (tace_amd.library), so
        # the reference's make_fx / torch.export path traces this module
        rowptr, eid = library.receiver_csr(edge_index, Nn)
        src, dst = edge_index[0], edge_index[1]
        blocks = library.tece_rotate_in(x_lc, wigner, src, dst, w, L)
        ms, md, mw = blocks[:n], blocks[n:2 * n], blocks[2 * n:]
        key = self.key_proj.blocks(ms, self.mixing)
        query = self.query_proj.blocks(md, self.mixing)
        rp = self.radial_proj(radial_basis)
        T = self.tmin + (self.tmax - self.tmin) * torch.sigmoid(self.temperature_logit)
        score = library.tece_score(query, key, rp, (T * self.attention_scale).detach(), L, H)
        alpha = library.tece_softmax(score, rowptr, eid)
        o = library.tece_edge_ace(self._shared_input_gemms(mw), L, self.A)
        m = self.linear_down.blocks(o, self.mixing)
        out = library.tece_rotate_out(m, alpha, wigner, rowptr, eid, dst, L, H)
        return gm_to_e3nn(out, irreps)
