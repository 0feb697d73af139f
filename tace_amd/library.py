"""The HIP operators of the plug-in slots as torch custom operators.

``torch.library`` operators in the ``tace_amd`` namespace: opaque nodes for
``make_fx`` / ``torch.export`` / AOTInductor, each with a fake (shape-only)
implementation for tracing and its backward registered as a custom operator
too, so a traced ``torch.autograd.grad`` (forces) stays inside the graph.
This is the pattern the reference uses for its LAMMPS exchange operators
(``tace/models/lammps.py:38-80``) and what its export path
(``tace/models/compile/aot.py:206-273``: ``make_fx`` then ``torch.export``)
needs from the operators in the ``fused_tp`` slots.

* ``tace_amd::uvu_scatter(x, y, w, edge_index, key, channels)``: the uvu
  tensor product + receiver scatter of ``O3ScatterTensorProduct.fused_tp``
  (``tace/models/_e3nn/fused.py:259-271``), edges in any order; backward
  ``tace_amd::uvu_scatter_backward`` -> (grad_x, grad_y, grad_w).
* ``tace_amd::uuu(x1, x2, w, key, channels)``: the uuu product of
  ``uuuTensorProduct.fused_tp`` (``fused.py:90-95``), ``w`` the optional
  per-node path weights; backward ``tace_amd::uuu_backward``.

Operators run the library's kernels; there is no CPU implementation.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import ops

Tensor = torch.Tensor


# ------------------------------------------------------------------- uvu ----
@torch.library.custom_op("tace_amd::uvu_scatter", mutates_args=(), device_types="cuda")
def uvu_scatter(x: Tensor, y: Tensor, w: Tensor, edge_index: Tensor, key: str, channels: int) -> Tensor:
    plan = ops.EdgePlan.from_edge_index(edge_index, x.shape[0])
    return ops.launch_edge_tp_fwd(x.contiguous(), y.contiguous(), w.contiguous(), plan, ops.find_variant(key),
                                  channels)


@uvu_scatter.register_fake
def _uvu_scatter_fake(x, y, w, edge_index, key, channels):
    return x.new_empty(x.shape[0], channels * ops.find_variant(key).dout)


@torch.library.custom_op("tace_amd::uvu_scatter_backward", mutates_args=(), device_types="cuda")
def uvu_scatter_backward(x: Tensor, y: Tensor, w: Tensor, edge_index: Tensor, grad_out: Tensor, key: str,
                         channels: int) -> Tuple[Tensor, Tensor, Tensor]:
    plan = ops.EdgePlan.from_edge_index(edge_index, x.shape[0])
    gx, gy, gw = ops.launch_edge_tp_bwd(x.contiguous(), y.contiguous(), w.contiguous(), grad_out.contiguous(), plan,
                                        ops.find_variant(key), channels)
    return gx, gy, gw


@uvu_scatter_backward.register_fake
def _uvu_scatter_backward_fake(x, y, w, edge_index, grad_out, key, channels):
    return torch.empty_like(x), torch.empty_like(y), torch.empty_like(w)


def _uvu_setup(ctx, inputs, output):
    x, y, w, edge_index, key, channels = inputs
    ctx.save_for_backward(x, y, w, edge_index)
    ctx.key, ctx.channels = key, channels


def _uvu_backward(ctx, grad_out):
    x, y, w, edge_index = ctx.saved_tensors
    gx, gy, gw = uvu_scatter_backward(x, y, w, edge_index, grad_out, ctx.key, ctx.channels)
    return gx, gy, gw, None, None, None


uvu_scatter.register_autograd(_uvu_backward, setup_context=_uvu_setup)


# ------------------------------------------------------------------- uuu ----
@torch.library.custom_op("tace_amd::uuu", mutates_args=(), device_types="cuda")
def uuu(x1: Tensor, x2: Tensor, w: Optional[Tensor], key: str, channels: int) -> Tensor:
    return ops.launch_uuu_fwd(x1.contiguous(), x2.contiguous(), None if w is None else w.contiguous(),
                              ops.find_variant(key), channels)


@uuu.register_fake
def _uuu_fake(x1, x2, w, key, channels):
    return x1.new_empty(x1.shape[0], channels * ops.find_variant(key).dout)


@torch.library.custom_op("tace_amd::uuu_backward", mutates_args=(), device_types="cuda")
def uuu_backward(x1: Tensor, x2: Tensor, w: Optional[Tensor], grad_out: Tensor, key: str,
                 channels: int) -> Tuple[Tensor, Tensor, Tensor]:
    g1, g2, gw = ops.launch_uuu_bwd(x1.contiguous(), x2.contiguous(), None if w is None else w.contiguous(),
                                    grad_out.contiguous(), ops.find_variant(key), channels)
    # a weightless product returns an empty weight gradient (schema: tensors only)
    return g1, g2, gw if gw is not None else x1.new_empty(0)


@uuu_backward.register_fake
def _uuu_backward_fake(x1, x2, w, grad_out, key, channels):
    return torch.empty_like(x1), torch.empty_like(x2), torch.empty_like(w) if w is not None else x1.new_empty(0)


def _uuu_setup(ctx, inputs, output):
    x1, x2, w, key, channels = inputs
    ctx.save_for_backward(x1, x2, w)
    ctx.key, ctx.channels, ctx.has_w = key, channels, w is not None


def _uuu_backward(ctx, grad_out):
    x1, x2, w = ctx.saved_tensors
    g1, g2, gw = uuu_backward(x1, x2, w, grad_out, ctx.key, ctx.channels)
    return g1, g2, gw if ctx.has_w else None, None, None


uuu.register_autograd(_uuu_backward, setup_context=_uuu_setup)
