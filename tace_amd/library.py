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
* The uvu and uuu backward operators are differentiable themselves (double
  backward for training with a force loss): their backward is written with
  the forward and backward operators.
* ``tace_amd::receiver_csr``, ``tece_rotate_in``, ``tece_score``,
  ``tece_softmax``, ``tece_edge_ace``, ``tece_rotate_out`` (each with a
  ``*_backward``): the kernels of the TECE convolution slot
  (``HipTeceConvolution``) and of exported TECE programs, edge features as
  lists of SO(2) blocks.
* ``tace_amd::graph_sum`` / ``graph_gather``: fixed-order per-graph sums
  (energies, the strain gradient) and their transpose.
* ``tace_amd::lammps_forward_exchange`` / ``lammps_reverse_exchange``: the
  per-layer ghost exchange of exported LAMMPS programs
  (``tace/models/lammps.py:38-80``), through ``use_lammps_data``.

Operators run the library's kernels; there is no CPU implementation.
"""

from __future__ import annotations

import threading
from contextlib import contextmanager
from typing import Any, Iterator, List, Optional, Tuple

import torch

from . import ops

Tensor = torch.Tensor


# ------------------------------------------------------------ per graph ----
# Per-graph sums of node rows and their transpose (the gather of per-graph
# rows to the nodes), each the other's backward: the energy sum and the strain
# displacement of stress (``scatter_sum(..., batch)``, tace/models/_e3nn/tace.py:364, 416;
# ``sym[batch]``, tace/models/utils.py:50-79) in a fixed order.
@torch.library.custom_op("tace_amd::graph_sum", mutates_args=(), device_types="cuda")
def graph_sum(values: Tensor, ptr: Tensor, batch: Tensor) -> Tensor:
    return ops._graph_sum(values, ptr)


@graph_sum.register_fake
def _graph_sum_fake(values, ptr, batch):
    return values.new_empty((ptr.shape[0] - 1,) + tuple(values.shape[1:]))


@torch.library.custom_op("tace_amd::graph_gather", mutates_args=(), device_types="cuda")
def graph_gather(values: Tensor, ptr: Tensor, batch: Tensor) -> Tensor:
    return values.index_select(0, batch)


@graph_gather.register_fake
def _graph_gather_fake(values, ptr, batch):
    return values.new_empty((batch.shape[0],) + tuple(values.shape[1:]))


def _graph_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[1], inputs[2])


def _graph_sum_backward(ctx, g):
    ptr, batch = ctx.saved_tensors
    return graph_gather(g, ptr, batch), None, None


def _graph_gather_backward(ctx, g):
    ptr, batch = ctx.saved_tensors
    return graph_sum(g, ptr, batch), None, None


graph_sum.register_autograd(_graph_sum_backward, setup_context=_graph_setup)
graph_gather.register_autograd(_graph_gather_backward, setup_context=_graph_setup)


# ------------------------------------------------------- LAMMPS exchange ----
# The per-layer ghost exchange of an exported LAMMPS program
# (tace/models/lammps.py:13-80: ``use_lammps_mliap_data`` and the
# lammps_forward_exchange / lammps_reverse_exchange operators).  A program has
# no Python object to hold LAMMPS's ML-IAP data, so the caller makes it current
# for the call (``use_lammps_data``) and the operators read it from there.
_LAMMPS_DATA = threading.local()


@contextmanager
def use_lammps_data(data: Any) -> Iterator[None]:
    """Makes ``data`` (LAMMPS KOKKOS ML-IAP data: forward_exchange /
    reverse_exchange) the exchange target of the exported program's operators
    on this thread for the duration of the block."""
    prev = getattr(_LAMMPS_DATA, "data", None)
    _LAMMPS_DATA.data = data
    try:
        yield
    finally:
        _LAMMPS_DATA.data = prev


def _lammps_data():
    data = getattr(_LAMMPS_DATA, "data", None)
    if data is None:
        raise RuntimeError("LAMMPS ghost exchange called outside use_lammps_data(...)")
    return data


@torch.library.custom_op("tace_amd::lammps_forward_exchange", mutates_args=(), device_types="cuda")
def lammps_forward_exchange(rows: Tensor) -> Tensor:
    """Ghost rows replaced by their owners' rows (rows in LAMMPS atom order)."""
    flat = rows.reshape(rows.shape[0], -1).contiguous()
    out = torch.empty_like(flat)
    _lammps_data().forward_exchange(flat, out, out.shape[1])
    return out.view(rows.shape)


@lammps_forward_exchange.register_fake
def _lammps_forward_exchange_fake(rows):
    return torch.empty_like(rows)


@torch.library.custom_op("tace_amd::lammps_reverse_exchange", mutates_args=(), device_types="cuda")
def lammps_reverse_exchange(grad: Tensor) -> Tensor:
    """The transpose: ghost-row gradients summed into their owners' rows."""
    flat = grad.reshape(grad.shape[0], -1).contiguous()
    out = torch.empty_like(flat)
    _lammps_data().reverse_exchange(flat, out, out.shape[1])
    return out.view(grad.shape)


@lammps_reverse_exchange.register_fake
def _lammps_reverse_exchange_fake(grad):
    return torch.empty_like(grad)


def _lammps_forward_exchange_backward(ctx, g):
    return lammps_reverse_exchange(g)


lammps_forward_exchange.register_autograd(_lammps_forward_exchange_backward)


# ------------------------------------------------------------------- uvu ----
@torch.library.custom_op("tace_amd::uvu_scatter", mutates_args=(), device_types="cuda")
def uvu_scatter(x: Tensor, y: Tensor, w: Tensor, edge_index: Tensor, key: str, channels: int,
                layout: int = 0) -> Tensor:
    plan = ops.EdgePlan.from_edge_index(edge_index, x.shape[0])
    return ops.launch_edge_tp_fwd(x.contiguous(), y.contiguous(), w.contiguous(), plan, ops.find_variant(key),
                                  channels, layout)


@uvu_scatter.register_fake
def _uvu_scatter_fake(x, y, w, edge_index, key, channels, layout=0):
    return x.new_empty(x.shape[0], channels * ops.find_variant(key).dout)


@torch.library.custom_op("tace_amd::uvu_scatter_backward", mutates_args=(), device_types="cuda")
def uvu_scatter_backward(x: Tensor, y: Tensor, w: Tensor, edge_index: Tensor, grad_out: Tensor, key: str,
                         channels: int, layout: int = 0) -> Tuple[Tensor, Tensor, Tensor]:
    plan = ops.EdgePlan.from_edge_index(edge_index, x.shape[0])
    gx, gy, gw = ops.launch_edge_tp_bwd(x.contiguous(), y.contiguous(), w.contiguous(), grad_out.contiguous(), plan,
                                        ops.find_variant(key), channels, layout)
    return gx, gy, gw


@uvu_scatter_backward.register_fake
def _uvu_scatter_backward_fake(x, y, w, edge_index, grad_out, key, channels, layout=0):
    return torch.empty_like(x), torch.empty_like(y), torch.empty_like(w)


def _uvu_setup(ctx, inputs, output):
    x, y, w, edge_index, key, channels, layout = inputs
    ctx.save_for_backward(x, y, w, edge_index)
    ctx.key, ctx.channels, ctx.layout = key, channels, layout


def _uvu_backward(ctx, grad_out):
    x, y, w, edge_index = ctx.saved_tensors
    gx, gy, gw = uvu_scatter_backward(x, y, w, edge_index, grad_out, ctx.key, ctx.channels, ctx.layout)
    return gx, gy, gw, None, None, None, None


uvu_scatter.register_autograd(_uvu_backward, setup_context=_uvu_setup)


# Double backward (training with a force loss, create_graph=True).  The
# product is trilinear in (x, y, w) and its backward (gx, gy, gw) is
# multilinear in (x, y, w, g) with each output free of its own operand:
# gx(y, w, g), gy(x, w, g), gw(x, y, g).  For upstream gradients (ax, ay, aw)
# of (gx, gy, gw):
#   d/dg = TP(ax, y, w) + TP(x, ay, w) + TP(x, y, aw)
#   d/dx = gx-part of bwd(x, ay, w, g) + of bwd(x, y, aw, g)
#   d/dy = gy-part of bwd(ax, y, w, g) + of bwd(x, y, aw, g)
#   d/dw = gw-part of bwd(ax, y, w, g) + of bwd(x, ay, w, g)
# -- the forward and backward operators again (themselves differentiable).
def _uvu_bwd_setup(ctx, inputs, output):
    x, y, w, edge_index, grad_out, key, channels, layout = inputs
    ctx.save_for_backward(x, y, w, edge_index, grad_out)
    ctx.key, ctx.channels, ctx.layout = key, channels, layout


def _uvu_bwd_backward(ctx, ax, ay, aw):
    x, y, w, ei, g = ctx.saved_tensors
    key, C, lay = ctx.key, ctx.channels, ctx.layout
    zx, zy, zw = (a if a is not None else torch.zeros_like(t) for a, t in ((ax, x), (ay, y), (aw, w)))
    gg = (uvu_scatter(zx, y, w, ei, key, C, lay) + uvu_scatter(x, zy, w, ei, key, C, lay)
          + uvu_scatter(x, y, zw, ei, key, C, lay))
    bx = uvu_scatter_backward(zx, y, w, ei, g, key, C, lay)   # (., gy, gw) with x -> ax
    by = uvu_scatter_backward(x, zy, w, ei, g, key, C, lay)   # (gx, ., gw) with y -> ay
    bw = uvu_scatter_backward(x, y, zw, ei, g, key, C, lay)   # (gx, gy, .) with w -> aw
    return by[0] + bw[0], bx[1] + bw[1], bx[2] + by[2], None, gg, None, None, None


uvu_scatter_backward.register_autograd(_uvu_bwd_backward, setup_context=_uvu_bwd_setup)


# ------------------------------------------------------------------- uuu ----
@torch.library.custom_op("tace_amd::uuu", mutates_args=(), device_types="cuda")
def uuu(x1: Tensor, x2: Tensor, w: Optional[Tensor], key: str, channels: int, layout: int = 0) -> Tensor:
    return ops.launch_uuu_fwd(x1.contiguous(), x2.contiguous(), None if w is None else w.contiguous(),
                              ops.find_variant(key), channels, layout)


@uuu.register_fake
def _uuu_fake(x1, x2, w, key, channels, layout=0):
    return x1.new_empty(x1.shape[0], channels * ops.find_variant(key).dout)


@torch.library.custom_op("tace_amd::uuu_backward", mutates_args=(), device_types="cuda")
def uuu_backward(x1: Tensor, x2: Tensor, w: Optional[Tensor], grad_out: Tensor, key: str,
                 channels: int, layout: int = 0) -> Tuple[Tensor, Tensor, Tensor]:
    g1, g2, gw = ops.launch_uuu_bwd(x1.contiguous(), x2.contiguous(), None if w is None else w.contiguous(),
                                    grad_out.contiguous(), ops.find_variant(key), channels, layout)
    # a weightless product returns an empty weight gradient (schema: tensors only)
    return g1, g2, gw if gw is not None else x1.new_empty(0)


@uuu_backward.register_fake
def _uuu_backward_fake(x1, x2, w, grad_out, key, channels, layout=0):
    return torch.empty_like(x1), torch.empty_like(x2), torch.empty_like(w) if w is not None else x1.new_empty(0)


def _uuu_setup(ctx, inputs, output):
    x1, x2, w, key, channels, layout = inputs
    ctx.save_for_backward(x1, x2, w)
    ctx.key, ctx.channels, ctx.has_w, ctx.layout = key, channels, w is not None, layout


def _uuu_backward(ctx, grad_out):
    x1, x2, w = ctx.saved_tensors
    g1, g2, gw = uuu_backward(x1, x2, w, grad_out, ctx.key, ctx.channels, ctx.layout)
    return g1, g2, gw if ctx.has_w else None, None, None, None


uuu.register_autograd(_uuu_backward, setup_context=_uuu_setup)


# Double backward of the uuu product: (g1, g2, gw) are multilinear in
# (x1, x2, w, g) with g1 free of x1, g2 free of x2 and gw free of w (the same
# scheme as the uvu one above).  Identical inputs pass the same tensor twice;
# autograd adds the two contributions.
def _uuu_bwd_setup(ctx, inputs, output):
    x1, x2, w, grad_out, key, channels, layout = inputs
    ctx.save_for_backward(x1, x2, w, grad_out)
    ctx.key, ctx.channels, ctx.has_w, ctx.layout = key, channels, w is not None, layout


def _uuu_bwd_backward(ctx, a1, a2, aw):
    x1, x2, w, g = ctx.saved_tensors
    key, C, lay = ctx.key, ctx.channels, ctx.layout
    z1 = a1 if a1 is not None else torch.zeros_like(x1)
    z2 = a2 if a2 is not None else torch.zeros_like(x2)
    gg = uuu(z1, x2, w, key, C, lay) + uuu(x1, z2, w, key, C, lay)
    b1 = uuu_backward(z1, x2, w, g, key, C, lay)   # (., g2, gw) with x1 -> a1
    b2 = uuu_backward(x1, z2, w, g, key, C, lay)   # (g1, ., gw) with x2 -> a2
    d1, d2 = b2[0], b1[1]
    dw = None
    if ctx.has_w:
        dw = b1[2] + b2[2]
        if aw is not None and aw.numel():
            gg = gg + uuu(x1, x2, aw, key, C, lay)
            bw = uuu_backward(x1, x2, aw, g, key, C, lay)
            d1, d2 = d1 + bw[0], d2 + bw[1]
    return d1, d2, dw, gg, None, None, None


uuu_backward.register_autograd(_uuu_bwd_backward, setup_context=_uuu_bwd_setup)


# ------------------------------------------------------- per-species linear ----
# ``e3nnElementLinear`` (tace/models/linear.py:377-481) for the exported model:
# features in node order (group-major), the species of every node as an int64
# tensor.  Inside the operator the rows are grouped by species and the
# segmented GEMM runs (what the eager model does once per forward with its
# species plan); the operator's backward gives the input gradient (exported
# models are evaluated with frozen parameters).
_LIN_LAYOUTS = {}


def _lin_layout(irreps_in: str, irreps_out: str):
    from .model import _LinearLayout
    key = (irreps_in, irreps_out)
    if key not in _LIN_LAYOUTS:
        _LIN_LAYOUTS[key] = _LinearLayout(irreps_in, irreps_out)
    return _LIN_LAYOUTS[key]


def _gm_take(x: Tensor, gm, idx: Tensor) -> Tensor:
    """Rows ``idx`` of group-major features (every block gathered by node)."""
    Z = x.shape[0]
    flat = x.reshape(-1)
    out = [flat[Z * s:Z * (s + m * d)].view(Z, d * m).index_select(0, idx).reshape(-1) for (s, m, d) in gm.blocks]
    return torch.cat(out).view(idx.shape[0], -1)


def _element_linear_sorted(x, weight, bias, species, irreps_in, irreps_out, alpha):
    from .model import SpeciesPlan, _LinearFn
    lay = _lin_layout(irreps_in, irreps_out)
    sp = SpeciesPlan(torch.nn.functional.one_hot(species, weight.shape[0]).to(x.dtype))
    xs = _gm_take(x, lay.gin, sp.perm).contiguous()
    return lay, sp, xs


@torch.library.custom_op("tace_amd::element_linear", mutates_args=(), device_types="cuda")
def element_linear(x: Tensor, weight: Tensor, bias: Optional[Tensor], species: Tensor, irreps_in: str,
                   irreps_out: str, alpha: float) -> Tensor:
    from .model import _LinearFn
    lay, sp, xs = _element_linear_sorted(x, weight, bias, species, irreps_in, irreps_out, alpha)
    ys = _LinearFn.apply(xs, weight, bias, lay, sp.ranges, alpha)
    return _gm_take(ys, lay.gout, sp.inv)


@element_linear.register_fake
def _element_linear_fake(x, weight, bias, species, irreps_in, irreps_out, alpha):
    return x.new_empty(x.shape[0], _lin_layout(irreps_in, irreps_out).dim_out)


@torch.library.custom_op("tace_amd::element_linear_backward", mutates_args=(), device_types="cuda")
def element_linear_backward(x: Tensor, weight: Tensor, species: Tensor, grad_out: Tensor, irreps_in: str,
                            irreps_out: str, alpha: float) -> Tensor:
    from .model import _LinearFn
    lay, sp, xs = _element_linear_sorted(x, weight, None, species, irreps_in, irreps_out, alpha)
    gs = _gm_take(grad_out.contiguous(), lay.gout, sp.perm)
    with torch.enable_grad():
        xs = xs.detach().requires_grad_(True)
        ys = _LinearFn.apply(xs, weight.detach(), None, lay, sp.ranges, alpha)
        (gx,) = torch.autograd.grad(ys, xs, gs)
    return _gm_take(gx, lay.gin, sp.inv)


@element_linear_backward.register_fake
def _element_linear_backward_fake(x, weight, species, grad_out, irreps_in, irreps_out, alpha):
    return torch.empty_like(x)


def _element_linear_setup(ctx, inputs, output):
    x, weight, bias, species, irreps_in, irreps_out, alpha = inputs
    ctx.save_for_backward(x, weight, species)
    ctx.args = (irreps_in, irreps_out, alpha)


def _element_linear_bwd(ctx, grad_out):
    x, weight, species = ctx.saved_tensors
    gx = element_linear_backward(x, weight, species, grad_out, *ctx.args)
    return gx, None, None, None, None, None, None


element_linear.register_autograd(_element_linear_bwd, setup_context=_element_linear_setup)


# ------------------------------------------------------------------ TECE ----
# The kernels of the TECE convolution slot (HipTeceConvolution, replacing
# OAM20260705Convolution, tace/models/_e3nn/archive/oam_2026_07_05.py:756-823).
# Edge features are lists of SO(2) blocks (block 0 [E, (L+1) ch], block m
# [2E, (L+1-m) ch]).  Gradients that do not reach an output arrive as None
# and are taken as zeros.

def _zeros_for(grads, like):
    return [g.contiguous() if g is not None else torch.zeros_like(t) for g, t in zip(grads, like)]


@torch.library.custom_op("tace_amd::receiver_csr", mutates_args=(), device_types="cuda")
def receiver_csr(edge_index: Tensor, n_nodes: int) -> Tuple[Tensor, Tensor]:
    """(rowptr int32 [n_nodes+1], eid int32 [E]): the edges of each receiver
    (edge_index[1]) in edge order."""
    dst = edge_index[1]
    rp = torch.zeros(n_nodes + 1, dtype=torch.int64, device=dst.device)
    rp[1:] = torch.cumsum(torch.bincount(dst, minlength=n_nodes), 0)
    return rp.to(torch.int32), torch.argsort(dst, stable=True).to(torch.int32)


@receiver_csr.register_fake
def _receiver_csr_fake(edge_index, n_nodes):
    return (edge_index.new_empty(n_nodes + 1, dtype=torch.int32),
            edge_index.new_empty(edge_index.shape[1], dtype=torch.int32))


def _plan(rowptr, eid, src=None) -> ops.EdgePlan:
    n = rowptr.shape[0] - 1
    return ops.EdgePlan(n, eid.shape[0], rowptr, src if src is not None else eid, eid)


@torch.library.custom_op("tace_amd::tece_rotate_in", mutates_args=(), device_types="cuda")
def tece_rotate_in(x: Tensor, wigner: Tensor, rows_src: Tensor, rows_dst: Tensor, radial_w: Tensor,
                   lmax: int) -> List[Tensor]:
    ms, md, mw = ops.launch_rotate_in_fwd(x.contiguous(), wigner.contiguous(), rows_src.contiguous(),
                                          rows_dst.contiguous(), radial_w.contiguous(), lmax)
    return ms + md + mw


@tece_rotate_in.register_fake
def _tece_rotate_in_fake(x, wigner, rows_src, rows_dst, radial_w, lmax):
    E, C = wigner.shape[0], x.shape[2]
    mk = lambda ch: [x.new_empty(shp) for shp in ops.so2_block_shapes(E, lmax, ch)]
    return mk(C) + mk(C) + mk(2 * C)


@torch.library.custom_op("tace_amd::tece_rotate_in_backward", mutates_args=(), device_types="cuda")
def tece_rotate_in_backward(x: Tensor, wigner: Tensor, rows_src: Tensor, rows_dst: Tensor, radial_w: Tensor,
                            grads: List[Tensor], lmax: int) -> Tuple[Tensor, Tensor, Tensor]:
    n = lmax + 1
    g = [t.contiguous() for t in grads]
    gxs, gxd, gW, gwr = ops.launch_rotate_in_bwd(x.contiguous(), wigner.contiguous(), rows_src.contiguous(),
                                                 rows_dst.contiguous(), radial_w.contiguous(), g[:n], g[n:2 * n],
                                                 g[2 * n:], True)
    gx = ops.scatter_add_rows(ops.scatter_add_rows(torch.zeros_like(x), rows_src, gxs), rows_dst, gxd)
    return gx, gW, gwr


@tece_rotate_in_backward.register_fake
def _tece_rotate_in_backward_fake(x, wigner, rows_src, rows_dst, radial_w, grads, lmax):
    return torch.empty_like(x), torch.empty_like(wigner), torch.empty_like(radial_w)


def _rotate_in_setup(ctx, inputs, output):
    x, wigner, rows_src, rows_dst, radial_w, lmax = inputs
    ctx.save_for_backward(x, wigner, rows_src, rows_dst, radial_w)
    ctx.lmax = lmax
    ctx.like = [o.detach() for o in output]


def _rotate_in_backward(ctx, grads):
    x, wigner, rows_src, rows_dst, radial_w = ctx.saved_tensors
    gx, gW, gwr = tece_rotate_in_backward(x, wigner, rows_src, rows_dst, radial_w, _zeros_for(grads, ctx.like),
                                          ctx.lmax)
    return gx, gW, None, None, gwr, None


tece_rotate_in.register_autograd(_rotate_in_backward, setup_context=_rotate_in_setup)


@torch.library.custom_op("tace_amd::tece_score", mutates_args=(), device_types="cuda")
def tece_score(q: List[Tensor], k: List[Tensor], radial_proj: Tensor, tscale: Tensor, lmax: int,
               heads: int) -> Tensor:
    return ops.launch_score_fwd([t.contiguous() for t in q], [t.contiguous() for t in k], radial_proj.contiguous(),
                                tscale.contiguous(), lmax, heads)


@tece_score.register_fake
def _tece_score_fake(q, k, radial_proj, tscale, lmax, heads):
    return radial_proj.new_empty(radial_proj.shape[0], heads)


@torch.library.custom_op("tace_amd::tece_score_backward", mutates_args=(), device_types="cuda")
def tece_score_backward(q: List[Tensor], k: List[Tensor], radial_proj: Tensor, tscale: Tensor, grad: Tensor,
                        lmax: int, heads: int) -> List[Tensor]:
    gq, gk, grp = ops.launch_score_bwd([t.contiguous() for t in q], [t.contiguous() for t in k],
                                       radial_proj.contiguous(), tscale.contiguous(), grad.contiguous(), lmax, heads)
    return gq + gk + [grp]


@tece_score_backward.register_fake
def _tece_score_backward_fake(q, k, radial_proj, tscale, grad, lmax, heads):
    return [torch.empty_like(t) for t in q] + [torch.empty_like(t) for t in k] + [torch.empty_like(radial_proj)]


def _score_setup(ctx, inputs, output):
    q, k, radial_proj, tscale, lmax, heads = inputs
    ctx.save_for_backward(*q, *k, radial_proj, tscale)
    ctx.lmax, ctx.heads = lmax, heads


def _score_backward(ctx, grad):
    *qk, rp, tscale = ctx.saved_tensors
    n = ctx.lmax + 1
    out = tece_score_backward(list(qk[:n]), list(qk[n:]), rp, tscale, grad, ctx.lmax, ctx.heads)
    return out[:n], out[n:2 * n], out[2 * n], None, None, None


tece_score.register_autograd(_score_backward, setup_context=_score_setup)


@torch.library.custom_op("tace_amd::tece_softmax", mutates_args=(), device_types="cuda")
def tece_softmax(score: Tensor, rowptr: Tensor, eid: Tensor) -> Tensor:
    return ops.launch_softmax_fwd(score.contiguous(), _plan(rowptr, eid))


@tece_softmax.register_fake
def _tece_softmax_fake(score, rowptr, eid):
    return torch.empty_like(score)


@torch.library.custom_op("tace_amd::tece_softmax_backward", mutates_args=(), device_types="cuda")
def tece_softmax_backward(alpha: Tensor, grad: Tensor, rowptr: Tensor, eid: Tensor) -> Tensor:
    return ops.launch_softmax_bwd(alpha.contiguous(), grad.contiguous(), _plan(rowptr, eid))


@tece_softmax_backward.register_fake
def _tece_softmax_backward_fake(alpha, grad, rowptr, eid):
    return torch.empty_like(alpha)


def _softmax_setup(ctx, inputs, output):
    score, rowptr, eid = inputs
    ctx.save_for_backward(output, rowptr, eid)


def _softmax_backward(ctx, grad):
    alpha, rowptr, eid = ctx.saved_tensors
    return tece_softmax_backward(alpha, grad, rowptr, eid), None, None


tece_softmax.register_autograd(_softmax_backward, setup_context=_softmax_setup)


@torch.library.custom_op("tace_amd::tece_edge_ace", mutates_args=(), device_types="cuda")
def tece_edge_ace(ys: List[Tensor], lmax: int, hidden: int) -> List[Tensor]:
    return ops.launch_edge_ace_fwd([t.contiguous() for t in ys], lmax, hidden)


@tece_edge_ace.register_fake
def _tece_edge_ace_fake(ys, lmax, hidden):
    E, n = ys[0].shape[0], lmax + 1
    return [ys[0].new_empty(E if m == 0 else 2 * E, n * hidden) for m in range(lmax + 1)]


@torch.library.custom_op("tace_amd::tece_edge_ace_backward", mutates_args=(), device_types="cuda")
def tece_edge_ace_backward(ys: List[Tensor], grads: List[Tensor], lmax: int, hidden: int) -> List[Tensor]:
    return ops.launch_edge_ace_bwd([t.contiguous() for t in ys], [g.contiguous() for g in grads], lmax, hidden)


@tece_edge_ace_backward.register_fake
def _tece_edge_ace_backward_fake(ys, grads, lmax, hidden):
    return [torch.empty_like(y) for y in ys]


def _edge_ace_setup(ctx, inputs, output):
    ys, lmax, hidden = inputs
    ctx.save_for_backward(*ys)
    ctx.lmax, ctx.hidden = lmax, hidden
    ctx.like = [o.detach() for o in output]


def _edge_ace_backward(ctx, grads):
    ys = list(ctx.saved_tensors)
    return tece_edge_ace_backward(ys, _zeros_for(grads, ctx.like), ctx.lmax, ctx.hidden), None, None


tece_edge_ace.register_autograd(_edge_ace_backward, setup_context=_edge_ace_setup)


@torch.library.custom_op("tace_amd::tece_rotate_out", mutates_args=(), device_types="cuda")
def tece_rotate_out(m: List[Tensor], alpha: Tensor, wigner: Tensor, rowptr: Tensor, eid: Tensor, dst: Tensor,
                    lmax: int, heads: int) -> Tensor:
    """Receiver sums [N, (L+1)^2 C], group-major, rows = node ids (dst: the
    receiver of each edge, int64, for the backward)."""
    return ops.launch_rotate_out_fwd([t.contiguous() for t in m], alpha.contiguous(), wigner.contiguous(),
                                     _plan(rowptr, eid), None, lmax, heads)


@tece_rotate_out.register_fake
def _tece_rotate_out_fake(m, alpha, wigner, rowptr, eid, dst, lmax, heads):
    C = m[0].shape[1] // (lmax + 1)
    return alpha.new_empty(rowptr.shape[0] - 1, (lmax + 1) ** 2 * C)


@torch.library.custom_op("tace_amd::tece_rotate_out_backward", mutates_args=(), device_types="cuda")
def tece_rotate_out_backward(m: List[Tensor], alpha: Tensor, wigner: Tensor, grad: Tensor, dst: Tensor,
                             rowptr: Tensor, eid: Tensor, lmax: int, heads: int) -> List[Tensor]:
    gm, ga, gW = ops.launch_rotate_out_bwd([t.contiguous() for t in m], alpha.contiguous(), wigner.contiguous(),
                                           grad.contiguous(), dst.contiguous(), None, _plan(rowptr, eid), lmax, heads)
    return gm + [ga, gW]


@tece_rotate_out_backward.register_fake
def _tece_rotate_out_backward_fake(m, alpha, wigner, grad, dst, rowptr, eid, lmax, heads):
    return [torch.empty_like(t) for t in m] + [torch.empty_like(alpha), torch.empty_like(wigner)]


def _rotate_out_setup(ctx, inputs, output):
    m, alpha, wigner, rowptr, eid, dst, lmax, heads = inputs
    ctx.save_for_backward(*m, alpha, wigner, rowptr, eid, dst)
    ctx.lmax, ctx.heads = lmax, heads


def _rotate_out_backward(ctx, grad):
    *m, alpha, wigner, rowptr, eid, dst = ctx.saved_tensors
    out = tece_rotate_out_backward(list(m), alpha, wigner, grad, dst, rowptr, eid, ctx.lmax, ctx.heads)
    k = ctx.lmax + 1
    return out[:k], out[k], out[k + 1], None, None, None, None, None


tece_rotate_out.register_autograd(_rotate_out_backward, setup_context=_rotate_out_setup)
