"""Autograd operators over the HIP kernels of ``libtace_hip.so``.

Each operator checks device, dtype, contiguity and shapes on the host before
launching (the kernels trust these), launches on torch's current stream, and
raises if the native library is missing -- there is no CPU path.

* ``edge_basis``      radial basis x cutoff and SH of edge vectors
                      (``tace/models/radial.py:974-993``, ``angular.py:288-315``)
* ``edge_tp_scatter`` uvu tensor product fused with the receiver scatter
                      (``tace/models/_e3nn/fused.py:259-271``)
* ``uuu_tp``          node-level uuu product (``fused.py:90-95``)
* ``neighbour_list``  cell-list neighbour search (``dataset/neighbour_list.py:195-298``)
"""

from __future__ import annotations

import contextlib
import threading

import ctypes
import math
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _native as N


class KernelTimer:
    """Optional HIP-event bracketing of every native launch, on the stream the
    kernel runs on (torch's current stream).  ``ops.TIMER = KernelTimer()``
    enables it; ``summary()`` returns {name: (launches, total_ms, infos)} and
    ``phases()`` {name: (launches, first phase ms)} for the entry points that
    mark a phase event (the edge-TP backward: its product kernel alone)."""

    def __init__(self):
        self.events = {}
        self.mid = {}

    def start(self, name):
        e0 = torch.cuda.Event(enable_timing=True)
        e0.record()
        return name, e0

    def mark_phase(self, tok):
        """Arms ``tace_mark_phase_event`` for the next entry point call."""
        if tok is None:
            return None
        e = torch.cuda.Event(enable_timing=True)
        e.record()   # creates the underlying event; the library records it again
        N.lib().tace_mark_phase_event(ctypes.c_void_p(e.cuda_event))
        return e

    def stop(self, tok, info=None, mid=None):
        name, e0 = tok
        e1 = torch.cuda.Event(enable_timing=True)
        e1.record()
        self.events.setdefault(name, []).append((e0, e1, info))
        if mid is not None:
            self.mid.setdefault(name, []).append((e0, mid))

    def summary(self):
        torch.cuda.synchronize()
        return {k: (len(v), sum(a.elapsed_time(b) for a, b, _ in v), [i for _, _, i in v]) for k, v in self.events.items()}

    def phases(self):
        torch.cuda.synchronize()
        return {k: (len(v), sum(a.elapsed_time(b) for a, b in v)) for k, v in self.mid.items()}


TIMER = None


class _Mode(threading.local):
    """Per-thread switch of the operators' autograd form (see ``differentiable_twice``
    and ``export_mode``)."""

    double = False
    export = False


MODE = _Mode()


@contextlib.contextmanager
def differentiable_twice(on: bool = True):
    """Inside this context the model's operators take a form whose backward is
    itself differentiable: the edge and node tensor products on the HIP
    kernels through operators whose backward is written with the forward and
    backward operators (``_EdgeTPD``, ``_UUUD``), everything else (edge
    vectors, radial basis and harmonics, radial MLP, linears, gate) as plain
    torch operations.  This is what training with a force loss needs
    (``create_graph=True`` in ``tace/models/adapter.py:95-104``); outside it the
    inference operators run (first-order backward, frozen radial weights)."""
    prev = MODE.double
    MODE.double = bool(on)
    try:
        yield
    finally:
        MODE.double = prev


@contextlib.contextmanager
def export_mode():
    """The model as a graph that ``make_fx`` / ``torch.export`` can trace with
    symbolic node and edge counts: the operators of ``differentiable_twice``,
    with the kernels reached only through the ``torch.library`` operators of
    ``tace_amd.library`` (tensor products, per-species linears), no host-side
    plans (species order, receiver CSR, edge pairs are made inside those
    operators) and features in node order."""
    prev = (MODE.double, MODE.export)
    MODE.double, MODE.export = True, True
    try:
        yield
    finally:
        MODE.double, MODE.export = prev


class TracedEdges:
    """The edge list where an ``EdgePlan`` would be (export mode): the
    operators build their receiver CSR from ``edge_index`` themselves."""

    def __init__(self, edge_index: torch.Tensor, n_nodes):
        self.edge_index = edge_index
        self.n_nodes = n_nodes
        self.src = edge_index[0]
        self.n_edges = edge_index.shape[1]


def _t0(name):
    return TIMER.start(name) if TIMER is not None else None


def _t1(tok, info=None):
    if tok is not None:
        TIMER.stop(tok, info)


def variant_key(kind: str, in1: Sequence[int], in2: Sequence[int], out: Sequence[int]) -> str:
    j = lambda s: ",".join(str(int(v)) for v in s)
    return f"{kind}|{j(in1)}|{j(in2)}|{j(out)}"


@dataclass(frozen=True)
class TpVariant:
    vid: int
    key: str
    npath: int
    d1: int
    d2: int
    dout: int


_VCACHE = {}


def find_variant(key: str) -> TpVariant:
    if key not in _VCACHE:
        L = N.lib()
        vid = L.tace_tp_find(key.encode())
        if vid < 0:
            raise N.NativeError(L.tace_last_error().decode())
        a, b, c, d = (np.zeros(1, np.int32) for _ in range(4))
        N.check(L.tace_tp_dims(vid, a.ctypes.data, b.ctypes.data, c.ctypes.data, d.ctypes.data), "tace_tp_dims")
        _VCACHE[key] = TpVariant(vid, key, int(a[0]), int(b[0]), int(c[0]), int(d[0]))
    return _VCACHE[key]


def _req(t: torch.Tensor, name: str, dtype, shape=None):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (got {t.device})")
    if t.dtype != dtype:
        raise ValueError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")


# ------------------------------------------------------------ edge plan ----
@dataclass
class EdgePlan:
    """Receiver-CSR view of an edge list: edge ids sorted by ``dst``.

    ``eid`` is None when the edges are already grouped by receiver (as the GPU
    neighbour list emits them)."""

    n_nodes: int
    n_edges: int
    rowptr: torch.Tensor           # int32 [N+1]
    src: torch.Tensor              # int32 [E], sender of edge id
    eid: Optional[torch.Tensor]    # int32 [E] or None
    _sender: Optional[Tuple[torch.Tensor, torch.Tensor]] = None
    _pairs: Optional["EdgePairs"] = None

    def sender_csr(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """(s_rowptr int32 [N+1], s_slot int32 [E]): receiver-sorted slots grouped
        by sender, stable -- the fixed order of the grad_x segmented sum."""
        if self._sender is None:
            slot_src = self.src if self.eid is None else self.src[self.eid.long()]
            self._sender = group_by_key(slot_src, self.n_nodes)
        return self._sender

    def edge_pairs(self, shifts: torch.Tensor) -> "EdgePairs":
        """The edge pairs of this list (``tace_edge_pairs``), from the integer
        periodic shifts [E, 3] (edge-id order); cached on the plan."""
        if self._pairs is None:
            self._pairs = edge_pairs(self, shifts)
        return self._pairs

    @staticmethod
    def from_edge_index(edge_index: torch.Tensor, n_nodes: int) -> "EdgePlan":
        src, dst = edge_index[0], edge_index[1]
        E = int(src.shape[0])
        if E and (int(torch.minimum(src.min(), dst.min())) < 0
                  or int(torch.maximum(src.max(), dst.max())) >= n_nodes):
            raise ValueError("edge_index refers to nodes outside [0, n_nodes)")
        if E >= 2 ** 31 or n_nodes >= 2 ** 31:
            raise ValueError("edge/node counts exceed the int32 CSR indexing of the kernels")
        counts = torch.bincount(dst, minlength=n_nodes)
        rowptr = torch.zeros(n_nodes + 1, dtype=torch.int64, device=dst.device)
        rowptr[1:] = torch.cumsum(counts, 0)
        if E > 0 and bool((dst[1:] >= dst[:-1]).all()):
            eid = None
        else:
            eid = torch.argsort(dst, stable=True).to(torch.int32).contiguous()
        return EdgePlan(n_nodes, E, rowptr.to(torch.int32).contiguous(), src.to(torch.int32).contiguous(), eid)


class EdgePairs:
    """The two directions of every edge (``tace_edge_pairs``): ``w_rows``
    (int32 [E], by edge id) the row of each edge's pair, ``row_edges`` /
    ``row_partner`` (int32 [n_rows]) the lower edge id of each row and its
    reverse (-1: none).  A weight that depends on the edge length only is made
    once per row.

    The row count is made on the GPU; it is copied to pinned host memory
    without waiting, and the host waits for that copy only when ``n_rows``
    (or a row array) is first needed, by which time the GPU has later work
    queued and does not run dry."""

    def __init__(self, n_rows, w_rows: torch.Tensor, row_edges: torch.Tensor, row_partner: torch.Tensor):
        # n_rows: an int, or (pinned host int32 [1], event recorded after its copy)
        self._n = n_rows
        self.w_rows = w_rows
        self._row_edges, self._row_partner = row_edges, row_partner

    @property
    def n_rows(self) -> int:
        if not isinstance(self._n, int):
            host, ev = self._n
            ev.synchronize()
            self._n = int(host[0])
        return self._n

    @property
    def row_edges(self) -> torch.Tensor:
        return self._row_edges[:self.n_rows]

    @property
    def row_partner(self) -> torch.Tensor:
        return self._row_partner[:self.n_rows]


def edge_pairs(plan: EdgePlan, shifts: torch.Tensor) -> EdgePairs:
    E = plan.n_edges
    sh = shifts if shifts.dtype == torch.int32 else torch.round(shifts).to(torch.int32)
    _req(sh.contiguous(), "shifts", torch.int32, (E, 3))
    sh = sh.contiguous()
    dev = plan.rowptr.device
    work = torch.empty(3 * E + 2 * ((E + 1023) // 1024) + 4, dtype=torch.int32, device=dev)  # TACE_EDGE_PAIRS_WORK
    w_rows = torch.empty(E, dtype=torch.int32, device=dev)
    row_edges = torch.empty(max(E, 1), dtype=torch.int32, device=dev)
    row_partner = torch.empty(max(E, 1), dtype=torch.int32, device=dev)
    tok = _t0("edge_pairs")
    N.check(N.lib().tace_edge_pairs(plan.rowptr.data_ptr(), N.ptr(plan.eid), plan.src.data_ptr() if E else None,
                                    sh.data_ptr() if E else None, plan.n_nodes, E, work.data_ptr(), w_rows.data_ptr(),
                                    row_edges.data_ptr(), row_partner.data_ptr(), N.stream_ptr(dev)),
            "tace_edge_pairs")
    _t1(tok, (E,))
    host = torch.empty(1, dtype=torch.int32, pin_memory=True)
    host.copy_(work[3 * E:3 * E + 1], non_blocking=True)
    ev = torch.cuda.Event()
    ev.record(torch.cuda.current_stream(dev))
    return EdgePairs((host, ev), w_rows, row_edges, row_partner)


# ------------------------------------------------------- edge featurisation ----
class _EdgeBasis(torch.autograd.Function):
    @staticmethod
    def forward(ctx, vec, bessel_w, prefactor: float, cutoff: float, p: int, lmax: int):
        E = vec.shape[0]
        nb = bessel_w.shape[0]
        _req(vec, "edge_vector", vec.dtype, (E, 3))
        _req(bessel_w, "bessel_weights", vec.dtype, (nb,))
        R = torch.empty(E, nb, dtype=vec.dtype, device=vec.device)
        Y = torch.empty(E, (lmax + 1) ** 2, dtype=vec.dtype, device=vec.device)
        tok = _t0("edge_basis_fwd")
        N.check(N.lib().tace_edge_basis_fwd(N.dtype_code(vec.dtype), vec.data_ptr(), E, nb, bessel_w.data_ptr(),
                                            prefactor, cutoff, p, lmax, R.data_ptr(), Y.data_ptr(),
                                            N.stream_ptr(vec.device)), "tace_edge_basis_fwd")
        _t1(tok, (E,))
        ctx.save_for_backward(vec, bessel_w)
        ctx.args = (prefactor, cutoff, p, lmax)
        return R, Y

    @staticmethod
    def backward(ctx, gR, gY):
        vec, bw = ctx.saved_tensors
        prefactor, cutoff, p, lmax = ctx.args
        E, nb = vec.shape[0], bw.shape[0]
        gR = torch.zeros(E, nb, dtype=vec.dtype, device=vec.device) if gR is None else gR.contiguous()
        gY = torch.zeros(E, (lmax + 1) ** 2, dtype=vec.dtype, device=vec.device) if gY is None else gY.contiguous()
        gvec = torch.empty_like(vec)
        tok = _t0("edge_basis_bwd")
        N.check(N.lib().tace_edge_basis_bwd(N.dtype_code(vec.dtype), vec.data_ptr(), gR.data_ptr(), gY.data_ptr(), E,
                                            nb, bw.data_ptr(), prefactor, cutoff, p, lmax, gvec.data_ptr(),
                                            N.stream_ptr(vec.device)), "tace_edge_basis_bwd")
        _t1(tok, (E,))
        return gvec, None, None, None, None, None


def spherical_harmonics(u: torch.Tensor, lmax: int) -> torch.Tensor:
    """e3nn's real spherical harmonics of the rows of u [E, 3], component
    normalisation, polar axis y, m = -l..l within each l (the closed forms the
    edge-basis kernel evaluates), as torch operations: [E, (lmax + 1)^2]."""
    x, y, z = u[:, 0], u[:, 1], u[:, 2]
    out = [torch.ones_like(x)]
    if lmax >= 1:
        s3 = math.sqrt(3.0)
        out += [s3 * x, s3 * y, s3 * z]
    if lmax >= 2:
        s15, s5 = math.sqrt(15.0), math.sqrt(5.0)
        y2, xz2 = y * y, x * x + z * z
        q = [s15 * x * z, s15 * x * y, s5 * (y2 - 0.5 * xz2), s15 * y * z, 0.5 * s15 * (z * z - x * x)]
        out += q
    if lmax >= 3:
        c42, c7, c168 = math.sqrt(42.0) / 6.0, math.sqrt(7.0), math.sqrt(168.0) / 8.0
        t = 4.0 * y2 - xz2
        out += [c42 * (q[0] * z + q[4] * x), c7 * q[0] * y, c168 * t * x, 0.5 * c7 * y * (2.0 * y2 - 3.0 * xz2),
                c168 * t * z, c7 * q[4] * y, c42 * (q[4] * z - q[0] * x)]
    if lmax > 3:
        raise ValueError("spherical harmonics up to l = 3")
    return torch.stack(out, dim=1)


def _edge_basis_autograd(vec, bessel_w, prefactor: float, cutoff: float, p: int, lmax: int):
    """The edge-basis kernel's arithmetic as torch operations: length + 1e-9
    (adapter.py:347), j0 Bessel x C2 polynomial cutoff (radial.py:43-84,
    437-472), harmonics of vec / length (representation.py:321-324)."""
    r = torch.sqrt((vec * vec).sum(dim=1, keepdim=True)) + 1e-9
    x = r / cutoff
    c1, c2, c3 = (p + 1.0) * (p + 2.0) / 2.0, p * (p + 2.0), p * (p + 1.0) / 2.0
    xp = x ** p
    env = 1.0 - c1 * xp + c2 * (xp * x) - c3 * (xp * x * x)
    env = torch.where(r < cutoff, env, torch.zeros_like(env))
    R = prefactor * (torch.sin(bessel_w * r) / r) * env
    return R, spherical_harmonics(vec / r, lmax)


def edge_basis(vec: torch.Tensor, bessel_w: torch.Tensor, prefactor: float, cutoff: float, p: int,
               lmax: int) -> Tuple[torch.Tensor, torch.Tensor]:
    if MODE.double:
        return _edge_basis_autograd(vec, bessel_w, float(prefactor), float(cutoff), int(p), int(lmax))
    return _EdgeBasis.apply(vec.contiguous(), bessel_w.contiguous(), float(prefactor), float(cutoff), int(p),
                            int(lmax))


# ------------------------------------------------------ edge tensor product ----
def launch_edge_tp_fwd(x, y, w, plan: EdgePlan, var: TpVariant, C: int, layout: int = 0, node_map=None,
                       pairs: Optional[EdgePairs] = None):
    """``pairs``: w has one row per edge pair (``EdgePairs.n_rows``), edge e
    reads row ``pairs.w_rows[e]``."""
    Nn, E = plan.n_nodes, plan.n_edges
    dt = x.dtype
    _req(x, "x", dt, (Nn, C * var.d1))
    _req(y, "y", dt, (E, var.d2))
    _req(w, "w", dt, (E if pairs is None else pairs.n_rows, C * var.npath))
    out = torch.empty(Nn, C * var.dout, dtype=dt, device=x.device)
    tok = _t0("edge_tp_fwd:" + var.key)
    N.check(N.lib().tace_edge_tp_fwd_rows(var.vid, N.dtype_code(dt), x.data_ptr(), y.data_ptr(), w.data_ptr(),
                                          plan.rowptr.data_ptr(), N.ptr(plan.eid), plan.src.data_ptr(),
                                          N.ptr(node_map), None if pairs is None else pairs.w_rows.data_ptr(), Nn,
                                          E, C, layout, out.data_ptr(), N.stream_ptr(x.device)), "tace_edge_tp_fwd")
    _t1(tok, (Nn, E, C) if pairs is None else (Nn, E, C, pairs.n_rows))
    return out


def launch_edge_tp_bwd(x, y, w, gout, plan: EdgePlan, var: TpVariant, C: int, layout: int = 0, node_map=None,
                       need_x: bool = True, pairs: Optional[EdgePairs] = None):
    """(grad_x or None, grad_y, grad_w) of ``launch_edge_tp_fwd``; with
    ``pairs`` grad_w is per edge ([E, C*npath]), not per weight row."""
    _req(gout, "g_out", x.dtype, (plan.n_nodes, C * var.dout))
    gx = torch.empty_like(x) if need_x else None
    gy = torch.empty_like(y)
    gw = torch.empty(plan.n_edges, w.shape[1], dtype=w.dtype, device=w.device)
    s_rowptr, s_slot = plan.sender_csr() if need_x else (None, None)
    n_ws = N.lib().tace_edge_tp_workspace_elems(var.vid, plan.n_edges, C, int(need_x))
    if n_ws < 0:
        N.check(int(n_ws), "tace_edge_tp_workspace_elems")
    ws = torch.empty(max(n_ws, 1), dtype=x.dtype, device=x.device)
    tok = _t0("edge_tp_bwd:" + var.key)
    mid = TIMER.mark_phase(tok) if tok is not None else None
    N.check(N.lib().tace_edge_tp_bwd_rows(var.vid, N.dtype_code(x.dtype), x.data_ptr(), y.data_ptr(), w.data_ptr(),
                                          gout.data_ptr(), plan.rowptr.data_ptr(), N.ptr(plan.eid),
                                          plan.src.data_ptr(), N.ptr(node_map),
                                          None if pairs is None else pairs.w_rows.data_ptr(), plan.n_nodes,
                                          plan.n_edges, C, layout, N.ptr(s_rowptr), N.ptr(s_slot), ws.data_ptr(),
                                          ws.numel(), N.ptr(gx), gy.data_ptr(), gw.data_ptr(),
                                          N.stream_ptr(x.device)), "tace_edge_tp_bwd")
    if tok is not None:
        TIMER.stop(tok, (plan.n_nodes, plan.n_edges, C, need_x) if pairs is None
                   else (plan.n_nodes, plan.n_edges, C, need_x, pairs.n_rows), mid)
    return gx, gy, gw


class _EdgeTP(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, y, w, plan: EdgePlan, var: TpVariant, C: int, layout: int, node_map):
        out = launch_edge_tp_fwd(x, y, w, plan, var, C, layout, node_map)
        ctx.save_for_backward(x, y, w)
        ctx.plan, ctx.var, ctx.C, ctx.layout, ctx.node_map = plan, var, C, layout, node_map
        return out

    @staticmethod
    def backward(ctx, gout):
        x, y, w = ctx.saved_tensors
        gx, gy, gw = launch_edge_tp_bwd(x, y, w, gout.contiguous(), ctx.plan, ctx.var, ctx.C, ctx.layout,
                                        ctx.node_map, ctx.needs_input_grad[0])
        return gx, gy, gw, None, None, None, None, None


# Double backward of the edge product.  out = TP(x, y, w) is trilinear and its
# backward (gx, gy, gw) is multilinear in (x, y, w, g) with gx(y, w, g),
# gy(x, w, g), gw(x, y, g).  For upstream gradients (ax, ay, aw):
#   d/dg = TP(ax, y, w) + TP(x, ay, w) + TP(x, y, aw)
#   d/dx = gx of bwd(x, ay, w, g) + gx of bwd(x, y, aw, g)
#   d/dy = gy of bwd(ax, y, w, g) + gy of bwd(x, y, aw, g)
#   d/dw = gw of bwd(ax, y, w, g) + gw of bwd(x, ay, w, g)
# -- the same two operators again, so every order is differentiable.
class _EdgeTPD(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, y, w, plan: EdgePlan, var: TpVariant, C: int, layout: int, node_map):
        ctx.save_for_backward(x, y, w)
        ctx.args = (plan, var, C, layout, node_map)
        return launch_edge_tp_fwd(x, y, w, plan, var, C, layout, node_map)

    @staticmethod
    def backward(ctx, g):
        x, y, w = ctx.saved_tensors
        gx, gy, gw = _EdgeTPBwdD.apply(x, y, w, g.contiguous(), *ctx.args)
        return gx, gy, gw, None, None, None, None, None


class _EdgeTPBwdD(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, y, w, g, plan: EdgePlan, var: TpVariant, C: int, layout: int, node_map):
        ctx.save_for_backward(x, y, w, g)
        ctx.args = (plan, var, C, layout, node_map)
        return launch_edge_tp_bwd(x, y, w, g, plan, var, C, layout, node_map, True)

    @staticmethod
    def backward(ctx, ax, ay, aw):
        x, y, w, g = ctx.saved_tensors
        a = ctx.args
        zx, zy, zw = (t.contiguous() if t is not None else torch.zeros_like(r) for t, r in ((ax, x), (ay, y), (aw, w)))
        F, B = _EdgeTPD.apply, _EdgeTPBwdD.apply
        gg = F(zx, y, w, *a) + F(x, zy, w, *a) + F(x, y, zw, *a)
        bx, by, bw = B(zx, y, w, g, *a), B(x, zy, w, g, *a), B(x, y, zw, g, *a)
        return by[0] + bw[0], bx[1] + bw[1], bx[2] + by[2], gg, None, None, None, None, None


def edge_tp_scatter(x, y, w, plan: EdgePlan, var: TpVariant, C: int, layout: int = 0,
                    node_map: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused uvu tensor product + receiver scatter.  ``layout``: combination of
    LAYOUT_IN1_GROUPED (x, grad x) and LAYOUT_OUT_GROUPED (output, grad output).
    ``node_map`` (int32 [N]): row of node n in x and in the output when the
    features are stored in another order than the edges index (None: same)."""
    if MODE.export:
        from . import library
        if node_map is not None:
            raise ValueError("export mode keeps the features in node order (node_map None)")
        return library.uvu_scatter(x, y, w, plan.edge_index, var.key, C, int(layout))
    if node_map is not None:
        _req(node_map, "node_map", torch.int32, (plan.n_nodes,))
    if MODE.double:
        return _EdgeTPD.apply(x.contiguous(), y.contiguous(), w.contiguous(), plan, var, C, int(layout), node_map)
    return _EdgeTP.apply(x.contiguous(), y.contiguous(), w.contiguous(), plan, var, C, int(layout), node_map)


class _PairRadialTP(torch.autograd.Function):
    """The radial MLP's last layer (w = alpha h @ W, one row per edge pair)
    and the edge product that reads w through ``pairs.w_rows``, as one
    operator: the backward turns the per-edge grad_w into the gradient of the
    pair rows' h directly (the two edges' rows summed in float32 inside the
    last layer's input-gradient kernel), so no per-pair grad_w is formed."""

    @staticmethod
    def forward(ctx, x, y, h, W, alpha: float, plan: EdgePlan, pairs: EdgePairs, var: TpVariant, C: int,
                layout: int, node_map):
        w = radial_mlp_out(h, W, alpha)
        out = launch_edge_tp_fwd(x, y, w, plan, var, C, layout, node_map, pairs)
        ctx.save_for_backward(x, y, w, W)
        ctx.alpha, ctx.plan, ctx.pairs, ctx.var, ctx.C, ctx.layout, ctx.node_map = (alpha, plan, pairs, var, C,
                                                                                   layout, node_map)
        return out

    @staticmethod
    def backward(ctx, gout):
        x, y, w, W = ctx.saved_tensors
        pairs = ctx.pairs
        gx, gy, gw = launch_edge_tp_bwd(x, y, w, gout.contiguous(), ctx.plan, ctx.var, ctx.C, ctx.layout,
                                        ctx.node_map, ctx.needs_input_grad[0], pairs)
        gh = None
        if ctx.needs_input_grad[2]:
            if gw.dtype == torch.float32:
                gh = launch_mlp_out_bwd_pairs_f32(gw, pairs, W, ctx.alpha)
            else:
                ra = pairs.row_edges.long()
                rb = pairs.row_partner.long()
                g = gw.index_select(0, ra)
                has = rb >= 0
                g[has] += gw.index_select(0, rb[has])
                gh = torch.mm(g, W.t()).mul_(ctx.alpha)
        return gx, gy, gh, None, None, None, None, None, None, None, None


def edge_tp_scatter_pairs(x, y, h, W, alpha: float, plan: EdgePlan, pairs: EdgePairs, var: TpVariant, C: int,
                          layout: int = 0, node_map: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``edge_tp_scatter(x, y, w, ...)`` with w = alpha h @ W made once per
    edge pair (h [n_rows, 64], the radial MLP's last hidden activations of the
    pairs' lower edges) and read by both edges of each pair (``pairs.w_rows``).
    Gradients: x, y and h (W is a constant, as in ``radial_mlp_out``)."""
    if node_map is not None:
        _req(node_map, "node_map", torch.int32, (plan.n_nodes,))
    return _PairRadialTP.apply(x.contiguous(), y.contiguous(), h.contiguous(), W.detach().contiguous(), float(alpha),
                               plan, pairs, var, C, int(layout), node_map)


# ------------------------------------------ radial-fused edge tensor product ----
def rtp_supported(dtype, C: int, hidden: int) -> bool:
    """Whether the radial-fused kernels take this product: float32, channels a
    multiple of 64, 64 hidden features in front of the radial last layer."""
    return dtype == torch.float32 and C % 64 == 0 and hidden == 64


def launch_edge_rtp_fwd(x, y, h, W, alpha: float, plan: EdgePlan, var: TpVariant, C: int, layout: int = 0,
                        node_map=None):
    """``launch_edge_tp_fwd`` with w = alpha h @ W made inside the kernel."""
    Nn, E = plan.n_nodes, plan.n_edges
    f32 = torch.float32
    _req(x, "x", f32, (Nn, C * var.d1))
    _req(y, "y", f32, (E, var.d2))
    _req(h, "h", f32, (E, 64))
    _req(W, "w_last", f32, (64, C * var.npath))
    out = torch.empty(Nn, C * var.dout, dtype=f32, device=x.device)
    rows = torch.empty(max(E, 1), dtype=torch.int32, device=x.device)
    tok = _t0("edge_rtp_fwd:" + var.key)
    N.check(N.lib().tace_edge_rtp_fwd(var.vid, x.data_ptr(), y.data_ptr(), h.data_ptr(), W.data_ptr(), float(alpha),
                                      plan.rowptr.data_ptr(), N.ptr(plan.eid), plan.src.data_ptr(), N.ptr(node_map),
                                      Nn, E, C, layout, rows.data_ptr(), out.data_ptr(), N.stream_ptr(x.device)),
            "tace_edge_rtp_fwd")
    _t1(tok, (Nn, E, C))
    return out


def launch_edge_rtp_bwd(x, y, h, W, alpha: float, gout, plan: EdgePlan, var: TpVariant, C: int, layout: int = 0,
                        node_map=None, need_x: bool = True):
    """(grad_x or None, grad_y, grad_w) of ``launch_edge_rtp_fwd``; grad_w is
    the gradient of the per-edge weights alpha h @ W."""
    E = plan.n_edges
    _req(gout, "g_out", torch.float32, (plan.n_nodes, C * var.dout))
    gx = torch.empty_like(x) if need_x else None
    gy = torch.empty_like(y)
    gw = torch.empty(E, C * var.npath, dtype=torch.float32, device=x.device)
    s_rowptr, s_slot = plan.sender_csr() if need_x else (None, None)
    n_ws = N.lib().tace_edge_rtp_workspace_elems(var.vid, E, C, int(need_x))
    if n_ws < 0:
        N.check(int(n_ws), "tace_edge_rtp_workspace_elems")
    ws = torch.empty(max(n_ws, 1), dtype=torch.float32, device=x.device)
    rows = torch.empty(max(E, 1), dtype=torch.int32, device=x.device)
    tok = _t0("edge_rtp_bwd:" + var.key)
    N.check(N.lib().tace_edge_rtp_bwd(var.vid, x.data_ptr(), y.data_ptr(), h.data_ptr(), W.data_ptr(), float(alpha),
                                      gout.data_ptr(), plan.rowptr.data_ptr(), N.ptr(plan.eid), plan.src.data_ptr(),
                                      N.ptr(node_map), plan.n_nodes, E, C, layout, N.ptr(s_rowptr), N.ptr(s_slot),
                                      rows.data_ptr(), ws.data_ptr(), ws.numel(), N.ptr(gx), gy.data_ptr(),
                                      gw.data_ptr(), N.stream_ptr(x.device)), "tace_edge_rtp_bwd")
    _t1(tok, (plan.n_nodes, E, C, need_x))
    return gx, gy, gw


class _EdgeRTP(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, y, h, W, alpha: float, plan: EdgePlan, var: TpVariant, C: int, layout: int, node_map):
        out = launch_edge_rtp_fwd(x, y, h, W, alpha, plan, var, C, layout, node_map)
        ctx.save_for_backward(x, y, h, W)
        ctx.alpha, ctx.plan, ctx.var, ctx.C, ctx.layout, ctx.node_map = alpha, plan, var, C, layout, node_map
        return out

    @staticmethod
    def backward(ctx, gout):
        x, y, h, W = ctx.saved_tensors
        gx, gy, gw = launch_edge_rtp_bwd(x, y, h, W, ctx.alpha, gout.contiguous(), ctx.plan, ctx.var, ctx.C,
                                         ctx.layout, ctx.node_map, ctx.needs_input_grad[0])
        gh = None
        if ctx.needs_input_grad[2]:
            gh = (launch_mlp_out_bwd_f32(gw, W, ctx.alpha) if gw.shape[1] % 4 == 0
                  else torch.mm(gw, W.t()).mul_(ctx.alpha))
        gW = torch.mm(h.t(), gw).mul_(ctx.alpha) if ctx.needs_input_grad[3] else None
        return gx, gy, gh, gW, None, None, None, None, None, None


def edge_rtp_scatter(x, y, h, W, alpha: float, plan: EdgePlan, var: TpVariant, C: int, layout: int = 0,
                     node_map: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``edge_tp_scatter(x, y, alpha * h @ W, ...)`` with the radial MLP's last
    layer (``mlp.py:136-191``) made on MFMA inside the product kernels: the
    per-edge weights never go through HBM, in the forward or the backward.
    h [E, 64] (last hidden activations), W [64, C * npath]; float32, C a
    multiple of 64 (``rtp_supported``)."""
    if node_map is not None:
        _req(node_map, "node_map", torch.int32, (plan.n_nodes,))
    if not rtp_supported(x.dtype, C, h.shape[-1]):
        raise ValueError("edge_rtp_scatter: needs float32, channels a multiple of 64 and 64 hidden features")
    return _EdgeRTP.apply(x.contiguous(), y.contiguous(), h.contiguous(), W.contiguous(), float(alpha), plan, var, C,
                          int(layout), node_map)


# ------------------------------------------------------------ edge vectors ----
class _EdgeVectors(torch.autograd.Function):
    @staticmethod
    def forward(ctx, pos, lattice, shifts, plan: EdgePlan, dst: torch.Tensor, edge_graph):
        E = plan.n_edges
        dt = pos.dtype
        _req(pos, "positions", dt, (plan.n_nodes, 3))
        _req(shifts, "edge_shifts", dt, (E, 3))
        _req(lattice, "lattice", dt)
        vec = torch.empty(E, 3, dtype=dt, device=pos.device)
        N.check(N.lib().tace_edge_vec_fwd(N.dtype_code(dt), pos.data_ptr(), lattice.data_ptr(), plan.src.data_ptr(),
                                          dst.data_ptr(), shifts.data_ptr(), N.ptr(edge_graph), E, vec.data_ptr(),
                                          N.stream_ptr(pos.device)), "tace_edge_vec_fwd")
        ctx.save_for_backward(shifts)
        ctx.plan, ctx.edge_graph, ctx.nlat = plan, edge_graph, lattice.shape[0]
        return vec

    @staticmethod
    def backward(ctx, g):
        (shifts,) = ctx.saved_tensors
        plan = ctx.plan
        g = g.contiguous()
        gpos = glat = None
        if ctx.needs_input_grad[0] and plan.n_edges == 0:
            # no edge: every receiver and sender sum is empty (and the empty
            # per-edge tensors have no device pointer for the kernel)
            gpos = torch.zeros(plan.n_nodes, 3, dtype=g.dtype, device=g.device)
        elif ctx.needs_input_grad[0]:
            s_rowptr, s_slot = plan.sender_csr()
            gpos = torch.empty(plan.n_nodes, 3, dtype=g.dtype, device=g.device)
            N.check(N.lib().tace_edge_vec_bwd(N.dtype_code(g.dtype), g.data_ptr(), plan.rowptr.data_ptr(),
                                              N.ptr(plan.eid), s_rowptr.data_ptr(), s_slot.data_ptr(),
                                              plan.n_nodes, gpos.data_ptr(), N.stream_ptr(g.device)),
                    "tace_edge_vec_bwd")
        if ctx.needs_input_grad[1]:
            outer = (shifts.unsqueeze(2) * g.unsqueeze(1)).reshape(-1, 9)
            if ctx.edge_graph is None:
                glat = outer.sum(0).view(1, 3, 3)
            else:
                glat = scatter_add_rows(torch.zeros(ctx.nlat, 9, dtype=g.dtype, device=g.device),
                                        ctx.edge_graph.long(), outer).view(-1, 3, 3)
        return gpos, glat, None, None, None, None


def edge_vectors(pos, lattice, shifts, plan: EdgePlan, dst: torch.Tensor, edge_graph=None) -> torch.Tensor:
    """vec[e] = pos[dst] - pos[src] + shifts[e] . lattice[edge_graph[e]]
    (``tace/models/adapter.py:334-340``) with a deterministic CSR backward.
    ``dst`` int32 [E] in edge-id order; ``edge_graph`` int32 [E] or None (one graph)."""
    if MODE.double:
        # adapter.py:334-340 as torch operations (differentiable to any order)
        L = lattice[edge_graph.long()] if edge_graph is not None else lattice[0].expand(plan.n_edges, 3, 3)
        return pos[dst.long()] - pos[plan.src.long()] + torch.einsum("ei,eij->ej", shifts.to(pos.dtype), L)
    if dst.dtype != torch.int32:
        dst = dst.to(torch.int32)
    if edge_graph is not None and edge_graph.dtype != torch.int32:
        edge_graph = edge_graph.to(torch.int32)
    return _EdgeVectors.apply(pos.contiguous(), lattice.contiguous(), shifts.contiguous(), plan, dst.contiguous(),
                              None if edge_graph is None else edge_graph.contiguous())


# ---------------------------------------------------------------- uuu ----
LAYOUT_IN1_GROUPED, LAYOUT_OUT_GROUPED, LAYOUT_IN2_GROUPED = 1, 2, 4
LAYOUT_ALL_GROUPED = 7


def launch_uuu_fwd(x1, x2, w, var: TpVariant, C: int, layout: int = 0):
    Nn = x1.shape[0]
    dt = x1.dtype
    _req(x1, "x1", dt, (Nn, C * var.d1))
    _req(x2, "x2", dt, (Nn, C * var.d2))
    if w is not None:
        _req(w, "w", dt, (Nn, C * var.npath))
    out = torch.empty(Nn, C * var.dout, dtype=dt, device=x1.device)
    tok = _t0("uuu_fwd:" + var.key)
    N.check(N.lib().tace_uuu_fwd(var.vid, N.dtype_code(dt), x1.data_ptr(), x2.data_ptr(), N.ptr(w), Nn, C, layout,
                                 out.data_ptr(), N.stream_ptr(x1.device)), "tace_uuu_fwd")
    _t1(tok, (Nn, C))
    return out


def launch_uuu_bwd(x1, x2, w, gout, var: TpVariant, C: int, layout: int = 0,
                   acc1: Optional[torch.Tensor] = None, acc2: Optional[torch.Tensor] = None):
    """(grad_x1, grad_x2, grad_w or None) of ``launch_uuu_fwd``.  ``acc1`` /
    ``acc2``: tensors shaped like x1 / x2 that the gradient is added to in
    place (and returned) instead of a new tensor; both may be one tensor when
    x1 and x2 are (then it receives both gradients)."""
    _req(gout, "g_out", x1.dtype, (x1.shape[0], C * var.dout))
    for a, x, nm in ((acc1, x1, "acc1"), (acc2, x2, "acc2")):
        if a is not None:
            _req(a, nm, x.dtype, tuple(x.shape))
    g1 = acc1 if acc1 is not None else torch.empty_like(x1)
    g2 = acc2 if acc2 is not None else torch.empty_like(x2)
    accumulate = (1 if acc1 is not None else 0) | (2 if acc2 is not None else 0)
    gw = torch.empty_like(w) if w is not None else None
    n_ws = N.lib().tace_uuu_workspace_elems(var.vid, x1.shape[0], C, accumulate)
    if n_ws < 0:
        N.check(int(n_ws), "tace_uuu_workspace_elems")
    ws = torch.empty(n_ws, dtype=x1.dtype, device=x1.device) if n_ws else None
    tok = _t0("uuu_bwd:" + var.key)
    N.check(N.lib().tace_uuu_bwd(var.vid, N.dtype_code(x1.dtype), x1.data_ptr(), x2.data_ptr(), N.ptr(w),
                                 gout.data_ptr(), x1.shape[0], C, layout, g1.data_ptr(), g2.data_ptr(), N.ptr(gw),
                                 N.ptr(ws), int(n_ws), accumulate, N.stream_ptr(x1.device)), "tace_uuu_bwd")
    _t1(tok, (x1.shape[0], C))
    return g1, g2, gw


class _UUU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x1, x2, w, var: TpVariant, C: int, layout: int):
        out = launch_uuu_fwd(x1, x2, w, var, C, layout)
        ctx.save_for_backward(x1, x2, w)
        ctx.var, ctx.C, ctx.layout = var, C, layout
        return out

    @staticmethod
    def backward(ctx, gout):
        x1, x2, w = ctx.saved_tensors
        g1, g2, gw = launch_uuu_bwd(x1, x2, w, gout.contiguous(), ctx.var, ctx.C, ctx.layout)
        return g1, g2, gw, None, None, None


# Double backward of the node product: (g1, g2, gw) are multilinear in
# (x1, x2, w, g) with g1 free of x1, g2 free of x2 and gw free of w (the scheme
# of the edge product above).  Identical inputs pass one tensor twice and
# autograd adds the two contributions.
class _UUUD(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x1, x2, w, var: TpVariant, C: int, layout: int):
        ctx.save_for_backward(x1, x2, w)
        ctx.args = (var, C, layout)
        return launch_uuu_fwd(x1, x2, w, var, C, layout)

    @staticmethod
    def backward(ctx, g):
        x1, x2, w = ctx.saved_tensors
        g1, g2, gw = _UUUBwdD.apply(x1, x2, w, g.contiguous(), *ctx.args)
        return g1, g2, (gw if w is not None else None), None, None, None


class _UUUBwdD(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x1, x2, w, g, var: TpVariant, C: int, layout: int):
        ctx.save_for_backward(x1, x2, w, g)
        ctx.args = (var, C, layout)
        g1, g2, gw = launch_uuu_bwd(x1, x2, w, g, var, C, layout)
        return g1, g2, gw if gw is not None else x1.new_zeros(0)

    @staticmethod
    def backward(ctx, a1, a2, aw):
        x1, x2, w, g = ctx.saved_tensors
        a = ctx.args
        z1 = a1.contiguous() if a1 is not None else torch.zeros_like(x1)
        z2 = a2.contiguous() if a2 is not None else torch.zeros_like(x2)
        F, B = _UUUD.apply, _UUUBwdD.apply
        gg = F(z1, x2, w, *a) + F(x1, z2, w, *a)
        b1, b2 = B(z1, x2, w, g, *a), B(x1, z2, w, g, *a)
        d1, d2, dw = b2[0], b1[1], None
        if w is not None:
            dw = b1[2] + b2[2]
            if aw is not None and aw.numel():
                zw = aw.contiguous()
                gg = gg + F(x1, x2, zw, *a)
                bw = B(x1, x2, zw, g, *a)
                d1, d2 = d1 + bw[0], d2 + bw[1]
        return d1, d2, dw, gg, None, None, None


def uuu_tp(x1, x2, var: TpVariant, C: int, layout: int = 0, w: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``layout`` = 0 (e3nn operands), LAYOUT_OUT_GROUPED, IN1|OUT or
    IN1|OUT|IN2 (LAYOUT_ALL_GROUPED): the group-major layout of
    ``include/tace_hip.h`` for x1 / out / x2.  ``w`` [N, npath*C]: per-node
    path weights (bilinear-gate product basis)."""
    if MODE.export:
        from . import library
        return library.uuu(x1, x2, w, var.key, C, int(layout))
    if MODE.double:
        return _UUUD.apply(x1.contiguous(), x2.contiguous(), None if w is None else w.contiguous(), var, C,
                           int(layout))
    return _UUU.apply(x1.contiguous(), x2.contiguous(), None if w is None else w.contiguous(), var, C, int(layout))


# ---------------------------------------------------------------- TECE ops ----
class _EdgeWigner(torch.autograd.Function):
    @staticmethod
    def forward(ctx, vec, lmax: int):
        E = vec.shape[0]
        K = (lmax + 1) ** 2
        _req(vec, "edge_vector", vec.dtype, (E, 3))
        W = torch.empty(E, K, K, dtype=vec.dtype, device=vec.device)
        tok = _t0("edge_wigner_fwd")
        N.check(N.lib().tace_edge_wigner_fwd(N.dtype_code(vec.dtype), vec.data_ptr(), E, lmax, W.data_ptr(),
                                             N.stream_ptr(vec.device)), "tace_edge_wigner_fwd")
        _t1(tok, (E, K))
        ctx.save_for_backward(vec)
        ctx.lmax = lmax
        return W

    @staticmethod
    def backward(ctx, gW):
        (vec,) = ctx.saved_tensors
        gW = gW.contiguous()
        gv = torch.empty_like(vec)
        tok = _t0("edge_wigner_bwd")
        N.check(N.lib().tace_edge_wigner_bwd(N.dtype_code(vec.dtype), vec.data_ptr(), gW.data_ptr(), vec.shape[0],
                                             ctx.lmax, gv.data_ptr(), N.stream_ptr(vec.device)), "tace_edge_wigner_bwd")
        _t1(tok, (vec.shape[0], (ctx.lmax + 1) ** 2))
        return gv, None


def _edge_frame_autograd(vec: torch.Tensor) -> torch.Tensor:
    """The edge-frame kernel's rotation R [E, 3, 3] (R @ vec/|vec| = +y) as
    torch operations: quaternion charts q+ = (1+y, -z, 0, x), q- = (-z, 1-y,
    x, 0) (w, x, y, z), normalised with eps^2 = 1e-14 inside the root, q+
    flipped onto q-'s hemisphere, nlerp with the C-infinity step of (y+1)/2
    (rotation_matrix.py:16-88)."""
    def nrm(t):
        return torch.sqrt((t * t).sum(-1, keepdim=True) + 1e-14)

    u = vec / nrm(vec)
    x, y, z = u.unbind(-1)
    zero = torch.zeros_like(x)
    qp = torch.stack([1.0 + y, -z, zero, x], -1)
    qp = qp / nrm(qp)
    qn = torch.stack([-z, 1.0 - y, x, zero], -1)
    qn = qn / nrm(qn)
    s = 0.5 * (y + 1.0)
    tiny = torch.finfo(vec.dtype).eps
    sa = torch.where(s < tiny, torch.full_like(s, tiny), s)
    sb = torch.where(1.0 - s < tiny, torch.full_like(s, tiny), 1.0 - s)
    a, b = torch.exp(-1.0 / sa), torch.exp(-1.0 / sb)
    t = torch.where(s <= 0.0, torch.zeros_like(s), torch.where(s >= 1.0, torch.ones_like(s), a / (a + b)))
    qp = torch.where((qn * qp).sum(-1, keepdim=True) < 0.0, -qp, qp)
    t = t.unsqueeze(-1)
    q = (1.0 - t) * qn + t * qp
    q = q / nrm(q)
    w, a, b, c = q.unbind(-1)
    R = [[1 - 2 * (b * b + c * c), 2 * (a * b - w * c), 2 * (a * c + w * b)],
         [2 * (a * b + w * c), 1 - 2 * (a * a + c * c), 2 * (b * c - w * a)],
         [2 * (a * c - w * b), 2 * (b * c + w * a), 1 - 2 * (a * a + b * b)]]
    return torch.stack([torch.stack(r, -1) for r in R], -2)


def so2_m_rows(lmax: int) -> List[int]:
    """e3nn component (l^2 + l + m) of every row of the SO(2) m layout
    (mmax = lmax): m = 0 for l = 0..lmax, then per m the +m and the -m rows."""
    rows = [l * l + l for l in range(lmax + 1)]
    for m in range(1, lmax + 1):
        rows += [l * l + l + m for l in range(m, lmax + 1)] + [l * l + l - m for l in range(m, lmax + 1)]
    return rows


def _edge_wigner_autograd(vec: torch.Tensor, lmax: int) -> torch.Tensor:
    """The Wigner kernel as torch operations: D^0 = 1, D^1 = R, D^l = (2l+1)
    C^T (R (x) D^(l-1)) C with C = W3j(1, l-1, l) (wigner.py:330-357), the
    block-diagonal matrix's rows in the m layout."""
    from .so3 import wigner_3j

    R = _edge_frame_autograd(vec)
    E = vec.shape[0]
    blocks = [R.new_ones(E, 1, 1)]
    if lmax >= 1:
        blocks.append(R)
    for l in range(2, lmax + 1):
        cg = torch.as_tensor(wigner_3j(1, l - 1, l), dtype=R.dtype, device=R.device)
        u = torch.einsum("abm,eac,ebd->emcd", cg, R, blocks[l - 1])
        blocks.append((2 * l + 1) * torch.einsum("emcd,cdn->emn", u, cg))
    K = (lmax + 1) ** 2
    D = torch.block_diag(*[torch.ones(2 * l + 1, 2 * l + 1) for l in range(lmax + 1)]).to(R.device) > 0
    full = R.new_zeros(E, K, K)
    full = full.masked_scatter(D.unsqueeze(0).expand(E, K, K),
                               torch.cat([b.reshape(E, -1) for b in blocks], dim=1).reshape(-1))
    return full[:, so2_m_rows(lmax), :]


def edge_wigner(vec: torch.Tensor, lmax: int) -> torch.Tensor:
    """Edge-frame Wigner matrices [E, K, K] (rows in the SO(2) m layout,
    columns e3nn components); the inverse rotation is the transpose."""
    if MODE.double:
        return _edge_wigner_autograd(vec, int(lmax))
    return _EdgeWigner.apply(vec.contiguous(), int(lmax))


def so2_block_shapes(E: int, lmax: int, ch: int) -> List[Tuple[int, int]]:
    """Shapes of the SO(2) block layout of edge features with ``ch`` channels:
    block 0 [E, (lmax+1) ch], block m [2E, (lmax+1-m) ch] (row 2e = +m rows of
    edge e, 2e+1 = its -m rows)."""
    return [(E, (lmax + 1) * ch)] + [(2 * E, (lmax + 1 - m) * ch) for m in range(1, lmax + 1)]


def so2_to_blocks(x: torch.Tensor, lmax: int) -> List[torch.Tensor]:
    """[E, K, ch] in the m layout -> the SO(2) block layout (copies)."""
    E, _, ch = x.shape
    n = lmax + 1
    out, off = [x[:, :n].reshape(E, n * ch)], n
    for m in range(1, lmax + 1):
        k = n - m
        out.append(x[:, off:off + 2 * k].reshape(2 * E, k * ch))
        off += 2 * k
    return out


def so2_from_blocks(blocks: Sequence[torch.Tensor], lmax: int) -> torch.Tensor:
    """The SO(2) block layout -> [E, K, ch] in the m layout."""
    E = blocks[0].shape[0]
    n = lmax + 1
    ch = blocks[0].shape[1] // n
    return torch.cat([blocks[0].view(E, n, ch)] + [blocks[m].reshape(E, 2 * (n - m), ch)
                                                   for m in range(1, lmax + 1)], dim=1)


def _block_array(blocks) -> "ctypes.Array":
    ptrs = [None if t is None else t.data_ptr() for t in blocks]
    return (ctypes.c_void_p * 4)(*(ptrs + [None] * (4 - len(ptrs))))


def _req_blocks(blocks, name: str, dt, E: int, lmax: int, ch: int):
    if len(blocks) != lmax + 1:
        raise ValueError(f"{name}: {len(blocks)} blocks, expected lmax+1 = {lmax + 1}")
    for m, (t, shp) in enumerate(zip(blocks, so2_block_shapes(E, lmax, ch))):
        _req(t, f"{name}[{m}]", dt, shp)


# Raw launches of the TECE kernels, shared by the autograd operators below and
# the fused chunk operator of tece.py.  bf16_out=True stores the outputs that
# feed SO(2)-linear GEMMs as bfloat16 (TACE_F32_BF16, float32 arithmetic).
TACE_F32_BF16 = 2


def _tece_code(dt, bf16_out: bool) -> int:
    if bf16_out:
        if dt != torch.float32:
            raise ValueError("bfloat16 GEMM operands need float32 arithmetic")
        return TACE_F32_BF16
    return N.dtype_code(dt)


def launch_score_fwd(q, k, rp, tscale, lmax: int, H: int) -> torch.Tensor:
    E, dt = rp.shape[0], rp.dtype
    C = q[0].shape[1] // (lmax + 1)
    _req_blocks(q, "query", dt, E, lmax, C)
    _req_blocks(k, "key", dt, E, lmax, C)
    _req(rp, "radial_proj", dt, (E, 2 * H))
    _req(tscale, "tscale", dt, (H,))
    s = torch.empty(E, H, dtype=dt, device=rp.device)
    tok = _t0("tece_score_fwd")
    N.check(N.lib().tace_tece_score_fwd(N.dtype_code(dt), _block_array(q), _block_array(k), rp.data_ptr(),
                                        tscale.data_ptr(), E, lmax, C, H, s.data_ptr(), N.stream_ptr(rp.device)),
            "tace_tece_score_fwd")
    _t1(tok, (E, (lmax + 1) ** 2, C, H))
    return s


def launch_score_bwd(q, k, rp, tscale, gs, lmax: int, H: int, bf16_out: bool = False):
    E, dt = rp.shape[0], rp.dtype
    C = q[0].shape[1] // (lmax + 1)
    _req(gs, "g_score", dt, (E, H))
    odt = torch.bfloat16 if bf16_out else dt
    gq = [torch.empty(t.shape, dtype=odt, device=t.device) for t in q]
    gk = [torch.empty(t.shape, dtype=odt, device=t.device) for t in k]
    grp = torch.empty_like(rp)
    tok = _t0("tece_score_bwd")
    N.check(N.lib().tace_tece_score_bwd(_tece_code(dt, bf16_out), _block_array(q), _block_array(k), rp.data_ptr(),
                                        tscale.data_ptr(), gs.data_ptr(), E, lmax, C, H, _block_array(gq),
                                        _block_array(gk), grp.data_ptr(), N.stream_ptr(rp.device)),
            "tace_tece_score_bwd")
    _t1(tok, (E, (lmax + 1) ** 2, C, H, bf16_out))
    return gq, gk, grp


def launch_softmax_fwd(s, plan: EdgePlan) -> torch.Tensor:
    E, H = s.shape
    _req(s, "score", s.dtype, (plan.n_edges, H))
    a = torch.empty_like(s)
    tok = _t0("graph_softmax_fwd")
    N.check(N.lib().tace_graph_softmax_fwd(N.dtype_code(s.dtype), s.data_ptr(), plan.rowptr.data_ptr(),
                                           N.ptr(plan.eid), plan.n_nodes, H, a.data_ptr(), N.stream_ptr(s.device)),
            "tace_graph_softmax_fwd")
    _t1(tok, (E, H, plan.n_nodes))
    return a


def launch_softmax_bwd(a, ga, plan: EdgePlan) -> torch.Tensor:
    _req(ga, "g_alpha", a.dtype, tuple(a.shape))
    gs = torch.empty_like(a)
    tok = _t0("graph_softmax_bwd")
    N.check(N.lib().tace_graph_softmax_bwd(N.dtype_code(a.dtype), a.data_ptr(), ga.data_ptr(), plan.rowptr.data_ptr(),
                                           N.ptr(plan.eid), plan.n_nodes, a.shape[1], gs.data_ptr(),
                                           N.stream_ptr(a.device)), "tace_graph_softmax_bwd")
    _t1(tok, (a.shape[0], a.shape[1], plan.n_nodes))
    return gs


def launch_rotate_out_fwd(m, alpha, W, plan: EdgePlan, node_map, lmax: int, H: int,
                          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Receiver sums [n_nodes, K C] (group-major, rows node_map[n]); with
    ``out`` (a whole batch's output, any row count, node_map required) the
    sums of plan's receivers go into its rows node_map[n]."""
    E, dt = W.shape[0], W.dtype
    K = (lmax + 1) ** 2
    C = m[0].shape[1] // (lmax + 1)
    _req_blocks(m, "messages", dt, plan.n_edges, lmax, C)
    _req(alpha, "alpha", dt, (E, H))
    _req(W, "wigner", dt, (E, K, K))
    if node_map is not None:
        _req(node_map, "node_map", torch.int32, (plan.n_nodes,))
    if out is None:
        out = torch.empty(plan.n_nodes, K * C, dtype=dt, device=W.device)
    else:
        if node_map is None:
            raise ValueError("rotate-out into a given output needs the receivers' rows (node_map)")
        _req(out, "out", dt, (out.shape[0], K * C))
    tok = _t0("tece_rotate_out_fwd")
    N.check(N.lib().tace_tece_rotate_out_fwd(N.dtype_code(dt), _block_array(m), alpha.data_ptr(), W.data_ptr(),
                                             plan.rowptr.data_ptr(), N.ptr(plan.eid), N.ptr(node_map), plan.n_nodes,
                                             out.shape[0], lmax, C, H, out.data_ptr(), N.stream_ptr(W.device)),
            "tace_tece_rotate_out_fwd")
    _t1(tok, (plan.n_nodes, E, C, K, H))
    return out


def launch_rotate_out_bwd(m, alpha, W, gout, dst, node_map, plan: EdgePlan, lmax: int, H: int,
                          bf16_out: bool = False, gW_out: Optional[torch.Tensor] = None,
                          g_rows: Optional[int] = None):
    """(g_m, g_alpha, g_wigner) of the rotate-out; g_wigner into ``gW_out``
    when given (a contiguous tensor of W's shape).  ``g_rows``: the row count
    of gout when it is not plan.n_nodes (a whole batch's gradient read at
    rows node_map[dst[e]] for a chunk's edges)."""
    E, dt = W.shape[0], W.dtype
    K = (lmax + 1) ** 2
    C = m[0].shape[1] // (lmax + 1)
    n_rows = plan.n_nodes if g_rows is None else int(g_rows)
    _req(gout, "g_out", dt, (n_rows, K * C))
    _req(dst, "dst", torch.int64, (E,))
    odt = torch.bfloat16 if bf16_out else dt
    gm = [torch.empty(t.shape, dtype=odt, device=t.device) for t in m]
    ga = torch.empty_like(alpha)
    if gW_out is not None:
        _req(gW_out, "gW_out", dt, tuple(W.shape))
    gW = torch.empty_like(W) if gW_out is None else gW_out
    tok = _t0("tece_rotate_out_bwd")
    N.check(N.lib().tace_tece_rotate_out_bwd(_tece_code(dt, bf16_out), _block_array(m), alpha.data_ptr(),
                                             W.data_ptr(), gout.data_ptr(), dst.data_ptr(), N.ptr(node_map),
                                             n_rows, E, lmax, C, H, _block_array(gm), ga.data_ptr(),
                                             gW.data_ptr(), N.stream_ptr(W.device)), "tace_tece_rotate_out_bwd")
    _t1(tok, (plan.n_nodes, E, C, K, H, bf16_out))
    return gm, ga, gW


def launch_rotate_in_fwd(x, W, rows_src, rows_dst, wr, lmax: int, bf16_out: bool = False):
    Nr, K, C = x.shape
    E, dt = W.shape[0], x.dtype
    if K != (lmax + 1) ** 2:
        raise ValueError(f"edge_rotate_in: {K} components, expected (lmax+1)^2 = {(lmax + 1) ** 2}")
    nc = (lmax + 1) * (lmax + 2) // 2
    _req(x, "x", dt, (Nr, K, C))
    _req(W, "wigner", dt, (E, K, K))
    if wr is not None:
        _req(wr, "radial_w", dt, (E, nc * 2 * C))
    _req(rows_src, "rows_src", torch.int64, (E,))
    _req(rows_dst, "rows_dst", torch.int64, (E,))
    odt = torch.bfloat16 if bf16_out else dt
    mk = lambda ch: [torch.empty(shp, dtype=odt, device=x.device) for shp in so2_block_shapes(E, lmax, ch)]
    ms, md = mk(C), mk(C)
    mw = mk(2 * C) if wr is not None else []
    tok = _t0("edge_rotate_in_fwd")
    N.check(N.lib().tace_edge_rotate_in_fwd(_tece_code(dt, bf16_out), x.data_ptr(), W.data_ptr(),
                                            rows_src.data_ptr(), rows_dst.data_ptr(), N.ptr(wr), Nr, E, lmax, C,
                                            _block_array(ms), _block_array(md), _block_array(mw) if mw else None,
                                            N.stream_ptr(x.device)), "tace_edge_rotate_in_fwd")
    _t1(tok, (E, K, C, wr is not None, bf16_out))
    return ms, md, mw


# the rotate-in backward's receiver rows as run sums of each workgroup's four
# edges (tace_edge_rotate_in_bwd_runs) where the edges are in receiver-CSR
# order and 4 K C values fit in 64 KB of LDS
ROTIN_RUNS = 4


def rotate_in_runs_ok(x: torch.Tensor) -> bool:
    """Whether ``launch_rotate_in_bwd(..., runs=True)`` takes node features x [rows, K, C]."""
    K, C = x.shape[1], x.shape[2]
    return 4 * K * C * x.element_size() <= 65536


def launch_rotate_in_bwd(x, W, rows_src, rows_dst, wr, gms, gmd, gmw, need_gwr: bool, runs: bool = False,
                         gW_acc: Optional[torch.Tensor] = None):
    """Per-edge grad_x rows of the senders / receivers [E, K, C] each, g_wigner
    and (need_gwr) g_radial_w; gmw None = no gradient reaches m_w.  runs
    (edges in receiver-CSR order, ``rotate_in_runs_ok``): the receiver rows
    come as run sums at the runs' first positions
    (``tace_edge_rotate_in_bwd_runs``), for ``rows_accumulate(...,
    run=ROTIN_RUNS)``.  gW_acc: a Wigner gradient with zeros off the l blocks
    (the rotate-out backward's) that g_wigner is added into and returned as."""
    Nr, K, C = x.shape
    E = W.shape[0]
    gxs = torch.empty(E, K, C, dtype=x.dtype, device=x.device)
    gxd = torch.empty_like(gxs)
    if gW_acc is not None:
        _req(gW_acc, "gW_acc", W.dtype, tuple(W.shape))
    gW = torch.empty_like(W) if gW_acc is None else gW_acc
    gwr = None
    if wr is not None and need_gwr:
        gwr = torch.empty_like(wr) if gmw is not None else torch.zeros_like(wr)
    if runs and not rotate_in_runs_ok(x):
        raise ValueError("rotate-in backward by runs: 4 K C values exceed 64 KB")
    name = "tace_edge_rotate_in_bwd_runs" if runs else "tace_edge_rotate_in_bwd"
    tok = _t0("edge_rotate_in_bwd")
    N.check(getattr(N.lib(), name)(N.dtype_code(x.dtype), x.data_ptr(), W.data_ptr(), rows_src.data_ptr(),
                                   rows_dst.data_ptr(), N.ptr(wr), _block_array(gms), _block_array(gmd),
                                   _block_array(gmw) if gmw is not None else None, Nr, E,
                                   (int(math.isqrt(K)) - 1), C, gxs.data_ptr(), gxd.data_ptr(),
                                   gW.data_ptr(), N.ptr(gwr) if gmw is not None else None,
                                   int(gW_acc is not None), N.stream_ptr(x.device)), name)
    _t1(tok, (E, K, C, gmw is not None, bool(runs)))
    return gxs, gxd, gW, gwr


def bf16_fragment_order(B: torch.Tensor) -> torch.Tensor:
    """B [k, n] bfloat16 -> the MFMA fragment order of ``tace_so2_gemm_bf16``:
    per 16-column block and 32-k step, 512 values in lane order (lane 16 g + f
    holds B[32 s + 8 g + e][16 cb + f], e < 8), zeros past k and n."""
    if B.dim() != 2 or B.dtype != torch.bfloat16:
        raise ValueError("bf16_fragment_order: B must be a 2-D bfloat16 matrix")
    k, n = B.shape
    nks, nb = (k + 31) // 32, (n + 15) // 16
    P = B.new_zeros(32 * nks, 16 * nb)
    P[:k, :n] = B
    return P.view(nks, 4, 8, nb, 16).permute(3, 0, 1, 4, 2).contiguous().view(-1)


def so2_gemm_bf16(a: torch.Tensor, b_frag: torch.Tensor, n: int, k: int,
                  bias: Optional[torch.Tensor] = None, ktiled: bool = False) -> torch.Tensor:
    """``tace_so2_gemm_bf16``: a [m, k] bfloat16 @ B [k, n] (given in fragment
    order, ``bf16_fragment_order``) with float32 sums (+ bias [n] float32);
    returns float32 [m, n].  ktiled: the k-tiled kernel
    (``tace_so2_gemm_bf16_kt``, for large k)."""
    if not a.is_cuda or a.dim() != 2 or a.dtype != torch.bfloat16 or a.shape[1] != k or a.stride(1) != 1:
        raise ValueError("so2 gemm: a must be a bfloat16 GPU matrix [m, k] with unit column stride")
    nks, nb = (k + 31) // 32, (n + 15) // 16
    if b_frag.dtype != torch.bfloat16 or b_frag.numel() != nks * nb * 512 or not b_frag.is_contiguous():
        raise ValueError("so2 gemm: the weight is not in the fragment order of a [k, n] matrix")
    if bias is not None:
        _req(bias, "bias", torch.float32, (n,))
    m = a.shape[0]
    out = torch.empty(m, n, dtype=torch.float32, device=a.device)
    tok = _t0("so2_gemm_bf16")
    fn = "tace_so2_gemm_bf16_kt" if ktiled else "tace_so2_gemm_bf16"
    N.check(getattr(N.lib(), fn)(a.data_ptr(), a.stride(0), b_frag.data_ptr(), N.ptr(bias), out.data_ptr(), n, m, n, k,
                                 N.stream_ptr(a.device)), fn)
    _t1(tok, (m, n, k))
    return out


def rows_accumulate(out: torch.Tensor, rows: torch.Tensor, rowptr: torch.Tensor, slot: Optional[torch.Tensor] = None,
                    target: Optional[torch.Tensor] = None, run: int = 1) -> torch.Tensor:
    """out[target[s]] += sum of rows[slot[k]], k in [rowptr[s], rowptr[s+1])
    (``tace_rows_accumulate``: fixed order, no atomics); returns out.  run >
    1 (slot None): only each segment's first position and the multiples of
    run inside it are read (``tace_rows_accumulate_runs``)."""
    n_seg = rowptr.numel() - 1
    dt = out.dtype
    _req(out, "out", dt)
    _req(rows, "rows", dt, (rows.shape[0], out.shape[1]))
    _req(rowptr, "rowptr", torch.int32, (n_seg + 1,))
    if slot is not None:
        _req(slot, "slot", torch.int32, (rows.shape[0],))
    if target is not None:
        _req(target, "target", torch.int32, (n_seg,))
    if run != 1 and slot is not None:
        raise ValueError("rows_accumulate: run sums are read at CSR positions (slot must be None)")
    tok = _t0("rows_accumulate")
    if run != 1:
        N.check(N.lib().tace_rows_accumulate_runs(N.dtype_code(dt), rows.data_ptr(), rows.shape[0], out.shape[1],
                                                  rowptr.data_ptr(), N.ptr(target), n_seg, int(run), out.data_ptr(),
                                                  out.shape[0], N.stream_ptr(out.device)), "tace_rows_accumulate_runs")
    else:
        N.check(N.lib().tace_rows_accumulate(N.dtype_code(dt), rows.data_ptr(), rows.shape[0], out.shape[1],
                                             rowptr.data_ptr(), N.ptr(slot), N.ptr(target), n_seg, out.data_ptr(),
                                             out.shape[0], N.stream_ptr(out.device)), "tace_rows_accumulate")
    _t1(tok, (rows.shape[0], out.shape[1], min(n_seg, out.shape[0])))
    return out


def narrow_linear(x: torch.Tensor, m: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x [rows, k] @ m [k, n] (+ bias [n]) for k, n <= 64 (``tace_narrow_linear``;
    no autograd: the fused TECE operator's radial projection and its input
    gradient)."""
    dt = x.dtype
    rows, k = x.shape
    _req(x, "x", dt)
    _req(m, "m", dt, (k, m.shape[1]))
    n = m.shape[1]
    if bias is not None:
        _req(bias, "bias", dt, (n,))
    out = torch.empty(rows, n, dtype=dt, device=x.device)
    tok = _t0("narrow_linear")
    N.check(N.lib().tace_narrow_linear(N.dtype_code(dt), x.data_ptr(), rows, k, m.data_ptr(), N.ptr(bias), n,
                                       out.data_ptr(), N.stream_ptr(x.device)), "tace_narrow_linear")
    _t1(tok, (rows, k, n))
    return out


def _graph_sum(values: torch.Tensor, ptr: torch.Tensor) -> torch.Tensor:
    """[N, w] rows -> [B, w] sums over the contiguous node ranges of ``ptr``
    [B + 1], each range summed in node order (``tace_rows_accumulate``)."""
    v = values.reshape(values.shape[0], -1).contiguous()
    _req(v, "values", v.dtype)
    p = ptr if ptr.dtype == torch.int64 else ptr.to(torch.int64)
    p = p.contiguous()
    _req(p, "ptr", torch.int64, (p.numel(),))
    out = torch.empty(p.numel() - 1, v.shape[1], dtype=v.dtype, device=v.device)
    tok = _t0("graph_sum")
    N.check(N.lib().tace_graph_sum(N.dtype_code(v.dtype), v.data_ptr(), v.shape[0], v.shape[1], p.data_ptr(),
                                   out.shape[0], out.data_ptr(), N.stream_ptr(v.device)), "tace_graph_sum")
    _t1(tok, (v.shape[0], v.shape[1], out.shape[0]))
    return out.reshape((p.numel() - 1,) + tuple(values.shape[1:]))


class _GraphSum(torch.autograd.Function):
    """Per-graph sums of node rows in a fixed order (``scatter_sum(..., batch)``
    of ``tace/utils/torch_scatter.py:43-62`` without atomics); backward: the
    graph's gradient gathered to its nodes (``_GraphGather``)."""

    @staticmethod
    def forward(ctx, values, ptr, batch):
        ctx.save_for_backward(ptr, batch)
        return _graph_sum(values, ptr)

    @staticmethod
    def backward(ctx, g):
        ptr, batch = ctx.saved_tensors
        return _GraphGather.apply(g, ptr, batch), None, None


class _GraphGather(torch.autograd.Function):
    """values[batch] for per-graph rows; backward: per-graph sums in a fixed
    order (``_GraphSum``), so both directions are repeatable bit for bit."""

    @staticmethod
    def forward(ctx, values, ptr, batch):
        ctx.save_for_backward(ptr, batch)
        return values.index_select(0, batch)

    @staticmethod
    def backward(ctx, g):
        ptr, batch = ctx.saved_tensors
        return _GraphSum.apply(g, ptr, batch), None, None


def graph_sum(values: torch.Tensor, ptr: torch.Tensor, batch: torch.Tensor) -> torch.Tensor:
    """Sum of node rows ``values`` [N, ...] per graph ([B, ...]); the nodes of
    graph b are rows ptr[b]..ptr[b+1]-1 and ``batch`` [N] their graph
    (collated batches hold both).  The same bits on every run, differentiable
    (twice as well)."""
    if MODE.export:
        from . import library
        return library.graph_sum(values, ptr, batch)
    if not values.is_cuda:
        return torch.zeros((ptr.numel() - 1,) + tuple(values.shape[1:]), dtype=values.dtype,
                           device=values.device).index_add(0, batch, values)
    return _GraphSum.apply(values, ptr, batch)


def graph_gather(values: torch.Tensor, ptr: torch.Tensor, batch: torch.Tensor) -> torch.Tensor:
    """``values[batch]`` for per-graph rows, with a fixed-order backward."""
    if MODE.export:
        from . import library
        return library.graph_gather(values, ptr, batch)
    if not values.is_cuda:
        return values.index_select(0, batch)
    return _GraphGather.apply(values, ptr, batch)


def scatter_add_rows(out: torch.Tensor, index: torch.Tensor, src: torch.Tensor) -> torch.Tensor:
    """out[index[e]] += src[e] (rows of any trailing shape).  On the GPU
    every row's terms are summed in edge order by ``tace_rows_accumulate``
    over a CSR of ``index`` (no atomics: the same bits on every run); on the
    CPU ``index_add_``.  Returns out."""
    E = src.shape[0]
    if E == 0:
        return out
    if not src.is_cuda or (torch.is_grad_enabled() and src.requires_grad):
        # CPU, or a sum that must stay differentiable
        return out.index_add_(0, index, src)
    n = out.shape[0]
    rp, slot = sender_csr(index.long(), n)
    return rows_accumulate(out.view(n, -1), src.reshape(E, -1).contiguous(), rp, slot).view(out.shape)


def group_by_key(keys: torch.Tensor, n_keys: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """(rowptr int32 [n_keys+1], order int32 [E]) of keys in [0, n_keys): the
    positions grouped by key, in position order within a key (a stable sort
    of 32-bit keys, half the radix passes of 64-bit ones), and each key's
    range from a binary search of the sorted keys (no atomics, no host
    synchronisation)."""
    if n_keys >= 2 ** 31:
        raise ValueError("group_by_key: more than 2^31 keys")
    k32 = keys.to(torch.int32)
    srt, order = torch.sort(k32, stable=True)
    bounds = torch.arange(n_keys + 1, dtype=torch.int32, device=keys.device)
    rp = torch.searchsorted(srt, bounds, out_int32=True)
    return rp.contiguous(), order.to(torch.int32).contiguous()


def sender_csr(rows_src: torch.Tensor, n_rows: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """(rowptr int32 [n_rows+1], slot int32 [E]): the edges grouped by sender
    row, in edge order within a sender."""
    return group_by_key(rows_src, n_rows)


def _pad4(lst):
    return [N.ptr(t) for t in lst] + [None] * (4 - len(lst))


def launch_edge_ace_fwd(ys, lmax: int, A: int, bf16_out: bool = False):
    n = lmax + 1
    y0 = ys[0]
    E, dt = y0.shape[0], y0.dtype
    P = len(edge_ace_paths(lmax))
    _req(y0, "y0", dt, (E, P * n * A + n * A + (n * (lmax + 1) + n) * A))
    for m in range(1, lmax + 1):
        _req(ys[m], f"y{m}", dt, (2 * E, 2 * n * A))
    odt = torch.bfloat16 if bf16_out else dt
    outs = [torch.empty(E if m == 0 else 2 * E, n * A, dtype=odt, device=y0.device) for m in range(lmax + 1)]
    tok = _t0("tece_edge_ace_fwd")
    N.check(N.lib().tace_tece_edge_ace_fwd(_tece_code(dt, bf16_out), *_pad4(list(ys)), E, lmax, A, *_pad4(outs),
                                           N.stream_ptr(y0.device)), "tace_tece_edge_ace_fwd")
    _t1(tok, (E, A, lmax, bf16_out))
    return outs


def launch_edge_ace_bwd(ys, gos, lmax: int, A: int, bf16_out: bool = False):
    E, dt = ys[0].shape[0], ys[0].dtype
    for m, g in enumerate(gos):
        _req(g, f"g_o{m}", dt, (E if m == 0 else 2 * E, (lmax + 1) * A))
    odt = torch.bfloat16 if bf16_out else dt
    gys = [torch.empty(y.shape, dtype=odt, device=y.device) for y in ys]
    tok = _t0("tece_edge_ace_bwd")
    N.check(N.lib().tace_tece_edge_ace_bwd(_tece_code(dt, bf16_out), *_pad4(list(ys)), *_pad4(list(gos)), E, lmax, A,
                                           *_pad4(gys), N.stream_ptr(ys[0].device)), "tace_tece_edge_ace_bwd")
    _t1(tok, (E, A, lmax, bf16_out))
    return gys


class _TeceScore(torch.autograd.Function):
    @staticmethod
    def forward(ctx, rp, tscale, lmax: int, H: int, C: int, *qk):
        n = lmax + 1
        q, k = list(qk[:n]), list(qk[n:])
        s = launch_score_fwd(q, k, rp, tscale, lmax, H)
        ctx.save_for_backward(rp, tscale, *q, *k)
        ctx.lmax, ctx.H = lmax, H
        return s

    @staticmethod
    def backward(ctx, gs):
        rp, tscale, *qk = ctx.saved_tensors
        n = ctx.lmax + 1
        gq, gk, grp = launch_score_bwd(qk[:n], qk[n:], rp, tscale, gs.contiguous(), ctx.lmax, ctx.H)
        # the attention temperature is a model parameter: no gradient on this
        # (inference) path, as the calculators freeze parameters
        return (grp, None, None, None, None) + tuple(gq) + tuple(gk)


def tece_score(q: Sequence[torch.Tensor], k: Sequence[torch.Tensor], radial_proj, tscale, lmax: int,
               heads: int) -> torch.Tensor:
    """Radial-rotary complex QK score [E, heads] of query / key in the SO(2)
    block layout (tscale = attention scale x temperature)."""
    if tscale.requires_grad:
        raise ValueError("tece_score: the temperature gradient is not computed (parameters must be frozen)")
    C = q[0].shape[1] // (lmax + 1)
    return _TeceScore.apply(radial_proj.contiguous(), tscale.contiguous(), int(lmax), int(heads), C,
                            *[t.contiguous() for t in q], *[t.contiguous() for t in k])


class _GraphSoftmax(torch.autograd.Function):
    @staticmethod
    def forward(ctx, s, plan: EdgePlan):
        a = launch_softmax_fwd(s, plan)
        ctx.save_for_backward(a)
        ctx.plan = plan
        return a

    @staticmethod
    def backward(ctx, ga):
        (a,) = ctx.saved_tensors
        return launch_softmax_bwd(a, ga.contiguous(), ctx.plan), None


def graph_softmax(score: torch.Tensor, plan: EdgePlan) -> torch.Tensor:
    """Softmax of ``score`` [E, H] over each receiver's in-edges (receiver CSR)."""
    return _GraphSoftmax.apply(score.contiguous(), plan)


class _TeceRotateOut(torch.autograd.Function):
    @staticmethod
    def forward(ctx, alpha, W, plan: EdgePlan, node_map, dst, lmax: int, H: int, C: int, *m):
        out = launch_rotate_out_fwd(list(m), alpha, W, plan, node_map, lmax, H)
        ctx.save_for_backward(alpha, W, node_map, dst, *m)
        ctx.plan, ctx.lmax, ctx.H = plan, lmax, H
        return out

    @staticmethod
    def backward(ctx, gout):
        alpha, W, node_map, dst, *m = ctx.saved_tensors
        gm, ga, gW = launch_rotate_out_bwd(m, alpha, W, gout.contiguous(), dst, node_map, ctx.plan, ctx.lmax, ctx.H)
        return (ga, gW, None, None, None, None, None, None) + tuple(gm)


def tece_rotate_out(m: Sequence[torch.Tensor], alpha, W, plan: EdgePlan, node_map, dst, lmax: int,
                    heads: int) -> torch.Tensor:
    """sum_{e -> n} W[e]^T (alpha[e] m[e]) per receiver n for messages in the
    SO(2) block layout, written in the group-major layout of C x (0..lmax) at
    rows node_map[n] ([N, K*C])."""
    dst = dst.long().contiguous()
    if dst.shape != (plan.n_edges,):
        raise ValueError(f"tece_rotate_out: dst has shape {tuple(dst.shape)}, expected ({plan.n_edges},)")
    C = m[0].shape[1] // (lmax + 1)
    return _TeceRotateOut.apply(alpha.contiguous(), W.contiguous(), plan, node_map, dst, int(lmax), int(heads), C,
                                *[t.contiguous() for t in m])


class _EdgeRotateIn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, W, wr, rows_src, rows_dst, lmax: int):
        ms, md, mw = launch_rotate_in_fwd(x, W, rows_src, rows_dst, wr, lmax)
        ctx.save_for_backward(x, W, wr, rows_src, rows_dst)
        ctx.lmax, ctx.n = lmax, lmax + 1
        ctx.set_materialize_grads(False)
        return tuple(ms + md + mw)

    @staticmethod
    def backward(ctx, *g):
        x, W, wr, rows_src, rows_dst = ctx.saved_tensors
        n = ctx.n
        g = [t.contiguous() if t is not None else None for t in g]
        gms, gmd, gmw = g[:n], g[n:2 * n], g[2 * n:]
        has_w = any(t is not None for t in gmw)
        gxs, gxd, gW, gwr = launch_rotate_in_bwd(x, W, rows_src, rows_dst, wr, gms, gmd, gmw if has_w else None,
                                                 ctx.needs_input_grad[2])
        gx = None
        if ctx.needs_input_grad[0]:
            gx = scatter_add_rows(scatter_add_rows(torch.zeros_like(x), rows_src, gxs), rows_dst, gxd)
        return gx, gW, gwr, None, None, None


def edge_rotate_in(x: torch.Tensor, W: torch.Tensor, rows_src: torch.Tensor, rows_dst: torch.Tensor, lmax: int,
                   radial_w: Optional[torch.Tensor] = None):
    """Edge-frame messages m = W[e] @ [x[rows_src[e]] | x[rows_dst[e]]] for node
    features x [rows, K, C] (l layout), in the SO(2) block layout: returns
    (m_src, m_dst) block lists (first / last C channels) and, with radial
    weights [E, ncomp * 2C], also the radially weighted m_w block list (2C
    channels; +m and -m rows share a weight component)."""
    out = _EdgeRotateIn.apply(x.contiguous(), W.contiguous(), None if radial_w is None else radial_w.contiguous(),
                              rows_src.long().contiguous(), rows_dst.long().contiguous(), int(lmax))
    n = lmax + 1
    blocks = [list(out[i * n:(i + 1) * n]) for i in range(len(out) // n)]
    return tuple(blocks)


# ---- TECE rotate-in / rotate-out, twice differentiable (training) ----------
# Both are multilinear: rotate-in m_s = W x_src, m_d = W x_dst, m_w = w (.)
# [m_s | m_d] in (x, W, w), rotate-out out = sum_e W_e^T (alpha_e m_e) in (m,
# alpha, W), and every gradient of their backward is free of its own operand
# (grad_x(W, w, g), grad_W(x, w, g), grad_w(x, W, g)).  So the backward of the
# backward is made of the forward and backward operators again, as for the
# edge tensor product: for upstream gradients (a_x, a_W, a_w) of the backward's
# outputs, d/dg = f(a_x, W, w) + f(x, a_W, w) + f(x, W, a_w); d/dx = the x part
# of bwd(x, a_W, w, g) + of bwd(x, W, a_w, g); and so on.  Rotate-in's m_s and
# m_d do not depend on w, so the a_w terms use m_w and its gradient alone.
def _rot_in_zero_sd(blocks, n):
    return [torch.zeros_like(t) for t in blocks[:2 * n]] + list(blocks[2 * n:])


class _RotInD(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, W, wr, rows_src, rows_dst, lmax: int):
        ms, md, mw = launch_rotate_in_fwd(x, W, rows_src, rows_dst, wr, lmax)
        ctx.save_for_backward(x, W, wr, rows_src, rows_dst)
        ctx.lmax = lmax
        ctx.like = [(t.shape, t.dtype) for t in ms + md + mw]
        return tuple(ms + md + mw)

    @staticmethod
    def backward(ctx, *g):
        x, W, wr, rs, rd = ctx.saved_tensors
        g = [t.contiguous() if t is not None else torch.zeros(shp, dtype=dt, device=x.device)
             for t, (shp, dt) in zip(g, ctx.like)]
        gx, gW, gwr = _RotInBwdD.apply(x, W, wr, rs, rd, ctx.lmax, *g)
        return gx, gW, gwr, None, None, None


class _RotInBwdD(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, W, wr, rs, rd, lmax: int, *g):
        n = lmax + 1
        gxs, gxd, gW, gwr = launch_rotate_in_bwd(x, W, rs, rd, wr, list(g[:n]), list(g[n:2 * n]),
                                                 list(g[2 * n:]), True)
        Nr, K, C = x.shape
        gx = scatter_add_rows(scatter_add_rows(torch.zeros_like(x), rs, gxs), rd, gxd)
        ctx.save_for_backward(x, W, wr, rs, rd, *g)
        ctx.lmax = lmax
        return gx, gW, gwr

    @staticmethod
    def backward(ctx, ax, aW, aw):
        x, W, wr, rs, rd, *g = ctx.saved_tensors
        L, n = ctx.lmax, ctx.lmax + 1
        zx = ax if ax is not None else torch.zeros_like(x)
        zW = aW if aW is not None else torch.zeros_like(W)
        zw = aw if aw is not None else torch.zeros_like(wr)
        fwd = lambda a, b, c: _RotInD.apply(a.contiguous(), b.contiguous(), c.contiguous(), rs, rd, L)
        bwd = lambda a, b, c, gg: _RotInBwdD.apply(a.contiguous(), b.contiguous(), c.contiguous(), rs, rd, L, *gg)
        f1, f2, f3 = fwd(zx, W, wr), fwd(x, zW, wr), fwd(x, W, zw)
        dg = [a + b + (c if k >= 2 * n else 0.0) for k, (a, b, c) in enumerate(zip(f1, f2, f3))]
        gw_only = _rot_in_zero_sd(g, n)
        b1 = bwd(zx, W, wr, g)          # W and w parts with x -> a_x
        b2 = bwd(x, zW, wr, g)          # x and w parts with W -> a_W
        b3 = bwd(x, W, zw, gw_only)     # x and W parts with w -> a_w (m_w only)
        return (b2[0] + b3[0], b1[1] + b3[1], b1[2] + b2[2], None, None, None) + tuple(dg)


def edge_rotate_in_twice(x, W, rows_src, rows_dst, lmax: int, radial_w):
    """``edge_rotate_in`` (radial weights required) whose backward is
    differentiable again (training with a force loss)."""
    out = _RotInD.apply(x.contiguous(), W.contiguous(), radial_w.contiguous(), rows_src.long().contiguous(),
                        rows_dst.long().contiguous(), int(lmax))
    n = lmax + 1
    return [list(out[i * n:(i + 1) * n]) for i in range(3)]


class _RotOutD(torch.autograd.Function):
    @staticmethod
    def forward(ctx, alpha, W, plan: EdgePlan, node_map, dst, lmax: int, H: int, *m):
        out = launch_rotate_out_fwd(list(m), alpha, W, plan, node_map, lmax, H)
        ctx.save_for_backward(alpha, W, node_map, dst, *m)
        ctx.plan, ctx.lmax, ctx.H = plan, lmax, H
        return out

    @staticmethod
    def backward(ctx, gout):
        alpha, W, node_map, dst, *m = ctx.saved_tensors
        out = _RotOutBwdD.apply(alpha, W, gout.contiguous(), ctx.plan, node_map, dst, ctx.lmax, ctx.H, *m)
        ga, gW, gm = out[0], out[1], out[2:]
        return (ga, gW, None, None, None, None, None) + tuple(gm)


class _RotOutBwdD(torch.autograd.Function):
    @staticmethod
    def forward(ctx, alpha, W, gout, plan: EdgePlan, node_map, dst, lmax: int, H: int, *m):
        gm, ga, gW = launch_rotate_out_bwd(list(m), alpha, W, gout, dst, node_map, plan, lmax, H)
        ctx.save_for_backward(alpha, W, gout, node_map, dst, *m)
        ctx.plan, ctx.lmax, ctx.H = plan, lmax, H
        return (ga, gW) + tuple(gm)

    @staticmethod
    def backward(ctx, aa, aW, *am):
        alpha, W, gout, node_map, dst, *m = ctx.saved_tensors
        plan, L, H = ctx.plan, ctx.lmax, ctx.H
        za = aa if aa is not None else torch.zeros_like(alpha)
        zW = aW if aW is not None else torch.zeros_like(W)
        zm = [a if a is not None else torch.zeros_like(t) for a, t in zip(am, m)]
        fwd = lambda a, b, mm: _RotOutD.apply(a.contiguous(), b.contiguous(), plan, node_map, dst, L, H,
                                              *[t.contiguous() for t in mm])
        bwd = lambda a, b, mm: _RotOutBwdD.apply(a.contiguous(), b.contiguous(), gout, plan, node_map, dst, L, H,
                                                 *[t.contiguous() for t in mm])
        dg = fwd(alpha, W, zm) + fwd(za, W, m) + fwd(alpha, zW, m)
        b_m = bwd(alpha, W, zm)    # alpha and W parts with m -> a_m
        b_a = bwd(za, W, m)        # m and W parts with alpha -> a_alpha
        b_W = bwd(alpha, zW, m)    # m and alpha parts with W -> a_W
        ga = b_m[0] + b_W[0]
        gW = b_m[1] + b_a[1]
        gm = [p + q for p, q in zip(b_a[2:], b_W[2:])]
        return (ga, gW, dg, None, None, None, None, None) + tuple(gm)


def tece_rotate_out_twice(m, alpha, W, plan: EdgePlan, node_map, dst, lmax: int, heads: int) -> torch.Tensor:
    """``tece_rotate_out`` whose backward is differentiable again."""
    return _RotOutD.apply(alpha.contiguous(), W.contiguous(), plan, node_map, dst.long().contiguous(), int(lmax),
                          int(heads), *[t.contiguous() for t in m])


def launch_mlp_hidden_fwd(radial, weights, n_layers: int) -> torch.Tensor:
    """Hidden layers of the radial MLP: the last hidden activations h [E, 64]
    (the backward recomputes the rest from ``radial``)."""
    E, n_in = radial.shape
    dt = radial.dtype
    width = 64
    _req(radial, "radial", dt, (E, n_in))
    _req(weights, "weights", dt, (n_in * width + (n_layers - 1) * width * width,))
    h = torch.empty(E, width, dtype=dt, device=radial.device)
    tok = _t0("radial_mlp_fwd")
    N.check(N.lib().tace_radial_mlp_fwd(N.dtype_code(dt), radial.data_ptr(), E, n_in, n_layers, weights.data_ptr(),
                                        h.data_ptr(), N.stream_ptr(radial.device)), "tace_radial_mlp_fwd")
    _t1(tok, (E, n_in, n_layers))
    return h


def launch_mlp_hidden_bwd(radial, gh, weights, n_layers: int) -> torch.Tensor:
    """grad of ``radial`` from the grad of the last hidden activations."""
    E, n_in = radial.shape
    _req(gh, "g_h", radial.dtype, (E, 64))
    g = torch.empty(E, n_in, dtype=radial.dtype, device=radial.device)
    tok = _t0("radial_mlp_bwd")
    N.check(N.lib().tace_radial_mlp_bwd(N.dtype_code(radial.dtype), radial.data_ptr(), gh.data_ptr(), E, n_in,
                                        n_layers, weights.data_ptr(), g.data_ptr(), N.stream_ptr(radial.device)),
            "tace_radial_mlp_bwd")
    _t1(tok, (E, n_in, n_layers))
    return g


class _RadialMlp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, radial, weights, n_layers: int):
        h = launch_mlp_hidden_fwd(radial, weights, n_layers)
        ctx.save_for_backward(radial, weights)
        ctx.n_layers = n_layers
        return h

    @staticmethod
    def backward(ctx, gh):
        radial, weights = ctx.saved_tensors
        return launch_mlp_hidden_bwd(radial, gh.contiguous(), weights, ctx.n_layers), None, None


def launch_mlp_out_f32(h, W, alpha: float) -> torch.Tensor:
    """alpha h @ W in float32 on the bf16 MFMA, both operands split into three
    bf16 terms (h [E, 64], W [64, n_out])."""
    E = h.shape[0]
    _req(h, "h", torch.float32, (E, 64))
    _req(W, "weight", torch.float32, (64, W.shape[1]))
    out = torch.empty(E, W.shape[1], dtype=torch.float32, device=h.device)
    tok = _t0("radial_mlp_out")
    N.check(N.lib().tace_radial_mlp_out_f32(h.data_ptr(), W.data_ptr(), E, W.shape[1], float(alpha), out.data_ptr(),
                                            N.stream_ptr(h.device)), "tace_radial_mlp_out_f32")
    _t1(tok, (E, W.shape[1]))
    return out


def launch_mlp_out_bwd_f32(g, W, alpha: float) -> torch.Tensor:
    """alpha g @ W^T (g [E, n_out], W [64, n_out]): the last layer's input
    gradient, in float32 on the bf16 MFMA (three-term split)."""
    E, n = g.shape
    _req(g, "g_out", torch.float32, (E, n))
    _req(W, "weight", torch.float32, (64, n))
    gh = torch.empty(E, 64, dtype=torch.float32, device=g.device)
    tok = _t0("radial_mlp_out_bwd")
    N.check(N.lib().tace_radial_mlp_out_bwd_f32(g.data_ptr(), W.data_ptr(), E, n, float(alpha), gh.data_ptr(),
                                                N.stream_ptr(g.device)), "tace_radial_mlp_out_bwd_f32")
    _t1(tok, (E, n))
    return gh


def launch_mlp_out_bwd_pairs_f32(g, pairs: EdgePairs, W, alpha: float) -> torch.Tensor:
    """alpha (g[row_edges] + g[row_partner]) @ W^T per pair row: the last
    layer's input gradient for weights shared by the two edges of a pair."""
    E, n = g.shape
    _req(g, "g_out", torch.float32, (E, n))
    _req(W, "weight", torch.float32, (64, n))
    gh = torch.empty(pairs.n_rows, 64, dtype=torch.float32, device=g.device)
    tok = _t0("radial_mlp_out_bwd")
    N.check(N.lib().tace_radial_mlp_out_bwd_pairs_f32(g.data_ptr(), pairs.row_edges.data_ptr(),
                                                      pairs.row_partner.data_ptr(), pairs.n_rows, n, float(alpha),
                                                      W.data_ptr(), gh.data_ptr(), N.stream_ptr(g.device)),
            "tace_radial_mlp_out_bwd_pairs_f32")
    _t1(tok, (E, n))
    return gh


class _MlpOut(torch.autograd.Function):
    @staticmethod
    def forward(ctx, h, W, alpha: float):
        out = launch_mlp_out_f32(h, W, alpha)
        ctx.save_for_backward(W)
        ctx.alpha = alpha
        return out

    @staticmethod
    def backward(ctx, g):
        (W,) = ctx.saved_tensors
        return launch_mlp_out_bwd_f32(g.contiguous(), W, ctx.alpha), None, None


def radial_mlp_out(h: torch.Tensor, W: torch.Tensor, alpha: float) -> torch.Tensor:
    """alpha h @ W for the width-64 last hidden activations: the fp32 MFMA
    kernel for float32 (weights as constants: gradient to h only), a GEMM
    otherwise."""
    if h.dtype == torch.float32:
        return _MlpOut.apply(h.contiguous(), W.detach().contiguous(), float(alpha))
    return h.new_empty(h.shape[0], W.shape[1]).addmm_(h, W, beta=0.0, alpha=alpha)


def radial_mlp_hidden(radial: torch.Tensor, mats: Sequence[torch.Tensor]) -> torch.Tensor:
    """silu(... silu(radial @ mats[0]) ... @ mats[-1]) for width-64 hidden
    layers (scales folded into ``mats``): the last hidden activations [E, 64].
    The matrices are constants here: gradients flow to ``radial`` only."""
    flat = torch.cat([m.detach().reshape(-1) for m in mats]).to(radial.dtype).contiguous()
    return _RadialMlp.apply(radial.contiguous(), flat, len(mats))


# ------------------------------------------------------ per-species linears ----
# output blocks of at least this many columns whose tiles have one
# contribution with k <= 256 (or none) go to tace_seg_linear_presplit_ks
# (pre-split plans only; None: every tile to the tile kernel)
SEG_KS_MIN_N = 256
# columns per tace_seg_linear_presplit_ks task
SEG_KS_CHUNK = 1024
# pre-split plans' tiles read the weights in fragment order
# (tace_seg_linear_presplit_frag) when every instruction has a
# fragment-order block; False: the planes of tace_seg_linear_presplit
SEG_TILE_FRAG = True
# fragment-order tile launches of at most SEG_SPLIT_MAX_TILES tiles (too
# few to fill the GPU) may split each tile's k over several workgroups
# (tace_seg_linear_presplit_frag_split): SEG_SPLIT_SLOTS is the number of
# tile workgroups the GPU runs at once (two per CU; None: never split), a
# split takes at least SEG_SPLIT_MIN_STEPS 32-k steps.  Measured: the
# 1,024-atom alloy's model step 3.24 -> 2.90 ms; the ragged batch's 342-tile
# launches were slower split (uneven tile heights), hence the tile limit
SEG_SPLIT_SLOTS = 512
SEG_SPLIT_MIN_STEPS = 8
SEG_SPLIT_MAX_TILES = 192


def seg_split_count(n_tiles: int, nks_min: int, nks_max: int) -> int:
    """Splits per tile (1: none) for n_tiles tiles of nks_min .. nks_max
    32-k steps: the fewest time units by a model in which the launch runs in
    rounds of SEG_SPLIT_SLOTS workgroups, a workgroup takes one unit per step
    plus one, and the partial sums' launch takes two."""
    if SEG_SPLIT_SLOTS is None or n_tiles <= 0 or n_tiles > SEG_SPLIT_MAX_TILES:
        return 1
    slots = int(SEG_SPLIT_SLOTS)
    best, best_c = 1, -(-n_tiles // slots) * (nks_max + 1)
    for S in range(2, min(64, nks_min // max(1, SEG_SPLIT_MIN_STEPS)) + 1):
        c = -(-n_tiles * S // slots) * (-(-nks_max // S) + 1) + 2
        if c < best_c:
            best, best_c = S, c
    return best


class SegLinearPlan:
    """Device tables of ``tace_seg_linear`` for one direction of one
    per-species linear over one set of species row ranges.

    out_blocks: per output block (s, n, d, bias_off): element column offset s
    of the block in the group-major feature row (the block starts at element
    Z*s), width n, 2l+1 = d, bias offset within one species' bias (None = no
    bias).  ins: (out_block, s_in, k, w_off, trans, scale) contributions (k =
    input block width, w_off = weight offset within one species' weights).
    ranges: [(species or None, a, b)] node ranges (species-sorted rows; None =
    the shared weight).  w_stride / b_stride: elements per species of weight /
    bias.  x_numel / y_numel / w_numel / b_numel: sizes every offset is
    checked against before the tables go to the device.  tile: (rows, cols)
    of the output tiles (float32 MFMA kernel: (128, 128); FMA kernel:
    (64, 64))."""

    def __init__(self, Z, out_blocks, ins, ranges, w_stride, b_stride, x_numel, y_numel, w_numel, b_numel, device,
                 tile: Tuple[int, int] = (64, 64), split_weights: bool = False,
                 frag: Optional[Tuple[int, int]] = None):
        TM, TN = tile
        self.tile = tuple(tile)
        # split_weights: w_off / w_stride / w_numel index the pre-split planes
        # (one plane), where a contribution's block is n columns of ceil8(k)
        self.split_weights = bool(split_weights)
        if self.split_weights and self.tile != (128, 128):
            raise ValueError("pre-split weights run on the 128 x 128 float32 MFMA tiles")
        tiles, contribs, scales, tasks = [], [], [], []
        nc = 0
        # frag: (per-species stride, size) of the fragment-order weights that
        # the short-k tasks read; an instruction's offset there is its 7th item
        # (-1: not split that way)
        self.frag_numel = frag[1] if frag is not None else 0
        # the tiles read B in fragment order too (tace_seg_linear_presplit_frag)
        # when every instruction has a fragment-order block
        self.tile_frag = bool(self.split_weights and frag is not None and SEG_TILE_FRAG
                              and all(len(c) > 6 and c[6] >= 0 for c in ins))
        for ob, (s_o, n, d, boff) in enumerate(out_blocks):
            mine = [c for c in ins if c[0] == ob]
            if (self.split_weights and frag is not None and SEG_KS_MIN_N is not None and n >= SEG_KS_MIN_N
                    and len(mine) <= 1 and all(c[2] <= 256 and c[6] >= 0 for c in mine)):
                tasks += self._ks_tasks(Z, s_o, n, d, boff, mine, ranges, frag[0], b_stride)
                continue
            c0s = np.arange(0, n, TN, dtype=np.int64)
            for (sp, a, b) in ranges:
                if b <= a:
                    continue
                r0 = np.arange(a * d, b * d, TM, dtype=np.int64)
                rows = np.minimum(b * d - r0, TM)
                R, Cc = np.meshgrid(r0, c0s, indexing="ij")
                Rows = np.broadcast_to(rows[:, None], R.shape)
                T = R.size
                t = np.zeros((T, 8), dtype=np.int64)
                t[:, 0] = Z * s_o + R.ravel() * n
                t[:, 1] = Rows.ravel()
                t[:, 2] = n
                t[:, 3] = Cc.ravel()
                t[:, 4] = -1 if boff is None else boff + (0 if sp is None else sp * b_stride)
                k_each = len(mine)
                t[:, 5] = nc + np.arange(T, dtype=np.int64) * k_each
                t[:, 6] = t[:, 5] + k_each
                nc += T * k_each
                tiles.append(t)
                if k_each:
                    c = np.zeros((T, k_each, 4), dtype=np.int64)
                    for j, (_, s_i, k, w_off, trans, sc, *_f) in enumerate(mine):
                        c[:, j, 0] = Z * s_i + R.ravel() * k
                        c[:, j, 1] = k
                        if self.tile_frag:
                            c[:, j, 2] = _f[0] + (0 if sp is None else sp * frag[0])
                        else:
                            c[:, j, 2] = w_off + (0 if sp is None else sp * w_stride)
                        c[:, j, 3] = int(trans)
                    contribs.append(c.reshape(-1, 4))
                    scales.append(np.tile(np.array([m[5] for m in mine], dtype=np.float64), T))
        t = np.concatenate(tiles) if tiles else np.zeros((0, 8), dtype=np.int64)
        c = np.concatenate(contribs) if contribs else np.zeros((0, 4), dtype=np.int64)
        s = np.concatenate(scales) if scales else np.zeros(0, dtype=np.float64)
        # every access of every tile inside its array
        if len(t):
            last_col = np.minimum(t[:, 3] + TN, t[:, 2])
            if (t[:, 0] + (t[:, 1] - 1) * t[:, 2] + last_col).max() > y_numel:
                raise ValueError("seg linear plan: output tile out of range")
            if (t[:, 4] >= 0).any() and (t[:, 4] + t[:, 2])[t[:, 4] >= 0].max() > b_numel:
                raise ValueError("seg linear plan: bias out of range")
        if len(c):
            rows_c = np.repeat(t[:, 1], t[:, 6] - t[:, 5])
            n_c = np.repeat(t[:, 2], t[:, 6] - t[:, 5])
            if (c[:, 0] + rows_c * c[:, 1]).max() > x_numel:
                raise ValueError("seg linear plan: input tile out of range")
            if self.tile_frag:
                fsz = 3 * ((n_c + 15) // 16 * 16) * ((c[:, 1] + 31) // 32 * 32)
                if (c[:, 2] + fsz).max() > self.frag_numel:
                    raise ValueError("seg linear plan: fragment-order weight out of range")
            else:
                kw = (c[:, 1] + 7) // 8 * 8 if self.split_weights else c[:, 1]
                if (c[:, 2] + kw * n_c).max() > w_numel:
                    raise ValueError("seg linear plan: weight out of range")
            if self.split_weights and (c[:, 2] % 8).any():
                raise ValueError("seg linear plan: pre-split weight blocks must start on 8-element boundaries")
        self.n_tiles = len(t)
        # every contribution's x rows start on a 16-byte boundary (offsets and
        # k multiples of 4): the fragment-order tiles' aligned A loads
        self.tile_aligned = bool(len(c) == 0 or (((c[:, 0] % 4) == 0) & ((c[:, 1] % 4) == 0)).all())
        # k split over `splits` workgroups per tile when the tiles are too few
        # to fill the GPU (fragment-order tiles with one contribution each)
        self.splits = 1
        if self.tile_frag and len(t) and ((t[:, 6] - t[:, 5]) == 1).all():
            nks = (c[t[:, 5], 1] + 31) // 32
            self.splits = seg_split_count(len(t), int(nks.min()), int(nks.max()))
        self.x_numel, self.y_numel, self.w_numel, self.b_numel = x_numel, y_numel, w_numel, b_numel
        # multiply-adds x 2 of the whole launch (rows x valid columns x summed k
        # of every tile): the algorithmic flops of the GEMMs, padding excluded
        self.flops = 0
        if len(t) and len(c):
            ksum = np.concatenate([[0], np.cumsum(c[:, 1])])
            self.flops = int(2 * (t[:, 1] * np.minimum(TN, t[:, 2] - t[:, 3]) * (ksum[t[:, 6]] - ksum[t[:, 5]])).sum())
        self.tiles = torch.from_numpy(np.ascontiguousarray(t)).to(device)
        self.contribs = torch.from_numpy(np.ascontiguousarray(c) if len(c) else np.zeros((1, 4), np.int64)).to(device)
        self.scales = torch.from_numpy(s if len(s) else np.zeros(1)).to(device)
        # short-k tasks (tace_seg_linear_presplit_ks), checked like the tiles
        k_t = np.asarray(tasks, dtype=np.int64).reshape(-1, 10)
        if len(k_t):
            if (k_t[:, 0] + (k_t[:, 1] - 1) * k_t[:, 2] + k_t[:, 4]).max() > y_numel:
                raise ValueError("seg linear plan: output task out of range")
            if (k_t[:, 0] < 0).any() or (k_t[:, 4] > k_t[:, 2]).any() or (k_t[:, 3] >= k_t[:, 4]).any():
                raise ValueError("seg linear plan: bad task columns")
            hb = k_t[:, 5] >= 0
            if hb.any() and (k_t[hb, 5] + k_t[hb, 4]).max() > b_numel:
                raise ValueError("seg linear plan: bias out of range")
            hk = k_t[:, 7] > 0
            if hk.any():
                if (k_t[hk, 6] + k_t[hk, 1] * k_t[hk, 7]).max() > x_numel:
                    raise ValueError("seg linear plan: input task out of range")
                fsz = 3 * ((k_t[hk, 2] + 15) // 16 * 16) * ((k_t[hk, 7] + 31) // 32 * 32)
                if (k_t[hk, 8] + fsz).max() > self.frag_numel or (k_t[hk, 8] % 8).any():
                    raise ValueError("seg linear plan: fragment-order weights of a task out of range")
            self.flops += int(2 * (k_t[:, 1] * (k_t[:, 4] - k_t[:, 3]) * k_t[:, 7]).sum())
        self.n_ks = len(k_t)
        # one launch per task height (128 rows: k <= 128, 64 rows: k <= 256)
        self.ks_groups = []
        if len(k_t):
            by_k = {int(k): self._ks_rows(int(k)) for k in np.unique(k_t[:, 7])}
            hts = np.array([by_k[int(k)] for k in k_t[:, 7]], dtype=np.int64)
            for R in (128, 64):
                sel = k_t[hts == R]
                if len(sel):
                    if (sel[:, 1] > R).any():
                        raise ValueError("seg linear plan: a task is taller than its kernel's tile")
                    if (sel[:, 7] > (128 if R == 128 else 256)).any():
                        raise ValueError("seg linear plan: a task's k exceeds its kernel's limit")
                    self.ks_groups.append((R, len(sel), torch.from_numpy(np.ascontiguousarray(sel)).to(device)))

    @staticmethod
    def _ks_rows(k: int) -> int:
        """Task height of ``tace_seg_linear_presplit_ks`` for contributions of
        width k (k = 0: a block without contribution, 128 rows)."""
        R = N.lib().tace_seg_linear_ks_rows(int(k))
        if R <= 0:
            raise ValueError(f"seg linear plan: no short-k task kernel for k = {k}")
        return R

    def _ks_tasks(self, Z, s_o, n, d, boff, mine, ranges, f_stride, b_stride):
        """Tasks of one output block (one contribution with k <= 128, or
        none): column chunk-major, so that the workgroups running at one time
        on an XCD share a chunk's weight columns in its L2."""
        out = []
        R = self._ks_rows(mine[0][2] if mine else 0)   # the task height for this k
        for cb in range(0, n, SEG_KS_CHUNK):
            ce = min(n, cb + SEG_KS_CHUNK)
            for (sp, a, b) in ranges:
                if b <= a:
                    continue
                for r0 in range(a * d, b * d, R):
                    rows = min(b * d - r0, R)
                    bo = -1 if boff is None else boff + (0 if sp is None else sp * b_stride)
                    if mine:
                        s_i, k, f_off = mine[0][1], mine[0][2], mine[0][6]
                        out.append((Z * s_o + r0 * n, rows, n, cb, ce, bo, Z * s_i + r0 * k, k,
                                    f_off + (0 if sp is None else sp * f_stride), 0))
                    else:
                        out.append((Z * s_o + r0 * n, rows, n, cb, ce, bo, 0, 0, 0, 0))
        return out


def _addend_ptr(addend: Optional[torch.Tensor], y: torch.Tensor):
    """Device pointer of the term added to every output (None: no term):
    y itself (y += ...) or a tensor of y's dtype and size apart from y."""
    if addend is None:
        return None
    if addend.dtype != y.dtype or addend.numel() != y.numel() or not addend.is_contiguous() \
            or addend.device != y.device:
        raise ValueError("seg linear: the addend must be a contiguous tensor of the output's dtype, size and device")
    if addend.data_ptr() != y.data_ptr():
        a0, a1 = addend.data_ptr(), addend.data_ptr() + addend.numel() * addend.element_size()
        y0, y1 = y.data_ptr(), y.data_ptr() + y.numel() * y.element_size()
        if a0 < y1 and y0 < a1:
            raise ValueError("seg linear: the addend overlaps the output without being it")
    return addend.data_ptr()


def seg_linear(x: torch.Tensor, y: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor], plan: SegLinearPlan,
               alpha: float, addend: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Runs ``plan`` (``tace_seg_linear``) from x into y (every element of y
    that a tile covers is overwritten, with ``addend`` added: y itself for
    y += ..., or a separate tensor); returns y."""
    dt = x.dtype
    for t, nm, n in ((x, "x", plan.x_numel), (y, "y", plan.y_numel), (w, "weight", plan.w_numel)):
        _req(t, nm, dt)
        if t.numel() != n:
            raise ValueError(f"seg linear: {nm} has {t.numel()} elements, the plan was built for {n}")
    if bias is not None:
        _req(bias, "bias", dt)
        if bias.numel() != plan.b_numel:
            raise ValueError("seg linear: bias size differs from the plan's")
    tok = _t0("seg_linear")
    N.check(N.lib().tace_seg_linear(N.dtype_code(dt), plan.tile[0], plan.tile[1], x.data_ptr(), y.data_ptr(),
                                    _addend_ptr(addend, y), w.data_ptr(),
                                    None if bias is None else bias.data_ptr(), plan.tiles.data_ptr(), plan.n_tiles,
                                    plan.contribs.data_ptr(), plan.scales.data_ptr(), float(alpha),
                                    N.stream_ptr(x.device)), "tace_seg_linear")
    _t1(tok, (plan.x_numel, plan.y_numel, plan.w_numel, plan.flops))
    return y


def bf16x3_split_blocks(w: torch.Tensor, blocks, scales, plane_stride: int, frag: bool = False) -> torch.Tensor:
    """``tace_bf16x3_split_blocks``: the three bf16 terms of scale x each
    weight block (table rows: src_off, cols, k, transpose, dst_off, layout),
    column-major runs of ceil8(k) into int16 planes [3 * plane_stride]
    (layout 0), or with ``frag`` in MFMA fragment order into one int16 buffer
    [plane_stride] (layout 1)."""
    _req(w, "weight", torch.float32)
    tab = np.asarray(blocks, dtype=np.int64).reshape(-1, 6)
    if len(tab):
        if (tab[:, 5] != (1 if frag else 0)).any():
            raise ValueError("bf16x3 split: every block must have the requested layout")
        if frag:
            size = 3 * ((tab[:, 1] + 15) // 16 * 16) * ((tab[:, 2] + 31) // 32 * 32)
        else:
            size = tab[:, 1] * ((tab[:, 2] + 7) // 8 * 8)
        if (tab[:, 0] + tab[:, 1] * tab[:, 2]).max() > w.numel():
            raise ValueError("bf16x3 split: source block out of range")
        if (tab[:, 4] + size).max() > plane_stride:
            raise ValueError("bf16x3 split: destination block out of range")
    planes = torch.zeros((1 if frag else 3) * plane_stride, dtype=torch.int16, device=w.device)
    tb = torch.from_numpy(np.ascontiguousarray(tab)).to(w.device)
    sc = torch.tensor(list(scales), dtype=torch.float64, device=w.device)
    for b0 in range(0, len(tab), 65535):
        b1 = min(len(tab), b0 + 65535)
        N.check(N.lib().tace_bf16x3_split_blocks(w.data_ptr(), tb[b0:b1].data_ptr(), sc[b0:b1].data_ptr(), b1 - b0,
                                                 planes.data_ptr(), plane_stride, N.stream_ptr(w.device)),
                "tace_bf16x3_split_blocks")
    return planes


def seg_linear_presplit(x: torch.Tensor, y: torch.Tensor, planes: Optional[torch.Tensor], plane_stride: int,
                        bias: Optional[torch.Tensor], plan: SegLinearPlan, alpha: float,
                        frag: Optional[torch.Tensor] = None, addend: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Runs a ``split_weights`` plan: its tiles with the weight planes of
    ``bf16x3_split_blocks`` (``tace_seg_linear_presplit``; planes may be None
    when the plan's tiles read the fragment-order weights instead,
    ``tace_seg_linear_presplit_frag``), and its short-k tasks
    (``tace_seg_linear_presplit_ks``) with the fragment-order weights
    ``frag``; ``addend`` as in ``seg_linear``; returns y."""
    if not plan.split_weights:
        raise ValueError("seg linear: the plan indexes flat weights, not pre-split planes")
    for t, nm, n in ((x, "x", plan.x_numel), (y, "y", plan.y_numel)):
        _req(t, nm, torch.float32)
        if t.numel() != n:
            raise ValueError(f"seg linear: {nm} has {t.numel()} elements, the plan was built for {n}")
    if (plan.n_ks or plan.tile_frag) and (frag is None or frag.dtype != torch.int16
                                          or frag.numel() < plan.frag_numel):
        raise ValueError("seg linear: the plan needs its fragment-order weights")
    if not plan.tile_frag and (planes is None or planes.dtype != torch.int16 or planes.numel() != 3 * plane_stride
                               or plane_stride < plan.w_numel):
        raise ValueError("seg linear: weight planes do not match the plan")
    if bias is not None:
        _req(bias, "bias", torch.float32)
        if bias.numel() != plan.b_numel:
            raise ValueError("seg linear: bias size differs from the plan's")
    tok = _t0("seg_linear")
    st = N.stream_ptr(x.device)
    b_ptr = None if bias is None else bias.data_ptr()
    a_ptr = _addend_ptr(addend, y)
    if plan.tile_frag and plan.splits > 1:
        pe = plan.n_tiles * plan.splits * 16384
        partials = torch.empty(pe, dtype=torch.float32, device=x.device)
        N.check(N.lib().tace_seg_linear_presplit_frag_split(x.data_ptr(), y.data_ptr(), a_ptr, frag.data_ptr(), b_ptr,
                                                            plan.tiles.data_ptr(), plan.n_tiles,
                                                            plan.contribs.data_ptr(), int(plan.tile_aligned),
                                                            plan.splits, partials.data_ptr(), pe, float(alpha), st),
                "tace_seg_linear_presplit_frag_split")
    elif plan.tile_frag:
        N.check(N.lib().tace_seg_linear_presplit_frag(x.data_ptr(), y.data_ptr(), a_ptr, frag.data_ptr(), b_ptr,
                                                      plan.tiles.data_ptr(), plan.n_tiles, plan.contribs.data_ptr(),
                                                      int(plan.tile_aligned), float(alpha), st),
                "tace_seg_linear_presplit_frag")
    else:
        N.check(N.lib().tace_seg_linear_presplit(x.data_ptr(), y.data_ptr(), a_ptr, planes.data_ptr(), plane_stride,
                                                 b_ptr,
                                                 plan.tiles.data_ptr(), plan.n_tiles, plan.contribs.data_ptr(),
                                                 float(alpha), st), "tace_seg_linear_presplit")
    if plan.n_ks:
        for R, n_t, tasks in plan.ks_groups:
            N.check(N.lib().tace_seg_linear_presplit_ks(x.data_ptr(), y.data_ptr(), a_ptr, frag.data_ptr(), b_ptr,
                                                        tasks.data_ptr(), n_t, R, float(alpha), st),
                    "tace_seg_linear_presplit_ks")
    _t1(tok, (plan.x_numel, plan.y_numel, plan.w_numel, plan.flops))
    return y


def edge_ace_paths(lmax: int) -> List[Tuple[int, int, int, bool]]:
    """(m3, m1, m2, is_sum) of the complex edge-ACE product in weight order."""
    out = []
    for m3 in range(lmax + 1):
        for m1 in range(lmax + 1):
            for m2 in range(m1 + 1):
                if m1 + m2 == m3:
                    out.append((m3, m1, m2, True))
                elif m1 - m2 == m3:
                    out.append((m3, m1, m2, False))
    return out


class _EdgeAce(torch.autograd.Function):
    @staticmethod
    def forward(ctx, lmax: int, A: int, *ys):
        outs = launch_edge_ace_fwd(list(ys), lmax, A)
        ctx.save_for_backward(*ys)
        ctx.lmax, ctx.A = lmax, A
        return tuple(outs)

    @staticmethod
    def backward(ctx, *gos):
        ys = ctx.saved_tensors
        lmax, A = ctx.lmax, ctx.A
        E = ys[0].shape[0]
        gos = [g.contiguous() if g is not None else torch.zeros(E if m == 0 else 2 * E, (lmax + 1) * A,
                                                                 dtype=ys[0].dtype, device=ys[0].device)
               for m, g in enumerate(gos)]
        return (None, None) + tuple(launch_edge_ace_bwd(list(ys), gos, lmax, A))


def tece_edge_ace(ys: Sequence[torch.Tensor], lmax: int, hidden: int) -> Tuple[torch.Tensor, ...]:
    """Gate + complex edge-ACE product on the stacked SO(2) GEMM outputs (block
    layouts of ``include/tace_hip.h``): returns the per-m blocks (o0 [E, n*A],
    o_m [2E, n*A])."""
    return _EdgeAce.apply(int(lmax), int(hidden), *[y.contiguous() for y in ys])


def to_grouped(x: torch.Tensor, ls: Sequence[int], C: int) -> torch.Tensor:
    """e3nn layout [N, C*D] -> group-major layout (same shape; test helper)."""
    Nn = x.shape[0]
    cols, off = [], 0
    groups = _runs(ls)
    parts = []
    for l, cnt in groups:
        d = 2 * l + 1
        blk = x[:, C * off:C * (off + cnt * d)].reshape(Nn, cnt, C, d)
        parts.append(blk.permute(0, 3, 1, 2).reshape(-1))
        off += cnt * d
    return torch.cat(parts).view(Nn, -1)


def from_grouped(x: torch.Tensor, ls: Sequence[int], C: int) -> torch.Tensor:
    """group-major layout -> e3nn layout (test helper)."""
    Nn = x.shape[0]
    flat = x.reshape(-1)
    cols, pos = [], 0
    for l, cnt in _runs(ls):
        d = 2 * l + 1
        n = Nn * d * cnt * C
        cols.append(flat[pos:pos + n].view(Nn, d, cnt, C).permute(0, 2, 3, 1).reshape(Nn, -1))
        pos += n
    return torch.cat(cols, dim=1)


def _runs(ls: Sequence[int]):
    out = []
    for l in ls:
        if out and out[-1][0] == l:
            out[-1][1] += 1
        else:
            out.append([l, 1])
    return [(l, c) for l, c in out]


# ------------------------------------------------------------ neighbours ----
def neighbour_list(positions: torch.Tensor, cell, pbc, cutoff: float):
    """GPU cell-list neighbour search (float64).

    Returns ``(rowptr int32 [N+1], src int32 [E], shifts int32 [E,3])`` with
    edges grouped by receiver: receiver of slot k is the n with
    rowptr[n] <= k < rowptr[n+1].  Edge vector = r[dst] - r[src] + S.cell."""
    _req(positions, "positions", torch.float64)
    n = positions.shape[0]
    dev = positions.device
    cell_np = np.ascontiguousarray(np.asarray(cell, dtype=np.float64).reshape(3, 3))
    pbc_np = np.ascontiguousarray(np.broadcast_to(np.asarray(pbc, dtype=np.int32), (3,)))
    L = N.lib()
    nbytes = L.tace_nl_workspace_bytes(n, cell_np.ctypes.data, pbc_np.ctypes.data, float(cutoff))
    if nbytes < 0:
        raise N.NativeError(L.tace_last_error().decode())
    ws = torch.empty(max(int(nbytes), 4), dtype=torch.uint8, device=dev)
    counts = torch.empty(n, dtype=torch.int32, device=dev)
    s = N.stream_ptr(dev)
    N.check(L.tace_nl_count(positions.data_ptr(), n, cell_np.ctypes.data, pbc_np.ctypes.data, float(cutoff),
                            ws.data_ptr(), int(nbytes), counts.data_ptr(), s), "tace_nl_count")
    rowptr = torch.empty(n + 1, dtype=torch.int32, device=dev)
    N.check(L.tace_scan_i32(counts.data_ptr(), n, rowptr.data_ptr(), s), "tace_scan_i32")
    E = int(rowptr[-1].item())
    src = torch.empty(E, dtype=torch.int32, device=dev)
    shifts = torch.empty(E, 3, dtype=torch.int32, device=dev)
    if E > 0:
        N.check(L.tace_nl_fill(positions.data_ptr(), n, cell_np.ctypes.data, pbc_np.ctypes.data, float(cutoff),
                               ws.data_ptr(), rowptr.data_ptr(), src.data_ptr(), shifts.data_ptr(), s),
                "tace_nl_fill")
    return rowptr, src, shifts


def neighbour_list_batch(positions: torch.Tensor, sizes: Sequence[int], cells, pbcs, cutoff: float,
                         mode: int = 0):
    """The cell-list neighbour search for a batch of structures in one pass
    (``tace_nl_batch_*``): one launch per phase for all structures, one host
    synchronisation for the total edge count.  ``positions`` [sum(sizes), 3]
    float64 (structures back to back); ``mode`` 0 automatic, 1 a thread per
    receiver, 2 a wavefront per receiver (same result).

    Returns ``(rowptr int32 [N+1], src int32 [E], shifts int32 [E,3])`` over
    the batch, node ids batch-global: receiver n's edges are slots
    rowptr[n]..rowptr[n+1], each structure's in the order ``neighbour_list``
    gives for it alone."""
    _req(positions, "positions", torch.float64)
    dev = positions.device
    L = N.lib()
    ns = len(sizes)
    n_tot = int(sum(sizes))
    if positions.shape[0] != n_tot:
        raise ValueError(f"positions has {positions.shape[0]} rows, sizes sum to {n_tot}")
    sizes_np = np.ascontiguousarray(np.asarray(sizes, dtype=np.int64))
    cells_np = np.ascontiguousarray(np.stack([np.asarray(c, dtype=np.float64).reshape(3, 3) for c in cells]))
    pbcs_np = np.ascontiguousarray(np.stack([np.broadcast_to(np.asarray(p, dtype=np.int32), (3,)) for p in pbcs]))
    na, nb = ctypes.c_int64(0), ctypes.c_int64(0)
    need = L.tace_nl_batch_plan(ns, sizes_np.ctypes.data, cells_np.ctypes.data, pbcs_np.ctypes.data, float(cutoff),
                                None, 0, ctypes.byref(na), ctypes.byref(nb))
    if need < 0:
        raise N.NativeError(L.tace_last_error().decode())
    host = np.zeros(need, dtype=np.uint8)
    if L.tace_nl_batch_plan(ns, sizes_np.ctypes.data, cells_np.ctypes.data, pbcs_np.ctypes.data, float(cutoff),
                            host.ctypes.data, need, ctypes.byref(na), ctypes.byref(nb)) < 0:
        raise N.NativeError(L.tace_last_error().decode())
    plan = torch.from_numpy(host).to(dev)
    wsb = L.tace_nl_batch_workspace_bytes(na.value, nb.value)
    if wsb < 0:
        raise N.NativeError(L.tace_last_error().decode())
    ws = torch.empty(max(wsb, 4), dtype=torch.uint8, device=dev)
    counts = torch.empty(max(n_tot, 1), dtype=torch.int32, device=dev)
    st = N.stream_ptr(dev)
    N.check(L.tace_nl_batch_count(positions.data_ptr(), n_tot, ns, plan.data_ptr(), nb.value, ws.data_ptr(), wsb,
                                  mode, counts.data_ptr(), st), "tace_nl_batch_count")
    rowptr = torch.empty(n_tot + 1, dtype=torch.int32, device=dev)
    N.check(L.tace_scan_i32(counts.data_ptr(), n_tot, rowptr.data_ptr(), st), "tace_scan_i32")
    E = int(rowptr[-1].item())
    src = torch.empty(E, dtype=torch.int32, device=dev)
    shifts = torch.empty(E, 3, dtype=torch.int32, device=dev)
    if E > 0:
        N.check(L.tace_nl_batch_fill(positions.data_ptr(), n_tot, ns, plan.data_ptr(), nb.value, ws.data_ptr(), wsb,
                                     mode, rowptr.data_ptr(), src.data_ptr(), shifts.data_ptr(), st),
                "tace_nl_batch_fill")
    return rowptr, src, shifts

