"""TECE radial-rotary edge convolution on MI355X.

``TeceConvolution`` has the parameters (names, shapes, init) of the
reference's ``OAM20260705Convolution`` with the flags of
``OAM20260705Interaction`` (``tace/models/_e3nn/archive/oam_2026_07_05.py:547-823``,
``tace/models/_e3nn/inter.py:440-519``: SO(2) linears of type "w1",
temperature, edge-ACE, graph softmax, radial phase, gate_m0).  The edge
frames, the gather + rotation into the edge frame with the radial weighting,
the rotary QK score, the graph softmax, the gate + complex edge-ACE product
and the attention-weighted inverse rotation + receiver sum run on the HIP
kernels of ``csrc/tece.hip``; the SO(2) linears are dense GEMMs (hipBLASLt
through torch), those sharing an input stacked into one GEMM per m.  Node
features come and go in the model's group-major, species-sorted layout.
"""

from __future__ import annotations

import math
from typing import List, Optional

import torch

from . import ops

class _MixedLinear(torch.autograd.Function):
    """y = x W^T (+ b) with x and W rounded to bfloat16 and fp32 accumulation
    and output (hipBLASLt); the input gradient likewise.  W is a constant."""

    @staticmethod
    def forward(ctx, x, wt, b):
        y = torch.mm(x.to(torch.bfloat16), wt, out_dtype=torch.float32)
        if b is not None:
            y += b
        ctx.save_for_backward(wt)
        return y

    @staticmethod
    def backward(ctx, g):
        (wt,) = ctx.saved_tensors
        return torch.mm(g.to(torch.bfloat16), wt.t(), out_dtype=torch.float32), None, None


def mix_linear(x, W, b, mixing):
    """``F.linear(x, W, b)`` for 2-D x; ``mixing`` = torch.bfloat16 runs the
    product on bf16 MFMA with fp32 accumulation (the "bf16 channel mixing"
    option of the TECE configuration), None in the input's precision."""
    if mixing is None or x.dtype != torch.float32:
        return torch.nn.functional.linear(x, W, b)
    return _MixedLinear.apply(x, W.detach().t().to(mixing).contiguous(), None if b is None else b.detach())


class torchLinear(torch.nn.Module):
    """``torchLinear`` (``tace/models/linear.py:210-244``): y = x (W/sqrt(in))^T + b,
    W ~ N(0,1) [out, in], b zeros."""

    def __init__(self, i: int, o: int, bias: bool = True):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.randn(o, i))
        self.bias = torch.nn.Parameter(torch.zeros(o)) if bias else None
        self.alpha = 1.0 / math.sqrt(i)

    def forward(self, x):
        return torch.nn.functional.linear(x, self.weight * self.alpha, self.bias)


class uvSO2MLinear(torch.nn.Module):
    """Weight type "w1" of ``uvSO2MLinear`` (``oam_2026_07_05.py:47-136``): one
    real map for the +m and the -m components."""

    def __init__(self, cin: int, cout: int, nin: int, nout: int):
        super().__init__()
        self.fc = torchLinear(nin * cin, nout * cout, bias=False)


class uvSO2Linear(torch.nn.Module):
    """``uvSO2Linear`` type "w1" (``oam_2026_07_05.py:138-247``) on [E, rows, C]
    features in the m layout; per m one GEMM over (component, channel)."""

    def __init__(self, mmax: int, lmax: int, cin: int, cout: int, nin: Optional[List[int]] = None,
                 nout: Optional[List[int]] = None):
        super().__init__()
        self.mmax, self.lmax, self.cin, self.cout = mmax, lmax, cin, cout
        self.nin = nin or [lmax + 1 - m for m in range(mmax + 1)]
        self.nout = nout or [lmax + 1 - m for m in range(mmax + 1)]
        self.m0_rlinear = torchLinear(cin * self.nin[0], cout * self.nout[0], bias=True)
        self.ms_clinear = torch.nn.ModuleList(
            uvSO2MLinear(cin, cout, self.nin[m], self.nout[m]) for m in range(1, mmax + 1))

    def forward(self, x, mixing=None):
        # every block is one 2-D GEMM over (edge[, +-m]) rows: the row slices
        # are made contiguous first (a strided 3-D operand would make torch
        # fall back to one tiny GEMM per edge)
        E = x.shape[0]
        f = self.m0_rlinear
        outs = [mix_linear(x[:, :self.nin[0]].reshape(E, -1), f.weight * f.alpha, f.bias, mixing)
                .view(E, self.nout[0], self.cout)]
        off = self.nin[0]
        for m in range(1, self.mmax + 1):
            n = self.nin[m]
            xm = x[:, off:off + 2 * n].contiguous().view(E * 2, n * self.cin)
            off += 2 * n
            fc = self.ms_clinear[m - 1].fc
            outs.append(mix_linear(xm, fc.weight * fc.alpha, None, mixing).view(E, 2 * self.nout[m], self.cout))
        return torch.cat(outs, dim=1)

    def blocks(self, xb, mixing=None):
        """The same map on the SO(2) block layout (``ops.so2_block_shapes``):
        one GEMM per block, no copies."""
        f = self.m0_rlinear
        out = [mix_linear(xb[0], f.weight * f.alpha, f.bias, mixing)]
        for m in range(1, self.mmax + 1):
            fc = self.ms_clinear[m - 1].fc
            out.append(mix_linear(xb[m], fc.weight * fc.alpha, None, mixing))
        return out


class TeceConvolution(torch.nn.Module):
    """``OAM20260705Convolution`` (see the module docstring)."""

    def __init__(self, mmax: int, lmax: int, C: int, num_head: int, edge_ace_hidden: int, num_radial: int):
        super().__init__()
        if mmax != lmax:
            raise NotImplementedError("TECE on the MI355X path needs mmax == lmax (the config-5 setting)")
        if C % num_head:
            raise ValueError("channels must be divisible by num_head")
        self.mmax, self.lmax, self.C, self.H, self.A = mmax, lmax, C, num_head, edge_ace_hidden
        # precision of the SO(2) channel mixing GEMMs: None = the features'
        # own, torch.bfloat16 = bf16 operands with fp32 accumulation
        self.mixing = None
        self.Ch = C // num_head
        n = lmax + 1
        A = edge_ace_hidden
        self.K = n * n
        self.num_components = sum(n - m for m in range(mmax + 1))
        self.weight_numel = self.num_components * C * 2
        self.num_gates = n * (mmax + 1)
        self.rows_full = n + 2 * n * mmax
        full = [n] * (mmax + 1)
        self.linear_up = uvSO2Linear(mmax, lmax, 2 * C, A, nout=[self.num_gates + n] + [n] * mmax)
        self.linear_glu = uvSO2Linear(mmax, lmax, 2 * C, A, nout=full)
        # one edge-ACE weight per path, row and hidden channel (uuuSO2TensorProduct)
        self.ece_weight_numel = len(ops.edge_ace_paths(lmax)) * n * A
        self.linear_coefs = uvSO2Linear(0, lmax, 2 * C, 1, nout=[self.ece_weight_numel])
        self.linear_down = uvSO2Linear(mmax, lmax, A, C, nin=full)
        self.query_proj = uvSO2Linear(mmax, lmax, C, C)
        self.key_proj = uvSO2Linear(mmax, lmax, C, C)
        self.radial_proj = torchLinear(num_radial, 2 * num_head)
        torch.nn.init.zeros_(self.radial_proj.weight)
        torch.nn.init.zeros_(self.radial_proj.bias)
        self.attention_scale = 1.0 / math.sqrt(self.Ch * self.rows_full)
        self.tmin, self.tmax = 0.25, 4.0
        self.temperature_logit = torch.nn.Parameter(
            torch.full((num_head,), math.log((1.0 - self.tmin) / (self.tmax - 1.0))))

    def _shared_input_gemms(self, mw):
        """linear_coefs, linear_glu and linear_up of the radially weighted
        messages (block layout, 2C channels): one GEMM per m block with the
        three weights stacked.  Returns y0 [E, coef | glu | up] and, per m > 0,
        y_m [2E, glu | up] (the edge-ACE kernel's input layout)."""
        lc, lg, lu = self.linear_coefs, self.linear_glu, self.linear_up
        f0 = [lc.m0_rlinear, lg.m0_rlinear, lu.m0_rlinear]
        W0 = torch.cat([f.weight * f.alpha for f in f0])
        b0 = torch.cat([f.bias for f in f0])
        ys = [mix_linear(mw[0], W0, b0, self.mixing)]
        for mm in range(1, self.mmax + 1):
            fg, fu = lg.ms_clinear[mm - 1].fc, lu.ms_clinear[mm - 1].fc
            ys.append(mix_linear(mw[mm], torch.cat([fg.weight * fg.alpha, fu.weight * fu.alpha]), None, self.mixing))
        return ys

    def node_components(self, x_gm):
        """Group-major C x (0..lmax) node features -> [rows, (L+1)^2, C] (l layout)."""
        Nn, C = x_gm.shape[0], self.C
        return torch.cat([x_gm.view(-1)[Nn * C * l * l:Nn * C * (l + 1) ** 2].view(Nn, 2 * l + 1, C)
                          for l in range(self.lmax + 1)], dim=1)

    def edges(self, x_lc, w, rows_src, rows_dst, plan: ops.EdgePlan, out_map, dst_out, wigner, R):
        """Messages of the edges of ``plan`` summed per receiver.  x_lc: node
        features [rows, K, C]; rows_src / rows_dst (int64): feature rows of each
        edge's sender / receiver; ``plan``: receiver CSR of these edges;
        ``out_map`` (int32 or None) / ``dst_out``: output row of each receiver /
        of each edge's receiver.  Returns [plan.n_nodes, K*C] group-major."""
        ms, md, mw = ops.edge_rotate_in(x_lc, wigner, rows_src, rows_dst, self.lmax, w)
        key = self.key_proj.blocks(ms, self.mixing)
        query = self.query_proj.blocks(md, self.mixing)
        rp = self.radial_proj(R)
        T = self.tmin + (self.tmax - self.tmin) * torch.sigmoid(self.temperature_logit)
        score = ops.tece_score(query, key, rp, (T * self.attention_scale).detach(), self.lmax, self.H)
        alpha = ops.graph_softmax(score, plan)
        o = ops.tece_edge_ace(self._shared_input_gemms(mw), self.lmax, self.A)
        m = self.linear_down.blocks(o, self.mixing)
        return ops.tece_rotate_out(m, alpha, wigner, plan, out_map, dst_out, self.lmax, self.H)

    def forward(self, x_gm, w, plan: ops.EdgePlan, node_map, src, dst, wigner, R):
        """x_gm: node features, group-major C x (0..lmax) in feature-row order;
        w: radial weights [E, weight_numel]; node_map[n] = feature row of node
        n; src/dst: edge endpoints (node ids); wigner [E, K, K] from
        ``ops.edge_wigner``; R: radial basis [E, num_radial].  Returns the
        receiver sums, group-major, in feature-row order."""
        rows = node_map.long()
        return self.edges(self.node_components(x_gm), w, rows[src], rows[dst], plan, node_map, dst, wigner, R)


def receiver_chunks(plan: ops.EdgePlan, max_edges: int):
    """Receiver ranges [n0, n1) whose in-edges (contiguous in a receiver-grouped
    edge list) number at most ``max_edges`` (or one receiver, if it alone has
    more), with their edge ranges [e0, e1)."""
    rp = plan.rowptr.cpu().tolist()
    out, n0, N = [], 0, plan.n_nodes
    while n0 < N:
        n1 = n0 + 1
        while n1 < N and rp[n1 + 1] - rp[n0] <= max_edges:
            n1 += 1
        out.append((n0, n1, rp[n0], rp[n1]))
        n0 = n1
    return out


def sub_plan(plan: ops.EdgePlan, n0: int, n1: int, e0: int, e1: int) -> ops.EdgePlan:
    """Receiver CSR of receivers n0..n1-1 and their edges e0..e1-1 (receiver-grouped edges)."""
    return ops.EdgePlan(n1 - n0, e1 - e0, (plan.rowptr[n0:n1 + 1] - e0).contiguous(),
                        plan.src[e0:e1].contiguous(), None)
