"""TECE radial-rotary edge convolution on MI355X.

``TeceConvolution`` has the parameters (names, shapes, init) of the
reference's ``OAM20260705Convolution`` with the flags of
``OAM20260705Interaction`` (``tace/models/_e3nn/archive/oam_2026_07_05.py:547-823``,
``tace/models/_e3nn/inter.py:440-519``: SO(2) linears of type "w1",
temperature, edge-ACE, graph softmax, radial phase, gate_m0).  The edge
frames, the rotary QK score, the graph softmax and the attention-weighted
inverse rotation + receiver sum run on the HIP kernels of ``csrc/tece.hip``;
the SO(2) linears are dense GEMMs (hipBLASLt through torch).  Node features
come and go in the model's group-major, species-sorted layout.
"""

from __future__ import annotations

import math
from typing import List, Optional

import torch

from . import ops

SIGMOID_CST = 1.8467055342154763  # ScaledSigmoid (tace/models/mlp.py:40-46)


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

    def forward(self, x):
        E = x.shape[0]
        outs = [self.m0_rlinear(x[:, :self.nin[0]].reshape(E, -1)).view(E, self.nout[0], self.cout)]
        off = self.nin[0]
        for m in range(1, self.mmax + 1):
            n = self.nin[m]
            y = self.ms_clinear[m - 1].fc(x[:, off:off + 2 * n].reshape(E, 2, n * self.cin))
            off += 2 * n
            outs.append(y.view(E, 2 * self.nout[m], self.cout))
        return torch.cat(outs, dim=1)


def _expand(mmax: int, lmax: int, full: bool) -> torch.Tensor:
    idx, off = [], 0
    for m in range(mmax + 1):
        n = lmax + 1 if full else lmax + 1 - m
        r = list(range(off, off + n))
        idx += r + (r if m > 0 else [])
        off += n
    return torch.tensor(idx, dtype=torch.long)


class ComplexProductBasis(torch.nn.Module):
    """SO(2) edge-ACE complex product with per-edge weights, m1 >= m2
    (``uuuSO2TensorProduct``, ``oam_2026_07_05.py:312-544``); no parameters."""

    def __init__(self, mmax: int, lmax: int, C: int):
        super().__init__()
        self.mmax, self.n, self.C = mmax, lmax + 1, C
        self.paths = []
        for m3 in range(mmax + 1):
            ps = []
            for m1 in range(mmax + 1):
                for m2 in range(mmax + 1):
                    if m1 >= m2:
                        if m1 + m2 == m3:
                            ps.append((m1, m2, "sum"))
                        elif abs(m1 - m2) == m3:
                            ps.append((m1, m2, "diff"))
            self.paths.append(ps)
        self.weight_numel = sum(len(p) for p in self.paths) * self.n * C

    def forward(self, x, y, ws):
        E, n, C = x.shape[0], self.n, self.C
        xs = [x[:, :n]] + [x[:, n + 2 * n * (m - 1):n + 2 * n * m].view(E, 2, n, C) for m in range(1, self.mmax + 1)]
        ys = [y[:, :n]] + [y[:, n + 2 * n * (m - 1):n + 2 * n * m].view(E, 2, n, C) for m in range(1, self.mmax + 1)]
        woff, outs = 0, []
        for m3, ps in enumerate(self.paths):
            re = im = None
            for (m1, m2, mode) in ps:
                w = ws[:, woff:woff + n * C].view(E, n, C)
                woff += n * C
                a, b = xs[m1], ys[m2]
                if m1 == 0 and m2 == 0:
                    zr, zi = a * b, None
                elif m2 == 0:
                    zr, zi = a[:, 0] * b, a[:, 1] * b
                else:
                    ar, ai, br, bi = a[:, 0], a[:, 1], b[:, 0], b[:, 1]
                    if mode == "sum":
                        zr, zi = ar * br - ai * bi, ar * bi + ai * br
                    else:
                        zr, zi = ar * br + ai * bi, ai * br - ar * bi
                re = zr * w if re is None else re + zr * w
                if m3 > 0:
                    im = zi * w if im is None else im + zi * w
            s = 1.0 / math.sqrt(len(ps))
            outs.append(re * s)
            if m3 > 0:
                outs.append(im * s)
        return torch.cat(outs, dim=1)


class TeceConvolution(torch.nn.Module):
    """``OAM20260705Convolution`` (see the module docstring)."""

    def __init__(self, mmax: int, lmax: int, C: int, num_head: int, edge_ace_hidden: int, num_radial: int):
        super().__init__()
        if mmax != lmax:
            raise NotImplementedError("TECE on the MI355X path needs mmax == lmax (the config-5 setting)")
        if C % num_head:
            raise ValueError("channels must be divisible by num_head")
        self.mmax, self.lmax, self.C, self.H = mmax, lmax, C, num_head
        self.Ch = C // num_head
        n = lmax + 1
        A = edge_ace_hidden
        self.K = n * n
        self.num_components = sum(n - m for m in range(mmax + 1))
        self.weight_numel = self.num_components * C * 2
        self.register_buffer("expand_index", _expand(mmax, lmax, False), persistent=False)
        self.register_buffer("gate_index", _expand(mmax, lmax, True), persistent=False)
        self.num_gates = n * (mmax + 1)
        self.rows_full = n + 2 * n * mmax
        full = [n] * (mmax + 1)
        self.linear_up = uvSO2Linear(mmax, lmax, 2 * C, A, nout=[self.num_gates + n] + [n] * mmax)
        self.linear_glu = uvSO2Linear(mmax, lmax, 2 * C, A, nout=full)
        self.ece = ComplexProductBasis(mmax, lmax, A)
        self.linear_coefs = uvSO2Linear(0, lmax, 2 * C, 1, nout=[self.ece.weight_numel])
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
        C = self.C
        E = w.shape[0]
        m = torch.bmm(wigner, torch.cat((x_lc.index_select(0, rows_src), x_lc.index_select(0, rows_dst)), dim=-1))
        key = self.key_proj(m[:, :, :C])
        query = self.query_proj(m[:, :, C:])
        rp = self.radial_proj(R)
        T = self.tmin + (self.tmax - self.tmin) * torch.sigmoid(self.temperature_logit)
        score = ops.tece_score(query, key, rp, (T * self.attention_scale).detach(), self.lmax, self.H)
        alpha = ops.graph_softmax(score, plan)
        m = w.view(E, self.num_components, 2 * C).index_select(1, self.expand_index) * m
        coefs = torch.sigmoid(self.linear_coefs(m).squeeze(-1)) * SIGMOID_CST
        m2 = self.linear_glu(m)
        mu = self.linear_up(m)
        gate, m = mu[:, :self.num_gates], mu[:, self.num_gates:self.num_gates + self.rows_full]
        g = (torch.sigmoid(gate) * SIGMOID_CST).index_select(1, self.gate_index)
        m = m + g * m + self.ece(m, m2, coefs)
        m = self.linear_down(m)
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
