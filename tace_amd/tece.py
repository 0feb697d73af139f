"""TECE radial-rotary edge convolution on MI355X.

``TeceConvolution`` has the parameters (names, shapes, init) of the
reference's ``OAM20260705Convolution`` with the flags of
``OAM20260705Interaction`` (``tace/models/_e3nn/archive/oam_2026_07_05.py:547-823``,
``tace/models/_e3nn/inter.py:440-519``: SO(2) linears of type "w1",
temperature, edge-ACE, graph softmax, radial phase, gate_m0).  The edge
frames, the gather + rotation into the edge frame with the radial weighting,
the rotary QK score, the graph softmax, the gate + complex edge-ACE product
and the attention-weighted inverse rotation + receiver sum run on the HIP
kernels of ``csrc/tece_*.hip``; the SO(2) linears are GEMMs on the bf16 MFMA
kernels of ``csrc/so2_gemm.hip`` under bf16 channel mixing (torch GEMMs in
float32 / float64 otherwise), those sharing an input stacked into one GEMM per
m.  Node
features come and go in the model's group-major, species-sorted layout.
"""

from __future__ import annotations

import math
from typing import List, Optional

import torch

from . import ops

_SIGMOID_CST = 1.8467055342154763   # e3nn normalize2mom(sigmoid) (tace/models/mlp.py:43)

# frozen parameters run the convolution on the fused operator (_TeceFused);
# False keeps the per-operator autograd path (the reference for its tests)
FUSED = True
# training (twice differentiable): rotate-in and rotate-out on their kernels
# (_forward_train); False runs the whole convolution as torch operations
TRAIN_ON_KERNELS = True

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

    # ---- the convolution as torch operations (training: twice differentiable) --
    def _expand(self, full: bool) -> torch.Tensor:
        """Row -> component map of the radial weights (full=False, one per (m,
        l), shared by +m and -m rows) and of the gates (full=True, lmax+1 per m)
        (``so2_expand_index``, ``SO2Gate``)."""
        idx, off, n = [], 0, self.lmax + 1
        for m in range(self.mmax + 1):
            k = n if full else n - m
            r = list(range(off, off + k))
            idx += r + (r if m > 0 else [])
            off += k
        return torch.tensor(idx, dtype=torch.long)

    def _edge_ace_autograd(self, u, v, coefs):
        """u + g u + complex edge-ACE product (``oam_2026_07_05.py:782-790``,
        ``uuuSO2TensorProduct`` 312-516) on [E, rows, A] m-layout features
        (m = 0: n real rows; m > 0: n rows of the +m, then n of the -m part),
        per path weights ``coefs`` [E, P n A] in ``ops.edge_ace_paths`` order;
        each output m scaled by 1/sqrt(its number of paths)."""
        E, n, A = u.shape[0], self.lmax + 1, self.A

        def split(x):
            return [x[:, :n]] + [x[:, n + 2 * n * (m - 1):n + 2 * n * m].reshape(E, 2, n, A)
                                 for m in range(1, self.mmax + 1)]
        us, vs = split(u), split(v)
        by_m3 = {}
        for j, (m3, m1, m2, is_sum) in enumerate(ops.edge_ace_paths(self.lmax)):
            by_m3.setdefault(m3, []).append((j, m1, m2, is_sum))
        outs = []
        for m3 in range(self.mmax + 1):
            ps = by_m3[m3]
            re, im = 0.0, 0.0
            for (j, m1, m2, is_sum) in ps:
                w = coefs[:, j * n * A:(j + 1) * n * A].reshape(E, n, A)
                a, b = us[m1], vs[m2]
                if m1 == 0 and m2 == 0:
                    zr, zi = a * b, None
                elif m2 == 0:
                    zr, zi = a[:, 0] * b, a[:, 1] * b
                elif m1 == 0:
                    zr, zi = a * b[:, 0], a * b[:, 1]
                elif is_sum:
                    zr, zi = a[:, 0] * b[:, 0] - a[:, 1] * b[:, 1], a[:, 0] * b[:, 1] + a[:, 1] * b[:, 0]
                else:
                    zr, zi = a[:, 0] * b[:, 0] + a[:, 1] * b[:, 1], a[:, 1] * b[:, 0] - a[:, 0] * b[:, 1]
                re = re + zr * w
                if m3 > 0:
                    im = im + zi * w
            sc = 1.0 / math.sqrt(len(ps))
            outs.append(re * sc)
            if m3 > 0:
                outs.append(im * sc)
        return torch.cat(outs, dim=1)

    def _score_autograd(self, q, k, R):
        """Radial-rotary complex QK score [E, H] (``oam_2026_07_05.py:699-754``)
        on [E, K, C] m-layout query / key; the temperature is differentiated."""
        E, H, Ch, n = q.shape[0], self.H, self.Ch, self.lmax + 1
        rp = self.radial_proj(R)
        bias, phase = rp[:, :H], math.pi * torch.tanh(rp[:, H:])
        s = (q[:, :n].reshape(E, n, H, Ch) * k[:, :n].reshape(E, n, H, Ch)).sum(dim=(1, 3))
        off = n
        for m in range(1, self.mmax + 1):
            nm = n - m
            qm = q[:, off:off + 2 * nm].reshape(E, 2, nm, H, Ch)
            km = k[:, off:off + 2 * nm].reshape(E, 2, nm, H, Ch)
            off += 2 * nm
            c, sn = torch.cos(m * phase).view(E, 1, H, 1), torch.sin(m * phase).view(E, 1, H, 1)
            s = s + (qm[:, 0] * (c * km[:, 0] - sn * km[:, 1]) + qm[:, 1] * (sn * km[:, 0] + c * km[:, 1])).sum(
                dim=(1, 3))
        T = self.tmin + (self.tmax - self.tmin) * torch.sigmoid(self.temperature_logit)
        return s * (self.attention_scale * T) + bias

    def _forward_autograd(self, x_gm, w, node_map, src, dst, wigner, R):
        """The whole convolution as torch operations (the per-edge kernels'
        arithmetic; ``oam_2026_07_05.py:756-823``): what training with a force
        loss differentiates twice.  Same inputs and output as ``forward``."""
        Nn, E, C, K = x_gm.shape[0], w.shape[0], self.C, self.K
        x_lc = self.node_components(x_gm)
        if node_map is None:   # features in node order
            rs, rd = src, dst
        else:
            rows = node_map.long()
            rs, rd = rows[src], rows[dst]
        m = torch.bmm(wigner, torch.cat((x_lc[rs], x_lc[rd]), dim=-1))
        key, query = self.key_proj(m[:, :, :C]), self.query_proj(m[:, :, C:])
        score = self._score_autograd(query, key, R)
        dev = w.device
        m = w.view(E, self.num_components, 2 * C).index_select(1, self._expand(False).to(dev)) * m
        coefs = torch.sigmoid(self.linear_coefs(m).squeeze(-1)) * _SIGMOID_CST
        v = self.linear_glu(m)
        u = self.linear_up(m)
        gate, u = u[:, :self.num_gates], u[:, self.num_gates:self.num_gates + self.rows_full]
        g = (torch.sigmoid(gate) * _SIGMOID_CST).index_select(1, self._expand(True).to(dev))
        m = self.linear_down(u + g * u + self._edge_ace_autograd(u, v, coefs))
        # graph softmax over each receiver's in-edges (softmax.py:100-112):
        # exp(s - max) / (sum exp(s - max) + 1e-16), the max not differentiated
        H = self.H
        mx = torch.full((Nn, H), -math.inf, dtype=score.dtype, device=dev).scatter_reduce(
            0, rd.view(-1, 1).expand(-1, H), score.detach(), reduce="amax", include_self=True)
        ex = torch.exp(score - mx[rd])
        alpha = ex / (torch.zeros(Nn, H, dtype=score.dtype, device=dev).index_add(0, rd, ex) + 1e-16)[rd]
        m = (m.view(E, K, H, self.Ch) * alpha.view(E, 1, H, 1)).view(E, K, C)
        m = torch.bmm(wigner.transpose(1, 2), m)
        out = torch.zeros(Nn, K, C, dtype=m.dtype, device=dev).index_add(0, rd, m)
        # [rows, K, C] (l layout) -> group-major C x (0..lmax)
        return torch.cat([out[:, l * l:(l + 1) ** 2].reshape(-1) for l in range(self.lmax + 1)]).view(Nn, K * C)

    def _forward_train(self, x_gm, w, plan: ops.EdgePlan, node_map, src, dst, wigner, R):
        """Training (twice differentiable): the rotate-in and the rotate-out
        (gathers, rotations, radial weighting, attention weighting and
        receiver sums) on their HIP kernels through operators whose backward is
        differentiable again; score, graph softmax, gate, edge-ACE and the SO(2)
        linears as torch operations (``_forward_autograd``'s)."""
        Nn, E, C = x_gm.shape[0], w.shape[0], self.C
        L, H, n = self.lmax, self.H, self.lmax + 1
        rows = node_map.long() if node_map is not None else None
        rs, rd = (src, dst) if rows is None else (rows[src], rows[dst])
        ms, md, mw = ops.edge_rotate_in_twice(self.node_components(x_gm), wigner, rs, rd, L, w)
        key = ops.so2_from_blocks(self.key_proj.blocks(ms, self.mixing), L)
        query = ops.so2_from_blocks(self.query_proj.blocks(md, self.mixing), L)
        score = self._score_autograd(query, key, R)
        m = ops.so2_from_blocks(mw, L)
        coefs = torch.sigmoid(self.linear_coefs(m).squeeze(-1)) * _SIGMOID_CST
        v = self.linear_glu(m)
        u = self.linear_up(m)
        gate, u = u[:, :self.num_gates], u[:, self.num_gates:self.num_gates + self.rows_full]
        g = (torch.sigmoid(gate) * _SIGMOID_CST).index_select(1, self._expand(True).to(w.device))
        m = self.linear_down(u + g * u + self._edge_ace_autograd(u, v, coefs))
        # graph softmax over each receiver's in-edges (softmax.py:100-112)
        mx = torch.full((Nn, H), -math.inf, dtype=score.dtype, device=w.device).scatter_reduce(
            0, rd.view(-1, 1).expand(-1, H), score.detach(), reduce="amax", include_self=True)
        ex = torch.exp(score - mx[rd])
        alpha = ex / (torch.zeros(Nn, H, dtype=score.dtype, device=w.device).index_add(0, rd, ex) + 1e-16)[rd]
        return ops.tece_rotate_out_twice(ops.so2_to_blocks(m, L), alpha, wigner, plan, node_map, dst, L, H)

    def _forward_library(self, x_gm, w, plan, src, dst, wigner, R):
        """Export mode: the kernels as ``tace_amd::`` operators (opaque nodes
        of the traced program, each with its registered backward), features in
        node order, edges in any order (``plan``: ``ops.TracedEdges``)."""
        from . import library
        Nn, L, H, n = x_gm.shape[0], self.lmax, self.H, self.lmax + 1
        rowptr, eid = library.receiver_csr(plan.edge_index, Nn)
        blocks = library.tece_rotate_in(self.node_components(x_gm), wigner, src, dst, w, L)
        ms, md, mw = blocks[:n], blocks[n:2 * n], blocks[2 * n:]
        key = self.key_proj.blocks(ms, self.mixing)
        query = self.query_proj.blocks(md, self.mixing)
        T = self.tmin + (self.tmax - self.tmin) * torch.sigmoid(self.temperature_logit)
        score = library.tece_score(query, key, self.radial_proj(R), (T * self.attention_scale).detach(), L, H)
        alpha = library.tece_softmax(score, rowptr, eid)
        o = library.tece_edge_ace(self._shared_input_gemms(mw), L, self.A)
        m = self.linear_down.blocks(o, self.mixing)
        return library.tece_rotate_out(m, alpha, wigner, rowptr, eid, dst, L, H)

    def forward(self, x_gm, w, plan: ops.EdgePlan, node_map, src, dst, wigner, R):
        """x_gm: node features, group-major C x (0..lmax) in feature-row order;
        w: radial weights [E, weight_numel]; node_map[n] = feature row of node
        n; src/dst: edge endpoints (node ids); wigner [E, K, K] from
        ``ops.edge_wigner``; R: radial basis [E, num_radial].  Returns the
        receiver sums, group-major, in feature-row order."""
        if ops.MODE.export:
            return self._forward_library(x_gm, w, plan, src, dst, wigner, R)
        if ops.MODE.double:
            if TRAIN_ON_KERNELS and isinstance(plan, ops.EdgePlan):
                return self._forward_train(x_gm, w, plan, node_map, src, dst, wigner, R)
            return self._forward_autograd(x_gm, w, node_map, src, dst, wigner, R)
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


# ----------------------------------------------------------- fused operator --
# bf16 channel mixing: SO(2) GEMMs on tace_so2_gemm_bf16 / _kt (bias in the
# epilogue) where they measured faster than the library GEMM on fe101k
# (_so2_route); False: torch.mm / addmm (addmm copies the bias into the output
# and accumulates onto it); SO2_GEMM_ALL: every shape on the hand-written ones
SO2_GEMM = True
SO2_GEMM_ALL = False


# kernel per SO(2) GEMM shape (k, n, biased) under bf16 mixing: "kt" =
# tace_so2_gemm_bf16_kt (A through LDS in 64-k stages, 128 x 256 tiles), "lds"
# = tace_so2_gemm_bf16 (a row tile's whole k in LDS), None = the library
# (torch.mm / addmm).  Measured per call on the fe101k chunk shapes (2^20
# edges: block 0 has 1 M rows, blocks m > 0 2 M), library / lds / kt in ms:
#   biased:   384->384 1.22 / 0.77 / 0.72, 768->1152 3.90 / 3.06 / 2.52,
#             96->384 0.90 / 0.37 / 0.74
#   1 M rows: 384->96 0.30 / 0.33 / 0.25, 1152->768 2.03 / 3.24 / 2.14,
#             384->384 0.64 / 0.71 / 0.62
#   2 M rows: 256->256 0.68 / 0.89 / 0.65, 512->192 0.82 / 1.07 / 0.78,
#             96->256 0.56 / 0.55 / 0.76, 256->96 0.45 / 0.47 / 0.38,
#             192->512 1.21 / 1.19 / 1.23, 128->128 0.31 / 0.33 / 0.33,
#             256->192 0.59 / 0.78 / 0.54, 96->128 0.33 / 0.30 / 0.51,
#             128->96 0.35 / 0.29 / 0.28, 192->256 0.65 / 0.76 / 0.59
# (the library's bias costs a copy of the broadcast bias into the output plus
# a beta = 1 pass; k = 96 is not a multiple of 64, so the k-tiled kernel takes
# its slower general path).  Every shape takes a hand-written kernel: where
# the library is ahead (1152->768, 128->128) it is by 4-5%.
_SO2_TABLE = {
    (384, 384, True): "kt", (768, 1152, True): "kt", (96, 384, True): "lds",
    (384, 96, False): "kt", (1152, 768, False): "kt", (384, 384, False): "kt",
    (256, 256, False): "kt", (512, 192, False): "kt", (96, 256, False): "lds", (256, 96, False): "kt",
    (192, 512, False): "lds", (128, 128, False): "kt", (256, 192, False): "kt", (96, 128, False): "lds",
    (128, 96, False): "kt", (192, 256, False): "kt",
}


def _so2_route(k: int, n: int, bias: bool):
    """Kernel for the SO(2) GEMM [rows, k] x [k, n] (+ bias): "kt", "lds" or
    None (the library); see _SO2_TABLE."""
    if SO2_GEMM_ALL:
        return "kt" if k >= 256 else "lds"
    key = (k, n, bool(bias))
    if key in _SO2_TABLE:
        return _SO2_TABLE[key]
    return "kt" if k % 64 == 0 else "lds"


class _FusedParams:
    """Everything the fused TECE operator needs from the frozen modules,
    prepared once per forward: the SO(2) linears as W^T (forward GEMM
    operand) and W (input-gradient operand) in the mixing precision, the
    biases, the radial projection, the attention scale and the radial MLP."""

    def __init__(self, conv: "TeceConvolution", mlp, dtype):
        self.lmax, self.H, self.A, self.C = conv.lmax, conv.H, conv.A, conv.C
        self.mixing = conv.mixing if dtype == torch.float32 else None
        self.bf16 = self.mixing is not None
        op = self.mixing or dtype
        L = self.lmax

        def pair(W):
            W = W.detach().to(dtype)
            return W.t().to(op).contiguous(), W.to(op).contiguous()

        def so2(lin):
            f0 = lin.m0_rlinear
            mats = [pair(f0.weight * f0.alpha)] + [pair(lin.ms_clinear[m - 1].fc.weight * lin.ms_clinear[m - 1].fc.alpha)
                                                   for m in range(1, L + 1)]
            return [a for a, _ in mats], [b for _, b in mats], f0.bias.detach().to(dtype).contiguous()

        self.k_T, self.k_N, self.k_b = so2(conv.key_proj)
        self.q_T, self.q_N, self.q_b = so2(conv.query_proj)
        self.d_T, self.d_N, self.d_b = so2(conv.linear_down)
        lc, lg, lu = conv.linear_coefs, conv.linear_glu, conv.linear_up
        f0 = [lc.m0_rlinear, lg.m0_rlinear, lu.m0_rlinear]
        sh = [pair(torch.cat([f.weight * f.alpha for f in f0]))]
        for m in range(1, L + 1):
            fg, fu = lg.ms_clinear[m - 1].fc, lu.ms_clinear[m - 1].fc
            sh.append(pair(torch.cat([fg.weight * fg.alpha, fu.weight * fu.alpha])))
        self.s_T, self.s_N = [a for a, _ in sh], [b for _, b in sh]
        self.s_b = torch.cat([f.bias for f in f0]).detach().to(dtype).contiguous()
        rp = conv.radial_proj
        Wrp = (rp.weight * rp.alpha).detach().to(dtype)
        self.rp_T, self.rp_N, self.rp_b = Wrp.t().contiguous(), Wrp.contiguous(), rp.bias.detach().to(dtype)
        T = conv.tmin + (conv.tmax - conv.tmin) * torch.sigmoid(conv.temperature_logit.detach())
        self.tscale = (T * conv.attention_scale).to(dtype).contiguous()
        lins = [m for m in mlp.mlp if hasattr(m, "alpha")]
        self.mlp_flat = torch.cat([(m.weight * m.alpha).detach().reshape(-1) for m in lins[:-1]]).to(dtype).contiguous()
        self.mlp_layers = len(lins) - 1
        self.mlp_W = lins[-1].weight.detach().to(dtype).contiguous()
        self.mlp_alpha = float(lins[-1].alpha)
        self.mlp_WT_scaled = (lins[-1].weight * lins[-1].alpha).detach().to(dtype).t().contiguous()
        # fragment-order copies of the bf16 GEMM operands (by id of the operand;
        # each entry keeps its operand alive)
        self._frag = {}

    def _so2(self, x, B, b=None, kernel="lds"):
        """x @ B (+ b) on ``tace_so2_gemm_bf16`` or, kernel "kt", its k-tiled
        variant (bf16 operands, float32 sums, bias in the epilogue); B's
        fragment-order copy is made on first use."""
        f = self._frag.get(id(B))
        if f is None:
            f = self._frag[id(B)] = (ops.bf16_fragment_order(B), B)
        return ops.so2_gemm_bf16(x, f[0], B.shape[1], B.shape[0], b, ktiled=kernel == "kt")

    def mm(self, x, WT, b=None):
        """x @ WT (+ b): bf16 operands with float32 accumulation and output
        under bf16 mixing, else in the features' precision."""
        if self.bf16:
            r = _so2_route(WT.shape[0], WT.shape[1], b is not None) if SO2_GEMM else None
            if r is not None and x.dtype == torch.bfloat16:
                return self._so2(x, WT, b, r)
            if b is None:
                return torch.mm(x, WT, out_dtype=torch.float32)
            return torch.addmm(b, x, WT, out_dtype=torch.float32)
        return torch.mm(x, WT) if b is None else torch.addmm(b, x, WT)

    def mm_grad(self, g, WN):
        if self.bf16:
            r = _so2_route(WN.shape[0], WN.shape[1], False) if SO2_GEMM else None
            if r is not None and g.dtype == torch.bfloat16:
                return self._so2(g, WN, None, r)
            return torch.mm(g, WN, out_dtype=torch.float32)
        return torch.mm(g, WN)


def _fused_chunk_fwd(P: _FusedParams, x_lc, R, W, rs, rd, plan: ops.EdgePlan, out_map, save: bool,
                     need_out: bool = True, out=None):
    """One receiver chunk of the convolution (the sequence of
    ``TeceConvolution.edges`` with the radial MLP in front).  Returns the
    receiver sums (None without ``need_out``: a recompute for the backward;
    written into the whole batch's ``out`` at rows ``out_map`` when given)
    and, with ``save``, what the backward needs."""
    L, H, A = P.lmax, P.H, P.A
    h = ops.launch_mlp_hidden_fwd(R, P.mlp_flat, P.mlp_layers)
    if h.dtype == torch.float32:
        w = ops.launch_mlp_out_f32(h, P.mlp_W, P.mlp_alpha)
    else:
        w = torch.mm(h, P.mlp_W).mul_(P.mlp_alpha)
    del h
    ms, md, mw = ops.launch_rotate_in_fwd(x_lc, W, rs, rd, w, L, P.bf16)
    key = [P.mm(ms[m], P.k_T[m], P.k_b if m == 0 else None) for m in range(L + 1)]
    query = [P.mm(md[m], P.q_T[m], P.q_b if m == 0 else None) for m in range(L + 1)]
    del ms, md
    rp = ops.narrow_linear(R, P.rp_T, P.rp_b)
    alpha = ops.launch_softmax_fwd(ops.launch_score_fwd(query, key, rp, P.tscale, L, H), plan)
    ys = [P.mm(mw[m], P.s_T[m], P.s_b if m == 0 else None) for m in range(L + 1)]
    del mw
    o = ops.launch_edge_ace_fwd(ys, L, A, P.bf16)
    mb = [P.mm(o[m], P.d_T[m], P.d_b if m == 0 else None) for m in range(L + 1)]
    del o
    out = ops.launch_rotate_out_fwd(mb, alpha, W, plan, out_map, L, H, out=out) if need_out else None
    return out, ((w, query, key, rp, alpha, ys, mb) if save else None)


def _fused_chunk_bwd(P: _FusedParams, x_lc, R, W, rs, rd, plan: ops.EdgePlan, out_map, dst_out, recv_rows, saved,
                     g_out, gx, gR_out=None, gW_out=None):
    """Backward of one chunk: adds its grad_x into ``gx`` (per-edge rows
    summed over the receiver CSR -- receivers at feature rows ``recv_rows``
    -- and over a sender CSR, in fixed order) and returns (grad_R, grad_W)
    of its edges, written into ``gR_out`` / ``gW_out`` when given.  g_out
    is the whole batch's output gradient, read at rows out_map[dst_out[e]]."""
    L, H, A = P.lmax, P.H, P.A
    if saved is None:
        _, saved = _fused_chunk_fwd(P, x_lc, R, W, rs, rd, plan, out_map, True, need_out=False)
    w, q, k, rp, alpha, ys, mb = saved
    # the two rotations' Wigner gradients: the rotate-out's written (zeros
    # off the l blocks), the rotate-in's added on the blocks
    gm, g_alpha, gW = ops.launch_rotate_out_bwd(mb, alpha, W, g_out, dst_out, out_map, plan, L, H, P.bf16,
                                                gW_out=gW_out, g_rows=g_out.shape[0])
    go = [P.mm_grad(gm[m], P.d_N[m]) for m in range(L + 1)]
    del gm
    gys = ops.launch_edge_ace_bwd(ys, go, L, A, P.bf16)
    del go
    gmw = [P.mm_grad(gys[m], P.s_N[m]) for m in range(L + 1)]
    del gys
    g_score = ops.launch_softmax_bwd(alpha, g_alpha, plan)
    gq, gk, grp = ops.launch_score_bwd(q, k, rp, P.tscale, g_score, L, H, P.bf16)
    gms = [P.mm_grad(gk[m], P.k_N[m]) for m in range(L + 1)]
    gmd = [P.mm_grad(gq[m], P.q_N[m]) for m in range(L + 1)]
    del gq, gk
    gR = ops.narrow_linear(grp, P.rp_N)
    # edges in receiver-CSR order: the receiver rows come as run sums of each
    # workgroup's four edges, a quarter of the rows to write and read back
    runs = ops.ROTIN_RUNS if plan.eid is None and ops.rotate_in_runs_ok(x_lc) else 1
    gxs, gxd, gW, gw = ops.launch_rotate_in_bwd(x_lc, W, rs, rd, w, gms, gmd, gmw, True, runs=runs > 1, gW_acc=gW)
    Nr, E = x_lc.shape[0], rs.shape[0]
    g2 = gx.view(Nr, -1)
    ops.rows_accumulate(g2, gxd.view(E, -1), plan.rowptr, plan.eid, recv_rows, run=runs)
    del gxd
    ops.rows_accumulate(g2, gxs.view(E, -1), *ops.sender_csr(rs, Nr))
    del gxs
    if gw.dtype == torch.float32 and gw.shape[1] % 4 == 0:
        gh = ops.launch_mlp_out_bwd_f32(gw, P.mlp_W, P.mlp_alpha)
    else:
        gh = torch.mm(gw, P.mlp_WT_scaled)
    gR = torch.add(gR, ops.launch_mlp_hidden_bwd(R, gh, P.mlp_flat, P.mlp_layers), out=gR_out)
    return gR, gW


# HBM left free when chunk intermediates are kept for the backward: chunks
# whose intermediates (~28 KB per edge at C = 128, L = 2) would cut into it
# are recomputed in the backward instead
KEEP_RESERVE_BYTES = 40 << 30


def _free_bytes(device) -> int:
    """Device memory a new tensor can take: the driver's free memory plus what
    torch's caching allocator holds unused."""
    free, _total = torch.cuda.mem_get_info(device)
    return free + torch.cuda.memory_reserved(device) - torch.cuda.memory_allocated(device)


class _TeceFused(torch.autograd.Function):
    """The whole TECE convolution with the radial MLP as one operator, for
    frozen parameters: inputs x_lc [rows, K, C] (node features, l layout,
    feature-row order), R [E, n_radial], wigner [E, K, K]; output the
    receiver sums [N, K C], group-major, in feature-row order.  The backward
    is written out (recomputing each chunk's forward when there is more than
    one), so GEMM operands go between kernels and GEMMs in the mixing
    precision without casts, and all chunks add their grad_x into one buffer
    by segmented sums in a fixed order (no atomics: the forces repeat bit for
    bit).
    With several chunks, each chunk's intermediates are kept for the backward
    while that leaves ``KEEP_RESERVE_BYTES`` of HBM free; only the chunks
    beyond that are recomputed."""

    @staticmethod
    def forward(ctx, x_lc, R, W, P: _FusedParams, plan: ops.EdgePlan, rs, rd, dst, node_map, chunks):
        ctx.P, ctx.plan, ctx.chunks = P, plan, chunks
        L, C = P.lmax, P.C
        if chunks is None:
            out, ctx.saved_chunk = _fused_chunk_fwd(P, x_lc, R, W, rs, rd, plan, node_map, True)
        else:
            Nn = plan.n_nodes
            # every chunk's receiver sums straight into their rows of the output
            out = torch.empty(Nn, (L + 1) ** 2 * C, dtype=x_lc.dtype, device=x_lc.device)
            keep = any(ctx.needs_input_grad[:3])
            ctx.saved_chunks = []
            for n0, n1, e0, e1 in chunks:
                _, saved = _fused_chunk_fwd(P, x_lc, R[e0:e1], W[e0:e1], rs[e0:e1], rd[e0:e1],
                                            sub_plan(plan, n0, n1, e0, e1), node_map[n0:n1].contiguous(), keep,
                                            out=out)
                if saved is not None and _free_bytes(x_lc.device) < KEEP_RESERVE_BYTES:
                    saved, keep = None, False   # no room: this and later chunks are recomputed
                ctx.saved_chunks.append(saved)
            ctx.saved_chunk = None
        ctx.save_for_backward(x_lc, R, W, rs, rd, dst, node_map)
        return out

    @staticmethod
    def backward(ctx, g_out):
        x_lc, R, W, rs, rd, dst, node_map = ctx.saved_tensors
        P, plan, chunks = ctx.P, ctx.plan, ctx.chunks
        g_out = g_out.contiguous()
        gx = torch.zeros_like(x_lc)
        if chunks is None:
            gR, gW = _fused_chunk_bwd(P, x_lc, R, W, rs, rd, plan, node_map, dst, node_map, ctx.saved_chunk, g_out,
                                      gx)
            ctx.saved_chunk = None
            return gx, gR, gW, None, None, None, None, None, None, None
        gR, gW = torch.empty_like(R), torch.empty_like(W)
        for i, (n0, n1, e0, e1) in enumerate(chunks):
            saved, ctx.saved_chunks[i] = ctx.saved_chunks[i], None
            # the output gradient of the chunk's receivers read in place
            # (rows node_map[dst[e]] of the whole batch's)
            _fused_chunk_bwd(P, x_lc, R[e0:e1], W[e0:e1], rs[e0:e1], rd[e0:e1], sub_plan(plan, n0, n1, e0, e1),
                             node_map, dst[e0:e1], node_map[n0:n1].contiguous(), saved, g_out, gx,
                             gR_out=gR[e0:e1], gW_out=gW[e0:e1])
            del saved
        return gx, gR, gW, None, None, None, None, None, None, None


def fused_supported(conv: "TeceConvolution", mlp) -> bool:
    """The fused operator covers frozen parameters and the fused radial MLP."""
    mods = [conv, mlp]
    return (getattr(mlp, "fused", False)
            and not any(p.requires_grad for m in mods for p in m.parameters()))


def tece_fused(conv: "TeceConvolution", mlp, x_gm, node_map, R, plan: ops.EdgePlan, src, dst, wigner,
               chunk_edges: int):
    """TECE convolution + radial MLP (``OAM20260705Convolution.forward`` with
    ``edge_info``) on the fused operator; receiver chunks of at most
    ``chunk_edges`` edges when the graph has more."""
    P = _FusedParams(conv, mlp, x_gm.dtype)
    x_lc = conv.node_components(x_gm)
    rows = node_map.long()
    src, dst = src.long(), dst.long()
    if plan.n_edges <= chunk_edges:
        return _TeceFused.apply(x_lc, R, wigner, P, plan, rows[src].contiguous(), rows[dst].contiguous(),
                                dst.contiguous(), node_map, None)
    if plan.eid is not None:   # chunks need receiver-grouped edges
        order = plan.eid.long()
        R, wigner, src, dst = R[order], wigner[order], src[order], dst[order]
        plan = ops.EdgePlan(plan.n_nodes, plan.n_edges, plan.rowptr, src.to(torch.int32).contiguous(), None)
    return _TeceFused.apply(x_lc, R.contiguous(), wigner.contiguous(), P, plan, rows[src].contiguous(),
                            rows[dst].contiguous(), dst.contiguous(), node_map, receiver_chunks(plan, chunk_edges))
