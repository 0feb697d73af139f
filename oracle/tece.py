"""CPU restatement of the TECE edge convolution (test infrastructure).

``OAM20260705Convolution`` (``tace/models/_e3nn/archive/oam_2026_07_05.py:547-823``)
inside ``OAM20260705Interaction`` (``tace/models/_e3nn/inter.py:440-519``), its
edge frames (``tace/models/o2/rotation_matrix.py:74-88``,
``tace/models/o2/wigner.py:176-362``) and ``GraphSoftmax``
(``tace/models/softmax.py:80-114``), written from the reference's equations in
plain PyTorch.  Only ``tests/``, ``__graft_entry__.smoke`` and ``bench.py``'s
CPU baseline may import it.

Conventions restated:
* edge frame: a unit quaternion blended (C-infinity smooth step in y) between
  two charts, so that R(q) maps the edge direction onto +y;
* Wigner blocks D^0 = 1, D^1 = R, D^l = (2l+1) C^T (D^1 (x) D^(l-1)) C with
  C = W3j(1, l-1, l) (``wigner.py:330-357``);
* SO(2) component order ("m layout"): m = 0 for l = 0..L, then for every
  m = 1..mmax the +m components (l = m..L) followed by the -m components; the
  e3nn real-basis component k of degree l carries m = k - l (``wigner.py:38-66``);
* features inside the convolution are [E, components, channels].
"""

from __future__ import annotations

import math
from typing import List, Optional

import torch

from . import so3


# ------------------------------------------------------------ edge frames ----
def _nrm(x: torch.Tensor, eps: float = 1e-7) -> torch.Tensor:
    return torch.sqrt((x * x).sum(-1, keepdim=True) + eps * eps)


def _smooth_step(x: torch.Tensor) -> torch.Tensor:
    """C-infinity step: 0 for x <= 0, 1 for x >= 1, e^(-1/x) / (e^(-1/x) + e^(-1/(1-x)))."""
    x = x.clamp(0.0, 1.0)
    tiny = torch.finfo(x.dtype).eps
    a = torch.exp(-1.0 / x.clamp(min=tiny))
    b = torch.exp(-1.0 / (1.0 - x).clamp(min=tiny))
    mid = a / (a + b)
    return torch.where(x <= 0.0, torch.zeros_like(x), torch.where(x >= 1.0, torch.ones_like(x), mid))


def edge_rotation(vec: torch.Tensor) -> torch.Tensor:
    """R [E,3,3] with R @ (vec/|vec|) = +y (``rotation_matrix.py:74-88``):
    charts q+ = (1+y, -z, 0, x) and q- = (-z, 1-y, x, 0) (w, x, y, z order),
    normalised, blended by nlerp with weight smooth_step((y+1)/2)."""
    u = vec / _nrm(vec)
    x, y, z = u.unbind(-1)
    zero = torch.zeros_like(x)
    qp = torch.stack([1.0 + y, -z, zero, x], -1)
    qp = qp / _nrm(qp)
    qn = torch.stack([-z, 1.0 - y, x, zero], -1)
    qn = qn / _nrm(qn)
    t = _smooth_step(0.5 * (y + 1.0)).unsqueeze(-1)
    qp = torch.where((qn * qp).sum(-1, keepdim=True) < 0.0, -qp, qp)
    q = (1.0 - t) * qn + t * qp
    q = q / _nrm(q)
    w, a, b, c = q.unbind(-1)
    rows = [
        [1 - 2 * (b * b + c * c), 2 * (a * b - w * c), 2 * (a * c + w * b)],
        [2 * (a * b + w * c), 1 - 2 * (a * a + c * c), 2 * (b * c - w * a)],
        [2 * (a * c - w * b), 2 * (b * c + w * a), 1 - 2 * (a * a + b * b)],
    ]
    return torch.stack([torch.stack(r, -1) for r in rows], -2)


def wigner_blocks(R: torch.Tensor, lmax: int) -> List[torch.Tensor]:
    """[D^0, ..., D^lmax] from the l = 1 block by the W3j(1, l-1, l) recursion."""
    E = R.shape[0]
    out = [R.new_ones(E, 1, 1)]
    if lmax >= 1:
        out.append(R)
    for l in range(2, lmax + 1):
        cg = so3.w3j_torch(1, l - 1, l, R.dtype)  # [3, 2l-1, 2l+1]
        t = torch.einsum("abm,eac->ebmc", cg, R)
        t = torch.einsum("ebmc,ebd->emcd", t, out[l - 1])
        out.append(torch.einsum("emcd,cdn->emn", t, cg) * (2 * l + 1))
    return out


def m_order(lmax: int, mmax: int) -> List[int]:
    """e3nn component index (l^2 + l + m) of each row of the m layout."""
    rows = [l * l + l for l in range(lmax + 1)]
    for m in range(1, mmax + 1):
        rows += [l * l + l + m for l in range(m, lmax + 1)]
        rows += [l * l + l - m for l in range(m, lmax + 1)]
    return rows


def edge_wigner(vec: torch.Tensor, lmax: int, mmax: int):
    """(wigner, wigner_inv): wigner [E, K_m, (L+1)^2] maps l-layout edge features
    into the edge frame's m layout, wigner_inv [E, (L+1)^2, K_m] back
    (``wigner.py:231-239``; mmax = lmax, so the inverse rescale is 1)."""
    if mmax != lmax:
        raise NotImplementedError("the restatement covers mmax == lmax (the TECE configurations)")
    blocks = wigner_blocks(edge_rotation(vec), lmax)
    K = (lmax + 1) ** 2
    D = vec.new_zeros(vec.shape[0], K, K)
    for l, b in enumerate(blocks):
        D[:, l * l:(l + 1) ** 2, l * l:(l + 1) ** 2] = b
    W = D[:, m_order(lmax, mmax), :]
    return W, W.transpose(1, 2)


# ------------------------------------------------------------- SO(2) ops ----
class TorchLinear(torch.nn.Module):
    """``torchLinear`` (``tace/models/linear.py:210-244``): y = x (W/sqrt(in))^T + b,
    W ~ N(0,1) [out, in], b zeros."""

    def __init__(self, i: int, o: int, bias: bool = True):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.randn(o, i))
        self.bias = torch.nn.Parameter(torch.zeros(o)) if bias else None
        self.alpha = 1.0 / math.sqrt(i)

    def forward(self, x):
        return torch.nn.functional.linear(x, self.weight * self.alpha, self.bias)


class SO2MLinear(torch.nn.Module):
    """``uvSO2MLinear`` weight type "w1": one real linear map applied to the
    +m and the -m components alike (``oam_2026_07_05.py:47-136``)."""

    def __init__(self, cin: int, cout: int, nin: int, nout: int):
        super().__init__()
        self.fc = TorchLinear(nin * cin, nout * cout, bias=False)


class SO2Linear(torch.nn.Module):
    """``uvSO2Linear`` (type "w1", ``oam_2026_07_05.py:138-247``): per m a dense
    map over (component, channel); m = 0 with bias."""

    def __init__(self, mmax: int, lmax: int, cin: int, cout: int, nin: Optional[List[int]] = None,
                 nout: Optional[List[int]] = None):
        super().__init__()
        self.mmax, self.lmax, self.cin, self.cout = mmax, lmax, cin, cout
        self.nin = nin or [lmax + 1 - m for m in range(mmax + 1)]
        self.nout = nout or [lmax + 1 - m for m in range(mmax + 1)]
        self.m0_rlinear = TorchLinear(cin * self.nin[0], cout * self.nout[0], bias=True)
        self.ms_clinear = torch.nn.ModuleList(
            SO2MLinear(cin, cout, self.nin[m], self.nout[m]) for m in range(1, mmax + 1))

    def forward(self, x):
        B = x.shape[0]
        outs = [self.m0_rlinear(x[:, :self.nin[0]].reshape(B, -1)).view(B, self.nout[0], self.cout)]
        off = self.nin[0]
        for m in range(1, self.mmax + 1):
            n = self.nin[m]
            xm = x[:, off:off + 2 * n].reshape(B, 2, n * self.cin)
            off += 2 * n
            y = self.ms_clinear[m - 1].fc(xm)
            outs.append(y[:, 0].view(B, self.nout[m], self.cout))
            outs.append(y[:, 1].view(B, self.nout[m], self.cout))
        return torch.cat(outs, dim=1)


def scaled_sigmoid(x):
    return torch.sigmoid(x) * 1.8467055342154763  # ScaledSigmoid (tace/models/mlp.py:40-46)


def so2_expand(mmax: int, lmax: int, full: bool, start: int = 0) -> torch.Tensor:
    """Row -> weight/gate component map (``so2_expand_index``, ``SO2Gate``):
    per m one entry per component (lmax+1-m of them, or lmax+1 when ``full``),
    listed twice (for +m and -m) when m > 0."""
    idx, off = [], 0
    for m in range(start, mmax + 1):
        n = lmax + 1 if full else lmax + 1 - m
        r = list(range(off, off + n))
        idx += r + (r if m > 0 else [])
        off += n
    return torch.tensor(idx, dtype=torch.long)


class ComplexProduct(torch.nn.Module):
    """``uuuSO2TensorProduct`` with external per-edge weights, m1 >= m2
    (``oam_2026_07_05.py:312-516``): features of n = lmax+1 components for
    every m; m = 0 real [B, n, C], m > 0 complex (real block, imaginary
    block).  Paths into m3: m1 + m2 = m3 ("sum", z = x y) and |m1 - m2| = m3
    ("diff", z = x conj(y)); m3 = 0 keeps the real part; each output m is
    scaled by 1/sqrt(number of its paths)."""

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

    def _split(self, x):
        B, n, C = x.shape[0], self.n, self.C
        out = [x[:, :n]]
        for m in range(1, self.mmax + 1):
            out.append(x[:, n + 2 * n * (m - 1):n + 2 * n * m].reshape(B, 2, n, C))
        return out

    def forward(self, x, y, ws):
        B, n, C = x.shape[0], self.n, self.C
        xs, ys = self._split(x), self._split(y)
        woff = 0
        outs = []
        for m3, ps in enumerate(self.paths):
            re = 0.0
            im = 0.0
            for (m1, m2, mode) in ps:
                w = ws[:, woff:woff + n * C].reshape(B, n, C)
                woff += n * C
                a, b = xs[m1], ys[m2]
                if m1 == 0 and m2 == 0:
                    zr, zi = a * b, None
                elif m2 == 0:
                    zr, zi = a[:, 0] * b, a[:, 1] * b
                elif m1 == 0:
                    zr, zi = a * b[:, 0], a * b[:, 1]
                else:
                    ar, ai, br, bi = a[:, 0], a[:, 1], b[:, 0], b[:, 1]
                    if mode == "sum":
                        zr, zi = ar * br - ai * bi, ar * bi + ai * br
                    else:
                        zr, zi = ar * br + ai * bi, ai * br - ar * bi
                re = re + zr * w
                if m3 > 0:
                    im = im + zi * w
            s = 1.0 / math.sqrt(len(ps))
            outs.append(re * s)
            if m3 > 0:
                outs.append(im * s)
        return torch.cat(outs, dim=1)


def graph_softmax(score: torch.Tensor, dst: torch.Tensor, num_nodes: int, eps: float = 1e-16):
    """``GraphSoftmax`` (``softmax.py:100-112``, no rescale): per receiver and
    column, exp(s - max) / (sum exp(s - max) + eps), the max not differentiated."""
    H = score.shape[1]
    mx = torch.full((num_nodes, H), -math.inf, dtype=score.dtype)
    mx = mx.scatter_reduce(0, dst.view(-1, 1).expand(-1, H), score.detach(), reduce="amax", include_self=True)
    ex = torch.exp(score - mx[dst])
    den = torch.zeros(num_nodes, H, dtype=score.dtype).index_add(0, dst, ex) + eps
    return ex / den[dst]


class TeceConvolution(torch.nn.Module):
    """``OAM20260705Convolution`` with the ``OAM20260705Interaction`` flags
    (so2_linear_type "w1", temperature, edge-ACE, graph softmax, radial phase;
    ``inter.py:450-454``) and gate_m0."""

    def __init__(self, mmax: int, lmax: int, C: int, num_head: int, edge_ace_hidden: int,
                 num_radial: int):
        super().__init__()
        self.mmax, self.lmax, self.C, self.H = mmax, lmax, C, num_head
        self.Ch = C // num_head
        n = lmax + 1
        A = edge_ace_hidden
        self.num_components = sum(n - m for m in range(mmax + 1))
        self.weight_numel = self.num_components * C * 2
        self.register_buffer("expand_index", so2_expand(mmax, lmax, False), persistent=False)
        self.num_gates = n * (mmax + 1)
        self.rows_full = n + 2 * n * mmax
        full = [n] * (mmax + 1)
        self.linear_up = SO2Linear(mmax, lmax, 2 * C, A, nout=[self.num_gates + n] + [n] * mmax)
        self.register_buffer("gate_index", so2_expand(mmax, lmax, True), persistent=False)
        self.linear_glu = SO2Linear(mmax, lmax, 2 * C, A, nout=full)
        self.ece = ComplexProduct(mmax, lmax, A)
        self.linear_coefs = SO2Linear(0, lmax, 2 * C, 1, nout=[self.ece.weight_numel])
        self.linear_down = SO2Linear(mmax, lmax, A, C, nin=full)
        self.query_proj = SO2Linear(mmax, lmax, C, C)
        self.key_proj = SO2Linear(mmax, lmax, C, C)
        self.radial_proj = TorchLinear(num_radial, 2 * num_head)
        torch.nn.init.zeros_(self.radial_proj.weight)
        torch.nn.init.zeros_(self.radial_proj.bias)
        self.attention_scale = 1.0 / math.sqrt(self.Ch * self.rows_full)
        self.tmin, self.tmax = 0.25, 4.0
        self.temperature_logit = torch.nn.Parameter(
            torch.full((num_head,), math.log((1.0 - self.tmin) / (self.tmax - 1.0))))

    def score(self, q, k, R):
        """Radial-rotary complex QK score [E, H] (``oam_2026_07_05.py:699-754``)."""
        E, H, Ch, n = q.shape[0], self.H, self.Ch, self.lmax + 1
        rp = self.radial_proj(R)
        bias, phase = rp[:, :H], math.pi * torch.tanh(rp[:, H:])
        s = (q[:, :n].reshape(E, n, H, Ch) * k[:, :n].reshape(E, n, H, Ch)).sum(dim=(1, 3))
        off = n
        for m in range(1, self.mmax + 1):
            nm = self.lmax + 1 - m
            qm = q[:, off:off + 2 * nm].reshape(E, 2, nm, H, Ch)
            km = k[:, off:off + 2 * nm].reshape(E, 2, nm, H, Ch)
            off += 2 * nm
            c, sn = torch.cos(m * phase).view(E, 1, H, 1), torch.sin(m * phase).view(E, 1, H, 1)
            kr = c * km[:, 0] - sn * km[:, 1]
            ki = sn * km[:, 0] + c * km[:, 1]
            s = s + (qm[:, 0] * kr + qm[:, 1] * ki).sum(dim=(1, 3))
        T = self.tmin + (self.tmax - self.tmin) * torch.sigmoid(self.temperature_logit)
        return s * self.attention_scale * T + bias

    def forward(self, x_l, w, edge_index, wigner, wigner_inv, R):
        """x_l: node features [N, (L+1)^2, C] (l layout); w: radial weights
        [E, weight_numel]; returns the scattered messages [N, (L+1)^2, C]."""
        N, E = x_l.shape[0], w.shape[0]
        src, dst = edge_index[0], edge_index[1]
        m = torch.bmm(wigner, torch.cat((x_l[src], x_l[dst]), dim=-1))
        key = self.key_proj(m[:, :, :self.C])
        query = self.query_proj(m[:, :, self.C:])
        alpha = self.score(query, key, R)
        w = w.view(E, self.num_components, 2 * self.C).index_select(1, self.expand_index)
        m = w * m
        coefs = scaled_sigmoid(self.linear_coefs(m).squeeze(-1))
        m2 = self.linear_glu(m)
        m = self.linear_up(m)
        gate, m = m[:, :self.num_gates], m[:, self.num_gates:self.num_gates + self.rows_full]
        g = scaled_sigmoid(gate).index_select(1, self.gate_index)
        m = m + g * m + self.ece(m, m2, coefs)
        m = self.linear_down(m)
        alpha = graph_softmax(alpha, dst, N)
        m = (m.view(E, m.shape[1], self.H, self.Ch) * alpha.view(E, 1, self.H, 1)).view(E, m.shape[1], self.C)
        m = torch.bmm(wigner_inv, m)
        return torch.zeros(N, m.shape[1], self.C, dtype=m.dtype).index_add(0, dst, m)


def e3nn_to_lc(x: torch.Tensor, lmax: int, C: int) -> torch.Tensor:
    """e3nn mul_ir layout of C x (0, 1, ..., lmax) -> [N, (L+1)^2, C]
    (``LayoutTransform.forward``, ``tace/models/layout.py:60-70``)."""
    N = x.shape[0]
    parts, off = [], 0
    for l in range(lmax + 1):
        d = 2 * l + 1
        parts.append(x[:, off:off + C * d].reshape(N, C, d))
        off += C * d
    return torch.cat(parts, dim=-1).transpose(1, 2)


def lc_to_e3nn(x: torch.Tensor, lmax: int) -> torch.Tensor:
    """Inverse of ``e3nn_to_lc`` (``LayoutTransform.inverse``)."""
    N = x.shape[0]
    xt = x.transpose(1, 2)
    return torch.cat([xt[:, :, l * l:(l + 1) ** 2].reshape(N, -1) for l in range(lmax + 1)], dim=1)
