"""HIP code generator for the CG tensor-product kernels of the TACE path.

Every admissible coupling path is known when the model is built, so the
kernels are emitted with the Clebsch-Gordan coefficients (times
sqrt(2 l3 + 1), e3nn's "component" path normalisation) as compile-time
constants: the contraction becomes straight-line FMAs on registers, with no
coefficient tables, no dynamic register indexing and no scratch memory.

Kernel families (all templated on T = float / double):

* ``uvu`` edge tensor product fused with the receiver scatter
  (``O3ScatterTensorProduct``, ``tace/models/_e3nn/fused.py:172-271``):
  one 64-lane wavefront per receiver node, lanes = channels, accumulators
  for all output components in registers, edges streamed in CSR order; no
  atomics in the forward.  The backward walks the same receiver CSR and
  produces grad_w / grad_y per edge (grad_y reduced across lanes with
  cross-lane shuffles) and grad_x scattered to sender nodes.
* ``uuu`` node-level product (``uuuTensorProduct``, ``fused.py:17-95``):
  one thread per (node, channel).

A variant is identified by the l-lists of its operands, e.g.
``uvu|0|0,1,2,3|0,1,2,3``; ``tace_amd.ops`` derives the same key from the
model's irreps and the C-ABI verifies it against the compiled registry.
"""

from __future__ import annotations

import math
import os
import sys
from typing import Dict, List, Sequence, Tuple

_HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(_HERE)))

from tace_amd.so3 import Irrep, Irreps, generate_paths, wigner_3j  # noqa: E402


def _lit(v: float) -> str:
    return f"T({v!r})"


def _irreps_from_ls(ls: Sequence[int], mul: int = 1) -> Irreps:
    return Irreps([(mul, Irrep(l, (-1) ** l)) for l in ls])


def variant_key(kind: str, in1: Sequence[int], in2: Sequence[int], out: Sequence[int]) -> str:
    j = lambda s: ",".join(str(int(v)) for v in s)
    return f"{kind}|{j(in1)}|{j(in2)}|{j(out)}"


class Variant:
    def __init__(self, kind: str, in1: Sequence[int], in2: Sequence[int], out: Sequence[int]):
        assert kind in ("uvu", "uuu")
        self.kind = kind
        self.in1, self.in2, self.out = list(in1), list(in2), list(out)
        self.key = variant_key(kind, in1, in2, out)
        i1 = _irreps_from_ls(in1, 2)
        i2 = _irreps_from_ls(in2, 2 if kind == "uuu" else 1)
        o = _irreps_from_ls(out, 1)
        identical = kind == "uuu" and list(in1) == list(in2)
        self.paths, outs = generate_paths(o, i1, i2, kind, identical_inputs=identical)
        self.path_l = [(in1[i], in2[j], outs[k][1].l) for (i, j, k) in self.paths]
        self.path_blocks = [(i, j) for (i, j, _) in self.paths]
        self.d1 = [2 * l + 1 for l in in1]           # per-channel dims of in1 blocks
        self.d2 = [2 * l + 1 for l in in2]
        self.off1 = [sum(self.d1[:b]) for b in range(len(in1))]  # per-channel offsets (x C)
        self.off2 = [sum(self.d2[:b]) for b in range(len(in2))]
        self.dout = [2 * l3 + 1 for (_, _, l3) in self.path_l]
        self.offo = [sum(self.dout[:p]) for p in range(len(self.paths))]
        self.D1, self.D2, self.DO = sum(self.d1), sum(self.d2), sum(self.dout)
        self.name = (f"{kind}_" + "".join(map(str, in1)) + "_" + "".join(map(str, in2)) + "_"
                     + "".join(map(str, out)))
        if len(self.name) > 60:
            import hashlib
            self.name = f"{kind}_" + hashlib.sha1(self.key.encode()).hexdigest()[:12]
        self.cg = []
        for (l1, l2, l3) in self.path_l:
            W = wigner_3j(l1, l2, l3) * math.sqrt(2 * l3 + 1)
            nz = [(i, j, k, float(W[i, j, k])) for i in range(2 * l1 + 1) for j in range(2 * l2 + 1)
                  for k in range(2 * l3 + 1) if abs(W[i, j, k]) > 1e-13]
            self.cg.append(nz)

    # ---------------------------------------------------------------- uvu ----
    def _x_loads(self, ptr: str, guard: str) -> List[str]:
        out = []
        for b, d in enumerate(self.d1):
            for m in range(d):
                out.append(f"    const T x{b}_{m} = {guard} ? {ptr}[(size_t)C * {self.off1[b]} + (size_t)u * {d} + {m}] : T(0);")
        return out

    def _y_loads(self, ptr: str) -> List[str]:
        return [f"    const T y{b}_{m} = {ptr}[{self.off2[b] + m}];" for b, d in enumerate(self.d2) for m in range(d)]

    def _products(self) -> Tuple[List[str], Dict]:
        used = set()
        for p, (b1, b2) in enumerate(self.path_blocks):
            for (i, j, k, c) in self.cg[p]:
                used.add((b1, i, b2, j))
        lines = [f"    const T q{b1}_{i}_{b2}_{j} = x{b1}_{i} * y{b2}_{j};" for (b1, i, b2, j) in sorted(used)]
        return lines

    def _t_expr(self, p: int, k: int) -> str:
        b1, b2 = self.path_blocks[p]
        terms = [f"{_lit(c)} * q{b1}_{i}_{b2}_{j}" for (i, j, kk, c) in self.cg[p] if kk == k]
        return " + ".join(terms) if terms else "T(0)"

    def emit_uvu_fwd(self) -> str:
        P = len(self.paths)
        L = []
        L.append(f"template <typename T, bool OUT_GM>\n__global__ __launch_bounds__(64) void k_{self.name}_fwd(")
        L.append("    const T* __restrict__ x, const T* __restrict__ y, const T* __restrict__ w,")
        L.append("    const int* __restrict__ rowptr, const int* __restrict__ eid, const int* __restrict__ src,")
        L.append("    T* __restrict__ out, int n_nodes, int C) {")
        L.append("  const int n = blockIdx.x;")
        L.append("  if (n >= n_nodes) return;")
        L.append("  const int beg = rowptr[n], end = rowptr[n + 1];")
        L.append(f"  const size_t DX = (size_t)C * {self.D1}, WW = (size_t)C * {P};")
        L.append("  for (int cb = 0; cb < C; cb += 64) {")
        L.append("    const int u = cb + (int)threadIdx.x;")
        L.append("    const bool act = u < C;")
        for a in range(self.DO):
            L.append(f"    T a{a} = T(0);")
        L.append("    for (int e = beg; e < end; ++e) {")
        L.append("    const int ed = eid ? eid[e] : e;")
        L.append("    const T* xs = x + (size_t)src[ed] * DX;")
        L.append(f"    const T* ys = y + (size_t)ed * {self.D2};")
        L.append("    const T* ws = w + (size_t)ed * WW;")
        L += self._x_loads("xs", "act")
        L += self._y_loads("ys")
        for p in range(P):
            L.append(f"    const T w{p} = act ? ws[(size_t){p} * C + u] : T(0);")
        L += self._products()
        for p in range(P):
            for k in range(self.dout[p]):
                L.append(f"    a{self.offo[p] + k} += w{p} * ({self._t_expr(p, k)});")
        L.append("    }")
        L.append("    if (act) {")
        L.append("      const size_t N = (size_t)n_nodes;")
        for p in range(P):
            d = self.dout[p]
            for k in range(d):
                e3, gm = self._addr("out", p, k)
                L.append(f"      out[OUT_GM ? ({gm}) : ({e3})] = a{self.offo[p] + k};")
        L.append("    }")
        L.append("  }")
        L.append("}")
        return "\n".join(L)

    def emit_uvu_bwd(self) -> str:
        P = len(self.paths)
        L = []
        L.append(f"template <typename T, bool NEED_GX, bool OUT_GM>\n__global__ __launch_bounds__(64) void k_{self.name}_bwd(")
        L.append("    const T* __restrict__ x, const T* __restrict__ y, const T* __restrict__ w,")
        L.append("    const T* __restrict__ gout,")
        L.append("    const int* __restrict__ rowptr, const int* __restrict__ eid, const int* __restrict__ src,")
        L.append("    T* __restrict__ cbuf, T* __restrict__ gy, T* __restrict__ gw, int n_nodes, int C) {")
        L.append("  const int n = blockIdx.x;")
        L.append("  if (n >= n_nodes) return;")
        L.append("  const int beg = rowptr[n], end = rowptr[n + 1];")
        L.append(f"  const size_t DX = (size_t)C * {self.D1}, WW = (size_t)C * {P};")
        L.append("  for (int cb = 0; cb < C; cb += 64) {")
        L.append("    const int u = cb + (int)threadIdx.x;")
        L.append("    const bool act = u < C;")
        L.append("    const size_t N = (size_t)n_nodes;")
        for p in range(P):
            d = self.dout[p]
            for k in range(d):
                e3, gm = self._addr("out", p, k)
                L.append(f"    const T g{self.offo[p] + k} = act ? gout[OUT_GM ? ({gm}) : ({e3})] : T(0);")
        L.append("    for (int e = beg; e < end; ++e) {")
        L.append("    const int ed = eid ? eid[e] : e;")
        L.append("    const int s = src[ed];")
        L.append("    const T* xs = x + (size_t)s * DX;")
        L.append(f"    const T* ys = y + (size_t)ed * {self.D2};")
        L.append("    const T* ws = w + (size_t)ed * WW;")
        L += self._x_loads("xs", "act")
        L += self._y_loads("ys")
        for p in range(P):
            L.append(f"    const T w{p} = act ? ws[(size_t){p} * C + u] : T(0);")
        L += self._products()
        for b, d in enumerate(self.d1):
            for m in range(d):
                L.append(f"    T hx{b}_{m} = T(0);")
        for b, d in enumerate(self.d2):
            for m in range(d):
                L.append(f"    T hy{b}_{m} = T(0);")
        for p in range(P):
            b1, b2 = self.path_blocks[p]
            d = self.dout[p]
            L.append("    {")
            for k in range(d):
                L.append(f"      const T t{k} = {self._t_expr(p, k)};")
            gsum = " + ".join(f"g{self.offo[p] + k} * t{k}" for k in range(d))
            L.append(f"      if (act) gw[(size_t)ed * WW + (size_t){p} * C + u] = {gsum};")
            for k in range(d):
                L.append(f"      const T a{k} = w{p} * g{self.offo[p] + k};")
            for (i, j, k, c) in self.cg[p]:
                L.append(f"      if (NEED_GX) hx{b1}_{i} += {_lit(c)} * (y{b2}_{j} * a{k});")
                L.append(f"      hy{b2}_{j} += {_lit(c)} * (x{b1}_{i} * a{k});")
            L.append("    }")
        # grad_x contribution of this edge, one row per receiver-sorted slot;
        # summed per sender by k_seg_rowsum (deterministic, no atomics)
        L.append("    if (NEED_GX && act) {")
        L.append("      T* cb = cbuf + (size_t)e * DX;")
        for b, d in enumerate(self.d1):
            for m in range(d):
                L.append(f"      cb[(size_t)C * {self.off1[b]} + (size_t)u * {d} + {m}] = hx{b}_{m};")
        L.append("    }")
        L.append(f"    T* gys = gy + (size_t)ed * {self.D2};")
        for b, d in enumerate(self.d2):
            for m in range(d):
                L.append(f"    {{ const T v = wave_sum(hy{b}_{m}); if (threadIdx.x == 0) gys[{self.off2[b] + m}] = (cb == 0) ? v : gys[{self.off2[b] + m}] + v; }}")
        L.append("    }")
        L.append("  }")
        L.append("}")
        return "\n".join(L)

    # ---------------------------------------------------------------- uuu ----
    @staticmethod
    def _groups(ls: Sequence[int]):
        """Runs of equal l (what ``Irreps.simplify`` merges): per block
        (group id, index inside the group); per group (l, count, per-channel offset)."""
        blk, grp = [], []
        for l in ls:
            if grp and grp[-1][0] == l:
                blk.append((len(grp) - 1, grp[-1][1]))
                grp[-1][1] += 1
            else:
                blk.append((len(grp), 0))
                grp.append([l, 1])
        off, acc = [], 0
        for l, c in grp:
            off.append(acc)
            acc += c * (2 * l + 1)
        return blk, [(l, c, o) for (l, c), o in zip(grp, off)]

    def _addr(self, which: str, b: int, m: int) -> Tuple[str, str]:
        """(e3nn address, group-major address) of component m of block b of
        operand ``which`` (in1 / in2 / out) for channel u of node n.
        e3nn: n*C*D + C*off_b + u*d_b + m;  group-major: the whole batch's group
        g is one [N, 2l+1, count*C] matrix at N*C*goff_g."""
        ls = {"in1": self.in1, "in2": self.in2, "out": [l3 for (_, _, l3) in self.path_l]}[which]
        D = {"in1": self.D1, "in2": self.D2, "out": self.DO}[which]
        offs = {"in1": self.off1, "in2": self.off2, "out": self.offo}[which]
        d = 2 * ls[b] + 1
        e3 = f"(size_t)n * C * {D} + (size_t)C * {offs[b]} + (size_t)u * {d} + {m}"
        blk, grp = self._groups(ls)
        g, j = blk[b]
        l, cnt, goff = grp[g]
        gm = f"(size_t)N * C * {goff} + ((size_t)n * {2 * l + 1} + {m}) * ((size_t){cnt} * C) + (size_t){j} * C + u"
        return e3, gm

    def _ld(self, ptr: str, which: str, b: int, m: int, flag: str) -> str:
        e3, gm = self._addr(which, b, m)
        return f"({flag} ? {ptr}[{gm}] : {ptr}[{e3}])"

    def emit_uuu_fwd(self) -> str:
        P = len(self.paths)
        L = []
        L.append(f"template <typename T, bool IN1_GM, bool OUT_GM>\n__global__ __launch_bounds__(256) void k_{self.name}_fwd(")
        L.append("    const T* __restrict__ x1, const T* __restrict__ x2, T* __restrict__ out, int n_nodes, int C) {")
        L.append("  const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;")
        L.append("  const size_t n = t / (size_t)C; const int u = (int)(t % (size_t)C);")
        L.append("  const size_t N = (size_t)n_nodes;")
        L.append("  if (n >= N) return;")
        for bb, d in enumerate(self.d1):
            for m in range(d):
                L.append(f"  const T x{bb}_{m} = {self._ld('x1', 'in1', bb, m, 'IN1_GM')};")
        for bb, d in enumerate(self.d2):
            for m in range(d):
                L.append(f"  const T y{bb}_{m} = {self._ld('x2', 'in2', bb, m, 'false')};")
        for p in range(P):
            b1, b2 = self.path_blocks[p]
            d = self.dout[p]
            for k in range(d):
                terms = [f"{_lit(c)} * (x{b1}_{i} * y{b2}_{j})" for (i, j, kk, c) in self.cg[p] if kk == k]
                e3, gm = self._addr("out", p, k)
                L.append(f"  out[OUT_GM ? ({gm}) : ({e3})] = {' + '.join(terms) if terms else 'T(0)'};")
        L.append("}")
        return "\n".join(L)

    def emit_uuu_bwd(self) -> str:
        P = len(self.paths)
        L = []
        L.append(f"template <typename T, bool IN1_GM, bool OUT_GM>\n__global__ __launch_bounds__(256) void k_{self.name}_bwd(")
        L.append("    const T* __restrict__ x1, const T* __restrict__ x2, const T* __restrict__ gout,")
        L.append("    T* __restrict__ g1, T* __restrict__ g2, int n_nodes, int C) {")
        L.append("  const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;")
        L.append("  const size_t n = t / (size_t)C; const int u = (int)(t % (size_t)C);")
        L.append("  const size_t N = (size_t)n_nodes;")
        L.append("  if (n >= N) return;")
        for bb, d in enumerate(self.d1):
            for m in range(d):
                L.append(f"  const T x{bb}_{m} = {self._ld('x1', 'in1', bb, m, 'IN1_GM')};")
                L.append(f"  T hx{bb}_{m} = T(0);")
        for bb, d in enumerate(self.d2):
            for m in range(d):
                L.append(f"  const T y{bb}_{m} = {self._ld('x2', 'in2', bb, m, 'false')};")
                L.append(f"  T hy{bb}_{m} = T(0);")
        for p in range(P):
            b1, b2 = self.path_blocks[p]
            d = self.dout[p]
            L.append("  {")
            for k in range(d):
                L.append(f"    const T g{k} = {self._ld('gout', 'out', p, k, 'OUT_GM')};")
            for (i, j, k, c) in self.cg[p]:
                L.append(f"    hx{b1}_{i} += {_lit(c)} * (y{b2}_{j} * g{k});")
                L.append(f"    hy{b2}_{j} += {_lit(c)} * (x{b1}_{i} * g{k});")
            L.append("  }")
        for bb, d in enumerate(self.d1):
            for m in range(d):
                e3, gm = self._addr("in1", bb, m)
                L.append(f"  g1[IN1_GM ? ({gm}) : ({e3})] = hx{bb}_{m};")
        for bb, d in enumerate(self.d2):
            for m in range(d):
                e3, gm = self._addr("in2", bb, m)
                L.append(f"  g2[{e3}] = hy{bb}_{m};")
        L.append("}")
        return "\n".join(L)

    def emit(self) -> str:
        if self.kind == "uvu":
            return self.emit_uvu_fwd() + "\n\n" + self.emit_uvu_bwd()
        return self.emit_uuu_fwd() + "\n\n" + self.emit_uuu_bwd()


# ------------------------------------------------------------ variant sets ----
def model_variants(Lmax: int, lmax: int, correlation: int) -> List[Variant]:
    """All tensor-product variants one e3nnTACE model with these settings uses
    (cgtp interaction + CgtpACE product, natural parity, one fidelity,
    energy target), mirroring ``base.py:113-360`` irreps bookkeeping."""
    sh = list(range(lmax + 1))
    node_full = list(range(Lmax + 1))
    inter_out = list(range(lmax + 1)) if correlation != 1 else list(range(Lmax + 1))
    vs = [Variant("uvu", [0], sh, inter_out), Variant("uvu", node_full, sh, inter_out)]
    hidden = inter_out
    for last in (False, True):
        in1 = hidden
        for nu in range(2, correlation + 1):
            if nu == correlation:
                out = [0] if last else list(range(Lmax + 1))
            else:
                out = list(range(lmax + 1))
            v = Variant("uuu", in1, hidden, out)
            vs.append(v)
            in1 = [l3 for (_, _, l3) in v.path_l]
    return vs


SUPPORTED = [(1, 1, 2), (1, 1, 3), (2, 2, 2), (2, 2, 3), (3, 3, 2), (3, 3, 3), (2, 3, 3)]


def all_variants() -> List[Variant]:
    seen, out = set(), []
    for (Lm, lm, corr) in SUPPORTED:
        for v in model_variants(Lm, lm, corr):
            if v.key not in seen:
                seen.add(v.key)
                out.append(v)
    return out


# ------------------------------------------------------- spherical harmonics ----
def _sh_polys(lmax: int):
    """e3nn component-normalised real SH as sympy polynomials in (x, y, z)
    (homogeneous of degree l; Y^1 = sqrt(3)(x, y, z), polar axis y)."""
    import sympy as sp

    x, y, z = sp.symbols("x y z")
    s = sp.sqrt
    ys = [[sp.Integer(1)], [s(3) * x, s(3) * y, s(3) * z]]
    y2, x2z2 = y ** 2, x ** 2 + z ** 2
    s2 = [s(15) * x * z, s(15) * x * y, s(5) * (y2 - x2z2 / 2), s(15) * y * z, s(15) / 2 * (z ** 2 - x ** 2)]
    ys.append(s2)
    s3 = [s(42) / 6 * (s2[0] * z + s2[4] * x), s(7) * s2[0] * y, s(168) / 8 * (4 * y2 - x2z2) * x,
          s(7) / 2 * y * (2 * y2 - 3 * x2z2), s(168) / 8 * z * (4 * y2 - x2z2), s(7) * (s2[4] * y),
          s(42) / 6 * (s2[4] * z - s2[0] * x)]
    ys.append(s3)
    assert lmax <= 3
    return (x, y, z), ys[: lmax + 1]


def _poly_code(expr, syms, pw) -> str:
    import sympy as sp

    poly = sp.Poly(sp.expand(expr), *syms)
    terms = []
    for (a, b, c), coef in poly.terms():
        f = []
        if a:
            f.append(pw[("x", a)])
        if b:
            f.append(pw[("y", b)])
        if c:
            f.append(pw[("z", c)])
        mono = " * ".join(f) if f else "T(1)"
        terms.append(f"{_lit(float(coef))} * {mono}")
    return " + ".join(terms) if terms else "T(0)"


def emit_sh(lmax_all: int = 3) -> str:
    """Device functions sh_eval_L<T>(x, y, z, out) and sh_grad_L<T>(x, y, z, g, &dx, &dy, &dz)."""
    import sympy as sp

    L = []
    for lmax in range(0, lmax_all + 1):
        (x, y, z), ys = _sh_polys(lmax)
        pw = {}
        decl = []
        for v in ("x", "y", "z"):
            for k in range(1, 4):
                pw[(v, k)] = f"{v}{k}"
        decl.append("  const T x1 = x, y1 = y, z1 = z, x2 = x * x, y2 = y * y, z2 = z * z, x3 = x2 * x, y3 = y2 * y, z3 = z2 * z;")
        flat = [e for blk in ys for e in blk]
        L.append(f"template <typename T>\n__device__ __forceinline__ void sh_eval_{lmax}(T x, T y, T z, T* __restrict__ o) {{")
        L += decl
        for i, e in enumerate(flat):
            L.append(f"  o[{i}] = {_poly_code(e, (x, y, z), pw)};")
        L.append("}")
        L.append(f"template <typename T>\n__device__ __forceinline__ void sh_grad_{lmax}(T x, T y, T z, const T* __restrict__ g, T& dx, T& dy, T& dz) {{")
        L += decl
        for name, s in (("dx", x), ("dy", y), ("dz", z)):
            parts = []
            for i, e in enumerate(flat):
                de = sp.diff(sp.expand(e), s)
                if de != 0:
                    parts.append(f"g[{i}] * ({_poly_code(de, (x, y, z), pw)})")
            L.append(f"  {name} = {' + '.join(parts) if parts else 'T(0)'};")
        L.append("}")
    return "\n".join(L)


# -------------------------------------------------------------------- main ----
_TYPEDEFS = [
    "typedef void (*UvuFwd)(const void*, const void*, const void*, const int*, const int*, const int*, void*, int, int, int, hipStream_t);",
    "typedef void (*UvuBwd)(const void*, const void*, const void*, const void*, const int*, const int*, const int*, void*, void*, void*, int, int, int, hipStream_t);",
    "typedef void (*UuuFwd)(const void*, const void*, void*, int, int, int, hipStream_t);",
    "typedef void (*UuuBwd)(const void*, const void*, const void*, void*, void*, int, int, int, hipStream_t);",
]


def _launchers(v: Variant) -> List[str]:
    out = []
    for T, tag in (("float", "f"), ("double", "d")):
        if v.kind == "uvu":
            out.append(f"void L_{v.name}_fwd_{tag}(const void* x, const void* y, const void* w, const int* rp, const int* eid, const int* src, void* o, int n, int flags, int C, hipStream_t s) {{")
            out.append("  if (n <= 0) return;")
            for f in (0, 2):
                out.append(f"  if (flags == {f}) hipLaunchKernelGGL((k_{v.name}_fwd<{T}, {'true' if f else 'false'}>), dim3(n), dim3(64), 0, s, (const {T}*)x, (const {T}*)y, (const {T}*)w, rp, eid, src, ({T}*)o, n, C);")
            out.append("}")
            out.append(f"void L_{v.name}_bwd_{tag}(const void* x, const void* y, const void* w, const void* g, const int* rp, const int* eid, const int* src, void* gx, void* gy, void* gw, int n, int flags, int C, hipStream_t s) {{")
            out.append("  if (n <= 0) return;")
            for f in (0, 2):
                for gx in (True, False):
                    out.append(f"  if (flags == {f} && {'gx' if gx else '!gx'}) hipLaunchKernelGGL((k_{v.name}_bwd<{T}, {'true' if gx else 'false'}, {'true' if f else 'false'}>), dim3(n), dim3(64), 0, s, (const {T}*)x, (const {T}*)y, (const {T}*)w, (const {T}*)g, rp, eid, src, ({T}*)gx, ({T}*)gy, ({T}*)gw, n, C);")
            out.append("}")
        else:
            out.append(f"void L_{v.name}_fwd_{tag}(const void* x1, const void* x2, void* o, int n, int C, int flags, hipStream_t s) {{")
            out.append("  const size_t tot = (size_t)n * C; if (tot == 0) return;")
            out.append("  const dim3 g((unsigned)((tot + 255) / 256)), b(256);")
            for f in (0, 2, 3):  # in1 grouped implies out grouped (the product-basis chain)
                out.append(f"  if (flags == {f}) hipLaunchKernelGGL((k_{v.name}_fwd<{T}, {'true' if f & 1 else 'false'}, {'true' if f & 2 else 'false'}>), g, b, 0, s, (const {T}*)x1, (const {T}*)x2, ({T}*)o, n, C);")
            out.append("}")
            out.append(f"void L_{v.name}_bwd_{tag}(const void* x1, const void* x2, const void* go, void* g1, void* g2, int n, int C, int flags, hipStream_t s) {{")
            out.append("  const size_t tot = (size_t)n * C; if (tot == 0) return;")
            out.append("  const dim3 g((unsigned)((tot + 255) / 256)), b(256);")
            for f in (0, 2, 3):
                out.append(f"  if (flags == {f}) hipLaunchKernelGGL((k_{v.name}_bwd<{T}, {'true' if f & 1 else 'false'}, {'true' if f & 2 else 'false'}>), g, b, 0, s, (const {T}*)x1, (const {T}*)x2, (const {T}*)go, ({T}*)g1, ({T}*)g2, n, C);")
            out.append("}")
    return out


def emit_all(gen_dir: str) -> List[str]:
    """Writes gen/sh.inc, gen/registry.inc and one gen/v_<name>.hip per variant
    (compiled as separate translation units).  Returns the .hip paths."""
    os.makedirs(gen_dir, exist_ok=True)
    hdr = "// GENERATED by tace_amd/csrc/codegen.py -- do not edit."
    vs = all_variants()
    _write(os.path.join(gen_dir, "sh.inc"), [hdr, "#pragma once", emit_sh(3)])
    srcs = []
    for v in vs:
        body = [hdr, f"// variant {v.key}: {len(v.paths)} paths, per-channel dims in1={v.D1} in2={v.D2} out={v.DO}",
                '#include "../common.h"', *_TYPEDEFS, v.emit(), "", *_launchers(v)]
        path = os.path.join(gen_dir, f"v_{v.name}.hip")
        _write(path, body)
        srcs.append(path)
    reg = [hdr, "#pragma once", *_TYPEDEFS,
           "struct TpVariant {", "  const char* key; int kind; int npath; int d1; int d2; int dout;",
           "  UvuFwd fwd_f, fwd_d; UvuBwd bwd_f, bwd_d; UuuFwd ufwd_f, ufwd_d; UuuBwd ubwd_f, ubwd_d;", "};"]
    for v in vs:
        if v.kind == "uvu":
            reg += [f"void L_{v.name}_{k}_{t}({sig});" for k, sig in
                    (("fwd", "const void*, const void*, const void*, const int*, const int*, const int*, void*, int, int, int, hipStream_t"),
                     ("bwd", "const void*, const void*, const void*, const void*, const int*, const int*, const int*, void*, void*, void*, int, int, int, hipStream_t"))
                    for t in ("f", "d")]
        else:
            reg += [f"void L_{v.name}_{k}_{t}({sig});" for k, sig in
                    (("fwd", "const void*, const void*, void*, int, int, int, hipStream_t"),
                     ("bwd", "const void*, const void*, const void*, void*, void*, int, int, int, hipStream_t"))
                    for t in ("f", "d")]
    reg.append("static const TpVariant kVariants[] = {")
    for v in vs:
        n = v.name
        if v.kind == "uvu":
            reg.append(f"  {{\"{v.key}\", 0, {len(v.paths)}, {v.D1}, {v.D2}, {v.DO}, L_{n}_fwd_f, L_{n}_fwd_d, L_{n}_bwd_f, L_{n}_bwd_d, nullptr, nullptr, nullptr, nullptr}},")
        else:
            reg.append(f"  {{\"{v.key}\", 1, {len(v.paths)}, {v.D1}, {v.D2}, {v.DO}, nullptr, nullptr, nullptr, nullptr, L_{n}_fwd_f, L_{n}_fwd_d, L_{n}_bwd_f, L_{n}_bwd_d}},")
    reg.append("};")
    reg.append(f"static const int kNumVariants = {len(vs)};")
    _write(os.path.join(gen_dir, "registry.inc"), reg)
    return srcs


def _write(path: str, lines: List[str]) -> None:
    txt = "\n".join(lines) + "\n"
    if os.path.exists(path) and open(path).read() == txt:
        return  # unchanged: keep the mtime so the build can skip the object
    with open(path, "w") as f:
        f.write(txt)


if __name__ == "__main__":
    for p in emit_all(sys.argv[1] if len(sys.argv) > 1 else os.path.join(_HERE, "gen")):
        print(p)
