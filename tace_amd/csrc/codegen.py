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
    def __init__(self, kind: str, in1: Sequence[int], in2: Sequence[int], out: Sequence[int],
                 weighted: bool = False):
        assert kind in ("uvu", "uuu")
        assert not weighted or kind == "uuu"
        self.kind = kind
        self.weighted = weighted  # uuu with per-node path weights (bilinear gate)
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
    def _ld_x(self, node: str, b: int, m: int) -> str:
        e3, gm = self._addr("in1", b, m)
        e3, gm = e3.replace("(size_t)n ", f"(size_t){node} "), gm.replace("(size_t)n ", f"(size_t){node} ")
        return f"(IN1_GM ? x[{gm}] : x[{e3}])"

    def parts(self, cap: int = 40) -> List[List[int]]:
        """Input blocks split into consecutive parts whose paths hold at most
        ``cap`` output components per channel: one kernel per part, so the
        per-lane accumulators / output gradients of a part stay in registers
        at an occupancy of several wavefronts per SIMD.  Parts touch disjoint
        paths, x blocks, weights and outputs (grad_y is accumulated)."""
        out, cur, acc = [], [], 0
        for b in range(len(self.in1)):
            d3 = sum(self.dout[p] for p in range(len(self.paths)) if self.path_blocks[p][0] == b)
            if cur and acc + d3 > cap:
                out.append(cur)
                cur, acc = [], 0
            cur.append(b)
            acc += d3
        if cur:
            out.append(cur)
        return out

    def _part_paths(self, blocks: Sequence[int]) -> List[int]:
        return [p for p in range(len(self.paths)) if self.path_blocks[p][0] in blocks]

    def _block_pairs(self, paths: Sequence[int]):
        """Paths grouped by their (in1 block, in2 block); per group the (i, j)
        products x_i y_j that some path of the group couples."""
        groups = {}
        for p in paths:
            groups.setdefault(self.path_blocks[p], []).append(p)
        out = []
        for (b1, b2), ps in groups.items():
            pairs = sorted({(i, j) for p in ps for (i, j, k, c) in self.cg[p]})
            out.append((b1, b2, ps, pairs))
        return out

    def _edge_pipeline(self, L: List[str], blocks: Sequence[int], paths: Sequence[int]) -> None:
        """Head of the edge loop: the operands of the next edge are loaded
        while the current one is computed (x*, w*, y* hold the current edge;
        xn*, wn*, yn* the next one).  y is uniform over the workgroup."""
        xs = [(b, m) for b in blocks for m in range(self.d1[b])]
        L.append("  int e = beg;")
        L.append("  int ed = e < end ? (eid ? eid[e] : e) : 0;")
        L.append("  int s = e < end ? src[ed] : 0;")
        L.append("  if (map) s = map[s];")
        L.append("  int wr = e < end && wmap ? wmap[ed] : ed;  // weight row of the edge")
        for (b, m) in xs:
            L.append(f"  T x{b}_{m} = T(0);")
        L += [f"  T w{p} = T(0);" for p in paths]
        L += [f"  T y{j} = T(0);" for j in range(self.D2)]
        L.append("  if (e < end) {")
        for (b, m) in xs:
            L.append(f"    x{b}_{m} = {self._ld_x('s', b, m)};")
        L += [f"    w{p} = __builtin_nontemporal_load(&w[(size_t)wr * WW + (size_t){p} * C + u]);" for p in paths]
        L += [f"    y{j} = y[(size_t)ed * {self.D2} + {j}];" for j in range(self.D2)]
        L.append("  }")
        L.append("  for (; e < end; ++e) {")
        L.append("    const int en = e + 1 < end ? e + 1 : e;")
        L.append("    const int edn = eid ? eid[en] : en;")
        L.append("    const int sn = map ? map[src[edn]] : src[edn];")
        L.append("    const int wrn = wmap ? wmap[edn] : edn;")
        for (b, m) in xs:
            L.append(f"    const T xn{b}_{m} = {self._ld_x('sn', b, m)};")
        L += [f"    const T wn{p} = __builtin_nontemporal_load(&w[(size_t)wrn * WW + (size_t){p} * C + u]);" for p in paths]
        L += [f"    const T yn{j} = y[(size_t)edn * {self.D2} + {j}];" for j in range(self.D2)]

    def _edge_rotate(self, L: List[str], blocks: Sequence[int], paths: Sequence[int]) -> None:
        for b in blocks:
            for m in range(self.d1[b]):
                L.append(f"    x{b}_{m} = xn{b}_{m};")
        L += [f"    w{p} = wn{p};" for p in paths]
        L += [f"    y{j} = yn{j};" for j in range(self.D2)]
        L.append("    ed = edn;")
        L.append("    wr = wrn;")
        L.append("  }")

    def emit_uvu_fwd(self, q: int) -> str:
        """Part q of out[n] = sum over edges e -> n of w_e (.) CG(x[src e], y_e):
        the paths of the part's input blocks.  The products x_i y_j are shared
        by the paths of one (in1, in2) block pair."""
        P = len(self.paths)
        blocks = self.parts()[q]
        paths = self._part_paths(blocks)
        L = [f"template <typename T, bool IN1_GM, bool OUT_GM>\n__device__ __forceinline__ void f_{self.name}_fwd{q}(",
             "    const T* __restrict__ x, const T* __restrict__ y, const T* __restrict__ w,",
             "    const int* __restrict__ rowptr, const int* __restrict__ eid, const int* __restrict__ src,",
             "    const int* __restrict__ map, const int* __restrict__ wmap, T* __restrict__ out, int n_nodes, int C,",
             "    int n0) {",
             "  const int u = (int)threadIdx.x;",
             "  if (u >= C) return;",
             "  const int n = map ? map[n0] : n0;  // feature row of the receiver",
             "  const size_t N = (size_t)n_nodes;",
             "  const int beg = rowptr[n0], end = rowptr[n0 + 1];",
             f"  const size_t WW = (size_t)C * {P};"]
        for p in paths:
            L += [f"  T a{self.offo[p] + k} = T(0);" for k in range(self.dout[p])]
        self._edge_pipeline(L, blocks, paths)
        for (b1, b2, ps, pairs) in self._block_pairs(paths):
            o2 = self.off2[b2]
            L.append("    {")
            for (i, j) in pairs:
                L.append(f"      const T q{i}_{j} = x{b1}_{i} * y{o2 + j};")
            for p in ps:
                byk = {}
                for (i, j, k, c) in self.cg[p]:
                    byk.setdefault(k, []).append((i, j, c))
                for k in range(self.dout[p]):
                    if k in byk:
                        t = " + ".join(f"{_lit(c)} * q{i}_{j}" for i, j, c in byk[k])
                        L.append(f"      a{self.offo[p] + k} += w{p} * ({t});")
            L.append("    }")
        self._edge_rotate(L, blocks, paths)
        for p in paths:
            for k in range(self.dout[p]):
                e3, gm = self._addr("out", p, k)
                L.append(f"  out[OUT_GM ? ({gm}) : ({e3})] = a{self.offo[p] + k};")
        L.append("}")
        return "\n".join(L)

    def emit_uvu_bwd(self, q: int) -> str:
        """Part q (paths of the part's input blocks).  Per edge e (slot of
        receiver n, sender s), channel u, path p:
          psi_i   = sum_{j,k} c^p_ijk y_j g_pk         (g = grad of out[n])
          gw_p    = sum_i x_i psi_i
          hx_i   += w_p psi_i                            -> cbuf row of slot e
          hy_j   += sum_{i,k} c^p_ijk x_i (w_p g_pk)     -> summed over channels
        A workgroup is one wavefront: channel group ``cg`` (channels 64 cg ..
        64 cg + 63) of one receiver and part.  grad_y is reduced over its 64
        lanes (transposing butterfly, 17 shuffles for 16 values) into the
        (part, channel group) partial ``gy`` points at; ``k_sum_parts`` adds
        the partials in a fixed order: deterministic, no atomics and no
        barrier inside the edge loop."""
        P = len(self.paths)
        blocks = self.parts()[q]
        paths = self._part_paths(blocks)
        assert self.D2 <= 16
        L = [f"template <typename T, bool NEED_GX, bool IN1_GM, bool OUT_GM>\n__device__ __forceinline__ void f_{self.name}_bwd{q}(",
             "    const T* __restrict__ x, const T* __restrict__ y, const T* __restrict__ w,",
             "    const T* __restrict__ gout,",
             "    const int* __restrict__ rowptr, const int* __restrict__ eid, const int* __restrict__ src,",
             "    const int* __restrict__ map, const int* __restrict__ wmap, T* __restrict__ cbuf, T* __restrict__ gy,",
             "    T* __restrict__ gw, int n_nodes, int C, int n0, int cg) {",
             "  const int n = map ? map[n0] : n0;  // feature row of the receiver",
             "  const int lane = (int)threadIdx.x & 63;",
             "  const bool act = 64 * cg + lane < C;",
             "  const int u = act ? 64 * cg + lane : C - 1;  // this lane's channel",
             "  const size_t N = (size_t)n_nodes;",
             "  const int beg = rowptr[n0], end = rowptr[n0 + 1];",
             f"  const size_t WW = (size_t)C * {P}, DX = (size_t)C * {self.D1};"]
        for p in paths:
            for k in range(self.dout[p]):
                e3, gm = self._addr("out", p, k)
                # lanes past C contribute nothing: their grad_out is zero
                L.append(f"  const T g{self.offo[p] + k} = act ? gout[OUT_GM ? ({gm}) : ({e3})] : T(0);")
        self._edge_pipeline(L, blocks, paths)
        for b in blocks:
            for m in range(self.d1[b]):
                L.append(f"    T hx{b}_{m} = T(0);")
        L += [f"    T hy{j} = T(0);" for j in range(16)]
        for p in paths:
            b1, b2 = self.path_blocks[p]
            o, o2 = self.offo[p], self.off2[b2]
            L.append("    {")
            byjk, byik = {}, {}
            for (i, j, k, c) in self.cg[p]:
                byjk.setdefault((j, k), []).append((i, c))
                byik.setdefault((i, k), []).append((j, c))
            used_i = sorted({i for (i, j, k, c) in self.cg[p]})
            L += [f"      T psi{i} = T(0);" for i in used_i]
            for (j, k), ic in sorted(byjk.items()):
                L.append(f"      {{ const T r = y{o2 + j} * g{o + k};")
                L += [f"        psi{i} += {_lit(c)} * r;" for i, c in ic]
                L.append("      }")
            L.append(f"      if (act) __builtin_nontemporal_store("
                     f"{' + '.join(f'x{b1}_{i} * psi{i}' for i in used_i)}, &gw[(size_t)ed * WW + (size_t){p} * C + u]);")
            L.append("      if (NEED_GX) {")
            L += [f"        hx{b1}_{i} += w{p} * psi{i};" for i in used_i]
            L.append("      }")
            used_k = sorted({k for (i, j, k, c) in self.cg[p]})
            L += [f"      const T a{k} = w{p} * g{o + k};" for k in used_k]
            for (i, k), jc in sorted(byik.items()):
                L.append(f"      {{ const T z = x{b1}_{i} * a{k};")
                L += [f"        hy{o2 + j} += {_lit(c)} * z;" for j, c in jc]
                L.append("      }")
            L.append("    }")
        L.append("    if (NEED_GX && act) {")
        L.append("      T* __restrict__ cb = cbuf + (size_t)e * DX;")
        for b in blocks:
            for m in range(self.d1[b]):
                e3, gm = self._row_addr(b, m)
                L.append(f"      __builtin_nontemporal_store(hx{b}_{m}, &cb[IN1_GM ? ({gm}) : ({e3})]);")
        L.append("    }")
        L.append("    const T v = reduce16_lanes(hy0, hy1, hy2, hy3, hy4, hy5, hy6, hy7, hy8, hy9, hy10, hy11, hy12, hy13, hy14, hy15);")
        L.append("    const int jj = rev4(lane);")
        L.append(f"    if (lane < 16 && jj < {self.D2}) gy[(size_t)ed * {self.D2} + jj] = v;")
        self._edge_rotate(L, blocks, paths)
        L.append("}")
        return "\n".join(L)

    def emit_uvu_wrappers(self) -> str:
        """One launch runs every part: the workgroups of one receiver's parts
        are neighbours on the same XCD (tp_part_node), so memory-heavy and
        compute-heavy parts share the CUs instead of running one after the
        other.  The backward runs a wavefront per (part q, channel group cg)
        that writes grad_y partial q * ceil(C / 64) + cg."""
        nq = len(self.parts())
        a_f = "x, y, w, rowptr, eid, src, map, wmap, out, n_nodes, C, n0"
        a_b = ("x, y, w, gout, rowptr, eid, src, map, wmap, cbuf, gy + (size_t)(q * ncg + cg) * n_edges * %d, gw, "
               "n_nodes, C, n0, cg" % self.D2)
        L = [f"template <typename T, bool IN1_GM, bool OUT_GM>\n__global__ __launch_bounds__(512) void k_{self.name}_fwd(",
             "    const T* __restrict__ x, const T* __restrict__ y, const T* __restrict__ w,",
             "    const int* __restrict__ rowptr, const int* __restrict__ eid, const int* __restrict__ src,",
             "    const int* __restrict__ map, const int* __restrict__ wmap, T* __restrict__ out, int n_nodes, int C) {",
             "  int q;",
             f"  const int n0 = tp_part_node(n_nodes, {nq}, &q);",
             "  if (n0 < 0) return;"]
        for q in range(nq):
            L.append(f"  {'if' if q == 0 else 'else if'} (q == {q}) f_{self.name}_fwd{q}<T, IN1_GM, OUT_GM>({a_f});")
        L.append("}")
        L += [f"template <typename T, bool NEED_GX, bool IN1_GM, bool OUT_GM>\n__global__ __launch_bounds__(512) void k_{self.name}_bwd(",
              "    const T* __restrict__ x, const T* __restrict__ y, const T* __restrict__ w,",
              "    const T* __restrict__ gout,",
              "    const int* __restrict__ rowptr, const int* __restrict__ eid, const int* __restrict__ src,",
              "    const int* __restrict__ map, const int* __restrict__ wmap, T* __restrict__ cbuf, T* __restrict__ gy,",
              "    T* __restrict__ gw, int n_nodes, int n_edges, int C) {",
              "  // one wavefront per (receiver, part, channel group of 64)",
              "  const int ncg = (C + 63) >> 6;",
              "  int q;",
              f"  const int n0 = tp_part_node(n_nodes, {nq} * ncg, &q);",
              "  if (n0 < 0) return;",
              "  const int cg = q % ncg;",
              "  q /= ncg;"]
        for q in range(nq):
            L.append(f"  {'if' if q == 0 else 'else if'} (q == {q}) f_{self.name}_bwd{q}<T, NEED_GX, IN1_GM, OUT_GM>({a_b});")
        L.append("}")
        return "\n".join(L)

    # ------------------------------------------------- radial-fused uvu ----
    # The same products with the radial MLP's last layer folded in: the
    # per-edge weights w[e, p, u] = alpha sum_k h[e, k] Wl[k, p C + u] (64
    # hidden features, fp32) are made on MFMA inside the kernel and never go
    # through HBM.  A workgroup of 8 wavefronts owns 64 channels of one part
    # and walks the 16-edge blocks of a range of receivers; its wavefronts
    # split the work by unit, so matrix cores and vector ALUs run side by side
    # on every SIMD:
    #  * producers (wavefronts 0-3): wavefront v makes the weights of channels
    #    16 v .. 16 v + 15 for the 16 edges of block k + 1
    #    (v_mfma_f32_16x16x4f32; the B fragments of Wl stay in registers for
    #    the workgroup's life) into an LDS tile [16][P][64], and stages the
    #    block's y rows;
    #  * consumers (wavefronts 4-7): wavefront 4 + v takes edges 4 v .. 4 v + 3
    #    of block k with one lane per channel, as the unfused kernels do --
    #    edge ids, senders and y are uniform over the wavefront, x rows are
    #    read 256 bytes at a time (prefetched one block ahead) and the weights
    #    come from the tile.
    # Tiles are double-buffered: one barrier per block.  One part per in1
    # block, with all of the block's paths, so a grad-x row block comes from
    # one part.
    def rtp_parts(self) -> List[int]:
        return [b for b in range(len(self.in1)) if any(pb[0] == b for pb in self.path_blocks)]

    def _rtp_signature(self, kind: str, q: int) -> List[str]:
        if kind == "fwd":
            return [f"template <bool IN1_GM, bool OUT_GM>\n__device__ __forceinline__ void f_{self.name}_rfwd{q}(",
                    "    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ h,",
                    "    const float* __restrict__ Wl, float alpha,",
                    "    const int* __restrict__ rowptr, const int* __restrict__ eid, const int* __restrict__ src,",
                    "    const int* __restrict__ map, const int* __restrict__ srow, float* __restrict__ out,",
                    "    int n_nodes, int C, int n_begin, int n_end, int c0, float* __restrict__ tile,",
                    "    float* __restrict__ ytile, float* __restrict__ red) {"]
        return [f"template <bool NEED_GX, bool IN1_GM, bool OUT_GM>\n__device__ __forceinline__ void f_{self.name}_rbwd{q}(",
                "    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ h,",
                "    const float* __restrict__ Wl, float alpha, const float* __restrict__ gout,",
                "    const int* __restrict__ rowptr, const int* __restrict__ eid, const int* __restrict__ src,",
                "    const int* __restrict__ map, const int* __restrict__ srow, float* __restrict__ cbuf,",
                "    float* __restrict__ gy, float* __restrict__ gw, int n_nodes, int C, int n_begin, int n_end,",
                "    int c0, float* __restrict__ tile, float* __restrict__ ytile) {"]

    def _rtp_head(self, L: List[str], paths: Sequence[int]) -> None:
        P = len(paths)
        L += [f"  constexpr int RTP_ROW = {P * 64}, RTP_TILE = 16 * RTP_ROW;",
              "  typedef float T;",
              "  const int lane = (int)threadIdx.x & 63;",
              "  const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);",
              "  const bool prod = wv < 4;",
              "  const int cw = prod ? wv : wv - 4;  // producer: channel group; consumer: edge group",
              "  const int lrow = lane & 15, lgrp = lane >> 4;",
              "  const int u = c0 + lane;  // consumer lane's channel",
              "  const size_t N = (size_t)n_nodes;",
              f"  const size_t WW = (size_t)C * {len(self.paths)};",
              f"  float wf[{P}][16];",
              "  if (prod) {"]
        for pi, p in enumerate(paths):
            L.append("#pragma unroll")
            L.append(f"    for (int s = 0; s < 16; ++s) wf[{pi}][s] = "
                     f"Wl[(size_t)(16 * lgrp + s) * WW + (size_t){p} * C + c0 + 16 * cw + lrow];")
        L.append("  }")

    def _rtp_load(self, L: List[str], cur: str, av: str, yv: str, ind: str) -> None:
        """Producer: A fragment (h rows) and this thread's y value of block `cur`."""
        L += [f"{ind}{{",
              f"{ind}  const int ea = {cur}.b0 + lrow;",
              f"{ind}  const bool oka = ea < {cur}.end;",
              f"{ind}  rtp_a_frag(h, oka ? (eid ? eid[ea] : ea) : 0, oka, lgrp, {av});",
              f"{ind}  const int t = (int)threadIdx.x, ey = {cur}.b0 + (t >> 4), jy = t & 15;",
              f"{ind}  {yv} = ey < {cur}.end && jy < {self.D2} ? y[(size_t)(eid ? eid[ey] : ey) * {self.D2} + jy] : 0.0f;",
              f"{ind}}}"]

    def _rtp_produce(self, L: List[str], paths: Sequence[int], buf: str, av: str, yv: str, ind: str) -> None:
        """Producer: weights of the block whose A fragment is `av` into tile
        buffer `buf`; its y values (`yv`, one per thread) into ytile."""
        P = len(paths)
        L += [f"{ind}{{",
              f"{ind}  float* __restrict__ tb = tile + ({buf}) * RTP_TILE;",
              f"{ind}  ytile[({buf}) * 256 + (int)threadIdx.x] = {yv};",
              f"{ind}  rtp_f4 acc[{P}];"]
        for pi in range(P):
            L.append(f"{ind}  acc[{pi}] = rtp_f4{{0.0f, 0.0f, 0.0f, 0.0f}};")
        L.append("#pragma unroll")
        L.append(f"{ind}  for (int s = 0; s < 16; ++s) {{")
        for pi in range(P):
            L.append(f"{ind}    acc[{pi}] = __builtin_amdgcn_mfma_f32_16x16x4f32({av}[s], wf[{pi}][s], acc[{pi}], 0, 0, 0);")
        L.append(f"{ind}  }}")
        L.append("#pragma unroll")
        L.append(f"{ind}  for (int r = 0; r < 4; ++r) {{")
        for pi in range(P):
            L.append(f"{ind}    tb[(4 * lgrp + r) * RTP_ROW + {pi * 64} + 16 * cw + lrow] = alpha * acc[{pi}][r];")
        L.append(f"{ind}  }}")
        L.append(f"{ind}}}")

    def _rtp_xload(self, L: List[str], b: int, cur: str, pre: str, ind: str, decl: bool) -> None:
        """Consumer: x rows of its 4 edges of block `cur` into registers {pre}{rr}_{m}."""
        for rr in range(4):
            L.append(f"{ind}{{")
            L.append(f"{ind}  const int e = {cur}.b0 + 4 * cw + {rr};")
            L.append(f"{ind}  const int s = e < {cur}.end ? srow[e] : -1;")
            for m in range(self.d1[b]):
                L.append(f"{ind}  {pre}{rr}_{m} = s >= 0 ? {self._ld_x('s', b, m)} : T(0);")
            L.append(f"{ind}}}")

    def _rtp_edge_operands(self, L: List[str], b: int, paths: Sequence[int], rr: int) -> None:
        used_y = sorted({self.off2[self.path_blocks[p][1]] + j for p in paths for (_, j, _, _) in self.cg[p]})
        L += [f"          const int e = cur.b0 + 4 * cw + {rr};",
              "          const int ed = eid ? eid[e] : e;"]
        for m in range(self.d1[b]):
            L.append(f"          const T x{b}_{m} = xc{rr}_{m};")
        for j in used_y:
            L.append(f"          const T y{j} = yb[(e - cur.b0) * 16 + {j}];")
        L.append("          const float* __restrict__ wrow = tb + (e - cur.b0) * RTP_ROW + lane;")
        for pi, p in enumerate(paths):
            L.append(f"          const T w{p} = wrow[{pi * 64}];")

    def _rtp_fwd_edge(self, L: List[str], paths: Sequence[int]) -> None:
        for (b1, b2, ps, pairs) in self._block_pairs(paths):
            o2 = self.off2[b2]
            L.append("          {")
            for (i, j) in pairs:
                L.append(f"            const T q{i}_{j} = x{b1}_{i} * y{o2 + j};")
            for p in ps:
                byk = {}
                for (i, j, k, c) in self.cg[p]:
                    byk.setdefault(k, []).append((i, j, c))
                for k in range(self.dout[p]):
                    if k in byk:
                        t = " + ".join(f"{_lit(c)} * q{i}_{j}" for i, j, c in byk[k])
                        L.append(f"            a{self.offo[p] + k} += w{p} * ({t});")
            L.append("          }")

    def _rtp_bwd_edge(self, L: List[str], b: int, paths: Sequence[int]) -> None:
        for m in range(self.d1[b]):
            L.append(f"          T hx{b}_{m} = T(0);")
        L += [f"          T hy{j} = T(0);" for j in range(16)]
        for p in paths:
            b1, b2 = self.path_blocks[p]
            o, o2 = self.offo[p], self.off2[b2]
            L.append("          {")
            byjk, byik = {}, {}
            for (i, j, k, c) in self.cg[p]:
                byjk.setdefault((j, k), []).append((i, c))
                byik.setdefault((i, k), []).append((j, c))
            used_i = sorted({i for (i, j, k, c) in self.cg[p]})
            L += [f"            T psi{i} = T(0);" for i in used_i]
            for (j, k), ic in sorted(byjk.items()):
                L.append(f"            {{ const T t = y{o2 + j} * g{o + k};")
                L += [f"              psi{i} += {_lit(c)} * t;" for i, c in ic]
                L.append("            }")
            L.append(f"            __builtin_nontemporal_store("
                     f"{' + '.join(f'x{b1}_{i} * psi{i}' for i in used_i)}, &gw[(size_t)ed * WW + (size_t){p} * C + u]);")
            L.append("            if (NEED_GX) {")
            L += [f"              hx{b1}_{i} += w{p} * psi{i};" for i in used_i]
            L.append("            }")
            used_k = sorted({k for (i, j, k, c) in self.cg[p]})
            L += [f"            const T a{k} = w{p} * g{o + k};" for k in used_k]
            for (i, k), jc in sorted(byik.items()):
                L.append(f"            {{ const T z = x{b1}_{i} * a{k};")
                L += [f"              hy{o2 + j} += {_lit(c)} * z;" for j, c in jc]
                L.append("            }")
            L.append("          }")
        L.append("          if (NEED_GX) {")
        L.append("            float* __restrict__ cb = cbuf + (size_t)e * DX;")
        for m in range(self.d1[b]):
            e3, gm = self._row_addr(b, m)
            L.append(f"            __builtin_nontemporal_store(hx{b}_{m}, &cb[IN1_GM ? ({gm}) : ({e3})]);")
        L.append("          }")
        L.append("          const T v = reduce16_lanes(hy0, hy1, hy2, hy3, hy4, hy5, hy6, hy7, hy8, hy9, hy10, hy11, "
                 "hy12, hy13, hy14, hy15);")
        L.append("          const int jj = rev4(lane);")
        L.append(f"          if (lane < 16 && jj < {self.D2}) gy[(size_t)ed * {self.D2} + jj] = v;")

    def _rtp_out_store(self, L: List[str], paths: Sequence[int], ind: str, node: str, val) -> None:
        accs = [self.offo[p] + k for p in paths for k in range(self.dout[p])]
        for idx, k in enumerate(accs):
            p = next(pp for pp in paths if self.offo[pp] <= k < self.offo[pp] + self.dout[pp])
            e3, gm = self._addr("out", p, k - self.offo[p])
            e3, gm = e3.replace("(size_t)n ", f"(size_t){node} "), gm.replace("(size_t)n ", f"(size_t){node} ")
            L.append(f"{ind}out[OUT_GM ? ({gm}) : ({e3})] = {val(idx, k)};")

    def _rtp_body(self, L: List[str], b: int, paths: Sequence[int], kind: str) -> None:
        """Producer and consumer loops over the same block sequence, one
        barrier per block in each (the wavefronts of a role never run the
        other role's loop, so the two keep separate registers)."""
        accs = [self.offo[p] + k for p in paths for k in range(self.dout[p])]
        NA = len(accs)
        red_sum = lambda idx, k: (f"rb[{idx} * 64 + lane] + rb[({NA} + {idx}) * 64 + lane] + "
                                  f"rb[({2 * NA} + {idx}) * 64 + lane] + rb[({3 * NA} + {idx}) * 64 + lane]")
        if kind == "fwd":
            # receivers without edges: zeros (no block visits them)
            L.append("  if (!prod) {")
            L.append("    for (int n0 = n_begin + cw; n0 < n_end; n0 += 4) {")
            L.append("      if (rowptr[n0] == rowptr[n0 + 1]) {")
            L.append("        const int nz = map ? map[n0] : n0;")
            self._rtp_out_store(L, paths, "        ", "nz", lambda idx, k: "0.0f")
            L.append("      }")
            L.append("    }")
            L.append("  }")
        L.append("  RtpCur cur;")
        L.append("  if (!rtp_seek(cur, rowptr, n_begin, n_end)) return;")
        L.append("  RtpCur nxt = cur;")
        # ---- producers: the operands of block k + 2 are loaded while the
        # MFMAs of block k + 1 run
        L.append("  if (prod) {")
        L.append("    float av[16], an[16], yv = 0.0f, yn = 0.0f;")
        self._rtp_load(L, "cur", "av", "yv", "    ")
        L.append("    bool m1 = rtp_next(nxt, rowptr, n_end);  // nxt = block 1")
        L.append("    if (m1) {")
        self._rtp_load(L, "nxt", "an", "yn", "      ")
        L.append("    }")
        self._rtp_produce(L, paths, "0", "av", "yv", "    ")
        L.append("    __syncthreads();")
        L.append("    for (int k = 0;; ++k) {")
        L.append("      const bool more = m1;  // block k + 1 exists")
        L.append("      if (more) {")
        L.append("#pragma unroll")
        L.append("        for (int s = 0; s < 16; ++s) av[s] = an[s];")
        L.append("        yv = yn;")
        L.append("        m1 = rtp_next(nxt, rowptr, n_end);  // nxt = block k + 2")
        L.append("        if (m1) {")
        self._rtp_load(L, "nxt", "an", "yn", "          ")
        L.append("        }")
        self._rtp_produce(L, paths, "(k + 1) & 1", "av", "yv", "        ")
        L.append("      }")
        L.append("      __syncthreads();")
        L.append("      if (!more) break;")
        L.append("    }")
        L.append("    return;")
        L.append("  }")
        # ---- consumers
        for rr in range(4):
            for m in range(self.d1[b]):
                L.append(f"  T xc{rr}_{m} = T(0), xn{rr}_{m} = T(0);")
        self._rtp_xload(L, b, "cur", "xc", "  ", False)
        if kind == "fwd":
            L += [f"  T a{k} = T(0);" for k in accs]
            L.append("  int rp = 0, pend_n = -1;  // receiver whose 4 partial sums wait in red[rp ^ 1]")
        else:
            for p in paths:
                for k in range(self.dout[p]):
                    L.append(f"  T g{self.offo[p] + k} = T(0);")
        L.append("  __syncthreads();")
        L.append("  for (int k = 0;; ++k) {")
        L.append("    const bool more = rtp_next(nxt, rowptr, n_end);  // nxt = block k + 1")
        L.append("    const float* __restrict__ tb = tile + (k & 1) * RTP_TILE;")
        L.append("    const float* __restrict__ yb = ytile + (k & 1) * 256;")
        L.append("    const int n = map ? map[cur.n0] : cur.n0;  // feature row of the receiver")
        if kind == "fwd":
            # the previous receiver's totals, summed in a fixed order
            L.append("    if (pend_n >= 0) {")
            L.append("      const float* __restrict__ rb = red + (rp ^ 1) * " + str(4 * NA * 64) + ";")
            L.append("      if (cw == 0) {")
            self._rtp_out_store(L, paths, "        ", "pend_n", red_sum)
            L.append("      }")
            L.append("      pend_n = -1;")
            L.append("    }")
        else:
            L.append("    if (cur.b0 == cur.beg) {  // first block of the receiver: its output gradient")
            for p in paths:
                for k in range(self.dout[p]):
                    e3, gm = self._addr("out", p, k)
                    L.append(f"      g{self.offo[p] + k} = gout[OUT_GM ? ({gm}) : ({e3})];")
            L.append("    }")
        L.append("    if (more) {")
        self._rtp_xload(L, b, "nxt", "xn", "      ", False)
        L.append("    }")
        for rr in range(4):
            L.append(f"    if (cur.b0 + 4 * cw + {rr} < cur.end) {{")
            L.append("        {")
            self._rtp_edge_operands(L, b, paths, rr)
            if kind == "fwd":
                self._rtp_fwd_edge(L, paths)
            else:
                self._rtp_bwd_edge(L, b, paths)
            L.append("        }")
            L.append("    }")
        if kind == "fwd":
            L.append("    if (cur.b0 + 16 >= cur.end) {  // last block of the receiver: partial sums -> red")
            L.append("      float* __restrict__ rb = red + rp * " + str(4 * NA * 64) + ";")
            for idx, k in enumerate(accs):
                L.append(f"      rb[({NA} * cw + {idx}) * 64 + lane] = a{k};")
                L.append(f"      a{k} = T(0);")
            L.append("      pend_n = n;")
            L.append("      rp ^= 1;")
            L.append("    }")
        for rr in range(4):
            for m in range(self.d1[b]):
                L.append(f"    xc{rr}_{m} = xn{rr}_{m};")
        L.append("    __syncthreads();")
        L.append("    if (!more) break;")
        L.append("    cur = nxt;")
        L.append("  }")
        if kind == "fwd":
            L.append("  if (pend_n >= 0 && cw == 0) {")
            L.append("    const float* __restrict__ rb = red + (rp ^ 1) * " + str(4 * NA * 64) + ";")
            self._rtp_out_store(L, paths, "    ", "pend_n", red_sum)
            L.append("  }")

    def emit_rtp_fwd(self, b: int) -> str:
        paths = self._part_paths([b])
        L = self._rtp_signature("fwd", self.rtp_parts().index(b))
        self._rtp_head(L, paths)
        self._rtp_body(L, b, paths, "fwd")
        L.append("}")
        return "\n".join(L)

    def emit_rtp_bwd(self, b: int) -> str:
        """Part of in1 block b: per edge e (slot of receiver n), channel u and
        path p, with g = grad of out[n] and w from the MFMA tile,
          psi_i = sum_{j,k} c^p_ijk y_j g_pk,  gw_p = sum_i x_i psi_i,
          hx_i += w_p psi_i  (-> cbuf row of slot e),
          hy_j += sum_{i,k} c^p_ijk x_i (w_p g_pk)  (summed over the
        wavefront's 64 channels into this slot's grad_y partial)."""
        paths = self._part_paths([b])
        L = self._rtp_signature("bwd", self.rtp_parts().index(b))
        self._rtp_head(L, paths)
        L.append(f"  const size_t DX = (size_t)C * {self.D1};")
        self._rtp_body(L, b, paths, "bwd")
        L.append("}")
        return "\n".join(L)

    def _rtp_lds(self) -> Tuple[int, int]:
        """(tile floats, red floats) of the largest part: two tile buffers; two
        buffers of the 4 consumers' partial sums."""
        tiles, reds = [], []
        for b in self.rtp_parts():
            ps = self._part_paths([b])
            tiles.append(2 * 16 * 64 * len(ps))
            reds.append(2 * 4 * 64 * sum(self.dout[p] for p in ps))
        return max(tiles), max(reds)

    def emit_rtp_wrappers(self) -> str:
        parts = self.rtp_parts()
        nq = len(parts)
        nt, nr = self._rtp_lds()
        a_f = "x, y, h, Wl, alpha, rowptr, eid, src, map, srow, out, n_nodes, C, nb, ne, c0, tile, ytile, red"
        a_b = "x, y, h, Wl, alpha, gout, rowptr, eid, src, map, srow, cbuf, gy, gw, n_nodes, C, nb, ne, c0, tile, ytile"
        head = ["  int ph, nb, ne;",
                f"  if (!rtp_slot(n_nodes, {nq} * (C >> 6), per_range, &ph, &nb, &ne)) return;",
                f"  const int q = ph % {nq}, c0 = (ph / {nq}) * 64;"]
        L = [f"template <bool IN1_GM, bool OUT_GM>\n__global__ __launch_bounds__(512) RTP_OCC void k_{self.name}_rfwd(",
             "    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ h,",
             "    const float* __restrict__ Wl, float alpha,",
             "    const int* __restrict__ rowptr, const int* __restrict__ eid, const int* __restrict__ src,",
             "    const int* __restrict__ map, const int* __restrict__ srow, float* __restrict__ out, int n_nodes,",
             "    int C, int per_range) {",
             f"  __shared__ float tile[{nt}];",
             "  __shared__ float ytile[512];",
             f"  __shared__ float red[{nr}];"]
        L += head
        for qq in range(nq):
            L.append(f"  {'if' if qq == 0 else 'else if'} (q == {qq}) f_{self.name}_rfwd{qq}<IN1_GM, OUT_GM>({a_f});")
        L.append("}")
        L += [f"template <bool NEED_GX, bool IN1_GM, bool OUT_GM>\n__global__ __launch_bounds__(512) RTP_OCC void k_{self.name}_rbwd(",
              "    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ h,",
              "    const float* __restrict__ Wl, float alpha, const float* __restrict__ gout,",
              "    const int* __restrict__ rowptr, const int* __restrict__ eid, const int* __restrict__ src,",
              "    const int* __restrict__ map, const int* __restrict__ srow, float* __restrict__ cbuf,",
              "    float* __restrict__ gyp, float* __restrict__ gw, int n_nodes, int n_edges, int C, int per_range) {",
              f"  __shared__ float tile[{nt}];",
              "  __shared__ float ytile[512];"]
        L += head
        L.append(f"  float* __restrict__ gy = gyp + (size_t)ph * n_edges * {self.D2};")
        for qq in range(nq):
            L.append(f"  {'if' if qq == 0 else 'else if'} (q == {qq}) f_{self.name}_rbwd{qq}<NEED_GX, IN1_GM, OUT_GM>({a_b});")
        L.append("}")
        return "\n".join(L)

    def _row_addr(self, b: int, m: int) -> Tuple[str, str]:
        """Position of (block b, component m, channel u) inside one grad-x row
        of C*D1 values: e3nn order, or group-major order within the row (each
        group g of count blocks is a [(2l+1), count*C] matrix at C*goff_g)."""
        d = self.d1[b]
        e3 = f"(size_t)C * {self.off1[b]} + (size_t)u * {d} + {m}"
        blk, grp = self._groups(self.in1)
        g, j = blk[b]
        l, cnt, goff = grp[g]
        gm = f"(size_t)C * {goff} + ((size_t){m} * {cnt} + {j}) * C + u"
        return e3, gm

    def row_segments(self):
        """Group-major grad-x rows: per group (row offset / C, length / C) --
        a node's group g lives at N*C*goff_g + node*len_g in the batch layout."""
        _, grp = self._groups(self.in1)
        return [(goff, (2 * l + 1) * cnt) for (l, cnt, goff) in grp]

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
        L.append(f"template <typename T, bool IN1_GM, bool OUT_GM, bool IN2_GM>\n__global__ __launch_bounds__(256) void k_{self.name}_fwd(")
        L.append("    const T* __restrict__ x1, const T* __restrict__ x2, const T* __restrict__ w, T* __restrict__ out,")
        L.append("    int n_nodes, int C) {")
        L.append("  const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;")
        L.append("  const size_t n = t / (size_t)C; const int u = (int)(t % (size_t)C);")
        L.append("  const size_t N = (size_t)n_nodes;")
        L.append("  if (n >= N) return;")
        for bb, d in enumerate(self.d1):
            for m in range(d):
                L.append(f"  const T x{bb}_{m} = {self._ld('x1', 'in1', bb, m, 'IN1_GM')};")
        for bb, d in enumerate(self.d2):
            for m in range(d):
                L.append(f"  const T y{bb}_{m} = {self._ld('x2', 'in2', bb, m, 'IN2_GM')};")
        # weighted variants: per-node path weights w [N, P*C] (bilinear gate)
        if self.weighted:
            L.append(f"  const T* __restrict__ wn = w + n * {P} * (size_t)C + u;")
        for p in range(P):
            b1, b2 = self.path_blocks[p]
            d = self.dout[p]
            L.append(f"  {{ const T wp = {f'wn[(size_t){p} * C]' if self.weighted else 'T(1)'};")
            for k in range(d):
                terms = [f"{_lit(c)} * (x{b1}_{i} * y{b2}_{j})" for (i, j, kk, c) in self.cg[p] if kk == k]
                e3, gm = self._addr("out", p, k)
                val = f"({' + '.join(terms) if terms else 'T(0)'})"
                L.append(f"    out[OUT_GM ? ({gm}) : ({e3})] = {'wp * ' + val if self.weighted else val};")
            L.append("  }")
        L.append("}")
        return "\n".join(L)

    def uuu_parts(self, cap: int = 40) -> List[List[int]]:
        """in1 blocks split into consecutive parts of at most ``cap`` x
        components per channel (one block per part at least): the backward
        runs one part per thread so that x, grad_x and the part's output
        gradients fit in registers at several wavefronts per SIMD.  A part owns
        its blocks' grad_x rows; grad_x2 is summed over the parts' partials.
        Products with few output components (<= 128 per channel) stay whole:
        their registers fit, and the parts would only re-read x2."""
        if self.DO <= 128:
            return [[b for b in range(len(self.in1)) if any(pb[0] == b for pb in self.path_blocks)]]
        out, cur, acc = [], [], 0
        for b in range(len(self.in1)):
            if not any(pb[0] == b for pb in self.path_blocks):
                continue
            if cur and acc + self.d1[b] > cap:
                out.append(cur)
                cur, acc = [], 0
            cur.append(b)
            acc += self.d1[b]
        if cur:
            out.append(cur)
        return out

    def emit_uuu_bwd(self) -> str:
        P = len(self.paths)
        parts = self.uuu_parts()
        nq = len(parts)
        L = []
        for q, blocks in enumerate(parts):
            L.append(f"template <typename T, bool IN1_GM, bool OUT_GM, bool IN2_GM>\n__device__ __forceinline__ void f_{self.name}_bwd{q}(")
            L.append("    const T* __restrict__ x1, const T* __restrict__ x2, const T* __restrict__ w,")
            L.append("    const T* __restrict__ gout, T* __restrict__ g1, T* __restrict__ g2, T* __restrict__ gw,")
            L.append("    size_t n, int u, size_t N, int C) {")
            for bb in blocks:
                for m in range(self.d1[bb]):
                    L.append(f"  const T x{bb}_{m} = {self._ld('x1', 'in1', bb, m, 'IN1_GM')};")
                    L.append(f"  T hx{bb}_{m} = T(0);")
            for bb, d in enumerate(self.d2):
                for m in range(d):
                    L.append(f"  const T y{bb}_{m} = {self._ld('x2', 'in2', bb, m, 'IN2_GM')};")
                    L.append(f"  T hy{bb}_{m} = T(0);")
            if self.weighted:
                L.append(f"  const size_t wo = n * {P} * (size_t)C + u;")
            for p in range(P):
                b1, b2 = self.path_blocks[p]
                if b1 not in blocks:
                    continue
                d = self.dout[p]
                L.append("  {")
                for k in range(d):
                    L.append(f"    const T o{k} = {self._ld('gout', 'out', p, k, 'OUT_GM')};")
                if self.weighted:
                    # grad of the weight: sum_k gout_k t_k with t the unweighted path output
                    L.append("    if (gw) {")
                    tsum = []
                    for k in range(d):
                        terms = [f"{_lit(c)} * (x{b1}_{i} * y{b2}_{j})" for (i, j, kk, c) in self.cg[p] if kk == k]
                        if terms:
                            tsum.append(f"o{k} * ({' + '.join(terms)})")
                    L.append(f"      gw[wo + (size_t){p} * C] = {' + '.join(tsum) if tsum else 'T(0)'};")
                    L.append("    }")
                    L.append(f"    const T wp = w[wo + (size_t){p} * C];")
                    for k in range(d):
                        L.append(f"    const T g{k} = wp * o{k};")
                else:
                    for k in range(d):
                        L.append(f"    const T g{k} = o{k};")
                for (i, j, k, c) in self.cg[p]:
                    L.append(f"    hx{b1}_{i} += {_lit(c)} * (y{b2}_{j} * g{k});")
                    L.append(f"    hy{b2}_{j} += {_lit(c)} * (x{b1}_{i} * g{k});")
                L.append("  }")
            for bb in blocks:
                for m in range(self.d1[bb]):
                    e3, gm = self._addr("in1", bb, m)
                    L.append(f"  g1[IN1_GM ? ({gm}) : ({e3})] = hx{bb}_{m};")
            for bb, d in enumerate(self.d2):
                for m in range(d):
                    e3, gm = self._addr("in2", bb, m)
                    L.append(f"  g2[IN2_GM ? ({gm}) : ({e3})] = hy{bb}_{m};")
            L.append("}")
        # one launch runs every part: consecutive workgroups = the parts of the
        # same 256 (node, channel) pairs, so they share x2 in L2; part q writes
        # grad_x2 partial q (g2 itself when there is one part)
        L.append(f"template <typename T, bool IN1_GM, bool OUT_GM, bool IN2_GM>\n__global__ __launch_bounds__(256) void k_{self.name}_bwd(")
        L.append("    const T* __restrict__ x1, const T* __restrict__ x2, const T* __restrict__ w,")
        L.append("    const T* __restrict__ gout, T* __restrict__ g1, T* __restrict__ g2p, T* __restrict__ gw,")
        L.append("    int n_nodes, int C) {")
        L.append(f"  const int q = (int)(blockIdx.x % {nq});")
        L.append(f"  const size_t t = (size_t)(blockIdx.x / {nq}) * 256 + threadIdx.x;")
        L.append("  const size_t n = t / (size_t)C; const int u = (int)(t % (size_t)C);")
        L.append("  const size_t N = (size_t)n_nodes;")
        L.append("  if (n >= N) return;")
        L.append(f"  T* __restrict__ g2 = g2p + (size_t)q * N * C * {self.D2};")
        for q in range(nq):
            L.append(f"  {'if' if q == 0 else 'else if'} (q == {q}) f_{self.name}_bwd{q}<T, IN1_GM, OUT_GM, IN2_GM>("
                     "x1, x2, w, gout, g1, g2, gw, n, u, N, C);")
        L.append("}")
        return "\n".join(L)

    def emit(self) -> str:
        if self.kind == "uvu":
            nq = len(self.parts())
            rp = self.rtp_parts()
            return "\n\n".join([self.emit_uvu_fwd(q) for q in range(nq)] + [self.emit_uvu_bwd(q) for q in range(nq)]
                               + [self.emit_uvu_wrappers()] + [self.emit_rtp_fwd(b) for b in rp]
                               + [self.emit_rtp_bwd(b) for b in rp] + [self.emit_rtp_wrappers()])
        return self.emit_uuu_fwd() + "\n\n" + self.emit_uuu_bwd()


# ------------------------------------------------------------ variant sets ----
def model_variants(Lmax: int, lmax: int, correlation: int, bilinear: bool = False) -> List[Variant]:
    """All tensor-product variants one e3nnTACE model with these settings uses
    (cgtp interaction + CgtpACE product, natural parity, one fidelity,
    energy target), mirroring ``base.py:113-360`` irreps bookkeeping.  With
    the bilinear-gate product basis (correlation 2) the second operand is the
    hidden irreps plus one 0e block (``prod.py:83-87``)."""
    sh = list(range(lmax + 1))
    node_full = list(range(Lmax + 1))
    inter_out = list(range(lmax + 1)) if correlation != 1 else list(range(Lmax + 1))
    vs = [Variant("uvu", [0], sh, inter_out), Variant("uvu", node_full, sh, inter_out)]
    hidden = inter_out
    base = hidden + [0] if bilinear else hidden
    for last in (False, True):
        in1 = hidden
        for nu in range(2, correlation + 1):
            if nu == correlation:
                out = [0] if last else list(range(Lmax + 1))
            else:
                out = list(range(lmax + 1))
            v = Variant("uuu", in1, base, out, weighted=bilinear)
            vs.append(v)
            in1 = [l3 for (_, _, l3) in v.path_l]
    return vs


SUPPORTED = [(1, 1, 2), (1, 1, 3), (2, 2, 2), (2, 2, 3), (3, 3, 2), (3, 3, 3), (2, 3, 3)]
SUPPORTED_BILINEAR = [(1, 1, 2), (2, 2, 2), (3, 3, 2)]


def all_variants() -> List[Variant]:
    seen, out = set(), []
    for (Lm, lm, corr, bil) in [s + (False,) for s in SUPPORTED] + [s + (True,) for s in SUPPORTED_BILINEAR]:
        for v in model_variants(Lm, lm, corr, bil):
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


# ------------------------------------------------------------ wigner-D cg ----
def emit_wigner_cg(lmax_all: int = 3) -> str:
    """W3j(1, l-1, l) tables for the edge-frame Wigner-D recursion
    (``tace/models/o2/wigner.py:330-357``), flat [a][b][m]."""
    L = ["// W3j(1, l-1, l) (e3nn real basis, unit Frobenius norm): the coupling of the",
         "// Wigner-D recursion D^l = (2l+1) C^T (D^1 (x) D^(l-1)) C, flat [a][b][m].",
         "template <int L> struct WigCG;"]
    for l in range(2, lmax_all + 1):
        cg = wigner_3j(1, l - 1, l)
        vals = [repr(float(cg[a, b, m])) if abs(cg[a, b, m]) > 1e-14 else "0.0"
                for a in range(3) for b in range(2 * l - 1) for m in range(2 * l + 1)]
        L.append(f"template <> struct WigCG<{l}> {{ static constexpr double v[{3 * (2 * l - 1) * (2 * l + 1)}] = "
                 f"{{{', '.join(vals)}}}; }};")
    return "\n".join(L)


# -------------------------------------------------------------------- main ----
_UVU_FWD_SIG = ("const void*, const void*, const void*, const int*, const int*, const int*, const int*, const int*, "
                "void*, int, int, int, hipStream_t")
_UVU_BWD_SIG = ("const void*, const void*, const void*, const void*, const int*, const int*, const int*, const int*, "
                "const int*, void*, void*, void*, int, int, int, int, hipStream_t")
_RTP_FWD_SIG = ("const float*, const float*, const float*, const float*, float, const int*, const int*, const int*, "
                "const int*, const int*, float*, int, int, int, int, hipStream_t")
_RTP_BWD_SIG = ("const float*, const float*, const float*, const float*, float, const float*, const int*, const int*, "
                "const int*, const int*, const int*, float*, float*, float*, int, int, int, int, int, hipStream_t")
_UUU_FWD_SIG = "const void*, const void*, const void*, void*, int, int, int, hipStream_t"
_UUU_BWD_SIG = "const void*, const void*, const void*, const void*, void*, void*, void*, int, int, int, hipStream_t"
_TYPEDEFS = [
    f"typedef void (*UvuFwd)({_UVU_FWD_SIG});",
    f"typedef void (*UvuBwd)({_UVU_BWD_SIG});",
    f"typedef void (*UuuFwd)({_UUU_FWD_SIG});",
    f"typedef void (*UuuBwd)({_UUU_BWD_SIG});",
    f"typedef void (*RtpFwd)({_RTP_FWD_SIG});",
    f"typedef void (*RtpBwd)({_RTP_BWD_SIG});",
]


# uuu operand layouts compiled in (bit 1: x1 group-major, 2: out, 4: x2):
# all-e3nn (the slot adapter), the product-basis chain with e3nn node
# features (2, 3) and with group-major node features (7)
UUU_LAYOUTS = (0, 2, 3, 7)


def _b(v) -> str:
    return "true" if v else "false"


def _launchers(v: Variant) -> List[str]:
    out = []
    for T, tag in (("float", "f"), ("double", "d")):
        if v.kind == "uvu":
            # grid: parts x receivers padded to a multiple of 8 (tp_part_node); block: one lane per channel
            nq = len(v.parts())
            launch = f"const dim3 g((unsigned)((n + 7) / 8 * 8 * {nq})), b((unsigned)((C + 63) / 64 * 64));"
            out.append(f"void L_{v.name}_fwd_{tag}(const void* x, const void* y, const void* w, const int* rp, const int* eid, const int* src, const int* map, const int* wmap, void* o, int n, int flags, int C, hipStream_t s) {{")
            out.append("  if (n <= 0) return;")
            out.append("  " + launch)
            for f in range(4):
                out.append(f"  if (flags == {f}) hipLaunchKernelGGL((k_{v.name}_fwd<{T}, {_b(f & 1)}, {_b(f & 2)}>), g, b, 0, s, (const {T}*)x, (const {T}*)y, (const {T}*)w, rp, eid, src, map, wmap, ({T}*)o, n, C);")
            out.append("}")
            out.append(f"void L_{v.name}_bwd_{tag}(const void* x, const void* y, const void* w, const void* go, const int* rp, const int* eid, const int* src, const int* map, const int* wmap, void* cb, void* gy, void* gw, int n, int E, int flags, int C, hipStream_t s) {{")
            out.append("  if (n <= 0) return;")
            out.append(f"  const dim3 g((unsigned)((n + 7) / 8 * 8 * {nq} * ((C + 63) / 64))), b(64);")
            for f in range(4):
                for gx in (True, False):
                    out.append(f"  if (flags == {f} && {'cb' if gx else '!cb'}) hipLaunchKernelGGL((k_{v.name}_bwd<{T}, {_b(gx)}, {_b(f & 1)}, {_b(f & 2)}>), g, b, 0, s, (const {T}*)x, (const {T}*)y, (const {T}*)w, (const {T}*)go, rp, eid, src, map, wmap, ({T}*)cb, ({T}*)gy, ({T}*)gw, n, E, C);")
            out.append("}")
            if tag == "f":
                # radial-fused kernels (float32 only): grid from rtp_slot, 4 wavefronts of 16 channels
                nq = len(v.rtp_parts())
                launch = (f"const int nph = {nq} * (C / 64), nr = (n + per_range - 1) / per_range; "
                          "const dim3 g((unsigned)(8 * ((nr + 7) / 8) * nph)), b(512);")
                out.append(f"void L_{v.name}_rfwd(const float* x, const float* y, const float* h, const float* Wl, float alpha, const int* rp, const int* eid, const int* src, const int* map, const int* srow, float* o, int n, int flags, int C, int per_range, hipStream_t s) {{")
                out.append("  if (n <= 0) return;")
                out.append("  " + launch)
                for f in range(4):
                    out.append(f"  if (flags == {f}) hipLaunchKernelGGL((k_{v.name}_rfwd<{_b(f & 1)}, {_b(f & 2)}>), g, b, 0, s, x, y, h, Wl, alpha, rp, eid, src, map, srow, o, n, C, per_range);")
                out.append("}")
                out.append(f"void L_{v.name}_rbwd(const float* x, const float* y, const float* h, const float* Wl, float alpha, const float* go, const int* rp, const int* eid, const int* src, const int* map, const int* srow, float* cb, float* gy, float* gw, int n, int E, int flags, int C, int per_range, hipStream_t s) {{")
                out.append("  if (n <= 0) return;")
                out.append("  " + launch)
                for f in range(4):
                    for gx in (True, False):
                        out.append(f"  if (flags == {f} && {'cb' if gx else '!cb'}) hipLaunchKernelGGL((k_{v.name}_rbwd<{_b(gx)}, {_b(f & 1)}, {_b(f & 2)}>), g, b, 0, s, x, y, h, Wl, alpha, go, rp, eid, src, map, srow, cb, gy, gw, n, E, C, per_range);")
                out.append("}")
        else:
            out.append(f"void L_{v.name}_fwd_{tag}(const void* x1, const void* x2, const void* w, void* o, int n, int C, int flags, hipStream_t s) {{")
            out.append("  const size_t tot = (size_t)n * C; if (tot == 0) return;")
            out.append("  const dim3 g((unsigned)((tot + 255) / 256)), b(256);")
            for f in UUU_LAYOUTS:
                out.append(f"  if (flags == {f}) hipLaunchKernelGGL((k_{v.name}_fwd<{T}, {_b(f & 1)}, {_b(f & 2)}, {_b(f & 4)}>), g, b, 0, s, (const {T}*)x1, (const {T}*)x2, (const {T}*)w, ({T}*)o, n, C);")
            out.append("}")
            out.append(f"void L_{v.name}_bwd_{tag}(const void* x1, const void* x2, const void* w, const void* go, void* g1, void* g2, void* gw, int n, int C, int flags, hipStream_t s) {{")
            out.append("  const size_t tot = (size_t)n * C; if (tot == 0) return;")
            out.append(f"  const dim3 g((unsigned)((tot + 255) / 256 * {len(v.uuu_parts())})), b(256);")
            for f in UUU_LAYOUTS:
                out.append(f"  if (flags == {f}) hipLaunchKernelGGL((k_{v.name}_bwd<{T}, {_b(f & 1)}, {_b(f & 2)}, {_b(f & 4)}>), g, b, 0, s, (const {T}*)x1, (const {T}*)x2, (const {T}*)w, (const {T}*)go, ({T}*)g1, ({T}*)g2, ({T}*)gw, n, C);")
            out.append("}")
    return out


def emit_all(gen_dir: str) -> List[str]:
    """Writes gen/sh.inc, gen/registry.inc and one gen/v_<name>.hip per variant
    (compiled as separate translation units).  Returns the .hip paths."""
    os.makedirs(gen_dir, exist_ok=True)
    hdr = "// GENERATED by tace_amd/csrc/codegen.py -- do not edit."
    vs = all_variants()
    _write(os.path.join(gen_dir, "sh.inc"), [hdr, "#pragma once", emit_sh(3)])
    _write(os.path.join(gen_dir, "wigner.inc"), [hdr, "#pragma once", emit_wigner_cg(3)])
    srcs = []
    for v in vs:
        body = [hdr, f"// variant {v.key}: {len(v.paths)} paths, per-channel dims in1={v.D1} in2={v.D2} out={v.DO}",
                '#include "../common.h"', *_TYPEDEFS, v.emit(), "", *_launchers(v)]
        path = os.path.join(gen_dir, f"v_{v.name}.hip")
        _write(path, body)
        srcs.append(path)
    reg = [hdr, "#pragma once", *_TYPEDEFS,
           "struct TpVariant {",
           "  const char* key; int kind; int npath; int d1; int d2; int dout;",
           "  int weighted;                   // uuu: per-node path weights required",
           "  int nparts;                     // uvu: part kernels per launch (grad_y partials: nparts * ceil(C / 64))",
           "  int nseg; int seg[8][2];        // group-major grad-x row segments (offset / C, length / C)",
           "  UvuFwd fwd_f, fwd_d; UvuBwd bwd_f, bwd_d;",
           "  UuuFwd ufwd_f, ufwd_d; UuuBwd ubwd_f, ubwd_d;",
           "  int rnparts;                    // uvu: radial-fused parts (grad_y partials: rnparts * C / 64)",
           "  RtpFwd rfwd; RtpBwd rbwd;       // uvu: radial-fused kernels (float32)",
           "  int unparts;                    // uuu: backward parts (grad_x2 partials when > 1)", "};"]
    for v in vs:
        if v.kind == "uvu":
            reg += [f"void L_{v.name}_{k}_{t}({sig});" for k, sig in
                    (("fwd", _UVU_FWD_SIG), ("bwd", _UVU_BWD_SIG)) for t in ("f", "d")]
            reg += [f"void L_{v.name}_rfwd({_RTP_FWD_SIG});", f"void L_{v.name}_rbwd({_RTP_BWD_SIG});"]
        else:
            reg += [f"void L_{v.name}_{k}_{t}({sig});" for k, sig in
                    (("fwd", _UUU_FWD_SIG), ("bwd", _UUU_BWD_SIG)) for t in ("f", "d")]
    reg.append("static const TpVariant kVariants[] = {")
    for v in vs:
        n = v.name
        segs = v.row_segments() if v.kind == "uvu" else []
        assert len(segs) <= 8
        seg = "{" + ", ".join(f"{{{a}, {b}}}" for a, b in segs + [(0, 0)] * (8 - len(segs))) + "}"
        head = (f"\"{v.key}\", {0 if v.kind == 'uvu' else 1}, {len(v.paths)}, {v.D1}, {v.D2}, {v.DO}, "
                f"{int(v.weighted)}")
        if v.kind == "uvu":
            reg.append(f"  {{{head}, {len(v.parts())}, {len(segs)}, {seg}, L_{n}_fwd_f, L_{n}_fwd_d, L_{n}_bwd_f, "
                       f"L_{n}_bwd_d, nullptr, nullptr, nullptr, nullptr, {len(v.rtp_parts())}, L_{n}_rfwd, "
                       f"L_{n}_rbwd, 0}},")
        else:
            reg.append(f"  {{{head}, 0, 0, {seg}, nullptr, nullptr, nullptr, nullptr, "
                       f"L_{n}_fwd_f, L_{n}_fwd_d, L_{n}_bwd_f, L_{n}_bwd_d, 0, nullptr, nullptr, "
                       f"{len(v.uuu_parts())}}},")
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
