"""MI355X TACE model behind the reference model API.

``TACE(**cfg)`` accepts the reference ``e3nnTACE`` configuration
(``tace/models/_e3nn/tace.py:28-337``) and registers parameters and buffers
under the reference's names and shapes, so a reference ``state_dict`` loads
into it; ``TensorModel(TACE(**cfg))`` keeps ``TensorModel.forward(data)``
(``tace/models/adapter.py:23-452``).  The hot path runs on hand-written HIP
kernels (``tace_amd.ops``): edge featurisation, the fused edge tensor
product + receiver scatter and the uuu product basis; the node-level channel
mixing runs as species-grouped GEMMs.  There is no CPU execution path: the
native library must be present and the tensors on the GPU.

Supported configuration (the one the benchmark workloads use): linear node
embedding, identity edge embedding/update, ``cgtp`` atomic basis with
``sigmoid_gate`` (gate_m0), avg_num_neighbors scatter norm, BB element-aware
resnet, ``cgtp`` product basis (correlation 1-3, one expert), energy readout
with hidden [16], ``rms_forces`` scale, j0 Bessel x c2poly radial basis; and
the TECE configuration: ``uv_so2`` layers (radial-rotary edge convolution,
mmax = lmax) and the ``silu_bilineargate`` product basis (correlation 2).
Anything else raises ``NotImplementedError`` at construction.
"""

from __future__ import annotations

import collections
import copy
import math
import random
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from . import ops
from .so3 import Irrep, Irreps, generate_paths, possible_tp_irreps, spherical_harmonics_irreps

SIGMOID_CST = 1.8467055342154763  # e3nn normalize2mom(sigmoid)  (tace/models/mlp.py:43)
SILU_CST = 1.6791767923989418     # e3nn normalize2mom(silu)     (tace/models/mlp.py:34)


# ---------------------------------------------------------------- species ----
class SpeciesPlan:
    """Node order of the model's feature tensors: nodes grouped by species
    (``attrs.argmax``, stable), so that every per-species weight applies to
    one contiguous row range.  ``perm[r]`` = node stored in row r,
    ``node_map[n]`` (int32) = row of node n (what the edge kernels take)."""

    # (attrs, its version, natural, the plan's fields) of the last plan made
    # (the reference keeps attrs alive, so its identity cannot be reused)
    _last = None

    def __init__(self, attrs: torch.Tensor, exchange=None, pairs: Optional[ops.EdgePairs] = None,
                 natural: bool = False, counts: Optional[List[int]] = None):
        """counts: the number of nodes of each species (attrs column), when
        the caller knows them on the host; else they are read back from attrs."""
        self.attrs = attrs
        # LAMMPS ML-IAP data whose forward_exchange fills ghost rows before
        # every interaction layer >= 1 (several domains), or None
        self.exchange = exchange
        # edge pairs whose radial weights are made once (None: per edge)
        self.pairs = pairs
        self._pair_radial = None
        # the same node_attrs tensor as the last plan's, unchanged (an MD run
        # passes it every step): its order and species ranges again, without
        # reading the species counts back to the host
        last = SpeciesPlan._last
        if (last is not None and last[0] is attrs and last[1] == attrs._version and last[2] == natural
                and not attrs.requires_grad):
            self.species, self.perm, self.inv, self.node_map, self.ranges = last[3]
            return
        species = attrs.argmax(dim=-1)
        self.species = species
        if natural:
            # export mode: rows stay in node order; the per-species linears
            # group them inside their operator (tace_amd::element_linear)
            self.perm = self.inv = torch.arange(attrs.shape[0], device=attrs.device)
            self.node_map, self.ranges = None, None
        else:
            self.perm = torch.argsort(species, stable=True)
            inv = torch.empty_like(self.perm)
            inv[self.perm] = torch.arange(len(self.perm), device=self.perm.device)
            self.inv = inv
            self.node_map = inv.to(torch.int32)
            if counts is None or len(counts) != attrs.shape[1]:
                counts = torch.bincount(species, minlength=attrs.shape[1]).tolist()
            self.ranges = []
            acc = 0
            for s, c in enumerate(counts):
                if c:
                    self.ranges.append((s, acc, acc + c))
                acc += c
        if not attrs.requires_grad:
            SpeciesPlan._last = (attrs, attrs._version, natural,
                                 (self.species, self.perm, self.inv, self.node_map, self.ranges))

    def pair_radial(self, R: torch.Tensor) -> torch.Tensor:
        """R's rows of the edge pairs' lower edges (the radial MLP's input),
        gathered once per forward for all interaction layers."""
        if self._pair_radial is None or self._pair_radial[0] is not R:
            if ops.MODE.double or ops.MODE.export or not _RowGatherFn.fits(R):
                rows = R.index_select(0, self.pairs.row_edges)
            else:
                rows = _RowGatherFn.apply(R, self.pairs.row_edges)
            self._pair_radial = (R, rows)
        return self._pair_radial[1]


class _RowGatherFn(torch.autograd.Function):
    """R[rows] for distinct rows, moved as 16-byte elements (a row of 8
    float32 is two of them instead of eight 4-byte gathers); the backward
    writes each row's gradient back to its row (distinct rows: no sums) and
    zeros elsewhere."""

    @staticmethod
    def fits(R: torch.Tensor) -> bool:
        return (R.dim() == 2 and R.is_contiguous() and (R.shape[1] * R.element_size()) % 16 == 0
                and (R.storage_offset() * R.element_size()) % 16 == 0)

    @staticmethod
    def forward(ctx, R, rows):
        ctx.save_for_backward(rows)
        ctx.shape = R.shape
        return R.view(torch.complex128).index_select(0, rows).view(R.dtype)

    @staticmethod
    def backward(ctx, g):
        (rows,) = ctx.saved_tensors
        gR = g.new_zeros(ctx.shape)
        gR.view(torch.complex128).index_copy_(0, rows.long(), g.contiguous().view(torch.complex128))
        return gR, None


# ------------------------------------------------------------ feature layout ----
class GMLayout:
    """Group-major batch layout of features with (simplified) irreps: block b
    of the whole batch is one row-major [Z, 2l+1, mul_b] matrix at element
    offset Z * s_b (s_b = sum of mul*dim of the blocks before it).  A block's
    rows for nodes a..b are then one contiguous [(b-a)(2l+1), mul] GEMM
    operand, and a block of C-channel irreps is what the tensor-product
    kernels read and write (``TACE_LAYOUT_*_GROUPED``)."""

    def __init__(self, irreps):
        # one block per entry of ``irreps``: for simplified irreps this is the
        # kernels' group-major layout; unsimplified irreps (adjacent equal
        # entries) stay separate blocks, which only the model's own code reads
        self.irreps = Irreps(irreps)
        self.blocks, s = [], 0
        for m, ir in self.irreps:
            self.blocks.append((s, m, ir.dim))
            s += m * ir.dim
        self.dim = s

    def block(self, x: torch.Tensor, b: int, a: int = 0, c: Optional[int] = None) -> torch.Tensor:
        """Rows of nodes a..c of block b as a [(c-a)*(2l+1), mul] view."""
        Z = x.shape[0]
        s, m, d = self.blocks[b]
        c = Z if c is None else c
        return x.view(-1)[Z * s + a * d * m:Z * s + c * d * m].view((c - a) * d, m)


def e3nn_to_gm(x: torch.Tensor, irreps) -> torch.Tensor:
    """e3nn mul_ir layout -> group-major layout of the same irreps."""
    lay = GMLayout(irreps)
    Z = x.shape[0]
    out = torch.empty_like(x)
    col = 0
    for b, (s, m, d) in enumerate(lay.blocks):
        lay.block(out, b).view(Z, d, m).copy_(x[:, col:col + m * d].view(Z, m, d).transpose(1, 2))
        col += m * d
    return out


def gm_to_e3nn(x: torch.Tensor, irreps) -> torch.Tensor:
    """group-major layout -> e3nn mul_ir layout."""
    lay = GMLayout(irreps)
    Z = x.shape[0]
    cols = [lay.block(x, b).view(Z, d, m).transpose(1, 2).reshape(Z, m * d) for b, (s, m, d) in enumerate(lay.blocks)]
    return torch.cat(cols, dim=1)


class _GhostExchangeFn(torch.autograd.Function):
    """``GhostExchange`` (``tace/models/lammps.py:82-102``) on this model's
    node features (group-major rows in species order): every row goes out in
    LAMMPS atom order and e3nn's mul_ir layout, ``forward_exchange`` replaces
    the ghost rows by their owners' rows (possibly from another domain), and
    the backward's ``reverse_exchange`` sums ghost-row gradients into their
    owners."""

    @staticmethod
    def forward(ctx, x, irreps, sp: "SpeciesPlan", lmp_data):
        rows = gm_to_e3nn(x, irreps).index_select(0, sp.inv).contiguous()
        out = torch.empty_like(rows)
        lmp_data.forward_exchange(rows, out, rows.shape[1])
        ctx.irreps, ctx.sp, ctx.lmp = irreps, sp, lmp_data
        return e3nn_to_gm(out.index_select(0, sp.perm), irreps)

    @staticmethod
    def backward(ctx, g):
        rows = gm_to_e3nn(g.contiguous(), ctx.irreps).index_select(0, ctx.sp.inv).contiguous()
        gin = torch.empty_like(rows)
        ctx.lmp.reverse_exchange(rows, gin, rows.shape[1])
        return e3nn_to_gm(gin.index_select(0, ctx.sp.perm), ctx.irreps), None, None, None


# the ghost exchange of an exported LAMMPS program: the tace_amd::
# lammps_forward_exchange operator on the LAMMPS data the caller makes current
# (library.use_lammps_data), as AOTI_LAMMPS_GHOST_EXCHANGE marks it in
# tace/models/lammps.py:12, 126-130
LAMMPS_PROGRAM_EXCHANGE = object()


def _exchange_ghosts(x: torch.Tensor, irreps, sp: "SpeciesPlan", layer: int) -> torch.Tensor:
    """``handle_lammps`` (``tace/models/lammps.py:105-134``, called after
    linear_up at ``_e3nn/inter.py:228``): no exchange in layer 0 (ghost
    features come from their own embedding), the owners' rows from layer 1."""
    if sp.exchange is None or layer == 0:
        return x
    if sp.exchange is LAMMPS_PROGRAM_EXCHANGE:
        # export mode: rows in node (LAMMPS atom) order
        from . import library
        return e3nn_to_gm(library.lammps_forward_exchange(gm_to_e3nn(x, irreps)), irreps)
    return _GhostExchangeFn.apply(x, irreps, sp, sp.exchange)


# ---------------------------------------------------------------- linears ----
# the interaction's radial last layer inside the edge-product kernels
# (ops.edge_rtp_scatter; float32, C % 64 == 0).  Off: on the 12k-atom water
# box the fused kernels take 12.6 ms (forward) and 23.3 ms (backward) per
# layer against 8.2 ms and 8.5 ms for the last layer's own MFMA kernel plus
# the product kernels -- the weight slice each wavefront keeps for its MFMAs
# (112 registers at 7 paths) leaves the product math 1-2 wavefronts per SIMD,
# too few to keep the vector ALUs busy.
RADIAL_FUSED_TP = False

# per-species linears over at least this many species ranges run as one
# segmented-GEMM launch (tace_seg_linear); fewer run one library GEMM per
# instruction and species.  float32 (the bf16x3 MFMA kernel): every
# per-species linear takes the segmented kernel -- on the 2-species water box
# it measured 72.3 against 72.7 ms/step with library GEMMs, on 1-species bcc Fe
# 375.8 against 379.3 ms/step.  float64 runs the segmented launch on a 64x64
# FMA tile kernel, which only pays for itself once the library path needs
# many small GEMMs (several species).
SEG_LINEAR_MIN_RANGES = {torch.float32: 1, torch.float64: 3}
# tile edge of the float32 segmented GEMM: 128 = MFMA kernel (float32 as three
# bf16 terms), 64 = FMA kernel
SEG_LINEAR_TILE_F32 = 128
# float32 shared-weight linears (e3nnLinear) with at least this many
# instructions run as one segmented-GEMM launch too (None: one library GEMM
# per instruction).  Water box: 62.4 against 63.0 ms/step model time (89
# library launches per step replaced by 28 segmented ones)
SEG_LINEAR_SHARED_MIN_INS = 1
# the 128 MFMA kernel reads weights split into bf16 terms once per weight
# version (tace_seg_linear_presplit) instead of splitting them in every launch
SEG_LINEAR_PRESPLIT = True
# radial MLP of the cgtp interactions once per edge pair (both directions of
# an edge have the same length), when the graph's periodic shifts are known
PAIR_RADIAL = True


class _LinearLayout:
    """e3nn ``o3.Linear`` bookkeeping: instructions (i_in, i_out) between equal
    irreps in i_in-major order, path weight (sum of mul_in into i_out)^-1/2,
    flat weight of row-major [mul_in, mul_out] blocks (``linear.py:282-374``);
    bias on the 0e output blocks."""

    def __init__(self, irreps_in, irreps_out):
        self.irreps_in = Irreps(irreps_in)
        self.irreps_out = Irreps(irreps_out)
        ins = [(i, o) for i, (_, a) in enumerate(self.irreps_in) for o, (_, b) in enumerate(self.irreps_out) if a == b]
        fan = {}
        for i, o in ins:
            fan[o] = fan.get(o, 0) + self.irreps_in[i][0]
        self.ins, off = [], 0
        for i, o in ins:
            mi, mo = self.irreps_in[i][0], self.irreps_out[o][0]
            self.ins.append((i, o, off, mi, mo, fan[o] ** -0.5))
            off += mi * mo
        self.weight_numel = off
        self.bias_blocks, b = [], 0
        for o, (m, ir) in enumerate(self.irreps_out):
            if ir.l == 0 and ir.p == 1:
                self.bias_blocks.append((o, b, m))
                b += m
        self.bias_numel = b
        self.gin, self.gout = GMLayout(self.irreps_in), GMLayout(self.irreps_out)
        self.dim_in, self.dim_out = self.gin.dim, self.gout.dim
        self.read = {i for (i, *_r) in self.ins}
        self.written = {o for (_, o, *_r) in self.ins}
        self._seg = collections.OrderedDict()
        self._split = {}
        # pre-split weight planes (tace_bf16x3_split_blocks): per instruction
        # the block's offset in one species' planes, its columns and k; per
        # direction ("fwd": B = W, "bwd": B = W^T)
        self.split_blocks = {}
        # the same in MFMA fragment order (layout 1: tace_seg_linear_presplit_ks
        # and tace_seg_linear_presplit_frag)
        self.frag_blocks = {}
        for kind in ("fwd", "bwd"):
            blocks, acc, fblocks, facc = [], 0, [], 0
            for (i, o, off, mi, mo, pw) in self.ins:
                cols, k = (mo, mi) if kind == "fwd" else (mi, mo)
                blocks.append((acc, cols, k))
                acc += cols * ((k + 7) // 8 * 8)
                fblocks.append((facc, cols, k))
                facc += 3 * ((cols + 15) // 16 * 16) * ((k + 31) // 32 * 32)
            self.split_blocks[kind] = (blocks, acc)
            self.frag_blocks[kind] = (fblocks, facc)

    def split_weights(self, kind: str, weight: torch.Tensor, frag: bool = False) -> Tuple[torch.Tensor, int]:
        """The three bf16 terms of every (species, instruction) weight block
        with its path weight folded in, in the column layout of
        ``tace_seg_linear_presplit`` ("fwd": B = W, "bwd": B = W^T); returns
        (planes int16 [3 * stride], plane stride).  ``frag``: the blocks in
        the MFMA fragment order of ``tace_seg_linear_presplit_ks`` and
        ``tace_seg_linear_presplit_frag`` instead (one buffer; the stride is
        its size).  Cached until the weight changes (its version counter or
        storage)."""
        w = weight.detach()
        key = (w.data_ptr(), w._version, tuple(w.shape), str(w.device))
        ck = (kind, frag)
        hit = self._split.get(ck)
        if hit is not None and hit[0] == key:
            return hit[1], hit[2]
        blocks, per = (self.frag_blocks if frag else self.split_blocks)[kind]
        S = 1 if w.dim() == 1 else w.shape[0]
        # never empty: a plan whose short-k tasks are all zero blocks still
        # passes a valid pointer
        stride = max(64, (S * per + 63) // 64 * 64)
        tab, sc = [], []
        for sp in range(S):
            for (dst, cols, k), (i, o, off, mi, mo, pw) in zip(blocks, self.ins):
                if dst < 0:
                    continue
                tab.append((sp * self.weight_numel + off, cols, k, 1 if kind == "fwd" else 0, sp * per + dst,
                            1 if frag else 0))
                sc.append(pw)
        planes = ops.bf16x3_split_blocks(w.contiguous().view(-1), tab, sc, stride, frag=frag)
        # the entry keeps the weight alive, so no other tensor can take its
        # address (and version) while the planes are cached
        self._split[ck] = (key, planes, stride, w)
        return planes, stride

    def seg_plan(self, kind: str, rr, Z: int, x: torch.Tensor, weight: torch.Tensor,
                 bias: Optional[torch.Tensor]) -> ops.SegLinearPlan:
        """``tace_seg_linear`` tables of the forward ("fwd": x -> out, bias
        added) or the input gradient ("bwd": g_out -> g_x, W^T) over species
        ranges ``rr`` of Z rows; the last few are cached."""
        tile = (128, 128) if x.dtype == torch.float32 and SEG_LINEAR_TILE_F32 == 128 else (64, 64)
        presplit = tile == (128, 128) and SEG_LINEAR_PRESPLIT
        key = (kind, tuple(rr), Z, str(x.device), bias is not None, weight.numel(), tile, presplit, ops.SEG_TILE_FRAG,
               ops.SEG_SPLIT_SLOTS, ops.SEG_SPLIT_MIN_STEPS, ops.SEG_SPLIT_MAX_TILES)
        plan = self._seg.get(key)
        if plan is not None:
            self._seg.move_to_end(key)
            return plan
        if kind == "fwd":
            boffs = {o: boff for (o, boff, m) in self.bias_blocks} if bias is not None else {}
            outs = [(s, m, d, boffs.get(o)) for o, (s, m, d) in enumerate(self.gout.blocks)]
            ins = [(o, self.gin.blocks[i][0], mi, off, False, pw) for (i, o, off, mi, mo, pw) in self.ins]
            xn, yn = Z * self.dim_in, Z * self.dim_out
        else:
            outs = [(s, m, d, None) for (s, m, d) in self.gin.blocks]
            ins = [(i, self.gout.blocks[o][0], mo, off, True, pw) for (i, o, off, mi, mo, pw) in self.ins]
            xn, yn = Z * self.dim_out, Z * self.dim_in
        if presplit:
            # weight offsets into the pre-split planes instead of the flat weight
            blocks, per = self.split_blocks[kind]
            fblocks, fper = self.frag_blocks[kind]
            ins = [(a, b, k, blocks[j][0], tr, pw, fblocks[j][0]) for j, (a, b, k, _off, tr, pw) in enumerate(ins)]
            S = 1 if weight.dim() == 1 else weight.shape[0]
            plan = ops.SegLinearPlan(Z, outs, ins, rr, per, self.bias_numel, xn, yn, S * per,
                                     0 if bias is None else bias.numel(), x.device, tile, split_weights=True,
                                     frag=(fper, S * fper))
        else:
            plan = ops.SegLinearPlan(Z, outs, ins, rr, self.weight_numel, self.bias_numel, xn, yn, weight.numel(),
                                     0 if bias is None else bias.numel(), x.device, tile)
        self._seg[key] = plan
        if len(self._seg) > 16:
            self._seg.popitem(last=False)
        return plan


def _linear_route(x: torch.Tensor, weight: torch.Tensor, lay: "_LinearLayout", ranges):
    """(non-empty species ranges, whether the segmented-GEMM kernel runs) of
    one linear on x: shared weights take the whole row range."""
    Z = x.shape[0]
    shared = weight.dim() == 1
    rr = [(None, 0, Z)] if shared else ranges
    rr = [r for r in rr if r[2] > r[1]]
    seg = not shared and len(rr) >= SEG_LINEAR_MIN_RANGES.get(x.dtype, 1)
    if shared and x.dtype == torch.float32 and SEG_LINEAR_SHARED_MIN_INS is not None:
        seg = len(lay.ins) >= SEG_LINEAR_SHARED_MIN_INS and Z > 0
    return rr, seg


def _linear_apply(x, weight, bias, lay: "_LinearLayout", rr, seg: bool, alpha: float, kind: str = "fwd",
                  out: Optional[torch.Tensor] = None, addend: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One direction of an e3nn linear on group-major rows: ``kind`` "fwd"
    (x -> out = alpha (x W + bias)) or "bwd" (g_out -> g_x = alpha g_out W^T,
    no bias), plus ``addend`` when given (``out`` itself for out += ..., or a
    separate tensor).  Per instruction and species range one GEMM, or all of
    them in one segmented-GEMM launch (``seg``)."""
    fwd = kind == "fwd"
    gin, gout_l = (lay.gin, lay.gout) if fwd else (lay.gout, lay.gin)
    dim = lay.dim_out if fwd else lay.dim_in
    Z = x.shape[0]
    if out is None:
        out = x.new_empty(Z, dim)
    if not fwd:
        bias = None
    shared = weight.dim() == 1
    if seg:
        plan = lay.seg_plan(kind, rr, Z, x, weight, bias)
        if plan.split_weights:
            fr = lay.split_weights(kind, weight, frag=True)[0] if plan.n_ks or plan.tile_frag else None
            pl = (None, 0) if plan.tile_frag else lay.split_weights(kind, weight)
            return ops.seg_linear_presplit(x, out, *pl, bias, plan, alpha, frag=fr, addend=addend)
        return ops.seg_linear(x, out, weight, bias, plan, alpha, addend=addend)
    acc = addend is not None
    if acc and addend.data_ptr() != out.data_ptr():
        out.copy_(addend)
    done = set()
    for (i, o, off, mi, mo, pw) in lay.ins:
        src, dst = (i, o) if fwd else (o, i)
        for (sp, a, b) in rr:
            W = (weight if shared else weight[sp])[off:off + mi * mo].view(mi, mo)
            gout_l.block(out, dst, a, b).addmm_(gin.block(x, src, a, b), W if fwd else W.t(),
                                                beta=1.0 if acc or (dst, sp) in done else 0.0, alpha=pw * alpha)
            done.add((dst, sp))
    if not acc:
        hit = lay.written if fwd else lay.read
        for o in range(len(gout_l.blocks)):
            if o not in hit:
                gout_l.block(out, o).zero_()
    if bias is not None:
        for (o, boff, m) in lay.bias_blocks:
            for (sp, a, b) in rr:
                bv = (bias if shared else bias[sp])[boff:boff + m]
                lay.gout.block(out, o, a, b).add_(bv, alpha=alpha)
    return out


class _LinearFn(torch.autograd.Function):
    """e3nn ``o3.Linear`` on group-major features: per instruction and species
    range one GEMM written in place into the output (``addmm_``, path weight
    and ``alpha`` in the GEMM's scale), bias added to the 0e blocks, or all
    of them in one segmented-GEMM launch.  ``weight`` [numel] (shared) or
    [S, numel] with ``ranges`` = [(species, a, b)] over species-sorted rows.
    out = alpha * (linear(x) + bias)."""

    @staticmethod
    def forward(ctx, x, weight, bias, lay: _LinearLayout, ranges, alpha: float):
        rr, seg = _linear_route(x, weight, lay, ranges)
        ctx.save_for_backward(x, weight, bias)
        ctx.lay, ctx.rr, ctx.alpha, ctx.seg = lay, rr, alpha, seg
        return _linear_apply(x, weight, bias, lay, rr, seg, alpha)

    @staticmethod
    def backward(ctx, gout):
        x, weight, bias = ctx.saved_tensors
        lay, rr, alpha = ctx.lay, ctx.rr, ctx.alpha
        gout = gout.contiguous()
        shared = weight.dim() == 1
        gx = None
        if ctx.needs_input_grad[0]:
            gx = _linear_apply(gout, weight, None, lay, rr, ctx.seg, alpha, kind="bwd")
        gw = torch.zeros_like(weight) if ctx.needs_input_grad[1] else None
        gb = torch.zeros_like(bias) if bias is not None and ctx.needs_input_grad[2] else None
        if gw is not None:
            for (i, o, off, mi, mo, pw) in lay.ins:
                for (sp, a, b) in rr:
                    tgt = (gw if shared else gw[sp])[off:off + mi * mo].view(mi, mo)
                    tgt.addmm_(lay.gin.block(x, i, a, b).t(), lay.gout.block(gout, o, a, b), alpha=pw * alpha)
        if gb is not None:
            for (o, boff, m) in lay.bias_blocks:
                for (sp, a, b) in rr:
                    tgt = (gb if shared else gb[sp])[boff:boff + m]
                    tgt += lay.gout.block(gout, o, a, b).sum(0) * alpha
        return gx, gw, gb, None, None, None


def _linear_autograd(x, weight, bias, lay: _LinearLayout, ranges, alpha: float) -> torch.Tensor:
    """``_LinearFn`` as plain torch operations (differentiable to any order):
    per output block and species range, the sum over its instructions of
    pw * x_block @ W, plus the bias on 0e blocks, times alpha; group-major out."""
    Z = x.shape[0]
    shared = weight.dim() == 1
    rr = [(None, 0, Z)] if shared else [r for r in ranges if r[2] > r[1]]
    if Z == 0 or not rr:
        return x.new_zeros(Z, lay.dim_out)
    boffs = {o: (boff, m) for (o, boff, m) in lay.bias_blocks}
    flat = []
    for o, (_s, m_o, d_o) in enumerate(lay.gout.blocks):
        parts = []
        for (sp, a, b) in rr:
            acc = None
            for (i, oo, off, mi, mo, pw) in lay.ins:
                if oo != o:
                    continue
                W = (weight if shared else weight[sp])[off:off + mi * mo].view(mi, mo)
                t = torch.mm(lay.gin.block(x, i, a, b), W) * pw
                acc = t if acc is None else acc + t
            if acc is None:
                acc = x.new_zeros((b - a) * d_o, m_o)
            if bias is not None and o in boffs:
                boff, m = boffs[o]
                acc = acc + (bias if shared else bias[sp])[boff:boff + m]
            parts.append(acc)
        flat.append((torch.cat(parts, 0) if len(parts) > 1 else parts[0]).reshape(-1))
    return (torch.cat(flat) * alpha).view(Z, lay.dim_out)


class e3nnLinear(torch.nn.Module):
    """Parameters ``weight`` [numel] ~ N(0,1), ``bias`` [#0e] zeros
    (``linear.py:282-374``); group-major input and output."""

    def __init__(self, irreps_in, irreps_out, bias: bool = True):
        super().__init__()
        self.lay = _LinearLayout(irreps_in, irreps_out)
        self.irreps_in, self.irreps_out = self.lay.irreps_in, self.lay.irreps_out
        self.weight = torch.nn.Parameter(torch.randn(self.lay.weight_numel))
        self.bias = torch.nn.Parameter(torch.zeros(self.lay.bias_numel)) if bias and self.lay.bias_numel else None

    def forward(self, x, alpha: float = 1.0):
        if ops.MODE.double:
            return _linear_autograd(x.contiguous(), self.weight, self.bias, self.lay, None, float(alpha))
        return _LinearFn.apply(x.contiguous(), self.weight, self.bias, self.lay, None, float(alpha))


class e3nnElementLinear(torch.nn.Module):
    """Per-species weights ``weight`` [S, numel], ``bias`` [S, #0e]
    (``linear.py:377-481``): one GEMM per (species, instruction) on the
    species-sorted rows of group-major features."""

    def __init__(self, irreps_in, irreps_out, num_elements: int, bias: bool = True):
        super().__init__()
        self.lay = _LinearLayout(irreps_in, irreps_out)
        self.irreps_in, self.irreps_out = self.lay.irreps_in, self.lay.irreps_out
        self.num_elements = num_elements
        self.weight = torch.nn.Parameter(torch.randn(num_elements, self.lay.weight_numel))
        self.bias = (torch.nn.Parameter(torch.zeros(num_elements, self.lay.bias_numel))
                     if bias and self.lay.bias_numel else None)

    def forward(self, x: torch.Tensor, sp: SpeciesPlan, alpha: float = 1.0) -> torch.Tensor:
        if ops.MODE.export:
            from . import library
            return library.element_linear(x.contiguous(), self.weight, self.bias, sp.species, str(self.irreps_in),
                                          str(self.irreps_out), float(alpha))
        if ops.MODE.double:
            return _linear_autograd(x.contiguous(), self.weight, self.bias, self.lay, sp.ranges, float(alpha))
        return _LinearFn.apply(x.contiguous(), self.weight, self.bias, self.lay, sp.ranges, float(alpha))


class mlpLinear(torch.nn.Module):
    """``x @ (weight * alpha)``, weight [in, out] ~ U(-sqrt3, sqrt3) (``linear.py:247-279``)."""

    def __init__(self, in_dim, out_dim, alpha):
        super().__init__()
        self.alpha = alpha
        self.weight = torch.nn.Parameter(torch.empty(in_dim, out_dim).uniform_(-math.sqrt(3), math.sqrt(3)))

    def forward(self, x):
        # x @ (weight * alpha) with alpha in the GEMM's scale
        return x.new_empty(x.shape[0], self.weight.shape[1]).addmm_(x, self.weight, beta=0.0, alpha=self.alpha)


class MLP(torch.nn.Module):
    """Radial MLP (``mlp.py:136-191``): alpha = gain/sqrt(h_in), SiLU between
    layers.  Width-64 hidden layers run in one HIP kernel per direction
    (``ops.radial_mlp_hidden``) and the wide last layer on a float32 MFMA
    kernel (three-term bf16 split, ``ops.radial_mlp_out``), the weights as
    constants: the inference path
    freezes parameters."""

    def __init__(self, dims):
        super().__init__()
        mods = []
        for layer, (a, b) in enumerate(zip(dims, dims[1:])):
            mods.append(mlpLinear(a, b, (1.0 if layer == 0 else math.sqrt(2.0)) / math.sqrt(a)))
            if layer != len(dims) - 2:
                mods.append(torch.nn.SiLU())
        self.mlp = torch.nn.Sequential(*mods)
        self.fused = len(dims) >= 3 and all(h == 64 for h in dims[1:-1]) and dims[0] <= 32 and len(dims) - 2 <= 4

    def forward(self, x):
        if not self.fused or ops.MODE.double:
            return self.mlp(x)
        return ops.radial_mlp_out(self.hidden(x), *self.last_layer())

    def hidden(self, x):
        """The last hidden activations [E, 64] (fused MLPs only)."""
        lins = [m for m in self.mlp if isinstance(m, mlpLinear)]
        return ops.radial_mlp_hidden(x, [m.weight * m.alpha for m in lins[:-1]])

    def last_layer(self):
        """(weight [64, n_out], alpha) of the last linear layer: the MLP's
        output is alpha * hidden(x) @ weight.  The weight is a constant here,
        as in ``forward``: gradients flow to the hidden activations only."""
        last = [m for m in self.mlp if isinstance(m, mlpLinear)][-1]
        return last.weight.detach(), float(last.alpha)


# ------------------------------------------------------------------ blocks ----
def _ls(irreps: Irreps) -> List[int]:
    return [ir.l for _, ir in irreps]


class O3ScatterTensorProduct(torch.nn.Module):
    """Edge uvu tensor product + scatter to receivers, on the HIP kernel
    (replaces ``tace/models/_e3nn/fused.py:172-271``; no parameters)."""

    def __init__(self, irreps_in1, irreps_in2, irreps_out):
        super().__init__()
        self.irreps_in1, self.irreps_in2 = Irreps(irreps_in1), Irreps(irreps_in2)
        paths, self.irreps_out = generate_paths(Irreps(irreps_out), self.irreps_in1, self.irreps_in2, "uvu")
        self.C = self.irreps_in1[0][0]
        assert all(m == self.C for m, _ in self.irreps_in1) and all(m == 1 for m, _ in self.irreps_in2)
        self.weight_numel = self.C * len(paths)
        self.key = ops.variant_key("uvu", _ls(self.irreps_in1), _ls(self.irreps_in2), _ls(Irreps(irreps_out)))

    def forward(self, x, y, w, plan: ops.EdgePlan, layout: int = 0, node_map=None):
        return ops.edge_tp_scatter(x, y, w, plan, ops.find_variant(self.key), self.C, layout, node_map)

    def paired(self, x, y, h, W, alpha: float, plan: ops.EdgePlan, pairs: ops.EdgePairs, layout: int = 0,
               node_map=None):
        """forward(x, y, alpha * h @ W, ...) with the weights made once per edge
        pair (``ops.edge_tp_scatter_pairs``; h holds the pairs' rows)."""
        return ops.edge_tp_scatter_pairs(x, y, h, W, alpha, plan, pairs, ops.find_variant(self.key), self.C, layout,
                                         node_map)

    def radial_fused(self, x, y, h, W, alpha: float, plan: ops.EdgePlan, layout: int = 0, node_map=None):
        """forward(x, y, alpha * h @ W, ...) with the radial last layer inside
        the product kernels (``ops.edge_rtp_scatter``)."""
        return ops.edge_rtp_scatter(x, y, h, W, alpha, plan, ops.find_variant(self.key), self.C, layout, node_map)


class uuuTensorProduct(torch.nn.Module):
    """Node uuu product on the HIP kernel (replaces ``fused.py:17-95``)."""

    def __init__(self, irreps_in1, irreps_in2, irreps_out, identical_inputs: bool):
        super().__init__()
        self.irreps_in1, self.irreps_in2 = Irreps(irreps_in1), Irreps(irreps_in2)
        paths, self.irreps_out = generate_paths(Irreps(irreps_out), self.irreps_in1, self.irreps_in2, "uuu",
                                                identical_inputs)
        self.C = self.irreps_in1[0][0]
        self.weight_numel = self.C * len(paths)
        self.key = ops.variant_key("uuu", _ls(self.irreps_in1), _ls(self.irreps_in2), _ls(Irreps(irreps_out)))

    def forward(self, x1, x2, layout: int = 0, w=None):
        return ops.uuu_tp(x1, x2, ops.find_variant(self.key), self.C, layout, w)


class _GateFn(torch.autograd.Function):
    """``O3Gate`` with gate_m0 (``tace/models/_e3nn/nonlinear.py:27-42, 93-143``)
    on group-major features.  Input irreps (gates + gated).simplify(): the
    first ng*C scalars of block 0 are the gates (one C-block per gated irrep),
    then come the gated irreps (a gated 0e shares block 0).  Each gated block
    [Z, 2l+1, C] is scaled by normalize2mom(sigmoid)(its gate) [Z, 1, C]
    (e3nn's elementwise product with sqrt(2l+1) W3j(l,0,l) is exactly that)."""

    @staticmethod
    def forward(ctx, x, lin: GMLayout, lout: GMLayout, C: int):
        Z = x.shape[0]
        ng = len(lout.blocks)
        X0 = lin.block(x, 0).view(Z, -1)
        g = torch.sigmoid(X0[:, :ng * C]).mul_(SIGMOID_CST)
        out = x.new_empty(Z, lout.dim)
        for k, src in enumerate(_gated_blocks(x, lin, lout, C)):
            torch.mul(src, g[:, k * C:(k + 1) * C].unsqueeze(1), out=lout.block(out, k).view(Z, -1, C))
        ctx.save_for_backward(x, g)
        ctx.lay = (lin, lout, C)
        return out

    @staticmethod
    def backward(ctx, gout):
        x, g = ctx.saved_tensors
        lin, lout, C = ctx.lay
        gout = gout.contiguous()
        Z = x.shape[0]
        ng = len(lout.blocks)
        gx = torch.empty_like(x)
        X0g = lin.block(gx, 0).view(Z, -1)
        gg = x.new_empty(Z, ng * C)
        srcs = _gated_blocks(x, lin, lout, C)
        dsts = _gated_blocks(gx, lin, lout, C)
        for k in range(ng):
            go = lout.block(gout, k).view(Z, -1, C)
            gk = g[:, k * C:(k + 1) * C]
            torch.mul(go, gk.unsqueeze(1), out=dsts[k])
            if go.shape[1] == 1:
                torch.mul(go[:, 0], srcs[k][:, 0], out=gg[:, k * C:(k + 1) * C])
            else:
                torch.sum(go * srcs[k], dim=1, out=gg[:, k * C:(k + 1) * C])
        # d/dz [CST * sigmoid(z)] = g * (1 - g / CST) = g - g^2 / CST
        torch.mul(gg, torch.addcmul(g, g, g, value=-1.0 / SIGMOID_CST), out=X0g[:, :ng * C])
        return gx, None, None, None


def _gate(x: torch.Tensor, lin: GMLayout, lout: GMLayout, C: int) -> torch.Tensor:
    """``_GateFn``; inside ``ops.differentiable_twice`` as plain torch operations."""
    if not ops.MODE.double:
        return _GateFn.apply(x, lin, lout, C)
    Z = x.shape[0]
    ng = len(lout.blocks)
    g = torch.sigmoid(lin.block(x, 0).view(Z, -1)[:, :ng * C]) * SIGMOID_CST
    out = [(src * g[:, k * C:(k + 1) * C].unsqueeze(1)).reshape(-1)
           for k, src in enumerate(_gated_blocks(x, lin, lout, C))]
    return torch.cat(out).view(Z, lout.dim)


def _gated_blocks(x: torch.Tensor, lin: GMLayout, lout: GMLayout, C: int) -> List[torch.Tensor]:
    """[Z, 2l+1, C] views of the gated irreps inside the gate's input."""
    Z = x.shape[0]
    ng = len(lout.blocks)
    X0 = lin.block(x, 0).view(Z, -1)
    out, b = [], 1
    for k, (s, m, d) in enumerate(lout.blocks):
        if k == 0 and d == 1:
            out.append(X0[:, ng * C:ng * C + C].unsqueeze(1))
        else:
            out.append(lin.block(x, b).view(Z, d, C))
            b += 1
    return out


class O3CgtpInteraction(torch.nn.Module):
    """``O3CgtpInteraction`` (``tace/models/_e3nn/inter.py:28-285``), BB resnet."""

    def __init__(self, layer, num_layers, irreps_in, C, Lmax, lmax, correlation, num_elements, avg_num_neighbors,
                 radial_hidden, num_radial):
        super().__init__()
        self.layer = layer
        self.avg_num_neighbors = float(avg_num_neighbors)
        self.irreps_in = Irreps(irreps_in)
        sh = spherical_harmonics_irreps(lmax)
        tp_out = possible_tp_irreps(self.irreps_in, sh, False, Lmax if correlation == 1 else lmax)
        self.irreps_out = (tp_out * C).regroup()
        if layer == num_layers - 1:
            irreps_sc = (Irreps("0e") * C).regroup()
        else:
            irreps_sc = (possible_tp_irreps(self.irreps_in, sh, False, Lmax) * C).regroup()
        self.linear_up = e3nnLinear(self.irreps_in, self.irreps_in, bias=True)
        self.rejector = O3ScatterTensorProduct(self.irreps_in, sh, self.irreps_out)
        self.gated = Irreps([(C, ir) for _, ir in self.irreps_out])
        gates = Irreps([(C, Irrep("0e")) for _ in self.gated])
        self.linear_nonlinearity = e3nnLinear(self.gated, self.irreps_out, bias=True)
        self.linear_down = e3nnLinear(self.rejector.irreps_out.simplify(), (gates + self.gated).simplify(), bias=True)
        self.C = C
        self._gate_lay = (GMLayout(self.linear_down.irreps_out), GMLayout(self.gated))
        self.edge_info = MLP([num_radial] + list(radial_hidden) + [self.rejector.weight_numel])
        if layer > 0:
            self.resnetBB = e3nnElementLinear(self.irreps_in, irreps_sc, num_elements, bias=True)

    def forward(self, x, sp: SpeciesPlan, R, Y, plan: ops.EdgePlan):
        """x: group-major node features in species-sorted row order."""
        if hasattr(self, "resnetBB") and not (ops.MODE.double or ops.MODE.export) \
                and _frozen(self.linear_up, self.resnetBB):
            up, sc = _SharedInputLinearsFn.apply(x.contiguous(), self.linear_up, None, self.resnetBB, sp.ranges)
        else:
            sc = self.resnetBB(x, sp) if hasattr(self, "resnetBB") else None
            up = self.linear_up(x)
        x = _exchange_ghosts(up, self.linear_up.irreps_out, sp, self.layer)
        lay = ops.LAYOUT_IN1_GROUPED | ops.LAYOUT_OUT_GROUPED
        pairs = sp.pairs
        if ops.MODE.double:
            m = self.rejector(x, Y, self.edge_info(R), plan, lay, sp.node_map)
        elif pairs is not None and self.edge_info.fused:
            # the radial weights depend on the edge length only: made once per
            # edge pair and read by both directions
            h = self.edge_info.hidden(sp.pair_radial(R))
            m = self.rejector.paired(x, Y, h, *self.edge_info.last_layer(), plan, pairs, lay, sp.node_map)
        elif RADIAL_FUSED_TP and self.edge_info.fused and ops.rtp_supported(x.dtype, self.rejector.C, 64):
            m = self.rejector.radial_fused(x, Y, self.edge_info.hidden(R), *self.edge_info.last_layer(), plan, lay,
                                           sp.node_map)
        else:
            m = self.rejector(x, Y, self.edge_info(R), plan, lay, sp.node_map)
        # linear_down(m) / avg_num_neighbors, the division in the GEMM scale
        m = self.linear_down(m, alpha=1.0 / self.avg_num_neighbors)
        m = self.linear_nonlinearity(_gate(m, *self._gate_lay, self.C))
        return m, sc


class TeceInteraction(torch.nn.Module):
    """``OAM20260705Interaction`` (``tace/models/_e3nn/inter.py:440-519``): the
    cgtp interaction's linears, radial MLP and gate around the TECE
    convolution (``tace_amd.tece``), without scatter normalisation."""

    def __init__(self, layer, num_layers, irreps_in, C, Lmax, lmax, mmax, num_elements, radial_hidden, num_radial,
                 num_head, edge_ace_hidden):
        super().__init__()
        from .tece import TeceConvolution
        self.layer = layer
        self.irreps_in = Irreps(irreps_in)
        if self.irreps_in.lmax < 1:
            raise ValueError("uv_so2 interactions need l > 0 inputs (inter.py:458-461)")
        sh = spherical_harmonics_irreps(lmax)
        self.irreps_out = (possible_tp_irreps(self.irreps_in, sh, False, lmax) * C).regroup()
        if [ir.l for _, ir in self.irreps_out] != list(range(lmax + 1)):
            raise NotImplementedError("TECE output must be one C block per l = 0..lmax")
        if layer == num_layers - 1:
            irreps_sc = (Irreps("0e") * C).regroup()
        else:
            irreps_sc = (possible_tp_irreps(self.irreps_in, sh, False, Lmax) * C).regroup()
        self.linear_up = e3nnLinear(self.irreps_in, self.irreps_in, bias=True)
        self.rejector = TeceConvolution(mmax, lmax, C, num_head, edge_ace_hidden, num_radial)
        self.gated = Irreps([(C, ir) for _, ir in self.irreps_out])
        gates = Irreps([(C, Irrep("0e")) for _ in self.gated])
        self.linear_nonlinearity = e3nnLinear(self.gated, self.irreps_out, bias=True)
        self.linear_down = e3nnLinear(Irreps([(C, ir) for _, ir in self.irreps_out]), (gates + self.gated).simplify(),
                                      bias=True)
        self.edge_info = MLP([num_radial] + list(radial_hidden) + [self.rejector.weight_numel])
        if layer > 0:
            self.resnetBB = e3nnElementLinear(self.irreps_in, irreps_sc, num_elements, bias=True)
        self.C = C
        self._gate_lay = (GMLayout(self.linear_down.irreps_out), GMLayout(self.gated))
        # edges per receiver chunk: above this the convolution runs chunk by
        # chunk (the fused operator keeps a chunk's intermediates for the
        # backward while HBM allows, else recomputes them).  At the 101k-atom
        # bcc Fe box: 2^18 -> 333, 2^19 -> 321, 2^20 -> 317 ms/step (171, 180,
        # 196 GB peak); 2^21: 316 ms at 230 GB
        self.chunk_edges = 1 << 20

    def forward(self, x, sp: SpeciesPlan, R, plan: ops.EdgePlan, src, dst, wigner):
        from . import tece
        sc = self.resnetBB(x, sp) if hasattr(self, "resnetBB") else None
        x = _exchange_ghosts(self.linear_up(x), self.linear_up.irreps_out, sp, self.layer)
        if ops.MODE.double:
            # training: the whole convolution as torch operations (twice differentiable)
            msg = self.rejector(x, self.edge_info(R), plan, sp.node_map, src, dst, wigner, R)
        elif tece.FUSED and tece.fused_supported(self.rejector, self.edge_info):
            msg = tece.tece_fused(self.rejector, self.edge_info, x, sp.node_map, R, plan, src, dst, wigner,
                                  self.chunk_edges)
        elif plan.n_edges <= self.chunk_edges:
            msg = self.rejector(x, self.edge_info(R), plan, sp.node_map, src, dst, wigner, R)
        else:
            msg = self._chunked(x, sp, R, plan, src, dst, wigner)
        m = self.linear_down(msg)
        m = self.linear_nonlinearity(_gate(m, *self._gate_lay, self.C))
        return m, sc


    def _chunked(self, x, sp: SpeciesPlan, R, plan: ops.EdgePlan, src, dst, wigner):
        """The convolution over receiver chunks, each under activation
        checkpointing; chunk outputs are assembled in node order and moved to
        the group-major feature-row order."""
        from torch.utils.checkpoint import checkpoint

        from .tece import receiver_chunks, sub_plan
        if plan.eid is not None:  # group the edges by receiver first
            order = plan.eid.long()
            R, wigner, src, dst = R[order], wigner[order], src[order], dst[order]
            plan = ops.EdgePlan(plan.n_nodes, plan.n_edges, plan.rowptr, src.to(torch.int32).contiguous(), None)
        conv, C, L = self.rejector, self.C, self.rejector.lmax
        x_lc = conv.node_components(x)
        rows = sp.node_map.long()
        outs = []
        for n0, n1, e0, e1 in receiver_chunks(plan, self.chunk_edges):
            pc = sub_plan(plan, n0, n1, e0, e1)
            rs, rd, dl = rows[src[e0:e1]], rows[dst[e0:e1]], dst[e0:e1] - n0

            def run(x_lc, R_c, W_c, pc=pc, rs=rs, rd=rd, dl=dl):
                return conv.edges(x_lc, self.edge_info(R_c), rs, rd, pc, None, dl, W_c, R_c)

            outs.append(checkpoint(run, x_lc, R[e0:e1], wigner[e0:e1], use_reentrant=False))
        blocks = []
        for l in range(L + 1):
            d = 2 * l + 1
            node_order = torch.cat([o.view(-1)[o.shape[0] * C * l * l:o.shape[0] * C * (l + 1) ** 2]
                                    .view(o.shape[0], d, C) for o in outs])
            blocks.append(node_order.index_select(0, sp.perm).reshape(-1))
        return torch.cat(blocks).view(x.shape[0], -1)


class _SplitUpFn(torch.autograd.Function):
    """``CgtpACE._split_up_torch`` with a one-pass backward: the gradient of
    ``linear_up``'s output is written block by block into one uninitialised
    tensor (every element is covered: the path weights' SiLU gradient, then
    the node and base halves of each doubled block), instead of autograd's
    zero-filled full-size gradient per slice and their sums."""

    @staticmethod
    def forward(ctx, u, mod):
        ctx.mod = mod
        ctx.save_for_backward(u)
        return mod._split_up_torch(u)

    @staticmethod
    def backward(ctx, g_node, g_base, g_ws):
        (u,) = ctx.saved_tensors
        mod = ctx.mod
        C, lay = mod.C, mod._up_lay
        gu = torch.empty_like(u)
        g0 = lay.block(gu, 0)
        if g_ws is None:
            g0.zero_()
        else:
            torch.ops.aten.silu_backward.grad_input(g_ws.contiguous().view(g0.shape), lay.block(u, 0), grad_input=g0)
        # the node and base halves of every doubled block in one strided copy each
        dbl = mod._doubled_rows(gu)
        R = dbl.shape[0]
        for half, g in ((dbl[:, :C], g_node), (dbl[:, C:], g_base)):
            if g is None:
                half.zero_()
            else:
                half.copy_(g.reshape(-1)[:R * C].view(R, C))
        return gu, None


def _frozen(*mods: torch.nn.Module) -> bool:
    """No parameter of these modules takes a gradient (the inference path)."""
    return not any(p.requires_grad for m in mods for p in m.parameters())


class _SharedInputLinearsFn(torch.autograd.Function):
    """Two linears of one input as one autograd node (the interaction's
    linear_up and its resnet linear, ``inter.py:212-227``): the second's input
    gradient is added to the first's in its GEMM epilogue instead of autograd
    summing two gradient tensors."""

    @staticmethod
    def forward(ctx, x, lin_a, ranges_a, lin_b, ranges_b):
        ra = _linear_route(x, lin_a.weight, lin_a.lay, ranges_a)
        rb = _linear_route(x, lin_b.weight, lin_b.lay, ranges_b)
        ctx.args = (lin_a, ra, lin_b, rb)
        return (_linear_apply(x, lin_a.weight, lin_a.bias, lin_a.lay, *ra, 1.0),
                _linear_apply(x, lin_b.weight, lin_b.bias, lin_b.lay, *rb, 1.0))

    @staticmethod
    def backward(ctx, ga, gb):
        lin_a, ra, lin_b, rb = ctx.args
        gx = None
        if ga is not None:
            gx = _linear_apply(ga.contiguous(), lin_a.weight, None, lin_a.lay, *ra, 1.0, kind="bwd")
        if gb is not None:
            gx = _linear_apply(gb.contiguous(), lin_b.weight, None, lin_b.lay, *rb, 1.0, kind="bwd", out=gx,
                               addend=gx)
        return gx, None, None, None, None


class _ProductBasisFn(torch.autograd.Function):
    """``CgtpACE.forward`` (``prod.py:216-266``) without path weights as one
    autograd node: out = linear(sum_nu coefs[nu - 1](f_nu)) + sc with f_1 = x,
    f_nu = uuu(f_{nu-1}, x).  The coefficient linears add into one buffer in
    their GEMM epilogues; in the backward each f_nu's gradient through its
    coefficient linear is added in that GEMM's epilogue to the one through
    the next product, and the products' gradients of x are added to g_x in
    their part sums (the uuu backward's accumulate mode)."""

    @staticmethod
    def forward(ctx, x, sc, mod: "CgtpACE", sp):
        ranges = None if mod.agnostic else sp.ranges
        routes = []

        def coef(k, inp, acc=None):
            L = mod.coefs[k]
            r = _linear_route(inp, L.weight, L.lay, ranges)
            routes.append(r)
            return _linear_apply(inp, L.weight, L.bias, L.lay, *r, 1.0, out=acc, addend=acc)

        outs = coef(0, x)
        feats, x1s = x, []
        for nu in range(2, mod.correlation + 1):
            ace = mod.aces[nu - 2]
            f = ops.launch_uuu_fwd(feats, x, None, ops.find_variant(ace.key), ace.C, ops.LAYOUT_ALL_GROUPED)
            x1s.append(feats)
            coef(nu - 1, f, outs)
            feats = f
        L = mod.linear
        fr = _linear_route(outs, L.weight, L.lay, None)
        ctx.routes, ctx.final, ctx.mod, ctx.has_sc = routes, fr, mod, sc is not None
        ctx.save_for_backward(x, *x1s[1:])
        return _linear_apply(outs, L.weight, L.bias, L.lay, *fr, 1.0, addend=sc)

    @staticmethod
    def backward(ctx, g):
        mod = ctx.mod
        x, *fs = ctx.saved_tensors   # fs: f_2 .. f_{correlation-1}
        g = g.contiguous()
        L = mod.linear
        g_outs = _linear_apply(g, L.weight, None, L.lay, *ctx.final, 1.0, kind="bwd")

        def coef_bwd(k):
            C = mod.coefs[k]
            return _linear_apply(g_outs, C.weight, None, C.lay, *ctx.routes[k], 1.0, kind="bwd")

        g_x = coef_bwd(0)
        if mod.correlation >= 2:
            g_f = coef_bwd(mod.correlation - 1)
            for nu in range(mod.correlation, 2, -1):
                ace = mod.aces[nu - 2]
                # the gradient of f_{nu-1} through this product (new), then
                # through its coefficient linear (added in the GEMM epilogue)
                g_prev, _, _ = ops.launch_uuu_bwd(fs[nu - 3], x, None, g_f, ops.find_variant(ace.key), ace.C,
                                                  ops.LAYOUT_ALL_GROUPED, acc2=g_x)
                C = mod.coefs[nu - 2]
                _linear_apply(g_outs, C.weight, None, C.lay, *ctx.routes[nu - 2], 1.0, kind="bwd", out=g_prev,
                              addend=g_prev)
                g_f = g_prev
            # f_2 = uuu(x, x): both of its gradients into g_x
            ace = mod.aces[0]
            ops.launch_uuu_bwd(x, x, None, g_f, ops.find_variant(ace.key), ace.C, ops.LAYOUT_ALL_GROUPED, acc1=g_x,
                               acc2=g_x)
        return g_x, (g if ctx.has_sc else None), None, None


class CgtpACE(torch.nn.Module):
    """``CgtpACE`` (``tace/models/_e3nn/prod.py:20-266``): nu-chain of uuu products
    and per-species coefficient linears, evaluated on species-sorted nodes."""

    def __init__(self, layer, num_layers, irreps_in, C, Lmax, lmax, correlation, num_elements, agnostic=False,
                 bilinear: bool = False):
        super().__init__()
        last = layer == num_layers - 1
        self.correlation = correlation
        self.agnostic = agnostic
        self.bilinear = bilinear
        if bilinear and correlation != 2:
            raise ValueError("the bilinear-gate product basis needs correlation 2 (prod.py:83-84)")
        irreps_in = Irreps(irreps_in)
        hidden = Irreps([(C, ir) for _, ir in irreps_in])
        tp_out = []
        for nu in range(2, correlation + 1):
            if nu == correlation:
                tp_out.append((Irreps("0e") * C).regroup() if last else
                              (possible_tp_irreps(hidden, hidden, False, Lmax) * C).regroup())
            else:
                tp_out.append(possible_tp_irreps(hidden, hidden, False, lmax))
        if correlation == 1:
            coefs_out = Irreps([(C, ir) for _, ir in irreps_in if ir.l <= Lmax])
        else:
            coefs_out = (possible_tp_irreps(irreps_in, irreps_in, False, Lmax) * C).regroup()
        if last:
            coefs_out = (Irreps("0e") * C).regroup()
        self.irreps_out = Irreps([(C, ir) for _, ir in coefs_out])

        def mk(irr):
            if agnostic:
                return e3nnLinear(irr, coefs_out, bias=True)
            return e3nnElementLinear(irr, coefs_out, num_elements, bias=True)

        self.coefs = torch.nn.ModuleList([mk(Irreps([(C, ir) for _, ir in hidden]).simplify())])
        self.aces = torch.nn.ModuleList()
        # bilinear gate (prod.py:83-87, 126-147, 178-214): second operand =
        # hidden irreps + a C x 0e block of ones, per-node path weights
        base = hidden + Irreps([(C, Irrep("0e"))]) if bilinear else hidden
        in1 = hidden
        for nu in range(2, correlation + 1):
            ace = uuuTensorProduct(in1, base, tp_out[nu - 2], identical_inputs=(nu == 2 and not bilinear))
            self.aces.append(ace)
            self.coefs.append(mk(Irreps([(C, ir) for _, ir in ace.irreps_out]).simplify()))
            in1 = ace.irreps_out
        self.linear = e3nnLinear(Irreps([(C, ir) for _, ir in coefs_out]), self.irreps_out, bias=True)
        self.C = C
        if bilinear:
            self.num_gate = sum(a.weight_numel for a in self.aces)
            self.double = [(2 * C, ir) for _, ir in hidden]
            self.linear_up = e3nnLinear(irreps_in, Irreps(f"{self.num_gate}x0e") + Irreps(self.double), bias=True)
            self._up_lay = GMLayout(self.linear_up.irreps_out)

    def _split_up(self, x):
        """linear_up output -> (node features, base features + ones, path weights),
        all group-major (``prod.py:178-214``)."""
        u = self.linear_up(x)
        if not ops.MODE.double:
            return _SplitUpFn.apply(u, self)
        return self._split_up_torch(u)

    def _split_up_torch(self, u):
        """The doubled blocks follow the path weights in ``u`` and the node
        blocks follow each other in the group-major output in the same order,
        so every doubled block's rows [Z (2l+1), 2C] together are one [R, 2C]
        matrix whose halves are the node and base features: one strided copy
        each (and a block of ones after the base features)."""
        Z, C = u.shape[0], self.C
        ws = torch.nn.functional.silu(self._up_lay.block(u, 0))
        dbl = self._doubled_rows(u)
        node = dbl[:, :C].contiguous().view(Z, -1)
        R = dbl.shape[0]
        base = u.new_empty(Z, (R // Z + 1) * C)
        bf = base.view(-1)
        bf[:R * C].view(R, C).copy_(dbl[:, C:])
        bf[R * C:].fill_(1.0)
        return node, base, ws

    def _doubled_rows(self, u):
        """All doubled blocks of ``linear_up``'s output as one [Z sum(2l+1), 2C] view."""
        Z, C = u.shape[0], self.C
        s0 = self._up_lay.blocks[1][0]
        return u.view(-1)[Z * s0:].view(-1, 2 * C)

    def forward(self, x, sp: SpeciesPlan, sc):
        """x: group-major node features in species-sorted row order."""
        if not (self.bilinear or ops.MODE.double or ops.MODE.export) and _frozen(self):
            return _ProductBasisFn.apply(x.contiguous(), None if sc is None else sc.contiguous(), self, sp)
        ws = base = None
        if self.bilinear:
            x, base, ws = self._split_up(x)
        if self.agnostic:
            outs = self.coefs[0](x)
        else:
            outs = self.coefs[0](x, sp)
        feats = x
        for nu in range(2, self.correlation + 1):
            if self.bilinear:
                feats = self.aces[nu - 2](feats, base, ops.LAYOUT_ALL_GROUPED, ws)
            else:
                feats = self.aces[nu - 2](feats, x, ops.LAYOUT_ALL_GROUPED)
            outs = outs + (self.coefs[nu - 1](feats) if self.agnostic else self.coefs[nu - 1](feats, sp))
        outs = self.linear(outs)
        return outs + sc if sc is not None else outs


class ScalarReadOut(torch.nn.Module):
    """Last-layer ``ScalarReadOut`` (``tace/models/_e3nn/readout.py:36-84``)."""

    def __init__(self, irreps_in, hidden=(16,)):
        super().__init__()
        dims = [Irreps(irreps_in)] + [Irreps(f"{h}x0e") for h in hidden] + [Irreps("1x0e")]
        self.linear2 = torch.nn.ModuleList(e3nnLinear(a, b, bias=False) for a, b in zip(dims, dims[1:]))

    def forward(self, x):
        for lin in self.linear2[:-1]:
            x = torch.nn.functional.silu(lin(x)) * SILU_CST
        return self.linear2[-1](x)


class _Buffers(torch.nn.Module):
    pass


class LinearNodeEmbedding(torch.nn.Module):
    def __init__(self, S, C):
        super().__init__()
        self.elem_emb1 = e3nnLinear(f"{S}x0e", f"{C}x0e", bias=False)

    def forward(self, attrs):
        return self.elem_emb1(attrs)


class RadialBasis(torch.nn.Module):
    """Buffers of ``RadialBasis`` (j0 + c2poly, ``radial.py:43-84, 437-472, 877-993``)."""

    def __init__(self, cutoff, num_basis, p):
        super().__init__()
        self.cutoff_fn = _Buffers()
        self.cutoff_fn.register_buffer("p", torch.tensor(p, dtype=torch.int))
        self.cutoff_fn.register_buffer("cutoff", torch.tensor(cutoff, dtype=torch.get_default_dtype()))
        self.radial_fn = _Buffers()
        self.radial_fn.register_buffer("bessel_weights", math.pi / cutoff * torch.linspace(
            1.0, num_basis, num_basis, dtype=torch.get_default_dtype()))
        self.radial_fn.register_buffer("cutoff", torch.tensor(cutoff, dtype=torch.get_default_dtype()))
        self.radial_fn.register_buffer("prefactor", torch.tensor(math.sqrt(2.0 / cutoff),
                                                                 dtype=torch.get_default_dtype()))
        self.num_basis = num_basis


_SUPPORTED = dict(node_embedding="linear", edge_embedding="identity", edge_update="identity")


def _check_supported(cfg):
    for k, v in _SUPPORTED.items():
        if cfg.get(k, {}).get("type", v) != v:
            raise NotImplementedError(f"{k}.type={cfg[k]['type']!r} is not on the MI355X path")
    ab = cfg.get("atomic_basis", {})
    types = ab.get("type", "cgtp")
    types = types if isinstance(types, list) else [types]
    for t in types:
        if t not in ("cgtp", "uv_so2"):
            raise NotImplementedError(f"atomic_basis.type={t!r} is not on the MI355X path")
    if "uv_so2" in types:
        if cfg.get("mmax", cfg["lmax"]) != cfg["lmax"]:
            raise NotImplementedError("uv_so2 on the MI355X path needs mmax == lmax")
        if ab.get("edge_nonlinear", "so2_sigmoid_gate") != "so2_sigmoid_gate":
            raise NotImplementedError("uv_so2 needs edge_nonlinear=so2_sigmoid_gate")
    nl = ab.get("nonlinear", "sigmoid_gate")
    for t in (nl if isinstance(nl, list) else [nl]):
        if t != "sigmoid_gate":
            raise NotImplementedError(f"atomic_basis.nonlinear={t!r} is not on the MI355X path")
    if not ab.get("gate_m0", True) or ab.get("scatter_norm", "avg_num_neighbors") != "avg_num_neighbors":
        raise NotImplementedError("only gate_m0=True and scatter_norm=avg_num_neighbors are supported")
    rb = cfg.get("radial_basis", {})
    if rb.get("radial_basis", "j0") not in ("j0", "bessel") or rb.get("cutoff_fn", "c2poly") != "c2poly" \
            or not rb.get("apply_cutoff", True) or rb.get("bias", False) or rb.get("distance_transform"):
        raise NotImplementedError("only j0 Bessel x c2poly radial basis (apply_cutoff, no bias) is supported")
    pb = cfg.get("product_basis", {})
    if pb.get("type", "cgtp") not in ("cgtp",) and not isinstance(pb.get("type"), list):
        raise NotImplementedError("only product_basis.type=cgtp is supported")
    if pb.get("num_expert") not in (None, 1):
        raise NotImplementedError("mixture-of-experts product basis is not on the MI355X path")
    if pb.get("nonlinear") not in (None, "silu_bilineargate"):
        raise NotImplementedError(f"product_basis.nonlinear={pb.get('nonlinear')!r} is not on the MI355X path")
    if pb.get("nonlinear") == "silu_bilineargate":
        corr = pb.get("correlation", 3)
        if any(c != 2 for c in (corr if isinstance(corr, list) else [corr])):
            raise NotImplementedError("the bilinear-gate product basis needs correlation 2 (prod.py:83-84)")
    rs = cfg.get("resnet", {})
    if rs.get("type", "BB") != "BB" or rs.get("linear_type", "aware") != "aware" or rs.get("use_first_resnet"):
        raise NotImplementedError("only resnet type BB, element-aware, no first resnet is supported")
    if cfg.get("parity", False):
        raise NotImplementedError("parity=True is not on the MI355X path")
    if len(cfg.get("fidelity", [0])) != 1:
        raise NotImplementedError("multi-fidelity heads are not on the MI355X path")


class Representation(torch.nn.Module):
    """``Representation`` (``tace/models/_e3nn/representation.py:28-429``)."""

    def __init__(self, cfg):
        super().__init__()
        S = len(cfg["atomic_numbers"])
        C, L, Lmax = cfg["num_channel"], cfg["lmax"], cfg["Lmax"]
        self.register_buffer("atomic_numbers", torch.tensor(cfg["atomic_numbers"], dtype=torch.int64))
        rb = cfg["radial_basis"]
        self.radial_basis = RadialBasis(cfg["cutoff"], rb["num_radial_basis"], rb["polynomial_cutoff"])
        self.lmax = L
        self.node_embedding = LinearNodeEmbedding(S, C)
        nl = cfg["num_layers"]
        corr = cfg["product_basis"]["correlation"]
        corr = corr if isinstance(corr, list) else [corr] * nl
        self.interactions = torch.nn.ModuleList()
        self.products = torch.nn.ModuleList()
        ab = cfg.get("atomic_basis", {})
        types = ab.get("type", "cgtp")
        types = types if isinstance(types, list) else [types] * nl
        self.use_so2 = "uv_so2" in types
        pb = cfg["product_basis"]
        bilinear = pb.get("nonlinear") == "silu_bilineargate"
        irreps = Irreps(f"{C}x0e")
        for layer in range(nl):
            if types[layer] == "uv_so2":
                inter = TeceInteraction(layer, nl, irreps, C, Lmax, L, cfg.get("mmax", L), S, rb["hidden"],
                                        rb["num_radial_basis"], ab.get("num_head") or 1,
                                        ab.get("edge_ace_hidden") or C)
            else:
                inter = O3CgtpInteraction(layer, nl, irreps, C, Lmax, L, corr[layer], S, cfg["avg_num_neighbors"],
                                          rb["hidden"], rb["num_radial_basis"])
            self.interactions.append(inter)
            prod = CgtpACE(layer, nl, inter.irreps_out, C, Lmax, L, corr[layer], S, pb.get("agnostic", False),
                           bilinear)
            self.products.append(prod)
            irreps = prod.irreps_out

    def _basis_scalars(self):
        """(prefactor, cutoff, p) of the radial basis as Python numbers, read
        from the buffers once and again only after a buffer is replaced or
        written (reading a device scalar stops the host until the GPU idles)."""
        rb = self.radial_basis
        bufs = (rb.radial_fn.prefactor, rb.cutoff_fn.cutoff, rb.cutoff_fn.p)
        key = tuple((id(b), b._version) if torch.is_tensor(b) else (None, b) for b in bufs)
        cached = getattr(self, "_basis_cache", None)
        if cached is None or cached[0] != key or any(c is not b for c, b in zip(cached[2], bufs)):
            self._basis_cache = (key, (float(bufs[0]), float(bufs[1]), int(bufs[2])), bufs)
        return self._basis_cache[1]

    def edge_features(self, edge_vector: torch.Tensor):
        rb = self.radial_basis
        pref, cut, p = self._basis_scalars()
        return ops.edge_basis(edge_vector, rb.radial_fn.bessel_weights.to(edge_vector.dtype), pref, cut, p,
                              self.lmax)

    def forward(self, attrs, plan: ops.EdgePlan, edge_vector, sp: SpeciesPlan, edge_index=None):
        """Node features (group-major, rows in ``sp``'s species-sorted order)."""
        R, Y = self.edge_features(edge_vector)
        wigner = ops.edge_wigner(edge_vector, self.lmax) if self.use_so2 else None
        x = self.node_embedding(attrs.index_select(0, sp.perm))
        for inter, prod in zip(self.interactions, self.products):
            if isinstance(inter, TeceInteraction):
                x, sc = inter(x, sp, R, plan, edge_index[0], edge_index[1], wigner)
            else:
                x, sc = inter(x, sp, R, Y, plan)
            x = prod(x, sp, sc)
        return x


class TACE(torch.nn.Module):
    """MI355X ``e3nnTACE`` (energy readout; ``tace/models/_e3nn/tace.py:28-790``)."""

    def __init__(self, **cfg):
        super().__init__()
        cfg = copy.deepcopy(cfg)
        if "atomic_numbers" not in cfg or cfg["atomic_numbers"] is None:
            cfg["atomic_numbers"] = sorted({z for s in cfg["statistics"] for z in s["atomic_numbers"]})
        if "avg_num_neighbors" not in cfg:
            cfg["avg_num_neighbors"] = sum(s["avg_num_neighbors"] for s in cfg["statistics"]) / len(cfg["statistics"])
        _check_supported(cfg)
        self.model_config = cfg
        self.target_property = list(cfg["target_property"])
        self.embedding_property = list(cfg.get("embedding_property", []))
        self.statistics = cfg["statistics"]
        self.fidelity = cfg.get("fidelity", [dict(name="PBE", atomic_energy=None)])
        self.max_neighbors = cfg.get("max_neighbors")
        zs = cfg["atomic_numbers"]
        self.register_buffer("cutoff", torch.tensor(cfg["cutoff"], dtype=torch.get_default_dtype()))
        self.register_buffer("atomic_numbers", torch.tensor(zs, dtype=torch.int64))
        self.representation = Representation(cfg)
        C = cfg["num_channel"]
        self.energy_readouts = torch.nn.ModuleList([ScalarReadOut(f"{C}x0e", cfg["readout_emlp"]["hidden"])])
        stats = cfg["statistics"]
        self.atomic_energy_layer = _Buffers()
        self.atomic_energy_layer.register_buffer("atomic_energy", torch.tensor(
            [[float({int(k): v for k, v in s["atomic_energy"].items()}.get(z, 0.0)) for z in zs] for s in stats],
            dtype=torch.get_default_dtype()))
        self.scale_shift = _Buffers()
        self.scale_shift.register_buffer("atomic_numbers", torch.tensor(zs, dtype=torch.int64))
        self.scale_shift.register_buffer("scale", torch.tensor(
            [[float({int(k): v for k, v in s["rms_forces"].items()}.get(z, 1.0)) for z in zs] for s in stats],
            dtype=torch.get_default_dtype()))
        self.scale_shift.register_buffer("shift", torch.zeros(len(stats), len(zs), dtype=torch.get_default_dtype()))

    def energy(self, data, plan: ops.EdgePlan, edge_vector, exchange=None, pairs: Optional[ops.EdgePairs] = None):
        """Energy branch of ``readout_fn`` (``tace.py:356-418``) + ``ScaleShift``
        (``blocks.py:289-379``), fidelity 0.  ``exchange``: LAMMPS ML-IAP data
        for the per-layer ghost exchange (several domains).  ``pairs``: make
        the radial weights once per edge pair (the energy and its gradients
        with respect to positions and cell are unchanged; the gradient with
        respect to each edge vector is not split between the two directions,
        so callers that want per-edge gradients pass None)."""
        attrs, batch, ptr = data["node_attrs"], data["batch"], data["ptr"]
        num_graphs = ptr.numel() - 1
        sp = SpeciesPlan(attrs, exchange, pairs, natural=ops.MODE.export, counts=_opt(data, "_species_counts"))
        x = self.representation(attrs, plan, edge_vector, sp, data["edge_index"])
        # E0(Z_n) (OneHotToAtomicEnergy, blocks.py:250-286) as a masked row sum (a
        # [N, S] x [S, 1] product would be a library GEMM launch)
        e_base = (attrs * self.atomic_energy_layer.atomic_energy[0]).sum(-1)
        e_node = self.energy_readouts[0](x)[:, 0].index_select(0, sp.inv)  # back to node order
        num_nodes = ptr[1:] - ptr[:-1]
        ei = data["edge_index"]
        if isinstance(plan, ops.EdgePlan) and plan.n_nodes == attrs.shape[0]:
            # edges per graph from the receiver CSR (graph g's receivers are
            # nodes ptr[g] .. ptr[g+1]-1): no per-edge atomics on a few counters
            rp = plan.rowptr.long()
            num_edges = rp[ptr[1:]] - rp[ptr[:-1]]
        else:
            num_edges = torch.zeros(num_graphs, dtype=torch.int64, device=attrs.device)
            if ei.numel():
                num_edges = num_edges.index_add(0, batch[ei[1]], torch.ones_like(ei[1]))
        isolated = ((num_nodes == 1) & (num_edges == 0))[batch]
        scale = (attrs * self.scale_shift.scale[0]).sum(-1)
        e_node = e_node * torch.where(isolated, torch.zeros_like(scale), scale)
        shift = (attrs * self.scale_shift.shift[0]).sum(-1)
        e_node = e_node + torch.where(isolated, torch.zeros_like(shift), shift)
        # scatter_sum of the base and the model energies (tace.py:364, 416), per
        # graph in node order
        sums = ops.graph_sum(torch.stack([e_base, e_node], 1), ptr, batch)
        E = sums[:, 0] + sums[:, 1]
        return E, e_base + e_node


def set_tece_channel_mixing(model: torch.nn.Module, dtype: Optional[torch.dtype]):
    """Precision of the TECE SO(2) channel-mixing GEMMs: None (the model's
    own, default) or torch.bfloat16 (bf16 operands, fp32 accumulation and
    output; the configuration-5 option).  Returns the number of convolutions set."""
    from .tece import TeceConvolution
    if dtype not in (None, torch.bfloat16):
        raise ValueError("channel mixing precision must be None or torch.bfloat16")
    n = 0
    for m in model.modules():
        if isinstance(m, TeceConvolution):
            m.mixing = dtype
            n += 1
    return n


def _atomic_virials(vec, edge_forces, edge_index, lattice, batch, n_nodes):
    """``compute_atomic_virials_stresses`` (``tace/models/utils.py:82-115``):
    each edge's f (x) r split half to its sender and half to its receiver,
    symmetrised and negated; stresses = -virials / cell volume."""
    ev = edge_forces.unsqueeze(-1) * vec.unsqueeze(-2)  # [E, 3, 3], f_i r_j
    av = torch.zeros(n_nodes, 3, 3, dtype=vec.dtype, device=vec.device)
    ops.scatter_add_rows(ops.scatter_add_rows(av, edge_index[0], ev), edge_index[1], ev)
    av = -0.5 * (av + av.transpose(-1, -2)) / 2
    vol = torch.linalg.det(lattice).abs()
    st = -av / vol[batch].view(-1, 1, 1)
    return av, torch.where(st.abs() < 1e10, st, torch.zeros_like(st))


# ------------------------------------------------------------ caller API ----
# target properties whose first derivative this path computes (the
# first-derivative rows of the reference's PROPERTY table,
# tace/dataset/quantity.py), and the compute_* switches it honours
_FIRST_DERIVATIVE = ("forces", "stress", "virials", "edge_forces", "atomic_virials", "atomic_stresses")
_SUPPORTED_FLAGS = frozenset("compute_" + p for p in ("energy", "node_energy") + _FIRST_DERIVATIVE)


class ComputeFlags:
    """The reference's ``ComputeFlag`` (``tace/dataset/quantity.py:917-922``):
    one boolean ``compute_<property>`` per property, False unless set.
    Callers switch outputs on and off through it (``interface/torchsim/
    torchsim.py:131-137``, ``interface/lammps/mliap.py:25-34``)."""

    def __init__(self, **on: bool):
        for k, v in on.items():
            setattr(self, k, bool(v))

    def __getattr__(self, name: str) -> bool:
        if name.startswith("compute_"):
            return False
        raise AttributeError(name)

    def enabled(self) -> List[str]:
        return sorted(k for k, v in vars(self).items() if v)

    def __repr__(self) -> str:
        return f"ComputeFlags({', '.join(self.enabled())})"


class TorchElement:
    """The model's element table, as ``TorchElement``
    (``tace/dataset/element.py:41-64``): sorted atomic numbers, ``z2idx`` and
    ``z2onehot`` (an atomic number outside the table raises in ``one_hot``)."""

    def __init__(self, zs: Sequence[int]):
        self.zs = sorted(int(z) for z in zs)
        self.num_elements = len(self.zs)
        self.lookup_table = torch.full((max(self.zs) + 1,), -1, dtype=torch.int64)
        self.lookup_table[torch.tensor(self.zs, dtype=torch.int64)] = torch.arange(self.num_elements)

    def z2idx(self, z: torch.Tensor) -> torch.Tensor:
        return self.lookup_table[z]

    def z2onehot(self, zs: torch.Tensor) -> torch.Tensor:
        idx = self.lookup_table.to(zs.device)[zs]
        return torch.nn.functional.one_hot(idx, num_classes=self.num_elements)

    def __len__(self) -> int:
        return len(self.zs)


def _opt(data, key: str):
    """data[key] or None, for plain dicts and torch_geometric batches alike."""
    return data[key] if key in data else None


class TensorModel(torch.nn.Module):
    """``TensorModel`` (``tace/models/adapter.py:23-452``) for energy, forces,
    stress/virials, edge forces and per-atom virials/stresses:
    ``forward(data) -> {energy, node_energy, forces, virials, stress,
    edge_forces, atomic_virials, atomic_stresses}`` (None where not computed).
    Which derivatives are taken follows ``flags`` (set from the target
    properties, ``adapter.py:410-426``, and overridable by the caller) and
    ``compute_first_derivative`` (``adapter.py:95``)."""

    def __init__(self, readout_fn: TACE):
        super().__init__()
        self.readout_fn = readout_fn
        self.fidelity_idx = 0
        self.lmp = False
        self._set_target_property()

    def _set_target_property(self) -> None:
        """``adapter.py:410-431``: flags and derivative switches from the
        target properties (no second-derivative targets on this path)."""
        tp = self.get_target_property()
        self.flags = ComputeFlags(**{f"compute_{k}": True for k in tp})
        self.compute_first_derivative = any(p in _FIRST_DERIVATIVE for p in tp)
        self.compute_second_derivative = False
        self.retain_graph = False
        self.create_graph = False

    # getters used by the ASE / TorchSim / LAMMPS callers (adapter.py:386-452)
    def get_cutoff(self) -> float:
        return float(self.readout_fn.cutoff.item())

    def get_atomic_numbers(self):
        return [int(z) for z in self.readout_fn.atomic_numbers.cpu().tolist()]

    def get_torch_element(self) -> TorchElement:
        return TorchElement(self.get_atomic_numbers())

    def get_model_dtype(self):
        return self.readout_fn.cutoff.dtype

    def get_target_property(self):
        return list(set(self.readout_fn.target_property))

    def get_embedding_property(self):
        return list(self.readout_fn.embedding_property)

    def get_max_neighbors(self):
        return self.readout_fn.max_neighbors

    def get_fidelity_idx(self) -> int:
        return int(self.fidelity_idx)

    def reset_fidelity_idx(self, fidelity_idx=0):
        if fidelity_idx is not None:
            self.fidelity_idx = fidelity_idx

    def reset_target_property(self, target_property):
        self.readout_fn.target_property = list(target_property)
        self._set_target_property()

    def load_state_dict(self, state_dict, strict: bool = True, assign: bool = False):
        """``load_state_dict`` that also takes a reference checkpoint as saved
        (``lightning/lit_model.py:597-610`` calls it on the model
        ``create_model`` built): keys of e3nn's internal modules are dropped
        and matrix-form weights (``TACE_USE_MATRIX_WEIGHT=1``,
        ``linear.py:322-327, 417-425``) are concatenated into the flat form."""
        sd = _reference_state_dict(self.state_dict(), state_dict)
        return super().load_state_dict(sd, strict=strict, assign=assign)

    @staticmethod
    def _ghost_owners(lmp_data, nlocal: int, nghosts: int, like: torch.Tensor) -> Optional[torch.Tensor]:
        """Local atom that each of the nlocal + nghosts LAMMPS atoms stands
        for, from one width-2 ``forward_exchange`` of (local index, a random
        token of this call) (``models/lammps.py:82-102`` semantics: ghost rows
        are copied from their owners).  None when some ghost's row carries
        another token: it is owned by another domain, and the model then runs
        the per-layer exchange instead."""
        ntotal = nlocal + nghosts
        ids = torch.arange(ntotal, device=like.device)
        if nghosts == 0:
            return ids
        if lmp_data is None or not hasattr(lmp_data, "forward_exchange"):
            raise RuntimeError("LAMMPS mode with ghost atoms needs lmp_data with forward_exchange")
        token = 1.0 + random.random()
        col = torch.zeros(ntotal, 2, dtype=like.dtype, device=like.device)
        col[:nlocal, 0] = torch.arange(nlocal, device=like.device, dtype=like.dtype)
        col[:nlocal, 1] = token
        out = torch.empty_like(col)
        lmp_data.forward_exchange(col, out, 2)
        if bool((out[nlocal:, 1] != token).any()):
            return None
        owner = out[:, 0].round().long()
        owner[:nlocal] = ids[:nlocal]
        if bool(((owner < 0) | (owner >= nlocal)).any()):
            raise RuntimeError("ghost exchange returned owners outside the local atoms")
        return owner

    def _forward_lammps(self, data: Dict[str, torch.Tensor]) -> Dict[str, Optional[torch.Tensor]]:
        """LAMMPS ML-IAP mode (``adapter.py:286-312``, ``mliap.py:113-151``):
        LAMMPS supplies pair vectors ``edge_vector`` [E, 3] for edges
        ``edge_index`` = [neighbour j, local i] over nlocal + nghosts atoms
        (``natoms``); returns the local energies and ``edge_forces`` =
        dE/d(edge_vector).  A ghost atom's features equal its owner's in every
        layer >= 1 (the reference's per-layer ghost exchange).  When every
        ghost is owned by this domain, each ghost sender is replaced by its
        owner and the graph is the periodic one on the local atoms (the sender
        CSR sums what the exchange's reverse pass would); otherwise the model
        runs on all nlocal + nghosts rows and exchanges the ghost rows through
        ``lmp_data`` before every interaction layer >= 1, as the reference
        does (``_e3nn/inter.py:228``, ``models/lammps.py:105-134``)."""
        vec = data["edge_vector"]
        if not vec.is_cuda:
            raise RuntimeError("tace_amd.TensorModel runs on the GPU only (edge_vector is on %s)" % vec.device)
        if not vec.requires_grad:
            vec = vec.detach().requires_grad_(True)
        ei = data["edge_index"]
        if ops.MODE.export:
            # exported program (LAMMPS AOTI inputs, tace/models/compile/aot.py:35-43):
            # nlocal from batch, every row of node_attrs a node, the ghost
            # exchange through the operator in every layer >= 1
            nlocal, n = data["batch"].shape[0], data["node_attrs"].shape[0]
            exchange = LAMMPS_PROGRAM_EXCHANGE
            plan = ops.TracedEdges(ei, n)
        else:
            nlocal, nghosts = (int(v) for v in data["natoms"])
            if ei.numel() and int(ei[1].max()) >= nlocal:
                raise ValueError("LAMMPS mode: every edge's receiver (edge_index[1]) must be a local atom")
            lmp_data = _opt(data, "lmp_data")
            owner = self._ghost_owners(lmp_data, nlocal, nghosts, vec)
            if owner is not None:
                ei = torch.stack([owner[ei[0]], ei[1]])
                n = nlocal
                exchange = None
            else:
                n = nlocal + nghosts
                exchange = lmp_data
            plan = ops.EdgePlan.from_edge_index(ei, n)
        attrs = data["node_attrs"][:n]
        d = dict(node_attrs=attrs, edge_index=ei, batch=torch.zeros(n, dtype=torch.int64, device=vec.device),
                 ptr=torch.arange(2, dtype=torch.int64, device=vec.device) * n)
        _, e_node = self.readout_fn.energy(d, plan, vec, exchange)
        e_node = e_node[:nlocal]
        E = e_node.sum().view(1)
        out: Dict[str, Optional[torch.Tensor]] = dict(energy=E.detach(), node_energy=e_node.detach(), forces=None,
                                                      stress=None, virials=None, edge_forces=None)
        if self.flags.compute_edge_forces:
            (g,) = torch.autograd.grad(E, [vec], grad_outputs=torch.ones_like(E), allow_unused=True)
            out["edge_forces"] = torch.zeros_like(vec) if g is None else g  # dE/dr_ij, as LAMMPS expects
        return out

    def forward(self, data: Dict[str, torch.Tensor]) -> Dict[str, Optional[torch.Tensor]]:
        if self.lmp or ("edge_vector" in data and "natoms" in data):
            return self._forward_lammps(data)
        fl = self.flags
        unsupported = [k for k in fl.enabled() if k not in _SUPPORTED_FLAGS]
        if unsupported:
            raise NotImplementedError(f"{unsupported} are not computed on the MI355X path")
        # adapter.py:69-87: the gradient inputs follow the flags
        want_f = fl.compute_forces
        want_s = fl.compute_stress or fl.compute_virials
        want_e = fl.compute_edge_forces or fl.compute_atomic_virials or fl.compute_atomic_stresses
        if (want_f or want_s or want_e) and not self.compute_first_derivative:
            raise RuntimeError("flags request derivatives but compute_first_derivative is False")
        dt = self.get_model_dtype()
        pos = data["positions"]
        if not pos.is_cuda:
            raise RuntimeError("tace_amd.TensorModel runs on the GPU only (positions are on %s)" % pos.device)
        pos = pos.detach().to(dt).requires_grad_(want_f or want_s or want_e)
        lattice, batch = data["lattice"].to(dt), data["batch"]
        shifts = data["edge_shifts"]
        if shifts.dtype != dt:
            shifts = shifts.to(dt)
        num_graphs = data["ptr"].numel() - 1
        inputs = [pos] if want_f else []
        if want_s:
            # compute_symmetric_displacement (tace/models/utils.py:50-79)
            disp = torch.zeros(num_graphs, 3, 3, dtype=pos.dtype, device=pos.device, requires_grad=True)
            sym = 0.5 * (disp + disp.transpose(-1, -2))
            # r + r . sym(eps), L + L . sym(eps) as broadcast products and sums over
            # the 3-long axis (batched 3 x 3 products would be library GEMM launches)
            pos_s = pos + (pos.unsqueeze(-1) * ops.graph_gather(sym, data["ptr"], batch)).sum(1)
            lat_s = lattice + (lattice.unsqueeze(-1) * sym.unsqueeze(1)).sum(2)
            inputs.append(disp)
        else:
            pos_s, lat_s = pos, lattice
        ei = data["edge_index"]
        if ops.MODE.export:
            plan = ops.TracedEdges(ei, pos.shape[0])
        else:
            plan = _opt(data, "_edge_plan") or ops.EdgePlan.from_edge_index(ei, pos.shape[0])
        # adapter.py:95-104: training (or create_graph) keeps the graph of the
        # derivatives, so that a loss on forces / stress can be differentiated
        # with respect to the parameters; the operators then take their
        # twice-differentiable form
        cg = bool(self.training or self.create_graph)
        with ops.differentiable_twice(cg or ops.MODE.export):
            return self._forward_graph(data, pos, lattice, batch, shifts, num_graphs, inputs, pos_s, lat_s, ei, plan,
                                       want_f, want_s, want_e, cg)

    def _forward_graph(self, data, pos, lattice, batch, shifts, num_graphs, inputs, pos_s, lat_s, ei, plan,
                       want_f: bool, want_s: bool, want_e: bool, cg: bool):
        pairs = None
        if PAIR_RADIAL and not ops.MODE.export and plan.n_edges and not want_e and not cg:
            sh32 = _opt(data, "_shifts32")
            pairs = plan.edge_pairs(sh32 if sh32 is not None else shifts)
        # prepare_graph (adapter.py:334-347) on the HIP edge-vector kernel; the
        # +1e-9 of the length is applied in the edge-basis kernel
        dst32 = _opt(data, "_dst32")
        if dst32 is None:
            dst32 = ei[1].to(torch.int32)
        egraph = None if (num_graphs == 1 and not ops.MODE.export) else batch[ei[0]].to(torch.int32)
        vec = ops.edge_vectors(pos_s, lat_s, shifts, plan, dst32, egraph)
        E, e_node = self.readout_fn.energy(data, plan, vec, pairs=pairs)
        out: Dict[str, Optional[torch.Tensor]] = dict(energy=E, node_energy=e_node, forces=None, virials=None,
                                                      stress=None, edge_forces=None, atomic_virials=None,
                                                      atomic_stresses=None)
        if want_e:
            inputs.append(vec)
        if inputs:
            grads = torch.autograd.grad(E, inputs, grad_outputs=torch.ones_like(E), allow_unused=True,
                                        retain_graph=cg or self.retain_graph, create_graph=cg)
            k = 0
            if want_f:
                out["forces"] = -grads[0] if grads[0] is not None else torch.zeros_like(pos)
                k = 1
            if want_s:
                V = -grads[k] if grads[k] is not None else torch.zeros_like(lattice)
                vol = torch.linalg.det(lattice).abs().view(-1, 1, 1)
                S = -V / vol
                out["virials"] = V
                out["stress"] = torch.where(S.abs() < 1e10, S, torch.zeros_like(S))
            if want_e:
                ef = grads[-1] if grads[-1] is not None else torch.zeros_like(vec)
                out["edge_forces"] = ef
                out["atomic_virials"], out["atomic_stresses"] = _atomic_virials(vec.detach(), ef, ei, lattice, batch,
                                                                                pos.shape[0])
        if not cg:
            out["energy"] = out["energy"].detach()
            out["node_energy"] = out["node_energy"].detach()
        return out


# ------------------------------------------------------------- checkpoints ----
_E3NN_INTERNAL = ("output_mask", "_compiled", ".tp.", ".sc.", ".act_gates.", ".mul.", "._bias_index",
                  "._bias_mask", ".cut.")


def _reference_state_dict(own: Dict[str, torch.Tensor], state_dict: Dict[str, torch.Tensor]) -> Dict[str, torch.Tensor]:
    """A reference ``state_dict`` mapped onto this model's keys.

    * Matrix-form weights (``TACE_USE_MATRIX_WEIGHT=1``): ``e3nnLinear``
      stores one ``weight.<i>`` of shape ``path_shape`` per o3.Linear
      instruction and ``e3nnElementLinear`` one of shape ``(num_elements,
      *path_shape)`` (``tace/models/linear.py:322-327, 417-425``); the flat
      weight is their concatenation in instruction order, per element
      (``linear.py:351-356, 444-456``).  The element bias of that form is
      ``(num_elements * bias_numel,)`` viewed per element (``linear.py:426-427,
      457-461``).
    * Keys that only e3nn's internal modules register (output masks,
      compiled-graph constants) are dropped.
    Everything else is passed through for ``load_state_dict`` to judge."""
    sd = dict(state_dict)
    for k, ref in own.items():
        if k in sd:
            v = sd[k]
            if k.endswith(".bias") and ref.dim() == 2 and v.dim() == 1 and v.numel() == ref.numel():
                sd[k] = v.reshape(ref.shape)
            continue
        if not k.endswith(".weight") or f"{k}.0" not in sd:
            continue
        parts, i = [], 0
        while f"{k}.{i}" in sd:
            parts.append(sd.pop(f"{k}.{i}"))
            i += 1
        if ref.dim() == 1:
            flat = torch.cat([p.reshape(-1) for p in parts])
        else:
            flat = torch.cat([p.reshape(ref.shape[0], -1) for p in parts], dim=-1)
        if flat.shape != ref.shape:
            raise RuntimeError(f"matrix-form weights of {k} concatenate to {tuple(flat.shape)}, "
                               f"expected {tuple(ref.shape)}")
        sd[k] = flat
    return {k: v for k, v in sd.items() if k in own or not any(t in k for t in _E3NN_INTERNAL)}


def load_reference_state_dict(model: torch.nn.Module, state_dict: Dict[str, torch.Tensor]):
    """``load_state_dict(strict=True)`` semantics for every parameter and buffer
    this model owns, from a reference checkpoint in either weight form; keys
    that only e3nn's internal modules register are ignored."""
    own = model.state_dict()
    sd = _reference_state_dict(own, state_dict)
    unknown = [k for k in sd if k not in own]
    if unknown:
        raise RuntimeError(f"unexpected keys in state_dict: {unknown[:8]}")
    missing = [k for k in own if k not in sd]
    if missing:
        raise RuntimeError(f"missing keys in state_dict: {missing[:8]}")
    torch.nn.Module.load_state_dict(model, sd, strict=True)
    return model


def create_model(cfg: Dict) -> TensorModel:
    """``create_model`` (``tace/lightning/torch_model.py:54-114``) for the MI355X path."""
    return TensorModel(TACE(**cfg))
