"""CPU-side checks of the native boundary and the model structure (no GPU)."""

import os
import re

import numpy as np
import pytest
import torch

from tace_amd import _native, configs, model as pm
from tace_amd.csrc import codegen
from oracle import model as om

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    txt = open(os.path.join(ROOT, "include", "tace_hip.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(tace_\w+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    declared = _header_functions()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_native.EXPORTED)
    hdr = open(os.path.join(ROOT, "include", "tace_hip.h")).read()
    assert lib.tace_abi_version() == int(re.search(r"TACE_HIP_ABI_VERSION (\d+)", hdr).group(1))


def test_channel_limit_and_layout_checks():
    """Channel counts beyond TACE_MAX_CHANNELS and unknown layout flags are
    refused before any device work."""
    lib = _native.lib()
    vid = lib.tace_tp_find(b"uvu|0,1,2,3|0,1,2,3|0,1,2,3")
    rc = lib.tace_edge_tp_fwd(vid, 0, None, None, None, None, None, None, None, 4, 0, 513, 0, None, None)
    assert rc < 0 and b"channels" in lib.tace_last_error()
    rc = lib.tace_edge_tp_fwd(vid, 0, None, None, None, None, None, None, None, 4, 0, 64, 4, None, None)
    assert rc < 0 and b"layout" in lib.tace_last_error()


@pytest.mark.parametrize("C,H,ok", [(48, 1, False), (96, 16, False), (128, 4, True), (192, 1, True), (160, 1, False)])
def test_rotate_out_head_width_check(C, H, ok):
    """The head sums of the rotate-out and score kernels add a head's lanes
    with power-of-two shuffles: a per-head width must divide 64 or be a
    multiple of 64, and other widths are refused before any device work (an
    accepted call gets as far as its null-pointer check)."""
    lib = _native.lib()
    rc = lib.tace_tece_rotate_out_bwd(0, None, None, None, None, None, None, 10, 5, 2, C, H, None, None, None, None)
    assert rc < 0
    assert (b"null pointer" in lib.tace_last_error()) == ok, lib.tace_last_error()


@pytest.mark.parametrize("in1,lmax", [([0], 2), ([0, 1, 2, 3], 3), ([0, 1, 2], 2)])
def test_generated_contraction_order_matches_oracle(in1, lmax):
    """CPU restatement of the contractions the generated edge kernels perform
    (forward t = CG(x, y) per (in1, in2) block pair; backward
    psi_i = sum_jk c y_j g_k, gw = x . psi, grad_x += w psi,
    grad_y_j += sum_ik c x_i w g_k) agrees with the oracle."""
    from oracle import so3 as oso3

    v = codegen.Variant("uvu", in1, list(range(lmax + 1)), list(range(lmax + 1)))
    g = torch.Generator().manual_seed(3)
    Nn, E, C = 5, 14, 3
    src = torch.randint(0, Nn, (E,), generator=g)
    dst = torch.randint(0, Nn, (E,), generator=g)
    irr = [(C, (l, (-1) ** l)) for l in in1]
    tp = om.ScatterTP(irr, oso3.sh_irreps(lmax), [(1, (l, (-1) ** l)) for l in range(lmax + 1)]).double()
    x = torch.randn(Nn, C * v.D1, generator=g, dtype=torch.float64, requires_grad=True)
    y = torch.randn(E, v.D2, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(E, C * len(v.paths), generator=g, dtype=torch.float64, requires_grad=True)
    out_o = tp(x, y, w, torch.stack([src, dst]))
    go = torch.randn(out_o.shape, generator=g, dtype=torch.float64)
    gx_o, gy_o, gw_o = torch.autograd.grad((out_o * go).sum(), [x, y, w])

    X = x.detach().numpy()
    Y, W, G = y.detach().numpy(), w.detach().numpy().reshape(E, -1, C), go.numpy()

    def xi(node, b, i):  # e3nn layout: block b is [C, 2l+1]
        return X[node, C * v.off1[b] + np.arange(C) * v.d1[b] + i]

    def oi(p, k):
        return C * v.offo[p] + np.arange(C) * v.dout[p] + k

    out = np.zeros((Nn, C * v.DO))
    gx, gw, gy = np.zeros_like(X), np.zeros_like(W), np.zeros_like(Y)
    for e in range(E):
        s, n = int(src[e]), int(dst[e])
        for p, (b1, b2) in enumerate(v.path_blocks):
            o2 = v.off2[b2]
            psi = {}
            for (i, j, k, c) in v.cg[p]:
                out[n, oi(p, k)] += W[e, p] * c * xi(s, b1, i) * Y[e, o2 + j]
                psi[i] = psi.get(i, 0) + c * Y[e, o2 + j] * G[n, oi(p, k)]
                gy[e, o2 + j] += (c * xi(s, b1, i) * W[e, p] * G[n, oi(p, k)]).sum()
            for i, ps in psi.items():
                gw[e, p] += xi(s, b1, i) * ps
                gx[s, C * v.off1[b1] + np.arange(C) * v.d1[b1] + i] += W[e, p] * ps
    np.testing.assert_allclose(out, out_o.detach().numpy(), rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(gx, gx_o.numpy(), rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(gw.reshape(E, -1), gw_o.numpy(), rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(gy, gy_o.numpy(), rtol=1e-11, atol=1e-11)


def test_kernel_parts_partition_the_paths():
    """The part splits of the generated kernels: every path in exactly one
    part; a part of the radial-fused uvu kernels and of the uuu backward
    holds whole in1 blocks (so each grad-x row block comes from one part);
    the uuu backward's parts respect their component cap and only products
    with many outputs are split; the registry records the part counts the
    launchers size their grids and workspaces with."""
    reg = open(os.path.join(ROOT, "tace_amd", "csrc", "gen", "registry.inc")).read()
    for v in codegen.all_variants():
        if v.kind == "uvu":
            parts = [v._part_paths([b]) for b in v.rtp_parts()]
            assert sorted(p for ps in parts for p in ps) == list(range(len(v.paths))), v.name
            assert f"{len(v.rtp_parts())}, L_{v.name}_rfwd, L_{v.name}_rbwd" in reg, v.name
        else:
            parts = v.uuu_parts()
            blocks = [b for bs in parts for b in bs]
            assert len(blocks) == len(set(blocks)), v.name
            covered = sorted(p for p in range(len(v.paths)) if v.path_blocks[p][0] in blocks)
            assert covered == list(range(len(v.paths))), v.name
            if v.DO <= 128:
                assert len(parts) == 1, v.name
            else:
                for bs in parts:
                    assert len(bs) == 1 or sum(v.d1[b] for b in bs) <= 40, (v.name, bs)
            assert reg.count(f"L_{v.name}_bwd_d, 0, nullptr, nullptr, {len(parts)}}}") == 1, v.name


def test_bf16_fragment_order_layout():
    """``ops.bf16_fragment_order``: element (k, n) of B lands at the lane and
    slot of the MFMA B operand the header states (per 16-column block cb and
    32-k step s: offset (cb nks + s) 512 + (16 g + f) 8 + e for k = 32 s + 8 g
    + e, n = 16 cb + f), zeros past k and n."""
    import torch
    from tace_amd import ops
    k, n = 70, 37
    B = (torch.arange(k * n, dtype=torch.float32).view(k, n) % 251 + 1).to(torch.bfloat16)
    f = ops.bf16_fragment_order(B)
    nks, nb = 3, 3
    assert f.numel() == nks * nb * 512
    for kk in range(32 * nks):
        for nn in range(16 * nb):
            s, g, e = kk // 32, (kk % 32) // 8, kk % 8
            cb, fl = nn // 16, nn % 16
            v = f[(cb * nks + s) * 512 + (16 * g + fl) * 8 + e]
            want = B[kk, nn] if kk < k and nn < n else torch.tensor(0, dtype=torch.bfloat16)
            assert v == want, (kk, nn)
