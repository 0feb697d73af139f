"""The allocation-free edge-TP backward (tace_edge_tp_bwd_noalloc) against the
workspace entry point (tace_edge_tp_bwd), through the C ABI.

Both run the same kernels, so every output must be bit-identical.  Two calls
in a row, the second on a smaller graph, check that the shared device scratch
carries nothing from one call into the next; an oversized request must be
refused before any device work.
"""

import ctypes

import pytest
import torch

from tace_amd import _native as N
from tace_amd import ops

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20  # TACE_NOALLOC_SCRATCH_BYTES


def _graph(n_nodes, n_edges, seed, device):
    g = torch.Generator().manual_seed(seed)
    src = torch.randint(0, n_nodes, (n_edges,), generator=g)
    dst = torch.randint(0, n_nodes - 2, (n_edges,), generator=g)  # the last receivers get no edges
    return ops.EdgePlan.from_edge_index(torch.stack([src, dst]).to(device), n_nodes), g


def _inputs(plan, var, C, dtype, g, device):
    x = torch.randn(plan.n_nodes, C * var.d1, generator=g, dtype=torch.float64).to(dtype).to(device)
    y = torch.randn(plan.n_edges, var.d2, generator=g, dtype=torch.float64).to(dtype).to(device)
    w = torch.randn(plan.n_edges, C * var.npath, generator=g, dtype=torch.float64).to(dtype).to(device)
    gout = torch.randn(plan.n_nodes, C * var.dout, generator=g, dtype=torch.float64).to(dtype).to(device)
    return x, y, w, gout


def _bwd(noalloc, x, y, w, gout, plan, var, C, layout, need_x):
    L = N.lib()
    gx = torch.full_like(x, float("nan")) if need_x else None
    gy = torch.full_like(y, float("nan"))
    gw = torch.full_like(w, float("nan"))
    s_rowptr, s_slot = plan.sender_csr()
    common = (var.vid, N.dtype_code(x.dtype), x.data_ptr(), y.data_ptr(), w.data_ptr(), gout.data_ptr(),
              plan.rowptr.data_ptr(), N.ptr(plan.eid), plan.src.data_ptr(), None, plan.n_nodes, plan.n_edges, C,
              layout, s_rowptr.data_ptr(), s_slot.data_ptr())
    tail = (N.ptr(gx), gy.data_ptr(), gw.data_ptr(), N.stream_ptr(x.device))
    if noalloc:
        N.check(L.tace_edge_tp_bwd_noalloc(*common, *tail), "tace_edge_tp_bwd_noalloc")
    else:
        n_ws = L.tace_edge_tp_workspace_elems(var.vid, plan.n_edges, C, int(need_x))
        N.check(0 if n_ws >= 0 else int(n_ws), "tace_edge_tp_workspace_elems")
        ws = torch.full((max(n_ws, 1),), float("nan"), dtype=x.dtype, device=x.device)
        N.check(L.tace_edge_tp_bwd(*common, ws.data_ptr(), ws.numel(), *tail), "tace_edge_tp_bwd")
    torch.cuda.synchronize()
    return gx, gy, gw


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("in1,lmax,C,layout", [([0, 1, 2, 3], 3, 64, 3), ([0], 3, 128, 0), ([0, 1, 2], 2, 96, 1)])
def test_noalloc_matches_workspace_entry_point(cuda, dtype, in1, lmax, C, layout):
    var = ops.find_variant(ops.variant_key("uvu", in1, list(range(lmax + 1)), list(range(lmax + 1))))
    # the first call is larger than the second: a stale scratch row or grad_y
    # partial from the first call would show up in the second
    for step, (n_nodes, n_edges) in enumerate([(61, 900), (23, 170)]):
        plan, g = _graph(n_nodes, n_edges, 11 * step + C + len(in1), cuda)
        x, y, w, gout = _inputs(plan, var, C, dtype, g, cuda)
        es = 4 if dtype == torch.float32 else 8
        assert N.lib().tace_edge_tp_workspace_elems(var.vid, n_edges, C, 1) * es <= SCRATCH_BYTES
        print(f"[no_alloc] {var.key} C={C} {dtype} layout={layout} call {step}: N={n_nodes} E={n_edges}",
              flush=True)
        for need_x in (True, False):
            want = _bwd(False, x, y, w, gout, plan, var, C, layout, need_x)
            got = _bwd(True, x, y, w, gout, plan, var, C, layout, need_x)
            for name, a, b in zip(("grad_x", "grad_y", "grad_w"), got, want):
                if b is None:
                    assert a is None
                    continue
                assert torch.isfinite(b).all(), name
                assert torch.equal(a, b), f"{name} differs (call {step}, need_x={need_x})"


def test_noalloc_refuses_oversized_workspace(cuda):
    var = ops.find_variant(ops.variant_key("uvu", [0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3]))
    C, E = 128, 1 << 20  # 1 M edges x 128 channels x 16 floats: far above the scratch
    L = N.lib()
    assert L.tace_edge_tp_workspace_elems(var.vid, E, C, 1) * 4 > SCRATCH_BYTES
    # rejected on the host before any pointer is touched, so null pointers are safe
    rc = L.tace_edge_tp_bwd_noalloc(var.vid, N.F32, None, None, None, None, None, None, None, None, 1000, E, C, 0,
                                    None, None, ctypes.c_void_p(1), None, None, None)
    assert rc < 0
    assert b"scratch" in L.tace_last_error()
