"""Whole-model export (GPU): ``TensorModel`` energy + forces (+ stress) traced
with ``make_fx`` and exported with ``torch.export`` (dynamic atom and edge
counts; ``tace/models/compile/aot.py:206-273``), saved and loaded as a .pt2
program, run on structures of other sizes: the eager model's results."""

import numpy as np
import pytest
import torch

from oracle import neighbours as onl
from tace_amd import configs, data, export, model as pm, ops, structures

pytestmark = pytest.mark.gpu


def _model(preset, zs, avg, cuda, seed, **over):
    cfg = configs.model_cfg(preset, zs, avg, **over)
    torch.manual_seed(seed)
    torch.set_default_dtype(torch.float64)
    try:
        m = pm.create_model(cfg)
    finally:
        torch.set_default_dtype(torch.float32)
    return m.to(cuda).eval(), cfg


def _graph(structs, cfg, cuda):
    edges = [onl.neighbour_list(s["positions"], s["cell"], s["pbc"], cfg["cutoff"]) for s in structs]
    return data.collate(structs, edges, cfg["atomic_numbers"], dtype=torch.float64, device=cuda)


def _compare(got, want, keys):
    for k in keys:
        a, b = got[k], want[k]
        assert a.shape == b.shape, k
        assert (a - b).abs().max().item() <= 1e-10 * max(1.0, b.abs().max().item()), k


@pytest.mark.parametrize("preset,over", [("si64", dict(num_channel=16)), ("fcc1024", dict(num_channel=16))])
def test_exported_model_matches_eager(cuda, tmp_path, preset, over):
    if preset == "si64":
        sample = [structures.si_diamond(seed=1)]
        other = [structures.si_diamond(reps=(2, 2, 3), seed=2)]
        zs = [14]
    else:
        sample = [structures.fcc_alloy(reps=(2, 2, 2), seed=3)]
        other = [structures.fcc_alloy(reps=(3, 2, 2), seed=4)]
        zs = sorted({int(z) for s in sample + other for z in s["numbers"]})
    m, cfg = _model(preset, zs, 30.0, cuda, seed=1, **over)
    if preset == "si64":
        m.reset_target_property(["energy", "forces", "stress"])
    else:
        m.reset_target_property(["energy", "forces"])
    print(f"[export] {preset}: tracing", flush=True)
    path = export.save_program(m, _graph(sample, cfg, cuda), str(tmp_path / "model.pt2"))
    loaded = export.load_program(path)
    for structs in (sample, other):
        g = _graph(structs, cfg, cuda)
        _compare(loaded(g), m(g), loaded.output_keys)


def test_exported_tece_model_matches_eager(cuda, tmp_path):
    """The config-5 TECE architecture: the convolution's kernels, the tensor
    products and the per-species linears as operators in the program."""
    s = structures.bcc_fe(reps=(2, 2, 2), seed=5)
    m, cfg = _model("tece", [26], 40.0, cuda, seed=2, num_channel=16, num_head=2, edge_ace_hidden=8)
    m.reset_target_property(["energy", "forces"])
    path = export.save_program(m, _graph([s], cfg, cuda), str(tmp_path / "tece.pt2"))
    loaded = export.load_program(path)
    for st in (s, structures.bcc_fe(reps=(3, 2, 2), seed=6)):
        g = _graph([st], cfg, cuda)
        ops.TIMER = ops.KernelTimer()
        try:
            got = loaded(g)
            launched = set(ops.TIMER.summary())
        finally:
            ops.TIMER = None
        _compare(got, m(g), loaded.output_keys)
        # the program runs the convolution's kernels, forward and backward
        for k in ("edge_rotate_in_fwd", "edge_rotate_in_bwd", "tece_rotate_out_fwd", "tece_rotate_out_bwd"):
            assert k in launched, k


def test_exported_model_takes_other_graph_counts(cuda, tmp_path):
    """A program exported on a two-graph batch runs batches of three graphs
    and of one (dynamic graph count, ``_graph_dynamic_shapes``,
    tace/models/compile/aot.py:513-530), with stress."""
    rng = np.random.default_rng(3)
    zs = [3, 8, 14]
    mk = lambda k: [structures.random_crystal(rng, int(rng.integers(5, 12)), zs) for _ in range(k)]
    sample, other, single = mk(2), mk(3), mk(1)
    m, cfg = _model("si64", zs, 30.0, cuda, seed=4, num_channel=16)
    m.reset_target_property(["energy", "forces", "stress"])
    path = export.save_program(m, _graph(sample, cfg, cuda), str(tmp_path / "multi.pt2"))
    loaded = export.load_program(path)
    assert loaded.get_cutoff() == cfg["cutoff"] and loaded.get_atomic_numbers() == cfg["atomic_numbers"]
    for structs in (sample, other, single):
        g = _graph(structs, cfg, cuda)
        _compare(loaded(g), m(g), loaded.output_keys)
