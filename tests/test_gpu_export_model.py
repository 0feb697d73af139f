"""Whole-model export (GPU): ``TensorModel`` energy + forces (+ stress) traced
with ``make_fx`` and exported with ``torch.export`` (dynamic atom and edge
counts; ``tace/models/compile/aot.py:206-273``), saved and loaded as a .pt2
program, run on structures of other sizes: the eager model's results."""

import numpy as np
import pytest
import torch

from oracle import neighbours as onl
from tace_amd import configs, data, export, model as pm, structures

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
    """The config-5 TECE architecture (its convolution as torch operations in
    the program, the tensor products and per-species linears as operators)."""
    s = structures.bcc_fe(reps=(2, 2, 2), seed=5)
    m, cfg = _model("tece", [26], 40.0, cuda, seed=2, num_channel=16, num_head=2, edge_ace_hidden=8)
    m.reset_target_property(["energy", "forces"])
    path = export.save_program(m, _graph([s], cfg, cuda), str(tmp_path / "tece.pt2"))
    loaded = export.load_program(path)
    for st in (s, structures.bcc_fe(reps=(3, 2, 2), seed=6)):
        g = _graph([st], cfg, cuda)
        _compare(loaded(g), m(g), loaded.output_keys)
