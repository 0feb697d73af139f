"""Training with a force loss through the whole model (GPU).

In training mode (or with ``create_graph``) ``TensorModel`` keeps the graph of
its derivatives (``tace/models/adapter.py:95-104``), so a loss on energies,
forces and stress can be differentiated with respect to the parameters: the
double backward of force-matching training (``lightning/lit_model.py:150``).
The tensor products and the TECE convolution's rotate-in and rotate-out run
on the HIP kernels through operators whose backward is differentiable again;
the
gradients of such a loss with respect to every parameter must equal torch
autograd through the CPU oracle (float64, 1e-10 relative), and the forces of
the training path those of the inference path.
"""

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import neighbours as onl
from tace_amd import configs, data, model as pm, ops, structures

pytestmark = pytest.mark.gpu


def _pair(structs, preset, cuda, seed, **over):
    rc = configs.PRESETS[preset]["cutoff"]
    edges = [onl.neighbour_list(s["positions"], s["cell"], s["pbc"], rc) for s in structs]
    zs = sorted({int(z) for s in structs for z in s["numbers"]})
    nat = sum(len(s["positions"]) for s in structs)
    cfg = configs.model_cfg(preset, zs, sum(e[0].shape[1] for e in edges) / nat, **over)
    torch.manual_seed(seed)
    ref = om.TACE(cfg).double()
    # non-zero biases and a spread of weights, so that no gradient vanishes by symmetry
    g = torch.Generator().manual_seed(seed + 7)
    with torch.no_grad():
        for name, p in ref.named_parameters():
            if name.endswith("bias"):
                p.copy_(0.1 * torch.randn(p.shape, generator=g, dtype=p.dtype))
    torch.set_default_dtype(torch.float64)
    try:
        gpu = pm.create_model(cfg)
    finally:
        torch.set_default_dtype(torch.float32)
    pm.load_reference_state_dict(gpu.readout_fn, ref.state_dict())
    d64 = data.collate(structs, edges, cfg["atomic_numbers"], dtype=torch.float64)
    dg = data.collate(structs, edges, cfg["atomic_numbers"], dtype=torch.float64, device=cuda)
    return ref, gpu.to(cuda), d64, dg


def _loss(out, stress, seed):
    """Energy + force (+ stress) loss against fixed random targets."""
    g = torch.Generator().manual_seed(seed)
    E, F = out["energy"], out["forces"]
    tE = torch.randn(E.shape, generator=g, dtype=E.dtype).to(E.device)
    tF = torch.randn(F.shape, generator=g, dtype=F.dtype).to(F.device)
    loss = ((E - tE) ** 2).sum() + 10.0 * ((F - tF) ** 2).sum()
    if stress:
        S = out["stress"]
        tS = torch.randn(S.shape, generator=g, dtype=S.dtype).to(S.device)
        loss = loss + 100.0 * ((S - tS) ** 2).sum()
    return loss


CASES = [
    # config 1 architecture (L = 2), one species, stress
    ("si64", lambda: [structures.si_diamond(seed=1)], True, dict(num_channel=16)),
    # config 2 architecture (L = 3): four species -> several per-species weight ranges
    ("fcc1024", lambda: [structures.fcc_alloy(reps=(2, 2, 2), seed=4)], False, dict(num_channel=16)),
    # a ragged batch of triclinic crystals with stress
    ("ragged128", lambda: [structures.random_crystal(np.random.default_rng(5 + i), 10 + 4 * i, [3, 8, 14])
                           for i in range(2)], True, dict(num_channel=16, num_layers=2)),
    # a crystal, a single atom without neighbours and two atoms beyond the cutoff, with stress
    ("si64", lambda: [structures.si_diamond(seed=2),
                      dict(positions=np.zeros((1, 3)), cell=np.eye(3) * 20.0, numbers=np.array([14]),
                           pbc=(True,) * 3),
                      dict(positions=np.array([[1.0, 1.0, 1.0], [8.5, 1.2, 0.9]]), cell=np.eye(3) * 20.0,
                           numbers=np.array([14, 14]), pbc=(True,) * 3)], True, dict(num_channel=16)),
]


@pytest.mark.parametrize("preset,make,stress,over", CASES,
                         ids=[c[0] for c in CASES[:-1]] + ["si64_isolated_atoms"])
def test_force_loss_parameter_gradients_match_oracle(cuda, preset, make, stress, over):
    structs = make()
    ref, gpu, d64, dg = _pair(structs, preset, cuda, seed=3, **over)
    targets = ["energy", "forces"] + (["stress"] if stress else [])
    gpu.reset_target_property(targets)
    gpu.train()
    print(f"[train] {preset}: {sum(len(s['positions']) for s in structs)} atoms, stress={stress}", flush=True)
    out = gpu(dg)
    assert out["forces"].requires_grad and out["energy"].requires_grad
    loss = _loss(out, stress, seed=11)
    names = [n for n, p in gpu.readout_fn.named_parameters() if p.requires_grad]
    params = [dict(gpu.readout_fn.named_parameters())[n] for n in names]
    grads = torch.autograd.grad(loss, params)

    want = om.compute(ref, d64, forces=True, stress=stress, create_graph=True)
    rp = dict(ref.named_parameters())
    wgrads = torch.autograd.grad(_loss(want, stress, seed=11), [rp[n] for n in names], allow_unused=True)

    assert abs(loss.item() - _loss(want, stress, seed=11).item()) <= 1e-10 * abs(loss.item())
    worst = 0.0
    for n, gg, gw in zip(names, grads, wgrads):
        gw = torch.zeros_like(rp[n]) if gw is None else gw
        scale = gw.abs().max().item()
        err = (gg.cpu() - gw).abs().max().item()
        assert err <= 1e-10 * max(scale, 1e-30) + 1e-14, (n, err, scale)
        worst = max(worst, err / max(scale, 1e-30))
    print(f"[train] {preset}: {len(names)} parameter tensors, worst relative gradient error {worst:.2e}", flush=True)


def test_training_and_inference_forces_agree(cuda):
    """The same model in training mode (twice-differentiable operators) and in
    eval mode (inference kernels) gives the same energies and forces."""
    ref, gpu, d64, dg = _pair([structures.fcc_alloy(reps=(2, 2, 2), seed=6)], "fcc1024", cuda, seed=5,
                              num_channel=32)
    gpu.reset_target_property(["energy", "forces"])
    gpu.train()
    a = gpu(dg)
    gpu.eval()
    b = gpu(dg)
    assert (a["energy"].detach() - b["energy"]).abs().max().item() <= 1e-11 * b["energy"].abs().max().item()
    assert (a["forces"].detach() - b["forces"]).abs().max().item() <= 1e-11 * max(b["forces"].abs().max().item(), 1.0)


def _perturb_tece(module, seed):
    """Random radial phase / bias and temperatures (zero / fixed at init), so
    that the rotary and temperature terms carry gradients."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in module.named_parameters():
            if "radial_proj" in name:
                p.copy_(0.7 * torch.randn(p.shape, generator=g, dtype=p.dtype))
            elif "temperature_logit" in name:
                p.copy_(torch.randn(p.shape, generator=g, dtype=p.dtype))


def test_tece_force_loss_parameter_gradients_match_oracle(cuda):
    """Config-5 architecture (TECE edge cluster expansion with radial rotary
    attention, bilinear-gate product basis) on a distorted bcc Fe slice: the
    gradients of an energy + force loss with respect to every parameter,
    including the radial projection and the attention temperatures."""
    s = structures.bcc_fe(reps=(2, 2, 2), seed=4)
    rc = configs.PRESETS["tece"]["cutoff"]
    edges = [onl.neighbour_list(s["positions"], s["cell"], s["pbc"], rc)]
    cfg = configs.model_cfg("tece", [26], edges[0][0].shape[1] / len(s["positions"]), num_channel=16, num_head=2,
                            edge_ace_hidden=8)
    torch.manual_seed(6)
    ref = om.TACE(cfg).double()
    _perturb_tece(ref, 9)
    torch.set_default_dtype(torch.float64)
    try:
        gpu = pm.create_model(cfg)
    finally:
        torch.set_default_dtype(torch.float32)
    pm.load_reference_state_dict(gpu.readout_fn, ref.state_dict())
    gpu = gpu.to(cuda)
    gpu.reset_target_property(["energy", "forces"])
    d64 = data.collate([s], edges, cfg["atomic_numbers"], dtype=torch.float64)
    dg = data.collate([s], edges, cfg["atomic_numbers"], dtype=torch.float64, device=cuda)
    # the training path's energies and forces equal the inference kernels'
    gpu.eval()
    inf = gpu(dg)
    gpu.train()
    ops.TIMER = ops.KernelTimer()
    try:
        out = gpu(dg)
        fwd_launched = set(ops.TIMER.summary())
    finally:
        ops.TIMER = None
    # the convolution's rotate-in / rotate-out kernels in training, forward and force backward
    for k in ("edge_rotate_in_fwd", "edge_rotate_in_bwd", "tece_rotate_out_fwd", "tece_rotate_out_bwd"):
        assert k in fwd_launched, k
    assert (out["energy"].detach() - inf["energy"]).abs().max().item() <= 1e-11 * inf["energy"].abs().max().item()
    assert (out["forces"].detach() - inf["forces"]).abs().max().item() <= 1e-11 * max(inf["forces"].abs().max().item(),
                                                                                    1.0)
    loss = _loss(out, False, seed=13)
    names = [n for n, p in gpu.readout_fn.named_parameters() if p.requires_grad]
    own = dict(gpu.readout_fn.named_parameters())
    grads = torch.autograd.grad(loss, [own[n] for n in names])
    want = om.compute(ref, d64, forces=True, create_graph=True)
    rp = dict(ref.named_parameters())
    wgrads = torch.autograd.grad(_loss(want, False, seed=13), [rp[n] for n in names], allow_unused=True)
    checked = 0
    for n, gg, gw in zip(names, grads, wgrads):
        gw = torch.zeros_like(rp[n]) if gw is None else gw
        scale = gw.abs().max().item()
        err = (gg.cpu() - gw).abs().max().item()
        assert err <= 1e-10 * max(scale, 1e-30) + 1e-14, (n, err, scale)
        checked += ("temperature_logit" in n or "radial_proj" in n) and scale > 0
    assert checked >= 2   # the rotary and temperature parameters have gradients
