"""The model API the reference's callers use, replayed on the CPU.

Every call ``TACEAseCalc.__init__`` (``tace/interface/ase/calculator.py:64-127``)
and ``TACETorchSimCalc.__init__`` (``tace/interface/torchsim/torchsim.py:
103-170``) make on the model, the loading path of ``load_tace``
(``tace/lightning/lit_model.py:564-610`` -> ``create_model``,
``tace/lightning/torch_model.py:54-114``), and both checkpoint weight forms
(``tace/models/linear.py:282-481``).  The forward passes run on the GPU
(``tests/test_gpu_boundary.py``); here only what happens before any kernel.
"""

import importlib

import pytest
import torch

from tace_amd import configs, model as pm


def _cfg(**over):
    return configs.model_cfg("si64", [1, 8, 14], 20.0, num_channel=8, **over)


def _model(cfg=None):
    torch.manual_seed(0)
    return pm.create_model(cfg or _cfg())


# ----------------------------------------------------------- element table ----
def test_torch_element_matches_the_reference_table():
    el = _model().get_torch_element()
    assert el.zs == [1, 8, 14] and el.num_elements == 3 and len(el) == 3
    z = torch.tensor([14, 1, 8, 8, 1])
    assert torch.equal(el.z2idx(z), torch.tensor([2, 0, 1, 1, 0]))
    oh = el.z2onehot(z)
    assert oh.dtype == torch.int64 and oh.shape == (5, 3)
    assert torch.equal(oh.argmax(-1), torch.tensor([2, 0, 1, 1, 0])) and torch.equal(oh.sum(-1), torch.ones(5).long())
    with pytest.raises(RuntimeError):  # an element outside the table: one_hot of -1
        el.z2onehot(torch.tensor([6]))


# ------------------------------------------------------------------ flags ----
def test_flags_follow_the_target_properties():
    m = _model()
    assert set(m.get_target_property()) == {"energy", "forces", "stress"}
    assert m.flags.compute_energy and m.flags.compute_forces and m.flags.compute_stress
    assert not m.flags.compute_virials and not m.flags.compute_edge_forces and not m.flags.compute_hessian
    assert m.compute_first_derivative and not m.compute_second_derivative
    m.reset_target_property(["energy"])
    assert not m.flags.compute_forces and not m.compute_first_derivative
    m.reset_target_property(["energy", "forces", "atomic_virials"])
    assert m.flags.compute_atomic_virials and m.compute_first_derivative


def test_unsupported_or_inconsistent_flags_are_refused_before_any_work():
    m = _model()
    m.flags.compute_hessian = True  # a second-derivative target this path does not compute
    with pytest.raises(NotImplementedError, match="compute_hessian"):
        m({})
    m = _model()
    m.reset_target_property(["energy"])
    m.flags.compute_forces = True  # without compute_first_derivative the reference has no gradients
    with pytest.raises(RuntimeError, match="compute_first_derivative"):
        m({})


def test_ase_calculator_init_calls():
    """calculator.py:98-127 after load_tace: eval, freeze, getters."""
    model = _model()
    model.eval()
    for p in model.parameters():
        p.requires_grad = False
    assert model.get_model_dtype() == torch.float32
    assert set(model.get_target_property()) == {"energy", "forces", "stress"}
    assert model.get_embedding_property() == []
    assert model.get_max_neighbors() is None
    assert model.get_cutoff() == 5.0
    assert model.get_torch_element().zs == [1, 8, 14]
    assert model.get_fidelity_idx() == 0
    model.reset_fidelity_idx(0)
    model.reset_fidelity_idx(None)  # fidelity_idx=None keeps the current one
    assert model.get_fidelity_idx() == 0


@pytest.mark.parametrize("compute_forces,compute_stress", [(True, True), (True, False), (False, False)])
def test_torchsim_init_calls(compute_forces, compute_stress):
    """torchsim.py:131-153: flags set by the caller, atomic numbers copied
    onto the model, element table taken from it."""
    cfg = _cfg()
    cfg["target_property"] = ["energy", "forces"]
    model = _model(cfg)
    assert hasattr(model, "flags")
    model.flags.compute_forces = compute_forces
    model.flags.compute_stress = compute_stress
    model.compute_first_derivative = compute_forces or compute_stress
    model.reset_fidelity_idx(None)
    model.eval()
    for p in model.parameters():
        p.requires_grad = False
    assert model.get_cutoff() == 5.0
    model.atomic_numbers = torch.tensor(model.get_atomic_numbers(), dtype=torch.int64)
    attrs = model.get_torch_element().z2onehot(torch.tensor([8, 1, 1])).to(model.get_model_dtype())
    assert attrs.dtype == torch.float32 and attrs.shape == (3, 3)
    # the stress switch is honoured although stress is not a target
    assert model.flags.compute_stress == compute_stress
    assert "compute_stress" not in [f"compute_{p}" for p in model.get_target_property()]


# ------------------------------------------------------------- checkpoints ----
def _matrix_form(model):
    """The state_dict the reference saves with TACE_USE_MATRIX_WEIGHT=1: every
    e3nn linear's flat weight split into one ``weight.<i>`` per o3.Linear
    instruction, shape ``path_shape`` (per element for the element linears),
    and the element bias flattened (linear.py:322-327, 417-427)."""
    sd = dict(model.state_dict())
    n = 0
    for name, mod in model.named_modules():
        if not isinstance(mod, (pm.e3nnLinear, pm.e3nnElementLinear)):
            continue
        key = f"{name}.weight"
        w = sd.pop(key)
        for i, (_i, _o, off, mi, mo, _pw) in enumerate(mod.lay.ins):
            if w.dim() == 1:
                sd[f"{key}.{i}"] = w[off:off + mi * mo].reshape(mi, mo).clone()
            else:
                sd[f"{key}.{i}"] = w[:, off:off + mi * mo].reshape(w.shape[0], mi, mo).clone()
        if isinstance(mod, pm.e3nnElementLinear) and f"{name}.bias" in sd:
            sd[f"{name}.bias"] = sd[f"{name}.bias"].reshape(-1).clone()
        n += 1
    assert n > 5
    return sd


def test_matrix_form_checkpoint_loads_into_the_flat_weights():
    src = _model()
    with torch.no_grad():
        for p in src.parameters():
            p.copy_(torch.randn_like(p))
    mat = _matrix_form(src)
    assert any(k.endswith(".weight.0") for k in mat)
    torch.manual_seed(1)
    dst = pm.create_model(_cfg())
    dst.load_state_dict(mat, strict=True)
    for k, v in src.state_dict().items():
        assert torch.equal(dst.state_dict()[k], v), k
    dst2 = pm.create_model(_cfg())
    pm.load_reference_state_dict(dst2.readout_fn, {k[len("readout_fn."):]: v for k, v in mat.items()})
    for k, v in src.state_dict().items():
        assert torch.equal(dst2.state_dict()[k], v), k
    # a malformed matrix form is refused
    bad = dict(mat)
    k0 = next(k for k in bad if k.endswith(".weight.0"))
    bad[k0] = bad[k0][..., :-1]
    with pytest.raises(RuntimeError, match="concatenate"):
        pm.create_model(_cfg()).load_state_dict(bad)


def test_e3nn_internal_keys_are_ignored_and_unknown_keys_refused():
    src = _model()
    sd = dict(src.state_dict())
    sd["readout_fn.representation.interactions.0.linear_up.linear.output_mask"] = torch.ones(3)
    m = pm.create_model(_cfg())
    m.load_state_dict(sd, strict=True)
    sd["readout_fn.not_a_parameter"] = torch.ones(1)
    with pytest.raises(RuntimeError):
        pm.create_model(_cfg()).load_state_dict(sd, strict=True)


def test_reference_create_model_path():
    """torch_model.py:54-114 with the model and wrapper classes named in the
    package's cfg: both are imported by path, the model takes the cfg with
    the extra ``_target_`` / ``wrapper`` keys, and load_tace's
    ``model.load_state_dict(state_dict, strict=True)`` (lit_model.py:597-610)
    loads a reference state_dict."""
    cfg = _cfg()
    cfg["_target_"] = "tace_amd.model.TACE"
    cfg["wrapper"] = {"_target_": "tace_amd.model.TensorModel"}
    mod, cls = cfg["_target_"].rsplit(".", 1)
    wmod, wcls = cfg["wrapper"]["_target_"].rsplit(".", 1)
    MODEL_CLS = getattr(importlib.import_module(mod), cls)
    WRAPPER_CLS = getattr(importlib.import_module(wmod), wcls)
    model = WRAPPER_CLS(MODEL_CLS(**cfg))
    src = _model()
    model.load_state_dict(_matrix_form(src), strict=True)
    for k, v in src.state_dict().items():
        assert torch.equal(model.state_dict()[k], v), k
