"""Host-side checks of the TorchSim calculator (CPU): argument validation and
the element table, as in ``tace/interface/torchsim/torchsim.py:157-193``."""

import pytest
import torch

from tace_amd import configs, model as pm
from tace_amd.torchsim import TACETorchSimCalc


def _model():
    return pm.create_model(configs.model_cfg("si64", [1, 8, 14], 20.0, num_channel=8))


def test_system_idx_length_must_match_atomic_numbers():
    with pytest.raises(ValueError, match="must match"):
        TACETorchSimCalc(_model(), device="cpu", atomic_numbers=torch.tensor([1, 8, 14]),
                         system_idx=torch.tensor([0, 0]))


def test_node_attrs_follow_the_model_element_table():
    calc = TACETorchSimCalc(_model(), device="cpu", atomic_numbers=torch.tensor([14, 1, 8, 8]),
                            system_idx=torch.tensor([0, 0, 1, 1]))
    assert torch.equal(calc.node_attrs.argmax(-1), torch.tensor([2, 0, 1, 1]))
    assert calc.n_systems == 2 and calc.n_atoms_per_system == [2, 2]
    assert calc.compute_forces and calc.compute_stress
    assert set(calc.model.get_target_property()) >= {"energy", "forces", "stress"}
    with pytest.raises(ValueError, match="element table"):
        calc._setup_node_attrs(torch.tensor([26]))


def test_model_instance_required():
    with pytest.raises(TypeError):
        TACETorchSimCalc("model.pt", device="cpu")
