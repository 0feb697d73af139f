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
    assert lib.tace_abi_version() == 4


def test_variant_registry_and_errors():
    lib = _native.lib()
    n = lib.tace_tp_num_variants()
    keys = {lib.tace_tp_variant_key(i).decode() for i in range(n)}
    assert {v.key for v in codegen.all_variants()} == keys
    assert lib.tace_tp_find(b"uvu|9|9|9") == -1
    assert b"no compiled" in lib.tace_last_error()
    # argument checks fire before any device work
    assert lib.tace_edge_tp_fwd(0, 0, None, None, None, None, None, None, 1, 1, 0, 0, None, None) < 0
    assert lib.tace_uuu_fwd(10 ** 6, 0, None, None, 1, 1, 0, None, None) < 0
    cell = np.zeros(9)
    pbc = np.ones(3, dtype=np.int32)
    assert lib.tace_nl_workspace_bytes(10, cell.ctypes.data, pbc.ctypes.data, 5.0) < 0
    assert b"singular" in lib.tace_last_error()


@pytest.mark.parametrize("preset,zs,C", [("si64", [14], 64), ("fcc1024", [26, 27, 28, 29], 16),
                                         ("water12k", [1, 8], 16)])
def test_product_and_oracle_share_state_dict_layout(preset, zs, C):
    cfg = configs.model_cfg(preset, zs, 30.0, num_channel=C)
    torch.manual_seed(0)
    o = om.TACE(cfg)
    p = pm.TACE(**cfg)
    so, sp = o.state_dict(), p.state_dict()
    assert list(so) == list(sp) or set(so) == set(sp)
    for k in so:
        assert so[k].shape == sp[k].shape, k
    pm.load_reference_state_dict(p, so)
    # every tensor-product variant the model needs is compiled in
    keys = {v.key for v in codegen.all_variants()}
    for mod in p.modules():
        if isinstance(mod, (pm.O3ScatterTensorProduct, pm.uuuTensorProduct)):
            assert mod.key in keys, mod.key


def test_unsupported_configuration_raises():
    cfg = configs.model_cfg("si64", [14], 30.0, num_channel=8)
    cfg["atomic_basis"]["type"] = "uv_so2"
    with pytest.raises(NotImplementedError):
        pm.TACE(**cfg)


def test_product_refuses_cpu_tensors():
    cfg = configs.model_cfg("si64", [14], 30.0, num_channel=8)
    m = pm.create_model(cfg)
    d = dict(positions=torch.zeros(2, 3), node_attrs=torch.ones(2, 1), edge_index=torch.zeros(2, 0, dtype=torch.long),
             edge_shifts=torch.zeros(0, 3), lattice=torch.eye(3)[None], batch=torch.zeros(2, dtype=torch.long),
             ptr=torch.tensor([0, 2]))
    with pytest.raises(RuntimeError, match="GPU"):
        m(d)


def test_slot_adapters_validate_the_reference_contract():
    from tace_amd import slot

    sh = "1x0e+1x1o+1x2e+1x3o"
    node = "128x0e+128x1o+128x2e+128x3o"
    tp = slot.e3nnHipScatterTensorProduct(node, sh, node)
    assert tp.weight_numel == 128 * 23
    from tace_amd.so3 import Irreps, generate_paths
    paths, actual = generate_paths(Irreps(node), Irreps(node), Irreps(sh), "uvu")
    ins = [(i, j, k, "uvu", True) for i, j, k in paths]
    slot.e3nnHipScatterTensorProduct(node, sh, actual, ins)
    with pytest.raises(ValueError):
        slot.e3nnHipScatterTensorProduct(node, sh, actual, ins[::-1])
    u = slot.e3nnHipUuuTensorProduct(node, node, "1x0e+1x1o+1x2e+1x3o", identical_inputs=True)
    assert u.C == 128
