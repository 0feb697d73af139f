"""Model configurations of the benchmark workloads, in the reference's cfg format.

``model_cfg`` returns the keyword dict that ``e3nnTACE(**cfg)``
(``tace/models/_e3nn/tace.py:28-62``) accepts, already merged with
``DEFAULT_MODEL_CONFIG`` for the keys this path reads
(``tace/models/_e3nn/default.py:10-177``), with "L" mapped to Lmax = lmax = L.
"""

from __future__ import annotations

import copy
from typing import Dict, List, Sequence

PRESETS = {
    # id: (channels, L, layers, cutoff, targets)
    "si64": dict(num_channel=64, L=2, num_layers=2, cutoff=5.0, target=["energy", "forces", "stress"]),
    "fcc1024": dict(num_channel=128, L=3, num_layers=2, cutoff=5.0, target=["energy", "forces"]),
    "water12k": dict(num_channel=128, L=3, num_layers=3, cutoff=6.0, target=["energy", "forces"]),
    "ragged128": dict(num_channel=256, L=3, num_layers=2, cutoff=6.0, target=["energy", "forces", "stress"]),
    # config 5: TECE edge cluster expansion with radial rotary attention; layer 0
    # cgtp (uv_so2 needs l > 0 inputs, inter.py:458-461), bilinear-gate product
    # basis (correlation 2, prod.py:83-84), agnostic coefficients
    "tece": dict(num_channel=128, L=2, mmax=2, num_layers=2, cutoff=5.0, target=["energy", "forces"],
                 atomic_basis_type=["cgtp", "uv_so2"], num_head=4, edge_ace_hidden=32, correlation=2,
                 product_nonlinear="silu_bilineargate", agnostic=True),
}


def statistics(atomic_numbers: Sequence[int], avg_num_neighbors: float) -> List[Dict]:
    """Fixed statistics stub in the reference format
    (``tace/dataset/statistics.py:342-447``): E0(z) = -0.1 z, rms_forces(z) = 1 + 0.01 z."""
    zs = sorted(int(z) for z in atomic_numbers)
    return [dict(atomic_numbers=zs, avg_num_neighbors=float(avg_num_neighbors),
                 atomic_energy={z: -0.1 * z for z in zs},
                 rms_forces={z: 1.0 + 0.01 * z for z in zs})]


def model_cfg(preset: str, atomic_numbers: Sequence[int], avg_num_neighbors: float, **over) -> Dict:
    p = dict(PRESETS[preset])
    p.update(over)
    L = p["L"]
    stats = statistics(atomic_numbers, avg_num_neighbors)
    cfg = dict(
        Lmax=L, lmax=L, mmax=p.get("mmax", 2), mag_Lmax=1, parity=False,
        num_channel=p["num_channel"], num_layers=p["num_layers"], cutoff=p["cutoff"],
        statistics=stats, target_property=list(p["target"]), embedding_property=[],
        max_neighbors=None,
        fidelity=[dict(name="PBE", atomic_energy=None)],
        node_embedding=dict(type="linear"),
        edge_embedding=dict(type="identity"),
        edge_update=dict(type="identity"),
        radial_basis=dict(bias=False, r_min=0.0, radial_basis="j0", num_radial_basis=8,
                          num_mag_radial_basis=10, distance_transform=None, cutoff_fn="c2poly",
                          polynomial_cutoff=5, order=0, trainable=False, apply_cutoff=True,
                          hidden=[64, 64, 64], gaussian_width=2.0, use_dydynamic_cutoff=False,
                          dydynamic_cutoff_mu=40),
        atomic_basis=dict(type=p.get("atomic_basis_type", "cgtp"), l1l2=None, scatter_norm="avg_num_neighbors",
                          nonlinear="sigmoid_gate", edge_nonlinear="so2_sigmoid_gate", gate_m0=True,
                          num_head=p.get("num_head"), edge_ace_hidden=p.get("edge_ace_hidden"),
                          scalar_act=None, tensor_act=None),
        resnet=dict(type="BB", linear_type="aware", use_first_resnet=False),
        product_basis=dict(type="cgtp", l1l2=None, correlation=p.get("correlation", 3),
                           num_expert=None, num_channel_per_expert=None, use_shared_expert=False,
                           nonlinear=p.get("product_nonlinear"), agnostic=p.get("agnostic", False),
                           return_components=None),
        readout_emlp=dict(bias=False, hidden=[16], use_alllayer=False, use_uie=False,
                          use_one_body_magmoms=True),
        scale_shift=dict(enable=True, scale_type="rms_forces", shift_type=None,
                         scale_trainable=False, shift_trainable=False, all_atoms=False, scale_zbl=True),
        short_range=dict(zbl=dict(enable=False, trainable=False)),
        long_range=dict(les=dict(enable=False)),
        universal_embedding={},
    )
    cfg["atomic_numbers"] = stats[0]["atomic_numbers"]
    cfg["avg_num_neighbors"] = stats[0]["avg_num_neighbors"]
    return copy.deepcopy(cfg)
