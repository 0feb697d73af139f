"""Graph batches in the reference's data-dict format.

``collate`` builds ``{positions, node_attrs, edge_index, edge_shifts, lattice,
batch, ptr}`` as ``from_atoms`` + torch_geometric collation produce them
(``tace/dataset/graph.py:36-161``; keys as used at
``tace/interface/torchsim/torchsim.py:261-274``), from structures and their
per-structure edge lists.  ``gpu_graph`` does the same on the GPU with the
HIP neighbour list, keeping edges grouped by receiver.
"""

from __future__ import annotations

from typing import Dict, List, Sequence, Tuple

import numpy as np
import torch


def one_hot(numbers: np.ndarray, atomic_numbers: Sequence[int], dtype) -> torch.Tensor:
    """``TorchElement.z2onehot`` (``tace/dataset/element.py:40-64``)."""
    zs = sorted(int(z) for z in atomic_numbers)
    lut = np.full(max(zs) + 1, -1, dtype=np.int64)
    lut[zs] = np.arange(len(zs))
    idx = lut[np.asarray(numbers)]
    if (idx < 0).any():
        raise ValueError("structure contains an element outside the model's atomic_numbers")
    out = torch.zeros(len(idx), len(zs), dtype=dtype)
    out[torch.arange(len(idx)), torch.from_numpy(idx)] = 1
    return out


def collate(structs: List[Dict], edges: List[Tuple[np.ndarray, np.ndarray]], atomic_numbers: Sequence[int],
            dtype=torch.float64, device="cpu") -> Dict[str, torch.Tensor]:
    """``edges[k] = (edge_index [2,E_k], shifts [E_k,3])`` per structure, local indexing."""
    pos, attrs, ei, sh, lat, batch, ptr = [], [], [], [], [], [], [0]
    off = 0
    for k, (s, (e, S)) in enumerate(zip(structs, edges)):
        n = len(s["positions"])
        pos.append(torch.as_tensor(np.asarray(s["positions"]), dtype=dtype))
        attrs.append(one_hot(s["numbers"], atomic_numbers, dtype))
        ei.append(torch.as_tensor(np.asarray(e), dtype=torch.int64) + off)
        sh.append(torch.as_tensor(np.asarray(S), dtype=dtype))
        lat.append(torch.as_tensor(np.asarray(s["cell"]), dtype=dtype).view(1, 3, 3))
        batch.append(torch.full((n,), k, dtype=torch.int64))
        off += n
        ptr.append(off)
    d = dict(positions=torch.cat(pos), node_attrs=torch.cat(attrs), edge_index=torch.cat(ei, 1),
             edge_shifts=torch.cat(sh), lattice=torch.cat(lat), batch=torch.cat(batch),
             ptr=torch.tensor(ptr, dtype=torch.int64))
    return {k: v.to(device) for k, v in d.items()}


def device_graph(p64: torch.Tensor, sizes: Sequence[int], cells, pbcs, cutoff: float) -> Dict[str, torch.Tensor]:
    """Edges of a batch whose float64 positions ``p64`` [sum(sizes), 3] are
    already on the GPU: one batched HIP cell-list search
    (``ops.neighbour_list_batch``), edges grouped by receiver
    (``edge_index[1]`` non-decreasing), node ids batch-global.  Returns
    edge_index (int64), integer edge_shifts (int32) and the receiver CSR plan
    the model's kernels take (``_edge_plan``, ``_dst32``)."""
    from .ops import EdgePlan, neighbour_list_batch

    n_tot = int(p64.shape[0])
    rowptr, src, shifts = neighbour_list_batch(p64, sizes, cells, pbcs, cutoff)
    E = src.shape[0]
    counts = (rowptr[1:] - rowptr[:-1]).to(torch.int64)
    dst = torch.repeat_interleave(torch.arange(n_tot, device=p64.device), counts, output_size=E)
    return dict(edge_index=torch.stack([src.to(torch.int64), dst]), edge_shifts=shifts,
                _edge_plan=EdgePlan(n_tot, E, rowptr, src, None), _dst32=dst.to(torch.int32), _shifts32=shifts)


def gpu_graph(structs: List[Dict], atomic_numbers: Sequence[int], cutoff: float, dtype=torch.float32,
              device="cuda") -> Dict[str, torch.Tensor]:
    """Batch built on the GPU (``device_graph``) from host structures; the
    result carries its receiver CSR plan."""
    sizes = [len(s["positions"]) for s in structs]
    dev = torch.device(device)
    up = lambda t: t.to(dev)
    p64 = up(torch.from_numpy(np.concatenate([np.asarray(s["positions"], dtype=np.float64).reshape(-1, 3)
                                              for s in structs])))
    g = device_graph(p64, sizes, [s["cell"] for s in structs], [s["pbc"] for s in structs], cutoff)
    sizes_t = torch.tensor(sizes, dtype=torch.int64)
    batch = up(torch.repeat_interleave(torch.arange(len(structs)), sizes_t))
    ptr = torch.zeros(len(structs) + 1, dtype=torch.int64)
    ptr[1:] = torch.cumsum(sizes_t, 0)
    attrs_h = torch.cat([one_hot(s["numbers"], atomic_numbers, dtype) for s in structs])
    lat = up(torch.from_numpy(np.stack([np.asarray(s["cell"], dtype=np.float64).reshape(3, 3)
                                        for s in structs])).to(dtype))
    g["edge_shifts"] = g["edge_shifts"].to(dtype)
    # per-species node counts (columns of node_attrs), known here on the host
    g["_species_counts"] = attrs_h.sum(0).to(torch.int64).tolist()
    return dict(positions=p64.to(dtype), node_attrs=up(attrs_h), lattice=lat, batch=batch, ptr=up(ptr), **g)


_CELLS: Dict = {}


def _device_cell(cell, dtype, device) -> torch.Tensor:
    """The lattice [1, 3, 3] on the device, kept per (values, dtype, device):
    an MD run passes the same cell every step.  Callers must not write to it."""
    a = np.ascontiguousarray(np.asarray(cell, dtype=np.float64).reshape(3, 3))
    key = (a.tobytes(), str(dtype), str(device))
    t = _CELLS.get(key)
    if t is None:
        if len(_CELLS) > 64:
            _CELLS.clear()
        t = _CELLS[key] = torch.as_tensor(a, dtype=dtype, device=device).view(1, 3, 3)
    return t


def resident_graph(pos64: torch.Tensor, cell, pbc, node_attrs: torch.Tensor, cutoff: float,
                   dtype=torch.float32) -> Dict[str, torch.Tensor]:
    """One periodic structure already resident on the GPU (float64 positions)
    -> model input dict, neighbour list rebuilt by the HIP cell list."""
    from .ops import EdgePlan, neighbour_list

    n = pos64.shape[0]
    dev = pos64.device
    rowptr, src, sh = neighbour_list(pos64, cell, pbc, cutoff)
    counts = (rowptr[1:] - rowptr[:-1]).to(torch.int64)
    dst = torch.repeat_interleave(torch.arange(n, device=dev), counts, output_size=int(src.shape[0]))
    # ptr [0, n] by a fill kernel, the lattice from a cache (host-to-device
    # copies of pageable memory wait for the GPU to go idle)
    ptr = torch.zeros(2, dtype=torch.int64, device=dev)
    ptr[1:] = n
    d = dict(positions=pos64.to(dtype), node_attrs=node_attrs,
             edge_index=torch.stack([src.to(torch.int64), dst]), edge_shifts=sh.to(dtype),
             lattice=_device_cell(cell, dtype, dev), batch=torch.zeros(n, dtype=torch.int64, device=dev), ptr=ptr)
    d["_edge_plan"] = EdgePlan(n, int(src.shape[0]), rowptr, src, None)
    d["_shifts32"] = sh
    return d


def mean_in_degree(edge_index: np.ndarray, n: int) -> float:
    return float(np.asarray(edge_index).shape[1]) / max(n, 1)
