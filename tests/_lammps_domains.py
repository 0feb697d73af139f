"""Two-domain LAMMPS ML-IAP run for tests/test_gpu_lammps.py (helper module,
not collected): a periodic bcc Fe cell split at x = L/2 into two domains, one
process each, with ghosts exchanged through a gloo stand-in for LAMMPS's
ML-IAP communication (``forward_exchange`` / ``reverse_exchange``,
``tace/models/lammps.py:82-102``)."""

import os

import numpy as np
import torch

from oracle import model as om
from oracle import neighbours as onl
from tace_amd import configs, data, structures

ZS = [26]
PRESETS = {"si64": dict(num_channel=16), "tece": dict(num_channel=32, edge_ace_hidden=16, num_head=2)}


def setup(preset: str = "si64"):
    """Structure, edges, domains and the oracle's energy and dE/d(edge vector)."""
    s = structures.bcc_fe(reps=(3, 3, 3), seed=12)
    rc = configs.PRESETS[preset]["cutoff"]
    ei, S = onl.neighbour_list(s["positions"], s["cell"], s["pbc"], rc)
    pos = torch.as_tensor(np.asarray(s["positions"]), dtype=torch.float64)
    cell = torch.as_tensor(np.asarray(s["cell"]), dtype=torch.float64)
    ei = torch.as_tensor(np.asarray(ei), dtype=torch.int64)
    S = torch.as_tensor(np.asarray(S), dtype=torch.float64)
    vec = pos[ei[1]] - pos[ei[0]] + S @ cell
    n = pos.shape[0]
    attrs = data.one_hot(s["numbers"], ZS, torch.float64)
    frac = torch.linalg.solve(cell.T, pos.T).T
    dom = (frac[:, 0] % 1.0 >= 0.5).long()
    cfg = configs.model_cfg(preset, ZS, ei.shape[1] / n, **PRESETS[preset])
    torch.manual_seed(21)
    ref = om.TACE(cfg).double()
    v = vec.clone().requires_grad_(True)
    E0, _ = ref.energy(attrs, ei, v, (v ** 2).sum(1, keepdim=True).sqrt() + 1e-9, torch.zeros(n, dtype=torch.int64),
                       torch.tensor([0, n]), 1)
    (gv0,) = torch.autograd.grad(E0.sum(), v)
    return dict(ei=ei, S=S, vec=vec, attrs=attrs, dom=dom, cfg=cfg, ref=ref, E0=E0.detach(), gv0=gv0)


class GlooExchange:
    """One domain's ML-IAP communication: every rank's local rows are
    gathered (host memory, gloo) and each ghost row copies its owner's row;
    backwards, every rank's ghost-row gradients are gathered and each rank
    sums those of the ghosts it owns into its local rows."""

    def __init__(self, nlocal, ghost_dom, ghost_idx, device):
        import torch.distributed as dist

        self.dist = dist
        self.nlocal, self.device = nlocal, device
        self.ghost_dom, self.ghost_idx = ghost_dom, ghost_idx
        objs = [None, None]
        dist.all_gather_object(objs, (nlocal, ghost_dom.tolist(), ghost_idx.tolist()))
        self.ranks = [(nl, torch.tensor(gd, dtype=torch.int64), torch.tensor(gi, dtype=torch.int64))
                      for nl, gd, gi in objs]

    def _gather(self, rows: torch.Tensor, n_max: int):
        pad = torch.zeros(n_max, rows.shape[1], dtype=rows.dtype)
        pad[:rows.shape[0]] = rows
        out = [torch.empty_like(pad) for _ in range(2)]
        self.dist.all_gather(out, pad)
        return out

    def forward_exchange(self, inp, out, n):
        loc = inp[:self.nlocal].detach().cpu()
        allrows = self._gather(loc, max(r[0] for r in self.ranks))
        ghosts = torch.empty(len(self.ghost_dom), inp.shape[1], dtype=inp.dtype)
        for d in (0, 1):
            sel = (self.ghost_dom == d).nonzero().squeeze(1)
            ghosts[sel] = allrows[d][self.ghost_idx[sel]]
        out[:self.nlocal] = inp[:self.nlocal]
        out[self.nlocal:] = ghosts.to(self.device)

    def reverse_exchange(self, gout, gin, n):
        gg = gout[self.nlocal:].detach().cpu()
        allg = self._gather(gg, max(len(r[1]) for r in self.ranks))
        me = self.dist.get_rank()
        acc = torch.zeros(self.nlocal, gout.shape[1], dtype=gout.dtype)
        for d, (_, gd, gi) in enumerate(self.ranks):
            mine = (gd == me).nonzero().squeeze(1)
            acc.index_add_(0, gi[mine], allg[d][mine])
        gin.zero_()
        gin[:self.nlocal] = gout[:self.nlocal] + acc.to(self.device)


def worker(rank: int, port: int, outdir: str, preset: str = "si64") -> None:
    import torch.distributed as dist

    from tace_amd import model as pm

    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    dist.init_process_group("gloo", rank=rank, world_size=2)
    try:
        dev = torch.device("cuda:0")
        st = setup(preset)
        ei, S, vec, attrs, dom = st["ei"], st["S"], st["vec"], st["attrs"], st["dom"]
        n = attrs.shape[0]
        local_idx = torch.zeros(n, dtype=torch.int64)
        for d in (0, 1):
            m = (dom == d).nonzero().squeeze(1)
            local_idx[m] = torch.arange(len(m))
        mine = (dom[ei[1]] == rank).nonzero().squeeze(1)      # edges whose receiver is local here
        nloc = int((dom == rank).sum())
        ghosts, sender = {}, []
        for k in mine.tolist():
            j, sh = int(ei[0, k]), tuple(int(t) for t in S[k].tolist())
            if sh == (0, 0, 0) and int(dom[j]) == rank:
                sender.append(int(local_idx[j]))
            else:
                sender.append(nloc + ghosts.setdefault((j, sh), len(ghosts)))
        gatoms = torch.tensor([j for (j, _) in ghosts], dtype=torch.int64)
        ex = GlooExchange(nloc, dom[gatoms], local_idx[gatoms], dev)
        locals_ = (dom == rank).nonzero().squeeze(1)
        lmp = dict(edge_vector=vec[mine].to(dev).requires_grad_(True),
                   node_attrs=torch.cat([attrs[locals_], attrs[gatoms]]).to(dev),
                   edge_index=torch.stack([torch.tensor(sender), local_idx[ei[1, mine]]]).to(dev),
                   batch=torch.zeros(nloc, dtype=torch.int64, device=dev),
                   ptr=torch.tensor([0, nloc], dtype=torch.int64, device=dev), lmp_data=ex,
                   natoms=(nloc, len(ghosts)))
        torch.set_default_dtype(torch.float64)
        try:
            m = pm.create_model(st["cfg"])
        finally:
            torch.set_default_dtype(torch.float32)
        pm.load_reference_state_dict(m.readout_fn, st["ref"].state_dict())
        m = m.to(dev)
        m.lmp = True   # what interface/lammps/mliap.py:25-37 does to the model
        m.flags.compute_forces = False
        m.flags.compute_edge_forces = True
        for p in m.parameters():
            p.requires_grad = False
        out = m(lmp)
        np.savez(os.path.join(outdir, f"dom{rank}.npz"), energy=out["energy"].cpu().numpy(),
                 edge_forces=out["edge_forces"].cpu().numpy(), mine=mine.numpy(),
                 n_ghost_foreign=np.array([int((dom[gatoms] != rank).sum())]))
    finally:
        dist.destroy_process_group()
