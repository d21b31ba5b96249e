"""Glue between synthetic batches and the CPU oracle (test helper)."""
from __future__ import annotations

import numpy as np
import torch

from oracle import gdn_tree as O


def np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().float().numpy()


def request_slices(batch):
    cu = batch.cu_seqlens.tolist()
    return [slice(cu[i], cu[i + 1]) for i in range(len(cu) - 1)]


def oracle_verify(batch, scale=None):
    """Per request: dict(o [n,hv,128], vn [hv,n,128], k [hv,n,128], G [hv,n],
    anc [n,n]) from the fp32 restatement."""
    out = []
    y, a, b = np32(batch.y), np32(batch.a), np32(batch.b)
    A_log, dtb = np32(batch.A_log), np32(batch.dt_bias)
    par = batch.parent.numpy()
    for r, sl in enumerate(request_slices(batch)):
        anc, depth, cidx = O.tree_struct(par[sl])
        S0 = np32(batch.state[r]).transpose(0, 2, 1)[None]  # [1, hv, K, V]
        res = O.tree_gdn_split(y[sl][None], a[sl][None], b[sl][None], A_log, dtb, S0, anc[None],
                               batch.hk, batch.hv, 128, 128, scale=scale)
        out.append(dict(o=res["o"][0], vn=res["vn"][0], k=res["k"][0], G=res["G"][0], anc=anc,
                        depth=depth, cidx=cidx))
    return out


def oracle_recurrent(batch, r, keep_states=False):
    sl = request_slices(batch)[r]
    S0 = np32(batch.state[r]).transpose(0, 2, 1)
    return O.recurrent_f64(np32(batch.y[sl]), np32(batch.a[sl]), np32(batch.b[sl]), np32(batch.A_log),
                           np32(batch.dt_bias), S0, batch.parent[sl].numpy(), batch.hk, batch.hv, 128, 128,
                           keep_states=keep_states)
