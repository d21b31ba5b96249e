"""Seeded synthetic inputs for the GDN tree-verify workloads.

Every request draws from its own CPU ``torch.Generator`` seeded with
``seed * 1_000_003 + layer * 1009 + request``, so a CPU checker and the GPU
see identical bytes.  Distributions (all workloads):

* q, k, v raw rows: bf16 N(0,1) packed as y = [q | k | v] (the kernel
  L2-normalises q and k per head);
* b ~ N(0,1) (beta = sigmoid(b)); a ~ N(0,1) with dt_bias = 0 and
  A_log = ln 0.5, so g = -0.5 softplus(a);
* S0: fp32 N(0, 0.02^2) per head in the pool's V-major layout [H, V, K];
* trees: node 0 is the root (parent -1); ``random`` draws parent[i] uniform
  in [0, i-1]; ``chain`` is parent[i] = i-1; ``bushy`` is depth <= 2.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

D = 128


def request_seed(seed: int, layer: int, req: int) -> int:
    return seed * 1_000_003 + layer * 1009 + req


def tree_parents(n: int, kind: str, gen: torch.Generator) -> torch.Tensor:
    """int32 parent indices of one tree (parent[0] = -1, parent[i] < i)."""
    p = torch.empty(n, dtype=torch.int32)
    p[0] = -1
    if n == 1:
        return p
    if kind == "chain":
        p[1:] = torch.arange(0, n - 1, dtype=torch.int32)
    elif kind == "random":
        u = torch.rand(n - 1, generator=gen, dtype=torch.float64)
        i = torch.arange(1, n, dtype=torch.float64)
        p[1:] = torch.clamp((u * i).floor(), max=i - 1).to(torch.int32)
    elif kind == "bushy":
        m = max(1, int(round(math.sqrt(n - 1))))
        m = min(m, n - 1)
        p[1:m + 1] = 0
        if n - 1 > m:
            p[m + 1:] = torch.randint(1, m + 1, (n - 1 - m,), generator=gen, dtype=torch.int32)
    else:
        raise ValueError(f"unknown tree kind {kind!r}")
    return p


def accepted_path(parent: torch.Tensor, max_len: int, gen: torch.Generator) -> torch.Tensor:
    """A seeded root-to-node walk: target length uniform in [1, max_len],
    each step to a uniformly chosen child, stopping early at a leaf."""
    n = parent.numel()
    children = [[] for _ in range(n)]
    for i in range(1, n):
        children[int(parent[i])].append(i)
    target = int(torch.randint(1, max_len + 1, (1,), generator=gen))
    path = [0]
    while len(path) < target and children[path[-1]]:
        ch = children[path[-1]]
        path.append(ch[int(torch.randint(0, len(ch), (1,), generator=gen))])
    return torch.tensor(path, dtype=torch.int32)


@dataclass
class Batch:
    """One layer's verify inputs for B requests (CPU or device tensors)."""
    y: torch.Tensor          # [rows, 2*hk*128 + hv*128] bf16
    a: torch.Tensor          # [rows, hv] f32
    b: torch.Tensor          # [rows, hv] f32
    A_log: torch.Tensor      # [hv] f32
    dt_bias: torch.Tensor    # [hv] f32
    state: torch.Tensor      # [B, hv, V, K] f32 (pool layout)
    parent: torch.Tensor     # [rows] int32 local parent index
    cu_seqlens: torch.Tensor  # [B+1] int32
    sizes: list
    hk: int
    hv: int

    @property
    def batch(self):
        return len(self.sizes)

    @property
    def n_max(self):
        return max(self.sizes)

    def to(self, device):
        kw = {f: getattr(self, f) for f in self.__dataclass_fields__}
        for f, v in kw.items():
            if isinstance(v, torch.Tensor):
                kw[f] = v.to(device)
        return Batch(**kw)


def make_batch(seed: int, layer: int, sizes, hk: int = 16, hv: int = 32, kinds="random",
               state: bool = True) -> Batch:
    """Inputs of one layer for requests with node counts ``sizes``."""
    sizes = list(sizes)
    if isinstance(kinds, str):
        kinds = [kinds] * len(sizes)
    C = 2 * hk * D + hv * D
    ys, as_, bs, ss, ps = [], [], [], [], []
    for r, (n, kind) in enumerate(zip(sizes, kinds)):
        g = torch.Generator().manual_seed(request_seed(seed, layer, r))
        ps.append(tree_parents(n, kind, g))
        ys.append(torch.randn(n, C, generator=g).to(torch.bfloat16))
        as_.append(torch.randn(n, hv, generator=g))
        bs.append(torch.randn(n, hv, generator=g))
        if state:
            ss.append(torch.randn(hv, D, D, generator=g) * 0.02)
    cu = torch.zeros(len(sizes) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(sizes, dtype=torch.int32), 0)
    return Batch(y=torch.cat(ys), a=torch.cat(as_), b=torch.cat(bs),
                 A_log=torch.full((hv,), math.log(0.5)), dt_bias=torch.zeros(hv),
                 state=torch.stack(ss) if state else torch.empty(0), parent=torch.cat(ps),
                 cu_seqlens=cu, sizes=sizes, hk=hk, hv=hv)


def ragged_sizes(batch: int, lo: int, hi: int, seed: int):
    """Per-request tree sizes uniform in [lo, hi] and a shape mix of thirds
    (chain / bushy / random)."""
    g = torch.Generator().manual_seed(seed * 1_000_003 + 7)
    sizes = torch.randint(lo, hi + 1, (batch,), generator=g).tolist()
    kinds = [("chain", "bushy", "random")[i % 3] for i in range(batch)]
    return sizes, kinds


def device_randn_(t: torch.Tensor, seed: int, std: float = 1.0) -> torch.Tensor:
    """Fill a (large) device tensor from a seeded device generator."""
    g = torch.Generator(device=t.device).manual_seed(seed)
    if t.dtype in (torch.float32, torch.float64):
        t.normal_(0.0, std, generator=g)
    else:
        tmp = torch.empty(t.shape, device=t.device, dtype=torch.float32).normal_(0.0, std, generator=g)
        t.copy_(tmp)
    return t
