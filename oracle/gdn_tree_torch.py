"""The split verify and the closed-form commit as batched PyTorch fp32 CPU ops.

TEST INFRASTRUCTURE ONLY -- the CPU baseline that ``bench.py``'s
``cpu_baseline`` leg times (and ``tests/`` pins), never the product.

It is the same algorithm as ``oracle.gdn_tree`` (the reference's
``_tree_prepare`` tree_kernels.py:135-164, the WY inverse of
fc1_block_inverse.py:10-83, ``_tree_finish`` tree_kernels.py:166-191 and the
closed commit tree_kernels.py:111-127), written as whole-batch torch ops so
that the baseline runs on every core: (I + A)^-1 comes from the library's
unit-lower triangular solve, and a batch of accepted paths is committed at
once through a per-request path mask.

Pinned by tests/test_oracle.py against ``oracle.gdn_tree`` (itself pinned by
the fp64 per-node recurrence and the sequential replay of accepted tokens).
"""
from __future__ import annotations

import torch


def tree_gdn_split(y, aa, bb, A_log, dt_bias, S0, anc, Hk: int, Hv: int, Dk: int, Dv: int, scale=None):
    """y [B, N, C] (bf16 values), aa, bb [B, N, Hv], S0 [B, Hv, Dk, Dv] (k, v),
    anc [B, N, N] ancestor-or-self 0/1.  Returns dict(o [B, N, Hv, Dv],
    vn [B, Hv, N, Dv], k [B, Hv, N, Dk], G [B, Hv, N])."""
    f = torch.float32
    y, aa, bb, S0, anc = (t.to(f) for t in (y, aa, bb, S0, anc))
    B, N, _ = y.shape
    R = Hv // Hk
    scale = Dk ** -0.5 if scale is None else scale
    KD = Hk * Dk
    q = y[:, :, :KD].reshape(B, N, Hk, Dk).transpose(1, 2)
    k = y[:, :, KD:2 * KD].reshape(B, N, Hk, Dk).transpose(1, 2)
    v = y[:, :, 2 * KD:2 * KD + Hv * Dv].reshape(B, N, Hv, Dv).transpose(1, 2)
    q = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6) * scale
    k = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    q = q.repeat_interleave(R, dim=1)
    k = k.repeat_interleave(R, dim=1)
    a = aa.transpose(1, 2) + dt_bias.to(f)[None, :, None]
    sp = torch.where(a > 20, a, torch.log1p(torch.exp(torch.clamp(a, max=20))))  # threshold 20 (:147)
    g = -torch.exp(A_log.to(f))[None, :, None] * sp
    beta = torch.sigmoid(bb.transpose(1, 2))
    G = torch.matmul(g, anc.transpose(1, 2))                  # [B, Hv, N]: sum over ancestors-or-self
    isanc = (anc > 0.5)[:, None]
    D = torch.where(isanc, torch.exp(G[..., :, None] - G[..., None, :]), torch.zeros((), dtype=f))
    strict = isanc & ~torch.eye(N, dtype=torch.bool)
    A = torch.where(strict, torch.matmul(k * beta[..., None], k.transpose(-1, -2)) * D, torch.zeros((), dtype=f))
    eye = torch.eye(N, dtype=f).expand(B, Hv, N, N)
    X = torch.linalg.solve_triangular(eye + A, eye, upper=False, unitriangular=True)
    eG = torch.exp(G)[..., None]
    vn = torch.matmul(X, beta[..., None] * (v - torch.matmul(k * eG, S0)))
    o = torch.matmul(q * eG, S0) + torch.matmul(torch.matmul(q, k.transpose(-1, -2)) * D, vn)
    return dict(o=o.transpose(1, 2), vn=vn, k=k, G=G)


def closed_commit(S0, k, vn, G, on, u):
    """S_u = e^{G_u} S0 + sum_t on_t e^{G_u - G_t} k_t vn_t^T for every request:
    S0 [B, Hv, Dk, Dv], k [B, Hv, N, Dk], vn [B, Hv, N, Dv], G [B, Hv, N],
    on [B, N] 0/1 (the accepted path's nodes), u [B] long (its last node)."""
    Gu = G.gather(2, u[:, None, None].expand(-1, G.shape[1], 1))  # [B, Hv, 1]
    w = torch.exp(Gu - G) * on[:, None, :].to(G.dtype)
    return torch.exp(Gu)[..., None] * S0 + torch.matmul((k * w[..., None]).transpose(-1, -2), vn)
