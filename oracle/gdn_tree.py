"""CPU oracle: restatement of DForkTree's GDN tree-verify path in numpy.

TEST INFRASTRUCTURE ONLY -- imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, never by the product package.

Conventions used throughout (they follow the reference's own):

* ``y``      [B, N, C] float32 holding bf16 values; C = 2*Hk*Dk + Hv*Dv laid out
             ``[q | k | v]`` (tree_kernels.py:142-143, :181).
* ``aa, bb`` [B, N, Hv] raw gate inputs a, b (tree_kernels.py:146, :150).
* ``S0``     [B, Hv, Dk, Dv] -- index (k, v), the view ``tree_gdn_split``
             receives (tree_kernels.py:185); the pool stores it V-major.
* ``anc``    [B, N, N] 0/1, ``anc[i, j] = 1`` iff j is an ancestor-or-self of i.
* v-head h reads q/k head ``h // (Hv // Hk)`` (tree_kernels.py:138).

Pinning (what fixes each function besides its own formula; tests/test_oracle.py):

=====================  =======================================================
function               pinned by
=====================  =======================================================
tree_struct            brute-force parent walks written independently in the
                       test; the reference's 5-squaring closure restated in
                       ``tree_struct_squaring`` agrees for depth <= 31; chain
                       special case (cidx of a chain = sliding window)
tree_links             definition check against a dict-of-children walk
block_invert           ``(I+A) X = I`` and scipy.linalg.solve_triangular
prepare/finish/split   ``recurrent_f64`` (independent fp64 per-node recurrence)
                       on random trees, chains (= sequential decoding), N=1,
                       beta=0 closed form, non-ancestor perturbation
                       invariance, topological relabelling invariance
tree_gdn_neumann       equals split for depth <= 15; differs beyond (documents
                       the reference's truncation)
recurrent_f64          chain == textbook sequential delta-rule decode written
                       in the test; one step == closed form
tree_conv              chain + zero state == numpy 1-D convolution (zero
                       padding 3) + SiLU; window == the last 3 inputs
closed_commit          ``replay_path_f64`` (sequential replay of the accepted
snapshot_commit        tokens) and the recurrent state at the accepted node
=====================  =======================================================

The only reference behaviour left unpinned is its TF32 rounding of ``tl.dot``
(absorbed by the rel-L2 2e-3 tolerance).
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


# --------------------------------------------------------------------------
# numeric helpers
# --------------------------------------------------------------------------
def bf16_round(x) -> np.ndarray:
    """Round to the nearest bfloat16 value (ties to even); result is float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).reshape(x.shape)


def softplus_thresh(a):
    """softplus with the threshold 20 of tree_kernels.py:147."""
    a = np.asarray(a)
    return np.where(a > 20.0, a, np.log(1.0 + np.exp(np.minimum(a, 20.0))))


# --------------------------------------------------------------------------
# tree structure (tree_ops.py:68-89, fc1_builder.py:38-47)
# --------------------------------------------------------------------------
def _parent_of(parent, i):
    """Node 0 is the root; any other node's parent is max(parent[i], 0),
    the clamp of tree_ops.py:73."""
    return -1 if i == 0 else max(int(parent[i]), 0)


def tree_struct(parent, kc: int = 4):
    """Ancestor-or-self matrix, depth and conv gather columns of one tree.

    Follows tree_ops.py:68-89 but with the exact closure (a parent walk) in
    place of the five squarings of :75-79, which stop at 31 edges.

    cidx[n, kc-1-r] = kc-1 + (r-th ancestor of n)   if r <= depth[n]
                    = kc-1 - (r - depth[n])         otherwise   (:81-88)
    Returns (anc [N,N] float32 0/1, depth [N] int64, cidx [N,kc] int64).
    """
    parent = np.asarray(parent, dtype=np.int64)
    n = parent.shape[0]
    anc = np.zeros((n, n), dtype=np.float32)
    depth = np.zeros(n, dtype=np.int64)
    cidx = np.zeros((n, kc), dtype=np.int64)
    for i in range(n):
        chain = [i]
        cur = i
        while cur != 0:
            cur = _parent_of(parent, cur)
            chain.append(cur)
            if len(chain) > n:
                raise ValueError("parent array has a cycle")
        anc[i, chain] = 1.0
        depth[i] = len(chain) - 1
        for r in range(kc):
            cidx[i, kc - 1 - r] = (kc - 1 + chain[r]) if r <= depth[i] else (kc - 1 - (r - depth[i]))
    return anc, depth, cidx


def tree_struct_squaring(parent, kc: int = 4):
    """The reference's closure verbatim in arithmetic (tree_ops.py:72-88):
    Anc = (I+P)(I+P^2)(I+P^4)(I+P^8)(I+P^16) > 0.5, complete up to 31 edges."""
    parent = np.asarray(parent, dtype=np.int64)
    n = parent.shape[0]
    P = np.zeros((n, n), dtype=np.float64)
    P[np.arange(1, n), np.maximum(parent[1:], 0)] = 1.0
    I = np.eye(n)
    Anc, Pk = I + P, P @ P
    for _ in range(4):
        Anc = Anc @ (I + Pk)
        Pk = Pk @ Pk
    Anc = (Anc > 0.5).astype(np.float32)
    depth = Anc.sum(1).astype(np.int64) - 1
    cols, Pr = [], I
    for r in range(kc):
        if r > 0:
            Pr = Pr @ P
        a_r = Pr.argmax(1)
        cols.append(np.where(r <= depth, kc - 1 + a_r, kc - 1 - (r - depth)))
    return Anc, depth, np.stack(cols[::-1], 1).astype(np.int64)


def tree_links(parent):
    """First child ``nxt`` and next sibling ``sib`` (fc1_builder.py:41-47),
    -1 where none.  Nodes are compared with the builder's own parent array
    (root -1)."""
    parent = np.asarray(parent, dtype=np.int64)
    n = parent.shape[0]
    u = np.arange(n)
    children = (parent[None, :] == u[:, None]) & (u[None, :] > 0)
    nxt = np.where(children, u[None, :], n).min(-1)
    sibling = (parent[:, None] == parent[None, :]) & (u[None, :] > u[:, None])
    sib = np.where(sibling, u[None, :], n).min(-1)
    return np.where(nxt < n, nxt, -1), np.where(sib < n, sib, -1)


def anc_bits(anc) -> np.ndarray:
    """Pack an ancestor matrix [..., N, N] (N <= 64) into uint64 row masks."""
    anc = np.asarray(anc) > 0.5
    n = anc.shape[-1]
    w = (np.uint64(1) << np.arange(n, dtype=np.uint64))
    return (anc.astype(np.uint64) * w).sum(-1, dtype=np.uint64)


# --------------------------------------------------------------------------
# split verify: prepare -> block inverse -> finish (tree_kernels.py:135-208)
# --------------------------------------------------------------------------
def _split_qkv(y, Hk, Hv, Dk, Dv):
    B, N, _ = y.shape
    KD = Hk * Dk
    q = y[:, :, :KD].reshape(B, N, Hk, Dk).transpose(0, 2, 1, 3)
    k = y[:, :, KD:2 * KD].reshape(B, N, Hk, Dk).transpose(0, 2, 1, 3)
    v = y[:, :, 2 * KD:2 * KD + Hv * Dv].reshape(B, N, Hv, Dv).transpose(0, 2, 1, 3)
    return q, k, v


def _gates(aa, bb, A_log, dt_bias, neg_exp_A, dtype):
    a = np.swapaxes(np.asarray(aa, dtype), 1, 2) + np.asarray(dt_bias, dtype)[None, :, None]
    sp = softplus_thresh(a).astype(dtype)
    if neg_exp_A is not None:
        dec = np.asarray(neg_exp_A, dtype)
    else:
        dec = -np.exp(np.asarray(A_log, dtype))
    g = dec[None, :, None] * sp
    b = np.swapaxes(np.asarray(bb, dtype), 1, 2)
    with np.errstate(over="ignore"):  # b -> -inf gives beta = 0 exactly
        beta = (1.0 / (1.0 + np.exp(-b))).astype(dtype)
    return g.astype(dtype), beta


def prepare(y, aa, bb, A_log, dt_bias, anc, Hk, Hv, Dk, scale=None, neg_exp_A=None):
    """fp32 restatement of ``_tree_prepare`` (tree_kernels.py:135-164).

    Returns q, k [B,Hv,N,Dk] (normalised, q scaled), g, G, beta [B,Hv,N] and
    A [B,Hv,N,N] = strict-ancestor-masked (beta_i k_i.k_j) e^{G_i-G_j}.
    """
    y = np.asarray(y, F32)
    R = Hv // Hk
    scale = Dk ** (-0.5) if scale is None else scale
    B, N, _ = y.shape
    KD = Hk * Dk
    q = y[:, :, :KD].reshape(B, N, Hk, Dk).transpose(0, 2, 1, 3)
    k = y[:, :, KD:2 * KD].reshape(B, N, Hk, Dk).transpose(0, 2, 1, 3)
    q = q * (1.0 / np.sqrt((q * q).sum(-1, dtype=F32) + F32(1e-6)))[..., None] * F32(scale)
    k = k * (1.0 / np.sqrt((k * k).sum(-1, dtype=F32) + F32(1e-6)))[..., None]
    q = np.repeat(q.astype(F32), R, axis=1)
    k = np.repeat(k.astype(F32), R, axis=1)
    g, beta = _gates(aa, bb, A_log, dt_bias, neg_exp_A, F32)
    anc = np.asarray(anc, F32)
    G = (anc[:, None, :, :] * g[:, :, None, :]).sum(-1, dtype=F32)
    isanc = anc[:, None] > 0.5
    N = anc.shape[-1]
    offd = ~np.eye(N, dtype=bool)
    with np.errstate(over="ignore"):
        D = np.where(isanc, np.exp(G[..., :, None] - G[..., None, :]), F32(0)).astype(F32)
    A = np.where(isanc & offd, np.matmul(k * beta[..., None], np.swapaxes(k, -1, -2)) * D, F32(0))
    return q, k, g, G, beta, A.astype(F32)


def _diag_inv16(a):
    """Forward substitution of one 16x16 unit-lower block
    (fc1_block_inverse.py:10-20): returns (I + strict_lower(a))^-1."""
    r = np.arange(16)
    lower = r[:, None] > r[None, :]
    inv = -np.where(lower, a, F32(0)).astype(F32)
    for i in range(2, 16):
        row = -a[..., i, :]
        row = np.where(r < i, row, F32(0))
        row = row + (row[..., :, None] * inv).sum(-2, dtype=F32)
        inv[..., i, :] = row
    return (inv + np.eye(16, dtype=F32)).astype(F32)


def block_invert(A):
    """(I + A)^-1 of a strictly-lower A, N in {16, 32, 64}: 16x16 diagonal
    blocks by forward substitution, off-diagonal blocks by
    b_ij = -d_i sum_{m=j}^{i-1} a_im x_mj (fc1_block_inverse.py:36-83)."""
    A = np.asarray(A, F32)
    n = A.shape[-1]
    if n not in (16, 32, 64):
        raise KeyError(n)
    nb = n // 16

    def blk(i, j):
        return A[..., 16 * i:16 * i + 16, 16 * j:16 * j + 16]

    d = [_diag_inv16(blk(i, i)) for i in range(nb)]
    X = np.zeros_like(A)
    xb = {(i, i): d[i] for i in range(nb)}
    for i in range(nb):
        for j in range(i):
            acc = None
            for m in range(j, i):
                t = np.matmul(blk(i, m), xb[m, j])
                acc = t if acc is None else acc + t
            xb[i, j] = -np.matmul(d[i], acc)
    for (i, j), v in xb.items():
        X[..., 16 * i:16 * i + 16, 16 * j:16 * j + 16] = v
    return X.astype(F32)


def finish(y, S0, anc, q, k, G, beta, X, Hk, Hv, Dk, Dv):
    """fp32 restatement of ``_tree_finish`` (tree_kernels.py:166-191).

    U = X(beta v); Wk = X(beta e^G k); vn = U - Wk S0;
    o = (e^G q) S0 + (q k^T o D) vn.   Returns o [B,N,Hv,Dv], vn [B,Hv,N,Dv].
    """
    y = np.asarray(y, F32)
    _, _, v = _split_qkv(y, Hk, Hv, Dk, Dv)
    anc = np.asarray(anc, F32)[:, None]
    with np.errstate(over="ignore"):
        D = np.where(anc > 0.5, np.exp(G[..., :, None] - G[..., None, :]), F32(0)).astype(F32)
    eG = np.exp(G).astype(F32)
    S0 = np.asarray(S0, F32)
    U = np.matmul(X, v * beta[..., None])
    Wk = np.matmul(X, k * beta[..., None] * eG[..., None])
    vn = U - np.matmul(Wk, S0)
    Pq = np.matmul(q, np.swapaxes(k, -1, -2)) * D
    o = np.matmul(q * eG[..., None], S0) + np.matmul(Pq, vn)
    return np.ascontiguousarray(o.transpose(0, 2, 1, 3)).astype(F32), vn.astype(F32)


def _pad_pow2(n):
    return max(16, 1 << (int(n) - 1).bit_length())


def tree_gdn_split(y, aa, bb, A_log, dt_bias, S0, anc, Hk, Hv, Dk, Dv, scale=None, neg_exp_A=None):
    """The split verify end to end (tree_kernels.py:193-208), batched.

    N that is not 16/32/64 is padded to the next of them with isolated,
    zero-input nodes (their rows/columns of anc are empty), which leaves the
    real nodes' results unchanged because A is ancestor-masked.
    Returns dict(o, vn, k, q, G, g, beta, X, A).
    """
    y = np.asarray(y, F32)
    B, N, C = y.shape
    NP = _pad_pow2(N)
    if NP != N:
        pad = NP - N
        y = np.concatenate([y, np.zeros((B, pad, C), F32)], 1)
        aa = np.concatenate([np.asarray(aa, F32), np.zeros((B, pad, Hv), F32)], 1)
        bb = np.concatenate([np.asarray(bb, F32), np.zeros((B, pad, Hv), F32)], 1)
        a2 = np.zeros((B, NP, NP), F32)
        a2[:, :N, :N] = anc
        anc = a2
    q, k, g, G, beta, A = prepare(y, aa, bb, A_log, dt_bias, anc, Hk, Hv, Dk, scale, neg_exp_A)
    if NP != N:  # padded nodes are masked exactly as the reference masks rows >= N (:149-151)
        g[..., N:] = 0
        beta[..., N:] = 0
        G[..., N:] = 0
    X = block_invert(A)
    o, vn = finish(y, S0, anc, q, k, G, beta, X, Hk, Hv, Dk, Dv)
    return dict(o=o[:, :N], vn=vn[:, :, :N], k=k[:, :, :N], q=q[:, :, :N], G=G[..., :N],
                g=g[..., :N], beta=beta[..., :N], X=X[..., :N, :N], A=A[..., :N, :N])


def tree_gdn_neumann(y, aa, bb, A_log, dt_bias, S0, anc, Hk, Hv, Dk, Dv, scale=None, neg_exp_A=None):
    """The single-kernel variant ``_tree_gdn_kernel`` (tree_kernels.py:35-81):
    same math, but X = (I-A)(I+A^2)(I+A^4)(I+A^8) = sum_{n<16} (-A)^n, which
    equals (I+A)^-1 only while every path has at most 15 edges."""
    y = np.asarray(y, F32)
    q, k, g, G, beta, A = prepare(y, aa, bb, A_log, dt_bias, anc, Hk, Hv, Dk, scale, neg_exp_A)
    n = A.shape[-1]
    I = np.eye(n, dtype=F32)
    X = I - A
    P = np.matmul(A, A)
    X = np.matmul(X, I + P)
    P = np.matmul(P, P)
    X = np.matmul(X, I + P)
    P = np.matmul(P, P)
    X = np.matmul(X, I + P)
    o, vn = finish(y, S0, anc, q, k, G, beta, X.astype(F32), Hk, Hv, Dk, Dv)
    return dict(o=o, vn=vn, k=k, G=G, X=X)


# --------------------------------------------------------------------------
# independent fp64 recurrence (the pin)
# --------------------------------------------------------------------------
def recurrent_f64(y, aa, bb, A_log, dt_bias, S0, parent, Hk, Hv, Dk, Dv, scale=None,
                  neg_exp_A=None, keep_states=False):
    """Gated delta rule run node by node on the tree, in float64.

    For node i with parent p (the root starts from S0):
        S~ = e^{g_i} S_p ;  u_i = beta_i (v_i - S~^T k_i) ;
        S_i = S~ + k_i u_i^T ;  o_i = S_i^T q_i
    with q, k normalised as in tree_kernels.py:144-145.  ``y`` [N, C] and the
    rest are ONE request.  Returns dict(o [N,Hv,Dv], vn [Hv,N,Dv], G [Hv,N],
    states [Hv,N,Dk,Dv] if keep_states).
    """
    y = np.asarray(y, np.float64)[None]
    N = y.shape[1]
    R = Hv // Hk
    scale = Dk ** (-0.5) if scale is None else scale
    q, k, v = _split_qkv(y, Hk, Hv, Dk, Dv)
    q, k, v = q[0], k[0], v[0]
    q = q / np.sqrt((q * q).sum(-1) + 1e-6)[..., None] * scale
    k = k / np.sqrt((k * k).sum(-1) + 1e-6)[..., None]
    q = np.repeat(q, R, axis=0)
    k = np.repeat(k, R, axis=0)
    g, beta = _gates(np.asarray(aa, np.float64)[None], np.asarray(bb, np.float64)[None],
                     A_log, dt_bias, neg_exp_A, np.float64)
    g, beta = g[0], beta[0]
    S0 = np.asarray(S0, np.float64)
    states = np.zeros((Hv, N, Dk, Dv))
    o = np.zeros((N, Hv, Dv))
    vn = np.zeros((Hv, N, Dv))
    G = np.zeros((Hv, N))
    for i in range(N):
        p = _parent_of(parent, i)
        Sp = S0 if p < 0 else states[:, p]
        Gp = 0.0 if p < 0 else G[:, p]
        St = np.exp(g[:, i])[:, None, None] * Sp
        u = beta[:, i][:, None] * (v[:, i] - np.einsum("hkv,hk->hv", St, k[:, i]))
        Si = St + k[:, i][:, :, None] * u[:, None, :]
        states[:, i] = Si
        vn[:, i] = u
        G[:, i] = Gp + g[:, i]
        o[i] = np.einsum("hkv,hk->hv", Si, q[:, i])
    out = dict(o=o, vn=vn, G=G, k=k, q=q, g=g, beta=beta)
    if keep_states:
        out["states"] = states
    return out


def replay_path_f64(y, aa, bb, A_log, dt_bias, S0, path, Hk, Hv, Dk, Dv, scale=None, neg_exp_A=None):
    """Sequential decode of the accepted tokens ``path`` (root first), fp64:
    the state a plain recurrent decoder holds after consuming them."""
    path = [int(t) for t in path]
    y = np.asarray(y)[path]
    aa = np.asarray(aa)[path]
    bb = np.asarray(bb)[path]
    chain = np.arange(len(path)) - 1
    r = recurrent_f64(y, aa, bb, A_log, dt_bias, S0, chain, Hk, Hv, Dk, Dv, scale, neg_exp_A,
                      keep_states=True)
    return r["states"][:, -1]


# --------------------------------------------------------------------------
# tree-parent causal conv1d (fc1_conv.py:7-27, tree_kernels.py:17-33)
# --------------------------------------------------------------------------
def tree_conv(x, conv_state, weight, bias, cidx, silu: bool = True):
    """y[n,c] = act(sum_j w[c,j] * xt[cidx[n,j], c] + b[c]), where
    xt = [conv_state[:, :KC-1] (as columns) || x (N tokens)].

    x [N, C]; conv_state [C, >=KC-1]; weight [C, KC]; bias [C] or None;
    cidx [N, KC].  Accumulates in fp32 in tap order (fc1_conv.py:15-22).
    Returns (y [N,C] float32 before output rounding,
             window [N, C, KC-1] = the values at taps 1..KC-1 (fc1_conv.py:23-24)).
    """
    x = np.asarray(x, F32)
    weight = np.asarray(weight, F32)
    KC = weight.shape[1]
    cs = np.asarray(conv_state, F32)[:, :KC - 1]
    xt = np.concatenate([cs.T, x], 0)
    cidx = np.asarray(cidx, np.int64)
    win = xt[cidx]  # [N, KC, C]
    acc = np.zeros((x.shape[0], x.shape[1]), F32)
    for j in range(KC):
        acc = acc + win[:, j, :] * weight[None, :, j]
    if bias is not None:
        acc = acc + np.asarray(bias, F32)[None]
    y = acc / (F32(1) + np.exp(-acc)) if silu else acc
    return y.astype(F32), np.ascontiguousarray(win[:, 1:, :].transpose(0, 2, 1))


# --------------------------------------------------------------------------
# closed-form accepted-path commit (tree_kernels.py:111-127, fc1_fused.py:26-49)
# --------------------------------------------------------------------------
def closed_commit(S, keys, values, gains, path, u=None, anc=None, dtype=F32):
    """S_u = e^{G_u} S + sum_t on_t e^{G_u - G_t} k_t vn_t^T for one request.

    S [H, Dk, Dv]; keys [H, N, Dk]; values [H, N, Dv]; gains [H, N];
    path: accepted node ids (-1 entries ignored).  ``u`` defaults to the last
    valid path entry (tree_kernels.py:118).  With ``anc`` given, a path node
    contributes only if it is an ancestor-or-self of u (fc1_fused.py:41);
    without it every listed node contributes (tree_kernels.py:119-122).
    """
    path = [int(t) for t in path]
    valid = [t for t in path if t >= 0]
    if u is None:
        u = valid[-1]
    S = np.asarray(S, dtype)
    keys, values, gains = (np.asarray(a, dtype) for a in (keys, values, gains))
    on = [t for t in valid if anc is None or anc[u, t] > 0.5]
    out = S * np.exp(gains[:, u])[:, None, None]
    if on:
        w = np.exp(gains[:, u][:, None] - gains[:, on])  # [H, T]
        kk = keys[:, on, :] * w[..., None]
        out = out + np.matmul(np.swapaxes(kk, -1, -2), values[:, on, :])
    return out.astype(dtype)
