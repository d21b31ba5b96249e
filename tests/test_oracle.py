"""CPU pins of the oracle (no GPU).  Each check is chosen so that a plausible
slip in the restatement -- a dropped term, a wrong sign, an index or a
transposed operand -- fails it."""
import numpy as np
import pytest
import scipy.linalg

from conftest import rel_l2
from oracle import gdn_tree as O

RNG = np.random.default_rng(1234)
D = 128


def rand_tree(n, kind, rng=RNG):
    p = np.full(n, -1, np.int64)
    for i in range(1, n):
        p[i] = i - 1 if kind == "chain" else rng.integers(0, i)
    return p


def inputs(n, hk=2, hv=4, rng=RNG, beta_zero=False):
    C = 2 * hk * D + hv * D
    y = O.bf16_round(rng.standard_normal((n, C)).astype(np.float32))
    aa = rng.standard_normal((n, hv)).astype(np.float32)
    bb = (np.full((n, hv), -1e4, np.float32) if beta_zero else rng.standard_normal((n, hv)).astype(np.float32))
    A_log = np.full(hv, np.log(0.5), np.float32)
    dtb = np.zeros(hv, np.float32)
    S0 = (rng.standard_normal((hv, D, D)) * 0.02).astype(np.float32)
    return y, aa, bb, A_log, dtb, S0


# ---------------------------------------------------------------- tree structure
def brute_ancestors(parent, i):
    out = {i}
    while i != 0:
        i = max(int(parent[i]), 0)
        out.add(i)
    return out


@pytest.mark.parametrize("n,kind", [(1, "random"), (5, "chain"), (32, "random"), (32, "chain"), (64, "random"),
                                    (64, "chain")])
def test_tree_struct_brute_force(n, kind):
    p = rand_tree(n, kind)
    anc, depth, cidx = O.tree_struct(p, 4)
    for i in range(n):
        a = brute_ancestors(p, i)
        assert set(np.nonzero(anc[i])[0]) == a
        assert depth[i] == len(a) - 1
        # cidx walks up the chain: column 3 is the node itself, column 3-r its r-th ancestor
        chain = sorted(a, key=lambda j: -len(brute_ancestors(p, j)))
        for r in range(4):
            want = 3 + chain[r] if r < len(chain) else 3 - (r - (len(chain) - 1))
            assert cidx[i, 3 - r] == want


def test_chain_cidx_is_sliding_window():
    n = 20
    _, _, cidx = O.tree_struct(np.arange(n) - 1, 4)
    xt_cols = np.arange(n)[:, None] + np.arange(4)[None, :]  # [state(3) || tokens]: token n at column 3+n
    assert np.array_equal(cidx, xt_cols)


def test_squaring_closure_agrees_to_31_edges_and_fails_beyond():
    for kind in ("random", "chain"):
        p = rand_tree(32, kind)
        for a, b in zip(O.tree_struct(p), O.tree_struct_squaring(p)):
            assert np.array_equal(a, b)
    p = np.arange(64) - 1  # a 63-edge chain: the reference's closure stops at 31 edges
    assert not np.array_equal(O.tree_struct(p)[0], O.tree_struct_squaring(p)[0])
    assert O.tree_struct(p)[1][-1] == 63 and O.tree_struct_squaring(p)[1][-1] == 31


def test_tree_links_definition():
    p = rand_tree(40, "random")
    nxt, sib = O.tree_links(p)
    kids = {u: [v for v in range(1, 40) if p[v] == u] for u in range(40)}
    for u in range(40):
        assert nxt[u] == (min(kids[u]) if kids[u] else -1)
        sibs = [v for v in range(u + 1, 40) if p[v] == p[u]] if u > 0 else []
        assert sib[u] == (min(sibs) if sibs else -1)


def test_anc_bits_roundtrip():
    p = rand_tree(64, "random")
    anc = O.tree_struct(p)[0]
    bits = O.anc_bits(anc)
    back = ((bits[:, None] >> np.arange(64, dtype=np.uint64)[None, :]) & np.uint64(1)).astype(np.float32)
    assert np.array_equal(back, anc)


# ---------------------------------------------------------------- block inverse
@pytest.mark.parametrize("n", [16, 32, 64])
def test_block_invert_against_scipy(n):
    A = np.tril(RNG.standard_normal((3, n, n)).astype(np.float32) * 0.3, -1)
    X = O.block_invert(A)
    for m in range(3):
        want = scipy.linalg.solve_triangular(np.eye(n) + A[m], np.eye(n), lower=True)
        assert np.abs(X[m] - want).max() < 1e-4
        assert np.abs((np.eye(n) + A[m]) @ X[m] - np.eye(n)).max() < 1e-4
        assert np.all(np.triu(X[m], 1) == 0)


def test_block_invert_ignores_upper_part():
    A = RNG.standard_normal((32, 32)).astype(np.float32) * 0.3
    assert np.array_equal(O.block_invert(A), O.block_invert(np.tril(A, -1)))


def test_block_invert_rejects_other_sizes():
    with pytest.raises(KeyError):
        O.block_invert(np.zeros((20, 20), np.float32))


# ---------------------------------------------------------------- verify math
def split(n, kind, **kw):
    y, aa, bb, A_log, dtb, S0 = inputs(n, **kw)
    p = rand_tree(n, kind)
    anc = O.tree_struct(p)[0]
    r = O.tree_gdn_split(y[None], aa[None], bb[None], A_log, dtb, S0[None], anc[None], 2, 4, D, D)
    f = O.recurrent_f64(y, aa, bb, A_log, dtb, S0, p, 2, 4, D, D, keep_states=True)
    return r, f, (y, aa, bb, A_log, dtb, S0, p, anc)


@pytest.mark.parametrize("n,kind", [(32, "random"), (32, "chain"), (16, "random"), (64, "random"), (64, "chain"),
                                    (7, "random"), (1, "random")])
def test_split_matches_fp64_recurrence(n, kind):
    r, f, _ = split(n, kind)
    assert rel_l2(r["o"][0], f["o"]) < 1e-5
    assert rel_l2(r["vn"][0], f["vn"]) < 1e-5
    assert rel_l2(r["G"][0], f["G"]) < 1e-6


def test_recurrence_chain_is_textbook_decode():
    """A chain tree is plain sequential gated-delta decoding, written here
    independently: S <- e^g S; S <- S + beta k (v - S^T k)^T; o = S^T q."""
    n, hk, hv = 12, 1, 2
    y, aa, bb, A_log, dtb, S0 = inputs(n, hk=hk, hv=hv)
    f = O.recurrent_f64(y, aa, bb, A_log, dtb, S0, np.arange(n) - 1, hk, hv, D, D)
    q = y[:, :D].astype(np.float64)
    k = y[:, D:2 * D].astype(np.float64)
    for h in range(hv):
        S = S0[h].astype(np.float64)
        for t in range(n):
            qt = q[t] / np.sqrt(q[t] @ q[t] + 1e-6) / np.sqrt(D)
            kt = k[t] / np.sqrt(k[t] @ k[t] + 1e-6)
            vt = y[t, 2 * D + h * D:2 * D + (h + 1) * D].astype(np.float64)
            a = float(aa[t, h])
            g = -np.exp(np.float64(A_log[h])) * (a if a > 20 else np.log1p(np.exp(a)))
            beta = 1 / (1 + np.exp(-float(bb[t, h])))
            S = np.exp(g) * S
            S = S + np.outer(kt, beta * (vt - S.T @ kt))
            assert np.allclose(S.T @ qt, f["o"][t, h], rtol=1e-9, atol=1e-12)


def test_beta_zero_is_pure_decay():
    y, aa, bb, A_log, dtb, S0 = inputs(16, beta_zero=True)
    p = rand_tree(16, "random")
    anc = O.tree_struct(p)[0]
    r = O.tree_gdn_split(y[None], aa[None], bb[None], A_log, dtb, S0[None], anc[None], 2, 4, D, D)
    G = r["G"][0]
    q = r["q"][0]
    want = np.einsum("hn,hnk,hkv->nhv", np.exp(G), q, S0)
    assert rel_l2(r["o"][0], want) < 1e-6
    assert np.abs(r["vn"]).max() < 1e-30


def test_non_ancestor_inputs_do_not_leak():
    r, f, (y, aa, bb, A_log, dtb, S0, p, anc) = split(32, "random")
    leaf = 31
    others = [j for j in range(32) if anc[leaf, j] < 0.5]
    y2, aa2, bb2 = y.copy(), aa.copy(), bb.copy()
    y2[others] = O.bf16_round(RNG.standard_normal((len(others), y.shape[1])).astype(np.float32))
    aa2[others] += 3.0
    bb2[others] -= 2.0
    r2 = O.tree_gdn_split(y2[None], aa2[None], bb2[None], A_log, dtb, S0[None], anc[None], 2, 4, D, D)
    assert np.allclose(r2["o"][0, leaf], r["o"][0, leaf], rtol=1e-5, atol=1e-7)
    changed = [j for j in others if not np.allclose(r2["o"][0, j], r["o"][0, j])]
    assert changed, "perturbing a node must change its own output"


def test_topological_relabelling_invariance():
    n = 24
    r, f, (y, aa, bb, A_log, dtb, S0, p, anc) = split(n, "random")
    # any order in which parents precede children: depth-first from the root
    kids = {u: [v for v in range(1, n) if p[v] == u] for u in range(n)}
    order, stack = [], [0]
    while stack:
        u = stack.pop()
        order.append(u)
        stack.extend(reversed(kids[u]))
    perm = np.array(order)
    inv = np.argsort(perm)
    p2 = np.array([-1] + [inv[p[perm[i]]] for i in range(1, n)])
    anc2 = O.tree_struct(p2)[0]
    r2 = O.tree_gdn_split(y[perm][None], aa[perm][None], bb[perm][None], A_log, dtb, S0[None], anc2[None], 2, 4, D, D)
    assert rel_l2(r2["o"][0], r["o"][0][perm]) < 1e-5


def test_single_node_is_one_recurrent_step():
    r, f, (y, aa, bb, A_log, dtb, S0, p, anc) = split(1, "random")
    st = f["states"][:, 0]
    assert rel_l2(r["o"][0][0], np.einsum("hkv,hk->hv", st, f["q"][:, 0])) < 1e-5


def test_neumann_variant_equals_split_to_depth_15_only():
    n = 32
    y, aa, bb, A_log, dtb, S0 = inputs(n)
    # identical keys and beta ~ 1 make A large enough for the truncation to show
    y[:, 2 * D:4 * D] = y[0:1, 2 * D:4 * D]
    bb[:] = 8.0
    aa[:] = -6.0  # g ~ 0: little decay
    for depth_limit, p in ((15, np.array([-1] + [max(i - 1, 0) if i <= 15 else 0 for i in range(1, n)])),
                           (31, np.arange(n) - 1)):
        anc = O.tree_struct(p)[0]
        a = O.tree_gdn_split(y[None], aa[None], bb[None], A_log, dtb, S0[None], anc[None], 2, 4, D, D)
        b = O.tree_gdn_neumann(y[None], aa[None], bb[None], A_log, dtb, S0[None], anc[None], 2, 4, D, D)
        err = rel_l2(b["o"], a["o"])
        if depth_limit == 15:
            assert err < 1e-5
        else:
            assert err > 1e-3


# ---------------------------------------------------------------- conv
def test_conv_chain_zero_state_is_conv1d():
    n, C = 16, 40
    x = O.bf16_round(RNG.standard_normal((n, C)).astype(np.float32))
    w = O.bf16_round(RNG.standard_normal((C, 4)).astype(np.float32) * 0.1)
    bias = RNG.standard_normal(C).astype(np.float32)
    cidx = O.tree_struct(np.arange(n) - 1, 4)[2]
    y, win = O.tree_conv(x, np.zeros((C, 3), np.float32), w, bias, cidx)
    xp = np.concatenate([np.zeros((3, C)), x.astype(np.float64)], 0)
    for c in range(C):
        full = np.convolve(xp[:, c], w[c, ::-1].astype(np.float64), mode="valid")  # causal, zero padding 3
        acc = full + bias[c]
        assert np.allclose(y[:, c], acc / (1 + np.exp(-acc)), rtol=1e-5, atol=1e-6)
    # the window is the last three inputs ending at the node's parent
    assert np.array_equal(win[:, :, 2], x)
    assert np.array_equal(win[1:, :, 1], x[:-1])


def test_conv_reads_old_state_at_the_root():
    C = 8
    cs = RNG.standard_normal((C, 3)).astype(np.float32)
    x = RNG.standard_normal((1, C)).astype(np.float32)
    w = RNG.standard_normal((C, 4)).astype(np.float32)
    y, win = O.tree_conv(x, cs, w, None, np.array([[0, 1, 2, 3]]), silu=False)
    assert np.allclose(y[0], (cs * w[:, :3]).sum(1) + x[0] * w[:, 3], rtol=1e-6)
    assert np.array_equal(win[0], np.concatenate([cs[:, 1:], x.T], 1))


# ---------------------------------------------------------------- commit
def test_closed_commit_equals_replay_and_recurrent_state():
    n = 32
    r, f, (y, aa, bb, A_log, dtb, S0, p, anc) = split(n, "random")
    u = n - 1
    path = sorted(np.nonzero(anc[u])[0], key=lambda j: O.tree_struct(p)[1][j])
    S_closed = O.closed_commit(S0, r["k"][0], r["vn"][0], r["G"][0], path, dtype=np.float64)
    S_replay = O.replay_path_f64(y, aa, bb, A_log, dtb, S0, path, 2, 4, D, D)
    assert rel_l2(S_closed, S_replay) < 1e-5
    assert rel_l2(S_replay, f["states"][:, u]) < 1e-12


def test_snapshot_at_inner_node_uses_ancestors_only():
    n = 32
    r, f, (y, aa, bb, A_log, dtb, S0, p, anc) = split(n, "chain")
    path = list(range(10))
    u = 4
    S_anc = O.closed_commit(S0, r["k"][0], r["vn"][0], r["G"][0], path, u=u, anc=anc, dtype=np.float64)
    assert rel_l2(S_anc, f["states"][:, u]) < 1e-5
    S_all = O.closed_commit(S0, r["k"][0], r["vn"][0], r["G"][0], path, u=u, anc=None, dtype=np.float64)
    assert rel_l2(S_all, f["states"][:, u]) > 1e-3


# ---------------------------------------------------------------- torch restatement (the CPU baseline)
@pytest.mark.parametrize("n,kind", [(16, "random"), (32, "chain"), (32, "random"), (48, "random")])
def test_torch_restatement_matches_oracle(n, kind):
    """oracle.gdn_tree_torch (the batched torch fp32 form bench.py times as
    its CPU baseline) against the numpy oracle, three requests at once: o, vn,
    k and G within 1e-5, and the batched path commit against closed_commit
    of each request's accepted walk."""
    import torch
    from oracle import gdn_tree_torch as T
    rng = np.random.default_rng(77 + n)
    reqs = [inputs(n, rng=rng) + (rand_tree(n, kind, rng),) for _ in range(3)]
    y, aa, bb = (np.stack([r[i] for r in reqs]) for i in range(3))
    A_log, dtb = reqs[0][3], reqs[0][4]
    S0 = np.stack([r[5] for r in reqs])
    anc = np.stack([O.tree_struct(r[6])[0] for r in reqs]).astype(np.float32)
    want = O.tree_gdn_split(y, aa, bb, A_log, dtb, S0, anc, 2, 4, D, D)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
    got = T.tree_gdn_split(t(y), t(aa), t(bb), t(A_log), t(dtb), t(S0), t(anc), 2, 4, D, D)
    for key in ("o", "vn", "k", "G"):
        assert rel_l2(got[key].numpy(), want[key]) < 1e-5, key
    # each request commits the walk from the root to its last node
    paths = [sorted(np.nonzero(anc[b, n - 1])[0]) for b in range(3)]
    on = torch.zeros(3, n)
    for b, pth in enumerate(paths):
        on[b, pth] = 1
    S = T.closed_commit(t(S0), got["k"], got["vn"], got["G"], on, torch.full((3,), n - 1, dtype=torch.long))
    for b in range(3):
        ref = O.closed_commit(S0[b], want["k"][b], want["vn"][b], want["G"][b], paths[b])
        assert rel_l2(S[b].numpy(), ref) < 1e-5
