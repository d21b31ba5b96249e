"""The per-request status words of the verify and commit entry points.

A packed request whose row span exceeds the launch's n_nodes is cut to its
first n_nodes rows (a valid tree: parents precede children), flagged with
DFT_STATUS_SPAN, and leaves the rows past the cut unwritten; every other
request of the launch still matches the oracle and reports 0.  A path entry
or commit end at or past its tree's size is ignored and flagged with
DFT_STATUS_PATH.  Tolerances as in the other parity tests (rel-L2 2e-3,
max-abs 1e-2 on bf16 outputs; indices and status words exact).
"""
import numpy as np
import pytest
import torch

from conftest import MAX_ABS_BF16, REL_L2, announce, max_abs, rel_l2
from _ref import np32, oracle_verify, request_slices
from oracle import gdn_tree as O

pytestmark = pytest.mark.gpu

SPAN, PATH = 1, 2
SENTINEL = 7.0


def _prefix_batch(batch, r, n):
    """The same batch with request r cut to its first n nodes (CPU)."""
    from dforktree_amd import synth
    sl = request_slices(batch)[r]
    keep = torch.ones(batch.y.shape[0], dtype=torch.bool)
    keep[sl.start + n:sl.stop] = False
    sizes = list(batch.sizes)
    sizes[r] = n
    cu = torch.zeros(len(sizes) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(sizes, dtype=torch.int32), 0)
    return synth.Batch(y=batch.y[keep], a=batch.a[keep], b=batch.b[keep], A_log=batch.A_log, dt_bias=batch.dt_bias,
                       state=batch.state, parent=batch.parent[keep], cu_seqlens=cu, sizes=sizes, hk=batch.hk,
                       hv=batch.hv)


@pytest.mark.parametrize("sizes,n_nodes,long", [([20, 40, 12, 32], 32, 1), ([20, 60, 40, 8], 48, 1),
                                                ([64, 9, 33], 40, 0)])
def test_verify_reports_a_request_past_n_nodes(cuda, sizes, n_nodes, long):
    from dforktree_amd import ops, synth
    announce(f"verify status: sizes={sizes} n_nodes={n_nodes}")
    kinds = ["random", "chain", "bushy", "random"][:len(sizes)]
    batch = synth.make_batch(41, 0, sizes, hk=2, hv=4, kinds=kinds)
    g = batch.to(cuda)
    rows = g.y.shape[0]
    ts = ops.tree_struct(g.parent, 4, cu_seqlens=g.cu_seqlens, n_nodes=max(sizes), batch=batch.batch,
                         want=("anc_bits",))
    o = torch.full((rows, batch.hv, 128), SENTINEL, device=cuda, dtype=torch.bfloat16)
    aux_v = torch.full((batch.hv, rows, 128), SENTINEL, device=cuda)
    status = torch.full((batch.batch,), -5, device=cuda, dtype=torch.int32)
    ops.tree_verify(g.y, g.a, g.b, g.A_log, g.dt_bias, g.state.transpose(-1, -2), hk=batch.hk, hv=batch.hv,
                    anc_bits=ts["anc_bits"], cu_seqlens=g.cu_seqlens, n_nodes=n_nodes, batch=batch.batch, o=o,
                    aux_v=aux_v, status=status)
    torch.cuda.synchronize()
    assert status.tolist() == [SPAN if r == long else 0 for r in range(batch.batch)]
    ref = oracle_verify(_prefix_batch(batch, long, n_nodes))
    oh, vh = np32(o), np32(aux_v)
    for r, sl in enumerate(request_slices(batch)):
        n = min(sizes[r], n_nodes)
        kept = slice(sl.start, sl.start + n)
        want = O.bf16_round(ref[r]["o"])
        assert rel_l2(oh[kept], want) <= REL_L2 and max_abs(oh[kept], want) <= MAX_ABS_BF16, f"request {r}: o"
        assert rel_l2(vh[:, kept], ref[r]["vn"]) <= REL_L2, f"request {r}: vn"
        if sizes[r] > n:  # the rows past the cut are left alone
            assert np.all(oh[sl.start + n:sl.stop] == SENTINEL) and np.all(vh[:, sl.start + n:sl.stop] == SENTINEL)


def test_status_is_optional_and_uniform_batches_report_zero(cuda):
    from dforktree_amd import ops, synth
    announce("verify status: uniform batch")
    batch = synth.make_batch(42, 0, [32] * 3, hk=2, hv=4)
    g = batch.to(cuda)
    ts = ops.tree_struct(g.parent, 4, batch=3, n_nodes=32, want=("anc_bits",))
    status = torch.full((3,), 9, device=cuda, dtype=torch.int32)
    kw = dict(hk=2, hv=4, anc_bits=ts["anc_bits"], batch=3, n_nodes=32)
    o1 = ops.tree_verify(g.y, g.a, g.b, g.A_log, g.dt_bias, g.state.transpose(-1, -2), status=status, **kw)
    o2 = ops.tree_verify(g.y, g.a, g.b, g.A_log, g.dt_bias, g.state.transpose(-1, -2), **kw)
    torch.cuda.synchronize()
    assert status.tolist() == [0, 0, 0] and torch.equal(o1, o2)


@pytest.mark.parametrize("raw", [False, True])
def test_commit_verify_reports_a_path_entry_past_the_tree(cuda, raw):
    """The fused entry: request 1's pending path names node 40 of a 32-node
    tree (ignored: the commit equals the one without it), request 2's next
    tree is longer than n_nodes.  raw: the commit reads step 1's raw k and v
    rows and recomputes the values (the kernel that copies the path's rows
    into LDS ahead of the state tile)."""
    from dforktree_amd import ops, synth
    announce("commit->verify status")
    hk, hv, B = 2, 4, 4
    b1 = synth.make_batch(43, 0, [32] * B, hk=hk, hv=hv, kinds=["random", "chain", "bushy", "random"])
    b2 = synth.make_batch(44, 0, [32, 32, 40, 32], hk=hk, hv=hv, kinds=["random", "chain", "bushy", "random"])
    pool = b1.state.clone().to(cuda)
    st = pool.transpose(-1, -2)
    g1, g2 = b1.to(cuda), b2.to(cuda)
    r1, r2 = g1.y.shape[0], g2.y.shape[0]
    k1, v1, G1 = (torch.zeros(hv, r1, 128, device=cuda), torch.zeros(hv, r1, 128, device=cuda),
                  torch.zeros(hv, r1, device=cuda))
    ts1 = ops.tree_struct(g1.parent, 4, batch=B, n_nodes=32, want=("anc_bits",))
    ops.tree_verify(g1.y, g1.a, g1.b, g1.A_log, g1.dt_bias, st, hk=hk, hv=hv, anc_bits=ts1["anc_bits"], batch=B,
                    n_nodes=32, aux_k=k1, aux_v=v1, aux_g=G1)
    gen = torch.Generator().manual_seed(45)
    idx = torch.full((B, 16), -1, dtype=torch.int32)
    walks = []
    for r, sl in enumerate(request_slices(b1)):
        w = synth.accepted_path(b1.parent[sl], 12, gen)
        idx[r, :len(w)] = w
        walks.append(w.tolist())
    idx[1, len(walks[1])] = 40  # past the 32-node tree: ignored, flagged
    ts2 = ops.tree_struct(g2.parent, 4, cu_seqlens=g2.cu_seqlens, n_nodes=40, batch=B, want=("anc_bits",))
    status = torch.full((B,), -5, device=cuda, dtype=torch.int32)
    if raw:
        rows = dict(pending_keys=None, pending_key_rows=g1.y[:, hk * 128:2 * hk * 128].unflatten(1, (hk, 128)),
                    pending_k_head_div=hv // hk, pending_values=None,
                    pending_value_rows=g1.y[:, 2 * hk * 128:].unflatten(1, (hv, 128)), pending_b=g1.b)
    else:
        rows = dict(pending_keys=k1, pending_values=v1)
    ops.tree_commit_verify(g2.y, g2.a, g2.b, g2.A_log, g2.dt_bias, st, hk=hk, hv=hv, anc_bits=ts2["anc_bits"],
                           cu_seqlens=g2.cu_seqlens, n_nodes=32, batch=B, pending_path=idx.to(cuda),
                           pending_gains=G1, prev_n_nodes=32, status=status, **rows)
    torch.cuda.synchronize()
    assert status.tolist() == [0, PATH, SPAN, 0]
    ref1 = oracle_verify(b1)
    got = np32(pool)
    for r in range(B):
        want = O.closed_commit(np32(b1.state[r]).transpose(0, 2, 1), ref1[r]["k"], ref1[r]["vn"], ref1[r]["G"],
                               walks[r])
        assert rel_l2(got[r].transpose(0, 2, 1), want) <= REL_L2, f"request {r}: committed state"


def test_commit_reports_spans_entries_and_ends(cuda):
    """dft_tree_commit: a packed request longer than n_nodes (SPAN), a path
    entry past the tree (PATH, ignored) and an end past the tree (PATH,
    nothing committed for it)."""
    from dforktree_amd import ops, synth
    announce("commit status")
    H, B, N = 4, 4, 32
    sizes = [32, 32, 36, 32]
    cu = torch.zeros(B + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(sizes), 0)
    rows = int(cu[-1])
    g = torch.Generator().manual_seed(46)
    S = (torch.randn(1, B, H, 128, 128, generator=g) * 0.02).to(cuda)
    keys = (torch.randn(1, H, rows, 128, generator=g) * 128 ** -0.5).to(cuda)
    vals = (torch.randn(1, H, rows, 128, generator=g) * 0.3).to(cuda)
    gains = (-torch.rand(1, H, rows, generator=g)).to(cuda)
    pars = [synth.tree_parents(n, "random", g) for n in sizes]
    idx = torch.full((B, 8), -1, dtype=torch.int32)
    walks = []
    for r in range(B):
        w = synth.accepted_path(pars[r][:N], 6, g)
        idx[r, :len(w)] = w
        walks.append(w.tolist())
    idx[1, 7] = N + 3          # an entry past the tree: ignored
    ends = torch.tensor([[walks[0][-1]], [walks[1][-1]], [walks[2][-1]], [N]], dtype=torch.int32)  # request 3: past
    dst = torch.zeros(1, B, N, H, 128, 128, device=cuda)
    status = torch.full((B,), -5, device=cuda, dtype=torch.int32)
    ops.tree_commit(S, keys, vals, gains, idx.to(cuda), n_nodes=N, ends=ends.to(cuda), cu_seqlens=cu.to(cuda), dst=dst,
                    status=status)
    torch.cuda.synchronize()
    assert status.tolist() == [0, PATH, SPAN, PATH]
    got = np32(dst)
    for r in range(B):
        sl = slice(int(cu[r]), int(cu[r]) + N)
        if r == 3:
            assert not got[0, 3].any(), "an end past the tree commits nothing"
            continue
        u = walks[r][-1]
        # the pool layout holds S as [H, V, K]; the closed form is written over [H, K, V]
        want = O.closed_commit(np32(S[0, r]).transpose(0, 2, 1), np32(keys[0, :, sl]), np32(vals[0, :, sl]),
                               np32(gains[0, :, sl]), walks[r])
        assert rel_l2(got[0, r, u].transpose(0, 2, 1), want) <= 1e-5, f"request {r}"
