"""GPU parity of the pipelined schedule in steady state, its walk check and
its flushes (dft_tree_commit_verify).

Steady state: step 0 is a plain verify; every later step is one fused
launch that commits the previous step's accepted walk (keys normalised from
that step's raw bf16 k rows, values recomputed from its raw v rows and b
gates, gains read from the buffer the previous launch wrote while this one
writes the other) and then verifies its own tree on the committed state.
That is the measured launch, run here at its shape (64 requests of 32-node
trees, full width) and at the ragged shape (128 packed requests of 8-64
nodes, both kernel widths, size-order records), four steps and a final
flush.  Every step's o and the pool after every step are checked against
the oracle chain: verify, closed-form commit of the walk
(tree_kernels.py:111-127), next verify on the committed state.

Walk check: with the previous step's ancestry rows a request whose path is
not a walk down from the root (ancestor missing, out of order, a
non-ancestor, a repeat, a path that does not start at the root) commits
nothing and gets DFT_STATUS_WALK, while the others still match the oracle.

Flush: a launch with n_nodes 0, or requests of span 0 in a packed batch,
commits the pending paths and verifies nothing for them.
"""
import numpy as np
import pytest
import torch

from conftest import MAX_ABS_BF16, REL_L2, announce, max_abs, rel_l2
from _ref import np32, oracle_verify, request_slices
from oracle import gdn_tree as O

pytestmark = pytest.mark.gpu

P = 16
WALK = 4  # DFT_STATUS_WALK


def _walks(batch, seed):
    """Accepted root-to-node walks of every request (-1 padded), their
    lengths, and the walks as lists (empty for a request without rows)."""
    from dforktree_amd import synth
    g = torch.Generator().manual_seed(seed)
    idx = torch.full((batch.batch, P), -1, dtype=torch.int32)
    lens = torch.zeros(batch.batch, dtype=torch.int32)
    walks = []
    for r, sl in enumerate(request_slices(batch)):
        w = synth.accepted_path(batch.parent[sl], P, g).tolist() if sl.stop > sl.start else []
        idx[r, :len(w)] = torch.tensor(w, dtype=torch.int32)
        lens[r] = len(w)
        walks.append(w)
    return idx, lens, walks


def _drop_rows(batch, empty):
    """The batch with the requests in ``empty`` cut to zero rows (their
    states kept): packed spans of 0."""
    from dforktree_amd.synth import Batch
    keep = [sl for r, sl in enumerate(request_slices(batch)) if r not in empty]
    cat = lambda t: torch.cat([t[sl] for sl in keep]) if keep else t[:0]
    sizes = [0 if r in empty else n for r, n in enumerate(batch.sizes)]
    cu = torch.zeros(len(sizes) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(sizes, dtype=torch.int32), 0)
    return Batch(y=cat(batch.y), a=cat(batch.a), b=cat(batch.b), A_log=batch.A_log, dt_bias=batch.dt_bias,
                 state=batch.state, parent=cat(batch.parent), cu_seqlens=cu, sizes=sizes, hk=batch.hk, hv=batch.hv)


def _oracle_step(batch, S):
    """The oracle's verify of every request with rows, on states S (K-major)."""
    from dforktree_amd.synth import Batch
    out = [None] * batch.batch
    rows = [r for r in range(batch.batch) if batch.sizes[r] > 0]
    if not rows:
        return out
    sub = _drop_rows(batch, ())
    sub = Batch(y=sub.y, a=sub.a, b=sub.b, A_log=sub.A_log, dt_bias=sub.dt_bias,
                state=torch.stack([torch.from_numpy(np.ascontiguousarray(S[r].transpose(0, 2, 1))) for r in rows]),
                parent=sub.parent, cu_seqlens=torch.tensor([0] + list(np.cumsum([batch.sizes[r] for r in rows])),
                                                           dtype=torch.int32),
                sizes=[batch.sizes[r] for r in rows], hk=batch.hk, hv=batch.hv)
    for r, ref in zip(rows, oracle_verify(sub)):
        out[r] = ref
    return out


class Chain:
    """Runs the pipelined schedule over ``batches`` (one layer): step 0 a
    plain verify, steps 1.. the fused launch on the previous step's walks,
    then (flush=True) one launch with n_nodes 0 that commits the last
    walks.  Keeps every step's o, status words and a snapshot of the pool."""

    def __init__(self, cuda, batches, *, packed, raw=True, ordered=False, walk_rows=False, paths=None,
                 flush=True, row_pad=0):
        from dforktree_amd import ops
        b0 = batches[0]
        hk, hv, B = b0.hk, b0.hv, b0.batch
        self.batches = batches
        self.pool = b0.state.clone().to(cuda)
        st = self.pool.transpose(-1, -2)
        gains = [None, None]
        saves = [None, None]
        self.outs, self.pools, self.status, self.walks = [], [], [], []
        prev = None
        for t, bt in enumerate(batches + ([None] if flush else [])):
            last = bt is None
            if last:  # the flush: every request without rows
                bt = _drop_rows(batches[-1], set(range(B)))
            g = bt.to(cuda)
            rows = g.y.shape[0]
            if row_pad:  # y rows row_pad elements longer: the raw rows are not 16-byte aligned
                C = g.y.shape[1]
                y = torch.zeros(rows, C + row_pad, dtype=g.y.dtype, device=cuda)[:, :C]
                y.copy_(g.y)
                g.y = y
            n_max = max(bt.sizes)
            kw = dict(batch=B, n_nodes=n_max)
            if packed or last:
                kw["cu_seqlens"] = g.cu_seqlens
                if ordered and n_max > 0:
                    kw["size_order"] = ops.size_order(g.cu_seqlens, n_max)
            if rows:
                bits = ops.tree_struct(g.parent, 4, cu_seqlens=g.cu_seqlens, n_nodes=n_max, batch=B,
                                       want=("anc_bits",))["anc_bits"]
            else:
                bits = torch.zeros(1, dtype=torch.int64, device=cuda)
            G = torch.zeros(hv, max(rows, 1), device=cuda)
            k = None if raw else torch.zeros(hk, max(rows, 1), 128, device=cuda)
            v = None if raw else torch.zeros(hv, max(rows, 1), 128, device=cuda)
            gains[t % 2], saves[t % 2] = G, (k, v)
            status = torch.full((B,), -7, dtype=torch.int32, device=cuda)
            common = dict(hk=hk, hv=hv, anc_bits=bits, aux_g=G[:, :rows], status=status, **kw)
            if not raw:
                common.update(aux_k=k[:, :rows], aux_v=v[:, :rows], aux_k_per_khead=True)
            if t == 0:
                o = ops.tree_verify(g.y, g.a, g.b, g.A_log, g.dt_bias, st, **common)
            else:
                pg, pbits, (pidx, plens), pk = prev
                pend = dict(pending_path=pidx.to(cuda), pending_path_len=plens.to(cuda), pending_gains=gains[(t - 1) % 2],
                            prev_cu_seqlens=pg.cu_seqlens, pending_k_head_div=hv // hk)
                if walk_rows:
                    pend["pending_anc_bits"] = pbits
                if raw:
                    pend.update(pending_keys=None, pending_key_rows=pg.y[:, hk * 128:2 * hk * 128].unflatten(1, (hk, 128)),
                                pending_values=None, pending_value_rows=pg.y[:, 2 * hk * 128:].unflatten(1, (hv, 128)),
                                pending_b=pg.b)
                else:
                    pend.update(pending_keys=pk[0], pending_values=pk[1])
                o = ops.tree_commit_verify(g.y, g.a, g.b, g.A_log, g.dt_bias, st, **pend, **common)
            if not last:
                idx, lens, walks = _walks(bt, 100 + t)
                if paths is not None:  # the caller's paths for this step (e.g. non-walks)
                    idx, lens, walks = paths(t, bt, idx, lens, walks)
                self.walks.append(walks)
                prev = (g, bits, (idx, lens), saves[t % 2])
                self.outs.append(o)
            self.pools.append(self.pool.clone())
            self.status.append(status)
        torch.cuda.synchronize()

    def check(self, committed=lambda t, r: True):
        """Every step's o and the pool after every step against the oracle
        chain; committed(t, r) says whether step t's walk of request r is
        committed (False: the slot must keep its state)."""
        B = self.batches[0].batch
        S = [np32(self.batches[0].state[r]).transpose(0, 2, 1) for r in range(B)]
        for t, bt in enumerate(self.batches):
            ref = _oracle_step(bt, S)
            o = np32(self.outs[t])
            for r, sl in enumerate(request_slices(bt)):
                if ref[r] is None:
                    continue
                want = O.bf16_round(ref[r]["o"])
                assert rel_l2(o[sl], want) <= REL_L2 and max_abs(o[sl], want) <= MAX_ABS_BF16, f"step {t} request {r}: o"
            for r in range(B):
                w = self.walks[t][r]
                if ref[r] is not None and w and committed(t, r):
                    S[r] = O.closed_commit(S[r], ref[r]["k"], ref[r]["vn"], ref[r]["G"], w)
            if t + 1 < len(self.pools):
                got = np32(self.pools[t + 1])
                for r in range(B):
                    assert rel_l2(got[r].transpose(0, 2, 1), S[r]) <= REL_L2, f"pool after step {t + 1}, request {r}"


def test_steady_state_bench_shape(cuda):
    """The measured launch in steady state at its shape: 64 requests of
    32-node random trees at full width (16 q/k heads, 32 v heads), raw key
    rows and recomputed values, gains alternating between two buffers, four
    steps and a flush, with the walk check on (every walk passes: status 0)."""
    from dforktree_amd import synth
    announce("steady state: 4 fused steps + flush, 64 x 32 full width")
    batches = [synth.make_batch(200 + t, 0, [32] * 64, hk=16, hv=32, kinds="random") for t in range(4)]
    ch = Chain(cuda, batches, packed=False, walk_rows=True)
    for t, s in enumerate(ch.status):
        assert torch.all(s == 0), f"step {t}: status {s.tolist()}"
    ch.check()


def test_steady_state_ragged_shape(cuda):
    """The ragged shape in steady state: 128 packed requests whose trees of
    8-64 nodes (chains, bushy, random) change size every step, so each step
    runs both kernel widths with size-order records; four steps and a flush."""
    from dforktree_amd import synth
    announce("steady state: 4 fused steps + flush, ragged 128 x 8-64 full width")
    batches = []
    for t in range(4):
        sizes, kinds = synth.ragged_sizes(128, 8, 64, seed=210 + t)
        batches.append(synth.make_batch(220 + t, 0, sizes, hk=16, hv=32, kinds=kinds))
    ch = Chain(cuda, batches, packed=True, ordered=True, walk_rows=True)
    for t, s in enumerate(ch.status):
        assert torch.all(s == 0), f"step {t}: status {s.tolist()}"
    ch.check()


@pytest.mark.parametrize("raw", [True, False])
def test_steady_state_saved_and_raw_forms_agree(cuda, raw):
    """Four steps and a flush at reduced width (2 q/k heads, 4 v heads) with
    packed trees on both sides of 32 nodes: the raw-row form and the
    saved-key/value form each match the oracle chain."""
    from dforktree_amd import synth
    announce(f"steady state small, raw={raw}")
    kinds = ["random", "chain", "bushy", "random", "chain", "bushy", "random", "random"]
    sz = [[40, 9, 64, 17, 33, 1, 50, 20], [12, 64, 30, 1, 50, 20, 33, 64], [5, 33, 64, 32, 16, 48, 2, 31],
          [64, 64, 8, 40, 32, 1, 17, 60]]
    batches = [synth.make_batch(230 + t, 0, sz[t], hk=2, hv=4, kinds=kinds) for t in range(4)]
    ch = Chain(cuda, batches, packed=True, raw=raw, ordered=True)
    ch.check()


def _non_walks(t, bt, idx, lens, walks):
    """Step 1's paths: request r gets a broken walk of kind r % 8 (0 and 6
    stay valid: a plain walk, and a walk with an unused -1 entry inside)."""
    if t != 1:
        return idx, lens, walks
    idx = torch.full_like(idx, -1)
    par = bt.parent
    out_w = []
    for r, sl in enumerate(request_slices(bt)):
        p = par[sl].tolist()
        n = len(p)
        depth = [0] * n
        for i in range(1, n):
            depth[i] = depth[p[i]] + 1
        u = max(range(n), key=lambda i: depth[i])  # the deepest node (depth >= 2 in these trees)
        w = [u]
        while p[w[-1]] >= 0:
            w.append(p[w[-1]])
        w = w[::-1][:6]  # its walk from the root, at most 6 entries
        kind = r % 8
        entries = list(w)
        if kind == 1 and len(w) >= 3:      # an ancestor missing
            entries = w[:1] + w[2:]
        elif kind == 2:                    # a non-ancestor appended
            x = next(i for i in range(1, n) if p[i] != w[-1] and i not in w)
            entries = w + [x]
        elif kind == 3:                    # a repeat
            entries = w + [w[-1]]
        elif kind == 4 and len(w) >= 3:    # out of order
            entries = [w[0], w[2], w[1]] + w[3:]
        elif kind == 5 and len(w) >= 2:    # not from the root
            entries = w[1:]
        elif kind == 6:                    # a walk with an unused entry inside: valid
            entries = w[:1] + [-1] + w[1:]
        elif kind == 7:                    # nothing pending
            entries = []
        idx[r, :len(entries)] = torch.tensor(entries, dtype=torch.int32)
        lens[r] = len(entries)
        out_w.append([e for e in entries if e >= 0])
    return idx, lens, out_w


BAD = {1, 2, 3, 4, 5}


@pytest.mark.parametrize("form", ["raw32", "raw32_unaligned", "saved32", "raw64", "saved64"])
def test_walk_check_drops_non_walks(cuda, form):
    """With the previous step's ancestry rows, requests whose pending path
    is not a walk down from the root commit nothing and get
    DFT_STATUS_WALK; every other request commits and matches the oracle
    chain.  Covers the 32-wide forms (raw rows copied ahead of the tile,
    raw rows in registers, saved keys and values) and the 64-wide ones."""
    from dforktree_amd import synth
    announce(f"walk check, form {form}")
    wide = form.endswith("64")
    n = 48 if wide else 32
    kinds = ["random", "bushy"] * 8
    batches = [synth.make_batch(240 + t + (10 if wide else 0), 0, [n] * 16, hk=2, hv=4, kinds=kinds)
               for t in range(3)]
    # raw32_unaligned: raw rows whose stride is not a multiple of 16 bytes take the register form
    ch = Chain(cuda, batches, packed=wide, raw=form.startswith("raw"), walk_rows=True, paths=_non_walks,
               row_pad=4 if form == "raw32_unaligned" else 0)
    st = ch.status[2].tolist()  # the launch that commits step 1's paths
    for r in range(16):
        want = WALK if (r % 8) in BAD else 0
        assert st[r] == want, f"request {r} (kind {r % 8}): status {st[r]}, want {want}"
    for s in (ch.status[1], ch.status[3]):
        assert torch.all(s == 0)
    ch.check(committed=lambda t, r: not (t == 1 and (r % 8) in BAD))


def test_walk_check_off_reports_nothing(cuda):
    """Without the ancestry rows there is no walk check: the same non-walks
    leave every status word 0 (the paths are committed as given)."""
    from dforktree_amd import synth
    announce("walk check off")
    batches = [synth.make_batch(260 + t, 0, [32] * 16, hk=2, hv=4, kinds="random") for t in range(2)]
    ch = Chain(cuda, batches + [synth.make_batch(262, 0, [32] * 16, hk=2, hv=4)], packed=False,
               paths=_non_walks)
    assert all(torch.all(s == 0) for s in ch.status)


@pytest.mark.parametrize("raw", [True, False])
def test_flush_with_empty_requests(cuda, raw):
    """A packed step in which some requests have no rows (span 0) beside
    trees on both sides of 32 nodes: those requests only commit their
    pending paths; the others commit and verify; a later step and the final
    n_nodes = 0 flush follow.  Against the oracle chain."""
    from dforktree_amd import synth
    announce(f"flush: empty requests in a packed step, raw={raw}")
    kinds = ["random", "chain", "bushy", "random"] * 2
    b0 = synth.make_batch(270, 0, [40, 9, 64, 17, 33, 12, 50, 20], hk=2, hv=4, kinds=kinds)
    b1 = _drop_rows(synth.make_batch(271, 0, [12, 64, 30, 5, 50, 20, 33, 64], hk=2, hv=4, kinds=kinds), {1, 3, 6})
    b2 = synth.make_batch(272, 0, [20, 33, 8, 64, 31, 2, 45, 16], hk=2, hv=4, kinds=kinds)
    for ordered in (False, True):
        ch = Chain(cuda, [b0, b1, b2], packed=True, raw=raw, ordered=ordered, walk_rows=True)
        assert all(torch.all(s == 0) for s in ch.status)
        ch.check()


@pytest.mark.parametrize("raw", [True, False])
def test_flush_uniform_batch_n_nodes_zero(cuda, raw):
    """A uniform 32-node step followed directly by the n_nodes = 0 flush:
    every slot holds its committed state, and a request without a path keeps
    its slot bit for bit."""
    from dforktree_amd import synth
    announce(f"flush: n_nodes 0 after a uniform step, raw={raw}")
    b0 = synth.make_batch(280, 0, [32] * 6, hk=2, hv=4, kinds=["random", "chain", "bushy"] * 2)

    def paths(t, bt, idx, lens, walks):
        idx[2], lens[2], walks[2] = -1, 0, []
        return idx, lens, walks

    ch = Chain(cuda, [b0], packed=False, raw=raw, paths=paths)
    assert torch.all(ch.status[1] == 0)
    assert torch.equal(ch.pools[1][2], ch.pools[0][2])
    ch.check()


def test_size_order_records_of_another_launch_are_ignored(cuda):
    """Records whose header names another n_nodes take no effect on the
    device (the launch runs as without them); the Python layer refuses
    records written for other n_nodes or from a changed cu_seqlens."""
    from dforktree_amd import ops, synth
    announce("size-order header check")
    b = synth.make_batch(290, 0, [40, 9, 48, 17, 33, 1], hk=2, hv=4)
    g = b.to(cuda)
    bits = ops.tree_struct(g.parent, 4, cu_seqlens=g.cu_seqlens, n_nodes=48, batch=6, want=("anc_bits",))["anc_bits"]
    common = dict(hk=2, hv=4, anc_bits=bits, cu_seqlens=g.cu_seqlens, batch=6)
    rec64 = ops.size_order(g.cu_seqlens, 64)
    with pytest.raises(ValueError, match="n_nodes=64"):
        ops.tree_verify(g.y, g.a, g.b, g.A_log, g.dt_bias, g.state.transpose(-1, -2), n_nodes=48,
                        size_order=rec64, **common)
    cu2 = g.cu_seqlens.clone()
    rec48 = ops.size_order(cu2, 48)
    cu2.add_(0)  # changed in place (same values): the records are stale by the version counter
    with pytest.raises(ValueError, match="another cu_seqlens"):
        ops.tree_verify(g.y, g.a, g.b, g.A_log, g.dt_bias, g.state.transpose(-1, -2), n_nodes=48,
                        size_order=rec48, **{**common, "cu_seqlens": cu2})
    # a copy of the n_nodes = 64 records is unknown to the Python layer: the device ignores its header
    o_ref = ops.tree_verify(g.y, g.a, g.b, g.A_log, g.dt_bias, g.state.transpose(-1, -2), n_nodes=48, **common)
    o_rec = ops.tree_verify(g.y, g.a, g.b, g.A_log, g.dt_bias, g.state.transpose(-1, -2), n_nodes=48,
                            size_order=rec64.clone(), **common)
    torch.cuda.synchronize()
    assert torch.equal(o_ref.view(torch.int16), o_rec.view(torch.int16))
