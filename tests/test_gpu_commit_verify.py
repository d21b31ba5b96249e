"""GPU parity of the fused commit -> verify entry point (dft_tree_commit_verify).

Step 1 verifies a batch of trees and saves k, vn, G; step 2 verifies new
trees through the fused entry, which first commits step 1's accepted paths
into each request's state slot.  Checked against the oracle chain
(closed-form commit of step 1, then the step-2 verify on the committed
state): node outputs within rel-L2 2e-3 (max-abs 1e-2 on bf16), committed
states within rel-L2 2e-3, a request without a valid path entry keeps its
slot bit for bit.  A second test checks that the fused entry equals the
separate in-place commit followed by the plain verify to fp32 rounding.
The raw-key form (the commit normalises step 1's bf16 k rows itself, and
step 1 saves no keys) is checked against the same oracle chain, and
against the saved-key form within rel-L2 1e-6 on the committed states.
So is the recomputed-value form (the commit recomputes the path's values
from step 1's raw bf16 v rows, b gates and the slot's state, and step 1
saves no values), and against the saved-value form within rel-L2 1e-5 on
the committed states (a different solve: fp32 products against the
verify's split-bf16 block inverse).
"""
import numpy as np
import pytest
import torch

from conftest import MAX_ABS_BF16, REL_L2, announce, max_abs, rel_l2
from _ref import np32, oracle_verify, request_slices
from oracle import gdn_tree as O

pytestmark = pytest.mark.gpu

P = 16


def _paths(batch, seed, empty=(), shorten=()):
    """Accepted root-to-node walks of every request, -1 padded to 16 columns;
    requests in ``empty`` get no entry, those in ``shorten`` a path_len one
    short of their walk."""
    from dforktree_amd import synth
    g = torch.Generator().manual_seed(seed)
    idx = torch.full((batch.batch, P), -1, dtype=torch.int32)
    lens = torch.zeros(batch.batch, dtype=torch.int32)
    walks = []
    for r, sl in enumerate(request_slices(batch)):
        w = synth.accepted_path(batch.parent[sl], P, g)
        if r in empty:
            w = w[:0]
        idx[r, :len(w)] = w
        lens[r] = len(w) - (1 if r in shorten and len(w) > 1 else 0)
        walks.append(w[:int(lens[r])].tolist())
    return idx, lens, walks


def _committed_states(batch1, walks):
    """Oracle: each request's state after committing its step-1 walk (k, v)."""
    ref = oracle_verify(batch1)
    out = []
    for r in range(batch1.batch):
        S0 = np32(batch1.state[r]).transpose(0, 2, 1)
        if walks[r]:
            out.append(O.closed_commit(S0, ref[r]["k"], ref[r]["vn"], ref[r]["G"], walks[r]))
        else:
            out.append(S0.copy())
    return out


def _run_chain(cuda, batch1, batch2, per_khead, packed, empty=(), shorten=(), path_dtype=torch.int32,
               raw_keys=False, raw_values=False, ordered=False, row_pad=0):
    """Step 1 verifies batch1 (saving k, vn, G); step 2 verifies batch2
    through the fused entry, committing step 1's walks first.  raw_keys: step
    1 saves no keys, and the commit reads step 1's raw bf16 k rows from its y.
    raw_values: step 1 saves no values, and the commit recomputes them from
    step 1's raw bf16 v rows (from its y) and b gates.  ordered: step 2's
    fused launch reads size-order records of its packed batch.  row_pad: the
    raw rows come from a copy of step 1's y whose rows are row_pad elements
    longer (not 16-byte multiples for row_pad = 4)."""
    from dforktree_amd import ops
    hk, hv, B = batch1.hk, batch1.hv, batch1.batch
    pool = batch1.state.clone().to(cuda)  # [B, hv, V, K]
    st = pool.transpose(-1, -2)
    g1, g2 = batch1.to(cuda), batch2.to(cuda)
    rows1, rows2 = g1.y.shape[0], g2.y.shape[0]
    kh = hk if per_khead else hv
    k1 = torch.zeros(kh, rows1, 128, device=cuda)
    v1 = torch.zeros(hv, rows1, 128, device=cuda)
    G1 = torch.zeros(hv, rows1, device=cuda)
    k2 = torch.zeros(kh, rows2, 128, device=cuda)
    v2 = torch.zeros(hv, rows2, 128, device=cuda)
    G2 = torch.zeros(hv, rows2, device=cuda)
    kw1 = dict(batch=B, n_nodes=batch1.n_max)
    kw2 = dict(batch=B, n_nodes=batch2.n_max)
    if packed:
        kw1["cu_seqlens"], kw2["cu_seqlens"] = g1.cu_seqlens, g2.cu_seqlens
        if ordered:
            kw2["size_order"] = ops.size_order(g2.cu_seqlens, batch2.n_max)
    ts1 = ops.tree_struct(g1.parent, 4, cu_seqlens=g1.cu_seqlens, n_nodes=batch1.n_max, batch=B, want=("anc_bits",))
    ts2 = ops.tree_struct(g2.parent, 4, cu_seqlens=g2.cu_seqlens, n_nodes=batch2.n_max, batch=B, want=("anc_bits",))
    ops.tree_verify(g1.y, g1.a, g1.b, g1.A_log, g1.dt_bias, st, hk=hk, hv=hv, anc_bits=ts1["anc_bits"],
                    aux_k=None if raw_keys else k1, aux_v=None if raw_values else v1, aux_g=G1,
                    aux_k_per_khead=per_khead, **kw1)
    idx, lens, walks = _paths(batch1, 5, empty, shorten)
    prev = dict(prev_cu_seqlens=g1.cu_seqlens) if packed else dict(prev_n_nodes=batch1.n_max)
    y1 = g1.y
    if row_pad:
        y1 = torch.empty(rows1, y1.shape[1] + row_pad, dtype=y1.dtype, device=cuda)[:, :y1.shape[1]]
        y1.copy_(g1.y)
    if raw_keys:  # the k part of step 1's y, [rows, hk, 128]
        keys = dict(pending_keys=None, pending_key_rows=y1[:, hk * 128:2 * hk * 128].unflatten(1, (hk, 128)),
                    pending_k_head_div=hv // hk)
    else:
        keys = dict(pending_keys=k1, pending_k_head_div=hv // kh)
    if raw_values:  # the v part of step 1's y, [rows, hv, 128], and its b gates
        keys.update(pending_values=None, pending_value_rows=y1[:, 2 * hk * 128:].unflatten(1, (hv, 128)),
                    pending_b=g1.b)
    else:
        keys.update(pending_values=v1)
    o2 = ops.tree_commit_verify(g2.y, g2.a, g2.b, g2.A_log, g2.dt_bias, st, hk=hk, hv=hv,
                                anc_bits=ts2["anc_bits"], pending_path=idx.to(path_dtype).to(cuda),
                                pending_gains=G1, pending_path_len=lens.to(cuda), **keys,
                                aux_k=k2, aux_v=v2, aux_g=G2, aux_k_per_khead=per_khead, **prev, **kw2)
    torch.cuda.synchronize()
    return pool, o2, (k2, v2, G2), walks


def _check_chain(batch1, batch2, pool, o2, aux2, walks, empty, per_khead):
    S1 = _committed_states(batch1, walks)
    got = np32(pool)
    for r in range(batch1.batch):
        if r in empty:
            assert np.array_equal(got[r], np32(batch1.state[r])), f"request {r}: slot touched without a path"
        else:
            assert rel_l2(got[r].transpose(0, 2, 1), S1[r]) <= REL_L2, f"request {r}: committed state"
    b2 = batch2.to("cpu")
    b2.state = torch.stack([torch.from_numpy(np.ascontiguousarray(s.transpose(0, 2, 1))) for s in S1])
    ref = oracle_verify(b2)
    o = np32(o2)
    k2, v2, G2 = (np32(t) for t in aux2)
    R = batch2.hv // batch2.hk
    for r, sl in enumerate(request_slices(b2)):
        want = O.bf16_round(ref[r]["o"])
        assert rel_l2(o[sl], want) <= REL_L2 and max_abs(o[sl], want) <= MAX_ABS_BF16, f"request {r}: o"
        assert rel_l2(v2[:, sl], ref[r]["vn"]) <= REL_L2, f"request {r}: vn"
        kref = ref[r]["k"][::R] if per_khead else ref[r]["k"]
        assert rel_l2(k2[:, sl], kref) <= 1e-5
        assert rel_l2(G2[:, sl], ref[r]["G"]) <= 1e-5


def test_commit_verify_uniform_chain(cuda):
    from dforktree_amd import synth
    announce("commit->verify uniform 32")
    kinds = ["random", "chain", "bushy", "random", "chain", "bushy"]
    batch1 = synth.make_batch(20, 0, [32] * 6, hk=2, hv=4, kinds=kinds)
    batch2 = synth.make_batch(21, 0, [32] * 6, hk=2, hv=4, kinds=kinds[::-1])
    empty, shorten = (2,), (4,)
    pool, o2, aux2, walks = _run_chain(cuda, batch1, batch2, per_khead=False, packed=False, empty=empty,
                                       shorten=shorten)
    _check_chain(batch1, batch2, pool, o2, aux2, walks, empty, per_khead=False)


@pytest.mark.parametrize("path_dtype", [torch.int32, torch.int64])
def test_commit_verify_packed_ragged_per_khead(cuda, path_dtype):
    """Packed rows of different sizes in the two steps (the 64-wide kernel),
    keys saved once per k-head, int32 and int64 paths."""
    from dforktree_amd import synth
    announce(f"commit->verify packed ragged {path_dtype}")
    sizes1, kinds = [40, 9, 64, 17, 33, 1], ["random", "chain", "bushy", "random", "chain", "bushy"]
    sizes2 = [12, 64, 30, 1, 50, 20]
    batch1 = synth.make_batch(22, 0, sizes1, hk=2, hv=4, kinds=kinds)
    batch2 = synth.make_batch(23, 0, sizes2, hk=2, hv=4, kinds=kinds)
    empty = (3,)
    pool, o2, aux2, walks = _run_chain(cuda, batch1, batch2, per_khead=True, packed=True, empty=empty,
                                       path_dtype=path_dtype)
    _check_chain(batch1, batch2, pool, o2, aux2, walks, empty, per_khead=True)


def test_commit_verify_size_order(cuda):
    """Packed trees on both sides of 32 nodes in both steps, recomputed
    values and raw keys: the fused launch reading size-order records commits
    and verifies bit for bit as the launch without them."""
    from dforktree_amd import synth
    announce("commit->verify with size-order records")
    sizes1, kinds = [40, 9, 64, 17, 33, 1, 50, 20], ["random", "chain", "bushy", "random"] * 2
    sizes2 = [12, 64, 30, 1, 50, 20, 33, 64]
    batch1 = synth.make_batch(52, 0, sizes1, hk=2, hv=4, kinds=kinds)
    batch2 = synth.make_batch(53, 0, sizes2, hk=2, hv=4, kinds=kinds)
    runs = [_run_chain(cuda, batch1, batch2, per_khead=True, packed=True, empty=(3,), shorten=(6,), raw_keys=True,
                       raw_values=True, ordered=ordered) for ordered in (False, True)]
    (pa, oa, auxa, walks), (pb, ob, auxb, _) = runs
    assert torch.equal(pa, pb) and torch.equal(oa.view(torch.int16), ob.view(torch.int16))
    for x, z in zip(auxa, auxb):
        assert torch.equal(x, z)
    _check_chain(batch1, batch2, pb, ob, auxb, walks, (3,), per_khead=True)


def test_commit_verify_bench_shape(cuda):
    """The measured shape: 64 requests of 32-node random trees at full width
    (2048 items, two generations of resident workgroups, so freed slots take
    further items), keys saved per k-head; one request without a path and
    one with a shortened path_len."""
    from dforktree_amd import synth
    announce("commit->verify bench shape 64 x 32")
    batch1 = synth.make_batch(40, 0, [32] * 64, hk=16, hv=32, kinds="random")
    batch2 = synth.make_batch(41, 0, [32] * 64, hk=16, hv=32, kinds="random")
    empty, shorten = (5,), (60,)
    pool, o2, aux2, walks = _run_chain(cuda, batch1, batch2, per_khead=True, packed=False, empty=empty,
                                       shorten=shorten)
    _check_chain(batch1, batch2, pool, o2, aux2, walks, empty, per_khead=True)


def test_commit_verify_ragged_bench_shape(cuda):
    """The ragged batch at full size in both steps: 128 packed requests with
    trees of 8-64 nodes at full width (both kernel sizes), a different tree
    size per request in the second step, keys saved per k-head; one request
    without a path and one with a shortened path_len."""
    from dforktree_amd import synth
    announce("commit->verify ragged bench shape 128 x 8-64")
    sizes1, kinds1 = synth.ragged_sizes(128, 8, 64, seed=3)
    sizes2, kinds2 = synth.ragged_sizes(128, 8, 64, seed=4)
    batch1 = synth.make_batch(42, 0, sizes1, hk=16, hv=32, kinds=kinds1)
    batch2 = synth.make_batch(43, 0, sizes2, hk=16, hv=32, kinds=kinds2)
    empty, shorten = (7,), (100,)
    pool, o2, aux2, walks = _run_chain(cuda, batch1, batch2, per_khead=True, packed=True, empty=empty,
                                       shorten=shorten)
    _check_chain(batch1, batch2, pool, o2, aux2, walks, empty, per_khead=True)


@pytest.mark.parametrize("sizes1,sizes2,packed", [([32] * 6, [32] * 6, False),
                                                   ([40, 9, 64, 17, 33, 1], [12, 64, 30, 1, 50, 20], True)])
def test_commit_verify_raw_key_rows(cuda, sizes1, sizes2, packed):
    """The commit reads the previous step's raw bf16 k rows (from its y) and
    normalises them itself; the step-1 verify saves no keys.  Against the
    oracle chain, and against the same chain through saved keys (the two
    normalise in a different order: committed states within 1e-6)."""
    from dforktree_amd import synth
    announce(f"commit->verify raw key rows packed={packed}")
    kinds = ["random", "chain", "bushy", "random", "chain", "bushy"]
    batch1 = synth.make_batch(24, 0, sizes1, hk=2, hv=4, kinds=kinds)
    batch2 = synth.make_batch(25, 0, sizes2, hk=2, hv=4, kinds=kinds[::-1])
    empty, shorten = (3,), (1,)
    pool, o2, aux2, walks = _run_chain(cuda, batch1, batch2, per_khead=True, packed=packed, empty=empty,
                                       shorten=shorten, raw_keys=True)
    _check_chain(batch1, batch2, pool, o2, aux2, walks, empty, per_khead=True)
    pool_s, o2_s, _, _ = _run_chain(cuda, batch1, batch2, per_khead=True, packed=packed, empty=empty,
                                    shorten=shorten)
    assert rel_l2(np32(pool), np32(pool_s)) <= 1e-6
    assert rel_l2(np32(o2), np32(o2_s)) <= 1e-5


def test_commit_verify_raw_key_rows_bench_shape(cuda):
    """The measured shape with raw key rows: 64 requests of 32-node trees at
    full width, the keys read from step 1's y."""
    from dforktree_amd import synth
    announce("commit->verify raw key rows, bench shape 64 x 32")
    batch1 = synth.make_batch(44, 0, [32] * 64, hk=16, hv=32, kinds="random")
    batch2 = synth.make_batch(45, 0, [32] * 64, hk=16, hv=32, kinds="random")
    empty, shorten = (9,), (33,)
    pool, o2, aux2, walks = _run_chain(cuda, batch1, batch2, per_khead=True, packed=False, empty=empty,
                                       shorten=shorten, raw_keys=True)
    _check_chain(batch1, batch2, pool, o2, aux2, walks, empty, per_khead=True)


@pytest.mark.parametrize("sizes1,sizes2,packed,b_dtype", [
    ([32] * 6, [32] * 6, False, torch.float32),
    ([32] * 6, [32] * 6, False, torch.bfloat16),
    ([40, 9, 64, 17, 33, 1], [12, 64, 30, 1, 50, 20], True, torch.float16)])
def test_commit_verify_recomputed_values(cuda, sizes1, sizes2, packed, b_dtype):
    """The commit recomputes the path's values from the previous step's raw
    bf16 v rows, b gates (fp32, bf16 or fp16, as the verify reads them) and
    the slot's state (both widths; with raw key rows too); the step-1 verify
    saves no values.  Against the oracle chain, and against the same chain
    through saved values."""
    from dforktree_amd import synth
    announce(f"commit->verify recomputed values packed={packed} b {b_dtype}")
    kinds = ["random", "chain", "bushy", "random", "chain", "bushy"]
    batch1 = synth.make_batch(46, 0, sizes1, hk=2, hv=4, kinds=kinds)
    batch2 = synth.make_batch(47, 0, sizes2, hk=2, hv=4, kinds=kinds[::-1])
    batch1.b, batch2.b = batch1.b.to(b_dtype), batch2.b.to(b_dtype)  # the oracle reads the same rounded gates
    empty, shorten = (2,), (5,)
    for raw_keys in (False, True):
        pool, o2, aux2, walks = _run_chain(cuda, batch1, batch2, per_khead=True, packed=packed, empty=empty,
                                           shorten=shorten, raw_keys=raw_keys, raw_values=True)
        _check_chain(batch1, batch2, pool, o2, aux2, walks, empty, per_khead=True)
        pool_s, o2_s, _, _ = _run_chain(cuda, batch1, batch2, per_khead=True, packed=packed, empty=empty,
                                        shorten=shorten, raw_keys=raw_keys)
        assert rel_l2(np32(pool), np32(pool_s)) <= 1e-5
        assert rel_l2(np32(o2), np32(o2_s)) <= 1e-4


@pytest.mark.parametrize("packed", [False, True])
def test_commit_verify_recomputed_values_unaligned_rows(cuda, packed):
    """Raw k and v rows whose row stride is not a multiple of 16 bytes take the
    32-wide kernel that loads them into registers; aligned rows take the one
    that copies them into LDS ahead of the state tile.  Both read the same
    values: bit-identical states, outputs and saves, and the oracle chain."""
    from dforktree_amd import synth
    announce(f"commit->verify recomputed values, aligned vs padded rows packed={packed}")
    sizes1, sizes2 = ([32, 7, 19, 1, 32, 25], [32, 12, 32, 4, 17, 30]) if packed else ([32] * 6, [32] * 6)
    kinds = ["random", "chain", "bushy", "random", "chain", "bushy"]
    batch1 = synth.make_batch(50, 0, sizes1, hk=2, hv=4, kinds=kinds)
    batch2 = synth.make_batch(51, 0, sizes2, hk=2, hv=4, kinds=kinds[::-1])
    empty, shorten = (3,), (5,)
    runs = [_run_chain(cuda, batch1, batch2, per_khead=True, packed=packed, empty=empty, shorten=shorten,
                       raw_keys=True, raw_values=True, row_pad=pad) for pad in (0, 4)]
    (pool_a, o_a, aux_a, walks), (pool_p, o_p, aux_p, _) = runs
    _check_chain(batch1, batch2, pool_p, o_p, aux_p, walks, empty, per_khead=True)
    assert torch.equal(pool_a, pool_p)
    assert torch.equal(o_a, o_p)
    for a, b in zip(aux_a, aux_p):
        assert torch.equal(a, b)


def test_commit_verify_recomputed_values_bench_shape(cuda):
    """The measured form at its shape: 64 requests of 32-node trees at full
    width, keys and values both from step 1's y (the verify saves neither)."""
    from dforktree_amd import synth
    announce("commit->verify raw keys + recomputed values, bench shape 64 x 32")
    batch1 = synth.make_batch(48, 0, [32] * 64, hk=16, hv=32, kinds="random")
    batch2 = synth.make_batch(49, 0, [32] * 64, hk=16, hv=32, kinds="random")
    empty, shorten = (11,), (40,)
    pool, o2, aux2, walks = _run_chain(cuda, batch1, batch2, per_khead=True, packed=False, empty=empty,
                                       shorten=shorten, raw_keys=True, raw_values=True)
    _check_chain(batch1, batch2, pool, o2, aux2, walks, empty, per_khead=True)


def test_commit_verify_equals_commit_then_verify(cuda):
    """Full layer width (16 q/k heads, 32 v heads) at 32 nodes: the fused entry
    against dft_tree_commit (in place) followed by dft_tree_verify."""
    from dforktree_amd import ops, synth
    announce("commit->verify vs separate kernels")
    B, N, hk, hv = 8, 32, 16, 32
    b1 = synth.make_batch(24, 0, [N] * B, hk=hk, hv=hv)
    b2 = synth.make_batch(25, 0, [N] * B, hk=hk, hv=hv)
    g1, g2 = b1.to(cuda), b2.to(cuda)
    rows = B * N
    k1 = torch.zeros(hk, rows, 128, device=cuda)
    v1 = torch.zeros(hv, rows, 128, device=cuda)
    G1 = torch.zeros(hv, rows, device=cuda)
    pool_a = b1.state.clone().to(cuda)
    ts1 = ops.tree_struct(g1.parent, 4, batch=B, n_nodes=N, want=("anc_bits",))["anc_bits"]
    ts2 = ops.tree_struct(g2.parent, 4, batch=B, n_nodes=N, want=("anc_bits",))["anc_bits"]
    ops.tree_verify(g1.y, g1.a, g1.b, g1.A_log, g1.dt_bias, pool_a.transpose(-1, -2), hk=hk, hv=hv, anc_bits=ts1,
                    batch=B, n_nodes=N, aux_k=k1, aux_v=v1, aux_g=G1, aux_k_per_khead=True)
    pool_b = pool_a.clone()
    idx, lens, _ = _paths(b1, 9)
    idx_d, lens_d = idx.to(cuda), lens.to(cuda)
    outs = []
    for fused, pool in ((True, pool_a), (False, pool_b)):
        aux = (torch.zeros(hk, rows, 128, device=cuda), torch.zeros(hv, rows, 128, device=cuda),
               torch.zeros(hv, rows, device=cuda))
        common = dict(hk=hk, hv=hv, anc_bits=ts2, batch=B, n_nodes=N, aux_k=aux[0], aux_v=aux[1], aux_g=aux[2],
                      aux_k_per_khead=True)
        if fused:
            o = ops.tree_commit_verify(g2.y, g2.a, g2.b, g2.A_log, g2.dt_bias, pool.transpose(-1, -2),
                                       pending_path=idx_d, pending_keys=k1, pending_values=v1, pending_gains=G1,
                                       pending_path_len=lens_d, prev_n_nodes=N, pending_k_head_div=hv // hk,
                                       **common)
        else:
            ops.tree_commit(pool.unsqueeze(0), k1.unsqueeze(0), v1.unsqueeze(0), G1.unsqueeze(0), idx_d, n_nodes=N,
                            path_len=lens_d, k_head_div=hv // hk)
            o = ops.tree_verify(g2.y, g2.a, g2.b, g2.A_log, g2.dt_bias, pool.transpose(-1, -2), **common)
        outs.append((o, aux))
    torch.cuda.synchronize()
    assert rel_l2(np32(pool_a), np32(pool_b)) <= 1e-6
    (oa, auxa), (ob, auxb) = outs
    assert rel_l2(np32(oa), np32(ob)) <= 1e-5
    for x, y in zip(auxa, auxb):
        assert rel_l2(np32(x), np32(y)) <= 1e-6


def test_commit_verify_recomputed_values_slots_int64_vhead_keys(cuda):
    """The recomputed-value form with keys saved per v-head (k_head_div 1),
    int64 path entries and state indices [2, -1, 1, 3] over a pool of 5
    slots: against the same launch with saved values (committed states within
    rel-L2 1e-5, o within 1e-4).  The slotless request verifies on slot 0 and
    commits nothing, so slots 0 and 4 keep their bits (no committing request
    owns slot 0, which the slotless one reads)."""
    from dforktree_amd import ops, synth
    announce("commit->verify recomputed values: v-head keys, int64 paths, slots")
    B, N, hk, hv = 4, 32, 2, 4
    b1 = synth.make_batch(54, 0, [N] * B, hk=hk, hv=hv, kinds=["random", "chain", "bushy", "random"])
    b2 = synth.make_batch(55, 0, [N] * B, hk=hk, hv=hv)
    g1, g2 = b1.to(cuda), b2.to(cuda)
    rows = B * N
    slots = torch.tensor([2, -1, 1, 3], dtype=torch.int32, device=cuda)
    pool0 = (torch.randn(5, hv, 128, 128, generator=torch.Generator().manual_seed(56)) * 0.02).to(cuda)
    k1 = torch.zeros(hv, rows, 128, device=cuda)
    v1 = torch.zeros(hv, rows, 128, device=cuda)
    G1 = torch.zeros(hv, rows, device=cuda)
    ts1 = ops.tree_struct(g1.parent, 4, batch=B, n_nodes=N, want=("anc_bits",))["anc_bits"]
    ts2 = ops.tree_struct(g2.parent, 4, batch=B, n_nodes=N, want=("anc_bits",))["anc_bits"]
    ops.tree_verify(g1.y, g1.a, g1.b, g1.A_log, g1.dt_bias, pool0.transpose(-1, -2), hk=hk, hv=hv, anc_bits=ts1,
                    batch=B, n_nodes=N, state_indices=slots, aux_k=k1, aux_v=v1, aux_g=G1)
    idx, lens, _ = _paths(b1, 57)
    idx_d, lens_d = idx.to(torch.int64).to(cuda), lens.to(cuda)
    common = dict(hk=hk, hv=hv, anc_bits=ts2, batch=B, n_nodes=N, state_indices=slots, pending_path=idx_d,
                  pending_keys=k1, pending_gains=G1, pending_path_len=lens_d, prev_n_nodes=N, pending_k_head_div=1)
    pools, outs = [], []
    for recompute in (False, True):
        pool = pool0.clone()
        vals = (dict(pending_values=None, pending_value_rows=g1.y[:, 2 * hk * 128:].unflatten(1, (hv, 128)),
                     pending_b=g1.b) if recompute else dict(pending_values=v1))
        outs.append(ops.tree_commit_verify(g2.y, g2.a, g2.b, g2.A_log, g2.dt_bias, pool.transpose(-1, -2), **vals,
                                           **common))
        pools.append(pool)
    torch.cuda.synchronize()
    for s_ in (0, 4):
        assert np.array_equal(np32(pools[1][s_]), np32(pool0[s_])), f"slot {s_} was written"
    for s_ in (1, 2, 3):
        assert not np.array_equal(np32(pools[1][s_]), np32(pool0[s_])), f"slot {s_} was not committed"
    assert rel_l2(np32(pools[1]), np32(pools[0])) <= 1e-5
    assert rel_l2(np32(outs[1]), np32(outs[0])) <= 1e-4


def test_commit_verify_negative_slot_commits_nothing(cuda):
    """State indices [2, -1, 1] over a pool of 4 slots, every request with a
    pending path: the request without a slot verifies on slot 0 (as the plain
    verify does) and commits nothing, so slots 0 and 3 keep their bits; the
    fused entry equals the separate commit (same slots) followed by the
    plain verify."""
    from dforktree_amd import ops, synth
    announce("commit->verify, negative state index")
    B, N, hk, hv = 3, 32, 2, 4
    b1 = synth.make_batch(26, 0, [N] * B, hk=hk, hv=hv)
    b2 = synth.make_batch(27, 0, [N] * B, hk=hk, hv=hv)
    g1, g2 = b1.to(cuda), b2.to(cuda)
    rows = B * N
    slots = torch.tensor([2, -1, 1], dtype=torch.int32, device=cuda)
    pool0 = (torch.randn(4, hv, 128, 128, generator=torch.Generator().manual_seed(28)) * 0.02).to(cuda)
    k1 = torch.zeros(hv, rows, 128, device=cuda)
    v1 = torch.zeros(hv, rows, 128, device=cuda)
    G1 = torch.zeros(hv, rows, device=cuda)
    ts1 = ops.tree_struct(g1.parent, 4, batch=B, n_nodes=N, want=("anc_bits",))["anc_bits"]
    ts2 = ops.tree_struct(g2.parent, 4, batch=B, n_nodes=N, want=("anc_bits",))["anc_bits"]
    ops.tree_verify(g1.y, g1.a, g1.b, g1.A_log, g1.dt_bias, pool0.transpose(-1, -2), hk=hk, hv=hv, anc_bits=ts1,
                    batch=B, n_nodes=N, state_indices=slots, aux_k=k1, aux_v=v1, aux_g=G1)
    idx, lens, _ = _paths(b1, 29)
    idx_d, lens_d = idx.to(cuda), lens.to(cuda)
    assert int(lens[1]) > 0, "the slotless request must have a pending path"
    pool_a, pool_b = pool0.clone(), pool0.clone()
    common = dict(hk=hk, hv=hv, anc_bits=ts2, batch=B, n_nodes=N, state_indices=slots)
    oa = ops.tree_commit_verify(g2.y, g2.a, g2.b, g2.A_log, g2.dt_bias, pool_a.transpose(-1, -2),
                                pending_path=idx_d, pending_keys=k1, pending_values=v1, pending_gains=G1,
                                pending_path_len=lens_d, prev_n_nodes=N, **common)
    ops.tree_commit(pool_b.unsqueeze(0), k1.unsqueeze(0), v1.unsqueeze(0), G1.unsqueeze(0), idx_d, n_nodes=N,
                    path_len=lens_d, src_slots=slots)
    ob = ops.tree_verify(g2.y, g2.a, g2.b, g2.A_log, g2.dt_bias, pool_b.transpose(-1, -2), **common)
    torch.cuda.synchronize()
    for s in (0, 3):
        assert np.array_equal(np32(pool_a[s]), np32(pool0[s])), f"fused entry wrote slot {s}"
        assert np.array_equal(np32(pool_b[s]), np32(pool0[s])), f"commit wrote slot {s}"
    for s in (1, 2):
        assert not np.array_equal(np32(pool_a[s]), np32(pool0[s])), f"slot {s} was not committed"
    assert rel_l2(np32(pool_a), np32(pool_b)) <= 1e-6
    assert rel_l2(np32(oa), np32(ob)) <= 1e-5


def test_commit_verify_many_items_chain_of_three(cuda):
    """Full layer width at 24 requests (768 items, one round of resident
    workgroups), three steps: plain verify, then two fused commit -> verify
    steps that alternate the save buffers; checked against the oracle chain."""
    from dforktree_amd import ops, synth
    announce("commit->verify many items, 3 steps")
    B, N, hk, hv = 24, 32, 16, 32
    steps = [synth.make_batch(30 + t, 0, [N] * B, hk=hk, hv=hv, kinds=["random", "chain", "bushy"] * 8)
             for t in range(3)]
    pool = steps[0].state.clone().to(cuda)
    rows = B * N
    saves = [tuple(torch.zeros(*sh, device=cuda) for sh in ((hk, rows, 128), (hv, rows, 128), (hv, rows)))
             for _ in range(2)]
    outs, walks_all = [], []
    S = [np32(steps[0].state[r]).transpose(0, 2, 1) for r in range(B)]
    for t, bt in enumerate(steps):
        g = bt.to(cuda)
        ts = ops.tree_struct(g.parent, 4, batch=B, n_nodes=N, want=("anc_bits",))["anc_bits"]
        k, v, G = saves[t % 2]
        common = dict(hk=hk, hv=hv, anc_bits=ts, batch=B, n_nodes=N, aux_k=k, aux_v=v, aux_g=G, aux_k_per_khead=True)
        if t == 0:
            o = ops.tree_verify(g.y, g.a, g.b, g.A_log, g.dt_bias, pool.transpose(-1, -2), **common)
        else:
            pk, pv, pG = saves[(t - 1) % 2]
            o = ops.tree_commit_verify(g.y, g.a, g.b, g.A_log, g.dt_bias, pool.transpose(-1, -2), pending_path=idx_d,
                                       pending_keys=pk, pending_values=pv, pending_gains=pG, pending_path_len=lens_d,
                                       prev_n_nodes=N, pending_k_head_div=hv // hk, **common)
        idx, lens, walks = _paths(bt, 40 + t)
        idx_d, lens_d = idx.to(cuda), lens.to(cuda)
        outs.append(np32(o))
        walks_all.append(walks)
    torch.cuda.synchronize()
    # oracle chain: verify step t on S, commit its walk, repeat
    for t, bt in enumerate(steps):
        b = bt.to("cpu")
        b.state = torch.stack([torch.from_numpy(np.ascontiguousarray(s.transpose(0, 2, 1))) for s in S])
        ref = oracle_verify(b)
        for r, sl in enumerate(request_slices(b)):
            want = O.bf16_round(ref[r]["o"])
            assert rel_l2(outs[t][sl], want) <= REL_L2 and max_abs(outs[t][sl], want) <= MAX_ABS_BF16, (t, r)
            if t < 2:
                S[r] = O.closed_commit(S[r], ref[r]["k"], ref[r]["vn"], ref[r]["G"], walks_all[t][r])
    # the pool holds the state after step 1's commit (step 2's walk is still pending)
    got = np32(pool)
    for r in range(B):
        assert rel_l2(got[r].transpose(0, 2, 1), S[r]) <= REL_L2, r
