"""GPU parity of the closed-form accepted-path commit.

Committed states: rel-L2 <= 2e-3 against the fp64 sequential replay of the
accepted tokens (the commit after a GPU verify), and 1e-5 against the fp32
closed form on the same saved inputs; path/ancestor index handling is exact
(a state the path does not reach is bit-identical to its input).
"""
import numpy as np
import pytest
import torch

from conftest import REL_L2, announce, rel_l2
from _ref import np32, request_slices
from oracle import gdn_tree as O

pytestmark = pytest.mark.gpu


def _aux(seed, L, H, rows):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(L, H, rows, 128, generator=g)
    k = k / k.norm(dim=-1, keepdim=True)
    v = torch.randn(L, H, rows, 128, generator=g) * 0.3
    gains = -torch.rand(L, H, rows, generator=g) * 2.0
    return k, v, gains


def _paths(pars, max_len, seed):
    from dforktree_amd import synth
    g = torch.Generator().manual_seed(seed)
    paths = [synth.accepted_path(p, max_len, g) for p in pars]
    P = max_len
    idx = torch.full((len(paths), P), -1, dtype=torch.int32)
    for i, p in enumerate(paths):
        idx[i, :len(p)] = p
    return paths, idx, torch.tensor([len(p) for p in paths], dtype=torch.int32)


def test_commit_inplace_closed_form(cuda):
    from dforktree_amd import ops, synth
    announce("commit in place closed form")
    L, B, H, N = 3, 6, 4, 32
    g = torch.Generator().manual_seed(0)
    pars = [synth.tree_parents(N, "random", g) for _ in range(B)]
    keys, vals, gains = _aux(1, L, H, B * N)
    S = torch.randn(L, B, H, 128, 128) * 0.02  # [L, slot, H, V, K]
    paths, idx, lens = _paths(pars, 16, 2)
    Sg = S.to(cuda)
    ops.tree_commit(Sg, keys.to(cuda), vals.to(cuda), gains.to(cuda), idx.to(cuda), n_nodes=N,
                    path_len=lens.to(cuda))
    torch.cuda.synchronize()
    got = np32(Sg)
    for l in range(L):
        for b in range(B):
            sl = slice(b * N, (b + 1) * N)
            want = O.closed_commit(np32(S[l, b]).transpose(0, 2, 1), np32(keys[l, :, sl]), np32(vals[l, :, sl]),
                                   np32(gains[l, :, sl]), paths[b].tolist())
            assert rel_l2(got[l, b].transpose(0, 2, 1), want) <= 1e-5, (l, b)


def test_commit_inplace_negative_slot_writes_nothing(cuda):
    """A request whose slot index is negative (a padded request) commits
    nothing: no slot changes for it, slot 0 included, while the other
    requests commit into their own slots."""
    from dforktree_amd import ops, synth
    announce("commit in place, negative slot")
    L, B, H, N = 2, 3, 4, 32
    g = torch.Generator().manual_seed(5)
    pars = [synth.tree_parents(N, "random", g) for _ in range(B)]
    keys, vals, gains = _aux(6, L, H, B * N)
    S = torch.randn(L, 4, H, 128, 128) * 0.02  # [L, slot, H, V, K]: slots 0 and 3 belong to nobody
    slots = torch.tensor([2, -1, 1], dtype=torch.int32)
    paths, idx, lens = _paths(pars, 16, 7)
    Sg = S.to(cuda)
    ops.tree_commit(Sg, keys.to(cuda), vals.to(cuda), gains.to(cuda), idx.to(cuda), n_nodes=N,
                    path_len=lens.to(cuda), src_slots=slots.to(cuda))
    torch.cuda.synchronize()
    got = np32(Sg)
    for s in (0, 3):
        assert np.array_equal(got[:, s], np32(S[:, s])), f"slot {s} was written"
    for l in range(L):
        for b in (0, 2):
            sl = slice(b * N, (b + 1) * N)
            s = int(slots[b])
            want = O.closed_commit(np32(S[l, s]).transpose(0, 2, 1), np32(keys[l, :, sl]), np32(vals[l, :, sl]),
                                   np32(gains[l, :, sl]), paths[b].tolist())
            assert rel_l2(got[l, s].transpose(0, 2, 1), want) <= 1e-5, (l, b)


def test_commit_full_size_pool(cuda):
    """Accept-and-commit at full size: 24 layers x 128 requests x 32 v-heads
    of 2 MiB fp32 state per request-layer (a 6 GiB pool, so byte offsets pass
    4 GiB), 32-node random trees, random accepted walks of length 1-16, keys
    per k-head (16 k-heads).  One launch commits everything in place; a spread
    of (layer, request) tiles, the first and last ones included, is checked
    against the fp32 closed form, and every committed value must be finite."""
    from dforktree_amd import ops, synth
    announce("commit in place, full-size pool (24 x 128 x 32 heads)")
    L, B, HK, HV, N, D = 24, 128, 16, 32, 32, 128
    rows = B * N
    S = synth.device_randn_(torch.empty(L, B, HV, D, D, device=cuda), 21, std=0.02)  # [L, slot, H, V, K]
    keys = synth.device_randn_(torch.empty(L, HK, rows, D, device=cuda), 22, std=D ** -0.5)
    vals = synth.device_randn_(torch.empty(L, HV, rows, D, device=cuda), 23, std=0.3)
    gains = synth.device_randn_(torch.empty(L, HV, rows, device=cuda), 24).abs_().neg_()
    g = torch.Generator().manual_seed(25)
    pars = [synth.tree_parents(N, "random", g) for _ in range(B)]
    paths, idx, lens = _paths(pars, 16, 26)
    picks = [(0, 0), (0, B - 1), (L - 1, 0), (L - 1, B - 1), (11, 64), (17, 63)]
    pg = torch.Generator().manual_seed(27)
    picks += [(int(torch.randint(0, L, (1,), generator=pg)), int(torch.randint(0, B, (1,), generator=pg)))
              for _ in range(10)]
    before = {lb: np32(S[lb[0], lb[1]]) for lb in picks}
    ops.tree_commit(S, keys, vals, gains, idx.to(cuda), n_nodes=N, path_len=lens.to(cuda), k_head_div=HV // HK)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(S).all())
    for l, b in picks:
        sl = slice(b * N, (b + 1) * N)
        kh = np32(keys[l, :, sl])[np.arange(HV) // (HV // HK)]  # v-head h uses k-head h // 2
        want = O.closed_commit(before[(l, b)].transpose(0, 2, 1), kh, np32(vals[l, :, sl]), np32(gains[l, :, sl]),
                               paths[b].tolist())
        assert rel_l2(np32(S[l, b]).transpose(0, 2, 1), want) <= 1e-5, (l, b, len(paths[b]))


def test_verify_then_commit_matches_replay(cuda):
    """Config-4 shape in miniature: verify every layer on the GPU (saving k, vn,
    G), commit the accepted root-to-node walk in place, compare with an fp64
    decoder that consumes only the accepted tokens."""
    from dforktree_amd import ops, synth
    announce("verify+commit vs replay")
    L, B, N, hk, hv = 2, 5, 32, 2, 4
    batches = [synth.make_batch(4, l, [N] * B, hk=hk, hv=hv, kinds=["random", "chain", "bushy", "random", "chain"])
               for l in range(L)]
    pars = [batches[0].parent[s] for s in request_slices(batches[0])]
    for bt in batches[1:]:  # same trees in every layer
        bt.parent = batches[0].parent.clone()
    rows = B * N
    keys = torch.zeros(L, hv, rows, 128, device=cuda)
    vals = torch.zeros(L, hv, rows, 128, device=cuda)
    gains = torch.zeros(L, hv, rows, device=cuda)
    state = torch.stack([bt.state for bt in batches]).to(cuda)  # [L, B, hv, V, K]
    ts = ops.tree_struct(batches[0].parent.to(cuda), 4, batch=B, n_nodes=N, want=("anc_bits",))
    for l, bt in enumerate(batches):
        gb = bt.to(cuda)
        ops.tree_verify(gb.y, gb.a, gb.b, gb.A_log, gb.dt_bias, state[l].transpose(-1, -2), hk=hk, hv=hv,
                        anc_bits=ts["anc_bits"], batch=B, n_nodes=N, aux_k=keys[l], aux_v=vals[l], aux_g=gains[l])
    paths, idx, lens = _paths(pars, 16, 3)
    ops.tree_commit(state, keys, vals, gains, idx.to(cuda), n_nodes=N, path_len=lens.to(cuda))
    torch.cuda.synchronize()
    got = np32(state)
    for l, bt in enumerate(batches):
        for b, sl in enumerate(request_slices(bt)):
            S0 = np32(bt.state[b]).transpose(0, 2, 1)
            want = O.replay_path_f64(np32(bt.y[sl]), np32(bt.a[sl]), np32(bt.b[sl]), np32(bt.A_log),
                                     np32(bt.dt_bias), S0, paths[b].tolist(), hk, hv, 128, 128)
            assert rel_l2(got[l, b].transpose(0, 2, 1), want) <= REL_L2, (l, b)


def test_snapshot_two_ends_with_ancestry(cuda):
    """fc1_fused snapshot form: two ends per request (last accepted and a
    tracked earlier step, or -1), ancestry-checked path, a separate
    destination cache indexed by node; untouched destinations stay intact."""
    from dforktree_amd import synth
    from dforktree_amd.plugin import fc1_fused
    announce("snapshot two ends")
    L, B, H, N = 2, 3, 4, 32
    g = torch.Generator().manual_seed(5)
    pars = [synth.tree_parents(N, "random", g) for _ in range(B)]
    keys, vals, gains = _aux(6, L, H, B * N)
    temporal = torch.randn(L, 4, H, 128, 128) * 0.02
    slots = torch.tensor([2, 0, 3], dtype=torch.int32)
    dsts = torch.tensor([1, 0, 2], dtype=torch.int32)
    paths, idx, lens = _paths(pars, 16, 7)
    # add an off-path node id to each path row to exercise the ancestry mask
    anc = torch.stack([torch.from_numpy(O.tree_struct(p.numpy())[0]) for p in pars])
    ends = torch.full((B, 2), -1, dtype=torch.int32)
    for b, p in enumerate(paths):
        ends[b, 0] = p[-1]
        if len(p) > 2:
            ends[b, 1] = p[len(p) // 2]
        if len(p) < 16:
            off = [u for u in range(N) if anc[b, p[-1], u] < 0.5]
            if off:
                idx[b, len(p)] = off[0]
    sentinel = 123.0
    out = torch.full((L, 3, N, H, 128, 128), sentinel)
    outg = out.to(cuda)
    for b in range(B):
        # snapshot_commit is the batch-1 hook form; call it per request with its own slice
        sl = slice(b * N, (b + 1) * N)
        fc1_fused.snapshot_commit(temporal.to(cuda), keys[:, :, sl].contiguous().to(cuda),
                                  vals[:, :, sl].contiguous().to(cuda), gains[:, :, sl].contiguous().to(cuda),
                                  anc[b].to(cuda), idx[b:b + 1].to(cuda), ends[b].to(cuda), slots[b:b + 1].to(cuda),
                                  dsts[b:b + 1].to(cuda), outg)
    torch.cuda.synchronize()
    got = outg.cpu()
    touched = torch.zeros(L, 3, N, dtype=torch.bool)
    for b in range(B):
        sl = slice(b * N, (b + 1) * N)
        for e in range(2):
            u = int(ends[b, e])
            if u < 0:
                continue
            touched[:, int(dsts[b]), u] = True
            for l in range(L):
                want = O.closed_commit(np32(temporal[l, int(slots[b])]).transpose(0, 2, 1), np32(keys[l, :, sl]),
                                       np32(vals[l, :, sl]), np32(gains[l, :, sl]), idx[b].tolist(), u=u,
                                       anc=anc[b].numpy())
                assert rel_l2(np32(got[l, int(dsts[b]), u]).transpose(0, 2, 1), want) <= 1e-5
    assert torch.all(got[~touched] == sentinel)


def test_closed_commit_dropin(cuda):
    """tree_kernels.closed_commit: states [L, H, DK, DV] (k-major), path src
    with the last index n on the device, in place."""
    from dforktree_amd import synth
    from dforktree_amd.plugin import tree_kernels as TK
    announce("closed_commit drop-in")
    L, H, N = 3, 4, 32
    g = torch.Generator().manual_seed(8)
    par = synth.tree_parents(N, "random", g)
    path = synth.accepted_path(par, 16, g)
    keys, vals, gains = _aux(9, L, H, N)
    S = torch.randn(L, H, 128, 128) * 0.02
    Sg = S.to(cuda)
    src = torch.zeros(16, dtype=torch.int64)
    src[:len(path)] = path
    n = torch.tensor([len(path) - 1], dtype=torch.int32)
    TK.closed_commit(Sg, keys.to(cuda), vals.to(cuda), gains.to(cuda), src.to(cuda), n.to(cuda))
    torch.cuda.synchronize()
    for l in range(L):
        want = O.closed_commit(np32(S[l]), np32(keys[l]), np32(vals[l]), np32(gains[l]), path.tolist())
        assert rel_l2(np32(Sg[l]), want) <= 1e-5


def test_config4_full_size_verify_then_commit_matches_replay(cuda):
    """The accept-and-commit workload at full size, after a real verify:
    24 layers x 128 requests of 32-node trees at full width (16 q/k heads,
    32 v heads, 2 MiB of fp32 state per request-layer: a 6 GiB pool).  Every
    layer is verified on the GPU (keys saved per k-head, vn, G), then each
    request's seeded accepted walk (length 1-16) is committed in place in
    one launch.  At least 16 (layer, request) tiles, the first and last
    included, must agree with an fp64 decoder that consumes only the
    accepted tokens (rel-L2 <= 2e-3).  Every 4th request is a chain, whose
    accepted walk is a prefix: there the replay is plain gated delta-rule
    decoding of the first tokens.  Every committed value must be finite."""
    import math
    from dforktree_amd import ops, synth
    announce("config4 full size: verify 24 x 128 x 32 heads, commit, replay")
    L, B, HK, HV, N, D = 24, 128, 16, 32, 32, 128
    C = 2 * HK * D + HV * D
    rows = B * N
    g = torch.Generator().manual_seed(80)
    kinds = ["chain" if b % 4 == 0 else "random" for b in range(B)]
    pars = [synth.tree_parents(N, k, g) for k in kinds]
    parent = torch.cat(pars).to(cuda)
    ts = ops.tree_struct(parent, 4, batch=B, n_nodes=N, want=("anc_bits",))
    S = synth.device_randn_(torch.empty(L, B, HV, D, D, device=cuda), 81, std=0.02)  # [L, slot, H, V, K]
    y = synth.device_randn_(torch.empty(L, rows, C, device=cuda, dtype=torch.bfloat16), 82)
    a = synth.device_randn_(torch.empty(L, rows, HV, device=cuda), 83)
    bb = synth.device_randn_(torch.empty(L, rows, HV, device=cuda), 84)
    A_log = torch.full((HV,), math.log(0.5), device=cuda)
    dt_bias = torch.zeros(HV, device=cuda)
    keys = torch.empty(L, HK, rows, D, device=cuda)
    vals = torch.empty(L, HV, rows, D, device=cuda)
    gains = torch.empty(L, HV, rows, device=cuda)
    picks = [(0, 0), (0, B - 1), (L - 1, 0), (L - 1, B - 1), (12, 4), (5, 64)]
    pg = torch.Generator().manual_seed(85)
    picks += [(int(torch.randint(0, L, (1,), generator=pg)), int(torch.randint(0, B, (1,), generator=pg)))
              for _ in range(12)]
    before = {(l, b): np32(S[l, b]) for l, b in picks}
    for l in range(L):
        ops.tree_verify(y[l], a[l], bb[l], A_log, dt_bias, S[l].transpose(-1, -2), hk=HK, hv=HV,
                        anc_bits=ts["anc_bits"], batch=B, n_nodes=N, aux_k=keys[l], aux_v=vals[l], aux_g=gains[l],
                        aux_k_per_khead=True)
    paths, idx, lens = _paths(pars, 16, 86)
    ops.tree_commit(S, keys, vals, gains, idx.to(cuda), n_nodes=N, path_len=lens.to(cuda), k_head_div=HV // HK)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(S).all())
    Al, dtb = np32(A_log), np32(dt_bias)
    for l, b in picks:
        sl = slice(b * N, (b + 1) * N)
        path = paths[b].tolist()
        if kinds[b] == "chain":
            assert path == list(range(len(path))), "a chain's accepted walk is a prefix"
        want = O.replay_path_f64(np32(y[l, sl]), np32(a[l, sl]), np32(bb[l, sl]), Al, dtb,
                                 before[(l, b)].transpose(0, 2, 1), path, HK, HV, D, D)
        err = rel_l2(np32(S[l, b]).transpose(0, 2, 1), want)
        assert err <= REL_L2, (l, b, len(path), err)
