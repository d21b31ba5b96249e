"""GPU parity of the fused tree verify against the CPU oracle.

Tolerances (stated for this path): node outputs and WY values within
rel-L2 <= 2e-3 of the fp32 recurrence, bf16 outputs within max-abs <= 1e-2;
the saved ancestry-derived gains G and the normalised keys within 1e-5.
"""
import numpy as np
import pytest
import torch

from conftest import MAX_ABS_BF16, REL_L2, announce, max_abs, rel_l2
from _ref import np32, oracle_recurrent, oracle_verify, request_slices
from oracle import gdn_tree as O

pytestmark = pytest.mark.gpu


def run_gpu(batch, dev, use_bits=False, o_dtype=torch.bfloat16, packed=None, state_indices=None, state=None,
            records=False, n_nodes=None):
    from dforktree_amd import ops
    g = batch.to(dev)
    rows = g.y.shape[0]
    uniform = len(set(batch.sizes)) == 1
    packed = (not uniform) if packed is None else packed
    aux_k = torch.zeros(batch.hv, rows, 128, device=dev)
    aux_v = torch.zeros(batch.hv, rows, 128, device=dev)
    aux_g = torch.zeros(batch.hv, rows, device=dev)
    st = (g.state if state is None else state).transpose(-1, -2)
    kw = dict(hk=batch.hk, hv=batch.hv, o_dtype=o_dtype, aux_k=aux_k, aux_v=aux_v, aux_g=aux_g,
              state_indices=state_indices)
    if packed:
        n_nodes = batch.n_max if n_nodes is None else n_nodes
        kw.update(cu_seqlens=g.cu_seqlens, n_nodes=n_nodes, batch=batch.batch)
        if records:  # size-order records: a launch over 32 nodes takes the mixed-width kernel
            kw["size_order"] = ops.size_order(g.cu_seqlens, n_nodes)
    else:
        kw.update(batch=batch.batch, n_nodes=batch.sizes[0])
    if use_bits or packed:
        ts = ops.tree_struct(g.parent, 4, cu_seqlens=g.cu_seqlens, n_nodes=batch.n_max, batch=batch.batch,
                             want=("anc_bits",))
        kw["anc_bits"] = ts["anc_bits"]
    else:
        anc = torch.stack([torch.from_numpy(O.tree_struct(p)[0]) for p in
                           [batch.parent[s].numpy() for s in request_slices(batch)]]).to(dev)
        kw["anc"] = anc
    o = ops.tree_verify(g.y, g.a, g.b, g.A_log, g.dt_bias, st, **kw)
    torch.cuda.synchronize()
    return o, aux_k, aux_v, aux_g


def check_against_oracle(batch, o, aux_k, aux_v, aux_g, o_bf16=True):
    ref = oracle_verify(batch)
    o, aux_k, aux_v, aux_g = (np32(t) for t in (o, aux_k, aux_v, aux_g))
    for r, sl in enumerate(request_slices(batch)):
        want_o = O.bf16_round(ref[r]["o"]) if o_bf16 else ref[r]["o"]
        assert rel_l2(o[sl], want_o) <= REL_L2, f"request {r}: o rel-L2 {rel_l2(o[sl], want_o):.3e}"
        if o_bf16:
            assert max_abs(o[sl], want_o) <= MAX_ABS_BF16
        assert rel_l2(aux_v[:, sl], ref[r]["vn"]) <= REL_L2, f"request {r}: vn"
        assert rel_l2(aux_k[:, sl], ref[r]["k"]) <= 1e-5, f"request {r}: k"
        assert rel_l2(aux_g[:, sl], ref[r]["G"]) <= 1e-5, f"request {r}: G"


@pytest.mark.parametrize("n,kind", [(32, "random"), (32, "chain"), (32, "bushy"), (16, "random"), (1, "random"),
                                    (20, "random"), (64, "random"), (64, "chain"), (48, "bushy"), (33, "random")])
def test_verify_single_request(cuda, n, kind):
    announce(f"verify single n={n} kind={kind}")
    batch = __import__("dforktree_amd.synth", fromlist=["x"]).make_batch(11, 0, [n], hk=2, hv=4, kinds=kind)
    check_against_oracle(batch, *run_gpu(batch, cuda))


def test_verify_config0_full_width(cuda):
    """Batch 1, 32 nodes, 16 q/k heads, 32 v heads, fp32 S0 -- and directly
    against the fp64 node-by-node recurrence as well."""
    from dforktree_amd import synth
    announce("verify config0 full width")
    batch = synth.make_batch(0, 0, [32], hk=16, hv=32)
    o, k, v, g = run_gpu(batch, cuda)
    check_against_oracle(batch, o, k, v, g)
    f = oracle_recurrent(batch, 0)
    assert rel_l2(np32(o), f["o"]) <= REL_L2
    assert rel_l2(np32(v), f["vn"]) <= REL_L2


def test_verify_fp32_output_tighter(cuda):
    """With fp32 outputs the hi/lo split keeps the result far inside the tolerance."""
    from dforktree_amd import synth
    announce("verify fp32 out")
    batch = synth.make_batch(5, 0, [32], hk=2, hv=4)
    o, k, v, g = run_gpu(batch, cuda, o_dtype=torch.float32)
    ref = oracle_verify(batch)[0]
    assert rel_l2(np32(o), ref["o"]) <= 5e-5
    assert rel_l2(np32(v), ref["vn"]) <= 5e-5


def test_verify_batched_uniform_bits(cuda):
    from dforktree_amd import synth
    announce("verify batched uniform anc_bits")
    batch = synth.make_batch(1, 0, [32] * 6, hk=2, hv=4, kinds=["random", "chain", "bushy"] * 2)
    check_against_oracle(batch, *run_gpu(batch, cuda, use_bits=True))


@pytest.mark.parametrize("hk,hv,records", [(2, 4, False), (2, 4, True), (2, 2, True), (1, 4, True), (2, 8, True)])
def test_verify_packed_ragged(cuda, hk, hv, records):
    """Packed varlen rows with cu_seqlens, sizes 1..64: two kernels without
    size-order records, the mixed-width kernel with them, whose v-head pairs
    (2j, 2j + 1) span one k-head (R = 2), two k-heads (R = 1) or half of one
    (R = 4)."""
    from dforktree_amd import synth
    announce(f"verify packed ragged hk={hk} hv={hv} records={records}")
    sizes, kinds = [8, 64, 17, 1, 33, 64, 40, 9], ["chain", "random", "bushy", "random", "chain", "bushy",
                                                 "random", "chain"]
    batch = synth.make_batch(3, 0, sizes, hk=hk, hv=hv, kinds=kinds)
    check_against_oracle(batch, *run_gpu(batch, cuda, packed=True, records=records))


@pytest.mark.parametrize("records", [False, True], ids=["two_kernels", "mixed_kernel"])
def test_verify_split_order_empty_requests_and_slots(cuda, records):
    """A launch split by tree size, as two kernels or (with size-order
    records) as the mixed-width kernel: empty requests between the others,
    permuted state slots with a -1 (read from slot 0), trees on both sides of
    32 nodes.  Every request matches the oracle and reports status 0."""
    from dforktree_amd import ops, synth
    announce(f"verify split order: empty requests, slots, records={records}")
    sizes = [40, 12, 64, 33, 9, 17, 64, 1, 48]
    batch = synth.make_batch(23, 0, sizes, hk=2, hv=4, kinds=["random", "chain", "bushy"] * 3)
    empty_at = [1, 5, 9]  # positions of the empty requests in the launch
    order = []            # launch position -> index into sizes (None: empty)
    it = iter(range(len(sizes)))
    for pos in range(len(sizes) + len(empty_at)):
        order.append(None if pos in empty_at else next(it))
    lens = [0 if r is None else sizes[r] for r in order]
    cu = torch.zeros(len(order) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    pool = torch.randn(len(order) + 1, 4, 128, 128) * 0.02
    slots = torch.randperm(len(order) + 1)[:len(order)].to(torch.int32)
    slots[3] = -1
    batch.state = torch.stack([pool[max(int(slots[p]), 0)] for p, r in enumerate(order) if r is not None])
    g = batch.to(cuda)
    rows = g.y.shape[0]
    ts = ops.tree_struct(g.parent, 4, cu_seqlens=g.cu_seqlens, n_nodes=64, batch=batch.batch, want=("anc_bits",))
    aux_k = torch.zeros(4, rows, 128, device=cuda)
    aux_v = torch.zeros(4, rows, 128, device=cuda)
    aux_g = torch.zeros(4, rows, device=cuda)
    status = torch.full((len(order),), -5, device=cuda, dtype=torch.int32)
    cu_d = cu.to(cuda)
    so = ops.size_order(cu_d, 64) if records else None
    o = ops.tree_verify(g.y, g.a, g.b, g.A_log, g.dt_bias, pool.to(cuda).transpose(-1, -2), hk=2, hv=4,
                        anc_bits=ts["anc_bits"], cu_seqlens=cu_d, n_nodes=64, batch=len(order),
                        state_indices=slots.to(cuda), aux_k=aux_k, aux_v=aux_v, aux_g=aux_g, status=status,
                        size_order=so)
    torch.cuda.synchronize()
    assert status.tolist() == [0] * len(order)
    check_against_oracle(batch, o, aux_k, aux_v, aux_g)


@pytest.mark.parametrize("sizes", [[5, 32, 17, 1, 30, 9], [33, 64, 40, 48]], ids=["all_small", "all_large"])
def test_verify_mixed_kernel_one_class(cuda, sizes):
    """Size-order records of a batch whose trees are all on one side of 32
    nodes (launched at n_nodes 64): the mixed-width kernel then runs only
    v-head pairs on the 32-wide body, or only 64-wide items.  Against the
    oracle."""
    from dforktree_amd import synth
    announce(f"verify mixed kernel, one size class: {sizes}")
    batch = synth.make_batch(31, 0, sizes, hk=2, hv=4, kinds=["random", "chain", "bushy"] * 2)
    check_against_oracle(batch, *run_gpu(batch, cuda, packed=True, records=True, n_nodes=64))


def size_order_records(cu, n_nodes):
    """The records dft_size_order writes, restated on the host: the counts,
    n_nodes and batch, then (request, first row, span, 0) for the requests of at most 32 nodes
    (span clamped to [0, n_nodes]) from the front and the others from the
    back, each class in request order."""
    B = len(cu) - 1
    n = [min(max(cu[r + 1] - cu[r], 0), n_nodes) for r in range(B)]
    small = [r for r in range(B) if n[r] <= 32]
    large = [r for r in range(B) if n[r] > 32]
    recs = [None] * B
    for j, r in enumerate(small):
        recs[j] = [r, cu[r], cu[r + 1] - cu[r], 0]
    for j, r in enumerate(large):
        recs[B - 1 - j] = [r, cu[r], cu[r + 1] - cu[r], 0]
    return [[len(small), len(large), n_nodes, B]] + recs


def test_verify_size_order(cuda):
    """1100 packed requests of 0-64 nodes (two chunks of the ordering
    workgroup) launched at n_nodes 60, so that those past 60 are cut
    (DFT_STATUS_SPAN): the records equal the host restatement, and the split
    launch that reads them writes o, the saves and the status words bit for
    bit as the launch without them."""
    from dforktree_amd import ops, synth
    announce("verify with size-order records, 1100 requests")
    g = torch.Generator().manual_seed(17)
    B, hk, hv = 1100, 1, 1
    sizes = torch.randint(0, 65, (B,), generator=g).tolist()
    rows = sum(sizes)
    cu = [0]
    for n in sizes:
        cu.append(cu[-1] + n)
    y = torch.randn(rows, 2 * hk * 128 + hv * 128, generator=g).to(torch.bfloat16).to(cuda)
    a, b = torch.randn(rows, hv, generator=g).to(cuda), torch.randn(rows, hv, generator=g).to(cuda)
    parents = torch.cat([synth.tree_parents(n, "random", g) for n in sizes if n]).to(cuda)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=cuda)
    state = (torch.randn(B, hv, 128, 128, generator=g) * 0.02).to(cuda)
    A_log, dt_bias = torch.full((hv,), -0.69, device=cuda), torch.zeros(hv, device=cuda)
    bits = ops.tree_struct(parents, 4, cu_seqlens=cu_d, n_nodes=64, batch=B, want=("anc_bits",))["anc_bits"]
    order = ops.size_order(cu_d, 60)
    torch.cuda.synchronize()
    assert order.cpu().tolist() == size_order_records(cu, 60)
    outs = []
    for so in (None, order):
        aux = [torch.full((hv, rows, 128), -3.0, device=cuda), torch.full((hv, rows, 128), -3.0, device=cuda),
               torch.full((hv, rows), -3.0, device=cuda)]
        status = torch.full((B,), -7, device=cuda, dtype=torch.int32)
        o = torch.full((rows, hv, 128), -3.0, device=cuda, dtype=torch.bfloat16)  # the cut rows stay unwritten
        ops.tree_verify(y, a, b, A_log, dt_bias, state.transpose(-1, -2), hk=hk, hv=hv, anc_bits=bits,
                        cu_seqlens=cu_d, n_nodes=60, batch=B, o=o, aux_k=aux[0], aux_v=aux[1], aux_g=aux[2],
                        status=status, size_order=so)
        torch.cuda.synchronize()
        outs.append([o.view(torch.int16), *(t.view(torch.int32) for t in aux), status])
    assert outs[0][-1].cpu().tolist() == [1 if n > 60 else 0 for n in sizes]  # DFT_STATUS_SPAN: the cut ones
    for x, z in zip(*outs):
        assert torch.equal(x, z)


def test_verify_split_beyond_ordered_batch(cuda):
    """300 requests (more than the split launch orders): the kernels take
    their requests by block id, skipping the other kernel's."""
    from dforktree_amd import synth
    announce("verify split, 300 requests")
    g = torch.Generator().manual_seed(5)
    sizes = torch.randint(1, 49, (300,), generator=g).tolist()
    batch = synth.make_batch(29, 0, sizes, hk=1, hv=1, kinds=["random", "chain", "bushy"] * 100)
    check_against_oracle(batch, *run_gpu(batch, cuda, packed=True))


def test_verify_state_indices(cuda):
    """Slots are read on the device: permuted slots, and -1 clamps to slot 0."""
    from dforktree_amd import synth
    announce("verify state_indices")
    batch = synth.make_batch(4, 0, [32] * 3, hk=2, hv=4)
    pool = torch.randn(5, 4, 128, 128) * 0.02
    slots = torch.tensor([3, -1, 4], dtype=torch.int32)
    batch.state = pool[slots.clamp(min=0).long()]
    o, k, v, g = run_gpu(batch, cuda, state=pool.to(cuda), state_indices=slots.to(cuda))
    check_against_oracle(batch, o, k, v, g)


def test_tree_gdn_split_dropin(cuda):
    """tree_kernels.tree_gdn_split with the plugin's argument forms: pool view,
    slot on device, cached neg_exp_A, aux buffers [Hv, N, D]."""
    from dforktree_amd import synth
    from dforktree_amd.plugin import tree_kernels as TK
    announce("tree_gdn_split drop-in")
    batch = synth.make_batch(6, 0, [32], hk=2, hv=4)
    anc = torch.from_numpy(O.tree_struct(batch.parent.numpy())[0])
    pool = (torch.randn(3, 4, 128, 128) * 0.02)
    batch.state = pool[2:3]
    g = batch.to(cuda)
    poolg = pool.to(cuda)
    keys = torch.zeros(4, 32, 128, device=cuda)
    vals = torch.zeros_like(keys)
    gains = torch.zeros(4, 32, device=cuda)
    neg = -g.A_log.exp()
    o = TK.tree_gdn_split(g.y, g.a, g.b, g.A_log, g.dt_bias, poolg[0].transpose(-1, -2), anc.to(cuda), 2, 4, 128, 128,
                          aux=(keys, vals, gains), neg_exp_A=neg,
                          state_indices=torch.tensor([2], device=cuda, dtype=torch.int32),
                          state_slot_stride=poolg.stride(0))
    torch.cuda.synchronize()
    assert o.shape == (32, 4, 128) and o.dtype == torch.bfloat16
    check_against_oracle(batch, o, keys, vals, gains)
    with pytest.raises(KeyError):
        TK.tree_gdn_split(g.y[:20], g.a[:20], g.b[:20], g.A_log, g.dt_bias, poolg[0].transpose(-1, -2),
                          anc[:20, :20].to(cuda), 2, 4, 128, 128)


def test_tree_gdn_fused_dropin(cuda):
    """tree_gdn_fused returns fp32 and, for N > 32, delegates to the split path."""
    from dforktree_amd import synth
    from dforktree_amd.plugin import tree_kernels as TK
    announce("tree_gdn_fused drop-in")
    for n in (24, 64):
        batch = synth.make_batch(7, 0, [n], hk=2, hv=4)
        anc = torch.from_numpy(O.tree_struct(batch.parent.numpy())[0]).to(cuda)
        g = batch.to(cuda)
        o = TK.tree_gdn_fused(g.y, g.a, g.b, g.A_log, g.dt_bias, g.state[0].transpose(-1, -2), anc, 2, 4, 128, 128)
        torch.cuda.synchronize()
        ref = oracle_verify(batch)[0]
        if n <= 32:
            assert o.dtype == torch.float32
            assert rel_l2(np32(o), ref["o"]) <= 5e-5
        else:
            assert o.dtype == torch.bfloat16
            assert rel_l2(np32(o), O.bf16_round(ref["o"])) <= REL_L2


def test_block_inverse_dropin(cuda):
    from dforktree_amd.plugin import fc1_block_inverse as FBI
    import scipy.linalg
    announce("block inverse")
    rng = np.random.default_rng(0)
    for n, inv in ((16, FBI.invert16), (32, FBI.invert32), (64, FBI.invert64)):
        A = np.tril(rng.standard_normal((8, n, n)).astype(np.float32) * 0.2, -1)
        X = torch.from_numpy(A + np.triu(np.ones((n, n), np.float32), 0)[None] * 7.0).to(cuda)  # junk above
        inv[8,](X, n, num_warps=4, num_stages=1)
        torch.cuda.synchronize()
        Xh = X.cpu().numpy()
        for m in range(8):
            want = scipy.linalg.solve_triangular(np.eye(n) + A[m], np.eye(n), lower=True)
            assert np.abs(Xh[m] - want).max() <= 1e-5
            assert np.all(np.triu(Xh[m], 1) == 0)


@pytest.mark.parametrize("sizes_kind", ["uniform32", "ragged64"])
def test_verify_more_items_than_resident_workgroups(cuda, sizes_kind):
    """More (request, head) items than resident workgroups, so freed slots
    take further items (and a packed batch runs both size classes)."""
    from dforktree_amd import synth
    announce(f"verify more items than slots {sizes_kind}")
    if sizes_kind == "uniform32":
        sizes = [32] * 40          # 40 x 32 heads = 1280 items (> 4 per CU x 256 CUs)
        kinds = ["random", "chain", "bushy", "random"] * 10
    else:
        sizes, kinds = synth.ragged_sizes(12, 8, 64, seed=3)  # 384 items (> 1 per CU x 256)
    batch = synth.make_batch(9, 0, sizes, hk=16, hv=32, kinds=kinds)
    check_against_oracle(batch, *run_gpu(batch, cuda, packed=(sizes_kind != "uniform32"), use_bits=True))


def test_verify_ragged_32_many_items(cuda):
    """Packed trees of 1-32 nodes with ancestry bits and more items than
    resident workgroups of the 32-wide kernel."""
    from dforktree_amd import synth
    announce("verify ragged <=32 many items")
    sizes, kinds = synth.ragged_sizes(40, 1, 32, seed=11)
    batch = synth.make_batch(12, 0, sizes, hk=16, hv=32, kinds=kinds)
    check_against_oracle(batch, *run_gpu(batch, cuda, packed=True, use_bits=True))


def test_verify_uniform_many_items_dense_ancestry(cuda):
    """The same width with dense ancestry matrices: one item per workgroup."""
    from dforktree_amd import synth
    announce("verify uniform 32 many items dense")
    batch = synth.make_batch(13, 0, [32] * 40, hk=16, hv=32, kinds=["random", "chain", "bushy", "random"] * 10)
    check_against_oracle(batch, *run_gpu(batch, cuda, packed=False, use_bits=False))


def test_verify_bench_shape(cuda):
    """The measured shape: 64 requests of 32-node random trees at full width
    (2048 items, two generations of resident workgroups), against the oracle."""
    from dforktree_amd import synth
    announce("verify bench shape 64 x 32")
    batch = synth.make_batch(14, 0, [32] * 64, hk=16, hv=32, kinds="random")
    check_against_oracle(batch, *run_gpu(batch, cuda, packed=False, use_bits=True))


@pytest.mark.parametrize("records", [False, True], ids=["two_kernels", "mixed_kernel"])
def test_verify_ragged_bench_shape(cuda, records):
    """The measured ragged batch at full size: 128 packed requests with trees
    of 8-64 nodes (chains, bushy and random thirds), 4507 nodes at full
    width, against the oracle: without size-order records as two kernels
    (64- and 32-wide), with them as the one mixed-width kernel (its 32-wide
    items in v-head pairs, two per workgroup)."""
    from dforktree_amd import synth
    announce(f"verify ragged bench shape 128 x 8-64 records={records}")
    sizes, kinds = synth.ragged_sizes(128, 8, 64, seed=3)
    batch = synth.make_batch(15, 0, sizes, hk=16, hv=32, kinds=kinds)
    check_against_oracle(batch, *run_gpu(batch, cuda, packed=True, use_bits=True, records=records))


def test_verify_kmajor_state_element_loads(cuda):
    """A k-major state ([hv, dk, dv] contiguous, v stride 1) takes the
    element-load path of the kernel; same results."""
    from dforktree_amd import synth
    announce("verify k-major state")
    batch = synth.make_batch(8, 0, [32, 17], hk=2, hv=4, kinds=["random", "chain"])
    st = batch.state.transpose(-1, -2).contiguous()           # [B, hv, K, V]
    o, k, v, g = run_gpu(batch, cuda, state=st.to(cuda).transpose(-1, -2), packed=True)
    check_against_oracle(batch, o, k, v, g)


def test_verify_kmajor_state_64_wide_split(cuda):
    """Element loads on the 64-wide kernel (late v rows, o staged in X) and
    the size split: a packed batch whose trees straddle 32 nodes."""
    from dforktree_amd import synth
    announce("verify k-major state, 64-wide split")
    batch = synth.make_batch(18, 0, [64, 9, 40, 33, 32, 1], hk=2, hv=4,
                             kinds=["chain", "random", "bushy", "random", "chain", "random"])
    st = batch.state.transpose(-1, -2).contiguous()
    o, k, v, g = run_gpu(batch, cuda, state=st.to(cuda).transpose(-1, -2), packed=True)
    check_against_oracle(batch, o, k, v, g)


@pytest.mark.parametrize("o_dtype", [torch.bfloat16, torch.float32])
def test_verify_64_wide_output_forms(cuda, o_dtype):
    """The 64-wide kernel with staged bf16 output (o staged in X) and with
    direct fp32 stores, trees of 33-64 nodes only."""
    from dforktree_amd import synth
    announce(f"verify 64-wide {o_dtype}")
    batch = synth.make_batch(19, 0, [64, 48, 33, 57], hk=2, hv=4, kinds=["random", "chain", "bushy", "random"])
    o, k, v, g = run_gpu(batch, cuda, o_dtype=o_dtype, packed=True)
    check_against_oracle(batch, o, k, v, g, o_bf16=(o_dtype == torch.bfloat16))


@pytest.mark.parametrize("case", ["b1_fp32_dense", "b4_packed_slots", "b5_one_workgroup"])
def test_verify_64_wide_column_split(cuda, case):
    """Launches over 32 nodes with at most 128 (request, v-head) items run
    each item on two workgroups (value columns split, state k halves split
    over wave pairs): batch 1 and 4 at full width (32 v-heads) take that
    form, batch 5 (160 items) the one-workgroup kernel.  fp32 output is held
    to 5e-5, as the one-workgroup kernel is."""
    from dforktree_amd import synth
    announce(f"verify 64-wide column split {case}")
    if case == "b1_fp32_dense":
        batch = synth.make_batch(21, 0, [64], hk=16, hv=32, kinds="random")
        o, k, v, g = run_gpu(batch, cuda, o_dtype=torch.float32)
        ref = oracle_verify(batch)[0]
        assert rel_l2(np32(o), ref["o"]) <= 5e-5
        assert rel_l2(np32(v), ref["vn"]) <= 5e-5
        check_against_oracle(batch, o, k, v, g, o_bf16=False)
    elif case == "b4_packed_slots":
        batch = synth.make_batch(22, 0, [64, 40, 9, 33], hk=16, hv=32, kinds=["chain", "random", "bushy", "random"])
        pool = torch.randn(6, 32, 128, 128) * 0.02
        slots = torch.tensor([5, 0, -1, 2], dtype=torch.int32)
        batch.state = pool[slots.clamp(min=0).long()]
        o, k, v, g = run_gpu(batch, cuda, packed=True, state=pool.to(cuda), state_indices=slots.to(cuda))
        check_against_oracle(batch, o, k, v, g)
    else:
        batch = synth.make_batch(23, 0, [48] * 5, hk=16, hv=32, kinds=["random", "chain", "bushy", "random", "chain"])
        check_against_oracle(batch, *run_gpu(batch, cuda, use_bits=True))


def test_verify_fp16_gates_and_output(cuda):
    """fp16 gate inputs a, b and an fp16 output o (DFT_F16 operands): the
    oracle takes the same fp16-rounded a, b; o is compared after fp16
    rounding of the oracle's output."""
    from dforktree_amd import ops, synth
    announce("verify fp16 a/b/o")
    batch = synth.make_batch(12, 0, [32, 32], hk=2, hv=4, kinds=["random", "bushy"])
    batch.a, batch.b = batch.a.half(), batch.b.half()
    g = batch.to(cuda)
    ts = ops.tree_struct(g.parent, 4, batch=2, n_nodes=32, want=("anc_bits",))
    vn = torch.zeros(4, 64, 128, device=cuda)
    o = ops.tree_verify(g.y, g.a, g.b, g.A_log, g.dt_bias, g.state.transpose(-1, -2), hk=2, hv=4,
                        anc_bits=ts["anc_bits"], batch=2, n_nodes=32, o_dtype=torch.float16, aux_v=vn)
    torch.cuda.synchronize()
    assert o.dtype == torch.float16
    ref = oracle_verify(batch)  # np32 of the fp16 a, b: the values the kernel reads
    for r, sl in enumerate(request_slices(batch)):
        want = ref[r]["o"].astype(np.float16).astype(np.float32)
        assert rel_l2(np32(o[sl]), want) <= REL_L2 and max_abs(np32(o[sl]), want) <= MAX_ABS_BF16, r
        assert rel_l2(np32(vn[:, sl]), ref[r]["vn"]) <= REL_L2, r


def test_conv_then_verify_config1_chain(cuda):
    """The full verify front end at batch 32 (32-node random trees, 16 q/k
    heads, 32 v heads, C = 8192): the tree conv (width 4, SiLU, zero state at
    the root, bf16 weights N(0, 0.1)) writes the y that the verify reads,
    checked against the oracle chain O.tree_conv -> bf16 -> tree_gdn_split."""
    from dforktree_amd import ops, synth
    announce("conv -> verify chain, config1 (batch 32, full width)")
    B, N, HK, HV, C = 32, 32, 16, 32, 8192
    batch = synth.make_batch(1, 0, [N] * B, hk=HK, hv=HV)  # a, b, S0, trees; y is replaced by the conv output
    g = torch.Generator().manual_seed(101)
    x = torch.randn(B * N, C, generator=g).to(torch.bfloat16)
    w = (torch.randn(C, 4, generator=g) * 0.1).to(torch.bfloat16)
    cs = torch.zeros(B, C, 3, dtype=torch.bfloat16)
    gb = batch.to(cuda)
    ts = ops.tree_struct(gb.parent, 4, batch=B, n_nodes=N, want=("anc_bits", "cidx"))
    y = ops.tree_conv(x.view(B, N, C).to(cuda), cs.to(cuda), w.to(cuda), None, ts["cidx"].view(B, N, 4))
    o = ops.tree_verify(y.view(B * N, C), gb.a, gb.b, gb.A_log, gb.dt_bias, gb.state.transpose(-1, -2), hk=HK, hv=HV,
                        anc_bits=ts["anc_bits"], batch=B, n_nodes=N)
    torch.cuda.synchronize()
    # the oracle chain
    ys = []
    for r, sl in enumerate(request_slices(batch)):
        cidx = O.tree_struct(batch.parent[sl].numpy(), 4)[2]
        ry, _ = O.tree_conv(np32(x[sl]), np32(cs[r]), np32(w), None, cidx)
        ys.append(torch.from_numpy(O.bf16_round(ry)).to(torch.bfloat16))
    batch.y = torch.cat(ys)
    yd = np32(y.view(B * N, C))
    assert max_abs(yd, np32(batch.y)) <= MAX_ABS_BF16, "conv output"
    ref = oracle_verify(batch)
    oh = np32(o)
    for r, sl in enumerate(request_slices(batch)):
        want = O.bf16_round(ref[r]["o"])
        assert rel_l2(oh[sl], want) <= REL_L2 and max_abs(oh[sl], want) <= MAX_ABS_BF16, f"request {r}"


def test_verify_misaligned_y_is_copied(cuda):
    """A y view that is contiguous but not 16-byte aligned (an odd element
    offset) is copied into an aligned buffer first: same outputs as the
    aligned y."""
    from dforktree_amd import ops, synth
    announce("verify misaligned y")
    batch = synth.make_batch(13, 0, [32, 32], hk=2, hv=4)
    g = batch.to(cuda)
    rows, C = g.y.shape
    big = torch.zeros(rows * C + 1, device=cuda, dtype=torch.bfloat16)
    ym = big[1:].view(rows, C)
    ym.copy_(g.y)
    assert ym.data_ptr() % 16 != 0 and ym.is_contiguous()
    ts = ops.tree_struct(g.parent, 4, batch=2, n_nodes=32, want=("anc_bits",))
    kw = dict(hk=2, hv=4, anc_bits=ts["anc_bits"], batch=2, n_nodes=32)
    o1 = ops.tree_verify(ym, g.a, g.b, g.A_log, g.dt_bias, g.state.transpose(-1, -2), **kw)
    o2 = ops.tree_verify(g.y, g.a, g.b, g.A_log, g.dt_bias, g.state.transpose(-1, -2), **kw)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
