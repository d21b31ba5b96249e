"""GPU parity of the tree-structure and tree-conv kernels.

Integer outputs (ancestor bits, Anc, depth, cidx, nxt/sib, the conv window
gathers) are compared bit for bit; the conv output is bf16, compared within
max-abs 1e-2 and rel-L2 2e-3 of the fp32 oracle.
"""
import numpy as np
import pytest
import torch

from conftest import MAX_ABS_BF16, REL_L2, announce, max_abs, rel_l2
from _ref import np32
from oracle import gdn_tree as O

pytestmark = pytest.mark.gpu


def _trees(seed):
    from dforktree_amd import synth
    g = torch.Generator().manual_seed(seed)
    sizes = [1, 2, 16, 31, 32, 33, 50, 64, 64, 64, 7, 40]
    kinds = ["random", "chain", "bushy", "random", "chain", "random", "bushy", "chain", "random", "bushy",
             "random", "chain"]
    return sizes, [synth.tree_parents(n, k, g) for n, k in zip(sizes, kinds)]


def test_tree_struct_packed_exact(cuda):
    from dforktree_amd import ops
    announce("tree_struct packed")
    sizes, pars = _trees(0)
    cu = torch.zeros(len(sizes) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(sizes), 0)
    r = ops.tree_struct(torch.cat(pars).to(cuda), 4, cu_seqlens=cu.to(cuda), n_nodes=64, batch=len(sizes))
    torch.cuda.synchronize()
    bits = r["anc_bits"].cpu().numpy().view(np.uint64)
    for i, (n, p) in enumerate(zip(sizes, pars)):
        sl = slice(int(cu[i]), int(cu[i + 1]))
        anc, depth, cidx = O.tree_struct(p.numpy())
        nxt, sib = O.tree_links(p.numpy())
        assert np.array_equal(bits[sl], O.anc_bits(anc)), f"tree {i}"
        assert np.array_equal(r["anc"][i, :n, :n].cpu().numpy(), anc)
        assert np.array_equal(r["depth"][sl].cpu().numpy(), depth)
        assert np.array_equal(r["cidx"][sl].cpu().numpy(), cidx)
        assert np.array_equal(r["nxt"][sl].cpu().numpy(), nxt)
        assert np.array_equal(r["sib"][sl].cpu().numpy(), sib)
        assert int(r["status"][i]) == 0


def test_tree_struct_status_flags(cuda):
    from dforktree_amd import ops
    announce("tree_struct status")
    bad = torch.tensor([[-1, 0, 3, 1], [-1, 0, 1, 2], [-1, 2, 3, 1]], dtype=torch.int32)
    r = ops.tree_struct(bad.to(cuda), 4, want=("anc_bits", "status"))
    torch.cuda.synchronize()
    assert r["status"].cpu().tolist() == [1, 0, 2]


def test_builder_tree_struct_matches_reference_closure(cuda):
    """builder.tree_struct (the opt-in for tree_ops.tree_struct) == the
    reference's squaring closure for N <= 32."""
    from dforktree_amd import builder, synth
    announce("builder.tree_struct")
    g = torch.Generator().manual_seed(1)
    for kind in ("random", "chain", "bushy"):
        p = synth.tree_parents(32, kind, g)
        anc, depth, cidx = builder.tree_struct(p.to(cuda).long(), 4)
        ra, rd, rc = O.tree_struct_squaring(p.numpy(), 4)
        assert anc.dtype == torch.float32 and depth.dtype == torch.int64 and cidx.dtype == torch.int64
        assert np.array_equal(anc.cpu().numpy(), ra)
        assert np.array_equal(depth.cpu().numpy(), rd)
        assert np.array_equal(cidx.cpu().numpy(), rc)


def _conv_inputs(seed, B, N, C, slots=None):
    from dforktree_amd import synth
    g = torch.Generator().manual_seed(seed)
    pars = [synth.tree_parents(N, k, g) for k in (["random", "chain", "bushy"] * B)[:B]]
    x = torch.randn(B, N, C, generator=g).to(torch.bfloat16)
    w = (torch.randn(C, 4, generator=g) * 0.1).to(torch.bfloat16)
    cs = torch.randn(slots or B, C, 3, generator=g).to(torch.bfloat16)
    cidx = torch.stack([torch.from_numpy(O.tree_struct(p.numpy())[2]) for p in pars]).int()
    return x, w, cs, cidx


def test_conv_config1_shapes(cuda):
    """Batch 32, 32-node trees, C = 8192, width 4, SiLU, zero state at the root."""
    from dforktree_amd import ops
    announce("conv config1")
    B, N, C = 32, 32, 8192
    x, w, cs, cidx = _conv_inputs(1, B, N, C)
    cs.zero_()
    iw = torch.zeros(B, N, C, 3, dtype=torch.bfloat16, device=cuda)
    y = ops.tree_conv(x.to(cuda), cs.to(cuda), w.to(cuda), None, cidx.to(cuda), iw=iw)
    torch.cuda.synchronize()
    yh, iwh = np32(y), np32(iw)
    for b in range(B):
        ry, rwin = O.tree_conv(np32(x[b]), np32(cs[b]), np32(w), None, cidx[b].numpy())
        want = O.bf16_round(ry)
        assert max_abs(yh[b], want) <= MAX_ABS_BF16 and rel_l2(yh[b], want) <= REL_L2
        assert np.array_equal(iwh[b], rwin), "window gathers must be bit-exact"


def test_conv_slots_bias_and_state(cuda):
    """Nonzero conv_state read through device slot indices, bias, and the
    window written to a different destination slot."""
    from dforktree_amd import ops
    announce("conv slots bias")
    B, N, C = 3, 32, 1000
    x, w, cs, cidx = _conv_inputs(2, B, N, C, slots=5)
    bias = torch.randn(C).to(torch.bfloat16)
    slots = torch.tensor([4, 0, 2], dtype=torch.int32)
    dsts = torch.tensor([1, 3, 0], dtype=torch.int64)
    iw = torch.zeros(4, N, C, 3, dtype=torch.bfloat16, device=cuda)
    y = ops.tree_conv(x.to(cuda), cs.to(cuda), w.to(cuda), bias.to(cuda), cidx.to(cuda), cs_indices=slots.to(cuda),
                      iw=iw, iw_indices=dsts.to(cuda))
    torch.cuda.synchronize()
    for b in range(B):
        ry, rwin = O.tree_conv(np32(x[b]), np32(cs[int(slots[b])]), np32(w), np32(bias), cidx[b].numpy())
        assert max_abs(np32(y[b]), O.bf16_round(ry)) <= MAX_ABS_BF16
        assert np.array_equal(np32(iw[int(dsts[b])]), rwin)


def test_tree_conv_fused_dropin(cuda):
    """tree_kernels.tree_conv_fused: 2-D conv_state [C, T], mixed0 [N, C]."""
    from dforktree_amd.plugin import tree_kernels as TK
    announce("tree_conv_fused drop-in")
    N, C = 32, 512
    x, w, cs, cidx = _conv_inputs(3, 1, N, C)
    bias = torch.randn(C).to(torch.bfloat16)
    cs2 = torch.randn(C, 5).to(torch.bfloat16)  # T = 5 columns, only the first 3 are read
    y = TK.tree_conv_fused(cs2.to(cuda), x[0].to(cuda), cidx[0].long().to(cuda), w.to(cuda), bias.to(cuda))
    torch.cuda.synchronize()
    ry, _ = O.tree_conv(np32(x[0]), np32(cs2), np32(w), np32(bias), cidx[0].numpy())
    assert y.shape == (N, C) and y.dtype == torch.bfloat16
    assert max_abs(np32(y), O.bf16_round(ry)) <= MAX_ABS_BF16


@pytest.mark.parametrize("case", ["f32_weight", "odd_channels", "fp32_state", "int64_cidx"])
def test_conv_general_layouts(cuda, case):
    """Layouts outside the 16-byte bf16 fast path (fp32 weights, a channel
    count that is not a multiple of 8), an fp32 conv state and 64-bit gather
    indices on the fast path: same results, window values rounded to the
    window's dtype."""
    from dforktree_amd import ops
    announce(f"conv general layout {case}")
    B, N = 2, 32
    C = 1003 if case == "odd_channels" else 1024
    x, w, cs, cidx = _conv_inputs(4, B, N, C)
    if case == "f32_weight":
        w = w.float()
    if case == "fp32_state":
        cs = torch.randn(B, C, 3) * 0.5
    if case == "int64_cidx":
        cidx = cidx.long()
    iw = torch.zeros(B, N, C, 3, dtype=torch.bfloat16, device=cuda)
    y = ops.tree_conv(x.to(cuda), cs.to(cuda), w.to(cuda), None, cidx.to(cuda), iw=iw)
    torch.cuda.synchronize()
    for b in range(B):
        ry, rwin = O.tree_conv(np32(x[b]), np32(cs[b]), np32(w), None, cidx[b].numpy())
        want = O.bf16_round(ry)
        assert max_abs(np32(y[b]), want) <= MAX_ABS_BF16 and rel_l2(np32(y[b]), want) <= REL_L2
        assert np.array_equal(np32(iw[b]), O.bf16_round(rwin))


@pytest.mark.parametrize("width", [2, 3, 5, 8])
def test_conv_other_widths(cuda, width):
    """The general-width conv (tree_kernels.py:17-33 takes any KC): the
    tree's gather columns for `width` taps (tree_ops.py:81-88), through
    ops.tree_conv over a batch (window included) and through the drop-in
    tree_conv_fused, against the oracle."""
    from dforktree_amd import ops, synth
    from dforktree_amd.plugin import tree_kernels as TK
    announce(f"conv width {width}")
    B, N, C = 3, 32, 1024
    g = torch.Generator().manual_seed(60 + width)
    pars = [synth.tree_parents(N, k, g) for k in ("random", "chain", "bushy")]
    x = torch.randn(B, N, C, generator=g).to(torch.bfloat16)
    w = (torch.randn(C, width, generator=g) * 0.1).to(torch.bfloat16)
    cs = torch.randn(B, C, max(width - 1, 1), generator=g).to(torch.bfloat16)
    bias = torch.randn(C, generator=g).to(torch.bfloat16)
    cidx = torch.stack([torch.from_numpy(O.tree_struct(p.numpy(), width)[2]) for p in pars])  # int64
    iw = torch.zeros(B, N, C, width - 1, dtype=torch.bfloat16, device=cuda)
    y = ops.tree_conv(x.to(cuda), cs.to(cuda), w.to(cuda), bias.to(cuda), cidx.to(cuda), iw=iw)
    y1 = TK.tree_conv_fused(cs[0].to(cuda), x[0].to(cuda), cidx[0].to(cuda), w.to(cuda), bias.to(cuda))
    torch.cuda.synchronize()
    for b in range(B):
        ry, rwin = O.tree_conv(np32(x[b]), np32(cs[b]), np32(w), np32(bias), cidx[b].numpy())
        want = O.bf16_round(ry)
        assert max_abs(np32(y[b]), want) <= MAX_ABS_BF16 and rel_l2(np32(y[b]), want) <= REL_L2, b
        assert np.array_equal(np32(iw[b]), rwin), "window gathers must be bit-exact"
        if b == 0:
            assert max_abs(np32(y1), want) <= MAX_ABS_BF16 and rel_l2(np32(y1), want) <= REL_L2


@pytest.mark.parametrize("layout", ["fast", "general"])
def test_conv_negative_slots(cuda, layout):
    """A negative conv-state slot (a padded request) reads slot 0, and a
    negative window slot writes no window: every window slot keeps what it
    held except the ones the valid requests own."""
    from dforktree_amd import ops
    announce(f"conv negative slots ({layout})")
    B, N, C = 3, 32, 1024
    x, w, cs, cidx = _conv_inputs(7, B, N, C, slots=3)
    if layout == "general":
        w = w.float()
    slots = torch.tensor([2, -1, 0], dtype=torch.int32)
    dsts = torch.tensor([1, -1, 2], dtype=torch.int32)
    iw = torch.full((4, N, C, 3), 5.0, dtype=torch.bfloat16, device=cuda)
    y = ops.tree_conv(x.to(cuda), cs.to(cuda), w.to(cuda), None, cidx.to(cuda), cs_indices=slots.to(cuda), iw=iw,
                      iw_indices=dsts.to(cuda))
    torch.cuda.synchronize()
    got = np32(iw)
    for b in range(B):
        ry, rwin = O.tree_conv(np32(x[b]), np32(cs[max(int(slots[b]), 0)]), np32(w), None, cidx[b].numpy())
        assert max_abs(np32(y[b]), O.bf16_round(ry)) <= MAX_ABS_BF16, b
        if int(dsts[b]) >= 0:
            assert np.array_equal(got[int(dsts[b])], rwin), b
    for untouched in (0, 3):
        assert np.all(got[untouched] == 5.0), f"window slot {untouched} was written"


@pytest.mark.parametrize("n", [1, 20, 32, 64])
def test_anc_pack_matches_oracle_bits(cuda, n):
    """dft_anc_pack: the dense ancestry (as tree_struct / the builder give it)
    packed into bit rows, bit-exact against the oracle's rows (bit 63 is the
    sign bit of the int64 row at n = 64); a batch of three trees at once."""
    from dforktree_amd import ops, synth
    announce(f"anc_pack n={n}")
    g = torch.Generator().manual_seed(90 + n)
    pars = [synth.tree_parents(n, k, g) for k in ("random", "chain", "bushy")]
    dense = np.stack([O.tree_struct(p.numpy())[0] for p in pars]).astype(np.float32)
    want = np.concatenate([O.anc_bits(d) for d in dense]).view(np.int64)
    got = ops.anc_pack(torch.from_numpy(dense).to(cuda))
    one = ops.anc_pack(torch.from_numpy(dense[1]).to(cuda))
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), want)
    assert np.array_equal(one.cpu().numpy(), want[n:2 * n])
