"""GPU: every entry point on the path replayed from a captured HIP graph.

The plugin's hooks run under graph capture, so the whole per-step sequence
(tree structure, conv, verify, the fused commit -> verify, the separate
commit, the standalone inverse, the packed masks) is captured once and
replayed three times.  Between replays the program does eager work of its
own: the state pools and the in-place inverse input are restored, every
output is refilled with a sentinel, an unrelated product runs, and the
device synchronises.  Every replay must reproduce the eager launch bit for
bit: the kernels use no atomics and no data-dependent reduction order, so
an eager run and a replay of the same launches agree exactly.
"""
import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu

P = 16
SENTINEL = {torch.float32: -3.0, torch.bfloat16: -3.0, torch.uint8: 0xA5, torch.int32: -7, torch.int64: -7}


def _paths(parent, cu, gen):
    """Accepted root-to-node walks, -1 padded to P columns, and their lengths."""
    from dforktree_amd import synth
    B = cu.numel() - 1
    idx = torch.full((B, P), -1, dtype=torch.int32)
    lens = torch.zeros(B, dtype=torch.int32)
    for r in range(B):
        w = synth.accepted_path(parent[int(cu[r]):int(cu[r + 1])], P, gen)
        idx[r, :len(w)] = w
        lens[r] = len(w)
    return idx, lens


class Step:
    """Inputs, in-place buffers and outputs of one step over a batch of trees."""

    def __init__(self, cuda, sizes, packed, seed):
        from dforktree_amd import synth
        kinds = ["random", "chain", "bushy"] * ((len(sizes) + 2) // 3)
        b1 = synth.make_batch(seed, 0, sizes, hk=2, hv=4, kinds=kinds[:len(sizes)])
        b2 = synth.make_batch(seed + 1, 0, sizes, hk=2, hv=4, kinds=kinds[::-1][:len(sizes)])
        self.packed, self.B, self.N, self.hk, self.hv = packed, b1.batch, b1.n_max, 2, 4
        self.g1, self.g2 = b1.to(cuda), b2.to(cuda)
        rows = self.g1.y.shape[0]
        gen = torch.Generator().manual_seed(seed + 2)
        idx, lens = _paths(b1.parent, b1.cu_seqlens, gen)
        self.idx, self.lens = idx.to(cuda), lens.to(cuda)
        idx2, _ = _paths(b2.parent, b2.cu_seqlens, gen)
        self.idx2 = idx2.to(cuda)
        # in-place inputs and their originals
        self.pool0 = self.g1.state.clone()                    # [B, hv, V, K]
        self.pool = self.pool0.clone()                        # fused commit -> verify
        self.rpool = self.pool0.clone()                       # the same with raw key rows
        self.vpool = self.pool0.clone()                       # raw key rows, recomputed values
        self.cpool0 = self.g1.state.clone().unsqueeze(0)      # [L=1, B, hv, V, K], separate commit
        self.cpool = self.cpool0.clone()
        n = 48
        a = torch.randn(6, n, n, generator=gen).tril(-1) * 0.3
        self.inv0 = a.to(cuda)
        self.inv = self.inv0.clone()
        self.plen = torch.tensor([0, 5, 64, 4096, 7, 100, 33, 1][:self.B], dtype=torch.int32).to(cuda)
        self.bits = (torch.rand(3 * 1000 + 13, generator=gen) < 0.4).to(cuda)
        self.cx = torch.randn(self.B, self.N, 2 * 2 * 128 + 4 * 128, generator=gen).to(torch.bfloat16).to(cuda)
        self.cw = (torch.randn(self.cx.shape[-1], 4, generator=gen) * 0.1).to(torch.bfloat16).to(cuda)
        self.cs = (torch.randn(self.B, self.cx.shape[-1], 3, generator=gen)).to(torch.bfloat16).to(cuda)
        # outputs (refilled with a sentinel before every run)
        f32 = dict(device=cuda, dtype=torch.float32)
        mask_bytes = sum((s * (int(p) + s) + 7) // 8 for s, p in zip(sizes, self.plen.tolist()))
        self.out = dict(
            o1=torch.empty(rows, 4, 128, device=cuda, dtype=torch.bfloat16),
            o2=torch.empty(rows, 4, 128, device=cuda, dtype=torch.bfloat16),
            k1=torch.empty(4, rows, 128, **f32), v1=torch.empty(4, rows, 128, **f32), G1=torch.empty(4, rows, **f32),
            k2=torch.empty(2, rows, 128, **f32), v2=torch.empty(4, rows, 128, **f32), G2=torch.empty(4, rows, **f32),
            o3=torch.empty(rows, 4, 128, device=cuda, dtype=torch.bfloat16),
            v3=torch.empty(4, rows, 128, **f32), G3=torch.empty(4, rows, **f32),
            o4=torch.empty(rows, 4, 128, device=cuda, dtype=torch.bfloat16), G4=torch.empty(4, rows, **f32),
            y=torch.empty_like(self.cx), iw=torch.empty(*self.cx.shape, 3, device=cuda, dtype=torch.bfloat16),
            mask=torch.empty(mask_bytes, device=cuda, dtype=torch.uint8),
            mind=torch.empty(self.B + 1, device=cuda, dtype=torch.int32),
            pb=torch.empty((self.bits.numel() + 7) // 8, device=cuda, dtype=torch.uint8),
            so1=torch.empty(self.B + 1, 4, device=cuda, dtype=torch.int32),
            so2=torch.empty(self.B + 1, 4, device=cuda, dtype=torch.int32),
        )

    def reset(self):
        self.pool.copy_(self.pool0)
        self.rpool.copy_(self.pool0)
        self.vpool.copy_(self.pool0)
        self.cpool.copy_(self.cpool0)
        self.inv.copy_(self.inv0)
        for t in self.out.values():
            t.fill_(SENTINEL[t.dtype])

    def shape_kw(self, g, order=None):
        kw = dict(batch=self.B, n_nodes=self.N)
        if self.packed:
            kw["cu_seqlens"] = g.cu_seqlens
            if order is not None:  # the packed step's size-order records (written by run)
                kw["size_order"] = order
        return kw

    def run(self):
        """The step's launches; returns the tree-structure outputs (fresh tensors)."""
        from dforktree_amd import ops
        o, g1, g2 = self.out, self.g1, self.g2
        sk = dict(cu_seqlens=g1.cu_seqlens) if self.packed else {}
        ts1 = ops.tree_struct(g1.parent, 4, batch=self.B, n_nodes=self.N, want=("anc_bits", "cidx", "depth"),
                              index_dtype=torch.int32, **sk)
        ts2 = ops.tree_struct(g2.parent, 4, batch=self.B, n_nodes=self.N, want=("anc_bits",),
                              **(dict(cu_seqlens=g2.cu_seqlens) if self.packed else {}))
        if not self.packed:
            cidx = ts1["cidx"].view(self.B, self.N, 4)
            ops.tree_conv(self.cx, self.cs, self.cw, None, cidx, y=o["y"], iw=o["iw"])
        else:
            ops.size_order(g1.cu_seqlens, self.N, out=o["so1"])
            ops.size_order(g2.cu_seqlens, self.N, out=o["so2"])
        st = self.pool.transpose(-1, -2)
        ops.tree_verify(g1.y, g1.a, g1.b, g1.A_log, g1.dt_bias, st, hk=2, hv=4, anc_bits=ts1["anc_bits"],
                        o=o["o1"], aux_k=o["k1"], aux_v=o["v1"], aux_g=o["G1"], **self.shape_kw(g1, o["so1"]))
        prev = dict(prev_cu_seqlens=g1.cu_seqlens) if self.packed else dict(prev_n_nodes=self.N)
        ops.tree_commit_verify(g2.y, g2.a, g2.b, g2.A_log, g2.dt_bias, st, hk=2, hv=4, anc_bits=ts2["anc_bits"],
                               pending_path=self.idx, pending_keys=o["k1"], pending_values=o["v1"],
                               pending_gains=o["G1"], pending_path_len=self.lens, o=o["o2"], aux_k=o["k2"],
                               aux_v=o["v2"], aux_g=o["G2"], aux_k_per_khead=True, **prev,
                               **self.shape_kw(g2, o["so2"]))
        # the fused entry again, its keys normalised from step 1's raw k rows
        ops.tree_commit_verify(g2.y, g2.a, g2.b, g2.A_log, g2.dt_bias, self.rpool.transpose(-1, -2), hk=2, hv=4,
                               anc_bits=ts2["anc_bits"], pending_path=self.idx, pending_keys=None,
                               pending_key_rows=g1.y[:, 256:512].unflatten(1, (2, 128)), pending_values=o["v1"],
                               pending_gains=o["G1"], pending_path_len=self.lens, pending_k_head_div=2, o=o["o3"],
                               aux_v=o["v3"], aux_g=o["G3"], **prev, **self.shape_kw(g2))
        # and with the path's values recomputed from step 1's raw v rows and b gates (vpool holds the
        # state step 1 read)
        ops.tree_commit_verify(g2.y, g2.a, g2.b, g2.A_log, g2.dt_bias, self.vpool.transpose(-1, -2), hk=2, hv=4,
                               anc_bits=ts2["anc_bits"], pending_path=self.idx, pending_keys=None,
                               pending_key_rows=g1.y[:, 256:512].unflatten(1, (2, 128)), pending_values=None,
                               pending_value_rows=g1.y[:, 512:].unflatten(1, (4, 128)), pending_b=g1.b,
                               pending_gains=o["G1"], pending_path_len=self.lens, pending_k_head_div=2, o=o["o4"],
                               aux_g=o["G4"], **prev, **self.shape_kw(g2, o["so2"]))
        ops.tree_commit(self.cpool, o["k2"][None], o["v2"][None], o["G2"][None], self.idx2, n_nodes=self.N,
                        k_head_div=2, **(dict(cu_seqlens=g2.cu_seqlens) if self.packed else {}))
        ops.block_inverse_(self.inv)
        ops.tree_mask_pack(ts1["anc_bits"], self.plen, out=o["mask"], out_indptr=o["mind"], **self.shape_kw(g1))
        ops.packbits(self.bits, "little", out=o["pb"])
        return ts1

    def snapshot(self, ts):
        got = {k: t.clone() for k, t in self.out.items()}
        got.update(pool=self.pool.clone(), rpool=self.rpool.clone(), vpool=self.vpool.clone(), cpool=self.cpool.clone(),
                   inv=self.inv.clone())
        got.update({f"ts_{k}": v.clone() for k, v in ts.items()})
        return got


def _bits(t):
    if t.dtype == torch.float32:
        return t.view(torch.int32)
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16)
    return t


def _replays(cuda, step):
    step.reset()
    torch.cuda.synchronize()
    want = step.snapshot(step.run())
    torch.cuda.synchronize()
    for name in ("o1", "o2", "o3", "o4", "k2", "mask", "pb"):
        assert not torch.equal(want[name], torch.full_like(want[name], SENTINEL[want[name].dtype])), name
    assert not torch.equal(want["pool"], step.pool0) and not torch.equal(want["cpool"], step.cpool0)
    assert not torch.equal(want["vpool"], step.pool0)

    # capture on a side stream after one warm-up there, as torch.cuda.graph requires
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step.reset()
        step.run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    step.reset()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ts = step.run()
    torch.cuda.synchronize()

    other = torch.randn(512, 512, device=cuda)
    for rep in range(3):
        step.reset()
        other = other @ other.T / 512.0  # eager work of the program's own between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = step.snapshot(ts)
        for name, w in want.items():
            assert torch.equal(_bits(got[name]), _bits(w)), f"replay {rep}: {name} differs from the eager run"


def test_graph_replay_uniform(cuda):
    announce("graph replay: uniform 4 x 32, every entry point")
    _replays(cuda, Step(cuda, [32] * 4, packed=False, seed=70))


def test_graph_replay_packed_ragged(cuda):
    """Both size classes (the 64-wide and 32-wide kernels) in one capture."""
    announce("graph replay: packed ragged 8 requests, 1-64 nodes")
    _replays(cuda, Step(cuda, [40, 9, 64, 17, 33, 1, 20, 64], packed=True, seed=80))
