"""A seeded sweep of verify configurations against the oracle: head counts
and GQA ratios, tree sizes 1-64 across the 32/64-wide split, tree shapes,
packed and uniform batches, bf16 / fp32 outputs, ancestry as bits or dense
matrices, and a commit of each case's accepted paths.  Every case is printed
before it runs; tolerances as the rest of the suite (rel-L2 2e-3, max-abs
1e-2 on bf16 outputs)."""
import numpy as np
import pytest
import torch

from conftest import REL_L2, announce, rel_l2
from _ref import np32, oracle_verify, request_slices
from oracle import gdn_tree as O
from test_gpu_verify import check_against_oracle, run_gpu

pytestmark = pytest.mark.gpu

KINDS = ("random", "chain", "bushy")


def _case(seed):
    g = np.random.default_rng(1000 + seed)
    hk = int(g.choice([1, 2, 4]))
    hv = hk * int(g.choice([1, 2, 4]))
    batch = int(g.integers(1, 6))
    uniform = bool(g.integers(0, 2))
    if uniform:
        n = int(g.choice([1, 5, 16, 31, 32, 33, 47, 64]))
        sizes = [n] * batch
    else:
        sizes = [int(x) for x in g.integers(1, 65, size=batch)]
    kinds = [KINDS[int(k)] for k in g.integers(0, 3, size=batch)]
    o_dtype = torch.bfloat16 if g.integers(0, 3) else torch.float32
    use_bits = (not uniform) or bool(g.integers(0, 2))
    return hk, hv, sizes, kinds, uniform, o_dtype, use_bits


@pytest.mark.parametrize("seed", range(16))
def test_verify_sweep(cuda, seed):
    from dforktree_amd import ops, synth
    hk, hv, sizes, kinds, uniform, o_dtype, use_bits = _case(seed)
    announce(f"sweep {seed}: hk={hk} hv={hv} sizes={sizes} kinds={kinds} uniform={uniform} o={o_dtype} "
             f"bits={use_bits}")
    batch = synth.make_batch(500 + seed, 0, sizes, hk=hk, hv=hv, kinds=kinds)
    o, k, v, gg = run_gpu(batch, cuda, use_bits=use_bits, o_dtype=o_dtype, packed=not uniform)
    check_against_oracle(batch, o, k, v, gg, o_bf16=(o_dtype == torch.bfloat16))
    # commit every request's accepted path from the saves just written, in place
    gen = torch.Generator().manual_seed(seed)
    P = 16
    idx = torch.full((batch.batch, P), -1, dtype=torch.int32)
    walks = []
    for r, sl in enumerate(request_slices(batch)):
        w = synth.accepted_path(batch.parent[sl], P, gen)
        idx[r, :len(w)] = w
        walks.append(w.tolist())
    state = batch.state.clone().to(cuda).unsqueeze(0)  # [L=1, B, hv, V, K]
    n_max = max(sizes)
    if uniform:
        ops.tree_commit(state, k.unsqueeze(0), v.unsqueeze(0), gg.unsqueeze(0), idx.to(cuda), n_nodes=n_max)
    else:
        ops.tree_commit(state, k.unsqueeze(0), v.unsqueeze(0), gg.unsqueeze(0), idx.to(cuda), n_nodes=n_max,
                        cu_seqlens=batch.cu_seqlens.to(cuda))
    torch.cuda.synchronize()
    ref = oracle_verify(batch)
    got = np32(state[0])
    for r in range(batch.batch):
        S0 = np32(batch.state[r]).transpose(0, 2, 1)
        want = O.closed_commit(S0, ref[r]["k"], ref[r]["vn"], ref[r]["G"], walks[r])
        assert rel_l2(got[r].transpose(0, 2, 1), want) <= REL_L2, f"request {r}: committed state"
