"""GPU parity of the bit-packed attention masks (dft_packbits,
dft_tree_mask_pack) against numpy.packbits and the oracle's tree mask:
bit-exact bytes and byte offsets, little and big bit order, empty and
ragged segments, prefixes that leave rows unaligned to bytes, a too-small
output buffer (bytes dropped, status set, nothing written past it)."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import gdn_tree as O
from oracle import mask as M

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bitorder", ["little", "big"])
def test_packbits_single(cuda, bitorder):
    from dforktree_amd import ops
    g = torch.Generator().manual_seed(3)
    for n in [1, 7, 8, 9, 31, 32, 33, 1000, 4096 * 64 + 5, 3_000_001]:
        announce(f"packbits n={n} {bitorder}")
        x = torch.randint(0, 3, (n,), generator=g, dtype=torch.uint8)
        got = ops.packbits(x.to(cuda), bitorder).cpu().numpy()
        assert np.array_equal(got, M.packbits(x.numpy(), bitorder)), n
    xb = torch.rand(37, 53, generator=g) > 0.5  # bool, 2-D: flattened row-major
    assert np.array_equal(ops.packbits(xb.to(cuda)).cpu().numpy(), M.packbits(xb.numpy()))


def test_segment_packbits(cuda):
    from dforktree_amd import ops
    announce("segment_packbits ragged")
    g = torch.Generator().manual_seed(4)
    lens = [0, 1, 7, 8, 9, 0, 100, 1023, 4161, 64]
    indptr = np.concatenate([[0], np.cumsum(lens)])
    x = torch.randint(0, 2, (int(indptr[-1]),), generator=g, dtype=torch.uint8).bool()
    for dt in (torch.int32, torch.int64):
        packed, new = ops.segment_packbits(x.to(cuda), torch.tensor(indptr, dtype=dt).to(cuda))
        want, want_ip = M.segment_packbits(x.numpy(), indptr)
        assert np.array_equal(packed.cpu().numpy(), want)
        assert new.cpu().numpy().tolist() == want_ip.tolist()


def _batch(seed, sizes, kinds):
    g = np.random.default_rng(seed)
    parents, ancs = [], []
    for n, kind in zip(sizes, kinds):
        p = np.full(n, -1, np.int64)
        for i in range(1, n):
            p[i] = i - 1 if kind == "chain" else (int(g.integers(0, min(i, 2))) if kind == "bushy" else int(g.integers(0, i)))
        parents.append(p)
        ancs.append(O.tree_struct(p)[0])
    return parents, ancs


@pytest.mark.parametrize("bitorder", ["little", "big"])
def test_tree_mask_pack_ragged(cuda, bitorder):
    from dforktree_amd import ops
    announce(f"tree_mask_pack ragged {bitorder}")
    sizes = [1, 8, 13, 32, 64, 40, 3, 64, 17, 2]
    kinds = ["chain", "bushy", "random"] * 4
    plens = [0, 1, 7, 8, 100, 4096, 4099, 3, 0, 12345]
    parents, ancs = _batch(5, sizes, kinds[:len(sizes)])
    cu = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]), dtype=torch.int32).to(cuda)
    par = torch.tensor(np.concatenate(parents), dtype=torch.int32).to(cuda)
    bits = ops.tree_struct(par, 4, cu_seqlens=cu, n_nodes=64, batch=len(sizes), want=("anc_bits",))["anc_bits"]
    for pdt in (torch.int32, torch.int64):
        packed, ip = ops.tree_mask_pack(bits, torch.tensor(plens, dtype=pdt).to(cuda), cu_seqlens=cu,
                                        bitorder=bitorder)
        want, want_ip = M.tree_masks_packed(ancs, plens, bitorder)
        assert ip.cpu().numpy().tolist() == want_ip.tolist()
        assert np.array_equal(packed.cpu().numpy(), want)


def test_tree_mask_pack_uniform_matches_packbits_of_bool_mask(cuda):
    """The plan's single-request case: packing fc1_branch64's boolean mask
    with dft_packbits and building it from the bits give the same bytes."""
    from dforktree_amd import ops
    announce("tree_mask_pack uniform vs packbits")
    n, plen = 64, 3001
    parents, ancs = _batch(6, [n], ["random"])
    par = torch.tensor(parents[0], dtype=torch.int64).to(cuda)
    st = ops.tree_struct(par, 4, want=("anc_bits", "anc"))
    boolmask = torch.cat((torch.ones((n, plen), device=cuda, dtype=torch.bool), st["anc"][0].bool()), dim=1)
    a = ops.packbits(boolmask.flatten())
    b, ip = ops.tree_mask_pack(st["anc_bits"], torch.tensor([plen], device=cuda))
    assert torch.equal(a, b)
    assert ip.cpu().tolist() == [0, (n * (plen + n) + 7) // 8]
    assert np.array_equal(b.cpu().numpy(), M.tree_mask_packed(ancs[0], plen))


def test_tree_mask_pack_capacity(cuda):
    """A buffer one request too small: the fitting bytes are exact, the
    guard bytes behind the capacity are untouched, status is 1."""
    from dforktree_amd import ops
    announce("tree_mask_pack capacity")
    sizes, plens = [32, 32, 32], [10, 20, 30]
    parents, ancs = _batch(7, sizes, ["random"] * 3)
    par = torch.tensor(np.concatenate(parents), dtype=torch.int64).to(cuda)
    bits = ops.tree_struct(par, 4, batch=3, n_nodes=32, want=("anc_bits",))["anc_bits"]
    want, want_ip = M.tree_masks_packed(ancs, plens)
    cap = int(want_ip[2]) + 5
    buf = torch.full((cap + 64,), 0xA5, dtype=torch.uint8, device=cuda)
    status = torch.zeros(1, dtype=torch.int32, device=cuda)
    out, ip = ops.tree_mask_pack(bits, torch.tensor(plens, device=cuda), n_nodes=32, out=buf[:cap], status=status)
    got = buf.cpu().numpy()
    assert np.array_equal(got[:cap], want[:cap])
    assert (got[cap:] == 0xA5).all()
    assert int(status.item()) == 1
    assert ip.cpu().numpy().tolist() == want_ip.tolist()


def test_plan_override_packs_on_the_device(cuda, monkeypatch):
    """fc1_plan's fast path on stand-ins for flashinfer / SGLang with the
    wrapper's buffers on the GPU: dft_packbits writes the mask bytes into
    the plan's own buffer, bit-exact with numpy.packbits."""
    import fake_flashinfer
    mods, calls, saved = fake_flashinfer.install_fakes()
    try:
        from dforktree_amd.plugin import fc1_plan as P
        P.install()
        n, plen = 64, 1237
        parents, ancs = _batch(8, [n], ["random"])
        mask = torch.cat((torch.ones(n, plen, dtype=torch.bool), torch.from_numpy(ancs[0] > 0.5)), dim=1).flatten()
        monkeypatch.setattr(P, "HOST_KV_LEN", plen + n)
        w = mods["flashinfer"].BatchPrefillWithPagedKVCacheWrapper(device=cuda)
        announce("plan override on the device")
        res = w.plan(qo_indptr=torch.tensor([0, n], device=cuda), paged_kv_indptr=None, paged_kv_indices=None,
                     paged_kv_last_page_len=None, num_qo_heads=8, num_kv_heads=1, head_dim_qk=128, page_size=1,
                     custom_mask=mask.to(cuda))
        torch.cuda.synchronize()
        assert res == "fast_plan"
        nbytes = (n * (plen + n) + 7) // 8
        assert np.array_equal(w._custom_mask_buf[:nbytes].cpu().numpy(), M.tree_mask_packed(ancs[0], plen))
        assert w._mask_indptr_buf.cpu().tolist() == [0, nbytes]
        assert int(w._custom_mask_buf[nbytes:].sum().item()) == 0
    finally:
        fake_flashinfer.remove_fakes(saved)
