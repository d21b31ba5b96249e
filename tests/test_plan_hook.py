"""CPU routing of the plan override (fc1_plan.py:8-35) on stand-ins for
flashinfer and SGLang: the guards that send a call to the original plan,
and on the fast path the packed bytes, the mask indptr and the host lengths
handed to fast_prefill_plan.  The packing itself is swapped for
numpy.packbits here (the GPU test runs dft_packbits)."""
import numpy as np
import pytest
import torch

import fake_flashinfer

N, PLEN = 32, 77


@pytest.fixture
def plan_mod(monkeypatch):
    mods, calls, saved = fake_flashinfer.install_fakes()
    from dforktree_amd.plugin import fc1_plan as P

    def np_packbits(x, bitorder="little", *, out=None, status=None):
        p = torch.from_numpy(np.packbits(x.cpu().numpy().reshape(-1) != 0, bitorder=bitorder))
        out[:p.numel()].copy_(p)
        return out[:p.numel()]

    monkeypatch.setattr(P._ops, "packbits", np_packbits)
    monkeypatch.setattr(P, "HOST_KV_LEN", None)
    P.install()
    yield P, mods["flashinfer"].BatchPrefillWithPagedKVCacheWrapper, calls
    fake_flashinfer.remove_fakes(saved)


def _args(mask):
    return dict(qo_indptr=torch.tensor([0, N]), paged_kv_indptr=torch.tensor([0, PLEN + N]),
                paged_kv_indices=torch.arange(PLEN + N), paged_kv_last_page_len=torch.tensor([1]),
                num_qo_heads=8, num_kv_heads=1, head_dim_qk=128, page_size=1, custom_mask=mask)


def _mask(seed=0):
    g = torch.Generator().manual_seed(seed)
    anc = torch.rand(N, N, generator=g) > 0.5
    return torch.cat((torch.ones(N, PLEN, dtype=torch.bool), anc), dim=1).flatten()


def test_fast_path_packs_into_the_wrapper(plan_mod, monkeypatch):
    P, W, calls = plan_mod
    monkeypatch.setattr(P, "HOST_KV_LEN", PLEN + N)
    w = W()
    mask = _mask()
    assert w.plan(**_args(mask)) == "fast_plan"
    nbytes = (N * (PLEN + N) + 7) // 8
    assert np.array_equal(w._custom_mask_buf[:nbytes].numpy(), np.packbits(mask.numpy(), bitorder="little"))
    assert w._mask_indptr_buf.tolist() == [0, nbytes]
    name, kw = calls[-1]
    assert name == "fast_plan"
    assert kw["qo_indptr_host"] == [0, N] and kw["kv_indptr_host"] == [0, PLEN + N] and kw["kv_lens_host"] == [PLEN + N]
    assert kw["max_q_len"] == N and kw["max_kv_len"] == PLEN + N and kw["num_qo_heads"] == 8
    # positional arguments bind the same way; begin_forward is the same override
    a = _args(mask)
    pos = [a.pop(k) for k in ("qo_indptr", "paged_kv_indptr", "paged_kv_indices", "paged_kv_last_page_len",
                              "num_qo_heads", "num_kv_heads", "head_dim_qk", "page_size")]
    assert w.begin_forward(*pos, **a) == "fast_plan"


@pytest.mark.parametrize("case", ["no_host_len", "no_mask", "no_graph", "other_backend", "not_compiled"])
def test_guards_fall_back_to_the_original_plan(plan_mod, monkeypatch, case):
    P, W, calls = plan_mod
    if case != "no_host_len":
        monkeypatch.setattr(P, "HOST_KV_LEN", PLEN + N)
    w = W(graph=case != "no_graph", backend="fa3" if case == "other_backend" else "fa2",
          compiled=case != "not_compiled")
    args = _args(None if case == "no_mask" else _mask())
    assert w.plan(**args) == "original_plan"
    assert calls[-1][0] == "original_plan"
    assert int(w._mask_indptr_buf.sum()) == 0


def test_tree_sizes_are_checked(plan_mod, monkeypatch):
    P, W, calls = plan_mod
    monkeypatch.setattr(P, "HOST_KV_LEN", 10)
    with pytest.raises(AssertionError):
        W().plan(**dict(_args(torch.ones(12 * 10, dtype=torch.bool)), qo_indptr=torch.tensor([0, 12])))


def test_refused_packing_falls_back_to_the_original_plan(plan_mod, monkeypatch):
    """A packing the library refuses before launching goes to flashinfer's
    own plan; a launch failure propagates."""
    from dforktree_amd import _lib
    P, W, calls = plan_mod
    monkeypatch.setattr(P, "HOST_KV_LEN", PLEN + N)
    for status, falls_back in ((_lib.DFT_ERR_UNSUPPORTED, True), (_lib.DFT_ERR_INVALID, True),
                               (_lib.DFT_ERR_LAUNCH, False)):
        def refuse(*args, _status=status, **kw):
            raise _lib.DftError("dft_packbits", _status, "forced by the test")
        monkeypatch.setattr(P._ops, "packbits", refuse)
        if falls_back:
            assert W().plan(**_args(_mask())) == "original_plan"
            assert calls[-1][0] == "original_plan"
        else:
            with pytest.raises(_lib.DftError):
                W().plan(**_args(_mask()))
