"""The SGLang hooks of fc1_fused / fc1_conv, on the CPU: which calls go to
the MI355X operators, with which arguments, and which fall back to the
original SGLang function (fc1_fused.py:59-95, fc1_conv.py:33-45).  The
operators themselves are replaced by recorders here; their arithmetic is
covered by the GPU parity tests."""
import types

import pytest
import torch

from fake_sglang import install_fakes, remove_fakes


@pytest.fixture
def hooked(monkeypatch):
    from dforktree_amd import fc1_conv, fc1_fused as F

    def step_indices(batch, accept_index, accept_lens, draft_token_num):
        last = accept_index.gather(1, (accept_lens.long() - 1)[:, None])
        return last, getattr(batch, "track", None)

    mods, calls, saved = install_fakes(step_indices)
    monkeypatch.setattr(F, "CTX", F.Context(device="cpu"))
    monkeypatch.setattr(F, "NATIVE_REFERENCE", False)
    F.install()
    fc1_conv.install()
    yield F, fc1_conv, mods, calls
    remove_fakes(saved)


def _verify_args(nn, hk=16, hv=32):
    A_log = torch.log(torch.full((hv,), 0.5))
    dt_bias = torch.zeros(hv)
    q = torch.zeros(1, nn, hk, 128, dtype=torch.bfloat16)
    v = torch.zeros(1, nn, hv, 128, dtype=torch.bfloat16)
    a = torch.zeros(1, nn, hv)
    return A_log, dt_bias, q, q, v, a, a.clone()


def test_verify_hook_routes_tree_verifies_to_split(hooked, monkeypatch):
    F, _, mods, calls = hooked
    seen = []

    def fake_split(*args, **kw):
        seen.append((args, kw))
        return torch.zeros(F.NN, 32, 128)

    monkeypatch.setattr(F.TK, "tree_gdn_split", fake_split)
    K = mods["sglang.srt.layers.attention.linear.kernels.gdn_triton"].TritonGDNKernel
    F.CTX.current_mixed = torch.zeros(F.NN, 8192, dtype=torch.bfloat16)
    pool = torch.zeros(3, 32, 128, 128)
    A_log, dt_bias, q, k, v, a, b = _verify_args(F.NN)
    slots, islots = torch.tensor([2]), torch.tensor([1])
    out = K().target_verify(A_log, dt_bias, q, k, v, a, b, cache_steps=F.NN, ssm_states=pool, cache_indices=slots,
                            intermediate_state_indices=islots)
    assert out.shape == (1, F.NN, 32, 128)
    (args, kw), = seen
    y, aa, bb, A, dtb, S0, anc, Hk, Hv, Dk, Dv = args
    assert y is F.CTX.current_mixed and anc is F.CTX.anc
    assert aa.shape == (F.NN, 32) and (Hk, Hv, Dk, Dv) == (16, 32, 128, 128)
    assert S0.shape == (32, 128, 128) and S0.stride() == pool[0].transpose(-1, -2).stride()
    assert kw["state_indices"] is slots and kw["state_slot_stride"] == pool.stride(0)
    assert torch.allclose(kw["neg_exp_A"], -A_log.exp())
    keys, vals, gains = kw["aux"]
    assert keys.data_ptr() == F.CTX.keys[0].data_ptr() and gains.data_ptr() == F.CTX.gains[0].data_ptr()
    assert F.CTX.inter_indices is islots
    # a second layer (another A_log) gets the next aux slice; the first keeps its index
    A2 = A_log.clone()
    K().target_verify(A2, dt_bias, q, k, v, a, b, cache_steps=F.NN, ssm_states=pool, cache_indices=slots,
                      intermediate_state_indices=islots)
    K().target_verify(A_log, dt_bias, q, k, v, a, b, cache_steps=F.NN, ssm_states=pool, cache_indices=slots,
                      intermediate_state_indices=islots)
    assert [s[1]["aux"][0].data_ptr() for s in seen] == [F.CTX.keys[i].data_ptr() for i in (0, 1, 0)]
    assert calls.names() == []


def test_verify_hook_falls_back_for_other_step_counts(hooked):
    F, _, mods, calls = hooked
    K = mods["sglang.srt.layers.attention.linear.kernels.gdn_triton"].TritonGDNKernel
    A_log, dt_bias, q, k, v, a, b = _verify_args(8)
    assert K().target_verify(A_log, dt_bias, q, k, v, a, b, cache_steps=8) == "original_verify"
    assert calls.names() == ["original_verify"]


def test_routing_hook(hooked, monkeypatch):
    F, _, mods, calls = hooked
    B = mods["sglang.srt.layers.attention.linear.gdn_backend"].GDNAttnBackend
    assert B()._target_verify_supports_strided_qkv(draft_token_num=F.NN) is True
    assert B()._target_verify_supports_strided_qkv(draft_token_num=F.NN - 1) is False
    monkeypatch.setattr(F, "NATIVE_REFERENCE", True)
    assert B()._target_verify_supports_strided_qkv(draft_token_num=F.NN) is False
    assert calls.names() == ["original_routing", "original_routing"]


def _worker(temporal, inter, slots):
    pool = types.SimpleNamespace(
        get_speculative_mamba2_params_all_layers=lambda: types.SimpleNamespace(temporal=temporal,
                                                                               intermediate_ssm=inter),
        get_mamba_indices=lambda req_pool_indices: slots)
    return types.SimpleNamespace(model_runner=types.SimpleNamespace(req_to_token_pool=pool))


@pytest.mark.parametrize("track", [None, 3])
def test_commit_hook_snapshots_both_ends_then_calls_original(hooked, monkeypatch, track):
    F, _, mods, calls = hooked
    seen = []
    monkeypatch.setattr(F, "snapshot_commit", lambda *args: seen.append(args))
    commit = mods["sglang.srt.speculative.eagle_worker_common"].commit_mamba_states_after_verify
    temporal, inter, slots = torch.zeros(2, 3, 4, 1, 1), torch.zeros(2, 2, F.NN, 4, 1, 1), torch.tensor([2])
    F.CTX.inter_indices = torch.tensor([1])
    accept_index = torch.tensor([[0, 5, 9, -1]], dtype=torch.int32)
    batch = types.SimpleNamespace(req_pool_indices=torch.tensor([0]),
                                  track=None if track is None else torch.tensor([[track]]))
    out = commit(_worker(temporal, inter, slots), batch, torch.tensor([3]), accept_index, F.NN)
    assert out == "original_commit"
    assert calls.names() == ["step_indices", "original_commit"]
    (args,), = [seen]
    S, keys, vals, gains, anc, acc, ends, sl, isl, dst = args
    assert S is temporal and dst is inter and sl is slots and isl is F.CTX.inter_indices
    assert keys is F.CTX.keys and anc is F.CTX.anc and acc is accept_index
    assert ends.tolist() == [[9, -1 if track is None else track]]


def test_commit_hook_skips_other_draft_sizes(hooked, monkeypatch):
    F, _, mods, calls = hooked
    monkeypatch.setattr(F, "snapshot_commit", lambda *args: pytest.fail("must not commit"))
    commit = mods["sglang.srt.speculative.eagle_worker_common"].commit_mamba_states_after_verify
    batch = types.SimpleNamespace(req_pool_indices=torch.tensor([0]))
    assert commit(None, batch, torch.tensor([1]), torch.tensor([[0]]), F.NN - 1) == "original_commit"
    assert calls.names() == ["original_commit"]


def test_conv_hook_routes_batch1_tree_verifies(hooked, monkeypatch):
    F, conv_mod, mods, calls = hooked
    seen = []

    def fake_conv(x, conv_state, weight, bias, cidx, csi, isi, iw, out):
        seen.append((x, cidx, csi, isi, iw))
        out.fill_(1.0)
        return out

    monkeypatch.setattr(conv_mod, "conv", fake_conv)
    backend = mods["sglang.srt.layers.attention.linear.gdn_backend"]
    C = 96
    x = torch.zeros(1, F.NN, C, dtype=torch.bfloat16).transpose(1, 2)   # [1, C, NN] strided view
    cs, w, iw = torch.zeros(3, C, 3), torch.zeros(C, 4), torch.zeros(2, F.NN, C, 3)
    csi, isi = torch.tensor([2]), torch.tensor([1])
    res = backend.causal_conv1d_update(x, cs, w, None, "silu", conv_state_indices=csi, intermediate_state_indices=isi,
                                       intermediate_conv_window=iw)
    assert res.shape == (1, C, F.NN) and torch.all(res == 1)
    assert F.CTX.current_mixed.shape == (F.NN, C) and F.CTX.current_mixed.data_ptr() == res.data_ptr()
    (sx, cidx, scsi, sisi, siw), = seen
    assert sx is x and scsi is csi and sisi is isi and siw is iw
    # the placeholder gather rows [0, 1, 2, 3 + n] until the builder's cidx is copied in (fc1_conv.py:39-40)
    want = torch.cat((torch.arange(3).expand(F.NN, 3), torch.arange(3, 3 + F.NN)[:, None]), 1)
    assert torch.equal(cidx.long(), want) and cidx.dtype == torch.int32
    # fallbacks: batch > 1, another token count, or native reference mode
    assert backend.causal_conv1d_update(torch.zeros(2, C, F.NN), cs, w) == "original_conv"
    assert backend.causal_conv1d_update(torch.zeros(1, C, 7), cs, w) == "original_conv"
    monkeypatch.setattr(F, "NATIVE_REFERENCE", True)
    assert backend.causal_conv1d_update(x, cs, w) == "original_conv"
    assert calls.names() == ["original_conv"] * 3
