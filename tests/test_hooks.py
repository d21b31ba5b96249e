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
    from dforktree_amd.plugin import fc1_conv, fc1_fused as F

    def step_indices(batch, accept_index, accept_lens, draft_token_num):
        last = accept_index.gather(1, (accept_lens.long() - 1)[:, None])
        return last, getattr(batch, "track", None)

    mods, calls, saved = install_fakes(step_indices)
    monkeypatch.setattr(F, "CTX", F.Context(device="cpu"))
    monkeypatch.setattr(F, "NATIVE_REFERENCE", False)
    packed = []  # the hook's dft_anc_pack launches, recorded (no device here)
    monkeypatch.setattr(F._ops, "anc_pack", lambda anc, out=None: packed.append((anc, out)) or out)
    F.packed = packed
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
    mixed = torch.zeros(F.NN, 8192, dtype=torch.bfloat16)
    F.CTX.current_mixed = mixed
    pool = torch.zeros(3, 32, 128, 128)
    A_log, dt_bias, q, k, v, a, b = _verify_args(F.NN)
    slots, islots = torch.tensor([2]), torch.tensor([1])
    out = K().target_verify(A_log, dt_bias, q, k, v, a, b, cache_steps=F.NN, ssm_states=pool, cache_indices=slots,
                            intermediate_state_indices=islots)
    assert out.shape == (1, F.NN, 32, 128)
    (args, kw), = seen
    y, aa, bb, A, dtb, S0, anc, Hk, Hv, Dk, Dv = args
    assert y is mixed and anc is F.CTX.anc
    # the conv output is consumed: a verify never reads another layer's
    assert F.CTX.current_mixed is None and F.CTX.saved == {0}
    assert aa.shape == (F.NN, 32) and (Hk, Hv, Dk, Dv) == (16, 32, 128, 128)
    assert S0.shape == (32, 128, 128) and S0.stride() == pool[0].transpose(-1, -2).stride()
    assert kw["state_indices"] is slots and kw["state_slot_stride"] == pool.stride(0)
    # layer 0 packs this step's CTX.anc into bit rows, which the verify reads
    assert kw["anc_bits"] is F.CTX.anc_bits
    assert len(F.packed) == 1 and F.packed[0][0] is F.CTX.anc and F.packed[0][1] is F.CTX.anc_bits
    assert torch.allclose(kw["neg_exp_A"], -A_log.exp())
    keys, vals, gains = kw["aux"]
    assert keys.data_ptr() == F.CTX.keys[0].data_ptr() and gains.data_ptr() == F.CTX.gains[0].data_ptr()
    assert F.CTX.inter_indices is islots
    # a second layer (another A_log) gets the next aux slice; the first keeps its index
    A2 = A_log.clone()
    for A in (A2, A_log):
        F.CTX.current_mixed = mixed
        K().target_verify(A, dt_bias, q, k, v, a, b, cache_steps=F.NN, ssm_states=pool, cache_indices=slots,
                          intermediate_state_indices=islots)
    assert [s[1]["aux"][0].data_ptr() for s in seen] == [F.CTX.keys[i].data_ptr() for i in (0, 1, 0)]
    assert calls.names() == [] and F.CTX.saved == {0, 1}
    assert len(F.packed) == 2, "packed once per forward: at layer 0 only"


def test_anc_is_packed_at_layer_0_even_when_its_conv_fell_back(hooked, monkeypatch):
    """Layer 0's conv ran in SGLang (no current_mixed): its verify falls back,
    but this step's tree is still packed, so a later layer verified here and
    the step's commit read this step's bit rows."""
    F, _, mods, calls = hooked
    seen = []
    monkeypatch.setattr(F.TK, "tree_gdn_split", lambda *args, **kw: seen.append(kw) or torch.zeros(F.NN, 32, 128))
    K = mods["sglang.srt.layers.attention.linear.kernels.gdn_triton"].TritonGDNKernel
    pool = torch.zeros(3, 32, 128, 128)
    A_log, dt_bias, q, k, v, a, b = _verify_args(F.NN)
    kw = dict(cache_steps=F.NN, ssm_states=pool, cache_indices=torch.tensor([2]),
              intermediate_state_indices=torch.tensor([1]))
    F.CTX.current_mixed = None
    assert K().target_verify(A_log, dt_bias, q, k, v, a, b, **kw) == "original_verify"
    assert len(F.packed) == 1 and F.packed[0][1] is F.CTX.anc_bits and F.CTX.saved == set()
    F.CTX.current_mixed = torch.zeros(F.NN, 8192, dtype=torch.bfloat16)
    K().target_verify(A_log.clone(), dt_bias, q, k, v, a, b, **kw)  # layer 1, verified here
    assert len(F.packed) == 1 and seen[0]["anc_bits"] is F.CTX.anc_bits and F.CTX.saved == {1}
    assert calls.names() == ["original_verify"]


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
    monkeypatch.setattr(F, "snapshot_commit", lambda *args, **kw: seen.append(args + (kw,)))
    commit = mods["sglang.srt.speculative.eagle_worker_common"].commit_mamba_states_after_verify
    temporal, inter, slots = torch.zeros(2, 3, 4, 1, 1), torch.zeros(2, 2, F.NN, 4, 1, 1), torch.tensor([2])
    F.CTX.inter_indices = torch.tensor([1])
    F.CTX.saved = {0, 1}   # both layers verified here
    accept_index = torch.tensor([[0, 5, 9, -1]], dtype=torch.int32)
    batch = types.SimpleNamespace(req_pool_indices=torch.tensor([0]),
                                  track=None if track is None else torch.tensor([[track]]))
    out = commit(_worker(temporal, inter, slots), batch, torch.tensor([3]), accept_index, F.NN)
    assert out == "original_commit"
    assert calls.names() == ["step_indices", "original_commit"]
    (args,), = [seen]
    S, keys, vals, gains, anc, acc, ends, sl, isl, dst, kw = args
    assert kw["anc_bits"] is F.CTX.anc_bits
    assert S.data_ptr() == temporal.data_ptr() and S.shape == temporal.shape
    assert dst.data_ptr() == inter.data_ptr() and dst.shape == inter.shape
    assert sl is slots and isl is F.CTX.inter_indices
    assert keys.data_ptr() == F.CTX.keys.data_ptr() and keys.shape[0] == 2
    assert anc is F.CTX.anc and acc is accept_index
    assert ends.tolist() == [[9, -1 if track is None else track]]


def test_commit_hook_skips_other_draft_sizes(hooked, monkeypatch):
    F, _, mods, calls = hooked
    monkeypatch.setattr(F, "snapshot_commit", lambda *args, **kw: pytest.fail("must not commit"))
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


def _refusal(status):
    from dforktree_amd import _lib

    def raise_status(*args, **kw):
        raise _lib.DftError("dft_stub", status, "forced by the test")
    return raise_status


def test_refused_verify_falls_back_and_is_not_committed(hooked, monkeypatch):
    """A verify the library refuses (nothing launched) runs SGLang's own
    kernel (fc1_fused.py:61-62), and the commit then leaves that layer to
    SGLang's snapshot."""
    from dforktree_amd import _lib
    F, _, mods, calls = hooked
    K = mods["sglang.srt.layers.attention.linear.kernels.gdn_triton"].TritonGDNKernel
    A_log, dt_bias, q, k, v, a, b = _verify_args(F.NN)
    kw = dict(cache_steps=F.NN, ssm_states=torch.zeros(3, 32, 128, 128), cache_indices=torch.tensor([0]),
              intermediate_state_indices=torch.tensor([0]))
    F.CTX.saved = {0}
    for status in (_lib.DFT_ERR_UNSUPPORTED, _lib.DFT_ERR_INVALID):
        monkeypatch.setattr(F.TK, "tree_gdn_split", _refusal(status))
        F.CTX.current_mixed = torch.zeros(F.NN, 8192, dtype=torch.bfloat16)
        assert K().target_verify(A_log, dt_bias, q, k, v, a, b, **kw) == "original_verify"
        assert F.CTX.saved == set() and F.CTX.current_mixed is None
    assert calls.names() == ["original_verify"] * 2
    # a launch failure is not a refusal: it propagates
    monkeypatch.setattr(F.TK, "tree_gdn_split", _refusal(_lib.DFT_ERR_LAUNCH))
    F.CTX.current_mixed = torch.zeros(F.NN, 8192, dtype=torch.bfloat16)
    with pytest.raises(_lib.DftError):
        K().target_verify(A_log, dt_bias, q, k, v, a, b, **kw)
    # no layer was verified here: the commit launches nothing and calls SGLang's commit
    monkeypatch.setattr(F, "snapshot_commit", lambda *args, **kw: pytest.fail("must not commit"))
    commit = mods["sglang.srt.speculative.eagle_worker_common"].commit_mamba_states_after_verify
    batch = types.SimpleNamespace(req_pool_indices=torch.tensor([0]))
    assert commit(None, batch, torch.tensor([1]), torch.tensor([[0]]), F.NN) == "original_commit"


def test_refused_conv_falls_back_and_so_does_the_next_verify(hooked, monkeypatch):
    """fc1_conv.py:34-35: a refused conv runs SGLang's conv; the verify of
    that layer then has no tree input and falls back too."""
    from dforktree_amd import _lib
    F, conv_mod, mods, calls = hooked
    backend = mods["sglang.srt.layers.attention.linear.gdn_backend"]
    K = mods["sglang.srt.layers.attention.linear.kernels.gdn_triton"].TritonGDNKernel
    monkeypatch.setattr(F.TK, "tree_gdn_split", lambda *a, **k: pytest.fail("must not verify"))
    C = 96
    x = torch.zeros(1, C, F.NN, dtype=torch.bfloat16)
    cs, w, iw = torch.zeros(3, C, 3), torch.zeros(C, 4), torch.zeros(2, F.NN, C, 3)
    conv_kw = dict(conv_state_indices=torch.tensor([0]), intermediate_state_indices=torch.tensor([0]),
                   intermediate_conv_window=iw)
    monkeypatch.setattr(conv_mod._ops, "tree_conv", _refusal(_lib.DFT_ERR_UNSUPPORTED))
    F.CTX.current_mixed = torch.zeros(F.NN, C, dtype=torch.bfloat16)   # a previous layer's output
    assert backend.causal_conv1d_update(x, cs, w, None, "silu", **conv_kw) == "original_conv"
    assert F.CTX.current_mixed is None
    A_log, dt_bias, q, k, v, a, b = _verify_args(F.NN)
    out = K().target_verify(A_log, dt_bias, q, k, v, a, b, cache_steps=F.NN, ssm_states=torch.zeros(1, 32, 128, 128),
                            cache_indices=torch.tensor([0]), intermediate_state_indices=torch.tensor([0]))
    assert out == "original_verify"
    assert calls.names() == ["original_conv", "original_verify"]
    # a conv that falls back on its guard clears the stale output as well
    F.CTX.current_mixed = torch.zeros(F.NN, C, dtype=torch.bfloat16)
    assert backend.causal_conv1d_update(torch.zeros(2, C, F.NN), cs, w) == "original_conv"
    assert F.CTX.current_mixed is None
    monkeypatch.setattr(conv_mod._ops, "tree_conv", _refusal(_lib.DFT_ERR_LAUNCH))
    with pytest.raises(_lib.DftError):
        backend.causal_conv1d_update(x, cs, w, None, "silu", **conv_kw)


def test_commit_covers_only_layers_verified_here(hooked, monkeypatch):
    """Layers whose verify fell back keep SGLang's snapshots: the commit
    launches over the runs of layers verified here, and a refusal there is
    raised (falling back would leave those layers without a snapshot)."""
    from dforktree_amd import _lib
    F, _, mods, calls = hooked
    seen = []
    monkeypatch.setattr(F, "snapshot_commit", lambda *args, **kw: seen.append(args + (kw,)))
    commit = mods["sglang.srt.speculative.eagle_worker_common"].commit_mamba_states_after_verify
    L = 6
    temporal, inter = torch.zeros(L, 3, 4, 1, 1), torch.zeros(L, 2, F.NN, 4, 1, 1)
    F.CTX.inter_indices = torch.tensor([1])
    F.CTX.saved = {0, 1, 3, 5}
    batch = types.SimpleNamespace(req_pool_indices=torch.tensor([0]), track=None)
    accept_index = torch.tensor([[0, 2, -1]], dtype=torch.int32)
    assert commit(_worker(temporal, inter, torch.tensor([2])), batch, torch.tensor([2]), accept_index,
                  F.NN) == "original_commit"
    got = [(args[0].data_ptr() - temporal.data_ptr()) // temporal.stride(0) // 4 for args in seen]
    assert got == [0, 3, 5] and [args[0].shape[0] for args in seen] == [2, 1, 1]
    for args in seen:
        l0 = (args[0].data_ptr() - temporal.data_ptr()) // temporal.stride(0) // 4
        assert args[1].data_ptr() == F.CTX.keys[l0].data_ptr() and args[1].shape[0] == args[0].shape[0]
        assert args[9].data_ptr() == inter[l0].data_ptr() and args[9].shape[0] == args[0].shape[0]
    assert F.layer_runs({0, 1, 3, 5}) == [(0, 2), (3, 4), (5, 6)] and F.layer_runs(set()) == []
    monkeypatch.setattr(F, "snapshot_commit", _refusal(_lib.DFT_ERR_UNSUPPORTED))
    with pytest.raises(_lib.DftError):
        commit(_worker(temporal, inter, torch.tensor([2])), batch, torch.tensor([2]), accept_index, F.NN)
