"""The drop-in as SGLang would drive it, on the GPU: the fc1_conv and
fc1_fused hooks installed over stand-in SGLang entry points, run for two GDN
layers of one 64-node tree at full width (16 q/k heads, 32 v heads, C =
8192), then the accept-and-commit hook.  Checked against the oracle:

* conv output (bf16) within max-abs 1e-2 / rel-L2 2e-3, window bit-exact;
* verify output within the same bounds, computed by the oracle from the
  conv output the GPU produced (the verify's own input);
* snapshots at the last and the tracked accepted node within rel-L2 2e-3 of
  the closed form over the oracle's keys, values and gains; every other
  snapshot slot untouched.
"""
import types

import numpy as np
import pytest
import torch

from conftest import MAX_ABS_BF16, REL_L2, announce, max_abs, rel_l2
from _ref import np32
from fake_sglang import install_fakes, remove_fakes
from oracle import gdn_tree as O

pytestmark = pytest.mark.gpu


def test_hooked_layers_then_commit(cuda, monkeypatch):
    from dforktree_amd import synth
    from dforktree_amd.plugin import fc1_conv, fc1_fused as F
    announce("hooked conv + verify x2 layers + snapshot commit")

    def step_indices(batch, accept_index, accept_lens, draft_token_num):
        last = accept_index.gather(1, (accept_lens.long() - 1)[:, None])
        return last, batch.track

    mods, calls, saved = install_fakes(step_indices)
    try:
        monkeypatch.setattr(F, "CTX", F.Context())
        monkeypatch.setattr(F, "NATIVE_REFERENCE", False)
        F.install()
        fc1_conv.install()
        NN, C, L, HK, HV = F.NN, 8192, 2, 16, 32
        gen = torch.Generator().manual_seed(21)
        parent = synth.tree_parents(NN, "random", gen)
        anc, depth, cidx = O.tree_struct(parent.numpy())
        # what fc1_branch64.verify_branch does before the forward pass
        F.CTX.cidx = fc1_conv.default_cidx(NN, cuda)
        F.CTX.anc.copy_(torch.from_numpy(anc))
        F.CTX.cidx.copy_(torch.from_numpy(cidx))

        temporal = torch.randn(L, 3, HV, 128, 128, generator=gen) * 0.02
        conv_state = torch.randn(3, C, 3, generator=gen).to(torch.bfloat16)
        weight = (torch.randn(C, 4, generator=gen) * 0.1).to(torch.bfloat16)
        xs = [torch.randn(1, NN, C, generator=gen).to(torch.bfloat16) for _ in range(L)]
        aa = [torch.randn(1, NN, HV, generator=gen).to(torch.bfloat16) for _ in range(L)]
        bb = [torch.randn(1, NN, HV, generator=gen).to(torch.bfloat16) for _ in range(L)]
        A_logs = [torch.log(torch.full((HV,), 0.5 + 0.2 * l)) for l in range(L)]
        dt_bias = torch.zeros(HV)
        slot, islot = torch.tensor([2], dtype=torch.int32), torch.tensor([1], dtype=torch.int32)

        tg = temporal.to(cuda)
        csg, wg = conv_state.to(cuda), weight.to(cuda)
        iws = [torch.zeros(2, NN, C, 3, dtype=torch.bfloat16, device=cuda) for _ in range(L)]
        backend = mods["sglang.srt.layers.attention.linear.gdn_backend"]
        K = mods["sglang.srt.layers.attention.linear.kernels.gdn_triton"].TritonGDNKernel
        q = torch.empty(1, NN, HK, 128, dtype=torch.bfloat16, device=cuda)
        v = torch.empty(1, NN, HV, 128, dtype=torch.bfloat16, device=cuda)
        ys, outs = [], []
        for l in range(L):
            x = xs[l].to(cuda).transpose(1, 2)          # [1, C, NN] view, as SGLang passes it
            res = backend.causal_conv1d_update(x, csg, wg, None, "silu", conv_state_indices=slot.to(cuda),
                                               intermediate_state_indices=islot.to(cuda),
                                               intermediate_conv_window=iws[l])
            ys.append(res[0].transpose(0, 1).clone())
            out = K().target_verify(A_logs[l].to(cuda), dt_bias.to(cuda), q, q, v, aa[l].to(cuda), bb[l].to(cuda),
                                    cache_steps=NN, ssm_states=tg[l], cache_indices=slot.to(cuda),
                                    intermediate_state_indices=islot.to(cuda))
            outs.append(out)

        path = synth.accepted_path(parent, 16, gen)
        accept_index = torch.full((1, 16), -1, dtype=torch.int32)
        accept_index[0, :len(path)] = path
        track = int(path[len(path) // 2]) if len(path) > 2 else -1
        batch = types.SimpleNamespace(req_pool_indices=torch.tensor([0], device=cuda),
                                      track=torch.tensor([[track]], dtype=torch.int32, device=cuda))
        sentinel = 321.0
        inter = torch.full((L, 2, NN, HV, 128, 128), sentinel, device=cuda)
        pool = types.SimpleNamespace(
            get_speculative_mamba2_params_all_layers=lambda: types.SimpleNamespace(temporal=tg,
                                                                                   intermediate_ssm=inter),
            get_mamba_indices=lambda req_pool_indices: slot.to(cuda))
        worker = types.SimpleNamespace(model_runner=types.SimpleNamespace(req_to_token_pool=pool))
        commit = mods["sglang.srt.speculative.eagle_worker_common"].commit_mamba_states_after_verify
        assert commit(worker, batch, torch.tensor([len(path)], device=cuda), accept_index.to(cuda), NN) \
            == "original_commit"
        torch.cuda.synchronize()
        assert calls.names() == ["step_indices", "original_commit"]

        touched = torch.zeros(L, 2, NN, dtype=torch.bool)
        for l in range(L):
            ry, win = O.tree_conv(np32(xs[l][0]), np32(conv_state[2]), np32(weight), None, cidx)
            y_gpu = np32(ys[l])
            assert max_abs(y_gpu, O.bf16_round(ry)) <= MAX_ABS_BF16 and rel_l2(y_gpu, O.bf16_round(ry)) <= REL_L2
            assert np.array_equal(np32(iws[l][1]), win), "conv window must be bit-exact"
            assert np.all(np32(iws[l][0]) == 0), "only the intermediate slot is written"
            S0 = np32(temporal[l, 2]).transpose(0, 2, 1)
            ref = O.tree_gdn_split(y_gpu[None], np32(aa[l][0])[None], np32(bb[l][0])[None], np32(A_logs[l]),
                                   np32(dt_bias), S0[None], anc[None], HK, HV, 128, 128)
            o = np32(outs[l][0])
            want = O.bf16_round(ref["o"][0])
            assert outs[l].shape == (1, NN, HV, 128)
            assert rel_l2(o, want) <= REL_L2 and max_abs(o, want) <= MAX_ABS_BF16, f"layer {l} o"
            for u in (int(path[-1]), track):
                if u < 0:
                    continue
                touched[l, 1, u] = True
                snap = O.closed_commit(S0, ref["k"][0], ref["vn"][0], ref["G"][0], path.tolist(), u=u, anc=anc)
                got = np32(inter[l, 1, u]).transpose(0, 2, 1)
                assert rel_l2(got, snap) <= REL_L2, f"layer {l} snapshot at node {u}"
        assert torch.all(inter.cpu()[~touched] == sentinel)
    finally:
        remove_fakes(saved)
