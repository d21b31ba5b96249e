"""A stand-in for the four SGLang 0.5.22 entry points the DForkTree hooks
patch (fc1_fused.py:51-97, fc1_conv.py:29-46).  SGLang is not installed; the
stand-ins record how they are called so tests can check the hooks' routing
and fallbacks, and the package's ``install()`` functions patch them exactly
as they would patch SGLang."""
from __future__ import annotations

import sys
import types

MODULES = (
    "sglang", "sglang.srt", "sglang.srt.layers", "sglang.srt.layers.attention",
    "sglang.srt.layers.attention.linear", "sglang.srt.layers.attention.linear.kernels",
    "sglang.srt.layers.attention.linear.kernels.gdn_triton", "sglang.srt.layers.attention.linear.gdn_backend",
    "sglang.srt.speculative", "sglang.srt.speculative.eagle_worker_common", "sglang.srt.speculative.spec_utils",
)


class Calls(list):
    def names(self):
        return [c[0] for c in self]


def install_fakes(step_indices=None):
    """Put fresh stand-in modules into sys.modules; returns (modules, calls).
    ``step_indices(batch, accept_index, accept_lens, draft_token_num)`` plays
    SGLang's ``_verify_commit_step_indices`` (returns ``last, track``)."""
    calls = Calls()
    mods = {name: types.ModuleType(name) for name in MODULES}
    for name, mod in mods.items():
        parent, _, leaf = name.rpartition(".")
        if parent:
            setattr(mods[parent], leaf, mod)

    class TritonGDNKernel:
        def target_verify(self, A_log, dt_bias, q, k, v, a, b, **kw):
            calls.append(("original_verify", kw))
            return "original_verify"

    class GDNAttnBackend:
        def _target_verify_supports_strided_qkv(self, **kwargs):
            calls.append(("original_routing", kwargs))
            return False

    def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None, **kw):
        calls.append(("original_conv", kw))
        return "original_conv"

    def commit_mamba_states_after_verify(target_worker, batch, accept_lens, accept_index, draft_token_num,
                                         prepared_step_indices=None):
        calls.append(("original_commit", draft_token_num))
        return "original_commit"

    def _verify_commit_step_indices(batch, accept_index, accept_lens, draft_token_num):
        calls.append(("step_indices", draft_token_num))
        return step_indices(batch, accept_index, accept_lens, draft_token_num)

    mods["sglang.srt.layers.attention.linear.kernels.gdn_triton"].TritonGDNKernel = TritonGDNKernel
    backend = mods["sglang.srt.layers.attention.linear.gdn_backend"]
    backend.GDNAttnBackend = GDNAttnBackend
    backend.causal_conv1d_update = causal_conv1d_update
    mods["sglang.srt.speculative.eagle_worker_common"].commit_mamba_states_after_verify = \
        commit_mamba_states_after_verify
    mods["sglang.srt.speculative.spec_utils"]._verify_commit_step_indices = _verify_commit_step_indices
    saved = {name: sys.modules.get(name) for name in MODULES}
    sys.modules.update(mods)
    return mods, calls, saved


def remove_fakes(saved):
    for name, mod in saved.items():
        if mod is None:
            sys.modules.pop(name, None)
        else:
            sys.modules[name] = mod
