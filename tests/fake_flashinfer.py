"""A stand-in for the flashinfer wrapper and the SGLang planner that
fc1_plan.py:8-35 patches (neither is installed).  The stand-ins record their
calls so tests can check the plan override's routing, its fallbacks and the
buffers it fills."""
from __future__ import annotations

import sys
import types

import torch

MODULES = ("flashinfer", "sglang", "sglang.srt", "sglang.srt.layers", "sglang.srt.layers.attention",
           "sglang.srt.layers.attention.flashinfer_backend")


def install_fakes():
    calls = []
    mods = {name: types.ModuleType(name) for name in MODULES}
    for name, mod in mods.items():
        parent, _, leaf = name.rpartition(".")
        if parent:
            setattr(mods[parent], leaf, mod)

    class BatchPrefillWithPagedKVCacheWrapper:
        def __init__(self, backend="fa2", graph=True, compiled=True, mask_bytes=1 << 16, device="cpu"):
            self._backend = backend
            self.is_cuda_graph_enabled = graph
            self._cached_module = object() if compiled else None
            self._custom_mask_buf = torch.zeros(mask_bytes, dtype=torch.uint8, device=device)
            self._mask_indptr_buf = torch.zeros(2, dtype=torch.int32, device=device)

        def plan(self, qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len, num_qo_heads,
                 num_kv_heads, head_dim_qk, page_size, head_dim_vo=None, custom_mask=None, packed_custom_mask=None,
                 causal=False):
            calls.append(("original_plan", custom_mask is not None))
            return "original_plan"

        begin_forward = plan

    def fast_prefill_plan(self, qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len, num_qo_heads,
                          num_kv_heads, head_dim_qk, page_size, qo_indptr_host, kv_indptr_host, kv_lens_host,
                          max_q_len, max_kv_len, head_dim_vo=None, causal=False):
        calls.append(("fast_plan", dict(num_qo_heads=num_qo_heads, page_size=page_size,
                                        qo_indptr_host=qo_indptr_host.tolist(), kv_indptr_host=kv_indptr_host.tolist(),
                                        kv_lens_host=kv_lens_host.tolist(), max_q_len=max_q_len, max_kv_len=max_kv_len)))
        return "fast_plan"

    mods["flashinfer"].BatchPrefillWithPagedKVCacheWrapper = BatchPrefillWithPagedKVCacheWrapper
    mods["sglang.srt.layers.attention.flashinfer_backend"].fast_prefill_plan = fast_prefill_plan
    saved = {name: sys.modules.get(name) for name in MODULES}
    sys.modules.update(mods)
    return mods, calls, saved


def remove_fakes(saved):
    for name, mod in saved.items():
        if mod is None:
            sys.modules.pop(name, None)
        else:
            sys.modules[name] = mod
