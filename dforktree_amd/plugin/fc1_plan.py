"""Drop-in for dforktree/fc1_plan.py on MI355X: the tree-attention plan override.

``install()`` wraps flashinfer's ``BatchPrefillWithPagedKVCacheWrapper.plan``
(and ``begin_forward``) as fc1_plan.py:8-35 does.  A call takes the fast
path when all of these hold:
  * ``HOST_KV_LEN`` is set (fc1_branch64.py:38 sets it to prefix + nodes);
  * a ``custom_mask`` is passed;
  * the wrapper runs under graph capture with the ``fa2`` backend and a
    compiled module.
The fast path:
  * packs the boolean mask (little bit order) straight into the wrapper's
    own mask buffer with ``dft_packbits``, with no allocation and no
    host read-back;
  * sets the mask indptr to [0, bytes];
  * calls SGLang's ``fast_prefill_plan`` with the host-side lengths.
Any other call goes to the original ``plan``, and so does one whose packing
the library refuses before launching (DFT_ERR_INVALID / DFT_ERR_UNSUPPORTED).

``pack_tree_mask()`` is the direct form for callers that hold the tree's
ancestry bits. It builds the packed mask of fc1_branch64.py:39 (ones over
the prefix, Anc over the draft nodes) with ``dft_tree_mask_pack``, without
the boolean [n, prefix + n] tensor.
"""
from __future__ import annotations

import inspect

import torch

try:
    from dforktree_amd import _lib, ops as _ops
except ImportError:  # bare import, with the package itself not on sys.path
    import pathlib
    import sys
    sys.path.append(str(pathlib.Path(__file__).resolve().parents[2]))
    from dforktree_amd import _lib, ops as _ops

HOST_KV_LEN = None
TREE_SIZES = (16, 32, 64)


def _bind(names, args, kwargs) -> dict:
    """plan()'s arguments by name (positional ones in signature order)."""
    values = dict(zip(names, args))
    values.update(kwargs)
    return values


def _takes_fast_path(wrapper, values) -> bool:
    return (HOST_KV_LEN is not None and values.get("custom_mask") is not None
            and bool(getattr(wrapper, "is_cuda_graph_enabled", False))
            and getattr(wrapper, "_backend", None) == "fa2"
            and getattr(wrapper, "_cached_module", None) is not None)


def pack_mask_into(wrapper, mask: torch.Tensor, n_queries: int, kv_len: int) -> int:
    """Packs a single request's boolean mask into the wrapper's buffers and
    returns its byte count (fc1_plan.py:26-28)."""
    nbytes = (n_queries * kv_len + 7) // 8
    buf = wrapper._custom_mask_buf
    if buf.numel() < nbytes:
        raise ValueError(f"custom mask needs {nbytes} bytes, the plan buffer holds {buf.numel()}")
    _ops.packbits(mask.reshape(-1), "little", out=buf[:nbytes])
    ind = wrapper._mask_indptr_buf
    ind.copy_(torch.tensor([0, nbytes], dtype=ind.dtype, device=ind.device), non_blocking=True)
    return nbytes


def pack_tree_mask(anc_bits: torch.Tensor, prefix_len: torch.Tensor, **kw):
    """The packed tree mask from ancestry bits (see ops.tree_mask_pack)."""
    return _ops.tree_mask_pack(anc_bits, prefix_len, **kw)


def install():
    import flashinfer
    from sglang.srt.layers.attention.flashinfer_backend import fast_prefill_plan

    cls = flashinfer.BatchPrefillWithPagedKVCacheWrapper
    original = cls.plan
    names = list(inspect.signature(original).parameters)[1:]
    fast_names = set(inspect.signature(fast_prefill_plan).parameters) - {"self"}

    def plan(self, *args, **kwargs):
        values = _bind(names, args, kwargs)
        if not _takes_fast_path(self, values):
            return original(self, *args, **kwargs)
        mask = values["custom_mask"]
        qo = values["qo_indptr"]
        # one request, one token per page, a 16/32/64-node tree against the host-known KV length
        assert qo.numel() == 2 and values["page_size"] == 1
        n = mask.numel() // HOST_KV_LEN
        assert n in TREE_SIZES and n * HOST_KV_LEN == mask.numel()
        try:
            pack_mask_into(self, mask, n, HOST_KV_LEN)
        except _lib.DftError as err:
            if err.status not in (_lib.DFT_ERR_INVALID, _lib.DFT_ERR_UNSUPPORTED):
                raise
            return original(self, *args, **kwargs)  # nothing was launched: the plan flashinfer would make
        kv_host = torch.tensor([0, HOST_KV_LEN], dtype=torch.int32)
        fast = {k: v for k, v in values.items() if k in fast_names}
        fast.update(qo_indptr_host=torch.tensor([0, n], dtype=torch.int32), kv_indptr_host=kv_host,
                    kv_lens_host=kv_host[1:], max_q_len=n, max_kv_len=HOST_KV_LEN)
        return fast_prefill_plan(self, **fast)

    cls.plan = plan
    cls.begin_forward = plan
