"""Drop-in for dforktree/fc1_conv.py on MI355X: the tree-parent conv hook.

``install()`` patches SGLang's ``gdn_backend.causal_conv1d_update`` like
fc1_conv.py:29-46: for a batch-1 verify of NN tokens it runs the gfx950
tree conv (width 4, SiLU) over ``[conv_state || tokens]`` with the gather
columns ``CTX.cidx``, writes each node's 3-column window into
``intermediate_conv_window``, stashes the [NN, C] output in
``fc1_fused.CTX.current_mixed`` for the verify hook, and returns the
[1, C, NN] view.  Anything else goes to the original SGLang function, and
so does a call the library refuses before launching (DFT_ERR_INVALID /
DFT_ERR_UNSUPPORTED); ``current_mixed`` is then cleared, so the next
verify falls back as well instead of reading another layer's output.
"""
from __future__ import annotations

import torch

if __package__:
    from . import fc1_fused as F
else:  # bare import from this directory
    import fc1_fused as F
try:
    from dforktree_amd import _lib, ops as _ops
except ImportError:  # bare import, with the package itself not on sys.path
    import pathlib
    import sys
    sys.path.append(str(pathlib.Path(__file__).resolve().parents[2]))
    from dforktree_amd import _lib, ops as _ops


def default_cidx(nn, device):
    """Placeholder gather rows [0, 1, 2, 3+n] used until the builder's real
    cidx is copied in (fc1_conv.py:39-40)."""
    return torch.cat((torch.arange(3, device=device).expand(nn, 3),
                      torch.arange(3, 3 + nn, device=device)[:, None]), 1).int()


def conv(x, conv_state, weight, bias, cidx, conv_state_indices, intermediate_state_indices, intermediate_conv_window,
         out):
    """fc1_conv.py:7-27 for one request: x [1, C, N] (any strides),
    conv_state [slots, C, 3], weight [C, 4] (or [C, 1, 4]), out [1, N, C]."""
    w2 = weight.reshape(weight.shape[0], -1)
    _ops.tree_conv(x.transpose(1, 2), conv_state, w2, bias, cidx, silu=True, cs_indices=conv_state_indices,
                   y=out, iw=intermediate_conv_window, iw_indices=intermediate_state_indices)
    return out


def install():
    from sglang.srt.layers.attention.linear import gdn_backend as backend
    original = backend.causal_conv1d_update

    def call(x, conv_state, weight, bias=None, activation=None, **kw):
        if F.CTX is not None:
            F.CTX.current_mixed = None
        if F.NATIVE_REFERENCE or x.ndim != 3 or x.shape[0] != 1 or x.shape[-1] != F.NN:
            return original(x, conv_state, weight, bias, activation, **kw)
        assert weight.shape[-1] == 4 and activation in ['silu', 'swish', True]
        if F.CTX is None:
            F.CTX = F.Context()
        if getattr(F.CTX, 'cidx', None) is None:
            F.CTX.cidx = default_cidx(F.NN, x.device)
        out = torch.empty((1, F.NN, x.shape[1]), device=x.device, dtype=x.dtype)
        try:
            conv(x, conv_state, weight, bias, F.CTX.cidx, kw['conv_state_indices'], kw['intermediate_state_indices'],
                 kw['intermediate_conv_window'], out)
        except _lib.DftError as err:
            if not F.refused(err):
                raise
            return original(x, conv_state, weight, bias, activation, **kw)
        F.CTX.current_mixed = out[0]
        return out.transpose(1, 2)

    backend.causal_conv1d_update = call
