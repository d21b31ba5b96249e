"""Drop-in for dforktree/tree_kernels.py on MI355X.

Same public names, signatures and argument meaning as the reference module
(tree_kernels.py:13-14, :83-108, :129-132, :193-208); the work runs in the
gfx950 HIP library through the C ABI.  Launch-tuning arguments of the Triton
kernels (BV, num_warps, BC) are accepted and ignored.

Differences, all deliberate:
* ``tree_gdn_fused`` inverts (I+A) exactly; the reference's Neumann product
  (tree_kernels.py:62-68) is exact only for paths of at most 15 edges.
* Dk = Dv = 128 only (the layer shape of the target model); other head dims
  raise ``DftError`` (DFT_ERR_UNSUPPORTED).
"""
from __future__ import annotations

import torch

try:
    from dforktree_amd import ops as _ops
    from dforktree_amd import _lib
except ImportError:  # bare import, with the package itself not on sys.path
    import pathlib
    import sys
    sys.path.append(str(pathlib.Path(__file__).resolve().parents[2]))
    from dforktree_amd import ops as _ops
    from dforktree_amd import _lib


def available():
    """tree_kernels.py:13-14: a GPU is present and the kernels can run."""
    return torch.cuda.is_available() and _lib.LIB_PATH.exists()


def _pow2(n):
    """tree_kernels.py:83-84."""
    return max(16, 1 << (int(n) - 1).bit_length())


def tree_conv_fused(conv_state, mixed0, cidx, w2, bias, BC=1024):
    """tree_kernels.py:86-93: y[n,c] = SiLU(sum_j w2[c,j] xt[cidx[n,j], c] + bias[c])
    with xt = [conv_state[:, :KC-1] as columns || mixed0 rows]."""
    N, C = mixed0.shape
    KC = cidx.shape[1]
    assert mixed0.stride(1) == 1 and w2.is_contiguous()
    y = torch.empty(N, C, device=mixed0.device, dtype=mixed0.dtype)
    assert w2.shape == (C, KC)
    # cidx goes to the kernel as it is: int32 and int64 are both read on the device
    _ops.tree_conv(mixed0.unsqueeze(0), conv_state, w2, bias, cidx, silu=True, y=y.unsqueeze(0))
    return y


def tree_gdn_fused(y, aa0, bb0, A_log, dt_bias, S0, Anc, Hk, Hv, Dk, Dv, scale=None, BV=16, num_warps=4, aux=None,
                   neg_exp_A=None):
    """tree_kernels.py:95-108: single-pass verify with fp32 output; N > 32
    goes to ``tree_gdn_split`` exactly as the reference delegates."""
    N = y.shape[0]
    if N > 32:
        return tree_gdn_split(y, aa0, bb0, A_log, dt_bias, S0, Anc, Hk, Hv, Dk, Dv, scale=scale, aux=aux,
                              neg_exp_A=neg_exp_A)
    BN = _pow2(N)
    assert BN <= 64, 'Invalid n-gram input or configuration'
    assert y.stride(1) == 1 and Dv % BV == 0
    o = torch.empty(N, Hv, Dv, device=y.device, dtype=torch.float32)
    _verify(y, aa0, bb0, A_log, dt_bias, S0, Anc, Hk, Hv, scale, aux, neg_exp_A, None, 0, o)
    return o


def closed_commit(states, keys, values, gains, src, n):
    """tree_kernels.py:129-132: in place, for every (layer, head),
    S <- e^{G_u} S + sum_{t<=n} e^{G_u - G_src[t]} k_src[t] v_src[t]^T with
    u = src[n]; states [L, H, DK, DV], at most 16 path entries (BT=16)."""
    L, H, DK, DV = states.shape
    N = keys.shape[2]
    P = min(int(src.numel()), 16)
    nn = n if isinstance(n, torch.Tensor) else torch.tensor([int(n)], device=states.device, dtype=torch.int32)
    _ops.tree_commit(states.unsqueeze(1), keys, values, gains, src.reshape(1, -1)[:, :P], n_nodes=N,
                     path_len=nn.reshape(1), len_is_last=True, kv_layout=True)


def tree_gdn_split(y, aa0, bb0, A_log, dt_bias, S0, Anc, Hk, Hv, Dk, Dv, scale=None, BV=64, num_warps=8, aux=None,
                   neg_exp_A=None, state_indices=None, state_slot_stride=0, anc_bits=None):
    """tree_kernels.py:193-208: the verify entry the SGLang hook calls
    (fc1_fused.py:74).  Returns o [N, Hv, Dv] in y.dtype; with
    aux=(k [Hv,N,Dk], vn [Hv,N,Dv], G [Hv,N]) also saves the commit inputs.
    S0 is the [Hv, Dk, Dv] view of slot 0; the slot max(state_indices[0], 0)
    is read on the device and offset by state_slot_stride.  ``anc_bits``
    (an extension: Anc packed to int64 rows by ``ops.anc_pack``) replaces
    the dense Anc when given."""
    N = y.shape[0]
    BN = _pow2(N)
    assert BN <= 64 and Dv % BV == 0
    if N not in (16, 32, 64):
        raise KeyError(N)  # the reference dispatches invert{16,32,64} by N (:206)
    o = torch.empty(N, Hv, Dv, device=y.device, dtype=y.dtype)
    _verify(y, aa0, bb0, A_log, dt_bias, S0, Anc, Hk, Hv, scale, aux, neg_exp_A, state_indices, state_slot_stride, o,
            anc_bits)
    return o


def _verify(y, aa0, bb0, A_log, dt_bias, S0, Anc, Hk, Hv, scale, aux, neg_exp_A, state_indices, slot_stride, o,
            anc_bits=None):
    N = y.shape[0]
    k, vn, G = aux if aux is not None else (None, None, None)
    tree = dict(anc=Anc) if anc_bits is None else dict(anc_bits=anc_bits)
    _ops.tree_verify(y, aa0.reshape(N, -1), bb0.reshape(N, -1), A_log, dt_bias, S0, hk=Hk, hv=Hv, batch=1, n_nodes=N,
                     scale=scale, neg_exp_A=neg_exp_A, state_indices=state_indices,
                     state_slot_stride=slot_stride if state_indices is not None else 0, o=o,
                     aux_k=k, aux_v=vn, aux_g=G, **tree)
