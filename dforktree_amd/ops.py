"""Torch-facing operators over the HIP library (batched and packed-varlen).

Tensors are caller-owned device tensors passed as pointer + element strides;
launches go on the current HIP stream of the tensors' device and nothing here
synchronises with the host, so every operator can be captured in a HIP graph.
Per-request slot and path indices stay on the device.

These are the building blocks of the reference-named modules in
``dforktree_amd.plugin`` (``tree_kernels``, ``fc1_fused``, ``fc1_conv``,
``fc1_block_inverse``, ``fc1_plan``), of ``dforktree_amd.builder`` and of
the batched API the reference lacks (it is batch-1 only: fc1_fused.py:69,
fc1_branch64.py:13).
"""
from __future__ import annotations

import ctypes as C
import weakref
from typing import Optional

import torch

from . import _lib
from ._lib import (DFT_BF16, DFT_BITS_BIG, DFT_BITS_LITTLE, DFT_F16, DFT_F32, DFT_I32, DFT_I64, AncPackArgs,
                   CommitArgs, ConvArgs, MaskArgs, PackbitsArgs, PendingArgs, TreeArgs, VerifyArgs, check, load)

_FLOAT_TAG = {torch.float32: DFT_F32, torch.bfloat16: DFT_BF16, torch.float16: DFT_F16}
_INDEX_TAG = {torch.int32: DFT_I32, torch.int64: DFT_I64}
D_HEAD = 128
MAX_NODES = 64


def _ftag(t: torch.Tensor, name: str) -> int:
    try:
        return _FLOAT_TAG[t.dtype]
    except KeyError:
        raise TypeError(f"{name}: unsupported dtype {t.dtype}") from None


def _itag(t: torch.Tensor, name: str) -> int:
    try:
        return _INDEX_TAG[t.dtype]
    except KeyError:
        raise TypeError(f"{name}: index tensor must be int32 or int64, got {t.dtype}") from None


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _device_of(*ts) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("dforktree_amd operators take GPU tensors (HIP device memory)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _idx_vec(t: Optional[torch.Tensor], name: str):
    if t is None:
        return None, DFT_I32
    if t.dim() != 1:
        t = t.reshape(-1)
    if t.stride(0) != 1:
        t = t.contiguous()
    return t, _itag(t, name)


# ---------------------------------------------------------------------------
# tree verify
# ---------------------------------------------------------------------------
def tree_verify(y: torch.Tensor, a: torch.Tensor, b: torch.Tensor, A_log: Optional[torch.Tensor],
                dt_bias: torch.Tensor, state: torch.Tensor, *, hk: int, hv: int,
                anc: Optional[torch.Tensor] = None, anc_bits: Optional[torch.Tensor] = None,
                batch: Optional[int] = None, n_nodes: Optional[int] = None,
                cu_seqlens: Optional[torch.Tensor] = None, scale: Optional[float] = None,
                neg_exp_A: Optional[torch.Tensor] = None, state_indices: Optional[torch.Tensor] = None,
                state_slot_stride: Optional[int] = None, o: Optional[torch.Tensor] = None,
                o_dtype: Optional[torch.dtype] = None, aux_k: Optional[torch.Tensor] = None,
                aux_v: Optional[torch.Tensor] = None, aux_g: Optional[torch.Tensor] = None,
                aux_k_per_khead: bool = False, status: Optional[torch.Tensor] = None,
                size_order: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused tree verify of every (request, v-head).

    y [rows, 2*hk*128 + hv*128] bf16 with channel stride 1; a, b [rows, hv];
    state: S0 viewed as [slots, hv, dk, dv] (index k, v; any strides -- pass
    ``pool.transpose(-1, -2)`` for a V-major pool) or [hv, dk, dv] for one slot;
    the tree as ``anc`` [batch, N, N] / [N, N] 0/1 or ``anc_bits`` [rows]
    int64 bit masks.  Rows of request b start at cu_seqlens[b] (packed) or
    b*n_nodes.  Returns o [rows, hv, dv]; aux_k [hv|hk, rows, dk],
    aux_v [hv, rows, dv], aux_g [hv, rows] are filled when given.  ``status``
    (int32 [batch]) receives every request's DFT_STATUS_* bits: a packed
    request longer than n_nodes is cut to n_nodes rows (DFT_STATUS_SPAN).
    ``size_order``: the records ``size_order(cu_seqlens, n_nodes)`` wrote for
    this packed batch (once per step, shared by every layer); a launch split
    by tree size then runs each class's requests first in its kernel.
    """
    args, o, dev, _keep = _verify_args(
        y, a, b, A_log, dt_bias, state, hk=hk, hv=hv, anc=anc, anc_bits=anc_bits, batch=batch, n_nodes=n_nodes,
        cu_seqlens=cu_seqlens, scale=scale, neg_exp_A=neg_exp_A, state_indices=state_indices,
        state_slot_stride=state_slot_stride, o=o, o_dtype=o_dtype, aux_k=aux_k, aux_v=aux_v, aux_g=aux_g,
        aux_k_per_khead=aux_k_per_khead, status=status, size_order=size_order)
    check("dft_tree_verify", load().dft_tree_verify(C.byref(args), _stream(dev)))
    return o


# Which cu_seqlens each size-order record tensor was written from (host-side
# bookkeeping: id of the records -> (weak reference to them, the cu_seqlens
# tensor's data pointer and version counter, n_nodes, batch)).  A verify
# given records of other cu_seqlens would take the wrong rows; the device
# only sees the header's n_nodes and batch.
_SIZE_ORDER_SOURCE = {}


def size_order(cu_seqlens: torch.Tensor, n_nodes: int, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The packed batch's requests by size class (``dft_size_order``):
    int32 [batch + 1, 4], row 0 = (requests of at most 32 nodes, the others,
    n_nodes, batch), then one (request, first row, span, 0) record per
    request, the small ones from the front and the others from the back.
    Pass it as ``size_order`` to every verify of the step; the verify refuses
    records written from another cu_seqlens tensor or before an in-place
    change of it.  ``out`` (int32, contiguous, 16-byte aligned, at least
    [batch + 1, 4]) avoids the allocation."""
    if cu_seqlens.dtype != torch.int32:
        raise TypeError("cu_seqlens must be int32")
    source = (cu_seqlens.data_ptr(), cu_seqlens._version)
    cu_seqlens = cu_seqlens.contiguous()
    batch = cu_seqlens.numel() - 1
    dev = cu_seqlens.device
    if out is None:
        out = torch.empty(batch + 1, 4, device=dev, dtype=torch.int32)
    _check_size_order(out, batch, dev)
    check("dft_size_order", load().dft_size_order(cu_seqlens.data_ptr(), batch, int(n_nodes), out.data_ptr(),
                                                  _stream(dev)))
    for k in [k for k, v in _SIZE_ORDER_SOURCE.items() if v[0]() is None]:
        del _SIZE_ORDER_SOURCE[k]
    _SIZE_ORDER_SOURCE[id(out)] = (weakref.ref(out), *source, int(n_nodes), batch)
    return out


def _check_size_order_source(t, cu_seqlens, n_nodes, batch):
    """Refuse records that ``size_order`` wrote for another batch.  Records
    written by other means are not known here (the device then checks the
    header's n_nodes and batch only)."""
    ent = _SIZE_ORDER_SOURCE.get(id(t))
    if ent is None or ent[0]() is not t:
        return
    _, ptr, ver, nn, b = ent
    if (nn, b) != (int(n_nodes), batch):
        raise ValueError(f"size_order was written for n_nodes={nn}, batch={b}; this launch has "
                         f"n_nodes={n_nodes}, batch={batch}")
    if (ptr, ver) != (cu_seqlens.data_ptr(), cu_seqlens._version):
        raise ValueError("size_order was written from another cu_seqlens (or before it was changed in place): "
                         "call size_order(cu_seqlens, n_nodes) again for this batch")


def _check_size_order(t, batch, dev):
    if t.dtype != torch.int32 or not t.is_contiguous() or t.numel() < 4 * (batch + 1) or t.data_ptr() % 16:
        raise ValueError(f"size_order must be a contiguous, 16-byte aligned int32 tensor of at least "
                         f"{4 * (batch + 1)} entries")
    if t.device != dev:
        raise ValueError(f"size_order is on {t.device}, the inputs on {dev}")


def _status_ptr(status, batch, dev):
    if status is None:
        return None
    if status.dtype != torch.int32 or not status.is_contiguous() or status.numel() < batch:
        raise ValueError(f"status must be a contiguous int32 tensor of at least {batch} entries")
    if status.device != dev:
        raise ValueError(f"status is on {status.device}, the inputs on {dev}")
    return status.data_ptr()


def _verify_args(y, a, b, A_log, dt_bias, state, *, hk, hv, anc, anc_bits, batch, n_nodes, cu_seqlens, scale,
                 neg_exp_A, state_indices, state_slot_stride, o, o_dtype, aux_k, aux_v, aux_g, aux_k_per_khead,
                 status=None, size_order=None):
    """Validate the verify operands and fill the C descriptor; returns
    (args, o, device, tensors that must outlive the launch call)."""
    dev = _device_of(y, a, b, A_log, dt_bias, state, anc, anc_bits, cu_seqlens, neg_exp_A,
                     state_indices, o, aux_k, aux_v, aux_g)
    if y.dim() != 2 or y.stride(1) != 1:
        raise ValueError("y must be [rows, channels] with channel stride 1")
    if y.dtype != torch.bfloat16:
        raise TypeError("y must be bfloat16")
    rows = y.shape[0]
    if y.shape[1] < 2 * hk * D_HEAD + hv * D_HEAD:
        raise ValueError(f"y has {y.shape[1]} channels, need {2 * hk * D_HEAD + hv * D_HEAD}")
    if y.data_ptr() % 16 or y.stride(0) % 8:
        # the kernels copy q/k/v rows as 16-byte pieces: a fresh buffer with
        # the row pitch rounded up to 8 elements (a contiguous but misaligned
        # view would stay misaligned under .contiguous())
        pitch = -(-y.shape[1] // 8) * 8
        y = torch.empty(rows, pitch, device=y.device, dtype=y.dtype)[:, :y.shape[1]].copy_(y)
    cu_given = cu_seqlens
    if cu_seqlens is not None:
        if batch is None:
            batch = cu_seqlens.numel() - 1
        if n_nodes is None:
            raise ValueError("packed input needs n_nodes (the largest request) on the host")
        if cu_seqlens.dtype != torch.int32:
            raise TypeError("cu_seqlens must be int32")
        cu_seqlens = cu_seqlens.contiguous()
    else:
        if n_nodes is None and batch is None:
            batch, n_nodes = 1, rows
        elif n_nodes is None:
            n_nodes = rows // batch
        elif batch is None:
            batch = rows // max(n_nodes, 1)
        if batch * n_nodes > rows:
            raise ValueError(f"batch*n_nodes = {batch * n_nodes} exceeds the {rows} rows of y")
    if n_nodes > MAX_NODES:
        raise ValueError(f"at most {MAX_NODES} nodes per request, got {n_nodes}")
    for t, nm in ((a, "a"), (b, "b")):
        if t.dim() != 2 or t.shape[1] < hv or t.stride(1) != 1:
            raise ValueError(f"{nm} must be [rows, hv] with stride 1 along heads")
    if state.dim() == 3:
        s_slot = 0 if state_slot_stride is None else state_slot_stride
        s_h, s_k, s_v = state.stride()
        shp = state.shape
    elif state.dim() == 4:
        s_slot, s_h, s_k, s_v = state.stride()
        if state_slot_stride is not None:
            s_slot = state_slot_stride
        shp = state.shape[1:]
    else:
        raise ValueError("state must be [hv, dk, dv] or [slots, hv, dk, dv]")
    if tuple(shp) != (hv, D_HEAD, D_HEAD):
        raise ValueError(f"state head block must be ({hv}, 128, 128), got {tuple(shp)}")
    if state.dtype != torch.float32:
        raise TypeError("state must be float32")
    if (anc is None) == (anc_bits is None):
        raise ValueError("give exactly one of anc / anc_bits")
    anc_row = anc_req = 0
    if anc is not None:
        if anc.dtype != torch.float32:
            anc = anc.float()
        if anc.stride(-1) != 1:
            anc = anc.contiguous()
        anc_row = anc.stride(-2)
        anc_req = anc.stride(0) if anc.dim() == 3 else 0
    if anc_bits is not None:
        if anc_bits.dtype != torch.int64:
            raise TypeError("anc_bits must be int64 (uint64 bit masks)")
        anc_bits = anc_bits.contiguous()
    if o is None:
        o = torch.empty(rows, hv, D_HEAD, device=dev, dtype=o_dtype or y.dtype)
    if o.stride(-1) != 1:
        raise ValueError("o must have stride 1 along dv")
    si, si_tag = _idx_vec(state_indices, "state_indices")
    scale = D_HEAD ** -0.5 if scale is None else float(scale)

    args = VerifyArgs()
    args.batch, args.n_nodes, args.hk, args.hv = batch, n_nodes, hk, hv
    args.dk = args.dv = D_HEAD
    args.scale = scale
    args.flags = _lib.DFT_VERIFY_AUX_K_PER_KHEAD if aux_k_per_khead else 0
    args.y, args.y_row_stride, args.cu_seqlens = y.data_ptr(), y.stride(0), _ptr(cu_seqlens)
    args.a, args.a_row_stride, args.a_dtype = a.data_ptr(), a.stride(0), _ftag(a, "a")
    args.b, args.b_row_stride, args.b_dtype = b.data_ptr(), b.stride(0), _ftag(b, "b")
    if A_log is not None:
        args.A_log, args.A_log_dtype = A_log.data_ptr(), _ftag(A_log, "A_log")
    args.dt_bias, args.dt_bias_dtype = dt_bias.data_ptr(), _ftag(dt_bias, "dt_bias")
    if neg_exp_A is not None:
        if neg_exp_A.dtype != torch.float32:
            raise TypeError("neg_exp_A must be float32")
        args.neg_exp_A = neg_exp_A.data_ptr()
    args.anc_f32, args.anc_row_stride, args.anc_req_stride = _ptr(anc), anc_row, anc_req
    args.anc_bits = _ptr(anc_bits)
    args.state = state.data_ptr()
    args.state_slot_stride, args.state_h_stride = s_slot, s_h
    args.state_k_stride, args.state_v_stride = s_k, s_v
    args.state_indices, args.state_indices_dtype = _ptr(si), si_tag
    args.o, args.o_row_stride, args.o_h_stride, args.o_dtype = o.data_ptr(), o.stride(0), o.stride(1), _ftag(o, "o")
    if aux_k is not None:
        _check_aux(aux_k, "aux_k", torch.float32)
        args.aux_k, args.aux_k_h_stride, args.aux_k_row_stride = aux_k.data_ptr(), aux_k.stride(0), aux_k.stride(1)
    if aux_v is not None:
        _check_aux(aux_v, "aux_v", torch.float32)
        args.aux_v, args.aux_v_h_stride, args.aux_v_row_stride = aux_v.data_ptr(), aux_v.stride(0), aux_v.stride(1)
    if aux_g is not None:
        _check_aux(aux_g, "aux_g", torch.float32, dims=2)
        args.aux_g, args.aux_g_h_stride, args.aux_g_row_stride = aux_g.data_ptr(), aux_g.stride(0), aux_g.stride(1)
    args.status = _status_ptr(status, batch, dev)
    if size_order is not None:
        if cu_seqlens is None:
            raise ValueError("size_order goes with a packed batch (cu_seqlens)")
        _check_size_order(size_order, batch, dev)
        _check_size_order_source(size_order, cu_given, n_nodes, batch)
        args.size_order = size_order.data_ptr()
    return args, o, dev, (y, cu_seqlens, anc, anc_bits, si)


def tree_commit_verify(y: torch.Tensor, a: torch.Tensor, b: torch.Tensor, A_log: Optional[torch.Tensor],
                       dt_bias: torch.Tensor, state: torch.Tensor, *, hk: int, hv: int,
                       pending_path: torch.Tensor, pending_keys: Optional[torch.Tensor],
                       pending_values: Optional[torch.Tensor], pending_gains: torch.Tensor,
                       pending_path_len: Optional[torch.Tensor] = None,
                       pending_key_rows: Optional[torch.Tensor] = None,
                       pending_value_rows: Optional[torch.Tensor] = None, pending_b: Optional[torch.Tensor] = None,
                       prev_cu_seqlens: Optional[torch.Tensor] = None, prev_n_nodes: Optional[int] = None,
                       pending_k_head_div: int = 1, anc: Optional[torch.Tensor] = None,
                       anc_bits: Optional[torch.Tensor] = None, batch: Optional[int] = None,
                       n_nodes: Optional[int] = None, cu_seqlens: Optional[torch.Tensor] = None,
                       scale: Optional[float] = None, neg_exp_A: Optional[torch.Tensor] = None,
                       state_indices: Optional[torch.Tensor] = None, state_slot_stride: Optional[int] = None,
                       o: Optional[torch.Tensor] = None, o_dtype: Optional[torch.dtype] = None,
                       aux_k: Optional[torch.Tensor] = None, aux_v: Optional[torch.Tensor] = None,
                       aux_g: Optional[torch.Tensor] = None, aux_k_per_khead: bool = False,
                       status: Optional[torch.Tensor] = None,
                       size_order: Optional[torch.Tensor] = None,
                       pending_anc_bits: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``tree_verify`` with the previous step's accepted path committed into
    each request's state slot on the way in (one read of the state, one
    write back).  The pending_* tensors are the previous step's saves
    (keys [hv or hk, rows, 128], values [hv, rows, 128], gains [hv, rows])
    and its accepted path [batch, P <= 16] (-1 padded); they must not alias
    this step's aux outputs.  Instead of saved keys (pending_keys None),
    ``pending_key_rows`` may give the previous step's raw bf16 key rows
    [rows, hk, 128], e.g. ``prev_y[:, hk*128:2*hk*128].unflatten(1, (hk, 128))``,
    which the commit normalises itself: the verify then needs no aux_k.
    Likewise, instead of saved values (pending_values None), the commit can
    recompute the path's values from the previous step's raw bf16 value rows
    ``pending_value_rows`` [rows, hv, 128] (``prev_y[:, 2*hk*128:]``) and b
    gates ``pending_b`` [rows, hv], with the state the slot holds: then the
    verify needs no aux_v.  That form requires every pending path to be a
    walk from its tree's root (each entry's ancestors are the entries before
    it), as an accepted path is, and the slot to hold the state the previous
    verify read.  Previous rows of request b start at prev_cu_seqlens[b] or
    b * prev_n_nodes.  Returns o.  ``status`` and ``size_order`` as in
    ``tree_verify``; status adds DFT_STATUS_PATH for a pending entry past the
    previous tree (the entry is ignored).  ``pending_anc_bits``: the previous
    step's ancestry rows (``tree_struct(..., want=("anc_bits",))`` of that
    step); with them a path whose valid entries are not a walk down from the
    root is not committed, and its request gets DFT_STATUS_WALK.
    With ``n_nodes=0`` (every request's tree empty) the launch only commits
    the pending paths: the flush of requests that leave the batch."""
    args, o, dev, _keep = _verify_args(
        y, a, b, A_log, dt_bias, state, hk=hk, hv=hv, anc=anc, anc_bits=anc_bits, batch=batch, n_nodes=n_nodes,
        cu_seqlens=cu_seqlens, scale=scale, neg_exp_A=neg_exp_A, state_indices=state_indices,
        state_slot_stride=state_slot_stride, o=o, o_dtype=o_dtype, aux_k=aux_k, aux_v=aux_v, aux_g=aux_g,
        aux_k_per_khead=aux_k_per_khead, status=status, size_order=size_order)
    _device_of(pending_path, pending_keys, pending_key_rows, pending_values, pending_value_rows, pending_b,
               pending_gains, pending_path_len, prev_cu_seqlens, y)
    if (pending_keys is None) == (pending_key_rows is None):
        raise ValueError("give either pending_keys or pending_key_rows")
    if (pending_values is None) == (pending_value_rows is None):
        raise ValueError("give either pending_values or pending_value_rows")
    if (pending_value_rows is None) != (pending_b is None):
        raise ValueError("pending_value_rows and pending_b go together")
    for t, nm, dims in ((pending_keys, "pending_keys", 3), (pending_values, "pending_values", 3),
                        (pending_gains, "pending_gains", 2)):
        if t is not None:
            _check_aux(t, nm, torch.float32, dims=dims)
    for t, nm in ((pending_key_rows, "pending_key_rows"), (pending_value_rows, "pending_value_rows")):
        if t is not None:
            _check_aux(t, nm, torch.bfloat16, dims=3)
            if t.shape[-1] != 128:
                raise ValueError(f"{nm} is [rows, heads, 128]")
    if pending_b is not None and (pending_b.dim() != 2 or pending_b.stride(1) != 1):
        raise ValueError("pending_b is [rows, hv] with unit stride along hv")
    saves = [t for t in (pending_keys, pending_values, pending_gains) if t is not None]
    for out in (aux_k, aux_v, aux_g):
        if out is not None and any(out.data_ptr() == t.data_ptr() for t in saves):
            raise ValueError("the pending saves must not alias this step's aux outputs")
    path = pending_path.unsqueeze(0) if pending_path.dim() == 1 else pending_path
    if path.stride(1) != 1:
        path = path.contiguous()
    if path.shape[1] > 16 or path.shape[1] < 1:
        raise ValueError("pending paths hold 1 to 16 entries")
    c = PendingArgs()
    c.path_cols, c.k_head_div = path.shape[1], pending_k_head_div
    c.path, c.path_req_stride, c.path_dtype = path.data_ptr(), path.stride(0), _itag(path, "pending_path")
    pl, c.path_len_dtype = _idx_vec(pending_path_len, "pending_path_len")
    c.path_len = _ptr(pl)
    if prev_cu_seqlens is not None:
        if prev_cu_seqlens.dtype != torch.int32:
            raise TypeError("prev_cu_seqlens must be int32")
        prev_cu_seqlens = prev_cu_seqlens.contiguous()
        c.prev_cu_seqlens = prev_cu_seqlens.data_ptr()
    else:
        if prev_n_nodes is None:
            raise ValueError("give prev_cu_seqlens or prev_n_nodes")
        c.prev_n_nodes = prev_n_nodes
    if pending_keys is not None:
        c.keys, c.k_h_stride, c.k_row_stride = pending_keys.data_ptr(), *pending_keys.stride()[:2]
    else:  # [rows, heads, 128]: row stride first
        c.key_rows = pending_key_rows.data_ptr()
        c.kr_row_stride, c.kr_h_stride = pending_key_rows.stride(0), pending_key_rows.stride(1)
    if pending_values is not None:
        c.values, c.v_h_stride, c.v_row_stride = pending_values.data_ptr(), *pending_values.stride()[:2]
    else:  # [rows, hv, 128]: row stride first
        c.value_rows = pending_value_rows.data_ptr()
        c.vr_row_stride, c.vr_h_stride = pending_value_rows.stride(0), pending_value_rows.stride(1)
        c.prev_b, c.pb_row_stride = pending_b.data_ptr(), pending_b.stride(0)
        c.prev_b_dtype = _ftag(pending_b, "pending_b")
    c.gains, c.g_h_stride, c.g_row_stride = pending_gains.data_ptr(), *pending_gains.stride()
    if pending_anc_bits is not None:
        if pending_anc_bits.dtype != torch.int64:
            raise TypeError("pending_anc_bits must be int64 (uint64 bit masks)")
        if pending_anc_bits.device != dev:
            raise ValueError(f"pending_anc_bits is on {pending_anc_bits.device}, the inputs on {dev}")
        pending_anc_bits = pending_anc_bits.contiguous()
        c.prev_anc_bits = pending_anc_bits.data_ptr()
    check("dft_tree_commit_verify", load().dft_tree_commit_verify(C.byref(args), C.byref(c), _stream(dev)))
    return o


def _check_aux(t, name, dtype, dims=3):
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}")
    if t.dim() != dims or (dims == 3 and t.stride(-1) != 1):
        raise ValueError(f"{name} has the wrong shape or strides: {tuple(t.shape)} {t.stride()}")


# ---------------------------------------------------------------------------
# tree conv
# ---------------------------------------------------------------------------
def tree_conv(x: torch.Tensor, conv_state: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
              cidx: torch.Tensor, *, silu: bool = True, cs_indices: Optional[torch.Tensor] = None,
              y: Optional[torch.Tensor] = None, iw: Optional[torch.Tensor] = None,
              iw_indices: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Tree-parent causal conv1d over a batch of trees.

    x [batch, N, C] pre-conv tokens (any strides); conv_state [slots, C, >=W-1]
    or [C, >=W-1]; weight [C, W]; bias [C] or None; cidx [batch, N, W] or
    [N, W] (shared).  Writes y [batch, N, C] (x.dtype by default) and, when
    given, the window iw [islots, N, C, W-1].
    """
    dev = _device_of(x, conv_state, weight, bias, cidx, cs_indices, y, iw, iw_indices)
    if x.dim() == 2:
        x = x.unsqueeze(0)
    B, N, Cn = x.shape
    W = weight.shape[-1]
    if weight.dim() != 2 or weight.shape[0] != Cn:
        raise ValueError(f"weight must be [C, W] = [{Cn}, W]")
    cs = conv_state if conv_state.dim() == 3 else conv_state.unsqueeze(0)
    if cs.shape[1] != Cn or cs.shape[2] < W - 1:
        raise ValueError("conv_state must be [slots, C, >=W-1]")
    if conv_state.dim() == 2 and cs_indices is not None:
        raise ValueError("a 2-D conv_state has a single slot")
    ci = cidx if cidx.dim() == 3 else cidx.unsqueeze(0)
    if ci.shape[1] != N or ci.shape[2] != W or ci.stride(2) != 1:
        ci = ci.contiguous()
        if ci.shape[1] != N or ci.shape[2] != W:
            raise ValueError(f"cidx must be [batch, {N}, {W}] or [{N}, {W}]")
    ci_req = ci.stride(0) if ci.shape[0] == B else 0
    if ci.shape[0] not in (1, B):
        raise ValueError("cidx batch must be 1 or match x")
    if y is None:
        y = torch.empty(B, N, Cn, device=dev, dtype=x.dtype)
    y3 = y if y.dim() == 3 else y.view(B, N, Cn)
    if y3.stride(2) != 1:
        raise ValueError("y must have channel stride 1")
    a = ConvArgs()
    a.batch, a.n_nodes, a.channels, a.width, a.silu = B, N, Cn, W, int(bool(silu))
    a.x, a.x_req_stride, a.x_node_stride, a.x_chan_stride = x.data_ptr(), x.stride(0), x.stride(1), x.stride(2)
    a.x_dtype = _ftag(x, "x")
    a.conv_state, a.cs_slot_stride, a.cs_chan_stride, a.cs_col_stride = cs.data_ptr(), *cs.stride()
    a.cs_dtype = _ftag(cs, "conv_state")
    csi, a.cs_indices_dtype = _idx_vec(cs_indices, "cs_indices")
    a.cs_indices = _ptr(csi)
    a.weight, a.w_chan_stride, a.w_tap_stride, a.w_dtype = weight.data_ptr(), *weight.stride(), _ftag(weight, "weight")
    if bias is not None:
        a.bias, a.bias_dtype = bias.data_ptr(), _ftag(bias, "bias")
    a.cidx, a.cidx_req_stride, a.cidx_node_stride, a.cidx_dtype = ci.data_ptr(), ci_req, ci.stride(1), _itag(ci, "cidx")
    a.y, a.y_req_stride, a.y_node_stride, a.y_dtype = y3.data_ptr(), y3.stride(0), y3.stride(1), _ftag(y3, "y")
    if iw is not None:
        if iw.dim() != 4 or iw.shape[1] < N or iw.shape[2] != Cn or iw.shape[3] < W - 1:
            raise ValueError("iw must be [islots, N, C, W-1]")
        a.iw, a.iw_slot_stride, a.iw_node_stride, a.iw_chan_stride, a.iw_col_stride = iw.data_ptr(), *iw.stride()
        a.iw_dtype = _ftag(iw, "iw")
    iwi, a.iw_indices_dtype = _idx_vec(iw_indices, "iw_indices")
    a.iw_indices = _ptr(iwi)
    check("dft_tree_conv", load().dft_tree_conv(C.byref(a), _stream(dev)))
    return y


# ---------------------------------------------------------------------------
# commit
# ---------------------------------------------------------------------------
def tree_commit(src: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, gains: torch.Tensor,
                path: torch.Tensor, *, n_nodes: int, path_len: Optional[torch.Tensor] = None,
                len_is_last: bool = False, ends: Optional[torch.Tensor] = None,
                anc: Optional[torch.Tensor] = None, anc_bits: Optional[torch.Tensor] = None,
                cu_seqlens: Optional[torch.Tensor] = None, src_slots: Optional[torch.Tensor] = None,
                dst: Optional[torch.Tensor] = None, dst_slots: Optional[torch.Tensor] = None,
                kv_layout: bool = False, k_head_div: int = 1, status: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Closed-form commit of the accepted path for every (layer, request, head).

    src: states [L, slots, H, rows=V, cols=K] (pool layout; ``kv_layout=True``
    for [.., K, V]); keys [L, H', T, 128], values [L, H, T, 128], gains
    [L, H, T] as saved by ``tree_verify`` (T = total node rows); path
    [batch, P] accepted local node ids (-1 padded).  In place when ``dst`` is
    None; otherwise dst is [L, dslots, N, H, rows, cols] and receives S_u at
    node u for every end in ``ends`` [batch, E] (-1 = skip).  ``anc`` /
    ``anc_bits`` restrict the sum to ancestors of u (fc1_fused.py:41).
    ``status`` (int32 [batch]) receives every request's DFT_STATUS_* bits.
    """
    dev = _device_of(src, keys, values, gains, path, path_len, ends, anc, anc_bits, cu_seqlens,
                     src_slots, dst, dst_slots)
    if src.dim() != 5 or tuple(src.shape[-2:]) != (D_HEAD, D_HEAD):
        raise ValueError("src must be [L, slots, H, 128, 128]")
    L, _, H = src.shape[:3]
    for t, nm in ((src, "src"), (keys, "keys"), (values, "values"), (gains, "gains")):
        if t.dtype != torch.float32:
            raise TypeError(f"{nm} must be float32")
    if keys.dim() != 4 or values.dim() != 4 or gains.dim() != 3:
        raise ValueError("keys/values must be [L, H, rows, 128], gains [L, H, rows]")
    if keys.stride(-1) != 1 or values.stride(-1) != 1:
        raise ValueError("keys/values need stride 1 along the head dim")
    if path.dim() == 1:
        path = path.unsqueeze(0)
    if path.stride(1) != 1:
        path = path.contiguous()
    B, P = path.shape
    if P > MAX_NODES or n_nodes > MAX_NODES:
        raise ValueError(f"paths and trees are limited to {MAX_NODES} nodes")
    if P < 1:
        raise ValueError("a path holds at least one entry (-1 for none)")
    a = CommitArgs()
    a.n_layers, a.batch, a.hv, a.dk, a.dv = L, B, H, D_HEAD, D_HEAD
    a.n_nodes, a.path_cols = n_nodes, P
    a.k_head_div = k_head_div
    flags = _lib.DFT_COMMIT_KV if kv_layout else 0
    if len_is_last:
        flags |= _lib.DFT_COMMIT_LEN_IS_LAST
    a.path, a.path_req_stride, a.path_dtype = path.data_ptr(), path.stride(0), _itag(path, "path")
    pl, a.path_len_dtype = _idx_vec(path_len, "path_len")
    a.path_len = _ptr(pl)
    if ends is not None:
        if ends.dim() == 1:
            ends = ends.unsqueeze(1) if B > 1 or ends.numel() == 1 else ends.unsqueeze(0)
        ends = ends.contiguous()
        a.n_ends = ends.shape[1]
        a.ends, a.ends_req_stride, a.ends_dtype = ends.data_ptr(), ends.stride(0), _itag(ends, "ends")
    else:
        a.n_ends = 1
    if anc is not None or anc_bits is not None:
        flags |= _lib.DFT_COMMIT_CHECK_ANC
        if anc_bits is not None:
            if anc_bits.dtype != torch.int64:
                raise TypeError("anc_bits must be int64")
            anc_bits = anc_bits.contiguous()
            a.anc_bits = anc_bits.data_ptr()
        else:
            anc = anc.float().contiguous()
            a.anc_f32, a.anc_row_stride = anc.data_ptr(), anc.stride(-2)
            a.anc_req_stride = anc.stride(0) if anc.dim() == 3 else 0
    a.flags = flags
    if cu_seqlens is not None:
        if cu_seqlens.dtype != torch.int32:
            raise TypeError("cu_seqlens must be int32")
        cu_seqlens = cu_seqlens.contiguous()
        a.cu_seqlens = cu_seqlens.data_ptr()
    a.keys, a.k_layer_stride, a.k_h_stride, a.k_row_stride = keys.data_ptr(), *keys.stride()[:3]
    a.values, a.v_layer_stride, a.v_h_stride, a.v_row_stride = values.data_ptr(), *values.stride()[:3]
    a.gains, a.g_layer_stride, a.g_h_stride, a.g_row_stride = gains.data_ptr(), *gains.stride()
    a.src = src.data_ptr()
    (a.src_layer_stride, a.src_slot_stride, a.src_h_stride, a.src_row_stride, a.src_col_stride) = src.stride()
    ss, a.src_slots_dtype = _idx_vec(src_slots, "src_slots")
    a.src_slots = _ptr(ss)
    if dst is None:
        a.dst = a.src
        (a.dst_layer_stride, a.dst_slot_stride, a.dst_h_stride, a.dst_row_stride, a.dst_col_stride) = src.stride()
        a.dst_node_stride = 0
        if a.n_ends != 1:
            raise ValueError("an in-place commit takes one end per request")
    else:
        if dst.dim() != 6 or tuple(dst.shape[-2:]) != (D_HEAD, D_HEAD) or dst.dtype != torch.float32:
            raise ValueError("dst must be float32 [L, slots, N, H, 128, 128]")
        a.dst = dst.data_ptr()
        (a.dst_layer_stride, a.dst_slot_stride, a.dst_node_stride, a.dst_h_stride, a.dst_row_stride,
         a.dst_col_stride) = dst.stride()
    ds, a.dst_slots_dtype = _idx_vec(dst_slots, "dst_slots")
    a.dst_slots = _ptr(ds)
    a.status = _status_ptr(status, B, dev)
    check("dft_tree_commit", load().dft_tree_commit(C.byref(a), _stream(dev)))
    return src if dst is None else dst


# ---------------------------------------------------------------------------
# tree structure and the standalone inverse
# ---------------------------------------------------------------------------
def tree_struct(parent: torch.Tensor, kc: int = 4, *, batch: Optional[int] = None,
                n_nodes: Optional[int] = None, cu_seqlens: Optional[torch.Tensor] = None,
                want=("anc_bits", "anc", "depth", "cidx", "nxt", "sib", "status"),
                index_dtype: torch.dtype = torch.int64) -> dict:
    """Ancestor bits / dense Anc / depth / cidx / nxt / sib of a batch of trees
    given by parent indices [rows] (or [batch, N])."""
    dev = _device_of(parent, cu_seqlens)
    if parent.dim() == 2:
        batch, n_nodes = parent.shape
        parent = parent.reshape(-1)
    parent = parent.contiguous()
    rows = parent.numel()
    if cu_seqlens is not None:
        batch = cu_seqlens.numel() - 1 if batch is None else batch
        if n_nodes is None:
            raise ValueError("packed input needs n_nodes (the largest request)")
        cu_seqlens = cu_seqlens.contiguous()
    else:
        if batch is None and n_nodes is None:
            batch, n_nodes = 1, rows
        elif n_nodes is None:
            n_nodes = rows // batch
        elif batch is None:
            batch = rows // max(n_nodes, 1)
    if n_nodes > MAX_NODES:
        raise ValueError(f"at most {MAX_NODES} nodes per tree")
    out = {}
    a = TreeArgs()
    a.batch, a.n_nodes, a.kc = batch, n_nodes, kc
    a.parent, a.parent_dtype = parent.data_ptr(), _itag(parent, "parent")
    a.cu_seqlens = _ptr(cu_seqlens)
    if "anc_bits" in want:
        out["anc_bits"] = torch.zeros(rows, device=dev, dtype=torch.int64)
        a.anc_bits = out["anc_bits"].data_ptr()
    if "anc" in want:
        out["anc"] = torch.zeros(batch, n_nodes, n_nodes, device=dev, dtype=torch.float32)
        a.anc_f32, a.anc_row_stride, a.anc_req_stride = out["anc"].data_ptr(), n_nodes, n_nodes * n_nodes
    if "depth" in want:
        out["depth"] = torch.empty(rows, device=dev, dtype=index_dtype)
        a.depth, a.depth_dtype = out["depth"].data_ptr(), _itag(out["depth"], "depth")
    if "cidx" in want:
        out["cidx"] = torch.empty(rows, kc, device=dev, dtype=index_dtype)
        a.cidx, a.cidx_dtype = out["cidx"].data_ptr(), _itag(out["cidx"], "cidx")
    a.link_dtype = _INDEX_TAG[index_dtype]
    if "nxt" in want:
        out["nxt"] = torch.empty(rows, device=dev, dtype=index_dtype)
        a.nxt = out["nxt"].data_ptr()
    if "sib" in want:
        out["sib"] = torch.empty(rows, device=dev, dtype=index_dtype)
        a.sib = out["sib"].data_ptr()
    if "status" in want:
        out["status"] = torch.empty(batch, device=dev, dtype=torch.int32)
        a.status = out["status"].data_ptr()
    check("dft_tree_struct", load().dft_tree_struct(C.byref(a), _stream(dev)))
    return out


def anc_pack(anc: torch.Tensor, *, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Dense 0/1 ancestry [N, N] or [batch, N, N] (any float dtype cast to
    fp32 first) -> int64 bit rows [batch * N]: bit j of row i = anc[i][j] >
    0.5 for j <= i.  With `out` nothing is allocated (for a fp32 input with
    unit column stride)."""
    dev = _device_of(anc, out)
    a3 = anc if anc.dim() == 3 else anc.unsqueeze(0)
    if a3.dim() != 3 or a3.shape[1] != a3.shape[2] or a3.shape[1] > MAX_NODES:
        raise ValueError(f"anc must be [N, N] or [batch, N, N] with N <= {MAX_NODES}")
    if a3.dtype != torch.float32 or a3.stride(2) != 1:
        a3 = a3.float().contiguous()
    B, n = a3.shape[0], a3.shape[1]
    if out is None:
        out = torch.empty(B * n, device=dev, dtype=torch.int64)
    if out.dtype != torch.int64 or not out.is_contiguous() or out.numel() < B * n:
        raise ValueError(f"out must be a contiguous int64 tensor of at least {B * n} entries")
    a = AncPackArgs()
    a.batch, a.n_nodes = B, n
    a.anc, a.anc_row_stride, a.anc_req_stride = a3.data_ptr(), a3.stride(1), a3.stride(0)
    a.anc_bits = out.data_ptr()
    check("dft_anc_pack", load().dft_anc_pack(C.byref(a), _stream(dev)))
    return out


def block_inverse_(x: torch.Tensor) -> torch.Tensor:
    """In place: x[..., n, n] (strictly-lower A, fp32) <- (I + A)^-1, n <= 64."""
    dev = _device_of(x)
    if x.dtype != torch.float32 or x.dim() < 2 or x.shape[-1] != x.shape[-2]:
        raise ValueError("x must be float32 [..., n, n]")
    if not x.is_contiguous():
        raise ValueError("x must be contiguous (it is updated in place)")
    n = x.shape[-1]
    mats = x.numel() // max(n * n, 1)
    check("dft_block_inverse", load().dft_block_inverse(x.data_ptr(), mats, n, n * n, _stream(dev)))
    return x


# ---------------------------------------------------------------------------
# bit-packed attention masks (fc1_plan.py:26, fc1_branch64.py:39)
# ---------------------------------------------------------------------------
_BIT_ORDER = {"little": DFT_BITS_LITTLE, "big": DFT_BITS_BIG}


def _bit_order(bitorder: str) -> int:
    try:
        return _BIT_ORDER[bitorder]
    except KeyError:
        raise ValueError(f"bitorder must be 'little' or 'big', got {bitorder!r}") from None


def _byte_view(x: torch.Tensor, name: str) -> torch.Tensor:
    if x.dtype not in (torch.bool, torch.uint8, torch.int8):
        raise TypeError(f"{name}: expected a bool or uint8 tensor, got {x.dtype}")
    x = x.reshape(-1)
    if not x.is_contiguous():
        x = x.contiguous()
    return x.view(torch.uint8)


def _out_bytes(out: Optional[torch.Tensor], nbytes: Optional[int], dev) -> torch.Tensor:
    if out is None:
        return torch.empty(nbytes, device=dev, dtype=torch.uint8)
    if out.dtype != torch.uint8 or not out.is_contiguous():
        raise TypeError("out: expected a contiguous uint8 tensor")
    if out.device != dev:
        raise ValueError(f"out is on {out.device}, the input on {dev}")
    return out


def packbits(x: torch.Tensor, bitorder: str = "little", *, out: Optional[torch.Tensor] = None,
             status: Optional[torch.Tensor] = None) -> torch.Tensor:
    """flashinfer.packbits (as fc1_plan.py:26 calls it): x (bool / uint8, any
    shape) flattened and packed 8 elements per byte with numpy.packbits
    semantics; returns the ceil(x.numel() / 8) bytes.  With `out` the bytes
    are written into it (no allocation; bytes past its end are dropped and
    `status` is set to 1)."""
    dev = _device_of(x, out, status)
    xb = _byte_view(x, "x")
    nbytes = (xb.numel() + 7) // 8
    o = _out_bytes(out, nbytes, dev)
    a = PackbitsArgs()
    a.n_segments, a.bit_order = 1, _bit_order(bitorder)
    a.x, a.n = xb.data_ptr(), xb.numel()
    a.out, a.out_capacity = o.data_ptr(), o.numel()
    a.status = _ptr(status)
    if xb.numel():
        check("dft_packbits", load().dft_packbits(C.byref(a), _stream(dev)))
    return o if out is None else o[:nbytes]


def segment_packbits(x: torch.Tensor, indptr: torch.Tensor, bitorder: str = "little", *,
                     out: Optional[torch.Tensor] = None, out_indptr: Optional[torch.Tensor] = None,
                     status: Optional[torch.Tensor] = None):
    """flashinfer.segment_packbits: segment s = x[indptr[s]:indptr[s+1]] is
    packed on its own; returns (packed, new_indptr) with new_indptr[s] the
    byte offset of segment s.  Without `out` the total size is read back to
    the host once (as flashinfer does); with `out` nothing is."""
    dev = _device_of(x, indptr, out, out_indptr, status)
    xb = _byte_view(x, "x")
    ip, ip_tag = _idx_vec(indptr, "indptr")
    segs = ip.numel() - 1
    if segs < 0:
        raise ValueError("indptr needs at least one entry")
    if out is None:
        lens = (ip[1:] - ip[:-1]).clamp_min(0).to(torch.int64)
        out = torch.empty(int(((lens + 7) // 8).sum().item()), device=dev, dtype=torch.uint8)
    else:
        out = _out_bytes(out, None, dev)
    if out_indptr is None:
        out_indptr = torch.zeros(segs + 1, device=dev, dtype=ip.dtype)
    a = PackbitsArgs()
    a.n_segments, a.bit_order = segs, _bit_order(bitorder)
    a.x, a.n = xb.data_ptr(), xb.numel()
    a.indptr, a.indptr_dtype = ip.data_ptr(), ip_tag
    a.out, a.out_capacity = out.data_ptr(), out.numel()
    a.out_indptr, a.out_indptr_dtype = out_indptr.data_ptr(), _itag(out_indptr, "out_indptr")
    a.status = _ptr(status)
    if segs:
        check("dft_packbits", load().dft_packbits(C.byref(a), _stream(dev)))
    return out, out_indptr


def tree_mask_pack(anc_bits: torch.Tensor, prefix_len: torch.Tensor, *, batch: Optional[int] = None,
                   n_nodes: Optional[int] = None, cu_seqlens: Optional[torch.Tensor] = None,
                   bitorder: str = "little", out: Optional[torch.Tensor] = None,
                   out_indptr: Optional[torch.Tensor] = None, status: Optional[torch.Tensor] = None):
    """The packed tree attention mask, straight from the ancestry bits.

    Request b (nodes row0(b) ..; n_b <= 64) with prefix_len[b] committed
    tokens contributes the row-major n_b x (plen_b + n_b) mask
    [ones(n_b, plen_b) | Anc_b] (fc1_branch64.py:39), packed as one segment
    (fc1_plan.py:26).  Returns (packed, mask_indptr).  Without `out` the
    total size is computed on the host from prefix_len and cu_seqlens (one
    read-back); the plan's preallocated buffer as `out` avoids it."""
    dev = _device_of(anc_bits, prefix_len, cu_seqlens, out, out_indptr, status)
    if anc_bits.dtype not in (torch.int64, torch.uint64) or not anc_bits.is_contiguous():
        raise TypeError("anc_bits: expected a contiguous 64-bit tensor (tree_struct's anc_bits)")
    pl, pl_tag = _idx_vec(prefix_len, "prefix_len")
    if cu_seqlens is not None:
        cu_seqlens = cu_seqlens.contiguous()
        if cu_seqlens.dtype != torch.int32:
            raise TypeError("cu_seqlens must be int32")
        batch = cu_seqlens.numel() - 1 if batch is None else batch
        n_nodes = MAX_NODES if n_nodes is None else n_nodes
    else:
        if batch is None:
            batch = pl.numel()
        if n_nodes is None:
            n_nodes = anc_bits.numel() // max(batch, 1)
    if n_nodes > MAX_NODES:
        raise ValueError(f"at most {MAX_NODES} nodes per tree")
    if pl.numel() < batch:
        raise ValueError(f"prefix_len has {pl.numel()} entries for {batch} requests")
    if out is None:
        if cu_seqlens is not None:
            n = (cu_seqlens[1:batch + 1] - cu_seqlens[:batch]).clamp(0, MAX_NODES).to(torch.int64)
        else:
            n = torch.full((batch,), n_nodes, device=dev, dtype=torch.int64)
        bits = n * (pl[:batch].to(torch.int64).clamp_min(0) + n)
        out = torch.empty(int(((bits + 7) // 8).sum().item()), device=dev, dtype=torch.uint8)
    else:
        out = _out_bytes(out, None, dev)
    if out_indptr is None:
        out_indptr = torch.zeros(batch + 1, device=dev, dtype=torch.int32)
    a = MaskArgs()
    a.batch, a.n_nodes, a.bit_order = batch, n_nodes, _bit_order(bitorder)
    a.cu_seqlens = _ptr(cu_seqlens)
    a.anc_bits = anc_bits.data_ptr()
    a.prefix_len, a.prefix_len_dtype = pl.data_ptr(), pl_tag
    a.out, a.out_capacity = out.data_ptr(), out.numel()
    a.out_indptr, a.out_indptr_dtype = out_indptr.data_ptr(), _itag(out_indptr, "out_indptr")
    a.status = _ptr(status)
    if batch:
        check("dft_tree_mask_pack", load().dft_tree_mask_pack(C.byref(a), _stream(dev)))
    return out, out_indptr
