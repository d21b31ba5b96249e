"""Drop-in for dforktree/fc1_fused.py on MI355X: the SGLang GDN adapter.

Keeps the reference's module surface -- ``NN``, ``BS``, ``Context``, ``CTX``,
``NATIVE_REFERENCE``, ``snapshots`` and ``install()`` (fc1_fused.py:4-97) --
and routes the three hooked SGLang entry points to the gfx950 library:

* ``TritonGDNKernel.target_verify``  -> ``tree_kernels.tree_gdn_split`` on the
  conv output stashed in ``CTX.current_mixed`` (fc1_fused.py:59-75); the
  first GDN layer of each forward packs ``CTX.anc`` into bit rows
  (``CTX.anc_bits``, one ``dft_anc_pack`` launch), which every layer's
  verify and the commit read instead of the dense matrix;
* ``commit_mamba_states_after_verify`` -> the snapshot commit into
  ``intermediate_ssm`` at the last / tracked accepted node, then SGLang's own
  commit copies it to the live state (fc1_fused.py:77-87);
* ``GDNAttnBackend._target_verify_supports_strided_qkv`` -> True for tree
  verifies of NN tokens (fc1_fused.py:91-95).

Shape guards fall back to the original SGLang functions exactly where the
reference does (``cache_steps != NN``, ``draft_token_num != NN``).  So does a
call the library refuses before launching anything (status
DFT_ERR_INVALID / DFT_ERR_UNSUPPORTED, e.g. a head dim other than 128), and
a verify whose layer has no conv output from the conv hook (that conv ran in
SGLang).  The commit then covers only the layers this module verified: the
others hold SGLang's own snapshots.  Unlike the reference's snapshot
kernel, an end of -1 (no tracked step) reads no state at all.
"""
from __future__ import annotations

import logging
import os

NN = int(os.environ.get('FC1_TREE_N', '64'))
BS = int(os.environ.get('FC1_DRAFT_BLOCK', '24'))

import torch  # noqa: E402

if __package__:
    from . import tree_kernels as TK
else:  # bare import from this directory (fc1_plugin's sys.path insert)
    import tree_kernels as TK
try:
    from dforktree_amd import _lib, ops as _ops
except ImportError:  # bare import, with the package itself not on sys.path
    import pathlib
    import sys
    sys.path.append(str(pathlib.Path(__file__).resolve().parents[2]))
    from dforktree_amd import _lib, ops as _ops

_log = logging.getLogger(__name__)

N_LAYERS = 24   # GDN layers of the target model (fc1_fused.py:15)
N_HEADS = 32    # GDN v-heads (fc1_fused.py:15)
D_HEAD = 128


class Context:
    """Per-process verify context (fc1_fused.py:12-20): the tree's ancestor
    matrix and, per GDN layer, the normalised keys, WY values and cumulative
    decays that the commit consumes."""

    def __init__(self, device='cuda'):
        self.anc = torch.eye(NN, device=device, dtype=torch.float32)
        # anc packed to bit rows, once per forward by the first layer's verify
        self.anc_bits = torch.zeros(NN, device=device, dtype=torch.int64)
        self.keys = torch.empty(N_LAYERS, N_HEADS, NN, D_HEAD, device=device)
        self.values = torch.empty_like(self.keys)
        self.gains = torch.empty(N_LAYERS, N_HEADS, NN, device=device)
        self.layers = {}
        self.inter_indices = None
        self.current_mixed = None  # the conv hook's [NN, C] output, consumed by the next verify
        self.saved = set()         # layers whose last verify ran here and saved keys/values/gains

    def layer(self, A_log):
        """Layer index by first sight of A_log's storage, plus the cached
        -exp(A_log) (fc1_fused.py:65-68)."""
        key = A_log.data_ptr()
        if key not in self.layers:
            self.layers[key] = (len(self.layers), -A_log.float().exp())
        return self.layers[key]


CTX = None
NATIVE_REFERENCE = False
COLLECT_LAYER = False
LAYER_STATS = []


def snapshot_commit(temporal, keys, values, gains, anc, accept_index, ends, slots, inter_indices,
                    intermediate_ssm, anc_bits=None):
    """fc1_fused.py:26-49 for every (layer, head, end):
    intermediate_ssm[l, dst, u, h] = e^{G_u} S + sum_t on_t e^{G_u-G_t} k_t vn_t^T,
    on_t = path node t is an ancestor-or-self of u; u in ``ends`` (-1 = skip).
    temporal [L, slots, H, V, K]; keys/values [>=L, H, NN, 128];
    accept_index [batch, P] (-1 padded); ends [batch*E] or [batch, E].
    ``anc_bits`` (anc packed to rows) replaces the dense anc when given."""
    L = temporal.shape[0]
    Bq = accept_index.shape[0] if accept_index.dim() == 2 else 1
    n = anc.shape[-1]
    tree = dict(anc=anc) if anc_bits is None else dict(anc_bits=anc_bits)
    _ops.tree_commit(temporal, keys[:L], values[:L], gains[:L], accept_index.reshape(Bq, -1), n_nodes=n,
                     ends=ends.reshape(Bq, -1), src_slots=slots, dst=intermediate_ssm, dst_slots=inter_indices,
                     **tree)


class _Snapshots:
    """Keeps the reference's launch form ``snapshots[grid](S, K, V, G, A, Path,
    Ends, Slot, InterSlot, Out, NN, BS, *strides)``; grid and strides come
    from the tensors themselves."""

    def __getitem__(self, grid):
        def launch(S, K, V, G, A, Path, Ends, Slot, InterSlot, Out, nn_, bs_, *strides, num_warps=4):
            path = Path.reshape(Path.shape[0] if Path.dim() == 2 else 1, -1)[:, :int(bs_)]
            snapshot_commit(S, K, V, G, A, path, Ends, Slot, InterSlot, Out)
        return launch


snapshots = _Snapshots()


def _context():
    global CTX
    if CTX is None:
        CTX = Context()
    return CTX


def refused(err) -> bool:
    """True for a library status that launched nothing and names a request
    this build does not take (DFT_ERR_INVALID, DFT_ERR_UNSUPPORTED): the hook
    hands such a call to SGLang's own function, as the reference's guards do
    (fc1_fused.py:61-62, :92-94; fc1_conv.py:34-35)."""
    if isinstance(err, _lib.DftError) and err.status in (_lib.DFT_ERR_INVALID, _lib.DFT_ERR_UNSUPPORTED):
        _log.warning("dforktree_amd: %s; running SGLang's own kernel instead", err)
        return True
    return False


def layer_runs(layers):
    """Sorted layer indices as [start, stop) runs of consecutive layers."""
    runs = []
    for li in sorted(layers):
        if runs and runs[-1][1] == li:
            runs[-1][1] = li + 1
        else:
            runs.append([li, li + 1])
    return [tuple(r) for r in runs]


def install():
    """Patch SGLang's GDN verify, mamba commit and routing (fc1_fused.py:51-97)."""
    from sglang.srt.layers.attention.linear.kernels.gdn_triton import TritonGDNKernel
    from sglang.srt.speculative import eagle_worker_common as common
    from sglang.srt.speculative.spec_utils import _verify_commit_step_indices
    from sglang.srt.layers.attention.linear.gdn_backend import GDNAttnBackend
    original_verify = TritonGDNKernel.target_verify
    original_commit = common.commit_mamba_states_after_verify
    original_routing = GDNAttnBackend._target_verify_supports_strided_qkv

    def fused(self, A_log, dt_bias, q, k, v, a, b, **kw):
        if kw['cache_steps'] != NN:
            return original_verify(self, A_log, dt_bias, q, k, v, a, b, **kw)
        ctx = _context()
        li, neg = ctx.layer(A_log)
        assert li < N_LAYERS and q.shape[0] == 1 and q.shape[1] == NN
        if li == 0:
            # the first GDN layer of a forward: CTX.anc is this step's tree (fc1_branch64.py:29).  Packed
            # whatever this layer does, so that later layers and the commit never read the previous step's
            # rows (CTX.anc is a fixed [NN, NN] fp32 buffer: nothing to refuse)
            _ops.anc_pack(ctx.anc, out=ctx.anc_bits)
        # the conv hook's output for this layer; None when this layer's conv ran in SGLang
        y, ctx.current_mixed = ctx.current_mixed, None
        ctx.saved.discard(li)
        if y is None:
            return original_verify(self, A_log, dt_bias, q, k, v, a, b, **kw)
        pool = kw['ssm_states']
        try:
            out = TK.tree_gdn_split(y, a.reshape(NN, -1), b.reshape(NN, -1), A_log, dt_bias,
                                    pool[0].transpose(-1, -2), ctx.anc, q.shape[2], v.shape[2], q.shape[3],
                                    v.shape[3], aux=(ctx.keys[li], ctx.values[li], ctx.gains[li]), neg_exp_A=neg,
                                    state_indices=kw['cache_indices'], state_slot_stride=pool.stride(0),
                                    anc_bits=ctx.anc_bits)
        except _lib.DftError as err:
            if not refused(err):
                raise
            return original_verify(self, A_log, dt_bias, q, k, v, a, b, **kw)
        ctx.inter_indices = kw['intermediate_state_indices']
        ctx.saved.add(li)
        return out.unsqueeze(0)

    def fused_commit(target_worker, batch, accept_lens, accept_index, draft_token_num, prepared_step_indices=None):
        if CTX is not None and CTX.saved and draft_token_num == NN and accept_index.numel():
            last, track = _verify_commit_step_indices(batch=batch, accept_index=accept_index,
                                                      accept_lens=accept_lens, draft_token_num=draft_token_num)
            if track is None:
                track = torch.full_like(last, -1)
            ends = torch.stack((last.reshape(-1), track.reshape(-1)), 1)
            pool = target_worker.model_runner.req_to_token_pool
            state = pool.get_speculative_mamba2_params_all_layers()
            slots = pool.get_mamba_indices(batch.req_pool_indices)
            # Only the layers verified here have no snapshot from SGLang's own verify.  A refusal
            # here cannot fall back: those layers' snapshots would be missing, so it is raised.
            for l0, l1 in layer_runs(CTX.saved):
                snapshot_commit(state.temporal[l0:l1], CTX.keys[l0:l1], CTX.values[l0:l1], CTX.gains[l0:l1],
                                CTX.anc, accept_index, ends, slots, CTX.inter_indices,
                                state.intermediate_ssm[l0:l1], anc_bits=CTX.anc_bits)
        return original_commit(target_worker, batch, accept_lens, accept_index, draft_token_num, prepared_step_indices)

    def direct_routing(self, **kwargs):
        if not NATIVE_REFERENCE and kwargs['draft_token_num'] == NN:
            return True
        return original_routing(self, **kwargs)

    GDNAttnBackend._target_verify_supports_strided_qkv = direct_routing
    TritonGDNKernel.target_verify = fused
    common.commit_mamba_states_after_verify = fused_commit
