"""Benchmark of the GDN tree-verify hot path on one MI355X.

Workload (the state-bandwidth-bound stacked step): 24 GDN layers, batch 64,
one random recursive 32-node tree per request, 16 q/k heads, 32 v heads,
dk = dv = 128, a distinct fp32 2 MiB state per request per layer (3 GiB).
Every step verifies each layer's trees and commits each request's accepted
root-to-node path (length 1-16) into its state, for all 24 layers.  Two
schedules of that work are timed:

* pipelined (``value``): one launch per layer of dft_tree_commit_verify,
  which commits the previous step's accepted path into the state tile as it
  streams in, writes the committed tile back and verifies this step's tree
  on it (steady state: one commit and one verify per layer and step);
* separate: one dft_tree_verify launch per layer, then one dft_tree_commit
  launch for all layers, as the reference's hooks order them.

Inputs are resident in HBM before timing starts.  Printed: one JSON line.
``value`` = verified nodes / s / layer = batch * nodes / (step time / 24).
``roofline`` is for the kernel with the most time per step, from HIP-event
timing of the step (24 launches of that kernel); ``cpu_baseline`` times the
batched PyTorch fp32 CPU restatement (oracle/gdn_tree_torch.py, pinned
against the numpy oracle) on one layer of the same workload.  Beside the
headline: the launch with saved keys / values, the separate schedule, the
conv and mask kernels, the ragged batch, 64-node trees at batch 64 and the
batch-1 plugin path.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, vendor figure
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, vendor figure
B, L, N, HK, HV, D = 64, 24, 32, 16, 32, 128
MAX_PATH = 16


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-ragged", action="store_true", help="skip the packed ragged workload's line")
    ap.add_argument("--no-plugin", action="store_true", help="skip the batch-1 plugin path's line")
    ap.add_argument("--no-nn64", action="store_true", help="skip the 64-node trees' line")
    ap.add_argument("--only-plugin", action="store_true", help="time the batch-1 plugin path alone")
    ap.add_argument("--only-ragged", action="store_true", help="time the packed ragged workload alone")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of a HIP graph")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 1 GiB device copy (the reference point for HBM byte counters)")
    return ap.parse_args()


class Workload:
    """Device buffers of the stacked step; every tensor preallocated.  n:
    nodes per tree (32 for the headline; 64, the reference's default tree
    size FC1_TREE_N of fc1_fused.py:4, for its own line)."""

    def __init__(self, dev, seed=2, n=N):
        import torch
        from dforktree_amd import ops, synth
        self.n = n
        C = 2 * HK * D + HV * D
        rows = B * n
        self.rows = rows
        self.y = synth.device_randn_(torch.empty(L, rows, C, device=dev, dtype=torch.bfloat16), seed)
        # the previous step's y: the pipelined commit reads its raw k rows
        self.y_prev = synth.device_randn_(torch.empty(L, rows, C, device=dev, dtype=torch.bfloat16), seed + 7)
        self.a = synth.device_randn_(torch.empty(L, rows, HV, device=dev, dtype=torch.bfloat16), seed + 1)
        self.b = synth.device_randn_(torch.empty(L, rows, HV, device=dev, dtype=torch.bfloat16), seed + 2)
        # and its b gates, from which the pipelined commit can recompute the path's values
        self.b_prev = synth.device_randn_(torch.empty(L, rows, HV, device=dev, dtype=torch.bfloat16), seed + 8)
        self.A_log = torch.full((HV,), -0.6931471805599453, device=dev)
        self.dt_bias = torch.zeros(HV, device=dev)
        self.neg = -self.A_log.exp()
        # pool layout [layer, slot, head, V, K]
        self.state = synth.device_randn_(torch.empty(L, B, HV, D, D, device=dev), seed + 3, std=0.02)
        g = torch.Generator().manual_seed(seed)
        parents = [synth.tree_parents(n, "random", g) for _ in range(B)]
        paths = [synth.accepted_path(p, MAX_PATH, g) for p in parents]
        self.path_lens = [len(p) for p in paths]
        idx = torch.full((B, MAX_PATH), -1, dtype=torch.int32)
        for i, p in enumerate(paths):
            idx[i, :len(p)] = p
        self.accept = idx.to(dev)
        self.parent = torch.cat(parents).to(dev)
        self.anc_bits = ops.tree_struct(self.parent, 4, batch=B, n_nodes=n, want=("anc_bits",))["anc_bits"]
        self.o = torch.empty(L, rows, HV, D, device=dev, dtype=torch.bfloat16)
        self.keys = torch.empty(L, HK, rows, D, device=dev)   # one key set per k-head
        self.vals = torch.empty(L, HV, rows, D, device=dev)
        self.gains = torch.empty(L, HV, rows, device=dev)
        # the pipelined schedule reads the previous step's saves from one set
        # and writes this step's into the other
        self.keys2, self.vals2, self.gains2 = (torch.empty_like(t) for t in (self.keys, self.vals, self.gains))

    def verify(self, l):
        from dforktree_amd import ops
        ops.tree_verify(self.y[l], self.a[l], self.b[l], self.A_log, self.dt_bias, self.state[l].transpose(-1, -2),
                        hk=HK, hv=HV, anc_bits=self.anc_bits, batch=B, n_nodes=self.n, neg_exp_A=self.neg,
                        o=self.o[l], aux_k=self.keys[l], aux_v=self.vals[l], aux_g=self.gains[l], aux_k_per_khead=True)

    def commit(self):
        from dforktree_amd import ops
        ops.tree_commit(self.state, self.keys, self.vals, self.gains, self.accept, n_nodes=self.n, k_head_div=HV // HK)

    def step(self):
        for l in range(L):
            self.verify(l)
        self.commit()

    def fused(self, l, raw_keys=True, raw_values=True):
        """One layer of the pipelined schedule.  raw_keys: the commit reads the
        previous step's raw k rows from its y and normalises them, so this
        step's verify saves no keys; else it reads the previous step's saved
        keys and this step saves its own.  raw_values: likewise the commit
        recomputes the path's values from the previous step's raw v rows and
        b gates, so this step's verify saves no values."""
        from dforktree_amd import ops
        if raw_keys:
            keys = dict(pending_keys=None, aux_k=None,
                        pending_key_rows=self.y_prev[l][:, HK * D:2 * HK * D].unflatten(1, (HK, D)))
        else:
            keys = dict(pending_keys=self.keys[l], aux_k=self.keys2[l])
        if raw_values:
            keys.update(pending_values=None, aux_v=None, pending_b=self.b_prev[l],
                        pending_value_rows=self.y_prev[l][:, 2 * HK * D:].unflatten(1, (HV, D)))
        else:
            keys.update(pending_values=self.vals[l], aux_v=self.vals2[l])
        ops.tree_commit_verify(self.y[l], self.a[l], self.b[l], self.A_log, self.dt_bias,
                               self.state[l].transpose(-1, -2), hk=HK, hv=HV, anc_bits=self.anc_bits, batch=B,
                               n_nodes=self.n, neg_exp_A=self.neg, o=self.o[l], aux_g=self.gains2[l],
                               aux_k_per_khead=True, pending_path=self.accept, pending_gains=self.gains[l],
                               prev_n_nodes=self.n, pending_k_head_div=HV // HK, **keys)

    def fused_step(self):
        for l in range(L):
            self.fused(l)

    def conv_setup(self, dev, seed=5):
        """Front end of one layer: tree-parent conv1d (width 4, SiLU) over the
        pre-conv tokens, writing the verify input and each node's window."""
        import torch
        from dforktree_amd import ops, synth
        C = 2 * HK * D + HV * D
        self.cx = synth.device_randn_(torch.empty(B, N, C, device=dev, dtype=torch.bfloat16), seed)
        self.cw = synth.device_randn_(torch.empty(C, 4, device=dev, dtype=torch.bfloat16), seed + 1, std=0.1)
        self.cs = torch.zeros(B, C, 3, device=dev, dtype=torch.bfloat16)
        self.cidx = ops.tree_struct(self.parent, 4, batch=B, n_nodes=N, want=("cidx",),
                                    index_dtype=torch.int32)["cidx"].view(B, N, 4)
        self.cy = torch.empty(B, N, C, device=dev, dtype=torch.bfloat16)
        self.ciw = torch.empty(B, N, C, 3, device=dev, dtype=torch.bfloat16)

    def conv(self):
        from dforktree_amd import ops
        ops.tree_conv(self.cx, self.cs, self.cw, None, self.cidx, y=self.cy, iw=self.ciw)

    MASK_PREFIX = 4096  # committed tokens ahead of each request's draft tree

    def mask_setup(self, dev):
        """The attention layers' packed tree mask: ones over a 4096-token
        prefix, the ancestry over the 32 draft nodes, per request."""
        import torch
        self.mplen = torch.full((B,), self.MASK_PREFIX, device=dev, dtype=torch.int32)
        nbytes = B * ((N * (self.MASK_PREFIX + N) + 7) // 8)
        self.mout = torch.empty(nbytes, device=dev, dtype=torch.uint8)
        self.mind = torch.empty(B + 1, device=dev, dtype=torch.int32)

    def mask(self):
        from dforktree_amd import ops
        ops.tree_mask_pack(self.anc_bits, self.mplen, n_nodes=N, out=self.mout, out_indptr=self.mind)

    def mask_bytes_per_launch(self):
        # packed bytes written, ancestry words and prefix lengths read
        return B * ((N * (self.MASK_PREFIX + N) + 7) // 8 + N * 8 + 4)

    def conv_bytes_per_launch(self):
        C = 2 * HK * D + HV * D
        # tokens read once (parents' rows are re-gathered from cache), output and window written
        return B * (N * C * 2 + N * C * 2 + N * C * 3 * 2 + N * 4 * 4) + C * 4 * 2

    # ---- algorithmic bytes: every mandatory tensor touched once
    def verify_bytes_per_launch(self):
        C = 2 * HK * D + HV * D
        n = self.n
        per_req = (HV * D * D * 4          # S0 read
                   + n * C * 2             # y = [q|k|v] bf16 read
                   + 2 * n * HV * 2        # a, b bf16 read
                   + n * 8                 # ancestor bit masks
                   + n * HV * D * 2        # o bf16 write
                   + HV * n * D * 4        # vn fp32 write
                   + HV * n * 4            # G write
                   + HK * n * D * 4)       # normalised k fp32 write (per k-head)
        return B * per_req

    def fused_bytes_per_launch(self, raw_keys=True, raw_values=True):
        """verify bytes + the committed tile written back + the path's saves.
        raw_keys: no keys are saved, and the path's keys are read as raw bf16
        rows (per k-head) instead of saved fp32 ones.  raw_values: no values
        are saved, and the path's values are recomputed from raw bf16 v rows
        and bf16 b gates."""
        tot = 0
        for ell in self.path_lens:
            tot += (HV * D * D * 4                                # state write
                    + ell * HK * D * (2 if raw_keys else 4)      # path keys (per k-head)
                    + ell * HV * D * (2 if raw_values else 4)    # path values (raw v rows)
                    + (ell * HV * 2 if raw_values else 0)        # path b gates
                    + ell * HV * 4                               # path gains
                    + MAX_PATH * 4)                              # path indices
        key_saves = B * HK * self.n * D * 4 if raw_keys else 0
        value_saves = B * HV * self.n * D * 4 if raw_values else 0
        return self.verify_bytes_per_launch() - key_saves - value_saves + tot

    def commit_bytes_per_launch(self):
        tot = 0
        for ell in self.path_lens:
            tot += (2 * HV * D * D * 4           # state read + write
                    + ell * (HK + HV) * D * 4    # path keys (per k-head) and values
                    + (ell + 1) * HV * 4         # path and end gains
                    + MAX_PATH * 4)              # path indices
        return L * tot

    def state_bytes_per_step(self):
        return L * B * 3 * HV * D * D * 4   # verify read + commit read and write, as the separate kernels need

    def state_bytes_moved_pipelined(self):
        return L * B * 2 * HV * D * D * 4   # one read and one write per request-layer


class RaggedWorkload:
    """The packed ragged batch: 128 requests with trees of 8-64 nodes (a third
    each chains, bushy depth-2 trees and random recursive trees), 24 layers of
    distinct state; verify only.  With the size-order records one launch is
    the mixed-width kernel (the 33-64-node trees on the 64-wide body, then the
    others' v-head pairs on the 32-wide one); without them, two kernels."""
    RB = 128

    def __init__(self, dev, seed=3):
        import torch
        from dforktree_amd import ops, synth
        self.sizes, kinds = synth.ragged_sizes(self.RB, 8, 64, seed=seed)
        rows = sum(self.sizes)
        self.rows = rows
        C = 2 * HK * D + HV * D
        self.y = synth.device_randn_(torch.empty(L, rows, C, device=dev, dtype=torch.bfloat16), seed + 10)
        self.a = synth.device_randn_(torch.empty(L, rows, HV, device=dev, dtype=torch.bfloat16), seed + 11)
        self.b = synth.device_randn_(torch.empty(L, rows, HV, device=dev, dtype=torch.bfloat16), seed + 12)
        self.A_log = torch.full((HV,), -0.6931471805599453, device=dev)
        self.dt_bias = torch.zeros(HV, device=dev)
        self.neg = -self.A_log.exp()
        self.state = synth.device_randn_(torch.empty(L, self.RB, HV, D, D, device=dev), seed + 13, std=0.02)
        g = torch.Generator().manual_seed(seed)
        parents = torch.cat([synth.tree_parents(n, k, g) for n, k in zip(self.sizes, kinds)]).to(dev)
        self.cu = torch.tensor([0] + torch.tensor(self.sizes).cumsum(0).tolist(), dtype=torch.int32, device=dev)
        self.anc_bits = ops.tree_struct(parents, 4, cu_seqlens=self.cu, n_nodes=64, batch=self.RB,
                                        want=("anc_bits",))["anc_bits"]
        # the requests by size class, once per step like the tree structure: the launch reads them to run as
        # the one mixed-width kernel
        self.order = ops.size_order(self.cu, 64)
        self.o = torch.empty(L, rows, HV, D, device=dev, dtype=torch.bfloat16)
        self.keys = torch.empty(L, HK, rows, D, device=dev)
        self.vals = torch.empty(L, HV, rows, D, device=dev)
        self.gains = torch.empty(L, HV, rows, device=dev)

    def verify(self, l, ordered=True):
        from dforktree_amd import ops
        ops.tree_verify(self.y[l], self.a[l], self.b[l], self.A_log, self.dt_bias, self.state[l].transpose(-1, -2),
                        hk=HK, hv=HV, anc_bits=self.anc_bits, batch=self.RB, n_nodes=64, cu_seqlens=self.cu,
                        neg_exp_A=self.neg, o=self.o[l], aux_k=self.keys[l], aux_v=self.vals[l],
                        aux_g=self.gains[l], aux_k_per_khead=True, size_order=self.order if ordered else None)

    def bytes_per_launch(self, lo=0, hi=64):
        """Algorithmic bytes of the requests with lo <= nodes <= hi: per
        request the 2 MiB state, and per node its y row, o, vn, key (per
        k-head), G, a, b and ancestry word."""
        C = 2 * HK * D + HV * D
        node = C * 2 + HV * D * 2 + HV * D * 4 + HK * D * 4 + HV * 4 + 2 * HV * 2 + 8
        return sum(D * D * 4 * HV + n * node for n in self.sizes if lo <= n <= hi)

    def by_class(self):
        """(requests, algorithmic bytes) of the two size classes: the trees of
        33-64 nodes (the 64-wide body) and the rest (the 32-wide body)."""
        wide = [n for n in self.sizes if n > 32]
        return {"33-64 nodes": (len(wide), self.bytes_per_launch(33, 64)),
                "1-32 nodes": (self.RB - len(wide), self.bytes_per_launch(0, 32))}


class PluginWorkload:
    """The path the SGLang plugin drives today: batch 1 (fc1_branch64.py:13,
    fc1_fused.py:69), one NN-node random tree per step, 24 GDN layers at full
    width.  Per layer the hooked conv (fc1_conv.py:33-45: x [1, C, NN] as a
    transposed view, the pool's conv state and intermediate window read
    through device slot indices) writes the verify input, then
    tree_gdn_split (fc1_fused.py:74) verifies on the dense fp32 CTX.anc,
    saving keys per v-head as the reference's Context holds them.  As the
    verify hook does, the first layer packs the dense CTX.anc into bit rows
    (dft_anc_pack) and every layer's verify reads those; the verify on the
    dense matrix is timed beside it.  Per step the two-end snapshot commit
    (fc1_fused.py:77-87) writes the states at the last accepted node and at
    a tracked earlier one into the intermediate cache."""
    SLOTS, ISLOTS = 4, 2

    def __init__(self, dev, nn, seed=7):
        import torch
        from dforktree_amd import ops, synth
        from dforktree_amd.plugin import fc1_conv, tree_kernels
        self.nn = nn
        C = 2 * HK * D + HV * D
        self.x = synth.device_randn_(torch.empty(L, nn, C, device=dev, dtype=torch.bfloat16), seed)
        self.cw = synth.device_randn_(torch.empty(C, 4, device=dev, dtype=torch.bfloat16), seed + 1, std=0.1)
        self.conv_state = synth.device_randn_(torch.empty(L, self.SLOTS, C, 3, device=dev, dtype=torch.bfloat16),
                                              seed + 2)
        self.iwin = torch.zeros(L, self.ISLOTS, nn, C, 3, device=dev, dtype=torch.bfloat16)
        self.a = synth.device_randn_(torch.empty(L, 1, nn, HV, device=dev, dtype=torch.bfloat16), seed + 3)
        self.b = synth.device_randn_(torch.empty(L, 1, nn, HV, device=dev, dtype=torch.bfloat16), seed + 4)
        self.A_log = torch.full((HV,), -0.6931471805599453, device=dev)
        self.dt_bias = torch.zeros(HV, device=dev)
        self.neg = -self.A_log.exp()
        # SGLang's pools: temporal [L, slots, H, V, K], intermediate_ssm [L, islots, NN, H, V, K]
        self.temporal = synth.device_randn_(torch.empty(L, self.SLOTS, HV, D, D, device=dev), seed + 5, std=0.02)
        self.inter = torch.empty(L, self.ISLOTS, nn, HV, D, D, device=dev)
        self.slot = torch.tensor([2], device=dev, dtype=torch.int32)
        self.islot = torch.tensor([1], device=dev, dtype=torch.int32)
        g = torch.Generator().manual_seed(seed)
        parent = synth.tree_parents(nn, "random", g)
        ts = ops.tree_struct(parent.to(dev), 4, batch=1, n_nodes=nn, want=("anc", "anc_bits", "cidx"),
                             index_dtype=torch.int32)
        self.anc, self.cidx = ts["anc"][0], ts["cidx"]
        self.anc_bits = torch.zeros(nn, device=dev, dtype=torch.int64)  # the hook's CTX.anc_bits
        path = synth.accepted_path(parent, MAX_PATH, g)
        self.accept = torch.full((1, MAX_PATH), -1, device=dev, dtype=torch.int32)
        self.accept[0, :len(path)] = path.to(dev)
        track = int(path[len(path) // 2])
        self.ends = torch.tensor([[int(path[-1]), track]], device=dev, dtype=torch.int32)
        # the reference's Context: keys per v-head (fc1_fused.py:16)
        self.keys = torch.empty(L, HV, nn, D, device=dev)
        self.values = torch.empty_like(self.keys)
        self.gains = torch.empty(L, HV, nn, device=dev)
        self.y = torch.empty(L, 1, nn, C, device=dev, dtype=torch.bfloat16)
        self.o = torch.empty(L, nn, HV, D, device=dev, dtype=torch.bfloat16)
        self._conv, self._tk = fc1_conv, tree_kernels

    def conv(self, l):
        x = self.x[l].t().unsqueeze(0)  # [1, C, NN], token stride C
        self._conv.conv(x, self.conv_state[l], self.cw, None, self.cidx, self.slot, self.islot, self.iwin[l], self.y[l])

    def verify_dense(self, l):
        pool = self.temporal[l]
        self._tk.tree_gdn_split(self.y[l, 0], self.a[l].reshape(self.nn, -1), self.b[l].reshape(self.nn, -1),
                                self.A_log, self.dt_bias, pool[0].transpose(-1, -2), self.anc, HK, HV, D, D,
                                aux=(self.keys[l], self.values[l], self.gains[l]), neg_exp_A=self.neg,
                                state_indices=self.slot, state_slot_stride=pool.stride(0))

    def pack(self):
        from dforktree_amd import ops
        ops.anc_pack(self.anc, out=self.anc_bits)

    def verify_bits(self, l):
        pool = self.temporal[l]
        self._tk.tree_gdn_split(self.y[l, 0], self.a[l].reshape(self.nn, -1), self.b[l].reshape(self.nn, -1),
                                self.A_log, self.dt_bias, pool[0].transpose(-1, -2), self.anc, HK, HV, D, D,
                                aux=(self.keys[l], self.values[l], self.gains[l]), neg_exp_A=self.neg,
                                state_indices=self.slot, state_slot_stride=pool.stride(0), anc_bits=self.anc_bits)

    def layers(self):
        """What the hooks launch per forward: the pack at the first layer, then conv + verify per layer."""
        for l in range(L):
            self.conv(l)
            if l == 0:
                self.pack()
            self.verify_bits(l)

    def commit(self):
        from dforktree_amd.plugin import fc1_fused
        fc1_fused.snapshot_commit(self.temporal, self.keys, self.values, self.gains, self.anc, self.accept, self.ends,
                                  self.slot, self.islot, self.inter, anc_bits=self.anc_bits)


def plugin_lines(dev, reps, warmup, eager):
    """µs per layer and per step of the batch-1 plugin path at NN = 32 and 64."""
    import torch
    lines = {}
    for nn in (32, 64):
        pw = PluginWorkload(dev, nn)
        torch.cuda.synchronize()
        t_layers = time_graph(pw.layers, reps, warmup, eager) / L
        t_conv = time_graph(lambda: [pw.conv(l) for l in range(L)], reps, warmup, eager) / L
        t_dense = time_graph(lambda: [pw.verify_dense(l) for l in range(L)], reps, warmup, eager) / L
        t_bits = time_graph(lambda: [pw.verify_bits(l) for l in range(L)], reps, warmup, eager) / L
        t_pack = time_graph(lambda: [pw.pack() for _ in range(L)], reps, warmup, eager) / L
        t_commit = time_graph(pw.commit, reps, warmup, eager)
        lines[f"nn{nn}"] = {"conv_plus_verify_us_per_layer": round(t_layers * 1e3, 2),
                            "conv_us_per_layer": round(t_conv * 1e3, 2),
                            "verify_us_per_layer": round(t_bits * 1e3, 2),
                            "verify_dense_anc_us_per_layer": round(t_dense * 1e3, 2),
                            "anc_pack_us_per_step": round(t_pack * 1e3, 2),
                            "snapshot_commit_us_per_step": round(t_commit * 1e3, 2),
                            "step_us": round((t_layers * L + t_commit) * 1e3, 1)}
        del pw
        torch.cuda.empty_cache()
    lines["workload"] = ("batch 1, one random tree per step, 24 layers at full width: CTX.anc packed to bit rows "
                         "once per step, hooked conv + tree_gdn_split per layer, two-end snapshot commit per step")
    return lines


def copy_rate(dev, reps=20):
    """Achievable HBM rate on this GPU: GB/s (bytes read + bytes written) of
    the streaming copy kernel built beside the library
    (dforktree_amd/calib/stream_copy.hip: 16-byte non-temporal loads and
    stores) over a 1 GiB buffer, four times the memory-side cache, timed as
    a HIP graph of back-to-back copies like the layers.  torch's copy_ of the
    same buffers is reported beside it.  None if the copy library is absent."""
    import ctypes
    import torch
    path = ROOT / "dforktree_amd" / "libdft_stream_copy.so"
    if not path.exists():
        return None
    lib = ctypes.CDLL(str(path))
    lib.dft_calib_stream_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    nbytes = 1 << 30
    src = torch.ones(nbytes // 4, device=dev)
    dst = torch.empty_like(src)

    def kernel_copy():
        rc = lib.dft_calib_stream_copy(src.data_ptr(), dst.data_ptr(), nbytes,
                                       ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc != 0:
            raise RuntimeError(f"dft_calib_stream_copy returned {rc}")

    ms = time_graph(kernel_copy, reps, 3)
    if not torch.equal(dst[::4096], src[::4096]):
        raise RuntimeError("stream copy produced a wrong result")
    ms_torch = time_graph(lambda: dst.copy_(src), reps, 3)
    del src, dst
    return {"kernel": "stream_copy_kernel (16-byte non-temporal load + store per thread)", "bytes": 2 * nbytes,
            "achieved": round(2 * nbytes / (ms * 1e-3) / 1e9, 1),
            "torch_copy": round(2 * nbytes / (ms_torch * 1e-3) / 1e9, 1), "unit": "GB/s"}


def time_graph(fn, reps, warmup, eager=False):
    """ms per call of fn (a sequence of launches), HIP events on the current stream."""
    import torch
    if eager:
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def _cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(seconds):
    """The CPU baseline: one layer of the workload (64 requests x 32 nodes,
    verify + commit of each accepted path) through the batched PyTorch fp32
    restatement (oracle/gdn_tree_torch.py, pinned against the numpy oracle),
    repeated for ~`seconds`.  torch gets one thread per core this process may
    run on (capped by OMP_NUM_THREADS when the environment sets it, the CPU
    share of the box); the trees' ancestry and the path masks are built
    outside the timed region, as the GPU path gets them once per step."""
    import numpy as np
    import torch
    from dforktree_amd import synth
    from oracle import gdn_tree as O
    from oracle import gdn_tree_torch as T
    affinity = len(os.sched_getaffinity(0))
    threads = min(affinity, int(os.environ.get("OMP_NUM_THREADS", affinity) or affinity))
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    bt = synth.make_batch(2, 0, [N] * B, hk=HK, hv=HV)
    y = bt.y.float().reshape(B, N, -1)
    a = bt.a.reshape(B, N, -1)
    b = bt.b.reshape(B, N, -1)
    S0 = bt.state.transpose(-1, -2).contiguous()  # (k, v)
    par = bt.parent.reshape(B, N)
    g = torch.Generator().manual_seed(3)
    paths = [synth.accepted_path(p, MAX_PATH, g) for p in par]
    anc = torch.from_numpy(np.stack([O.tree_struct(p.numpy())[0] for p in par]).astype(np.float32))
    on = torch.zeros(B, N)
    for i, p in enumerate(paths):
        on[i, p.long()] = 1
    u = torch.tensor([int(p[-1]) for p in paths])

    def layer():
        r = T.tree_gdn_split(y, a, b, bt.A_log, bt.dt_bias, S0, anc, HK, HV, D, D)
        return T.closed_commit(S0, r["k"], r["vn"], r["G"], on, u)

    with torch.inference_mode():
        layer()  # warm-up
        times = []
        t_end = time.perf_counter() + seconds
        while time.perf_counter() < t_end or len(times) < 3:
            t0 = time.perf_counter()
            layer()
            times.append(time.perf_counter() - t0)
    torch.set_num_threads(prev_threads)
    t = float(np.median(times))
    return {"value": B * N / t, "unit": "nodes/s/layer", "cores": threads, "kind": "port",
            "affinity_cores": affinity, "cpu_model": _cpu_model(),
            "sample": f"{len(times)} x one layer of the workload ({B} requests x {N} nodes, verify + "
                      f"commit of the accepted paths) through the batched PyTorch fp32 restatement "
                      f"(torch {torch.__version__}, {threads} threads), median {t * 1e3:.0f} ms"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the path shards by request and "
              f"head group with no exchange step, so every rank would run an independent copy of this "
              f"single-GPU workload)", file=sys.stderr)
        sys.exit(2)
    import torch
    dev = torch.device("cuda:0")
    if args.only_plugin:
        print(json.dumps({"plugin": plugin_lines(dev, max(args.steps, 10), args.warmup, args.eager)}), flush=True)
        return
    if args.only_ragged:
        rw = RaggedWorkload(dev)
        t = time_graph(lambda: [rw.verify(l) for l in range(L)], max(args.steps, 10), args.warmup, args.eager) / L
        if args.copy_calibration:
            src = torch.ones(1 << 28, device=dev)
            dst = torch.empty_like(src)
            for _ in range(3):
                dst.copy_(src)
            torch.cuda.synchronize()
        print(json.dumps({"ragged_us_per_layer": round(t * 1e3, 2), "bytes_per_launch": rw.bytes_per_launch(),
                          "classes": rw.by_class()}), flush=True)
        return
    w = Workload(dev)
    torch.cuda.synchronize()

    reps_kernel = max(args.steps, 10)
    # the separate schedule first: it fills both save sets the pipelined one reads
    t_verify_layers = time_graph(lambda: [w.verify(l) for l in range(L)], reps_kernel, args.warmup, args.eager)
    t_verify = t_verify_layers / L
    t_commit = time_graph(w.commit, reps_kernel, args.warmup, args.eager)
    t_step_sep = time_graph(w.step, args.steps, args.warmup, args.eager)
    for l in range(L):
        w.verify(l)
    torch.cuda.synchronize()
    # the same launch reading saved values (raw key rows), and saved keys and values
    t_fused_sv = time_graph(lambda: [w.fused(l, raw_values=False) for l in range(L)], reps_kernel, args.warmup,
                            args.eager) / L
    t_fused_saved = time_graph(lambda: [w.fused(l, raw_keys=False, raw_values=False) for l in range(L)], reps_kernel,
                               args.warmup, args.eager) / L
    # the step is 24 launches of the dominant kernel: its launch time is taken from this one timing
    t_step = time_graph(w.fused_step, args.steps, args.warmup, args.eager)
    t_fused = t_step / L
    # conv and mask run once per layer in a step: 24 back-to-back launches per replay, as for verify
    w.conv_setup(dev)
    t_conv = time_graph(lambda: [w.conv() for _ in range(L)], reps_kernel, args.warmup, args.eager) / L
    w.mask_setup(dev)
    t_mask = time_graph(lambda: [w.mask() for _ in range(L)], reps_kernel, args.warmup, args.eager) / L
    ragged = None
    if not args.no_ragged:
        rw = RaggedWorkload(dev)  # both workloads fit together (about 17 GB)
        t_ragged = time_graph(lambda: [rw.verify(l) for l in range(L)], reps_kernel, args.warmup, args.eager) / L
        t_two = time_graph(lambda: [rw.verify(l, ordered=False) for l in range(L)], reps_kernel, args.warmup,
                           args.eager) / L
        ragged = {"workload": "packed ragged batch: 128 requests, trees of 8-64 nodes (chains / bushy / random), "
                              "verify as one mixed-width launch from the size-order records (the 33-64-node trees "
                              "on the 64-wide body first, then the others' v-head pairs on the 32-wide body)",
                  "nodes": rw.rows, "us_per_layer": round(t_ragged * 1e3, 2),
                  "two_kernels_us_per_layer": round(t_two * 1e3, 2),
                  "nodes_per_s_per_layer": round(rw.rows / (t_ragged * 1e-3), 1),
                  "hbm_frac": round(rw.bytes_per_launch() / (t_ragged * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    nn64 = None
    if not args.no_ragged:
        del rw
    if not args.no_nn64:
        torch.cuda.empty_cache()
        w64 = Workload(dev, seed=4, n=64)  # the reference's default tree size (FC1_TREE_N, fc1_fused.py:4)
        t64_v = time_graph(lambda: [w64.verify(l) for l in range(L)], reps_kernel, args.warmup, args.eager) / L
        t64_f = time_graph(w64.fused_step, reps_kernel, args.warmup, args.eager) / L
        nn64 = {"workload": "batch 64, uniform 64-node random recursive trees, 24 layers (the reference's default "
                            "tree size); verify, and the pipelined commit -> verify (raw key rows, recomputed values)",
                "verify_us_per_layer": round(t64_v * 1e3, 2),
                "verify_nodes_per_s_per_layer": round(B * 64 / (t64_v * 1e-3), 1),
                "verify_hbm_frac": round(w64.verify_bytes_per_launch() / (t64_v * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "commit_verify_us_per_layer": round(t64_f * 1e3, 2),
                "nodes_per_s_per_layer": round(B * 64 / (t64_f * 1e-3), 1),
                "hbm_frac": round(w64.fused_bytes_per_launch() / (t64_f * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "algorithmic_bytes_per_launch": w64.fused_bytes_per_launch()}
        del w64
    plugin = None
    if not args.no_plugin:
        torch.cuda.empty_cache()
        plugin = plugin_lines(dev, reps_kernel, args.warmup, args.eager)
    if args.copy_calibration:
        src = torch.ones(1 << 28, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    torch.cuda.empty_cache()
    copy = copy_rate(dev)

    vb, cb, fb = w.verify_bytes_per_launch(), w.commit_bytes_per_launch(), w.fused_bytes_per_launch()
    kernels = {"tree_commit_verify_kernel": dict(ms=t_fused, bytes=fb, per_step=L)}
    dom = max(kernels, key=lambda k: kernels[k]["ms"] * kernels[k]["per_step"])
    kd = kernels[dom]
    achieved = kd["bytes"] / (kd["ms"] * 1e-3) / 1e9
    traffic = None
    prof = ROOT / "profiles" / "hbm_traffic.json"
    if prof.exists():
        try:
            traffic = json.loads(prof.read_text()).get(dom, {}).get("traffic_bytes_per_launch")
        except (ValueError, OSError):
            traffic = None
    # MFMA work per launch of the dominant kernel, counted by rocprofv3 (MOPS x 512 FLOP, hi/lo splits included),
    # over this run's live kernel time
    mfma = None
    mprof = ROOT / "profiles" / "mfma.json"
    if mprof.exists():
        try:
            mf = json.loads(mprof.read_text()).get(dom, {}).get("bf16_flops_per_launch")
        except (ValueError, OSError):
            mf = None
        if mf:
            tflops = mf / (kd["ms"] * 1e-3) / 1e12
            mfma = {"kernel": dom, "dtype": "bf16", "flops_per_launch": mf, "achieved": round(tflops, 1),
                    "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)}
    value = B * N / (t_step * 1e-3 / L)
    frac = lambda nbytes, ms: round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)  # noqa: E731
    out = {
        "metric": "GDN tree-verify nodes/sec/layer (bs64, 32-node tree) + % HBM peak",
        "value": round(value, 1),
        "unit": "nodes/s/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "stacked GDN tree verify + accepted-path commit", "batch": B, "nodes": N,
                   "layers": L, "qk_heads": HK, "v_heads": HV, "dk": D, "dv": D, "tree": "random recursive",
                   "accepted_path": "random walk, length 1-16",
                   "schedule": "pipelined: each layer's launch commits the previous step's path (its keys "
                               "normalised from the previous step's raw k rows, its values recomputed from the "
                               "previous step's raw v rows and b gates), then verifies",
                   "timing": "eager" if args.eager else "hip graph"},
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes_per_launch": kd["bytes"],
                     # what a streaming copy reaches on this GPU, and the kernel's rate against it
                     "copy": copy, "frac_of_copy": round(achieved / copy["achieved"], 4) if copy else None},
        "mfma": mfma,
        "commit_verify_us_per_layer": round(t_fused * 1e3, 2),
        # the same launch with the values saved by the verify and read back by the next commit (keys from the
        # raw rows), and with both keys and values saved
        "commit_verify_saved_values": {"us_per_layer": round(t_fused_sv * 1e3, 2),
                                       "hbm_frac": frac(w.fused_bytes_per_launch(raw_values=False), t_fused_sv)},
        "commit_verify_saved_keys": {"us_per_layer": round(t_fused_saved * 1e3, 2),
                                     "hbm_frac": frac(w.fused_bytes_per_launch(raw_keys=False, raw_values=False),
                                                      t_fused_saved)},
        # state bytes per unit time: what the pipelined schedule moves (one read and one write per
        # request-layer), and an equivalent that also credits the separate verify's own state read, which the
        # fused launch does not perform (3 x 2 MiB per request-layer: the bytes the separate kernels need)
        "state_traffic": {"moved_hbm_frac": frac(w.state_bytes_moved_pipelined(), t_step),
                          "moved_bytes_per_step": w.state_bytes_moved_pipelined(),
                          "separate_equivalent_hbm_frac": frac(w.state_bytes_per_step(), t_step),
                          "separate_equivalent_bytes_per_step": w.state_bytes_per_step()},
        "separate": {"ms_per_step": round(t_step_sep, 4), "value": round(B * N / (t_step_sep * 1e-3 / L), 1),
                     "verify_us_per_layer": round(t_verify * 1e3, 2), "verify_hbm_frac": frac(vb, t_verify),
                     "commit_ms": round(t_commit, 4), "commit_hbm_frac": frac(cb, t_commit),
                     "state_traffic_hbm_frac": frac(w.state_bytes_per_step(), L * t_verify + t_commit)},
        "verify_only_nodes_per_s_per_layer": round(B * N / (t_verify * 1e-3), 1),
        "conv_us_per_layer": round(t_conv * 1e3, 2),
        "conv_hbm_frac": frac(w.conv_bytes_per_launch(), t_conv),
        "mask_pack_us": round(t_mask * 1e3, 2),
        "mask_pack_hbm_frac": frac(w.mask_bytes_per_launch(), t_mask),
        "ragged": ragged,
        "nn64": nn64,
        "plugin": plugin,
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
