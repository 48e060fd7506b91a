#!/usr/bin/env python3
"""Benchmark of the padded-CSR training hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload c5-95-rigl] [--no-extra]
                    [--graph-steps S] [--no-graph] [--no-cpu]

Prints ONE JSON line (rank 0). Workloads (BASELINE.json `configs`):

  c5-95-rigl (default, configs[4]: the largest single-GPU configuration)
      one 16384x16384 layer at 95% sparsity, Zipf(1.1) rows, N = 4096 tokens;
      one step = forward Y, dW on the live slots, dX through the cached
      transpose, then a RigL rewrite (G = dY.X^T, drop the 30% smallest |w|,
      regrow at the top-|G| dead positions) and the device transpose
      rebuild. value = tokens / s of that step. The same line carries the
      99%-sparsity layer's RigL step under "extra" (--no-extra skips it).
  c5-95, c5-99, c5-99-rigl   the same layers without / with RigL
  c4  (configs[3]) 60M mini-GPT train step + SET, 8192 tokens
  c3  (configs[2]) 10M char-GPT forward+backward, 8192 tokens
  c2  (configs[1]) 2-layer MLP 784->512->10, batch 256, train step
  c1  (configs[0]) one 512x784 layer, 78 live columns per row, N=256

Steps of workloads whose topology is fixed are replayed from HIP graphs
(--graph-steps consecutive steps per graph for sub-millisecond steps);
topology-changing steps (RigL, SET) run eagerly. Inputs and weights are
resident in HBM before the timed region starts. Each path kernel's average
duration is then measured with HIP events around back-to-back launches on the
step's own tensors (queued behind a GPU sleep so no host gap enters the
interval); `roofline.achieved` is the dominant path kernel's algorithmic
bytes per launch divided by that duration, `roofline.compute` its 2*nnz*N
flops against the published fp32 peak.

The CPU baseline runs the same step with the reference's own kernels
(oracle/_ref: csrc/kernels/*.cpp compiled at the reference flags, OpenMP
threads = OMP_NUM_THREADS, plus a 1-thread row) and torch CPU ops for the
dense parts, timed over a bounded sample on this host.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

# The CPU baseline's OpenMP threads are bound to consecutive physical cores,
# as the reference's published OpenMP numbers were measured; libgomp reads
# these when it loads, so they are set before anything imports it. A
# caller's own setting wins.
os.environ.setdefault("OMP_PROC_BIND", "close")
os.environ.setdefault("OMP_PLACES", "cores")

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "SpMM fwd+dX+dW achieved HBM GB/s & effective GFLOP/s; train-step tokens/s"
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3  # MI355X published fp32 peak (vector, packed; = dense fp32 MFMA)
# The kernels run on the VALU with packed fp32 disabled at compile time (some
# packed forms have given wrong results on this hardware), so the non-packed
# rate is their practical ceiling: 256 CUs x 64 fma/clk x 2.4 GHz x 2 flops.
VALU_NONPACKED_TFLOPS = 78.6
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X published dense bf16 matrix-core peak


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c5-95-rigl",
                    choices=["c1", "c2", "c3", "c4", "c5-95", "c5-99", "c5-95-rigl",
                             "c5-99-rigl"])
    ap.add_argument("--no-graph", action="store_true", help="time eager launches")
    ap.add_argument("--graph-steps", type=int, default=20,
                    help="training steps captured per HIP graph (graph-captured workloads)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true",
                    help="c5-95-rigl only: skip the c5-99-rigl line reported beside it")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="approximate CPU-baseline budget")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--only-kernel", default=None,
                    help="build the workload, then time only this kernel label (e.g. spmm_fwd, "
                         "sddmm_dw, 'spmm_dx[qkv 768x2304]') and print its timing: a short "
                         "run for profiler counter passes")
    ap.add_argument("--kernel-reps", type=int, default=30,
                    help="timed calls per kernel label in the kernel-timing phase (after 3 "
                         "warm-up calls; the median is reported)")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="after the run, copy a buffer of this many MiB three times (a "
                         "known-size reference dispatch for HBM byte counters)")
    return ap.parse_args()


# ───────────────────────────── byte / flop model ─────────────────────────────
# Algorithmic (compulsory) traffic per launch: f32/i32 = 4 B, i64 = 8 B.

def bytes_fwd(nnz, M, K, N):  # values+cols, row_start+row_nnz, X read, Y written
    return 8 * nnz + 8 * M + 4 * K * N + 4 * M * N


def bytes_dw(nnz, cap, M, K, N):  # cols, row arrays, dY + X read, dW (all slots) written
    return 4 * nnz + 8 * M + 4 * M * N + 4 * K * N + 4 * cap


def bytes_backward_fused(nnz, cap, M, K, N):  # dW as bytes_dw; dX as the forward on WT,
    # its values gathered through perm (i64) instead of refreshed first
    return bytes_dw(nnz, cap, M, K, N) + bytes_fwd(nnz, K, M, N) + 8 * nnz


def bytes_refresh(nnz, capT):  # perm (i64) read, gathered values, WT values written
    return 8 * capT + 4 * nnz + 4 * capT


def flops(nnz, N):
    return 2 * nnz * N


# ───────────────────────────── timing helpers ────────────────────────────────

KERNEL_WARMUP = 3
KERNEL_REPS = 30


def graph_call_us(fn, calls: int = 20, reps: int = 11) -> float:
    """Per-call time of `fn` replayed from a HIP graph of `calls` consecutive
    calls (median over `reps` replays, divided by `calls`): for kernels of a
    few microseconds, whose one-call event interval is mostly launch
    overhead. Only for calls that a graph can hold (no host reads)."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(KERNEL_WARMUP):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(calls):
            fn()
    g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) * 1e3 / calls)
    return sorted(ts)[reps // 2]


def kernel_time_ms(fn, reps: int | None = None):
    """Per-call device time of `fn` (one kernel label) as the reference's
    profiler measures it (examples/profile_dw_baseline.py:94-128): KERNEL_WARMUP
    untimed calls, then `reps` calls, each between two HIP events on the
    current stream, queued behind a GPU sleep so no host launch gap enters an
    interval. Returns (median ms, mean ms, reps)."""
    import torch

    for _ in range(KERNEL_WARMUP):
        fn()
    torch.cuda.synchronize()
    reps = KERNEL_REPS if reps is None else max(1, int(reps))
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    torch.cuda._sleep(int(2e7))  # keeps the GPU busy while the launches queue up
    ev[0].record()
    for i in range(reps):
        fn()
        ev[i + 1].record()
    torch.cuda.synchronize()
    ts = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(reps))
    mid = reps // 2
    median = ts[mid] if reps % 2 else 0.5 * (ts[mid - 1] + ts[mid])
    return median, sum(ts) / reps, reps


def stage(msg: str) -> None:
    """Progress marker on stderr, flushed, so a failing run names its stage."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def timed_loop(step, steps: int):
    import torch

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def timed_run(run_steps, steps: int):
    """Wall time of run_steps(steps), synchronized on both sides."""
    import torch

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run_steps(steps)
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def capture(step_body, warm_iters: int = 3, steps: int = 1):
    """Capture `steps` consecutive step_body() calls into one HIP graph after
    warming it on a side stream; returns the graph, each step's output and the
    graph's node types (read before the graph is instantiated)."""
    import torch

    from sparsecore_amd import _lib

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warm_iters):
            step_body()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(g):
        outs = [step_body() for _ in range(steps)]
    nodes = _lib.graph_node_types(g)
    g.instantiate()
    return g, outs, nodes


class GraphSteps:
    """Runs n training steps as replays of an S-step graph plus, for n mod S,
    a one-step graph. A replay costs a fixed few microseconds of launch
    latency on top of its kernels, which a sub-100 us step feels; a graph of
    S steps pays it once per S steps. Every step is still executed in full."""

    def __init__(self, big, S, one):
        self.big, self.S, self.one = big, S, one

    def run(self, n):
        for _ in range(n // self.S):
            self.big.replay()
        for _ in range(n % self.S):
            self.one.replay()


# ───────────────────────────── workload C2 ───────────────────────────────────

class C2:
    name = "c2"
    desc = ("2-layer MLP 784->512->10, SparseLinear 90%/90%, fp32, ReLU, cross-entropy, "
            "batch 256, SGD lr 0.01")
    batch = 256

    def __init__(self, dev, seed):
        import torch
        import torch.nn as nn

        import sparsecore_amd as slk

        self.seed = seed
        torch.manual_seed(seed)
        self.l1 = slk.SparseLinear(784, 512, sparsity=0.9)
        self.l2 = slk.SparseLinear(512, 10, sparsity=0.9)
        self.model = nn.Sequential(self.l1, nn.ReLU(), self.l2).to(dev)
        g = torch.Generator().manual_seed(seed + 1)
        self.x = torch.rand(self.batch, 784, generator=g).to(dev)
        self.labels = torch.randint(0, 10, (self.batch,), generator=g).to(dev)
        # foreach=False: torch's multi-tensor SGD kernel gives each 64Ki-element
        # chunk one workgroup, so these four small tensors run on 4 workgroups
        # (≈20 µs); one elementwise update per tensor fills the GPU instead.
        self.opt = torch.optim.SGD(self.model.parameters(), lr=0.01, foreach=False)
        self.dev = dev

    def body(self):
        import torch.nn.functional as F

        self.opt.zero_grad(set_to_none=True)
        loss = F.cross_entropy(self.model(self.x), self.labels)
        loss.backward()
        self.opt.step()
        # detached: the caller must not keep this step's autograd graph (and its
        # AccumulateGrad nodes, bound to the stream they ran on) alive
        return loss.detach()

    def params(self):
        return [p for p in self.model.parameters()]

    def tokens_per_step(self):
        return self.batch

    def kernels(self):
        """(name, launch fn, bytes, flops) of the HIP kernels one step runs."""
        import torch

        from sparsecore_amd import _lib, ops

        out = []
        N = self.batch
        x_col = self.x.t().contiguous()
        h = torch.relu(self.l1(self.x)).detach()
        h_col = h.t().contiguous()
        for tag, layer, X in (("l1", self.l1, x_col), ("l2", self.l2, h_col)):
            W = layer._csr
            M, K = W.nrows, W.ncols
            dW = torch.empty(W.total_capacity, device=self.dev)
            view = W._view()
            if ops._narrow_layer(W):
                # the narrow path: token-major store, and dW + dbias + dX in one
                # launch from the token-major gradient (no transpose cache)
                Yt = torch.empty(N, M, device=self.dev)
                dYt = torch.randn(N, M, device=self.dev)
                db = torch.empty(M, device=self.dev)
                dX = torch.empty(K, N, device=self.dev)
                out.append((f"spmm_fwd_t[{tag} {M}x{K}]",
                            lambda view=view, X=X, Yt=Yt: _lib.spmm_t(view, X, Yt),
                            bytes_fwd(W.nnz, M, K, N), flops(W.nnz, N)))
                out.append((f"backward_narrow[{tag} {M}x{K}]",
                            lambda view=view, dYt=dYt, X=X, dW=dW, db=db, dX=dX:
                                _lib.backward_narrow(view, dYt, X, dW, db, dX, _lib.SLK_DW_SIMD),
                            bytes_dw(W.nnz, W.total_capacity, M, K, N) +
                            bytes_fwd(W.nnz, K, M, N), 2 * flops(W.nnz, N)))
                continue
            Y = torch.empty(M, N, device=self.dev)
            dY = torch.randn(M, N, device=self.dev)
            out.append((f"spmm_fwd[{tag} {M}x{K}]",
                        lambda view=view, X=X, Y=Y: _lib.spmm(view, X, Y),
                        bytes_fwd(W.nnz, M, K, N), flops(W.nnz, N)))
            out.append((f"sddmm_dw[{tag} {M}x{K}]",
                        lambda view=view, dY=dY, X=X, dW=dW: _lib.sddmm(view, dY, X, dW,
                                                                       _lib.SLK_DW_SIMD),
                        bytes_dw(W.nnz, W.total_capacity, M, K, N), flops(W.nnz, N)))
            if tag == "l2":  # layer 1's input needs no gradient, so no dX there
                WT = ops._cached_transpose(W)
                perm = ops._transpose_cache[id(W)][3]
                dX = torch.empty(K, N, device=self.dev)
                vT = WT._view()
                out.append((f"spmm_dx[{tag} {K}x{M}]",
                            lambda vT=vT, dY=dY, dX=dX: _lib.spmm(vT, dY, dX),
                            bytes_fwd(WT.nnz, K, M, N), flops(W.nnz, N)))
                out.append((f"transpose_refresh[{tag}]",
                            lambda W=W, perm=perm, WT=WT: _lib.transpose_refresh(
                                W.values, perm, WT.values),
                            bytes_refresh(W.nnz, WT.total_capacity), 0))
        return out

    def spmm_layer(self):
        return self.l1._csr


# ─────────────────────────── workloads C3 / C4 ───────────────────────────────

class GPTWork:
    """Char-level decoder-only transformer with SparseLinear projections.

    Attention projections (fused QKV D->3D and O D->D, as the reference's
    demo_15_mini_gpt.py builds them) are SparseLinear at `attn_sparsity`; FFN
    up/down are SparseLinear at `ffn_sparsity`; embeddings, LayerNorms and the
    LM head are dense. Subclasses fix the configuration."""

    name = desc = ""
    d_model = n_layers = n_heads = d_ff = vocab = ctx = batch = 0
    attn_sparsity, ffn_sparsity = 0.7, 0.9
    train = False       # SGD step (lr 0.01) inside the step
    set_update = False  # SET drop/regrow + device transpose rebuild inside the step
    dynamic = False     # topology changes every step (no graph capture)

    def __init__(self, dev, seed, with_set: bool = True):
        import torch
        import torch.nn as nn
        import torch.nn.functional as F

        import sparsecore_amd as slk

        cfg = type(self)
        D, H, d_ff, ctx, vocab = cfg.d_model, cfg.n_heads, cfg.d_ff, cfg.ctx, cfg.vocab
        sa, sf = cfg.attn_sparsity, cfg.ffn_sparsity

        class Attn(nn.Module):
            def __init__(self):
                super().__init__()
                self.qkv = slk.SparseLinear(D, 3 * D, sparsity=sa, bias=False)
                self.o = slk.SparseLinear(D, D, sparsity=sa, bias=False)

            def forward(self, x):
                B, T, C = x.shape
                q, k, v = self.qkv(x).chunk(3, dim=-1)
                q = q.reshape(B, T, H, C // H).transpose(1, 2)
                k = k.reshape(B, T, H, C // H).transpose(1, 2)
                v = v.reshape(B, T, H, C // H).transpose(1, 2)
                a = F.scaled_dot_product_attention(q, k, v, is_causal=True)
                return self.o(a.transpose(1, 2).reshape(B, T, C))

        class Block(nn.Module):
            def __init__(self):
                super().__init__()
                self.ln1 = nn.LayerNorm(D)
                self.attn = Attn()
                self.ln2 = nn.LayerNorm(D)
                self.up = slk.SparseLinear(D, d_ff, sparsity=sf, bias=False)
                self.down = slk.SparseLinear(d_ff, D, sparsity=sf, bias=False)

            def forward(self, x):
                x = x + self.attn(self.ln1(x))
                return x + self.down(F.gelu(self.up(self.ln2(x))))

        n_layers = cfg.n_layers

        class GPT(nn.Module):
            def __init__(self):
                super().__init__()
                self.tok = nn.Embedding(vocab, D)
                self.pos = nn.Embedding(ctx, D)
                self.blocks = nn.ModuleList([Block() for _ in range(n_layers)])
                self.ln_f = nn.LayerNorm(D)
                self.head = nn.Linear(D, vocab, bias=False)

            def forward(self, idx):
                x = self.tok(idx) + self.pos(torch.arange(idx.shape[1], device=idx.device))
                for b in self.blocks:
                    x = b(x)
                return self.head(self.ln_f(x))

        self.seed = seed
        torch.manual_seed(seed)
        self.model = GPT().to(dev)
        g = torch.Generator().manual_seed(seed + 1)
        self.idx = torch.randint(0, vocab, (self.batch, ctx), generator=g).to(dev)
        self.tgt = torch.randint(0, vocab, (self.batch, ctx), generator=g).to(dev)
        self.dev = dev
        self.opt = torch.optim.SGD(self.model.parameters(), lr=0.01) if cfg.train else None
        self.algo = None
        if cfg.set_update and with_set:
            self.algo = slk.SET(sparsity=sf, drop_fraction=0.3, update_freq=1, seed=seed)
            self.model.apply(self.algo)

    def body(self):
        import torch.nn.functional as F

        for p in self.model.parameters():
            p.grad = None
        logits = self.model(self.idx)
        loss = F.cross_entropy(logits.reshape(-1, self.vocab), self.tgt.reshape(-1))
        loss.backward()
        if self.opt is not None:
            self.opt.step()
        if self.algo is not None:
            self.topology_update()
        return loss.detach()

    def topology_update(self):
        """SET on every sparse layer; SET then rebuilds the layers' transposes on
        the device in one batch."""
        self.algo.step()

    def params(self):
        return list(self.model.parameters())

    def tokens_per_step(self):
        return self.batch * self.ctx

    def sparse_layers(self):
        b = self.model.blocks[0]
        return [("qkv", b.attn.qkv), ("o", b.attn.o), ("up", b.up), ("down", b.down)]

    def kernels(self):
        """The HIP kernels of block 0's four sparse layers at N = batch*ctx tokens."""
        import torch

        from sparsecore_amd import _lib, ops

        N = self.batch * self.ctx
        out = []
        for tag, layer in self.sparse_layers():
            W = layer._csr
            M, K = W.nrows, W.ncols
            X = torch.randn(K, N, device=self.dev)
            Y = torch.empty(M, N, device=self.dev)
            dY = torch.randn(M, N, device=self.dev)
            dW = torch.empty(W.total_capacity, device=self.dev)
            dX = torch.empty(K, N, device=self.dev)
            WT = ops._cached_transpose(W)
            v, vT = W._view(), WT._view()
            out.append((f"spmm_fwd[{tag} {M}x{K}]", lambda v=v, X=X, Y=Y: _lib.spmm(v, X, Y),
                        bytes_fwd(W.nnz, M, K, N), flops(W.nnz, N)))
            out.append((f"sddmm_dw[{tag} {M}x{K}]",
                        lambda W=W, dY=dY, X=X, dW=dW: _lib.sddmm(ops._sddmm_view(W, X), dY, X, dW,
                                                                  _lib.SLK_DW_SIMD),
                        bytes_dw(W.nnz, W.total_capacity, M, K, N), flops(W.nnz, N)))
            out.append((f"spmm_dx[{tag} {K}x{M}]", lambda vT=vT, dY=dY, dX=dX: _lib.spmm(vT, dY, dX),
                        bytes_fwd(W.nnz, K, M, N), flops(W.nnz, N)))
        return out

    def spmm_layer(self):
        return self.model.blocks[0].up._csr


class C3(GPTWork):
    """10M-param char-level decoder, d_model 384, 6 layers,
    6 heads, FFN 1536, vocab 65, context 256, batch 32 (8192 tokens), fp32,
    QKV/O at 70%, FFN at 90%. One step = forward + backward (no optimizer
    step, as the config specifies); value = tokens / s."""

    name = "c3"
    d_model, n_layers, n_heads, d_ff, vocab, ctx, batch = 384, 6, 6, 1536, 65, 256, 32
    desc = ("10M char GPT: d384 6L 6H FFN1536 vocab65 ctx256 batch32 (8192 tokens), fp32; "
            "QKV/O SparseLinear 70%, FFN SparseLinear 90%; forward+backward")


class C4(GPTWork):
    """60M-param mini-GPT, d_model 768, 8 layers, 12 heads,
    FFN 3072, vocab 65, context 512, batch 16 (8192 tokens), fp32, attention
    projections at 70%, FFN at 90%. One step = forward, backward, SGD update
    (lr 0.01), then one SET rewrite of every sparse layer (drop the 30%
    smallest |w| per layer, regrow at uniform-random empty columns, zero-init)
    and the device transpose rebuild of every layer. value = tokens / s."""

    name = "c4"
    d_model, n_layers, n_heads, d_ff, vocab, ctx, batch = 768, 8, 12, 3072, 65, 512, 16
    train = set_update = dynamic = True
    desc = ("60M mini-GPT: d768 8L 12H FFN3072 vocab65 ctx512 batch16 (8192 tokens), fp32; "
            "QKV/O SparseLinear 70%, FFN SparseLinear 90%; forward+backward+SGD, then SET "
            "(drop 30% smallest |w| per layer, uniform regrow) + device transpose rebuild "
            "every step")

    def kernels(self):
        """Block 0's SpMM/SDDMM kernels plus one layer's topology update."""
        from sparsecore_amd import _lib, ops

        out = super().kernels()
        W = self.model.blocks[0].up._csr
        k = max(1, int(0.3 * W.nnz))
        seed = [0]

        def set_up():
            seed[0] += 1
            W._drop_grow(k, _lib.SLK_GROW_RANDOM, None, seed[0])

        def rebuild():
            ops._transpose_cache.pop(id(W), None)
            ops._cached_transpose(W)

        out.append(("set_drop_grow[up 3072x768]", set_up, 0, 0))
        out.append(("transpose_rebuild[up 3072x768]", rebuild,
                    8 * W.nrows + 8 * W.nnz + 16 * int(1.2 * W.nnz + W.ncols) + 12 * W.ncols, 0))
        return out


# ───────────────────────── single-layer workloads (C1, C5) ────────────────────

def zipf_row_counts(M: int, K: int, density: float, s: float, seed: int):
    """nnz_i = min(K, c * rank^-s) with c water-filled so the total is density*M*K,
    assigned to rows in a seeded random order."""
    import numpy as np

    target = int(round(density * M * K))
    ranks = np.arange(1, M + 1, dtype=np.float64) ** (-s)
    lo, hi = 0.0, float(K) * M
    for _ in range(200):
        mid = 0.5 * (lo + hi)
        if np.minimum(K, np.floor(mid * ranks)).sum() < target:
            lo = mid
        else:
            hi = mid
    counts = np.minimum(K, np.floor(hi * ranks)).astype(np.int64)
    short = target - int(counts.sum())
    for i in range(M):  # hand the rounding remainder to the largest non-full rows
        if short <= 0:
            break
        add = min(short, K - int(counts[i]))
        counts[i] += add
        short -= add
    return counts[np.random.default_rng(seed).permutation(M)]


def device_rows_csr(counts, K: int, sigma: float, seed: int, dev, padding_ratio=0.2):
    """Row i gets counts[i] distinct uniform columns and N(0, sigma) values, all
    drawn on the device (13.4M entries at C5-95% would be slow on the host)."""
    import torch

    from sparsecore_amd import layout

    M = len(counts)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    cnt = torch.as_tensor(counts, device=dev)
    rows, cols = [], []
    chunk = max(1, (1 << 25) // max(K, 1))
    for r0 in range(0, M, chunk):
        r1 = min(M, r0 + chunk)
        scores = torch.rand(r1 - r0, K, generator=g, device=dev)
        order = torch.argsort(scores, dim=1)
        rank = torch.empty_like(order)
        rank.scatter_(1, order, torch.arange(K, device=dev).expand(r1 - r0, K))
        r, c = (rank < cnt[r0:r1, None]).nonzero(as_tuple=True)
        rows.append(r + r0)
        cols.append(c)
        del scores, order, rank
    rows = torch.cat(rows)
    cols = torch.cat(cols)
    vals = torch.randn(rows.numel(), generator=g, device=dev) * sigma
    return layout.from_coo(rows, cols, vals, (M, K), padding_ratio=padding_ratio)


class LayerWork:
    """One SparseLinear-shaped layer: Y = W·X, dW = SDDMM(dY, X), dX = Wᵀ·dY via
    the cached transpose (refresh + SpMM) — the three kernels of the path; a
    small layer's backward is one launch (dW and dX, W's values read through
    the transpose's slot map), as ops' backward runs it."""

    def __init__(self, name, desc, W, X, dY, rigl: bool = False):
        import torch

        from sparsecore_amd import ops

        self.name, self.desc = name, desc
        self.W, self.X, self.dY = W, X, dY
        self.rigl = self.dynamic = rigl
        self.M, self.K = W.nrows, W.ncols
        self.N = X.shape[1]
        self.dev = X.device
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ops._cached_transpose(W)  # topology fixed: build once
        torch.cuda.synchronize()
        self.rebuild_ms = 1e3 * (time.perf_counter() - t0)

    def fused(self) -> bool:
        """The backward as one launch (slk_backward_fused), as ops' backward
        chooses it for this layer."""
        from sparsecore_amd import ops

        return ops._fused_backward(self.W, self.N, "simd")

    def body(self):
        from sparsecore_amd import ops

        Y = ops._launch_spmm(self.W, self.X)
        # dW (SIMD order) and dX = Wᵀ·dY as the autograd backward computes
        # them: separate launches through the transpose cache, or one launch
        # for a small layer
        dW, dX = ops._spmm_backward(self.W, self.X, self.dY, "simd", True, True)
        if self.rigl:
            self.topology_update()
        return Y, dW, dX

    def topology_update(self):
        """RigL: drop the 30% smallest |w|, regrow at the top-|G| dead
        positions, G = dY·Xᵀ (the grows certified from the matrix-core
        approximation, exact G where it cannot decide), then rebuild the
        transpose on the device."""
        from sparsecore_amd import ops

        # the rewrite and the rebuild of the cached transpose, one host read
        ops._rigl_update_cached(self.W, max(1, int(0.3 * self.W.nnz)), self.dY, self.X)

    def params(self):
        return []

    def _WT(self):
        from sparsecore_amd import ops

        return ops._cached_transpose(self.W)

    def step_bytes(self):
        W, WT = self.W, self._WT()
        M, K, N = self.M, self.K, self.N
        if self.fused():
            return bytes_fwd(W.nnz, M, K, N) + bytes_backward_fused(W.nnz, W.total_capacity,
                                                                    M, K, N)
        return (bytes_fwd(W.nnz, M, K, N) + bytes_dw(W.nnz, W.total_capacity, M, K, N)
                + bytes_refresh(W.nnz, WT.total_capacity) + bytes_fwd(W.nnz, K, M, N))

    def step_flops(self):
        return 3 * flops(self.W.nnz, self.N)

    def kernels(self):
        import torch

        from sparsecore_amd import _lib, ops

        W = self.W
        M, K, N = self.M, self.K, self.N
        WT = self._WT()
        perm = ops._transpose_cache[id(W)][3]
        Y = torch.empty(M, N, device=self.dev)
        dW = torch.empty(W.total_capacity, device=self.dev)
        dX = torch.empty(K, N, device=self.dev)
        v, vT = ops._spmm_view(W, self.X), ops._spmm_view(WT, self.dY)
        if self.fused():
            WTs, perm_s = ops._cached_transpose_structure(W)
            return [
                ("spmm_fwd", lambda: _lib.spmm(v, self.X, Y), bytes_fwd(W.nnz, M, K, N),
                 flops(W.nnz, N)),
                ("backward_fused", lambda: _lib.backward_fused(W._view(), WTs._view(), perm_s,
                                                               self.dY, self.X, dW, None, dX),
                 bytes_backward_fused(W.nnz, W.total_capacity, M, K, N), 2 * flops(W.nnz, N)),
            ] + (self._rigl_kernels() if self.rigl else [])
        return [
            ("spmm_fwd", lambda: _lib.spmm(v, self.X, Y), bytes_fwd(W.nnz, M, K, N),
             flops(W.nnz, N)),
            ("sddmm_dw", lambda: _lib.sddmm(ops._sddmm_view(W, self.X), self.dY, self.X, dW,
                                            _lib.SLK_DW_SIMD),
             bytes_dw(W.nnz, W.total_capacity, M, K, N), flops(W.nnz, N)),
            ("transpose_refresh", lambda: _lib.transpose_refresh(W.values, perm, WT.values),
             bytes_refresh(W.nnz, WT.total_capacity), 0),
            ("spmm_dx", lambda: _lib.spmm(vT, self.dY, dX), bytes_fwd(W.nnz, K, M, N),
             flops(W.nnz, N)),
        ] + (self._rigl_kernels() if self.rigl else [])

    def _rigl_kernels(self):
        import torch

        from sparsecore_amd import _lib, ops

        W = self.W
        M, K, N = self.M, self.K, self.N
        G = torch.empty(M, K, device=self.dev)
        Gc = torch.empty(M, K, dtype=torch.uint8, device=self.dev)
        nd = torch.empty(M, device=self.dev)
        nx = torch.empty(K, device=self.dev)
        k = max(1, int(0.3 * W.nnz))

        def rebuild():
            ops._transpose_cache.pop(id(W), None)
            ops._cached_transpose(W)

        return [
            ("rigl_norms", lambda: _lib.rigl_norms(self.dY, self.X, nd, nx),
             4 * (M * N + K * N + M + K), 0),
            ("dense_grad_approx", lambda: _lib.dense_grad_approx(self.dY, self.X, G, Gc),
             4 * (M * N + K * N + M * K) + M * K, 2 * M * K * N),
            ("rigl_update", lambda: W._rigl_update(k, self.dY, self.X), 0, 0),
            ("transpose_rebuild", rebuild,
             8 * M + 8 * W.nnz + 16 * int(1.2 * W.nnz + K) + 12 * K, 0),
        ]


def make_c1(dev, seed):
    import numpy as np
    import torch

    from sparsecore_amd import PaddedCSR

    M, K, N = 512, 784, 256
    rng = np.random.default_rng(seed)
    W_dense = torch.zeros(M, K)
    for i in range(M):
        cols = torch.from_numpy(np.sort(rng.choice(K, 78, replace=False)))
        W_dense[i, cols] = torch.from_numpy(rng.normal(0, 0.02, 78).astype(np.float32))
    W = PaddedCSR.from_dense(W_dense, padding_ratio=0.2).to(dev)
    X = torch.from_numpy(rng.standard_normal((K, N)).astype(np.float32)).to(dev)
    dY = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(dev)
    return LayerWork("c1", "one 512x784 layer, 78 live/row (90%), values N(0,0.02), pr 0.2, N=256",
                     W, X, dY)


def make_c5(dev, seed, density, rigl=False):
    import torch

    M = K = 16384
    N = 4096
    counts = zipf_row_counts(M, K, density, 1.1, seed)
    W = device_rows_csr(counts, K, 0.01, seed + 1, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 2)
    X = torch.randn(K, N, generator=g, device=dev)
    dY = torch.randn(M, N, generator=g, device=dev)
    pct = int(round(100 * (1 - density)))
    extra = ("; step = fwd + dW + dX + RigL rewrite (drop 30% smallest |w|, regrow at the "
             "top-|G| dead positions, G = dY.X^T with the reference's dense_grad arithmetic: "
             "certified from a matrix-core approximation, exact where undecided) + device "
             "transpose rebuild") if rigl else ""
    return LayerWork(f"c5-{pct}" + ("-rigl" if rigl else ""),
                     f"16384x16384 at {pct}% sparsity, Zipf(1.1) rows (max {int(counts.max())}, "
                     f"min {int(counts.min())}), values N(0,0.01), N=4096" + extra, W, X, dY,
                     rigl=rigl)


# ───────────────────────────── CPU baseline ──────────────────────────────────

def _host_info() -> dict:
    """The host the CPU baseline ran on: CPU model, sockets, NUMA nodes, the
    GPU's NUMA node, and the CPUs this process may use."""
    import glob

    info = {"nproc": os.cpu_count()}
    try:
        info["cpus_allowed"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        pass
    try:
        txt = Path("/proc/cpuinfo").read_text()
        models = [ln.split(":", 1)[1].strip() for ln in txt.splitlines()
                  if ln.startswith("model name")]
        info["cpu_model"] = models[0] if models else None
        info["sockets"] = len({ln.split(":", 1)[1].strip() for ln in txt.splitlines()
                               if ln.startswith("physical id")}) or None
    except OSError:
        pass
    info["numa_nodes"] = len(glob.glob("/sys/devices/system/node/node[0-9]*")) or None
    try:
        import torch

        pr = torch.cuda.get_device_properties(0)
        bdf = "%04x:%02x:%02x.0" % (getattr(pr, "pci_domain_id", 0), pr.pci_bus_id,
                                    pr.pci_device_id)
        info["gpu_pci"] = bdf
        info["gpu_numa_node"] = int(Path(f"/sys/bus/pci/devices/{bdf}/numa_node").read_text())
    except Exception:  # best effort: attribute names and sysfs layout vary
        pass
    return info


def _set_threads(n: int) -> None:
    """OpenMP threads of the reference kernels (libgomp's ICV of this thread,
    read by every later parallel region it starts) and torch's CPU threads."""
    import ctypes

    import torch

    try:
        ctypes.CDLL("libgomp.so.1").omp_set_num_threads(int(n))
    except OSError:
        pass
    torch.set_num_threads(int(n))


def cpu_baseline(work, seconds: float):
    """The same step on this host's cores with the reference's own kernels:
    at OMP_NUM_THREADS threads (the box's CPU share), then a 1-thread row."""
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    _set_threads(threads)
    out = _cpu_run(work, seconds, threads)
    one_ok = isinstance(work, C2) or (isinstance(work, LayerWork) and
                                      (work.rigl or work.M * work.K <= 1 << 22))
    if not one_ok:
        out["one_thread"] = "skipped: one step on one thread exceeds the CPU budget"
    elif "error" not in out:
        _set_threads(1)
        one = _cpu_run(work, max(4.0, seconds / 2), 1)
        _set_threads(threads)
        out["one_thread"] = {k: one.get(k) for k in ("value", "unit", "cores", "sample")}
    out["host"] = _host_info()
    out["threads_note"] = ("cores = OpenMP/torch threads used; binding: " + _omp_binding())
    return out


def _omp_binding() -> str:
    """The OpenMP binding libgomp applies (OMP_PROC_BIND / OMP_PLACES, set by
    this script before anything loads libgomp)."""
    import ctypes

    names = {0: "false", 1: "true", 2: "primary", 3: "close", 4: "spread"}
    try:
        gomp = ctypes.CDLL("libgomp.so.1")
        bind = names.get(gomp.omp_get_proc_bind(), "?")
        places = gomp.omp_get_num_places()
    except (OSError, AttributeError):
        return "libgomp not found"
    return (f"OMP_PROC_BIND={os.environ.get('OMP_PROC_BIND')} (libgomp: {bind}), "
            f"OMP_PLACES={os.environ.get('OMP_PLACES')} (libgomp: {places} places)")


def _cpu_run(work, seconds: float, threads: int):
    """One timed CPU-baseline leg at `threads` threads."""
    import numpy as np
    import torch

    import oracle

    kind = "reference" if oracle.ref_available() else "port"

    class HostLayer:
        """Reference-path layer: RefCsr values aliased with a torch Parameter."""

        def __init__(self, csr):
            self.c = oracle.Csr(csr.nrows, csr.ncols, csr.values.detach().cpu().numpy(),
                                csr.col_indices.cpu().numpy(), csr.row_start.cpu().numpy(),
                                csr.row_nnz.cpu().numpy(), csr.row_capacity.cpu().numpy())
            if kind == "reference":
                self.r = oracle.RefCsr(self.c)
                self.values = torch.from_numpy(self.r.values_view())
                WT, perm = oracle.transpose_with_perm(self.c)
                self.rt = oracle.RefCsr(WT)
                self.wt_values = self.rt.values_view()
                self.perm = perm
                self.live = perm >= 0
            else:
                self.values = torch.from_numpy(self.c.values)
                self.WT, self.perm = oracle.transpose_with_perm(self.c)
                self.live = self.perm >= 0

        def fwd(self, X):
            if kind == "reference":
                Y = np.empty((self.c.nrows, X.shape[1]), np.float32)
                self.r.spmm_into(X, Y)
                return Y
            return oracle.spmm(self.c, X)

        def dw(self, dY, X):
            if kind == "reference":
                dW = np.empty(self.c.total_capacity, np.float32)
                self.r.sddmm_into(dY, X, dW)
                return dW
            return oracle.sddmm(self.c, dY, X)

        def set_update(self, rng):
            self.topo_update("random", seed=int(rng.integers(0, 2**63)))

        def topo_update(self, rule, seed=0, G=None):
            """SET / RigL on this layer (router.py:378-478 / :598-732 restated in
            oracle.drop_grow), rows written back through the reference's
            rewrite_row, then the transpose rebuilt (layout.py:460-536 restated)."""
            if kind == "reference":
                vals, cols, nnz, _ = self.r.arrays()
                c = oracle.Csr(self.c.nrows, self.c.ncols, vals, cols, self.c.row_start, nnz,
                               self.c.row_capacity)
            else:
                c = self.c
            q = oracle.drop_grow(c, max(1, int(0.3 * c.nnz)), rule, G=G, seed=seed)
            if kind == "reference":
                for i in range(q.nrows):
                    s0, n = int(q.row_start[i]), int(q.row_nnz[i])
                    if n:
                        self.r.rewrite_row(i, q.col_indices[s0:s0 + n], q.values[s0:s0 + n])
                self.c = q
                WT, self.perm = oracle.transpose_with_perm(q)
                self.rt = oracle.RefCsr(WT)
                self.wt_values = self.rt.values_view()
            else:
                self.c.col_indices[:] = q.col_indices
                self.c.values[:] = q.values
                self.WT, self.perm = oracle.transpose_with_perm(self.c)
            self.live = self.perm >= 0

        def dx(self, dY):
            # cache hit: refresh WT values through perm (ops.py:83-94), then SpMM
            if kind == "reference":
                self.wt_values[self.live] = self.values.numpy()[self.perm[self.live]]
                out = np.empty((self.rt.p.nrows, dY.shape[1]), np.float32)
                self.rt.spmm_into(dY, out)
                return out
            self.WT.values[self.live] = self.values.numpy()[self.perm[self.live]]
            return oracle.spmm(self.WT, dY)

    class RefFn(torch.autograd.Function):
        @staticmethod
        def forward(ctx, values, layer, X):
            ctx.layer = layer
            ctx.save_for_backward(X)
            return torch.from_numpy(layer.fwd(X.detach().contiguous().numpy()))

        @staticmethod
        def backward(ctx, dY):
            (X,) = ctx.saved_tensors
            dYc = dY.detach().contiguous().numpy()
            layer = ctx.layer
            dW = torch.from_numpy(layer.dw(dYc, X.detach().numpy()))
            dX = torch.from_numpy(layer.dx(dYc))  # the reference always computes dX
            return dW, None, dX

    class RefLinear(torch.nn.Module):
        """SparseLinear.forward (nn.py:210-245) over the reference's kernels."""

        def __init__(self, sl):
            super().__init__()
            self.hl = HostLayer(sl._csr)
            self.w = torch.nn.Parameter(self.hl.values)
            self.bias = (None if sl.bias is None
                         else torch.nn.Parameter(sl.bias.detach().cpu().clone()))
            self.fin, self.fout = sl.in_features, sl.out_features

        def forward(self, x):
            shp = x.shape
            X_col = x.reshape(-1, self.fin).contiguous().t().contiguous()
            y = RefFn.apply(self.w, self.hl, X_col).t()
            if self.bias is not None:
                y = y + self.bias
            return y.reshape(shp[:-1] + (self.fout,))

    def swap_sparse(module):
        import sparsecore_amd as slk

        for name, child in list(module.named_children()):
            if isinstance(child, slk.SparseLinear):
                setattr(module, name, RefLinear(child))
            else:
                swap_sparse(child)

    if isinstance(work, (C2, GPTWork)):
        # same seed on the CPU: identical weights and inputs, then the
        # SparseLinear layers run on the reference kernels
        if isinstance(work, GPTWork):
            host = type(work)(torch.device("cpu"), work.seed, with_set=False)
        else:
            host = type(work)(torch.device("cpu"), work.seed)
        swap_sparse(host.model)
        if isinstance(work, C2):
            opt = torch.optim.SGD(host.model.parameters(), lr=0.01)

            def step():
                opt.zero_grad(set_to_none=True)
                loss = torch.nn.functional.cross_entropy(host.model(host.x), host.labels)
                loss.backward()
                opt.step()

            sample = "C2 train steps (MLP 784->512->10, batch 256)"
        else:
            opt = torch.optim.SGD(host.model.parameters(), lr=0.01) if work.train else None
            refs = [m for m in host.model.modules() if isinstance(m, RefLinear)]
            set_rng = np.random.default_rng(work.seed)

            def step():
                for prm in host.model.parameters():
                    prm.grad = None
                logits = host.model(host.idx)
                torch.nn.functional.cross_entropy(logits.reshape(-1, host.vocab),
                                                  host.tgt.reshape(-1)).backward()
                if opt is not None:
                    opt.step()
                if work.set_update:
                    for rl in refs:
                        rl.hl.set_update(set_rng)

            if work.set_update:
                sample = (f"{work.name.upper()} train steps (fwd+bwd+SGD on the reference kernels; "
                          f"SET on {len(refs)} layers: numpy restatement of router.py with the "
                          f"reference's rewrite_row; numpy transpose rebuild), "
                          f"{work.tokens_per_step()} tokens")
            else:
                sample = (f"{work.name.upper()} forward+backward steps, "
                          f"{work.tokens_per_step()} tokens")
        unit_per_step = work.tokens_per_step()
        unit = "tokens/s"
    elif work.rigl:
        return _cpu_rigl_sample(work, HostLayer, kind, threads, seconds,
                                row_div=16 if threads > 1 else 64)
    else:
        hl = HostLayer(work.W)
        X = work.X.cpu().numpy()
        dY = work.dY.cpu().numpy()

        def step():
            hl.fwd(X)
            hl.dw(dY, X)
            hl.dx(dY)

        unit_per_step = work.step_bytes() / 1e9
        unit = "GB/s"
        sample = f"{work.name} fwd+dW+dX steps ({work.M}x{work.K}, N={work.N})"

    # 3 warm-up steps (1 where a step takes more than a twentieth of the
    # budget), then up to 30 steps timed one by one within the budget; the
    # median step is reported
    t0 = time.perf_counter()
    step()
    if time.perf_counter() - t0 < seconds / 20:
        for _ in range(2):
            step()
    times = []
    t_all = time.perf_counter()
    while len(times) < 30:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_all > seconds:
            break
    times.sort()
    n = len(times)
    med = times[n // 2] if n % 2 else 0.5 * (times[n // 2 - 1] + times[n // 2])
    return {"value": unit_per_step / med, "unit": unit, "cores": threads, "kind": kind,
            "sample": f"median of {n} timed {sample} (after warm-up), OpenMP/torch "
                      f"threads={threads}, ms/step median={1e3 * med:.3f} "
                      f"mean={1e3 * sum(times) / n:.3f}"}


def _cpu_rigl_sample(work, HostLayer, kind, threads, seconds, row_div=16):
    """C5 RigL step on the host, sampled on the first 1/row_div of W's rows
    (the rows are a random permutation of the Zipf ranks): fwd + dW + dX on
    the reference kernels, the reference's dense_grad, the RigL rewrite and
    the transpose rebuild. Each part's time is scaled to the full layer
    (kernel and rewrite parts by the nnz ratio, dense_grad by the row
    ratio)."""
    import types

    import oracle

    W = work.W
    M, K, N = work.M, work.K, work.N
    Ms = max(1, M // row_div)
    end = int(W.row_start[Ms].item()) if Ms < M else W.total_capacity
    sl = types.SimpleNamespace(nrows=Ms, ncols=K, values=W.values[:end],
                               col_indices=W.col_indices[:end], row_start=W.row_start[:Ms],
                               row_nnz=W.row_nnz[:Ms], row_capacity=W.row_capacity[:Ms])
    hl = HostLayer(sl)
    nnz_s = hl.c.nnz
    X = work.X.cpu().numpy()
    dY = work.dY[:Ms].cpu().numpy()
    dense = oracle.ref_dense_grad if kind == "reference" else oracle.dense_grad
    t_k = t_g = t_u = 0.0
    n = 0
    t_all = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        hl.fwd(X)
        hl.dw(dY, X)
        hl.dx(dY)
        t1 = time.perf_counter()
        G = dense(dY, X)
        t2 = time.perf_counter()
        hl.topo_update("gradient", G=G)
        t3 = time.perf_counter()
        if n > 0:  # the first step is the warmup
            t_k += t1 - t0
            t_g += t2 - t1
            t_u += t3 - t2
        n += 1
        if n >= 3 and time.perf_counter() - t_all > seconds:
            break
    steps = n - 1
    r_nnz, r_rows = W.nnz / max(nnz_s, 1), M / Ms
    est = (t_k * r_nnz + t_g * r_rows + t_u * r_nnz) / steps
    return {"value": N / est, "unit": "tokens/s", "cores": threads, "kind": kind,
            "sample": f"{steps} RigL steps on rows 0..{Ms - 1} of {M} (nnz {nnz_s} of {W.nnz}), "
                      f"scaled to the full layer: fwd+dW+dX {1e3 * t_k / steps:.1f} ms x "
                      f"{r_nnz:.2f}, dense_grad {1e3 * t_g / steps:.1f} ms x {r_rows:.0f}, "
                      f"rewrite+rebuild {1e3 * t_u / steps:.1f} ms x {r_nnz:.2f} = "
                      f"{1e3 * est:.0f} ms/step, OpenMP threads={threads}"}


# ───────────────────────────── main ──────────────────────────────────────────

def build_work(name: str, dev, seed: int):
    if name == "c2":
        return C2(dev, seed)
    if name == "c3":
        return C3(dev, seed)
    if name == "c4":
        return C4(dev, seed)
    if name == "c1":
        return make_c1(dev, seed)
    return make_c5(dev, seed, 0.05 if name.startswith("c5-95") else 0.01,
                   rigl=name.endswith("rigl"))


def calibrate_copy(args, dev) -> None:
    """A known-size reference dispatch for HBM byte counters: three copies of
    --calibrate-copy-mib MiB."""
    import torch

    if args.calibrate_copy_mib <= 0:
        return
    stage(f"copy calibration: {args.calibrate_copy_mib} MiB x 3")
    n = args.calibrate_copy_mib * (1 << 20) // 4
    src = torch.ones(n, device=dev)
    dst = torch.empty(n, device=dev)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def measure(work, args):
    """Warmup, graph capture (where the topology is fixed), the timed region
    and the per-kernel timings of one workload. Returns the fields of its
    bench line."""
    import torch

    stage(f"{work.name}: eager warmup")
    work.body()
    eager_s = timed_loop(work.body, max(1, args.warmup)) / max(1, args.warmup)

    use_graph = not args.no_graph and not getattr(work, "dynamic", False)
    graph_ok = False
    # Several steps per graph only where a replay's launch latency is a visible
    # share of the step (sub-millisecond steps: C1, C2), one step otherwise.
    # A graph that holds memset nodes is not replayed at all (the step runs
    # eagerly): memset nodes have left memory uncleared on replays after the
    # first on these machines, and library code records them (rocprim's
    # partition zeroes its selected-item count with hipMemsetAsync; torch's
    # embedding backward runs that partition, torch's multi-block reductions
    # zero their semaphores the same way). A partition whose count starts
    # from the previous replay's total writes its outputs past their end.
    S = max(1, min(args.graph_steps, args.steps)) if eager_s < 1e-3 else 1
    graph_nodes = None
    if use_graph:
        params = work.params()
        snap = [p.detach().clone() for p in params]
        stage(f"eager reference steps for the graph check (2 x {S} steps)")
        eager_flat = []
        for _ in range(2 * S):
            o = work.body()
            eager_flat += [t.detach().clone() for t in (o if isinstance(o, tuple) else (o,))]
            del o
        eager_params = [p.detach().clone() for p in params]
        with torch.no_grad():
            for p, s in zip(params, snap):
                p.copy_(s)
        torch.cuda.synchronize()
        stage(f"graph capture ({S} steps per graph)")
        g, gouts, graph_nodes = capture(work.body, steps=S)
        g1 = None
        if args.steps % S or args.warmup % S:
            g1, _, nodes1 = capture(work.body)
            for k, v in nodes1.items():
                graph_nodes[k] = graph_nodes.get(k, 0) + v
        stage(f"graph node types: {graph_nodes}")
        with torch.no_grad():
            for p, s in zip(params, snap):
                p.copy_(s)
        graph_ok = not graph_nodes.get("memset")
        if not graph_ok:
            print(f"bench.py: the captured step holds {graph_nodes['memset']} memset nodes; "
                  f"not replaying it, timing eager launches", file=sys.stderr)
        else:
            stage("graph replay check (two replays, every step against eager)")
        if graph_ok:
            for r in range(2):
                g.replay()
                torch.cuda.synchronize()
                got = [t for o in gouts for t in (o if isinstance(o, tuple) else (o,))]
                want = eager_flat[r * len(got):(r + 1) * len(got)]
                graph_ok = graph_ok and len(want) == len(got) and all(
                    torch.equal(a, b) for a, b in zip(got, want))
            graph_ok = graph_ok and all(torch.equal(p, e) for p, e in zip(params, eager_params))
            if not graph_ok:
                print("bench.py: graph replay differs from eager; timing eager launches",
                      file=sys.stderr)
        if not graph_ok:
            del g, g1, gouts  # release the graphs' private memory pool
            with torch.no_grad():
                for p, s in zip(params, snap):
                    p.copy_(s)
        if graph_ok:
            runner = GraphSteps(g, S, g1)
            run_steps = runner.run
        else:
            def run_steps(n):
                for _ in range(n):
                    work.body()
        run_steps(args.warmup)
    else:
        def run_steps(n):
            for _ in range(n):
                work.body()

    stage(f"{work.name}: timed region, {args.steps} steps "
          f"(graph={graph_ok if use_graph else False})")
    elapsed = timed_run(run_steps, args.steps)
    ms_per_step = 1e3 * elapsed / args.steps
    topo_ms = 0.0
    if getattr(work, "algo", None) is not None or getattr(work, "rigl", False):
        stage("topology update timing (SET/RigL + transpose rebuild)")
        reps = 5
        topo_ms = 1e3 * timed_loop(work.topology_update, reps) / reps

    kern = []
    path_labels = ("spmm_fwd", "sddmm_dw", "transpose_refresh", "spmm_dx", "backward_fused")
    for name, fn, nbytes, nflops in work.kernels():
        stage(f"kernel timing: {name}")
        ms, mean_ms, reps = kernel_time_ms(fn)
        kern.append({"kernel": name, "median_us": round(ms * 1e3, 3),
                     "mean_us": round(mean_ms * 1e3, 3), "bytes": nbytes,
                     "flops": nflops, "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "timed_calls": reps, "warmup_calls": KERNEL_WARMUP})
        if graph_ok and name in path_labels and ms < 0.1:
            # microsecond kernels: also the per-call time inside a graph,
            # which the graph-replayed step pays
            kern[-1]["graph_us"] = round(graph_call_us(fn), 3)
    # roofline on the path's dominant kernel (forward SpMM, dX SpMM or dW SDDMM)
    dom = max((k for k in kern if k["kernel"].startswith(("spmm", "sddmm", "backward_"))),
              key=lambda k: k["median_us"])
    achieved = dom["bytes"] / (dom["median_us"] * 1e-6) / 1e9
    tflops = dom["flops"] / (dom["median_us"] * 1e-6) / 1e12
    # HBM bytes per launch of the dominant kernel, from the committed
    # rocprofv3 FETCH_SIZE/WRITE_SIZE summary of this workload (if any)
    traffic = None
    tf = ROOT / "profiles" / f"traffic_{work.name}.json"
    if not tf.exists():  # a RigL workload's layer is the static workload's layer
        tf = ROOT / "profiles" / f"traffic_{work.name.removesuffix('-rigl')}.json"
    if tf.exists():
        tj = json.loads(tf.read_text())
        traffic = tj.get(dom["kernel"], tj.get(dom["kernel"].split("[")[0]))

    if isinstance(work, C2):
        value = work.tokens_per_step() * args.steps / elapsed
        unit = "tokens/s"
        W = work.spmm_layer()
        l1 = [k for k in kern if "[l1" in k["kernel"]]
        spmm_us = sum(k["median_us"] for k in kern)
        path = {"spmm_kernels_us_per_step": round(spmm_us, 2),
                "layer1_fwd_dw_GBps": round(sum(k["bytes"] for k in l1) /
                                            (sum(k["median_us"] for k in l1) * 1e-6) / 1e9, 1),
                "layer1_fwd_dw_GFLOPs": round(sum(k["flops"] for k in l1) /
                                              (sum(k["median_us"] for k in l1) * 1e-6) / 1e9, 1),
                "layer1_nnz": W.nnz}
        config = {"workload": "c2: " + work.desc, "global_batch": work.batch,
                  "l1_dx": "not computed (the input needs no grad; the reference computes "
                           "and discards it)",
                  "graph": graph_ok, "graph_steps": S if graph_ok else 0}
        if graph_nodes and graph_nodes.get("memset"):
            config["graph_refused"] = f"{graph_nodes['memset']} memset nodes"
    elif isinstance(work, GPTWork):
        value = work.tokens_per_step() * args.steps / elapsed
        unit = "tokens/s"
        per_block_us = sum(k["median_us"] for k in kern
                           if k["kernel"].startswith(("spmm", "sddmm")))
        path = {"block0_sparse_kernels_us": round(per_block_us, 1),
                "block0_sparse_GBps": round(sum(k["bytes"] for k in kern) /
                                            (per_block_us * 1e-6) / 1e9, 1),
                "block0_sparse_GFLOPs": round(sum(k["flops"] for k in kern) /
                                              (per_block_us * 1e-6) / 1e9, 1),
                "sparse_kernel_share_of_step": round(work.n_layers * per_block_us * 1e-3 /
                                                     ms_per_step, 3)}
        if work.algo is not None:
            path["topology_update_ms_per_step"] = round(topo_ms, 3)
        config = {"workload": f"{work.name}: {work.desc}", "global_batch": work.batch,
                  "seq_len": work.ctx, "graph": graph_ok,
                  "graph_steps": S if graph_ok else 0}
        if graph_nodes and graph_nodes.get("memset"):
            config["graph_refused"] = f"{graph_nodes['memset']} memset nodes"
    else:
        path_k = [k for k in kern if k["kernel"] in ("spmm_fwd", "sddmm_dw", "transpose_refresh",
                                                      "spmm_dx", "backward_fused")]
        path_us = sum(k["median_us"] for k in path_k)
        path = {"fwd_dw_dx_us": round(path_us, 1),
                **({"fwd_dw_dx_graph_us": round(sum(k["graph_us"] for k in path_k), 2)}
                   if path_k and all("graph_us" in k for k in path_k) else {}),
                "fwd_dw_dx_GBps": round(work.step_bytes() / (path_us * 1e-6) / 1e9, 1),
                "fwd_dw_dx_GFLOPs": round(work.step_flops() / (path_us * 1e-6) / 1e9, 1),
                "step_bytes_fwd_dw_dx": work.step_bytes(), "nnz": work.W.nnz}
        if work.rigl:
            value = work.N * args.steps / elapsed
            unit = "tokens/s"
            path["topology_update_ms_per_step"] = round(topo_ms, 3)
            config = {"workload": f"{work.name}: {work.desc}", "graph": False}
        else:
            value = work.step_bytes() * args.steps / elapsed / 1e9
            unit = "GB/s"
            path["GFLOP/s"] = round(work.step_flops() * args.steps / elapsed / 1e9, 1)
            config = {"workload": f"{work.name}: {work.desc}", "graph": graph_ok,
                      "graph_steps": S if graph_ok else 0,
                      "transpose_rebuild_ms": round(work.rebuild_ms, 3)}
            if graph_nodes and graph_nodes.get("memset"):
                config["graph_refused"] = f"{graph_nodes['memset']} memset nodes"
    roofline_mfma = None
    apx = [k for k in kern if k["kernel"] == "dense_grad_approx"]
    if apx:
        # RigL's matrix-core pass: three bf16 products (x_h·y_h, x_h·y_l,
        # x_l·y_h) of 2·M·K·N flops each, against the dense bf16 peak
        t = 3 * apx[0]["flops"] / (apx[0]["median_us"] * 1e-6) / 1e12
        roofline_mfma = {"kernel": "dense_grad_approx", "achieved": round(t, 1),
                         "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(t / MFMA_BF16_PEAK_TFLOPS, 4)}
    return {
        "value": value, "unit": unit, "ms_per_step": ms_per_step, "config": config,
        "path": path, "kernels": kern,
        "roofline": {"bound": "hbm", "kernel": dom["kernel"], "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     # the same kernel's 2*nnz*N flops against the published
                     # fp32 peak, and against the non-packed VALU rate the
                     # kernels actually compute at (MFMA is not used)
                     "compute": {"achieved": round(tflops, 3), "unit": "TFLOP/s",
                                 "peak": FP32_PEAK_TFLOPS,
                                 "frac": round(tflops / FP32_PEAK_TFLOPS, 4),
                                 "frac_of_nonpacked_valu": round(tflops / VALU_NONPACKED_TFLOPS,
                                                                 4)},
                     **({"mfma": roofline_mfma} if roofline_mfma else {})},
    }


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              f"the multi-GPU sharding is a design note, not a measured path.", file=sys.stderr)
        sys.exit(2)
    import torch

    import sparsecore_amd

    if not torch.cuda.is_available():
        sys.exit("bench.py needs a HIP device")
    if not sparsecore_amd.native_available():
        sys.exit("bench.py: libsparsecore_amd.so is not built (python -m sparsecore_amd.build)")
    dev = torch.device("cuda:0")
    global KERNEL_REPS
    KERNEL_REPS = max(1, args.kernel_reps)
    stage(f"workload {args.workload}: building")
    work = build_work(args.workload, dev, args.seed)
    if args.only_kernel is not None:
        got = [k for k in work.kernels() if k[0] == args.only_kernel]
        if not got:
            sys.exit(f"bench.py: no kernel label {args.only_kernel!r} in {args.workload}: "
                     f"{[k[0] for k in work.kernels()]}")
        name, fn, nbytes, nflops = got[0]
        stage(f"kernel timing: {name}")
        ms, mean_ms, reps = kernel_time_ms(fn)
        calibrate_copy(args, dev)
        print(json.dumps({"workload": args.workload, "kernel": name,
                          "median_us": round(ms * 1e3, 3), "mean_us": round(mean_ms * 1e3, 3),
                          "bytes": nbytes, "flops": nflops, "reps": reps}), flush=True)
        return
    m = measure(work, args)
    line = {
        "metric": METRIC,
        "value": round(m["value"], 3),
        "unit": m["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(m["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": m["config"],
        "path": m["path"],
        "kernels": m["kernels"],
        "roofline": m["roofline"],
        "cpu_baseline": None,
    }
    calibrate_copy(args, dev)
    if not args.no_cpu:
        stage("cpu baseline")
        try:
            line["cpu_baseline"] = cpu_baseline(work, args.cpu_seconds)
        except Exception as e:  # the baseline is reported, never required
            line["cpu_baseline"] = {"error": repr(e)}
    if args.workload == "c5-95-rigl" and not args.no_extra:
        del work
        torch.cuda.empty_cache()
        stage("extra workload c5-99-rigl: building")
        w99 = build_work("c5-99-rigl", dev, args.seed)
        m99 = measure(w99, args)
        line["extra"] = {"c5-99-rigl": {
            "value": round(m99["value"], 3), "unit": m99["unit"],
            "ms_per_step": round(m99["ms_per_step"], 5), "config": m99["config"],
            "path": m99["path"], "kernels": m99["kernels"], "roofline": m99["roofline"]}}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
