#!/usr/bin/env python3
"""Benchmark of the paged-KV hot path: decode attention + KV append at Qwen3-1.7B shape.

Workload (the metric's configuration): 28 layers, 16 query heads over 8 kv
heads, head_dim 128; 32 sequences with contexts uniform in [256, 4096] (after the step's append), one
new token each per step; f16 K/V in 16-token pages scattered by a seeded permutation of an 8,192-page
pool (131,072 tokens: the "28k-token pool" of the config cannot hold the ~69.6k tokens the batch
needs); q/k/v activations N(0, 1), resident in HBM before timing.

A step is what a serving step does on this path: the host plans it (page allocation through the
BlockManager, packing, one upload), then for each of the 28 layers the fused QK-norm + RoPE + KV
append and the paged decode attention (+ split merge) run on the GPU. Contexts grow by one token per
step, as in decoding.

Prints one JSON line (the driver's contract); a human summary goes to stderr.
"""
from __future__ import annotations

import argparse
import contextlib
import gc
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

N_LAYERS, H, KVH, D = 28, 16, 8, 128
BATCH, CTX_LO, CTX_HI = 32, 256, 4096
POOL_PAGES = 8192
PAGE = 16
SEED = 20261005
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16 MFMA (no sparsity)
KV_BYTES_PER_TOKEN = 2 * KVH * D * 2  # f16 K + V of one token, one layer: 4096 B
# Per new token per layer: qkv in 8 KiB + q out 4 KiB + KV append 4 KiB + q in 4 KiB + attention out 4 KiB
# when the append is its own launch; the fused append + attention keeps q on chip (16 KiB).
TOKEN_BYTES = 8192 + 4096 + 4096 + 4096 + 4096
FUSED_TOKEN_BYTES = 8192 + 4096 + 4096
METRIC = "paged decode-attn+append tokens/s and % HBM peak (Qwen3-1.7B shape, batch 32)"


@contextlib.contextmanager
def collector_paused():
    """Python's cyclic garbage collector off inside a timed region, after one full collection (as timeit does).
    The step loop here stands in for an engine's C++ loop, which has no collector. A collection of an older
    generation that lands inside a timed region stalls this host thread for tens of milliseconds, long enough for
    the GPU to run out of queued steps: at BASELINE config 3 plain runs read 3.78-4.20 ms/step depending on where
    it landed (one ~45 ms idle window in the GPU trace), and 3.772-3.776 ms/step with the collector off."""
    gc.collect()
    was = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Workload:
    """Config 2 on the GPU path."""

    def __init__(self, total_steps: int, split_len: int = 512, graph: bool = False, block: bool = False):
        import torch

        from ember_amd import BlockManager
        from ember_amd.paged_kv import PagedKv

        self.torch = torch
        rng = np.random.default_rng(SEED)
        self.ctx_after = rng.integers(CTX_LO, CTX_HI + 1, BATCH)  # context after the first step's append
        self.ctx = self.ctx_after - 1                             # cached before the first step
        max_ctx = int(self.ctx_after.max()) + total_steps + PAGE
        self.max_blocks = (max_ctx + PAGE - 1) // PAGE
        # Pages scattered over the pool: take every block, give them back in a seeded random order,
        # so the allocator's free stack hands them out permuted.
        self.bm = BlockManager(POOL_PAGES, False)
        every = [self.bm.allocate() for _ in range(POOL_PAGES)]
        self.bm.release_all([every[i] for i in rng.permutation(POOL_PAGES)])
        # The engine's block tables, kept as one array and extended in place as pages are allocated.
        self.tables = np.zeros((BATCH, self.max_blocks), np.int32)
        self.n_blocks = [0] * BATCH
        for s in range(BATCH):
            self._ensure(s, int(self.ctx[s]))
        self.tokens = np.zeros(BATCH, np.int32)
        self.query_start = np.arange(BATCH + 1, dtype=np.int32)
        self.stream = torch.cuda.Stream()
        self.kv = PagedKv(n_layers=N_LAYERS, n_heads=H, n_kv_heads=KVH, rms_eps=1e-6, rope_theta=1e6,
                          max_position=self.max_blocks * PAGE, num_blocks=POOL_PAGES, max_batch_tokens=BATCH,
                          max_seqs=BATCH, dtype=torch.float16, split_len=split_len, stream=self.stream)
        g = torch.Generator(device="cuda").manual_seed(SEED)
        with torch.cuda.stream(self.stream):
            for layer in range(N_LAYERS):  # cached K/V: random f16 in every page (the values do not matter)
                self.kv.pool_view(layer, "k").normal_(generator=g)
                self.kv.pool_view(layer, "v").normal_(generator=g)
            self.qkv = torch.randn((N_LAYERS, BATCH, (H + 2 * KVH) * D), generator=g, device="cuda",
                                   dtype=torch.float16)
            self.qn = 1 + 0.1 * torch.randn((N_LAYERS, D), generator=g, device="cuda")
            self.kn = 1 + 0.1 * torch.randn((N_LAYERS, D), generator=g, device="cuda")
            self.out = torch.empty((BATCH, H, D), device="cuda", dtype=torch.float16)
        self.stream.synchronize()
        # Per-layer device addresses, checked once here: the timed loop calls the C ABI directly, as a C++
        # engine's layer loop would, without per-call Python tensor checks.
        for t in (self.qkv, self.qn, self.kn, self.out):
            assert t.is_cuda and t.is_contiguous()
        self.layer_args = [(self.qkv[layer].data_ptr(), self.qn[layer].data_ptr(), self.kn[layer].data_ptr())
                           for layer in range(N_LAYERS)]
        # Graph replay: the step's launches for all layers as one hipGraph (the batch of 32 is its own token
        # bucket, so no padding rows are read or written).
        self.graph = graph
        self.graph_io = [(self.qkv[layer], self.out, self.qn[layer], self.kn[layer], None) for layer in range(N_LAYERS)]
        self.sum_ctx_timed = 0
        self.alloc_s = 0.0
        self.block = block
        if block:
            self._init_block(g)

    def _init_block(self, g) -> None:
        """The whole attention block per layer (input RMSNorm, qkv GEMV, append + attention, o GEMV into the f32
        residual), with random weights of its own per layer (704 MB in all), called through the C ABI."""
        import ctypes

        from ember_amd import _lib

        torch, HID, NQKV = self.torch, H * D, (H + 2 * KVH) * D
        with torch.cuda.stream(self.stream):
            self.w_qkv = [torch.randn((NQKV, HID), generator=g, device="cuda", dtype=torch.float16) * 0.02
                          for _ in range(N_LAYERS)]
            self.w_o = [torch.randn((HID, HID), generator=g, device="cuda", dtype=torch.float16) * 0.02
                        for _ in range(N_LAYERS)]
            self.in_norm = [torch.ones(HID, device="cuda") for _ in range(N_LAYERS)]
            self.h = torch.randn((BATCH, HID), generator=g, device="cuda")
            self.xn = torch.empty((BATCH, HID), device="cuda", dtype=torch.float16)
            self.qkv_buf = torch.empty((BATCH, NQKV), device="cuda", dtype=torch.float16)
        from ember_amd import kernels as K

        with torch.cuda.stream(self.stream):
            self.p_qkv = [K.gemv_pack(w, stream=self.stream) for w in self.w_qkv]
            self.p_o = [K.gemv_pack(w, stream=self.stream) for w in self.w_o]
        ws_bytes = max(int(_lib.lib().ember_hip_gemv_workspace_bytes(BATCH, n, HID)) for n in (NQKV, HID))
        self.gemv_ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")  # both GEMVs, one stream
        torch.cuda.synchronize()  # the zero fill ran on torch's stream
        self.block_args = []
        for layer in range(N_LAYERS):
            n = _lib.NormArgs()
            n.x, n.w, n.out, n.R, n.hidden, n.eps = (self.h.data_ptr(), self.in_norm[layer].data_ptr(),
                                                     self.xn.data_ptr(), BATCH, HID, 1e-6)
            gq = _lib.GemvArgs()
            gq.A, gq.lda, gq.W, gq.M, gq.N, gq.K = self.xn.data_ptr(), HID, self.p_qkv[layer].data_ptr(), BATCH, NQKV, HID
            gq.C, gq.ldc, gq.epilogue = self.qkv_buf.data_ptr(), NQKV, _lib.EPILOGUE_STORE_F16
            go = _lib.GemvArgs()
            go.A, go.lda, go.W, go.M, go.N, go.K = self.out.data_ptr(), HID, self.p_o[layer].data_ptr(), BATCH, HID, HID
            go.C, go.ldc, go.epilogue = self.h.data_ptr(), HID, _lib.EPILOGUE_ADD_F32
            for ga in (gq, go):
                ga.workspace, ga.workspace_bytes = self.gemv_ws.data_ptr(), ws_bytes
                ga.w_packed = 1  # the weights as a backend keeps them, in the GEMV's packed layout
            self.block_args.append((ctypes.byref(n), ctypes.byref(gq), ctypes.byref(go), n, gq, go,
                                    self.qn[layer].data_ptr(), self.kn[layer].data_ptr()))
        self.block_weight_bytes = N_LAYERS * (NQKV * HID * 2 + HID * HID * 2)

    def _ensure(self, s: int, upto: int) -> None:
        need = (upto + PAGE - 1) // PAGE
        while self.n_blocks[s] < need:
            b = self.bm.allocate()
            if b < 0:
                raise RuntimeError("the page pool is exhausted")
            self.tables[s, self.n_blocks[s]] = b
            self.n_blocks[s] += 1

    def step(self) -> int:
        from ember_amd import _lib
        from ember_amd.paged_kv import StepBatch

        t0 = time.perf_counter()
        for s in range(BATCH):
            self._ensure(s, int(self.ctx[s]) + 1)
        self.alloc_s += time.perf_counter() - t0
        pos = self.ctx.astype(np.int32)
        b = StepBatch(tokens=self.tokens, positions=pos, query_start=self.query_start, context_len=pos + 1,
                      block_tables=self.tables.reshape(-1), max_blocks=self.max_blocks)
        if self.graph and self.kv.decode_graph(b, self.graph_io):
            self.ctx += 1
            return int(pos.sum() + BATCH)
        self.kv.plan(b)
        layer_fn, h, out = _lib.lib().ember_kv_layer, self.kv._h, self.out.data_ptr()
        if self.block:
            lib, st, qkv = _lib.lib(), self.stream.cuda_stream, self.qkv_buf.data_ptr()
            for layer, (na, ga, oa, _n, _g, _o, qn, kn) in enumerate(self.block_args):
                if (lib.ember_hip_rmsnorm_rows(na, st) != _lib.OK or lib.ember_hip_gemv(ga, st) != _lib.OK
                        or layer_fn(h, layer, qkv, qn, kn, None, out) != _lib.OK or lib.ember_hip_gemv(oa, st) != _lib.OK):
                    _lib.check(-1, "attention block")
            self.ctx += 1
            return int(pos.sum() + BATCH)
        for layer, (qkv, qn, kn) in enumerate(self.layer_args):
            if layer_fn(h, layer, qkv, qn, kn, None, out) != _lib.OK:
                _lib.check(-1, "kv_layer")
        self.ctx += 1
        return int(pos.sum() + BATCH)  # sum of contexts after this step's append


TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic_config2.json"


def measured_traffic():
    """HBM bytes per decode launch as the rocprofv3 FETCH_SIZE / WRITE_SIZE passes measured them (scaled by the
    copy-kernel calibration), read from the summary committed with those passes, with the algorithmic bytes of
    the launches those passes covered: (traffic, traffic / algorithmic). (None, None) without a summary. The
    counters cannot run beside this timing, so the figure is that committed measurement, not this run's."""
    try:
        t = json.loads(TRAFFIC_FILE.read_text())
        total = float(t["fetch_bytes_per_launch"]) + float(t["write_bytes_per_launch"])
        ratio = total / float(t["algorithmic_bytes_per_launch"])
    except (OSError, ValueError, KeyError, ZeroDivisionError):
        return None, None
    log(f"[bench] HBM traffic per launch (committed rocprofv3 PMC passes, {TRAFFIC_FILE.name}): {total / 1e6:.1f} MB, "
        f"{ratio:.3f} x the algorithmic bytes of the launches it measured")
    return round(total), round(ratio, 4)


def copy_calibration(steps: int) -> int:
    """Known-size HBM traffic for scaling the rocprofv3 FETCH_SIZE / WRITE_SIZE counters: each launch of the
    page-copy kernel reads and writes exactly 2,048 pages x 28 layers x (K + V) x 32 KiB = 3.76 GB."""
    import torch

    from ember_amd import kernels as K

    n_pages, per_page = 4096, KVH * PAGE * D  # elements of one layer's K page (all kv heads)
    pool_k = torch.zeros(N_LAYERS * n_pages * per_page, dtype=torch.float16, device="cuda")
    pool_v = torch.zeros_like(pool_k)
    rng = np.random.default_rng(SEED)
    src = rng.permutation(n_pages)[: n_pages // 2]
    dst = np.setdiff1d(np.arange(n_pages), src)
    rng.shuffle(dst)
    for _ in range(steps):
        K.copy_pages(pool_k, pool_v, src, dst, n_layers=N_LAYERS, layer_stride=n_pages * per_page, n_kv=KVH,
                     num_blocks=n_pages)
    torch.cuda.synchronize()
    per_launch = src.size * N_LAYERS * 2 * per_page * 2
    print(json.dumps({"copy_pages_launches": steps, "bytes_read_per_launch": per_launch,
                      "bytes_written_per_launch": per_launch}), flush=True)
    return 0


def cpu_baseline(seconds: float) -> dict:
    """The oracle (the reference's f32 CPU path, restated) on one layer of the same batch, threads = the
    host's CPU share. Reported as tokens/s for 28 layers (per-layer time x 28)."""
    import oracle

    # hardware_concurrency() on a one-GPU box shows the whole host, but this job's CPU share is 16 threads
    # (OMP_NUM_THREADS says the same there): the baseline uses the share and names the host's count beside it.
    host_cpus = os.cpu_count() or 1
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else host_cpus
    threads = min(16, affinity)
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    rng = np.random.default_rng(SEED)
    ctx_after = rng.integers(CTX_LO, CTX_HI + 1, BATCH)
    perm = rng.permutation(POOL_PAGES).astype(np.int32)
    pages = (ctx_after + PAGE - 1) // PAGE
    mb = int(pages.max()) + 1
    tables = np.zeros((BATCH, mb), np.int32)
    at = 0
    for s in range(BATCH):
        tables[s, :pages[s]] = perm[at:at + pages[s]]
        at += pages[s]
    k = rng.standard_normal((POOL_PAGES, KVH, PAGE, D), dtype=np.float32)
    v = rng.standard_normal((POOL_PAGES, KVH, PAGE, D), dtype=np.float32)
    qkv = rng.standard_normal((BATCH, (H + 2 * KVH) * D), dtype=np.float32)
    inv = oracle.inv_freq(1e6, D)
    ones = np.ones(D, np.float32)
    pos = (ctx_after - 1).astype(np.int32)
    qs = np.arange(BATCH + 1, dtype=np.int32)

    def one_step():
        q = oracle.append_layer(qkv, pos, qs, tables, k, v, n_heads=H, n_kv=KVH, inv_freq_=inv, q_norm=ones,
                                k_norm=ones, num_blocks=POOL_PAGES, kv_f16=False)
        oracle.attention_layer(q, pos, qs, tables, k, v, n_heads=H, n_kv=KVH, num_blocks=POOL_PAGES, kv_f16=False,
                               threads=threads)

    one_step()  # warm up (threads, pages)
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        one_step()
        times.append(time.perf_counter() - t0)
    per_layer = float(np.median(times))
    cpu_model = ""
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                cpu_model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": BATCH / (per_layer * N_LAYERS),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"1 of {N_LAYERS} layers of the same 32-sequence batch (sum of contexts {int(ctx_after.sum())}), "
                   f"f32 KV, median of {len(times)} steps ({per_layer * 1e3:.1f} ms/layer) x {N_LAYERS} layers; "
                   f"{threads} threads = this job's CPU share (host: {host_cpus} CPUs, {affinity} in this process's "
                   f"affinity); {cpu_model or platform.processor()}"),
    }


# ---- BASELINE configs 3, 4 and 5 (reported beside the metric; `--config N`) ----

class PathBench:
    """The GPU path plus the engine-side bookkeeping a config needs: a BlockManager over the pool, block
    tables kept as one array, pools filled with random f16 K/V, per-layer q/k/v activations."""

    def __init__(self, *, pool_pages, max_seqs, max_blocks, max_tokens, split_len, prefix_caching=False, seed,
                 qkv_tokens=None, shared_qkv=False):
        import torch

        from ember_amd import BlockManager
        from ember_amd.paged_kv import PagedKv

        self.torch = torch
        self.rng = np.random.default_rng(seed)
        self.bm = BlockManager(pool_pages, prefix_caching)
        every = [self.bm.allocate() for _ in range(pool_pages)]  # pages handed out in a seeded random order
        self.bm.release_all([every[i] for i in self.rng.permutation(pool_pages)])
        self.max_blocks = max_blocks
        self.tables = np.zeros((max_seqs, max_blocks), np.int32)
        self.blocks = [[] for _ in range(max_seqs)]
        self.stream = torch.cuda.Stream()
        self.kv = PagedKv(n_layers=N_LAYERS, n_heads=H, n_kv_heads=KVH, rms_eps=1e-6, rope_theta=1e6,
                          max_position=max_blocks * PAGE, num_blocks=pool_pages, max_batch_tokens=max_tokens,
                          max_seqs=max_seqs, dtype=torch.float16, split_len=split_len, stream=self.stream)
        g = torch.Generator(device="cuda").manual_seed(seed)
        with torch.cuda.stream(self.stream):
            for layer in range(N_LAYERS):
                self.kv.pool_view(layer, "k").normal_(generator=g)
                self.kv.pool_view(layer, "v").normal_(generator=g)
            rows = qkv_tokens or max_tokens
            if shared_qkv:  # one buffer read by every layer (the values are synthetic either way)
                self.qkv = torch.randn((rows, (H + 2 * KVH) * D), generator=g, device="cuda",
                                       dtype=torch.float16).expand(N_LAYERS, -1, -1)
            else:
                self.qkv = torch.randn((N_LAYERS, rows, (H + 2 * KVH) * D), generator=g, device="cuda",
                                       dtype=torch.float16)
            self.qn = 1 + 0.1 * torch.randn((N_LAYERS, D), generator=g, device="cuda")
            self.kn = 1 + 0.1 * torch.randn((N_LAYERS, D), generator=g, device="cuda")
            self.out = torch.empty((max_tokens, H, D), device="cuda", dtype=torch.float16)
        self.stream.synchronize()
        self.alloc_s = 0.0

    def ensure(self, s: int, upto: int) -> None:
        t0 = time.perf_counter()
        while len(self.blocks[s]) * PAGE < upto:
            b = self.bm.allocate()
            if b < 0:
                raise RuntimeError("the page pool is exhausted")
            self.tables[s, len(self.blocks[s])] = b
            self.blocks[s].append(b)
        self.alloc_s += time.perf_counter() - t0

    def release(self, s: int) -> None:
        t0 = time.perf_counter()
        self.bm.release_all(self.blocks[s])
        self.blocks[s] = []
        self.alloc_s += time.perf_counter() - t0

    def run(self, seqs, positions, query_start) -> None:
        """Plans and runs one step of all layers for the sequences `seqs` (rows of the block tables)."""
        from ember_amd import _lib
        from ember_amd.paged_kv import StepBatch

        positions = np.asarray(positions, np.int32)
        qs = np.asarray(query_start, np.int32)
        tab = self.tables[np.asarray(seqs)]
        ctx = np.array([positions[qs[i + 1] - 1] + 1 for i in range(len(seqs))], np.int32)
        mb = int(max(1, (ctx.max() + PAGE - 1) // PAGE))
        b = StepBatch(tokens=np.zeros(positions.size, np.int32), positions=positions, query_start=qs,
                      context_len=ctx, block_tables=np.ascontiguousarray(tab[:, :mb]).reshape(-1), max_blocks=mb)
        self.kv.plan(b)
        fn, h, out = _lib.lib().ember_kv_layer, self.kv._h, self.out.data_ptr()
        for layer in range(N_LAYERS):
            if fn(h, layer, self.qkv[layer].data_ptr(), self.qn[layer].data_ptr(), self.kn[layer].data_ptr(), None,
                  out) != _lib.OK:
                _lib.check(-1, "kv_layer")


def _timed(path, step, steps, warmup):
    """Bare pass (the step time), then a pass with HIP events around every paged-decode launch."""
    for _ in range(warmup):
        step()
    path.stream.synchronize()
    path.alloc_s = 0.0
    bytes_ = 0
    with collector_paused():
        t0 = time.perf_counter()
        for _ in range(steps):
            bytes_ += step()
        path.stream.synchronize()
        wall = time.perf_counter() - t0
    alloc_us = path.alloc_s / steps * 1e6
    path.kv.set_timing(True)
    path.kv.timing()
    path.kv.prefill_timing()
    timed_bytes = 0
    with collector_paused():
        for _ in range(steps):
            timed_bytes += step()
        path.stream.synchronize()
    path.timed_bytes = timed_bytes / steps  # the step bytes of the pass the events timed
    launches, kernel_ms = path.kv.timing()
    path.prefill_timed = path.kv.prefill_timing()  # (launches, total ms) of the prefill tiles in the same pass
    path.kv.set_timing(False)
    return wall / steps, bytes_ / steps, alloc_us, launches, kernel_ms


def run_config5(args) -> dict:
    """speculative verify on the paged cache at Qwen3-1.7B shape. 64 sequences with
    contexts U[512, 4096]; each step appends the last accepted token and 4 draft tokens per sequence and
    attends with q_len 5 (causal inside the window: one 5-token run per sequence through the fused
    append + attention kernel), then rolls back to a seeded accepted count U{0..4}: the context grows by
    1 + accepted, and the rejected slots are overwritten by the next step. Bytes count each sequence's
    K/V once per layer."""
    B5, Q = 64, 5
    rng = np.random.default_rng(SEED + 5)
    ctx = rng.integers(512, 4097, B5).astype(np.int64)
    total = args.warmup + 2 * args.steps
    max_ctx = int(ctx.max()) + Q * total + PAGE
    mb = (max_ctx + PAGE - 1) // PAGE
    pages = int(((ctx + Q * total) // PAGE + 2).sum())
    path = PathBench(pool_pages=pages, max_seqs=B5, max_blocks=mb, max_tokens=B5 * Q, split_len=args.split_len, seed=SEED + 5)
    acc_rng = np.random.default_rng(SEED + 55)
    qs = np.arange(B5 + 1, dtype=np.int32) * Q

    def step():
        for s in range(B5):
            path.ensure(s, int(ctx[s]) + Q)
        pos = (ctx[:, None] + np.arange(Q)[None, :]).reshape(-1)
        path.run(range(B5), pos, qs)
        kv_bytes = KV_BYTES_PER_TOKEN * int((ctx + Q).sum())
        ctx[:] += 1 + acc_rng.integers(0, Q, B5)
        return N_LAYERS * (kv_bytes + FUSED_TOKEN_BYTES * B5 * Q)

    step_s, step_bytes, alloc_us, launches, kernel_ms = _timed(path, step, args.steps, args.warmup)
    gbs = step_bytes / step_s / 1e9
    kernel_us = kernel_ms / max(launches, 1) * 1e3
    kernel_gbs = path.timed_bytes / N_LAYERS / (kernel_us * 1e-6) / 1e9
    return {
        "metric": "speculative verify rows/s and % HBM peak (Qwen3-1.7B shape, batch 64, q_len 5)",
        "value": round(B5 * Q / step_s, 1), "unit": "query rows/s", "ms_per_step": round(step_s * 1e3, 4),
        "step_gb": round(step_bytes / 1e9, 4), "step_hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "decode_kernel_avg_us": round(kernel_us, 2),
        "decode_kernel_hbm_frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
        "host_blockmanager_us_per_step": round(alloc_us, 2),
        "config": {"workload": "BASELINE configs[4]: 64 sequences, context U[512,4096], 4 drafts + 1 per sequence "
                               "verified in one fused launch per layer, rollback to accepted U{0..4}, 28 layers",
                   "split_len": args.split_len},
    }


def run_linear(args) -> dict:
    """The layer either side of the path at config 2's shape (32 tokens, Qwen3-1.7B: hidden 2048, q 16 x 128,
    kv 8 x 128): the input RMSNorm, the qkv projection (N 4096, K 2048, f16 out) and the output projection
    (N 2048, K 2048, added into the f32 residual), in the reference's order (cuda_backend.cu:350-362). Each
    of the 28 layers has its own random weights (672 MB in all, more than the 256 MB last-level cache), so W
    streams from HBM as in a real step. The pass is timed as launched one by one; each kernel's time is a
    hipGraph of its 28 launches replayed between two HIP events: a launch's share of back-to-back work on
    the GPU, free of the host's launch rate. Consecutive launches overlap one's start with the other's end,
    so it can read below a rocprof duration."""
    import torch

    from ember_amd import kernels as K

    M, HID, NQKV = BATCH, H * D, (H + 2 * KVH) * D
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(SEED + 7)
    w_qkv = [torch.randn((NQKV, HID), generator=g, device=dev, dtype=torch.float16) * 0.02 for _ in range(N_LAYERS)]
    w_o = [torch.randn((HID, HID), generator=g, device=dev, dtype=torch.float16) * 0.02 for _ in range(N_LAYERS)]
    norm_w = [torch.ones(HID, device=dev) for _ in range(N_LAYERS)]
    h = torch.randn((M, HID), generator=g, device=dev)
    xn = torch.empty((M, HID), device=dev, dtype=torch.float16)
    qkv = torch.empty((M, NQKV), device=dev, dtype=torch.float16)
    att = torch.randn((M, HID), generator=g, device=dev).half()
    # One zeroed workspace for both projections (they never overlap); neither splits K at these shapes (None).
    ws = max((K.gemv_workspace(M, n, HID, dev) for n in (NQKV, HID)),
             key=lambda t: 0 if t is None else t.numel(), default=None)
    p_qkv = [K.gemv_pack(w) for w in w_qkv]  # W as a backend keeps it: the GEMV's packed layout
    p_o = [K.gemv_pack(w) for w in w_o]
    torch.cuda.synchronize()
    names = ["rmsnorm_rows", "gemv qkv (store_f16)", "gemv o (add_f32)"]

    def ops(l):
        return [lambda: K.rmsnorm_rows(h, norm_w[l], xn, 1e-6),
                lambda: K.gemv(xn, w_qkv[l], qkv, 0, workspace=ws, packed=p_qkv[l]),
                lambda: K.gemv(att, w_o[l], h, 2, workspace=ws, packed=p_o[l])]

    def layer(l):
        for op in ops(l):
            op()

    for _ in range(args.warmup):
        for l in range(N_LAYERS):
            layer(l)
    torch.cuda.synchronize()
    with collector_paused():
        t0 = time.perf_counter()
        for _ in range(args.steps):
            for l in range(N_LAYERS):
                layer(l)
        torch.cuda.synchronize()
        step_s = (time.perf_counter() - t0) / args.steps
    tot = []
    for i in range(len(names)):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for l in range(N_LAYERS):
                ops(l)[i]()
        graph.replay()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with collector_paused():
            start.record()
            for _ in range(args.steps):
                graph.replay()
            stop.record()
            torch.cuda.synchronize()
        tot.append(start.elapsed_time(stop))
        del graph
    us = [t / (args.steps * N_LAYERS) * 1e3 for t in tot]
    bytes_ = [M * HID * 4 + HID * 4 + M * HID * 2,
              NQKV * HID * 2 + M * HID * 2 + M * NQKV * 2,
              HID * HID * 2 + M * HID * 2 + 2 * M * HID * 4]
    kern = {n: {"avg_us": round(u, 2), "bytes": b_, "gbs": round(b_ / u / 1e3, 1),
                "hbm_frac": round(b_ / u / 1e3 / HBM_PEAK_GBS, 4)} for n, u, b_ in zip(names, us, bytes_)}
    gemv_bytes = bytes_[1] + bytes_[2]
    gemv_gbs = gemv_bytes / (us[1] + us[2]) / 1e3
    log(f"[bench] linear layers: {step_s * 1e3:.3f} ms per 28-layer pass; " +
        "; ".join(f"{n} {k['avg_us']} us = {k['gbs']} GB/s" for n, k in kern.items()))
    return {
        "metric": "decode-size linear layers either side of the path: GB/s and % HBM peak (Qwen3-1.7B shape, "
                  "32 tokens)",
        "value": round(gemv_gbs, 1), "unit": "GB/s", "ms_per_step": round(step_s * 1e3, 4),
        "step_hbm_frac": round(gemv_gbs / HBM_PEAK_GBS, 4), "kernels": kern,
        "config": {"workload": "28 layers of rmsnorm_rows (32 x 2048) + qkv GEMV (4096 x 2048, f16 out) + "
                               "o GEMV (2048 x 2048, added into the f32 residual), own random weights per layer"},
    }


def run_backend(args) -> dict:
    """Whole-model decode through HipBackend (ember::Backend, device "hip"): a synthetic Qwen3-0.6B-shaped model
    (28 layers, hidden 1024, 16 q / 8 kv heads, MLP 3072, tied 151,936-token vocabulary, N(0, 0.02) weights in the
    safetensors layout the backend loads), 8 sequences with 128-token prompts, then greedy decode steps (forward +
    sample). Each step is timed with the whole step replayed as one hipGraph (BackendOptions.cuda_graphs, the
    reference's default) and, on a second backend over the same files, launched eagerly (~200 launches).
    Bytes per step: every weight once plus the K/V of every context token."""
    import tempfile

    from ember_amd import _lib
    from ember_amd.backend import BackendOptions, SampleRequest, SamplingParams, create_backend
    from ember_amd.paged_kv import StepBatch

    sys.path.insert(0, str(ROOT / "tests"))
    from synthetic_model import write_model

    B, PROMPT, LAYERS, VOCAB, HID, INTER, QD, KVD = 8, 128, 28, 151936, 1024, 3072, 2048, 1024
    weight_bytes = 2 * (LAYERS * ((QD + 2 * KVD) * HID + HID * QD + 2 * INTER * HID + HID * INTER) + VOCAB * HID)
    kv_token_bytes = LAYERS * 2 * KVD * 2  # K and V of one token, every layer, f16
    n_steps = args.warmup + args.steps
    width = (PROMPT + n_steps + PAGE) // PAGE + 1
    greedy = [SampleRequest(SamplingParams(temperature=0.0))] * B
    rng = np.random.default_rng(SEED + 11)
    prompts = rng.integers(3, VOCAB, (B, PROMPT)).tolist()

    def batch(new_tokens, lens, rows):
        toks, pos, qs, ctx, tab = [], [], [0], [], []
        for i, (t, n) in enumerate(zip(new_tokens, lens)):
            toks += t
            pos += list(range(n, n + len(t)))
            qs.append(qs[-1] + len(t))
            ctx.append(n + len(t))
            tab += [i * width + p for p in range(width)]
        return StepBatch(tokens=toks, positions=pos, query_start=qs, context_len=ctx, block_tables=tab,
                         max_blocks=width, logit_rows=list(rows))

    results = {}
    with tempfile.TemporaryDirectory() as td:
        log(f"[bench] writing a synthetic {LAYERS}-layer Qwen3-0.6B-shaped model ({weight_bytes / 1e9:.2f} GB f16)")
        write_model(Path(td), layers=LAYERS, vocab=VOCAB)
        captures = _lib.lib().ember_backend_graph_captures
        timed_captures = 0
        for graphs in (True, False):
            be = create_backend(td, BackendOptions(max_batch_tokens=B * PROMPT, max_seqs=B, kv_cache_tokens=B * width * PAGE,
                                                   cuda_graphs=graphs))
            be.forward(batch(prompts, [0] * B, [PROMPT * (i + 1) - 1 for i in range(B)]))
            nxt, lens = be.sample(greedy), [PROMPT] * B
            ctx_sum = 0
            with collector_paused():
                for step in range(n_steps):
                    if step == args.warmup:
                        t0, ctx_sum, c0 = time.perf_counter(), 0, captures()
                    be.forward(batch([[t] for t in nxt], lens, range(B)))
                    nxt = be.sample(greedy)  # waits for the step's logits
                    lens = [n + 1 for n in lens]
                    ctx_sum += sum(lens)
                wall = time.perf_counter() - t0
            if graphs:
                timed_captures = captures() - c0
            be.close()
            results[graphs] = (wall / args.steps, ctx_sum / args.steps)
            log(f"[bench] backend decode, graphs {'on' if graphs else 'off'}: {wall / args.steps * 1e3:.3f} ms/step")
    step_s, ctx = results[True]
    step_bytes = weight_bytes + kv_token_bytes * ctx
    return {
        "metric": "whole-model greedy decode tokens/s through HipBackend (Qwen3-0.6B shape, batch 8)",
        "value": round(B / step_s, 1), "unit": "tokens/s", "ms_per_step": round(step_s * 1e3, 4),
        "step_gb": round(step_bytes / 1e9, 4), "step_hbm_frac": round(step_bytes / step_s / 1e9 / HBM_PEAK_GBS, 4),
        "eager_ms_per_step": round(results[False][0] * 1e3, 4),
        "graph_captures_timed": timed_captures,
        "config": {"workload": "synthetic Qwen3-0.6B-shaped model (28 layers, tied 151,936 vocabulary), 8 sequences, "
                               "128-token prompts, greedy decode steps (forward + sample) as one replayed graph each; "
                               "eager_ms_per_step: the same steps launched one by one"},
    }


def run_block(args) -> dict:
    """Config 2's decode step with the whole attention block per layer (input RMSNorm, qkv GEMV, the fused
    append + paged attention, o GEMV into the f32 residual), 28 layers: the attention half of a Qwen3-1.7B
    layer on MI355X. Bytes: the decode path's (K/V of every context token, the new tokens' traffic) plus every
    layer's qkv and o weights once."""
    torch = __import__("torch")
    w = Workload(args.warmup + 2 * args.steps, args.split_len, block=True)
    for _ in range(args.warmup):
        w.step()
    w.stream.synchronize()
    sum_ctx = 0
    with collector_paused():
        t0 = time.perf_counter()
        for _ in range(args.steps):
            sum_ctx += w.step()
        w.stream.synchronize()
        torch.cuda.synchronize()
        step_s = (time.perf_counter() - t0) / args.steps
    kv_bytes = N_LAYERS * (KV_BYTES_PER_TOKEN * sum_ctx / args.steps + TOKEN_BYTES * BATCH)
    step_bytes = kv_bytes + w.block_weight_bytes
    gbs = step_bytes / step_s / 1e9
    log(f"[bench] attention block: {step_s * 1e3:.3f} ms/step, {BATCH / step_s:.0f} tokens/s, "
        f"{gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of peak)")
    return {
        "metric": "attention-block decode tokens/s and % HBM peak (Qwen3-1.7B shape, batch 32: input RMSNorm + "
                  "qkv GEMV + paged append/attention + o GEMV, 28 layers)",
        "value": round(BATCH / step_s, 1), "unit": "tokens/s", "ms_per_step": round(step_s * 1e3, 4),
        "step_gb": round(step_bytes / 1e9, 4), "step_hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "config": {"workload": "BASELINE configs[1] (batch 32, context U[256,4096], 8192-page pool) with the "
                               "attention block's RMSNorm and projections, own random weights per layer",
                   "split_len": args.split_len},
    }


def run_config3(args) -> dict:
    """a continuous-batching mixed step at Qwen3-1.7B shape. 64 sequences share one
    1024-token system prefix held in 64 sealed, refcounted pages (prefix cache: match_prefix). 4 of them
    prefill their own 2048-token prompts in 512-token chunks (MFMA tiles), staggered so one finishes and a
    new one is admitted every step; 60 decode one token each, with own context U[128, 2048] after the
    prefix. Two decode sequences are a fork sharing every page, the partial last one included, so their
    first step copies that page on write. Bytes count each sequence's context once per layer."""
    NSEQ, NPRE, PREFIX, CHUNK, NCHUNK = 64, 4, 1024, 512, 4
    rng = np.random.default_rng(SEED + 3)
    total = args.warmup + 2 * args.steps
    own = rng.integers(128, 2049, NSEQ - NPRE)
    max_ctx = PREFIX + max(CHUNK * NCHUNK, int(own.max()) + total) + PAGE
    mb = (max_ctx + PAGE - 1) // PAGE
    pages = PREFIX // PAGE + int((own + total).sum()) // PAGE + 2 * NSEQ + (NPRE + 2) * CHUNK * NCHUNK // PAGE + 64
    path = PathBench(pool_pages=pages, max_seqs=NSEQ, max_blocks=mb, max_tokens=NPRE * CHUNK + NSEQ, split_len=args.split_len,
                prefix_caching=True, seed=SEED + 3)
    bm = path.bm
    prefix = rng.integers(0, 150000, PREFIX).astype(np.int32)
    # The prefix, computed once (its K/V are already in the pools) and sealed into the prefix cache.
    path.ensure(0, PREFIX)
    parent = 0
    for i, b in enumerate(path.blocks[0]):
        parent = bm.seal(b, parent, prefix[i * PAGE:(i + 1) * PAGE])
    prefix_blocks = list(path.blocks[0])
    path.release(0)  # sealed and unreferenced: held by the prefix cache until a sequence matches it

    def admit(s, n_own):  # a sequence starting with the prefix: the cache hands out the shared pages
        got = bm.match_prefix(np.concatenate([prefix, np.zeros(1, np.int32)]))
        assert got == prefix_blocks, "the prefix cache missed"
        path.blocks[s] = list(got)
        path.tables[s, :len(got)] = got
        path.ensure(s, PREFIX + n_own)

    ctx = np.zeros(NSEQ, np.int64)
    for s in range(NPRE, NSEQ - 1):
        admit(s, int(own[s - NPRE]))
        ctx[s] = PREFIX + int(own[s - NPRE])
    # the fork: sequence NSEQ-1 shares every page of sequence NSEQ-2, partial last page included
    src = NSEQ - 2
    bm.share(path.blocks[src])
    path.blocks[NSEQ - 1] = list(path.blocks[src])
    path.tables[NSEQ - 1, :len(path.blocks[src])] = path.blocks[src]
    ctx[NSEQ - 1] = ctx[src]
    assert ctx[src] % PAGE, "the fork's last page must be partial"
    shared_last = path.blocks[src][-1]
    assert bm.refcount(shared_last) == 2 and bm.refcount(prefix_blocks[0]) == NSEQ - NPRE
    chunk_of = list(range(NPRE))  # staggered prompts: sequence i starts at chunk i
    for s in range(NPRE):
        admit(s, CHUNK * NCHUNK)
    cow = {"copies": 0}
    prefill_flops = []  # per step, per layer

    def step():
        # copy-on-write before any write into a shared page
        for s in range(NPRE, NSEQ):
            last = path.blocks[s][-1] if ctx[s] % PAGE else None
            if last is not None and bm.refcount(last) > 1:
                nb = bm.copy_on_write(last)
                if nb < 0:
                    raise RuntimeError("no block for copy-on-write")
                if nb != last:
                    path.kv.copy_blocks([last], [nb])
                    path.blocks[s][-1] = nb
                    path.tables[s, len(path.blocks[s]) - 1] = nb
                    cow["copies"] += 1
        pos, qs = [], [0]
        kv_tokens = 0
        flops = 0  # prefill tiles, per layer: QK and PV, 2 flops per multiply-add, over keys 0..pos of every head
        for s in range(NPRE):
            c0 = PREFIX + CHUNK * chunk_of[s]
            pos.append(np.arange(c0, c0 + CHUNK))
            qs.append(qs[-1] + CHUNK)
            kv_tokens += c0 + CHUNK
            flops += 4 * D * H * (CHUNK * c0 + CHUNK * (CHUNK + 1) // 2)
        prefill_flops.append(flops)
        for s in range(NPRE, NSEQ):
            path.ensure(s, int(ctx[s]) + 1)
            pos.append(np.array([ctx[s]]))
            qs.append(qs[-1] + 1)
            kv_tokens += int(ctx[s]) + 1
        path.run(range(NSEQ), np.concatenate(pos), qs)
        ctx[NPRE:] += 1
        for s in range(NPRE):  # the next chunk; a finished prompt makes room for a new one
            chunk_of[s] += 1
            if chunk_of[s] == NCHUNK:
                path.release(s)
                admit(s, CHUNK * NCHUNK)
                chunk_of[s] = 0
        return N_LAYERS * (KV_BYTES_PER_TOKEN * kv_tokens + TOKEN_BYTES * (NPRE * CHUNK + NSEQ - NPRE))

    step_s, step_bytes, alloc_us, launches, kernel_ms = _timed(path, step, args.steps, args.warmup)
    assert cow["copies"] == 1, f"expected one copy-on-write, saw {cow['copies']}"
    assert bm.refcount(prefix_blocks[0]) == NSEQ and bm.check() == "", bm.check()
    gbs = step_bytes / step_s / 1e9
    T = NPRE * CHUNK + NSEQ - NPRE
    p_launches, p_ms = path.prefill_timed
    p_us = p_ms / max(p_launches, 1) * 1e3
    p_tflops = float(np.mean(prefill_flops[-args.steps:])) / (p_us * 1e-6) / 1e12 if p_launches else None
    return {
        "metric": "continuous-batching mixed step tokens/s and % HBM peak (Qwen3-1.7B shape, 4 x 512 prefill + 60 decode)",
        "value": round(T / step_s, 1), "unit": "tokens/s", "ms_per_step": round(step_s * 1e3, 4),
        "step_gb": round(step_bytes / 1e9, 4), "step_hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "decode_kernel_avg_us": round(kernel_ms / max(launches, 1) * 1e3, 2),
        "prefill_kernel_avg_us": round(p_us, 2),
        "prefill_mfma": None if p_tflops is None else {
            "achieved": round(p_tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(p_tflops / MFMA_F16_PEAK_TFLOPS, 4)},
        "host_blockmanager_us_per_step": round(alloc_us, 2), "cow_copies": cow["copies"],
        "prefix_refcount": bm.refcount(prefix_blocks[0]),
        "config": {"workload": "BASELINE configs[2]: 64 sequences sharing a 1024-token prefix (64 sealed pages), "
                               "4 x 512-token prefill chunks (MFMA tiles) + 60 decodes (own context U[128,2048]), "
                               "one forked pair copying its shared partial page on write, 28 layers",
                   "split_len": args.split_len},
    }


def run_config4(args) -> dict:
    """large-pool decode sized for 288 GB of HBM. A 2,097,152-token pool (131,072
    pages, 112 KiB of f16 K/V per token over 28 layers: 224 GiB) and 256 sequences with contexts
    log-uniform in [512, 16384]. Each step decodes one token for every running sequence, preempts the
    newest 8 (their pages go back to the pool) and resumes the 8 preempted the step before, as the
    reference's engine does (engine.cpp:195-205, :302-335): their pages are allocated again and their whole
    contexts re-prefilled in the same step through the plan, which routes each resumed context (>= 16 new
    tokens) to the MFMA prefill tiles (cuda_backend.cu:174-179) while the running sequences decode. GB/s counts
    the decode's K/V once per sequence plus the re-prefill's K/V once per resumed sequence and every new
    token's bytes."""
    import torch

    POOL, NSEQ, PRE = 131072, 256, 8
    free = torch.cuda.mem_get_info()[0]
    need = 2 * N_LAYERS * (POOL + 1) * KVH * PAGE * D * 2
    if need > free * 0.95:
        raise RuntimeError(f"config 4 needs {need / 2**30:.0f} GiB of pool, {free / 2**30:.0f} GiB free")
    rng = np.random.default_rng(SEED + 4)
    ctx = np.exp(rng.uniform(np.log(512), np.log(16384), NSEQ)).astype(np.int64)
    total = args.warmup + 2 * args.steps
    mb = (int(ctx.max()) + total + 2 * PAGE) // PAGE
    resume_rows = PRE * (int(ctx.max()) + total)
    path = PathBench(pool_pages=POOL, max_seqs=NSEQ, max_blocks=mb, max_tokens=NSEQ + resume_rows,
                     split_len=args.split_len, seed=SEED + 4, shared_qkv=True)
    for s in range(NSEQ):
        path.ensure(s, int(ctx[s]))
    order = list(range(NSEQ))  # admission order: the newest are preempted
    paused = []
    prefill_flops, resumed_tokens = [], []

    def step():
        nonlocal paused
        running = [s for s in order if s not in paused]
        for s in paused:  # resume: fresh pages for the whole context, recomputed below
            path.ensure(s, int(ctx[s]))
        for s in running:
            path.ensure(s, int(ctx[s]) + 1)
        seqs = running + paused
        pos = [np.array([ctx[s]]) for s in running] + [np.arange(0, ctx[s]) for s in paused]
        qs = np.concatenate([[0], np.cumsum([p.size for p in pos])])
        path.run(seqs, np.concatenate(pos), qs)
        # per layer: QK and PV over keys 0..pos of every head, 2 flops per multiply-add
        prefill_flops.append(sum(4 * D * H * int(ctx[s]) * (int(ctx[s]) + 1) // 2 for s in paused))
        resumed_tokens.append(int(sum(int(ctx[s]) for s in paused)))
        kv_bytes = KV_BYTES_PER_TOKEN * (int((ctx[running] + 1).sum()) + resumed_tokens[-1])
        new_tokens = len(running) + resumed_tokens[-1]
        ctx[running] += 1
        # the resumed rejoin at the back; the newest 8 running are preempted and their pages freed
        newest = running[-PRE:]
        for s in newest:
            path.release(s)
        order[:] = [s for s in order if s not in newest] + newest
        paused = newest
        return N_LAYERS * (kv_bytes + TOKEN_BYTES * new_tokens)

    step_s, step_bytes, alloc_us, launches, kernel_ms = _timed(path, step, args.steps, args.warmup)
    gbs = step_bytes / step_s / 1e9
    p_launches, p_ms = path.prefill_timed
    p_us = p_ms / max(p_launches, 1) * 1e3
    p_tflops = float(np.mean(prefill_flops[-args.steps:])) / (p_us * 1e-6) / 1e12 if p_launches else None
    d_us = kernel_ms / max(launches, 1) * 1e3
    return {
        "metric": "large-pool decode tokens/s, % HBM peak and page-allocator overhead (2M-token pool, 256 sequences)",
        "value": round((NSEQ - PRE) / step_s, 1), "unit": "decode tokens/s", "ms_per_step": round(step_s * 1e3, 4),
        "step_gb": round(step_bytes / 1e9, 4), "step_hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "decode_kernel_avg_us": round(d_us, 2),
        "prefill_kernel_avg_us": round(p_us, 2),
        "resumed_tokens_per_step": round(float(np.mean(resumed_tokens[-args.steps:])), 1),
        "prefill_share_of_step": round(N_LAYERS * p_us * 1e-6 / step_s, 4),
        "decode_share_of_step": round(N_LAYERS * d_us * 1e-6 / step_s, 4),
        "prefill_mfma": None if p_tflops is None else {
            "achieved": round(p_tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(p_tflops / MFMA_F16_PEAK_TFLOPS, 4)},
        "host_blockmanager_us_per_step": round(alloc_us, 2),
        "config": {"workload": "BASELINE configs[3]: 2,097,152-token f16 pool (224 GiB over 28 layers), 256 sequences "
                               "with context logU[512,16384], each step preempting the newest 8 and re-prefilling the "
                               "8 preempted the step before (whole contexts through the plan: MFMA prefill tiles) "
                               "beside the running 248's decode", "split_len": args.split_len},
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample length (0 = skip)")
    ap.add_argument("--split-len", type=int, default=512, help="keys per decode split (a multiple of 16)")
    ap.add_argument("--graph", action="store_true",
                    help="run each step as a replayed hipGraph of all layers (the timing pass stays eager)")
    ap.add_argument("--config", type=int, default=2, choices=[2, 3, 4, 5],
                    help="BASELINE config: 2 = the metric (default); 3, 4, 5 print their own line")
    ap.add_argument("--block", action="store_true",
                    help="config 2 with the whole attention block per layer (RMSNorm, qkv/o GEMVs); its own line")
    ap.add_argument("--linear", action="store_true",
                    help="time the layer either side of the path (input RMSNorm, qkv and o GEMVs); its own line")
    ap.add_argument("--backend", action="store_true",
                    help="whole-model decode through HipBackend on a synthetic Qwen3-0.6B-shaped model; its own line")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only the known-size page copy used to scale the HBM byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (this path has no multi-GPU "
              "part to measure; see DESIGN.md for how it would shard)", file=sys.stderr)
        return 2
    if args.copy_calibration:
        return copy_calibration(args.steps)
    if args.config != 2 or args.linear or args.block or args.backend:
        import torch

        from ember_amd import lib

        lib()
        assert torch.cuda.is_available(), "bench.py needs a GPU"
        log("[bench] linear layers" if args.linear else "[bench] attention block" if args.block
            else "[bench] whole-model decode" if args.backend else f"[bench] BASELINE config {args.config}")
        fn = (run_linear if args.linear else run_block if args.block else run_backend if args.backend
              else {3: run_config3, 4: run_config4, 5: run_config5}[args.config])
        line = fn(args)
        line.update({"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
                     "vs_baseline": None, "dtype": "f16", "data": "synthetic, seeded"})
        log(f"[bench] {line['ms_per_step']:.3f} ms/step, {line['value']:.0f} {line['unit']}, "
            f"{line['step_hbm_frac']:.1%} of peak HBM")
        print(json.dumps(line), flush=True)
        return 0

    import torch

    from ember_amd import lib

    lib()  # fails loudly when the HIP library is not built
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    log(f"[bench] setting up config 2 ({N_LAYERS} layers, batch {BATCH}, {POOL_PAGES}-page pool)")
    # Two passes over the same growing batch: the first is timed bare (the metric: nothing but the path
    # runs), the second with start/stop events around every decode launch (the kernel's average duration
    # for the roofline; the events add host-visible gaps between launches, so that pass is not the metric).
    w = Workload(args.warmup + 2 * args.steps, args.split_len, args.graph)
    for _ in range(args.warmup):
        w.step()
    w.stream.synchronize()
    w.alloc_s = 0.0
    sum_ctx = 0
    captures0 = w.kv.graph_captures()
    torch.cuda.synchronize()
    with collector_paused():
        t0 = time.perf_counter()
        for _ in range(args.steps):
            sum_ctx += w.step()
        w.stream.synchronize()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    # graphs captured inside the timed window (a new bucket layout); 0 means every timed step relaunched a kept graph
    timed_captures = w.kv.graph_captures() - captures0
    alloc_us = w.alloc_s / args.steps * 1e6

    w.graph = False  # events cannot sit inside a graph: the timing pass launches layer by layer
    w.kv.set_timing(True)
    w.kv.timing()  # start from zero
    sum_ctx_inst = 0
    with collector_paused():
        t1 = time.perf_counter()
        for _ in range(args.steps):
            sum_ctx_inst += w.step()
        w.stream.synchronize()
        wall_inst = time.perf_counter() - t1
    launches, kernel_ms = w.kv.timing()
    w.kv.set_timing(False)

    ms_per_step = wall * 1e3 / args.steps
    tokens_s = BATCH * args.steps / wall
    # Decode kernel roofline: algorithmic bytes per launch = K+V of every context token, plus per new token
    # either the query (4 KiB, unfused) or, fused, qkv in (8 KiB) + its K/V written (4 KiB) + the output (4 KiB).
    fused = w.kv.fused()
    per_token = FUSED_TOKEN_BYTES if fused else 4096
    token_bytes = FUSED_TOKEN_BYTES if fused else TOKEN_BYTES
    step_bytes = N_LAYERS * (KV_BYTES_PER_TOKEN * sum_ctx / args.steps + token_bytes * BATCH)
    step_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    kernel_bytes = (KV_BYTES_PER_TOKEN * sum_ctx_inst + per_token * BATCH * args.steps) * N_LAYERS
    kernel_gbs = kernel_bytes / (kernel_ms * 1e-3) / 1e9 if kernel_ms > 0 else 0.0
    avg_us = kernel_ms / max(launches, 1) * 1e3
    log(f"[bench] {args.steps} steps in {wall:.3f} s: {ms_per_step:.3f} ms/step, {tokens_s:.0f} tokens/s, "
        f"step {step_gbs:.0f} GB/s ({step_gbs / HBM_PEAK_GBS:.1%} of peak)")
    log(f"[bench] instrumented pass {wall_inst * 1e3 / args.steps:.3f} ms/step; paged_decode_kernel: {launches} "
        f"launches, avg {avg_us:.1f} us, {kernel_gbs:.0f} GB/s ({kernel_gbs / HBM_PEAK_GBS:.1%}); "
        f"host BlockManager {alloc_us:.1f} us/step")
    traffic, traffic_ratio = measured_traffic()

    cpu = None
    if args.cpu_seconds > 0:
        log("[bench] timing the CPU baseline (oracle, f32 KV)")
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu['value']:.1f} tokens/s on {cpu['cores']} threads")

    line = {
        "metric": METRIC,
        "value": round(tokens_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: N(0,1) q/k/v activations and random f16 K/V pages, seeded",
        "config": {
            "workload": "BASELINE configs[1]: batched paged decode, Qwen3-1.7B KV shape, 28 layers, "
                        "16 q / 8 kv heads, d=128, 32 sequences, context U[256,4096], 1 new token each per step, "
                        "f16 KV in 16-token pages scattered over an 8192-page pool",
            "global_batch": BATCH,
            "layers": N_LAYERS,
            "accumulate": "f32",
            "step_gb": round(step_bytes / 1e9, 4),
            "step_hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
            "split_len": args.split_len,
            "graph": args.graph,
            "graph_captures": {"total": w.kv.graph_captures(), "timed": timed_captures} if args.graph else None,
            "host_blockmanager_us_per_step": round(alloc_us, 2),
        },
        "roofline": {
            "kernel": "paged_decode_kernel<f16, rows 2, fused append + merge>" if fused else "paged_decode_kernel",
            "bound": "hbm",
            "achieved": round(kernel_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_ratio": traffic_ratio,
            "traffic_source": f"profiles/{TRAFFIC_FILE.name} (rocprofv3 FETCH_SIZE / WRITE_SIZE passes, copy-kernel "
                              "calibrated; committed, not measured in this run)" if traffic else None,
            "avg_launch_us": round(avg_us, 2),
            "timed_launches": launches,
            "bytes_per_launch": round(kernel_bytes / max(launches, 1)),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
