"""Launchers of the gfx950 kernels through the C ABI, for torch tensors.

Mirrors the reference's launcher seam (src/backend/cuda/kernels.cuh:74-120):
``qk_norm_rope_store`` (-> ember_hip_kv_append), ``paged_attention``
(-> ember_hip_paged_decode), ``prefill_attention`` (-> ember_hip_prefill_attn),
plus ``copy_pages`` (copy-on-write). Device tensors carry activations and pools;
the step's integer arrays are given as host arrays, checked here (every index a
kernel will follow is in range), then uploaded. Launches go to the current torch
stream unless ``stream`` is given.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._lib import BLOCK_SIZE, MAX_RUN, PREFILL_TILE, AttnArgs, CopyArgs, EmberError, PrefillArgs, QkvArgs, check

HEAD_DIM = 128


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float16:
        return _lib.DTYPE_F16
    if t.dtype == torch.float32:
        return _lib.DTYPE_F32
    raise EmberError(f"unsupported dtype {t.dtype}")


def _stream_handle(stream) -> int:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def _dev(t: torch.Tensor, name: str) -> int:
    if not t.is_cuda or not t.is_contiguous():
        raise EmberError(f"{name} must be a contiguous device tensor")
    return t.data_ptr()


def _opt(t: torch.Tensor | None, name: str) -> int | None:
    return None if t is None else _dev(t, name)


def _ints(a, device) -> torch.Tensor:
    return torch.as_tensor(np.ascontiguousarray(np.asarray(a, dtype=np.int32)), device=device)


@dataclass
class StepInts:
    """A step's integers on the host (the StepBatch fields the kernels read) and their device copies.

    positions [T], token_seq [T], block_tables [S, max_blocks].
    """

    positions: np.ndarray
    token_seq: np.ndarray
    block_tables: np.ndarray
    num_blocks: int  # blocks in each layer's pool (every table entry a kernel reads must be below it)

    def __post_init__(self):
        self.positions = np.ascontiguousarray(np.asarray(self.positions, dtype=np.int32).reshape(-1))
        self.token_seq = np.ascontiguousarray(np.asarray(self.token_seq, dtype=np.int32).reshape(-1))
        bt = np.asarray(self.block_tables, dtype=np.int32)
        self.block_tables = np.ascontiguousarray(bt.reshape(bt.shape[0], -1))
        T, S, W = self.positions.size, self.block_tables.shape[0], self.block_tables.shape[1]
        if self.token_seq.size != T:
            raise EmberError("positions and token_seq differ in length")
        if T and (self.token_seq.min() < 0 or self.token_seq.max() >= S):
            raise EmberError("token_seq names a sequence without a block table")
        if T and (self.positions.min() < 0 or self.positions.max() >= W * BLOCK_SIZE):
            raise EmberError("a position lies beyond its block table")
        for t in range(T):  # every page up to each token's position must be a pool block
            pages = self.block_tables[self.token_seq[t], : self.positions[t] // BLOCK_SIZE + 1]
            if pages.size and (pages.min() < 0 or pages.max() >= self.num_blocks):
                raise EmberError(f"token {t} reads a block outside the pool of {self.num_blocks}")
        self._dev = None

    @property
    def T(self) -> int:
        return int(self.positions.size)

    @property
    def max_blocks(self) -> int:
        return int(self.block_tables.shape[1])

    def device(self, device="cuda"):
        if self._dev is None:
            self._dev = (_ints(self.positions, device), _ints(self.token_seq, device), _ints(self.block_tables, device))
        return self._dev


def inv_freq(theta: float, head_dim: int = HEAD_DIM) -> np.ndarray:
    """Rotary frequencies in f32, as the reference computes them (cpu_backend.cpp:85-88)."""
    i = np.arange(head_dim // 2, dtype=np.float32)
    return (np.float32(1.0) / np.power(np.float32(theta), (2 * i) / np.float32(head_dim), dtype=np.float32)).astype(np.float32)


def qk_norm_rope_store(qkv, q_out, k_pool, v_pool, ints: StepInts, *, n_heads, n_kv, inv_freq_dev, q_norm=None,
                       k_norm=None, bias=None, eps=1e-6, stream=None):
    """QK-RMSNorm + RoPE + K/V page write for one layer (≙ cuda::qk_norm_rope_store)."""
    T = ints.T
    width = (n_heads + 2 * n_kv) * HEAD_DIM
    if qkv.numel() != T * width or q_out.numel() != T * n_heads * HEAD_DIM:
        raise EmberError("qkv / q_out sizes do not match the step")
    if k_pool.numel() < ints.num_blocks * n_kv * BLOCK_SIZE * HEAD_DIM or v_pool.numel() != k_pool.numel():
        raise EmberError("pools are smaller than num_blocks pages")
    pos, seq, tab = ints.device(qkv.device)
    a = QkvArgs()
    a.qkv, a.q_out = _dev(qkv, "qkv"), _dev(q_out, "q_out")
    a.k_cache, a.v_cache = _dev(k_pool, "k_pool"), _dev(v_pool, "v_pool")
    a.q_norm, a.k_norm, a.bias = _opt(q_norm, "q_norm"), _opt(k_norm, "k_norm"), _opt(bias, "bias")
    a.inv_freq = _dev(inv_freq_dev, "inv_freq")
    a.positions, a.token_seq, a.block_tables = pos.data_ptr(), seq.data_ptr(), tab.data_ptr()
    a.max_blocks, a.T, a.n_heads, a.n_kv, a.head_dim = ints.max_blocks, T, n_heads, n_kv, HEAD_DIM
    a.eps, a.num_blocks, a.dtype = eps, ints.num_blocks, _dtype_code(qkv)
    check(_lib.lib().ember_hip_kv_append(a, _stream_handle(stream)), "kv_append")


def decode_runs(ints: StepInts, token_list, max_run: int = MAX_RUN, group: int = 1):
    """Cuts a list of tokens into runs of consecutive tokens of one sequence, at most max_run each and at
    most 16 // group (a decode work-group holds at most 16 query rows: group heads x run tokens), the cap
    the C++ planner applies."""
    max_run = max(1, min(max_run, 16 // group))
    first, count = [], []
    i, tl = 0, list(token_list)
    while i < len(tl):
        j = i + 1
        while (j < len(tl) and j - i < max_run and tl[j] == tl[j - 1] + 1
               and ints.token_seq[tl[j]] == ints.token_seq[tl[i]] and ints.positions[tl[j]] == ints.positions[tl[j - 1]] + 1):
            j += 1
        first.append(i)
        count.append(j - i)
        i = j
    return np.asarray(first, np.int32), np.asarray(count, np.int32)


def work_list(run_ctx, split_len: int) -> np.ndarray:
    """(run, split) items, every full split first, then the partial last splits longest first
    (the order the C++ planner uses)."""
    full, partial = [], []
    for r, ctx in enumerate(int(c) for c in run_ctx):
        full += [(r, s) for s in range(ctx // split_len)]
        if ctx % split_len:
            partial.append((ctx % split_len, r, ctx // split_len))
    partial.sort(key=lambda x: -x[0])  # stable: equal sizes keep run order
    items = full + [(r, s) for _, r, s in partial]
    return np.asarray(items, np.int32).reshape(-1, 2)


def paged_attention(q, k_pool, v_pool, out, ints: StepInts, *, n_heads, n_kv, token_list=None, runs=None,
                    split_len=512, num_splits=None, scratch=None, use_work_list=False, merge_in_kernel=False,
                    work_desc=True, stream=None):
    """Paged decode attention (≙ cuda::paged_attention).

    token_list: tokens to process (None = all). runs: (run_first, run_count) over
    token_list positions, or None for one token per run. num_splits defaults to
    what the longest context needs at split_len keys per split. use_work_list:
    dispatch through a sorted (run, split) list instead of the dense grid.
    merge_in_kernel: merge the splits in the last work-group of each (run, kv
    head) instead of a second launch. work_desc: with the work list, also pass
    the per-item descriptors the C++ plan uploads (EmberAttnArgs::work_desc).
    """
    a, keep = _attn_args(q, k_pool, v_pool, out, ints, n_heads=n_heads, n_kv=n_kv, token_list=token_list, runs=runs,
                         split_len=split_len, num_splits=num_splits, scratch=scratch, use_work_list=use_work_list,
                         merge_in_kernel=merge_in_kernel, work_desc=work_desc)
    if a is None:
        return keep
    check(_lib.lib().ember_hip_paged_decode(a, _stream_handle(stream)), "paged_decode")
    return keep  # the caller keeps the uploads alive until the stream has run


def decode_step(qkv, k_pool, v_pool, out, ints: StepInts, *, n_heads, n_kv, inv_freq_dev, q_norm=None, k_norm=None,
                bias=None, eps=1e-6, runs=None, split_len=512, num_splits=None, use_work_list=False,
                merge_in_kernel=False, work_desc=True, stream=None):
    """Append + attention in one launch (ember_hip_decode_step); every token of the step is listed, each
    sequence's tokens forming one run of consecutive positions."""
    T = ints.T
    width = (n_heads + 2 * n_kv) * HEAD_DIM
    if qkv.numel() != T * width:
        raise EmberError("qkv does not match the step")
    a, keep = _attn_args(None, k_pool, v_pool, out, ints, n_heads=n_heads, n_kv=n_kv, token_list=None, runs=runs,
                         split_len=split_len, num_splits=num_splits, scratch=None, use_work_list=use_work_list,
                         merge_in_kernel=merge_in_kernel, work_desc=work_desc, dtype_of=qkv)
    seqs = ints.token_seq.tolist()
    if runs is None and len(set(seqs)) != len(seqs):
        raise EmberError("a sequence with several tokens needs them as one run")
    if runs is not None:  # one run per sequence, consecutive positions (the kernel relies on both)
        seen = set()
        for f, c in zip(*runs):
            s = int(ints.token_seq[f])
            if s in seen or np.any(np.diff(ints.positions[f:f + c]) != 1):
                raise EmberError("each sequence's tokens must form one run of consecutive positions")
            seen.add(s)
    pos, seq, tab = ints.device(qkv.device)
    qa = QkvArgs()
    qa.qkv, qa.q_out = _dev(qkv, "qkv"), None
    qa.k_cache, qa.v_cache = a.k_cache, a.v_cache
    qa.q_norm, qa.k_norm, qa.bias = _opt(q_norm, "q_norm"), _opt(k_norm, "k_norm"), _opt(bias, "bias")
    qa.inv_freq = _dev(inv_freq_dev, "inv_freq")
    qa.positions, qa.token_seq, qa.block_tables = pos.data_ptr(), seq.data_ptr(), tab.data_ptr()
    qa.max_blocks, qa.T, qa.n_heads, qa.n_kv, qa.head_dim = ints.max_blocks, T, n_heads, n_kv, HEAD_DIM
    qa.eps, qa.num_blocks, qa.dtype = eps, ints.num_blocks, _dtype_code(qkv)
    check(_lib.lib().ember_hip_decode_step(qa, a, _stream_handle(stream)), "decode_step")
    return keep


def _attn_args(q, k_pool, v_pool, out, ints: StepInts, *, n_heads, n_kv, token_list, runs, split_len, num_splits,
               scratch, use_work_list, merge_in_kernel, work_desc=True, dtype_of=None):
    tl = np.arange(ints.T, dtype=np.int32) if token_list is None else np.asarray(token_list, np.int32)
    n = int(tl.size)
    if n == 0:
        return None, []
    if tl.min() < 0 or tl.max() >= ints.T:
        raise EmberError("token_list names a token outside the step")
    if (q is not None and q.numel() < ints.T * n_heads * HEAD_DIM) or out.numel() < ints.T * n_heads * HEAD_DIM:
        raise EmberError("q / out are smaller than the step")
    if k_pool.numel() < ints.num_blocks * n_kv * BLOCK_SIZE * HEAD_DIM:
        raise EmberError("pools are smaller than num_blocks pages")
    ctx = int(ints.positions[tl].max()) + 1
    if num_splits is None:
        num_splits = max(1, math.ceil(ctx / split_len))
    if num_splits * split_len < ctx:
        raise EmberError("num_splits x split_len does not cover the context")
    dev = k_pool.device
    pos, seq, tab = ints.device(dev)
    tl_dev = _ints(tl, dev)
    a = AttnArgs()
    a.token_index = tl_dev.data_ptr()
    a.q = None if q is None else _dev(q, "q")
    a.k_cache, a.v_cache = _dev(k_pool, "k_pool"), _dev(v_pool, "v_pool")
    a.positions, a.token_seq, a.block_tables = pos.data_ptr(), seq.data_ptr(), tab.data_ptr()
    a.max_blocks, a.T, a.n_heads, a.n_kv, a.head_dim = ints.max_blocks, n, n_heads, n_kv, HEAD_DIM
    a.scale = 1.0 / math.sqrt(HEAD_DIM)
    a.out = _dev(out, "out")
    a.num_splits, a.split_len = num_splits, split_len
    keep = [tl_dev]
    if num_splits > 1:
        need = n * n_heads * num_splits
        if scratch is None:
            scratch = (torch.empty(need * HEAD_DIM, dtype=torch.float32, device=dev),
                       torch.empty(need * 2, dtype=torch.float32, device=dev))
        if scratch[0].numel() < need * HEAD_DIM or scratch[1].numel() < need * 2:
            raise EmberError("split scratch too small")
        a.part_acc, a.part_ml = _dev(scratch[0], "part_acc"), _dev(scratch[1], "part_ml")
        keep.append(scratch)
    a.num_blocks, a.dtype = ints.num_blocks, _dtype_code(q if q is not None else dtype_of)
    if runs is not None:
        rf, rc = (np.asarray(x, np.int32) for x in runs)
        if rf.size != rc.size or rc.min() < 1 or rc.max() > MAX_RUN or rf.min() < 0 or (rf + rc).max() > n:
            raise EmberError("malformed runs")
        for f, c in zip(rf, rc):  # one sequence per run
            if len(set(ints.token_seq[tl[f:f + c]].tolist())) != 1:
                raise EmberError("a run spans two sequences")
        rf_dev, rc_dev = _ints(rf, dev), _ints(rc, dev)
        keep += [rf_dev, rc_dev]
        a.run_first, a.run_count, a.num_runs, a.max_run = rf_dev.data_ptr(), rc_dev.data_ptr(), int(rf.size), int(rc.max())
        run_ctx = [int(ints.positions[tl[f:f + c]].max()) + 1 for f, c in zip(rf, rc)]
    else:
        rf, rc = np.arange(n, dtype=np.int32), np.ones(n, np.int32)
        run_ctx = [int(ints.positions[t]) + 1 for t in tl]
    if use_work_list:
        items = work_list(run_ctx, split_len)
        if items.size and items[:, 1].max() >= num_splits:
            raise EmberError("num_splits is too small for the work list")
        w_dev = _ints(items.reshape(-1), dev)
        keep.append(w_dev)
        a.work, a.num_work = w_dev.data_ptr(), int(items.shape[0])
        if work_desc:
            desc = np.full((items.shape[0], 16), -1, np.int32)
            for i, (r, sp) in enumerate(items.tolist()):
                toks = tl[rf[r]:rf[r] + rc[r]]
                pos = ints.positions[toks]
                seq = int(ints.token_seq[toks[0]])
                counting = (np.diff(toks) == 1).all() and (np.diff(pos) == 1).all()
                desc[i, :8] = (r, sp, rf[r], rc[r], seq, pos.min(), pos.max(), toks[0] if counting else -1)
                p0 = sp * split_len // BLOCK_SIZE
                last = min(int(pos.max()) + 1, (sp + 1) * split_len) - 1
                for j in range(8):
                    if p0 + j <= last // BLOCK_SIZE:
                        desc[i, 8 + j] = ints.block_tables[seq, p0 + j]
            d_dev = _ints(desc.reshape(-1), dev)
            keep.append(d_dev)
            a.work_desc = d_dev.data_ptr()
    if merge_in_kernel:
        counters = torch.zeros(len(run_ctx) * n_kv, dtype=torch.int32, device=dev)
        keep.append(counters)
        a.merge_counters = counters.data_ptr()
    return a, keep


def prefill_attention(q, k_pool, v_pool, out, ints: StepInts, *, n_heads, n_kv, tiles, stream=None,
                      heads_per_group=0):
    """Causal prefill attention of query tiles on MFMA (≙ cuda::prefill_attention).

    tiles: (start, end, seq) triples, each up to PREFILL_TILE consecutive tokens start..end-1 of
    sequence seq; every token attends to its sequence's keys 0..its position, which must already be in
    the pools. f16 only. heads_per_group: 0 (the launcher's choice), 1 or 2 (even G): the same bits.
    """
    if not tiles:
        return []
    t = np.asarray(tiles, np.int32).reshape(-1, 3)
    if (t[:, 1] <= t[:, 0]).any() or (t[:, 1] - t[:, 0] > PREFILL_TILE).any() or t[:, 0].min() < 0 \
            or t[:, 1].max() > ints.T:
        raise EmberError("malformed tiles")
    for s0, e0, sq in t.tolist():
        if (ints.token_seq[s0:e0] != sq).any():
            raise EmberError("a tile spans tokens of another sequence")
    if q.numel() < ints.T * n_heads * HEAD_DIM or out.numel() < ints.T * n_heads * HEAD_DIM:
        raise EmberError("q / out are smaller than the step")
    if k_pool.numel() < ints.num_blocks * n_kv * BLOCK_SIZE * HEAD_DIM:
        raise EmberError("pools are smaller than num_blocks pages")
    dev = k_pool.device
    pos, seq, tab = ints.device(dev)
    ts, te, tq = (_ints(np.ascontiguousarray(t[:, i]), dev) for i in range(3))
    a = PrefillArgs()
    a.q, a.k_cache, a.v_cache = _dev(q, "q"), _dev(k_pool, "k_pool"), _dev(v_pool, "v_pool")
    a.tile_start, a.tile_end, a.tile_seq = ts.data_ptr(), te.data_ptr(), tq.data_ptr()
    a.positions, a.block_tables = pos.data_ptr(), tab.data_ptr()
    a.num_tiles, a.max_blocks, a.n_heads, a.n_kv, a.head_dim = int(t.shape[0]), ints.max_blocks, n_heads, n_kv, HEAD_DIM
    a.scale = 1.0 / math.sqrt(HEAD_DIM)
    a.out = _dev(out, "out")
    a.num_blocks, a.dtype = ints.num_blocks, _dtype_code(q)
    a.heads_per_group = heads_per_group
    check(_lib.lib().ember_hip_prefill_attn(a, _stream_handle(stream)), "prefill_attn")
    return [ts, te, tq]


def copy_pages(k_pool, v_pool, src, dst, *, n_layers, layer_stride, n_kv, num_blocks, stream=None):
    """Copies whole pages src[i] -> dst[i] over every layer (the device half of copy-on-write)."""
    s, d = np.asarray(src, np.int32), np.asarray(dst, np.int32)
    if s.size != d.size:
        raise EmberError("src / dst differ in length")
    if s.size == 0:
        return
    if min(s.min(), d.min()) < 0 or max(s.max(), d.max()) >= num_blocks:
        raise EmberError("a page pair lies outside the pool")
    if k_pool.numel() < n_layers * layer_stride:
        raise EmberError("pools are smaller than n_layers x layer_stride")
    dev = k_pool.device
    sd, dd = _ints(s, dev), _ints(d, dev)
    a = CopyArgs()
    a.k_cache, a.v_cache = _dev(k_pool, "k_pool"), _dev(v_pool, "v_pool")
    a.src_blocks, a.dst_blocks, a.n = sd.data_ptr(), dd.data_ptr(), int(s.size)
    a.n_layers, a.layer_stride, a.n_kv, a.head_dim = n_layers, layer_stride, n_kv, HEAD_DIM
    a.num_blocks, a.dtype = num_blocks, _dtype_code(k_pool)
    check(_lib.lib().ember_hip_copy_pages(a, _stream_handle(stream)), "copy_pages")
    return (sd, dd)


def gemv_workspace(M: int, N: int, K: int, device="cuda"):
    """A zeroed workspace for gemv at this shape (uint8 tensor), or None when the shape does not split K."""
    n = int(_lib.lib().ember_hip_gemv_workspace_bytes(M, N, K))
    return torch.zeros(n, dtype=torch.uint8, device=device) if n > 0 else None


def gemv_pack(w, stream=None):
    """W (f16 [N, K]) laid out for gemv(..., packed=True): a flat f16 device tensor (N rounded up to 16 rows)."""
    if w.dtype != torch.float16 or w.dim() != 2:
        raise EmberError("gemv_pack: w must be f16 [N, K]")
    N, K = w.shape
    n = int(_lib.lib().ember_hip_gemv_packed_bytes(N, K))
    if n <= 0:
        raise EmberError(f"gemv_pack: K must be a positive multiple of 32 (got {K})")
    out = torch.empty(n // 2, dtype=torch.float16, device=w.device)
    check(_lib.lib().ember_hip_gemv_pack(_dev(w, "w"), N, K, out.data_ptr(), _stream_handle(stream)), "gemv_pack")
    return out


def gemv(a, w, c, epilogue: int, stream=None, workspace=None, packed=None):
    """C = A . W^T for decode-sized batches (≙ cuda::gemm with GemmKernel::gemv_tc, k_gemm.cu:302-425).

    a: f16 [M, K] (M <= 64, K a multiple of 32); w: f16 [N, K]; c: per epilogue, f16 [M, N] (store_f16),
    f32 [M, N] (store_f32; add_f32 adds into it) or f16 [M, N / 2] (silu_mul, W rows interleaving gate and up).
    workspace: None, or a zeroed device tensor of at least gemv_workspace's size, which lets a shape with few
    output features split K over more work-groups (not shared by launches that overlap in time).
    packed: None, or gemv_pack(w): the kernel then reads W from that layout (the same bits); w still gives N, K.
    """
    if a.dtype != torch.float16 or w.dtype != torch.float16 or a.dim() != 2 or w.dim() != 2 or a.shape[1] != w.shape[1]:
        raise EmberError("gemv: a [M, K] and w [N, K] must be f16 with the same K")
    M, K = a.shape
    N = w.shape[0]
    cols = N // 2 if epilogue == _lib.EPILOGUE_SILU_MUL else N
    want = torch.float32 if epilogue in (_lib.EPILOGUE_STORE_F32, _lib.EPILOGUE_ADD_F32) else torch.float16
    if c.dtype != want or tuple(c.shape) != (M, cols):
        raise EmberError(f"gemv: c must be {want} [{M}, {cols}]")
    g = _lib.GemvArgs()
    g.A, g.lda, g.W, g.M, g.N, g.K = _dev(a, "a"), K, _dev(w, "w"), M, N, K
    g.C, g.ldc, g.epilogue = _dev(c, "c"), cols, epilogue
    if workspace is not None:
        g.workspace, g.workspace_bytes = _dev(workspace, "workspace"), workspace.numel() * workspace.element_size()
    if packed is not None:
        g.W, g.w_packed = _dev(packed, "packed w"), 1
    check(_lib.lib().ember_hip_gemv(g, _stream_handle(stream)), "gemv")


def rmsnorm_rows(x, w, out, eps: float, rows=None, stream=None):
    """out[r] = rmsnorm(x[rows[r] if rows else r]) * w as f16 (≙ cuda::rmsnorm_rows, kernels.cuh:70-72)."""
    if x.dtype != torch.float32 or w.dtype != torch.float32 or out.dtype != torch.float16:
        raise EmberError("rmsnorm_rows: x and w f32, out f16")
    hidden = x.shape[-1]
    R = out.shape[0]
    keep = []
    n = _lib.NormArgs()
    n.x, n.w, n.out, n.R, n.hidden, n.eps = _dev(x, "x"), _dev(w, "w"), _dev(out, "out"), R, hidden, eps
    if rows is not None:
        r = _ints(np.asarray(rows, np.int32), x.device)
        keep.append(r)
        n.rows = r.data_ptr()
    check(_lib.lib().ember_hip_rmsnorm_rows(n, _stream_handle(stream)), "rmsnorm_rows")
    return keep
