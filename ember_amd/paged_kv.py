"""Python handle on the C++ paged-KV path (ember::HipPagedKv through the C ABI).

Mirrors what the reference's CudaBackend does around attention each step
(src/backend/cuda/cuda_backend.cu:134-205 forward, :345-368 the layer loop):
``plan(batch)`` once per step, then ``layer(l, qkv, ...)`` per layer.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from ._lib import EmberError, KvConfig, StepBatchC, check, last_error


@dataclass
class StepBatch:
    """The reference's ember::StepBatch (src/backend/backend.hpp:56-76)."""

    tokens: list = field(default_factory=list)
    positions: list = field(default_factory=list)
    query_start: list = field(default_factory=lambda: [0])
    context_len: list = field(default_factory=list)
    block_tables: list = field(default_factory=list)
    max_blocks: int = 0
    logit_rows: list = field(default_factory=list)

    def num_tokens(self) -> int:
        return len(self.tokens)

    def num_seqs(self) -> int:
        return len(self.context_len)


def _arr(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.int32).reshape(-1))


class PagedKv:
    def __init__(self, *, n_layers, n_heads, n_kv_heads, head_dim=128, rms_eps=1e-6, rope_theta=1e6,
                 max_position, num_blocks, max_batch_tokens=2048, max_seqs=64, dtype=torch.float16, qk_norm=True,
                 split_len=512, stream=None):
        self.stream = stream if stream is not None else torch.cuda.current_stream()
        c = KvConfig()
        c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim = n_layers, n_heads, n_kv_heads, head_dim
        c.rms_eps, c.rope_theta, c.max_position, c.num_blocks = rms_eps, rope_theta, max_position, num_blocks
        c.max_batch_tokens, c.max_seqs = max_batch_tokens, max_seqs
        c.dtype = _lib.DTYPE_F16 if dtype == torch.float16 else _lib.DTYPE_F32
        c.qk_norm, c.split_len = 1 if qk_norm else 0, split_len
        self.cfg = c
        self.dtype = dtype
        # The destructor is bound here: at interpreter exit the module's globals may be gone before this object.
        self._destroy = _lib.lib().ember_kv_destroy
        self._h = _lib.lib().ember_kv_create(c, self.stream.cuda_stream)
        if not self._h:
            raise EmberError(last_error())
        self.n_layers, self.n_heads, self.n_kv, self.head_dim = n_layers, n_heads, n_kv_heads, head_dim
        self.num_blocks = num_blocks

    def close(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._destroy(h)

    def __del__(self):
        self.close()

    @staticmethod
    def _batch(b: StepBatch):
        arrs = [_arr(b.tokens), _arr(b.positions), _arr(b.query_start), _arr(b.context_len), _arr(b.block_tables)]
        sb = StepBatchC()
        sb.tokens, sb.positions, sb.query_start, sb.context_len, sb.block_tables = (a.ctypes.data for a in arrs)
        sb.num_tokens, sb.num_seqs, sb.max_blocks = len(b.tokens), len(b.context_len), b.max_blocks
        return sb, arrs

    def plan(self, b: StepBatch) -> None:
        sb, _keep = self._batch(b)
        check(_lib.lib().ember_kv_plan(self._h, sb), "kv_plan")

    def decode_graph(self, b: StepBatch, layers) -> bool:
        """A pure decode step of <= 64 tokens, planned and run for every layer as one replayed hipGraph.
        layers: per layer (qkv, out, q_norm, k_norm, bias) device tensors (or None for the optional ones),
        qkv and out holding token_bucket(T) rows; they must stay the same between steps to reuse a graph.
        Returns False (nothing enqueued) when the step does not qualify."""
        sb, _keep = self._batch(b)
        io = (_lib.LayerIo * len(layers))()
        ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        for i, (qkv, out, qn, kn, bias) in enumerate(layers):
            io[i].qkv, io[i].out, io[i].q_norm, io[i].k_norm, io[i].bias = ptr(qkv), ptr(out), ptr(qn), ptr(kn), ptr(bias)
        code = _lib.lib().ember_kv_decode_graph(self._h, sb, io, len(layers))
        if code == 1:
            return False
        check(code, "kv_decode_graph")
        return True

    def graph_captures(self) -> int:
        """Graphs decode_graph has captured on this path so far (a launch of a kept graph does not count)."""
        return int(_lib.lib().ember_kv_graph_captures(self._h))

    def layer(self, layer: int, qkv: torch.Tensor, out: torch.Tensor, q_norm=None, k_norm=None, bias=None) -> None:
        for t in (qkv, out):
            if not t.is_cuda or not t.is_contiguous() or t.dtype != self.dtype:
                raise EmberError("qkv / out must be contiguous device tensors of the pool dtype")
        ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        check(_lib.lib().ember_kv_layer(self._h, layer, qkv.data_ptr(), ptr(q_norm), ptr(k_norm), ptr(bias),
                                        out.data_ptr()), "kv_layer")

    def attention_block(self, layer: int, h: torch.Tensor, in_norm: torch.Tensor, w_qkv: torch.Tensor,
                        w_o: torch.Tensor, *, xn: torch.Tensor, qkv: torch.Tensor, att: torch.Tensor, q_norm=None,
                        k_norm=None, bias=None) -> None:
        """One layer's attention block in the reference's order (cuda_backend.cu:350-362), for a planned step of
        at most 64 tokens and f16 pools: xn = rmsnorm(h) * in_norm (f16), qkv = xn . w_qkv^T (f16), the append +
        attention of `layer` into att, then h += att . w_o^T (the f32 residual).
        h: f32 [T, hidden]; in_norm: f32 [hidden]; w_qkv: f16 [(n_heads + 2 n_kv) head_dim, hidden];
        w_o: f16 [hidden, n_heads head_dim]; xn, qkv, att: f16 scratch of [T, hidden], [T, w_qkv rows] and
        [T, n_heads, head_dim]."""
        from . import _lib as L
        from . import kernels as K

        if self.dtype != torch.float16:
            raise EmberError("attention_block: f16 pools only (the GEMV takes f16 activations)")
        T = h.shape[0]
        if T > 64:
            raise EmberError("attention_block: at most 64 tokens (decode-sized GEMV)")
        # One workspace, sized for 64 tokens, serves both projections: they run one after the other on the stream.
        need = max(int(L.lib().ember_hip_gemv_workspace_bytes(64, w.shape[0], w.shape[1])) for w in (w_qkv, w_o))
        if need > 0 and (getattr(self, "_gemv_ws", None) is None or self._gemv_ws.numel() < need):
            self._gemv_ws = torch.zeros(need, dtype=torch.uint8, device=h.device)
        ws = getattr(self, "_gemv_ws", None) if need > 0 else None
        K.rmsnorm_rows(h, in_norm, xn, self.cfg.rms_eps, stream=self.stream)
        K.gemv(xn, w_qkv, qkv, L.EPILOGUE_STORE_F16, stream=self.stream, workspace=ws)
        self.layer(layer, qkv, att, q_norm, k_norm, bias)
        K.gemv(att.view(T, -1), w_o, h, L.EPILOGUE_ADD_F32, stream=self.stream, workspace=ws)

    def copy_blocks(self, src, dst) -> None:
        s, d = _arr(src), _arr(dst)
        p = ctypes.POINTER(ctypes.c_int32)
        check(_lib.lib().ember_kv_copy_blocks(self._h, s.ctypes.data_as(p), d.ctypes.data_as(p), s.size), "kv_copy_blocks")

    def pool_view(self, layer: int, which: str = "k") -> torch.Tensor:
        """A torch view of one layer's K or V pool, [num_blocks + 1, n_kv, 16, head_dim] (last block = spare)."""
        fn = _lib.lib().ember_kv_k_pool if which == "k" else _lib.lib().ember_kv_v_pool
        addr = fn(self._h, layer)
        if not addr:
            raise EmberError(last_error())
        n = (self.num_blocks + 1) * self.n_kv * 16 * self.head_dim
        return _wrap_device(addr, n, self.dtype).view(self.num_blocks + 1, self.n_kv, 16, self.head_dim)

    def layer_stride(self) -> int:
        return int(_lib.lib().ember_kv_layer_stride(self._h))

    def spare_block(self) -> int:
        return int(_lib.lib().ember_kv_spare_block(self._h))

    def set_timing(self, on: bool) -> None:
        _lib.lib().ember_kv_set_timing(self._h, 1 if on else 0)

    def timing(self) -> tuple[int, float]:
        """(launches, total ms) of the paged-decode kernel since the last call, from HIP events."""
        n, ms = ctypes.c_int32(), ctypes.c_double()
        check(_lib.lib().ember_kv_timing(self._h, ctypes.byref(n), ctypes.byref(ms)), "kv_timing")
        return n.value, ms.value

    def prefill_timing(self) -> tuple[int, float]:
        """(launches, total ms) of the prefill-tile kernel since the last call, from HIP events."""
        n, ms = ctypes.c_int32(), ctypes.c_double()
        check(_lib.lib().ember_kv_prefill_timing(self._h, ctypes.byref(n), ctypes.byref(ms)), "kv_prefill_timing")
        return n.value, ms.value

    def plan_info(self) -> tuple[int, int, int, bool]:
        """(decode runs, prefill tiles, splits, fused) of the current plan."""
        r, t, s, f = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        _lib.lib().ember_kv_plan_info(self._h, ctypes.byref(r), ctypes.byref(t), ctypes.byref(s), ctypes.byref(f))
        return r.value, t.value, s.value, bool(f.value)

    def fused(self) -> bool:
        """Whether the current plan appends and attends in one launch per layer."""
        return self.plan_info()[3]


def _wrap_device(addr: int, numel: int, dtype: torch.dtype) -> torch.Tensor:
    """A non-owning torch tensor over device memory the C++ side owns (DLPack-free, via __cuda_array_interface__)."""
    typestr = {torch.float16: "<f2", torch.float32: "<f4"}[dtype]

    class _Holder:
        __cuda_array_interface__ = {"shape": (numel,), "typestr": typestr, "data": (addr, False), "version": 2,
                                    "strides": None}

    return torch.as_tensor(_Holder(), device="cuda")
