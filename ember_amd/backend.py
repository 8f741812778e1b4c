"""Python handle on ember::Backend with device "hip" (src/backend/backend.hpp:94-125), through the C ABI.

``create_backend(model_dir, options)`` opens a Hugging Face model directory (config.json, generation_config.json,
model.safetensors) on the GPU; the methods keep the reference's names and meaning: ``forward(batch)`` appends the
batch's K/V and keeps the logits of ``batch.logit_rows`` on the device, ``sample``, ``token_probs``, ``logits``,
``set_capture_hidden`` / ``captured_hidden``. Errors the reference throws raise EmberError.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import EmberError, check, last_error
from .paged_kv import StepBatch

_I32P, _F32P = ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_float)


@dataclass
class SamplingParams:
    """ember::SamplingParams (backend.hpp:28-34)."""

    temperature: float = 1.0  # 0 = greedy
    top_p: float = 1.0
    top_k: int = 0
    min_p: float = 0.0
    seed: int = 0


@dataclass
class SampleRequest:
    """ember::SampleRequest (backend.hpp:78-81)."""

    params: SamplingParams = field(default_factory=SamplingParams)
    counter: int = 0


@dataclass
class BackendOptions:
    """The ember::BackendOptions fields the HIP backend reads (backend.hpp:35-48)."""

    max_batch_tokens: int = 2048
    max_seqs: int = 64
    max_logit_rows: int = 0
    kv_cache_bytes: int = 0
    kv_cache_tokens: int = 0
    memory_fraction: float = 0.0
    gpu: int = 0
    cuda_graphs: bool = True  # pure decode steps replay one graph of the whole step (backend.hpp:46)


def _params(reqs) -> ctypes.Array:
    arr = (_lib.SampleParams * max(1, len(reqs)))()
    for i, r in enumerate(reqs):
        p = r.params
        arr[i].temperature, arr[i].top_p, arr[i].min_p, arr[i].top_k = p.temperature, p.top_p, p.min_p, p.top_k
        arr[i].seed, arr[i].counter = p.seed & 0xFFFFFFFFFFFFFFFF, r.counter & 0xFFFFFFFFFFFFFFFF
    return arr


class Backend:
    def __init__(self, model_dir: str, options: BackendOptions | None = None):
        o = options or BackendOptions()
        c = _lib.BackendOptions()
        c.max_batch_tokens, c.max_seqs, c.max_logit_rows = o.max_batch_tokens, o.max_seqs, o.max_logit_rows
        c.kv_cache_bytes, c.kv_cache_tokens, c.memory_fraction, c.gpu = (o.kv_cache_bytes, o.kv_cache_tokens,
                                                                        o.memory_fraction, o.gpu)
        c.graphs = 1 if o.cuda_graphs else -1
        # The destructor is bound here: at interpreter exit the module's globals may be gone before this object.
        self._destroy = _lib.lib().ember_backend_destroy
        self._h = _lib.lib().ember_backend_create(str(model_dir).encode(), c)
        if not self._h:
            raise EmberError(last_error())
        info = _lib.ModelInfo()
        check(_lib.lib().ember_backend_info(self._h, info), "backend_info")
        self.info = info

    def close(self) -> None:
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._destroy(h)

    def __del__(self):
        self.close()

    def name(self) -> str:
        return "hip"

    def num_kv_blocks(self) -> int:
        return int(self.info.num_kv_blocks)

    @property
    def vocab_size(self) -> int:
        return int(self.info.vocab_size)

    def forward(self, b: StepBatch) -> None:
        from .paged_kv import PagedKv

        sb, keep = PagedKv._batch(b)
        rows = np.ascontiguousarray(np.asarray(b.logit_rows, np.int32).reshape(-1))
        check(_lib.lib().ember_backend_forward(self._h, sb, rows.ctypes.data_as(_I32P), rows.size), "backend_forward")
        del keep

    def sample(self, requests) -> list[int]:
        out = np.zeros(max(1, len(requests)), np.int32)
        check(_lib.lib().ember_backend_sample(self._h, _params(requests), len(requests), out.ctypes.data_as(_I32P)),
              "backend_sample")
        return out[:len(requests)].tolist()

    def token_probs(self, requests, rows, tokens) -> np.ndarray:
        r = np.ascontiguousarray(np.asarray(rows, np.int32))
        t = np.ascontiguousarray(np.asarray(tokens, np.int32))
        out = np.zeros(max(1, r.size), np.float32)
        check(_lib.lib().ember_backend_token_probs(self._h, _params(requests), len(requests), r.ctypes.data_as(_I32P),
                                                   t.ctypes.data_as(_I32P), r.size, out.ctypes.data_as(_F32P)),
              "backend_token_probs")
        return out[:r.size]

    def logits(self, row: int) -> np.ndarray:
        out = np.zeros(self.vocab_size, np.float32)
        check(_lib.lib().ember_backend_logits(self._h, row, out.ctypes.data_as(_F32P), out.size), "backend_logits")
        return out

    def set_capture_hidden(self, on: bool) -> None:
        check(_lib.lib().ember_backend_set_capture_hidden(self._h, 1 if on else 0), "backend_set_capture_hidden")

    def captured_hidden(self) -> np.ndarray:
        out = np.zeros((self.info.n_layers + 1) * self.info.hidden, np.float32)
        n = _lib.lib().ember_backend_captured_hidden(self._h, out.ctypes.data_as(_F32P), out.size)
        if n < 0:
            check(n, "backend_captured_hidden")
        return out[:n]


def create_backend(model_dir: str, options: BackendOptions | None = None) -> Backend:
    """ember::create_backend with device "hip" (backend.hpp:125)."""
    return Backend(model_dir, options)
