"""Python handle on the CPU oracle (oracle/oracle.cpp) - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
package, and only as the checker. The product (ember_amd/) never does.
Every function restates a piece of the reference's CPU path; see oracle.h for
the reference lines each follows and what pins it. ref_lib() loads the pieces of
the reference itself that compile here (oracle/_ref, built by `make ref` where
the reference tree is present), against which tests check the restatements.
"""
from __future__ import annotations

import ctypes
import subprocess
from ctypes import (POINTER, c_char_p, c_double, c_float, c_int32, c_int64, c_uint8, c_uint16, c_uint32, c_uint64,
                    c_void_p)
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
PAGE = 16

_F32P, _I32P, _U16P = POINTER(c_float), POINTER(c_int32), POINTER(c_uint16)

_PROTOS = {
    "ember_oracle_f16_to_f32": (c_float, [c_uint16]),
    "ember_oracle_f32_to_f16": (c_uint16, [c_float]),
    "ember_oracle_f16_to_f32_n": (None, [_U16P, _F32P, c_int64]),
    "ember_oracle_f32_to_f16_n": (None, [_F32P, _U16P, c_int64]),
    "ember_oracle_inv_freq": (None, [c_double, c_int32, _F32P]),
    "ember_oracle_rmsnorm": (None, [_F32P, _F32P, c_int32, c_float, _F32P]),
    "ember_oracle_rope": (None, [_F32P, c_int32, c_int32, _F32P]),
    "ember_oracle_linear": (None, [_U16P, _U16P, c_int32, c_int32, c_int32, c_int32, _F32P, c_int32]),
    "ember_oracle_linear_mt": (None, [_U16P, _U16P, c_int32, c_int32, c_int32, c_int32, _F32P, c_int32, c_int32]),
    "ember_oracle_rng_mix": (c_uint64, [c_uint64]),
    "ember_oracle_gumbel": (c_float, [c_uint64, c_uint64, ctypes.c_uint32]),
    "ember_oracle_sampling_distribution": (c_int32, [_F32P, c_int32, c_float, c_float, c_int32, c_float, _I32P, _F32P]),
    "ember_oracle_sample": (c_int32, [_F32P, c_int32, c_float, c_float, c_int32, c_float, c_uint64, c_uint64]),
    "ember_oracle_dot": (c_float, [_F32P, _F32P, c_int32]),
    "ember_oracle_cache_offset": (c_int64, [_I32P, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32]),
    "ember_oracle_append_layer": (c_int32, [_F32P, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p,
                                            c_float, _F32P, _I32P, _I32P, c_int32, _I32P, c_int32, _F32P, c_void_p,
                                            c_void_p, c_int32, c_int32]),
    "ember_oracle_attention_layer": (c_int32, [_F32P, c_int32, c_int32, c_int32, c_int32, _I32P, _I32P, c_int32, _I32P,
                                               c_int32, c_void_p, c_void_p, c_int32, c_int32, c_int32, _F32P, c_int32]),
    "ember_oracle_bm_create": (c_void_p, [c_int32, c_int32]),
    "ember_oracle_bm_destroy": (None, [c_void_p]),
    "ember_oracle_bm_num_blocks": (c_int32, [c_void_p]),
    "ember_oracle_bm_available": (c_int32, [c_void_p]),
    "ember_oracle_bm_cached": (c_int32, [c_void_p]),
    "ember_oracle_bm_allocate": (c_int32, [c_void_p]),
    "ember_oracle_bm_release": (c_int32, [c_void_p, c_int32]),
    "ember_oracle_bm_release_all": (c_int32, [c_void_p, _I32P, c_int32]),
    "ember_oracle_bm_block_hash": (c_uint64, [c_uint64, _I32P, c_int32]),
    "ember_oracle_fnv1a_words": (c_uint64, [c_uint64, _I32P, c_int32]),
    "ember_oracle_fmix64": (c_uint64, [c_uint64]),
    "ember_oracle_bm_match_prefix": (c_int32, [c_void_p, _I32P, c_int32, _I32P]),
    "ember_oracle_bm_seal": (c_uint64, [c_void_p, c_int32, c_uint64, _I32P, c_int32]),
    "ember_oracle_bm_refcount": (c_int32, [c_void_p, c_int32]),
    "ember_oracle_bm_hit_tokens": (c_uint64, [c_void_p]),
    "ember_oracle_bm_lookup_tokens": (c_uint64, [c_void_p]),
    "ember_oracle_bm_check": (c_int32, [c_void_p, c_char_p, c_int32]),
    "ember_oracle_bm_states": (None, [c_void_p, POINTER(c_uint8)]),
    "ember_oracle_bm_share": (c_int32, [c_void_p, _I32P, c_int32]),
    "ember_oracle_bm_copy_on_write": (c_int32, [c_void_p, c_int32]),
}

_lib = None


REF_TREE = Path("/root/reference/src")
REF_LIB_PATH = HERE / "_ref" / "libember_ref.so"
_REF_PROTOS = {
    "ember_ref_rng_mix": (c_uint64, [c_uint64]),
    "ember_ref_gumbel_noise": (c_float, [c_uint64, c_uint64, c_uint32]),
    "ember_ref_sample_uniform": (c_double, [c_uint64, c_uint64]),
    "ember_ref_sampling_distribution": (c_int32, [_F32P, c_int32, c_float, c_float, c_int32, c_float, _I32P, _F32P]),
    "ember_ref_sample_host": (c_int32, [_F32P, c_int32, c_float, c_float, c_int32, c_float, c_uint64, c_uint64]),
    "ember_ref_dot_avx2": (c_float, [_F32P, _F32P, c_int32]),
}
_ref_lib = None


def build() -> Path:
    """Compiles oracle/liboracle.so with the committed Makefile, and oracle/_ref from the reference's own sources
    when the reference tree is present (not on a GPU box, which uses what was built)."""
    subprocess.run(["make", "-B", "-s", "-C", str(HERE)], check=True)
    if REF_TREE.is_dir():
        subprocess.run(["make", "-B", "-s", "-C", str(HERE), "ref"], check=True)
    return LIB_PATH


def ref_lib():
    """The reference's host sampler and AVX2 dot product as built into oracle/_ref, or None when not built."""
    global _ref_lib
    if _ref_lib is None and REF_LIB_PATH.exists():
        h = ctypes.CDLL(str(REF_LIB_PATH))
        for name, (res, args) in _REF_PROTOS.items():
            fn = getattr(h, name)
            fn.restype, fn.argtypes = res, args
        _ref_lib = h
    return _ref_lib


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        h = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _PROTOS.items():
            fn = getattr(h, name)
            fn.restype, fn.argtypes = res, args
        _lib = h
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


# ---- scalar pieces ----

def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(np.asarray(h, dtype=np.uint16))
    out = np.empty(h.shape, np.float32)
    lib().ember_oracle_f16_to_f32_n(_p(h, _U16P), _p(out, _F32P), h.size)
    return out


def f32_to_f16(f) -> np.ndarray:
    f = _f32(f)
    out = np.empty(f.shape, np.uint16)
    lib().ember_oracle_f32_to_f16_n(_p(f, _F32P), _p(out, _U16P), f.size)
    return out


def inv_freq(theta: float, head_dim: int) -> np.ndarray:
    out = np.empty(head_dim // 2, np.float32)
    lib().ember_oracle_inv_freq(theta, head_dim, _p(out, _F32P))
    return out


def rmsnorm(x, w, eps: float) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    out = np.empty_like(x)
    lib().ember_oracle_rmsnorm(_p(x, _F32P), _p(w, _F32P), x.size, eps, _p(out, _F32P))
    return out


def linear(a_f16, w_f16, epilogue: int, c=None, threads: int = 1) -> np.ndarray:
    """C = A . W^T (f16 bits in, double sums, f32 out) with an epilogue; c is the f32 C that add_f32 adds to.
    threads > 1 spreads the outputs over threads with bit-identical results."""
    a = np.ascontiguousarray(np.asarray(a_f16, np.float16)).view(np.uint16)
    w = np.ascontiguousarray(np.asarray(w_f16, np.float16)).view(np.uint16)
    M, K = a.shape
    N = w.shape[0]
    cols = N // 2 if epilogue == 3 else N
    out = np.zeros((M, cols), np.float32) if c is None else np.array(c, np.float32, copy=True)
    if threads > 1:
        lib().ember_oracle_linear_mt(_p(a, _U16P), _p(w, _U16P), M, N, K, epilogue, _p(out, _F32P), cols, threads)
    else:
        lib().ember_oracle_linear(_p(a, _U16P), _p(w, _U16P), M, N, K, epilogue, _p(out, _F32P), cols)
    return out


# ---- sampling ----

def rng_mix(z: int) -> int:
    return int(lib().ember_oracle_rng_mix(z & 0xFFFFFFFFFFFFFFFF))


def gumbel(seed: int, counter: int, token: int) -> float:
    return float(lib().ember_oracle_gumbel(seed & 0xFFFFFFFFFFFFFFFF, counter & 0xFFFFFFFFFFFFFFFF, token))


def sampling_distribution(logits, temperature=1.0, top_p=1.0, top_k=0, min_p=0.0):
    """(tokens, probabilities) of the kept set, most likely first (sampling_host.cpp:20-66)."""
    x = _f32(logits)
    toks = np.empty(x.size, np.int32)
    probs = np.empty(x.size, np.float32)
    n = lib().ember_oracle_sampling_distribution(_p(x, _F32P), x.size, temperature, top_p, top_k, min_p,
                                                 _p(toks, _I32P), _p(probs, _F32P))
    return toks[:n].copy(), probs[:n].copy()


def sample(logits, temperature=1.0, top_p=1.0, top_k=0, min_p=0.0, seed=0, counter=0) -> int:
    """One draw of the host sampler (sampling_host.cpp:68-85)."""
    x = _f32(logits)
    return int(lib().ember_oracle_sample(_p(x, _F32P), x.size, temperature, top_p, top_k, min_p,
                                         seed & 0xFFFFFFFFFFFFFFFF, counter & 0xFFFFFFFFFFFFFFFF))


def rope(x, pos: int, inv_freq_: np.ndarray) -> np.ndarray:
    x = _f32(x).copy()
    f = _f32(inv_freq_)
    lib().ember_oracle_rope(_p(x, _F32P), x.size, pos, _p(f, _F32P))
    return x


def dot(a, b) -> float:
    a, b = _f32(a), _f32(b)
    return float(lib().ember_oracle_dot(_p(a, _F32P), _p(b, _F32P), a.size))


def cache_offset(block_tables, num_blocks, n_kv, head_dim, seq, layer, kv_head, pos) -> int:
    bt = _i32(block_tables)
    return int(lib().ember_oracle_cache_offset(_p(bt, _I32P), bt.shape[-1], num_blocks, n_kv, head_dim, seq, layer,
                                               kv_head, pos))


# ---- one layer of the path ----

def append_layer(qkv, positions, query_start, block_tables, k_cache, v_cache, *, n_heads, n_kv, inv_freq_, eps=1e-6,
                 q_norm=None, k_norm=None, bias=None, num_blocks, kv_f16: bool, head_dim=128) -> np.ndarray:
    """QK-norm + RoPE + store for one layer (cpu_backend.cpp:146-172). Writes k_cache/v_cache
    (f32 arrays, or uint16 f16 bits when kv_f16) in place; returns q [T, n_heads, D] f32."""
    qkv = _f32(qkv)
    T = qkv.shape[0]
    pos, qs, bt = _i32(positions), _i32(query_start), _i32(block_tables)
    q_out = np.empty((T, n_heads, head_dim), np.float32)
    want = np.uint16 if kv_f16 else np.float32
    assert k_cache.dtype == want and v_cache.dtype == want and k_cache.flags.c_contiguous and v_cache.flags.c_contiguous
    opt = lambda a: None if a is None else _f32(a)  # noqa: E731
    qn, kn, bs = opt(q_norm), opt(k_norm), opt(bias)
    f = _f32(inv_freq_)
    rc = lib().ember_oracle_append_layer(
        _p(qkv, _F32P), T, n_heads, n_kv, head_dim, None if qn is None else qn.ctypes.data,
        None if kn is None else kn.ctypes.data, None if bs is None else bs.ctypes.data, eps, _p(f, _F32P),
        _p(pos, _I32P), _p(qs, _I32P), qs.size - 1, _p(bt, _I32P), bt.shape[-1], _p(q_out, _F32P),
        k_cache.ctypes.data, v_cache.ctypes.data, num_blocks, 1 if kv_f16 else 0)
    if rc != 0:
        raise ValueError("oracle append: a slot falls outside the pool")
    return q_out


def attention_layer(q, positions, query_start, block_tables, k_cache, v_cache, *, n_heads, n_kv, num_blocks,
                    kv_f16: bool, q_f16: bool = False, threads: int = 1, head_dim=128) -> np.ndarray:
    """Causal paged attention of every token (cpu_backend.cpp:173-198); out [T, n_heads, D] f32."""
    q = _f32(q)
    T = q.shape[0]
    pos, qs, bt = _i32(positions), _i32(query_start), _i32(block_tables)
    out = np.empty((T, n_heads, head_dim), np.float32)
    rc = lib().ember_oracle_attention_layer(
        _p(q, _F32P), T, n_heads, n_kv, head_dim, _p(pos, _I32P), _p(qs, _I32P), qs.size - 1, _p(bt, _I32P),
        bt.shape[-1], k_cache.ctypes.data, v_cache.ctypes.data, num_blocks, 1 if kv_f16 else 0, 1 if q_f16 else 0,
        _p(out, _F32P), threads)
    if rc != 0:
        raise ValueError("oracle attention: malformed step")
    return out


# ---- block manager ----

class BlockManager:
    """The oracle restatement of block_manager.cpp:9-139, same method names as the reference."""

    def __init__(self, num_blocks: int, prefix_caching: bool):
        self._h = lib().ember_oracle_bm_create(num_blocks, 1 if prefix_caching else 0)
        if not self._h:
            raise ValueError("the KV cache has no blocks")

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            lib().ember_oracle_bm_destroy(h)

    def num_blocks(self):
        return lib().ember_oracle_bm_num_blocks(self._h)

    def available(self):
        return lib().ember_oracle_bm_available(self._h)

    def used(self):
        return self.num_blocks() - self.available()

    def cached(self):
        return lib().ember_oracle_bm_cached(self._h)

    def allocate(self):
        return lib().ember_oracle_bm_allocate(self._h)

    def release(self, b):
        if lib().ember_oracle_bm_release(self._h, b) != 0:
            raise ValueError(f"releasing free block {b}")

    def release_all(self, blocks):
        a = _i32(list(blocks))
        if lib().ember_oracle_bm_release_all(self._h, _p(a, _I32P), a.size) != 0:
            raise ValueError("releasing a free block")

    @staticmethod
    def block_hash(parent, tokens):
        a = _i32(list(tokens))
        return int(lib().ember_oracle_bm_block_hash(parent, _p(a, _I32P), a.size))

    def match_prefix(self, tokens):
        a = _i32(list(tokens))
        out = np.empty(max(1, a.size // PAGE), np.int32)
        n = lib().ember_oracle_bm_match_prefix(self._h, _p(a, _I32P), a.size, _p(out, _I32P))
        return out[:n].tolist()

    def seal(self, block, parent, tokens):
        a = _i32(list(tokens))
        h = int(lib().ember_oracle_bm_seal(self._h, block, parent, _p(a, _I32P), a.size))
        if h == 0:
            raise ValueError("sealing a block that is not full")
        return h

    def refcount(self, b):
        return lib().ember_oracle_bm_refcount(self._h, b)

    def hit_tokens(self):
        return int(lib().ember_oracle_bm_hit_tokens(self._h))

    def lookup_tokens(self):
        return int(lib().ember_oracle_bm_lookup_tokens(self._h))

    def check(self):
        buf = ctypes.create_string_buffer(512)
        lib().ember_oracle_bm_check(self._h, buf, len(buf))
        return buf.value.decode()

    def states(self):
        out = np.empty(self.num_blocks(), np.uint8)
        lib().ember_oracle_bm_states(self._h, out.ctypes.data_as(POINTER(c_uint8)))
        return out.tolist()

    def share(self, blocks):
        a = _i32(list(blocks))
        if lib().ember_oracle_bm_share(self._h, _p(a, _I32P), a.size) != 0:
            raise ValueError("sharing a block that is not held")

    def copy_on_write(self, b):
        return lib().ember_oracle_bm_copy_on_write(self._h, b)


def fnv1a_words(parent: int, tokens) -> int:
    a = _i32(list(tokens))
    return int(lib().ember_oracle_fnv1a_words(parent, _p(a, _I32P), a.size))


def fmix64(h: int) -> int:
    return int(lib().ember_oracle_fmix64(h))
