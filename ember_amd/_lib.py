"""ctypes binding of include/ember_hip.h.

The shared library is built in-tree by ember_amd.build (``__graft_entry__.build()``).
There is no fallback: if the library is missing, loading raises, so nothing can
silently run on another code path.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_double, c_float, c_int32, c_int64, c_uint8, c_uint64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libember_hip.so"

# Constants of include/ember_hip.h.
ABI_VERSION = 7
BLOCK_SIZE = 16
PREFILL_TILE = 64
MAX_RUN = 8
MAX_SPLIT_LEN = 1024
STATIC_MAX_PARTIALS = 49152
STATIC_MAX_COUNTERS = 16384
OK = 0
ERR_INVALID = -1
DTYPE_F16 = 0
DTYPE_F32 = 1
EPILOGUE_STORE_F16 = 0
EPILOGUE_STORE_F32 = 1
EPILOGUE_ADD_F32 = 2
EPILOGUE_SILU_MUL = 3


class EmberError(RuntimeError):
    """A failure reported through the C ABI (the reference's ember::Error)."""


class QkvArgs(ctypes.Structure):
    _fields_ = [
        ("qkv", c_void_p), ("q_out", c_void_p), ("k_cache", c_void_p), ("v_cache", c_void_p),
        ("q_norm", c_void_p), ("k_norm", c_void_p), ("bias", c_void_p), ("inv_freq", c_void_p),
        ("positions", c_void_p), ("token_seq", c_void_p), ("block_tables", c_void_p),
        ("max_blocks", c_int32), ("T", c_int32), ("n_heads", c_int32), ("n_kv", c_int32), ("head_dim", c_int32),
        ("eps", c_float), ("num_blocks", c_int32), ("dtype", c_int32),
    ]


class AttnArgs(ctypes.Structure):
    _fields_ = [
        ("token_index", c_void_p), ("q", c_void_p), ("k_cache", c_void_p), ("v_cache", c_void_p),
        ("positions", c_void_p), ("token_seq", c_void_p), ("block_tables", c_void_p),
        ("max_blocks", c_int32), ("T", c_int32), ("n_heads", c_int32), ("n_kv", c_int32), ("head_dim", c_int32),
        ("scale", c_float), ("out", c_void_p), ("num_splits", c_int32), ("split_len", c_int32),
        ("part_acc", c_void_p), ("part_ml", c_void_p), ("num_blocks", c_int32), ("dtype", c_int32),
        ("run_first", c_void_p), ("run_count", c_void_p), ("num_runs", c_int32), ("max_run", c_int32),
        ("work", c_void_p), ("num_work", c_int32), ("merge_counters", c_void_p), ("work_desc", c_void_p),
    ]


class PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("q", c_void_p), ("k_cache", c_void_p), ("v_cache", c_void_p),
        ("tile_start", c_void_p), ("tile_end", c_void_p), ("tile_seq", c_void_p),
        ("positions", c_void_p), ("block_tables", c_void_p),
        ("num_tiles", c_int32), ("max_blocks", c_int32), ("n_heads", c_int32), ("n_kv", c_int32), ("head_dim", c_int32),
        ("scale", c_float), ("out", c_void_p), ("num_blocks", c_int32), ("dtype", c_int32),
        ("heads_per_group", c_int32),
    ]


class CopyArgs(ctypes.Structure):
    _fields_ = [
        ("k_cache", c_void_p), ("v_cache", c_void_p), ("src_blocks", c_void_p), ("dst_blocks", c_void_p),
        ("n", c_int32), ("n_layers", c_int32), ("layer_stride", c_int64),
        ("n_kv", c_int32), ("head_dim", c_int32), ("num_blocks", c_int32), ("dtype", c_int32),
    ]


class KvConfig(ctypes.Structure):
    _fields_ = [
        ("n_layers", c_int32), ("n_heads", c_int32), ("n_kv_heads", c_int32), ("head_dim", c_int32),
        ("rms_eps", c_float), ("rope_theta", c_double), ("max_position", c_int32), ("num_blocks", c_int32),
        ("max_batch_tokens", c_int32), ("max_seqs", c_int32), ("dtype", c_int32), ("qk_norm", c_int32),
        ("split_len", c_int32),
    ]


class StepBatchC(ctypes.Structure):
    _fields_ = [
        ("tokens", c_void_p), ("positions", c_void_p), ("query_start", c_void_p), ("context_len", c_void_p),
        ("block_tables", c_void_p), ("num_tokens", c_int32), ("num_seqs", c_int32), ("max_blocks", c_int32),
    ]


class LayerIo(ctypes.Structure):
    _fields_ = [("qkv", c_void_p), ("q_norm", c_void_p), ("k_norm", c_void_p), ("bias", c_void_p), ("out", c_void_p)]


class GemvArgs(ctypes.Structure):
    _fields_ = [
        ("A", c_void_p), ("lda", c_int32), ("W", c_void_p), ("M", c_int32), ("N", c_int32), ("K", c_int32),
        ("C", c_void_p), ("ldc", c_int32), ("epilogue", c_int32), ("workspace", c_void_p), ("workspace_bytes", c_int64), ("w_packed", c_int32),
    ]


class NormArgs(ctypes.Structure):
    _fields_ = [
        ("x", c_void_p), ("rows", c_void_p), ("R", c_int32), ("hidden", c_int32), ("w", c_void_p), ("eps", c_float),
        ("out", c_void_p),
    ]


class EmbedArgs(ctypes.Structure):
    _fields_ = [("tokens", c_void_p), ("T", c_int32), ("table", c_void_p), ("vocab", c_int32), ("hidden", c_int32),
                ("out", c_void_p)]


class SampleParams(ctypes.Structure):
    _fields_ = [("temperature", c_float), ("top_p", c_float), ("min_p", c_float), ("top_k", c_int32),
                ("seed", c_uint64), ("counter", c_uint64)]


class SampleArgs(ctypes.Structure):
    _fields_ = [("logits", c_void_p), ("R", c_int32), ("vocab", c_int32), ("params", c_void_p), ("out", c_void_p)]


class ProbArgs(ctypes.Structure):
    _fields_ = [("logits", c_void_p), ("vocab", c_int32), ("params", c_void_p), ("rows", c_void_p),
                ("tokens", c_void_p), ("n", c_int32), ("out", c_void_p), ("R", c_int32)]


class BackendOptions(ctypes.Structure):
    _fields_ = [("max_batch_tokens", c_int32), ("max_seqs", c_int32), ("max_logit_rows", c_int32),
                ("kv_cache_bytes", c_int64), ("kv_cache_tokens", c_int32), ("memory_fraction", c_double),
                ("gpu", c_int32), ("graphs", c_int32)]


class ModelInfo(ctypes.Structure):
    _fields_ = [("vocab_size", c_int32), ("hidden", c_int32), ("intermediate", c_int32), ("n_layers", c_int32),
                ("n_heads", c_int32), ("n_kv_heads", c_int32), ("head_dim", c_int32), ("num_kv_blocks", c_int32),
                ("max_logit_rows", c_int32)]


STRUCTS = [QkvArgs, AttnArgs, PrefillArgs, CopyArgs, KvConfig, StepBatchC, LayerIo, GemvArgs, NormArgs, EmbedArgs,
           SampleParams, SampleArgs, ProbArgs, BackendOptions, ModelInfo]

# name -> (restype, argtypes); every extern "C" symbol of include/ember_hip.h.
PROTOTYPES = {
    "ember_hip_kv_append": (c_int32, [POINTER(QkvArgs), c_void_p]),
    "ember_hip_paged_decode": (c_int32, [POINTER(AttnArgs), c_void_p]),
    "ember_hip_paged_decode_static": (c_int32, [POINTER(AttnArgs), c_void_p]),
    "ember_hip_decode_step": (c_int32, [POINTER(QkvArgs), POINTER(AttnArgs), c_void_p]),
    "ember_hip_prefill_attn": (c_int32, [POINTER(PrefillArgs), c_void_p]),
    "ember_hip_copy_pages": (c_int32, [POINTER(CopyArgs), c_void_p]),
    "ember_hip_gemv": (c_int32, [POINTER(GemvArgs), c_void_p]),
    "ember_hip_gemv_workspace_bytes": (c_int64, [c_int32, c_int32, c_int32]),
    "ember_hip_gemv_packed_bytes": (c_int64, [c_int32, c_int32]),
    "ember_hip_gemv_pack": (c_int32, [c_void_p, c_int32, c_int32, c_void_p, c_void_p]),
    "ember_hip_rmsnorm_rows": (c_int32, [POINTER(NormArgs), c_void_p]),
    "ember_hip_embed": (c_int32, [POINTER(EmbedArgs), c_void_p]),
    "ember_hip_sample": (c_int32, [POINTER(SampleArgs), c_void_p]),
    "ember_hip_token_probs": (c_int32, [POINTER(ProbArgs), c_void_p]),
    "ember_hip_last_error": (c_char_p, []),
    "ember_hip_abi_version": (c_int32, []),
    "ember_hip_sizeof": (c_int32, [c_int32]),
    "ember_bm_create": (c_void_p, [c_int32, c_int32]),
    "ember_bm_destroy": (None, [c_void_p]),
    "ember_bm_num_blocks": (c_int32, [c_void_p]),
    "ember_bm_available": (c_int32, [c_void_p]),
    "ember_bm_used": (c_int32, [c_void_p]),
    "ember_bm_cached": (c_int32, [c_void_p]),
    "ember_bm_allocate": (c_int32, [c_void_p]),
    "ember_bm_release": (c_int32, [c_void_p, c_int32]),
    "ember_bm_release_all": (c_int32, [c_void_p, POINTER(c_int32), c_int32]),
    "ember_bm_block_hash": (c_uint64, [c_uint64, POINTER(c_int32), c_int32]),
    "ember_bm_match_prefix": (c_int32, [c_void_p, POINTER(c_int32), c_int32, POINTER(c_int32)]),
    "ember_bm_seal": (c_uint64, [c_void_p, c_int32, c_uint64, POINTER(c_int32), c_int32]),
    "ember_bm_prefix_caching": (c_int32, [c_void_p]),
    "ember_bm_refcount": (c_int32, [c_void_p, c_int32]),
    "ember_bm_hit_tokens": (c_uint64, [c_void_p]),
    "ember_bm_lookup_tokens": (c_uint64, [c_void_p]),
    "ember_bm_check": (c_int32, [c_void_p, c_char_p, c_int32]),
    "ember_bm_states": (None, [c_void_p, POINTER(c_uint8)]),
    "ember_bm_share": (c_int32, [c_void_p, POINTER(c_int32), c_int32]),
    "ember_bm_copy_on_write": (c_int32, [c_void_p, c_int32]),
    "ember_kv_create": (c_void_p, [POINTER(KvConfig), c_void_p]),
    "ember_kv_destroy": (None, [c_void_p]),
    "ember_kv_plan": (c_int32, [c_void_p, POINTER(StepBatchC)]),
    "ember_kv_layer": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "ember_kv_decode_graph": (c_int32, [c_void_p, POINTER(StepBatchC), POINTER(LayerIo), c_int32]),
    "ember_kv_graph_captures": (c_int64, [c_void_p]),
    "ember_kv_copy_blocks": (c_int32, [c_void_p, POINTER(c_int32), POINTER(c_int32), c_int32]),
    "ember_kv_k_pool": (c_void_p, [c_void_p, c_int32]),
    "ember_kv_v_pool": (c_void_p, [c_void_p, c_int32]),
    "ember_kv_layer_stride": (c_int64, [c_void_p]),
    "ember_kv_spare_block": (c_int32, [c_void_p]),
    "ember_kv_plan_info": (c_int32, [c_void_p, POINTER(c_int32), POINTER(c_int32), POINTER(c_int32), POINTER(c_int32)]),
    "ember_kv_set_timing": (c_int32, [c_void_p, c_int32]),
    "ember_kv_timing": (c_int32, [c_void_p, POINTER(c_int32), POINTER(c_double)]),
    "ember_kv_prefill_timing": (c_int32, [c_void_p, POINTER(c_int32), POINTER(c_double)]),
    "ember_backend_create": (c_void_p, [c_char_p, POINTER(BackendOptions)]),
    "ember_backend_destroy": (None, [c_void_p]),
    "ember_backend_graph_replays": (c_int64, []),
    "ember_backend_graph_captures": (c_int64, []),
    "ember_backend_info": (c_int32, [c_void_p, POINTER(ModelInfo)]),
    "ember_backend_forward": (c_int32, [c_void_p, POINTER(StepBatchC), POINTER(c_int32), c_int32]),
    "ember_backend_sample": (c_int32, [c_void_p, POINTER(SampleParams), c_int32, POINTER(c_int32)]),
    "ember_backend_token_probs": (c_int32, [c_void_p, POINTER(SampleParams), c_int32, POINTER(c_int32),
                                            POINTER(c_int32), c_int32, POINTER(c_float)]),
    "ember_backend_logits": (c_int32, [c_void_p, c_int32, POINTER(c_float), c_int32]),
    "ember_backend_set_capture_hidden": (c_int32, [c_void_p, c_int32]),
    "ember_backend_captured_hidden": (c_int32, [c_void_p, POINTER(c_float), c_int32]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded libember_hip.so with every prototype set; raises if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` first"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.ember_hip_abi_version() != ABI_VERSION:
            raise ImportError(f"{LIB_PATH} has ABI {handle.ember_hip_abi_version()}, expected {ABI_VERSION}")
        for i, st in enumerate(STRUCTS):
            if handle.ember_hip_sizeof(i) != ctypes.sizeof(st):
                raise ImportError(f"struct layout mismatch for {st.__name__}")
        _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().ember_hip_last_error()
    return msg.decode() if msg else ""


def check(code: int, what: str = "") -> int:
    """Raises EmberError for a negative or hipError_t return code."""
    if code != OK:
        raise EmberError(f"{what or 'ember'} failed ({code}): {last_error()}")
    return code
