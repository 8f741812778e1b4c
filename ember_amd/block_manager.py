"""Python mirror of ember::BlockManager (src/kvcache/block_manager.hpp:25-67).

Same method names, argument meaning and error behaviour as the reference's C++
class; every call goes through the C ABI to the C++ implementation in
ember_amd/csrc/host/kvcache/block_manager.cpp. Errors the reference throws as
ember::Error raise EmberError here.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import numpy as np

from ._lib import BLOCK_SIZE, EmberError, last_error, lib

_I32P = ctypes.POINTER(ctypes.c_int32)


def _i32(values: Sequence[int]) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(values, dtype=np.int32).reshape(-1))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_I32P)


class BlockManager:
    def __init__(self, num_blocks: int, prefix_caching: bool):
        # The destructor is bound here: at interpreter exit the module's globals may be gone before this object.
        self._destroy = lib().ember_bm_destroy
        self._h = lib().ember_bm_create(int(num_blocks), 1 if prefix_caching else 0)
        if not self._h:
            raise EmberError(last_error())

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._destroy(h)

    # -- sizes (block_manager.hpp:29-33) --
    def num_blocks(self) -> int:
        return lib().ember_bm_num_blocks(self._h)

    def available(self) -> int:
        return lib().ember_bm_available(self._h)

    def used(self) -> int:
        return lib().ember_bm_used(self._h)

    def cached(self) -> int:
        return lib().ember_bm_cached(self._h)

    # -- allocation (:35-40) --
    def allocate(self) -> int:
        return lib().ember_bm_allocate(self._h)

    def release(self, block: int) -> None:
        if lib().ember_bm_release(self._h, int(block)) != 0:
            raise EmberError(last_error())

    def release_all(self, blocks: Sequence[int]) -> None:
        a = _i32(blocks)
        if lib().ember_bm_release_all(self._h, _ptr(a), a.size) != 0:
            raise EmberError(last_error())

    # -- prefix cache (:42-52) --
    @staticmethod
    def block_hash(parent: int, tokens: Sequence[int]) -> int:
        a = _i32(tokens)
        return int(lib().ember_bm_block_hash(int(parent), _ptr(a), a.size))

    def match_prefix(self, tokens: Sequence[int]) -> list[int]:
        a = _i32(tokens)
        out = np.empty(max(1, a.size // BLOCK_SIZE), dtype=np.int32)
        n = lib().ember_bm_match_prefix(self._h, _ptr(a), a.size, _ptr(out))
        if n < 0:
            raise EmberError(last_error())
        return out[:n].tolist()

    def seal(self, block: int, parent: int, tokens: Sequence[int]) -> int:
        a = _i32(tokens)
        h = int(lib().ember_bm_seal(self._h, int(block), int(parent), _ptr(a), a.size))
        if h == 0:
            raise EmberError(last_error())
        return h

    def prefix_caching(self) -> bool:
        return bool(lib().ember_bm_prefix_caching(self._h))

    def refcount(self, block: int) -> int:
        r = lib().ember_bm_refcount(self._h, int(block))
        if r < 0:
            raise EmberError(last_error())
        return r

    def hit_tokens(self) -> int:
        return int(lib().ember_bm_hit_tokens(self._h))

    def lookup_tokens(self) -> int:
        return int(lib().ember_bm_lookup_tokens(self._h))

    def check(self) -> str:
        buf = ctypes.create_string_buffer(512)
        lib().ember_bm_check(self._h, buf, len(buf))
        return buf.value.decode()

    def states(self) -> list[int]:
        out = np.empty(self.num_blocks(), dtype=np.uint8)
        lib().ember_bm_states(self._h, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)))
        return out.tolist()

    # -- additions: fork / copy-on-write --
    def share(self, blocks: Sequence[int]) -> None:
        a = _i32(blocks)
        if lib().ember_bm_share(self._h, _ptr(a), a.size) != 0:
            raise EmberError(last_error())

    def copy_on_write(self, block: int) -> int:
        r = lib().ember_bm_copy_on_write(self._h, int(block))
        if r < -1:
            raise EmberError(last_error())
        return r
