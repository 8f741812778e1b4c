"""The C ABI library loads without a GPU and exports every function include/*.h declares."""
import ctypes
import re
from pathlib import Path

import ember_amd
from ember_amd import _lib

HEADERS = sorted((Path(__file__).resolve().parent.parent / "include").glob("*.h"))


def _declared():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"\b(ember_\w+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_every_declared_function_is_exported_and_bound():
    names = _declared()
    assert len(names) > 30
    so = ctypes.CDLL(str(_lib.LIB_PATH))
    for n in sorted(names):
        assert hasattr(so, n), f"{n} is declared in include/ but not exported"
    assert names == set(_lib.PROTOTYPES), "the ctypes binding and the header disagree"


def test_struct_layouts_and_version():
    lib = ember_amd.lib()
    assert lib.ember_hip_abi_version() == _lib.ABI_VERSION
    for i, st in enumerate(_lib.STRUCTS):
        assert lib.ember_hip_sizeof(i) == ctypes.sizeof(st), st.__name__
    assert lib.ember_hip_sizeof(99) == -1


def test_launchers_reject_bad_arguments_without_a_gpu():
    lib = ember_amd.lib()
    a = _lib.QkvArgs()
    a.head_dim, a.n_heads, a.n_kv = 64, 16, 8
    assert lib.ember_hip_kv_append(a, None) == _lib.ERR_INVALID
    assert "head_dim 64" in _lib.last_error()
    at = _lib.AttnArgs()
    at.head_dim, at.n_heads, at.n_kv = 128, 16, 1  # 16 query heads per kv head: more than 8
    assert lib.ember_hip_paged_decode(at, None) == _lib.ERR_INVALID
    at.n_kv, at.max_blocks, at.num_blocks, at.T, at.num_splits, at.split_len = 8, 4, 4, 1, 1, 24
    assert lib.ember_hip_paged_decode(at, None) == _lib.ERR_INVALID  # split_len not a multiple of 16
    assert "split_len" in _lib.last_error()
    at.split_len = _lib.MAX_SPLIT_LEN + 16  # a split's block ids must fit one 64-lane register
    assert lib.ember_hip_paged_decode(at, None) == _lib.ERR_INVALID
    assert "split_len" in _lib.last_error()
    pf = _lib.PrefillArgs()
    pf.head_dim, pf.n_heads, pf.n_kv, pf.dtype = 128, 16, 8, _lib.DTYPE_F32
    assert lib.ember_hip_prefill_attn(pf, None) == _lib.ERR_INVALID
    pf.dtype, pf.max_blocks, pf.num_blocks, pf.num_tiles, pf.scale = _lib.DTYPE_F16, 4, 4, 1, 0.0
    assert lib.ember_hip_prefill_attn(pf, None) == _lib.ERR_INVALID  # the block max is taken before scaling
    assert "scale" in _lib.last_error()
    assert lib.ember_hip_copy_pages(None, None) == _lib.ERR_INVALID
    g = _lib.GemvArgs()
    g.M, g.N, g.K, g.lda, g.ldc, g.epilogue = 65, 16, 64, 64, 16, 0  # M above 64
    assert lib.ember_hip_gemv(g, None) == _lib.ERR_INVALID
    assert "M must be 1..64" in _lib.last_error()
    g.M, g.K, g.lda = 4, 40, 40  # K not a multiple of 32
    assert lib.ember_hip_gemv(g, None) == _lib.ERR_INVALID
    g.K, g.lda, g.N, g.epilogue = 64, 64, 15, _lib.EPILOGUE_SILU_MUL  # silu_mul needs an even N
    assert lib.ember_hip_gemv(g, None) == _lib.ERR_INVALID
    assert "even N" in _lib.last_error()
    g.N, g.epilogue = 16, 0  # null pointers
    assert lib.ember_hip_gemv(g, None) == _lib.ERR_INVALID
    g.A, g.W, g.C = 16, 16, 16  # (never dereferenced: the workspace check comes first)
    g.workspace, g.workspace_bytes = 16, -1
    assert lib.ember_hip_gemv(g, None) == _lib.ERR_INVALID
    assert "workspace" in _lib.last_error()
    g.workspace, g.workspace_bytes = 8, 64  # misaligned
    assert lib.ember_hip_gemv(g, None) == _lib.ERR_INVALID
    assert lib.ember_hip_rmsnorm_rows(None, None) == _lib.ERR_INVALID
    n = _lib.NormArgs()
    n.R, n.hidden = 2, 0
    assert lib.ember_hip_rmsnorm_rows(n, None) == _lib.ERR_INVALID
    # T = 0 is a no-op, not an error
    at.split_len, at.T = 512, 0
    assert lib.ember_hip_paged_decode(at, None) == _lib.OK


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    import pytest

    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libember_hip.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(ImportError):
        _lib.lib()


def test_gemv_workspace_sizes():
    """The K split is taken only when N / 16 gives fewer than 256 work-groups and the slice would be wider than
    4096, in powers of two up to 4, with at least 256 of K per slice; its workspace is the 16-feature counters
    (padded to 256 bytes) plus the slice sums."""
    lib = _lib.lib()
    size = lib.ember_hip_gemv_workspace_bytes
    assert size(32, 4096, 2048) == 0  # 256 work-groups already: no split
    assert size(32, 2048, 2048) == 0  # the o projection: K 2048 is not split
    assert size(64, 1024, 3072) == 0  # nor 3072
    assert size(32, 2048, 4096) == 0  # nor 4096
    assert size(8, 2048, 6144) == 512 + 2 * 128 * 1 * 1024  # Qwen3-1.7B's down projection: 2 slices of 3072
    assert size(16, 1024, 12288) == 256 + 4 * 64 * 1 * 1024  # 4 slices of 3072
    assert size(32, 4096, 8192) == 0  # 256 work-groups already
    assert size(3, 130, 256) == 0  # K too short to split
    assert size(65, 2048, 6144) == 0 and size(32, 2048, 40) == 0  # invalid shapes: no workspace


def test_gemv_pack_sizes_and_errors():
    lib = _lib.lib()
    assert lib.ember_hip_gemv_packed_bytes(4096, 1024) == 4096 * 1024 * 2
    assert lib.ember_hip_gemv_packed_bytes(37, 64) == 48 * 64 * 2  # rows rounded up to 16
    assert lib.ember_hip_gemv_packed_bytes(37, 40) == 0
    assert lib.ember_hip_gemv_pack(None, 16, 64, None, None) == _lib.ERR_INVALID
    assert lib.ember_hip_gemv_pack(16, 16, 40, 16, None) == _lib.ERR_INVALID
    assert "multiple of 32" in _lib.last_error()
    g = _lib.GemvArgs()
    g.M, g.N, g.K, g.lda, g.ldc, g.epilogue, g.w_packed = 1, 16, 64, 64, 16, 0, 2
    g.A, g.W, g.C = 16, 16, 16
    assert lib.ember_hip_gemv(g, None) == _lib.ERR_INVALID
    assert "w_packed" in _lib.last_error()
