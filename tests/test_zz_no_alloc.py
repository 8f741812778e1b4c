"""ember_hip_paged_decode_static (the entry point that allocates nothing) against ember_hip_paged_decode.

Both are called through the C ABI on the same step; the static variant takes its split partials and merge
counters from the library's static device array. Outputs must be bit-identical, on two calls in a row (the
second with a smaller step, so the array holds the first call's contents), and both within the f16 bound of
the float64 reference.
"""
import ctypes

import numpy as np
import pytest
import torch

from ember_amd import _lib
from ember_amd import kernels as K
from helpers import D, PAGE, attention_f64, make_step, rel_err

pytestmark = pytest.mark.gpu

H, KVH = 16, 8


def _bits(t):
    return t.cpu().numpy().view(np.uint16)


def _run_both(rng, device, ctx_after, new_tokens, NB):
    step = make_step(rng, ctx_after, new_tokens, NB)
    ints = K.StepInts(step.positions, step.token_seq, step.tables, NB)
    k_pool = (0.5 * torch.randn((NB, KVH, PAGE, D), device=device)).to(torch.float16)
    v_pool = (0.5 * torch.randn((NB, KVH, PAGE, D), device=device)).to(torch.float16)
    q = torch.randn((step.T, H, D), device=device).to(torch.float16)
    runs = K.decode_runs(ints, range(step.T), group=H // KVH)
    out_ref = torch.full((step.T, H, D), float("nan"), dtype=torch.float16, device=device)
    keep = K.paged_attention(q, k_pool, v_pool, out_ref, ints, n_heads=H, n_kv=KVH, runs=runs, use_work_list=True,
                             merge_in_kernel=True)
    out_static = torch.full_like(out_ref, float("nan"))
    a, keep2 = K._attn_args(q, k_pool, v_pool, out_static, ints, n_heads=H, n_kv=KVH, token_list=None, runs=runs,
                            split_len=512, num_splits=None, scratch=None, use_work_list=True, merge_in_kernel=False)
    a.part_acc, a.part_ml, a.merge_counters = None, None, None  # the static scratch replaces them
    splits = a.num_splits
    _lib.check(_lib.lib().ember_hip_paged_decode_static(ctypes.byref(a), torch.cuda.current_stream().cuda_stream),
               "paged_decode_static")
    torch.cuda.synchronize()
    del keep, keep2
    assert splits > 1, "the step must use split partials (the scratch) to test anything"
    assert np.array_equal(_bits(out_static), _bits(out_ref)), "static-scratch decode differs from paged_decode"
    want = attention_f64(q.float().cpu().numpy(), step, k_pool.float().cpu().numpy(), v_pool.float().cpu().numpy(),
                         H, KVH)
    assert rel_err(out_static.float().cpu().numpy(), want) < 2e-3
    return splits


def test_static_scratch_decode_equals_paged_decode_twice(rng, device):
    """A 28-sequence step with contexts up to 4096 (8 splits) and 5-token verify runs, then a smaller step of 6
    sequences with shorter contexts: bit-identical to ember_hip_paged_decode both times."""
    NB = 8192
    ctx = rng.integers(256, 4097, 28)
    ctx[3] = 4096  # the longest context sets 8 splits
    new = np.where(np.arange(28) % 4 == 0, 5, 1)
    assert _run_both(rng, device, ctx, new, NB) == 8
    ctx2 = rng.integers(600, 1500, 6)
    assert _run_both(rng, device, ctx2, np.ones(6, int), NB) <= 3


def test_static_scratch_rejects_oversized_steps_and_caller_scratch(device):
    """More partials than the static array holds, or caller scratch given, is refused before any launch."""
    lib = _lib.lib()
    a = _lib.AttnArgs()
    a.head_dim, a.n_heads, a.n_kv, a.max_blocks, a.num_blocks, a.split_len, a.dtype = 128, 16, 8, 256, 64, 512, 0
    a.T, a.num_splits = _lib.STATIC_MAX_PARTIALS // 16 + 1, 1
    assert lib.ember_hip_paged_decode_static(ctypes.byref(a), None) == _lib.ERR_INVALID
    assert "exceed the static scratch" in _lib.last_error()
    a.T, a.num_splits = 1, 2
    dummy = torch.zeros(4, device=device)
    a.part_acc = dummy.data_ptr()
    assert lib.ember_hip_paged_decode_static(ctypes.byref(a), None) == _lib.ERR_INVALID
    assert "must be NULL" in _lib.last_error()
