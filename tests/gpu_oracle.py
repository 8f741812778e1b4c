"""The oracle beside the GPU path at full workload sizes.

A full-size pool (config 4: 131,072 pages) cannot be mirrored page for page in the oracle's memory, so a
step is checked on a snapshot: the pages the step's sequences read are gathered from the GPU pools before the
step (f16 bits), renumbered compactly (a page shared by several sequences stays one page), and the oracle's
append + attention run on that compact copy. After the step the same pages are gathered again and compared
with what the oracle wrote: every slot the step does not write bit-exact, new V slots bit-exact, new K slots
within one ulp of the stored format or 2^-20 absolute (near-zero rotations).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

import oracle

PAGE, D = 16, 128


@dataclass
class Snapshot:
    blocks: np.ndarray     # [U] pool blocks, ascending
    tables: np.ndarray     # [S, max_blocks] compact page numbers (0..U-1; -1 past a sequence's pages)
    k: np.ndarray          # [U + 1, n_kv, 16, D] f16 bits (uint16) or f32; the last page is a spare of zeros
    v: np.ndarray
    f16: bool


def snapshot(kv, layer: int, tables, pages_per_seq) -> Snapshot:
    """Gathers the pages tables[s, :pages_per_seq[s]] of one layer's K and V pools."""
    tables = np.asarray(tables, np.int32)
    pages_per_seq = [int(p) for p in pages_per_seq]
    used = np.concatenate([tables[s, :p] for s, p in enumerate(pages_per_seq)] + [np.zeros(0, np.int32)])
    blocks, inverse = np.unique(used, return_inverse=True)
    compact = np.full(tables.shape, -1, np.int32)
    at = 0
    for s, p in enumerate(pages_per_seq):
        compact[s, :p] = inverse[at:at + p]
        at += p
    idx = torch.from_numpy(blocks.astype(np.int64)).to("cuda")
    f16 = kv.dtype == torch.float16
    out = []
    for which in ("k", "v"):
        pages = _bits(kv.pool_view(layer, which)[idx], f16)
        full = np.zeros((blocks.size + 1,) + pages.shape[1:], pages.dtype)
        full[:blocks.size] = pages
        out.append(full)
    return Snapshot(blocks, compact, out[0], out[1], f16)


def _bits(t: torch.Tensor, f16: bool) -> np.ndarray:
    """f16 pages as their bits (uint16), f32 pages as they are."""
    a = t.cpu().numpy()
    return a.view(np.uint16) if f16 else a


def oracle_layer(snap: Snapshot, qkv, positions, query_start, *, n_heads, n_kv, q_norm, k_norm, inv_freq, eps=1e-6,
                 subset=None, threads=16):
    """The oracle's append (into snap's compact pools, f16 or f32 as the GPU's) then attention of the step's
    tokens, or of the tokens in `subset` (indices into the step, ascending) only. qkv: [T, (n_heads + 2 n_kv) * D]
    (f16 values for f16 pools). Returns [len(subset) or T, n_heads, D] f32."""
    positions = np.asarray(positions, np.int32)
    query_start = np.asarray(query_start, np.int32)
    q = oracle.append_layer(np.asarray(qkv, np.float32), positions, query_start, snap.tables, snap.k, snap.v,
                            n_heads=n_heads, n_kv=n_kv, inv_freq_=inv_freq, eps=eps, q_norm=q_norm, k_norm=k_norm,
                            num_blocks=snap.k.shape[0], kv_f16=snap.f16)
    if subset is None:
        pos, qs, tab, qq = positions, query_start, snap.tables, q
    else:
        subset = np.asarray(subset, np.int64)
        seq_of = np.searchsorted(query_start, subset, side="right") - 1
        seqs, counts = np.unique(seq_of, return_counts=True)
        pos, qq = positions[subset], q[subset]
        qs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
        tab = snap.tables[seqs]
    return oracle.attention_layer(qq, pos, qs, tab, snap.k, snap.v, n_heads=n_heads, n_kv=n_kv,
                                  num_blocks=snap.k.shape[0], kv_f16=snap.f16, q_f16=snap.f16, threads=threads)


def check_pages_after(kv, layer: int, snap: Snapshot, written) -> None:
    """Compares the GPU's pages (gathered again after the step) with the oracle's snapshot after its append.
    written: (compact page, slot) pairs the step wrote. Untouched slots and new V slots must be bit-exact,
    new K slots within one ulp or 2^-20 absolute (the GPU's and the CPU's rsqrt / sincos roundings)."""
    idx = torch.from_numpy(snap.blocks.astype(np.int64)).to("cuda")
    gk = _bits(kv.pool_view(layer, "k")[idx], snap.f16)
    gv = _bits(kv.pool_view(layer, "v")[idx], snap.f16)
    ok, ov = snap.k[:snap.blocks.size], snap.v[:snap.blocks.size]
    mask = np.zeros(ok.shape[:1] + ok.shape[2:3], bool)  # [U, 16]: slots written this step
    for page, slot in written:
        mask[page, slot] = True
    if not np.array_equal(gv, ov):
        bad = (gv != ov).any(axis=(1, 3))
        pg, sl = np.nonzero(bad)
        where = []
        for p, s_ in zip(pg[:4], sl[:4]):
            writers = [t for t, (wp, ws) in enumerate(written) if wp == p and ws == s_]
            h = int(np.nonzero((gv[p, :, s_] != ov[p, :, s_]).any(axis=1))[0][0])
            d = np.nonzero(gv[p, h, s_] != ov[p, h, s_])[0]
            where.append(dict(block=int(snap.blocks[p]), slot=int(s_), written=bool(mask[p, s_]), writers=writers,
                              head=h, dims=d[:6].tolist(), gpu=gv[p, h, s_, d[:3]].tolist(),
                              oracle=ov[p, h, s_, d[:3]].tolist()))
        raise AssertionError(f"V differs from the oracle's in {pg.size} slots of {np.unique(pg).size} pages "
                             f"({int((bad & mask).sum())} of them written this step): {where}")
    differs = (gk != ok).any(axis=(1, 3))  # [U, 16]: slots whose K differs anywhere
    assert not (differs & ~mask).any(), "K slots the step does not write changed"
    pg, sl = np.nonzero(differs)
    if pg.size:
        # One ulp of the stored format (|d| <= 2^-10 |k| in f16, 2^-20 |k| in f32; the rounding of the same f32
        # value can cross one boundary), plus 2^-20 absolute: where the rotation x cos - y sin cancels to near
        # zero, the GPU's and the CPU's f32 cos / sin / product roundings (a few 2^-24 of |x|) are many f16
        # subnormal ulps (2^-24 each).
        f = (lambda a: a.view(np.float16).astype(np.float64)) if snap.f16 else (lambda a: a.astype(np.float64))
        g, o = f(gk[pg, :, sl]), f(ok[pg, :, sl])
        bound = (2.0 ** -10 if snap.f16 else 2.0 ** -20) * np.abs(o) + 2.0 ** -20
        excess = np.abs(g - o) - bound
        i = np.unravel_index(int(np.argmax(excess)), excess.shape)
        assert excess[i] <= 0, f"a new K value differs beyond its bound: gpu {g[i]!r}, oracle {o[i]!r}"


def written_slots(snap: Snapshot, positions, query_start):
    """(compact page, slot) of every token the step appends."""
    out = []
    for s in range(len(query_start) - 1):
        for t in range(query_start[s], query_start[s + 1]):
            p = int(positions[t])
            out.append((int(snap.tables[s, p // PAGE]), p % PAGE))
    return out
