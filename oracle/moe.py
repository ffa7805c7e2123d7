"""CPU restatement of the MoE expert dispatch (numpy).  TEST INFRASTRUCTURE.

Reference semantics (``/root/reference/model/architecture/``):
  * moe_infer: argsort of the flat picks, bincount, offsets, one expert MLP
    per segment of gathered tokens, output * weight, scatter_add_ into the
    token rows .......................................... moe.py:288-341
  * shared expert added to the routed sum ................ moe.py:272-273
  * segment_reduce_weighted: per token, sum of w_p * x_p over its segment
    of a target-sorted list (searchsorted offsets) ....... moe_kernels.py:6-125
  * fused_scatter_add_weighted: the same for an unsorted target list
    (argsort by target first) ........................... moe_kernels.py:128-171

This build's dispatch layout (what the HIP kernels produce) is restated
here exactly: moe_align groups the entries (t, j) -- j < top_k the routed
pick topk_idx[t, j], then the S shared experts E .. E+S-1 with weight 1 --
by expert, experts in index order, entries of an expert in flat order
t * (top_k + S) + j, each expert's segment padded to 128 rows.

Pinning (tests/test_oracle_moe.py):
  moe_align          -- brute force (a scan per expert over all entries);
                        invariants: every kept entry appears once, rows of
                        an expert hold that expert's entries in flat order,
                        padding rows are -1 / weight 0, tiles past the last
                        segment are -1, capacity never exceeded.
  grouped_gemm       -- one expert with identity rows equals fp8.fp8_gemm
                        (pinned itself); each tile equals fp8.fp8_gemm of
                        the gathered rows against its expert's weights.
  moe_combine        -- scalar loops over (t, j).
  segment_reduce_weighted / scatter_add_weighted
                     -- np.add.at scatter and a one-hot matrix product
                        agree with the segment form; an unsorted list equals
                        its target-sorted permutation.
"""
from __future__ import annotations

import numpy as np

from . import fp8 as F

TILE = 128


def align_tiles(T: int, top_k: int, E: int, S: int) -> int:
    """Capacity in 128-row tiles: ceil((T*(top_k+S) + (E+S)*127) / 128)."""
    if T <= 0:
        return 0
    n = T * (top_k + S)
    return (n + (E + S) * (TILE - 1) + TILE - 1) // TILE


def entries(topk_idx, topk_w, E: int, S: int):
    """Flat (token, expert, weight) list; out-of-range picks get expert -1."""
    idx = np.asarray(topk_idx, np.int64)
    w = np.asarray(topk_w, np.float32)
    T, k = idx.shape
    out = []
    for t in range(T):
        for j in range(k + S):
            if j < k:
                e = int(idx[t, j])
                out.append((t, e if 0 <= e < E else -1, float(w[t, j])))
            else:
                out.append((t, E + j - k, 1.0))
    return out


def moe_align(topk_idx, topk_w, E: int, S: int = 0, num_tiles=None):
    """Returns (row_token int32 [P], row_weight float32 [P], tile_expert
    int32 [P/128], entry_row int32 [T, top_k+S]), P = num_tiles*128."""
    idx = np.asarray(topk_idx, np.int64)
    T, k = idx.shape
    ent = entries(topk_idx, topk_w, E, S)
    tiles = align_tiles(T, k, E, S) if num_tiles is None else num_tiles
    row_token = np.full(tiles * TILE, -1, np.int32)
    row_weight = np.zeros(tiles * TILE, np.float32)
    tile_expert = np.full(tiles, -1, np.int32)
    entry_row = np.full(len(ent), -1, np.int32)
    base = 0
    for e in range(E + S):
        mine = [i for i, (_, ee, _) in enumerate(ent) if ee == e]
        for r, i in enumerate(mine):
            row_token[base + r] = ent[i][0]
            row_weight[base + r] = ent[i][2]
            entry_row[i] = base + r
        padded = -(-len(mine) // TILE) * TILE
        tile_expert[base // TILE:(base + padded) // TILE] = e
        base += padded
    assert base <= tiles * TILE
    return row_token, row_weight, tile_expert, entry_row.reshape(T, k + S)


def grouped_gemm(a, a_s, row_index, tile_expert, b, b_s, bias=None, round_bf16=True):
    """Per tile i with e = tile_expert[i] >= 0: rows 128i..128i+127 of the
    result = fp8_gemm(a[rows], a_s[rows], b[e], b_s[e]) (+ bias[e]); row
    index -1 reads row 0; tiles with e < 0 stay NaN (unwritten).
    b: codes [E, N, K], b_s [E, ceil(N/128), K/128], bias [E, N]."""
    tile_expert = np.asarray(tile_expert)
    tiles = len(tile_expert)
    N = b.shape[1]
    out = np.full((tiles * TILE, N), np.nan, np.float64)
    for i, e in enumerate(tile_expert):
        if e < 0:
            continue
        rows = np.arange(i * TILE, (i + 1) * TILE)
        src = rows if row_index is None else np.maximum(np.asarray(row_index)[rows], 0)
        out[rows] = F.fp8_gemm(a[src], a_s[src], b[e], b_s[e], None if bias is None else bias[e],
                               round_bf16=round_bf16)
    return out


def moe_combine(out, entry_row, topk_idx, topk_w, E: int, S: int = 0, down_bias=None):
    """y[t] = bf16(sum_j out[entry_row[t, j]] + sum_j w_tj * down_bias[e_tj]),
    dropped entries (-1) skipped; float64 sums."""
    entry_row = np.asarray(entry_row)
    T = entry_row.shape[0]
    ent = entries(topk_idx, topk_w, E, S)
    kk = entry_row.shape[1]
    y = np.zeros((T, out.shape[1]), np.float64)
    for t in range(T):
        for j in range(kk):
            r = entry_row[t, j]
            if r < 0:
                continue
            y[t] += out[r]
            if down_bias is not None:
                _, e, w = ent[t * kk + j]
                y[t] += w * np.asarray(down_bias, np.float64)[e]
    return F.bf16_round(y.astype(np.float32))


def segment_reduce_weighted(x, w, sorted_idx, num_tokens: int) -> np.ndarray:
    """y[t] = sum over the segment of p with sorted_idx[p] == t of w[p]*x[p]
    (segments by searchsorted, as moe_kernels.py:99-101); float64."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    sidx = np.asarray(sorted_idx, np.int64)
    bounds = np.searchsorted(sidx, np.arange(num_tokens + 1), side="left")
    y = np.zeros((num_tokens, x.shape[1]), np.float64)
    for t in range(num_tokens):
        s, e = bounds[t], bounds[t + 1]
        if e > s:
            y[t] = (w[s:e, None] * x[s:e]).sum(0)
    return y


def scatter_add_weighted(x, token_idx, w, num_tokens: int) -> np.ndarray:
    """y[t] = sum over i with token_idx[i] == t of w[i]*x[i] (any order;
    indices outside [0, num_tokens) dropped); float64 via np.add.at."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    idx = np.asarray(token_idx, np.int64)
    keep = (idx >= 0) & (idx < num_tokens)
    y = np.zeros((num_tokens, x.shape[1]), np.float64)
    np.add.at(y, idx[keep], w[keep, None] * x[keep])
    return y
