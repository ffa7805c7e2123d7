"""CPU restatement of the paged-KV path (numpy).  TEST INFRASTRUCTURE.

KV pool layout per layer (``/root/reference/engine/model_runner.py:184-190``):
``k_cache``/``v_cache`` = [num_blocks, block_size, num_kv_heads, head_dim];
``slot_mapping`` int64 with -1 = skip (padding, :303); ``block_tables`` int32
[B, max_blocks] padded with -1 (:262-266); ``context_lens`` int64 (:275).

Pinning (tests/test_oracle_paged.py):
  store_kvcache  -- poison-filled pool: exactly the targeted slots change,
                    bitwise; -1 slots skipped.
  sdpa           -- the reference's own golden vectors
                    tests/_snapshots/test_scaled_dot_product_attention.npz and
                    test_4d_...npz (seeded inputs, conftest.py:253-280),
                    checked to 1e-6.
  paged_decode   -- equals ``sdpa`` on the gathered K/V; L=1 gives v0;
                    constant V gives V; invariant under a permutation of the
                    block pool with remapped tables; L=0 gives zeros.
  decode_slots   -- brute force slot(b,t) = bt[b][t//BS]*BS + t%BS.
  prefill_attention -- a whole prompt (lq == lk) equals ``sdpa`` with the
                    lower-triangular mask (the reference's causal
                    scaled_dot_product_attention, utils.py:51-63 with
                    GQA.py:126-130's causal mask); a cached prefix (lq < lk)
                    equals the last lq rows of the whole prompt's result;
                    paged keys equal the same keys stored contiguously.
"""
from __future__ import annotations

import numpy as np


def store_kvcache(key, value, k_cache, v_cache, slot_mapping):
    """In place: for t with slot_mapping[t] != -1,
    k_cache.reshape(NB*BS, Hkv, D)[slot] = key[t] (same for v).

    The write the reference's missing attention layer performs with the
    slot contract of engine/model_runner.py:226-230 (prefill), :261 (decode)
    and :303 (-1 padding).  Works on any dtype (bit copy)."""
    NB, BS, H, D = k_cache.shape
    kc = k_cache.reshape(NB * BS, H, D)
    vc = v_cache.reshape(NB * BS, H, D)
    for t, slot in enumerate(np.asarray(slot_mapping, dtype=np.int64)):
        if slot == -1:
            continue
        kc[slot] = key[t]
        vc[slot] = value[t]


def sdpa(q, k, v, mask=None, scale=None, dtype=np.float64):
    """softmax(q k^T * scale, masked) v -- model/attention/utils.py:51-63
    (scores divided by sqrt(d_k) when scale is None; mask True = keep;
    softmax subtracts the row max, utils.py:8-12)."""
    q = np.asarray(q, dtype)
    k = np.asarray(k, dtype)
    v = np.asarray(v, dtype)
    d = q.shape[-1]
    if scale is None:
        s = (q @ np.swapaxes(k, -1, -2)) / dtype(np.sqrt(d))
    else:
        s = (q @ np.swapaxes(k, -1, -2)) * dtype(scale)
    if mask is not None:
        s = np.where(mask, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    return (e / e.sum(axis=-1, keepdims=True)) @ v


def gather_kv(cache, block_table, length):
    """Rows 0..length-1 of one sequence: cache[bt[t // BS], t % BS]."""
    BS = cache.shape[1]
    t = np.arange(length)
    blocks = np.asarray(block_table, dtype=np.int64)[t // BS]
    return cache[blocks, t % BS]


def paged_decode(q, k_cache, v_cache, context_lens, block_tables, scale, dtype=np.float64):
    """o[b, h] = softmax_t(scale * q[b,h] . K[b,t,h//G]) V[b,t,h//G], t < L_b.

    GQA head map h -> h // (Hq/Hkv) as model/attention/GQA.py:118-125
    (repeat_interleave of kv heads); SDPA math as utils.py:51-63.
    L_b == 0 (graph padding rows, model_runner.py:305) gives zeros.
    q: [B, Hq, D]; caches [NB, BS, Hkv, D]; returns float64/32 [B, Hq, D]."""
    q = np.asarray(q, dtype)
    B, Hq, D = q.shape
    Hkv = k_cache.shape[2]
    G = Hq // Hkv
    out = np.zeros((B, Hq, D), dtype)
    for b in range(B):
        L = int(context_lens[b])
        if L == 0:
            continue
        K = gather_kv(k_cache, block_tables[b], L).astype(dtype)  # [L, Hkv, D]
        V = gather_kv(v_cache, block_tables[b], L).astype(dtype)
        Kh = np.repeat(K.transpose(1, 0, 2), G, axis=0)  # [Hq, L, D]
        Vh = np.repeat(V.transpose(1, 0, 2), G, axis=0)
        out[b] = sdpa(q[b][:, None, :], Kh, Vh, scale=scale, dtype=dtype)[:, 0, :]
    return out


def decode_slots(block_tables, context_lens, block_size):
    """Slot of each sequence's newest token (position L-1):
    bt[b][(L-1)//BS]*BS + (L-1)%BS.  This is the slot
    engine/model_runner.py:261 means; the reference's formula there
    (block_table[-1]*BS + last_block_num_tokens - 1) gives block_id*BS - 1
    when L % BS == 0 (engine/sequence.py:67-69), which this restatement does
    not copy.  L == 0 -> -1."""
    out = np.full(len(context_lens), -1, dtype=np.int64)
    for b, L in enumerate(context_lens):
        L = int(L)
        if L > 0:
            out[b] = int(block_tables[b][(L - 1) // block_size]) * block_size + (L - 1) % block_size
    return out


def prefill_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, scale, block_tables=None, dtype=np.float64):
    """Varlen causal prefill attention (the flash_attn_varlen_func call named
    at engine/model_runner.py:291-292, causal=True).

    Sequence i: queries q[cu_q[i]:cu_q[i+1]] (lq tokens) at positions
    lk-lq .. lk-1 of its context of lk = cu_k[i+1]-cu_k[i] keys; query p
    attends to keys 0..p.  Keys: k[cu_k[i]:cu_k[i+1]] (contiguous, [Tk, Hkv,
    D]) or, with block_tables, gathered from the pool k = [NB, BS, Hkv, D].
    GQA head map h -> h // (Hq/Hkv).  Returns [Tq, Hq, D]."""
    q = np.asarray(q, dtype)
    Tq, Hq, D = q.shape
    Hkv = k.shape[-2]
    G = Hq // Hkv
    out = np.zeros((Tq, Hq, D), dtype)
    cu_q = np.asarray(cu_seqlens_q, np.int64)
    cu_k = np.asarray(cu_seqlens_k, np.int64)
    for i in range(len(cu_q) - 1):
        qs, qe = int(cu_q[i]), int(cu_q[i + 1])
        lq, lk = qe - qs, int(cu_k[i + 1] - cu_k[i])
        if lq == 0:
            continue
        if block_tables is not None:
            K = gather_kv(k, block_tables[i], lk)
            V = gather_kv(v, block_tables[i], lk)
        else:
            K = k[int(cu_k[i]):int(cu_k[i + 1])]
            V = v[int(cu_k[i]):int(cu_k[i + 1])]
        Kh = np.repeat(np.asarray(K, dtype).transpose(1, 0, 2), G, axis=0)  # [Hq, lk, D]
        Vh = np.repeat(np.asarray(V, dtype).transpose(1, 0, 2), G, axis=0)
        pos_q = np.arange(lk - lq, lk)
        mask = np.arange(lk)[None, :] <= pos_q[:, None]                      # [lq, lk]
        out[qs:qe] = sdpa(q[qs:qe].transpose(1, 0, 2), Kh, Vh, mask=mask, scale=scale,
                          dtype=dtype).transpose(1, 0, 2)
    return out
