"""Float64 closed forms of the attention part of the verification path (oracle).

Test infrastructure only (see oracle/__init__.py).

Reference semantics restated:
  prefix attention + LSE     runtime/tree_attention.py:414-446, LSE layout of
                             runtime/attention_compat.py:103-132 ([B, H, M])
  tree block                 runtime/tree_attention.py:40-63 with the mask
                             conversion of _maybe_to_int8_mask (:449-460)
  hybrid merge               llama_target_model.py:862-866 / runtime/tree_attention.py:535-539
  GQA expansion              llama_target_model.py:543-560 (q head h reads kv head h // G)
  bundle verify              runtime/bundle_verifier.py:259-297 (masked attention + LSE [B, M, H])
  paged gather               core/kv_cache/paged_kv.py:56-65, 325-340
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import numpy as np


def masked_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray,
                     mask: Optional[np.ndarray] = None) -> Tuple[np.ndarray, np.ndarray]:
    """Softmax attention of one batch element in float64.

    q [M, H, D]; k, v [N, Hk, D] with H % Hk == 0 (head h reads kv head h // (H/Hk));
    mask [M, N] bool shared by all heads (None = all visible).
    Returns O [M, H, D] and natural-log LSE [M, H]; a row with no visible key
    has O = 0 and LSE = -inf.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    M, H, D = q.shape
    N, Hk, _ = k.shape
    G = H // Hk
    out = np.zeros((M, H, D))
    lse = np.full((M, H), -np.inf)
    if N == 0:
        return out, lse
    scale = 1.0 / math.sqrt(D)
    for h in range(H):
        kh = h // G
        s = (q[:, h, :] @ k[:, kh, :].T) * scale
        if mask is not None:
            s = np.where(mask, s, -np.inf)
        m = s.max(axis=1)
        ok = np.isfinite(m)
        ms = np.where(ok, m, 0.0)
        p = np.exp(s - ms[:, None])
        l = p.sum(axis=1)
        o = p @ v[:, kh, :]
        out[:, h, :] = np.where(ok[:, None], o / np.where(ok, l, 1.0)[:, None], 0.0)
        lse[:, h] = np.where(ok, ms + np.log(np.where(ok, l, 1.0)), -np.inf)
    return out, lse


def prefix_attention(q, k, v) -> Tuple[np.ndarray, np.ndarray]:
    """prefix_attention_forward for one batch: O [M, H, D], LSE [H, M] (flash layout)."""
    o, lse = masked_attention(q, k, v, None)
    return o, lse.T.copy()


def tree_block_keep(tree_mask: np.ndarray, M: int) -> np.ndarray:
    """Lower-right M x M block of a tree mask as keep-booleans (_maybe_to_int8_mask).

    Float masks keep where == 0 (additive masks); integer / bool masks keep where != 0.
    """
    blk = np.asarray(tree_mask)[..., -M:, -M:]
    blk = blk.reshape(blk.shape[-2], blk.shape[-1]) if blk.ndim > 2 and blk.shape[0] == 1 else blk
    if np.issubdtype(blk.dtype, np.floating):
        return blk == 0
    return blk != 0


def tree_attention(q, k_t, v_t, keep: np.ndarray, prefix_lse_hm: np.ndarray):
    """tree_attention_forward for one batch.

    q [M, H, D], k_t/v_t [M, Hk, D], keep [M, M] bool, prefix_lse_hm [H, M].
    Returns current_out [M, H, D], weight [M, H] = sigmoid(prefix_lse - tree_lse),
    tree_lse [M, H].
    """
    o_t, lse_t = masked_attention(q, k_t, v_t, keep)
    w = 1.0 / (1.0 + np.exp(-(np.asarray(prefix_lse_hm, dtype=np.float64).T - lse_t)))
    return o_t, w, lse_t


def hybrid_merge(o_t, w, o_p):
    """out = O_tree * (1 - w) + O_prefix * w (llama_target_model.py:862-866)."""
    return o_t * (1.0 - w[..., None]) + o_p * w[..., None]


def merge_lse(o_a, lse_a, o_b, lse_b):
    """Exact two-way combine of attention results over disjoint key sets."""
    m = np.maximum(lse_a, lse_b)
    ms = np.where(np.isfinite(m), m, 0.0)
    wa = np.exp(lse_a - ms)
    wb = np.exp(lse_b - ms)
    tot = wa + wb
    lse = np.where(tot > 0, ms + np.log(np.where(tot > 0, tot, 1.0)), -np.inf)
    den = np.where(tot > 0, tot, 1.0)
    o = (o_a * wa[..., None] + o_b * wb[..., None]) / den[..., None]
    return o, lse


def ancestor_mask(parent: Sequence[int]) -> np.ndarray:
    """[M, M] bool: j is i or an ancestor of i (runtime/draft_tree.py:188-214)."""
    M = len(parent)
    keep = np.zeros((M, M), dtype=bool)
    for i in range(M):
        j, steps = i, 0
        while 0 <= j < M and steps <= M:
            keep[i, j] = True
            if parent[j] == j:
                break
            j = parent[j]
            steps += 1
    return keep


def tree_verify(q, k_all, v_all, n_prefix: int, parent: Sequence[int]):
    """Attention of the tree queries over prefix + ancestors-or-self, in one pass.

    q [M, H, D]; k_all, v_all [n_prefix + M, Hk, D] (tree K/V after the prefix).
    Returns O [M, H, D], LSE [M, H].
    """
    M = q.shape[0]
    mask = np.zeros((M, n_prefix + M), dtype=bool)
    mask[:, :n_prefix] = True
    mask[:, n_prefix:] = ancestor_mask(parent)
    return masked_attention(q, k_all[:n_prefix + M], v_all[:n_prefix + M], mask)


def paged_gather(pool_kv: np.ndarray, page_table: Sequence[int], n: int) -> np.ndarray:
    """Tokens [0, n) of one K or V pool half [P, Hk, ps, D] -> [n, Hk, D]."""
    ps = pool_kv.shape[2]
    tok = np.arange(n)
    pt = np.asarray(page_table)
    return pool_kv[pt[tok // ps], :, tok % ps, :]


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (round-to-nearest-even), returned as float32."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(a), a, out)


def half_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to float16 (round-to-nearest-even), returned as float32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def rope_16bit(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, f16: bool = False) -> np.ndarray:
    """x * cos + rotate_half(x) * sin as torch evaluates it on bf16/f16 tensors
    (llama_target_model.py:408-427, 452-473): each product and the sum rounded
    to the 16-bit dtype.  x [..., M, D] (token axis -2), cos/sin [M, D]; all
    values already representable in the dtype."""
    rnd = half_round if f16 else bf16_round
    x = np.asarray(x, dtype=np.float32)
    d = x.shape[-1] // 2
    rot = np.concatenate([-x[..., d:], x[..., :d]], axis=-1)
    return rnd(rnd(x * cos) + rnd(rot * sin))
