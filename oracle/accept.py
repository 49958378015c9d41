"""CPU restatement of the tree acceptance walk (oracle).

Test infrastructure only (see oracle/__init__.py).

``greedy_walk`` restates draft/tree_verification.py:100-182 step by step
(numpy argmax returns the first maximal index and the first NaN, as
torch.argmax does).  ``typical_walk`` applies the posterior criterion of
Cai et al. 2024 (Medusa): accept node i iff
    p_T(draft[i] | parent) > min(eps, alpha * exp(-H(p_T(. | parent))))
with p_T = softmax(logits / T) and H its exact entropy (0 log 0 = 0),
evaluated in float64; T, eps and alpha are taken as the float32 values the
C ABI receives.  The reference has no typical mode, so this function defines
it.
``brute_force_greedy`` is an independent formulation used to pin
``greedy_walk``: a node is accepted iff every edge on its root path matches.
``kv_commit`` restates the KV compaction after the walk
(draft/tree_verification.py:197-217): a gather of the accepted rows into a
temporary, then a copy to the front of the tree's slots.
"""

from __future__ import annotations

from typing import List, Sequence, Tuple

import numpy as np


def parent_ext(parent_ref: Sequence[int]) -> np.ndarray:
    """[0] + (parent + 1) with self-references mapped to the root (:120-125)."""
    p = np.asarray(parent_ref, dtype=np.int64)
    rows = np.arange(p.size, dtype=np.int64)
    p = np.where(p == rows, -1, p)
    return np.concatenate([np.zeros(1, dtype=np.int64), p + 1])


def _walk(ok: np.ndarray, pe: np.ndarray, pos: np.ndarray, max_depth: int, draft: np.ndarray,
          next_tokens: np.ndarray):
    ok = ok.copy()
    ok[0] = True
    max_hops = min(int(max_depth) + 2, int(pe.size))
    for _ in range(max_hops):
        nxt = ok & ok[pe]
        if np.array_equal(nxt, ok):
            break
        ok = nxt
    masked = np.where(ok, pos, 0)
    max_id = int(np.argmax(masked))
    back = pe.tolist()
    back[0] = -1
    ids: List[int] = []
    cur = max_id
    while cur != -1:
        ids.append(cur)
        cur = back[cur]
    ids.reverse()
    toks = [int(draft[i]) for i in ids]
    return toks, ids, len(ids) - 1, int(next_tokens[max_id]), max_id


def greedy_walk(logits: np.ndarray, draft: Sequence[int], parent_ref: Sequence[int], pos: Sequence[int],
                max_depth: int) -> Tuple[List[int], List[int], int, int, int]:
    """Returns (best_candidate, best_candidate_id, accept_length, next_token, max_id)."""
    logits = np.asarray(logits)
    next_tokens = np.argmax(logits, axis=-1)
    draft = np.asarray(draft, dtype=np.int64)
    pe = parent_ext(parent_ref)
    ok = draft == next_tokens[pe]
    return _walk(ok, pe, np.asarray(pos, dtype=np.int64), max_depth, draft, next_tokens)


def softmax_stats(row: np.ndarray, temperature: float = 1.0) -> Tuple[np.ndarray, float]:
    """p = softmax(row / T) and its entropy H = -sum p log p (float64)."""
    y = np.asarray(row, dtype=np.float64) / temperature
    m = y.max()
    e = np.exp(y - m)
    z = e.sum()
    p = e / z
    # 0 log 0 = 0: entries with p = 0 (y = -inf) add nothing to sum p*y.
    ent = float(m + np.log(z) - (p * np.where(p > 0, y, 0.0)).sum())
    return p, ent


def f32(x: float) -> float:
    """x rounded to float32 (the C ABI's argument type), as a Python float."""
    return float(np.float32(x))


def typical_prob_thr(row: np.ndarray, tok: int, temperature: float, eps: float, alpha: float) -> Tuple[float, float]:
    """(p_T(tok), min(eps, alpha * exp(-H))) with float32-rounded T, eps, alpha."""
    p, ent = softmax_stats(row, f32(temperature))
    return float(p[tok]), float(min(f32(eps), f32(alpha) * np.exp(-ent)))


def typical_accept(row: np.ndarray, tok: int, temperature: float, eps: float, alpha: float) -> bool:
    if tok < 0 or tok >= np.asarray(row).size:
        return False
    prob, thr = typical_prob_thr(row, tok, temperature, eps, alpha)
    return bool(prob > thr)


def typical_walk(logits: np.ndarray, draft: Sequence[int], parent_ref: Sequence[int], pos: Sequence[int],
                 max_depth: int, temperature: float = 1.0, eps: float = 0.09,
                 alpha: float = 0.3) -> Tuple[List[int], List[int], int, int, int]:
    logits = np.asarray(logits)
    next_tokens = np.argmax(logits, axis=-1)
    draft = np.asarray(draft, dtype=np.int64)
    pe = parent_ext(parent_ref)
    ok = np.zeros(pe.size, dtype=bool)
    for i in range(1, pe.size):
        ok[i] = typical_accept(logits[pe[i]], int(draft[i]), temperature, eps, alpha)
    return _walk(ok, pe, np.asarray(pos, dtype=np.int64), max_depth, draft, next_tokens)


def brute_force_greedy(logits: np.ndarray, draft: Sequence[int], parent: Sequence[int],
                       pos: Sequence[int]) -> Tuple[List[int], int, int]:
    """Independent greedy acceptance from per-node parents (parent[0] = -1).

    Returns (path ids, accept_length, next_token); winner = deepest accepted
    position, lowest index on ties (pos >= 0 assumed).
    """
    nxt = np.argmax(np.asarray(logits), axis=-1)
    M = len(parent)
    best, best_pos = 0, None
    for i in range(M):
        node, good = i, True
        while node != 0:
            p = parent[node]
            if int(draft[node]) != int(nxt[p]):
                good = False
                break
            node = p
        if good and (best_pos is None or pos[i] > best_pos):
            best, best_pos = i, pos[i]
    path, node = [], best
    while node != -1:
        path.append(node)
        node = parent[node] if node != 0 else -1
    path.reverse()
    return path, len(path) - 1, int(nxt[best])


def kv_commit(cache: np.ndarray, start: int, path: Sequence[int]) -> np.ndarray:
    """draft/tree_verification.py:197-217 on one cache tensor [..., S, D]:
    select_indices = path + start; tgt = data[..., select_indices, :] (a new
    array); data[..., start:start + len(path), :] = tgt.  Returns a copy."""
    out = np.array(cache, copy=True)
    sel = np.asarray(path, dtype=np.int64) + int(start)
    tgt = out[..., sel, :].copy()
    out[..., int(start):int(start) + sel.size, :] = tgt
    return out
