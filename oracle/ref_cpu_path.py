"""The reference's PyTorch CPU path of one verification step (oracle / CPU baseline).

Test infrastructure only (see oracle/__init__.py).  Restates, op for op, what
the reference runs when no GPU kernel is available, so that it can be timed
on the host cores as the CPU baseline and cross-checked against the float64
closed forms:

  repeat_kv                        llama_target_model.py:543-560 (applied :795-796)
  prefix attention (fallback)      runtime/tree_attention.py:439-446
  tree attention (naive)           runtime/tree_attention.py:40-63
  merge                            llama_target_model.py:862-866
  greedy acceptance walk           draft/tree_verification.py:100-182
"""

from __future__ import annotations

import math

import torch


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[B, Hk, L, D] -> [B, Hk * n_rep, L, D] (materialised copy)."""
    b, hk, l, d = x.shape
    if n_rep == 1:
        return x
    return x[:, :, None, :, :].expand(b, hk, n_rep, l, d).reshape(b, hk * n_rep, l, d)


def prefix_attention_cpu(q, k, v):
    """q [B, M, H, D], k/v [B, N, H, D] -> out [B, M, H, D] (v dtype), lse [B, H, M] f32."""
    scale = 1.0 / math.sqrt(q.shape[-1])
    qh = q.transpose(1, 2).float()
    kh = k.transpose(1, 2).float()
    vh = v.transpose(1, 2)
    scores = torch.matmul(qh, kh.transpose(-2, -1)) * scale
    weights = torch.softmax(scores, dim=-1).to(v.dtype)
    out = torch.matmul(weights, vh).transpose(1, 2)
    lse = torch.logsumexp(scores, dim=-1)
    return out, lse


def tree_attention_naive(q, k, v, tree_mask, prefix_lse, bsz, q_len, num_heads, hidden_dim):
    """Additive tree mask [B, 1, T, T] -> (current_out [B, M, H, D], weight [B, M, H, 1])."""
    keep = (tree_mask[:, :, -q_len:, -q_len:] == 0).to(torch.int8)
    scale = 1.0 / math.sqrt(hidden_dim)
    qh = q.transpose(1, 2)
    kh = k.permute(0, 2, 3, 1)
    vh = v.transpose(1, 2)
    s = (torch.matmul(qh, kh) * scale).to(torch.float32)
    s = s.masked_fill(keep.expand(-1, num_heads, -1, -1) == 0, -float("inf"))
    w_att = torch.softmax(s, dim=-1).to(qh.dtype)
    cur = torch.matmul(w_att, vh).permute(0, 2, 1, 3)
    lse_t = s.logsumexp(dim=-1, keepdim=True).transpose(1, 2)
    plse = prefix_lse.reshape(bsz, num_heads, q_len, -1).transpose(1, 2)
    weight = torch.sigmoid(plse - lse_t).to(qh.dtype)
    return cur, weight


def additive_tree_mask(keep: torch.Tensor) -> torch.Tensor:
    """[M, M] keep-bool -> [1, 1, M, M] float additive mask (llama_target_model.py:1325-1330)."""
    m = torch.zeros(keep.shape, dtype=torch.float32)
    m.masked_fill_(~keep, torch.finfo(torch.float32).min)
    return m[None, None]


def hybrid_verify_cpu(q, k_cache, v_cache, cache_len: int, tree_mask_add):
    """One layer's hybrid verify attention as the reference does it on CPU.

    q [B, M, H, D]; k_cache/v_cache [B, Hk, L, D] with the tree K/V at
    [cache_len, cache_len + M); tree_mask_add [B, 1, M, M] additive.
    Returns out [B, M, H, D].
    """
    B, M, H, D = q.shape
    n_rep = H // k_cache.shape[1]
    k = repeat_kv(k_cache[:, :, :cache_len + M], n_rep).transpose(1, 2)
    v = repeat_kv(v_cache[:, :, :cache_len + M], n_rep).transpose(1, 2)
    p_o, p_lse = prefix_attention_cpu(q, k[:, :cache_len], v[:, :cache_len])
    cur, w = tree_attention_naive(q, k[:, cache_len:], v[:, cache_len:], tree_mask_add, p_lse, B, M, H, D)
    out = cur * (1.0 - w) + p_o.to(cur.dtype) * w
    return out


def greedy_walk_torch(logits, draft, parent, position_ids, max_depth):
    """draft/tree_verification.py:100-182 with torch CPU ops.

    logits [1, M, V]; draft [1, M]; parent [M-1]; position_ids [M].
    Returns (best_candidate, best_candidate_id, accept_length, next_token, max_id).
    """
    next_tokens = torch.argmax(logits, dim=-1)
    par = parent.clone()
    rows = torch.arange(par.numel(), dtype=par.dtype)
    par = torch.where(par == rows, torch.full_like(par, -1), par)
    pe = torch.cat([torch.zeros(1, dtype=par.dtype), par + 1])
    ok = draft[0].eq(next_tokens[0].index_select(0, pe))
    ok[0] = True
    for _ in range(min(int(max_depth) + 2, int(pe.numel()))):
        nxt = ok & ok.index_select(0, pe)
        if torch.equal(nxt, ok):
            break
        ok = nxt
    max_id = int(torch.argmax(torch.where(ok, position_ids, torch.zeros_like(position_ids))).item())
    back = pe.tolist()
    back[0] = -1
    ids, cur = [], max_id
    while cur != -1:
        ids.append(cur)
        cur = back[cur]
    ids.reverse()
    toks = [int(draft[0, i]) for i in ids]
    return toks, ids, len(ids) - 1, int(next_tokens[0, max_id]), max_id
