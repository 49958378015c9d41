"""Tree acceptance on MI355X: the verify_new contract with a gfx950 acceptance kernel.

Drop-in for ``verify`` / ``verify_new`` of the reference's
``diffspec/draft/tree_verification.py`` (:66-257).  Lines :100-182 of the
reference — per-node argmax, the ancestor closure, the deepest-node winner,
the traceback and the next token — run in kernel 4 (libdsv.so), which
returns the accepted path, its tokens and the next token in one small
device buffer, read back with a single device-to-host copy instead of the
reference's four (:112-118).  The remainder of verify_new (hazard tracker,
tree budget, KV compaction, next-tree construction by the draft model, root
prepend) follows the reference.

Acceptance modes:
  * ``greedy`` — the reference rule (``logits_processor is None``).
  * ``sample`` — the reference's sampling branch (``logits_processor`` given,
    :103-106): the warpers of ``prepare_logits_processor`` (:15-32;
    temperature, top-p, top-k), one draw per node from softmax of the warped
    logits, then the same walk.  The draw is a seeded counter-based
    Gumbel-max (libdsv's dsv_tree_accept_sample) instead of
    ``torch.multinomial``: same distribution, reproducible from its seed,
    which ``verify_new`` takes from torch's default generator (so
    ``torch.manual_seed`` fixes it, as it fixes the reference's draws).
  * ``typical`` — posterior (typical) acceptance of Cai et al. 2024 (Medusa):
    accept node i iff p_T(draft[i] | parent) > min(eps, alpha * exp(-H)),
    with H the entropy of p_T(. | parent); the reference has no such mode.
"""

from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch

from .. import _ext
from ..core.bundle_scheduler import BundleScheduler

__all__ = ["tree_accept", "evaluate_tree", "kv_commit", "verify", "verify_new", "prepare_logits_processor",
           "SamplingParams"]


class SamplingParams:
    """The warpers of the reference's sampling branch: temperature, then top-p,
    then top-k (prepare_logits_processor, draft/tree_verification.py:15-32)."""

    def __init__(self, temperature: float = 1.0, top_p: float = 1.0, top_k: int = 0):
        self.temperature, self.top_p, self.top_k = float(temperature), float(top_p), int(top_k)

    def __repr__(self) -> str:
        return f"SamplingParams(temperature={self.temperature}, top_p={self.top_p}, top_k={self.top_k})"


def prepare_logits_processor(temperature: float = 0.0, repetition_penalty: float = 0.0, top_p: float = 0.0,
                             top_k: int = 0) -> Optional[SamplingParams]:
    """Mirror of the reference's prepare_logits_processor (:15-32): None (greedy)
    for temperature <= 1e-5, else the warpers to apply.  The repetition penalty
    is refused: the reference's only call (:104) passes input_ids=None, which
    RepetitionPenaltyLogitsProcessor cannot take."""
    if temperature > 1e-5:
        if repetition_penalty > 1.0:
            raise NotImplementedError("the repetition penalty needs the input ids, which verify_new does not pass")
        return SamplingParams(temperature=temperature if temperature != 1.0 else 1.0,
                              top_p=top_p if 1e-8 <= top_p < 1.0 else 1.0, top_k=top_k if top_k > 0 else 0)
    return None


def _sampling_params(logits_processor) -> SamplingParams:
    """SamplingParams from this module's prepare_logits_processor or from the
    transformers LogitsProcessorList the reference builds (temperature, top-p,
    top-k warpers in that order)."""
    if isinstance(logits_processor, SamplingParams):
        return logits_processor
    T, p, k, rank = 1.0, 1.0, 0, -1
    order = {"TemperatureLogitsWarper": 0, "TopPLogitsWarper": 1, "TopKLogitsWarper": 2}
    for proc in logits_processor:
        name = type(proc).__name__
        if name not in order:
            raise NotImplementedError(f"{name} is not supported by the sampling acceptance kernel")
        if order[name] <= rank:
            raise NotImplementedError("the warpers must come in the order temperature, top-p, top-k")
        rank = order[name]
        if getattr(proc, "min_tokens_to_keep", 1) != 1 or getattr(proc, "filter_value", float("-inf")) != float("-inf"):
            raise NotImplementedError(f"{name}: only min_tokens_to_keep=1 and filter_value=-inf are supported")
        if name == "TemperatureLogitsWarper":
            T = float(proc.temperature)
        elif name == "TopPLogitsWarper":
            p = float(proc.top_p)
        else:
            k = int(proc.top_k)
    return SamplingParams(T, p, k)


def tree_accept(logits: torch.Tensor, draft: torch.Tensor, parent: torch.Tensor, pos: torch.Tensor,
                max_hops: int, mode: str = "greedy", temperature: float = 1.0,
                posterior_threshold: float = 0.09, posterior_alpha: float = 0.3,
                return_next: bool = False, top_p: float = 1.0, top_k: int = 0,
                seed: int = 0) -> Dict[str, torch.Tensor]:
    """Batched acceptance of T independent trees (kernel 4).

    ``mode`` is "greedy", "typical" or "sample" (temperature, top_p, top_k and
    the 64-bit ``seed`` of the counter-based draw; ``next`` then holds the
    per-node draws).

    Args:
        logits: [T, M, V] (or [M, V]) bf16/f16/f32 target logits per node.
        draft: [T, M] int64 draft token per node (node 0 = root).
        parent: [T, M-1] int64, reference convention (parent[k] is the parent
            of node k+1 among non-root nodes; -1 or k itself = the root).
        pos: [T, M] or [M] int64 position ids.
        max_hops: closure rounds; the reference uses min(max_depth + 2, M).
    Returns:
        dict of device tensors: ``path`` [T, M] (node ids root..winner, then -1),
        ``tokens`` [T, M], ``info`` [T, 4] = (winner, accept_length, next_token,
        path_len or -1 on a malformed tree) and, if asked, ``next`` [T, M].
    """
    if logits.dim() == 2:
        logits = logits.unsqueeze(0)
    if draft.dim() == 1:
        draft = draft.unsqueeze(0)
    if parent.dim() == 1:
        parent = parent.unsqueeze(0)
    dev = _ext.require_gpu(logits, draft, parent, pos)
    T, M, V = logits.shape
    if draft.dtype != torch.int64:
        draft = draft.to(torch.int64)
    if parent.dtype != torch.int64:
        parent = parent.to(torch.int64)
    if pos.dtype != torch.int64:
        pos = pos.to(torch.int64)
    lib = _ext.load()
    path = torch.empty((T, M), dtype=torch.int64, device=dev)
    tokens = torch.empty((T, M), dtype=torch.int64, device=dev)
    info = torch.empty((T, 4), dtype=torch.int64, device=dev)
    nxt = torch.empty((T, M), dtype=torch.int64, device=dev) if return_next else None
    ws = _ext.workspace(lib.dsv_accept_workspace_bytes(T, M, V), dev)
    if mode == "sample":
        rc = lib.dsv_tree_accept_sample(_ext.desc(logits), _ext.desc(draft), _ext.desc(parent), _ext.desc(pos),
                                        int(max_hops), float(temperature), float(top_p), int(top_k),
                                        int(seed) & 0xFFFFFFFFFFFFFFFF, _ext.desc(path), _ext.desc(tokens),
                                        _ext.desc(info), _ext.desc(nxt), ws.data_ptr(), ws.numel(),
                                        _ext.stream_of(dev))
    else:
        mode_id = {"greedy": _ext.ACCEPT_GREEDY, "typical": _ext.ACCEPT_TYPICAL}[mode]
        rc = lib.dsv_tree_accept(mode_id, _ext.desc(logits), _ext.desc(draft), _ext.desc(parent), _ext.desc(pos),
                                 int(max_hops), float(temperature), float(posterior_threshold),
                                 float(posterior_alpha), _ext.desc(path), _ext.desc(tokens), _ext.desc(info),
                                 _ext.desc(nxt), ws.data_ptr(), ws.numel(), _ext.stream_of(dev))
    _ext.check(rc, "tree_accept")
    out = {"path": path, "tokens": tokens, "info": info}
    if return_next:
        out["next"] = nxt
    return out


def lmhead_tree_accept(hidden: torch.Tensor, weight: torch.Tensor, draft: torch.Tensor, parent: torch.Tensor,
                       pos: torch.Tensor, max_hops: int, mode: str = "greedy", temperature: float = 1.0,
                       posterior_threshold: float = 0.09, posterior_alpha: float = 0.3,
                       return_next: bool = False, return_logits: bool = False) -> Dict[str, torch.Tensor]:
    """lm_head fused with the acceptance of T trees (kernel 5 + kernel 4's walk).

    Same results as ``tree_accept(lm_head(hidden), ...)`` with bf16 logits
    (the reference's ``self.base_model.lm_head`` output, draft/diffspec_model.py:229-231,
    walked by draft/tree_verification.py:100-182), without writing the
    ``[T, M, V]`` logits to memory.

    Args:
        hidden: [T, M, Dm] or [M, Dm] bf16 final hidden states of the tree nodes
            (after the final norm); Dm a multiple of 64.
        weight: [V, Dm] bf16 lm_head weight (``nn.Linear.weight``).
        draft, parent, pos, max_hops, mode, ...: as :func:`tree_accept`.
        return_logits: also write the bf16 logits ``[T, M, V]`` (returned as ``logits``).
    """
    if hidden.dim() == 2:
        hidden = hidden.unsqueeze(0)
    if draft.dim() == 1:
        draft = draft.unsqueeze(0)
    if parent.dim() == 1:
        parent = parent.unsqueeze(0)
    dev = _ext.require_gpu(hidden, weight, draft, parent, pos)
    T, M, _ = hidden.shape
    V = weight.shape[0]
    if draft.dtype != torch.int64:
        draft = draft.to(torch.int64)
    if parent.dtype != torch.int64:
        parent = parent.to(torch.int64)
    if pos.dtype != torch.int64:
        pos = pos.to(torch.int64)
    mode_id = {"greedy": _ext.ACCEPT_GREEDY, "typical": _ext.ACCEPT_TYPICAL}[mode]
    lib = _ext.load()
    path = torch.empty((T, M), dtype=torch.int64, device=dev)
    tokens = torch.empty((T, M), dtype=torch.int64, device=dev)
    info = torch.empty((T, 4), dtype=torch.int64, device=dev)
    nxt = torch.empty((T, M), dtype=torch.int64, device=dev) if return_next else None
    logits = torch.empty((T, M, V), dtype=torch.bfloat16, device=dev) if return_logits else None
    ws = _ext.workspace(lib.dsv_lmhead_accept_workspace_bytes(T, M, V), dev)
    rc = lib.dsv_lmhead_accept(mode_id, _ext.desc(hidden), _ext.desc(weight), _ext.desc(draft), _ext.desc(parent),
                               _ext.desc(pos), int(max_hops), float(temperature), float(posterior_threshold),
                               float(posterior_alpha), _ext.desc(path), _ext.desc(tokens), _ext.desc(info),
                               _ext.desc(nxt), _ext.desc(logits), ws.data_ptr(), ws.numel(), _ext.stream_of(dev))
    _ext.check(rc, "lmhead_tree_accept")
    out = {"path": path, "tokens": tokens, "info": info}
    if return_next:
        out["next"] = nxt
    if return_logits:
        out["logits"] = logits
    return out


def kv_commit(kv: torch.Tensor, start: int, path: torch.Tensor, info: torch.Tensor,
              page_table: Optional[torch.Tensor] = None, tree: int = 0) -> None:
    """Accepted-path KV commit on the GPU (reference draft/tree_verification.py:197-217).

    Tokens [start, start + n) of every row of ``kv`` receive tokens
    start + path[0..n), n = info[3], every read before any write (the
    reference's ``data[..., start:start+n, :] = data[..., start + path, :]``).
    ``path`` / ``info`` are the device outputs of :func:`tree_accept`
    (``[T, M]`` / ``[T, 4]``, or one tree's rows), so no host round trip is
    needed.  ``kv`` is a page pool ``[L, 2, P, Hk, page, D]`` with
    ``page_table``, or a dense cache ``[..., S, D]`` (1..4 leading dims);
    bf16/f16/f32 with 16-byte token rows.
    """
    _ext.require_gpu(kv, path, info)
    lib = _ext.load()
    rc = lib.dsv_kv_commit(_ext.desc(kv), _ext.desc(page_table), int(start), _ext.desc(path), _ext.desc(info),
                           int(tree), _ext.stream_of(kv.device))
    _ext.check(rc, "kv_commit")


# Bytes of tree rows the commit kernel stages per cache row (dsv_kv_commit:
# M * row bytes <= 256 threads x 16 chunks x 16 bytes).
KV_COMMIT_MAX_TREE_BYTES = 256 * 16 * 16


def _kv_commit_ok(t: torch.Tensor, M: int) -> bool:
    """Whether the commit kernel takes this dense cache tensor as it is, for an M-node tree."""
    es = t.element_size()
    return (t.is_cuda and t.dtype in (torch.bfloat16, torch.float16, torch.float32) and 3 <= t.dim() <= 6
            and t.stride(-1) == 1 and (t.shape[-1] * es) % 16 == 0 and t.data_ptr() % 16 == 0
            and all((st * es) % 16 == 0 for st in t.stride()[:-1])
            and M * t.shape[-1] * es <= KV_COMMIT_MAX_TREE_BYTES)


def _evaluate_tree_dev(logits, draft, parent, position_ids, max_depth, mode, temperature, posterior_threshold,
                       posterior_alpha, top_p=1.0, top_k=0, seed=0):
    M = draft.shape[-1]
    pos = position_ids[0] if position_ids.dim() == 2 else position_ids
    max_hops = min(int(max_depth) + 2, M)
    r = tree_accept(logits.reshape(1, M, -1), draft.reshape(1, M), parent.reshape(1, M - 1), pos, max_hops,
                    mode=mode, temperature=temperature, posterior_threshold=posterior_threshold,
                    posterior_alpha=posterior_alpha, top_p=top_p, top_k=top_k, seed=seed)
    host = torch.cat([r["info"], r["path"], r["tokens"]], dim=1).cpu()[0].tolist()
    winner, accept_length, _, plen = host[:4]
    if plen < 0:
        raise RuntimeError("malformed draft tree: the parent chain does not reach the root")
    ids = host[4:4 + plen]
    toks = host[4 + M:4 + M + plen]
    next_token = r["info"][:, 2:3]
    return (toks, ids, int(accept_length), next_token, int(winner)), r


def evaluate_tree(logits: torch.Tensor, draft: torch.Tensor, parent: torch.Tensor, position_ids: torch.Tensor,
                  max_depth: int, mode: str = "greedy", temperature: float = 1.0,
                  posterior_threshold: float = 0.09,
                  posterior_alpha: float = 0.3) -> Tuple[list, list, int, torch.Tensor, int]:
    """Lines :100-182 of verify_new for one tree.

    Returns (best_candidate tokens, best_candidate node ids, accept_length,
    next_token [1, 1] on the device, max_id).
    """
    return _evaluate_tree_dev(logits, draft, parent, position_ids, max_depth, mode, temperature,
                              posterior_threshold, posterior_alpha)[0]


def verify(input_ids, logits, draft, position_ids, hidden_states, tree_attention_mask, past_key_values_data,
           current_length_data, parent, model, nodes, threshold, max_depth, logits_processor, hazard_tracker=None):
    """Redirects to verify_new (reference :66-72)."""
    return verify_new(input_ids, logits, draft, position_ids, hidden_states, tree_attention_mask,
                      past_key_values_data, current_length_data, parent, model, nodes, threshold, max_depth,
                      logits_processor, hazard_tracker)


@torch.no_grad()
def verify_new(input_ids, logits, draft, position_ids, hidden_states, tree_attention_mask, past_key_values_data,
               current_length_data, parent, model, nodes, threshold, max_depth, logits_processor,
               hazard_tracker=None, acceptance: str = "greedy", temperature: float = 1.0,
               posterior_threshold: float = 0.09, posterior_alpha: float = 0.3, sample_seed: Optional[int] = None):
    """Verify the draft tree and advance the generation state (reference :76-257).

    With ``logits_processor`` (this module's ``prepare_logits_processor`` or
    the reference's transformers warper list) the draw per node is sampled
    (mode "sample"); its seed is ``sample_seed`` or, by default, one draw from
    torch's default generator.

    Returns (input_ids, best_candidate, accept_length, next_draft,
    next_position_ids, next_tree_attention_mask, next_parent).
    """
    top_p, top_k, seed = 1.0, 0, 0
    if logits_processor is not None:
        sp = _sampling_params(logits_processor)
        acceptance, temperature, top_p, top_k = "sample", sp.temperature, sp.top_p, sp.top_k
        seed = int(sample_seed) if sample_seed is not None else int(torch.randint(0, 2 ** 62, (1,)).item())

    # 1-2. Acceptance walk on the GPU (reference :100-182).
    (best_candidate, best_candidate_id, accept_length, next_token, max_id), acc = _evaluate_tree_dev(
        logits, draft, parent, position_ids, max_depth, acceptance, temperature, posterior_threshold,
        posterior_alpha, top_p, top_k, seed)
    next_token = next_token.to(draft.device)
    pos_all = position_ids[0] if position_ids.dim() == 2 else position_ids

    if getattr(model.draft_model, "enable_bundle_scheduling", False):
        scheduler = getattr(model.draft_model, "bundle_scheduler", None)
        if scheduler is None:
            scheduler = BundleScheduler(bundle_size=3, max_bundles=100, device=str(draft.device))
            model.draft_model.bundle_scheduler = scheduler
        par = parent.detach().to("cpu").tolist()
        parent_map = {0: -1}
        for k, p in enumerate(par):
            parent_map[k + 1] = (-1 if p == k else p) + 1
        children = set(parent_map.values()) - {-1}
        leaf_ids = [i for i in range(len(par) + 1) if i not in children]
        pos_cpu = pos_all.detach().to("cpu").tolist()
        depth_map = {i: int(pos_cpu[i]) for i in range(len(pos_cpu))}
        bundles = scheduler.schedule_bundles({"leaf_ids": leaf_ids, "parent_map": parent_map,
                                              "depth_map": depth_map}, return_tensors=False)
        model.draft_model.last_bundle_stats = {"num_leaves": len(leaf_ids), "num_bundles": len(bundles),
                                               "avg_prefix_length": scheduler.avg_prefix_length}

    if hazard_tracker is not None:
        observed_tree_depth = int(max(0, int((pos_all.max() - pos_all[0]).item())))
        first_reject_depth = -1 if accept_length >= observed_tree_depth else int(accept_length)
        hazard_tracker.update(first_reject_depth)

    budget_controller = getattr(model, "tree_budget_controller", None)
    next_nodes = int(nodes)
    if budget_controller is not None:
        next_nodes = budget_controller.observe(int(accept_length))
    model.draft_model.last_tree_node_budget = next_nodes

    # 3. Compact the accepted KV rows and update the cache length (reference :197-217).
    start = int(current_length_data[0].item()) - int(draft.size(1))
    select_indices = torch.tensor(best_candidate_id, device=input_ids.device, dtype=torch.long) + start
    if getattr(model.draft_model, "use_retrieval_cache", False) and getattr(model.draft_model,
                                                                             "retrieval_condition", False):
        prev_input_len = input_ids.shape[1]
        last_query_index = best_candidate_id[-1]
        last_attn_scores = model.draft_model.attn_scores[:, :, last_query_index, :].mean(dim=1).squeeze()
        abs_ids = torch.tensor(best_candidate_id, device=last_attn_scores.device) + prev_input_len
        model.draft_model.attn_scores_final = torch.cat(
            (last_attn_scores[:prev_input_len], last_attn_scores[abs_ids]), dim=0)
    n_sel = len(best_candidate_id)
    # Cache tensors the commit kernel takes are compacted on the GPU from the
    # walk's device-side path; other layouts take the reference's gather + copy.
    for data in past_key_values_data:
        if (_kv_commit_ok(data, int(draft.size(1))) and start + int(draft.size(1)) <= data.shape[-2]
                and data.device == acc["path"].device):
            kv_commit(data, start, acc["path"], acc["info"])
        else:
            tgt = data[..., select_indices.to(data.device), :]
            data[..., start:start + n_sel, :].copy_(tgt, non_blocking=True)
    current_length_data.fill_(start + n_sel)

    # 4. Append the accepted path and build the next draft tree (reference :219-257).
    input_ids = torch.cat(
        [input_ids, torch.tensor(best_candidate, device=input_ids.device, dtype=input_ids.dtype).unsqueeze(0)],
        dim=-1)
    new_accept_hidden = hidden_states[:, torch.tensor(best_candidate_id, device=hidden_states.device), :]
    next_draft, next_position_ids, next_tree_attention_mask, next_parent = model.draft_model.build_speculative_tree(
        new_accept_hidden, input_ids=torch.cat((input_ids, next_token.to(input_ids.device)), dim=1),
        head=model.base_model.lm_head, nodes=next_nodes, threshold=threshold, max_depth=max_depth)
    next_draft = torch.cat([next_token.to(next_draft.device), next_draft], dim=-1)
    root_pos_val = (pos_all[max_id] + 1).to(next_position_ids.device)
    next_position_ids = torch.cat([root_pos_val.view(1), next_position_ids], dim=-1)
    m = next_tree_attention_mask
    m = torch.cat([torch.zeros(1, m.size(1), dtype=m.dtype, device=m.device), m], dim=0)
    m = torch.cat([torch.ones(m.size(0), 1, dtype=m.dtype, device=m.device), m], dim=1)
    return input_ids, best_candidate, accept_length, next_draft, next_position_ids, m, next_parent
