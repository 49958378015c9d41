"""Seeded synthetic inputs of the tree-verification workloads.

The reference ships no datasets or checkpoints for this path; its benchmark
shapes are reproduced with generators whose every choice is fixed here, so
the GPU runs, the CPU oracle and the benchmark all see identical inputs.

Tree generator (node 0 is the root): node i draws its parent uniformly from
the nodes j in [max(0, i - window), i) whose out-degree is below
``max_outdeg`` and whose depth is below ``max_depth``; if none qualifies, the
nearest earlier qualifying node is used.  Parents therefore precede children
(the depth-sorted-parent property of runtime/draft_tree.py:234-236 that the
verification path relies on).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch


# ----------------------------------------------------------------------------
# Trees
# ----------------------------------------------------------------------------

def make_tree(M: int, max_depth: int = 8, max_outdeg: int = 4, window: int = 8,
              seed: int = 0) -> Tuple[List[int], List[int]]:
    """Return (parent, depth) lists of an M-node tree; parent[0] = -1."""
    rng = np.random.default_rng(seed)
    parent = [-1] * M
    depth = [0] * M
    outdeg = [0] * M
    for i in range(1, M):
        cand = [j for j in range(max(0, i - window), i) if outdeg[j] < max_outdeg and depth[j] < max_depth]
        if cand:
            p = cand[int(rng.integers(len(cand)))]
        else:
            p = next((j for j in range(i - 1, -1, -1) if outdeg[j] < max_outdeg and depth[j] < max_depth), None)
            if p is None:
                raise ValueError("tree capacity exhausted (raise max_outdeg or max_depth)")
        parent[i] = p
        depth[i] = depth[p] + 1
        outdeg[p] += 1
    return parent, depth


def parent_to_reference(parent: List[int]) -> List[int]:
    """Per-node parents -> verify_new's ``parent`` ([M-1], -1 = root child).

    Node k+1's parent among the non-root nodes is parent[k+1] - 1
    (draft/tree_verification.py:120-125 undoes exactly this shift).
    """
    return [parent[i] - 1 for i in range(1, len(parent))]


def ancestor_mask(parent: List[int]) -> np.ndarray:
    """[M, M] bool, mask[i, j] = j is i or an ancestor of i."""
    M = len(parent)
    mask = np.zeros((M, M), dtype=bool)
    for i in range(M):
        j, steps = i, 0
        while j >= 0 and steps <= M:
            mask[i, j] = True
            j = parent[j]
            steps += 1
    return mask


# ----------------------------------------------------------------------------
# Attention inputs
# ----------------------------------------------------------------------------

@dataclass
class TreeVerifyInputs:
    q: torch.Tensor            # [B, M, H, D]
    kv_pages: torch.Tensor     # [L, 2, P, Hk, page_size, D]
    page_table: torch.Tensor   # [n_pages] int32, logical -> physical
    n_prefix: int
    parent: List[int]
    depth: List[int]
    page_size: int

    @property
    def M(self) -> int:
        return self.q.shape[1]

    def logical_kv(self, layer: int = 0, kv: int = 0, n: Optional[int] = None) -> torch.Tensor:
        """Gather tokens [0, n) of one layer into [B=1, n, Hk, D] (contiguous)."""
        n = self.n_prefix + self.M if n is None else n
        ps = self.page_size
        tok = torch.arange(n, device=self.page_table.device)
        phys = self.page_table.long()[tok // ps]
        x = self.kv_pages[layer, kv][phys, :, tok % ps, :]  # [n, Hk, D]
        return x.unsqueeze(0)


def make_tree_verify_inputs(n_prefix: int, M: int, H: int = 32, Hk: int = 8, D: int = 128,
                            page_size: int = 16, layers: int = 1, dtype=torch.bfloat16,
                            scale: float = 0.5, seed: int = 0, tree_seed: int = 0, max_depth: int = 8,
                            max_outdeg: int = 4, device: str = "cuda") -> TreeVerifyInputs:
    """Single-layer paged tree verify inputs (batch 1).

    The pool holds ``layers`` independent layers so a benchmark can rotate
    through distinct KV sets.  Q and the pool are N(0, 1) * scale cast to
    ``dtype``; the page table is a seeded random permutation of the pages that
    hold tokens [0, n_prefix + M) (the tree's K/V follow the prefix).
    """
    n_tok = n_prefix + M
    n_pages = (n_tok + page_size - 1) // page_size
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    q = (torch.randn((1, M, H, D), generator=g, device=device) * scale).to(dtype)
    pool = torch.empty((layers, 2, n_pages, Hk, page_size, D), dtype=dtype, device=device)
    for l in range(layers):
        for kv in range(2):
            pool[l, kv] = (torch.randn((n_pages, Hk, page_size, D), generator=g, device=device) * scale).to(dtype)
    perm = np.random.default_rng(seed + 1).permutation(n_pages).astype(np.int32)
    pt = torch.from_numpy(perm).to(device)
    parent, depth = make_tree(M, max_depth=max_depth, max_outdeg=max_outdeg, seed=tree_seed)
    return TreeVerifyInputs(q=q, kv_pages=pool, page_table=pt, n_prefix=n_prefix, parent=parent, depth=depth,
                            page_size=page_size)


# ----------------------------------------------------------------------------
# Acceptance inputs
# ----------------------------------------------------------------------------

PLANT_VALUE = 20.0  # logit given to each node's planted top token


@dataclass
class AcceptInputs:
    logits: torch.Tensor     # [T, M, V]
    draft: torch.Tensor      # [T, M] int64
    parent_ref: torch.Tensor  # [T, M-1] int64 (verify_new convention)
    pos: torch.Tensor        # [T, M] int64
    parents: List[List[int]]
    depths: List[List[int]]
    planted_len: List[int]


def make_accept_inputs(T: int = 8, M: int = 64, V: int = 128256, dtype=torch.bfloat16, sigma: float = 3.0,
                       seed: int = 0, max_depth: int = 8, max_outdeg: int = 4, pos_offset: int = 0,
                       device: str = "cuda") -> AcceptInputs:
    """T independent trees with N(0, sigma) logits, a planted top token per
    node and a planted accepted path of seeded length 1..max_depth."""
    rng = np.random.default_rng(seed)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    logits = (torch.randn((T, M, V), generator=g, device=device) * sigma)
    top = torch.from_numpy(rng.integers(0, V, size=(T, M))).to(device)
    logits.scatter_(2, top.unsqueeze(-1), PLANT_VALUE)
    logits = logits.to(dtype)
    draft = rng.integers(0, V, size=(T, M))
    parents, depths, plens = [], [], []
    for t in range(T):
        parent, depth = make_tree(M, max_depth=max_depth, max_outdeg=max_outdeg, seed=seed * 1000 + t)
        want = int(rng.integers(1, max_depth + 1))
        cands = [i for i in range(M) if depth[i] == want] or [int(np.argmax(depth))]
        node = cands[int(rng.integers(len(cands)))]
        plens.append(depth[node])
        top_t = top[t].cpu().numpy()
        while node > 0:
            draft[t, node] = top_t[parent[node]]
            node = parent[node]
        parents.append(parent)
        depths.append(depth)
    pref = torch.tensor([parent_to_reference(p) for p in parents], dtype=torch.int64, device=device)
    pos = torch.tensor([[pos_offset + d for d in dep] for dep in depths], dtype=torch.int64, device=device)
    return AcceptInputs(logits=logits, draft=torch.from_numpy(draft).to(device), parent_ref=pref, pos=pos,
                        parents=parents, depths=depths, planted_len=plens)


# ----------------------------------------------------------------------------
# Llama-3.1-8B-shaped verification step
# ----------------------------------------------------------------------------

class LlamaVerifyStep:
    """One target-side verification step of a Llama-3.1-8B-shaped model over a
    draft tree, with seeded random weights (no checkpoint exists offline).

    Shape: ``layers`` decoder layers (32), hidden 4096, 32 query / 8 KV heads
    of 128, FFN 14336, vocab 128256, RoPE theta 5e5, bf16 weights N(0, 0.02).
    Every layer's K/V prefix (``n_prefix`` tokens) sits in a page pool behind
    a random-permutation page table; the tree's K/V follow it in the same
    pages.  The tree nodes' inputs are their draft tokens' embeddings.

    Per layer (llama_target_model.py:834-867 around the hot path): RMSNorm,
    QKV projection, RoPE of q and k at the nodes' positions with the tree K/V
    written into the pages (dsv_kv_append), the fused tree verify (kernels 1
    and 3), o_proj, RMSNorm, SwiGLU MLP; then the final norm and the lm_head
    with the greedy walk (draft/diffspec_model.py:229-231 and
    draft/tree_verification.py:100-182).  Projections, norms and the MLP are
    torch ops (hipBLASLt GEMMs): scaffolding around the hot path.
    """

    def __init__(self, n_prefix: int = 65536, M: int = 64, layers: int = 32, hidden: int = 4096, H: int = 32,
                 Hk: int = 8, D: int = 128, ffn: int = 14336, vocab: int = 128256, theta: float = 5e5,
                 seed: int = 5, device: str = "cuda"):
        self.N, self.M, self.L, self.hid, self.H, self.Hk, self.D, self.F, self.V = (
            n_prefix, M, layers, hidden, H, Hk, D, ffn, vocab)
        self.dev = device
        self.inp = make_tree_verify_inputs(n_prefix=n_prefix, M=M, H=H, Hk=Hk, D=D, layers=layers, device=device,
                                           seed=seed, tree_seed=seed)
        g = torch.Generator(device=device)
        g.manual_seed(seed)

        def w(*shape):
            return (torch.randn(shape, generator=g, device=device) * 0.02).to(torch.bfloat16)

        # nn.Linear weight layout [out_features, in_features], applied as x @ W.T
        self.layers = [dict(qkv=w((H + 2 * Hk) * D, hidden), o=w(hidden, H * D), gu=w(2 * ffn, hidden),
                            d=w(hidden, ffn)) for _ in range(layers)]
        self.lm_head = w(vocab, hidden)
        # token embeddings at the scale of a trained model's (unit-RMS rows)
        self.embed = w(vocab, hidden) * 50
        self.par = torch.tensor(self.inp.parent, dtype=torch.int64, device=device)
        self.pref = torch.tensor([parent_to_reference(self.inp.parent)], dtype=torch.int64, device=device)
        self.pos = torch.tensor([n_prefix + d for d in self.inp.depth], dtype=torch.int64, device=device)
        self.draft = torch.randint(0, vocab, (1, M), generator=g, device=device)
        inv = 1.0 / (theta ** (torch.arange(0, D, 2, device=device, dtype=torch.float32) / D))
        ang = self.pos.float()[:, None] * inv[None, :]
        self.cos = torch.cat([ang.cos(), ang.cos()], -1).to(torch.bfloat16)
        self.sin = torch.cat([ang.sin(), ang.sin()], -1).to(torch.bfloat16)
        self.max_hops = min(max(self.inp.depth) + 2, M)

    @staticmethod
    def rms(t: torch.Tensor) -> torch.Tensor:
        tf = t.float()
        return (tf * torch.rsqrt(tf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(torch.bfloat16)

    def hidden(self, capture: Sequence[int] = (), verify_hook=None
               ) -> Tuple[torch.Tensor, Dict[int, Tuple[torch.Tensor, torch.Tensor]]]:
        """The 32 layers over the tree; returns the final normed hidden states
        [M, hidden] and, for the layers in ``capture``, (rotated q [M, H, D],
        attention output [M, H, D]).  ``verify_hook(layer, phase)``, when
        given, is called right before (phase 0) and right after (phase 1)
        each layer's fused tree verify (a measurement hook)."""
        from .runtime.cache_state import append_tree_kv
        from .runtime.tree_attention import tree_verify

        M, H, Hk, D, F, N = self.M, self.H, self.Hk, self.D, self.F, self.N
        inp = self.inp
        caps = {}
        x = self.embed[self.draft[0]]
        for l in range(self.L):
            W = self.layers[l]
            qkv = self.rms(x) @ W["qkv"].T
            q = append_tree_kv(qkv[:, H * D:(H + Hk) * D].view(M, Hk, D), qkv[:, (H + Hk) * D:].view(M, Hk, D),
                               inp.kv_pages[l, 0], inp.kv_pages[l, 1], N, cos=self.cos, sin=self.sin,
                               page_table=inp.page_table, q=qkv[:, :H * D].view(M, H, D))
            if verify_hook is not None:
                verify_hook(l, 0)
            o, _ = tree_verify(q.unsqueeze(0), inp.kv_pages[l, 0], inp.kv_pages[l, 1], N, self.par,
                               page_table=inp.page_table)
            if verify_hook is not None:
                verify_hook(l, 1)
            if l in capture:
                caps[l] = (q.clone(), o[0].clone())
            x = x + o.view(M, H * D) @ W["o"].T
            gu = self.rms(x) @ W["gu"].T
            x = x + (torch.nn.functional.silu(gu[:, :F].float()) * gu[:, F:].float()).to(torch.bfloat16) @ W["d"].T
        return self.rms(x), caps

    def step(self, verify_hook=None) -> Dict[str, torch.Tensor]:
        """The whole verification step: layers, then the lm_head fused with the
        greedy walk (kernel 5 + kernel 4's walk)."""
        from .draft.tree_verification import lmhead_tree_accept

        xn, _ = self.hidden(verify_hook=verify_hook)
        return lmhead_tree_accept(xn.unsqueeze(0), self.lm_head, self.draft, self.pref, self.pos, self.max_hops)

    def torch_logits(self, xn: torch.Tensor) -> torch.Tensor:
        """The reference's bf16 lm_head logits [1, M, V] (nn.Linear: x @ W.T)."""
        return (xn @ self.lm_head.T).unsqueeze(0)

    def plant_path(self, node: Optional[int] = None) -> List[int]:
        """Make the draft agree with the target along the root path of ``node``
        (default: the first deepest node), top-down: the token of each path
        node becomes the argmax of torch's logits at its parent, whose hidden
        state depends only on tokens already fixed.  One pass of the layers per
        edge.  Returns the path (root first)."""
        if node is None:
            node = int(np.argmax(self.inp.depth))
        path = [node]
        while path[-1] > 0:
            path.append(self.inp.parent[path[-1]])
        path.reverse()
        for par, child in zip(path[:-1], path[1:]):
            xn, _ = self.hidden()
            self.draft[0, child] = int(torch.argmax(self.torch_logits(xn)[0, par].float()))
        return path
