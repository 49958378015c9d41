"""GPU parity of the lm_head fused with the acceptance (dsv_lmhead_accept).

* logits: the fused kernel's bf16 logits (written on request) against the
  fp64 oracle h . W^T rounded to bf16: within one bf16 step of the exactly
  rounded value (fp32 accumulation), and equal for nearly all entries;
* statistics and walk: bit-exact against kernel 4 run over those same logits
  (greedy: argmax per node, path, tokens, info; typical: the same on seeded
  cases), and next tokens equal to torch.argmax of those logits."""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from diffspec_mi355x import workloads as wl
from diffspec_mi355x.draft.tree_verification import lmhead_tree_accept, tree_accept

pytestmark = pytest.mark.gpu


def _case(gpu, T, M, Dm, V, seed, sigma=0.1, max_depth=6):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn((T, M, Dm), generator=g).to(torch.bfloat16).to(gpu)
    w = (torch.randn((V, Dm), generator=g) * sigma).to(torch.bfloat16).to(gpu)
    rng = np.random.default_rng(seed)
    parents, depths = [], []
    for t in range(T):
        p, d = wl.make_tree(M, max_depth=max_depth, max_outdeg=4, seed=seed * 10 + t)
        parents.append(p)
        depths.append(d)
    # plant a path of argmax tokens (torch fp32 logits) so that walks accept
    ref = (h.float() @ w.float().T).argmax(-1).cpu().numpy()
    draft = rng.integers(0, V, size=(T, M))
    for t in range(T):
        node = int(np.argmax(depths[t]))
        while node > 0:
            draft[t, node] = ref[t, parents[t][node]]
            node = parents[t][node]
    pref = torch.tensor([wl.parent_to_reference(p) for p in parents], dtype=torch.int64, device=gpu)
    pos = torch.tensor([[100 + x for x in d] for d in depths], dtype=torch.int64, device=gpu)
    return h, w, torch.from_numpy(draft).to(gpu), pref, pos, max_depth


def _check_logits(h, w, lg):
    hd, wd = h.double().cpu().numpy(), w.double().cpu().numpy()
    exact = hd @ wd.T
    want = oa.bf16_round(exact.astype(np.float32))
    got = lg.float().cpu().numpy()
    # one bf16 step (8 significant bits) at the larger magnitude, plus the
    # fp32 accumulation error sqrt(Dm) * 2^-24 * sum |h w| (x4), which
    # matters where the sum cancels to a small value
    mag = np.maximum(np.maximum(np.abs(got), np.abs(want)), 1e-30)
    ulp = np.exp2(np.floor(np.log2(mag)) - 7)
    acc = 4 * np.sqrt(hd.shape[1]) * 2.0 ** -24 * (np.abs(hd) @ np.abs(wd).T)
    diff = np.abs(got - want)
    assert np.all(diff <= ulp + acc), float((diff / (ulp + acc)).max())
    assert np.mean(diff == 0) > 0.98


@pytest.mark.parametrize("T,M,Dm,V", [(1, 64, 512, 5000), (2, 20, 128, 1000), (3, 40, 256, 3000), (1, 1, 64, 300),
                                       (1, 5, 192, 700), (2, 3, 320, 260)])
@pytest.mark.parametrize("mode", ["greedy", "typical"])
def test_fused_matches_kernel4_on_its_logits(gpu, T, M, Dm, V, mode):
    print(f"[lmhead] T={T} M={M} Dm={Dm} V={V} mode={mode}", flush=True)
    h, w, draft, pref, pos, md = _case(gpu, T, M, Dm, V, seed=T * 7 + M)
    hops = min(md + 2, M)
    r = lmhead_tree_accept(h, w, draft, pref, pos, hops, mode=mode, return_next=True, return_logits=True)
    torch.cuda.synchronize()
    lg = r["logits"]
    _check_logits(h.reshape(T * M, Dm), w, lg.reshape(T * M, V))
    ref = tree_accept(lg, draft, pref, pos, hops, mode=mode, return_next=True)
    torch.cuda.synchronize()
    assert torch.equal(r["next"], ref["next"])
    assert torch.equal(r["next"], lg.argmax(-1))
    assert torch.equal(r["info"], ref["info"])
    assert torch.equal(r["path"], ref["path"]) and torch.equal(r["tokens"], ref["tokens"])
    if M > 1:
        assert int(r["info"][:, 1].max()) >= 1   # the planted paths are (at least partly) accepted


def test_fused_random_shapes(gpu):
    """20 random fused lm_head calls: 1-3 trees of 1 to 100 nodes, hidden
    sizes 64 to 1024, vocabularies of 1 to 20000 (around the 256-row slices),
    greedy and typical; the written logits within one bf16 step of fp64, the
    walk and next tokens bit-exact against kernel 4 on those logits."""
    rng = np.random.default_rng(92)
    for case in range(20):
        T = int(rng.integers(1, 4))
        M = int(rng.choice([1, 2, 7, 33, 64, 100]))
        Dm = int(rng.choice([64, 128, 192, 256, 320, 512, 1024]))
        V = int(rng.choice([1, 2, 255, 256, 257, 1000, 5000, 20000]))
        mode = "greedy" if rng.integers(2) == 0 else "typical"
        print(f"[lmhead random] case {case}: T={T} M={M} Dm={Dm} V={V} {mode}", flush=True)
        h, w, draft, pref, pos, md = _case(gpu, T, M, Dm, V, seed=900 + case)
        hops = min(md + 2, M)
        r = lmhead_tree_accept(h, w, draft, pref, pos, hops, mode=mode, return_next=True, return_logits=True)
        torch.cuda.synchronize()
        lg = r["logits"]
        _check_logits(h.reshape(T * M, Dm), w, lg.reshape(T * M, V))
        ref = tree_accept(lg, draft, pref, pos, hops, mode=mode, return_next=True)
        torch.cuda.synchronize()
        assert torch.equal(r["next"], ref["next"]) and torch.equal(r["next"], lg.argmax(-1))
        assert torch.equal(r["info"], ref["info"])
        assert torch.equal(r["path"], ref["path"]) and torch.equal(r["tokens"], ref["tokens"])


def test_without_logits_output_and_llama_shape(gpu):
    # Llama-3.1-8B lm_head: Dm 4096, V 128256; 64 nodes.  The logits are
    # checked on a vocabulary subset against the fp64 oracle.
    T, M, Dm, V = 1, 64, 4096, 128256
    h, w, draft, pref, pos, md = _case(gpu, T, M, Dm, V, seed=11, sigma=0.02)
    hops = min(md + 2, M)
    r1 = lmhead_tree_accept(h, w, draft, pref, pos, hops, return_next=True)
    r2 = lmhead_tree_accept(h, w, draft, pref, pos, hops, return_next=True, return_logits=True)
    torch.cuda.synchronize()
    lg = r2["logits"]
    for k in ("next", "info", "path", "tokens"):
        assert torch.equal(r1[k], r2[k])
    ref = tree_accept(lg, draft, pref, pos, hops, return_next=True)
    torch.cuda.synchronize()
    assert torch.equal(r1["next"], ref["next"]) and torch.equal(r1["info"], ref["info"])
    cols = torch.from_numpy(np.random.default_rng(0).choice(V, 3000, replace=False)).to(gpu)
    _check_logits(h[0], w[cols], lg[0][:, cols])


def test_strided_hidden_temperature_and_shared_positions(gpu):
    # hidden rows at a padded stride (a [T, M, Dm] view of a wider buffer),
    # typical acceptance at temperature 0.7, one [M] position row for all trees
    T, M, Dm, V = 2, 24, 256, 2000
    h, w, draft, pref, pos, md = _case(gpu, T, M, Dm, V, seed=23)
    wide = torch.zeros((T, M, Dm + 64), dtype=torch.bfloat16, device=gpu)
    wide[..., :Dm] = h
    hv = wide[..., :Dm]
    assert hv.stride(1) == Dm + 64
    pos1 = pos[0]
    hops = min(md + 2, M)
    r = lmhead_tree_accept(hv, w, draft, pref, pos1, hops, mode="typical", temperature=0.7, return_next=True,
                           return_logits=True)
    torch.cuda.synchronize()
    _check_logits(h.reshape(T * M, Dm), w, r["logits"].reshape(T * M, V))
    ref = tree_accept(r["logits"], draft, pref, pos1, hops, mode="typical", temperature=0.7, return_next=True)
    torch.cuda.synchronize()
    for k in ("next", "info", "path", "tokens"):
        assert torch.equal(r[k], ref[k]), k


@pytest.mark.parametrize("delta", [1e-6, -1e-6])
def test_typical_near_the_threshold_rechecked_from_the_written_logits(gpu, delta):
    """With its logits written, the fused path re-decides near-threshold nodes
    from them exactly as kernel 4 does.  Hidden rows that are unit vectors
    make every logit an exact copy of one weight column, so rows within a
    relative 1e-6 of the typical threshold (then rounded to bf16, many
    inside the fp32 margin) can be planted as the roots' distributions."""
    from oracle import accept as oacc
    from test_gpu_accept import _near_threshold_rows
    V, Dm, temperature = 20000, 64, 0.9
    rng = np.random.default_rng(77 + (delta > 0))
    rows, _ = _near_threshold_rows(24, V, delta, 0.5, rng, temperature=temperature)
    T = min(rows.shape[0], Dm // 2)
    rows16 = torch.from_numpy(rows[:T]).to(torch.bfloat16)
    r16 = np.array([np.divide(*oacc.typical_prob_thr(rows16[t].double().numpy(), 0, temperature, 0.09, 0.3))
                    for t in range(T)])
    assert (np.abs(r16 - 1) < 5e-3).sum() >= T // 3, r16     # inside the margin: re-checked
    w = torch.zeros((V, Dm), dtype=torch.bfloat16)
    h = torch.zeros((T, 2, Dm), dtype=torch.bfloat16)
    for t in range(T):
        w[:, 2 * t] = rows16[t]
        h[t, 0, 2 * t] = 1.0                                    # the root's logits: row t
        h[t, 1, 2 * t + 1] = 1.0                                # the child's: zeros
    draft = torch.zeros((T, 2), dtype=torch.int64)               # the child drafts token 0
    pref = torch.full((T, 1), -1, dtype=torch.int64)
    pos = torch.tensor([0, 1])
    r = lmhead_tree_accept(h.to(gpu), w.to(gpu), draft.to(gpu), pref.to(gpu), pos.to(gpu), 2, mode="typical",
                           temperature=temperature, posterior_threshold=0.09, posterior_alpha=0.3,
                           return_logits=True)
    lg = r["logits"].float().cpu().numpy()
    assert np.array_equal(lg[:, 0], rows16.float().numpy())
    info = r["info"].cpu().numpy()
    for t in range(T):
        w_toks, w_ids, w_alen, w_next, w_id = oacc.typical_walk(lg[t], draft[t].numpy(), [-1], pos.numpy(), 8,
                                                                 temperature=temperature, eps=0.09, alpha=0.3)
        assert info[t].tolist() == [w_id, w_alen, w_next, len(w_ids)], f"tree {t}"
