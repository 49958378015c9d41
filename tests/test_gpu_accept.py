"""GPU parity of the acceptance kernel (4) against the oracle walk: accepted
path, its tokens, accept length and next token must be bit-exact."""

import numpy as np
import pytest
import torch

from oracle import accept as oacc
from diffspec_mi355x import workloads as wl
from diffspec_mi355x.draft.tree_verification import evaluate_tree, tree_accept, verify_new

pytestmark = pytest.mark.gpu


def run_and_compare(logits, draft, parent_ref, pos, max_depth, mode="greedy", **kw):
    T, M = draft.shape
    r = tree_accept(logits, draft, parent_ref, pos, min(max_depth + 2, M), mode=mode, return_next=True, **kw)
    info = r["info"].cpu().numpy()
    path = r["path"].cpu().numpy()
    toks = r["tokens"].cpu().numpy()
    lg = logits.float().cpu().numpy()
    for t in range(T):
        p = pos[t] if pos.dim() == 2 else pos
        args = (lg[t], draft[t].cpu().numpy(), parent_ref[t].cpu().tolist(), p.cpu().numpy(), max_depth)
        if mode == "greedy":
            w_toks, w_ids, w_alen, w_next, w_id = oacc.greedy_walk(*args)
        else:
            w_toks, w_ids, w_alen, w_next, w_id = oacc.typical_walk(
                *args, temperature=kw["temperature"], eps=kw["posterior_threshold"], alpha=kw["posterior_alpha"])
        L = len(w_ids)
        assert info[t].tolist() == [w_id, w_alen, w_next, L], f"tree {t}"
        assert path[t, :L].tolist() == w_ids and (path[t, L:] == -1).all()
        assert toks[t, :L].tolist() == w_toks and (toks[t, L:] == -1).all()
        assert r["next"][t].cpu().tolist() == np.argmax(lg[t], axis=-1).tolist()
    return info


@pytest.mark.parametrize("mode", ["greedy", "typical"])
def test_accept_8x64_vocab128256_bit_exact(gpu, mode):
    """8 trees x 64 nodes, bf16 logits [8, 64, 128256] N(0, 3) with a
    planted top token per node and a planted path of length 1..8."""
    a = wl.make_accept_inputs(T=8, M=64, V=128256, device=str(gpu), pos_offset=1000)
    kw = dict(temperature=1.0, posterior_threshold=0.09, posterior_alpha=0.3) if mode == "typical" else {}
    info = run_and_compare(a.logits, a.draft, a.parent_ref, a.pos, 8, mode=mode, **kw)
    assert all(info[t, 1] >= a.planted_len[t] for t in range(8))


@pytest.mark.parametrize("mode", ["greedy", "typical"])
def test_accept_fp32_64_nodes_vocab128256_seed1(gpu, mode):
    """The CPU reference workload's walk at its own size: fp32 logits
    [1, 64, 128256] N(0, 3) from seed 1, draft ids uniform over the vocab from
    the same generator (nothing planted), the 64-node tree of seed 0 (depth
    <= 8, out-degree <= 4)."""
    M, V = 64, 128256
    g = torch.Generator().manual_seed(1)
    logits = torch.randn((1, M, V), generator=g) * 3.0
    draft = torch.randint(0, V, (1, M), generator=g)
    parent, depth = wl.make_tree(M, seed=0)
    pref = torch.tensor([wl.parent_to_reference(parent)], dtype=torch.int64)
    pos = torch.tensor([4096 + d for d in depth], dtype=torch.int64)
    kw = dict(temperature=1.0, posterior_threshold=0.09, posterior_alpha=0.3) if mode == "typical" else {}
    run_and_compare(logits.to(gpu), draft.to(gpu), pref.to(gpu), pos.to(gpu), 8, mode=mode, **kw)
    # and with the root's argmax planted along the chain to a deep node, so the walk has a path to follow
    lg = logits[0].numpy()
    node = int(np.argmax(depth))
    while node > 0:
        draft[0, node] = int(np.argmax(lg[parent[node]]))
        node = parent[node]
    info = run_and_compare(logits.to(gpu), draft.to(gpu), pref.to(gpu), pos.to(gpu), 8, mode=mode, **kw)
    if mode == "greedy":
        assert info[0, 1] == max(depth)


def test_accept_random_shapes_bit_exact(gpu):
    """40 random acceptance calls against the oracle walk: 1-4 trees of 1 to
    1024 nodes, vocabularies of 3 to 50257, bf16 / f16 / f32 logits of spread
    0.3 to 3 (planted paths), greedy and typical (temperature 0.5 to 1.7)."""
    rng = np.random.default_rng(5)
    for case in range(40):
        T = int(rng.integers(1, 5))
        M = int(rng.choice([1, 2, 9, 64, 100, 256, 300, 1024]))
        V = int(rng.choice([3, 100, 1000, 32000, 50257]))
        dtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(3))]
        mode = "greedy" if rng.integers(2) == 0 else "typical"
        sigma = float(rng.choice([0.3, 1.0, 3.0]))
        depth = int(rng.integers(1, 13))
        while sum(6 ** k for k in range(depth + 1)) < M:
            depth += 1
        temp = float(rng.choice([0.5, 1.0, 1.7]))
        print(f"[accept random] case {case}: T={T} M={M} V={V} {dtype} {mode} sigma={sigma} depth={depth} "
              f"temperature={temp}", flush=True)
        a = wl.make_accept_inputs(T=T, M=M, V=V, dtype=dtype, sigma=sigma, seed=300 + case, max_depth=depth,
                                  max_outdeg=6, pos_offset=int(rng.integers(0, 100000)), device=str(gpu))
        kw = dict(temperature=temp, posterior_threshold=0.09, posterior_alpha=0.3) if mode == "typical" else {}
        run_and_compare(a.logits, a.draft, a.parent_ref, a.pos, depth, mode=mode, **kw)


def test_typical_accepts_runner_up_that_greedy_rejects(gpu):
    V, M = 5000, 6
    lg = torch.full((1, M, V), -4.0)
    lg[0, :, 10] = 3.0
    lg[0, :, 11] = 2.9   # runner-up with high probability
    lg[0, 2, 12] = 3.5   # node 2's distribution has a different top token
    draft = torch.tensor([[0, 11, 10, 12, 11, 10]])
    parent_ref = torch.tensor([[-1, 0, 1, -1, 3]])  # nodes 1..5 -> parents 0,1,2,0,4
    pos = torch.tensor([0, 1, 2, 3, 1, 2])
    kw = dict(temperature=1.0, posterior_threshold=0.09, posterior_alpha=0.3)
    gi = run_and_compare(lg.to(torch.bfloat16).to(gpu), draft.to(gpu), parent_ref.to(gpu), pos.to(gpu), 8)
    ti = run_and_compare(lg.to(torch.bfloat16).to(gpu), draft.to(gpu), parent_ref.to(gpu), pos.to(gpu), 8,
                         mode="typical", **kw)
    assert gi[0, 1] < ti[0, 1]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_typical_entropy_with_neg_inf_logits_and_tails(gpu, dtype):
    """-inf logits have p = 0 and add nothing to the entropy (0 log 0 = 0);
    the vocabulary is a multiple of neither 8 nor a range.  The draft token's
    p (~0.01) lies between alpha*exp(-H) (~1e-4) and eps (0.09), so the
    entropy decides the test: a NaN entropy would fall back to eps and reject."""
    V, M = 5003, 3
    lg = torch.zeros((1, M, V))
    lg[0, :, 100:140] = float("-inf")
    lg[0, :, 7] = 3.9
    lg[0, :, V - 1] = float("-inf")  # in the tail past the last 16-byte vector
    draft = torch.tensor([[0, 7, 7]])
    parent_ref = torch.tensor([[-1, 0]])
    pos = torch.arange(M)
    kw = dict(temperature=1.0, posterior_threshold=0.09, posterior_alpha=0.3)
    info = run_and_compare(lg.to(dtype).to(gpu), draft.to(gpu), parent_ref.to(gpu), pos.to(gpu), 8,
                           mode="typical", **kw)
    assert info[0, 1] == 2


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_logit_dtypes_and_vocab_tails(gpu, dtype):
    # vocab not a multiple of the 16-byte vector width nor of the chunk size
    a = wl.make_accept_inputs(T=3, M=40, V=16384 * 2 + 77, dtype=dtype, device=str(gpu), seed=5)
    run_and_compare(a.logits, a.draft, a.parent_ref, a.pos, 8)
    run_and_compare(a.logits, a.draft, a.parent_ref, a.pos, 8, mode="typical", temperature=0.7,
                    posterior_threshold=0.09, posterior_alpha=0.3)


def test_bf16_ties_take_first_index(gpu):
    V, M = 40000, 4
    lg = torch.zeros((1, M, V))
    lg[0, :, [17, 39000, 20000]] = 5.0  # exact ties across vocab chunks
    draft = torch.tensor([[0, 17, 17, 39000]])
    parent_ref = torch.tensor([[-1, 0, 1]])
    pos = torch.arange(M)
    info = run_and_compare(lg.to(torch.bfloat16).to(gpu), draft.to(gpu), parent_ref.to(gpu), pos.to(gpu), 8)
    assert info[0, 2] == 17 and info[0, 1] == 2


def test_nan_ranks_first_like_torch_argmax(gpu):
    V = 1000
    lg = torch.randn((1, 3, V))
    lg[0, 1, 500] = float("nan")
    lg[0, 1, 700] = float("nan")
    r = tree_accept(lg.to(gpu), torch.tensor([[0, 1, 2]], device=gpu), torch.tensor([[-1, 0]], device=gpu),
                    torch.arange(3, device=gpu), 4, return_next=True)
    assert r["next"][0].cpu().tolist() == torch.argmax(lg[0], -1).tolist()


def test_bounded_closure_semantics(gpu):
    M, V = 12, 64
    lg = torch.zeros((1, M, V))
    lg[0, :, 1] = 1
    draft = torch.ones((1, M), dtype=torch.long)
    draft[0, 1] = 2
    parent_ref = torch.tensor([[-1] + list(range(M - 2))])
    pos = torch.arange(M)
    info = run_and_compare(lg.to(gpu), draft.to(gpu), parent_ref.to(gpu), pos.to(gpu), max_depth=2)
    assert info[0, 0] == M - 1


def test_malformed_parent_is_reported(gpu):
    lg = torch.zeros((1, 4, 16), device=gpu)
    r = tree_accept(lg, torch.zeros((1, 4), dtype=torch.long, device=gpu),
                    torch.tensor([[-1, 7, 0]], device=gpu), torch.arange(4, device=gpu), 4)
    assert r["info"][0, 3].item() == -1


class _FakeDraftModel:
    def __init__(self, dev):
        self.dev = dev
        self.enable_bundle_scheduling = True
        self.use_retrieval_cache = False

    def build_speculative_tree(self, hidden, input_ids, head, nodes, threshold, max_depth):
        self.seen_input_ids = input_ids.clone()
        d = torch.tensor([[5, 6, 7]], device=self.dev)
        pos = torch.tensor([1, 2, 2], device=self.dev)
        mask = torch.tensor([[1, 0, 0], [1, 1, 0], [1, 0, 1]], device=self.dev)
        par = torch.tensor([-1, 0, 0], device=self.dev)
        return d, pos, mask, par


class _FakeModel:
    def __init__(self, dev):
        self.draft_model = _FakeDraftModel(dev)
        self.base_model = type("B", (), {"lm_head": None})()


def test_verify_new_contract_with_kv_compaction(gpu):
    a = wl.make_accept_inputs(T=1, M=16, V=3000, device=str(gpu), seed=9, pos_offset=50)
    M = 16
    L = 80
    kv = [torch.randn(2, 1, 2, L, 8, device=gpu) for _ in range(2)]
    kv_before = [x.clone() for x in kv]
    cur_len = torch.tensor([L - 4], dtype=torch.long)  # 60 prefix + 16 tree
    start = L - 4 - M
    input_ids = torch.arange(10, device=gpu).unsqueeze(0)
    hidden = torch.randn(1, M, 4, device=gpu)
    model = _FakeModel(gpu)
    res = verify_new(input_ids, a.logits, a.draft, a.pos, hidden, None, kv, cur_len,
                     a.parent_ref[0], model, nodes=3, threshold=0.1, max_depth=8, logits_processor=None)
    ids_out, best, alen, nd, npos, nmask, npar = res
    w = oacc.greedy_walk(a.logits[0].float().cpu().numpy(), a.draft[0].cpu().numpy(), a.parent_ref[0].tolist(),
                         a.pos[0].cpu().numpy(), 8)
    assert best == w[0] and alen == w[2]
    assert ids_out[0, 10:].tolist() == w[0]
    assert nd[0, 0].item() == w[3] and nd.shape == (1, 4)
    assert npos[0].item() == int(a.pos[0, w[4]]) + 1
    assert nmask.shape == (4, 4) and nmask[0].tolist() == [1, 0, 0, 0]
    assert cur_len.item() == start + len(w[1])
    sel = torch.tensor(w[1], device=gpu) + start
    for x, x0 in zip(kv, kv_before):
        assert torch.equal(x[..., start:start + len(w[1]), :], x0[..., sel, :])
    assert model.draft_model.last_bundle_stats["num_bundles"] >= 1


def _edge_rows(V):
    """Rows that exercise the ordering of 16-bit keys (V a multiple of 8, so
    rows are 16-byte aligned and the packed-key sweep runs)."""
    g = torch.Generator().manual_seed(11)
    lg = torch.randn((7, V), generator=g)
    lg[0] = -lg[0].abs() - 1.0                     # all negative
    lg[1, 2] = lg[1, 3] = lg[1, 1000] = 9.0        # ties inside one dword and across threads
    lg[2] = -1.0
    lg[2, 5] = -0.0                                # -0 == +0: first one wins
    lg[2, 9] = 0.0
    lg[3] = float("-inf")                          # all -inf: index 0
    lg[4, 100] = lg[4, V - 3] = float("inf")       # +inf ties across chunks
    lg[5, 20] = lg[5, V - 10] = float("nan")       # first NaN wins
    return lg


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_packed_key_sweep_edge_rows(gpu, dtype):
    V = 16384 * 2 + 8 * 41
    lg = _edge_rows(V).to(dtype)
    M = lg.shape[0]
    want = torch.argmax(lg.float(), -1).tolist()
    r = tree_accept(lg.unsqueeze(0).to(gpu), torch.zeros((1, M), dtype=torch.int64, device=gpu),
                    torch.full((1, M - 1), -1, dtype=torch.int64, device=gpu), torch.arange(M, device=gpu), 4,
                    return_next=True)
    assert r["next"][0].cpu().tolist() == want


def test_packed_key_sweep_strided_rows_with_short_tail(gpu):
    # rows of a wider, 16-byte aligned buffer: the vocab tail (V % 8 != 0) is
    # read by the scalar tail path of the packed-key sweep
    a = wl.make_accept_inputs(T=2, M=24, V=16384 + 8 * 300 + 5, dtype=torch.bfloat16, device=str(gpu), seed=9)
    V = a.logits.shape[-1]
    wide = torch.full((2, 24, V + 3), -100.0, dtype=torch.bfloat16, device=gpu)
    wide[..., :V] = a.logits
    wide[1, 5, V - 2] = 50.0                       # maximum inside the tail
    lg = wide[..., :V]
    assert lg.stride(1) * 2 % 16 == 0
    run_and_compare(lg, a.draft, a.parent_ref, a.pos, 8)
    run_and_compare(lg, a.draft, a.parent_ref, a.pos, 8, mode="typical", temperature=1.0,
                    posterior_threshold=0.09, posterior_alpha=0.3)


@pytest.mark.parametrize("M", [200, 300])
def test_verify_new_takes_the_reference_copy_beyond_the_commit_kernel_limit(gpu, M):
    """A 200- or 300-node tree with 128-element fp32 cache rows (M x 512 B,
    above the commit kernel's 64 KiB of staged tree rows) takes the
    reference's gather + copy instead of raising, with the same result."""
    from diffspec_mi355x.draft.tree_verification import _kv_commit_ok
    a = wl.make_accept_inputs(T=1, M=M, V=3000, device=str(gpu), seed=3, max_outdeg=6, pos_offset=50)
    L = M + 40
    kv = [torch.randn(2, 1, 2, L, 128, device=gpu) for _ in range(2)]
    assert not _kv_commit_ok(kv[0], M)             # the fallback branch is the one taken
    kv_before = [x.clone() for x in kv]
    cur_len = torch.tensor([L], dtype=torch.long)
    start = L - M
    model = _FakeModel(gpu)
    res = verify_new(torch.arange(10, device=gpu).unsqueeze(0), a.logits, a.draft, a.pos,
                     torch.randn(1, M, 4, device=gpu), None, kv, cur_len, a.parent_ref[0], model, nodes=3,
                     threshold=0.1, max_depth=8, logits_processor=None)
    w = oacc.greedy_walk(a.logits[0].float().cpu().numpy(), a.draft[0].cpu().numpy(), a.parent_ref[0].tolist(),
                         a.pos[0].cpu().numpy(), 8)
    assert res[1] == w[0] and res[2] == w[2]
    sel = torch.tensor(w[1], device=gpu) + start
    for x, x0 in zip(kv, kv_before):
        assert torch.equal(x[..., start:start + len(w[1]), :], x0[..., sel, :])


def _log_ratio(x, temperature, eps, alpha, delta):
    prob, thr = oacc.typical_prob_thr(x.astype(np.float32), 0, temperature, eps, alpha)
    return np.log(prob) - np.log(thr) - np.log1p(delta)


def _bisect_f32(f, x, j, lo, hi, side):
    """Set x[j] to the float32 value in [lo, hi] next to the root of f, on the
    side where sign(f) == side; False if f does not change sign there."""
    x[j] = lo
    flo = f(x)
    x[j] = hi
    if flo * f(x) > 0:
        return False
    for _ in range(200):
        mid = 0.5 * (lo + hi)
        x[j] = mid
        if (f(x) > 0) == (flo > 0):
            lo = mid
        else:
            hi = mid
    best = None
    for c in [np.float32(lo), np.float32(hi), np.nextafter(np.float32(lo), np.float32(-np.inf)),
              np.nextafter(np.float32(hi), np.float32(np.inf))]:
        x[j] = float(c)
        v = f(x) * side
        if v >= 0 and (best is None or v < best[1]):
            best = (float(c), v)
    if best is None:
        return False
    x[j] = best[0]
    return True


def _near_threshold_rows(n, V, delta, sigma, rng, temperature=1.0, eps=0.09, alpha=0.3):
    """fp32 rows whose token 0 has p = (1 + delta) * min(eps, alpha * exp(-H))
    under softmax(row / T), to within |delta| / 4, with delta down to 1e-9:
    token 0's logit is solved first (bisection in float64, rounded to a
    neighbouring float32), then token 1's logit, started far below the others
    where its mass is negligible, tunes the ratio finely (raising it moves the
    ratio by its tiny mass, in a direction probed first).  Returns the rows
    and their float64 ratios p / threshold."""
    rows, got = [], []
    f = lambda x: _log_ratio(x, temperature, eps, alpha, delta)
    lo1 = -60.0 * temperature
    for _ in range(n):
        x = rng.normal(0, sigma, V).astype(np.float64)
        x[1] = lo1
        if not _bisect_f32(f, x, 0, -30.0 * temperature, 30.0 * temperature, 1):
            continue
        f0 = f(x)
        x[1] = x[0]
        up = f(x) > f0                   # does raising token 1's logit raise the ratio?
        x[1] = lo1
        if not _bisect_f32(f, x, 0, -30.0 * temperature, 30.0 * temperature, -1 if up else 1):
            continue
        if not _bisect_f32(f, x, 1, lo1, x[0], 1):
            continue
        prob, thr = oacc.typical_prob_thr(x.astype(np.float32), 0, temperature, eps, alpha)
        ratio = prob / thr
        if np.sign(ratio - 1.0) == np.sign(delta) and abs(ratio - 1.0 - delta) <= abs(delta) / 4:
            rows.append(x.astype(np.float32))
            got.append(ratio)
    return np.stack(rows), np.array(got)


@pytest.mark.parametrize("delta", [2e-3, -2e-3, 1e-6, -1e-6, 1e-9, -1e-9])
@pytest.mark.parametrize("sigma", [0.5, 3.0])
def test_typical_decision_near_the_threshold(gpu, delta, sigma):
    """The typical test p > min(eps, alpha * exp(-H)) is bit-exact against the
    float64 oracle arbitrarily close to the threshold: the kernel decides from
    the sweep's fp32 statistics only outside a margin of about 1% (relative)
    and re-decides the nodes inside it from float64 statistics of the
    parent's row.  fp32 rows with p at (1 + delta) times the threshold, delta
    from 2e-3 down to 1e-9, both signs; sigma 0.5 gives flat rows (threshold
    alpha * exp(-H)), sigma 3 peaked ones (threshold eps for many).  The same
    rows rounded to bf16 land within a few percent of their own thresholds,
    some within 0.5% (a third of the flat ones), where the margin re-checks
    them; the oracle decides them from the rounded values."""
    rng = np.random.default_rng(int(abs(np.log10(abs(delta))) * 10) + int(sigma * 10) + (delta > 0))
    rows, ratio = _near_threshold_rows(24, 20000, delta, sigma, rng, temperature=0.9)
    T = rows.shape[0]
    assert T >= 12
    print(f"[typical near threshold] delta={delta} sigma={sigma}: {T} rows, "
          f"ratio-1 in [{(ratio - 1).min():.3e}, {(ratio - 1).max():.3e}]", flush=True)
    draft = torch.zeros((T, 2), dtype=torch.int64)                     # the child's token is token 0
    parent_ref = torch.full((T, 1), -1, dtype=torch.int64)
    pos = torch.tensor([0, 1])
    kw = dict(temperature=0.9, posterior_threshold=0.09, posterior_alpha=0.3)
    for dtype in (torch.float32, torch.bfloat16):
        lg = torch.from_numpy(np.stack([rows, rows], axis=1)).to(dtype)   # [T, 2, V]: root and its child
        if dtype == torch.bfloat16:
            r16 = np.array([np.divide(*oacc.typical_prob_thr(lg[t, 0].double().numpy(), 0, 0.9, 0.09, 0.3))
                            for t in range(T)])
            # inside the margin (re-checked): many of the flat rows, a few peaked ones
            assert (np.abs(r16 - 1) < 5e-3).sum() >= (T // 3 if sigma < 1 else 2), r16
        info = run_and_compare(lg.to(gpu), draft.to(gpu), parent_ref.to(gpu), pos.to(gpu), 8, mode="typical", **kw)
        if dtype == torch.float32:
            assert (info[:, 1] == (1 if delta > 0 else 0)).all()


def _accept_into(ws, logits, draft, parent_ref, pos, max_hops, mode, kw):
    """dsv_tree_accept through the C ABI over a caller-owned workspace."""
    from diffspec_mi355x import _ext
    lib = _ext.load()
    T, M, V = logits.shape
    dev = logits.device
    path = torch.empty((T, M), dtype=torch.int64, device=dev)
    tokens = torch.empty_like(path)
    info = torch.empty((T, 4), dtype=torch.int64, device=dev)
    assert ws.numel() >= lib.dsv_accept_workspace_bytes(T, M, V)
    mode_id = {"greedy": _ext.ACCEPT_GREEDY, "typical": _ext.ACCEPT_TYPICAL}[mode]
    rc = lib.dsv_tree_accept(mode_id, _ext.desc(logits), _ext.desc(draft), _ext.desc(parent_ref), _ext.desc(pos),
                             int(max_hops), float(kw.get("temperature", 1.0)),
                             float(kw.get("posterior_threshold", 0.09)), float(kw.get("posterior_alpha", 0.3)),
                             _ext.desc(path), _ext.desc(tokens), _ext.desc(info), _ext.desc(None), ws.data_ptr(),
                             ws.numel(), _ext.stream_of(dev))
    _ext.check(rc, "tree_accept")
    return path.cpu().numpy(), tokens.cpu().numpy(), info.cpu().numpy()


@pytest.mark.parametrize("mode", ["greedy", "typical"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_acceptance_needs_no_cleared_workspace(gpu, mode, dtype):
    """The result must not depend on what the workspace held before: zeros,
    all ones, random bytes, the statistics of a call over other trees, and the
    same workspace reused call after call.  bf16 rows take the streaming
    sweep, f32 rows the generic one."""
    kw = dict(temperature=1.0, posterior_threshold=0.09, posterior_alpha=0.3) if mode == "typical" else {}
    T, M, V = 8, 64, 50000
    a = wl.make_accept_inputs(T=T, M=M, V=V, dtype=dtype, device=str(gpu), seed=21, pos_offset=300)
    other = wl.make_accept_inputs(T=T, M=M, V=V, dtype=dtype, device=str(gpu), seed=22, pos_offset=300)
    lg = a.logits.float().cpu().numpy()
    want = []
    for t in range(T):
        args = (lg[t], a.draft[t].cpu().numpy(), a.parent_ref[t].cpu().tolist(), a.pos[t].cpu().numpy(), 8)
        if mode == "greedy":
            want.append(oacc.greedy_walk(*args))
        else:
            want.append(oacc.typical_walk(*args, temperature=1.0, eps=0.09, alpha=0.3))

    def check(res, label):
        path, toks, info = res
        for t, (w_toks, w_ids, w_alen, w_next, w_id) in enumerate(want):
            L = len(w_ids)
            assert info[t].tolist() == [w_id, w_alen, w_next, L], f"{label}: tree {t}"
            assert path[t, :L].tolist() == w_ids and (path[t, L:] == -1).all(), f"{label}: tree {t}"
            assert toks[t, :L].tolist() == w_toks and (toks[t, L:] == -1).all(), f"{label}: tree {t}"

    from diffspec_mi355x import _ext
    nbytes = _ext.load().dsv_accept_workspace_bytes(T, M, V)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
    g = torch.Generator(device=gpu).manual_seed(5)
    run = lambda x: _accept_into(ws, x.logits, x.draft, x.parent_ref, x.pos, 10, mode, kw)
    for label, fill in [("zeros", lambda: ws.zero_()), ("ones", lambda: ws.fill_(255)),
                        ("random", lambda: ws.copy_(torch.randint(0, 256, (nbytes,), generator=g, device=gpu,
                                                                  dtype=torch.uint8)))]:
        fill()
        check(run(a), label)
    run(other)
    check(run(a), "after a call over other trees")
    for k in range(3):
        check(run(a), f"reused {k}")
