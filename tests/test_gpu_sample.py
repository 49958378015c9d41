"""GPU parity of the sampling acceptance (dsv_tree_accept_sample) against the
oracle (oracle/sampling.py): per-node draws, accepted path, tokens, accept
length and next token bit-exact; the draws' frequencies against the warped
softmax by a chi-square test; verify_new driven by the reference's own
transformers warper list."""

import numpy as np
import pytest
import torch
from scipy import stats

from oracle import sampling as sp
from diffspec_mi355x import workloads as wl
from diffspec_mi355x.draft.tree_verification import prepare_logits_processor, tree_accept, verify_new

pytestmark = pytest.mark.gpu

DT = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def run_and_compare(logits, draft, parent_ref, pos, max_depth, temperature, top_p, top_k, seed):
    T, M = draft.shape
    r = tree_accept(logits, draft, parent_ref, pos, min(max_depth + 2, M), mode="sample", temperature=temperature,
                    top_p=top_p, top_k=top_k, seed=seed, return_next=True)
    info, path, toks, nxt = (r[k].cpu().numpy() for k in ("info", "path", "tokens", "next"))
    lg = logits.float().cpu().numpy()
    for t in range(T):
        p = pos[t] if pos.dim() == 2 else pos
        w_toks, w_ids, w_alen, w_next, w_id, draws = sp.sample_walk(
            lg[t], DT[logits.dtype], draft[t].cpu().numpy(), parent_ref[t].cpu().tolist(), p.cpu().numpy(),
            max_depth, temperature, top_p, top_k, seed, tree=t)
        assert nxt[t].tolist() == draws.tolist(), f"tree {t} draws"
        L = len(w_ids)
        assert info[t].tolist() == [w_id, w_alen, w_next, L], f"tree {t}"
        assert path[t, :L].tolist() == w_ids and toks[t, :L].tolist() == w_toks
    return r


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("temperature,top_p,top_k", [(1.0, 1.0, 0), (0.7, 0.9, 0), (1.3, 1.0, 20), (0.8, 0.5, 10),
                                                     (1.0, 0.05, 0), (1.0, 1.0, 1)])
def test_sample_walk_bit_exact(gpu, dtype, temperature, top_p, top_k):
    print(f"[sample] {dtype} T={temperature} top_p={top_p} top_k={top_k}", flush=True)
    a = wl.make_accept_inputs(T=2, M=16, V=3000 + 5, dtype=dtype, sigma=2.0, device=str(gpu), seed=11)
    run_and_compare(a.logits, a.draft, a.parent_ref, a.pos, 8, temperature, top_p, top_k, seed=12345)


def test_sample_random_warper_combinations(gpu):
    """30 random sampling calls, bit-exact against the oracle: 1-3 trees of 1
    to 200 nodes, vocabularies of 2 to 32000, bf16 / f16 / f32 logits of
    spread 0.1 to 8, temperature 0.3 to 1.5, top-p 1 down to 0.001, top-k 0
    to 1000, random 64-bit seeds."""
    rng = np.random.default_rng(91)
    for case in range(30):
        T = int(rng.integers(1, 4))
        V = int(rng.choice([2, 7, 1000, 5003, 32000]))
        M = int(rng.choice([1, 5, 64, 200]))
        dtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(3))]
        temp = float(rng.choice([0.3, 0.7, 1.0, 1.5]))
        top_p = float(rng.choice([1.0, 0.95, 0.5, 0.05, 0.001]))
        top_k = int(rng.choice([0, 1, 5, 50, 1000]))
        sigma = float(rng.choice([0.1, 1.0, 3.0, 8.0]))
        depth = int(rng.integers(1, 10))
        while sum(6 ** k for k in range(depth + 1)) < M:
            depth += 1
        seed = int(rng.integers(0, 2 ** 63))
        print(f"[sample random] case {case}: T={T} M={M} V={V} {dtype} temperature={temp} top_p={top_p} "
              f"top_k={top_k} sigma={sigma}", flush=True)
        a = wl.make_accept_inputs(T=T, M=M, V=V, dtype=dtype, sigma=sigma, seed=500 + case, max_depth=depth,
                                  max_outdeg=6, device=str(gpu))
        run_and_compare(a.logits, a.draft, a.parent_ref, a.pos, depth, temp, top_p, top_k, seed)


def test_sample_full_vocab_64_nodes(gpu):
    """bf16 [1, 64, 128256] N(0, 3) logits, temperature 0.7, top-p 0.9, top-k 50."""
    a = wl.make_accept_inputs(T=1, M=64, V=128256, device=str(gpu), seed=21)
    run_and_compare(a.logits, a.draft, a.parent_ref, a.pos, 8, 0.7, 0.9, 50, seed=2 ** 63 + 5)
    run_and_compare(a.logits, a.draft, a.parent_ref, a.pos, 8, 1.0, 1.0, 0, seed=7)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("T,V", [(1, 32768), (8, 20003)])
def test_sample_temperature_alone_rows_and_workgroups(gpu, dtype, T, V):
    """Temperature alone at 64 rows (16-bit logits: several workgroups per
    row, each over a run of the row's vocabulary ranges; f32: the sweep
    kernel) and at 512 rows (one workgroup per row, f32 included), on peaked,
    flat, all-negative and NaN-holding rows: bit-exact against the oracle."""
    M = 64
    g = torch.Generator().manual_seed(17 + T)
    lg = torch.randn((T, M, V), generator=g) * 3.0
    lg[:, ::4, 123] += 30.0                         # a planted favourite on a quarter of the rows
    lg[:, 1::8] -= 60.0                             # all-negative rows
    lg[:, 2::16, 500:520] = float("nan")
    lg = lg.to(dtype).to(gpu)
    a = wl.make_accept_inputs(T=T, M=M, V=V, device=str(gpu), seed=5)
    for temperature in (0.7, 1.0):
        print(f"[sample temperature alone] {dtype} T={T} V={V} temperature={temperature}", flush=True)
        run_and_compare(lg, a.draft, a.parent_ref, a.pos, 8, temperature, 1.0, 0, seed=1000 + T)


def test_sample_many_rows(gpu):
    """8 trees x 64 nodes = 512 rows, at least two per CU: the select kernel
    runs its 512-thread workgroups (fewer rows take 1024 threads)."""
    a = wl.make_accept_inputs(T=8, M=64, V=8192 + 3, device=str(gpu), seed=31)
    run_and_compare(a.logits, a.draft, a.parent_ref, a.pos, 8, 0.7, 0.9, 50, seed=77)
    run_and_compare(a.logits, a.draft, a.parent_ref, a.pos, 8, 1.0, 0.8, 0, seed=78)
    flat = (torch.randn((8, 64, 8192 + 3), generator=torch.Generator().manual_seed(3)) * 0.5).to(torch.bfloat16)
    run_and_compare(flat.to(gpu), a.draft, a.parent_ref, a.pos, 8, 1.0, 0.9, 0, seed=79)
    run_and_compare(flat.to(gpu), a.draft, a.parent_ref, a.pos, 8, 1.0, 1.0, 100, seed=80)


@pytest.mark.parametrize("sigma,top_p,top_k", [(0.3, 0.9, 0), (0.3, 1.0, 3000), (3.0, 1.0, 2000), (3.0, 0.999, 0),
                                             (3.0, 0.5, 7)])
def test_sample_full_vocab_flat_and_peaked_rows(gpu, sigma, top_p, top_k):
    """bf16 [1, 16, 128256] N(0, sigma) logits: flat rows whose top-p set or
    top-k is too large for the select kernel's candidate list (the radix
    selection and the sweep draw them), and peaked rows drawn from the
    candidates."""
    print(f"[sample] full vocab sigma={sigma} top_p={top_p} top_k={top_k}", flush=True)
    a = wl.make_accept_inputs(T=1, M=16, V=128256, device=str(gpu), seed=31)
    g = torch.Generator().manual_seed(31)
    lg = (torch.randn((1, 16, 128256), generator=g) * sigma).to(torch.bfloat16).to(gpu)  # no planted token
    run_and_compare(lg, a.draft, a.parent_ref, a.pos, 8, 1.0, top_p, top_k, seed=77)


def test_sample_random_configurations(gpu):
    """40 random (dtype, vocabulary, spread, temperature, top-p, top-k, seed)
    configurations, peaked and flat rows, aligned and unaligned vocabularies:
    every draw bit-exact against the oracle (the fp32 filters, the head
    choice, the tail bounds and the radix kernel all take part)."""
    rng = np.random.default_rng(2026)
    dts = [torch.bfloat16, torch.float16, torch.float32]
    for case in range(40):
        dtype = dts[case % 3]
        V = int(rng.choice([777, 4099, 8192, 20000, 33333]))
        sigma = float(rng.choice([0.3, 1.0, 3.0, 8.0]))
        temperature = float(rng.choice([1.0, 0.5, 0.8, 1.7]))
        top_p = float(rng.choice([1.0, 0.99, 0.9, 0.6, 0.2]))
        top_k = int(rng.choice([0, 0, 1, 5, 50, 700]))
        seed = int(rng.integers(0, 2 ** 63))
        print(f"[sample random {case}] {dtype} V={V} sigma={sigma} T={temperature} p={top_p} k={top_k}", flush=True)
        g = torch.Generator().manual_seed(case)
        lg = (torch.randn((2, 6, V), generator=g) * sigma)
        if case % 4 == 0:
            lg[:, :, int(rng.integers(0, V))] += 10.0 * sigma  # a planted favourite
        lg = lg.to(dtype).to(gpu)
        a = wl.make_accept_inputs(T=2, M=6, V=V, device=str(gpu), seed=case)
        run_and_compare(lg, a.draft, a.parent_ref, a.pos, 8, temperature, top_p, top_k, seed)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_sample_ties_at_the_top_p_cut(gpu, dtype):
    """Rows of a few repeated values, so the top-p cut falls inside a tie
    group (kept: its highest indices) and top-k ties are all kept; with
    rows whose largest logit is -0 or negative, rows of -inf and NaNs of both
    signs, also drawn with temperature alone."""
    M, V = 8, 4099
    g = torch.Generator().manual_seed(5)
    lg = torch.randint(-3, 3, (1, M, V), generator=g).float().to(dtype)
    lg[0, 2] = -lg[0, 2].abs()                      # at most -0
    lg[0, 7] -= 10.0                                # all negative
    lg[0, 3] = float("-inf")
    lg[0, 3, 17] = 2.0                              # one finite logit
    lg[0, 4, :] = float("-inf")                     # none: token 0
    lg[0, 5, 100:200] = float("nan")                # NaN counts as -inf
    if dtype == torch.float32:                      # signalling NaNs, both signs
        snan = torch.tensor([0x7F800001, -0x7FFFFF], dtype=torch.int32).view(dtype)
    else:
        snan = torch.tensor([0x7F81, -0x7F], dtype=torch.int16).view(dtype)
    lg[0, 6, 10], lg[0, 6, 4000] = snan[0], snan[1]
    draft = torch.randint(0, V, (1, M), generator=g)
    parent_ref = torch.tensor([[-1, 0, 1, 2, 3, 4, 5]])
    pos = torch.arange(M)
    for temperature, top_p, top_k in [(1.0, 0.3, 0), (1.0, 0.77, 0), (1.0, 0.5, 7), (1.0, 1.0, 3), (1.0, 1.0, 0),
                                      (0.6, 1.0, 0)]:
        print(f"[sample ties] {dtype} T={temperature} top_p={top_p} top_k={top_k}", flush=True)
        run_and_compare(lg.to(gpu), draft.to(gpu), parent_ref.to(gpu), pos.to(gpu), 8, temperature, top_p, top_k,
                        seed=99)
    r = tree_accept(lg.to(gpu), draft.to(gpu), parent_ref.to(gpu), pos.to(gpu), 8, mode="sample", top_p=0.9, seed=4,
                    return_next=True)
    assert r["next"][0, 3].item() == 17 and r["next"][0, 4].item() == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_sample_tiny_and_huge_logits(gpu, dtype):
    """Rows of subnormal-range logits (the warper's product and quotient among
    the subnormals), rows of logits in the thousands (the fp32 bound on L
    widens with |m|), and a planted favourite among tiny values: every draw
    bit-exact against the oracle."""
    M, V = 6, 8195
    g = torch.Generator().manual_seed(12)
    base = torch.randn((1, M, V), generator=g)
    tiny = {torch.bfloat16: 1e-39, torch.float16: 1e-6, torch.float32: 1e-41}[dtype]  # subnormal in the dtype
    lg = base.clone()
    lg[0, 0] *= tiny
    lg[0, 1] *= tiny
    lg[0, 1, 77] = 3.0
    lg[0, 2] *= 300.0 if dtype == torch.float16 else 2000.0
    lg[0, 3] = lg[0, 3] * 2.0 + (500.0 if dtype == torch.float16 else 4000.0)
    lg[0, 4] *= 40.0
    lg = lg.to(dtype)
    draft = torch.randint(0, V, (1, M), generator=g)
    parent_ref = torch.tensor([[-1, 0, 1, 2, 3]])
    pos = torch.arange(M)
    for temperature, top_p, top_k in [(0.3, 1.0, 5), (0.7, 0.9, 0), (1.0, 0.5, 0), (1.3, 1.0, 40), (0.7, 0.95, 20),
                                      (0.7, 1.0, 0), (1.0, 1.0, 0)]:
        print(f"[sample tiny/huge] {dtype} T={temperature} top_p={top_p} top_k={top_k}", flush=True)
        run_and_compare(lg.to(gpu), draft.to(gpu), parent_ref.to(gpu), pos.to(gpu), 8, temperature, top_p, top_k,
                        seed=41)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_sample_rows_with_infinite_logits(gpu, dtype):
    """Rows holding +inf logits (one, two tied, with NaNs beside), and f16 rows
    whose warped values overflow to +inf at temperature 0.7: every +inf entry
    has the maximum's mass, the others none; ties drawn by the lowest index."""
    M, V = 6, 4099
    g = torch.Generator().manual_seed(8)
    lg = torch.randint(-3, 3, (1, M, V), generator=g).float()
    lg[0, 1, 50] = float("inf")
    lg[0, 2, 60] = float("inf")
    lg[0, 2, 70] = float("inf")
    lg[0, 3, 80] = float("inf")
    lg[0, 3, 90:95] = float("nan")
    lg[0, 4, 1000] = 50000.0                        # f16: 50000 / 0.7 rounds to +inf
    lg[0, 4, 2000] = 60000.0
    lg[0, 5, 3000] = 40000.0                        # f16: 40000 / 0.7 = 57142.9 stays finite
    lg = lg.to(dtype)
    draft = torch.randint(0, V, (1, M), generator=g)
    parent_ref = torch.tensor([[-1, 0, 1, 2, 3]])
    pos = torch.arange(M)
    for temperature, top_p, top_k in [(1.0, 1.0, 0), (0.7, 1.0, 0), (0.7, 0.9, 0), (1.0, 1.0, 5), (1.3, 0.5, 7)]:
        print(f"[sample inf] {dtype} T={temperature} top_p={top_p} top_k={top_k}", flush=True)
        run_and_compare(lg.to(gpu), draft.to(gpu), parent_ref.to(gpu), pos.to(gpu), 8, temperature, top_p, top_k,
                        seed=31)


def test_sample_top_p_total_mass_above_2_62(gpu):
    """Rows whose fixed-point total mass L lies just above 2^62 (V = 8000, so
    S = 50 and L < 2^63): four logits tied at the maximum and a flat tail that
    brings L to 4096.01 * 2^50, with top_p = 2^-12, so that the exact cut
    P * L / 2^32 lies just above one tie's mass and keeps two of the four
    tied entries (the two highest indices).  An upper bound of L capped at
    2^62 would keep one.  The sixteen nodes draw between the two kept entries;
    every draw is checked against the oracle."""
    V, M, h = 8000, 16, 4
    a = np.float32(-0.66990507)
    row = np.full(V, a, dtype=np.float32)
    row[:h] = 0.0
    q = sp.fixed_masses(row.astype(np.float64))
    L = int(q.sum(dtype=np.uint64))
    assert 2 ** 62 < L < 2 ** 62 + 2 ** 50 // 10
    top_p = 2.0 ** -12
    assert sp.kept_mask(row.astype(np.float64), top_p, 0).sum() == 2
    for shift in (0, 3001):                         # the tied entries at the front, then mid-row
        lg = torch.from_numpy(np.roll(row, shift)).reshape(1, 1, V).repeat(1, M, 1)
        g = torch.Generator().manual_seed(shift)
        draft = torch.randint(0, V, (1, M), generator=g)
        parent_ref = torch.tensor([list(range(-1, M - 2))])
        pos = torch.arange(M)
        print(f"[sample L>2^62] shift {shift}", flush=True)
        r = run_and_compare(lg.to(gpu), draft.to(gpu), parent_ref.to(gpu), pos.to(gpu), 8, 1.0, top_p, 0, seed=17)
        draws = set(r["next"][0].cpu().tolist())
        assert draws == {shift + 2, shift + 3}, draws


@pytest.mark.parametrize("temperature,top_p,top_k", [(1.0, 1.0, 0), (0.6, 0.85, 0), (1.5, 1.0, 6)])
def test_sample_frequencies_follow_the_warped_softmax(gpu, temperature, top_p, top_k):
    """4096 draws of one 24-token row (512 trees x 8 nodes with the same logits)."""
    V, T, M = 24, 512, 8
    g = torch.Generator().manual_seed(3)
    row = torch.randn(V, generator=g) * 1.5
    lg = row.expand(T, M, V).contiguous().to(gpu)
    draft = torch.zeros((T, M), dtype=torch.int64, device=gpu)
    parent_ref = torch.full((T, M - 1), -1, dtype=torch.int64, device=gpu)
    pos = torch.arange(M, device=gpu)
    r = tree_accept(lg, draft, parent_ref, pos, 4, mode="sample", temperature=temperature, top_p=top_p, top_k=top_k,
                    seed=2024, return_next=True)
    draws = r["next"].reshape(-1).cpu().numpy()
    y = sp.warp_temperature(row.numpy(), temperature, "f32")
    keep = sp.kept_mask(y, top_p, top_k)
    p = np.where(keep, np.exp(y - y.max()), 0.0)
    p /= p.sum()
    counts = np.bincount(draws, minlength=V)
    assert counts[~keep].sum() == 0
    kept = np.nonzero(keep)[0]
    assert stats.chisquare(counts[kept], draws.size * p[kept]).pvalue > 1e-4
    # and bit-exact with the oracle on a few of those trees
    for t in (0, 1, 511):
        want = [sp.sample_row(row.numpy(), "f32", temperature, top_p, top_k, 2024, t, i) for i in range(M)]
        assert r["next"][t].cpu().tolist() == want


class _Draft:
    def __init__(self, dev):
        self.dev, self.enable_bundle_scheduling = dev, False

    def build_speculative_tree(self, hidden, input_ids, head, nodes, threshold, max_depth):
        return (torch.tensor([[5, 6]], device=self.dev), torch.tensor([1, 2], device=self.dev),
                torch.tensor([[1, 0], [1, 1]], device=self.dev), torch.tensor([-1, 0], device=self.dev))


class _Model:
    def __init__(self, dev):
        self.draft_model = _Draft(dev)
        self.base_model = type("B", (), {"lm_head": None})()


def test_verify_new_with_the_reference_warper_list(gpu):
    """verify_new given transformers' processor list (what the reference's
    prepare_logits_processor builds) samples with a seed drawn from torch's
    default generator: torch.manual_seed fixes the result."""
    from transformers.generation.logits_process import (LogitsProcessorList, TemperatureLogitsWarper,
                                                        TopKLogitsWarper, TopPLogitsWarper)
    a = wl.make_accept_inputs(T=1, M=16, V=2000, sigma=1.0, device=str(gpu), seed=4, pos_offset=30)
    procs = LogitsProcessorList([TemperatureLogitsWarper(0.8), TopPLogitsWarper(0.9), TopKLogitsWarper(40)])
    L = 60
    kv = [torch.randn(2, 1, 2, L, 8, device=gpu)]
    for lp in (procs, prepare_logits_processor(temperature=0.8, top_p=0.9, top_k=40)):
        torch.manual_seed(77)
        seed = int(torch.randint(0, 2 ** 62, (1,)).item())
        torch.manual_seed(77)
        res = verify_new(torch.arange(5, device=gpu).unsqueeze(0), a.logits, a.draft, a.pos,
                         torch.randn(1, 16, 4, device=gpu), None, kv, torch.tensor([L - 4]), a.parent_ref[0],
                         _Model(gpu), nodes=3, threshold=0.1, max_depth=8, logits_processor=lp)
        w = sp.sample_walk(a.logits[0].float().cpu().numpy(), "bf16", a.draft[0].cpu().numpy(),
                           a.parent_ref[0].tolist(), a.pos[0].cpu().numpy(), 8, 0.8, 0.9, 40, seed)
        assert res[1] == w[0] and res[2] == w[2] and res[3][0, 0].item() == w[3]
