"""CPU restatement of the sampling acceptance walk (oracle).

Test infrastructure only (see oracle/__init__.py).

The reference's sampling branch (draft/tree_verification.py:103-106) warps
the target logits with the processors of prepare_logits_processor
(:15-32: temperature, then top-p, then top-k, all from transformers), draws
one token per node with torch.multinomial over softmax of the warped logits,
and runs the greedy walk with those draws in place of the argmax.  torch's
RNG cannot be reproduced across implementations, so the draw is restated as
a seeded, counter-based Gumbel-max: token = argmax over kept v of
y_v + G_v, G_v = -ln(-ln U_v), which samples softmax(y) over the kept set
exactly.  Every quantity the decision depends on is computed here with the
same sequence of IEEE-754 double operations the kernel performs (each one
correctly rounded, no fused multiply-add, no library transcendental), so the
kernel's tokens equal these bit for bit.

Definitions (per node row x of the logits, vocabulary V):
  y        x if T == 1, else x / T in float32 rounded to the logits' dtype
           (transformers' TemperatureLogitsWarper on a tensor of that dtype);
           NaN counts as -inf, -0 as +0
  order    descending by (y, index): among equal values the higher index
           ranks first (transformers sorts ascending with a stable sort and
           cuts from the low end)
  q_v      exp(y_v - max y) in fixed point: rint(p * 2^S), S = 63 - bitlen(V),
           p from det_exp2; L = sum q
  top-p    (1e-8 <= top_p < 1) keep v iff (q-mass ranked above v) < Tq,
           Tq = ceil(P * L / 2^32), P = rint(top_p * 2^32): the smallest
           head of the order whose mass reaches top_p (TopPLogitsWarper)
  top-k    (k > 0) keep v iff y_v >= the k-th largest y (with multiplicity),
           applied after top-p, which is the same as intersecting with the
           top-k set of the unfiltered row (TopKLogitsWarper)
  U_v      Philox4x32-10 (Salmon et al. 2011, the Random123 generator) with
           key (seed mod 2^32, seed >> 32) and counter (v >> 2, node, tree, 0):
           output word v & 3, w, gives U = (w + 0.5) * 2^-32 in (0, 1)
  G_v      -det_ln(-det_ln(U_v))
  token    argmax over kept v of y_v + G_v (double), lowest index on ties;
           0 when nothing is kept (a row without a finite logit)
"""

from __future__ import annotations

from typing import List, Sequence, Tuple

import numpy as np

from .accept import _walk, parent_ext
from .attention import bf16_round, half_round

U64 = np.uint64
MASK32 = U64(0xFFFFFFFF)

PHILOX_M0, PHILOX_M1 = 0xD2511F53, 0xCD9E8D57
PHILOX_W0, PHILOX_W1 = 0x9E3779B9, 0xBB67AE85


# ln(2)^k / k!, k = 0..17, and 1 / (2k + 1), k = 0..11, as correctly rounded doubles.
EXP2_C = [float.fromhex(h) for h in (
    "0x1.0000000000000p+0", "0x1.62e42fefa39efp-1", "0x1.ebfbdff82c58fp-3", "0x1.c6b08d704a0c0p-5",
    "0x1.3b2ab6fba4e77p-7", "0x1.5d87fe78a6731p-10", "0x1.430912f86c787p-13", "0x1.ffcbfc588b0c7p-17",
    "0x1.62c0223a5c824p-20", "0x1.b5253d395e7c4p-24", "0x1.e4cf5158b8ecap-28", "0x1.e8cac7351bb25p-32",
    "0x1.c3bd650fc2986p-36", "0x1.816193166d0f9p-40", "0x1.314964d5878a9p-44", "0x1.c36e843b04022p-49",
    "0x1.38e89ae79f8b4p-53", "0x1.98444b41c25a8p-58")]
ATANH_C = [float.fromhex(h) for h in (
    "0x1.0000000000000p+0", "0x1.5555555555555p-2", "0x1.999999999999ap-3", "0x1.2492492492492p-3",
    "0x1.c71c71c71c71cp-4", "0x1.745d1745d1746p-4", "0x1.3b13b13b13b14p-4", "0x1.1111111111111p-4",
    "0x1.e1e1e1e1e1e1ep-5", "0x1.af286bca1af28p-5", "0x1.8618618618618p-5", "0x1.642c8590b2164p-5")]
LN2 = float.fromhex("0x1.62e42fefa39efp-1")
LOG2E = float.fromhex("0x1.71547652b82fep+0")
SQRT_HALF = float.fromhex("0x1.6a09e667f3bcdp-1")


# ----------------------------------------------------------------------------
# Counter-based uniforms
# ----------------------------------------------------------------------------

def philox4x32_10(c0, c1, c2, c3, k0: int, k1: int):
    """Philox4x32 with 10 rounds on arrays of 32-bit counter words (held in
    uint64), key (k0, k1): the four output words."""
    c = [np.asarray(x, dtype=U64) & MASK32 for x in (c0, c1, c2, c3)]
    c = list(np.broadcast_arrays(*c))
    k0, k1 = int(k0) & 0xFFFFFFFF, int(k1) & 0xFFFFFFFF
    for r in range(10):
        if r:
            k0 = (k0 + PHILOX_W0) & 0xFFFFFFFF
            k1 = (k1 + PHILOX_W1) & 0xFFFFFFFF
        p0 = c[0] * U64(PHILOX_M0)          # < 2^64: exact in uint64
        p1 = c[2] * U64(PHILOX_M1)
        c = [(p1 >> U64(32)) ^ c[1] ^ U64(k0), p1 & MASK32, (p0 >> U64(32)) ^ c[3] ^ U64(k1), p0 & MASK32]
    return c


def uniforms(seed: int, tree: int, node: int, V: int) -> np.ndarray:
    """U_v in (0, 1) for v in [0, V) of one node."""
    v = np.arange(V, dtype=U64)
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    words = np.stack(philox4x32_10(v >> U64(2), U64(node), U64(tree), U64(0), seed & 0xFFFFFFFF, seed >> 32))
    w = words[(v & U64(3)).astype(np.int64), np.arange(V)]
    return (w.astype(np.float64) + 0.5) * 2.0 ** -32


# ----------------------------------------------------------------------------
# Deterministic ln and 2^x (single correctly rounded double operations only)
# ----------------------------------------------------------------------------

def det_ln(x: np.ndarray) -> np.ndarray:
    """ln x for finite x > 0: x = m 2^e, m in [sqrt(1/2), sqrt(2)),
    ln m = 2 atanh(s), s = (m - 1) / (m + 1), by Horner in s^2."""
    x = np.asarray(x, dtype=np.float64)
    m, e = np.frexp(x)
    small = m < SQRT_HALF
    m = np.where(small, m * 2.0, m)
    e = np.where(small, e - 1, e).astype(np.float64)
    s = (m - 1.0) / (m + 1.0)
    s2 = s * s
    p = np.full_like(s, ATANH_C[-1])
    for c in ATANH_C[-2::-1]:
        p = p * s2
        p = p + c
    t = s * p
    return e * LN2 + (t + t)


def det_exp2(u: np.ndarray) -> np.ndarray:
    """2^u for u <= 0 (0 below -200 and at -inf): u = n + f, f in [0, 1),
    2^f = sum (f ln 2)^k / k! by Horner in f, then scaled by 2^n."""
    u = np.asarray(u, dtype=np.float64)
    low = ~(u >= -200.0)
    uu = np.where(low, 0.0, u)
    n = np.floor(uu)
    f = uu - n
    p = np.full_like(f, EXP2_C[-1])
    for c in EXP2_C[-2::-1]:
        p = p * f
        p = p + c
    return np.where(low, 0.0, np.ldexp(p, n.astype(np.int64)))


# ----------------------------------------------------------------------------
# Warpers and the kept set
# ----------------------------------------------------------------------------

def warp_temperature(x: np.ndarray, temperature: float, dtype: str) -> np.ndarray:
    """y = x / T in float32 rounded to the logits dtype ('bf16', 'f16', 'f32');
    T == 1 leaves x as it is.  NaN -> -inf, -0 -> +0."""
    x = np.asarray(x, dtype=np.float32)
    if temperature != 1.0:
        y = x / np.float32(temperature)
        y = bf16_round(y) if dtype == "bf16" else (half_round(y) if dtype == "f16" else y)
    else:
        y = x
    y = np.where(np.isnan(y), -np.inf, y).astype(np.float32)
    return np.where(y == 0, np.float32(0.0), y).astype(np.float64)


def fixed_masses(y: np.ndarray) -> np.ndarray:
    """q_v = rint(exp(y_v - max y) * 2^S), S = 63 - bitlen(V); y == max gives 2^S."""
    V = y.size
    S = 63 - int(V).bit_length()
    m = y.max()
    if not np.isfinite(m) and m < 0:
        return np.zeros(V, dtype=U64)
    with np.errstate(invalid="ignore"):  # m = +inf: inf - inf where y == m, replaced by 0
        d = np.where(y == m, 0.0, y - m)
    p = det_exp2(d * LOG2E)
    return np.rint(np.ldexp(p, S)).astype(U64)


def top_p_threshold(L: int, top_p: float) -> int:
    P = int(np.rint(np.float64(np.float32(top_p)) * 2.0 ** 32))
    return (P * int(L) + (1 << 32) - 1) >> 32


def kept_mask(y: np.ndarray, top_p: float, top_k: int) -> np.ndarray:
    """The kept set of the warpers (module docstring), by an explicit sort."""
    V = y.size
    keep = np.ones(V, dtype=bool)
    if 1e-8 <= top_p < 1.0:
        q = fixed_masses(y)
        Tq = top_p_threshold(int(q.sum(dtype=U64)), top_p)
        order = np.lexsort((np.arange(V), y))[::-1]          # descending (y, index)
        qs = q[order]
        above = np.concatenate([np.zeros(1, dtype=U64), np.cumsum(qs, dtype=U64)[:-1]])
        k = np.zeros(V, dtype=bool)
        k[order] = above < U64(Tq)
        keep &= k
    if top_k > 0:
        kk = min(int(top_k), V)
        kth = np.sort(y)[::-1][kk - 1]
        keep &= y >= kth
    return keep


def sample_row(x: np.ndarray, dtype: str, temperature: float, top_p: float, top_k: int, seed: int, tree: int,
               node: int) -> int:
    """The sampled token of one node row."""
    y = warp_temperature(x, temperature, dtype)
    keep = kept_mask(y, top_p, top_k) & (y > -np.inf)
    if not keep.any():
        return 0
    g = -det_ln(-det_ln(uniforms(seed, tree, node, y.size)))
    z = np.where(keep, y + g, -np.inf)
    return int(np.argmax(z))


def sample_walk(logits: np.ndarray, dtype: str, draft: Sequence[int], parent_ref: Sequence[int],
                pos: Sequence[int], max_depth: int, temperature: float, top_p: float, top_k: int, seed: int,
                tree: int = 0) -> Tuple[List[int], List[int], int, int, int, np.ndarray]:
    """The walk of draft/tree_verification.py:100-182 with sampled next tokens.

    Returns (best_candidate, best_candidate_id, accept_length, next_token,
    max_id, per-node samples)."""
    logits = np.asarray(logits)
    M = logits.shape[0]
    samples = np.array([sample_row(logits[i], dtype, temperature, top_p, top_k, seed, tree, i) for i in range(M)],
                       dtype=np.int64)
    draft = np.asarray(draft, dtype=np.int64)
    pe = parent_ext(parent_ref)
    ok = draft == samples[pe]
    return (*_walk(ok, pe, np.asarray(pos, dtype=np.int64), max_depth, draft, samples), samples)
