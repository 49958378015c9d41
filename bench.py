#!/usr/bin/env python3
"""Benchmark of the tree-verification hot path on one MI355X.

Workload (the headline configuration): one layer of bf16 tree verification,
Llama-3.1-8B attention shape (32 query heads, 8 KV heads, head_dim 128),
batch 1, a 65536-token prefix in 16-token pages behind a random-permutation
page table, a 64-node draft tree (parents from the seeded generator, depth
<= 8, out-degree <= 4) whose K/V follow the prefix in the same pages.  One
step = the fused verify: kernel 1 (split-K flash-decoding over the pages plus
the ancestor-masked tree split) and kernel 3 (LSE merge) -> O [64, 32, 128]
bf16 + LSE [64, 32].  Four distinct KV layers are rotated so the 256 MiB
per-layer K/V set is not served from the 256 MB Infinity Cache.

Also measured (extra fields): the acceptance kernel on 8 trees x 64 nodes x
vocab 128256 bf16 (greedy, typical, sampling), the 128K / 128-node
bundle-packed verify, the 32-layer Llama-3.1-8B-shaped step, and the CPU
baseline — the reference's own torch CPU path (repeat_kv -> fp32
matmul/softmax/logsumexp prefix -> naive tree -> sigmoid merge) on the same
workload, its greedy walk, and the 4096-token fp32 layer, timed on the host
cores.

Prints ONE JSON line.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "specdiff-ae_amd"))
sys.path.insert(0, str(REPO))

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD public spec

# Untimed continuous load before every timed measurement (set by --settle-ms).
# After an idle gap the GPU first runs at a boost clock for about 2 ms, then
# 25-50 % slower for 10-20 ms while its power management settles, then at the
# steady state a serving loop sees; each measurement starts in the last.
SETTLE_MS = 60.0


def settle(fn, ms=None, batch=10):
    """Runs fn untimed, `batch` calls between synchronisations, for about
    `ms` milliseconds (SETTLE_MS by default)."""
    ms = SETTLE_MS if ms is None else ms
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(batch):
            fn()
        torch.cuda.synchronize()


def algorithmic_bytes(n_prefix, M, H, Hk, D, elem=2, out_elem=2, page_size=16):
    kv = 2 * n_prefix * Hk * D * elem
    q = M * H * D * elem
    tree_kv = 2 * M * Hk * D * elem
    o = M * H * D * out_elem
    lse = 4 * M * H
    pt = 4 * ((n_prefix + M + page_size - 1) // page_size)
    return {"step": kv + q + tree_kv + o + lse + pt, "kernel1": kv + q + tree_kv + pt, "prefix_kv": kv}


class HipEvents:
    """hipEvent_t pairs from the HIP runtime torch loaded (same soname)."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self, n):
        evs = []
        for _ in range(n):
            e = ctypes.c_void_p()
            rc = self.hip.hipEventCreate(ctypes.byref(e))
            if rc != 0:
                raise RuntimeError(f"hipEventCreate failed ({rc})")
            evs.append(e)
        return evs

    def record(self, e, stream):
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        rc = self.hip.hipEventRecord(e, ctypes.c_void_p(stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        rc = self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def destroy(self, evs):
        for e in evs:
            self.hip.hipEventDestroy(e)


def measured_traffic():
    """HBM bytes per kernel-1 launch from the committed rocprofv3 counter passes.

    profiles/attn_splitk_64k_traffic.json holds FETCH_SIZE and WRITE_SIZE (KiB
    per dispatch) of kernel 1 on this workload and of a 1 GiB device copy, with
    the commands that produced them; each counter is scaled by bytes / counter
    of the copy.  Returns None when the file is absent.
    """
    f = REPO / "profiles" / "attn_splitk_64k_traffic.json"
    if not f.exists():
        return None
    d = json.loads(f.read_text())
    return int(d["kernel_fetch_kib"] * 1024 * d["fetch_scale"] + d["kernel_write_kib"] * 1024 * d["write_scale"])


def bench_verify(args, lib, ev):
    from diffspec_mi355x import workloads as wl
    from diffspec_mi355x.runtime.tree_attention import tree_verify

    n_prefix, M, H, Hk, D = args.n_prefix, args.nodes, 32, 8, 128
    inp = wl.make_tree_verify_inputs(n_prefix=n_prefix, M=M, H=H, Hk=Hk, D=D, layers=args.layers,
                                     device="cuda", seed=0, tree_seed=0)
    par = torch.tensor(inp.parent, dtype=torch.int64, device="cuda")
    pools = [(inp.kv_pages[l, 0], inp.kv_pages[l, 1]) for l in range(args.layers)]

    def step(i, arm=None):
        if arm is not None:
            lib.dsv_set_timing_events(arm[0], arm[1])
        k, v = pools[i % len(pools)]
        return tree_verify(inp.q, k, v, n_prefix, par, page_table=inp.page_table)

    # Settle (untimed steps for args.settle_ms), then the W warm-up steps,
    # then the K timed ones.
    it = iter(range(1 << 62))
    settle(lambda: step(next(it)), args.settle_ms, batch=20)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # Timed region: K whole steps (kernel 1 + kernel 3), device clock.
    st0, st1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    st0.record()
    for i in range(args.steps):
        step(i)
    st1.record()
    torch.cuda.synchronize()
    t_wall = time.perf_counter() - t_wall
    total_ms = st0.elapsed_time(st1)

    # Kernel 1 alone: a second pass of K steps with a HIP event pair attached
    # to every kernel-1 launch (hipExtLaunchKernel start/stop events on the
    # launch stream: the kernel's own start and end).  Timed events cost the
    # step a few us, which is why they stay out of the pass above.
    k1 = ev.create(2 * args.steps)
    se0, se1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    se0.record()
    for i in range(args.steps):
        step(i, arm=(k1[2 * i], k1[2 * i + 1]))
    se1.record()
    torch.cuda.synchronize()
    k1_ms = [ev.elapsed_ms(k1[2 * i], k1[2 * i + 1]) for i in range(args.steps)]
    ev.destroy(k1)
    return inp, total_ms / args.steps, k1_ms, t_wall, se0.elapsed_time(se1) / args.steps


def bench_prefix_sweep(args, lib, ev):
    """The metric's step (64 nodes, H 32, Hk 8, D 128, paged bf16) over prefix
    lengths from 4K to 512K tokens, with enough KV layers rotated that the
    layers together exceed the 256 MB Infinity Cache: us per step, kernel 1
    (launch-attached events) and its algorithmic HBM rate."""
    import types
    rows = []
    for n in (4096, 16384, 65536, 262144, 524288):
        per_layer = 2 * n * 8 * 128 * 2
        layers = max(1, min(24, -(-320 * 2 ** 20 // per_layer)))
        sub = types.SimpleNamespace(**vars(args))
        sub.n_prefix, sub.layers = n, layers
        print(f"[bench] prefix sweep: N={n} layers={layers}", file=sys.stderr, flush=True)
        inp, ms_step, k1_ms, _, _ = bench_verify(sub, lib, ev)
        del inp
        torch.cuda.empty_cache()
        nb = algorithmic_bytes(n, args.nodes, 32, 8, 128)["kernel1"]
        k1 = statistics.mean(k1_ms) * 1e3
        rows.append({"n_prefix": n, "kv_layers_rotated": layers, "us_per_step": round(ms_step * 1e3, 2),
                     "kernel1_us": round(k1, 2), "kernel1_hbm_gbs": round(nb / (k1 * 1e-6) / 1e9, 1),
                     "kernel1_hbm_frac": round(nb / (k1 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
    return rows


def bench_bundle_packed_128k(args, lib, ev):
    """128K paged prefix, 128-node tree (depth <= 12, out-degree <= 6), query
    rows packed in bundle order (8 bundles).  MFMA-bound: 512 flop/B.  A step
    computes the bundle order on the GPU from the device parent array
    (dsv_bundle_order), then runs the fused verify with it."""
    from diffspec_mi355x import workloads as wl
    from diffspec_mi355x.core.bundle_scheduler import bundle_row_order, bundle_row_order_device
    from diffspec_mi355x.runtime.tree_attention import tree_verify

    N, M, H, Hk, D, layers = 131072, 128, 32, 8, 128, 3
    inp = wl.make_tree_verify_inputs(n_prefix=N, M=M, H=H, Hk=Hk, D=D, layers=layers, device="cuda", seed=2,
                                     tree_seed=2, max_depth=12, max_outdeg=6)
    par = torch.tensor(inp.parent, dtype=torch.int64, device="cuda")
    host_perm = torch.tensor(bundle_row_order(inp.parent, num_bundles=8), dtype=torch.int32, device="cuda")
    if not torch.equal(bundle_row_order_device(par, num_bundles=8), host_perm):
        raise RuntimeError("device bundle order differs from the host scheduler's")
    pools = [(inp.kv_pages[l, 0], inp.kv_pages[l, 1]) for l in range(layers)]

    def step(i, arm=None):
        perm = bundle_row_order_device(par, num_bundles=8)
        if arm is not None:
            lib.dsv_set_timing_events(arm[0], arm[1])
        k, v = pools[i % layers]
        return tree_verify(inp.q, k, v, N, par, page_table=inp.page_table, row_perm=perm, check_row_perm=False)

    n = 20
    it = iter(range(1 << 62))
    settle(lambda: step(next(it)), args.settle_ms, batch=5)
    for i in range(10):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(n):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    us_step = e0.elapsed_time(e1) / n * 1e3
    evs = ev.create(2 * n)
    for i in range(n):
        step(i, arm=(evs[2 * i], evs[2 * i + 1]))
    torch.cuda.synchronize()
    k1_us = statistics.mean(ev.elapsed_ms(evs[2 * i], evs[2 * i + 1]) for i in range(n)) * 1e3
    ev.destroy(evs)
    # Bundle order: device time per launch vs the host scheduler + copy.
    order_us = device_us(lambda: bundle_row_order_device(par, num_bundles=8))
    t0 = time.perf_counter()
    reps = 20
    for _ in range(reps):
        hp = torch.tensor(bundle_row_order(par.tolist(), num_bundles=8), dtype=torch.int32).to("cuda")
    torch.cuda.synchronize()
    host_us = (time.perf_counter() - t0) / reps * 1e6
    nb = algorithmic_bytes(N, M, H, Hk, D)
    flops = 4 * M * H * N * D + 4 * M * H * M * D
    # the tree block counted over visible keys only: 4*H*D * sum_i |anc(i)|
    anc = [0] * M
    for i in range(M):
        j, c = i, 0
        while j >= 0 and c <= M:
            c += 1
            j = inp.parent[j] if j > 0 else -1
        anc[i] = c
    flops_masked = 4 * M * H * N * D + 4 * H * D * sum(anc)
    return {"workload": "tree-verify attention, N=131072, M=128 (8 bundles, row-packed), paged bf16 KV, "
                        f"{layers} KV layers rotated", "us_per_step": round(us_step, 3),
            "kernel1_avg_us": round(k1_us, 3), "kernel1_tflops": round(flops / (k1_us * 1e-6) / 1e12, 1),
            "kernel1_mfma_frac": round(flops / (k1_us * 1e-6) / 2.5e15, 4),
            "kernel1_hbm_gbs": round(nb["kernel1"] / (k1_us * 1e-6) / 1e9, 1),
            "kernel1_hbm_frac": round(nb["kernel1"] / (k1_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "flops_dense": flops, "flops_masked": flops_masked, "bytes_per_launch": nb["kernel1"],
            "bundle_order": {"device_us": round(order_us, 2),
                             "host_scheduler_us": round(host_us, 1),
                             "timing": "device: HIP graph replay; host: parent to host, Python "
                                       "scheduler, permutation to the device"}}


def device_us(fn, calls=10, reps=20):
    """Device time per call of fn: `calls` calls captured once in a HIP graph,
    replayed `reps` times (host launch cost excluded) after the graph has been
    replayed untimed for SETTLE_MS.  fn records no memset nodes."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(calls):
            fn()
    g.replay()
    torch.cuda.synchronize()
    settle(g.replay, batch=1)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (reps * calls) * 1e3


def bench_llama8b_step(args, lib, ev):
    """One verify step of a Llama-3.1-8B-shaped target (32 layers, hidden 4096,
    32/8 heads, FFN 14336, vocab 128256, RoPE theta 5e5) over a 64-node tree
    with a 65536-token paged prefix per layer, random N(0, 0.02) bf16 weights
    (workloads.LlamaVerifyStep).  The draft is planted along the root path of
    a deepest node from the target's own argmax, so the walk accepts that
    path.  Per layer: RMSNorm, QKV projection, RoPE + tree K/V into the pages
    (dsv_kv_append), the fused tree verify (kernels 1 and 3), o_proj, RMSNorm,
    SwiGLU MLP; then the final norm and the lm_head fused with the greedy walk
    (kernel 5 + kernel 4's walk).  Projections, norms and the MLP are torch
    (hipBLASLt) ops: measurement scaffolding around the hot path."""
    from diffspec_mi355x import workloads as wl
    from diffspec_mi355x.runtime.cache_state import append_tree_kv
    from diffspec_mi355x.runtime.tree_attention import tree_verify

    st = wl.LlamaVerifyStep(device="cuda")
    path = st.plant_path()
    inp, N, M, L, H, Hk, D = st.inp, st.N, st.M, st.L, st.H, st.Hk, st.D
    for _ in range(3):
        r = st.step()
    torch.cuda.synchronize()
    settle(st.step, batch=1)
    n = 10
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n):
        r = st.step()
    e1.record()
    torch.cuda.synchronize()
    us_eager = e0.elapsed_time(e1) / n * 1e3
    # Device time of the step: the whole 32-layer step captured in a HIP graph
    # and replayed (Python launch overhead excluded; eager launching leaves the
    # GPU idle between this scaffolding's small torch ops).
    us_step = device_us(st.step, calls=1, reps=5)
    # Attention's device time inside the step: in eager steps, each layer's
    # fused verify (kernels 1 and 3, over that layer's own KV pages) is timed
    # from a HIP event attached to its kernel-1 launch (the kernel's start)
    # to an event recorded on the stream right after the call (after kernel
    # 3).  The host enqueues kernel 3 and that event while kernel 1 runs, so
    # the interval holds no host gap.
    attn_steps = []
    stream = torch.cuda.current_stream().cuda_stream
    for _ in range(3):
        evs = ev.create(3 * L)

        def hook(l, phase):
            if phase == 0:
                lib.dsv_set_timing_events(evs[3 * l], evs[3 * l + 1])
            else:
                ev.record(evs[3 * l + 2], stream)

        st.step(verify_hook=hook)
        torch.cuda.synchronize()
        attn_steps.append([ev.elapsed_ms(evs[3 * l], evs[3 * l + 2]) * 1e3 for l in range(L)])
        ev.destroy(evs)
    per_layer = [statistics.median(s_[l] for s_ in attn_steps) for l in range(L)]
    attn_us = sum(per_layer)
    commit = bench_commit(inp, N, M, L, Hk, D, n)
    # The append alone (one layer): q/k RoPE + tree K/V into the pages, one
    # launch, against the reference's ops (RoPE of q and k in bf16 torch ops,
    # then the K/V writes into the pages).
    x0 = st.embed[st.draft[0]]
    qkv = st.rms(x0) @ st.layers[0]["qkv"].T
    qs, ks, vs = (qkv[:, :H * D].view(M, H, D), qkv[:, H * D:(H + Hk) * D].view(M, Hk, D),
                  qkv[:, (H + Hk) * D:].view(M, Hk, D))
    tok = torch.arange(N, N + M, device="cuda")
    phys = inp.page_table.long()[tok // inp.page_size]
    slot = tok % inp.page_size

    def rope_ref(t):  # the reference's op sequence on [M, heads, D]
        c, s_ = st.cos[:, None, :], st.sin[:, None, :]
        return (t * c) + (torch.cat((-t[..., D // 2:], t[..., :D // 2]), -1) * s_)

    def ours():
        append_tree_kv(ks, vs, inp.kv_pages[0, 0], inp.kv_pages[0, 1], N, cos=st.cos, sin=st.sin,
                       page_table=inp.page_table, q=qs)

    def theirs():
        rope_ref(qs)
        inp.kv_pages[0, 0][phys, :, slot, :] = rope_ref(ks)
        inp.kv_pages[0, 1][phys, :, slot, :] = vs

    app = {"us": round(device_us(ours), 2), "reference_ops_us": round(device_us(theirs), 2),
           "timing": "device time per call, HIP graph of 10 calls replayed"}
    lmh = bench_lmhead(st)
    wbytes = sum(t.numel() * 2 for W in st.layers for t in W.values()) + st.lm_head.numel() * 2
    kvbytes = L * algorithmic_bytes(N, M, H, Hk, D)["prefix_kv"]
    alen = int(r["info"][0, 1])
    return {"workload": "Llama-3.1-8B-shaped verify step: 32 layers, 64-node tree, 65536-token paged prefix per "
                        "layer, random bf16 weights, draft planted along a root path, lm_head + greedy acceptance",
            "us_per_step": round(us_step, 1), "us_per_step_eager": round(us_eager, 1),
            "timing": "us_per_step: device time of the step, HIP graph replayed; us_per_step_eager: eager "
                      "launches (host-bound: the torch scaffolding's launches leave the GPU idle)",
            "attention_us_per_step": round(attn_us, 1), "attention_share": round(attn_us / us_step, 3),
            "attention_us_per_layer": {"min": round(min(per_layer), 2), "median": round(statistics.median(per_layer), 2),
                                       "max": round(max(per_layer), 2)},
            "attention_timing": "sum over the 32 layers of each layer's fused verify inside the step (its own KV "
                                "pages): kernel-1 start event to an event after kernel 3, median of 3 eager steps",
            "weight_bytes": wbytes, "kv_bytes": kvbytes,
            "hbm_gbs": round((wbytes + kvbytes) / (us_step * 1e-6) / 1e9, 1),
            "planted_path_len": len(path), "accept_length": alen,
            "tokens_per_s": round((alen + 1) / (us_step * 1e-6), 1),
            "lmhead_accept_share": round(lmh["fused_us"] / us_step, 4), "kv_commit": commit,
            "kv_append_one_layer": dict(app, bytes=(M * (H + 2 * Hk) * D * 2) * 2), "lmhead_accept": lmh}


def bench_lmhead(st):
    """lm_head + greedy acceptance of a 64-node tree (Dm 4096, V 128256):
    the fused kernel against torch's lm_head (hipBLASLt, x @ W^T) followed by
    kernel 4 on the materialised bf16 logits.  Agreement of the fused walk
    with the walk over torch's logits is counted over 8 seeds of hidden
    states (per-node next tokens, and whole results: path, tokens, info)."""
    from diffspec_mi355x.draft.tree_verification import lmhead_tree_accept, tree_accept

    xn = st.rms(st.embed[st.draft[0]])
    V, hid = st.lm_head.shape
    M = xn.shape[0]
    args = (st.draft, st.pref, st.pos, st.max_hops)
    fused = device_us(lambda: lmhead_tree_accept(xn.unsqueeze(0), st.lm_head, *args), calls=5, reps=10)
    mm = device_us(lambda: xn @ st.lm_head.T, calls=5, reps=10)
    unfused = device_us(lambda: tree_accept((xn @ st.lm_head.T).unsqueeze(0), *args), calls=5, reps=10)
    nb = V * hid * 2 + M * hid * 2
    same_next, same_walk, nodes = 0, 0, 0
    g = torch.Generator(device="cuda")
    for seed in range(8):
        g.manual_seed(100 + seed)
        h = st.rms(torch.randn((M, hid), generator=g, device="cuda").to(torch.bfloat16))
        rf = lmhead_tree_accept(h.unsqueeze(0), st.lm_head, *args, return_next=True)
        ru = tree_accept((h @ st.lm_head.T).unsqueeze(0), *args, return_next=True)
        same_next += int((rf["next"] == ru["next"]).sum())
        nodes += M
        same_walk += int(torch.equal(rf["info"], ru["info"]) and torch.equal(rf["path"], ru["path"])
                         and torch.equal(rf["tokens"], ru["tokens"]))
    return {"workload": "lm_head [128256 x 4096] bf16 over 64 tree nodes + greedy walk",
            "fused_us": round(fused, 2), "torch_lm_head_us": round(mm, 2),
            "torch_lm_head_plus_kernel4_us": round(unfused, 2), "bytes": nb,
            "fused_hbm_gbs": round(nb / (fused * 1e-6) / 1e9, 1),
            "fused_hbm_frac": round(nb / (fused * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "next_token_agreement_with_torch_logits": round(same_next / nodes, 4),
            "walk_agreement_with_torch_logits": f"{same_walk}/8 seeds",
            "timing": "device time per call, HIP graph of 5 calls replayed"}


def bench_commit(inp, N, M, L, Hk, D, n):
    """Accepted-path KV commit over all 32 layers of the page pool, path of 9
    nodes (depth 8) from device memory, against the reference's op sequence
    (per layer and K/V cache: gather of the selected rows, copy to the front;
    draft/tree_verification.py:197-217) on dense caches of the same rows."""
    from diffspec_mi355x.draft.tree_verification import kv_commit

    path_nodes = [0, 1, 3, 7, 12, 20, 33, 47, 60]
    path = torch.full((1, M), -1, dtype=torch.int64, device="cuda")
    path[0, :len(path_nodes)] = torch.tensor(path_nodes, device="cuda")
    info = torch.tensor([[path_nodes[-1], len(path_nodes) - 1, 0, len(path_nodes)]], dtype=torch.int64, device="cuda")
    us = device_us(lambda: kv_commit(inp.kv_pages, N, path, info, page_table=inp.page_table))
    # The reference's sequence on dense per-layer caches [2, 1, Hk, S, D]
    # holding the same rows (S = the tree's slots plus a prefix tail).
    S, start = 1024, 1024 - M
    dense = [torch.randn((2, 1, Hk, S, D), device="cuda").to(torch.bfloat16) for _ in range(L)]
    sel = torch.tensor(path_nodes, dtype=torch.long, device="cuda") + start

    def ref():
        for data in dense:
            tgt = data[..., sel, :]
            data[..., start:start + sel.numel(), :].copy_(tgt, non_blocking=True)

    us_ref = device_us(ref, calls=2)
    moved = 2 * L * 2 * Hk * len(path_nodes) * D * 2
    return {"layers": L, "path_nodes": len(path_nodes), "bytes_moved": moved, "us": round(us, 2),
            "reference_ops_us": round(us_ref, 1), "reference_ops_launches": 2 * L,
            "timing": "device time per call, HIP graph replayed"}


def bench_fp32_4k():
    """The 4096-token fp32 layer on the GPU: N=4096, M=64, GQA 32/8, D=128,
    Q / K-V prefix / K-V tree drawn N(0, 1) fp32 in that order (seed 0), the
    64-node tree; fp32 tensors straight into the fp32 kernel (kernel 1's fp32
    variant + kernel 3).  Then the greedy walk over [1, 64, 128256] fp32
    N(0, 3) logits (seed 1) with uniform draft tokens.  Device time per call,
    HIP graph replayed."""
    from diffspec_mi355x import workloads as wl
    from diffspec_mi355x.draft.tree_verification import tree_accept
    from diffspec_mi355x.runtime.tree_attention import tree_verify

    g = torch.Generator().manual_seed(0)
    M, H, Hk, D, N = 64, 32, 8, 128, 4096
    q = torch.randn(1, M, H, D, generator=g)
    kp, vp = torch.randn(1, N, Hk, D, generator=g), torch.randn(1, N, Hk, D, generator=g)
    kt, vt = torch.randn(1, M, Hk, D, generator=g), torch.randn(1, M, Hk, D, generator=g)
    parent, depth = wl.make_tree(M, seed=0)
    q, kc, vc = q.cuda(), torch.cat([kp, kt], 1).cuda(), torch.cat([vp, vt], 1).cuda()
    par = torch.tensor(parent, dtype=torch.int64, device="cuda")
    attn = device_us(lambda: tree_verify(q, kc, vc, N, par, out_dtype=torch.float32))
    g = torch.Generator().manual_seed(1)
    V = 128256
    logits = (torch.randn((1, M, V), generator=g) * 3.0).cuda()
    draft = torch.randint(0, V, (1, M), generator=g).cuda()
    pref = torch.tensor([wl.parent_to_reference(parent)], dtype=torch.int64, device="cuda")
    pos = torch.tensor(depth, dtype=torch.int64, device="cuda")
    walk = device_us(lambda: tree_accept(logits, draft, pref, pos, 10))
    flops = 4 * M * H * (N + M) * D
    return {"workload": "tree-verify attention, 1 layer, N=4096, M=64, fp32 dense KV; greedy walk over "
                        "[1, 64, 128256] fp32 logits",
            "attention_us": round(attn, 2), "greedy_walk_us": round(walk, 2), "total_us": round(attn + walk, 2),
            "attention_tflops_fp32": round(flops / (attn * 1e-6) / 1e12, 1),
            "timing": "device time per call, HIP graph of 10 calls replayed"}


def bench_accept(args, lib, ev):
    from diffspec_mi355x import workloads as wl
    from diffspec_mi355x.draft.tree_verification import tree_accept

    T, M, V = 8, 64, 128256
    a = wl.make_accept_inputs(T=T, M=M, V=V, device="cuda", pos_offset=65536)
    res = {}
    kws = {"greedy": {}, "typical": {}, "sample": dict(temperature=0.7, top_p=0.9, top_k=50, seed=1234),
           "sample_temperature_only": dict(temperature=0.7, seed=1234)}
    for name, kw in kws.items():
        mode = "sample" if name.startswith("sample") else name
        for _ in range(3):
            tree_accept(a.logits, a.draft, a.parent_ref, a.pos, 10, mode=mode, **kw)
        torch.cuda.synchronize()
        settle(lambda: tree_accept(a.logits, a.draft, a.parent_ref, a.pos, 10, mode=mode, **kw))
        n = 20
        evs = ev.create(2 * n)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(n):
            lib.dsv_set_timing_events(evs[2 * i], evs[2 * i + 1])
            r = tree_accept(a.logits, a.draft, a.parent_ref, a.pos, 10, mode=mode, **kw)
        e1.record()
        torch.cuda.synchronize()
        sweep = statistics.median(ev.elapsed_ms(evs[2 * i], evs[2 * i + 1]) for i in range(n))
        ev.destroy(evs)
        # Device time of the whole call (sweep + walk kernels), free of the
        # host-side launch cost: 10 calls captured in a HIP graph and the graph
        # replayed (the acceptance path records no memset nodes); every
        # captured call's result is checked against the eager one.
        per_graph, replays = 10, 4
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            rgs = [tree_accept(a.logits, a.draft, a.parent_ref, a.pos, 10, mode=mode, **kw) for _ in range(per_graph)]
        g.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(x["info"], r["info"]) for x in rgs), "graph replay differs from the eager call"
        e2, e3 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e2.record()
        for i in range(replays):
            g.replay()
        e3.record()
        torch.cuda.synchronize()
        assert all(torch.equal(x["info"], r["info"]) for x in rgs), "graph replay differs from the eager call"
        res[name] = {"us_total": e2.elapsed_time(e3) / (replays * per_graph) * 1e3,
                     "us_total_eager": e0.elapsed_time(e1) / n * 1e3,
                     "us_vocab_sweep": sweep * 1e3, "accept_lengths": r["info"][:, 1].tolist()}
        if mode == "sample":
            res[name]["params"] = {k: v for k, v in kw.items() if k != "seed"}
    nbytes = T * M * V * 2
    for mode in res:
        res[mode]["sweep_gbs"] = nbytes / (res[mode]["us_vocab_sweep"] * 1e-6) / 1e9
    return res


def _cpu_median_us(fn, seconds, max_runs):
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or not times:
        t0 = time.perf_counter()
        out = fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= max_runs:
            break
    return statistics.median(times) * 1e6, len(times), out


def cpu_baseline(inp, args):
    """The reference's CPU path (oracle/ref_cpu_path.py), bounded samples:
    the verify attention of the same layer (repeat_kv -> fp32 prefix ->
    naive tree -> sigmoid merge), the greedy walk over [1, 64, 128256] fp32
    N(0, 3) logits (seed 1; draft/tree_verification.py:100-182), and the
    4096-token fp32 layer (seed 0) with the same walk."""
    from diffspec_mi355x import workloads as wl
    from oracle import ref_cpu_path as rc
    from oracle import attention as oa

    # Every core of the affinity mask, unless the machine caps this process's
    # CPU share through OMP_NUM_THREADS (a shared host may give each GPU's
    # process a fixed number of threads).
    affinity = len(os.sched_getaffinity(0))
    cores = min(affinity, int(os.environ.get("OMP_NUM_THREADS", affinity)))
    torch.set_num_threads(cores)
    n_prefix, M = inp.n_prefix, inp.M
    k = inp.logical_kv(0, 0)[0].float().cpu().transpose(0, 1).unsqueeze(0).contiguous()  # [1, Hk, L, D]
    v = inp.logical_kv(0, 1)[0].float().cpu().transpose(0, 1).unsqueeze(0).contiguous()
    q = inp.q.float().cpu()
    mask = rc.additive_tree_mask(torch.from_numpy(oa.ancestor_mask(inp.parent)))
    attn_us, n_attn, out = _cpu_median_us(lambda: rc.hybrid_verify_cpu(q, k, v, n_prefix, mask), args.cpu_seconds,
                                          args.cpu_max_steps)
    del k, v

    # The greedy walk of one step: logits [1, 64, 128256] fp32 N(0, 3), seed 1,
    # uniform draft tokens (seed 1), the 64-node tree of the generator.
    V = 128256
    g = torch.Generator().manual_seed(1)
    logits = torch.randn((1, M, V), generator=g) * 3.0
    draft = torch.randint(0, V, (1, M), generator=g)
    parent, depth = wl.make_tree(M, seed=0)
    pref = torch.tensor(wl.parent_to_reference(parent), dtype=torch.int64)
    pos = torch.tensor(depth, dtype=torch.int64)
    walk_us, n_walk, _ = _cpu_median_us(lambda: rc.greedy_walk_torch(logits, draft, pref, pos, 8), 3.0, 20)

    # The 4096-token fp32 layer: Q, K/V prefix, K/V tree drawn N(0, 1) in that
    # order (seed 0), GQA 32/8, D 128, the same 64-node tree.
    g = torch.Generator().manual_seed(0)
    H, Hk, D, N1 = 32, 8, 128, 4096
    q1 = torch.randn(1, M, H, D, generator=g)
    kp, vp = torch.randn(1, N1, Hk, D, generator=g), torch.randn(1, N1, Hk, D, generator=g)
    kt, vt = torch.randn(1, M, Hk, D, generator=g), torch.randn(1, M, Hk, D, generator=g)
    k1 = torch.cat([kp, kt], 1).transpose(1, 2).contiguous()
    v1 = torch.cat([vp, vt], 1).transpose(1, 2).contiguous()
    mask1 = rc.additive_tree_mask(torch.from_numpy(oa.ancestor_mask(parent)))
    c1_us, n_c1, _ = _cpu_median_us(lambda: rc.hybrid_verify_cpu(q1, k1, v1, N1, mask1), 3.0, 20)
    return {"value": attn_us, "unit": "us/verify-step", "cores": cores,
            "affinity_cores": affinity, "threads": torch.get_num_threads(), "kind": "port",
            "sample": f"{n_attn} full verify steps (1 layer, N={n_prefix}, M={M}, bf16 inputs upcast to fp32), "
                      f"median",
            "greedy_walk_us": round(walk_us, 1),
            "greedy_walk_sample": f"{n_walk} walks over [1, {M}, {V}] fp32 N(0, 3) logits (seed 1), median",
            "value_with_walk_us": round(attn_us + walk_us, 1),
            "config_4096_fp32": {"attention_us": round(c1_us, 1), "greedy_walk_us": round(walk_us, 1),
                                 "total_us": round(c1_us + walk_us, 1),
                                 "sample": f"{n_c1} verify steps (1 layer, N=4096, M=64, fp32 N(0, 1), seed 0), "
                                           f"median; the walk as above"}}, out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--settle-ms", type=float, default=60.0,
                    help="untimed continuous load before the warm-up steps (clock ramp)")
    ap.add_argument("--n-prefix", type=int, default=65536)
    ap.add_argument("--nodes", type=int, default=64)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--cpu-max-steps", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-accept", action="store_true")
    ap.add_argument("--no-bundle-128k", action="store_true")
    ap.add_argument("--no-llama-step", action="store_true")
    ap.add_argument("--no-prefix-sweep", action="store_true",
                    help="skip the step at prefix lengths 4K to 512K (prefix_sweep)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device-to-device copy (scale reference for the FETCH_SIZE / WRITE_SIZE "
                         "counters) and exit")
    args = ap.parse_args()
    global SETTLE_MS
    SETTLE_MS = args.settle_ms
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (got --gpus {args.gpus}). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)

    if args.copy_calibration:
        n = 1 << 30
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": n, "copy_calibration_bytes_written": n}), flush=True)
        return

    from diffspec_mi355x import _ext

    lib = _ext.load()
    ev = HipEvents()
    print(f"[bench] verify: N={args.n_prefix} M={args.nodes} steps={args.steps} warmup={args.warmup}", file=sys.stderr,
          flush=True)
    inp, ms_step, k1_ms, t_wall, ms_step_ev = bench_verify(args, lib, ev)
    nb = algorithmic_bytes(args.n_prefix, args.nodes, 32, 8, 128)
    us_step = ms_step * 1e3
    k1_us = statistics.mean(k1_ms) * 1e3
    k1_med = statistics.median(k1_ms) * 1e3
    achieved = nb["kernel1"] / (k1_us * 1e-6) / 1e9
    line = {
        "metric": "verify-step us & HBM GB/s (% peak) at 64K ctx, 64-node tree, 1 MI355X",
        "value": round(us_step, 3),
        "unit": "us/verify-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)*0.5 Q/K/V, random-permutation page table, generated tree)",
        "config": {"workload": "tree-verify attention, 1 layer, paged bf16 KV", "n_prefix": args.n_prefix,
                   "tree_nodes": args.nodes, "q_heads": 32, "kv_heads": 8, "head_dim": 128, "page_size": 16,
                   "batch": 1, "kv_layers_rotated": args.layers},
        "hbm_gbs_step": round(nb["step"] / (us_step * 1e-6) / 1e9, 1),
        "hbm_frac_step": round(nb["step"] / (us_step * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": {"kernel": "attn_splitk_kernel (kernel 1: prefix splits + tree split)", "bound": "hbm",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "traffic_source": "profiles/attn_splitk_64k_traffic.json: rocprofv3 FETCH_SIZE and WRITE_SIZE "
                                       "per dispatch of this kernel on this workload (two counter passes), scaled "
                                       "by a 1 GiB copy; re-measured whenever kernel 1 changes",
                     "bytes_per_launch": nb["kernel1"], "avg_us": round(k1_us, 3), "median_us": round(k1_med, 3),
                     "timing": "HIP start/stop events attached to each kernel-1 launch (hipExtLaunchKernel), "
                               "second pass of K steps", "us_per_step_in_that_pass": round(ms_step_ev * 1e3, 3)},
        "wall_s_timed": round(t_wall, 4),
    }
    if not args.no_prefix_sweep:
        line["prefix_sweep"] = bench_prefix_sweep(args, lib, ev)
    if not args.no_bundle_128k:
        print("[bench] bundle-packed verify (N=131072, M=128)", file=sys.stderr, flush=True)
        line["bundle_packed_128k"] = bench_bundle_packed_128k(args, lib, ev)
    if not args.no_llama_step:
        print("[bench] Llama-3.1-8B-shaped verify step (32 layers)", file=sys.stderr, flush=True)
        line["llama8b_verify_step"] = bench_llama8b_step(args, lib, ev)
    if not args.no_accept:
        print("[bench] acceptance kernel", file=sys.stderr, flush=True)
        line["acceptance"] = bench_accept(args, lib, ev)
        print("[bench] fp32 4096-token layer", file=sys.stderr, flush=True)
        line["config_4096_fp32"] = bench_fp32_4k()
    if not args.no_cpu:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        cb, _ = cpu_baseline(inp, args)
        line["cpu_baseline"] = cb
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
