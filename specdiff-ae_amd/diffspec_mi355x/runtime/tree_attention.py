"""Tree-attention runtime for DiffSpec target adapters, on MI355X (gfx950) HIP kernels.

Drop-in for the reference module ``diffspec/runtime/tree_attention.py``:
same function names, argument meaning, shapes and return layouts.  The work
is done by libdsv.so (kernel 1: split-K flash-decoding over the prefix;
kernel 2: tree-masked block with an in-LDS ancestor bitmask; kernel 3: wave64
LSE merge).  There is no Triton, no PyTorch math fallback and no CPU path:
CPU tensors raise.

Differences from the reference, all deliberate:
  * GQA-native: key/value may carry Hk heads with num_heads % Hk == 0 (the
    reference requires the repeat_kv-expanded form, which is still accepted).
  * The tree mask is read by the kernel itself in its native dtype, with the
    conversion rule of ``_maybe_to_int8_mask`` (runtime/tree_attention.py:449-460):
    float masks keep where == 0, int8/uint8/bool masks keep where != 0.
  * Errors raise instead of silently falling back (runtime/tree_attention.py:493-525).
"""

from __future__ import annotations

import torch

from .. import _ext

__all__ = [
    "TRITON_AVAILABLE",
    "HIP_AVAILABLE",
    "prefix_attention_forward",
    "tree_attention_forward",
    "tree_verify",
]

# The reference exposes TRITON_AVAILABLE; this backend never uses Triton.
TRITON_AVAILABLE = False
HIP_AVAILABLE = True


def _check_4d(name: str, t: torch.Tensor, shape) -> None:
    if tuple(t.shape) != tuple(shape):
        raise AssertionError(f"{name} shape {tuple(t.shape)} != {tuple(shape)}")


def prefix_attention_forward(query_states, key_states, value_states, bsz, q_len, num_heads, hidden_dim,
                             n_keys: int = -1):
    """Non-causal attention of the tree queries over the prefix, with LSE.

    Mirrors runtime/tree_attention.py:414-446.

    Args:
        query_states: [B, M, H, D] bf16/f16 on a ROCm device.
        key_states, value_states: [B, N, Hk, D], Hk divides H.
        n_keys: attend to keys [0, n_keys) only (flash_attn cache_seqlens); -1 = all.

    Returns:
        out: [B, M, H, D] in the query dtype.
        lse: [B, H, M] float32 (flash-attn ``return_softmax_lse`` layout).
    """
    dev = _ext.require_gpu(query_states, key_states, value_states)
    B, M, H, D = bsz, q_len, num_heads, hidden_dim
    _check_4d("query_states", query_states, (B, M, H, D))
    lib = _ext.load()
    out = torch.empty_like(query_states)
    lse = torch.empty((B, H, M), dtype=torch.float32, device=dev)
    N = key_states.shape[1]
    nk = N if n_keys is None or n_keys < 0 else int(n_keys)
    ws_bytes = lib.dsv_attn_workspace_bytes(B, M, H, key_states.shape[2], D, nk, 0, 0)
    ws = _ext.workspace(ws_bytes, dev)
    q_d, k_d, v_d = _ext.desc(query_states), _ext.desc(key_states), _ext.desc(value_states)
    o_d, l_d = _ext.desc(out), _ext.desc(lse)
    rc = lib.dsv_prefix_attention_forward(q_d, k_d, v_d, nk, o_d, l_d, ws.data_ptr(), ws.numel(),
                                          _ext.stream_of(dev))
    _ext.check(rc, "prefix_attention_forward")
    return out, lse


def tree_attention_forward(query_states, key_states, value_states, tree_mask, cache_lens, prefix_lse, bsz, q_len,
                           num_heads, hidden_dim, return_lse: bool = False):
    """Tree-masked attention over the post-cache block and the merge weight.

    Mirrors runtime/tree_attention.py:462-541.

    Args:
        query_states: [B, M, H, D]
        key_states, value_states: [B, M, Hk, D] (post-cache tree block)
        tree_mask: [B, 1, T, T] or [B, T, T]; only the last M x M block is used
        cache_lens: unused (signature compatibility)
        prefix_lse: [B, H, M] (flash layout; reshaped like the reference)

    Returns:
        current_out: [B, M, H, D] in the query dtype
        weight: [B, M, H, 1] in the query dtype = sigmoid(prefix_lse - tree_lse)
        (and tree_lse [B, M, H] float32 when return_lse=True)
    """
    dev = _ext.require_gpu(query_states, key_states, value_states, tree_mask, prefix_lse)
    B, M, H, D = bsz, q_len, num_heads, hidden_dim
    assert query_states.shape[:3] == (B, M, H) and query_states.shape[3] == D, \
        f"query_states shape {query_states.shape} != {(B, M, H, D)}"
    if key_states.shape[:2] != (B, M) or key_states.shape[3] != D or value_states.shape != key_states.shape:
        raise AssertionError("key/value must be post-cache block")
    lib = _ext.load()
    # Same reinterpretation as the reference: reshape(B, H, M, -1), first column.
    plse = prefix_lse.reshape(B, H, M, -1)[..., 0]
    if plse.dtype != torch.float32:
        plse = plse.float()
    mask = tree_mask
    if mask.dtype not in (torch.float32, torch.float16, torch.bfloat16, torch.int8, torch.uint8, torch.bool):
        mask = mask.float()
    current_out = torch.empty_like(query_states)
    weight = torch.empty((B, M, H, 1), dtype=query_states.dtype, device=dev)
    tree_lse = torch.empty((B, M, H), dtype=torch.float32, device=dev) if return_lse else None
    ws_bytes = lib.dsv_attn_workspace_bytes(B, M, H, key_states.shape[2], D, 0, 0, 1)
    ws = _ext.workspace(ws_bytes, dev)
    args = [_ext.desc(query_states), _ext.desc(key_states), _ext.desc(value_states), _ext.desc(mask),
            _ext.desc(plse), _ext.desc(current_out), _ext.desc(weight), _ext.desc(tree_lse)]
    rc = lib.dsv_tree_attention_forward(*args, ws.data_ptr(), ws.numel(), _ext.stream_of(dev))
    _ext.check(rc, "tree_attention_forward")
    if return_lse:
        return current_out, weight, tree_lse
    return current_out, weight


def _check_row_perm(row_perm: torch.Tensor, M: int) -> None:
    """A caller-supplied query packing order must be a permutation of [0, M)."""
    if row_perm.dim() != 1 or row_perm.numel() != M:
        raise ValueError(f"row_perm must be a [M] = [{M}] permutation (got shape {tuple(row_perm.shape)})")
    ok = torch.equal(torch.sort(row_perm.to(torch.int64)).values,
                     torch.arange(M, device=row_perm.device, dtype=torch.int64))
    if not ok:
        raise ValueError("row_perm is not a permutation of [0, M): rows of the missing nodes would stay unwritten")


def tree_verify(query_states, k_cache, v_cache, n_prefix: int, parent, page_table=None, row_perm=None,
                out_dtype=None, return_lse: bool = True, check_row_perm: bool = True):
    """Fused hybrid tree verification: prefix + tree block + LSE merge.

    Computes what llama_target_model.py:834-867 computes with three calls and
    three elementwise passes (prefix_attention_forward, tree_attention_forward,
    out = cur*(1-w) + prefix*w), in one split-K launch plus one merge launch.

    Args:
        query_states: [B, M, H, D]
        k_cache, v_cache: either page-pool halves [P, Hk, page_size, D]
            (kv_pages[layer, 0] / kv_pages[layer, 1]) with ``page_table``
            [n_pages] or [B, n_pages], or contiguous caches [B, L, Hk, D].
            The tree's K/V rows are tokens [n_prefix, n_prefix + M).
        parent: [M] or [B, M] int32/int64, parent node of each node (< 0 = root).
        row_perm: optional int32 [M] query packing order (bundle order), a
            permutation of [0, M).
        check_row_perm: verify that ``row_perm`` is a permutation (one device
            sort and a host read); pass False for an order that is one by
            construction, such as ``bundle_row_order_device``'s output.

    Returns:
        out [B, M, H, D] (out_dtype, default the query dtype) and lse [B, M, H] float32.
    """
    dev = _ext.require_gpu(query_states, k_cache, v_cache, parent, page_table, row_perm)
    B, M, H, D = query_states.shape
    lib = _ext.load()
    out = torch.empty((B, M, H, D), dtype=out_dtype or query_states.dtype, device=dev)
    lse = torch.empty((B, M, H), dtype=torch.float32, device=dev) if return_lse else None
    if page_table is not None:
        Hk, ps = k_cache.shape[1], k_cache.shape[2]
    else:
        Hk, ps = k_cache.shape[2], 0
    ws_bytes = lib.dsv_attn_workspace_bytes(B, M, H, Hk, D, int(n_prefix), ps, 1)
    ws = _ext.workspace(ws_bytes, dev)
    if row_perm is not None:
        if check_row_perm:
            _check_row_perm(row_perm, M)
        if row_perm.dtype != torch.int32:
            row_perm = row_perm.to(torch.int32)
    args = [_ext.desc(query_states), _ext.desc(k_cache), _ext.desc(v_cache), _ext.desc(page_table)]
    rc = lib.dsv_tree_verify(*args, int(n_prefix), _ext.desc(parent), _ext.desc(row_perm), _ext.desc(out),
                             _ext.desc(lse), ws.data_ptr(), ws.numel(), _ext.stream_of(dev))
    _ext.check(rc, "tree_verify")
    return out, lse
