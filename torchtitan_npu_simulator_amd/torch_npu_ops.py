"""MI355X implementations of the torch_npu DSA ops the reference calls.

Same names, argument meanings and return conventions as the ``torch_npu`` calls in the
reference's ``converters/kernels/dsa.py`` (paths relative to the reference repository):

* ``npu_lightning_indexer``            dsa.py:217-226, binding ops/aclnn/lightning_indexer/binding.cpp:12-36
* ``npu_sparse_flash_attention``       dsa.py:238-253 (attention_mode=2, MLA absorb)
* ``npu_sparse_lightning_indexer_grad_kl_loss``  dsa.py:159-177,
                                       binding ops/aclnn/sparse_lightning_indexer_grad_kl_loss/binding.cpp:12-36

Every op runs on the HIP library (``libdsa_mi355x.so``) on the tensors' GPU and raises
if the library or a GPU is missing; nothing here computes on the CPU.

Layouts "BSND" and "TND".  ``sparse_mode`` 3 is the causal rule aligned bottom-right
(query row s may see key t <= s + (S_k - S_q)); 0 means no causal mask.  An explicit
``q_offset`` overrides it (one GPU's context-parallel share sees Q rows starting at
``q_offset`` against the KV prefix).

"TND" packs sequences along the token axis (query [T,N,D], key [T_k,1,D], indices
[T,1,K] holding sequence-local key positions).  Its sequence boundaries come either as
``actual_seq_lengths_*`` in torch_npu's TND convention (cumulative END offsets, one per
sequence, the last equal to T) or as ``cu_seqlens_*`` (``[0, ends...]``, the A5 ops'
convention, converters/kernels/npu_smla.py:457-479, :754-768).  In "BSND",
``actual_seq_lengths_*`` are per-batch valid lengths: rows past a batch's query length
get no selection (-1) and keys past its key length are never candidates.
"""

from __future__ import annotations

import itertools
import math
import warnings
import weakref

import torch

from . import _lib
from ._lib import check, host_i32, load_library, ptr, require_gpu_tensor, stream_of

__all__ = [
    "npu_lightning_indexer",
    "npu_sparse_flash_attention",
    "npu_sparse_lightning_indexer_grad_kl_loss",
    "sparse_mla_fwd",
    "sparse_mla_bwd",
    "attn_mass",
    "indexer_kl_grad_from_mass",
    "indexer_scores",
    "topk_select",
    "quantize_fp8_per_row",
    "compressor_pool",
    "compressor_pool_tnd",
    "indexer_prep",
    "rope_cos_sin",
    "mla_absorb",
    "mla_absorb_q",
    "mla_absorb_out",
    "lightning_indexer_varlen",
    "sparse_mla_fwd_varlen",
    "sparse_mla_bwd_varlen",
    "attn_mass_varlen",
    "indexer_kl_grad_from_mass_varlen",
    "to_cu_seqlens",
    "npu_sparse_attn_shared_kv",
    "npu_sparse_attn_sharedkv_metadata",
    "npu_sparse_attn_sharedkv",
    "npu_sparse_attn_sharedkv_grad",
    "SparseAttnSharedKV",
    "v4_attention_indices",
    "v4_indexer_kl_grad",
]

_SCORE_BUDGET_BYTES = 1 << 30  # fp32 score rows materialised per indexer chunk
_NO_MASK_OFFSET = 1 << 40


def _resolve_q_offset(sparse_mode: int, s_q: int, s_k_tokens: int, q_offset: int | None) -> int:
    if q_offset is not None:
        return int(q_offset)
    if sparse_mode == 3:
        return max(0, s_k_tokens - s_q)
    if sparse_mode == 0:
        return _NO_MASK_OFFSET
    raise ValueError(f"sparse_mode={sparse_mode} is not supported (0 or 3)")


def _band_cuts(sparse_mode: int, s_q: int, s_k: int, q_off: int, pre_tokens: int, next_tokens: int) -> bool:
    """Whether the pre_tokens / next_tokens band removes any key the mode's own rule admits.

    The band of query row s is t in [a(s) - pre_tokens, a(s) + next_tokens] with a(s) = s
    (sparse_mode 0, top-left aligned) or s + q_off (sparse_mode 3, the bottom-right causal
    diagonal, which also bounds t from above)."""
    pre, nxt = int(pre_tokens), int(next_tokens)
    if sparse_mode == 3:
        return pre < s_q - 1 + q_off or nxt < 0
    return pre < s_q - 1 or nxt < s_k - 1


def _band_mask_indices(idx, sparse_mode: int, q_off: int, pre_tokens: int, next_tokens: int):
    """Slot indices [B,S,K] with every key outside the row's band set to -1 (see _band_cuts)."""
    S = idx.shape[1]
    a = torch.arange(S, device=idx.device, dtype=torch.int64).view(1, S, 1)
    if sparse_mode == 3:
        a = a + int(q_off)
    t = idx.long()
    ok = (t >= a - int(pre_tokens)) & (t <= a + int(next_tokens))
    return torch.where(ok, idx, torch.full_like(idx, -1))


def _banded_indexer(query, k3, weights, K, query_scale, key_scale, sparse_mode, q_off, pre_tokens, next_tokens,
                    index_offset, return_value):
    """Indexer + top-k under a band that cuts keys: scores per row chunk (dsa_indexer_fwd_ws),
    keys below the band's lower edge set to NaN (never a candidate), the upper edge given to
    dsa_topk as its causal offset."""
    B, S = query.shape[:2]
    s_k = k3.shape[1]
    pre, nxt = int(pre_tokens), int(next_tokens)
    up_off = min(q_off, q_off + nxt) if sparse_mode == 3 else min(nxt, _NO_MASK_OFFSET)
    lo_off = (q_off if sparse_mode == 3 else 0) - pre
    idx = torch.empty(B, S, K, dtype=torch.int32, device=query.device)
    vals = torch.empty(B, S, K, dtype=torch.float32, device=query.device) if return_value else None
    rows = max(1, min(S, _SCORE_BUDGET_BYTES // (4 * max(1, s_k) * B)))
    t = torch.arange(s_k, device=query.device).view(1, 1, s_k)
    for r0 in range(0, S, rows):
        r1 = min(S, r0 + rows)
        qs = None if query_scale is None else query_scale[:, r0:r1]
        sc = indexer_scores(query[:, r0:r1], k3, weights[:, r0:r1], q_scale=qs, k_scale=key_scale,
                            q_offset=r0 + up_off)
        lo = torch.arange(r0, r1, device=query.device).view(1, -1, 1) + lo_off
        sc.masked_fill_(t < lo, float("nan"))
        i_c, v_c = topk_select(sc, K, q_offset=r0 + up_off, index_offset=index_offset, return_values=return_value)
        idx[:, r0:r1] = i_c
        if return_value:
            vals[:, r0:r1] = v_c
    return idx, vals


def to_cu_seqlens(cu_seqlens=None, actual_seq_lengths=None, total=None) -> list[int]:
    """Host ``[0, end_0, end_1, ...]`` from A5-style ``cu_seqlens`` or torch_npu-style TND
    ``actual_seq_lengths`` (cumulative ends); checks the last end against ``total``."""
    if cu_seqlens is not None:
        cu = list(_lib.host_ints(cu_seqlens))
        if not cu or cu[0] != 0:
            raise ValueError("cu_seqlens must start with 0")
    elif actual_seq_lengths is not None:
        cu = [0] + list(_lib.host_ints(actual_seq_lengths))
    else:
        raise ValueError("TND layout needs cu_seqlens or actual_seq_lengths")
    if any(b < a for a, b in zip(cu[:-1], cu[1:])):
        raise ValueError(f"sequence boundaries must be non-decreasing: {cu}")
    if total is not None and cu[-1] != total:
        raise ValueError(f"sequence boundaries end at {cu[-1]} but the packed tensor has {total} tokens")
    return cu


def _on_device(x) -> bool:
    return isinstance(x, torch.Tensor) and x.is_cuda


def seq_bounds(cu_seqlens=None, actual_seq_lengths=None, total=None):
    """Sequence boundaries of a packed batch: a GPU tensor stays on the device (int32
    [0, end_0, end_1, ...], built there from ``cu_seqlens`` or from the cumulative ends
    ``actual_seq_lengths`` without reading them, so the ops take their device paths with no
    host synchronisation); anything else becomes the validated host list of
    ``to_cu_seqlens``."""
    src = cu_seqlens if cu_seqlens is not None else actual_seq_lengths
    if _on_device(src):
        t = src.reshape(-1).to(torch.int32)
        if cu_seqlens is None:
            t = torch.cat([t.new_zeros(1), t])
        return t.contiguous()
    return to_cu_seqlens(cu_seqlens, actual_seq_lengths, total)


def _device_bounds(*bounds, device):
    """Each of ``bounds`` (host list, CPU or GPU tensor, or None) as a device int32 tensor."""
    out = []
    for b in bounds:
        if b is None or _on_device(b):
            out.append(None if b is None else b.reshape(-1).to(device=device, dtype=torch.int32).contiguous())
        else:
            vals = b.tolist() if isinstance(b, torch.Tensor) else list(b)
            out.append(torch.tensor(vals, dtype=torch.int32, device=device))
    return out


# ---------------------------------------------------------------------------
# lightning indexer + top-k
# ---------------------------------------------------------------------------
def quantize_fp8_per_row(x: torch.Tensor):
    """OCP fp8-e4m3fn with one fp32 scale per row of the last dim (dsa_quantize_fp8_rows):
    scale = max(amax|row| / 448, 1e-12), q = e4m3fn(x / scale) (correctly rounded fp32
    divisions, round-to-nearest-even cast).  Returns (q like x in
    torch.float8_e4m3fn, scale fp32 x.shape[:-1])."""
    lib = load_library()
    require_gpu_tensor(x, "x")
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.float()
    x = x.contiguous()
    d = x.shape[-1]
    rows = x.numel() // d if d else 0
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    scale = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    if rows:
        check(lib.dsa_quantize_fp8_rows(ptr(x), _lib.dtype_code(x.dtype), ptr(q), ptr(scale), rows, d,
                                        stream_of(x.device)), "dsa_quantize_fp8_rows")
    return q, scale


def indexer_scores(q_idx, k_idx, weights, *, q_scale=None, k_scale=None, q_offset=0, cmp_ratio=1, out=None,
                   linear_split=True):
    """fp32 index scores [B,S,S_k] (-inf where invalid) from dsa_indexer_fwd_ws.

    ``linear_split`` gives the fp8 H_I=64 kernel its pre-pass workspace (relu(x) = (x + |x|)/2
    with the linear part on the MFMA); False runs the relu-form kernels of dsa_indexer_fwd.
    """
    lib = load_library()
    for t, n in ((q_idx, "query"), (k_idx, "key"), (weights, "weights")):
        require_gpu_tensor(t, n)
    if k_idx.dim() == 4:
        k_idx = k_idx.squeeze(2)
    B, S, H, D = q_idx.shape
    s_k = k_idx.shape[1]
    if q_idx.dtype != k_idx.dtype:
        raise ValueError("query and key must share a dtype")
    q_idx = q_idx.contiguous()
    k_idx = k_idx.contiguous()
    w = weights.float().contiguous()
    qs = None if q_scale is None else q_scale.float().contiguous()
    ks = None if k_scale is None else k_scale.float().contiguous()
    if out is None:
        out = torch.empty(B, S, s_k, dtype=torch.float32, device=q_idx.device)
    dt = _lib.dtype_code(q_idx.dtype)
    ws_bytes = int(lib.dsa_indexer_fwd_workspace_size(B, S, H, D, dt)) if linear_split else 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q_idx.device) if ws_bytes else None
    check(
        lib.dsa_indexer_fwd_ws(ptr(q_idx), ptr(qs), ptr(k_idx), ptr(ks), ptr(w), ptr(out), dt, B, S, s_k, H, D,
                               out.stride(1), int(q_offset), int(cmp_ratio), ptr(ws), ws_bytes,
                               stream_of(q_idx.device)),
        "dsa_indexer_fwd_ws",
    )
    return out


def topk_select(scores, k, *, q_offset=0, cmp_ratio=1, index_offset=0, return_values=False, candidates=True):
    """int32 [B,S,k] top-k indices (ascending index order, -1 padded) of fp32 scores.  Rows
    longer than 16384 keys go through candidate lists (dsa_topk_ws) unless ``candidates`` is
    False (dsa_topk's multi-pass selection; the same result)."""
    lib = load_library()
    require_gpu_tensor(scores, "scores")
    B, S, s_k = scores.shape
    if scores.stride(2) != 1:
        scores = scores.contiguous()
    idx = torch.empty(B, S, k, dtype=torch.int32, device=scores.device)
    vals = torch.empty(B, S, k, dtype=torch.float32, device=scores.device) if return_values else None
    if not candidates:
        check(
            lib.dsa_topk(ptr(scores), ptr(idx), ptr(vals), B, S, s_k, scores.stride(1), k, int(q_offset),
                         int(cmp_ratio), int(index_offset), stream_of(scores.device)),
            "dsa_topk",
        )
        return idx, vals
    ws_bytes = int(lib.dsa_topk_workspace_size(B, S, s_k, k))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=scores.device) if ws_bytes else None
    check(
        lib.dsa_topk_ws(ptr(scores), ptr(idx), ptr(vals), B, S, s_k, scores.stride(1), k, int(q_offset),
                        int(cmp_ratio), int(index_offset), ptr(ws), ws_bytes, stream_of(scores.device)),
        "dsa_topk",
    )
    return idx, vals


def _values_dtype(query: torch.Tensor) -> torch.dtype:
    """dtype of sparse_values: the query's, as the binding allocates them (lightning_indexer/
    binding.cpp:29); bf16 for this build's fp8 queries."""
    return torch.bfloat16 if query.dtype == torch.float8_e4m3fn else query.dtype


def npu_lightning_indexer(
    query,
    key,
    weights,
    actual_seq_lengths_query=None,
    actual_seq_lengths_key=None,
    block_table=None,
    layout_query="BSND",
    layout_key="BSND",
    sparse_count=2048,
    sparse_mode=3,
    pre_tokens=(1 << 63) - 1,
    next_tokens=(1 << 63) - 1,
    cmp_ratio=1,
    return_value=False,
    *,
    query_scale=None,
    key_scale=None,
    q_offset=None,
    index_offset=0,
    cu_seqlens_q=None,
    cu_seqlens_k=None,
    cmp_residual_k=None,
):
    """Fused lightning indexer + per-query top-k.

    query [B,S,H_I,D_I], key [B,S_k,1,D_I] (or [B,S_k,D_I]), weights [B,S,H_I]; bf16, or
    fp8-e4m3fn with ``query_scale`` [B,S,H_I] / ``key_scale`` [B,S_k] (this build's
    extension for the fp8 indexer).  Returns (sparse_indices int32 [B,S,1,K],
    sparse_values [B,S,1,K] in the query's dtype (bf16 for fp8 queries; -inf in padded
    slots) or None): the chosen key indices in ascending order with -1 padding (reference
    binding shapes and dtypes: lightning_indexer/binding.cpp:27-29).  Rows are processed in
    chunks so the fp32 score buffer stays under 1 GiB.

    TND: query [T,H_I,D_I], key [T_k,1,D_I], weights [T,H_I], scales [T,H_I] / [T_k];
    returns [T,1,K] with sequence-local indices (see ``lightning_indexer_varlen``).
    """
    if block_table is not None:
        raise NotImplementedError("paged KV (block_table) is not supported")
    if layout_query not in ("BSND", "TND") or layout_key != layout_query:
        raise NotImplementedError(f"layouts {layout_query}/{layout_key} (BSND/BSND or TND/TND)")
    if layout_query == "TND":
        kt = key.reshape(key.shape[0], key.shape[-1])
        cu_q = seq_bounds(cu_seqlens_q, actual_seq_lengths_query, query.shape[0])
        cu_k = seq_bounds(cu_seqlens_k, actual_seq_lengths_key, kt.shape[0])
        idx, vals = lightning_indexer_varlen(query, kt, weights, cu_q, cu_k, sparse_count, sparse_mode=sparse_mode,
                                             cmp_ratio=cmp_ratio, cmp_residual_k=cmp_residual_k,
                                             return_value=return_value, query_scale=query_scale, key_scale=key_scale,
                                             index_offset=index_offset)
        return idx.unsqueeze(1), (vals.to(_values_dtype(query)).unsqueeze(1) if return_value else None)
    if actual_seq_lengths_query is not None or actual_seq_lengths_key is not None:
        idx, vals = _bsnd_lengths_indexer(query, key, weights, actual_seq_lengths_query, actual_seq_lengths_key,
                                          sparse_count, sparse_mode, cmp_ratio, return_value, query_scale, key_scale,
                                          index_offset)
        return idx, (vals.to(_values_dtype(query)) if return_value else None)
    k3 = key.squeeze(2) if key.dim() == 4 else key
    B, S, H, D = query.shape
    s_k = k3.shape[1]
    q_off = _resolve_q_offset(sparse_mode, S, s_k * cmp_ratio, q_offset)
    if _band_cuts(sparse_mode, S, s_k, q_off, pre_tokens, next_tokens):
        if int(cmp_ratio) != 1:
            raise NotImplementedError("a pre_tokens / next_tokens band over compressed keys (cmp_ratio > 1)")
        idx, vals = _banded_indexer(query, k3, weights, int(sparse_count), query_scale, key_scale, sparse_mode, q_off,
                                    pre_tokens, next_tokens, index_offset, return_value)
    else:
        idx, vals = lightning_indexer(query, k3, weights, int(sparse_count), query_scale=query_scale,
                                      key_scale=key_scale, q_offset=q_off, cmp_ratio=cmp_ratio,
                                      index_offset=index_offset, return_value=return_value)
    return idx.unsqueeze(2), (vals.to(_values_dtype(query)).unsqueeze(2) if return_value else None)


def lightning_indexer_workspace_bytes(lib, B, S, s_k, H, D, dt, budget=None) -> int:
    """Workspace of one dsa_lightning_indexer call under a score budget (default
    ``_SCORE_BUDGET_BYTES``): every row of every batch at once when they fit, else one batch
    at a time in chunks of as many rows as fit (the C entry picks the same split from the
    workspace size it is given)."""
    budget = _SCORE_BUDGET_BYTES if budget is None else int(budget)
    if B * S * s_k * 4 <= budget:
        return int(lib.dsa_lightning_indexer_workspace_size(B, S, s_k, H, D, dt, S))
    return int(lib.dsa_lightning_indexer_workspace_size(1, S, s_k, H, D, dt, max(1, budget // (4 * s_k))))


def lightning_indexer(query, key, weights, k, *, query_scale=None, key_scale=None, q_offset=0, cmp_ratio=1,
                      index_offset=0, return_value=False):
    """Index scores + per-row top-k in one library call (dsa_lightning_indexer).

    query [B,S,H_I,D_I], key [B,S_k,D_I] (bf16, or fp8-e4m3fn with query_scale [B,S,H_I] and
    key_scale [B,S_k]), weights [B,S,H_I].  Returns (indices int32 [B,S,k], values fp32
    [B,S,k] or None).  The fp32 score rows live in a workspace of at most 1 GiB: every row of
    every batch at once when they fit, else batch by batch in row chunks."""
    lib = load_library()
    for t, n in ((query, "query"), (key, "key"), (weights, "weights")):
        require_gpu_tensor(t, n)
    if query.dtype != key.dtype:
        raise ValueError("query and key must share a dtype")
    B, S, H, D = query.shape
    s_k = key.shape[1]
    q = query.contiguous()
    kk = key.contiguous()
    w = weights.float().contiguous()
    qs = None if query_scale is None else query_scale.float().contiguous()
    ks = None if key_scale is None else key_scale.float().contiguous()
    dt = _lib.dtype_code(q.dtype)
    idx = torch.empty(B, S, k, dtype=torch.int32, device=q.device)
    vals = torch.empty(B, S, k, dtype=torch.float32, device=q.device) if return_value else None
    ws_bytes = lightning_indexer_workspace_bytes(lib, B, S, s_k, H, D, dt)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    check(
        lib.dsa_lightning_indexer(ptr(q), ptr(qs), ptr(kk), ptr(ks), ptr(w), ptr(idx), ptr(vals), dt, B, S, s_k, H, D,
                                  int(k), int(q_offset), int(cmp_ratio), int(index_offset), ptr(ws), ws_bytes,
                                  stream_of(q.device)),
        "dsa_lightning_indexer",
    )
    return idx, vals


def _bsnd_lengths_indexer(query, key, weights, len_q, len_k, sparse_count, sparse_mode, cmp_ratio, return_value,
                          query_scale, key_scale, index_offset):
    """BSND with per-batch valid lengths: batch b is one sequence of its first len_q[b]
    queries and len_k[b] keys; its padded rows select nothing (-1)."""
    k3 = key.squeeze(2) if key.dim() == 4 else key
    B, S = query.shape[:2]
    s_k = k3.shape[1]
    lq = [S] * B if len_q is None else [int(v) for v in (len_q.tolist() if isinstance(len_q, torch.Tensor) else len_q)]
    lk = [s_k] * B if len_k is None else [int(v) for v in (len_k.tolist() if isinstance(len_k, torch.Tensor) else len_k)]
    if len(lq) != B or len(lk) != B or any(not 0 <= v <= S for v in lq) or any(not 0 <= v <= s_k for v in lk):
        raise ValueError(f"actual sequence lengths {lq} / {lk} do not fit B={B}, S={S}, S_k={s_k}")
    K = int(sparse_count)
    idx = torch.full((B, S, K), -1, dtype=torch.int32, device=query.device)
    vals = torch.full((B, S, K), float("-inf"), dtype=torch.float32, device=query.device) if return_value else None
    for b in range(B):
        if lq[b] == 0:
            continue
        qs = None if query_scale is None else query_scale[b, : lq[b]]
        ks = None if key_scale is None else key_scale[b, : lk[b]]
        i_b, v_b = lightning_indexer_varlen(query[b, : lq[b]], k3[b, : lk[b]], weights[b, : lq[b]], [0, lq[b]],
                                            [0, lk[b]], K, sparse_mode=sparse_mode, cmp_ratio=cmp_ratio,
                                            return_value=return_value, query_scale=qs, key_scale=ks,
                                            index_offset=index_offset)
        idx[b, : lq[b]] = i_b
        if return_value:
            vals[b, : lq[b]] = v_b
    return idx.unsqueeze(2), (vals.unsqueeze(2) if return_value else None)


def lightning_indexer_varlen(query, key, weights, cu_seqlens_q, cu_seqlens_k, sparse_count, *, sparse_mode=3,
                             cmp_ratio=1, cmp_residual_k=None, return_value=False, query_scale=None, key_scale=None,
                             index_offset=0):
    """Indexer scores + top-k over a packed varlen batch (dsa_lightning_indexer_varlen).

    query [T,H_I,D_I], key [T_k,D_I] (bf16, or fp8-e4m3fn with query_scale [T,H_I] and
    key_scale [T_k]), weights [T,H_I].  Sequence i's queries see its own keys only;
    indices are sequence-local (+ index_offset), -1 padded.  With compressed keys
    (cmp_ratio > 1), ``cmp_residual_k[i]`` original tokens follow the last whole block.
    Returns (indices int32 [T,K], values fp32 [T,K] or None).

    Bounds given as GPU tensors are read on the device (dsa_lightning_indexer_tnd: no host
    synchronisation, the same indices bit for bit) when the shape has a tile kernel (D_I
    128, H_I a multiple of 16 up to 128, bf16 or fp8); otherwise, and for host bounds, the
    host schedule (dsa_lightning_indexer_varlen) runs, reading GPU bounds back once per
    tensor version.
    """
    lib = load_library()
    for t, n in ((query, "query"), (key, "key"), (weights, "weights")):
        require_gpu_tensor(t, n)
    key = key.reshape(key.shape[0], key.shape[-1])
    T, H, D = query.shape
    T_k = key.shape[0]
    if query.dtype != key.dtype:
        raise ValueError("query and key must share a dtype")
    if any(_on_device(b) for b in (cu_seqlens_q, cu_seqlens_k, cmp_residual_k)):
        res = _lightning_indexer_tnd(query, key, weights, cu_seqlens_q, cu_seqlens_k, sparse_count, sparse_mode,
                                     cmp_ratio, cmp_residual_k, return_value, query_scale, key_scale, index_offset)
        if res is not None:
            return res
    cu_q = to_cu_seqlens(cu_seqlens_q, None, T)
    cu_k = to_cu_seqlens(cu_seqlens_k, None, T_k)
    if len(cu_q) != len(cu_k):
        raise ValueError("cu_seqlens_q and cu_seqlens_k describe different numbers of sequences")
    n_seq = len(cu_q) - 1
    res = None
    if cmp_residual_k is not None:
        res = list(_lib.host_ints(cmp_residual_k))  # a device tensor is read back once per version
        if len(res) != n_seq:
            raise ValueError("cmp_residual_k needs one entry per sequence")
    q = query.contiguous()
    k = key.contiguous()
    w = weights.float().contiguous()
    qs = None if query_scale is None else query_scale.float().contiguous()
    ks = None if key_scale is None else key_scale.float().contiguous()
    K = int(sparse_count)
    idx = torch.empty(T, K, dtype=torch.int32, device=q.device)
    vals = torch.empty(T, K, dtype=torch.float32, device=q.device) if return_value else None
    max_k = max(max(b - a for a, b in zip(cu_k[:-1], cu_k[1:])), 1)
    max_q = max(max(b - a for a, b in zip(cu_q[:-1], cu_q[1:])), 1)
    rows = max(1, min(max_q, _SCORE_BUDGET_BYTES // (4 * max_k)))
    # + the linear-split pieces of the chunk's rows (fp8, H_I=64), after a 256-byte boundary,
    # + for rows longer than 16384 keys the top-k candidate lists (8 bytes per entry, twice K
    # rounded to 4096 or 8192 entries, and a count per row), after another
    lin = int(lib.dsa_indexer_fwd_workspace_size(1, 1, H, D, _lib.dtype_code(q.dtype)))
    cand = rows * (8 * (4096 if K <= 2048 else 8192) + 4) + 768 if max_k > 16384 else 0
    ws = torch.empty(rows * max_k + ((rows * lin + 256) // 4 if lin else 0) + cand // 4, dtype=torch.float32,
                     device=q.device)
    if T == 0:
        return idx, vals
    check(
        lib.dsa_lightning_indexer_varlen(ptr(q), ptr(qs), ptr(k), ptr(ks), ptr(w), ptr(idx), ptr(vals), ptr(ws),
                                         ws.numel() * 4, _lib.dtype_code(q.dtype), host_i32(cu_q), host_i32(cu_k),
                                         host_i32(res), n_seq, H, D, K, int(cmp_ratio), int(sparse_mode),
                                         int(index_offset), stream_of(q.device)),
        "dsa_lightning_indexer_varlen",
    )
    return idx, vals


def _lightning_indexer_tnd(query, key, weights, cu_seqlens_q, cu_seqlens_k, sparse_count, sparse_mode, cmp_ratio,
                           cmp_residual_k, return_value, query_scale, key_scale, index_offset):
    """lightning_indexer_varlen with device sequence bounds (dsa_lightning_indexer_tnd): the
    windows are read on the device, so nothing is copied back.  None if the shape has no tile
    kernel (the host schedule then serves it)."""
    lib = load_library()
    T, H, D = query.shape
    T_k = key.shape[0]
    K = int(sparse_count)
    dt = _lib.dtype_code(query.dtype)
    ld = (T_k + 3) // 4 * 4
    max_rows = max(1, _SCORE_BUDGET_BYTES // (4 * ld))
    ws_bytes = int(lib.dsa_lightning_indexer_tnd_workspace_size(max(T, 1), T_k, H, D, dt, K, max_rows))
    if ws_bytes <= 0:
        return None
    dev = query.device
    cu_q, cu_k, res = _device_bounds(cu_seqlens_q, cu_seqlens_k, cmp_residual_k, device=dev)
    if cu_q.numel() != cu_k.numel() or cu_q.numel() < 2:
        raise ValueError("cu_seqlens_q and cu_seqlens_k describe different numbers of sequences")
    n_seq = cu_q.numel() - 1
    if res is not None and res.numel() != n_seq:
        raise ValueError("cmp_residual_k needs one entry per sequence")
    q = query.contiguous()
    k = key.contiguous()
    w = weights.float().contiguous()
    qs = None if query_scale is None else query_scale.float().contiguous()
    ks = None if key_scale is None else key_scale.float().contiguous()
    idx = torch.empty(T, K, dtype=torch.int32, device=dev)
    vals = torch.empty(T, K, dtype=torch.float32, device=dev) if return_value else None
    if T == 0:
        return idx, vals
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    check(
        lib.dsa_lightning_indexer_tnd(ptr(q), ptr(qs), ptr(k), ptr(ks), ptr(w), ptr(idx), ptr(vals), dt, ptr(cu_q),
                                      ptr(cu_k), ptr(res), n_seq, T, T_k, H, D, K, int(cmp_ratio), int(sparse_mode),
                                      int(index_offset), ptr(ws), ws_bytes, stream_of(dev)),
        "dsa_lightning_indexer_tnd",
    )
    return idx, vals


_global_idx_entry = None  # (key, source tensors, global indices [T,K] int32)


def tnd_global_indices(indices, cu_seqlens_q, cu_seqlens_k, t_k):
    """Sequence-local slot indices [T,K] of a packed batch as global key rows
    (dsa_tnd_global_indices): slot v of a row of sequence i becomes cu_seqlens_k[i] + v if it
    passes that sequence's causal rule, else -1, so the fixed-length kernels run the batch
    as one [1, T] problem with no causal test.  ``cu_seqlens_*`` are device int32 tensors.
    The last result is kept (with the tensors it came from, so their addresses cannot be
    reused while it lives) for the other ops of the same step: forward, backward, mass and
    indexer KL all take the same indices."""
    global _global_idx_entry
    lib = load_library()
    key = tuple((t.data_ptr(), t._version, tuple(t.shape), tuple(t.stride())) for t in
                (indices, cu_seqlens_q, cu_seqlens_k)) + (indices.device, int(t_k))
    e = _global_idx_entry
    if e is not None and e[0] == key:
        return e[2]
    _global_idx_entry = None
    T, K = indices.shape
    out = torch.empty(T, K, dtype=torch.int32, device=indices.device)
    check(lib.dsa_tnd_global_indices(ptr(indices), ptr(out), ptr(cu_seqlens_q), ptr(cu_seqlens_k),
                                     cu_seqlens_q.numel() - 1, T, int(t_k), K, stream_of(indices.device)),
          "dsa_tnd_global_indices")
    _global_idx_entry = (key, (indices, cu_seqlens_q, cu_seqlens_k), out)
    return out


def _varlen_global(indices, cu_seqlens_q, cu_seqlens_kv, T, T_kv, device):
    """Global indices [T,K] when the sequence bounds are on the device, else None."""
    if not (_on_device(cu_seqlens_q) or _on_device(cu_seqlens_kv)):
        return None
    cu_q, cu_k = _device_bounds(cu_seqlens_q, cu_seqlens_kv, device=device)
    if cu_q.numel() != cu_k.numel() or cu_q.numel() < 2:
        raise ValueError("cu_seqlens_q and cu_seqlens_kv describe different numbers of sequences")
    return tnd_global_indices(indices.reshape(T, -1).to(torch.int32).contiguous(), cu_q, cu_k, T_kv)


# ---------------------------------------------------------------------------
# gathered sparse MLA attention
# ---------------------------------------------------------------------------
def sparse_mla_fwd(q, kv, indices, scale, *, d_v=512, q_offset=0, sinks=None):
    """(out [B,S,H,d_v], softmax_max [B,S,H], softmax_sum [B,S,H]) from dsa_sparse_mla_fwd.

    q [B,S,H,D_qk] bf16/fp32, kv [B,S_kv,D_qk] (v = kv[..., :d_v]), indices [B,S,K] int32.
    ``sinks`` [H] (DeepSeek-V4's per-head attention sink) selects dsa_sparse_mla_fwd_sink: the
    sink joins every row's softmax with no value, and the statistics returned include it.
    """
    global _attn_mass_entry
    _attn_mass_entry = None  # a mass kept by the last backward (take_attn_mass) is not for this call
    lib = load_library()
    require_gpu_tensor(q, "q")
    B, S, H, D = q.shape
    s_kv = kv.shape[1]
    K = indices.shape[-1]
    q = q.contiguous()
    kv = kv.contiguous()
    indices = indices.reshape(B, S, K).to(torch.int32).contiguous()
    out = torch.empty(B, S, H, d_v, dtype=q.dtype, device=q.device)
    smax = torch.empty(B, S, H, dtype=torch.float32, device=q.device)
    ssum = torch.empty(B, S, H, dtype=torch.float32, device=q.device)
    if sinks is not None:
        sk = _sink_vector(sinks, H, q.device)
        check(
            lib.dsa_sparse_mla_fwd_sink(ptr(q), ptr(kv), ptr(indices), ptr(sk), ptr(out), ptr(smax), ptr(ssum),
                                        _lib.dtype_code(q.dtype), B, S, s_kv, H, D, d_v, K, float(scale),
                                        int(q_offset), stream_of(q.device)),
            "dsa_sparse_mla_fwd_sink",
        )
        return out, smax, ssum
    check(
        lib.dsa_sparse_mla_fwd(ptr(q), ptr(kv), ptr(indices), ptr(out), ptr(smax), ptr(ssum), _lib.dtype_code(q.dtype),
                               B, S, s_kv, H, D, d_v, K, float(scale), int(q_offset), stream_of(q.device)),
        "dsa_sparse_mla_fwd",
    )
    return out, smax, ssum


def _sink_vector(sinks, H, device):
    sk = sinks.to(device=device, dtype=torch.float32).reshape(-1).contiguous()
    if sk.numel() != H:
        raise ValueError(f"sinks has {sk.numel()} entries, the call has {H} heads")
    return sk


_pair_csr_entry = None  # (key, the index tensor, CSR buffer)
_share_pair_csr = True  # False: each reduction builds its own CSR inside the library call


def pair_csr(indices, s_k, q_offset=0):
    """The key-major CSR of the usable (row, slot) pairs of ``indices`` [B,S,K] int32 over s_k
    keys (dsa_pair_csr_build), shared by the attention backward's dKV reduction and the
    indexer KL op's dK_index reduction, which use the same index tensor.  One CSR is kept,
    with a reference to the index tensor it was built from (so that storage cannot be freed
    and its address reused while the entry lives); it is rebuilt when the index data (address,
    shape, strides or version, which views of one storage share), the key count or the offset
    changes."""
    global _pair_csr_entry
    lib = load_library()
    B, S, K = indices.shape
    key = (indices.data_ptr(), indices._version, tuple(indices.shape), tuple(indices.stride()), indices.device,
           int(s_k), int(q_offset))
    e = _pair_csr_entry
    if e is not None and e[0] == key:
        return e[2]
    _pair_csr_entry = None  # (the old buffer goes before the new one is allocated)
    nbytes = int(lib.dsa_pair_csr_size(B, S, s_k, K))
    csr = torch.empty(nbytes, dtype=torch.uint8, device=indices.device)
    check(lib.dsa_pair_csr_build(ptr(indices), B, S, s_k, K, int(q_offset), ptr(csr), nbytes,
                                 stream_of(indices.device)), "dsa_pair_csr_build")
    _pair_csr_entry = (key, indices, csr)
    return csr


_attn_mass_entry = None  # (key, the tensors the mass came from, mass [B,S,K] fp32)
_share_attn_mass = True  # False: the indexer KL op always recomputes its target mass


def _attn_mass_key(q, kv, indices, smax, ssum, scale, q_offset):
    # address, version (shared by every view of a storage), shape, strides and dtype of each
    # input, so a different view, a copy or an in-place change of any of them misses
    return tuple((t.data_ptr(), t._version, tuple(t.shape), tuple(t.stride()), t.dtype)
                 for t in (q, kv, indices, smax, ssum)) + (q.device, float(scale), int(q_offset))


def take_attn_mass(q, kv, indices, smax, ssum, scale, q_offset=0):
    """The head-summed attention mass that the last op-level attention backward left for
    exactly these inputs (same tensors, unchanged since), or None; the entry is used once.

    ``npu_sparse_flash_attention``'s backward forms P for every (row, head, slot) anyway, so
    it keeps the mass (``bwd_sdp_kernel`` writes it; bitwise equal to ``dsa_attn_mass`` on
    the same inputs) for the indexer KL op that a torch_npu-style layer calls next with the
    same query, key, indices and softmax statistics (reference converters/kernels/dsa.py:
    159-177 after :238-253).  The entry holds the index and statistics tensors it was made
    for (so their addresses cannot be reused while it lives; softmax statistics belong to
    one query / key pair) but not the query and key, and it is dropped by the next attention
    forward or replaced by the next backward."""
    global _attn_mass_entry
    e = _attn_mass_entry
    if e is None or e[0] != _attn_mass_key(q, kv, indices, smax, ssum, scale, q_offset):
        return None
    _attn_mass_entry = None
    return e[2]


def sparse_mla_bwd(q, kv, indices, out, dout, smax, ssum, scale, *, q_offset=0, workspace_bytes=None,
                   return_mass=False, sinks=None):
    """(dq like q, dkv fp32 [B,S_kv,D_qk]) from dsa_sparse_mla_bwd, plus the head-summed
    attention mass [B,S,K] fp32 when ``return_mass`` (bf16 path; the same quantity as
    ``attn_mass``, taken from the probabilities the backward recomputes anyway), plus
    d sinks [H] fp32 last when ``sinks`` is given (dsa_sparse_mla_bwd_sink; smax / ssum must
    then be the statistics sparse_mla_fwd returned with the same sinks).

    ``workspace_bytes`` caps the scratch (fewer bytes -> more query-row chunks).
    """
    global _attn_mass_entry
    lib = load_library()
    B, S, H, D = q.shape
    s_kv = kv.shape[1]
    K = indices.shape[-1]
    d_v = out.shape[-1]
    indices = indices.reshape(B, S, K).to(torch.int32).contiguous()
    # without return_mass the bf16 path still writes the mass (a few % of the score kernel)
    # and keeps it for the indexer KL op of the same layer (take_attn_mass)
    keep = _share_attn_mass and not return_mass and sinks is None and q.dtype == torch.bfloat16
    if keep:
        _attn_mass_entry = None  # (the old mass goes before the new one is allocated)
        keep_key = _attn_mass_key(q, kv, indices, smax, ssum, scale, q_offset)
        keep_refs = (indices, smax, ssum)
    q, kv, out, dout = (t.contiguous() for t in (q, kv, out, dout))
    dq = torch.empty_like(q)
    dkv = torch.zeros(B, s_kv, D, dtype=torch.float32, device=q.device)
    mass = torch.empty(B, S, K, dtype=torch.float32, device=q.device) if (return_mass or keep) else None
    ws_bytes = int(lib.dsa_sparse_mla_bwd_workspace_size(B, S, s_kv, H, D, K))
    if workspace_bytes is not None:
        ws_bytes = int(workspace_bytes)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    res = (dq, dkv, mass) if return_mass else (dq, dkv)
    # one chunk of rows: the dKV reduction takes the shared pair CSR (also the indexer loss's)
    csr = None
    if _share_pair_csr and q.dtype == torch.bfloat16 and \
            int(lib.dsa_sparse_mla_bwd_chunk_rows(B, S, s_kv, D, K, ws_bytes)) >= S:
        csr = pair_csr(indices, s_kv, q_offset)
    sk = dsink = None
    if sinks is not None:
        sk = _sink_vector(sinks, H, q.device)
        dsink = torch.zeros(H, dtype=torch.float32, device=q.device)
    check(
        lib.dsa_sparse_mla_bwd_ex(ptr(q), ptr(kv), ptr(indices), ptr(out), ptr(dout), ptr(smax), ptr(ssum), ptr(dq),
                                  ptr(dkv), ptr(mass), ptr(sk), ptr(dsink), ptr(csr),
                                  0 if csr is None else csr.numel(), ptr(ws), ws_bytes, _lib.dtype_code(q.dtype), B,
                                  S, s_kv, H, D, d_v, K, float(scale), int(q_offset), stream_of(q.device)),
        "dsa_sparse_mla_bwd",
    )
    if keep:
        _attn_mass_entry = (keep_key, keep_refs, mass)
    return res + (dsink,) if sinks is not None else res


def attn_mass(q, kv, indices, smax, ssum, scale, *, q_offset=0):
    """Head-summed softmax mass [B,S,K] at the selected slots (dsa_attn_mass)."""
    lib = load_library()
    B, S, H, D = q.shape
    s_kv = kv.shape[1]
    K = indices.shape[-1]
    q = q.contiguous()
    kv = kv.contiguous()
    indices = indices.reshape(B, S, K).to(torch.int32).contiguous()
    mass = torch.empty(B, S, K, dtype=torch.float32, device=q.device)
    check(
        lib.dsa_attn_mass(ptr(q), ptr(kv), ptr(indices), ptr(smax.contiguous()), ptr(ssum.contiguous()), ptr(mass),
                          _lib.dtype_code(q.dtype), B, S, s_kv, H, D, K, float(scale), int(q_offset),
                          stream_of(q.device)),
        "dsa_attn_mass",
    )
    return mass


def _varlen_seqs(cu_seqlens_q, cu_seqlens_kv, T, T_kv):
    cu_q = to_cu_seqlens(cu_seqlens_q, None, T)
    cu_k = to_cu_seqlens(cu_seqlens_kv, None, T_kv)
    if len(cu_q) != len(cu_k):
        raise ValueError("cu_seqlens_q and cu_seqlens_kv describe different numbers of sequences")
    return cu_q, cu_k, len(cu_q) - 1


def sparse_mla_fwd_varlen(q, kv, indices, scale, cu_seqlens_q, cu_seqlens_kv, *, d_v=512):
    """Packed varlen forward (dsa_sparse_mla_fwd_varlen): q [T,H,D_qk], kv [T_kv,D_qk],
    indices [T,K] sequence-local; returns (out [T,H,d_v], softmax_max [T,H], softmax_sum [T,H]).
    With GPU-tensor bounds the batch runs as one launch on global key rows
    (tnd_global_indices), with no host read; with host bounds, one launch per sequence."""
    lib = load_library()
    require_gpu_tensor(q, "q")
    T, H, D = q.shape
    kv = kv.reshape(kv.shape[0], kv.shape[-1]).contiguous()
    g = _varlen_global(indices, cu_seqlens_q, cu_seqlens_kv, T, kv.shape[0], q.device)
    if g is not None:  # device bounds: one launch over the batch
        out, smax, ssum = sparse_mla_fwd(q.unsqueeze(0), kv.unsqueeze(0), g.unsqueeze(0), scale, d_v=d_v,
                                         q_offset=_NO_MASK_OFFSET)
        return out[0], smax[0], ssum[0]
    cu_q, cu_k, n_seq = _varlen_seqs(cu_seqlens_q, cu_seqlens_kv, T, kv.shape[0])
    K = indices.shape[-1]
    q = q.contiguous()
    indices = indices.reshape(T, K).to(torch.int32).contiguous()
    out = torch.empty(T, H, d_v, dtype=q.dtype, device=q.device)
    smax = torch.empty(T, H, dtype=torch.float32, device=q.device)
    ssum = torch.empty(T, H, dtype=torch.float32, device=q.device)
    if T:
        check(
            lib.dsa_sparse_mla_fwd_varlen(ptr(q), ptr(kv), ptr(indices), ptr(out), ptr(smax), ptr(ssum),
                                          _lib.dtype_code(q.dtype), host_i32(cu_q), host_i32(cu_k), n_seq, H, D, d_v,
                                          K, float(scale), stream_of(q.device)),
            "dsa_sparse_mla_fwd_varlen",
        )
    return out, smax, ssum


def sparse_mla_bwd_varlen(q, kv, indices, out, dout, smax, ssum, scale, cu_seqlens_q, cu_seqlens_kv, *,
                          return_mass=False, workspace_bytes=None):
    """Packed varlen backward (dsa_sparse_mla_bwd_varlen): (dq like q, dkv fp32 [T_kv,D_qk])
    and, with ``return_mass``, the head-summed attention mass [T,K] fp32."""
    lib = load_library()
    T, H, D = q.shape
    kv = kv.reshape(kv.shape[0], kv.shape[-1]).contiguous()
    T_kv = kv.shape[0]
    g = _varlen_global(indices, cu_seqlens_q, cu_seqlens_kv, T, T_kv, q.device)
    if g is not None:  # device bounds: one launch over the batch
        res = sparse_mla_bwd(q.unsqueeze(0), kv.unsqueeze(0), g.unsqueeze(0), out.unsqueeze(0), dout.unsqueeze(0),
                             smax.unsqueeze(0), ssum.unsqueeze(0), scale, q_offset=_NO_MASK_OFFSET,
                             workspace_bytes=workspace_bytes, return_mass=return_mass)
        return tuple(t[0] for t in res)
    cu_q, cu_k, n_seq = _varlen_seqs(cu_seqlens_q, cu_seqlens_kv, T, T_kv)
    K = indices.shape[-1]
    d_v = out.shape[-1]
    q, out, dout = (t.contiguous() for t in (q, out, dout))
    indices = indices.reshape(T, K).to(torch.int32).contiguous()
    dq = torch.empty_like(q)
    dkv = torch.zeros(T_kv, D, dtype=torch.float32, device=q.device)
    mass = torch.empty(T, K, dtype=torch.float32, device=q.device) if return_mass else None
    hq, hk = host_i32(cu_q), host_i32(cu_k)
    ws_bytes = int(lib.dsa_sparse_mla_bwd_varlen_workspace_size(hq, hk, n_seq, H, D, K))
    if workspace_bytes is not None:
        ws_bytes = int(workspace_bytes)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    if T:
        check(
            lib.dsa_sparse_mla_bwd_varlen(ptr(q), ptr(kv), ptr(indices), ptr(out), ptr(dout), ptr(smax.contiguous()),
                                          ptr(ssum.contiguous()), ptr(dq), ptr(dkv), ptr(mass), ptr(ws), ws_bytes,
                                          _lib.dtype_code(q.dtype), hq, hk, n_seq, H, D, d_v, K, float(scale),
                                          stream_of(q.device)),
            "dsa_sparse_mla_bwd_varlen",
        )
    return (dq, dkv, mass) if return_mass else (dq, dkv)


def attn_mass_varlen(q, kv, indices, smax, ssum, scale, cu_seqlens_q, cu_seqlens_kv):
    """Head-summed softmax mass [T,K] of a packed varlen batch (dsa_attn_mass_varlen)."""
    lib = load_library()
    T, H, D = q.shape
    kv = kv.reshape(kv.shape[0], kv.shape[-1]).contiguous()
    g = _varlen_global(indices, cu_seqlens_q, cu_seqlens_kv, T, kv.shape[0], q.device)
    if g is not None:  # device bounds: one launch over the batch
        return attn_mass(q.unsqueeze(0), kv.unsqueeze(0), g.unsqueeze(0), smax.unsqueeze(0), ssum.unsqueeze(0), scale,
                         q_offset=_NO_MASK_OFFSET)[0]
    cu_q, cu_k, n_seq = _varlen_seqs(cu_seqlens_q, cu_seqlens_kv, T, kv.shape[0])
    K = indices.shape[-1]
    q = q.contiguous()
    indices = indices.reshape(T, K).to(torch.int32).contiguous()
    mass = torch.empty(T, K, dtype=torch.float32, device=q.device)
    if T:
        check(
            lib.dsa_attn_mass_varlen(ptr(q), ptr(kv), ptr(indices), ptr(smax.contiguous()), ptr(ssum.contiguous()),
                                     ptr(mass), _lib.dtype_code(q.dtype), host_i32(cu_q), host_i32(cu_k), n_seq, H, D,
                                     K, float(scale), stream_of(q.device)),
            "dsa_attn_mass_varlen",
        )
    return mass


def _packed_view(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor | None:
    """If ``a`` and ``b`` are the two halves of one contiguous last-dim split, return the whole."""
    if a.dtype != b.dtype or a.shape[:-1] != b.shape[:-1] or a.stride() != b.stride() or a.stride(-1) != 1:
        return None
    width = a.shape[-1] + b.shape[-1]
    if b.data_ptr() != a.data_ptr() + a.shape[-1] * a.element_size():
        return None
    full = a.as_strided(a.shape[:-1] + (width,), a.stride())
    return full if full.is_contiguous() else None


def _cat_last(a, b):
    packed = _packed_view(a, b)
    return packed if packed is not None else torch.cat([a, b], dim=-1).contiguous()


class _SparseFlashAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q_nope, k_nope, q_pe, k_pe, indices, scale, q_offset):
        q = _cat_last(q_nope, q_pe)  # [B,S,H,576]
        kv = _cat_last(k_nope, k_pe)  # [B,S_kv,1,576]
        B, S, H, _ = q.shape
        kv3 = kv.reshape(kv.shape[0], kv.shape[1], kv.shape[-1])
        out, smax, ssum = sparse_mla_fwd(q, kv3, indices, scale, d_v=q_nope.shape[-1], q_offset=q_offset)
        ctx.save_for_backward(q, kv3, indices, out, smax, ssum)
        ctx.scale = scale
        ctx.q_offset = q_offset
        ctx.split = (q_nope.shape[-1], q_pe.shape[-1])
        ctx.kv_shape = kv.shape
        ctx.mark_non_differentiable(smax, ssum)
        return out, smax, ssum

    @staticmethod
    def backward(ctx, dout, _dmax, _dsum):
        q, kv3, indices, out, smax, ssum = ctx.saved_tensors
        dq, dkv = sparse_mla_bwd(q, kv3, indices, out, dout.contiguous(), smax, ssum, ctx.scale, q_offset=ctx.q_offset)
        dnope, dpe = ctx.split
        dkv = dkv.to(kv3.dtype).reshape(ctx.kv_shape)
        return dq[..., :dnope], dkv[..., :dnope], dq[..., dnope:], dkv[..., dnope:], None, None, None


class MassLink:
    """Hands the head-summed attention mass [B,S,K] from a layer's attention backward to the
    same layer's indexer-loss backward, so the loss's target is not recomputed.

    The link holds no tensor between forward and backward: the attention node owns its
    inputs through ``save_for_backward`` (so saved-tensor hooks, and with them activation
    checkpointing, see them), and ``attn`` is only a weak reference to that node, through
    which a backward of the loss alone (attention node not run) reaches the saved forward
    statistics.  ``mass`` is set by each run of the attention backward and kept until the
    graph is freed, so a second backward with ``retain_graph=True`` finds it again."""

    __slots__ = ("mass", "attn", "scale", "q_offset")

    def __init__(self):
        self.mass = None
        self.attn = None
        self.scale = None
        self.q_offset = 0

    def recompute_mass(self):
        """The mass from the attention node's saved forward statistics (``dsa_attn_mass``)."""
        node = self.attn() if self.attn is not None else None
        if node is None:
            raise RuntimeError("the indexer loss of this DSA layer takes its target from the layer's attention, "
                               "whose autograd node is gone; backpropagate through the attention output as well")
        q, kv3, indices, _out, smax, ssum = node.saved_tensors
        return attn_mass(q, kv3, indices, smax, ssum, self.scale, q_offset=self.q_offset)


class _SparseFlashAttentionLinked(torch.autograd.Function):
    """Absorb-mode attention on whole 576-column rows (query [B,S,H,576], key [B,S_kv,1,576],
    any strides: each becomes one contiguous copy at most, no split and re-concatenation)
    whose backward also produces the attention mass (the fused output of
    dsa_sparse_mla_bwd) into ``link``.  ``after`` is the indexer loss's (zero) output: as an
    input here it makes the loss node's backward wait for this one."""

    @staticmethod
    def forward(ctx, query, key, indices, scale, q_offset, d_v, after, link):
        q = query.contiguous()
        kv3 = key.reshape(key.shape[0], key.shape[1], key.shape[-1]).contiguous()
        out, smax, ssum = sparse_mla_fwd(q, kv3, indices, scale, d_v=d_v, q_offset=q_offset)
        ctx.save_for_backward(q, kv3, indices, out, smax, ssum)
        ctx.scale = scale
        ctx.q_offset = q_offset
        ctx.kv_shape = key.shape
        ctx.link = link
        link.attn = weakref.ref(ctx)  # (the node itself; no tensor is kept in the link)
        link.scale = scale
        link.q_offset = q_offset
        ctx.mark_non_differentiable(smax, ssum)
        return out, smax, ssum

    @staticmethod
    def backward(ctx, dout, _dmax, _dsum):
        q, kv3, indices, out, smax, ssum = ctx.saved_tensors
        dq, dkv, mass = sparse_mla_bwd(q, kv3, indices, out, dout.contiguous(), smax, ssum, ctx.scale,
                                       q_offset=ctx.q_offset, return_mass=True)
        ctx.link.mass = mass
        return dq, dkv.to(kv3.dtype).reshape(ctx.kv_shape), None, None, None, None, None, None


def sparse_flash_attention_linked(query, key, sparse_indices, scale_value, after, link, *, d_v=512, sparse_mode=3):
    """Absorb-mode sparse attention (``npu_sparse_flash_attention`` semantics, BSND) on whole
    rows - query [B,S,H,576] = [q_nope | q_pe], key [B,S_kv,1,576] = [k_nope | k_pe], the value
    being the first ``d_v`` columns of the key - for a layer whose indexer loss takes its
    target from this attention's backward: returns (out [B,S,H,d_v], softmax_max,
    softmax_sum) and, in backward, leaves the head-summed mass [B,S,K] in ``link.mass`` (a
    ``MassLink``).  ``after`` is the loss's output tensor (see _SparseFlashAttentionLinked)."""
    q_off = _resolve_q_offset(sparse_mode, query.shape[1], key.shape[1], None)
    idx = sparse_indices.reshape(query.shape[0], query.shape[1], -1).to(torch.int32).contiguous()
    return _SparseFlashAttentionLinked.apply(query, key, idx, float(scale_value), q_off, int(d_v), after, link)


class _SparseFlashAttentionTND(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q_nope, k_nope, q_pe, k_pe, indices, scale, cu_q, cu_k):
        q = _cat_last(q_nope, q_pe)  # [T,H,576]
        kv = _cat_last(k_nope, k_pe)  # [T_kv,1,576]
        kv2 = kv.reshape(kv.shape[0], kv.shape[-1])
        out, smax, ssum = sparse_mla_fwd_varlen(q, kv2, indices, scale, cu_q, cu_k, d_v=q_nope.shape[-1])
        ctx.save_for_backward(q, kv2, indices, out, smax, ssum)
        ctx.scale = scale
        ctx.cu = (cu_q, cu_k)
        ctx.split = (q_nope.shape[-1], q_pe.shape[-1])
        ctx.kv_shape = kv.shape
        ctx.mark_non_differentiable(smax, ssum)
        return out, smax, ssum

    @staticmethod
    def backward(ctx, dout, _dmax, _dsum):
        q, kv2, indices, out, smax, ssum = ctx.saved_tensors
        dq, dkv = sparse_mla_bwd_varlen(q, kv2, indices, out, dout.contiguous(), smax, ssum, ctx.scale, *ctx.cu)
        dnope, _ = ctx.split
        dkv = dkv.to(kv2.dtype).reshape(ctx.kv_shape)
        return dq[..., :dnope], dkv[..., :dnope], dq[..., dnope:], dkv[..., dnope:], None, None, None, None


def npu_sparse_flash_attention(
    query,
    key,
    value,
    sparse_indices,
    block_table=None,
    query_rope=None,
    key_rope=None,
    scale_value=1.0,
    sparse_block_size=1,
    layout_query="BSND",
    layout_kv="BSND",
    sparse_mode=3,
    attention_mode=2,
    return_softmax_lse=True,
    *,
    actual_seq_lengths_query=None,
    actual_seq_lengths_kv=None,
    cu_seqlens_q=None,
    cu_seqlens_kv=None,
    q_offset=None,
):
    """Gathered sparse MLA attention in absorb mode (attention_mode=2).

    query [B,S,H,512] (q_nope), key [B,S_kv,1,512] (k_nope), value (must be k_nope: the
    absorbed latent is both key and value), query_rope [B,S,H,64], key_rope [B,S_kv,1,64],
    sparse_indices [B,S,1,K] int32 (-1 = empty).  Returns (out [B,S,H,512], softmax_max
    [B,S,H], softmax_sum [B,S,H]); differentiable in query/key/query_rope/key_rope, with
    the value gradient folded into the key gradient (dKV_latent = dK_nope + dV).

    TND: query [T,H,512], key [T_kv,1,512], ropes [T,H,64] / [T_kv,1,64], sparse_indices
    [T,1,K] sequence-local; sequences from ``actual_seq_lengths_*`` (cumulative ends) or
    ``cu_seqlens_*``; causal within each sequence (sparse_mode 3).
    """
    if attention_mode != 2:
        raise NotImplementedError("only attention_mode=2 (MLA absorb) is supported")
    if block_table is not None or sparse_block_size != 1:
        raise NotImplementedError("sparse_block_size=1 and no block_table")
    if layout_query not in ("BSND", "TND") or layout_kv != layout_query:
        raise NotImplementedError(f"layouts {layout_query}/{layout_kv} (BSND/BSND or TND/TND)")
    if query_rope is None or key_rope is None:
        raise ValueError("query_rope and key_rope are required in absorb mode")
    if layout_query == "TND":
        if sparse_mode != 3 or q_offset is not None:
            raise NotImplementedError("TND runs the per-sequence causal rule (sparse_mode=3) only")
        cu_q = seq_bounds(cu_seqlens_q, actual_seq_lengths_query, query.shape[0])
        cu_k = seq_bounds(cu_seqlens_kv, actual_seq_lengths_kv, key.shape[0])
        idx = sparse_indices.reshape(query.shape[0], -1)
        return _SparseFlashAttentionTND.apply(query, key, query_rope, key_rope, idx, float(scale_value), cu_q, cu_k)
    if actual_seq_lengths_query is not None or actual_seq_lengths_kv is not None:
        raise NotImplementedError("BSND with actual_seq_lengths: pack the batch as TND instead")
    s_kv = key.shape[1]
    q_off = _resolve_q_offset(sparse_mode, query.shape[1], s_kv, q_offset)
    idx = sparse_indices.reshape(query.shape[0], query.shape[1], -1)
    out, smax, ssum = _SparseFlashAttention.apply(query, key, query_rope, key_rope, idx, float(scale_value), q_off)
    return out, smax, ssum


# ---------------------------------------------------------------------------
# DeepSeek-V4 shared-KV sparse attention: sliding window + compressed KV + sink
# ---------------------------------------------------------------------------
def v4_attention_indices(B, S, device, *, win_left=127, win_right=0, cmp_ratio=1, n_cmp=0, cmp_indices=None):
    """int32 [B,S,W(+K)] slot indices over cat(ori_kv, cmp_kv), -1 = empty.

    Window slots: ori tokens t in [s - win_left, s + win_right] (reference
    GetWindowTopkIdxs, models/deepseek_v4/model.py:467-471, is the win_right = 0 case).
    Compressed slots (cmp_ratio > 1, ``n_cmp`` compressed rows): ``cmp_indices`` as given
    (offset by S, as LiCompute returns them), or every causal block t < (s+1)//r
    offset by S (GetCompressTopkIdxs, :483-488; the ratio-128 layers).
    """
    W = win_left + win_right + 1
    s_pos = torch.arange(S, device=device).view(S, 1)
    w = s_pos - win_left + torch.arange(W, device=device).view(1, W)
    w = torch.where((w >= 0) & (w < S), w, torch.full_like(w, -1))
    idx = w.unsqueeze(0).expand(B, S, W)
    if cmp_ratio > 1 and n_cmp > 0:
        if cmp_indices is None:
            t = torch.arange(n_cmp, device=device).view(1, n_cmp)
            c = torch.where(t < (s_pos + 1) // cmp_ratio, t + S, torch.full_like(t, -1))
            cmp_indices = c.unsqueeze(0).expand(B, S, n_cmp)
        idx = torch.cat([idx, cmp_indices.to(device=device, dtype=idx.dtype)], dim=-1)
    return idx.to(torch.int32).contiguous()


def _cu_device(cu, device) -> torch.Tensor:
    """int64 device copy of a cu_seqlens-style tensor or list (no host read of a device tensor)."""
    if isinstance(cu, torch.Tensor):
        return cu.to(device=device, dtype=torch.int64).reshape(-1)
    return torch.tensor([int(v) for v in cu], dtype=torch.int64, device=device)


def sharedkv_tnd_indices(cu_seqlens_q, cu_seqlens_ori_kv, T, T_ori, device, *, win_left=127, win_right=0,
                         cmp_ratio=1, cu_seqlens_cmp_kv=None, cmp_residual_kv=None, cmp_indices=None, max_cmp=0,
                         window=True):
    """int32 [T, W(+K)] slot indices of a packed ("TND") shared-KV batch over the rows of
    cat(ori_kv [T_ori], cmp_kv), -1 = empty; built on the device from the cu_seqlens tensors
    (no host read).

    Query t of sequence i (position p = t - cu_seqlens_q[i]) sees the ori rows of its own
    sequence at positions [p - win_left, p + win_right] (ori_mask_mode 4; ori and query
    tokens are the same positions, as in the reference's global TND batch) and, with
    compressed keys (cmp_ratio > 1, cmp_mask_mode 3), the compressed rows c of its sequence
    with c < (p + 1 + o_i) // cmp_ratio, o_i = max(0, cmp_ratio * n_i + residual_i - len_i)
    (n_i compressed rows, residual_i original tokens after the last whole block): for ratio 4
    the entries of ``cmp_indices`` [T, K] (sequence-local, as the indexer returns them; -1
    and entries outside that rule stay empty), otherwise every such row, in ``max_cmp``
    (>= the longest compressed sequence) slots.  The same rules over one sequence are what
    ``v4_attention_indices`` builds for a BSND batch.  ``window=False`` leaves the window
    columns out (the compressed rows alone, numbered from ``T_ori``).
    """
    cu_q = _cu_device(cu_seqlens_q, device)
    cu_o = _cu_device(cu_seqlens_ori_kv if cu_seqlens_ori_kv is not None else cu_seqlens_q, device)
    t = torch.arange(T, device=device)
    seq = torch.searchsorted(cu_q[1:].contiguous(), t, right=True).clamp_(max=cu_q.numel() - 2)
    pos = t - cu_q[seq]
    len_o = (cu_o[seq + 1] - cu_o[seq]).view(T, 1)
    W = int(win_left) + int(win_right) + 1
    j = pos.view(T, 1) - int(win_left) + torch.arange(W, device=device).view(1, W)
    win = torch.where((j >= 0) & (j < len_o), cu_o[seq].view(T, 1) + j, torch.full_like(j, -1))
    if not window:
        win = win[:, :0]
    if cmp_ratio <= 1 or cu_seqlens_cmp_kv is None:
        return win.to(torch.int32).contiguous()
    r = int(cmp_ratio)
    cu_c = _cu_device(cu_seqlens_cmp_kv, device)
    n_c = cu_c[seq + 1] - cu_c[seq]
    res = _cu_device(cmp_residual_kv, device)[seq] if cmp_residual_kv is not None else torch.zeros_like(n_c)
    len_q = cu_q[seq + 1] - cu_q[seq]
    off = (r * n_c + res - len_q).clamp(min=0)
    lim = torch.minimum((pos + 1 + off) // r, n_c).view(T, 1)
    base = (int(T_ori) + cu_c[seq]).view(T, 1)
    if cmp_indices is not None:
        c = cmp_indices.reshape(T, -1).to(torch.int64)
    else:
        c = torch.arange(int(max_cmp), device=device).view(1, -1).expand(T, -1)
    cmp = torch.where((c >= 0) & (c < lim), base + c, torch.full_like(c, -1))
    return torch.cat([win, cmp], dim=1).to(torch.int32).contiguous()


def _pad_rows(x: torch.Tensor, width: int) -> torch.Tensor:
    if x.shape[-1] == width:
        return x.contiguous()
    pad = x.new_zeros(*x.shape[:-1], width - x.shape[-1])
    return torch.cat([x, pad], dim=-1).contiguous()


def attn_sink_fold_(out, smax, ssum, sinks):
    """In place (dsa_attn_sink_fold): out [.., H, d_v] *= a / s2 and (smax, ssum) <- (m2, s2)
    with m2 = max(smax, sink), a = ssum e^(smax - m2), s2 = a + e^(sink - m2)."""
    lib = load_library()
    H, dv = out.shape[-2], out.shape[-1]
    rows = out.numel() // (H * dv) if out.numel() else 0
    if rows:
        check(lib.dsa_attn_sink_fold(ptr(out), ptr(smax), ptr(ssum), ptr(sinks.float().contiguous()),
                                     _lib.dtype_code(out.dtype), rows, H, dv, stream_of(out.device)),
              "dsa_attn_sink_fold")
    return out, smax, ssum


def attn_sink_grad(out, dout, m2, s2, sinks):
    """d sink [H] fp32 = - sum over rows of e^(sink - m2) / s2 * rowsum(dout * out)
    (dsa_attn_sink_grad)."""
    lib = load_library()
    H, dv = out.shape[-2], out.shape[-1]
    rows = out.numel() // (H * dv) if out.numel() else 0
    dsink = torch.zeros(H, dtype=torch.float32, device=out.device)
    if rows:
        check(lib.dsa_attn_sink_grad(ptr(out), ptr(dout), ptr(m2), ptr(s2), ptr(sinks.float().contiguous()),
                                     ptr(dsink), _lib.dtype_code(out.dtype), rows, H, dv, stream_of(out.device)),
              "dsa_attn_sink_grad")
    return dsink


_SHAREDKV_MAGIC = 0x44534B56  # "DSKV": first word of the metadata record
_LAYOUT_CODES = {"BSND": 1, "TND": 2, "SBH": 3, "BSH": 4}


def npu_sparse_attn_sharedkv_metadata(
    cu_seqlens_q=None,
    seqused_ori_kv=None,
    seqused_cmp_kv=None,
    seqused_q=None,
    seqused_kv=None,
    num_heads_q=1,
    num_heads_kv=1,
    head_dim=512,
    batch_size=1,
    max_seqlen_q=0,
    max_seqlen_kv=0,
    ori_topk=0,
    cmp_topk=0,
    cmp_ratio=1,
    ori_mask_mode=4,
    cmp_mask_mode=3,
    ori_win_left=127,
    ori_win_right=0,
    layout_q="SBH",
    layout_kv="SBH",
    has_ori_kv=True,
    has_cmp_kv=False,
    *,
    device=None,
):
    """Launch metadata of the shared-KV attention (reference binding
    ``npu_sparse_attn_sharedkv_metadata``, ops/aclnn/sparse_attn_sharedkv/binding.cpp:12-28):
    an int32 [1024] device tensor, as the binding returns.

    Here the gathered-attention kernels schedule themselves from the shapes, so the record
    only carries the problem description (magic, version, heads, head_dim, batch, sequence
    lengths, top-k, ratio, mask modes, window, layout codes, which KV sets exist) for
    ``npu_sparse_attn_sharedkv`` to check against its own arguments; the host copy of the
    record rides on the tensor, so the check reads no device memory.
    """
    if num_heads_kv != 1:
        raise NotImplementedError(f"num_heads_kv={num_heads_kv}: the shared KV has one head")
    if ori_mask_mode != 4 or cmp_mask_mode != 3:
        raise NotImplementedError("mask modes: band window (4) over ori_kv, causal (3) over cmp_kv")
    for name, t in (("seqused_ori_kv", seqused_ori_kv), ("seqused_cmp_kv", seqused_cmp_kv),
                    ("seqused_q", seqused_q), ("seqused_kv", seqused_kv)):
        if t is not None and t.numel():
            raise NotImplementedError(f"{name} (per-batch used lengths) is not supported")
    if device is None:
        device = cu_seqlens_q.device if cu_seqlens_q is not None else torch.device("cuda", torch.cuda.current_device())
    rec = [_SHAREDKV_MAGIC, 1, int(num_heads_q), int(num_heads_kv), int(head_dim), int(batch_size),
           int(max_seqlen_q), int(max_seqlen_kv), int(ori_topk), int(cmp_topk), int(cmp_ratio), int(ori_mask_mode),
           int(cmp_mask_mode), int(ori_win_left), int(ori_win_right), _LAYOUT_CODES.get(str(layout_q), 0),
           _LAYOUT_CODES.get(str(layout_kv), 0), int(bool(has_ori_kv)), int(bool(has_cmp_kv))]
    meta = torch.zeros(1024, dtype=torch.int32)
    meta[: len(rec)] = torch.tensor(rec, dtype=torch.int32)
    meta = meta.to(device)
    meta._dsa_record = tuple(rec)
    return meta


def _check_sharedkv_metadata(metadata, query, cmp_kv, cmp_ratio, ori_win_left, ori_win_right):
    rec = getattr(metadata, "_dsa_record", None) if metadata is not None else None
    if rec is None:
        return
    if query.dim() == 3:  # TND: [T, N, D]; the record's batch size counts sequences
        H, D = query.shape[1:]
        B = rec[5]
    else:
        B, S, H, D = query.shape
    want = dict(num_heads_q=(2, H), head_dim=(4, D), batch_size=(5, B), cmp_ratio=(10, cmp_ratio),
                ori_win_left=(13, ori_win_left), ori_win_right=(14, ori_win_right), has_cmp_kv=(18, int(cmp_kv is not None)))
    for name, (i, v) in want.items():
        if rec[i] != int(v):
            raise ValueError(f"metadata was built for {name}={rec[i]}, the call has {v}")


def _sharedkv_prepare(query, ori_kv, cmp_kv, cmp_sparse_indices, cmp_ratio, ori_win_left, ori_win_right, tnd=None):
    """Kernel operands of the shared-KV attention: query and cat(ori_kv, cmp_kv) rows as the
    gathered-attention kernels take them (bf16: 512-column rows, the kernels' rope-less
    width, zero-padded when D < 512; fp32: as given) and the [B,S,W(+K)] slot indices over
    the concatenated rows.  ``tnd`` (a dict of cu_seqlens_q / cu_seqlens_ori_kv /
    cu_seqlens_cmp_kv / cmp_residual_kv / max_cmp) marks a packed batch: query [T,N,D],
    ori_kv [T_ori,(1,)D], cmp_kv [T_c,(1,)D], cmp_sparse_indices [T,(1,)K] sequence-local;
    it runs as one [1,T] batch whose slot indices keep every query inside its sequence."""
    if tnd is not None:
        T, H, D = query.shape
        ori = ori_kv.reshape(1, ori_kv.shape[0], ori_kv.shape[-1])
        cmp = None if cmp_kv is None else cmp_kv.reshape(1, cmp_kv.shape[0], cmp_kv.shape[-1])
        cmp_ratio = int(cmp_ratio) if cmp is not None else 1
        ci = None
        if cmp_ratio == 4:
            if cmp_sparse_indices is None:
                raise ValueError("cmp_ratio 4 needs cmp_sparse_indices")
            ci = cmp_sparse_indices.reshape(T, -1)
        idx = sharedkv_tnd_indices(tnd["cu_seqlens_q"], tnd.get("cu_seqlens_ori_kv"), T, ori.shape[1], query.device,
                                   win_left=int(ori_win_left), win_right=int(ori_win_right), cmp_ratio=cmp_ratio,
                                   cu_seqlens_cmp_kv=tnd.get("cu_seqlens_cmp_kv"),
                                   cmp_residual_kv=tnd.get("cmp_residual_kv"), cmp_indices=ci,
                                   max_cmp=int(tnd.get("max_cmp", 0)))
        query = query.reshape(1, T, H, D)
        idx = idx.unsqueeze(0)
    else:
        B, S, H, D = query.shape
        ori = ori_kv.reshape(ori_kv.shape[0], ori_kv.shape[1], ori_kv.shape[-1])
        cmp = None if cmp_kv is None else cmp_kv.reshape(cmp_kv.shape[0], cmp_kv.shape[1], cmp_kv.shape[-1])
        if cmp_sparse_indices is not None and cmp_sparse_indices.dim() == 4:
            cmp_sparse_indices = cmp_sparse_indices.squeeze(2)
        n_cmp = 0 if cmp is None else cmp.shape[1]
        idx = v4_attention_indices(B, S, query.device, win_left=int(ori_win_left), win_right=int(ori_win_right),
                                   cmp_ratio=int(cmp_ratio), n_cmp=n_cmp,
                                   cmp_indices=cmp_sparse_indices if cmp_ratio == 4 else None)
    kv = ori if cmp is None else torch.cat([ori, cmp], dim=1)
    bf16 = query.dtype == torch.bfloat16
    if bf16 and D > 512:
        raise NotImplementedError(f"bf16 shared-KV attention needs head_dim <= 512 (got {D})")
    # bf16: 512-column rows (k = v = the whole row; the kernels' d_qk = d_v = 512 variant,
    # no rope columns).  fp32: the exact kernel takes any width.
    dqk, dv = (512, 512) if bf16 else (D, D)
    W = int(ori_win_left) + int(ori_win_right) + 1
    return dict(q=_pad_rows(query, dqk), kv=_pad_rows(kv, dqk), idx=idx, D=D, dv=dv, s_ori=ori.shape[1],
                has_cmp=cmp is not None, W=W, tnd=tnd is not None)


def _sharedkv_forward(prep, sinks, scale):
    """(out [B,S,H,dv] with the sink folded in, m2, s2): the row statistics include the sink."""
    return sparse_mla_fwd(prep["q"], prep["kv"], prep["idx"], scale, d_v=prep["dv"], q_offset=_NO_MASK_OFFSET,
                          sinks=sinks)


def _sharedkv_backward(prep, out, dout, m2, s2, sinks, scale, *, return_cmp_mass=False):
    """(dq [B,S,H,D], d_ori [B,S_ori,D], d_cmp [B,S_c,D] or None, d_sink [H] or None), fp32 dKV;
    with ``return_cmp_mass`` also the head-summed probability [B,S,K] at the compressed slots
    (from the probabilities the bf16 backward recomputes; dsa_attn_mass on the fp32 path)."""
    D, dv = prep["D"], prep["dv"]
    dout = _pad_rows(dout.reshape(out.shape[:-1] + dout.shape[-1:]).to(out.dtype), dv) if dv != D else \
        dout.reshape(out.shape).contiguous().to(out.dtype)
    # P_j = exp(x_j - lse) with lse = m2 + log s2 includes the sink, and the kernel's
    # delta = rowsum(dO * O) uses the sink-scaled O: dQ and dKV are exact.  The sink has no
    # value: d sink = -sum over rows of p_sink * rowsum(dO o O), from the same delta pass.
    bf16 = prep["q"].dtype == torch.bfloat16
    fused_mass = return_cmp_mass and bf16
    res = sparse_mla_bwd(prep["q"], prep["kv"], prep["idx"], out, dout, m2, s2, scale, q_offset=_NO_MASK_OFFSET,
                         sinks=sinks, return_mass=fused_mass)
    dq, dkv = res[0], res[1]
    mass = res[2] if fused_mass else None
    dsink = res[-1] if sinks is not None else None
    if return_cmp_mass and mass is None:
        mass = attn_mass(prep["q"], prep["kv"], prep["idx"], m2, s2, scale, q_offset=_NO_MASK_OFFSET)
    dkv = dkv[..., :D]
    s_ori = prep["s_ori"]
    out4 = (dq[..., :D], dkv[:, :s_ori], (dkv[:, s_ori:] if prep["has_cmp"] else None), dsink)
    if return_cmp_mass:
        return out4 + (mass[..., prep["W"]:],)
    return out4


def _check_sharedkv_args(layout_q, layout_kv, ori_sparse_indices, block_tables, seq_tensors, ori_mask_mode,
                         cmp_mask_mode):
    """Returns True for a packed (TND) call: both layouts TND and cu_seqlens_q given (the
    first of ``seq_tensors``); BSND takes no cu_seqlens / seqused tensors."""
    if (layout_q, layout_kv) not in (("BSND", "BSND"), ("TND", "TND")):
        raise NotImplementedError(f"layouts {layout_q}/{layout_kv}: BSND/BSND or TND/TND")
    if ori_sparse_indices is not None:
        raise NotImplementedError("ori_sparse_indices: the window over ori_kv is the band of ori_mask_mode 4")
    if any(t is not None for t in block_tables):
        raise NotImplementedError("paged KV (block tables) is not supported")
    if ori_mask_mode != 4 or cmp_mask_mode != 3:
        raise NotImplementedError("mask modes: band window (4) over ori_kv, causal (3) over cmp_kv")
    if layout_q == "TND":
        if seq_tensors[0] is None:
            raise ValueError("layout TND needs cu_seqlens_q")
        if any(t is not None and t.numel() for t in seq_tensors[3:]):
            raise NotImplementedError("seqused_* (per-sequence used lengths) is not supported")
        return True
    if any(t is not None and t.numel() for t in seq_tensors):
        raise NotImplementedError("cu_seqlens / seqused arguments need layout TND")
    return False


def npu_sparse_attn_sharedkv(
    query,
    ori_kv=None,
    cmp_kv=None,
    ori_sparse_indices=None,
    cmp_sparse_indices=None,
    ori_block_table=None,
    cmp_block_table=None,
    cu_seqlens_q=None,
    cu_seqlens_ori_kv=None,
    cu_seqlens_cmp_kv=None,
    seqused_q=None,
    seqused_kv=None,
    sinks=None,
    metadata=None,
    softmax_scale=1.0,
    cmp_ratio=1,
    ori_mask_mode=4,
    cmp_mask_mode=3,
    ori_kv_stride=0,
    cmp_kv_stride=0,
    ori_win_left=127,
    ori_win_right=0,
    layout_q="BSND",
    layout_kv="BSND",
    return_softmax_lse=True,
):
    """Shared-KV sparse attention forward (reference binding ``npu_sparse_attn_sharedkv``,
    ops/aclnn/sparse_attn_sharedkv/binding.cpp:30-60; math of SparseAttention.forward,
    models/deepseek_v4/model.py:573-623).

    query [B,S,N,D]; ori_kv [B,S,1,D] (window keys, also the values); cmp_kv [B,S_c,1,D] or
    None; cmp_sparse_indices [B,S,1,K] int32, the selected compressed rows offset by S as
    LiCompute returns them (-1 empty; ratio 4 only, every causal block t < (s+1)//r
    otherwise); sinks [N] fp32 (a per-head logit with no value) or None.  Each query sees
    the ori tokens of its band [s - ori_win_left, s + ori_win_right] and its compressed rows.
    Layout TND (packed sequences, ``cu_seqlens_q`` / ``cu_seqlens_ori_kv`` /
    ``cu_seqlens_cmp_kv``): query [T,N,D], ori_kv [T,1,D], cmp_kv [T_c,1,D],
    cmp_sparse_indices [T,1,K] sequence-local; the same rules hold inside each sequence
    (``sharedkv_tnd_indices``).  Returns (attn_out like query, softmax_lse fp32 [B,S,N,1]
    (TND: [T,N,1]) = the natural-log logsumexp of every logit of the row including the
    sink, or None without ``return_softmax_lse``).  Not differentiable by itself:
    ``npu_sparse_attn_sharedkv_grad`` is its backward.
    """
    tnd = _check_sharedkv_args(layout_q, layout_kv, ori_sparse_indices, (ori_block_table, cmp_block_table),
                               (cu_seqlens_q, cu_seqlens_ori_kv, cu_seqlens_cmp_kv, seqused_q, seqused_kv),
                               ori_mask_mode, cmp_mask_mode)
    if ori_kv is None:
        raise NotImplementedError("ori_kv is required (the window keys)")
    require_gpu_tensor(query, "query")
    _check_sharedkv_metadata(metadata, query, cmp_kv, cmp_ratio, ori_win_left, ori_win_right)
    geo = _sharedkv_tnd_args(cu_seqlens_q, cu_seqlens_ori_kv, cu_seqlens_cmp_kv, None, cmp_kv, cmp_ratio) if tnd else None
    prep = _sharedkv_prepare(query.contiguous(), ori_kv.contiguous(), cmp_kv, cmp_sparse_indices, int(cmp_ratio),
                             ori_win_left, ori_win_right, tnd=geo)
    sk = None if sinks is None else sinks.float().contiguous()
    out, m2, s2 = _sharedkv_forward(prep, sk, float(softmax_scale))
    D = prep["D"]
    out = out[..., :D].contiguous() if prep["dv"] != D else out
    lse = (m2 + torch.log(s2)).unsqueeze(-1) if return_softmax_lse else None
    if tnd:
        out = out.reshape(query.shape)
        lse = None if lse is None else lse.reshape(*query.shape[:2], 1)
    return out, lse


def _sharedkv_tnd_args(cu_seqlens_q, cu_seqlens_ori_kv, cu_seqlens_cmp_kv, cmp_residual_kv, cmp_kv, cmp_ratio,
                       max_cmp=None):
    """The ``tnd`` argument of _sharedkv_prepare; ``max_cmp`` (the longest compressed
    sequence, the slot count of the every-causal-block rule) is read from cu_seqlens_cmp_kv
    when not given (a device tensor is read back once per version)."""
    geo = dict(cu_seqlens_q=cu_seqlens_q, cu_seqlens_ori_kv=cu_seqlens_ori_kv, cu_seqlens_cmp_kv=cu_seqlens_cmp_kv,
               cmp_residual_kv=cmp_residual_kv, max_cmp=0)
    if cmp_kv is not None and int(cmp_ratio) > 1:
        if cu_seqlens_cmp_kv is None:
            raise ValueError("compressed KV in layout TND needs cu_seqlens_cmp_kv")
        if max_cmp is None:
            cu = _lib.host_ints(cu_seqlens_cmp_kv)
            max_cmp = max([b - a for a, b in zip(cu[:-1], cu[1:])] or [0])
        geo["max_cmp"] = int(max_cmp)
    return geo


def npu_sparse_attn_sharedkv_grad(
    query,
    ori_kv,
    cmp_kv=None,
    d_out=None,
    out=None,
    lse=None,
    ori_sparse_indices=None,
    cmp_sparse_indices=None,
    cu_seqlens_q=None,
    cu_seqlens_ori_kv=None,
    cu_seqlens_cmp_kv=None,
    sinks=None,
    scale_value=1.0,
    cmp_ratio=1,
    ori_mask_mode=4,
    cmp_mask_mode=3,
    ori_win_left=127,
    ori_win_right=0,
    layout="BSND",
):
    """Backward of ``npu_sparse_attn_sharedkv`` (reference binding
    ``npu_sparse_attn_sharedkv_grad``, ops/aclnn/sparse_attn_sharedkv/binding.cpp:62-88): from
    the forward's output and softmax_lse, returns (d_query like query, d_ori_kv like ori_kv,
    d_cmp_kv like cmp_kv or None, d_sinks like sinks), allocated in the inputs' dtypes as the
    binding does."""
    tnd = _check_sharedkv_args(layout, layout, ori_sparse_indices, (), (cu_seqlens_q, cu_seqlens_ori_kv,
                                                                       cu_seqlens_cmp_kv), ori_mask_mode, cmp_mask_mode)
    if d_out is None or out is None or lse is None or sinks is None:
        raise ValueError("d_out, out, lse and sinks are required")
    geo = _sharedkv_tnd_args(cu_seqlens_q, cu_seqlens_ori_kv, cu_seqlens_cmp_kv, None, cmp_kv, cmp_ratio) if tnd else None
    res = _sharedkv_grad(query, ori_kv, cmp_kv, d_out, out, lse, cmp_sparse_indices, sinks, scale_value, cmp_ratio,
                         ori_win_left, ori_win_right, geo)
    return res[:4]


def _sharedkv_grad(query, ori_kv, cmp_kv, d_out, out, lse, cmp_sparse_indices, sinks, scale_value, cmp_ratio,
                   ori_win_left, ori_win_right, geo, return_cmp_mass=False):
    """npu_sparse_attn_sharedkv_grad's work (BSND, or TND with ``geo``); with
    ``return_cmp_mass`` also the head-summed probability at each compressed slot, fp32
    [B,S,K] (TND: [T,K])."""
    prep = _sharedkv_prepare(query.contiguous(), ori_kv.contiguous(), cmp_kv, cmp_sparse_indices, int(cmp_ratio),
                             ori_win_left, ori_win_right, tnd=geo)
    D, dv = prep["D"], prep["dv"]
    shp = prep["q"].shape[:-1]
    o = out.reshape(*shp, out.shape[-1]).to(prep["q"].dtype)
    o = _pad_rows(o, dv) if dv != D else o.contiguous()
    m2 = lse.reshape(shp).float().contiguous()
    s2 = torch.ones_like(m2)
    res = _sharedkv_backward(prep, o, d_out.reshape(*shp, d_out.shape[-1]), m2, s2, sinks.float().contiguous(),
                             float(scale_value), return_cmp_mass=return_cmp_mass)
    dq, d_ori, d_cmp, dsink = res[:4]
    d_ori = d_ori.reshape(ori_kv.shape).to(ori_kv.dtype)
    d_cmp = None if d_cmp is None or cmp_ratio <= 1 else d_cmp.reshape(cmp_kv.shape).to(cmp_kv.dtype)
    out4 = (dq.reshape(query.shape).to(query.dtype), d_ori, d_cmp, dsink.reshape(sinks.shape).to(sinks.dtype))
    if return_cmp_mass:
        mass = res[4]
        return out4 + (mass.reshape(query.shape[0], -1) if geo is not None else mass,)
    return out4


class SparseAttnSharedKV(torch.autograd.Function):
    """The reference's autograd wrapper of the shared-KV op (converters/kernels/npu_smla.py:192-348),
    same arguments and order: metadata, forward with the LSE saved, and the binding-level
    gradient in backward (query, ori_kv, cmp_kv and sinks)."""

    @staticmethod
    def forward(ctx, query, ori_kv, cmp_kv, cu_seq_lens_q, cu_seq_lens_ori_kv, cu_seq_lens_cmp_kv, ori_sparse_indices,
                cmp_sparse_indices, sinks, softmax_scale, cmp_ratio, ori_mask_mode, cmp_mask_mode, ori_win_left,
                ori_win_right, num_heads_q, num_heads_kv, head_dim, batch_size, max_seq_len_q, max_seq_len_kv, topk,
                layout_q, layout_kv):
        tnd = _check_sharedkv_args(layout_q, layout_kv, ori_sparse_indices, (),
                                   (cu_seq_lens_q, cu_seq_lens_ori_kv, cu_seq_lens_cmp_kv), ori_mask_mode,
                                   cmp_mask_mode)
        metadata = npu_sparse_attn_sharedkv_metadata(
            cu_seq_lens_q, None, None, None, None, num_heads_q, num_heads_kv, head_dim, batch_size, max_seq_len_q,
            max_seq_len_kv, 0, topk, cmp_ratio, ori_mask_mode, cmp_mask_mode, ori_win_left, ori_win_right, layout_q,
            layout_kv, ori_kv is not None, cmp_kv is not None, device=query.device)
        _check_sharedkv_metadata(metadata, query, cmp_kv, cmp_ratio, ori_win_left, ori_win_right)
        # the kernels' operands are kept for backward (the bf16 path pads query rows to 512)
        geo = _sharedkv_tnd_args(cu_seq_lens_q, cu_seq_lens_ori_kv, cu_seq_lens_cmp_kv, None, cmp_kv,
                                 cmp_ratio) if tnd else None
        prep = _sharedkv_prepare(query, ori_kv, cmp_kv, cmp_sparse_indices, int(cmp_ratio), ori_win_left,
                                 ori_win_right, tnd=geo)
        sk = None if sinks is None else sinks.float().contiguous()
        out, m2, s2 = _sharedkv_forward(prep, sk, float(softmax_scale))
        ctx.prep = prep
        ctx.q_shape = query.shape
        ctx.save_for_backward(out, m2, s2, sk)
        ctx.softmax_scale = float(softmax_scale)
        ctx.in_dtypes = (ori_kv.dtype, None if cmp_kv is None else cmp_kv.dtype, None if sinks is None else sinks.dtype)
        ctx.shapes = (ori_kv.shape, None if cmp_kv is None else cmp_kv.shape, None if sinks is None else sinks.shape)
        ctx.cmp_ratio = int(cmp_ratio)
        D = prep["D"]
        res = out[..., :D] if prep["dv"] != D else out
        return res.reshape(query.shape)

    @staticmethod
    def backward(ctx, grad_output):
        out, m2, s2, sk = ctx.saved_tensors
        dq, d_ori, d_cmp, dsink = _sharedkv_backward(ctx.prep, out, grad_output, m2, s2, sk, ctx.softmax_scale)
        dq = dq.reshape(ctx.q_shape)
        ori_dt, cmp_dt, sink_dt = ctx.in_dtypes
        ori_shape, cmp_shape, sink_shape = ctx.shapes
        d_ori = d_ori.reshape(ori_shape).to(ori_dt)
        if d_cmp is not None and ctx.cmp_ratio > 1:
            d_cmp = d_cmp.reshape(cmp_shape).to(cmp_dt)
        else:
            d_cmp = None
        ctx.prep = None
        dsink = None if dsink is None else dsink.reshape(sink_shape).to(sink_dt)
        return (dq, d_ori, d_cmp, *([None] * 5), dsink, *([None] * 15))


def npu_sparse_attn_shared_kv(
    query,
    ori_kv,
    cmp_kv,
    cmp_sparse_indices,
    sinks,
    softmax_scale,
    cmp_ratio,
    ori_mask_mode=4,
    cmp_mask_mode=3,
    ori_win_left=127,
    ori_win_right=0,
):
    """DeepSeek-V4 shared-KV sparse attention (reference npu_sparse_attn_shared_kv,
    converters/kernels/npu_smla.py:351-402; math of SparseAttention.forward,
    models/deepseek_v4/model.py:573-623).

    query [B,S,H,D], ori_kv [B,S,D] (window keys), cmp_kv [B,S/r,D] or None (compressed
    keys), cmp_sparse_indices [B,S,K] int (top-k compressed rows offset by S, -1 empty;
    ratio 4) or None (every causal block), sinks [H] fp32.  Keys and values are the same
    rows (k = v).  Each query sees the ori tokens of its band [s - ori_win_left,
    s + ori_win_right] and the selected compressed rows; the softmax also includes the
    head's sink logit, which carries no value.  Returns [B,S,H,D] (contiguous),
    differentiable in query, ori_kv, cmp_kv and sinks through ``SparseAttnSharedKV``.
    bf16 rows need D <= 512 (MFMA path); fp32 rows any D.
    """
    batch_size, max_seq_len_q, num_heads_q, head_dim = query.size()
    max_seq_len_kv = ori_kv.size(1)
    topk = 0 if cmp_ratio != 4 else cmp_sparse_indices.size(-1)
    layout_q = layout_kv = "BSND"
    query = query.contiguous()
    ori_kv = (ori_kv if ori_kv.dim() == 4 else ori_kv.unsqueeze(2)).contiguous()  # [B,S,1,D]
    if cmp_kv is not None:
        cmp_kv = (cmp_kv if cmp_kv.dim() == 4 else cmp_kv.unsqueeze(2)).contiguous()
    if cmp_ratio == 4:
        cmp_sparse_indices = cmp_sparse_indices.to(torch.int32)
        if cmp_sparse_indices.dim() == 3:
            cmp_sparse_indices = cmp_sparse_indices.unsqueeze(2)
        cmp_sparse_indices = cmp_sparse_indices.contiguous()
    else:
        cmp_sparse_indices = None
    out = SparseAttnSharedKV.apply(query, ori_kv, cmp_kv, None, None, None, None, cmp_sparse_indices, sinks,
                                   float(softmax_scale), int(cmp_ratio), ori_mask_mode, cmp_mask_mode, ori_win_left,
                                   ori_win_right, num_heads_q, 1, head_dim, batch_size, max_seq_len_q,
                                   max_seq_len_kv, topk, layout_q, layout_kv)
    return out.contiguous()


def v4_indexer_kl_grad(q, kv, kv_compress, attn_sink, q_indexer, k_indexer, weights, compress_topk_idxs, offset,
                       softmax_scale, window_size=128, *, eps=1e-10, grad_scale=1.0):
    """DeepSeek-V4 indexer KL loss and its gradients (reference LiLoss, models/deepseek_v4/
    model.py:366-456, the loss of DSAIndexerLoss with eps 1e-10 and loss_scale =
    softmax_scale).  The target is the main attention's probability at each selected
    compressed row (combined softmax over the window keys, the compressed keys and the
    head's sink), averaged over heads: dsa_attn_mass over the same gathered slots as
    npu_sparse_attn_shared_kv with the sink folded into the row statistics.  The student
    scores and the gradients come from dsa_indexer_kl_grad.

    q [B,S,H,D], kv [B,S,D], kv_compress [B,S_c,D], attn_sink [H], q_indexer [B,S,H_I,D_I],
    k_indexer [B,S_c,D_I], weights [B,S,H_I], compress_topk_idxs [B,S,K] (offset by
    ``offset``, -1 empty).  Returns (dq_indexer fp32, dk_indexer fp32 [B,S_c,D_I],
    dweights fp32, loss_rows fp32 [B,S]); gradients are scaled by ``grad_scale``.
    """
    B, S, H, D = q.shape
    cmp = compress_topk_idxs.to(torch.int32)
    local = torch.where(cmp < 0, cmp, cmp - int(offset)).contiguous()
    n_cmp = kv_compress.shape[1]
    idx = v4_attention_indices(B, S, q.device, win_left=window_size - 1, cmp_ratio=2, n_cmp=n_cmp,
                               cmp_indices=torch.where(local < 0, local, local + kv.shape[1]))
    W = window_size
    bf16 = q.dtype == torch.bfloat16
    if bf16 and D > 512:
        raise NotImplementedError(f"bf16 DeepSeek-V4 indexer loss needs head_dim <= 512 (got {D})")
    # bf16: the 512-column kernels (k = v = the whole row, no rope columns); fp32: any width
    dqk, dv = (512, 512) if bf16 else (D, D)
    q_ext = _pad_rows(q.detach(), dqk)
    kv_ext = _pad_rows(torch.cat([kv.detach(), kv_compress.detach()], dim=1), dqk)
    _, m2, s2 = sparse_mla_fwd(q_ext, kv_ext, idx, softmax_scale, d_v=dv, q_offset=_NO_MASK_OFFSET,
                               sinks=attn_sink.detach())
    mass = attn_mass(q_ext, kv_ext, idx, m2, s2, softmax_scale, q_offset=_NO_MASK_OFFSET)
    dist = (mass[..., W:] / H).contiguous()
    return indexer_kl_grad_from_mass(q_indexer, k_indexer, weights, local, dist, q_offset=_NO_MASK_OFFSET,
                                     loss_scale=softmax_scale, eps=eps, grad_scale=grad_scale)


def npu_sparse_lightning_indexer_grad_kl_loss(
    query,
    key,
    query_index,
    key_index,
    weight,
    sparse_indices,
    softmax_max,
    softmax_sum,
    scale_value=1.0,
    *,
    query_rope=None,
    key_rope=None,
    actual_seq_qlen=None,
    actual_seq_klen=None,
    layout="BSND",
    sparse_mode=3,
    pre_tokens=65536,
    next_tokens=65536,
    deterministic=False,
    cmp_ratio=1,
    q_offset=None,
    loss_scale=1.0,
    eps=1e-8,
    grad_scale=1.0,
    cu_seqlens_q=None,
    cu_seqlens_k=None,
):
    """(d_query_index, d_key_index, d_weights, loss fp32[1]) of the indexer KL loss, the
    gradients in the dtypes of query_index / key_index / weight as the binding allocates them
    (sparse_lightning_indexer_grad_kl_loss/binding.cpp:26-29).

    The main-attention target mass at the selected keys is the one the op-level attention
    backward left for exactly these query / key, indices and statistics (take_attn_mass),
    or else recomputed from (query || query_rope, key || key_rope, softmax_max,
    softmax_sum) - bitwise the same mass either way; ``loss`` is the token SUM
    (the caller divides by B*S, reference dsa.py:73).  ``cmp_ratio`` > 1: key / key_index
    are compressed rows (binding.cpp:17) and sparse_indices come from the indexer's
    compressed rule t < (s+1)//r, so the -1 slots carry the validity and no causal test is
    applied on top.  ``deterministic``: always met on the MFMA path - d_key_index sums each
    key's contributions in fp32 in a fixed order (the key-major pair list is placed row by
    row, and the partial sums of keys that straddle reduction segments are added in segment
    order), with no float atomics, so equal inputs give equal bits; the exact fp32 kernel of
    other shapes scatters with fp32 atomics, so ``deterministic=True`` warns there.
    """
    if deterministic and not _kl_mfma_shape(query_index, key_index):
        _warn_nondeterministic()
    out_dtypes = (query_index.dtype, key_index.dtype, weight.dtype)
    if layout == "TND":
        if sparse_mode != 3 or q_offset is not None or int(cmp_ratio) != 1:
            raise NotImplementedError("TND runs the per-sequence causal rule (sparse_mode=3, cmp_ratio=1) only")
        q = _cat_last(query, query_rope) if query_rope is not None else query.contiguous()
        kv = _cat_last(key, key_rope) if key_rope is not None else key.contiguous()
        kv2 = kv.reshape(kv.shape[0], kv.shape[-1])
        cu_q = seq_bounds(cu_seqlens_q, actual_seq_qlen, q.shape[0])
        cu_k = seq_bounds(cu_seqlens_k, actual_seq_klen, kv2.shape[0])
        idx = sparse_indices.reshape(q.shape[0], -1).to(torch.int32).contiguous()
        mass = attn_mass_varlen(q, kv2, idx, softmax_max, softmax_sum, scale_value, cu_q, cu_k)
        dq_i, dk_i, dw, loss_rows = indexer_kl_grad_from_mass_varlen(query_index, key_index, weight, idx, mass, cu_q,
                                                                     cu_k, loss_scale=loss_scale, eps=eps,
                                                                     grad_scale=grad_scale)
        return (dq_i.to(out_dtypes[0]), dk_i.reshape(key_index.shape).to(out_dtypes[1]), dw.to(out_dtypes[2]),
                loss_rows.sum().reshape(1))
    if layout != "BSND":
        raise NotImplementedError(f"layout {layout} (BSND or TND)")
    if actual_seq_qlen is not None or actual_seq_klen is not None:
        return _kl_loss_bsnd_lengths(query, key, query_index, key_index, weight, sparse_indices, softmax_max,
                                     softmax_sum, scale_value, query_rope, key_rope, actual_seq_qlen, actual_seq_klen,
                                     sparse_mode, cmp_ratio, q_offset, loss_scale, eps, grad_scale, out_dtypes)
    q = _cat_last(query, query_rope) if query_rope is not None else query.contiguous()
    kv = _cat_last(key, key_rope) if key_rope is not None else key.contiguous()
    B, S, H, D = q.shape
    kv3 = kv.reshape(B, kv.shape[1], D)
    s_kv = kv3.shape[1]
    if int(cmp_ratio) > 1:
        q_off = _NO_MASK_OFFSET if q_offset is None else int(q_offset)
    else:
        q_off = _resolve_q_offset(sparse_mode, S, s_kv, q_offset)
    idx = sparse_indices.reshape(B, S, -1).to(torch.int32).contiguous()
    if int(cmp_ratio) == 1 and _band_cuts(sparse_mode, S, s_kv, q_off, pre_tokens, next_tokens):
        # selected keys outside the band count as unusable slots in the target and the student
        idx = _band_mask_indices(idx, sparse_mode, q_off, pre_tokens, next_tokens).contiguous()
    elif int(cmp_ratio) != 1 and (int(pre_tokens) < s_kv * int(cmp_ratio) or int(next_tokens) < 0):
        raise NotImplementedError("a pre_tokens / next_tokens band over compressed keys (cmp_ratio > 1)")
    mass = take_attn_mass(q, kv3, idx, softmax_max, softmax_sum, scale_value, q_off)
    if mass is None:
        mass = attn_mass(q, kv3, idx, softmax_max, softmax_sum, scale_value, q_offset=q_off)
    dq_i, dk_i, dw, loss_rows = indexer_kl_grad_from_mass(query_index, key_index, weight, idx, mass, q_offset=q_off,
                                                          loss_scale=loss_scale, eps=eps, grad_scale=grad_scale)
    return (dq_i.to(out_dtypes[0]), dk_i.reshape(key_index.shape).to(out_dtypes[1]), dw.to(out_dtypes[2]),
            loss_rows.sum().reshape(1))


def _kl_loss_bsnd_lengths(query, key, query_index, key_index, weight, sparse_indices, softmax_max, softmax_sum,
                          scale_value, query_rope, key_rope, len_q, len_k, sparse_mode, cmp_ratio, q_offset,
                          loss_scale, eps, grad_scale, out_dtypes):
    """BSND with per-batch valid lengths (``actual_seq_qlen`` / ``actual_seq_klen``, the
    binding's actual_seq_lengths_query / _key): batch b is one sequence of its first len_q[b]
    query rows and len_k[b] key rows, causal bottom-right within those lengths (sparse_mode 3).
    The valid rows are packed into one TND batch for the varlen kernels and the gradients
    scattered back; padded query rows and keys get zero gradients and add no loss."""
    if sparse_mode != 3 or q_offset is not None or int(cmp_ratio) != 1:
        raise NotImplementedError("BSND with actual sequence lengths runs the per-sequence causal rule "
                                  "(sparse_mode=3, cmp_ratio=1) only")
    q = _cat_last(query, query_rope) if query_rope is not None else query.contiguous()
    kv = _cat_last(key, key_rope) if key_rope is not None else key.contiguous()
    B, S, H, D = q.shape
    kv3 = kv.reshape(B, kv.shape[1], D)
    s_k = kv3.shape[1]
    ki3 = key_index.reshape(B, key_index.shape[1], key_index.shape[-1])

    def _lens(v, n):
        vals = [n] * B if v is None else [int(x) for x in (v.tolist() if isinstance(v, torch.Tensor) else v)]
        if len(vals) != B or any(not 0 <= x <= n for x in vals):
            raise ValueError(f"actual sequence lengths {vals} do not fit B={B}, length {n}")
        return vals

    lq, lk = _lens(len_q, S), _lens(len_k, s_k)
    rows_q = torch.cat([torch.arange(n, device=q.device) + b * S for b, n in enumerate(lq)])
    rows_k = torch.cat([torch.arange(n, device=q.device) + b * s_k for b, n in enumerate(lk)])
    cu_q = torch.tensor([0] + list(itertools.accumulate(lq)), dtype=torch.int32, device=q.device)
    cu_k = torch.tensor([0] + list(itertools.accumulate(lk)), dtype=torch.int32, device=q.device)
    idx = sparse_indices.reshape(B * S, -1).to(torch.int32)
    flat = lambda t, n: t.reshape(B * n, *t.shape[2:])  # noqa: E731
    qt, kvt = flat(q, S)[rows_q], kv3.reshape(B * s_k, D)[rows_k]
    it = idx[rows_q].contiguous()
    mass = attn_mass_varlen(qt, kvt, it, flat(softmax_max, S)[rows_q], flat(softmax_sum, S)[rows_q], scale_value,
                            cu_q, cu_k)
    dq_t, dk_t, dw_t, loss_rows = indexer_kl_grad_from_mass_varlen(
        flat(query_index, S)[rows_q], ki3.reshape(B * ki3.shape[1], -1)[rows_k], flat(weight, S)[rows_q], it, mass,
        cu_q, cu_k, loss_scale=loss_scale, eps=eps, grad_scale=grad_scale)
    dq_i = torch.zeros(B * S, *query_index.shape[2:], dtype=out_dtypes[0], device=q.device)
    dk_i = torch.zeros(B * ki3.shape[1], ki3.shape[-1], dtype=out_dtypes[1], device=q.device)
    dw = torch.zeros(B * S, *weight.shape[2:], dtype=out_dtypes[2], device=q.device)
    dq_i[rows_q] = dq_t.to(out_dtypes[0])
    dk_i[rows_k] = dk_t.to(out_dtypes[1])
    dw[rows_q] = dw_t.to(out_dtypes[2])
    return (dq_i.reshape(query_index.shape), dk_i.reshape(key_index.shape), dw.reshape(weight.shape),
            loss_rows.sum().reshape(1))


_warned_nondeterministic = False


def _kl_mfma_shape(query_index, key_index) -> bool:
    """The KL MFMA kernel's shapes (H_I = 64, D_I = 128), whose d_key_index is bitwise
    reproducible; other shapes take the exact fp32 kernel."""
    return query_index.shape[-2] == 64 and query_index.shape[-1] == 128 and key_index.shape[-1] == 128


def _warn_nondeterministic():
    global _warned_nondeterministic
    if not _warned_nondeterministic:
        _warned_nondeterministic = True
        warnings.warn("npu_sparse_lightning_indexer_grad_kl_loss(deterministic=True): shapes other than H_I=64, "
                      "D_I=128 run the exact fp32 kernel, whose d_key_index is reproducible to fp32 rounding only "
                      "(fp32 atomics)", stacklevel=3)


def _grad_scale_args(grad_scale, device):
    """(host float, device fp32 scalar or None): a tensor upstream gradient stays on the device."""
    if isinstance(grad_scale, torch.Tensor):
        if grad_scale.numel() != 1:
            raise ValueError("grad_scale must be a scalar")
        return 1.0, grad_scale.detach().reshape(1).to(device=device, dtype=torch.float32)
    return float(grad_scale), None


def indexer_kl_grad_from_mass(query_index, key_index, weight, indices, mass, *, q_offset=0, loss_scale=1.0, eps=1e-8,
                              grad_scale=1.0, return_softmax=False):
    """(dq_idx fp32, dk_idx fp32 [B,S_k,D_I], dw fp32, loss_rows fp32 [B,S]) given the target mass;
    ``grad_scale`` (a float or a device scalar tensor) multiplies the gradients.  With
    ``return_softmax`` a fifth tensor follows: the indexer's softmax over the slots [B,S,K]
    fp32 (0 at unusable slots; dsa_indexer_kl_grad_softmax)."""
    lib = load_library()
    ki = key_index.squeeze(2) if key_index.dim() == 4 else key_index
    qi = query_index.to(torch.bfloat16).contiguous()
    ki = ki.to(torch.bfloat16).contiguous()
    w = weight.float().contiguous()
    B, S, HI, DI = qi.shape
    s_k = ki.shape[1]
    idx = indices.reshape(B, S, -1).to(torch.int32).contiguous()
    K = idx.shape[-1]
    mass = mass.float().contiguous()
    dev = qi.device
    dq_i = torch.empty(B, S, HI, DI, dtype=torch.float32, device=dev)
    dk_i = torch.zeros(B, s_k, DI, dtype=torch.float32, device=dev)
    dw = torch.empty(B, S, HI, dtype=torch.float32, device=dev)
    loss_rows = torch.empty(B, S, dtype=torch.float32, device=dev)
    ws_bytes = int(lib.dsa_indexer_kl_grad_workspace_size(B, S, s_k, HI, DI, K))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    gsf, gsd = _grad_scale_args(grad_scale, dev)
    sm = torch.empty(B, S, K, dtype=torch.float32, device=dev) if return_softmax else None
    # one chunk of rows: the dK_index reduction takes the shared pair CSR (the attention
    # backward's, when it ran on the same indices)
    csr = None
    if _share_pair_csr and ws_bytes > 0 and int(lib.dsa_indexer_kl_grad_chunk_rows(B, S, s_k, K, ws_bytes)) >= S:
        csr = pair_csr(idx, s_k, q_offset)
    check(
        lib.dsa_indexer_kl_grad_ex(ptr(qi), ptr(ki), ptr(w), ptr(idx), ptr(mass), ptr(dq_i), ptr(dk_i), ptr(dw),
                                   ptr(loss_rows), ptr(sm), ptr(csr), 0 if csr is None else csr.numel(), ptr(ws),
                                   ws_bytes, B, S, s_k, HI, DI, K, int(q_offset), float(loss_scale), float(eps), gsf,
                                   ptr(gsd), stream_of(dev)),
        "dsa_indexer_kl_grad",
    )
    return (dq_i, dk_i, dw, loss_rows, sm) if return_softmax else (dq_i, dk_i, dw, loss_rows)


def indexer_kl_grad_from_mass_varlen(query_index, key_index, weight, indices, mass, cu_seqlens_q, cu_seqlens_k, *,
                                     loss_scale=1.0, eps=1e-8, grad_scale=1.0):
    """Packed varlen indexer KL gradients (dsa_indexer_kl_grad_varlen): query_index
    [T,H_I,D_I], key_index [T_k,D_I] (or [T_k,1,D_I]), weight [T,H_I], indices [T,K]
    sequence-local, mass [T,K].  Returns (dq_idx [T,H_I,D_I], dk_idx [T_k,D_I], dw [T,H_I],
    loss_rows [T]), all fp32."""
    lib = load_library()
    qi = query_index.to(torch.bfloat16).contiguous()
    ki = key_index.reshape(key_index.shape[0], key_index.shape[-1]).to(torch.bfloat16).contiguous()
    w = weight.float().contiguous()
    T, HI, DI = qi.shape
    T_k = ki.shape[0]
    g = _varlen_global(indices, cu_seqlens_q, cu_seqlens_k, T, T_k, qi.device)
    if g is not None:  # device bounds: one launch over the batch
        res = indexer_kl_grad_from_mass(qi.unsqueeze(0), ki.unsqueeze(0), w.unsqueeze(0), g.unsqueeze(0),
                                        mass.reshape(T, -1).unsqueeze(0), q_offset=_NO_MASK_OFFSET,
                                        loss_scale=loss_scale, eps=eps, grad_scale=grad_scale)
        return tuple(t[0] for t in res)
    cu_q, cu_k, n_seq = _varlen_seqs(cu_seqlens_q, cu_seqlens_k, T, T_k)
    idx = indices.reshape(T, -1).to(torch.int32).contiguous()
    K = idx.shape[-1]
    mass = mass.float().contiguous()
    dev = qi.device
    dq_i = torch.empty(T, HI, DI, dtype=torch.float32, device=dev)
    dk_i = torch.zeros(T_k, DI, dtype=torch.float32, device=dev)
    dw = torch.empty(T, HI, dtype=torch.float32, device=dev)
    loss_rows = torch.empty(T, dtype=torch.float32, device=dev)
    hq, hk = host_i32(cu_q), host_i32(cu_k)
    ws_bytes = int(lib.dsa_indexer_kl_grad_varlen_workspace_size(hq, hk, n_seq, HI, DI, K))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    gsf, gsd = _grad_scale_args(grad_scale, dev)
    if T:
        check(
            lib.dsa_indexer_kl_grad_varlen(ptr(qi), ptr(ki), ptr(w), ptr(idx), ptr(mass), ptr(dq_i), ptr(dk_i),
                                           ptr(dw), ptr(loss_rows), ptr(ws), ws_bytes, hq, hk, n_seq, HI, DI, K,
                                           float(loss_scale), float(eps), gsf, ptr(gsd), stream_of(dev)),
            "dsa_indexer_kl_grad_varlen",
        )
    return dq_i, dk_i, dw, loss_rows


# ---------------------------------------------------------------------------
# block KV compressor (V4)
# ---------------------------------------------------------------------------
def rope_cos_sin(freqs_cis: torch.Tensor) -> torch.Tensor:
    """The fp32 [n_pos, rope_dim/2, 2] (cos, sin) table the kernels take, from a complex
    ``freqs_cis`` [n_pos, rope_dim/2] (torch.view_as_real), or an already-real table."""
    t = torch.view_as_real(freqs_cis) if freqs_cis.is_complex() else freqs_cis
    return t.float().contiguous()


def _rope_args(freqs_cis, rope_dim, device):
    if freqs_cis is None:
        return None, 0, 0
    cs = rope_cos_sin(freqs_cis).to(device)
    if cs.shape[-2] * 2 != rope_dim:
        raise ValueError(f"freqs_cis covers {cs.shape[-2] * 2} rope features, rope_dim is {rope_dim}")
    return cs, cs.shape[0], rope_dim


def indexer_prep(x, freqs_cis=None, *, positions=None, pos_offset=0, rope_dim=64, rope_start=0, interleaved=False,
                 hadamard=True, fp8=True, return_bf16=True, layout="BSND"):
    """Indexer input producer (dsa_indexer_prep): RoPE, the Hadamard ``rotate_activation`` and
    the fp8-e4m3 per-row quantisation of query / key rows in one HIP pass.

    x bf16: "BSND" [B,S,H,128] (queries) or [B,S,128] (keys); "TND" [T,H,128] or [T,128].
    The RoPE position of token row r is ``positions`` (int [B,S] or [T]) or
    ``pos_offset + s`` (BSND) / ``pos_offset + t`` (TND);
    ``freqs_cis`` [n_pos, rope_dim/2] complex (or its real view) is the reference's rope
    cache, None skips the RoPE.  V3.2 (models/deepseek_v32/model.py:264-282): rope_start 0,
    interleaved False; V4 (models/deepseek_v4/model.py:343-357): rope_start 64, interleaved
    True.  Returns (y bf16 like x or None, q8 float8_e4m3fn like x or None, scale fp32
    x.shape[:-1] or None).
    """
    lib = load_library()
    require_gpu_tensor(x, "x")
    if x.dtype != torch.bfloat16:
        raise ValueError("indexer_prep takes bf16 rows (the model dtype)")
    if x.shape[-1] != 128:
        raise ValueError(f"indexer_prep takes 128-feature rows (got {x.shape[-1]})")
    x = x.contiguous()
    if layout == "BSND" and x.dim() in (3, 4):
        B, S = x.shape[:2]
        rows, H, seq_len = B * S, (x.shape[2] if x.dim() == 4 else 1), S
    elif layout == "TND" and x.dim() in (2, 3):
        rows, H = x.shape[0], (x.shape[1] if x.dim() == 3 else 1)
        seq_len = max(rows, 1)
    else:
        raise ValueError(f"indexer_prep: shape {tuple(x.shape)} does not fit layout {layout}")
    cs, n_pos, rd = _rope_args(freqs_cis, rope_dim, x.device)
    pos = None
    if positions is not None and rd:
        pos = positions.reshape(-1).to(device=x.device, dtype=torch.int32).contiguous()
        if pos.numel() != rows:
            raise ValueError(f"positions has {pos.numel()} entries for {rows} rows")
    y = torch.empty_like(x) if return_bf16 else None
    q8 = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device) if fp8 else None
    sc = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device) if fp8 else None
    if rows:
        check(lib.dsa_indexer_prep(ptr(x), ptr(y), ptr(q8), ptr(sc), rows, H, 128, seq_len, ptr(cs), n_pos, ptr(pos),
                                   int(pos_offset), rd, int(rope_start), int(bool(interleaved)), int(bool(hadamard)),
                                   stream_of(x.device)), "dsa_indexer_prep")
    return y, q8, sc


def compressor_pool(kv, score, ape, ratio, *, overlap=None, norm_weight=None, norm_eps=1e-6, out_dtype=None,
                    freqs_cis=None, rope_dim=64, positions=None):
    """Softmax-gated pooling of ``ratio``-token blocks (dsa_compressor_fwd).

    kv, score [B,S,coff*D] fp32 (the wkv / wgate projections; coff = 2 with overlap, which
    defaults to ``ratio == 4`` as in the reference), ape [ratio, coff*D] fp32.  Returns
    [B,S/ratio,D]: the pooled fp32 rows, or with ``norm_weight`` the RMSNorm of the
    bf16-rounded pooled rows times the weight, in ``out_dtype`` (default bf16).  With
    ``freqs_cis`` the last ``rope_dim`` features are rotated (interleaved pairs) at each
    block's first-token position, ``positions`` [B,S] or c*ratio
    (Compressor._forward_bsnd, models/deepseek_v4/model.py:218-220).
    """
    lib = load_library()
    require_gpu_tensor(kv, "kv")
    if overlap is None:
        overlap = ratio == 4
    B, S, CD = kv.shape
    coff = 2 if overlap else 1
    D = CD // coff
    if out_dtype is None:
        out_dtype = torch.bfloat16 if norm_weight is not None else torch.float32
    kv = kv.float().contiguous()
    score = score.float().contiguous()
    ape = ape.float().contiguous()
    nw = None if norm_weight is None else norm_weight.float().contiguous()
    out = torch.empty(B, S // ratio, D, dtype=out_dtype, device=kv.device)
    cs, n_pos, rd = _rope_args(freqs_cis, rope_dim, kv.device)
    pos = None
    if cs is not None and positions is not None:
        pos = positions.reshape(-1).to(device=kv.device, dtype=torch.int32).contiguous()
        if pos.numel() != B * S:
            raise ValueError(f"positions has {pos.numel()} entries for {B * S} tokens")
    check(
        lib.dsa_compressor_fwd(ptr(kv), ptr(score), ptr(ape), ptr(nw), ptr(out), _lib.dtype_code(out_dtype), B, S, D,
                               int(ratio), int(bool(overlap)), float(norm_eps), ptr(cs), n_pos, rd, ptr(pos),
                               stream_of(kv.device)),
        "dsa_compressor_fwd",
    )
    return out


def compressor_pool_tnd(kv, score, ape, ratio, block_starts, positions=None, *, overlap=None, norm_weight=None,
                        norm_eps=1e-6, out_dtype=None, freqs_cis=None, rope_dim=64):
    """Softmax-gated pooling over a packed varlen batch (dsa_compressor_fwd_tnd;
    reference Compressor._forward_tnd, models/deepseek_v4/model.py:223-274).

    kv, score [T,coff*D] fp32; block_starts [n_blocks] (tnd.compressed_block_starts); with
    overlap, positions [T] (request-local) decide which blocks take the previous block's
    first half.  Returns [n_blocks,D] like ``compressor_pool``; with ``freqs_cis`` the last
    ``rope_dim`` features of block c are rotated at positions[block_starts[c]]
    (models/deepseek_v4/model.py:266-273).
    """
    lib = load_library()
    require_gpu_tensor(kv, "kv")
    if overlap is None:
        overlap = ratio == 4
    T, CD = kv.shape[-2], kv.shape[-1]
    coff = 2 if overlap else 1
    D = CD // coff
    if out_dtype is None:
        out_dtype = torch.bfloat16 if norm_weight is not None else torch.float32
    kv = kv.reshape(T, CD).float().contiguous()
    score = score.reshape(T, CD).float().contiguous()
    ape = ape.float().contiguous()
    nw = None if norm_weight is None else norm_weight.float().contiguous()
    bs = block_starts.to(device=kv.device, dtype=torch.int64).contiguous()
    pos = None
    cs, n_pos, rd = _rope_args(freqs_cis, rope_dim, kv.device)
    if overlap or cs is not None:
        if positions is None:
            raise ValueError("overlap pooling and the RoPE epilogue need the token positions")
        pos = positions.reshape(-1).to(device=kv.device, dtype=torch.int32).contiguous()
        if pos.numel() != T:
            raise ValueError(f"positions has {pos.numel()} entries for {T} tokens")
    out = torch.empty(bs.numel(), D, dtype=out_dtype, device=kv.device)
    check(
        lib.dsa_compressor_fwd_tnd(ptr(kv), ptr(score), ptr(ape), ptr(nw), ptr(out), _lib.dtype_code(out_dtype), T, D,
                                   int(ratio), int(bool(overlap)), ptr(bs), bs.numel(), ptr(pos), float(norm_eps),
                                   ptr(cs), n_pos, rd, stream_of(kv.device)),
        "dsa_compressor_fwd_tnd",
    )
    return out


# ---------------------------------------------------------------------------
# MLA weight absorption around the absorbed attention
# ---------------------------------------------------------------------------
def _rows_view(x):
    """``x`` [..., H, D] with a unit last stride and its (token, head) rows at a fixed stride
    ``ld`` (token stride H * ld), as the absorb kernel addresses them; copies otherwise.
    Returns (x, ld)."""
    H, D = x.shape[-2], x.shape[-1]
    ld = x.stride(-2)
    ok = x.stride(-1) == 1 and ld >= D and ld % 8 == 0 and x.data_ptr() % 16 == 0
    expected = H * ld
    for i in range(x.dim() - 3, -1, -1):
        if x.shape[i] != 1 and x.stride(i) != expected:
            ok = False
        expected *= x.shape[i]
    if not ok:
        x = x.contiguous()
        ld = D
    return x, ld


def mla_absorb(a, wt, *, append=None):
    """c[t, h, :N] = a[t, h, :K] . wt[h]^T, c[t, h, N:] = append[t, h] (dsa_mla_absorb).

    a [..., H, K] bf16 (rows may be a strided view, e.g. the first 512 columns of a 576-wide
    gradient), wt [H, N, K] bf16, append [..., H, E] or None; (K, N) = (128, 512) or
    (512, 128).  Returns c [..., H, N + E] bf16, contiguous."""
    lib = load_library()
    require_gpu_tensor(a, "a")
    a, lda = _rows_view(a.to(torch.bfloat16))
    H, K = a.shape[-2], a.shape[-1]
    N = wt.shape[1]
    if wt.shape != (H, N, K):
        raise ValueError(f"weight {tuple(wt.shape)} does not fit rows [.., {H}, {K}]")
    lead = a.shape[:-2]
    tokens = math.prod(lead)
    wt = wt.to(torch.bfloat16).contiguous()
    E, lde = 0, 0
    if append is not None:
        append, lde = _rows_view(append.to(torch.bfloat16))
        E = append.shape[-1]
    out = torch.empty(*lead, H, N + E, dtype=torch.bfloat16, device=a.device)
    check(lib.dsa_mla_absorb(ptr(a), lda, ptr(wt), ptr(out), N + E, ptr(append), lde, E, tokens, H, K, N,
                             stream_of(a.device)), "dsa_mla_absorb")
    return out


class _AbsorbQ(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q_nope, q_pe, w_uk):
        wt = w_uk.transpose(1, 2).contiguous()  # [H, 512, 128]
        q = mla_absorb(q_nope, wt, append=q_pe)
        ctx.save_for_backward(q_nope, w_uk)
        ctx.rope = q_pe.shape[-1]
        return q

    @staticmethod
    def backward(ctx, dq):
        q_nope, w_uk = ctx.saved_tensors
        R = w_uk.shape[-1]
        dq = dq.to(torch.bfloat16)
        d_nope = mla_absorb(dq[..., :R], w_uk.to(torch.bfloat16).contiguous())  # [.., H, 128]
        # d w_uk[h] = sum_t q_nope[t, h]^T dq[t, h, :R]: a plain batched GEMM (hipBLASLt)
        H = q_nope.shape[-2]
        qn = q_nope.reshape(-1, H, q_nope.shape[-1]).permute(1, 2, 0).contiguous().float()
        dqa = dq[..., :R].reshape(-1, H, R).transpose(0, 1).contiguous().float()
        d_w = torch.bmm(qn, dqa).to(w_uk.dtype)
        return d_nope.to(q_nope.dtype), dq[..., R:].to(q_nope.dtype), d_w


class _AbsorbOut(torch.autograd.Function):
    @staticmethod
    def forward(ctx, out, w_uv_t):
        wt = w_uv_t.transpose(1, 2).contiguous()  # [H, 128, 512]
        y = mla_absorb(out, wt)
        ctx.save_for_backward(out, w_uv_t)
        return y

    @staticmethod
    def backward(ctx, dy):
        out, w_uv_t = ctx.saved_tensors
        dy = dy.to(torch.bfloat16)
        d_out = mla_absorb(dy, w_uv_t.to(torch.bfloat16).contiguous())  # [.., H, 512]
        H = out.shape[-2]
        o = out.reshape(-1, H, out.shape[-1]).permute(1, 2, 0).contiguous().float()
        g = dy.reshape(-1, H, dy.shape[-1]).transpose(0, 1).contiguous().float()
        d_w = torch.bmm(o, g).to(w_uv_t.dtype)
        return d_out.to(out.dtype), d_w


def mla_absorb_q(q_nope, q_pe, w_uk):
    """The absorbed query of MLA (reference PreAttention, models/deepseek_v32/model.py:520-535):
    ``cat([einsum("bshq,hqr->bshr", q_nope, w_uk), q_pe], -1)`` in one kernel.
    q_nope [B,S,H,128], q_pe [B,S,H,64], w_uk [H,128,512] bf16 -> q [B,S,H,576];
    differentiable in all three (the weight gradient is a batched GEMM)."""
    return _AbsorbQ.apply(q_nope, q_pe, w_uk)


def mla_absorb_out(out, w_uv_t):
    """The output projection of absorbed MLA (reference PostAttention,
    models/deepseek_v32/model.py:574-575): ``einsum("bshr,hrv->bshv", out, w_uv_t)`` on the
    BSND attention output [B,S,H,512] with w_uv_t [H,512,128] -> [B,S,H,128] (contiguous,
    so .view(B, S, H*128) feeds wo); differentiable in both."""
    return _AbsorbOut.apply(out, w_uv_t)


def default_softmax_scale(d_qk: int) -> float:
    return 1.0 / math.sqrt(d_qk)
