"""MI355X implementations of the torch_npu DSA ops the reference calls.

Same names, argument meanings and return conventions as the ``torch_npu`` calls in the
reference's ``converters/kernels/dsa.py`` (paths relative to the reference repository):

* ``npu_lightning_indexer``            dsa.py:217-226, binding ops/aclnn/lightning_indexer/binding.cpp:12-36
* ``npu_sparse_flash_attention``       dsa.py:238-253 (attention_mode=2, MLA absorb)
* ``npu_sparse_lightning_indexer_grad_kl_loss``  dsa.py:159-177,
                                       binding ops/aclnn/sparse_lightning_indexer_grad_kl_loss/binding.cpp:12-36

Every op runs on the HIP library (``libdsa_mi355x.so``) on the tensors' GPU and raises
if the library or a GPU is missing; nothing here computes on the CPU.

Layout "BSND" throughout.  ``sparse_mode`` 3 is the causal rule aligned bottom-right
(query row s may see key t <= s + (S_k - S_q)); 0 means no causal mask.  An explicit
``q_offset`` overrides it (one GPU's context-parallel share sees Q rows starting at
``q_offset`` against the KV prefix).
"""

from __future__ import annotations

import math

import torch

from . import _lib
from ._lib import check, load_library, ptr, require_gpu_tensor, stream_of

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


# ---------------------------------------------------------------------------
# lightning indexer + top-k
# ---------------------------------------------------------------------------
def quantize_fp8_per_row(x: torch.Tensor):
    """OCP fp8-e4m3fn with one fp32 scale (amax/448) per row of the last dim."""
    xf = x.float()
    scale = (xf.abs().amax(dim=-1) / 448.0).clamp_min(1e-12)
    return (xf / scale.unsqueeze(-1)).to(torch.float8_e4m3fn), scale


def indexer_scores(q_idx, k_idx, weights, *, q_scale=None, k_scale=None, q_offset=0, cmp_ratio=1, out=None):
    """fp32 index scores [B,S,S_k] (-inf where invalid) from dsa_indexer_fwd."""
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
    check(
        lib.dsa_indexer_fwd(ptr(q_idx), ptr(qs), ptr(k_idx), ptr(ks), ptr(w), ptr(out), _lib.dtype_code(q_idx.dtype),
                            B, S, s_k, H, D, out.stride(1), int(q_offset), int(cmp_ratio),
                            stream_of(q_idx.device)),
        "dsa_indexer_fwd",
    )
    return out


def topk_select(scores, k, *, q_offset=0, cmp_ratio=1, index_offset=0, return_values=False):
    """int32 [B,S,k] top-k indices (ascending index order, -1 padded) of fp32 scores."""
    lib = load_library()
    require_gpu_tensor(scores, "scores")
    B, S, s_k = scores.shape
    if scores.stride(2) != 1:
        scores = scores.contiguous()
    idx = torch.empty(B, S, k, dtype=torch.int32, device=scores.device)
    vals = torch.empty(B, S, k, dtype=torch.float32, device=scores.device) if return_values else None
    check(
        lib.dsa_topk(ptr(scores), ptr(idx), ptr(vals), B, S, s_k, scores.stride(1), k, int(q_offset), int(cmp_ratio),
                     int(index_offset), stream_of(scores.device)),
        "dsa_topk",
    )
    return idx, vals


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
):
    """Fused lightning indexer + per-query top-k.

    query [B,S,H_I,D_I], key [B,S_k,1,D_I] (or [B,S_k,D_I]), weights [B,S,H_I]; bf16, or
    fp8-e4m3fn with ``query_scale`` [B,S,H_I] / ``key_scale`` [B,S_k] (this build's
    extension for the fp8 indexer).  Returns (sparse_indices int32 [B,S,1,K],
    sparse_values fp32 [B,S,1,K] or None): the chosen key indices in ascending order with
    -1 padding (reference binding shape: lightning_indexer/binding.cpp:28).  Rows are
    processed in chunks so the fp32 score buffer stays under 1 GiB.
    """
    if layout_query != "BSND" or layout_key != "BSND":
        raise NotImplementedError("only the BSND layout is supported")
    if block_table is not None or actual_seq_lengths_query is not None or actual_seq_lengths_key is not None:
        raise NotImplementedError("paged / varlen indexer inputs are not supported by this op (use dsa.varlen)")
    k3 = key.squeeze(2) if key.dim() == 4 else key
    B, S, H, D = query.shape
    s_k = k3.shape[1]
    q_off = _resolve_q_offset(sparse_mode, S, s_k * cmp_ratio, q_offset)
    K = int(sparse_count)
    idx = torch.empty(B, S, K, dtype=torch.int32, device=query.device)
    vals = torch.empty(B, S, K, dtype=torch.float32, device=query.device) if return_value else None
    rows = max(1, min(S, _SCORE_BUDGET_BYTES // max(1, 4 * s_k * B)))
    buf = torch.empty(B, rows, s_k, dtype=torch.float32, device=query.device)
    for r0 in range(0, S, rows):
        r1 = min(S, r0 + rows)
        sc = buf[:, : r1 - r0]
        for b in range(B):
            qs = None if query_scale is None else query_scale[b : b + 1, r0:r1]
            ks = None if key_scale is None else key_scale[b : b + 1]
            indexer_scores(query[b : b + 1, r0:r1], k3[b : b + 1], weights[b : b + 1, r0:r1], q_scale=qs,
                           k_scale=ks, q_offset=q_off + r0, cmp_ratio=cmp_ratio, out=sc[b : b + 1])
            i_b, v_b = topk_select(sc[b : b + 1], K, q_offset=q_off + r0, cmp_ratio=cmp_ratio,
                                   index_offset=index_offset, return_values=return_value)
            idx[b, r0:r1] = i_b[0]
            if return_value:
                vals[b, r0:r1] = v_b[0]
    return idx.unsqueeze(2), (vals.unsqueeze(2) if return_value else None)


# ---------------------------------------------------------------------------
# gathered sparse MLA attention
# ---------------------------------------------------------------------------
def sparse_mla_fwd(q, kv, indices, scale, *, d_v=512, q_offset=0):
    """(out [B,S,H,d_v], softmax_max [B,S,H], softmax_sum [B,S,H]) from dsa_sparse_mla_fwd.

    q [B,S,H,D_qk] bf16/fp32, kv [B,S_kv,D_qk] (v = kv[..., :d_v]), indices [B,S,K] int32.
    """
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
    check(
        lib.dsa_sparse_mla_fwd(ptr(q), ptr(kv), ptr(indices), ptr(out), ptr(smax), ptr(ssum), _lib.dtype_code(q.dtype),
                               B, S, s_kv, H, D, d_v, K, float(scale), int(q_offset), stream_of(q.device)),
        "dsa_sparse_mla_fwd",
    )
    return out, smax, ssum


def sparse_mla_bwd(q, kv, indices, out, dout, smax, ssum, scale, *, q_offset=0, workspace_bytes=None,
                   return_mass=False):
    """(dq like q, dkv fp32 [B,S_kv,D_qk]) from dsa_sparse_mla_bwd, plus the head-summed
    attention mass [B,S,K] fp32 when ``return_mass`` (bf16 path; the same quantity as
    ``attn_mass``, taken from the probabilities the backward recomputes anyway).

    ``workspace_bytes`` caps the scratch (fewer bytes -> more query-row chunks).
    """
    lib = load_library()
    B, S, H, D = q.shape
    s_kv = kv.shape[1]
    K = indices.shape[-1]
    d_v = out.shape[-1]
    q, kv, out, dout = (t.contiguous() for t in (q, kv, out, dout))
    indices = indices.reshape(B, S, K).to(torch.int32).contiguous()
    dq = torch.empty_like(q)
    dkv = torch.zeros(B, s_kv, D, dtype=torch.float32, device=q.device)
    mass = torch.empty(B, S, K, dtype=torch.float32, device=q.device) if return_mass else None
    ws_bytes = int(lib.dsa_sparse_mla_bwd_workspace_size(B, S, s_kv, H, D, K))
    if workspace_bytes is not None:
        ws_bytes = int(workspace_bytes)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    check(
        lib.dsa_sparse_mla_bwd(ptr(q), ptr(kv), ptr(indices), ptr(out), ptr(dout), ptr(smax), ptr(ssum), ptr(dq),
                               ptr(dkv), ptr(mass), ptr(ws), ws_bytes, _lib.dtype_code(q.dtype), B, S, s_kv, H, D, d_v,
                               K, float(scale), int(q_offset), stream_of(q.device)),
        "dsa_sparse_mla_bwd",
    )
    return (dq, dkv, mass) if return_mass else (dq, dkv)


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
    q_offset=None,
):
    """Gathered sparse MLA attention in absorb mode (attention_mode=2).

    query [B,S,H,512] (q_nope), key [B,S_kv,1,512] (k_nope), value (must be k_nope: the
    absorbed latent is both key and value), query_rope [B,S,H,64], key_rope [B,S_kv,1,64],
    sparse_indices [B,S,1,K] int32 (-1 = empty).  Returns (out [B,S,H,512], softmax_max
    [B,S,H], softmax_sum [B,S,H]); differentiable in query/key/query_rope/key_rope, with
    the value gradient folded into the key gradient (dKV_latent = dK_nope + dV).
    """
    if attention_mode != 2:
        raise NotImplementedError("only attention_mode=2 (MLA absorb) is supported")
    if layout_query != "BSND" or layout_kv != "BSND" or block_table is not None or sparse_block_size != 1:
        raise NotImplementedError("BSND, sparse_block_size=1, no block_table")
    if query_rope is None or key_rope is None:
        raise ValueError("query_rope and key_rope are required in absorb mode")
    s_kv = key.shape[1]
    q_off = _resolve_q_offset(sparse_mode, query.shape[1], s_kv, q_offset)
    idx = sparse_indices.reshape(query.shape[0], query.shape[1], -1)
    out, smax, ssum = _SparseFlashAttention.apply(query, key, query_rope, key_rope, idx, float(scale_value), q_off)
    return out, smax, ssum


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
    q_offset=None,
    loss_scale=1.0,
    eps=1e-8,
    grad_scale=1.0,
):
    """(d_query_index fp32, d_key_index fp32, d_weights fp32, loss fp32[1]) of the indexer KL loss.

    The main-attention target mass is recomputed from (query || query_rope, key ||
    key_rope, softmax_max, softmax_sum) at the selected keys; ``loss`` is the token SUM
    (the caller divides by B*S, reference dsa.py:73).
    """
    if actual_seq_qlen is not None or actual_seq_klen is not None or layout != "BSND":
        raise NotImplementedError("BSND without actual_seq_* only")
    lib = load_library()
    q = _cat_last(query, query_rope) if query_rope is not None else query.contiguous()
    kv = _cat_last(key, key_rope) if key_rope is not None else key.contiguous()
    B, S, H, D = q.shape
    kv3 = kv.reshape(B, kv.shape[1], D)
    s_kv = kv3.shape[1]
    q_off = _resolve_q_offset(sparse_mode, S, s_kv, q_offset)
    idx = sparse_indices.reshape(B, S, -1).to(torch.int32).contiguous()
    K = idx.shape[-1]
    mass = attn_mass(q, kv3, idx, softmax_max, softmax_sum, scale_value, q_offset=q_off)
    dq_i, dk_i, dw, loss_rows = indexer_kl_grad_from_mass(query_index, key_index, weight, idx, mass, q_offset=q_off,
                                                          loss_scale=loss_scale, eps=eps, grad_scale=grad_scale)
    return dq_i, dk_i.reshape(key_index.shape), dw, loss_rows.sum().reshape(1)


def indexer_kl_grad_from_mass(query_index, key_index, weight, indices, mass, *, q_offset=0, loss_scale=1.0, eps=1e-8,
                              grad_scale=1.0):
    """(dq_idx fp32, dk_idx fp32 [B,S_k,D_I], dw fp32, loss_rows fp32 [B,S]) given the target mass."""
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
    check(
        lib.dsa_indexer_kl_grad(ptr(qi), ptr(ki), ptr(w), ptr(idx), ptr(mass), ptr(dq_i), ptr(dk_i), ptr(dw),
                                ptr(loss_rows), ptr(ws), ws_bytes, B, S, s_k, HI, DI, K, int(q_offset),
                                float(loss_scale), float(eps), float(grad_scale), stream_of(dev)),
        "dsa_indexer_kl_grad",
    )
    return dq_i, dk_i, dw, loss_rows


# ---------------------------------------------------------------------------
# block KV compressor (V4)
# ---------------------------------------------------------------------------
def compressor_pool(kv, score, ape, ratio, *, overlap=None, norm_weight=None, norm_eps=1e-6, out_dtype=None):
    """Softmax-gated pooling of ``ratio``-token blocks (dsa_compressor_fwd).

    kv, score [B,S,coff*D] fp32 (the wkv / wgate projections; coff = 2 with overlap, which
    defaults to ``ratio == 4`` as in the reference), ape [ratio, coff*D] fp32.  Returns
    [B,S/ratio,D]: the pooled fp32 rows, or with ``norm_weight`` the RMSNorm of the
    bf16-rounded pooled rows times the weight, in ``out_dtype`` (default bf16).
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
    check(
        lib.dsa_compressor_fwd(ptr(kv), ptr(score), ptr(ape), ptr(nw), ptr(out), _lib.dtype_code(out_dtype), B, S, D,
                               int(ratio), int(bool(overlap)), float(norm_eps), stream_of(kv.device)),
        "dsa_compressor_fwd",
    )
    return out


def default_softmax_scale(d_qk: int) -> float:
    return 1.0 / math.sqrt(d_qk)
