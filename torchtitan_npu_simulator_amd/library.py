"""The DSA ops as ``torch.library`` custom ops (namespace ``dsa_mi355x``).

Each op wraps the same-named function of ``torch_npu_ops`` (and so the HIP library) and
carries a fake implementation that only computes output shapes and dtypes, so
``torch.compile`` / FakeTensor / meta tracing can pass through the attention path as
opaque nodes instead of excluding it from compilation (the reference leaves
``inner_attention`` out of compile, models/deepseek_v32/parallelize.py:606-609).  The
attention ops register their backward through ``register_autograd``.

Signatures follow the reference bindings (paths relative to the reference repository):

* ``npu_lightning_indexer``        ops/aclnn/lightning_indexer/binding.cpp:12-36
* ``npu_sparse_flash_attention``   converters/kernels/dsa.py:238-253 (absorb mode, BSND)
  and its ``_grad``
* ``npu_sparse_lightning_indexer_grad_kl_loss``
                                   ops/aclnn/sparse_lightning_indexer_grad_kl_loss/binding.cpp:12-36
* ``npu_sparse_attn_sharedkv_metadata`` / ``npu_sparse_attn_sharedkv`` / ``_grad``
                                   ops/aclnn/sparse_attn_sharedkv/binding.cpp:12-88

Custom ops cannot return ``None``: where a binding returns an undefined tensor (values
without ``return_value``, the LSE without ``return_softmax_lse``, d_cmp_kv without
compressed keys) these return an empty tensor.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch
from torch.library import custom_op

from . import torch_npu_ops as _ops

_NS = "dsa_mi355x"
_I64_MAX = (1 << 63) - 1


def _empty(like: torch.Tensor, dtype=None) -> torch.Tensor:
    return like.new_empty(0, dtype=dtype or like.dtype)


def _own(t: torch.Tensor) -> torch.Tensor:
    """A custom op's output may not be a view: copy slices of larger results."""
    return t.clone() if t._base is not None else t


# ---------------------------------------------------------------------------
# lightning indexer + top-k
# ---------------------------------------------------------------------------
@custom_op(f"{_NS}::npu_lightning_indexer", mutates_args=())
def npu_lightning_indexer(query: torch.Tensor, key: torch.Tensor, weights: torch.Tensor,
                          actual_seq_lengths_query: Optional[torch.Tensor] = None,
                          actual_seq_lengths_key: Optional[torch.Tensor] = None,
                          block_table: Optional[torch.Tensor] = None, layout_query: str = "BSND",
                          layout_key: str = "BSND", sparse_count: int = 2048, sparse_mode: int = 3,
                          pre_tokens: int = _I64_MAX, next_tokens: int = _I64_MAX, cmp_ratio: int = 1,
                          return_value: bool = False, query_scale: Optional[torch.Tensor] = None,
                          key_scale: Optional[torch.Tensor] = None) -> tuple[torch.Tensor, torch.Tensor]:
    idx, vals = _ops.npu_lightning_indexer(query, key, weights, actual_seq_lengths_query, actual_seq_lengths_key,
                                           block_table, layout_query, layout_key, sparse_count, sparse_mode,
                                           pre_tokens, next_tokens, cmp_ratio, return_value, query_scale=query_scale,
                                           key_scale=key_scale)
    return _own(idx), (_own(vals) if vals is not None else _empty(query, _ops._values_dtype(query)))


@npu_lightning_indexer.register_fake
def _(query, key, weights, actual_seq_lengths_query=None, actual_seq_lengths_key=None, block_table=None,
      layout_query="BSND", layout_key="BSND", sparse_count=2048, sparse_mode=3, pre_tokens=_I64_MAX,
      next_tokens=_I64_MAX, cmp_ratio=1, return_value=False, query_scale=None, key_scale=None):
    lead = (query.shape[0],) if layout_query == "TND" else (query.shape[0], query.shape[1])
    shape = (*lead, 1, sparse_count)
    idx = query.new_empty(shape, dtype=torch.int32)
    vdt = _ops._values_dtype(query)
    vals = query.new_empty(shape, dtype=vdt) if return_value else _empty(query, vdt)
    return idx, vals


# ---------------------------------------------------------------------------
# gathered sparse MLA attention (absorb mode, BSND)
# ---------------------------------------------------------------------------
@custom_op(f"{_NS}::npu_sparse_flash_attention", mutates_args=())
def npu_sparse_flash_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                               sparse_indices: torch.Tensor, query_rope: torch.Tensor, key_rope: torch.Tensor,
                               scale_value: float = 1.0, sparse_mode: int = 3
                               ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    q = _ops._cat_last(query, query_rope)
    kv = _ops._cat_last(key, key_rope)
    kv3 = kv.reshape(kv.shape[0], kv.shape[1], kv.shape[-1])
    q_off = _ops._resolve_q_offset(sparse_mode, query.shape[1], key.shape[1], None)
    idx = sparse_indices.reshape(query.shape[0], query.shape[1], -1)
    return _ops.sparse_mla_fwd(q, kv3, idx, float(scale_value), d_v=query.shape[-1], q_offset=q_off)


@npu_sparse_flash_attention.register_fake
def _(query, key, value, sparse_indices, query_rope, key_rope, scale_value=1.0, sparse_mode=3):
    B, S, H, dv = query.shape
    return (query.new_empty(B, S, H, dv), query.new_empty(B, S, H, dtype=torch.float32),
            query.new_empty(B, S, H, dtype=torch.float32))


@custom_op(f"{_NS}::npu_sparse_flash_attention_grad", mutates_args=())
def npu_sparse_flash_attention_grad(query: torch.Tensor, key: torch.Tensor, query_rope: torch.Tensor,
                                    key_rope: torch.Tensor, sparse_indices: torch.Tensor, out: torch.Tensor,
                                    d_out: torch.Tensor, softmax_max: torch.Tensor, softmax_sum: torch.Tensor,
                                    scale_value: float = 1.0, sparse_mode: int = 3
                                    ) -> tuple[torch.Tensor, torch.Tensor]:
    """(dq [B,S,H,D_qk] like query, dkv fp32 [B,S_kv,D_qk]): latent columns first, then rope."""
    q = _ops._cat_last(query, query_rope)
    kv = _ops._cat_last(key, key_rope)
    kv3 = kv.reshape(kv.shape[0], kv.shape[1], kv.shape[-1])
    q_off = _ops._resolve_q_offset(sparse_mode, query.shape[1], key.shape[1], None)
    idx = sparse_indices.reshape(query.shape[0], query.shape[1], -1)
    return _ops.sparse_mla_bwd(q, kv3, idx, out, d_out.contiguous(), softmax_max, softmax_sum, float(scale_value),
                               q_offset=q_off)


@npu_sparse_flash_attention_grad.register_fake
def _(query, key, query_rope, key_rope, sparse_indices, out, d_out, softmax_max, softmax_sum, scale_value=1.0,
      sparse_mode=3):
    B, S, H, dn = query.shape
    d = dn + query_rope.shape[-1]
    return query.new_empty(B, S, H, d), query.new_empty(B, key.shape[1], d, dtype=torch.float32)


def _sfa_setup(ctx, inputs, output):
    query, key, value, sparse_indices, query_rope, key_rope, scale_value, sparse_mode = inputs
    out, smax, ssum = output
    ctx.save_for_backward(query, key, query_rope, key_rope, sparse_indices, out, smax, ssum)
    ctx.scale_value = scale_value
    ctx.sparse_mode = sparse_mode
    ctx.key_shape = key.shape
    ctx.key_dtype = key.dtype


def _sfa_backward(ctx, d_out, _d_max, _d_sum):
    query, key, query_rope, key_rope, sparse_indices, out, smax, ssum = ctx.saved_tensors
    dq, dkv = npu_sparse_flash_attention_grad(query, key, query_rope, key_rope, sparse_indices, out, d_out, smax,
                                              ssum, ctx.scale_value, ctx.sparse_mode)
    dn = query.shape[-1]
    dkv = dkv.to(ctx.key_dtype)
    k_shape = ctx.key_shape
    d_key = dkv[..., :dn].reshape(k_shape)
    d_key_rope = dkv[..., dn:].reshape(*k_shape[:-1], dkv.shape[-1] - dn)
    # absorb mode: the value is the key's latent part; its gradient is inside d_key
    return dq[..., :dn], d_key, None, None, dq[..., dn:], d_key_rope, None, None


npu_sparse_flash_attention.register_autograd(_sfa_backward, setup_context=_sfa_setup)


# ---------------------------------------------------------------------------
# indexer KL loss + gradients
# ---------------------------------------------------------------------------
@custom_op(f"{_NS}::npu_sparse_lightning_indexer_grad_kl_loss", mutates_args=())
def npu_sparse_lightning_indexer_grad_kl_loss(
        query: torch.Tensor, key: torch.Tensor, query_index: torch.Tensor, key_index: torch.Tensor,
        weight: torch.Tensor, sparse_indices: torch.Tensor, softmax_max: Optional[torch.Tensor],
        softmax_sum: Optional[torch.Tensor], query_rope: Optional[torch.Tensor] = None,
        key_rope: Optional[torch.Tensor] = None, actual_seq_qlen: Optional[Sequence[int]] = None,
        actual_seq_klen: Optional[Sequence[int]] = None, layout: str = "BSND", sparse_mode: int = 3,
        pre_tokens: int = 65536, next_tokens: int = 65536, cmp_ratio: int = 1, scale_value: float = 1.0,
        deterministic: bool = False) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    res = _ops.npu_sparse_lightning_indexer_grad_kl_loss(
        query, key, query_index, key_index, weight, sparse_indices, softmax_max, softmax_sum, scale_value,
        query_rope=query_rope, key_rope=key_rope, actual_seq_qlen=actual_seq_qlen, actual_seq_klen=actual_seq_klen,
        layout=layout, sparse_mode=sparse_mode, pre_tokens=pre_tokens, next_tokens=next_tokens,
        deterministic=deterministic, cmp_ratio=cmp_ratio)
    return tuple(_own(t) for t in res)


@npu_sparse_lightning_indexer_grad_kl_loss.register_fake
def _(query, key, query_index, key_index, weight, sparse_indices, softmax_max, softmax_sum, query_rope=None,
      key_rope=None, actual_seq_qlen=None, actual_seq_klen=None, layout="BSND", sparse_mode=3, pre_tokens=65536,
      next_tokens=65536, cmp_ratio=1, scale_value=1.0, deterministic=False):
    return (torch.empty_like(query_index), torch.empty_like(key_index), torch.empty_like(weight),
            query.new_empty(1, dtype=torch.float32))


# ---------------------------------------------------------------------------
# DeepSeek-V4 shared-KV attention (window + compressed KV + sink)
# ---------------------------------------------------------------------------
@custom_op(f"{_NS}::npu_sparse_attn_sharedkv_metadata", mutates_args=())
def npu_sparse_attn_sharedkv_metadata(
        cu_seqlens_q: Optional[torch.Tensor], seqused_ori_kv: Optional[torch.Tensor],
        seqused_cmp_kv: Optional[torch.Tensor], seqused_q: Optional[torch.Tensor],
        seqused_kv: Optional[torch.Tensor], num_heads_q: int, num_heads_kv: int, head_dim: int, batch_size: int,
        max_seqlen_q: int, max_seqlen_kv: int, ori_topk: int, cmp_topk: int, cmp_ratio: int, ori_mask_mode: int,
        cmp_mask_mode: int, ori_win_left: int, ori_win_right: int, layout_q: str, layout_kv: str, has_ori_kv: bool,
        has_cmp_kv: bool, device: torch.device) -> torch.Tensor:
    return _ops.npu_sparse_attn_sharedkv_metadata(
        cu_seqlens_q, seqused_ori_kv, seqused_cmp_kv, seqused_q, seqused_kv, num_heads_q, num_heads_kv, head_dim,
        batch_size, max_seqlen_q, max_seqlen_kv, ori_topk, cmp_topk, cmp_ratio, ori_mask_mode, cmp_mask_mode,
        ori_win_left, ori_win_right, layout_q, layout_kv, has_ori_kv, has_cmp_kv, device=device)


@npu_sparse_attn_sharedkv_metadata.register_fake
def _(cu_seqlens_q, seqused_ori_kv, seqused_cmp_kv, seqused_q, seqused_kv, num_heads_q, num_heads_kv, head_dim,
      batch_size, max_seqlen_q, max_seqlen_kv, ori_topk, cmp_topk, cmp_ratio, ori_mask_mode, cmp_mask_mode,
      ori_win_left, ori_win_right, layout_q, layout_kv, has_ori_kv, has_cmp_kv, device):
    return torch.empty(1024, dtype=torch.int32, device=device)


@custom_op(f"{_NS}::npu_sparse_attn_sharedkv", mutates_args=())
def npu_sparse_attn_sharedkv(query: torch.Tensor, ori_kv: torch.Tensor, cmp_kv: Optional[torch.Tensor],
                             cmp_sparse_indices: Optional[torch.Tensor], sinks: torch.Tensor,
                             metadata: Optional[torch.Tensor], softmax_scale: float, cmp_ratio: int,
                             ori_mask_mode: int = 4, cmp_mask_mode: int = 3, ori_win_left: int = 127,
                             ori_win_right: int = 0, layout_q: str = "BSND", layout_kv: str = "BSND",
                             return_softmax_lse: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    out, lse = _ops.npu_sparse_attn_sharedkv(
        query, ori_kv, cmp_kv, None, cmp_sparse_indices, sinks=sinks, metadata=metadata, softmax_scale=softmax_scale,
        cmp_ratio=cmp_ratio, ori_mask_mode=ori_mask_mode, cmp_mask_mode=cmp_mask_mode, ori_win_left=ori_win_left,
        ori_win_right=ori_win_right, layout_q=layout_q, layout_kv=layout_kv, return_softmax_lse=return_softmax_lse)
    return _own(out), (_own(lse) if lse is not None else _empty(query, torch.float32))


@npu_sparse_attn_sharedkv.register_fake
def _(query, ori_kv, cmp_kv, cmp_sparse_indices, sinks, metadata, softmax_scale, cmp_ratio, ori_mask_mode=4,
      cmp_mask_mode=3, ori_win_left=127, ori_win_right=0, layout_q="BSND", layout_kv="BSND",
      return_softmax_lse=True):
    lse = query.new_empty(*query.shape[:-1], 1, dtype=torch.float32) if return_softmax_lse else \
        _empty(query, torch.float32)
    return torch.empty_like(query), lse


@custom_op(f"{_NS}::npu_sparse_attn_sharedkv_grad", mutates_args=())
def npu_sparse_attn_sharedkv_grad(query: torch.Tensor, ori_kv: torch.Tensor, cmp_kv: Optional[torch.Tensor],
                                  d_out: torch.Tensor, out: torch.Tensor, lse: torch.Tensor,
                                  cmp_sparse_indices: Optional[torch.Tensor], sinks: torch.Tensor,
                                  scale_value: float, cmp_ratio: int, ori_mask_mode: int = 4,
                                  cmp_mask_mode: int = 3, ori_win_left: int = 127, ori_win_right: int = 0,
                                  layout: str = "BSND"
                                  ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    dq, d_ori, d_cmp, dsink = _ops.npu_sparse_attn_sharedkv_grad(
        query, ori_kv, cmp_kv, d_out, out, lse, None, cmp_sparse_indices, sinks=sinks, scale_value=scale_value,
        cmp_ratio=cmp_ratio, ori_mask_mode=ori_mask_mode, cmp_mask_mode=cmp_mask_mode, ori_win_left=ori_win_left,
        ori_win_right=ori_win_right, layout=layout)
    return _own(dq), _own(d_ori), (_own(d_cmp) if d_cmp is not None else _empty(ori_kv)), _own(dsink)


@npu_sparse_attn_sharedkv_grad.register_fake
def _(query, ori_kv, cmp_kv, d_out, out, lse, cmp_sparse_indices, sinks, scale_value, cmp_ratio, ori_mask_mode=4,
      cmp_mask_mode=3, ori_win_left=127, ori_win_right=0, layout="BSND"):
    d_cmp = torch.empty_like(cmp_kv) if (cmp_kv is not None and cmp_ratio > 1) else _empty(ori_kv)
    return torch.empty_like(query), torch.empty_like(ori_kv), d_cmp, torch.empty_like(sinks)


def _sas_setup(ctx, inputs, output):
    (query, ori_kv, cmp_kv, cmp_sparse_indices, sinks, metadata, softmax_scale, cmp_ratio, ori_mask_mode,
     cmp_mask_mode, ori_win_left, ori_win_right, layout_q, layout_kv, return_softmax_lse) = inputs
    out, lse = output
    if not return_softmax_lse:
        raise RuntimeError("npu_sparse_attn_sharedkv needs return_softmax_lse=True for its backward")
    ctx.save_for_backward(query, ori_kv, cmp_kv, cmp_sparse_indices, sinks, out, lse)
    ctx.args = (softmax_scale, cmp_ratio, ori_mask_mode, cmp_mask_mode, ori_win_left, ori_win_right, layout_q)
    ctx.has_cmp = cmp_kv is not None and cmp_ratio > 1


def _sas_backward(ctx, d_out, _d_lse):
    query, ori_kv, cmp_kv, cmp_sparse_indices, sinks, out, lse = ctx.saved_tensors
    dq, d_ori, d_cmp, dsink = npu_sparse_attn_sharedkv_grad(query, ori_kv, cmp_kv, d_out, out, lse,
                                                            cmp_sparse_indices, sinks, *ctx.args)
    return (dq, d_ori, d_cmp if ctx.has_cmp else None, None, dsink, *([None] * 10))


npu_sparse_attn_sharedkv.register_autograd(_sas_backward, setup_context=_sas_setup)

__all__ = [
    "npu_lightning_indexer",
    "npu_sparse_flash_attention",
    "npu_sparse_flash_attention_grad",
    "npu_sparse_lightning_indexer_grad_kl_loss",
    "npu_sparse_attn_sharedkv_metadata",
    "npu_sparse_attn_sharedkv",
    "npu_sparse_attn_sharedkv_grad",
]
