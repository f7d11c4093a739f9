"""The packed-sequence ("global TND") DeepSeek-V4 attention ops on the MI355X kernels.

The reference's A5 branch calls these through ``cann_ops_transformer.ops`` (external,
closed; call sites in converters/kernels/npu_smla.py, paths relative to the reference
repository):

* ``sparse_flash_mla_metadata`` / ``sparse_flash_mla``                       :457-479, :672-686
* ``sparse_flash_mla_grad_metadata`` / ``sparse_flash_mla_grad``             :540-568, :689-704
* ``lightning_indexer_metadata`` / ``lightning_indexer``                     :753-769, :789-813
* ``sparse_lightning_indexer_kl_loss_grad_metadata`` /
  ``sparse_lightning_indexer_kl_loss_grad``                                  :584-598, :707-732

Same keyword names and returns as those call sites use.  Every op runs the packed batch
as one [1, T] problem whose slot indices keep each query inside its sequence
(``torch_npu_ops.sharedkv_tnd_indices``): the sliding window over the sequence's own
tokens (ori_mask_mode 4), the compressed rows it may see (cmp_mask_mode 3: row c of the
sequence when c < (p + 1) // cmp_ratio, p the query's position in the sequence), the
top-k of those rows for ratio 4.  The metadata a ``*_metadata`` op returns is an int32
device record of the problem (like ``npu_sparse_attn_sharedkv_metadata``) with the host
values the launches need riding on the tensor, so an op given metadata reads nothing
back from the device.
"""

from __future__ import annotations

from typing import Any

import torch

from . import _lib
from . import torch_npu_ops as npu

__all__ = [
    "sparse_flash_mla_metadata",
    "sparse_flash_mla_grad_metadata",
    "sparse_flash_mla",
    "sparse_flash_mla_grad",
    "lightning_indexer_metadata",
    "lightning_indexer",
    "sparse_lightning_indexer_kl_loss_grad_metadata",
    "sparse_lightning_indexer_kl_loss_grad",
]

_MAGIC = 0x534D4C41  # "SMLA": first word of the record
_LAYOUTS = {"TND": 3, "BSND": 1}


def _record(kind: int, fields: list[int], host: dict[str, Any], device) -> torch.Tensor:
    rec = [_MAGIC, kind] + [int(v) for v in fields]
    meta = torch.zeros(1024, dtype=torch.int32)
    meta[: len(rec)] = torch.tensor(rec, dtype=torch.int32)
    meta = meta.to(device)
    meta._dsa_record = tuple(rec)
    meta._dsa_host = host
    return meta


def _device_of(*tensors) -> torch.device:
    for t in tensors:
        if isinstance(t, torch.Tensor):
            return t.device
    return torch.device("cuda", torch.cuda.current_device())


def _max_len(cu) -> int:
    if cu is None:
        return 0
    v = _lib.host_ints(cu)
    return max([b - a for a, b in zip(v[:-1], v[1:])] or [0])


def _host(metadata) -> dict[str, Any]:
    return getattr(metadata, "_dsa_host", None) or {}


def _check_tnd(layout_q, layout_kv):
    if layout_q != "TND" or layout_kv != "TND":
        raise NotImplementedError(f"layouts {layout_q}/{layout_kv}: these ops take packed TND batches")


def _check_masks(ori_mask_mode, cmp_mask_mode):
    if ori_mask_mode != 4 or cmp_mask_mode != 3:
        raise NotImplementedError("mask modes: band window (4) over ori_kv, causal (3) over cmp_kv")


def sparse_flash_mla_metadata(*, cu_seqlens_q=None, cu_seqlens_ori_kv=None, cu_seqlens_cmp_kv=None,
                              cmp_residual_kv=None, ori_topk_length=None, cmp_topk_length=None, batch_size=1,
                              max_seqlen_q=0, max_seqlen_ori_kv=0, max_seqlen_cmp_kv=0, num_heads_q=1,
                              num_heads_kv=1, head_dim=512, cmp_topk=0, cmp_ratio=1, ori_mask_mode=4, cmp_mask_mode=3,
                              ori_win_left=127, ori_win_right=0, layout_q="TND", layout_kv="TND", has_ori_kv=True,
                              has_cmp_kv=False, ori_topk=None, _kind=1):
    """Record of a packed attention problem (the keywords of the reference's
    ``_sparse_attention_metadata_kwargs``, npu_smla.py:165-189).  ``max_seqlen_cmp_kv`` is
    the slot count of the every-causal-block rule (ratio 128); it is read from
    cu_seqlens_cmp_kv once when not given.  (``_kind``: 1 forward, 2 backward record.)"""
    _check_tnd(layout_q, layout_kv)
    _check_masks(ori_mask_mode, cmp_mask_mode)
    if num_heads_kv != 1:
        raise NotImplementedError(f"num_heads_kv={num_heads_kv}: the shared KV has one head")
    if ori_topk_length is not None or cmp_topk_length is not None or ori_topk:
        raise NotImplementedError("per-row top-k lengths / ori top-k: the window is the band of ori_mask_mode 4")
    if has_cmp_kv and cmp_ratio > 1 and not max_seqlen_cmp_kv:
        max_seqlen_cmp_kv = _max_len(cu_seqlens_cmp_kv)
    host = dict(max_cmp=int(max_seqlen_cmp_kv), cmp_ratio=int(cmp_ratio), num_heads_q=int(num_heads_q),
                head_dim=int(head_dim), win=(int(ori_win_left), int(ori_win_right)), has_cmp=bool(has_cmp_kv),
                cmp_topk=int(cmp_topk))
    fields = [num_heads_q, num_heads_kv, head_dim, batch_size, max_seqlen_q, max_seqlen_ori_kv, max_seqlen_cmp_kv,
              cmp_topk, cmp_ratio, ori_mask_mode, cmp_mask_mode, ori_win_left, ori_win_right, _LAYOUTS[layout_q],
              _LAYOUTS[layout_kv], int(bool(has_ori_kv)), int(bool(has_cmp_kv))]
    return _record(int(_kind), fields, host, _device_of(cu_seqlens_q, cu_seqlens_ori_kv))


def sparse_flash_mla_grad_metadata(**kwargs):
    """Record of the backward of the same problem (same keywords plus ``ori_topk``): kind 2
    in both the host tuple and the device record."""
    return sparse_flash_mla_metadata(**kwargs, _kind=2)


def _check_attn_metadata(metadata, query, cmp_ratio, ori_win_left, ori_win_right):
    h = _host(metadata)
    if not h:
        return
    want = dict(num_heads_q=(h["num_heads_q"], query.shape[1]), head_dim=(h["head_dim"], query.shape[2]),
                cmp_ratio=(h["cmp_ratio"], int(cmp_ratio)), window=(h["win"], (int(ori_win_left), int(ori_win_right))))
    for name, (have, got) in want.items():
        if have != got:
            raise ValueError(f"metadata was built for {name}={have}, the call has {got}")


def _geo(metadata, cu_q, cu_ori, cu_cmp, residual, cmp_kv, cmp_ratio):
    h = _host(metadata)
    return npu._sharedkv_tnd_args(cu_q, cu_ori, cu_cmp, residual, cmp_kv, cmp_ratio,
                                  max_cmp=h.get("max_cmp") if h else None)


def _kv2(t):
    return None if t is None else t.reshape(t.shape[0], t.shape[-1])


def sparse_flash_mla(query, *, ori_kv, cmp_kv=None, cmp_sparse_indices=None, ori_block_table=None,
                     cmp_block_table=None, cu_seqlens_q, cu_seqlens_ori_kv=None, cu_seqlens_cmp_kv=None,
                     cmp_residual_kv=None, sinks=None, metadata=None, softmax_scale=1.0, cmp_ratio=1,
                     ori_mask_mode=4, cmp_mask_mode=3, ori_win_left=127, ori_win_right=0, layout_q="TND",
                     layout_kv="TND", return_softmax_lse=True):
    """(out [T,N,D] like query, softmax_lse fp32 [T,N,1] or None): DeepSeek-V4 attention with
    the per-head sink over a packed batch (query [T,N,D], ori_kv [T,1,D], cmp_kv [T_c,1,D],
    cmp_sparse_indices [T,1,K] sequence-local, ratio 4)."""
    _check_tnd(layout_q, layout_kv)
    _check_masks(ori_mask_mode, cmp_mask_mode)
    if ori_block_table is not None or cmp_block_table is not None:
        raise NotImplementedError("paged KV (block tables) is not supported")
    npu.require_gpu_tensor(query, "query")
    _check_attn_metadata(metadata, query, cmp_ratio, ori_win_left, ori_win_right)
    cmp2 = _kv2(cmp_kv) if cmp_ratio > 1 else None
    geo = _geo(metadata, cu_seqlens_q, cu_seqlens_ori_kv, cu_seqlens_cmp_kv, cmp_residual_kv, cmp2, cmp_ratio)
    prep = npu._sharedkv_prepare(query.contiguous(), _kv2(ori_kv).contiguous(), cmp2, cmp_sparse_indices,
                                 int(cmp_ratio), ori_win_left, ori_win_right, tnd=geo)
    sk = None if sinks is None else sinks.float().contiguous()
    out, m2, s2 = npu._sharedkv_forward(prep, sk, float(softmax_scale))
    D = prep["D"]
    out = (out[..., :D] if prep["dv"] != D else out).reshape(query.shape).contiguous()
    lse = (m2 + torch.log(s2)).reshape(*query.shape[:2], 1) if return_softmax_lse else None
    return out, lse


def sparse_flash_mla_grad(query, grad_out, out, lse, *, ori_kv, cmp_kv=None, ori_sparse_indices=None,
                          cmp_sparse_indices=None, cu_seqlens_q, cu_seqlens_ori_kv=None, cu_seqlens_cmp_kv=None,
                          seqused_q=None, seqused_ori_kv=None, seqused_cmp_kv=None, cmp_residual_kv=None,
                          ori_topk_length=None, cmp_topk_length=None, sinks, metadata=None, softmax_scale=1.0,
                          cmp_ratio=1, ori_mask_mode=4, cmp_mask_mode=3, ori_win_left=127, ori_win_right=0,
                          layout_q="TND", layout_kv="TND"):
    """(dq like query, dori_kv like ori_kv, dcmp_kv like cmp_kv or None, dsinks like sinks,
    None, cmp_softmax_l1 fp32 [T,K] or None) from the forward's out and softmax_lse.

    cmp_softmax_l1[t, k] = the probability the row's softmax (over the window keys, the
    compressed keys and the sink) gives to its k-th compressed slot, averaged over the heads
    (0 for an empty slot): the target distribution of the V4 indexer loss
    (``LiLoss._current_selected_attn_dist``, models/deepseek_v4/model.py:421-456), taken from
    the probabilities this backward recomputes anyway.  Given for ratio 4 (None otherwise).
    The fifth entry (the ori-window counterpart) is None.
    """
    _check_tnd(layout_q, layout_kv)
    _check_masks(ori_mask_mode, cmp_mask_mode)
    if ori_sparse_indices is not None:
        raise NotImplementedError("ori_sparse_indices: the window over ori_kv is the band of ori_mask_mode 4")
    for name, t in (("seqused_q", seqused_q), ("seqused_ori_kv", seqused_ori_kv), ("seqused_cmp_kv", seqused_cmp_kv),
                    ("ori_topk_length", ori_topk_length), ("cmp_topk_length", cmp_topk_length)):
        if t is not None:
            raise NotImplementedError(f"{name} is not supported")
    _check_attn_metadata(metadata, query, cmp_ratio, ori_win_left, ori_win_right)
    cmp2 = _kv2(cmp_kv) if cmp_ratio > 1 else None
    geo = _geo(metadata, cu_seqlens_q, cu_seqlens_ori_kv, cu_seqlens_cmp_kv, cmp_residual_kv, cmp2, cmp_ratio)
    want_l1 = int(cmp_ratio) == 4 and cmp2 is not None
    res = npu._sharedkv_grad(query, ori_kv, cmp_kv if cmp2 is not None else None, grad_out, out, lse,
                             cmp_sparse_indices, sinks, softmax_scale, int(cmp_ratio), ori_win_left, ori_win_right,
                             geo, return_cmp_mass=want_l1)
    dq, d_ori, d_cmp, dsink = res[:4]
    l1 = (res[4] / query.shape[1]).contiguous() if want_l1 else None
    return dq, d_ori, d_cmp, dsink, None, l1


def lightning_indexer_metadata(n_heads, n_kv_heads, head_dim, topk, *, cu_seqlens_q=None, cu_seqlens_k=None,
                               cmp_residual_k=None, batch_size=1, max_seqlen_q=0, max_seqlen_k=0, layout_q="TND",
                               layout_k="TND", mask_mode=3, cmp_ratio=1):
    """Record of a packed indexer problem (keywords of npu_smla.py:797-812)."""
    _check_tnd(layout_q, layout_k)
    host = dict(n_heads=int(n_heads), head_dim=int(head_dim), topk=int(topk), cmp_ratio=int(cmp_ratio),
                mask_mode=int(mask_mode))
    fields = [n_heads, n_kv_heads, head_dim, topk, batch_size, max_seqlen_q, max_seqlen_k, mask_mode, cmp_ratio,
              _LAYOUTS[layout_q], _LAYOUTS[layout_k]]
    return _record(3, fields, host, _device_of(cu_seqlens_q, cu_seqlens_k))


def lightning_indexer(query, key, weights, sparse_count, *, cu_seqlens_q, cu_seqlens_k, cmp_residual_k=None,
                      metadata=None, layout_q="TND", layout_k="TND", mask_mode=3, cmp_ratio=1, return_value=0):
    """(indices int32 [T,1,K] sequence-local with -1 padding, values [T,1,K] in the query's
    dtype or None): lightning-indexer scores I[t, j] = sum_h w[t,h] relu(q[t,h].k[j]) over the
    sequence's compressed keys j < (p + 1 + o) // cmp_ratio (mask_mode 3), top ``sparse_count``
    per query (query [T,H,D], key [T_c,1,D], weights [T,H])."""
    _check_tnd(layout_q, layout_k)
    h = _host(metadata)
    if h and (h["topk"] != int(sparse_count) or h["cmp_ratio"] != int(cmp_ratio)):
        raise ValueError("metadata was built for another top-k or ratio")
    idx, vals = npu.lightning_indexer_varlen(query, key.reshape(key.shape[0], key.shape[-1]), weights, cu_seqlens_q,
                                             cu_seqlens_k, int(sparse_count), sparse_mode=int(mask_mode),
                                             cmp_ratio=int(cmp_ratio), cmp_residual_k=cmp_residual_k,
                                             return_value=bool(return_value))
    return idx.unsqueeze(1), (vals.to(npu._values_dtype(query)).unsqueeze(1) if return_value else None)


def sparse_lightning_indexer_kl_loss_grad_metadata(n_heads, n_kv_heads, head_dim, *, cu_seqlens_q=None,
                                                   cu_seqlens_k=None, cmp_residual_k=None, batch_size=1,
                                                   max_seqlen_q=0, max_seqlen_k=0, topk=0, layout_q="TND",
                                                   layout_k="TND", mask_mode=3, cmp_ratio=1):
    """Record of a packed indexer-loss problem (keywords of npu_smla.py:715-732)."""
    _check_tnd(layout_q, layout_k)
    host = dict(n_heads=int(n_heads), head_dim=int(head_dim), topk=int(topk), cmp_ratio=int(cmp_ratio))
    fields = [n_heads, n_kv_heads, head_dim, topk, batch_size, max_seqlen_q, max_seqlen_k, mask_mode, cmp_ratio,
              _LAYOUTS[layout_q], _LAYOUTS[layout_k]]
    return _record(4, fields, host, _device_of(cu_seqlens_q, cu_seqlens_k))


def sparse_lightning_indexer_kl_loss_grad(*, q, k, w, sparse_indices, attn_softmax_l1_norm, cmp_residual_k=None,
                                          cu_seqlens_q, cu_seqlens_k, metadata=None, layout_q="TND", layout_k="TND",
                                          mask_mode=3, cmp_ratio=1, eps=1e-10, grad_scale=1.0,
                                          return_loss_rows=False):
    """(dq [T,H,D], dk [T_c,1,D], dw [T,H], softmax_out) of the V4 indexer loss over a
    packed batch, unscaled (the caller multiplies by its loss scale, npu_smla.py:600-608).

    Per row: I_j = sum_h w[h] relu(q[h].k[idx_j]) over the used slots (sequence-local
    indices into the sequence's compressed keys), target t = l1 / sum(l1) from
    ``attn_softmax_l1_norm`` [T,K], row loss sum(l1) * KL(t || softmax(I)) (rows with
    sum(l1) <= eps add nothing) - DSAIndexerLoss with eps 1e-10 (dsa_indexer_loss.py:138-160),
    the form ``_compute_li_loss`` (npu_smla.py:405-420) logs.  ``grad_scale`` (a float or a
    device scalar) multiplies the gradients inside the kernel.  ``softmax_out`` [T,K] fp32 is
    the indexer's distribution over the slots, softmax of I over the usable slots and 0 at
    the others (written by the KL kernel from the row statistics it forms anyway);
    ``return_loss_rows`` appends the per-row losses [T] fp32.  Gradients are fp32 in the
    shapes of q / k / w.
    """
    _check_tnd(layout_q, layout_k)
    if int(mask_mode) != 3:
        raise NotImplementedError("mask_mode 3 (causal over the compressed keys) only")
    T = q.shape[0]
    kc = k.reshape(k.shape[0], k.shape[-1])
    idx = sparse_indices.reshape(T, -1)
    # sequence-local compressed-row indices -> rows of the packed key tensor, with the causal
    # rule re-applied (the indexer already leaves only visible rows)
    gidx = npu.sharedkv_tnd_indices(cu_seqlens_q, cu_seqlens_q, T, 0, q.device, cmp_ratio=int(cmp_ratio),
                                    cu_seqlens_cmp_kv=cu_seqlens_k, cmp_residual_kv=cmp_residual_k, cmp_indices=idx,
                                    window=False)
    dq, dk, dw, loss_rows, sm = npu.indexer_kl_grad_from_mass(
        q.unsqueeze(0), kc.unsqueeze(0), w.float().unsqueeze(0), gidx.unsqueeze(0),
        attn_softmax_l1_norm.float().reshape(1, T, -1).contiguous(), q_offset=npu._NO_MASK_OFFSET, loss_scale=1.0,
        eps=eps, grad_scale=grad_scale, return_softmax=True)
    res = (dq.reshape(q.shape), dk.reshape(k.shape), dw.reshape(w.shape), sm.reshape(T, -1))
    return res + (loss_rows.reshape(T),) if return_loss_rows else res
