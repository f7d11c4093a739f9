"""``npu_dsa``: DeepSeek-V3.2 DSA attention on the MI355X HIP kernels.

Drop-in for the reference's converters/kernels/dsa.py:
* ``dsa_forward`` replaces ``DSV32_SDPA.forward`` (dsa.py:195-277): lightning indexer +
  top-k, then gathered sparse MLA attention in absorb mode, then the indexer loss hook.
* ``LILossTrain`` (dsa.py:76-192): zero loss in forward, the fused KL loss and the
  indexer gradients in backward, scaled by the incoming gradient; the token-sum loss
  divided by B*S goes to the logging tracker.
* ``SparseLightningIndexerKLLoss`` (dsa.py:22-73) returns ``LILossTrain(...) / (B*S)``.

Inside ``dsa_forward`` the installed loss module is run through ``_LinkedIndexerLoss``, the
same deferred loss whose backward takes the main-attention mass from the layer's attention
backward (fused into dsa_sparse_mla_bwd) instead of recomputing it from the softmax
statistics: the loss node's zero output is an input of the attention op, so autograd runs
the attention backward first.  Called on its own, the module keeps the reference's
interface and takes the mass through the KL op (kept by the op-level attention backward
for the same tensors, or recomputed).
* ``NpuDSAConverter`` / ``DSAModelConfig`` registered as ``"npu_dsa"`` (dsa.py:283-309).
"""

from __future__ import annotations

import logging

import torch

from .. import torch_npu_ops as npu
from .convert_utils import replace_methods
from .dsa_indexer_loss import DSAIndexerLossLoggingHelper
from .model_custom_interface import ModelCustomConfig, ModelCustomConverter
from .registry import register_model_converter

logger = logging.getLogger(__name__)

_DSV32_MODEL_PACKAGE = "torchtitan_npu.models.deepseek_v32"


class LILossTrain(torch.autograd.Function):
    """Loss deferred to backward (activation recompute then does not redo the KL work)."""

    @staticmethod
    def forward(ctx, query, key, query_indexer, key_indexer, weights, sparse_indices, softmax_max, softmax_sum,
                layer_number=None, num_layers=0, scale_value=1.0, query_rope=None, key_rope=None,
                actual_seq_qlen=None, actual_seq_klen=None, layout="BSND", sparse_mode=3, pre_tokens=65536,
                next_tokens=65536):
        ctx.save_for_backward(query, key, query_indexer, key_indexer, weights, sparse_indices, softmax_max,
                              softmax_sum, query_rope, key_rope)
        ctx.layer_number = layer_number
        ctx.num_layers = num_layers
        ctx.scale_value = scale_value
        ctx.layout = layout
        ctx.sparse_mode = sparse_mode
        ctx.pre_tokens = pre_tokens
        ctx.next_tokens = next_tokens
        ctx.actual_seq_qlen = actual_seq_qlen
        ctx.actual_seq_klen = actual_seq_klen
        return torch.zeros(1, dtype=torch.float32, device=query.device)[0]

    @staticmethod
    def backward(ctx, *grad_output):
        (query, key, query_indexer, key_indexer, weights, sparse_indices, softmax_max, softmax_sum, query_rope,
         key_rope) = ctx.saved_tensors
        # the upstream gradient scales the KL gradients inside the kernel, read from the
        # device: no host round trip (the reference's `grad_output[0] != 1.0` test is one)
        g = grad_output[0]
        d_q, d_k, d_w, loss = npu.npu_sparse_lightning_indexer_grad_kl_loss(
            query, key, query_indexer, key_indexer, weights, sparse_indices, softmax_max, softmax_sum,
            scale_value=ctx.scale_value, query_rope=query_rope, key_rope=key_rope,
            actual_seq_qlen=ctx.actual_seq_qlen, actual_seq_klen=ctx.actual_seq_klen, layout=ctx.layout,
            sparse_mode=ctx.sparse_mode, pre_tokens=ctx.pre_tokens, next_tokens=ctx.next_tokens,
            grad_scale=g if isinstance(g, torch.Tensor) else float(g))
        bsz, sq = query.shape[0], query.shape[1]
        DSAIndexerLossLoggingHelper.save_loss_to_tracker(loss[0] / (bsz * sq), ctx.layer_number, ctx.num_layers)
        return (None, None, d_q.to(query_indexer.dtype), d_k.to(key_indexer.dtype), d_w.to(weights.dtype),
                *([None] * 14))


class _LinkedIndexerLoss(torch.autograd.Function):
    """LILossTrain for a layer's own attention (BSND, sparse_mode 3): zero in forward; in
    backward the KL loss and the indexer gradients, scaled by the upstream gradient, with the
    target mass from ``link`` (set by the attention backward; recomputed from the attention
    node's saved forward statistics only if that backward has not run)."""

    @staticmethod
    def forward(ctx, query_indexer, key_indexer, weights, sparse_indices, link, layer_number, num_layers):
        ctx.save_for_backward(query_indexer, key_indexer, weights, sparse_indices)
        ctx.link = link
        ctx.layer_number = layer_number
        ctx.num_layers = num_layers
        return torch.zeros((), dtype=torch.float32, device=query_indexer.device)

    @staticmethod
    def backward(ctx, grad):
        query_indexer, key_indexer, weights, idx = ctx.saved_tensors
        link = ctx.link
        mass = link.mass
        if mass is None:  # (a backward of the loss alone: the attention node did not run)
            mass = link.recompute_mass()
        g = grad if isinstance(grad, torch.Tensor) else float(grad)
        dq_i, dk_i, dw, loss_rows = npu.indexer_kl_grad_from_mass(query_indexer, key_indexer, weights, idx, mass,
                                                                  q_offset=link.q_offset, loss_scale=1.0, eps=1e-8,
                                                                  grad_scale=g)
        bsz, sq = query_indexer.shape[0], query_indexer.shape[1]
        DSAIndexerLossLoggingHelper.save_loss_to_tracker(loss_rows.sum() / (bsz * sq), ctx.layer_number,
                                                         ctx.num_layers)
        return (dq_i.to(query_indexer.dtype), dk_i.reshape(key_indexer.shape).to(key_indexer.dtype),
                dw.to(weights.dtype), None, None, None, None)


class SparseLightningIndexerKLLoss(torch.nn.Module):
    """Indexer KL loss module installed as ``inner_attention.compute_dsa_indexer_loss``."""

    def forward(self, query, key, query_indexer, key_indexer, weights, topk_indices, softmax_max, softmax_sum,
                scale_value=1.0, *, query_rope=None, key_rope=None, actual_seq_qlen=None, actual_seq_klen=None,
                layout="BSND", sparse_mode=3, pre_tokens=65536, next_tokens=65536, layer_number=None, num_layers=0):
        bsz, sq = query.shape[0], query.shape[1]
        loss = LILossTrain.apply(query, key, query_indexer, key_indexer, weights, topk_indices, softmax_max,
                                 softmax_sum, layer_number, num_layers, scale_value, query_rope, key_rope,
                                 actual_seq_qlen, actual_seq_klen, layout, sparse_mode, pre_tokens, next_tokens)
        return loss / (bsz * sq)


def dsa_forward(self, q, k, v, attn_mask=None, scale=None, q_indexer=None, k_indexer=None, weights=None,
                end_pos=None, index_topk=None):
    """Replacement for ``DSV32_SDPA.forward``: q [B,H,S,576], k [B,1,S,576], v [B,1,S,512],
    q_indexer [B,S,H_I,D_I], k_indexer [B,S,1,D_I], weights [B,S,H_I] -> (loss, out [B,H,S,512])."""
    if k.shape[1] != 1 or v.shape[1] != 1:
        raise NotImplementedError("Only support num_head_kv == 1 in dsa forward under absorb mode.")
    topk_indices, _ = npu.npu_lightning_indexer(q_indexer, k_indexer, weights, layout_query="BSND",
                                                layout_key="BSND", sparse_count=index_topk, sparse_mode=3,
                                                return_value=False)
    q = q.transpose(1, 2)
    k = k.transpose(1, 2)
    v = v.transpose(1, 2)
    nope, rope = self.config.kv_lora_rank, self.config.qk_rope_head_dim
    if type(self.compute_dsa_indexer_loss) is SparseLightningIndexerKLLoss:
        # the loss first (zero, deferred), then the attention with the loss's output as an
        # input: its backward runs before the loss's and hands over the attention mass.  The
        # attention takes the whole [nope | rope] rows (v = the first kv_lora_rank columns of
        # k, the absorb-mode alias), so no split / re-concatenation is made either way.
        bsz, sq = q.shape[0], q.shape[1]
        link = npu.MassLink()
        idx3 = topk_indices.reshape(bsz, sq, -1).to(torch.int32)
        z = _LinkedIndexerLoss.apply(q_indexer, k_indexer, weights, idx3, link, self.layer_number, self.num_layers)
        output, _, _ = npu.sparse_flash_attention_linked(q, k, topk_indices, scale, z, link, d_v=nope)
        return z / (bsz * sq), output.transpose(1, 2)
    q_nope, q_pe = torch.split(q, [nope, rope], dim=-1)
    k_nope, k_pe = torch.split(k, [nope, rope], dim=-1)
    output, softmax_max, softmax_sum = npu.npu_sparse_flash_attention(
        q_nope, k_nope, v, sparse_indices=topk_indices.to(torch.int32), block_table=None, query_rope=q_pe,
        key_rope=k_pe, scale_value=scale, sparse_block_size=1, layout_query="BSND", layout_kv="BSND", sparse_mode=3,
        attention_mode=2, return_softmax_lse=True)
    loss = self.compute_dsa_indexer_loss(
        q_nope.detach(), k_nope.detach(), q_indexer, k_indexer, weights, topk_indices, softmax_max, softmax_sum,
        scale_value=scale, query_rope=q_pe.detach(), key_rope=k_pe.detach(), actual_seq_qlen=None,
        actual_seq_klen=None, layout="BSND", layer_number=self.layer_number, num_layers=self.num_layers)
    return loss, output.transpose(1, 2)


class NpuDSAConverter(ModelCustomConverter):
    def convert(self, model) -> None:
        if self.model_name != "deepseek_v32":
            logger.info(f"NpuDSAConverter: skipped for model {self.model_name!r} (only deepseek_v32 is supported)")
            return
        count = replace_methods("DSV32_SDPA", "forward", dsa_forward, model=model, package=_DSV32_MODEL_PACKAGE)
        logger.info(f"  [DSV32_SDPA forward] Applied {count} replacement(s)")
        num_layers = len(model.layers)
        for layer_id, block in model.layers.named_children():
            inner = block.attention.inner_attention
            if not isinstance(getattr(inner, "compute_dsa_indexer_loss", None), SparseLightningIndexerKLLoss):
                inner.compute_dsa_indexer_loss = SparseLightningIndexerKLLoss()
            inner.layer_number = int(layer_id)
            inner.num_layers = num_layers


@register_model_converter("npu_dsa")
class DSAModelConfig(ModelCustomConfig):
    model_converter = NpuDSAConverter
