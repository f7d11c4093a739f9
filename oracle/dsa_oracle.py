"""CPU oracle for the DeepSeek sparse-attention (DSA) hot path.

TEST INFRASTRUCTURE ONLY.  This module is the checker that the HIP kernels of
``torchtitan_npu_simulator_amd`` are compared against.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product path never routes through it (the HIP library raises
when it is missing).

It restates, in plain PyTorch on the CPU (fp32 or fp64), the arithmetic of the
reference's torch-native DSA path.  Every function cites the reference lines it
follows (paths relative to the reference repository root):

* ``indexer_scores``       models/deepseek_v32/model.py:224-236 (bf16_index),
                           :378-388 (causal -inf mask); models/deepseek_v4/
                           model.py:647-652 (LiCompute einsum + ``t < (s+1)//r``)
* ``topk_select``          models/deepseek_v32/model.py:389-395;
                           models/deepseek_v4/model.py:653-655; the tie rule
                           (lower index wins, -0.0 == +0.0) is this build's
                           explicit contract for the unspecified torch.topk order
* ``sparse_mla_fwd``       models/deepseek_v32/model.py:391-404 (mask + SDPA over
                           the absorbed q/k/v of :519-535), gathered form
* ``dsv32_sdpa_dense``     models/deepseek_v32/model.py:335-420, the dense-mask
                           form exactly as written (small S only)
* ``sparse_mla_bwd``       autograd of ``sparse_mla_fwd`` plus the closed-form
                           flash-attention backward (for the latent alias
                           k_nope == v, models/deepseek_v32/model.py:527-528)
* ``attn_mass``            get_attn_scores, models/deepseek_v32/model.py:285-306
                           followed by the gather/zero of :410-413
* ``dsa_indexer_loss``     models/common/dsa_indexer_loss.py:138-160
* ``indexer_kl_loss_grad`` converters/kernels/dsa.py:76-192 (loss deferred to
                           backward; op returns the token SUM, caller divides by
                           B*S at :73 and :182-183)
* ``compressor_pool``      models/deepseek_v4/model.py:174-221 (overlap_transform
                           + softmax-gated pooling + RMSNorm)
* ``sparse_attn_sink``     models/deepseek_v4/model.py:573-623 (SparseAttention.forward:
                           window + compressed indices over cat(kv, kv_compress),
                           index mask, per-head sink logit appended to the softmax,
                           output = probs @ kv); ``v4_attn_indices`` builds its
                           index tensor (:581-592)
* ``v4_selected_attn_dist``  models/deepseek_v4/model.py:421-456 (LiLoss target: the
                           combined softmax at the selected compressed rows, averaged
                           over heads); the V4 loss is then ``indexer_kl_from_mass``
                           with loss_scale = softmax_scale, eps 1e-10 (:385, :412-417)
* ``window_topk_idxs``     models/deepseek_v4/model.py:467-471
* ``compress_topk_idxs``   models/deepseek_v4/model.py:483-488
* ``compressor_pool_tnd``  models/deepseek_v4/model.py:223-274 (Compressor._forward_tnd:
                           blocks gathered at block_starts, has_prev_block guard)
* ``lengths_to_cu_seqlens``, ``tnd_compressed_block_starts``
                           models/deepseek_v4/tnd.py:32-38, :87-94
* ``varlen_split``         per-sequence slices of a packed (TND) batch; the
                           varlen reference result is the per-sequence one
* ``rope_rotate``          apply_rotary_emb: models/deepseek_v32/model.py:173-193
                           (the indexer's non-interleaved layout viewed as interleaved
                           pairs and back), models/deepseek_v4/model.py:45-87
                           (interleaved); the complex product is torchtitan's
                           apply_rotary_emb_single_complex (an absent third-party
                           module: x as fp32 complex pairs times freqs_cis[pos], cast
                           back to x's dtype), restated here in fp64
* ``hadamard_rotate``      rotate_activation / hadamard_transform_ref,
                           models/deepseek_v32/model.py:196-221 and
                           models/deepseek_v4/model.py:90-111: F.linear with
                           scipy.linalg.hadamard(D) in the input dtype, then times
                           D^-0.5 in that dtype
* ``mla_absorb_q``, ``mla_absorb_out``
                           the absorbed-MLA einsums, models/deepseek_v32/model.py:
                           520-535 (q_nope . w_uk, then cat with q_pe) and :574-575
                           (output . w_uv_t), in fp64
* ``indexer_prep``         Indexer.forward's q / k producer:
                           models/deepseek_v32/model.py:264-282 (rope on the first
                           64 features, non-interleaved, then rotate) and
                           models/deepseek_v4/model.py:343-357 (rope on the last 64,
                           interleaved, then rotate), followed by this build's fp8
                           per-row quantisation (``quantize_e4m3_per_row``)

Which check pins each function (tests/test_oracle.py):

* indexer_scores: brute-force loops at S<=16; the H_I=1, w=1, q.k>=0 special
  case reduces to torch.matmul.
* topk_select: brute force by repeated arg-max at small sizes, adversarial ties
  and signed zeros; hypothesis sweep.
* sparse_mla_fwd / dsv32_sdpa_dense: K >= #valid reduces to dense causal
  F.scaled_dot_product_attention; gathered form == dense-mask form; lse equals
  torch.logsumexp of the masked logits.
* sparse_mla_bwd: fp64 torch.autograd.gradcheck of the gathered form, and the
  closed form equals autograd.
* attn_mass: rows sum to the number of heads (each head's softmax sums to 1).
* dsa_indexer_loss / indexer_kl_loss_grad: KL == 0 and zero gradient when the
  indexer distribution equals the target; fp64 gradcheck; reference's
  ``loss / (B*S)`` scaling.
* compressor_pool: uniform gates give the mean pool; first block gets no
  overlap contribution; r == 1 without overlap is the identity.
* sparse_attn_sink: a sink of -inf reduces it to sparse_mla_fwd with v = the
  whole row; brute-force loops over (s, h) on tiny inputs; fp64 gradcheck of
  the gradients to q, kv and the sink.
* v4_selected_attn_dist: equals the compressed-slot columns of sparse_attn_sink's
  probabilities summed over heads / H (recomputed from its lse); rows sum to at
  most 1.
* compressor_pool_tnd: one request whose length is a multiple of r equals
  compressor_pool on it; several such requests equal compressor_pool per request
  (the has_prev_block guard restarts the overlap at each request).
* TND metadata: the known answers of the reference's
  tests/unit_tests/models/test_deepseek_v4_tnd.py:65-79.
* rope_rotate: explicit per-pair loops (pair i = features (i, i + d/2) blocked,
  (2i, 2i + 1) interleaved); position 0 is the identity; rotating by the table and
  then by its conjugate restores the input; pair norms are preserved.
* hadamard_rotate: in fp64 it is orthogonal and symmetric, so applying it twice
  restores the input; the matrix is scipy.linalg.hadamard (entries +-1, H H = D I);
  a one-hot input gives the corresponding column times D^-0.5.
* indexer_prep: the composition of the two loops above with the reference's bf16
  rounding points, and quantize_e4m3_per_row of its output.
* mla_absorb_q / mla_absorb_out: per-head torch.matmul loops and the non-absorbed
  attention: with kv = [kv_latent, k_pe], the absorbed scores q_abs . kv equal the
  explicit q_nope . (kv_latent w_uk^T) + q_pe . k_pe, and the absorbed output
  (P kv_latent) w_uv equals P (kv_latent w_uv) (tests/test_oracle_prep.py).
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

__all__ = [
    "indexer_scores",
    "valid_key_count",
    "topk_select",
    "topk_select_numpy",
    "sparse_mla_fwd",
    "sparse_mla_bwd",
    "sparse_mla_bwd_closed_form",
    "dsv32_sdpa_dense",
    "attn_mass",
    "dsa_indexer_loss",
    "indexer_kl_loss_grad",
    "indexer_kl_from_mass",
    "compressor_pool",
    "sparse_attn_sink",
    "v4_attn_indices",
    "v4_selected_attn_dist",
    "window_topk_idxs",
    "compress_topk_idxs",
    "lengths_to_cu_seqlens",
    "tnd_compressed_block_starts",
    "compressor_pool_tnd",
    "varlen_split",
    "quantize_e4m3_per_row",
    "rope_rotate",
    "hadamard_rotate",
    "indexer_prep",
    "mla_absorb_q",
    "mla_absorb_out",
]


# ---------------------------------------------------------------------------
# a3: lightning-indexer scores
# ---------------------------------------------------------------------------
def valid_key_count(s: int, q_offset: int, cmp_ratio: int, s_k: int) -> int:
    """Number of keys query row ``s`` may attend to.

    V3.2 (cmp_ratio == 1): keys ``t <= s + q_offset``
    (models/deepseek_v32/model.py:378-388).  V4 compressed keys: block ``t`` is
    valid when ``t < (s + q_offset + 1) // r`` (models/deepseek_v4/model.py:650).
    Both are ``t < (s + q_offset + 1) // r``.
    """
    return max(0, min(s_k, (s + q_offset + 1) // cmp_ratio))


def indexer_scores(q_idx, k_idx, weights, *, q_offset=0, cmp_ratio=1, dtype=torch.float32):
    """I[b,s,t] = sum_h w[b,s,h] * relu(q_idx[b,s,h] . k_idx[b,t]), -inf where invalid.

    q_idx [B,S,H_I,D_I], k_idx [B,S_k,D_I] (or [B,S_k,1,D_I]), weights [B,S,H_I].
    Inputs are upcast to ``dtype`` first, as bf16_index does
    (models/deepseek_v32/model.py:228-229).
    """
    if k_idx.dim() == 4:
        k_idx = k_idx.squeeze(2)
    q = q_idx.to(dtype)
    k = k_idx.to(dtype)
    w = weights.to(dtype)
    p = torch.einsum("bshd,btd->bsht", q, k)
    score = (torch.relu(p) * w.unsqueeze(-1)).sum(dim=2)
    B, S, S_k = score.shape
    s_pos = torch.arange(S).unsqueeze(1)
    t_pos = torch.arange(S_k).unsqueeze(0)
    invalid = t_pos >= (s_pos + q_offset + 1) // cmp_ratio
    return score.masked_fill(invalid.unsqueeze(0), float("-inf"))


def quantize_e4m3_per_row(x: torch.Tensor):
    """OCP fp8-e4m3fn quantisation with one fp32 scale per row (last dim).

    scale = max(amax(|row|) / 448, 1e-12) (448 = largest finite e4m3fn; both the
    division and x / scale are correctly rounded fp32 divisions), q = x / scale rounded
    to the nearest e4m3fn value (ties to even).  Returns (q as torch.float8_e4m3fn, scale
    fp32 with the row shape).  The reference indexes in bf16 (fp8 is a QAT note there,
    models/deepseek_v4/model.py:646, :822), so this quantiser is the build's definition;
    the oracle's fp8 indexer computes on ``q.float() * scale`` (quantise, then
    dequantise), which is what the fp8 MFMA path must reproduce up to fp32 summation
    order.
    """
    xf = x.float()
    amax = xf.abs().amax(dim=-1).numpy()
    scale = torch.from_numpy(np.maximum(amax / np.float32(448.0), np.float32(1e-12)).astype(np.float32))
    q = (xf / scale.unsqueeze(-1)).to(torch.float8_e4m3fn)
    return q, scale


# ---------------------------------------------------------------------------
# a4: per-query top-k
# ---------------------------------------------------------------------------
def _orderable_keys(scores_f32: np.ndarray) -> np.ndarray:
    """Map fp32 to uint32 so that unsigned order == float order, -0.0 == +0.0."""
    s = np.ascontiguousarray(scores_f32, dtype=np.float32) + np.float32(0.0)  # -0.0 -> +0.0
    u = s.view(np.uint32)
    neg = (u >> np.uint32(31)).astype(bool)
    return np.where(neg, ~u, u | np.uint32(0x80000000)).astype(np.uint32)


def topk_select_numpy(scores: np.ndarray, k: int, n_valid: np.ndarray | None = None) -> np.ndarray:
    """Bit-exact reference selection on fp32 scores.

    Per row: among candidates t < n_valid[row] whose score is not NaN, take the
    first ``k`` of a stable descending sort by (score, then lower index) with
    -0.0 == +0.0.  Output: int32 [rows, k], the chosen indices in ascending
    index order, padded with -1.  (The reference's torch.topk leaves the tie
    order unspecified, models/deepseek_v32/model.py:390; this is the explicit
    rule the HIP select reproduces bit-exactly.)
    """
    scores = np.asarray(scores, dtype=np.float32)
    rows, n = scores.shape
    out = np.full((rows, k), -1, dtype=np.int32)
    keys = _orderable_keys(scores)
    for r in range(rows):
        nv = n if n_valid is None else int(min(n, max(0, n_valid[r])))
        row = scores[r, :nv]
        cand = np.nonzero(~np.isnan(row))[0]
        if cand.size == 0:
            continue
        kk = keys[r, cand].astype(np.int64)
        order = np.lexsort((cand, -kk))  # primary: key descending; secondary: index ascending
        chosen = np.sort(cand[order[:k]])
        out[r, : chosen.size] = chosen
    return out


def topk_select(scores: torch.Tensor, k: int, *, q_offset=0, cmp_ratio=1):
    """Top-k indices of masked indexer scores [B,S,S_k] -> int32 [B,S,k] (-1 padded).

    Validity follows ``valid_key_count``; entries outside it are never chosen
    (the reference marks them invalid after topk: models/deepseek_v32/
    model.py:391-395, models/deepseek_v4/model.py:654-655).
    """
    B, S, S_k = scores.shape
    nv = np.array([valid_key_count(s, q_offset, cmp_ratio, S_k) for s in range(S)], dtype=np.int64)
    out = np.stack([topk_select_numpy(scores[b].float().numpy(), k, nv) for b in range(B)])
    return torch.from_numpy(out)


def topk_values(scores: torch.Tensor, idx: torch.Tensor):
    """Scores at the selected indices, -inf at -1 slots (sparse_values)."""
    safe = idx.clamp_min(0).long()
    vals = torch.gather(scores.float(), -1, safe)
    return vals.masked_fill(idx < 0, float("-inf"))


# ---------------------------------------------------------------------------
# a5 / a6: gathered sparse MLA attention
# ---------------------------------------------------------------------------
def _attn_valid(idx: torch.Tensor, q_offset: int, s_kv: int) -> torch.Tensor:
    """Slot validity: idx >= 0, idx < S_kv and causal idx <= s + q_offset (sparse_mode 3)."""
    S = idx.shape[1]
    s_pos = torch.arange(S).view(1, S, 1)
    return (idx >= 0) & (idx < s_kv) & (idx <= s_pos + q_offset)


def sparse_mla_fwd(q, kv, idx, scale, *, d_v=512, q_offset=0, dtype=torch.float64, chunk=256):
    """O[b,s,h] = sum_{j in sel(s)} softmax_j(scale * q[b,s,h].kv[b,j]) kv[b,j,:d_v].

    q [B,S,H,D_qk], kv [B,S_kv,D_qk] (latent || rope; v = kv[..., :d_v]),
    idx [B,S,K] (-1 = empty slot).  Returns (out [B,S,H,d_v], lse [B,S,H]) in
    ``dtype``; lse is the natural-log logsumexp of the scaled logits (-inf for a
    row with no valid key, whose output is 0).  Duplicate indices count once
    per slot, like a gathered kernel; the reference's index_mask de-duplicates,
    so callers must pass distinct indices (top-k output always is).
    """
    B, S, H, D = q.shape
    s_kv = kv.shape[1]
    valid = _attn_valid(idx.long(), q_offset, s_kv)
    out = torch.zeros(B, S, H, d_v, dtype=dtype)
    lse = torch.full((B, S, H), float("-inf"), dtype=dtype)
    for b in range(B):
        for s0 in range(0, S, chunk):
            s1 = min(S, s0 + chunk)
            ii = idx[b, s0:s1].long().clamp(0, s_kv - 1)
            kk = kv[b].to(dtype)[ii]  # [c,K,D]
            vm = valid[b, s0:s1]  # [c,K]
            logits = torch.einsum("chd,ckd->chk", q[b, s0:s1].to(dtype), kk) * scale
            logits = logits.masked_fill(~vm.unsqueeze(1), float("-inf"))
            l = torch.logsumexp(logits, dim=-1)  # [c,H]
            p = torch.exp(logits - l.unsqueeze(-1))
            p = torch.nan_to_num(p, nan=0.0)
            out[b, s0:s1] = torch.einsum("chk,ckd->chd", p, kk[..., :d_v])
            lse[b, s0:s1] = l
    return out, lse


def sparse_mla_bwd(q, kv, idx, dout, scale, *, d_v=512, q_offset=0, dtype=torch.float64):
    """(dq, dkv) by autograd of ``sparse_mla_fwd`` (latent alias: dkv[:, :d_v] = dK_nope + dV)."""
    qq = q.detach().to(dtype).requires_grad_(True)
    kk = kv.detach().to(dtype).requires_grad_(True)
    out, _ = _sparse_mla_fwd_autograd(qq, kk, idx, scale, d_v, q_offset)
    (dq, dkv) = torch.autograd.grad(out, (qq, kk), dout.to(dtype))
    return dq, dkv


def _sparse_mla_fwd_autograd(q, kv, idx, scale, d_v, q_offset):
    B, S, H, D = q.shape
    s_kv = kv.shape[1]
    valid = _attn_valid(idx.long(), q_offset, s_kv)
    ii = idx.long().clamp(0, s_kv - 1)
    outs = []
    for b in range(B):
        kk = kv[b][ii[b]]  # [S,K,D]
        logits = torch.einsum("shd,skd->shk", q[b], kk) * scale
        logits = logits.masked_fill(~valid[b].unsqueeze(1), float("-inf"))
        m = logits.amax(dim=-1, keepdim=True).clamp_min(torch.finfo(logits.dtype).min)
        e = torch.exp(logits - m.detach())
        p = e / e.sum(dim=-1, keepdim=True).clamp_min(torch.finfo(logits.dtype).tiny)
        outs.append(torch.einsum("shk,skd->shd", p, kk[..., :d_v]))
    return torch.stack(outs), None


def sparse_mla_bwd_closed_form(q, kv, idx, out, lse, dout, scale, *, d_v=512, q_offset=0, dtype=torch.float64):
    """Flash-attention backward on the gathered set (what the HIP kernels compute).

    delta = sum(dO * O); P = exp(scale q.k - lse); dP = dO . v; dS = P (dP - delta);
    dq = scale sum_j dS k_j; dk_j += scale sum dS q; dv_j += sum P dO.
    Also returns the head-summed probability mass [B,S,K] used by the indexer loss.
    """
    B, S, H, D = q.shape
    s_kv = kv.shape[1]
    valid = _attn_valid(idx.long(), q_offset, s_kv)
    ii = idx.long().clamp(0, s_kv - 1)
    dq = torch.zeros(B, S, H, D, dtype=dtype)
    dkv = torch.zeros(B, s_kv, D, dtype=dtype)
    mass = torch.zeros(B, S, idx.shape[-1], dtype=dtype)
    for b in range(B):
        kk = kv[b].to(dtype)[ii[b]]
        qd = q[b].to(dtype)
        do = dout[b].to(dtype)
        delta = (do * out[b].to(dtype)).sum(-1)  # [S,H]
        logits = torch.einsum("shd,skd->shk", qd, kk) * scale
        p = torch.exp(logits - lse[b].to(dtype).unsqueeze(-1))
        p = p.masked_fill(~valid[b].unsqueeze(1), 0.0)
        dp = torch.einsum("shd,skd->shk", do, kk[..., :d_v])
        ds = p * (dp - delta.unsqueeze(-1))
        dq[b] = scale * torch.einsum("shk,skd->shd", ds, kk)
        dk = scale * torch.einsum("shk,shd->skd", ds, qd)
        dk[..., :d_v] += torch.einsum("shk,shd->skd", p, do)
        dk = dk * valid[b].unsqueeze(-1)
        dkv[b].index_add_(0, ii[b].reshape(-1), dk.reshape(-1, D))
        mass[b] = p.sum(dim=1)
    return dq, dkv, mass


def dsv32_sdpa_dense(q, k, v, q_indexer, k_indexer, weights, index_topk, scale, dtype=torch.float64):
    """DSV32_SDPA.forward in its dense-mask form (models/deepseek_v32/model.py:335-420).

    q [B,H,S,576], k [B,1,S,576], v [B,1,S,512], q_indexer [B,S,H_I,D_I],
    k_indexer [B,S,1,D_I], weights [B,S,H_I].  Returns (loss, out [B,H,S,512],
    topk_indices [B,S,K] with the reference's sentinel S-1 for invalid slots,
    valid_positions).  The selection uses ``topk_select`` (the tie rule) in place
    of torch.topk; everything after it is the reference's dense arithmetic.
    """
    bsz = q.shape[0]
    index_score = indexer_scores(q_indexer, k_indexer, weights, dtype=torch.float32)  # :363-369 + :378-388
    seqlen = index_score.size(1)
    k_eff = min(index_topk, seqlen)
    sel = topk_select(index_score, k_eff)  # ascending-index order, -1 padded
    topk_score = topk_values(index_score, sel)
    query_positions = torch.arange(seqlen).view(1, -1, 1)
    valid_positions = (sel >= 0) & (sel <= query_positions)
    topk_indices = torch.where(valid_positions, sel.long(), torch.full_like(sel.long(), seqlen - 1))
    attn_mask = torch.where(torch.triu(torch.ones(bsz, seqlen, seqlen), diagonal=1) == 1, float("-inf"), 0.0)
    index_mask = torch.full((bsz, seqlen, seqlen), float("-inf")).scatter_(-1, topk_indices, 0)
    masks = attn_mask + index_mask
    masks = (torch.isinf(masks) & (masks < 0)).unsqueeze(1)
    out = F.scaled_dot_product_attention(
        q.to(dtype), k.to(dtype), v.to(dtype), attn_mask=~masks, scale=scale, is_causal=False
    )
    # get_attn_scores (:285-306)
    attn = (q.to(dtype) @ k.to(dtype).transpose(-1, -2)) * scale
    attn = attn.masked_fill(masks, float("-inf"))
    attn = F.softmax(attn, dim=-1, dtype=torch.float32).sum(dim=1)
    selected = torch.gather(attn, -1, topk_indices).masked_fill(~valid_positions, 0.0)
    loss = dsa_indexer_loss(selected, topk_score, 1.0, eps=1e-8)
    return loss, out, topk_indices, valid_positions


def attn_mass(q, kv, idx, lse, scale, *, q_offset=0, dtype=torch.float64):
    """A[b,s,k] = sum_h exp(scale q[b,s,h].kv[idx] - lse[b,s,h]), 0 at invalid slots.

    get_attn_scores (models/deepseek_v32/model.py:285-306) gathered at the
    selected indices and zeroed at invalid slots (:410-413).
    """
    B, S, H, D = q.shape
    s_kv = kv.shape[1]
    valid = _attn_valid(idx.long(), q_offset, s_kv)
    ii = idx.long().clamp(0, s_kv - 1)
    out = torch.zeros(B, S, idx.shape[-1], dtype=dtype)
    for b in range(B):
        kk = kv[b].to(dtype)[ii[b]]
        logits = torch.einsum("shd,skd->shk", q[b].to(dtype), kk) * scale
        p = torch.exp(logits - lse[b].to(dtype).unsqueeze(-1)).masked_fill(~valid[b].unsqueeze(1), 0.0)
        out[b] = p.sum(dim=1)
    return out


# ---------------------------------------------------------------------------
# a7: indexer KL loss
# ---------------------------------------------------------------------------
def dsa_indexer_loss(selected_main_attn_dist, index_score, loss_scale, eps=1e-8, reduction="mean"):
    """DSAIndexerLoss.forward (models/common/dsa_indexer_loss.py:138-160).

    reduction="mean" is the module (mean over B*S tokens); "sum" is what the
    fused NPU op returns (converters/kernels/dsa.py:73 divides by B*S).
    """
    work = torch.float64 if selected_main_attn_dist.dtype == torch.float64 else torch.float32
    sel = selected_main_attn_dist.to(work).clamp_min(0)
    index_score = index_score.to(work)
    target_sum = sel.sum(dim=-1, keepdim=True)
    valid_target = target_sum > eps
    index_score = torch.where(valid_target, index_score, torch.zeros_like(index_score))
    ls = F.log_softmax(index_score, dim=-1, dtype=sel.dtype)
    t = sel / target_sum.clamp_min(eps)
    positive = t > 0
    ls = torch.where(positive, ls, torch.zeros_like(ls))
    log_t = t.clamp_min(eps).log()
    loss = (t * (log_t - ls)).sum(dim=-1)
    loss = target_sum.squeeze(-1) * loss
    loss = loss.mean() if reduction == "mean" else loss.sum()
    return loss * loss_scale


def indexer_kl_loss_grad(
    q, kv, q_idx, k_idx, weights, idx, lse, scale, *, q_offset=0, loss_scale=1.0, eps=1e-8, dtype=torch.float64
):
    """What npu_sparse_lightning_indexer_grad_kl_loss returns: (dq_idx, dk_idx, dw, loss_sum).

    The indexer scores are recomputed at the selected keys, the target is the
    head-summed main-attention mass at those keys, and the loss is the token SUM
    of DSAIndexerLoss's per-token term times ``loss_scale``; gradients flow
    only into (q_idx, k_idx, weights) (models/deepseek_v32/model.py:407-409).
    """
    mass = attn_mass(q, kv, idx, lse, scale, q_offset=q_offset, dtype=dtype)
    return indexer_kl_from_mass(q_idx, k_idx, weights, idx, mass, q_offset=q_offset, loss_scale=loss_scale, eps=eps,
                                dtype=dtype)


def indexer_kl_from_mass(q_idx, k_idx, weights, idx, mass, *, q_offset=0, loss_scale=1.0, eps=1e-8,
                         dtype=torch.float64):
    """KL loss SUM over tokens and its gradients given the target mass [B,S,K]."""
    s_k = k_idx.shape[-2] if k_idx.dim() == 3 else k_idx.shape[1]
    valid = _attn_valid(idx.long(), q_offset, s_k)
    qi = q_idx.detach().to(dtype).requires_grad_(True)
    ki = (k_idx.squeeze(2) if k_idx.dim() == 4 else k_idx).detach().to(dtype).requires_grad_(True)
    w = weights.detach().to(dtype).requires_grad_(True)
    ii = idx.long().clamp(0, s_k - 1)
    rows = []
    for b in range(q_idx.shape[0]):
        kk = ki[b][ii[b]]  # [S,K,D_I]
        p = torch.einsum("shd,skd->shk", qi[b], kk)
        sc = (torch.relu(p) * w[b].unsqueeze(-1)).sum(dim=1)
        rows.append(sc.masked_fill(~valid[b], float("-inf")))
    index_score = torch.stack(rows)
    target = mass.to(dtype).masked_fill(~valid, 0.0)
    loss = dsa_indexer_loss(target, index_score, loss_scale, eps=eps, reduction="sum")
    dq, dk, dw = torch.autograd.grad(loss, (qi, ki, w), allow_unused=True)
    return dq, dk, dw, loss.detach()


# ---------------------------------------------------------------------------
# a1: block KV compressor (V4)
# ---------------------------------------------------------------------------
def compressor_pool(kv, score, ape, ratio, *, overlap=None, norm_weight=None, norm_eps=1e-6, out_dtype=None,
                    freqs_cis=None, rope_dim=64, positions=None):
    """Softmax-gated pooling of token blocks (models/deepseek_v4/model.py:183-218).

    kv, score: [B,S,coff*D] fp32 (the wkv/wgate projections), ape [r,coff*D].
    With overlap (r == 4 in the reference, :150) slots r..2r-1 carry the current
    block's features D..2D and slots 0..r-1 the previous block's features 0..D;
    the first block's overlap slots are kv=0, score=-inf (overlap_transform,
    :174-181).  Returns the pooled [B,S/r,D] fp32, or, with ``norm_weight``,
    RMSNorm(pooled.to(out_dtype)) (:218) in float32.  With ``freqs_cis`` the last
    ``rope_dim`` features of the (out_dtype-rounded) row are rotated at the block's first
    position, positions[:, ::r] or c*r (:198-220), in fp64.
    """
    if overlap is None:
        overlap = ratio == 4
    B, S, CD = kv.shape
    coff = 2 if overlap else 1
    D = CD // coff
    if S % ratio:
        raise ValueError(f"seqlen ({S}) must be divisible by compress_ratio ({ratio})")
    kvb = kv.float().unflatten(1, (-1, ratio))
    sc = score.float().unflatten(1, (-1, ratio)) + ape.float()
    if overlap:
        nb = kvb.shape[1]
        kv2 = kvb.new_zeros(B, nb, 2 * ratio, D)
        sc2 = sc.new_full((B, nb, 2 * ratio, D), float("-inf"))
        kv2[:, :, ratio:] = kvb[..., D:]
        sc2[:, :, ratio:] = sc[..., D:]
        kv2[:, 1:, :ratio] = kvb[:, :-1, :, :D]
        sc2[:, 1:, :ratio] = sc[:, :-1, :, :D]
        kvb, sc = kv2, sc2
    pooled = (kvb * sc.softmax(dim=2)).sum(dim=2)
    if norm_weight is not None:
        x = pooled.to(out_dtype or torch.float32).float()
        rms = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + norm_eps)
        pooled = x * rms * norm_weight.float()
    if freqs_cis is None:
        return pooled
    nb = pooled.shape[1]
    cpos = positions[:, ::ratio] if positions is not None else torch.arange(nb).unsqueeze(0).expand(B, nb) * ratio
    x = pooled.to(out_dtype or torch.float32)
    rot = torch.stack([rope_rotate(x[b], freqs_cis, cpos[b], rope_dim=rope_dim, rope_start=D - rope_dim,
                                   interleaved=True, out_dtype=torch.float64) for b in range(B)])
    return rot


def compressor_pool_tnd(kv, score, ape, ratio, block_starts, positions, *, overlap=None, norm_weight=None,
                        norm_eps=1e-6, out_dtype=None, freqs_cis=None, rope_dim=64):
    """Compressor._forward_tnd pooling (models/deepseek_v4/model.py:223-265).

    kv, score: [T,coff*D] fp32 projections of the packed tokens; block c pools tokens
    block_starts[c] + [0, r).  With overlap, slots 0..r-1 take the PREVIOUS LISTED
    block's features 0..D (:248-249) unless the block's position is < r (the
    has_prev_block guard, :252-262) or it is the first block; those slots are kv=0,
    score=-inf.  Returns [n_blocks,D] fp32 (RMSNorm'd like compressor_pool with
    ``norm_weight``).
    """
    if overlap is None:
        overlap = ratio == 4
    T, CD = kv.shape
    coff = 2 if overlap else 1
    D = CD // coff
    bs = block_starts.long()
    rows = bs.unsqueeze(1) + torch.arange(ratio).unsqueeze(0)  # [n, r]
    kvb = kv.float()[rows]  # [n, r, coff*D]
    sc = score.float()[rows] + ape.float()
    if overlap:
        n = bs.numel()
        kv2 = kvb.new_zeros(n, 2 * ratio, D)
        sc2 = sc.new_full((n, 2 * ratio, D), float("-inf"))
        kv2[:, ratio:] = kvb[..., D:]
        sc2[:, ratio:] = sc[..., D:]
        kv2[1:, :ratio] = kvb[:-1, :, :D]
        sc2[1:, :ratio] = sc[:-1, :, :D]
        has_prev = positions.reshape(-1)[bs].ge(ratio).view(-1, 1, 1)
        kv2[:, :ratio] = torch.where(has_prev, kv2[:, :ratio], torch.zeros_like(kv2[:, :ratio]))
        sc2[:, :ratio] = torch.where(has_prev, sc2[:, :ratio], torch.full_like(sc2[:, :ratio], float("-inf")))
        kvb, sc = kv2, sc2
    pooled = (kvb * sc.softmax(dim=1)).sum(dim=1)
    if norm_weight is not None:
        x = pooled.to(out_dtype or torch.float32).float()
        rms = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + norm_eps)
        pooled = x * rms * norm_weight.float()
    if freqs_cis is None:
        return pooled
    # RoPE at each block's own position (:266-273)
    x = pooled.to(out_dtype or torch.float32)
    return rope_rotate(x, freqs_cis, positions.reshape(-1)[bs], rope_dim=rope_dim, rope_start=D - rope_dim,
                       interleaved=True, out_dtype=torch.float64)


def v4_attn_indices(bsz, seqlen, window_size, ratio, kv_len, cmp_idxs=None):
    """Index tensor of SparseAttention.forward (models/deepseek_v4/model.py:581-592): the
    sliding-window indices into kv_states, then (ratio > 1) the compressed ones into
    kv_compress offset by kv_len (``cmp_idxs``, already offset, or every causal block)."""
    idx = window_topk_idxs(window_size, bsz, seqlen)
    if ratio > 1:
        if cmp_idxs is None:
            cmp_idxs = compress_topk_idxs(ratio, bsz, seqlen, kv_len)
        idx = torch.cat([idx, cmp_idxs.to(idx.dtype)], dim=-1)
    return idx.int()


def sparse_attn_sink(q, kv, sink, idx, scale, *, dtype=torch.float64):
    """SparseAttention.forward math (models/deepseek_v4/model.py:600-623).

    q [B,S,H,D], kv [B,T,D] (cat of kv_states and kv_compress; k = v = the row), sink
    [H], idx [B,S,K] into kv (-1 = masked).  logits = scale q.k over the indexed keys
    (the reference's index mask adds bf16 min elsewhere, i.e. excludes them), the sink
    logit is appended, a softmax over [keys, sink] gives probs, and out = probs[:-1] @ kv.
    Returns (out [B,S,H,D], lse [B,S,H]) with lse = logsumexp over keys and sink.
    Differentiable in q, kv and sink (autograd in ``dtype``).
    """
    B, S, H, D = q.shape
    T = kv.shape[1]
    qd, kvd, sd = q.to(dtype), kv.to(dtype), sink.to(dtype)
    ii = idx.long()
    valid = (ii >= 0) & (ii < T)
    iic = ii.clamp(0, T - 1)
    outs, lses = [], []
    for b in range(B):
        kk = kvd[b][iic[b]]  # [S,K,D]
        logits = torch.einsum("shd,skd->shk", qd[b], kk) * scale
        logits = logits.masked_fill(~valid[b].unsqueeze(1), float("-inf"))
        comb = torch.cat([logits, sd.view(1, H, 1).expand(S, H, 1)], dim=-1)
        lse = torch.logsumexp(comb, dim=-1)
        p = torch.exp(comb - lse.unsqueeze(-1))[..., :-1]
        outs.append(torch.einsum("shk,skd->shd", p, kk))
        lses.append(lse)
    return torch.stack(outs), torch.stack(lses)


def v4_selected_attn_dist(q, kv, kv_compress, sink, cmp_idx, scale, window_size, *, dtype=torch.float64):
    """LiLoss._current_selected_attn_dist (models/deepseek_v4/model.py:421-456): the
    probability of the combined softmax (window keys, compressed keys, sink) at each
    selected compressed row, averaged over heads; 0 for -1 slots.  cmp_idx [B,S,K] are
    local compressed indices (offset removed)."""
    B, S, H, _ = q.shape
    kv_len = kv.shape[1]
    kv_all = torch.cat([kv, kv_compress], dim=1)
    cmp_off = torch.where(cmp_idx < 0, cmp_idx, cmp_idx + kv_len)
    idx = torch.cat([window_topk_idxs(window_size, B, S), cmp_off.to(torch.long)], dim=-1)
    T = kv_all.shape[1]
    ii = idx.long()
    valid = (ii >= 0) & (ii < T)
    iic = ii.clamp(0, T - 1)
    W = idx.shape[-1] - cmp_idx.shape[-1]
    rows = []
    for b in range(B):
        kk = kv_all[b].to(dtype)[iic[b]]
        logits = torch.einsum("shd,skd->shk", q[b].to(dtype), kk) * scale
        logits = logits.masked_fill(~valid[b].unsqueeze(1), float("-inf"))
        comb = torch.cat([logits, sink.to(dtype).view(1, H, 1).expand(S, H, 1)], dim=-1)
        p = torch.softmax(comb, dim=-1)[..., :-1]
        rows.append(p[..., W:].sum(dim=1) / H)
    dist = torch.stack(rows)
    return dist.masked_fill(cmp_idx < 0, 0.0)


def varlen_split(packed: torch.Tensor, cu_seqlens) -> list[torch.Tensor]:
    """The per-sequence slices packed[cu[i]:cu[i+1]] of a TND tensor."""
    cu = [int(v) for v in (cu_seqlens.tolist() if isinstance(cu_seqlens, torch.Tensor) else cu_seqlens)]
    return [packed[a:b] for a, b in zip(cu[:-1], cu[1:])]


# ---------------------------------------------------------------------------
# V4 index helpers and varlen metadata
# ---------------------------------------------------------------------------
def window_topk_idxs(window_size: int, bsz: int, seqlen: int):
    """GetWindowTopkIdxs.forward (models/deepseek_v4/model.py:467-471)."""
    base = torch.arange(seqlen).unsqueeze(1)
    w = (base - window_size + 1).clamp(0) + torch.arange(min(seqlen, window_size))
    w = torch.where(w > base, -1, w)
    return w.unsqueeze(0).expand(bsz, -1, -1)


def compress_topk_idxs(ratio: int, bsz: int, seqlen: int, offset: int):
    """GetCompressTopkIdxs.forward (models/deepseek_v4/model.py:483-488)."""
    m = torch.arange(seqlen // ratio).repeat(seqlen, 1)
    mask = m >= torch.arange(1, seqlen + 1).unsqueeze(1) // ratio
    return torch.where(mask, -1, m + offset).unsqueeze(0).expand(bsz, -1, -1)


def lengths_to_cu_seqlens(lengths: torch.Tensor) -> torch.Tensor:
    """[0, cumsum(lengths)] (models/deepseek_v4/tnd.py:32-38)."""
    return torch.cat((lengths.new_zeros((1,)), torch.cumsum(lengths, dim=0, dtype=lengths.dtype)))


def tnd_compressed_block_starts(flat_positions: torch.Tensor, ratio: int) -> torch.Tensor:
    """Token indices that start a whole ratio-block inside one request (tnd.py:87-94)."""
    n = flat_positions.numel()
    ti = torch.arange(n)
    end = ti + ratio - 1
    in_range = end < n
    end_pos = flat_positions[end.clamp_max(n - 1)]
    ok = flat_positions.remainder(ratio).eq(0) & in_range & end_pos.eq(flat_positions + ratio - 1)
    return torch.nonzero(ok, as_tuple=False).flatten()


def seeded_inputs(S, H, *, B=1, d_qk=576, d_v=512, h_idx=64, d_idx=128, topk=2048, seed=0, scale_inputs=True,
                  dtype=torch.bfloat16):
    """The seeded synthetic DSA inputs (fixed draw order: q, kv, q_idx, k_idx, w, dO).

    q, kv, q_idx, k_idx, dO ~ N(0,1); w ~ U(0,1) times H_I^-0.5 * D_I^-0.5 (the
    indexer's weight scaling, models/deepseek_v32/model.py:280-281).  With
    ``scale_inputs`` q is divided by sqrt(d_qk) ("N(0,1) scaled by 1/sqrt(d)").
    """
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S, H, d_qk, generator=g)
    if scale_inputs:
        q = q / math.sqrt(d_qk)
    kv = torch.randn(B, S, d_qk, generator=g)
    q_idx = torch.randn(B, S, h_idx, d_idx, generator=g)
    k_idx = torch.randn(B, S, d_idx, generator=g)
    w = torch.rand(B, S, h_idx, generator=g) * (h_idx ** -0.5) * (d_idx ** -0.5)
    dout = torch.randn(B, S, H, d_v, generator=g)
    return dict(q=q.to(dtype), kv=kv.to(dtype), q_idx=q_idx.to(dtype), k_idx=k_idx.to(dtype), w=w, dout=dout.to(dtype))


# ---------------------------------------------------------------------------
# the indexer input producer: RoPE, Hadamard rotation, fp8
# ---------------------------------------------------------------------------
def rope_rotate(x, freqs_cis, positions, *, rope_dim=64, rope_start=0, interleaved=True, out_dtype=None):
    """apply_rotary_emb on features [rope_start, rope_start + rope_dim) of x [N, ..., D]
    (models/deepseek_v32/model.py:173-193; models/deepseek_v4/model.py:45-87).

    Token n (the leading axis) is rotated by freqs_cis[positions[n]] (complex [n_pos,
    rope_dim/2]).  Interleaved: complex pair i is features (2i, 2i+1).  Not interleaved (the
    V3.2 indexer): the features are viewed as interleaved pairs first,
    ``x.view(..., 2, -1).transpose(-1, -2)``, so pair i is (i, i + rope_dim/2), and the
    result is put back with ``cat([y[..., 0::2], y[..., 1::2]])``.  The complex product
    (torchtitan's apply_rotary_emb_single_complex) is computed exactly in fp64 and cast to
    ``out_dtype`` (default: x's dtype), the reference's single rounding.
    """
    out_dtype = out_dtype or x.dtype
    fc = freqs_cis if freqs_cis.is_complex() else torch.view_as_complex(freqs_cis.float().contiguous())
    rot = fc.to(torch.complex128)[positions.long()]  # [N, rope_dim/2]
    xr = x[..., rope_start: rope_start + rope_dim].to(torch.float64)
    s = xr.shape
    if not interleaved:
        xr = xr.reshape(*s[:-1], 2, -1).transpose(-1, -2).reshape(*s)
    c = torch.view_as_complex(xr.reshape(*s[:-1], -1, 2).contiguous())
    shape = [rot.shape[0]] + [1] * (c.dim() - 2) + [rot.shape[1]]
    y = torch.view_as_real(c * rot.reshape(shape)).reshape(*s)
    if not interleaved:
        y = torch.cat([y[..., 0::2], y[..., 1::2]], dim=-1)
    out = x.to(torch.float64).clone()
    out[..., rope_start: rope_start + rope_dim] = y
    return out.to(out_dtype)


def hadamard_rotate(x, *, out_dtype=None):
    """rotate_activation (models/deepseek_v32/model.py:196-221; models/deepseek_v4/model.py:
    90-111): ``F.linear(x, H) * D^-0.5`` with H = scipy.linalg.hadamard(D) in x's dtype.
    The product is exact in fp64 and rounded to ``out_dtype`` (default x's dtype); the
    scaling then runs in fp32 on the rounded values and is rounded again, as a bf16 tensor
    times a Python float is in torch.  With out_dtype float64 nothing is rounded.
    """
    from scipy.linalg import hadamard

    out_dtype = out_dtype or x.dtype
    D = x.shape[-1]
    H = torch.tensor(hadamard(D), dtype=torch.float64)
    y = x.to(torch.float64) @ H.T
    if out_dtype == torch.float64:
        return y * D ** -0.5
    y = y.to(out_dtype)
    return (y.float() * np.float32(D ** -0.5)).to(out_dtype)


def indexer_prep(x, freqs_cis, positions, *, rope_dim=64, rope_start=0, interleaved=False, hadamard=True,
                 out_dtype=torch.bfloat16):
    """The indexer's q / k producer: RoPE (skipped when freqs_cis is None) then
    rotate_activation, with the reference's rounding points in ``out_dtype``; returns
    (y, q8, scale) with (q8, scale) = quantize_e4m3_per_row(y).  x [N, ..., D] with token
    positions [N].  V3.2: rope_start 0, not interleaved (models/deepseek_v32/model.py:
    264-282); V4: rope_start D - 64, interleaved (models/deepseek_v4/model.py:343-357)."""
    y = x
    if freqs_cis is not None:
        y = rope_rotate(y, freqs_cis, positions, rope_dim=rope_dim, rope_start=rope_start, interleaved=interleaved,
                        out_dtype=out_dtype)
    if hadamard:
        y = hadamard_rotate(y.to(out_dtype) if out_dtype != torch.float64 else y, out_dtype=out_dtype)
    q8, sc = quantize_e4m3_per_row(y.float())
    return y, q8, sc


# ---------------------------------------------------------------------------
# the MLA absorb einsums
# ---------------------------------------------------------------------------
def mla_absorb_q(q_nope, q_pe, w_uk, *, dtype=torch.float64):
    """PreAttention's absorbed query (models/deepseek_v32/model.py:520-535):
    ``cat([einsum("bshq,hqr->bshr", q_nope, w_uk), q_pe], -1)`` computed in ``dtype``."""
    q_abs = torch.einsum("bshq,hqr->bshr", q_nope.to(dtype), w_uk.to(dtype))
    return torch.cat([q_abs, q_pe.to(dtype)], dim=-1)


def mla_absorb_out(out, w_uv_t, *, dtype=torch.float64):
    """PostAttention's absorbed output projection (models/deepseek_v32/model.py:574-575),
    ``einsum("bhsr,hrv->bhsv", output, w_uv_t)``, on the BSND output [B,S,H,512]."""
    return torch.einsum("bshr,hrv->bshv", out.to(dtype), w_uv_t.to(dtype))
