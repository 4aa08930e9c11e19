"""CPU restatement of the reference attention path (test infrastructure only).

Every function states the reference lines it follows (paths relative to the
KempnerForge repository root).  Tensors use the layout the reference's
projections produce, ``q_proj(x).view(B, S, H, D)`` = BSHD
(``kempnerforge/model/attention.py:150-152``); the reference transposes to BHSD
before RoPE (``:160-162``), and so does this module, internally.

Numerics: RoPE is evaluated in the *input* dtype exactly as PyTorch eager
evaluates ``kempnerforge/model/position.py:65-71`` (tables cast to the input
dtype, every elementwise op rounded to that dtype).  Everything after RoPE is
evaluated in ``compute_dtype`` (float64 by default) from the rotated, input-dtype
values, which makes this the "fp32-or-better reference" the GPU kernels are
compared against.
"""

from __future__ import annotations

import math

import torch

__all__ = [
    "rope_tables",
    "apply_rope",
    "rotate_half_inverse",
    "gqa_expand",
    "attention_fwd",
    "attention_fwd_rows",
    "attention_fwd_rotated",
    "attention_bwd",
    "decode_step",
    "capture",
]


def rope_tables(head_dim: int, max_seq_len: int, theta: float = 10000.0):
    """RoPE cos/sin tables, float32 ``[max_seq_len, head_dim // 2]``.

    Follows ``kempnerforge/model/position.py:12-40``: ``inv = 1/theta^(2i/D)`` in
    float32 (``:32``), ``outer(arange(S), inv)`` (``:35-38``), ``cos, sin`` (``:40``).
    """
    assert head_dim % 2 == 0, f"head_dim must be even, got {head_dim}"
    freqs = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    positions = torch.arange(max_seq_len)
    table = torch.outer(positions, freqs)
    return table.cos(), table.sin()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Half-split rotation of ``x[..., S, D]`` by ``cos/sin[S, D/2]``.

    Follows ``kempnerforge/model/position.py:43-71``: halves ``x[..., :d]`` and
    ``x[..., d:]`` (``:58-60``), tables viewed to broadcast and cast to
    ``x.dtype`` (``:62-68``), ``cat([x1*c - x2*s, x2*c + x1*s])`` (``:71``).
    Each product and sum is a separate eager op, so for bfloat16 input every
    intermediate is rounded to bfloat16.
    """
    d = x.shape[-1] // 2
    x1, x2 = x[..., :d], x[..., d:]
    shape = [1] * (x.ndim - 2) + list(cos.shape)
    c = cos.view(*shape).to(x.dtype)
    s = sin.view(*shape).to(x.dtype)
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)


def rotate_half_inverse(g: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, table_dtype) -> torch.Tensor:
    """Backward of :func:`apply_rope` with respect to ``x`` (transposed rotation).

    ``r1 = x1 c - x2 s``, ``r2 = x2 c + x1 s`` ⇒ ``dx1 = g1 c + g2 s``,
    ``dx2 = g2 c - g1 s``, with ``c, s`` the tables after the cast to the input
    dtype (``kempnerforge/model/position.py:67-68``), evaluated in ``g.dtype``.
    """
    d = g.shape[-1] // 2
    g1, g2 = g[..., :d], g[..., d:]
    shape = [1] * (g.ndim - 2) + list(cos.shape)
    c = cos.view(*shape).to(table_dtype).to(g.dtype)
    s = sin.view(*shape).to(table_dtype).to(g.dtype)
    return torch.cat([g1 * c + g2 * s, g2 * c - g1 * s], dim=-1)


def gqa_expand(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """``repeat_interleave(n_rep, dim=1)`` on BHSD: query head ``h`` reads KV head
    ``h // n_rep`` (``kempnerforge/model/attention.py:89,173-175``)."""
    return x if n_rep == 1 else x.repeat_interleave(n_rep, dim=1)


def _rotated_bhsd(q, k, v, cos, sin):
    """RoPE'd q, k and plain v, transposed to BHSD, still in the input dtype
    (``kempnerforge/model/attention.py:160-166``)."""
    qr = apply_rope(q.transpose(1, 2), cos, sin)
    kr = apply_rope(k.transpose(1, 2), cos, sin)
    return qr, kr, v.transpose(1, 2)


def _causal_mask(sq: int, sk: int) -> torch.Tensor:
    """True where masked.  ``is_causal=True`` in SDPA aligns the mask top-left:
    query ``i`` sees keys ``j <= i`` (``kempnerforge/model/attention.py:229-231``,
    and the manual mask ``triu(1)`` at ``:272-276``)."""
    return torch.ones(sq, sk, dtype=torch.bool).triu(diagonal=1)


def _doc_mask(doc_ids) -> torch.Tensor:
    """True where masked: query ``i`` and key ``j`` of a packed sequence belong
    to different documents (``doc_ids[b,i] != doc_ids[b,j]``), ``[B,1,S,S]``.
    Follows ``kempnerforge/model/attention.py:211-216``: the explicit mask is
    ``causal & (doc_ids[:, :, None] == doc_ids[:, None, :])``."""
    d = torch.as_tensor(doc_ids)
    return (d.unsqueeze(2) != d.unsqueeze(1)).unsqueeze(1)


def _scores(qf, kf, causal, doc_ids=None, key_padding_mask=None):
    """Scaled scores with the masked entries at -inf.

    With ``doc_ids`` or ``key_padding_mask`` this is the reference's
    explicit-mask branch (``kempnerforge/model/attention.py:209-225``;
    ``kempnerforge/model/mot.py:188-196``): allowed = causal AND same document
    AND ``key_padding_mask[b, j]``, then the NaN guard ``allowed | ~allowed.any(
    -1)``, which unmasks a row that allows no key at all."""
    d = qf.shape[-1]
    s = torch.matmul(qf, kf.transpose(-2, -1)) * (d ** -0.5)
    if doc_ids is None and key_padding_mask is None:
        if causal:
            s = s.masked_fill(_causal_mask(s.shape[-2], s.shape[-1]), float("-inf"))
        return s
    masked = torch.zeros(1, 1, s.shape[-2], s.shape[-1], dtype=torch.bool)
    if causal:
        masked = masked | _causal_mask(s.shape[-2], s.shape[-1])
    if doc_ids is not None:
        masked = masked | _doc_mask(doc_ids)
    if key_padding_mask is not None:
        kpm = torch.as_tensor(key_padding_mask).bool()
        masked = masked | ~kpm.view(kpm.shape[0], 1, 1, -1)
    masked = masked & ~masked.all(dim=-1, keepdim=True)  # NaN guard
    return s.masked_fill(masked, float("-inf"))


def attention_fwd(q, k, v, cos, sin, *, causal: bool = True, compute_dtype=torch.float64,
                  doc_ids=None, key_padding_mask=None):
    """Causal GQA attention with fused RoPE; returns ``(out, lse)``.

    q ``[B,Sq,Hq,D]``, k/v ``[B,Sk,Hkv,D]`` (pre-RoPE), cos/sin ``[S, D/2]``
    float32 rows for positions ``0..S-1``.  out ``[B,Sq,Hq,D]`` and
    lse ``[B,Hq,Sq]`` (natural log of the softmax denominator of the scaled
    scores) in ``compute_dtype``.

    Follows ``kempnerforge/model/attention.py:160-175`` (transpose, RoPE, GQA
    expansion) and ``:228-231`` (``F.scaled_dot_product_attention`` with default
    scale ``D^-1/2`` and ``is_causal``).  The reference returns no LSE; it is the
    closed form ``log sum_j exp(s_ij)``.  With ``doc_ids [B,S]`` (packed
    sequences, ``:204-227``) a query also sees only keys of its own document;
    with ``key_padding_mask [B,S]`` (True = attend) only valid keys, and a row
    left with none attends every key (the NaN guard).
    """
    qr, kr, vt = _rotated_bhsd(q, k, v, cos, sin)
    n_rep = qr.shape[1] // kr.shape[1]
    qf = qr.to(compute_dtype)
    kf = gqa_expand(kr, n_rep).to(compute_dtype)
    vf = gqa_expand(vt, n_rep).to(compute_dtype)
    s = _scores(qf, kf, causal, doc_ids, key_padding_mask)
    lse = torch.logsumexp(s, dim=-1)
    p = torch.exp(s - lse.unsqueeze(-1))
    out = torch.matmul(p, vf)
    return out.transpose(1, 2).contiguous(), lse


def attention_fwd_rows(q, k, v, cos, sin, rows, *, heads=None, causal: bool = True,
                       compute_dtype=torch.float64):
    """Selected query rows of :func:`attention_fwd` without the full score matrix.

    ``rows`` is a 1-D index of query positions, ``heads`` an optional index of
    query heads.  Returns ``(out [B, len(rows), len(heads), D], lse [B,
    len(heads), len(rows)])`` equal to the matching slices of
    :func:`attention_fwd` (rows are independent given all keys), so full-size
    GPU outputs can be spot-checked in seconds.
    """
    rows = torch.as_tensor(rows, dtype=torch.long)
    Hq, Hkv = q.shape[2], k.shape[2]
    n_rep = Hq // Hkv
    heads = torch.arange(Hq) if heads is None else torch.as_tensor(heads, dtype=torch.long)
    kmax = int(rows.max()) + 1 if causal else k.shape[1]
    kr = apply_rope(k[:, :kmax].transpose(1, 2), cos[:kmax], sin[:kmax])
    qsel = q[:, rows][:, :, heads]
    qr = apply_rope(qsel.permute(0, 2, 1, 3), cos[rows], sin[rows])
    kf = kr[:, heads // n_rep].to(compute_dtype)
    vf = v[:, :kmax].transpose(1, 2)[:, heads // n_rep].to(compute_dtype)
    s = torch.matmul(qr.to(compute_dtype), kf.transpose(-2, -1)) * (q.shape[-1] ** -0.5)
    if causal:
        s = s.masked_fill(torch.arange(kmax)[None, :] > rows[:, None], float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    out = torch.matmul(torch.exp(s - lse.unsqueeze(-1)), vf)
    return out.transpose(1, 2).contiguous(), lse


def attention_fwd_rotated(q, k_cache, v_cache, cos, sin, *, causal: bool = True,
                          compute_dtype=torch.float64):
    """Forward over already-rotated keys in cache layout ``[B, Hkv, Sk, D]``.

    The multi-token-with-cache branch of ``Attention.forward``
    (``kempnerforge/model/attention.py:165-175,229-231``): q ``[B,Sq,Hq,D]`` is
    rotated with table rows ``0..Sq-1`` (the caller passes the rows for
    ``start_pos..``), keys come from the cache, and ``is_causal=True`` aligns
    the mask top-left even when ``Sq < Sk``.  Returns ``(out BSHD, lse)``.
    """
    qr = apply_rope(q.transpose(1, 2), cos, sin)
    n_rep = qr.shape[1] // k_cache.shape[1]
    qf = qr.to(compute_dtype)
    kf = gqa_expand(k_cache, n_rep).to(compute_dtype)
    vf = gqa_expand(v_cache, n_rep).to(compute_dtype)
    s = _scores(qf, kf, causal)
    lse = torch.logsumexp(s, dim=-1)
    out = torch.matmul(torch.exp(s - lse.unsqueeze(-1)), vf)
    return out.transpose(1, 2).contiguous(), lse


def attention_bwd(q, k, v, cos, sin, dout, *, causal: bool = True, compute_dtype=torch.float64,
                  doc_ids=None, key_padding_mask=None):
    """Gradients ``(dq, dk, dv)`` of :func:`attention_fwd`'s output, pre-RoPE, BSHD.

    The reference gets these from autograd (``scripts/train.py:850``) through
    SDPA backward, the ``repeat_interleave`` backward (sum over the ``n_rep``
    query heads of each KV group, ``kempnerforge/model/attention.py:173-175``)
    and the RoPE backward (transposed rotation with the dtype-cast tables,
    ``kempnerforge/model/position.py:65-71``).  Here the attention part is
    differentiated by autograd in ``compute_dtype`` starting from the rotated,
    input-dtype q/k, and the RoPE backward is applied in closed form.
    """
    qr, kr, vt = _rotated_bhsd(q, k, v, cos, sin)
    n_rep = qr.shape[1] // kr.shape[1]
    qf = qr.to(compute_dtype).detach().requires_grad_(True)
    kf = kr.to(compute_dtype).detach().requires_grad_(True)
    vf = vt.to(compute_dtype).detach().requires_grad_(True)
    with torch.enable_grad():
        s = _scores(qf, gqa_expand(kf, n_rep), causal, doc_ids, key_padding_mask)
        p = torch.softmax(s, dim=-1)
        out = torch.matmul(p, gqa_expand(vf, n_rep))
        out.backward(dout.transpose(1, 2).to(compute_dtype))
    dq = rotate_half_inverse(qf.grad, cos, sin, q.dtype)
    dk = rotate_half_inverse(kf.grad, cos, sin, k.dtype)
    return (
        dq.transpose(1, 2).contiguous(),
        dk.transpose(1, 2).contiguous(),
        vf.grad.transpose(1, 2).contiguous(),
    )


def attention_bwd_rounded_operands(q, k, v, cos, sin, dout, *, operand_dtype,
                                   causal: bool = True, doc_ids=None, key_padding_mask=None):
    """:func:`attention_bwd` with the products' 16-bit operands rounded: the
    closed-form flash-attention backward in float64 except that P (the operand of
    dV = P^T dO) and dS = P (dP - Delta) (the operand of dK and dQ) are rounded
    to ``operand_dtype``, and Delta = rowsum(dO * O) uses the output O as stored
    (rounded to the input dtype).  Any backward whose matrix products take bf16
    (fp16) P and dS operands, the reference's bf16 SDPA backward included, carries
    at least this rounding against exact arithmetic; the GPU tests use the
    difference to :func:`attention_bwd` as the error the operand format itself
    forces.  ``operand_dtype=None`` rounds nothing (and keeps O exact), which
    equals :func:`attention_bwd` to float64 rounding (``tests/test_oracle.py``).
    """
    qr, kr, vt = _rotated_bhsd(q, k, v, cos, sin)
    n_rep = qr.shape[1] // kr.shape[1]
    f64 = torch.float64
    rnd = (lambda x: x) if operand_dtype is None else (lambda x: x.to(operand_dtype).to(f64))
    qf, kf, vf = qr.to(f64), gqa_expand(kr, n_rep).to(f64), gqa_expand(vt, n_rep).to(f64)
    do = dout.transpose(1, 2).to(f64)
    scale = q.shape[-1] ** -0.5
    s = _scores(qf, kf, causal, doc_ids, key_padding_mask)
    p = torch.exp(s - torch.logsumexp(s, dim=-1, keepdim=True))
    o = torch.matmul(p, vf)
    o_stored = o if operand_dtype is None else o.to(q.dtype).to(f64)
    pr = rnd(p)
    dv = torch.matmul(pr.transpose(-2, -1), do)
    dp = torch.matmul(do, vf.transpose(-2, -1))
    delta = (do * o_stored).sum(-1, keepdim=True)
    ds = rnd(pr * (dp - delta))
    dq = torch.matmul(ds, kf) * scale
    dk = torch.matmul(ds.transpose(-2, -1), qf) * scale
    B, Hq, S, D = dk.shape
    dk = dk.view(B, Hq // n_rep, n_rep, S, D).sum(2)
    dv = dv.view(B, Hq // n_rep, n_rep, -1, D).sum(2)
    dq = rotate_half_inverse(dq, cos, sin, q.dtype)
    dk = rotate_half_inverse(dk, cos, sin, k.dtype)
    return (dq.transpose(1, 2).contiguous(), dk.transpose(1, 2).contiguous(),
            dv.transpose(1, 2).contiguous())


def decode_step(q_new, k_new, v_new, k_cache, v_cache, lens, cos_table, sin_table,
                *, compute_dtype=torch.float64):
    """One KV-cache decode step with a per-sequence cache fill level.

    q_new ``[B,1,Hq,D]``, k_new/v_new ``[B,1,Hkv,D]`` (pre-RoPE), caches
    ``[B,Hkv,Smax,D]`` (post-RoPE K, ``kempnerforge/model/attention.py:46-51``),
    ``lens[b]`` = tokens already cached for sequence ``b`` = the new token's
    position.  Returns ``(out [B,1,Hq,D] in compute_dtype, k_cache', v_cache')``.

    Per sequence this is the reference's decode: RoPE at ``start_pos``
    (``kempnerforge/model/transformer.py:418-425``), ``KVCache.update`` slice
    assignment (``kempnerforge/model/attention.py:54-70``), GQA expansion of the
    whole cache (``:173-175``) and SDPA with ``is_causal=False`` (``:229-231``).
    The reference holds one scalar ``seq_len`` for the batch; equal ``lens``
    reduce to exactly that.
    """
    B = q_new.shape[0]
    Hq, Hkv = q_new.shape[2], k_new.shape[2]
    n_rep = Hq // Hkv
    k_cache = k_cache.clone()
    v_cache = v_cache.clone()
    outs = []
    for b in range(B):
        pos = int(lens[b])
        c, s = cos_table[pos:pos + 1], sin_table[pos:pos + 1]
        qr = apply_rope(q_new[b:b + 1].transpose(1, 2), c, s)
        kr = apply_rope(k_new[b:b + 1].transpose(1, 2), c, s)
        k_cache[b:b + 1, :, pos:pos + 1] = kr
        v_cache[b:b + 1, :, pos:pos + 1] = v_new[b:b + 1].transpose(1, 2)
        kk = gqa_expand(k_cache[b:b + 1, :, : pos + 1], n_rep).to(compute_dtype)
        vv = gqa_expand(v_cache[b:b + 1, :, : pos + 1], n_rep).to(compute_dtype)
        sc = torch.matmul(qr.to(compute_dtype), kk.transpose(-2, -1)) * (q_new.shape[-1] ** -0.5)
        p = torch.softmax(sc, dim=-1)
        outs.append(torch.matmul(p, vv).transpose(1, 2))
    return torch.cat(outs, dim=0), k_cache, v_cache


def capture(q, k, v, cos, sin, *, causal: bool = True, compute_dtype=torch.float64,
            doc_ids=None, key_padding_mask=None):
    """Materialised attention probabilities; returns ``(out BSHD, P [B,Hq,Sq,Sk])``.

    Follows ``kempnerforge/model/attention.py:238-280``: ``QK^T * D^-1/2``
    (``:259-260``), ``masked_fill(triu(1), -inf)`` (``:272-276``), softmax over
    keys (``:278``), ``P @ V`` (``:279``), after the same RoPE and GQA expansion
    as the forward (``:160-175``).
    """
    qr, kr, vt = _rotated_bhsd(q, k, v, cos, sin)
    n_rep = qr.shape[1] // kr.shape[1]
    qf = qr.to(compute_dtype)
    kf = gqa_expand(kr, n_rep).to(compute_dtype)
    vf = gqa_expand(vt, n_rep).to(compute_dtype)
    p = torch.softmax(_scores(qf, kf, causal, doc_ids, key_padding_mask), dim=-1)
    out = torch.matmul(p, vf)
    return out.transpose(1, 2).contiguous(), p


def flops_fwd(B: int, Sq: int, Hq: int, D: int, causal: bool = True) -> float:
    """Algorithmic forward flops, ``4·D·P`` with ``P`` the attended (q, k) pairs;
    GQA is not discounted (``kempnerforge/metrics/mfu.py:97-98``)."""
    pairs = B * Hq * (Sq * (Sq + 1) // 2 if causal else Sq * Sq)
    return 4.0 * D * pairs


def logsumexp_closed_form(scores_row) -> float:
    """Scalar ``log(sum(exp(s)))`` with max subtraction, for brute-force checks."""
    m = max(scores_row)
    return m + math.log(sum(math.exp(x - m) for x in scores_row))
