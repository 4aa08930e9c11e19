"""CPU oracle for the attention path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU and in plain PyTorch (float64 by default), what
the reference computes on the attention path of KempnerForge:

* ``kempnerforge/model/position.py:12-71``   RoPE tables and ``apply_rope``
* ``kempnerforge/model/attention.py:29-70``  ``KVCache`` append
* ``kempnerforge/model/attention.py:116-236`` ``Attention.forward`` (RoPE → GQA
  expansion → causal / decode SDPA)
* ``kempnerforge/model/attention.py:238-280`` ``_attention_with_weights`` (capture)
* autograd backward of the above (SDPA backward, ``repeat_interleave`` backward,
  RoPE backward).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the CPU baseline.  The
product path (``kempnerforge_amd``) never imports it and has no CPU fallback.

Pinning (every function is checked by ``tests/test_oracle.py`` against something
that is not a retyping of its own formula):

* ``rope_tables``         closed form in numpy float64, cos²+sin²=1, position 0
  is the identity (reference ``tests/unit/test_model.py:67-106``).
* ``apply_rope``          scalar Python loop with explicit per-op rounding,
  pair-norm preservation, angle composition.
* ``attention_fwd``       ``torch.nn.functional.scaled_dot_product_attention``
  (library routine) after ``repeat_interleave``; scalar brute force on tiny
  shapes; LSE closed form (``exp(s - lse)`` sums to one; constant keys give
  ``lse = log(n) + s``).
* ``attention_bwd``       ``torch.autograd.gradcheck`` (finite differences) of the
  literal reference composition ``apply_rope → repeat_interleave → SDPA``.
* ``decode_step``         equal lengths reduce to a literal ``KVCache.update`` +
  SDPA(is_causal=False) restatement; decoding token t equals row t of the causal
  forward over t+1 tokens.
* ``capture``             rows sum to one, upper triangle zero, output equals
  ``attention_fwd``'s, ``P = exp(S - lse)``.
"""

from oracle.attention_ref import (  # noqa: F401
    apply_rope,
    attention_bwd,
    attention_fwd,
    attention_fwd_rows,
    attention_fwd_rotated,
    capture,
    decode_step,
    gqa_expand,
    rope_tables,
    rotate_half_inverse,
)
