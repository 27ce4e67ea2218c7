"""CPU oracle for the two hot operators -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference's own PyTorch oracles and
host-side metadata rules for ``packed_varlen_attn`` and ``packed_target_attn``.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import it, and only as the checker.  The product path
(``varlenabsorbflashattn_amd``) never imports, calls or falls back to it.

Modules
-------
meta    -- seqinfo->cu_seqlens, cu_seqlens validation, chunk tables, split plan
varlen  -- block-diagonal attention forward/backward (log2-domain LSE)
absorb  -- absorbed target attention forward/backward + explicit-K/V restatement

Parity pins (each checked in tests/test_oracle.py): every function here is
checked against an independent computation -- closed forms (uniform
attention, single-key segments, one-hot segment-id values, the LSE combine
identity, the absorb<->explicit identity), torch.autograd on a float64
restatement, central finite differences, and brute force on tiny inputs.
No function is left "parity unpinned".
"""
from . import meta, varlen, absorb  # noqa: F401
