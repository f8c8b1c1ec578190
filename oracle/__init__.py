"""CPU oracle for the paged-attention decode path - TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import anything from this package, and only as the checker (or, for
the baseline, as the timed CPU restatement).  The product path
(``paged_attention_decode_amd``) never imports it and has no CPU fallback.

Contents (each function cites the reference file:line it restates):

* ``reference.paged_attention_decode_reference`` - fp32 torch restatement of
  ``src/reference.py:8-54`` with the input validation of
  ``src/reference.py:57-112``.  Pinned by: ``torch.nn.functional.
  scaled_dot_product_attention`` on unpaged inputs (the reference's own
  ``tests/test_reference.py:7-36`` check), the float64 brute force below
  (independent page walk), closed-form known answers and invariants
  (``tests/test_oracle_*.py``).
* ``brute.decode_f64`` - float64 numpy brute force with its own page walk,
  written from the operator's definition (no code shared with
  ``reference``); the source of the committed golden fixtures.  Pinned by
  the same SDPA and closed-form checks.
* ``splitk`` - float64 model of the split-K decomposition of
  ``analysis/split_k_derivation.md:16-86`` (phase-1 partials, phase-2 merge
  with the ``-inf`` guard), in token-granular and page-aligned split modes.
  Pinned against ``brute`` (split invariance over many split counts,
  including empty splits), and by planted-mistake tests that show a dropped
  rescale, a dropped guard or a wrong merge index is caught.
* ``csr`` - the dense -> CSR page-index conversion of the reference's
  FlashInfer adapter (src/flashinfer_adapter.py:40-65) and its inverse.
  Pinned by hand-computed known answers and round trips.
"""
