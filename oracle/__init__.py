"""CPU oracle for the block-sparse attention path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package may import, call or
link anything under ``oracle/``; the only importers are ``tests/``,
``__graft_entry__.smoke()`` (as the checker) and the ``cpu_baseline`` leg of
``bench.py`` (as the timed CPU reference).  The product path never routes
through this code.

Modules and what each restates (all paths are into the reference
``rrroooyyywang/SparseAttentionInfer``):

* ``oracle.csr``        -- ``build_block_pairs_from_mask`` and
  ``kv_block_list_to_pairs`` (``sparse_attentions/patterns/base.py:36-133``),
  plus a brute-force token-loop builder used to pin them.
* ``oracle.bigbird``    -- BigBird layout helpers, the rotation hash that picks
  "random" blocks, the keep-ratio estimators and the CSR / padded-list / token
  mask builders of ``BigBirdPattern``, ``BigBirdKeepRatioPattern`` and
  ``BigBird2Pattern`` (``sparse_attentions/patterns/bigbird_pattern.py``), and
  the sliding window of ``local_window.py``.
* ``oracle.attention``  -- the dense masked attention of ``MaskedSdpaBackend``
  (``sparse_attentions/attention/masked_sdpa.py:23-68``) with
  ``causal_mask`` (``sparse_attentions/utils.py:6-12``), a float64 textbook
  attention, and a block-gather restatement of the Triton kernel's semantics
  (``kernels/triton/universal_sparse_attn.py:77-160``) used at sizes where the
  dense oracle does not fit.

How each function is pinned (none of the reference's own tests covers this
path, so the pins are golden vectors written from the reference in this
container, published numbers, and mathematics):

* CSR builders: brute force over tokens on random masks, invariants, and
  reference-written golden vectors (``tests/golden``).
* BigBird hash and layouts: the keep ratios the reference published in its
  benchmark CSVs (head 0), and reference-written golden vectors for every
  head, prefill and decode, keep-ratio groups and BigBird2.
* Attention: float64 textbook loops, the all-ones-mask == causal SDPA special
  case, single-key rows, decode over all keys, and the block-gather form
  against the dense form.
"""
