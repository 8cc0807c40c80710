"""CPU oracle for the beam-decode hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference beam_engine computes on
its decode path, so that the HIP implementation in ``beam_engine_amd`` can be
checked against it.  It is never the thing measured or shipped:

* only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
  ``bench.py`` may import it, and only as a checker or as the timed CPU
  baseline;
* ``beam_engine_amd`` never imports it and has no CPU fallback.

Modules (each function cites the reference file:line it restates):

``attention``   paged gather, partial softmax attention with (o, lse), the
                log-sum-exp merge, cascade / flat / tree attention.
``beam_state``  FIFO page allocator, trie fork / copy rules, cascade metadata,
                final ranking.
``topk``        log_softmax + per-row top-2B + global top-B selection with
                float64 scores and stable tie order.
``fasttree``    the FastTree SplitQ/SplitK cost model.

Parity pinning (what each function is checked against besides the HIP path):

* attention: fp64 brute force, closed forms (single token -> v, constant
  scores -> mean(V) and ln T), torch's scaled_dot_product_attention in fp64,
  merge identities (idempotence, -inf identity, associativity, union).
* beam_state: hand-derived golden fixtures from the reference's own test trees
  (tests/golden/cascade_fixtures.json) and the allocator/fork trace; the
  reconstruction invariant of the reference's verify_cascade_output.
* topk: brute-force stable sort over the whole pool, torch.log_softmax /
  torch.topk on CPU for tie-free rows.
* fasttree: hand-evaluated cost-model values.
"""
