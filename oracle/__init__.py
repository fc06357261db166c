# -*- coding: utf-8 -*-
"""CPU oracle for the RVC synthesis hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference's numpy inference path
(``runtime/nn.py`` + the numpy branches of ``runtime/backend.py`` and
``runtime/models/vits.py``) so the HIP backend can be checked against it on
identical seeded inputs.  Every function cites the reference file:line it
follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker / the timed CPU
baseline.  The product (``rvc-vulkan_amd/``) never imports it and has no CPU
fallback.

Pinning status (what checks each oracle function against something other
than itself; the tests named here live under ``tests/``):

* ``nn_ref.conv1d`` / ``conv_transpose1d`` / ``linear`` / ``embedding`` /
  ``layer_norm`` / ``softmax`` / ``leaky_relu`` / ``sigmoid`` / ``tanh``:
  float64 brute-force loops (``oracle/loops.py``) on tiny inputs, scipy
  ``correlate`` for conv1d, the adjoint identity <convT x, y> = <x, conv y>
  (test_oracle_ops.py).
* ``vits_ref.deweight_norm``: closed form and the ``g = ||v||`` special case.
* ``vits_ref.get_relative_embeddings`` / ``relative_to_absolute`` /
  ``absolute_to_relative``: brute-force index identities for P in
  {1,5,11,12,40} (test_oracle_ops.py).
* attention in ``TextEncoder.encode``: an explicit banded double loop in
  float64 (``loops.relpos_attention``).
* ``GeneratorNSF.sine_gen``: special cases (f0 == 0, constant f0) and the
  golden vectors written by importing the reference
  (``tests/golden/make_golden.py``).
* ``hubert_ref.gelu_erf``: the reference's own outputs on a grid and the
  exact-erf GELU within the A&S 7.1.26 bound; ``group_norm``: a float64
  per-group standardisation; ``pos_conv_weight``: the ``g = ||v||`` case;
  ``grouped_conv1d``: the equivalent block-diagonal dense conv;
  ``HubertRef`` stages (conv stack, projection, encoder entry, layer 1,
  version 1 and 2 outputs): reference golden vectors at T in {1600, 4000}
  (``tests/golden/make_golden_hubert.py``; test_oracle_hubert.py).
* ``VitsConfig``, ``TextEncoder.encode``, ``FlowBlock.reverse``,
  ``GeneratorNSF.forward`` and ``Synthesizer.infer_controlled``: golden
  vectors produced by the reference's own numpy code at reduced and full
  width (``tests/golden/*.npz``; test_oracle_golden.py).
"""
