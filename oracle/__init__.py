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
* ``Synthesizer.make_noise`` (nz drawn before ns from one
  ``RandomState(seed)``, ``RVC_FIXED_SEED``), ``infer(seed)``,
  ``phase_offsets``, ``sine_gen(seg_offsets)``, the partial ``prep_dec``
  (flow from ``max(head - 40, 0)``, decoder segment +- 16 frames),
  ``decode_batch(preps)`` over unequal chunks and
  ``infer(skip_head, return_length)``: the reference's own outputs for each
  (``tests/golden/make_golden_partial.py``; test_oracle_partial.py).
  ``phase_offsets`` is also compared bit for bit with the GPU's blocked scan
  at 16 383 - 70 001 frames (test_gpu_partial.py).
* the ``conv_formulation("taps")`` form of ``nn_ref.conv1d`` /
  ``conv_transpose1d`` (contiguous per-tap GEMMs, used by the full-size
  parity tests for speed): agrees with the default einsum form (the
  reference's sliding window with zero-stuffed dilation) and with the
  float64 loops on every decoder, flow and encoder op shape
  (test_oracle_ops.py).
* ``pipeline_ref`` (``vc_prepare``, ``search_l2``, ``change_rms``,
  interpolation, protect, int16) and ``rmvpe_ref`` (log-mel, U-Net,
  BiGRU, decode): the reference's own outputs written by
  ``tests/golden/make_golden_pipeline.py`` / ``make_golden_rmvpe.py``, plus
  torch routines and float64 loops where those leave a case open
  (test_oracle_pipeline.py, test_oracle_rmvpe.py).
"""
