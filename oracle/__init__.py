"""CPU oracle for the sparse-convolution hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the algorithms of the reference package
(trispconv/pytorch/indices.py, functional.py, weight.py and the inverse branch
of modules.py) so that the HIP path can be checked against it.  Only the
test-suite, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only to check results or as the timed CPU
baseline.  The product path (``trispconv_amd``) never imports it and has no
CPU fallback.

Pinning (what checks each function, so that a plausible mistake fails one):

* ``pairs.subm_pairs``     — reference golden fixtures (subm_*: exact output
  coordinates, features to 1e-4), dense ``conv3d`` closed form, brute-force
  enumeration of (in, out, k) triples on tiny grids (pair order and values).
* ``pairs.strided_pairs``  — golden fixtures (strided_*), closed-form output
  set "conv3d(occupancy, ones) > 0", dense ``conv3d``, brute force (order).
* ``pairs.inverse_pairs``  — golden fixtures (inverse_*), dense
  ``conv_transpose3d``, brute force on tiny grids, coordinate round trip.
* ``weights.normalize_weight`` — golden fixture subm_1x1x1_c16 (fold quirk),
  dense ``conv3d`` (KRSC permutation), explicit index formula on random data.
* ``conv.conv_forward``   — all of the above through the feature values.

All of these live in ``tests/test_oracle.py``; none of them restates the
oracle's own formula.
"""
