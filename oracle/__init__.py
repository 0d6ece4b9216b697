"""CPU oracle for the OmniWeave BiGEMM path — TEST INFRASTRUCTURE ONLY.

This package restates the upstream reference algorithm (``omniweave/models/routing.py``,
``omniweave/ops/reference.py``, ``omniweave/models/block.py``) on the CPU so that the HIP
backend in ``omniwave_amd`` can be checked against it.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it, and
only as the checker.  The product package never imports anything from here.

Modules
-------
``oracle.routing``  literal loop restatement of the route plans (integer work).
``oracle.bigemm``   pack -> gated two-sided einsum -> unpack in PyTorch on the CPU, the
                    block's RMSNorm/residual sequence, and an fp64 per-tile brute force.
``oracle.backbone`` the backbone's space_to_depth layout and stem (fp32).

How each function is pinned (tests named in brackets):

* route orders - golden vectors written by importing the reference's ``routing.py`` in
  the build container (``tests/golden/routes.json``) plus the reference's own coverage,
  count and schedule tests [tests/test_oracle_routing.py].
* ``pack_tiles`` / ``unpack_tiles`` - the reference's round-trip and zero-padding tests
  plus an element-by-element brute force [tests/test_oracle_ops.py].
* ``bigemm_delta_reference`` - the reference's closed-form single-tile test, its fp64
  gradcheck, and an fp64 per-tile brute force through the route tables that shares no
  code with the pack/einsum path [tests/test_oracle_ops.py].
* ``rmsnorm_reference`` - textbook RMS formula in fp64 and the reference's dtype sequence
  checked element-wise [tests/test_oracle_ops.py].
* ``space_to_depth_nhwc`` - an element loop over the definition (``space_to_depth_loops``)
  and the inverse property on an index image; ``stem_reference`` - a per-pixel fp64 dot
  product over the 4x4x3 patch written from the NCHW image directly [tests/test_backbone_glue.py].
"""
