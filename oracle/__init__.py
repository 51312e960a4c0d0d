"""CPU oracle for the FP8 paged-attention decode path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``flydsl_amd`` imports this package;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker.  The product path runs the HIP
kernels in ``flydsl_amd/csrc`` and fails loudly when they are not built.

Modules:
  torch_ref   restatement of the reference's torch path
              (tests/kernels/test_pa.py:177-429): KV-cache construction,
              quantisers, value-layout shuffle, masked attention, the paged
              gather of ``torch_mha_extend``; plus the per-slot partials and
              the log-sum-exp merge of kernels/pa_decode_swa.py:954-1130.
  np_ref      independent float64 NumPy brute force (explicit token loops)
              used to pin ``torch_ref``.
  plan        integer planning: split count, slot ranges, sliding-window
              tile mapping, and the work-list scheduler of
              kernels/pa_metadata.py.
  fp8         OCP e4m3fn decode/encode written from the format definition.
"""
