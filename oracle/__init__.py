"""CPU oracle for the QSRT encoder hot path -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (``qsrt_amd``) may import this package.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg use it, and only as the checker (or the timed CPU baseline), never as a
thing that is shipped or measured as the GPU result.

Contents (each function cites the reference file:line it restates):

* ``tables``   -- numpy restatement of the SQG E4M3 alphabets
                  (reference ``qsrt/sqg_e4m3.py``), with an independent
                  E4M3 round-to-nearest-even encoder.
* ``fmt``      -- numpy restatement of cyclic states, EXL word packing,
                  tensor-core permutation, Sylvester Hadamard and the
                  reference decode (``qsrt/qsrt.py``, ``qsrt/exl3_reference.py``).
* ``viterbi``  -- ctypes binding to ``viterbi_ref.c``: the tail-biting tile
                  Viterbi (``qsrt/csrc/qsrt_quantize_tiles_kernel.cuh``,
                  ``qsrt_quantize_tiles_k2_kernel.cuh``) in plain FP32 C, plus
                  a pure-Python exhaustive search for tiny trellises.
* ``ldlq``     -- float64 numpy restatement of block LDL, BlockLDLQ and the
                  regularisation/scale search (``qsrt/exl3_encoder_backend.py``).

Pinning status of every function is recorded next to it ("pinned by ...");
a function with no independent check says "parity unpinned".
"""
