"""CPU oracle for the trellis packed-linear decode-matmul.

TEST INFRASTRUCTURE ONLY. This package is the checker, never the product: only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import it. The product path (``trellis-everywhere_amd``) never calls into it and
fails loudly when its HIP library is missing.

Contents
--------
``trellis_np``   numpy restatement of the reference decode path (codebooks, packed
                 bit layout, wrapped-window decode, tile layout, block Hadamard,
                 restore, IP fold, dense matmul) plus the encode-side incoherence
                 processing used to build fixtures.
``torch_cpu``    the same decode-then-matmul written with torch CPU ops, used as the
                 timed CPU baseline (multi-threaded, as the reference runs on CPU).
``viterbi``      ctypes front end of ``viterbi.c``, a C restatement of the
                 reference's tail-biting Viterbi encoder (fixture generation only).

How each function is pinned (known-answer vectors, reference invariants, closed
forms, library routines) is listed in the module docstrings and exercised by
``tests/test_oracle_*.py``. Every oracle function has at least one such pin; none
is "parity unpinned".
"""
