"""CPU oracle for the packed-TCQ decode path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference TurboPress runtime
computes on its packed-TCQ path (``turbopress/runtime.py``,
``turbopress/trellis.py``, ``turbopress/hadamard.py``,
``turbopress/codebooks.py``).  It is the *checker*: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import it.  The product package ``turbopress_amd`` never imports,
links or executes anything under ``oracle/``.

Modules
-------
``tcq_oracle``      numpy restatement of the bit layout, trellis tables,
                    window decode, block FWHT, row decode and tiled forward.
``codebook_oracle`` torch-CPU restatement of the Lloyd-Max and
                    trellis-optimised codebooks (needs torch's RNG stream).
``tiled_baseline``  op-for-op torch-CPU restatement of the reference's
                    ``mode="tiled"`` forward, timed as the CPU baseline.
"""
