"""CPU oracle for the Leech-lattice quantization path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of the reference's
Leech-lattice weight-quantization path (alavicka/pollux ``castor.py``,
``pack.py`` and ``pollux.py``) so that the HIP implementation in
``pollux_amd`` can be checked against it.  It is the checker, never the thing
measured or shipped: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product path
(``pollux_amd``) never imports it and fails loudly when its HIP library is
missing.

Modules
-------
codebook    Golay code and the 196,561-entry codebook (castor.py:74-199, 263-266)
packing     18-bit pack / unpack (castor.py:226-260)
nn          exact (float64) nearest-neighbour scoring for the three reference
            semantics NN-B / NN-T / NN-P, with near-tie classification
            (castor.py:407-460, 544-557; pack.py:167-177)
optim       the H24 branch of the optimiser step with every rounding explicit
            (pollux.py:815-878)
torch_ref   the reference's CPU path restated with the same torch ops:
            NN-B / NN-P search (castor.py:544-557, pack.py:167-177), row RMS,
            normalisation, rescale, the pack-time sigma16 (castor.py:309-339,
            pack.py:164, pollux.py:874-884), fp16 materialisation and the
            dense linear (pollux.py:485-507) -- also the CPU baseline of
            bench.py

How each function is pinned (golden vectors, closed forms, invariants,
independent restatements) is listed in each module's header.
"""
