"""CPU oracle of the F-side routed-expert path: TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import anything here, and only to check or time against it. The
product package (``sgl-afd-plugin_amd/sgl_asap_amd``) never imports, links or runs this
code: its kernels are HIP, and it raises when the HIP library is missing.

Modules:
* ``formats``   - E2M1 / UE8M0 / e4m3fn codecs and the MX (per-32) and FP8-block
                  (1x128, 128x128) quantizers, numpy, bit-level.
* ``routing``   - the stable expert-contiguous permutation of local (token, k) pairs.
* ``experts``   - fp32 expert FFN on dequantized operands (torch CPU), finalize
                  (top-k weighted sum) and the A-side combine.
* ``transport`` - doorbell word, arena geometry and the F poller's rules, plain Python.

Every function cites the reference file:line it restates. How each one is pinned (known
answers, closed forms, library casts, brute force) is written in its docstring; the
checks are tests/test_oracle_*.py, tests/test_transport.py and tests/test_golden.py.
"""
