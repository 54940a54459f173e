"""Oracle: CPU restatements of the reference's hot-path algorithms.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or, for the CPU baseline, as the thing timed on the
host).  The product package ``boa-constrictor_amd/`` never imports it.

Modules:
  ora            -- ctypes binding of rc_oracle.c (range coder core, Q2 and XQ quantisers, exp).
  bigint_check   -- independent big-integer interval check of any encoder's output words.
  model_ref      -- torch-CPU fp32 restatement of BoaBytePredictor (step and teacher-forced forward).
  codec_ref      -- CPU restatement of codec.compress_CPU/decompress_CPU (the reported CPU baseline).
  weights_ref    -- the seeded weight generator's restatement used to pin the product's blob hashes.
"""
