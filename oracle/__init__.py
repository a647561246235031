"""CPU oracle for the Mamba3 SISO state scan -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed CPU
baseline.  The product path (``sigma-0_amd``) never imports it and has no CPU
fallback: it fails loudly when the HIP library is missing.

Contents:
  mamba3_ref  -- numpy restatement of the reference's pure-JAX chunked scan
                 (src/base_model/models/mamba3_jax.py:62-419) and of the decode
                 recurrence rnn_step (src/base_model/models/mamba3.py:498-562).
  pins        -- independent formulations used to pin the restatement: the
                 quadratic (attention) form computed by brute force and the
                 token-by-token recurrence.
  inputs      -- seeded input generators for the benchmark configurations.
"""
