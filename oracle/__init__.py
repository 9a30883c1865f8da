"""CPU oracle for the chunked GDN3 / KMD-2 recurrence.

TEST INFRASTRUCTURE ONLY.  This package restates, on the CPU and in plain
PyTorch (float64 by default), the sequential recurrences of the reference
repository PhantomG27249/GDNX.  It is the checker against which the HIP
library in ``gdnx_amd`` is compared.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it; the product path
(``gdnx_amd``) never imports, calls or links anything from here, and fails
loudly when its HIP library is missing instead of falling back to this code.

Modules:
  delta   -- dense decoupled-erase delta rule (KMD-2 ``scan`` semantics and the
             GDN3 dense / bridge regime), sequential and chunked forms.
  gdn3    -- GDN3 Kronecker-residual recurrence with circular residual buffer
             and two-timescale rearrangement-SVD compaction.
  inputs  -- seeded synthetic input generators for the benchmark configs.

Pinning status of every function is listed in each module header.
"""
