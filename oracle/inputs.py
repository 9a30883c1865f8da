"""Seeded synthetic inputs of the parity tests: the generators are the
benchmark's workload definitions (gdnx_amd/workloads.py, data only, no
recurrence maths), re-exported here so the tests and the oracle's checks read
their inputs from one place."""
from gdnx_amd.workloads import (TAUS, config0, config1, config2, config3, decode_inputs,  # noqa: F401
                                dense_inputs, partial_rope)
